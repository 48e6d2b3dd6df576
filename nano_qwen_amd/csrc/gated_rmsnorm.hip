// Gated RMS norm at the Gated DeltaNet output (gfx950).
//
// Reference: RMSNormGated.forward (layers/layernorm.py:143-157), applied as
// self.norm(out, z) in GatedDeltaNet (layers/gated_delta_net.py:205-207,
// 268-270), eager:
//   x = hidden.float(); x = x * rsqrt(mean(x^2) + eps)
//   x = x.to(dtype) * weight.to(dtype)          (16-bit product, rounded)
//   x = x * silu(gate.float())                   (fp32)
//   return x.to(dtype)
// several launches and temporaries there; one pass here.  A row (D
// elements) is D/8 adjacent lanes with 8 consecutive elements each; the sum
// of squares is each lane's 8 squares left to right, then a butterfly over
// the row's lanes, every operation rounded on its own.
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kThreads = 256;

template <class T>
__device__ inline float rnd16(float f) {
  asm("" : "+v"(f));  // keep the fp32 value: no fused product-and-narrow
  return T::to_float(T::from_float(f));
}

template <class T, int LPU>
__global__ __launch_bounds__(kThreads) void gated_rmsnorm_kernel(const uint8_t *x, int64_t x_rs, const uint8_t *z,
                                                                 int64_t z_rs, const float *w, float eps,
                                                                 uint8_t *out, int64_t o_rs, int64_t rows) {
#pragma clang fp contract(off)
  constexpr int D = LPU * 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t row = gid / LPU;
  const int l = static_cast<int>(gid % LPU);
  if (row >= rows) return;
  const u32x4 xr = load16(x + row * x_rs + l * 16);
  const u32x4 zr = load16(z + row * z_rs + l * 16);
  const f32x4 w0 = reinterpret_cast<const f32x4 *>(w + 8 * l)[0];
  const f32x4 w1 = reinterpret_cast<const f32x4 *>(w + 8 * l)[1];
  const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
  float xv[8], zv[8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    xv[2 * t] = T::to_float(static_cast<uint16_t>(xr[t] & 0xffffu));
    xv[2 * t + 1] = T::to_float(static_cast<uint16_t>(xr[t] >> 16));
    zv[2 * t] = T::to_float(static_cast<uint16_t>(zr[t] & 0xffffu));
    zv[2 * t + 1] = T::to_float(static_cast<uint16_t>(zr[t] >> 16));
  }
  float ss = xv[0] * xv[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) ss += xv[i] * xv[i];
#pragma unroll
  for (int off = LPU / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, LPU);
  const float r = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + eps);
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float n = rnd16<T>(xv[i] * r);
    const float nw = rnd16<T>(n * T::to_float(T::from_float(wv[i])));
    // silu(z) = z / (1 + e^-z) with the hardware exp2 and reciprocal (about
    // one fp32 ulp each): the output's single rounding moves by one 16-bit
    // ulp only for values within those few ulps of a rounding boundary, and
    // the pass stays memory-bound instead of paying for expf and a division
    const float silu = zv[i] * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(zv[i] * -1.4426950408889634f));
    y[i] = nw * silu;
  }
  u32x4 o;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float a0 = y[2 * t], a1 = y[2 * t + 1];
    asm("" : "+v"(a0), "+v"(a1));
    o[t] = T::pack2(a0, a1);
  }
  __builtin_nontemporal_store(o, reinterpret_cast<u32x4 *>(out + row * o_rs + l * 16));
}

template <class T>
void launch(const uint8_t *x, int64_t x_rs, const uint8_t *z, int64_t z_rs, const float *w, float eps, uint8_t *out,
            int64_t o_rs, int64_t rows, int d, unsigned blocks, hipStream_t s) {
  if (d == 64)
    gated_rmsnorm_kernel<T, 8><<<blocks, kThreads, 0, s>>>(x, x_rs, z, z_rs, w, eps, out, o_rs, rows);
  else if (d == 128)
    gated_rmsnorm_kernel<T, 16><<<blocks, kThreads, 0, s>>>(x, x_rs, z, z_rs, w, eps, out, o_rs, rows);
  else
    gated_rmsnorm_kernel<T, 32><<<blocks, kThreads, 0, s>>>(x, x_rs, z, z_rs, w, eps, out, o_rs, rows);
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_gated_rmsnorm(const void *x, int64_t x_row_stride, const void *gate, int64_t gate_row_stride,
                                const float *weight, float eps, void *out, int64_t out_row_stride, int64_t rows,
                                int dim, int dtype, void *stream) {
  if (rows < 0 || (dim != 64 && dim != 128 && dim != 256))
    return fail(rows < 0 ? NQ_EINVAL : NQ_EUNSUPPORTED, "gated_rmsnorm: rows %lld, dim %d (built: 64/128/256)",
                (long long)rows, dim);
  if (dtype != NQ_BF16 && dtype != NQ_F16) return fail(NQ_EUNSUPPORTED, "gated_rmsnorm: dtype %d (f16/bf16)", dtype);
  if (rows == 0) return NQ_OK;
  if (!x || !gate || !weight || !out) return fail(NQ_EINVAL, "gated_rmsnorm: null pointer");
  if (!aligned(x, 16) || !aligned(gate, 16) || !aligned(out, 16) || !aligned(weight, 16) ||
      (x_row_stride * 2) % 16 || (gate_row_stride * 2) % 16 || (out_row_stride * 2) % 16)
    return fail(NQ_EINVAL, "gated_rmsnorm: pointers and row strides must be 16-byte aligned");
  const int64_t lanes = rows * (dim / 8);
  const int64_t blocks = (lanes + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffffLL) return fail(NQ_EINVAL, "gated_rmsnorm: too many rows for one launch");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto *xp = static_cast<const uint8_t *>(x);
  const auto *zp = static_cast<const uint8_t *>(gate);
  auto *op = static_cast<uint8_t *>(out);
  if (dtype == NQ_BF16)
    launch<BF16>(xp, x_row_stride * 2, zp, gate_row_stride * 2, weight, eps, op, out_row_stride * 2, rows, dim,
                 static_cast<unsigned>(blocks), s);
  else
    launch<F16>(xp, x_row_stride * 2, zp, gate_row_stride * 2, weight, eps, op, out_row_stride * 2, rows, dim,
                static_cast<unsigned>(blocks), s);
  return check_launch("gated_rmsnorm");
}
