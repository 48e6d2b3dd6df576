// Causal depthwise conv1d + silu in front of the Gated DeltaNet (gfx950).
//
// Reference: GatedDeltaNet (layers/gated_delta_net.py)
//   prefill (:178-180, 207-213):  silu(conv1d(qkv)[:, :, :S]) with padding
//     K - 1 (a causal conv from zeros); the state kept for decode is the
//     last K - 1 raw inputs;
//   decode  (:218-227):  x = cat(conv_state, qkv); silu(conv1d(x)); the new
//     state is x[:, 1:].
// Per channel c and token t (window of the K inputs ending at t, earlier
// positions from the sequence's initial state or zero):
//   y = rnd(sum_j w[c][j] * x[t - K + 1 + j])    (fp32, j = 0 .. K-1 in order)
//   out = rnd(y / (1 + exp(-y)))
// with rnd = round to the 16-bit type, as torch computes the bf16 conv and the
// silu on its bf16 result.
//
// Prefill (conv_prefill8, channel counts that are multiples of 8 with
// 16-byte aligned rows): one lane per 8 channels and run of kRun8 tokens;
// the lane issues the 16-byte loads of all kRun8 + K - 1 input rows of its
// run before computing any output, so a wave keeps that many loads in
// flight, and stores each output row as one 16-byte store.  The runs of a
// sequence are independent, so prefill is parallel over tokens too.
// Decode and other channel counts (conv_kernel): one lane per pair of
// channels and run of kRun tokens, the last K - 1 inputs kept in registers
// as a sliding window.
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxK = 8;
constexpr int kRun = 32;  // tokens per lane and run

struct ConvArgs {
  const uint8_t *x;  // [T, C] rows (16-bit)
  int64_t x_rs;      // bytes
  const uint8_t *w;  // [C, K] (16-bit)
  const int32_t *cu;  // [N + 1], or null: one token per sequence (decode)
  uint8_t *state;     // [slots, C, K - 1] (16-bit)
  const int32_t *idx;  // [N]
  int64_t num_slots;
  int from_state;
  uint8_t *out;  // [T, C]
  int64_t o_rs;
  int C, K, N;
};

template <class T>
__device__ inline float ld16(const uint8_t *p, int64_t i) {
  return T::to_float(reinterpret_cast<const uint16_t *>(p)[i]);
}
template <class T>
__device__ inline float rnd16(float f) {
  asm("" : "+v"(f));
  return T::to_float(T::from_float(f));
}

// grid.x covers channel pairs, grid.y = sequence (decode: the token), and
// grid.z walks a prefill sequence's runs (run z, z + gridDim.z, ...).
template <class T>
__global__ __launch_bounds__(kThreads) void conv_kernel(const ConvArgs a) {
#pragma clang fp contract(off)
  const int c = 2 * (blockIdx.x * kThreads + threadIdx.x);
  const int n = blockIdx.y;
  if (c >= a.C) return;
  const int K = a.K;
  int64_t t0 = n, t1 = n + 1;
  if (a.cu) {
    t0 = a.cu[n];
    t1 = a.cu[n + 1];
  }
  const int32_t slot = a.idx[n];
  const bool has_slot = slot >= 0 && slot < a.num_slots;
  const int64_t sbase = (static_cast<int64_t>(has_slot ? slot : 0) * a.C) * (K - 1);
  float w0[kMaxK], w1[kMaxK];
#pragma unroll
  for (int j = 0; j < kMaxK; ++j)
    if (j < K) {
      w0[j] = ld16<T>(a.w, static_cast<int64_t>(c) * K + j);
      w1[j] = c + 1 < a.C ? ld16<T>(a.w, static_cast<int64_t>(c + 1) * K + j) : 0.f;
    }
  // Input at position p of this sequence (p < t0: the initial state or zero).
  auto in = [&](int64_t p, int ch) -> float {
    if (ch >= a.C) return 0.f;
    if (p >= t0) return ld16<T>(a.x + p * a.x_rs, ch);
    const int64_t back = t0 - p;  // 1 .. K-1
    if (!(a.from_state && has_slot) || back > K - 1) return 0.f;
    return ld16<T>(a.state, sbase + static_cast<int64_t>(ch) * (K - 1) + (K - 1 - back));
  };
  // Both channels of input position p as one 4-byte load (p >= t0), else
  // from the state or zero.
  auto in2 = [&](int64_t p, float &v0, float &v1) {
    if (p >= t0 && c + 1 < a.C) {
      const uint32_t w2 = *reinterpret_cast<const uint32_t *>(a.x + p * a.x_rs + 2 * c);
      v0 = T::to_float(static_cast<uint16_t>(w2 & 0xffffu));
      v1 = T::to_float(static_cast<uint16_t>(w2 >> 16));
    } else {
      v0 = in(p, c);
      v1 = in(p, c + 1);
    }
  };
  const int64_t nrun = (t1 - t0 + kRun - 1) / kRun;
  for (int64_t run = blockIdx.z; run < nrun; run += gridDim.z) {
    const int64_t ts = t0 + run * kRun, te = min(ts + kRun, t1);
    float h0[kMaxK], h1[kMaxK];  // window: inputs ts - K + 1 + j, j < K - 1
#pragma unroll
    for (int j = 0; j < kMaxK - 1; ++j)
      if (j < K - 1) in2(ts - K + 1 + j, h0[j], h1[j]);
    for (int64_t t = ts; t < te; ++t) {
      float x0, x1;
      in2(t, x0, x1);
      float y0 = 0.f, y1 = 0.f;
#pragma unroll
      for (int j = 0; j < kMaxK; ++j)
        if (j < K) {
          const float v0 = j < K - 1 ? h0[j] : x0, v1 = j < K - 1 ? h1[j] : x1;
          y0 += w0[j] * v0;
          y1 += w1[j] * v1;
        }
#pragma unroll
      for (int j = 0; j < kMaxK - 1; ++j)
        if (j < K - 1) {
          h0[j] = j + 1 < K - 1 ? h0[j + 1] : x0;
          h1[j] = j + 1 < K - 1 ? h1[j + 1] : x1;
        }
      y0 = rnd16<T>(y0);
      y1 = rnd16<T>(y1);
      const float s0 = y0 / (1.0f + expf(-y0)), s1 = y1 / (1.0f + expf(-y1));
      uint16_t *op = reinterpret_cast<uint16_t *>(a.out + t * a.o_rs) + c;
      if (c + 1 < a.C) {
        float r0 = s0, r1 = s1;
        asm("" : "+v"(r0), "+v"(r1));
        __builtin_nontemporal_store(T::pack2(r0, r1), reinterpret_cast<uint32_t *>(op));
      } else {
        op[0] = T::from_float(rnd16<T>(s0));
      }
    }
  }

  // The state after the sequence: its last K - 1 inputs, written by the
  // z = 0 workgroups.  Decode (grid.z = 1): the same lane read the old state
  // above.  Prefill never reads the state (it starts from zero, as the
  // reference does), so other token blocks cannot race with this write.
  if (!has_slot || blockIdx.z != 0) return;
  float keep0[kMaxK], keep1[kMaxK];
#pragma unroll
  for (int j = 0; j < kMaxK - 1; ++j)
    if (j < K - 1) {
      keep0[j] = in(t1 - (K - 1) + j, c);
      keep1[j] = in(t1 - (K - 1) + j, c + 1);
    }
#pragma unroll
  for (int j = 0; j < kMaxK - 1; ++j)
    if (j < K - 1) {
      uint16_t *sp = reinterpret_cast<uint16_t *>(a.state) + sbase;
      sp[static_cast<int64_t>(c) * (K - 1) + j] = T::from_float(keep0[j]);
      if (c + 1 < a.C) sp[static_cast<int64_t>(c + 1) * (K - 1) + j] = T::from_float(keep1[j]);
    }
}

constexpr int kRun8 = 16;  // tokens per lane and run (prefill, 8 channels per lane)

// Prefill from a zero state, 8 channels per lane (C % 8 == 0, rows 16-byte
// aligned).  grid.x covers channel groups, grid.z = sequence, grid.y walks
// the sequence's runs (run y, y + gridDim.y, ...).
template <class T, int K>
__global__ __launch_bounds__(kThreads) void conv_prefill8(const ConvArgs a) {
  const int c = 8 * (blockIdx.x * kThreads + threadIdx.x);
  if (c >= a.C) return;
  const int n = blockIdx.z;
  const int64_t t0 = a.cu[n], t1 = a.cu[n + 1];
  float w[8][K];
#pragma unroll
  for (int ch = 0; ch < 8; ++ch)
#pragma unroll
    for (int j = 0; j < K; ++j) w[ch][j] = ld16<T>(a.w, static_cast<int64_t>(c + ch) * K + j);
  // Eight channels of input position p (zero before the sequence: prefill
  // starts from a zero state).
  auto in8 = [&](int64_t p) -> u32x4 {
    return (p >= t0 && p < t1) ? *reinterpret_cast<const u32x4 *>(a.x + p * a.x_rs + 2 * c) : u32x4{0, 0, 0, 0};
  };
  // The eight channels of a row as floats, converted once per input row;
  // the empty asm keeps the compiler from converting again at every tap.
  auto unpack8 = [](const u32x4 &v, float (&f)[8]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f[2 * q] = T::to_float(static_cast<uint16_t>(v[q] & 0xffffu));
      f[2 * q + 1] = T::to_float(static_cast<uint16_t>(v[q] >> 16));
      asm("" : "+v"(f[2 * q]), "+v"(f[2 * q + 1]));
    }
  };
  const int64_t nrun = (t1 - t0 + kRun8 - 1) / kRun8;
  for (int64_t run = blockIdx.y; run < nrun; run += gridDim.y) {
    const int64_t ts = t0 + run * kRun8;
    // Input rows ts - K + 1 .. ts + kRun8 - 1 through a descriptor over the
    // rows of the sequence among them: a row before or after the sequence
    // lies outside it (its offset, negative or past the end, is out of
    // range as an unsigned number) and reads as zeros.
    const int64_t lo = ts - (K - 1) > t0 ? ts - (K - 1) : t0;
    const int64_t hi = ts + kRun8 < t1 ? ts + kRun8 : t1;
    const auto rs = make_rsrc(a.x + lo * a.x_rs, static_cast<uint32_t>((hi - lo) * a.x_rs));
    const int off0 = static_cast<int>((ts - (K - 1) - lo) * a.x_rs) + 2 * c;
    u32x4 xin[kRun8 + K - 1];
#pragma unroll
    for (int i = 0; i < kRun8 + K - 1; ++i)
      xin[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off0 + i * static_cast<int>(a.x_rs), 0, 0));
    const auto ors = make_rsrc(a.out + ts * a.o_rs, static_cast<uint32_t>((hi - ts) * a.o_rs));
    float win[K][8];  // input rows i .. i + K - 1 of output i
#pragma unroll
    for (int j = 0; j < K - 1; ++j) unpack8(xin[j], win[j + 1]);
#pragma unroll
    for (int i = 0; i < kRun8; ++i) {
#pragma unroll
      for (int j = 0; j < K - 1; ++j)
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) win[j][ch] = win[j + 1][ch];
      unpack8(xin[i + K - 1], win[K - 1]);
      float y[8];
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) {
        // The product of two 16-bit values is exact in float32, so the
        // fused multiply-add rounds exactly as the add after the multiply.
        y[ch] = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) y[ch] = __builtin_fmaf(w[ch][j], win[j][ch], y[ch]);
      }
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // Both sums rounded to 16 bits by one pack, then silu with the
        // hardware exp2 and reciprocal (about 1 ulp each), rounded again.
        const uint32_t yp = T::pack2(y[2 * q], y[2 * q + 1]);
        float r[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float v = T::to_float(static_cast<uint16_t>(h ? yp >> 16 : yp & 0xffffu));
          r[h] = v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f));
        }
        o[q] = T::pack2(r[0], r[1]);
      }
      // Rows past the sequence fall outside the descriptor and are dropped.
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), ors, i * static_cast<int>(a.o_rs) + 2 * c, 0, 2);
    }
  }
  // The state after the sequence: its last K - 1 inputs (zero before it).
  const int32_t slot = a.idx[n];
  if (slot < 0 || slot >= a.num_slots || blockIdx.y != 0) return;
  uint16_t *sp = reinterpret_cast<uint16_t *>(a.state) + static_cast<int64_t>(slot) * a.C * (K - 1);
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const u32x4 v = in8(t1 - (K - 1) + j);
#pragma unroll
    for (int ch = 0; ch < 8; ++ch)
      sp[static_cast<int64_t>(c + ch) * (K - 1) + j] = static_cast<uint16_t>((ch & 1) ? (v[ch >> 1] >> 16) : (v[ch >> 1] & 0xffffu));
  }
}

template <class T, int K>
int launch_prefill8(const ConvArgs &g, hipStream_t s) {
  const int groups = g.C / 8;
  // A sequence's runs are neighbours in dispatch order: its rows are read
  // and written as one region.
  dim3 grid((groups + kThreads - 1) / kThreads, 64, g.N);  // 64 runs at a time
  conv_prefill8<T, K><<<grid, kThreads, 0, s>>>(g);
  return check_launch("gdn_conv1d");
}
template <class T>
int launch_prefill8_k(const ConvArgs &g, hipStream_t s) {
  switch (g.K) {
    case 2: return launch_prefill8<T, 2>(g, s);
    case 3: return launch_prefill8<T, 3>(g, s);
    case 4: return launch_prefill8<T, 4>(g, s);
    case 5: return launch_prefill8<T, 5>(g, s);
    case 6: return launch_prefill8<T, 6>(g, s);
    case 7: return launch_prefill8<T, 7>(g, s);
    default: return launch_prefill8<T, 8>(g, s);
  }
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_gdn_conv1d(const void *x, int64_t x_row_stride, const void *weight, int kernel_size,
                             const int32_t *cu_seqlens, int num_seqs, void *conv_state,
                             const int32_t *state_indices, int64_t num_slots, int initial_state_from_slot,
                             void *out, int64_t out_row_stride, int channels, int dtype, void *stream) {
  if (num_seqs < 0 || channels <= 0 || kernel_size < 2 || kernel_size > kMaxK || num_slots < 0)
    return fail(NQ_EINVAL, "gdn_conv1d: bad sizes (seqs=%d channels=%d kernel=%d, kernel in [2, %d])", num_seqs,
                channels, kernel_size, kMaxK);
  if (dtype != NQ_BF16 && dtype != NQ_F16) return fail(NQ_EUNSUPPORTED, "gdn_conv1d: dtype %d (f16/bf16)", dtype);
  if (cu_seqlens && initial_state_from_slot)
    return fail(NQ_EUNSUPPORTED, "gdn_conv1d: prefill starts from a zero state (as the reference's does)");
  if (num_seqs == 0) return NQ_OK;
  if (!x || !weight || !conv_state || !state_indices || !out) return fail(NQ_EINVAL, "gdn_conv1d: null pointer");
  if (x_row_stride < channels || out_row_stride < channels)
    return fail(NQ_EINVAL, "gdn_conv1d: row strides %lld/%lld below the %d channels", static_cast<long long>(x_row_stride),
                static_cast<long long>(out_row_stride), channels);
  if (!aligned(out, 4) || (out_row_stride * 2) % 4 || !aligned(x, 4) || (x_row_stride * 2) % 4)
    return fail(NQ_EINVAL, "gdn_conv1d: x and out rows 4-byte aligned");
  if (num_seqs > 65535) return fail(NQ_EINVAL, "gdn_conv1d: too many sequences for one launch");
  ConvArgs g{};
  g.x = static_cast<const uint8_t *>(x);
  g.x_rs = x_row_stride * 2;
  g.w = static_cast<const uint8_t *>(weight);
  g.cu = cu_seqlens;
  g.state = static_cast<uint8_t *>(conv_state);
  g.idx = state_indices;
  g.num_slots = num_slots;
  g.from_state = cu_seqlens ? 0 : 1;
  g.out = static_cast<uint8_t *>(out);
  g.o_rs = out_row_stride * 2;
  g.C = channels;
  g.K = kernel_size;
  g.N = num_seqs;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The 8-channel prefill kernel addresses a run's input rows by 32-bit
  // offsets from the run's first row, negative ones included.
  if (cu_seqlens && channels % 8 == 0 && aligned(x, 16) && aligned(out, 16) && (x_row_stride * 2) % 16 == 0 &&
      (out_row_stride * 2) % 16 == 0 && g.x_rs * (kRun8 + kMaxK) < (int64_t{1} << 31) &&
      g.o_rs * kRun8 < (int64_t{1} << 31))
    return dtype == NQ_BF16 ? launch_prefill8_k<BF16>(g, s) : launch_prefill8_k<F16>(g, s);
  // Channel pairs over grid.x; the tokens of a prefill sequence over grid.z.
  const int pairs = (channels + 1) / 2;
  dim3 grid((pairs + kThreads - 1) / kThreads, num_seqs, cu_seqlens ? 64 : 1);  // 64 runs at a time
  if (dtype == NQ_BF16) conv_kernel<BF16><<<grid, kThreads, 0, s>>>(g);
  else conv_kernel<F16><<<grid, kThreads, 0, s>>>(g);
  return check_launch("gdn_conv1d");
}
