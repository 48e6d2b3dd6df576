// Fused q/k Gemma RMS norm + partial rotary embedding + KV-cache store (gfx950).
//
// Reference: the part of Qwen3_5Attention.forward between the projections
// and the attention call (models/qwen3_5.py:135-139):
//   query = q_norm(query); key = k_norm(key)          layers/layernorm.py:81-91
//   query, key = rotary_emb(positions, query, key)    layers/rotary_embedding.py:104-123
//   store_kvcache(key, value, k_cache, v_cache, ...)  layers/attention.py:62-63
// There q and k make three round trips through HBM over four launches; here
// one launch reads q, k and v once and writes q_out, k_out and the cache rows.
//
// One workgroup per token.  A head row (head_dim = D elements) is handled by
// D/8 adjacent lanes with 8 consecutive elements each (16 bytes in bf16).
// A row never straddles a wave, so its sum of squares is a butterfly over
// its lanes, and the rotary partner of element e (e +- R/2, R = rotary dim,
// a multiple of 16) sits R/16 lanes away: one lane shuffle per element.
// The token's rows are its Hq q rows, its Hkv k rows and (when a cache is
// given) its Hkv value rows, which are only copied (or quantized) into the
// value cache.
//
// Arithmetic, per row x of one head (fp32 throughout, `rnd` = round to the
// tensor's dtype, nearest even):
//   r = 1 / sqrt(sum(x*x) / D + eps)        IEEE sqrt and divide; the sum in
//                                           a fixed order (see the kernel)
//   y = rnd(rnd(x * r) * (w + weight_offset))
//       -- GemmaRMSNorm under torch.compile: x.to(dtype) rounds, the
//          1.0 + weight and the product stay fp32 until the output cast
//   for e < R (rotary part), with c, s = cos_sin_cache[pos][e mod R/2]:
//       e <  R/2: z = rnd(y[e] * c - y[e + R/2] * s)
//       e >= R/2: z = rnd(y[e] * c + y[e - R/2] * s)
//   for e >= R: z = y[e]
// Products are formed separately (no fused multiply-add), as in the
// reference's elementwise ops.  A position outside [0, max_position) makes
// the whole row NaN (the reference's table index would fail).
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kThreads = 256;

// Cache modes of the kernel.
enum { kNoCache = 0, kSameCache = 1, kFp8Cache = 2 };

// 8 consecutive elements <-> fp32.
template <int DT>
__device__ inline void load8(const void *p, float x[8]) {
  if constexpr (DT == NQ_F32) {
    const f32x4 a = reinterpret_cast<const f32x4 *>(p)[0];
    const f32x4 b = reinterpret_cast<const f32x4 *>(p)[1];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      x[t] = a[t];
      x[4 + t] = b[t];
    }
  } else {
    const u32x4 w = load16(p);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint16_t lo = static_cast<uint16_t>(w[t] & 0xffffu);
      const uint16_t hi = static_cast<uint16_t>(w[t] >> 16);
      if constexpr (DT == NQ_BF16) {
        x[2 * t] = BF16::to_float(lo);
        x[2 * t + 1] = BF16::to_float(hi);
      } else {
        x[2 * t] = F16::to_float(lo);
        x[2 * t + 1] = F16::to_float(hi);
      }
    }
  }
}

// Round an fp32 result to DT.  The empty asm materialises the fp32 value
// first: otherwise the compiler folds a product and its narrowing into one
// v_fma_mixlo_f16, which rounds once where the reference rounds twice (an
// fp32 product, then the cast).
template <int DT>
__device__ inline float rnd(float f) {
  if constexpr (DT != NQ_F32) asm("" : "+v"(f));
  if constexpr (DT == NQ_BF16) return BF16::to_float(BF16::from_float(f));
  else if constexpr (DT == NQ_F16) return F16::to_float(F16::from_float(f));
  else return f;
}

// Stores 8 values that are already representable in DT.  Every output is
// written once and not read back by this kernel: non-temporal stores (the
// streaming hint) take about a quarter off the kernel's time at cfg3 sizes.
template <int DT>
__device__ inline void store8(void *p, const float x[8]) {
  if constexpr (DT == NQ_F32) {
    __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f32x4 *>(p));
    __builtin_nontemporal_store(f32x4{x[4], x[5], x[6], x[7]}, reinterpret_cast<f32x4 *>(p) + 1);
  } else {
    u32x4 w;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      w[t] = DT == NQ_BF16 ? BF16::pack2(x[2 * t], x[2 * t + 1]) : F16::pack2(x[2 * t], x[2 * t + 1]);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(p));
  }
}

// 8 values -> 8 e4m3fn bytes, as nq_store_kvcache quantizes.
__device__ inline void store8_fp8(void *p, const float x[8], float inv) {
  u32x2 w;
  w[0] = fp8x4(x[0] * inv, x[1] * inv, x[2] * inv, x[3] * inv);
  w[1] = fp8x4(x[4] * inv, x[5] * inv, x[6] * inv, x[7] * inv);
  __builtin_nontemporal_store(w, reinterpret_cast<u32x2 *>(p));
}

struct Args {
  const char *q;
  int64_t q_row, q_head;  // strides in elements
  const char *k;
  int64_t k_row;
  const char *v;
  int64_t v_row;
  const int64_t *positions;
  const float *cos_sin;  // [max_position, R]: R/2 cosines, then R/2 sines
  int64_t max_position;
  int rot;  // R
  const char *q_w, *k_w;
  float eps, w_off;
  char *q_out;
  int64_t qo_row, qo_head;
  char *k_out;  // may be null
  int64_t ko_row;
  char *k_cache, *v_cache;
  const int32_t *slots;
  int64_t num_slots;
  const float *k_scale, *v_scale;
  int hq, hkv;
  int units;  // rows per token: hq + hkv, plus hkv value rows with a cache
};

// One workgroup per token.  Thread t always sits at lane l = t % LPU of its
// rows (256 is a multiple of LPU), so its weights and its cos/sin slice are
// loaded once; it then takes rows t / LPU, t / LPU + 256 / LPU, ... of the
// token's q rows, k rows and value rows, one row at a time.  (Issuing the
// loads of several rows first measured slower: the extra registers cost more
// occupancy than the deeper queue gains.)
template <int DT, int LPU, int CACHE>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(Args a) {
  // Every float operation rounds on its own (no contraction into FMA), so the
  // result is a fixed function of the inputs.
#pragma clang fp contract(off)
  constexpr int D = LPU * 8;
  constexpr int ES = DT == NQ_F32 ? 4 : 2;  // element bytes
  constexpr int RPP = kThreads / LPU;       // rows per pass of the workgroup
  const int64_t tok = blockIdx.x;
  const int l = threadIdx.x % LPU;
  const int r0 = threadIdx.x / LPU;
  const int e0 = 8 * l;
  const int lane = static_cast<int>(threadIdx.x & 63);

  const int64_t pos = a.positions[tok];
  const bool bad_pos = pos < 0 || pos >= a.max_position;
  int32_t slot = -1;
  if constexpr (CACHE != kNoCache) slot = a.slots[tok];
  const bool store = CACHE != kNoCache && slot >= 0 && slot < a.num_slots;

  float wq[8], wk[8];
  load8<DT>(a.q_w + e0 * ES, wq);
  load8<DT>(a.k_w + e0 * ES, wk);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    wq[i] += a.w_off;
    wk[i] += a.w_off;
  }
  // Rotary slice of this lane: elements [e0, e0 + 8) < R pair with e0 +- R/2.
  const int half = a.rot >> 1;
  const bool rot_lane = e0 < a.rot;
  const bool first = e0 < half;
  const int partner = rot_lane ? (first ? lane + (half >> 3) : lane - (half >> 3)) : lane;
  float c[8], sn[8];
  if (rot_lane) {
    const float *cs = a.cos_sin + (bad_pos ? 0 : pos) * a.rot + (first ? e0 : e0 - half);
    const f32x4 c0 = reinterpret_cast<const f32x4 *>(cs)[0];
    const f32x4 c1 = reinterpret_cast<const f32x4 *>(cs)[1];
    const f32x4 s0 = reinterpret_cast<const f32x4 *>(cs + half)[0];
    const f32x4 s1 = reinterpret_cast<const f32x4 *>(cs + half)[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = c0[i];
      c[4 + i] = c1[i];
      sn[i] = s0[i];
      sn[4 + i] = s1[i];
    }
  }

  for (int h = r0; h < a.units; h += RPP) {
    float x[8];
    {
      const char *src;
      if (h < a.hq) src = a.q + (tok * a.q_row + h * a.q_head + e0) * ES;
      else if (h < a.hq + a.hkv) src = a.k + (tok * a.k_row + (h - a.hq) * D + e0) * ES;
      else src = a.v + (tok * a.v_row + (h - a.hq - a.hkv) * D + e0) * ES;
      load8<DT>(src, x);
    }
    if (h >= a.hq + a.hkv) {  // value row: into the cache only
      if constexpr (CACHE != kNoCache) {
        if (store) {
          const int vh = h - a.hq - a.hkv;
          const int64_t dst_e = (static_cast<int64_t>(slot) * a.hkv + vh) * D + e0;
          if constexpr (CACHE == kSameCache) store8<DT>(a.v_cache + dst_e * ES, x);
          else store8_fp8(a.v_cache + dst_e, x, 1.0f / a.v_scale[vh]);
        }
      }
      continue;
    }
    const bool is_k = h >= a.hq;
    // r = 1 / sqrt(mean(x^2) + eps).  Summation order: each lane adds its 8
    // squares left to right, then a butterfly over the row's lanes (offsets
    // LPU/2, ..., 1); addition commutes, so every lane ends with the same sum.
    float ss = x[0] * x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) ss += x[i] * x[i];
#pragma unroll
    for (int off = LPU / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, LPU);
    float r = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + a.eps);
    if (bad_pos) r = __builtin_nanf("");
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = rnd<DT>(rnd<DT>(x[i] * r) * (is_k ? wk[i] : wq[i]));
    float yp[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) yp[i] = __shfl(y[i], partner, 64);
    if (rot_lane) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float a0 = y[i] * c[i];
        const float b0 = yp[i] * sn[i];
        y[i] = rnd<DT>(first ? a0 - b0 : a0 + b0);
      }
    }
    if (!is_k) {
      store8<DT>(a.q_out + (tok * a.qo_row + h * a.qo_head + e0) * ES, y);
      continue;
    }
    const int kh = h - a.hq;
    if (a.k_out) store8<DT>(a.k_out + (tok * a.ko_row + kh * D + e0) * ES, y);
    if constexpr (CACHE != kNoCache) {
      if (store) {
        const int64_t dst_e = (static_cast<int64_t>(slot) * a.hkv + kh) * D + e0;
        if constexpr (CACHE == kSameCache) store8<DT>(a.k_cache + dst_e * ES, y);
        else store8_fp8(a.k_cache + dst_e, y, 1.0f / a.k_scale[kh]);
      }
    }
  }
}

template <int DT, int LPU>
void launch(const Args &a, int cache, unsigned blocks, hipStream_t s) {
  if (cache == kNoCache) qk_norm_rope_kernel<DT, LPU, kNoCache><<<blocks, kThreads, 0, s>>>(a);
  else if (cache == kSameCache) qk_norm_rope_kernel<DT, LPU, kSameCache><<<blocks, kThreads, 0, s>>>(a);
  else qk_norm_rope_kernel<DT, LPU, kFp8Cache><<<blocks, kThreads, 0, s>>>(a);
}

template <int DT>
void launch_dt(const Args &a, int head_dim, int cache, unsigned blocks, hipStream_t s) {
  if (head_dim == 64) launch<DT, 8>(a, cache, blocks, s);
  else if (head_dim == 128) launch<DT, 16>(a, cache, blocks, s);
  else launch<DT, 32>(a, cache, blocks, s);
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_qk_norm_rope_store(
    const void *q, int64_t q_row_stride, int64_t q_head_stride, const void *k, int64_t k_row_stride,
    const void *v, int64_t v_row_stride, const int64_t *positions, const float *cos_sin_cache,
    int64_t max_position, int rotary_dim, const void *q_weight, const void *k_weight, float eps,
    float weight_offset, void *q_out, int64_t q_out_row_stride, int64_t q_out_head_stride,
    void *k_out, int64_t k_out_row_stride, void *k_cache, void *v_cache, const int32_t *slot_mapping,
    int64_t num_slots, int64_t num_tokens, int num_q_heads, int num_kv_heads, int head_dim, int dtype,
    int cache_dtype, const float *k_scale, const float *v_scale, void *stream) {
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_position < 0)
    return fail(NQ_EINVAL, "qk_norm_rope_store: bad sizes (tokens=%lld q_heads=%d kv_heads=%d dim=%d)",
                (long long)num_tokens, num_q_heads, num_kv_heads, head_dim);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(NQ_EUNSUPPORTED, "qk_norm_rope_store: head_dim %d not built (64, 128, 256)", head_dim);
  if (rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 16 != 0)
    return fail(NQ_EUNSUPPORTED, "qk_norm_rope_store: rotary_dim %d must be a multiple of 16 in [0, %d]",
                rotary_dim, head_dim);
  if (dtype != NQ_F32 && dtype != NQ_F16 && dtype != NQ_BF16)
    return fail(NQ_EUNSUPPORTED, "qk_norm_rope_store: dtype %d unsupported", dtype);
  if (num_tokens == 0) return NQ_OK;
  if (!q || !k || !positions || !q_weight || !k_weight || !q_out || (rotary_dim > 0 && !cos_sin_cache))
    return fail(NQ_EINVAL, "qk_norm_rope_store: null pointer");
  const int es = dtype == NQ_F32 ? 4 : 2;
  int cache = kNoCache;
  if (k_cache || v_cache) {
    if (!k_cache || !v_cache || !v || !slot_mapping || num_slots < 0)
      return fail(NQ_EINVAL, "qk_norm_rope_store: a cache store needs k_cache, v_cache, value and slot_mapping");
    if (cache_dtype == dtype) {
      cache = kSameCache;
    } else if (cache_dtype == NQ_FP8_E4M3) {
      if (!k_scale || !v_scale) return fail(NQ_EINVAL, "qk_norm_rope_store: fp8 cache needs k_scale/v_scale");
      cache = kFp8Cache;
    } else {
      return fail(NQ_EUNSUPPORTED, "qk_norm_rope_store: cache dtype %d with dtype %d", cache_dtype, dtype);
    }
  }
  // Every 8-element group is one (or two, fp32) 16-byte access.
  const bool al = aligned(q, 16) && aligned(k, 16) && aligned(q_out, 16) && aligned(q_weight, 16) &&
                  aligned(k_weight, 16) && (!k_out || aligned(k_out, 16)) &&
                  (!cos_sin_cache || aligned(cos_sin_cache, 16)) &&
                  (cache == kNoCache || (aligned(v, 16) && aligned(k_cache, 16) && aligned(v_cache, 16))) &&
                  (q_row_stride * es) % 16 == 0 && (q_head_stride * es) % 16 == 0 &&
                  (k_row_stride * es) % 16 == 0 && (v_row_stride * es) % 16 == 0 &&
                  (q_out_row_stride * es) % 16 == 0 && (q_out_head_stride * es) % 16 == 0 &&
                  (k_out_row_stride * es) % 16 == 0;
  if (!al) return fail(NQ_EINVAL, "qk_norm_rope_store: pointers and strides must be 16-byte aligned");
  const int64_t per_tok = static_cast<int64_t>(num_q_heads) + num_kv_heads + (cache ? num_kv_heads : 0);
  if (num_tokens > 0x7fffffffLL || per_tok > (1 << 20))
    return fail(NQ_EINVAL, "qk_norm_rope_store: too many tokens or heads for one launch");
  Args a;
  a.q = static_cast<const char *>(q);
  a.q_row = q_row_stride;
  a.q_head = q_head_stride;
  a.k = static_cast<const char *>(k);
  a.k_row = k_row_stride;
  a.v = static_cast<const char *>(v);
  a.v_row = v_row_stride;
  a.positions = positions;
  a.cos_sin = cos_sin_cache;
  a.max_position = rotary_dim > 0 ? max_position : INT64_MAX;
  a.rot = rotary_dim;
  a.q_w = static_cast<const char *>(q_weight);
  a.k_w = static_cast<const char *>(k_weight);
  a.eps = eps;
  a.w_off = weight_offset;
  a.q_out = static_cast<char *>(q_out);
  a.qo_row = q_out_row_stride;
  a.qo_head = q_out_head_stride;
  a.k_out = static_cast<char *>(k_out);
  a.ko_row = k_out_row_stride;
  a.k_cache = static_cast<char *>(k_cache);
  a.v_cache = static_cast<char *>(v_cache);
  a.slots = slot_mapping;
  a.num_slots = num_slots;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.units = static_cast<int>(per_tok);
  const unsigned blocks = static_cast<unsigned>(num_tokens);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == NQ_BF16) launch_dt<NQ_BF16>(a, head_dim, cache, blocks, s);
  else if (dtype == NQ_F16) launch_dt<NQ_F16>(a, head_dim, cache, blocks, s);
  else launch_dt<NQ_F32>(a, head_dim, cache, blocks, s);
  return check_launch("qk_norm_rope_store");
}
