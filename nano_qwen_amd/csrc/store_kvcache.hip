// Slot-mapped KV scatter (store_kvcache) for gfx950.
//
// Reference: layers/attention.py:10-40 -- one Triton program per token copies
// the token's Hkv*D key (and value) elements to cache row slot_mapping[i],
// skipping slot -1.  Here one 256-thread workgroup handles one token: the K
// row and the V row are moved as 16-byte vectors (global_load/store_dwordx4),
// so a 2 KiB bf16 row is one fully coalesced 128-lane transaction.  The fp8
// variant quantizes on the fly with per-kv-head scales (e4m3fn, RNE,
// saturating), converting 16 values per thread with v_cvt_pk_fp8_f32.
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kThreads = 256;

// Same-dtype copy.  `row_vecs` = row bytes / VEC.
template <int VEC>
__global__ __launch_bounds__(kThreads) void store_copy_kernel(
    const char *__restrict__ key, int64_t key_stride_b, const char *__restrict__ value,
    int64_t value_stride_b, char *__restrict__ k_cache, char *__restrict__ v_cache,
    const int32_t *__restrict__ slot_mapping, int64_t num_slots, int row_vecs) {
  const int64_t tok = blockIdx.x;
  const int32_t slot = slot_mapping[tok];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t row_b = static_cast<int64_t>(row_vecs) * VEC;
  const char *ksrc = key + tok * key_stride_b;
  const char *vsrc = value + tok * value_stride_b;
  char *kdst = k_cache + static_cast<int64_t>(slot) * row_b;
  char *vdst = v_cache + static_cast<int64_t>(slot) * row_b;
  for (int i = threadIdx.x; i < 2 * row_vecs; i += kThreads) {
    const bool is_v = i >= row_vecs;
    const int j = is_v ? i - row_vecs : i;
    const char *src = (is_v ? vsrc : ksrc) + static_cast<int64_t>(j) * VEC;
    char *dst = (is_v ? vdst : kdst) + static_cast<int64_t>(j) * VEC;
    if constexpr (VEC == 16) {
      store16(dst, load16(src));
    } else if constexpr (VEC == 4) {
      *reinterpret_cast<uint32_t *>(dst) = *reinterpret_cast<const uint32_t *>(src);
    } else if constexpr (VEC == 2) {
      *reinterpret_cast<uint16_t *>(dst) = *reinterpret_cast<const uint16_t *>(src);
    } else {
      *dst = *src;
    }
  }
}

// fp8 quantizing store: each thread produces 16 output bytes (16 elements,
// all of one kv head because head_dim % 16 == 0).  IN: 0 f32, 1 f16, 2 bf16.
template <int IN>
__global__ __launch_bounds__(kThreads) void store_fp8_kernel(
    const char *__restrict__ key, int64_t key_stride_b, const char *__restrict__ value,
    int64_t value_stride_b, uint8_t *__restrict__ k_cache, uint8_t *__restrict__ v_cache,
    const int32_t *__restrict__ slot_mapping, int64_t num_slots, int row_elems, int head_dim,
    const float *__restrict__ k_scale, const float *__restrict__ v_scale) {
  const int64_t tok = blockIdx.x;
  const int32_t slot = slot_mapping[tok];
  if (slot < 0 || slot >= num_slots) return;
  const int groups = row_elems / 16;
  for (int i = threadIdx.x; i < 2 * groups; i += kThreads) {
    const bool is_v = i >= groups;
    const int j = is_v ? i - groups : i;
    const int e0 = j * 16;
    const int h = e0 / head_dim;
    const float inv = 1.0f / (is_v ? v_scale[h] : k_scale[h]);
    const char *src = (is_v ? value + tok * value_stride_b : key + tok * key_stride_b);
    float x[16];
    if constexpr (IN == 0) {
      const float *s = reinterpret_cast<const float *>(src) + e0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        // Load as float vectors: this hipcc miscompiles __builtin_bit_cast
        // applied to an element of an ext_vector (every element reads as [0]).
        const f32x4 w = *reinterpret_cast<const f32x4 *>(s + 4 * c);
#pragma unroll
        for (int t = 0; t < 4; ++t) x[4 * c + t] = w[t];
      }
    } else {
      const uint16_t *s = reinterpret_cast<const uint16_t *>(src) + e0;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        u32x4 w = load16(s + 8 * c);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint16_t lo = static_cast<uint16_t>(w[t] & 0xffffu);
          const uint16_t hi = static_cast<uint16_t>(w[t] >> 16);
          if constexpr (IN == 1) {
            x[8 * c + 2 * t] = F16::to_float(lo);
            x[8 * c + 2 * t + 1] = F16::to_float(hi);
          } else {
            x[8 * c + 2 * t] = BF16::to_float(lo);
            x[8 * c + 2 * t + 1] = BF16::to_float(hi);
          }
        }
      }
    }
    u32x4 out;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      out[t] = fp8x4(x[4 * t] * inv, x[4 * t + 1] * inv, x[4 * t + 2] * inv, x[4 * t + 3] * inv);
    uint8_t *dst = (is_v ? v_cache : k_cache) + static_cast<int64_t>(slot) * row_elems + e0;
    store16(dst, out);
  }
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_store_kvcache(const void *key, int64_t key_row_stride, const void *value,
                                int64_t value_row_stride, void *k_cache, void *v_cache,
                                const int32_t *slot_mapping, int64_t num_tokens, int64_t num_slots,
                                int num_kv_heads, int head_dim, int in_dtype, int cache_dtype,
                                const float *k_scale, const float *v_scale, void *stream) {
  if (num_tokens < 0 || num_slots < 0 || num_kv_heads <= 0 || head_dim <= 0)
    return fail(NQ_EINVAL, "store_kvcache: bad sizes (tokens=%lld slots=%lld heads=%d dim=%d)",
                (long long)num_tokens, (long long)num_slots, num_kv_heads, head_dim);
  if (num_tokens == 0) return NQ_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(NQ_EINVAL, "store_kvcache: null pointer");
  if (num_tokens > 0x7fffffffLL) return fail(NQ_EINVAL, "store_kvcache: too many tokens");
  const int in_sz = elem_size(in_dtype);
  if (in_sz == 0 || in_dtype == NQ_FP8_E4M3 || elem_size(cache_dtype) == 0)
    return fail(NQ_EUNSUPPORTED, "store_kvcache: dtype in=%d cache=%d unsupported", in_dtype, cache_dtype);
  const int row_elems = num_kv_heads * head_dim;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t ks_b = key_row_stride * in_sz, vs_b = value_row_stride * in_sz;
  if (cache_dtype == in_dtype) {
    const int row_b = row_elems * in_sz;
    const bool a16 = row_b % 16 == 0 && ks_b % 16 == 0 && vs_b % 16 == 0 && aligned(key, 16) &&
                     aligned(value, 16) && aligned(k_cache, 16) && aligned(v_cache, 16);
    dim3 grid(static_cast<unsigned>(num_tokens));
    if (a16) {
      store_copy_kernel<16><<<grid, kThreads, 0, s>>>(
          (const char *)key, ks_b, (const char *)value, vs_b, (char *)k_cache, (char *)v_cache,
          slot_mapping, num_slots, row_b / 16);
    } else if (in_sz == 4) {
      store_copy_kernel<4><<<grid, kThreads, 0, s>>>(
          (const char *)key, ks_b, (const char *)value, vs_b, (char *)k_cache, (char *)v_cache,
          slot_mapping, num_slots, row_b / 4);
    } else {
      store_copy_kernel<2><<<grid, kThreads, 0, s>>>(
          (const char *)key, ks_b, (const char *)value, vs_b, (char *)k_cache, (char *)v_cache,
          slot_mapping, num_slots, row_b / 2);
    }
    return check_launch("store_kvcache");
  }
  if (cache_dtype != NQ_FP8_E4M3)
    return fail(NQ_EUNSUPPORTED, "store_kvcache: cache dtype %d needs in dtype %d", cache_dtype, in_dtype);
  if (!k_scale || !v_scale) return fail(NQ_EINVAL, "store_kvcache: fp8 cache needs k_scale/v_scale");
  if (head_dim % 16 != 0) return fail(NQ_EUNSUPPORTED, "store_kvcache: fp8 needs head_dim %% 16 == 0");
  if (ks_b % 16 || vs_b % 16 || !aligned(key, 16) || !aligned(value, 16) || !aligned(k_cache, 16) ||
      !aligned(v_cache, 16))
    return fail(NQ_EINVAL, "store_kvcache: fp8 path needs 16-byte aligned rows");
  dim3 grid(static_cast<unsigned>(num_tokens));
#define NQ_LAUNCH_FP8(IN)                                                                        \
  store_fp8_kernel<IN><<<grid, kThreads, 0, s>>>((const char *)key, ks_b, (const char *)value, \
                                                 vs_b, (uint8_t *)k_cache, (uint8_t *)v_cache,  \
                                                 slot_mapping, num_slots, row_elems, head_dim,  \
                                                 k_scale, v_scale)
  if (in_dtype == NQ_F32) NQ_LAUNCH_FP8(0);
  else if (in_dtype == NQ_F16) NQ_LAUNCH_FP8(1);
  else NQ_LAUNCH_FP8(2);
#undef NQ_LAUNCH_FP8
  return check_launch("store_kvcache(fp8)");
}
