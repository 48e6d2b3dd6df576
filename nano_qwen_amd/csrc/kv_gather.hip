// Paged fp8 K/V -> packed 16-bit K/V, dequantized (gfx950).
//
// Feeds the 16-bit prefill kernel from an fp8 cache: for each sequence s and
// key j < Lk_s (Lk_s = cu_k[s+1] - cu_k[s]), cache row
// block_tables[s][j / block_size] * block_size + j % block_size is written to
// packed row cu_k[s] + j as rnd(code * scale[h]) for every element of kv
// head h (rnd = round to the 16-bit type, nearest even; missing blocks give
// zeros).  That is exactly the "attention over the dequantized K/V" the fp8
// path is specified against.  One wave per key row, one lane per 16 fp8 bytes
// of it (16 elements of one head, since head_dim % 16 == 0): 16-byte loads
// and two 16-byte stores per lane.
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kThreads = 256;

template <class T>
__global__ __launch_bounds__(kThreads) void gather_dequant_kernel(
    const uint8_t *kc, const uint8_t *vc, const int32_t *bt, int64_t bt_stride, int max_blocks,
    int64_t num_blocks, const int32_t *cu_k, int block_size, int row_b, int head_dim, const float *ks,
    const float *vs, uint8_t *ok, uint8_t *ov, int max_seqlen_k, int64_t cap) {
  const int s = blockIdx.y;
  const int chunks = row_b / 16;  // 16-byte chunks per fp8 row
  // Rows written stay below `cap` (the output's rows) even if cu_seqlens_k
  // disagrees with it or with max_seqlen_k.
  const int64_t k0 = ld_const(cu_k + s);
  int64_t Lk = ld_const(cu_k + s + 1) - k0;
  Lk = k0 < 0 ? 0 : max<int64_t>(0, min<int64_t>(min<int64_t>(Lk, max_seqlen_k), cap - k0));
  // One wave per key row: the block-table entry is wave-uniform (a scalar
  // load); lane l moves chunks l, l + 64, ... of the row.
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave; j < Lk;
       j += static_cast<int64_t>(gridDim.x) * (kThreads / 64)) {
    const int bi = __builtin_amdgcn_readfirstlane(static_cast<int>(j / block_size));
    const int blk = bi < max_blocks ? ld_const(bt + static_cast<int64_t>(s) * bt_stride + bi) : -1;
    const bool ok_blk = blk >= 0 && blk < num_blocks;
    const int64_t row = static_cast<int64_t>(blk) * block_size + j % block_size;
    for (int c = lane; c < chunks; c += 64) {
      const int64_t src = row * row_b + c * 16;
      const int h = (c * 16) / head_dim;
      const u32x4 kw = ok_blk ? load16_stream(kc + src) : u32x4{0, 0, 0, 0};
      const u32x4 vw = ok_blk ? load16_stream(vc + src) : u32x4{0, 0, 0, 0};
      const float ksc = ks[h], vsc = vs[h];
      uint8_t *kd = ok + ((k0 + j) * row_b + c * 16) * 2;
      uint8_t *vd = ov + ((k0 + j) * row_b + c * 16) * 2;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u32x4 ko, vo;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint32_t kx = kw[2 * half + q], vx = vw[2 * half + q];
          const uint32_t kp[2] = {T::template fp8x2<false>(kx), T::template fp8x2<true>(kx)};
          const uint32_t vp[2] = {T::template fp8x2<false>(vx), T::template fp8x2<true>(vx)};
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            ko[2 * q + e] = T::pack2(T::to_float(static_cast<uint16_t>(kp[e] & 0xffffu)) * ksc,
                                     T::to_float(static_cast<uint16_t>(kp[e] >> 16)) * ksc);
            vo[2 * q + e] = T::pack2(T::to_float(static_cast<uint16_t>(vp[e] & 0xffffu)) * vsc,
                                     T::to_float(static_cast<uint16_t>(vp[e] >> 16)) * vsc);
          }
        }
        __builtin_nontemporal_store(ko, reinterpret_cast<u32x4 *>(kd) + half);
        __builtin_nontemporal_store(vo, reinterpret_cast<u32x4 *>(vd) + half);
      }
    }
  }
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_kv_gather_dequant(const void *k_cache, const void *v_cache, const int32_t *block_tables,
                                    int64_t bt_stride, int max_blocks_per_seq, int64_t num_blocks,
                                    const int32_t *cu_seqlens_k, int num_seqs, int max_seqlen_k, int block_size,
                                    int num_kv_heads, int head_dim, const float *k_scale, const float *v_scale,
                                    void *k_out, void *v_out, int64_t out_rows, int out_dtype, void *stream) {
  if (num_seqs < 0 || max_seqlen_k < 0 || out_rows < 0 || block_size <= 0 || num_kv_heads <= 0 || head_dim <= 0)
    return fail(NQ_EINVAL, "kv_gather_dequant: bad sizes");
  if (head_dim % 16) return fail(NQ_EUNSUPPORTED, "kv_gather_dequant: head_dim %% 16 != 0");
  if (out_dtype != NQ_BF16 && out_dtype != NQ_F16)
    return fail(NQ_EUNSUPPORTED, "kv_gather_dequant: out dtype %d (f16/bf16)", out_dtype);
  if (num_seqs == 0 || max_seqlen_k == 0 || out_rows == 0) return NQ_OK;
  if (!k_cache || !v_cache || !block_tables || !cu_seqlens_k || !k_scale || !v_scale || !k_out || !v_out)
    return fail(NQ_EINVAL, "kv_gather_dequant: null pointer");
  if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(k_out, 16) || !aligned(v_out, 16))
    return fail(NQ_EINVAL, "kv_gather_dequant: 16-byte alignment");
  if (num_seqs > 65535) return fail(NQ_EINVAL, "kv_gather_dequant: too many sequences");
  const int row_b = num_kv_heads * head_dim;
  const int64_t bx = (static_cast<int64_t>(max_seqlen_k) + kThreads / 64 - 1) / (kThreads / 64);  // rows / 4
  dim3 grid(static_cast<unsigned>(bx < 4096 ? bx : 4096), num_seqs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto *kc = static_cast<const uint8_t *>(k_cache);
  const auto *vc = static_cast<const uint8_t *>(v_cache);
  auto *ko = static_cast<uint8_t *>(k_out);
  auto *vo = static_cast<uint8_t *>(v_out);
  if (out_dtype == NQ_BF16)
    gather_dequant_kernel<BF16><<<grid, kThreads, 0, s>>>(kc, vc, block_tables, bt_stride, max_blocks_per_seq,
                                                          num_blocks, cu_seqlens_k, block_size, row_b, head_dim,
                                                          k_scale, v_scale, ko, vo, max_seqlen_k, out_rows);
  else
    gather_dequant_kernel<F16><<<grid, kThreads, 0, s>>>(kc, vc, block_tables, bt_stride, max_blocks_per_seq,
                                                         num_blocks, cu_seqlens_k, block_size, row_b, head_dim,
                                                         k_scale, v_scale, ko, vo, max_seqlen_k, out_rows);
  return check_launch("kv_gather_dequant");
}
