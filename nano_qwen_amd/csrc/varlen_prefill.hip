// Causal varlen prefill attention for gfx950 on bf16/f16 MFMA.
//
// Reference semantics: layers/attention.py:64-70 calls
// flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
// max_seqlen_k, softmax_scale, causal=True, block_table): sequence s owns query
// rows [cu_q[s], cu_q[s+1]) and Lk = cu_k[s+1]-cu_k[s] keys; query row i sees
// keys j <= i + (Lk - Lq) (causal mask aligned to the bottom-right corner, so
// a prefix-cache hit of P = Lk - Lq tokens is visible to every row).  With a
// block table (any prefix hit in the batch, engine/model_runner.py:275-276)
// K/V are the whole paged cache (layers/attention.py:65-66).
//
// Design (one workgroup = 4 waves = 128 query rows of one (sequence, head)):
//  * grid (Hq * num_seqs, ceil(max_seqlen_q / 128)), q tiles dispatched
//    last-row-first so the tiles with the most keys start earliest; tiles
//    past a sequence's end exit at once.
//  * K and V tiles of 64 keys are staged in LDS (fp8 caches are converted to
//    the operand type while staging); each wave keeps its 32 query rows in
//    registers as the B operand of S^T = K . Q^T (v_mfma_f32_16x16x32).
//  * The S^T accumulator layout is the B-operand layout of O^T += V^T . P^T,
//    so probabilities stay in registers; V^T operands are read transposed
//    from the row-major LDS tile.
//  * Online softmax in the log2 domain; key tiles beyond a wave's causal
//    limit are skipped, the diagonal tile is masked element-wise.
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kPWaves = 4;
constexpr int kPThreads = 64 * kPWaves;
constexpr int kBM = 128;  // query rows per workgroup (32 per wave)
constexpr int kBN = 64;   // keys per LDS tile

struct PrefillArgs {
  const uint8_t *q;
  int64_t q_rs, q_hs;  // bytes
  const uint8_t *k;
  const uint8_t *v;
  int64_t kv_rs;  // bytes per K/V row (token)
  const int32_t *cu_q;
  const int32_t *cu_k;
  const int32_t *block_tables;  // null: packed K/V
  int64_t bt_stride;
  int max_blocks;  // table width: entries past it are never read
  int64_t num_blocks;
  uint8_t *out;
  int64_t o_rs, o_hs;  // bytes
  int Hq, Hkv, G, block_size, num_seqs, n_qtiles;
  int causal;
  float scale_log2;
  const float *k_scale;
  const float *v_scale;
};

template <class T, bool FP8, int D>
struct PrefillTile {
  static constexpr int ROW = D + 8;  // LDS row stride in 16-bit elements (16-byte aligned rows)
  static constexpr int NKK = D / 32;
  static constexpr int NJ = D / 16;
  static constexpr int TILE_ELEMS = kBN * ROW;
  static constexpr int LDS_BYTES = 2 * TILE_ELEMS * 2;

  // Cache/packed row of key j of the sequence, or -1 when unavailable.
  __device__ static inline int64_t key_row(const PrefillArgs &a, int s, int k0, int j) {
    if (a.block_tables == nullptr) return static_cast<int64_t>(k0) + j;
    if (j / a.block_size >= a.max_blocks) return -1;
    const int blk = a.block_tables[s * a.bt_stride + j / a.block_size];
    if (blk < 0 || blk >= a.num_blocks) return -1;
    return static_cast<int64_t>(blk) * a.block_size + j % a.block_size;
  }

  // Stage K and V rows [kbase, kbase+64) of kv head kvh into LDS; keys at or
  // past key_end are zero.
  __device__ static inline void stage(const PrefillArgs &a, uint16_t *kt, uint16_t *vt, int s, int k0,
                                      int kvh, int kbase, int key_end) {
    if constexpr (!FP8) {
      constexpr int CH = D / 8;  // 16-byte chunks per row
      for (int c = threadIdx.x; c < kBN * CH; c += kPThreads) {
        const int r = c / CH, col = (c % CH) * 8;
        const int j = kbase + r;
        u32x4 kw{0, 0, 0, 0}, vw{0, 0, 0, 0};
        if (j < key_end) {
          const int64_t row = key_row(a, s, k0, j);
          if (row >= 0) {
            const int64_t off = row * a.kv_rs + (static_cast<int64_t>(kvh) * D + col) * 2;
            kw = load16(a.k + off);
            vw = load16(a.v + off);
          }
        }
        *reinterpret_cast<u32x4 *>(kt + r * ROW + col) = kw;
        *reinterpret_cast<u32x4 *>(vt + r * ROW + col) = vw;
      }
    } else {
      constexpr int CH = D / 16;  // 16-byte fp8 chunks per row
      for (int c = threadIdx.x; c < kBN * CH; c += kPThreads) {
        const int r = c / CH, col = (c % CH) * 16;
        const int j = kbase + r;
        u32x4 kw{0, 0, 0, 0}, vw{0, 0, 0, 0};
        if (j < key_end) {
          const int64_t row = key_row(a, s, k0, j);
          if (row >= 0) {
            const int64_t off = row * a.kv_rs + static_cast<int64_t>(kvh) * D + col;
            kw = load16(a.k + off);
            vw = load16(a.v + off);
          }
        }
        u32x4 k0w, k1w, v0w, v1w;
        k0w = u32x4{T::template fp8x2<false>(kw[0]), T::template fp8x2<true>(kw[0]),
                    T::template fp8x2<false>(kw[1]), T::template fp8x2<true>(kw[1])};
        k1w = u32x4{T::template fp8x2<false>(kw[2]), T::template fp8x2<true>(kw[2]),
                    T::template fp8x2<false>(kw[3]), T::template fp8x2<true>(kw[3])};
        v0w = u32x4{T::template fp8x2<false>(vw[0]), T::template fp8x2<true>(vw[0]),
                    T::template fp8x2<false>(vw[1]), T::template fp8x2<true>(vw[1])};
        v1w = u32x4{T::template fp8x2<false>(vw[2]), T::template fp8x2<true>(vw[2]),
                    T::template fp8x2<false>(vw[3]), T::template fp8x2<true>(vw[3])};
        *reinterpret_cast<u32x4 *>(kt + r * ROW + col) = k0w;
        *reinterpret_cast<u32x4 *>(kt + r * ROW + col + 8) = k1w;
        *reinterpret_cast<u32x4 *>(vt + r * ROW + col) = v0w;
        *reinterpret_cast<u32x4 *>(vt + r * ROW + col + 8) = v1w;
      }
    }
  }

  // K operand: lane (m, g) = key row `r0 + m`, dims 8g + 32kk + [0, 8).
  __device__ static inline u32x4 kfrag(const uint16_t *kt, int r0, int kk, int m, int g) {
    return *reinterpret_cast<const u32x4 *>(kt + (r0 + m) * ROW + 8 * g + 32 * kk);
  }

  // V^T operand of output block j over keys r0 .. r0+31:
  // lane (m, g) takes V[r0 + psi(g, i)][16j + m].
  __device__ static inline u32x4 vfrag(const uint16_t *vt, int r0, int j, int m, int g) {
    const uint16_t *c0 = vt + (r0 + 4 * g) * ROW + 16 * j + m;
    const uint16_t *c1 = c0 + 16 * ROW;
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = c0[i * ROW];
      e[4 + i] = c1[i * ROW];
    }
    return u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
  }
};

template <class T, bool FP8, int D>
__global__ __launch_bounds__(kPThreads) void varlen_prefill_kernel(const PrefillArgs a) {
  using PT = PrefillTile<T, FP8, D>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t *kt = reinterpret_cast<uint16_t *>(smem);
  uint16_t *vt = kt + PT::TILE_ELEMS;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, g = lane >> 4;
  const int h = blockIdx.x % a.Hq, s = blockIdx.x / a.Hq;
  const int qt = a.n_qtiles - 1 - static_cast<int>(blockIdx.y);
  const int q0 = a.cu_q[s], Lq = a.cu_q[s + 1] - q0;
  const int row_begin = qt * kBM;
  if (row_begin >= Lq) return;
  const int k0 = a.cu_k[s], Lk = a.cu_k[s + 1] - k0;
  const int P = Lk - Lq;
  const int kvh = h / a.G;
  const int row_last = min(row_begin + kBM, Lq) - 1;
  const int key_end = a.causal ? max(0, min(Lk, row_last + P + 1)) : Lk;
  const int n_kt = (key_end + kBN - 1) / kBN;

  const float kscale = FP8 ? a.k_scale[kvh] : 1.0f;
  const float vscale = FP8 ? a.v_scale[kvh] : 1.0f;
  const float sl2 = a.scale_log2 * kscale;

  // This wave's rows: wrow0 .. wrow0+31 (two 16-row sub-tiles).
  const int wrow0 = row_begin + 32 * wave;
  const bool wave_live = wrow0 < Lq;
  const int wrow_last = min(wrow0 + 31, Lq - 1);
  const int wave_key_end = a.causal ? min(Lk, wrow_last + P + 1) : Lk;

  u32x4 qf[2][PT::NKK];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int r = wrow0 + 16 * qs + m;
    const bool ok = r < Lq;
    const uint8_t *qp = a.q + static_cast<int64_t>(q0 + (ok ? r : 0)) * a.q_rs + static_cast<int64_t>(h) * a.q_hs;
#pragma unroll
    for (int kk = 0; kk < PT::NKK; ++kk)
      qf[qs][kk] = ok ? load16(qp + (8 * g + 32 * kk) * 2) : u32x4{0, 0, 0, 0};
  }

  float m_run[2] = {kNegInf, kNegInf}, l_run[2] = {0.f, 0.f};
  f32x4 o[2][PT::NJ];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int j = 0; j < PT::NJ; ++j) o[qs][j] = f32x4{0, 0, 0, 0};

  for (int ktile = 0; ktile < n_kt; ++ktile) {
    const int kbase = ktile * kBN;
    __syncthreads();
    PT::stage(a, kt, vt, s, k0, kvh, kbase, key_end);
    __syncthreads();
    if (!wave_live) continue;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int kb = kbase + 32 * hh;
      if (kb >= wave_key_end) break;
      f32x4 sc[2][2];
#pragma unroll
      for (int qs = 0; qs < 2; ++qs)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) sc[qs][ks] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int kk = 0; kk < PT::NKK; ++kk) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const u32x4 kf = PT::kfrag(kt, 32 * hh + 16 * ks, kk, m, g);
#pragma unroll
          for (int qs = 0; qs < 2; ++qs) sc[qs][ks] = T::mfma16x16x32(kf, qf[qs][kk], sc[qs][ks]);
        }
      }
      const bool need_mask = kb + 31 > wrow0 + P || kb + 31 >= Lk;
      u32x4 pb[2];
      float alpha[2];
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) {
        const int row = wrow0 + 16 * qs + m;
        const int lim = a.causal ? min(Lk - 1, row + P) : Lk - 1;  // last visible key
        float x[8];
        float mloc = kNegInf;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int j = kb + 16 * ks + 4 * g + rr;
            float v = sc[qs][ks][rr] * sl2;
            if (need_mask && j > lim) v = kNegInf;
            x[4 * ks + rr] = v;
            mloc = fmaxf(mloc, v);
          }
        mloc = xor_max(mloc, 16);
        mloc = xor_max(mloc, 32);
        const float m_new = fmaxf(m_run[qs], mloc);
        const float m_use = (m_new == kNegInf) ? 0.f : m_new;
        alpha[qs] = __builtin_amdgcn_exp2f(m_run[qs] - m_use);
        float psum = 0.f;
        uint32_t pw[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float p0 = __builtin_amdgcn_exp2f(x[2 * t] - m_use);
          const float p1 = __builtin_amdgcn_exp2f(x[2 * t + 1] - m_use);
          psum += p0 + p1;
          pw[t] = T::pack2(p0, p1);
        }
        l_run[qs] = l_run[qs] * alpha[qs] + psum;
        m_run[qs] = m_new;
        pb[qs] = u32x4{pw[0], pw[1], pw[2], pw[3]};
      }
#pragma unroll
      for (int j = 0; j < PT::NJ; ++j) {
        const u32x4 vf = PT::vfrag(vt, 32 * hh, j, m, g);
#pragma unroll
        for (int qs = 0; qs < 2; ++qs) {
          o[qs][j] *= alpha[qs];
          o[qs][j] = T::mfma16x16x32(vf, pb[qs], o[qs][j]);
        }
      }
    }
  }

  if (!wave_live) return;
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    float l = xor_sum(l_run[qs], 16);
    l = xor_sum(l, 32);
    const int row = wrow0 + 16 * qs + m;
    if (row >= Lq) continue;
    const float inv = l > 0.f ? vscale / l : 0.f;
    uint8_t *op = a.out + static_cast<int64_t>(q0 + row) * a.o_rs + static_cast<int64_t>(h) * a.o_hs;
#pragma unroll
    for (int j = 0; j < PT::NJ; ++j) {
      const f32x4 v = o[qs][j] * inv;
      *reinterpret_cast<u32x2 *>(op + (16 * j + 4 * g) * 2) = u32x2{T::pack2(v[0], v[1]), T::pack2(v[2], v[3])};
    }
  }
}

template <class T, bool FP8, int D>
int launch_prefill(const PrefillArgs &a, hipStream_t s) {
  using PT = PrefillTile<T, FP8, D>;
  dim3 grid(a.Hq * a.num_seqs, a.n_qtiles);
  varlen_prefill_kernel<T, FP8, D><<<grid, kPThreads, PT::LDS_BYTES, s>>>(a);
  return check_launch("varlen_prefill");
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_varlen_prefill(const void *q, int64_t q_row_stride, int64_t q_head_stride, const void *k,
                                 const void *v, int64_t kv_row_stride, const int32_t *cu_seqlens_q,
                                 const int32_t *cu_seqlens_k, int max_seqlen_q, int max_seqlen_k,
                                 const int32_t *block_tables, int64_t bt_stride, int max_blocks_per_seq,
                                 int64_t num_blocks, void *out, int64_t out_row_stride,
                                 int64_t out_head_stride, int num_seqs, int num_q_heads, int num_kv_heads,
                                 int head_dim, int block_size, float softmax_scale, int causal, int q_dtype,
                                 int kv_dtype, const float *k_scale, const float *v_scale, void *stream) {
  if (num_seqs == 0 || max_seqlen_q == 0) return NQ_OK;
  if (num_seqs < 0 || max_seqlen_q < 0 || max_seqlen_k < 0 || num_q_heads <= 0 || num_kv_heads <= 0)
    return fail(NQ_EINVAL, "varlen_prefill: bad sizes");
  if (num_q_heads % num_kv_heads != 0)
    return fail(NQ_EINVAL, "varlen_prefill: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads,
                num_kv_heads);
  if (head_dim != 128) return fail(NQ_EUNSUPPORTED, "varlen_prefill: head_dim %d (built: 128)", head_dim);
  if (q_dtype != NQ_BF16 && q_dtype != NQ_F16)
    return fail(NQ_EUNSUPPORTED, "varlen_prefill: q dtype %d (need f16/bf16)", q_dtype);
  const bool fp8 = kv_dtype == NQ_FP8_E4M3;
  if (!fp8 && kv_dtype != q_dtype)
    return fail(NQ_EUNSUPPORTED, "varlen_prefill: kv dtype %d with q dtype %d", kv_dtype, q_dtype);
  if (fp8 && (!k_scale || !v_scale)) return fail(NQ_EINVAL, "varlen_prefill: fp8 K/V needs scales");
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out) return fail(NQ_EINVAL, "varlen_prefill: null pointer");
  if (block_tables) {
    if (block_size <= 0 || block_size % kBN != 0)
      return fail(NQ_EUNSUPPORTED, "varlen_prefill: block_size %d must be a multiple of %d", block_size, kBN);
    if (max_blocks_per_seq <= 0 || bt_stride < max_blocks_per_seq)
      return fail(NQ_EINVAL, "varlen_prefill: block table width");
    if (static_cast<int64_t>(max_blocks_per_seq) * block_size < max_seqlen_k)
      return fail(NQ_EINVAL, "varlen_prefill: block table narrower than max_seqlen_k");
  }
  const int qsz = 2, ksz = fp8 ? 1 : 2;
  if ((q_row_stride * qsz) % 16 || (q_head_stride * qsz) % 16 || !aligned(q, 16) || (kv_row_stride * ksz) % 16 ||
      !aligned(k, 16) || !aligned(v, 16) || (out_row_stride * qsz) % 8 || (out_head_stride * qsz) % 8 ||
      !aligned(out, 8))
    return fail(NQ_EINVAL, "varlen_prefill: q/k/v/out alignment");
  const int n_qtiles = (max_seqlen_q + kBM - 1) / kBM;
  if (n_qtiles > 65535 || static_cast<int64_t>(num_q_heads) * num_seqs > 0x7fffffff)
    return fail(NQ_EINVAL, "varlen_prefill: grid too large");
  PrefillArgs a{};
  a.q = static_cast<const uint8_t *>(q);
  a.q_rs = q_row_stride * qsz;
  a.q_hs = q_head_stride * qsz;
  a.k = static_cast<const uint8_t *>(k);
  a.v = static_cast<const uint8_t *>(v);
  a.kv_rs = kv_row_stride * ksz;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.block_tables = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks_per_seq;
  a.num_blocks = num_blocks;
  a.out = static_cast<uint8_t *>(out);
  a.o_rs = out_row_stride * qsz;
  a.o_hs = out_head_stride * qsz;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.G = num_q_heads / num_kv_heads;
  a.block_size = block_size;
  a.num_seqs = num_seqs;
  a.n_qtiles = n_qtiles;
  a.causal = causal;
  a.scale_log2 = softmax_scale * kLog2e;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (q_dtype == NQ_BF16)
    return fp8 ? launch_prefill<BF16, true, 128>(a, st) : launch_prefill<BF16, false, 128>(a, st);
  return fp8 ? launch_prefill<F16, true, 128>(a, st) : launch_prefill<F16, false, 128>(a, st);
}
