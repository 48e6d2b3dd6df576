// Paged decode attention for gfx950: split-K flash-decoding on bf16/f16 MFMA.
//
// Reference semantics: layers/attention.py:71-74 calls
// flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
// cache_seqlens=context_lens, block_table=block_tables, causal=True): for each
// sequence b and query head h, softmax(scale * q[b,h] . K_b^T) V_b over the
// context_lens[b] cached tokens of kv head h / G, gathered through
// block_tables[b, t / block_size].
//
// Design (one workgroup = 4 waves = one (sequence, kv head, split)):
//  * GQA sharing: the G query heads of a kv head are the 16 columns of one
//    MFMA tile, so every K/V byte is read from HBM exactly once.
//  * S^T[token, head] = K . Q^T on v_mfma_f32_16x16x32 (K is the A operand,
//    loaded straight from HBM as 16-byte vectors in operand layout).  The
//    C layout (lane = head column, 4 token rows) is already the B-operand
//    layout of the PV product, so P never leaves registers.
//  * O^T[dim, head] += V^T . P^T: V needs token-contiguous operands, so each
//    wave stages its 32-token V tile through LDS (row-major) and reads it
//    back transposed.
//  * Online softmax in the log2 domain per head; the row max is reduced over
//    the 4 lane groups with two cross-lane exchanges.
//  * Split-K: split s of a sequence covers tokens [s*T, (s+1)*T); a split
//    whose sequence is shorter exits at once, so the grid (num_splits,
//    Hkv, B) depends only on host-known shapes and is graph-capture safe.
//    A one-split sequence writes `out` directly; otherwise each split writes
//    (O_s / l_s, log2-sum-exp) to the workspace and decode_reduce_kernel
//    merges them.
//  * fp8-e4m3 K/V are converted to the operand type in registers (exact);
//    k_scale is folded into the softmax scale and v_scale into the epilogue.
#include <stdlib.h>

#include <algorithm>

#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kStep = 32;  // tokens per wave step (two 16-token MFMA tiles)

struct DecodeArgs {
  const uint8_t *q;
  int64_t q_bs, q_hs;  // bytes
  const uint8_t *k_cache;
  const uint8_t *v_cache;
  const int32_t *block_tables;
  int64_t bt_stride;
  int max_tokens;  // table width * block_size: tokens past it are never read
  const int32_t *context_lens;
  uint8_t *out;
  int64_t o_bs, o_hs;  // bytes
  float *ws_o;         // [B, Hq, S, D]
  float *ws_lse;       // [B, Hq, S]
  int Hq, Hkv, G, block_size;
  int64_t num_blocks;
  int split_tokens, num_splits;
  float scale_log2;
  const float *k_scale;
  const float *v_scale;
};

// Per-head-dim constants.  16-bit K/V: lane group g holds dims 8g + 32kk + [0,8)
// of its token for MFMA kk; fp8 K/V: dims (D/4)g + 8kk + [0,8) so one lane's
// bytes are contiguous.
template <int D, bool FP8>
struct Geo {
  static constexpr int NKK = D / 32;                   // QK MFMAs per 16-token tile
  static constexpr int NJ = D / 16;                    // PV output blocks
  static constexpr int KLOADS = FP8 ? D / 64 : D / 32;  // 16-byte loads per lane per tile
  static constexpr int VROW = D + 4;                   // LDS V row stride (16-bit elems)
  static constexpr int ESZ = FP8 ? 1 : 2;
  __device__ static inline int lane_off(int g) { return FP8 ? (D / 4) * g : 8 * g; }  // elems
  __device__ static inline int load_stride() { return FP8 ? 16 : 32; }                 // elems
  __device__ static inline int dim0(int g, int kk) { return FP8 ? (D / 4) * g + 8 * kk : 8 * g + 32 * kk; }
};

template <int D, bool FP8>
struct StepRegs {
  u32x4 k[2][Geo<D, FP8>::KLOADS];
  u32x4 v[2][Geo<D, FP8>::KLOADS];
};

template <class T, bool FP8, int D>
struct DecodeWave {
  using Gm = Geo<D, FP8>;
  static constexpr int LDS_PER_WAVE_B =
      (kStep * Gm::VROW * 2 > (16 * D + 32) * 4) ? kStep * Gm::VROW * 2 : (16 * D + 32) * 4;

  // Issue the K/V loads of one 32-token step (tokens t0 .. t0+31 of the split).
  __device__ static inline void load(const DecodeArgs &a, const int32_t *bt_row, int kvh, int t0,
                                     int t_end, int m, int g, StepRegs<D, FP8> &r) {
    const int blk = bt_row[t0 / a.block_size];
    const bool ok = blk >= 0 && blk < a.num_blocks;
    const int64_t row0 = static_cast<int64_t>(blk) * a.block_size + (t0 % a.block_size);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const bool valid = ok && (t0 + 16 * i + m < t_end);
      const int64_t off =
          (((row0 + 16 * i + m) * a.Hkv + kvh) * D + Gm::lane_off(g)) * Gm::ESZ;
#pragma unroll
      for (int c = 0; c < Gm::KLOADS; ++c) {
        const int64_t o2 = off + static_cast<int64_t>(c) * Gm::load_stride() * Gm::ESZ;
        r.k[i][c] = valid ? load16_stream(a.k_cache + o2) : u32x4{0, 0, 0, 0};
        r.v[i][c] = valid ? load16_stream(a.v_cache + o2) : u32x4{0, 0, 0, 0};
      }
    }
  }

  // K operand of MFMA kk of tile i, in operand type.
  __device__ static inline u32x4 kfrag(const StepRegs<D, FP8> &r, int i, int kk) {
    if constexpr (!FP8) {
      return r.k[i][kk];
    } else {
      const u32x4 &w = r.k[i][kk / 2];
      const uint32_t w0 = w[(kk % 2) * 2], w1 = w[(kk % 2) * 2 + 1];
      return u32x4{T::template fp8x2<false>(w0), T::template fp8x2<true>(w0), T::template fp8x2<false>(w1),
                   T::template fp8x2<true>(w1)};
    }
  }

  // Write this wave's V tile (32 tokens x D, operand type) to LDS row-major.
  __device__ static inline void stage_v(uint16_t *vt, const StepRegs<D, FP8> &r, int m, int g) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint16_t *row = vt + (16 * i + m) * Gm::VROW;
#pragma unroll
      for (int c = 0; c < Gm::KLOADS; ++c) {
        if constexpr (!FP8) {
          const u32x4 &w = r.v[i][c];
          uint16_t *p = row + Gm::dim0(g, c);
          *reinterpret_cast<u32x2 *>(p) = u32x2{w[0], w[1]};
          *reinterpret_cast<u32x2 *>(p + 4) = u32x2{w[2], w[3]};
        } else {
          const u32x4 &w = r.v[i][c];
          uint16_t *p = row + Gm::lane_off(g) + 16 * c;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            *reinterpret_cast<u32x2 *>(p + 4 * t) = u32x2{T::template fp8x2<false>(w[t]), T::template fp8x2<true>(w[t])};
          }
        }
      }
    }
  }

  // V^T operand for output block j: lane (m, g) takes V[psi(g, i)][16j + m],
  // psi(g, i) = 4g + i (i < 4, tile 0) or 16 + 4g + i - 4 (tile 1).
  __device__ static inline u32x4 vfrag(const uint16_t *vt, int j, int m, int g) {
    const uint16_t *c0 = vt + (4 * g) * Gm::VROW + 16 * j + m;
    const uint16_t *c1 = c0 + 16 * Gm::VROW;
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = c0[i * Gm::VROW];
      e[4 + i] = c1[i * Gm::VROW];
    }
    return u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
  }
};

template <class T, bool FP8, int D, bool PIPE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(PIPE ? 2 : 3)))
void paged_decode_kernel(const DecodeArgs a) {
  using W = DecodeWave<T, FP8, D>;
  using Gm = Geo<D, FP8>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, g = lane >> 4;  // m: token row / head column, g: lane group
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = a.G;
  const int ctx = min(a.context_lens[b], a.max_tokens);
  const int t_begin = split * a.split_tokens;

  if (ctx <= 0) {  // padded graph row: defined zeros, no KV reads
    if (split == 0) {
      for (int it = threadIdx.x; it < G * D / 4; it += kThreads) {
        const int h = it / (D / 4), d4 = it % (D / 4);
        uint8_t *o = a.out + b * a.o_bs + (kvh * G + h) * a.o_hs + d4 * 8;
        *reinterpret_cast<u32x2 *>(o) = u32x2{0, 0};
      }
    }
    return;
  }
  if (t_begin >= ctx) return;
  const int t_end = min(t_begin + a.split_tokens, ctx);
  const bool single = ctx <= a.split_tokens;

  const float kscale = FP8 ? a.k_scale[kvh] : 1.0f;
  const float vscale = FP8 ? a.v_scale[kvh] : 1.0f;
  const float sl2 = a.scale_log2 * kscale;

  // Q^T operand: lane (m, g) = head column m, dims dim0(g, kk) + [0, 8).
  u32x4 qf[Gm::NKK];
  {
    const bool hv = m < G;
    const uint8_t *qp = a.q + b * a.q_bs + (kvh * G + (hv ? m : 0)) * a.q_hs;
#pragma unroll
    for (int kk = 0; kk < Gm::NKK; ++kk)
      qf[kk] = hv ? load16(qp + Gm::dim0(g, kk) * 2) : u32x4{0, 0, 0, 0};
  }

  const int32_t *bt_row = a.block_tables + b * a.bt_stride;
  uint16_t *vt = reinterpret_cast<uint16_t *>(smem + wave * W::LDS_PER_WAVE_B);

  float m_run = kNegInf, l_run = 0.f;
  f32x4 o[Gm::NJ];
#pragma unroll
  for (int j = 0; j < Gm::NJ; ++j) o[j] = f32x4{0, 0, 0, 0};

  auto compute = [&](int t0, const StepRegs<D, FP8> &r) {
    wave_lds_sync();  // previous step's V^T reads are done before overwriting
    W::stage_v(vt, r, m, g);
    f32x4 s[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      s[i] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int kk = 0; kk < Gm::NKK; ++kk) s[i] = T::mfma16x16x32(W::kfrag(r, i, kk), qf[kk], s[i]);
    }
    float x[8];
    float mloc = kNegInf;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const bool valid = t0 + 16 * i + 4 * g + rr < t_end;
        const float v = valid ? s[i][rr] * sl2 : kNegInf;
        x[4 * i + rr] = v;
        mloc = fmaxf(mloc, v);
      }
    mloc = xor_max(mloc, 16);
    mloc = xor_max(mloc, 32);
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
    uint32_t pw[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float p0 = __builtin_amdgcn_exp2f(x[2 * t] - m_use);
      const float p1 = __builtin_amdgcn_exp2f(x[2 * t + 1] - m_use);
      psum += p0 + p1;
      pw[t] = T::pack2(p0, p1);
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    const u32x4 pb{pw[0], pw[1], pw[2], pw[3]};
    wave_lds_sync();  // V tile visible to every lane of the wave
#pragma unroll
    for (int j = 0; j < Gm::NJ; ++j) {
      o[j] *= alpha;
      o[j] = T::mfma16x16x32(W::vfrag(vt, j, m, g), pb, o[j]);
    }
  };

  // Token loop: waves take interleaved 32-token steps.  With PIPE, step
  // n+1's loads are in flight while step n computes (two register sets,
  // fewer waves); without, latency is hidden by more resident waves.
  const int stride = kWaves * kStep;
  int t0 = t_begin + wave * kStep;
  if constexpr (PIPE) {
    StepRegs<D, FP8> ra, rb;
    if (t0 < t_end) W::load(a, bt_row, kvh, t0, t_end, m, g, ra);
    while (t0 < t_end) {
      int t1 = t0 + stride;
      if (t1 < t_end) W::load(a, bt_row, kvh, t1, t_end, m, g, rb);
      compute(t0, ra);
      t0 = t1;
      if (t0 >= t_end) break;
      t1 = t0 + stride;
      if (t1 < t_end) W::load(a, bt_row, kvh, t1, t_end, m, g, ra);
      compute(t0, rb);
      t0 = t1;
    }
  } else {
    for (; t0 < t_end; t0 += stride) {
      StepRegs<D, FP8> r;
      W::load(a, bt_row, kvh, t0, t_end, m, g, r);
      compute(t0, r);
    }
  }

  // ---- merge the 4 waves of the workgroup through LDS
  l_run = xor_sum(l_run, 16);
  l_run = xor_sum(l_run, 32);
  __syncthreads();  // every wave is done with its V tile (the merge buffers alias it)
  float *cb = reinterpret_cast<float *>(smem + wave * W::LDS_PER_WAVE_B);
#pragma unroll
  for (int j = 0; j < Gm::NJ; ++j) *reinterpret_cast<f32x4 *>(cb + m * D + 16 * j + 4 * g) = o[j];
  if (g == 0) {
    cb[16 * D + m] = m_run;
    cb[16 * D + 16 + m] = l_run;
  }
  __syncthreads();
  for (int it = threadIdx.x; it < G * D / 4; it += kThreads) {
    const int h = it / (D / 4), d4 = it % (D / 4);
    float mw[kWaves], M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mw[w] = reinterpret_cast<const float *>(smem + w * W::LDS_PER_WAVE_B)[16 * D + h];
      M = fmaxf(M, mw[w]);
    }
    float L = 0.f;
    f32x4 acc{0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float *cw = reinterpret_cast<const float *>(smem + w * W::LDS_PER_WAVE_B);
      const float e = (mw[w] == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
      L += cw[16 * D + 16 + h] * e;
      acc += *reinterpret_cast<const f32x4 *>(cw + h * D + 4 * d4) * e;
    }
    const float inv = (L > 0.f) ? vscale / L : 0.f;
    acc *= inv;
    const int head = kvh * G + h;
    if (single) {
      uint8_t *op = a.out + b * a.o_bs + head * a.o_hs + d4 * 8;
      *reinterpret_cast<u32x2 *>(op) = u32x2{T::pack2(acc[0], acc[1]), T::pack2(acc[2], acc[3])};
    } else {
      const int64_t idx = (static_cast<int64_t>(b) * a.Hq + head) * a.num_splits + split;
      *reinterpret_cast<f32x4 *>(a.ws_o + idx * D + 4 * d4) = acc;
      if (d4 == 0) a.ws_lse[idx] = (L > 0.f) ? M + __log2f(L) : kNegInf;
    }
  }
}

int env_int(const char *name, int dflt) {
  const char *v = getenv(name);
  if (!v || !*v) return dflt;
  return atoi(v);
}

// Merge the per-split partials of every (sequence, head) with >1 split.
template <class T, int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(const DecodeArgs a, int batch) {
  constexpr int kPer = D / 4;  // threads per (b, head)
  const int pair = blockIdx.x * (256 / kPer) + threadIdx.x / kPer;
  const int d4 = threadIdx.x % kPer;
  if (pair >= batch * a.Hq) return;
  const int b = pair / a.Hq, head = pair % a.Hq;
  const int ctx = min(a.context_lens[b], a.max_tokens);
  if (ctx <= a.split_tokens) return;  // single split or empty: written by the main kernel
  const int nact = min((ctx + a.split_tokens - 1) / a.split_tokens, a.num_splits);
  const int64_t base = static_cast<int64_t>(pair) * a.num_splits;
  float M = kNegInf;
  for (int s = 0; s < nact; ++s) M = fmaxf(M, a.ws_lse[base + s]);
  float W = 0.f;
  f32x4 acc{0, 0, 0, 0};
  if (M != kNegInf) {
    for (int s = 0; s < nact; ++s) {
      const float l = a.ws_lse[base + s];
      const float w = (l == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(l - M);
      W += w;
      acc += *reinterpret_cast<const f32x4 *>(a.ws_o + (base + s) * D + 4 * d4) * w;
    }
  }
  const float inv = W > 0.f ? 1.0f / W : 0.f;
  acc *= inv;
  uint8_t *op = a.out + b * a.o_bs + head * a.o_hs + d4 * 8;
  *reinterpret_cast<u32x2 *>(op) = u32x2{T::pack2(acc[0], acc[1]), T::pack2(acc[2], acc[3])};
}

template <class T, bool FP8, int D>
int launch_decode(const DecodeArgs &a, int batch, hipStream_t s) {
  using W = DecodeWave<T, FP8, D>;
  const size_t lds = static_cast<size_t>(kWaves) * W::LDS_PER_WAVE_B;
  dim3 grid(a.num_splits, a.Hkv, batch);
  static const bool pipe = env_int("NQ_DECODE_PIPE", 1) != 0;
  if (pipe)
    paged_decode_kernel<T, FP8, D, true><<<grid, kThreads, lds, s>>>(a);
  else
    paged_decode_kernel<T, FP8, D, false><<<grid, kThreads, lds, s>>>(a);
  int rc = check_launch("paged_decode");
  if (rc != NQ_OK || a.num_splits <= 1) return rc;
  constexpr int per_block = 256 / (D / 4);
  dim3 rgrid((batch * a.Hq + per_block - 1) / per_block);
  decode_reduce_kernel<T, D><<<rgrid, 256, 0, s>>>(a, batch);
  return check_launch("paged_decode(reduce)");
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_decode_plan(int batch, int num_q_heads, int num_kv_heads, int max_blocks_per_seq,
                              int block_size, int kv_dtype, int *num_splits, int *split_tokens) {
  if (!num_splits || !split_tokens || batch <= 0 || num_kv_heads <= 0 || max_blocks_per_seq <= 0 ||
      block_size <= 0)
    return fail(NQ_EINVAL, "decode_plan: bad arguments");
  (void)num_q_heads;
  (void)kv_dtype;
  const int64_t max_tokens = static_cast<int64_t>(max_blocks_per_seq) * block_size;
  int64_t split = env_int("NQ_DECODE_SPLIT_TOKENS", 512);
  split = (split + 127) / 128 * 128;
  if (split < 128) split = 128;
  if (max_tokens <= split) {
    *num_splits = 1;
    *split_tokens = static_cast<int>((max_tokens + 127) / 128 * 128);
    return NQ_OK;
  }
  *num_splits = static_cast<int>((max_tokens + split - 1) / split);
  *split_tokens = static_cast<int>(split);
  return NQ_OK;
}

extern "C" int64_t nq_decode_workspace_bytes(int batch, int num_q_heads, int head_dim, int num_splits) {
  if (num_splits <= 1) return 0;
  const int64_t n = static_cast<int64_t>(batch) * num_q_heads * num_splits;
  int64_t bytes = n * head_dim * 4;
  bytes = (bytes + 255) / 256 * 256;
  return bytes + (n * 4 + 255) / 256 * 256;
}

extern "C" int nq_paged_decode(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                               const void *k_cache, const void *v_cache, const int32_t *block_tables,
                               int64_t bt_stride, int max_blocks_per_seq, const int32_t *context_lens,
                               void *out, int64_t out_batch_stride, int64_t out_head_stride, int batch,
                               int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                               int64_t num_blocks, float softmax_scale, int num_splits, int split_tokens,
                               void *workspace, int64_t workspace_bytes, int q_dtype, int kv_dtype,
                               const float *k_scale, const float *v_scale, void *stream) {
  if (batch == 0) return NQ_OK;
  if (batch < 0 || batch > 65535 || num_q_heads <= 0 || num_kv_heads <= 0 || num_kv_heads > 65535)
    return fail(NQ_EINVAL, "paged_decode: bad batch/head counts");
  if (num_q_heads % num_kv_heads != 0)
    return fail(NQ_EINVAL, "paged_decode: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads,
                num_kv_heads);
  const int G = num_q_heads / num_kv_heads;
  if (G > 16) return fail(NQ_EUNSUPPORTED, "paged_decode: GQA group %d > 16", G);
  if (head_dim != 128) return fail(NQ_EUNSUPPORTED, "paged_decode: head_dim %d (built: 128)", head_dim);
  if (block_size <= 0 || block_size % 32 != 0)
    return fail(NQ_EUNSUPPORTED, "paged_decode: block_size %d must be a multiple of 32", block_size);
  if (q_dtype != NQ_BF16 && q_dtype != NQ_F16)
    return fail(NQ_EUNSUPPORTED, "paged_decode: q dtype %d (need f16/bf16)", q_dtype);
  const bool fp8 = kv_dtype == NQ_FP8_E4M3;
  if (!fp8 && kv_dtype != q_dtype)
    return fail(NQ_EUNSUPPORTED, "paged_decode: kv dtype %d with q dtype %d", kv_dtype, q_dtype);
  if (fp8 && (!k_scale || !v_scale)) return fail(NQ_EINVAL, "paged_decode: fp8 cache needs scales");
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out)
    return fail(NQ_EINVAL, "paged_decode: null pointer");
  if (max_blocks_per_seq <= 0 || bt_stride < max_blocks_per_seq)
    return fail(NQ_EINVAL, "paged_decode: block table width");
  if (num_splits <= 0 || split_tokens <= 0 || split_tokens % 128 != 0)
    return fail(NQ_EINVAL, "paged_decode: bad split plan (%d x %d)", num_splits, split_tokens);
  if (static_cast<int64_t>(num_splits) * split_tokens < static_cast<int64_t>(max_blocks_per_seq) * block_size)
    return fail(NQ_EINVAL, "paged_decode: split plan covers %lld < %lld tokens",
                (long long)num_splits * split_tokens, (long long)max_blocks_per_seq * block_size);
  if ((q_head_stride * 2) % 16 || (q_batch_stride * 2) % 16 || !aligned(q, 16) || (out_head_stride * 2) % 8 ||
      (out_batch_stride * 2) % 8 || !aligned(out, 8) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return fail(NQ_EINVAL, "paged_decode: q/out/cache alignment");
  DecodeArgs a{};
  a.q = static_cast<const uint8_t *>(q);
  a.q_bs = q_batch_stride * 2;
  a.q_hs = q_head_stride * 2;
  a.k_cache = static_cast<const uint8_t *>(k_cache);
  a.v_cache = static_cast<const uint8_t *>(v_cache);
  a.block_tables = block_tables;
  a.bt_stride = bt_stride;
  a.max_tokens = static_cast<int>(std::min<int64_t>(static_cast<int64_t>(max_blocks_per_seq) * block_size, 0x7fffffff));
  a.context_lens = context_lens;
  a.out = static_cast<uint8_t *>(out);
  a.o_bs = out_batch_stride * 2;
  a.o_hs = out_head_stride * 2;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.G = G;
  a.block_size = block_size;
  a.num_blocks = num_blocks;
  a.split_tokens = split_tokens;
  a.num_splits = num_splits;
  a.scale_log2 = softmax_scale * kLog2e;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  if (num_splits > 1) {
    const int64_t need = nq_decode_workspace_bytes(batch, num_q_heads, head_dim, num_splits);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
      return fail(NQ_EINVAL, "paged_decode: workspace %lld bytes < %lld needed (or unaligned)",
                  (long long)workspace_bytes, (long long)need);
    const int64_t n = static_cast<int64_t>(batch) * num_q_heads * num_splits;
    a.ws_o = static_cast<float *>(workspace);
    a.ws_lse = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + (n * head_dim * 4 + 255) / 256 * 256);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (q_dtype == NQ_BF16)
    return fp8 ? launch_decode<BF16, true, 128>(a, batch, s) : launch_decode<BF16, false, 128>(a, batch, s);
  return fp8 ? launch_decode<F16, true, 128>(a, batch, s) : launch_decode<F16, false, 128>(a, batch, s);
}
