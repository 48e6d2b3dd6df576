// Paged decode attention for gfx950: split-K flash-decoding on bf16/f16 MFMA.
//
// Reference semantics: layers/attention.py:71-74 calls
// flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
// cache_seqlens=context_lens, block_table=block_tables, causal=True): for each
// sequence b and query head h, softmax(scale * q[b,h] . K_b^T) V_b over the
// context_lens[b] cached tokens of kv head h / G, gathered through
// block_tables[b, t / block_size].
//
// Design (one workgroup = up to 8 waves = the kv heads of one (sequence, split)):
//  * GQA sharing: the G query heads of a kv head are the 16 columns of one
//    MFMA tile, so every K/V byte is read from HBM exactly once.
//  * K/V are streamed in full 128-byte lines per load instruction (the
//    access pattern that sustains HBM bandwidth) and each wave rearranges its
//    32-token tile through a swizzled LDS tile into MFMA operands.
//  * S^T[token, head] = K . Q^T on v_mfma_f32_16x16x32 (K is the A operand).
//    The C layout (lane = head column, 4 token rows) is already the B-operand
//    layout of the PV product, so P never leaves registers.
//  * O^T[dim, head] += V^T . P^T: the token-contiguous V^T operands come from
//    the row-major tile through ds_read_b64_tr_b16 (gfx950 transposing read).
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
#include <mutex>

#include "nq_device.hpp"

namespace nq {
namespace {

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
  const uint8_t *gate;  // null, or the output gate [B, Hq, D] (same type as out)
  int64_t g_bs, g_hs;   // bytes
  float *ws_o;         // split-K [B, Hq, S, D]; stream-K [W, 2, Hq, D]
  float *ws_lse;       // split-K [B, Hq, S]; stream-K [W, 2, Hq]
  int2 *sk_bnd;        // stream-K: [W] range starts (sequence, token)
  uint8_t *ws_raw;     // the caller's workspace and its size
  int64_t ws_bytes;
  int Hq, Hkv, G, block_size;
  int64_t num_blocks;
  int split_tokens, num_splits;
  float scale_log2;
  const float *k_scale;
  const float *v_scale;
  // Fused store of the new token (nq_paged_decode_store); k_new == null: none.
  const uint8_t *k_new;
  const uint8_t *v_new;
  int64_t kn_rs, vn_rs;         // bytes per row (token) of k_new / v_new
  const int32_t *slot_mapping;  // [batch]
  int new_dtype;                // element type of k_new / v_new
};

// Per-head-dim geometry.  K/V are streamed from HBM in "full-line" layout:
// one 16-byte load instruction covers whole 128-byte cache lines of a few
// tokens (a 16-bit token row of one kv head is 2*D bytes = D/8 chunks of 16 B;
// an fp8 row is D/16 chunks).  Measured on MI355X this reaches ~6.2-6.6 TB/s
// where the MFMA-operand layout (16 tokens x 64 B per instruction) stalls near
// 4-5.6 TB/s.  Each wave then rearranges the 32-token tile through its own
// LDS tile into MFMA operands.
template <int D, bool FP8>
struct Geo {
  static constexpr int NKK = D / 32;           // QK MFMAs per 16-token tile
  static constexpr int NJ = D / 16;            // PV output blocks
  static constexpr int ROWB = D * 2;           // LDS tile row: one token, 16-bit elements
  static constexpr int CHUNKS = ROWB / 16;     // 16-byte chunks per LDS row
  static constexpr int SRC_ROWB = FP8 ? D : D * 2;       // bytes of one token's head piece in HBM
  static constexpr int SRC_CHUNKS = SRC_ROWB / 16;
  static constexpr int TOK_PER_LOAD = 64 / SRC_CHUNKS;   // tokens covered by one load instruction
  static constexpr int RAW = kStep / TOK_PER_LOAD;       // load instructions per 32-token step
  static constexpr int TILE_B = kStep * ROWB;            // LDS bytes per wave
  // The swizzle below permutes chunks within aligned groups of 16; rows are a
  // multiple of 256 bytes apart, so a group's 16 chunks hit 16 distinct bank
  // quads for D = 128 and D = 256 alike.
  static_assert(CHUNKS % 16 == 0, "rows of whole 16-chunk groups");
};

// XOR swizzle of 16-byte chunks within an LDS row (row index mod 16).  It is
// a bijection, so a row written by 16 lanes stays conflict-free, and it makes
// both operand reads conflict-free: 16 rows x one logical chunk (K fragments,
// ds_read_b128) and 4 rows x 2 adjacent chunks (V^T fragments, ds_read_b64_tr_b16).
__device__ inline int swz(int row) { return ((row & 3) << 1) | ((row >> 2) & 1) | (row & 8); }

template <class T, bool FP8, int D>
struct DecodeWave {
  using Gm = Geo<D, FP8>;
  // The wave's 32-token tile, then the new token's K and V rows (16-bit,
  // unswizzled) for the fused store.
  static constexpr int LDS_PER_WAVE_B = Gm::TILE_B + 2 * Gm::ROWB;

  // 8 elements of the new token's row: row chunk c (elements 8c .. 8c+7) of
  // kv head kvh in `src` (a k_new / v_new row of type a.new_dtype), as the
  // cache stores it -- the same bits for a 16-bit cache; for an fp8 cache
  // the e4m3fn codes of x * (1 / scale) (saturating, RNE, as
  // nq_store_kvcache), returned widened to 16 bits (exact) in `wide` and as
  // codes in `codes` (two words).
  __device__ static inline void new_chunk(const DecodeArgs &a, const uint8_t *src, int kvh, int c, float scale,
                                          u32x4 &wide, u32x2 &codes) {
    if constexpr (!FP8) {
      wide = load16(src + (static_cast<int64_t>(kvh) * D + 8 * c) * 2);
      codes = u32x2{0, 0};
    } else {
      float x[8];
      if (a.new_dtype == NQ_F32) {
        const float *f = reinterpret_cast<const float *>(src) + kvh * D + 8 * c;
        // float vectors: this hipcc miscompiles __builtin_bit_cast of an
        // ext_vector element (every element reads as [0])
        const f32x4 w0 = *reinterpret_cast<const f32x4 *>(f), w1 = *reinterpret_cast<const f32x4 *>(f + 4);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          x[t] = w0[t];
          x[4 + t] = w1[t];
        }
      } else {
        const u32x4 w = load16(src + (static_cast<int64_t>(kvh) * D + 8 * c) * 2);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint16_t lo = static_cast<uint16_t>(w[t] & 0xffffu), hi = static_cast<uint16_t>(w[t] >> 16);
          x[2 * t] = a.new_dtype == NQ_F16 ? F16::to_float(lo) : BF16::to_float(lo);
          x[2 * t + 1] = a.new_dtype == NQ_F16 ? F16::to_float(hi) : BF16::to_float(hi);
        }
      }
      const float inv = 1.0f / scale;
      codes = u32x2{fp8x4(x[0] * inv, x[1] * inv, x[2] * inv, x[3] * inv),
                    fp8x4(x[4] * inv, x[5] * inv, x[6] * inv, x[7] * inv)};
      wide = u32x4{T::template fp8x2<false>(codes[0]), T::template fp8x2<true>(codes[0]),
                   T::template fp8x2<false>(codes[1]), T::template fp8x2<true>(codes[1])};
    }
  }

  // Fused store: the new token of sequence b, kv head kvh, to cache row
  // slot_mapping[b] when that slot lies in the pool (nq_store_kvcache's
  // rule).  Lanes 0 .. 2 * D / 8 - 1: chunk lane % (D / 8) of K (first half)
  // or V (second half).
  __device__ static inline void store_new(const DecodeArgs &a, int b, int kvh, int lane) {
    const int32_t slot = a.slot_mapping[b];
    if (slot < 0 || slot >= a.num_blocks * a.block_size) return;
    constexpr int NC = D / 8;  // 8-element chunks per row
    if (lane >= 2 * NC) return;
    const bool is_v = lane >= NC;
    const int c = is_v ? lane - NC : lane;
    const uint8_t *src = (is_v ? a.v_new : a.k_new) + b * (is_v ? a.vn_rs : a.kn_rs);
    u32x4 wide;
    u32x2 codes;
    new_chunk(a, src, kvh, c, FP8 ? (is_v ? a.v_scale : a.k_scale)[kvh] : 1.0f, wide, codes);
    const int64_t elem = (static_cast<int64_t>(slot) * a.Hkv + kvh) * D + 8 * c;
    uint8_t *dst = is_v ? const_cast<uint8_t *>(a.v_cache) : const_cast<uint8_t *>(a.k_cache);
    if constexpr (FP8)
      *reinterpret_cast<u32x2 *>(dst + elem) = codes;
    else
      store16(dst + elem * 2, wide);
  }

  // The new token's K and V rows into the wave's row buffer `nbuf` (K at 0,
  // V at ROWB), in the tile's 16-bit form.
  __device__ static inline void stage_new(const DecodeArgs &a, uint8_t *nbuf, int b, int kvh, int lane) {
    constexpr int NC = D / 8;
    if (lane >= 2 * NC) return;
    const bool is_v = lane >= NC;
    const int c = is_v ? lane - NC : lane;
    const uint8_t *src = (is_v ? a.v_new : a.k_new) + b * (is_v ? a.vn_rs : a.kn_rs);
    u32x4 wide;
    u32x2 codes;
    new_chunk(a, src, kvh, c, FP8 ? (is_v ? a.v_scale : a.k_scale)[kvh] : 1.0f, wide, codes);
    *reinterpret_cast<u32x4 *>(nbuf + (is_v ? Gm::ROWB : 0) + 16 * c) = wide;
  }

  // Overwrite row `row` of a staged tile with a buffered row (same swizzle
  // as stage): lanes 0 .. CHUNKS - 1, one 16-byte chunk each.  LDS
  // operations of one wave complete in order, so this write follows the
  // stage's.
  __device__ static inline void patch_row(uint8_t *tile, const uint8_t *row_buf, int row, int lane) {
    if (lane < Gm::CHUNKS) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(row_buf + 16 * lane);
      *reinterpret_cast<u32x4 *>(tile + row * Gm::ROWB + ((lane ^ swz(row)) << 4)) = v;
    }
  }

  // Cache row of token t0 of a step (t0 % 32 == 0, so the step stays inside
  // one block), or -1 if the table entry is not a valid block.  The split's
  // table entries were loaded once into `bt_lane` (lane i holds entry
  // first_blk + i), so no memory access -- and no wait on the vector-memory
  // counter, which would also wait for the K/V prefetch -- happens here.
  __device__ static inline int64_t step_row(const DecodeArgs &a, int bt_lane, int first_blk, int t0) {
    const int blk = __builtin_amdgcn_readlane(bt_lane, t0 / a.block_size - first_blk);
    if (blk < 0 || blk >= a.num_blocks) return -1;
    return static_cast<int64_t>(blk) * a.block_size + (t0 % a.block_size);
  }

  // Lane's byte offset, within a step's rows, of its chunk for load c = 0
  // (load c adds c * TOK_PER_LOAD rows).
  __device__ static inline int lane_voff(const DecodeArgs &a, int kvh, int lane) {
    const int tl = lane / Gm::SRC_CHUNKS, ch = lane % Gm::SRC_CHUNKS;
    return (tl * a.Hkv + kvh) * Gm::SRC_ROWB + ch * 16;
  }

  // Issue the loads of one 32-token step of K (or V): load c, lane l ->
  // token c*TOK_PER_LOAD + l/SRC_CHUNKS, chunk l%SRC_CHUNKS of kv head kvh.
  // One scalar buffer descriptor spans exactly the step's valid tokens, so
  // tokens past t_end (or a missing block) read as zeros with no branches.
  __device__ static inline void load(const uint8_t *base, const DecodeArgs &a, int64_t row0, int t0, int t_end,
                                     int voff0, u32x4 (&r)[Gm::RAW]) {
    const int row_b = a.Hkv * Gm::SRC_ROWB;
    const int nvalid = row0 >= 0 ? max(0, min(kStep, t_end - t0)) : 0;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + (row0 >= 0 ? row0 : 0) * row_b,
                                                static_cast<uint32_t>(nvalid * row_b));
#pragma unroll
    for (int c = 0; c < Gm::RAW; ++c) r[c] = buffer_load16_nt(rs, voff0 + c * Gm::TOK_PER_LOAD * row_b);
  }

  // Write one raw step into the wave's LDS tile (row-major tokens x D, 16-bit,
  // swizzled chunks); fp8 is converted to the operand type on the way.
  __device__ static inline void stage(uint8_t *tile, const u32x4 (&r)[Gm::RAW], int lane) {
    const int tl = lane / Gm::SRC_CHUNKS, ch = lane % Gm::SRC_CHUNKS;
#pragma unroll
    for (int c = 0; c < Gm::RAW; ++c) {
      const int row = c * Gm::TOK_PER_LOAD + tl;
      uint8_t *rp = tile + row * Gm::ROWB;
      if constexpr (!FP8) {
        *reinterpret_cast<u32x4 *>(rp + ((ch ^ swz(row)) << 4)) = r[c];
      } else {
        // A lane's 16 codes widen to logical chunks 2ch (dims 16ch..+7) and
        // 2ch + 1.  The first store takes chunk 2ch + f and the second the
        // other, with f chosen so that every 16 lanes of a store hit 16
        // distinct bank quads: at head_dim 128 those lanes are rows 2i, 2i + 1
        // (8 lanes each), whose swizzles agree in bits 0 and 3, so the two
        // rows take complementary chunk sets {c : c0 ^ c3 = f-parity}; at 256
        // they are one row, whose two 256-byte halves share banks.  (All
        // lanes storing 2ch first would put both rows on the same 8 quads.)
        const int f = D == 128 ? (((lane >> 3) ^ (lane >> 2)) & 1) : ((lane >> 3) & 1);
        const u32x4 w = f ? u32x4{r[c][2], r[c][3], r[c][0], r[c][1]} : r[c];
        const u32x4 first{T::template fp8x2<false>(w[0]), T::template fp8x2<true>(w[0]),
                          T::template fp8x2<false>(w[1]), T::template fp8x2<true>(w[1])};
        const u32x4 second{T::template fp8x2<false>(w[2]), T::template fp8x2<true>(w[2]),
                           T::template fp8x2<false>(w[3]), T::template fp8x2<true>(w[3])};
        *reinterpret_cast<u32x4 *>(rp + (((2 * ch + f) ^ swz(row)) << 4)) = first;
        *reinterpret_cast<u32x4 *>(rp + (((2 * ch + 1 - f) ^ swz(row)) << 4)) = second;
      }
    }
  }

  // K operand of MFMA kk of tile i: lane (m, g) = token 16i + m, dims
  // 8(g + 4kk) .. +8 (logical chunk g + 4kk).
  __device__ static inline u32x4 kfrag(const uint8_t *tile, int i, int kk, int m, int g) {
    const int row = 16 * i + m;
    return *reinterpret_cast<const u32x4 *>(tile + row * Gm::ROWB + (((g + 4 * kk) ^ swz(row)) << 4));
  }

  // V^T operand for output block j: lane (m, g) takes V[psi(g, i)][16j + m],
  // psi(g, i) = 4g + i (i < 4) or 16 + 4g + i - 4.  Two transposing reads:
  // lane 16g + 4k + q addresses row psi(g, k) (resp. psi(g, 4 + k)) at
  // elements 16j + 4q .. +3.
  __device__ static inline u32x4 vfrag(const uint8_t *tile, int j, int lane) {
    const int g = lane >> 4, k = (lane >> 2) & 3, q = lane & 3;
    const int r0 = 4 * g + k, r1 = r0 + 16;
    const int lc = 2 * j + (q >> 1), sub = (q & 1) * 8;
    const u32x2 lo = lds_read_tr16(reinterpret_cast<const uint16_t *>(
        tile + r0 * Gm::ROWB + ((lc ^ swz(r0)) << 4) + sub));
    const u32x2 hi = lds_read_tr16(reinterpret_cast<const uint16_t *>(
        tile + r1 * Gm::ROWB + ((lc ^ swz(r1)) << 4) + sub));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  }
};

// The work of one wave on one piece of a sequence: kv head kvh of sequence
// b over tokens [t_begin, t_end) (t_begin % 32 == 0, at most 63 blocks).  A
// piece that is the whole context (single) writes `out`; any other writes
// its heads' normalised partial O and log2-sum-exp to workspace row
// ws_row + head * ws_head_stride, for a merge pass.
template <class T, bool FP8, int D, int DEPTH>
__device__ __forceinline__ void decode_piece(const DecodeArgs &a, uint8_t *tile, int b, int kvh, int t_begin,
                                             int t_end, bool single, int64_t ws_row, int64_t ws_head_stride) {
  using W = DecodeWave<T, FP8, D>;
  using Gm = Geo<D, FP8>;
  const int lane = threadIdx.x & 63;
  const int m = lane & 15, g = lane >> 4;  // m: token row / head column, g: lane group
  const int G = a.G;
  const float kscale = FP8 ? a.k_scale[kvh] : 1.0f;
  const float vscale = FP8 ? a.v_scale[kvh] : 1.0f;
  const float sl2 = a.scale_log2 * kscale;
  const int32_t *bt_row = a.block_tables + b * a.bt_stride;

  // Q^T operand: lane (m, g) = head column m, dims 8(g + 4kk) .. +8.
  u32x4 qf[Gm::NKK];
  {
    const bool hv = m < G;
    const uint8_t *qp = a.q + b * a.q_bs + (kvh * G + (hv ? m : 0)) * a.q_hs;
#pragma unroll
    for (int kk = 0; kk < Gm::NKK; ++kk) qf[kk] = hv ? load16(qp + (8 * g + 32 * kk) * 2) : u32x4{0, 0, 0, 0};
  }

  // Raw K and V of DEPTH steps live in registers (one set per step in
  // flight); a set is refilled with the step DEPTH ahead as soon as it has
  // been copied to LDS, so those loads are in flight while the wave works
  // through the steps before it.  The refill is issued unconditionally (past
  // the split it is an empty descriptor: zeros, no memory traffic) so the
  // vector-memory wait counts are identical on every iteration and never
  // drain the prefetch.
  const int first_blk = t_begin / a.block_size;
  const int n_blk = (t_end - 1) / a.block_size - first_blk + 1;  // <= 64 (host plan)
  const int bt_lane = lane < n_blk ? bt_row[first_blk + lane] : -1;
  const int voff0 = W::lane_voff(a, kvh, lane);

  // Fused store: the piece that ends at the sequence's last token, when that
  // token's cache row is the slot the new token is stored to, takes the new
  // K/V rows from the inputs (as the store writes them) instead of from the
  // cache, so it needs no ordering against the store.  sub_t0: the step that
  // holds the token (-1: none).
  uint8_t *const nbuf = tile + Gm::TILE_B;
  int sub_t0 = -1, sub_row = 0;
  if (a.k_new && t_end == a.context_lens[b]) {
    const int t = t_end - 1;
    const int blk = __builtin_amdgcn_readlane(bt_lane, t / a.block_size - first_blk);
    if (blk >= 0 && blk < a.num_blocks &&
        a.slot_mapping[b] == static_cast<int64_t>(blk) * a.block_size + t % a.block_size) {
      W::stage_new(a, nbuf, b, kvh, lane);
      sub_t0 = __builtin_amdgcn_readfirstlane(t_begin + (t - t_begin) / kStep * kStep);
      sub_row = __builtin_amdgcn_readfirstlane(t - sub_t0);
    }
  }
  u32x4 kraw[DEPTH][Gm::RAW], vraw[DEPTH][Gm::RAW];
  int64_t rows[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    const int td = t_begin + d * kStep;
    rows[d] = td < t_end ? W::step_row(a, bt_lane, first_blk, td) : -1;
    W::load(a.k_cache, a, rows[d], td, t_end, voff0, kraw[d]);
    W::load(a.v_cache, a, rows[d], td, t_end, voff0, vraw[d]);
  }

  float m_run = kNegInf, l_run = 0.f;
  f32x4 o[Gm::NJ];
#pragma unroll
  for (int j = 0; j < Gm::NJ; ++j) o[j] = f32x4{0, 0, 0, 0};

  // One 32-token step on register set (kr, vr) holding tokens t0..t0+31 of
  // cache row `row`; returns the row of the step that refilled the set.
  auto step = [&](int t0, int64_t row, u32x4 (&kr)[Gm::RAW], u32x4 (&vr)[Gm::RAW]) -> int64_t {
    const int tn = t0 + DEPTH * kStep;
    const int64_t rown = (tn < t_end) ? W::step_row(a, bt_lane, first_blk, tn) : -1;
    wave_lds_sync();  // the previous step's V^T reads are issued before the tile is overwritten
    W::stage(tile, kr, lane);
    if (t0 == sub_t0) W::patch_row(tile, nbuf, sub_row, lane);
    W::load(a.k_cache, a, rown, tn, t_end, voff0, kr);  // empty past t_end
    wave_lds_sync();
    f32x4 s[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      s[i] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int kk = 0; kk < Gm::NKK; ++kk) s[i] = T::mfma16x16x32(W::kfrag(tile, i, kk, m, g), qf[kk], s[i]);
    }
    wave_lds_sync();  // K operand reads are issued before V overwrites the tile
    W::stage(tile, vr, lane);
    if (t0 == sub_t0) W::patch_row(tile, nbuf + Gm::ROWB, sub_row, lane);
    W::load(a.v_cache, a, rown, tn, t_end, voff0, vr);
    float x[8];
    float mloc = kNegInf;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const bool valid = row >= 0 && t0 + 16 * i + 4 * g + rr < t_end;
        const float v = valid ? s[i][rr] * sl2 : kNegInf;
        x[4 * i + rr] = v;
        mloc = fmaxf(mloc, v);
      }
    mloc = max32(max16(mloc));
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
      o[j] = T::mfma16x16x32(W::vfrag(tile, j, lane), pb, o[j]);
    }
    return rown;
  };

  for (int t0 = t_begin; t0 < t_end; t0 += DEPTH * kStep) {
    rows[0] = step(t0, rows[0], kraw[0], vraw[0]);
    if constexpr (DEPTH > 1) {
      if (t0 + kStep >= t_end) break;
      rows[1] = step(t0 + kStep, rows[1], kraw[1], vraw[1]);
    }
  }

  // ---- epilogue: lane (m, g) holds O^T[16j + 4g + r][head m]
  const float L = sum32(sum16(l_run));
  if (m >= G) return;
  const int head = kvh * G + m;
  const float inv = (L > 0.f) ? vscale / L : 0.f;
  if (single) {
    uint8_t *op = a.out + b * a.o_bs + head * a.o_hs;
    if (a.gate) {
      const uint8_t *gp = a.gate + b * a.g_bs + head * a.g_hs;
      u32x2 gr[Gm::NJ];
#pragma unroll
      for (int j = 0; j < Gm::NJ; ++j) gr[j] = *reinterpret_cast<const u32x2 *>(gp + (16 * j + 4 * g) * 2);
#pragma unroll
      for (int j = 0; j < Gm::NJ; ++j)
        *reinterpret_cast<u32x2 *>(op + (16 * j + 4 * g) * 2) = gate4<T>(o[j] * inv, gr[j]);
    } else {
#pragma unroll
      for (int j = 0; j < Gm::NJ; ++j) {
        const f32x4 v = o[j] * inv;
        *reinterpret_cast<u32x2 *>(op + (16 * j + 4 * g) * 2) = u32x2{T::pack2(v[0], v[1]), T::pack2(v[2], v[3])};
      }
    }
  } else {
    const int64_t idx = ws_row + static_cast<int64_t>(head) * ws_head_stride;
    float *wp = a.ws_o + idx * D;
#pragma unroll
    for (int j = 0; j < Gm::NJ; ++j) *reinterpret_cast<f32x4 *>(wp + 16 * j + 4 * g) = o[j] * inv;
    if (g == 0) a.ws_lse[idx] = (L > 0.f) ? m_run + __log2f(L) : kNegInf;
  }
}


// Zeros for the heads of kv head kvh of a padded graph row (ctx 0).
template <int D>
__device__ __forceinline__ void decode_zero_row(const DecodeArgs &a, int b, int kvh, int lane) {
  for (int it = lane; it < a.G * D / 4; it += 64) {
    const int h = it / (D / 4), d4 = it % (D / 4);
    uint8_t *o = a.out + b * a.o_bs + (kvh * a.G + h) * a.o_hs + d4 * 8;
    *reinterpret_cast<u32x2 *>(o) = u32x2{0, 0};
  }
}

// Split-K: one workgroup = HPW waves = HPW consecutive kv heads of one
// (sequence, split); wave w owns kv head blockIdx.y * HPW + w.  The waves of
// a workgroup step through the same tokens together, so the workgroup
// streams whole contiguous cache rows, and no cross-wave merge is needed:
// each wave owns its heads' softmax state.  The split index is the fastest
// grid dimension: dispatching a sequence's splits together measured 6%
// faster on cfg5 than all first splits first.
template <class T, bool FP8, int D, int HPW, int DEPTH, int WPE>
__global__ __launch_bounds__(64 * HPW) __attribute__((amdgpu_waves_per_eu(WPE)))
void paged_decode_kernel(const DecodeArgs a) {
  static_assert(DEPTH == 1 || DEPTH == 2, "prefetch depth");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int split = blockIdx.x, b = blockIdx.z;
  const int kvh = blockIdx.y * HPW + wave;
  if (kvh >= a.Hkv) return;  // whole wave; the kernel has no workgroup barrier
  // fused store: split 0's wave of each (sequence, kv head) writes the row
  if (a.k_new && split == 0) DecodeWave<T, FP8, D>::store_new(a, b, kvh, lane);
  const int ctx = min(a.context_lens[b], a.max_tokens);
  const int t_begin = split * a.split_tokens;
  if (ctx <= 0 || t_begin >= ctx) {
    if (ctx <= 0 && split == 0)  // padded graph row: defined zeros, no KV reads
      decode_zero_row<D>(a, b, kvh, lane);
    else if (split > 0)  // a split without tokens marks its partials empty for the merge
      for (int h = lane; h < a.G; h += 64)
        a.ws_lse[(static_cast<int64_t>(b) * a.Hq + kvh * a.G + h) * a.num_splits + split] = kNegInf;
    return;
  }
  const int t_end = min(t_begin + a.split_tokens, ctx);
  decode_piece<T, FP8, D, DEPTH>(a, smem + wave * DecodeWave<T, FP8, D>::LDS_PER_WAVE_B, b, kvh, t_begin, t_end,
                                 ctx <= a.split_tokens,
                                 static_cast<int64_t>(b) * a.Hq * a.num_splits + split, a.num_splits);
}

// ---------------------------------------------------------------- stream-K
// The contexts of the batch (clamped to [0, max_tokens]) laid end to end form
// T tokens; workgroup w of W takes tokens [B(w), B(w + 1)) with B(w) the
// token floor(w * T / W) rounded down to a multiple of 32 within its
// sequence, so every workgroup carries the same work whatever the lengths
// (a split-K grid of uneven splits leaves CUs idle while the longest splits
// finish).  A sequence that lies within one workgroup's range is written
// whole; a workgroup writes at most two partial pieces: slot 0 for a
// sequence that began in an earlier range, slot 1 for one that continues
// into a later range.  Workgroup w records B(w), and decode_merge_sk_kernel
// finds a sequence's pieces from those boundaries.  T < 2^31 (host check).
// A launch uses W = min(grid, max(one range per CU and group, T / 2048, the
// ranges that keep each within 61 blocks)) of its workgroups: every range
// then carries at least 2048 tokens where the batch has them (a range's
// fixed costs -- Q load, first-step latency, partial write -- stay small),
// and the rest record an empty range at the end (batch, 0) and exit.
constexpr int kSkMinPiece = 2048;
__device__ __forceinline__ int clamped_ctx(const DecodeArgs &a, int b) {
  return max(0, min(a.context_lens[b], a.max_tokens));
}
__device__ __forceinline__ int sk_total(const DecodeArgs &a, int batch, int lane) {
  int t = 0;
  for (int b0 = 0; b0 < batch; b0 += 64) t += b0 + lane < batch ? clamped_ctx(a, b0 + lane) : 0;
  return wave_sum_i32(t);
}
// Boundary B(w) as (sequence, token); B(W) = (batch, 0).  Whole waves.
__device__ __forceinline__ int2 sk_boundary(const DecodeArgs &a, int batch, int total, int w, int W, int lane) {
  if (w >= W) return int2{batch, 0};
  const int gpos = static_cast<int>(static_cast<int64_t>(w) * total / W);  // < total
  int base = 0;
  for (int b0 = 0; b0 < batch; b0 += 64) {
    const int c = b0 + lane < batch ? clamped_ctx(a, b0 + lane) : 0;
    const int incl = base + wave_iscan(c);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(incl > gpos);
    if (hit != 0) {
      const int l = static_cast<int>(__builtin_ctzll(hit));
      const int start = __builtin_amdgcn_readlane(incl - c, l);
      return int2{b0 + l, (gpos - start) & ~31};
    }
    base = __builtin_amdgcn_readlane(incl, 63);
  }
  return int2{batch, 0};  // not reached: gpos < T
}

// At most two waves per SIMD: the piece loop's state does not fit the
// register share of three (168 VGPRs) without spills.
template <class T, bool FP8, int D, int HPW, int DEPTH, int WPE>
__global__ __launch_bounds__(64 * HPW) __attribute__((amdgpu_waves_per_eu(WPE)))
void paged_decode_sk_kernel(const DecodeArgs a, int batch, int grid_w, int w_min) {
  static_assert(DEPTH == 1 || DEPTH == 2, "prefetch depth");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int w = blockIdx.x;
  const int kvh = blockIdx.y * HPW + wave;
  if (kvh >= a.Hkv) return;  // whole wave; the kernel has no workgroup barrier
  // fused store: workgroup w's wave of kv head kvh writes the rows of
  // sequences w, w + grid_w, ... after its pieces (the piece that reads a
  // new token takes it from the inputs, so the order does not matter)
  auto store_rows = [&]() {
    if (a.k_new)
      for (int b = w; b < batch; b += grid_w) DecodeWave<T, FP8, D>::store_new(a, b, kvh, lane);
  };
  const int total = sk_total(a, batch, lane);
  const int W = min(grid_w, max(w_min, max(total / kSkMinPiece, (total + 61 * a.block_size - 1) / (61 * a.block_size))));
  if (w >= W) {
    if (blockIdx.y == 0 && wave == 0 && lane == 0) a.sk_bnd[w] = int2{batch, 0};
    store_rows();
    return;
  }
  const int2 lo = sk_boundary(a, batch, total, w, W, lane);
  const int2 hi = sk_boundary(a, batch, total, w + 1, W, lane);
  if (blockIdx.y == 0 && wave == 0 && lane == 0) a.sk_bnd[w] = lo;
  uint8_t *tile = smem + wave * DecodeWave<T, FP8, D>::LDS_PER_WAVE_B;
  for (int b = lo.x; b < batch && (b < hi.x || (b == hi.x && hi.y > 0)); ++b) {
    const int ctx = clamped_ctx(a, b);
    const int t0 = b == lo.x ? lo.y : 0;
    const int t1 = b == hi.x ? hi.y : ctx;
    if (t1 <= t0) continue;
    const int slot = t0 > 0 ? 0 : 1;
    decode_piece<T, FP8, D, DEPTH>(a, tile, b, kvh, t0, t1, t0 == 0 && t1 == ctx,
                                   (static_cast<int64_t>(w) * 2 + slot) * a.Hq, 1);
  }
  store_rows();
}

int env_int(const char *name, int dflt) {
  const char *v = getenv(name);
  if (!v || !*v) return dflt;
  return atoi(v);
}

// Merge the per-split partials of every (sequence, head) with >1 split.
// nsplit: the splits the main kernel's grid had.  Every split of a row past
// the first either wrote its partials or marked them empty (lse -inf), so
// the merge needs no context length: it loads the lse values and partials
// of up to kMergeUnroll splits at once (one round trip per chunk of splits),
// and a row whose later splits are all empty (a single split, or a padded
// row) was written by the main kernel.
constexpr int kMergeUnroll = 16;
template <class T, int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(const DecodeArgs a, int batch, int nsplit) {
  constexpr int kPer = D / 4;  // threads per (b, head)
  const int pair = blockIdx.x * (256 / kPer) + threadIdx.x / kPer;
  const int d4 = threadIdx.x % kPer;
  if (pair >= batch * a.Hq) return;
  const int b = pair / a.Hq, head = pair % a.Hq;
  const int64_t base = static_cast<int64_t>(pair) * a.num_splits;
  // The splits in chunks of kMergeUnroll, each chunk's loads issued
  // together; the running maximum rescales the earlier chunks' sums (with
  // one chunk the weights are exp2(lse - max) directly).
  f32x4 acc{0, 0, 0, 0};
  float W = 0.f, M = kNegInf;
  bool multi = false;
#pragma unroll 1
  for (int c0 = 0; c0 < nsplit; c0 += kMergeUnroll) {
    float l[kMergeUnroll];
    f32x4 p[kMergeUnroll];
#pragma unroll
    for (int s = 0; s < kMergeUnroll; ++s) {
      l[s] = kNegInf;
      if (c0 + s < nsplit) {
        l[s] = a.ws_lse[base + c0 + s];
        p[s] = *reinterpret_cast<const f32x4 *>(a.ws_o + (base + c0 + s) * D + 4 * d4);
      }
    }
    float mc = kNegInf;
#pragma unroll
    for (int s = 0; s < kMergeUnroll; ++s) {
      if (c0 + s >= 1) multi |= l[s] != kNegInf;
      mc = fmaxf(mc, l[s]);
    }
    if (mc == kNegInf) continue;  // every split of the chunk is empty
    const float mn = fmaxf(M, mc);
    if (M != kNegInf) {
      const float r = __builtin_amdgcn_exp2f(M - mn);
      W *= r;
      acc *= r;
    }
    M = mn;
#pragma unroll
    for (int s = 0; s < kMergeUnroll; ++s)
      if (l[s] != kNegInf) {  // an empty split's partials are not read: they may be stale
        const float w = __builtin_amdgcn_exp2f(l[s] - M);
        W += w;
        acc += p[s] * w;
      }
  }
  if (!multi) return;  // a single split or a padded row: written by the main kernel
  const float inv = W > 0.f ? 1.0f / W : 0.f;
  acc *= inv;
  uint8_t *op = a.out + b * a.o_bs + head * a.o_hs + d4 * 8;
  if (a.gate)
    *reinterpret_cast<u32x2 *>(op) =
        gate4<T>(acc, *reinterpret_cast<const u32x2 *>(a.gate + b * a.g_bs + head * a.g_hs + d4 * 8));
  else
    *reinterpret_cast<u32x2 *>(op) = u32x2{T::pack2(acc[0], acc[1]), T::pack2(acc[2], acc[3])};
}

// Stream-K merge: every (sequence, head) whose tokens span several workgroup
// ranges gets the lse-weighted sum of its partials; padded rows (ctx 0) get
// zeros.  The pieces of sequence b are those of workgroups ws..we, where ws
// is the last range starting at or before (b, 0) (its piece is in slot 1)
// and we the last starting at or before (b, ctx - 1) (ws < w <= we: slot
// 0); a range with no tokens (equal consecutive starts) holds nothing.
// The range starts are staged in LDS (one load per thread) when they fit
// kSkLdsRanges entries, so the searches do not chain global-memory round
// trips.
constexpr int kSkLdsRanges = 4096;
template <class T, int D>
__global__ __launch_bounds__(256) void decode_merge_sk_kernel(const DecodeArgs a, int batch, int W) {
  constexpr int kPer = D / 4;  // threads per (b, head)
  __shared__ int2 lds_bnd[kSkLdsRanges];
  const bool staged = W <= kSkLdsRanges;
  if (staged) {
    for (int i = threadIdx.x; i < W; i += 256) lds_bnd[i] = a.sk_bnd[i];
    __syncthreads();
  }
  const int2 *bnd = staged ? lds_bnd : a.sk_bnd;
  const int pair = blockIdx.x * (256 / kPer) + threadIdx.x / kPer;
  const int d4 = threadIdx.x % kPer;
  if (pair >= batch * a.Hq) return;
  const int b = pair / a.Hq, head = pair % a.Hq;
  const int ctx = max(0, min(a.context_lens[b], a.max_tokens));
  uint8_t *op = a.out + b * a.o_bs + head * a.o_hs + d4 * 8;
  if (ctx == 0) {
    *reinterpret_cast<u32x2 *>(op) = u32x2{0, 0};
    return;
  }
  // Last range starting at or before (b, t); range 0 starts at or before
  // (b, 0) because sequence b has tokens.
  auto last_le = [&](int t) {
    int lo = 0, hi = W - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      const int2 s = bnd[mid];
      if (s.x < b || (s.x == b && s.y <= t)) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  };
  const int ws = last_le(0), we = last_le(ctx - 1);
  if (ws == we) return;  // written whole by the workgroup of range ws
  auto empty = [&](int w) {
    if (w + 1 >= W) return false;
    const int2 s0 = bnd[w], s1 = bnd[w + 1];
    return s0.x == s1.x && s0.y == s1.y;
  };
  auto row = [&](int w) { return (static_cast<int64_t>(w) * 2 + (w == ws ? 1 : 0)) * a.Hq + head; };
  float M = kNegInf;
  for (int w = ws; w <= we; ++w)
    if (!empty(w)) M = fmaxf(M, a.ws_lse[row(w)]);
  float Wsum = 0.f;
  f32x4 acc{0, 0, 0, 0};
  if (M != kNegInf) {
    for (int w = ws; w <= we; ++w) {
      if (empty(w)) continue;
      const int64_t r = row(w);
      const float l = a.ws_lse[r];
      const float wt = (l == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(l - M);
      Wsum += wt;
      acc += *reinterpret_cast<const f32x4 *>(a.ws_o + r * D + 4 * d4) * wt;
    }
  }
  const float inv = Wsum > 0.f ? 1.0f / Wsum : 0.f;
  acc *= inv;
  if (a.gate)
    *reinterpret_cast<u32x2 *>(op) =
        gate4<T>(acc, *reinterpret_cast<const u32x2 *>(a.gate + b * a.g_bs + head * a.g_hs + d4 * 8));
  else
    *reinterpret_cast<u32x2 *>(op) = u32x2{T::pack2(acc[0], acc[1]), T::pack2(acc[2], acc[3])};
}

// kv heads (= waves) per workgroup: 4 for 16-bit caches, 8 for fp8 with
// at least 8 kv heads (measured best on MI355X; eight 16-bit waves per
// workgroup and one prefetch step with more waves per SIMD both measured
// slower on the bench shapes).
int decode_heads_per_wg(int hkv, bool fp8) { return (fp8 && hkv >= 8) ? 8 : 4; }

// Calls f.template run<HPW, DEPTH, WPE>() for the decode kernels' launch
// shape: HPW kv heads (waves) per workgroup, DEPTH steps of raw K/V in
// flight, WPE waves per SIMD.  Register budget per wave = in-flight K/V +
// state: two steps deep (bf16: 2 waves/SIMD, fp8: 3).  head_dim 256: twice
// the raw K/V per step, one step in flight, one wave per SIMD.
template <bool FP8, int D, class F>
int with_decode_shape(int hpw, F &&f) {
  if constexpr (D == 256) {
    if constexpr (FP8) {
      if (hpw == 8) return f.template run<8, 1, 1>();
      return f.template run<4, 1, 1>();
    } else {
      return f.template run<4, 1, 1>();
    }
  } else {
    if (hpw == 8) return f.template run<8, 2, FP8 ? 3 : 2>();
    return f.template run<4, 2, FP8 ? 3 : 2>();
  }
}
template <bool FP8, int D>
int decode_hpw(int hkv) {
  const int hpw = decode_heads_per_wg(hkv, FP8);
  return (D == 256 && !FP8) ? 4 : hpw;  // eight waves of ~360 registers do not fit a CU
}

// Resident workgroups per CU of a kernel (cached per kernel and device).
int kernel_occupancy(const void *kernel, int threads, size_t lds) {
  struct Entry {
    const void *k;
    int dev, threads;
    size_t lds;
    int occ;
  };
  static std::mutex mu;
  static Entry cache[64];
  static int n = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n; ++i)
    if (cache[i].k == kernel && cache[i].dev == dev && cache[i].threads == threads && cache[i].lds == lds)
      return cache[i].occ;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, lds) != hipSuccess || occ < 1) {
    (void)hipGetLastError();
    occ = 1;
  }
  if (n < 64) cache[n++] = Entry{kernel, dev, threads, lds, occ};
  return occ;
}

// Stream-K applies to multi-split plans of at most 4096 sequences whose
// tokens (batch x table width) stay below 2^31 and fit 65535 ranges of at
// most 61 blocks each (a range's block-table entries are held one per lane,
// so a longer range would read wrong blocks past lane 63), for kernels with
// one resident workgroup per CU (the fp8 and head_dim-256 shapes): its grid
// is then one range per CU and group, all busy.  Measured on MI355X: cfg5
// (fp8, random contexts) 5.25 -> 6.0 TB/s against its split-K plan; the
// bf16 shapes, two workgroups per CU with already balanced split-K plans,
// lost 10-18%.  NQ_DECODE_STREAMK=0 keeps split-K.
constexpr int64_t kSkMaxRanges = 65535;  // grid.x of the stream-K kernel
bool sk_eligible(int batch, int64_t max_tokens, int block_size) {
  const int64_t total = batch * max_tokens;
  return env_int("NQ_DECODE_STREAMK", 1) != 0 && batch <= 4096 && total < (int64_t{1} << 31) &&
         (total + 61LL * block_size - 1) / (61LL * block_size) <= kSkMaxRanges;
}
int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }
int64_t sk_workspace_bytes(int64_t W, int Hq, int D) {
  return align256(W * 2 * Hq * D * 4) + align256(W * 2 * Hq * 4) + align256(W * 8);
}
// Workgroups per kv-head group: every resident slot of the device, and
// enough that no range exceeds 61 blocks (a range spans at most 63 block-
// table entries, one per lane, once its ends are rounded to 32 tokens).
int sk_workgroups(int occ, int groups, int batch, int64_t max_tokens, int block_size) {
  int64_t W = std::max<int64_t>(1, static_cast<int64_t>(device_cus()) * occ / groups);
  W = std::max<int64_t>(W, (batch * max_tokens + 61LL * block_size - 1) / (61LL * block_size));
  return static_cast<int>(std::min<int64_t>(W, kSkMaxRanges));  // sk_eligible keeps the 61-block bound within it
}

// Stream-K workgroups per group of a launch with these shapes on the
// kernel <T, FP8, D, H, DP, WP>, or 0 when it runs split-K: multi-split
// plans that sk_eligible accepts, on a kernel with one resident workgroup per
// CU, whose workspace holds the stream-K partials.
template <class T, bool FP8, int D, int H, int DP, int WP>
int sk_ranges(int batch, int hq, int hkv, int64_t max_tokens, int block_size, int num_splits, int64_t ws_bytes) {
  if (num_splits <= 1 || !sk_eligible(batch, max_tokens, block_size)) return 0;
  const size_t lds = static_cast<size_t>(H) * DecodeWave<T, FP8, D>::LDS_PER_WAVE_B;
  auto *kern = paged_decode_sk_kernel<T, FP8, D, H, DP, (WP > 2 ? 2 : WP)>;
  if (kernel_occupancy(reinterpret_cast<const void *>(kern), 64 * H, lds) != 1) return 0;
  const int W = sk_workgroups(1, (hkv + H - 1) / H, batch, max_tokens, block_size);
  return sk_workspace_bytes(W, hq, D) <= ws_bytes ? W : 0;
}

template <class T, bool FP8, int D>
struct DecodeLaunch {
  const DecodeArgs &a;
  int batch;
  hipStream_t s;
  template <int H, int DP, int WP>
  int run() const {
    const int groups = (a.Hkv + H - 1) / H;
    const size_t lds = static_cast<size_t>(H) * DecodeWave<T, FP8, D>::LDS_PER_WAVE_B;
    constexpr int per_block = 256 / (D / 4);
    const dim3 rgrid((batch * a.Hq + per_block - 1) / per_block);
    auto *kern = paged_decode_sk_kernel<T, FP8, D, H, DP, (WP > 2 ? 2 : WP)>;
    {
      const int W = sk_ranges<T, FP8, D, H, DP, WP>(batch, a.Hq, a.Hkv, a.max_tokens, a.block_size, a.num_splits,
                                                    a.ws_raw ? a.ws_bytes : 0);
      if (W > 0) {
        DecodeArgs k = a;
        k.ws_o = reinterpret_cast<float *>(a.ws_raw);
        k.ws_lse = reinterpret_cast<float *>(a.ws_raw + align256(static_cast<int64_t>(W) * 2 * a.Hq * D * 4));
        k.sk_bnd = reinterpret_cast<int2 *>(a.ws_raw + align256(static_cast<int64_t>(W) * 2 * a.Hq * D * 4) +
                                            align256(static_cast<int64_t>(W) * 2 * a.Hq * 4));
        kern<<<dim3(W, groups), 64 * H, lds, s>>>(k, batch, W, std::max(1, device_cus() / groups));
        const int rc = check_launch("paged_decode(stream-K)");
        if (rc != NQ_OK) return rc;
        decode_merge_sk_kernel<T, D><<<rgrid, 256, 0, s>>>(k, batch, W);
        return check_launch("paged_decode(stream-K merge)");
      }
    }
    // Splits past the table's tokens only size the workspace (for the
    // stream-K partials of another head_dim): no workgroups for them.
    const int64_t cover = (static_cast<int64_t>(a.max_tokens) + a.split_tokens - 1) / a.split_tokens;
    const int nsplit = static_cast<int>(std::min<int64_t>(a.num_splits, cover));
    paged_decode_kernel<T, FP8, D, H, DP, WP><<<dim3(nsplit, groups, batch), 64 * H, lds, s>>>(a);
    const int rc = check_launch("paged_decode");
    if (rc != NQ_OK || a.num_splits <= 1) return rc;
    decode_reduce_kernel<T, D><<<rgrid, 256, 0, s>>>(a, batch, nsplit);
    return check_launch("paged_decode(reduce)");
  }
};

// Schedule of a launch (1 stream-K, 0 split-K) for nq_decode_schedule.
template <bool FP8, int D>
struct DecodeSchedule {
  int batch, hq, hkv, block_size, num_splits;
  int64_t max_tokens, ws_bytes;
  template <int H, int DP, int WP>
  int run() const {
    return sk_ranges<BF16, FP8, D, H, DP, WP>(batch, hq, hkv, max_tokens, block_size, num_splits, ws_bytes) > 0;
  }
};

template <class T, bool FP8, int D>
int launch_decode(const DecodeArgs &a, int batch, hipStream_t s) {
  return with_decode_shape<FP8, D>(decode_hpw<FP8, D>(a.Hkv), DecodeLaunch<T, FP8, D>{a, batch, s});
}

// Stream-K workgroups per group the head_dim-D kernel would launch for
// these shapes, or 0 if it runs split-K.
template <bool FP8, int D>
struct SkPlanWorkgroups {
  int hkv, batch, block_size;
  int64_t max_tokens;
  template <int H, int DP, int WP>
  int run() const {
    const size_t lds = static_cast<size_t>(H) * DecodeWave<BF16, FP8, D>::LDS_PER_WAVE_B;
    const int occ = kernel_occupancy(
        reinterpret_cast<const void *>(paged_decode_sk_kernel<BF16, FP8, D, H, DP, (WP > 2 ? 2 : WP)>), 64 * H, lds);
    return occ == 1 ? sk_workgroups(1, (hkv + H - 1) / H, batch, max_tokens, block_size) : 0;
  }
};
template <bool FP8, int D>
int sk_plan_workgroups(int hkv, int batch, int64_t max_tokens, int block_size) {
  return with_decode_shape<FP8, D>(decode_hpw<FP8, D>(hkv), SkPlanWorkgroups<FP8, D>{hkv, batch, block_size, max_tokens});
}

}  // namespace
}  // namespace nq

using namespace nq;

// Largest split the decode kernel accepts: a split's block-table entries are
// held one per lane (64 per wave, one spare for the block after the split).
static int max_split_tokens(int block_size) { return static_cast<int>((63LL * block_size) / 128 * 128); }

// Split size: one split per workgroup should carry enough tokens that the
// workgroup's fixed costs (Q load, first-step latency, partial write) stay
// small, while the grid still spreads over every CU.  Measured on MI355X:
// 2048-token splits are best for the benchmark shapes; smaller batches get
// smaller splits (down to 512) so the grid keeps ~one workgroup per CU at the
// longest context the table allows.
extern "C" int nq_decode_plan(int batch, int num_q_heads, int num_kv_heads, int max_blocks_per_seq,
                              int block_size, int kv_dtype, int *num_splits, int *split_tokens) {
  if (!num_splits || !split_tokens || batch <= 0 || num_kv_heads <= 0 || max_blocks_per_seq <= 0 ||
      block_size <= 0)
    return fail(NQ_EINVAL, "decode_plan: bad arguments");
  if (num_q_heads <= 0) return fail(NQ_EINVAL, "decode_plan: bad arguments");
  const int64_t max_tokens = static_cast<int64_t>(max_blocks_per_seq) * block_size;
  const int hpw = decode_heads_per_wg(num_kv_heads, kv_dtype == NQ_FP8_E4M3);
  const int64_t groups = (num_kv_heads + hpw - 1) / hpw;
  int64_t split = env_int("NQ_DECODE_SPLIT_TOKENS", 0);
  if (split <= 0) {
    const int64_t per_cu = static_cast<int64_t>(batch) * groups * max_tokens / device_cus();
    split = 512;
    while (split < 2048 && split * 2 <= per_cu) split *= 2;
  }
  split = (split + 127) / 128 * 128;
  if (split < 128) split = 128;
  // a split's block-table entries are held one per lane: at most 63 blocks
  const int64_t max_split = max_split_tokens(block_size);
  if (split > max_split) split = max_split;
  if (max_tokens <= split) {
    *num_splits = 1;
    *split_tokens = static_cast<int>((max_tokens + 127) / 128 * 128);
    return NQ_OK;
  }
  int64_t ns = (max_tokens + split - 1) / split;
  // The workspace is sized from num_splits (nq_decode_workspace_bytes); a
  // multi-split decode runs as stream-K when that workspace also holds the
  // stream-K partials, so num_splits grows until it does, for whichever
  // head_dim (128 or 256; the plan does not know which) runs stream-K.
  if (sk_eligible(batch, max_tokens, block_size)) {
    const bool fp8 = kv_dtype == NQ_FP8_E4M3;
    const int w128 = fp8 ? sk_plan_workgroups<true, 128>(num_kv_heads, batch, max_tokens, block_size)
                         : sk_plan_workgroups<false, 128>(num_kv_heads, batch, max_tokens, block_size);
    const int w256 = fp8 ? sk_plan_workgroups<true, 256>(num_kv_heads, batch, max_tokens, block_size)
                         : sk_plan_workgroups<false, 256>(num_kv_heads, batch, max_tokens, block_size);
    auto fits = [&](int D, int W) {
      return W == 0 || nq_decode_workspace_bytes(batch, num_q_heads, D, static_cast<int>(ns)) >=
                           sk_workspace_bytes(W, num_q_heads, D);
    };
    while (ns < 65535 && !(fits(128, w128) && fits(256, w256))) ++ns;
  }
  *num_splits = static_cast<int>(ns);
  *split_tokens = static_cast<int>(split);
  return NQ_OK;
}

extern "C" int nq_decode_schedule(int batch, int num_q_heads, int num_kv_heads, int head_dim, int max_blocks_per_seq,
                                  int block_size, int kv_dtype, int num_splits, int64_t workspace_bytes) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_blocks_per_seq <= 0 || block_size <= 0 ||
      num_splits <= 0 || workspace_bytes < 0)
    return fail(NQ_EINVAL, "decode_schedule: bad arguments");
  if (head_dim != 128 && head_dim != 256)
    return fail(NQ_EUNSUPPORTED, "decode_schedule: head_dim %d (built: 128, 256)", head_dim);
  const int64_t max_tokens = std::min<int64_t>(static_cast<int64_t>(max_blocks_per_seq) * block_size, 0x7fffffff);
  const bool fp8 = kv_dtype == NQ_FP8_E4M3;
  if (head_dim == 256) {
    return fp8 ? with_decode_shape<true, 256>(decode_hpw<true, 256>(num_kv_heads),
                                              DecodeSchedule<true, 256>{batch, num_q_heads, num_kv_heads, block_size,
                                                                        num_splits, max_tokens, workspace_bytes})
               : with_decode_shape<false, 256>(decode_hpw<false, 256>(num_kv_heads),
                                               DecodeSchedule<false, 256>{batch, num_q_heads, num_kv_heads,
                                                                          block_size, num_splits, max_tokens,
                                                                          workspace_bytes});
  }
  return fp8 ? with_decode_shape<true, 128>(decode_hpw<true, 128>(num_kv_heads),
                                            DecodeSchedule<true, 128>{batch, num_q_heads, num_kv_heads, block_size,
                                                                      num_splits, max_tokens, workspace_bytes})
             : with_decode_shape<false, 128>(decode_hpw<false, 128>(num_kv_heads),
                                             DecodeSchedule<false, 128>{batch, num_q_heads, num_kv_heads, block_size,
                                                                        num_splits, max_tokens, workspace_bytes});
}

extern "C" int64_t nq_decode_workspace_bytes(int batch, int num_q_heads, int head_dim, int num_splits) {
  if (num_splits <= 1) return 0;
  const int64_t n = static_cast<int64_t>(batch) * num_q_heads * num_splits;
  int64_t bytes = n * head_dim * 4;
  bytes = (bytes + 255) / 256 * 256;
  return bytes + (n * 4 + 255) / 256 * 256;
}

static int paged_decode_impl(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                             const void *k_cache, const void *v_cache, const int32_t *block_tables,
                             int64_t bt_stride, int max_blocks_per_seq, const int32_t *context_lens,
                             void *out, int64_t out_batch_stride, int64_t out_head_stride, int batch,
                             int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                             int64_t num_blocks, float softmax_scale, int num_splits, int split_tokens,
                             void *workspace, int64_t workspace_bytes, int q_dtype, int kv_dtype,
                             const float *k_scale, const float *v_scale, const void *gate,
                             int64_t gate_batch_stride, int64_t gate_head_stride, void *stream,
                             const void *k_new = nullptr, int64_t k_new_row_stride = 0, const void *v_new = nullptr,
                             int64_t v_new_row_stride = 0, const int32_t *slot_mapping = nullptr,
                             int new_dtype = -1) {
  if (batch == 0) return NQ_OK;
  if (batch < 0 || batch > 65535 || num_q_heads <= 0 || num_kv_heads <= 0 || num_kv_heads > 65535)
    return fail(NQ_EINVAL, "paged_decode: bad batch/head counts");
  if (num_q_heads % num_kv_heads != 0)
    return fail(NQ_EINVAL, "paged_decode: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads,
                num_kv_heads);
  const int G = num_q_heads / num_kv_heads;
  if (G > 16) return fail(NQ_EUNSUPPORTED, "paged_decode: GQA group %d > 16", G);
  if (head_dim != 128 && head_dim != 256)
    return fail(NQ_EUNSUPPORTED, "paged_decode: head_dim %d (built: 128, 256)", head_dim);
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
  if (num_splits <= 0 || num_splits > 65535 || split_tokens <= 0 || split_tokens % 128 != 0)
    return fail(NQ_EINVAL, "paged_decode: bad split plan (%d x %d)", num_splits, split_tokens);
  // A split's block-table entries are held one per lane of a wave: a split
  // may span at most 63 blocks (the cap nq_decode_plan applies).
  if (split_tokens > max_split_tokens(block_size))
    return fail(NQ_EINVAL, "paged_decode: split_tokens %d > %d (63 blocks of %d)", split_tokens,
                max_split_tokens(block_size), block_size);
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
  if (gate && ((gate_batch_stride * 2) % 8 || (gate_head_stride * 2) % 8 || !aligned(gate, 8)))
    return fail(NQ_EINVAL, "paged_decode: gate must be 8-byte aligned with strides that are multiples of 4");
  a.gate = static_cast<const uint8_t *>(gate);
  a.g_bs = gate_batch_stride * 2;
  a.g_hs = gate_head_stride * 2;
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
  if (k_new) {
    // the fused store (nq_paged_decode_store): rows [batch, Hkv, D]
    const int nsz = elem_size(new_dtype);
    if (!v_new || !slot_mapping) return fail(NQ_EINVAL, "paged_decode_store: null k_new/v_new/slot_mapping");
    if (nsz == 0 || new_dtype == NQ_FP8_E4M3 || (!fp8 && new_dtype != kv_dtype))
      return fail(NQ_EUNSUPPORTED, "paged_decode_store: new rows of dtype %d into a cache of dtype %d", new_dtype,
                  kv_dtype);
    if (k_new_row_stride < static_cast<int64_t>(num_kv_heads) * head_dim ||
        v_new_row_stride < static_cast<int64_t>(num_kv_heads) * head_dim || (k_new_row_stride * nsz) % 16 ||
        (v_new_row_stride * nsz) % 16 || !aligned(k_new, 16) || !aligned(v_new, 16))
      return fail(NQ_EINVAL, "paged_decode_store: k_new/v_new rows must be 16-byte aligned [Hkv, D] rows");
    a.k_new = static_cast<const uint8_t *>(k_new);
    a.v_new = static_cast<const uint8_t *>(v_new);
    a.kn_rs = k_new_row_stride * nsz;
    a.vn_rs = v_new_row_stride * nsz;
    a.slot_mapping = slot_mapping;
    a.new_dtype = new_dtype;
  }
  if (num_splits > 1) {
    const int64_t need = nq_decode_workspace_bytes(batch, num_q_heads, head_dim, num_splits);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
      return fail(NQ_EINVAL, "paged_decode: workspace %lld bytes < %lld needed (or unaligned)",
                  (long long)workspace_bytes, (long long)need);
    const int64_t n = static_cast<int64_t>(batch) * num_q_heads * num_splits;
    a.ws_raw = static_cast<uint8_t *>(workspace);
    a.ws_bytes = workspace_bytes;
    a.ws_o = static_cast<float *>(workspace);
    a.ws_lse = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + (n * head_dim * 4 + 255) / 256 * 256);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (q_dtype == NQ_BF16)
    return head_dim == 256
               ? (fp8 ? launch_decode<BF16, true, 256>(a, batch, s) : launch_decode<BF16, false, 256>(a, batch, s))
               : (fp8 ? launch_decode<BF16, true, 128>(a, batch, s) : launch_decode<BF16, false, 128>(a, batch, s));
  return head_dim == 256
             ? (fp8 ? launch_decode<F16, true, 256>(a, batch, s) : launch_decode<F16, false, 256>(a, batch, s))
             : (fp8 ? launch_decode<F16, true, 128>(a, batch, s) : launch_decode<F16, false, 128>(a, batch, s));
}

extern "C" int nq_paged_decode(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                               const void *k_cache, const void *v_cache, const int32_t *block_tables,
                               int64_t bt_stride, int max_blocks_per_seq, const int32_t *context_lens,
                               void *out, int64_t out_batch_stride, int64_t out_head_stride, int batch,
                               int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                               int64_t num_blocks, float softmax_scale, int num_splits, int split_tokens,
                               void *workspace, int64_t workspace_bytes, int q_dtype, int kv_dtype,
                               const float *k_scale, const float *v_scale, void *stream) {
  return paged_decode_impl(q, q_batch_stride, q_head_stride, k_cache, v_cache, block_tables, bt_stride,
                           max_blocks_per_seq, context_lens, out, out_batch_stride, out_head_stride, batch,
                           num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, softmax_scale,
                           num_splits, split_tokens, workspace, workspace_bytes, q_dtype, kv_dtype, k_scale,
                           v_scale, nullptr, 0, 0, stream);
}

extern "C" int nq_paged_decode_gated(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                                     const void *k_cache, const void *v_cache, const int32_t *block_tables,
                                     int64_t bt_stride, int max_blocks_per_seq, const int32_t *context_lens,
                                     void *out, int64_t out_batch_stride, int64_t out_head_stride, int batch,
                                     int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                     int64_t num_blocks, float softmax_scale, int num_splits,
                                     int split_tokens, void *workspace, int64_t workspace_bytes, int q_dtype,
                                     int kv_dtype, const float *k_scale, const float *v_scale,
                                     const void *gate, int64_t gate_batch_stride, int64_t gate_head_stride,
                                     void *stream) {
  if (!gate) return fail(NQ_EINVAL, "paged_decode_gated: null gate");
  return paged_decode_impl(q, q_batch_stride, q_head_stride, k_cache, v_cache, block_tables, bt_stride,
                           max_blocks_per_seq, context_lens, out, out_batch_stride, out_head_stride, batch,
                           num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, softmax_scale,
                           num_splits, split_tokens, workspace, workspace_bytes, q_dtype, kv_dtype, k_scale,
                           v_scale, gate, gate_batch_stride, gate_head_stride, stream);
}

extern "C" int nq_paged_decode_store(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                                     void *k_cache, void *v_cache, const int32_t *block_tables, int64_t bt_stride,
                                     int max_blocks_per_seq, const int32_t *context_lens, const void *k_new,
                                     int64_t k_new_row_stride, const void *v_new, int64_t v_new_row_stride,
                                     const int32_t *slot_mapping, int new_dtype, void *out,
                                     int64_t out_batch_stride, int64_t out_head_stride, int batch,
                                     int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                     int64_t num_blocks, float softmax_scale, int num_splits, int split_tokens,
                                     void *workspace, int64_t workspace_bytes, int q_dtype, int kv_dtype,
                                     const float *k_scale, const float *v_scale, const void *gate,
                                     int64_t gate_batch_stride, int64_t gate_head_stride, void *stream) {
  if (!k_new) return fail(NQ_EINVAL, "paged_decode_store: null k_new");
  return paged_decode_impl(q, q_batch_stride, q_head_stride, k_cache, v_cache, block_tables, bt_stride,
                           max_blocks_per_seq, context_lens, out, out_batch_stride, out_head_stride, batch,
                           num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, softmax_scale,
                           num_splits, split_tokens, workspace, workspace_bytes, q_dtype, kv_dtype, k_scale,
                           v_scale, gate, gate_batch_stride, gate_head_stride, stream, k_new, k_new_row_stride,
                           v_new, v_new_row_stride, slot_mapping, new_dtype);
}

// ---------------------------------------------------------------------------
// nq_paged_decode_noalloc: the same kernels with the split-K partials in a
// static device array, for callers that cannot allocate.  Every call on a
// device shares that device's array; calls that overlap on one device (two
// streams, or two host threads) race on it.  The partials need no clearing:
// the merge reads only the splits the main kernel wrote in the same call.
namespace {
constexpr int64_t kScratchBytes = NQ_DECODE_NOALLOC_SCRATCH_BYTES;  // per device
constexpr int kMaxDevices = 64;
__device__ __attribute__((aligned(256))) uint8_t scratch[kScratchBytes];
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// Device address of the current device's copy of `scratch`, looked up once
// per device (each device holds its own copy at its own address).  The
// array's name is only a host-side handle: kernels get this address.
int scratch_address(void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(NQ_ELAUNCH, "paged_decode_noalloc: no current device (or device id %d >= %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(NQ_ELAUNCH, "paged_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return NQ_OK;
}
}  // namespace

extern "C" int nq_paged_decode_noalloc(const void *q, int64_t q_batch_stride, int64_t q_head_stride,
                                       const void *k_cache, const void *v_cache, const int32_t *block_tables,
                                       int64_t bt_stride, int max_blocks_per_seq, const int32_t *context_lens,
                                       void *out, int64_t out_batch_stride, int64_t out_head_stride, int batch,
                                       int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                       int64_t num_blocks, float softmax_scale, int num_splits, int split_tokens,
                                       int q_dtype, int kv_dtype, const float *k_scale, const float *v_scale,
                                       void *stream) {
  // The address is looked up on the first call on a device, whatever the
  // plan, so a caller's first (eager) call does it before any graph capture.
  void *ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != NQ_OK) return rc;
  if (num_splits > 1) {
    int64_t need = nq_decode_workspace_bytes(batch, num_q_heads, head_dim, num_splits);
    if (need > kScratchBytes && split_tokens > 0 && max_blocks_per_seq > 0) {
      // Splits past the table's tokens only size a caller's workspace for
      // stream-K partials; here the launch itself checks the array against
      // those, so the plan needs only the splits that cover the table.
      const int64_t cover = (static_cast<int64_t>(max_blocks_per_seq) * block_size + split_tokens - 1) / split_tokens;
      if (cover < num_splits) {
        num_splits = static_cast<int>(cover);
        need = nq_decode_workspace_bytes(batch, num_q_heads, head_dim, num_splits);
      }
    }
    if (need > kScratchBytes)
      return fail(NQ_EINVAL,
                  "paged_decode_noalloc: the plan (batch %d x %d heads x %d splits) needs %lld bytes of split-K "
                  "scratch, more than the static %lld",
                  batch, num_q_heads, num_splits, (long long)need, (long long)kScratchBytes);
  }
  return paged_decode_impl(q, q_batch_stride, q_head_stride, k_cache, v_cache, block_tables, bt_stride,
                           max_blocks_per_seq, context_lens, out, out_batch_stride, out_head_stride, batch,
                           num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, softmax_scale,
                           num_splits, split_tokens, ws, kScratchBytes, q_dtype, kv_dtype, k_scale, v_scale,
                           nullptr, 0, 0, stream);
}
