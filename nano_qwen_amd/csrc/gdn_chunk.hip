// Gated DeltaNet prefill in the chunked (WY) form, on MFMA (gfx950).
//
// Reference: chunk_gated_delta_rule (layers/gated_delta_net.py:44-82) with
// use_qk_l2norm_in_kernel=True -- the Triton kernels of layers/fla/:
// chunk_local_cumsum of the log decays, chunk_scaled_dot_kkt + solve_tril
// (the WY representation, chunk.py:23-72, wy_fast.py:23), the state pass
// over the chunks (chunk_delta_h.py:53) and the outputs (chunk_o.py:30) --
// with the gating computed before it (:197-198) and the final-state write to
// the pool after it (:210-214).
//
// Per sequence and value head, over chunks of C = 64 tokens with unit keys
// k_t, scaled unit queries q_t (x K^-1/2), beta_t = sigmoid(b_t), log decays
// g_t = -exp(A_log) softplus(a_t + dt_bias) and their in-chunk cumulative
// sums G_t, and the state S [V, K] entering the chunk:
//   A[i][j] = beta_i exp(G_i - G_j) (k_i . k_j)  (j < i),  T = (I + A)^-1
//   Tw = -T diag(beta exp(G)),  Tu = T diag(beta)
//   Y = K S^T,  D = Tu V + Tw Y               (the delta-rule updates)
//   P[i][j] = exp(G_i - G_j) (q_i . k_j)  (j <= i)
//   O = diag(exp(G)) Q S^T + P D
//   S <- exp(G_C) S + (diag(exp(G_C - G)) D)^T K
// which unrolls the per-token recurrence of nq_gdn_decode exactly in exact
// arithmetic.  (W = T diag(beta exp(G)) K and U = T diag(beta) V of the
// reference are never formed.)
//
// One 4-wave workgroup per (sequence, value head) walks the sequence's
// chunks; two fit on a CU (72 KiB of LDS, at most 256 VGPRs a wave).  Wave w
// owns value columns 32 w .. +31 of the state S^T [K][V], all 128 key rows of
// them, as float32 MFMA accumulators for the whole sequence: every
// state-dependent product of the chunk (Y = K S^T, Q S^T, the update
// solve, O += P D and the state update) is the wave's own, with no state
// copy through LDS and no barrier.  Only the chunk's shared inputs go
// through LDS: q and k as they are (their norms become per-token factors of
// the products' epilogues), V, the gates, A and P.
//
// The update D = Tu V + Tw Y is formed as the solution of
// (I + A) D = Z, Z = diag(beta) (V - diag(exp(G)) Y), by substitution over
// the four 16-token blocks of the chunk: D_j = T_jj (Z_j - sum_{m<j} A_jm D_m),
// with the inverses T_jj of the 16x16 diagonal blocks formed in float32 on
// the VALU (forward substitution, one lane per block and column) and the products on
// v_mfma_f32_16x16x16, whose accumulator rows are the next product's
// B-operand rows.  The other products run on v_mfma_f32_16x16x32 with
// 16-bit operands and float32 accumulation, as the reference's kernels do.
// A state block's accumulator row i holds key 32 s + 8 (i / 4) + 4 o + i % 4
// (block 2 s + o), so that the packed accumulators of blocks 2 s and 2 s + 1
// are the standard B operand of k-step s; the state update reads K down its
// columns in that order.
//
// LDS tiles are row-major with 16-byte chunks XOR-swizzled per row (128-
// column tiles: swz_r for row reads only, swz_c for tiles also read down
// their columns) or 8-byte pieces XOR-swizzled (64-column tiles, t64).
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kC = 64;         // tokens per chunk
constexpr int kD = 128;        // K = V
constexpr int kThreads = 256;  // 4 waves, one per SIMD; two workgroups per CU

struct ChunkArgs {
  const uint8_t *q, *k, *v;  // [T, H, K], [T, H, K], [T, HV, V] (dtype T)
  int64_t q_rs, k_rs, v_rs;  // bytes per token row
  const uint8_t *a, *b;      // [T, HV] (dtype T)
  int64_t a_rs, b_rs;
  const float *A_log, *dt_bias;  // [HV]
  float *state;                  // [num_slots, HV, V, K]
  const int32_t *idx;            // [num_seqs]
  int64_t num_slots;
  uint8_t *out;  // [T, HV, V]
  int64_t o_rs;
  const int32_t *cu;
  int H, HV, from_slot, num_seqs;
  float eps, scale;
};

constexpr int kSortSeqs = 64;  // batches up to this size run their longest sequences first

// LDS layout (bytes).
constexpr int kTile = kC * kD * 2;         // 64 x 128 16-bit values
constexpr int kOffK = 0;                   // K (unit keys) [t][k], swz_c
constexpr int kOffQ = kOffK + kTile;       // Q (scaled unit queries) [t][k], swz_r
constexpr int kOffV = kOffQ + kTile;       // V [t][v], swz_c
constexpr int kOffA = kOffV + kTile;       // 64 x 64 16-bit (t64): -A off the diagonal blocks, T_jj on them
constexpr int kOffP = kOffA + kC * kC * 2;  // P [i][j] (t64), zero above the diagonal blocks
constexpr int kOffB = kOffP + kC * kC * 2;  // the four diagonal 16x16 blocks of A, fp32 [b][i][j]
constexpr int kGates = 4 * kC * 4;          // G, beta, exp(G), exp(G_C - G): 64 fp32 each
constexpr int kOffG = kOffB + 4 * 256 * 4;  // two gate sets: this chunk's and the next one's
constexpr int kOffR = kOffG + 2 * kGates;    // 1 / |q| x K^-1/2 and 1 / |k| of the chunk's tokens: 64 fp32 each
constexpr int kOffW = kOffR + 2 * kC * 4;  // 256 bytes the L2 warm-up copies land in (never read)
constexpr int kLds = kOffW + 256;
static_assert(2 * kLds <= 160 * 1024, "two workgroups per CU");

// Chunk swizzles of the 128-column tiles (16 chunks a row).
__device__ inline int swz_r(int row) { return row & 15; }
__device__ inline int swz_c(int row) { return ((row & 7) << 1) | ((row >> 3) & 1); }

__device__ inline uint32_t lds_addr(const uint8_t *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t *)(p)));
}
__device__ inline uint32_t a128(uint32_t base, int row, int chunk, bool colwise) {
  return base + row * 256 + ((chunk ^ (colwise ? swz_c(row) : swz_r(row))) << 4);
}
// 8-byte piece `piece` (columns 4 piece .. +3) of row `row` of a 64-column 16-bit tile.
__device__ inline uint32_t t64(uint32_t base, int row, int piece) {
  return base + row * 128 + ((piece ^ (row & 15)) << 3);
}
__device__ inline float ldf(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) float *>(static_cast<uintptr_t>(addr));
}
__device__ inline void stf(uint32_t addr, float v) {
  *reinterpret_cast<__attribute__((address_space(3))) float *>(static_cast<uintptr_t>(addr)) = v;
}
__device__ inline f32x4 ldf4(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) f32x4 *>(static_cast<uintptr_t>(addr));
}
__device__ inline void stf4(uint32_t addr, const f32x4 &v) {
  *reinterpret_cast<__attribute__((address_space(3))) f32x4 *>(static_cast<uintptr_t>(addr)) = v;
}
__device__ inline u32x2 lds_load_b64(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x2 *>(static_cast<uintptr_t>(addr));
}
__device__ inline void lds_store_b64(uint32_t addr, const u32x2 &v) {
  *reinterpret_cast<__attribute__((address_space(3))) u32x2 *>(static_cast<uintptr_t>(addr)) = v;
}

__device__ inline float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }

template <int CTRL, int ROW_MASK>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}
// Sum over the 4 lanes of a quad; every lane gets the same bits.
__device__ inline float sum4(float v) {
  v += dpp_f<0xb1, 0xf>(v);       // quad_perm [1, 0, 3, 2]
  return v + dpp_f<0x4e, 0xf>(v);  // quad_perm [2, 3, 0, 1]
}
// Inclusive prefix sum over the wave: shifts by 1, 2, 4, 8 within each
// 16-lane row, then each row's running total into the rows after it
// (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3); lanes
// whose source is out of range add 0.
__device__ inline float wave_scan(float v) {
  v += dpp_f<0x111, 0xf>(v);  // row_shr:1
  v += dpp_f<0x112, 0xf>(v);  // row_shr:2
  v += dpp_f<0x114, 0xf>(v);  // row_shr:4
  v += dpp_f<0x118, 0xf>(v);  // row_shr:8
  v += dpp_f<0x142, 0xa>(v);  // row_bcast:15
  return v + dpp_f<0x143, 0xc>(v);  // row_bcast:31
}

template <class T>
__device__ inline f32x4 unpack2x2(uint32_t w0, uint32_t w1) {
  return f32x4{T::to_float(w0 & 0xffffu), T::to_float(w0 >> 16), T::to_float(w1 & 0xffffu), T::to_float(w1 >> 16)};
}
// a.x * b.x + a.y * b.y + c over packed 16-bit pairs (v_dot2_f32_*)
template <class T>
__device__ inline float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (T::dtype == NQ_BF16) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  } else {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
}
template <class T>
__device__ inline u32x2 pack4(const f32x4 &v) {
  return u32x2{T::pack2(v[0], v[1]), T::pack2(v[2], v[3])};
}
// B operand of a 16x16x32 k-step from two 16-row accumulator blocks: rows
// 4 (l / 16) .. +3 of `lo`, then of `hi` (the contraction order the A
// operand reads follow).
template <class T>
__device__ inline u32x4 pack8(const f32x4 &lo, const f32x4 &hi) {
  return u32x4{T::pack2(lo[0], lo[1]), T::pack2(lo[2], lo[3]), T::pack2(hi[0], hi[1]), T::pack2(hi[2], hi[3])};
}
__device__ inline u32x4 cat(const u32x2 &lo, const u32x2 &hi) { return u32x4{lo[0], lo[1], hi[0], hi[1]}; }

// Workgroup barrier after this wave's LDS writes complete, without the
// fence of __syncthreads(), which would also wait for the next chunk's
// global loads in flight and the output stores.
__device__ inline void lds_sync() {
  wait_lgkmcnt0();
  raw_barrier();
}

// A operand of the state update from the K tile read down its columns: lane
// l (i = l % 16, g = l / 16) takes key 32 sg + 8 (i / 4) + 4 o + i % 4 (row
// i of state block 2 sg + o) at tokens 32 s + 4 g .. +3 and 32 s + 16 + 4 g
// .. +3.  In a transposing read, lane 4 rho + p addresses row rho and an
// 8-byte piece, and lane i receives element i % 4 of the pieces of lanes
// i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4: piece p is keys 32 sg + 8 p + 4 o .. +3.
// `base` is the lane's address for s = 0, o = 0 (row 4 g + i / 4, the chunk
// of piece p; the swizzle depends on neither s nor the +16 rows).
__device__ inline u32x4 kt_op(uint32_t base, int o, int s) {
  return cat(lds_load_tr16<0>(base + 8 * o + 32 * 256 * s), lds_load_tr16<0>(base + 8 * o + 32 * 256 * s + 16 * 256));
}

template <class T>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_chunk_kernel(
    const ChunkArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t L = lds_addr(smem);
  const uint32_t LK = L + kOffK, LQ = L + kOffQ, LV = L + kOffV, LA = L + kOffA, LBD = L + kOffB;
  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);  // uniform: branches on it are scalar
  // The value heads of one key head read the same q and k: with enough heads
  // they get grid columns 8 apart, which the hardware places on the same XCD
  // (workgroup L on XCD L % 8), so the second reads them from that L2.
  int hv = blockIdx.x;
  {
    const int G = a.HV / a.H;
    if (G > 1 && a.HV % (8 * G) == 0) {
      const int i = hv & 7, j = hv >> 3;
      hv = (i + 8 * (j / G)) * G + j % G;
    }
    hv = __builtin_amdgcn_readfirstlane(hv);  // uniform: the head's constants load as scalars
  }
  // Workgroups start in grid order and a sequence's chunks run one after
  // another, so the longest sequences go first (row y of the grid takes the
  // sequence of rank y by length, ties by index); wave 0 ranks them.
  int n = blockIdx.y;
  if (a.num_seqs <= kSortSeqs) {
    if (wave == 0) {
      const int lane = tid0 & 63;
      const int len = lane < a.num_seqs ? a.cu[lane + 1] - a.cu[lane] : -1;
      int rank = 0;
      for (int s2 = 0; s2 < a.num_seqs; ++s2) {
        const int l2 = __builtin_amdgcn_readlane(len, s2);
        rank += (l2 > len || (l2 == len && s2 < lane)) ? 1 : 0;
      }
      const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < a.num_seqs && rank == static_cast<int>(blockIdx.y));
      if (lane == 0) *reinterpret_cast<__attribute__((address_space(3))) int *>(static_cast<uintptr_t>(L + kOffG)) =
          static_cast<int>(__builtin_ctzll(hit));
    }
    lds_sync();
    n = __builtin_amdgcn_readfirstlane(
        *reinterpret_cast<const __attribute__((address_space(3))) int *>(static_cast<uintptr_t>(L + kOffG)));
    lds_sync();  // read by every wave before the region is reused
  }
  const int h = hv / (a.HV / a.H);
  const int t0 = a.cu[n], t1 = a.cu[n + 1];
  const int slot = a.idx[n];
  const bool has = slot >= 0 && slot < a.num_slots;
  float *st = has ? a.state + (static_cast<int64_t>(slot) * a.HV + hv) * kD * kD : nullptr;
  // per-head gate constants, held in scalar registers
  const float neg_a = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, -expf(a.A_log[hv]))));
  const float dtb = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, a.dt_bias[hv])));

  // This wave's state: S^T blocks kb (keys, in the order above) x half hf
  // (value columns 32 wave + 16 hf .. +15); element r of lane l is key
  // 32 (kb / 2) + 8 (l / 16) + 4 (kb % 2) + r, value column 32 wave + 16 hf + l % 16.
  const int m0 = tid0 & 15, g0 = (tid0 >> 4) & 3;
  f32x4 S[8][2];
  auto state_at = [&](int kb, int hf) {
    return reinterpret_cast<f32x4 *>(st + (32 * wave + 16 * hf + m0) * kD + 32 * (kb >> 1) + 8 * g0 + 4 * (kb & 1));
  };
  if (has && a.from_slot) {
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) S[kb][hf] = *state_at(kb, hf);
  } else {
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) S[kb][hf] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Inputs of a chunk: q and k fetched one chunk ahead into registers (row
  // tid / 4, columns 32 (tid % 4) .. +31), through buffer descriptors over
  // the chunk's rows of this head: rows past the sequence are out of range
  // and read as zeros.
  u32x4 qv[4], kv[4];
  auto fetch = [&](int c0, int tid) {
    const int r = tid >> 2, e = tid & 3;
    const int rows = min(kC, t1 - c0);
    const auto rq = make_rsrc(a.q + static_cast<int64_t>(c0) * a.q_rs + h * kD * 2,
                              static_cast<uint32_t>((rows - 1) * a.q_rs + kD * 2));
    const auto rk = make_rsrc(a.k + static_cast<int64_t>(c0) * a.k_rs + h * kD * 2,
                              static_cast<uint32_t>((rows - 1) * a.k_rs + kD * 2));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col2 = (32 * e + 8 * j) * 2;
      qv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, r * static_cast<int>(a.q_rs) + col2, 0, 0));
      kv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, r * static_cast<int>(a.k_rs) + col2, 0, 0));
    }
  };
  // V of the chunk at c0 straight into its LDS tile (no registers): wave w
  // copies rows 16 w .. +15, four rows per copy; lane l of a copy lands in
  // chunk position l % 16 of row 4 q + l / 16 and so loads the logical chunk
  // the swizzle puts there.  Rows past the sequence read as zeros.
  auto copy_v = [&](int c0, int tid) {
    const int rows = min(kC, t1 - c0);
    const u32x4 rv = rsrc_words(a.v + static_cast<int64_t>(c0) * a.v_rs + hv * kD * 2,
                                static_cast<uint32_t>((rows - 1) * a.v_rs + kD * 2));
    const int l = tid & 63;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int row0 = 16 * wave + 4 * q4, row = row0 + (l >> 4);  // row0 uniform: M0
      const int chunk = (l & 15) ^ swz_c(row);
      dma16_opaque(LV + row0 * 256, rv, static_cast<uint32_t>(row * static_cast<int>(a.v_rs) + 16 * chunk));
    }
  };
  // The next chunk's q and k rows into L2 ahead of their fetch: one dword
  // of each 128-byte line, by LDS DMA into a scratch area nobody reads
  // (waves 0 and 1: q rows 0-31 and 32-63; waves 2 and 3: the same of k).
  // Rows past the sequence fall outside the descriptor.
  auto warm = [&](int c0, int tid) {
    const int rows = min(kC, t1 - c0);
    const uint8_t *src = wave < 2 ? a.q : a.k;
    const int64_t rs = wave < 2 ? a.q_rs : a.k_rs;
    const u32x4 rw = rsrc_words(src + static_cast<int64_t>(c0) * rs + h * kD * 2,
                                static_cast<uint32_t>((rows - 1) * rs + kD * 2));
    const int l = tid & 63, row = 32 * (wave & 1) + (l >> 1);
    dma4_opaque(L + kOffW, rw, static_cast<uint32_t>(row * static_cast<int>(rs) + 128 * (l & 1)));
  };
  // The gates of the chunk at c0 into gate set `set`: wave w copies field w
  // of the 64 tokens (one dword per lane) from the output rows; tokens past
  // the sequence read as zeros.
  auto copy_gates = [&](int c0, int set, int tid) {
    const int rows = min(kC, t1 - c0);
    const u32x4 rg = rsrc_words(a.out + static_cast<int64_t>(c0) * a.o_rs + hv * kD * 2,
                                static_cast<uint32_t>((rows - 1) * a.o_rs + 16));
    dma4_opaque(L + kOffG + set * kGates + kC * 4 * wave, rg,
                static_cast<uint32_t>((tid & 63) * static_cast<int>(a.o_rs) + 4 * wave));
  };
  // Gates of every chunk of the sequence up front (wave w: chunks w, w + 4,
  // ...; lane = token), into the first 16 bytes of each token's output row:
  // G, the in-chunk inclusive sum of the log decays, beta, exp(G) and
  // exp(G_C - G).  A chunk's copy reads them before its output overwrites
  // the row.
  if (t1 > t0) {
    const int lane = tid0 & 63;
    for (int c0 = t0 + kC * wave; c0 < t1; c0 += 4 * kC) {
      const int ck = min(kC, t1 - c0);
      float g = 0.f, beta = 0.f;
      const int64_t t = c0 + lane;
      if (lane < ck) {
        const float xa = T::to_float(reinterpret_cast<const uint16_t *>(a.a + t * a.a_rs)[hv]);
        const float xb = T::to_float(reinterpret_cast<const uint16_t *>(a.b + t * a.b_rs)[hv]);
        g = neg_a * softplus(xa + dtb);
        beta = 1.0f / (1.0f + expf(-xb));
      }
      g = wave_scan(g);
      // G_C = G of the chunk's last token (tokens past the sequence add 0)
      const float gc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, g), 63));
      if (lane < ck)
        *reinterpret_cast<f32x4 *>(a.out + t * a.o_rs + hv * kD * 2) = f32x4{g, beta, __expf(g), __expf(gc - g)};
    }
    // stores complete and seen by every wave, then the first chunk's gates
    // (the compiler's wait for the q and k fetched after them covers the copy)
    wait_vmcnt<0>();
    raw_barrier();
    copy_gates(t0, 0, tid0);
    fetch(t0, tid0);
    // P's blocks (0, 1) and (2, 3), read by O += P D and never written
    // otherwise: zero once
    if (wave < 2) lds_store_b64(t64(L + kOffP, 32 * wave + (tid0 & 15), 4 * (2 * wave + 1) + ((tid0 >> 4) & 3)), u32x2{0u, 0u});
  }
  // Per-lane LDS addresses of the operand reads, formed once: the tile
  // swizzles depend only on a row's low four bits, so every block, k-step or
  // row offset below is an immediate added to one of these.
  //   bK[x], bQ[x]: row m of the K and Q tiles, chunk 4 x + g (16-byte row reads)
  //   bKT[x]: the state update's transposing reads of K (kt_op, sg = x)
  //   bV[hf]: Z's transposing reads of V, columns 32 w + 16 hf ..
  //   bT[x]: row m, piece 4 x + g of the 64-column tiles (A; P 8 KiB on)
  uint32_t bK[4], bQ[4], bKT[4], bV[2], bT[4];
  {
    const int lane = tid0 & 63, m = lane & 15, g = lane >> 4;
    const int rr = 4 * g + (m >> 2), p = m & 3;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      bK[x] = a128(L + kOffK, m, 4 * x + g, true);
      bQ[x] = a128(L + kOffQ, m, 4 * x + g, false);
      bKT[x] = a128(L + kOffK, rr, 4 * x + p, true);
      bT[x] = t64(L + kOffA, m, 4 * x + g);
    }
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) bV[hf] = a128(L + kOffV, rr, 4 * wave + 2 * hf + (p >> 1), true) + 8 * (p & 1);
#pragma unroll
    for (int x = 0; x < 4; ++x) asm volatile("" : "+v"(bK[x]), "+v"(bQ[x]), "+v"(bKT[x]), "+v"(bT[x]));
    asm volatile("" : "+v"(bV[0]), "+v"(bV[1]));
  }
  for (int c0 = t0; c0 < t1; c0 += kC) {
    // this chunk's gate set (the next chunk's is copied during this one)
    const int gset = ((c0 - t0) / kC) & 1;
    const uint32_t LG = L + kOffG + gset * kGates, LB = LG + kC * 4, LEG = LB + kC * 4, LEC = LEG + kC * 4;
    const uint32_t LRQ = L + kOffR, LRK = LRQ + kC * 4;
    const int ck = min(kC, t1 - c0);
    // The thread index from an instruction the compiler cannot hoist: the
    // LDS addresses derived from it are recomputed per chunk instead of each
    // holding a register across the loop.
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int m = lane & 15, g = lane >> 4;
    const int wv = tid >> 6;  // the wave index for addresses (branches use the uniform `wave`)
    // ---- q and k rows into LDS as they are; their norms (float32) as
    // per-token factors 1 / |q| x K^-1/2 and 1 / |k|, which the products'
    // epilogues apply.
    {
      const int r = tid >> 2, e = tid & 3;
      float sq0 = 0.f, sq1 = 0.f, sk0 = 0.f, sk1 = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sq0 = dot2<T>(qv[j][0], qv[j][0], dot2<T>(qv[j][1], qv[j][1], sq0));
        sq1 = dot2<T>(qv[j][2], qv[j][2], dot2<T>(qv[j][3], qv[j][3], sq1));
        sk0 = dot2<T>(kv[j][0], kv[j][0], dot2<T>(kv[j][1], kv[j][1], sk0));
        sk1 = dot2<T>(kv[j][2], kv[j][2], dot2<T>(kv[j][3], kv[j][3], sk1));
      }
      const float sq = sum4(sq0 + sq1), sk = sum4(sk0 + sk1);
      if (e == 0) {
        stf(LRQ + 4 * r, a.scale * __builtin_amdgcn_rsqf(sq + a.eps));
        stf(LRK + 4 * r, __builtin_amdgcn_rsqf(sk + a.eps));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int chunk = 4 * e + j;
        lds_store_b128(a128(LQ, r, chunk, false), qv[j]);
        lds_store_b128(a128(LK, r, chunk, true), kv[j]);
      }
    }
    // V, and the next chunk's gates: their regions are free (the last
    // chunk's reads ended before its final barrier); issued after q and k are
    // consumed, so that the compiler's waits for those do not also wait for
    // these copies.  Completed by the vmcnt(0) before the barrier ahead of Z.
    copy_v(c0, tid);
    if (c0 + kC < t1) copy_gates(c0 + kC, gset ^ 1, tid);
    lds_sync();

    // ---- A and P by 16x16 blocks, formed transposed (rows j, columns i):
    // A[i][j] = beta_i exp(G_i - G_j) (k_i . k_j) for j < i, P[i][j] =
    // exp(G_i - G_j) (q_i . k_j) for j <= i (P's two blocks above the
    // diagonal that O += P D reads are zeroed once).  Wave w forms diagonal
    // block w of A (K_b K_b^T: one operand read per k-step) in float32; then
    // wave 0 inverts the four: T_bb = (I + A_bb)^-1 by forward substitution,
    // lane = block l / 16 and column l % 16, stored transposed in the
    // diagonal blocks of the 16-bit tile, while waves 1-3 form -A below the
    // diagonal blocks (16 bits) and P.
    // Element r of a block's accumulator: row j = 16 J + 4 g + r, column i = 16 I + m.
    // dec[r] = exp(G_i - G_j) / |k_j|, fa = beta_i / |k_i|, fp = 1 / |q_i| x K^-1/2
    auto decay = [&](int I, int J, f32x4 &dec, float &fa, float &fp) {
      const int i = 16 * I + m, jb = 16 * J + 4 * g;
      const float Gi = ldf(LG + 4 * i);
      fa = ldf(LB + 4 * i) * ldf(LRK + 4 * i);
      fp = ldf(LRQ + 4 * i);
      const f32x4 Gj = ldf4(LG + 4 * jb), rkj = ldf4(LRK + 4 * jb);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        // G_i <= G_j for tokens j <= i of the sequence; past it G reads 0
        dec[r] = __expf(jb + r <= i ? fminf(Gi - Gj[r], 0.f) : 0.f) * rkj[r];
    };
    // A^T and P^T of the pair (I, J), J < I: operands K_J, K_I, Q_I
    auto pair_job = [&](int I, int J) {
      f32x4 ca = f32x4{0.f, 0.f, 0.f, 0.f}, cp = ca;
      u32x4 kj[4], ki[4], qi[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        kj[s] = lds_load_b128<0>(bK[s] + 16 * 256 * J);
        ki[s] = lds_load_b128<0>(bK[s] + 16 * 256 * I);
        qi[s] = lds_load_b128<0>(bQ[s] + 16 * 256 * I);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        ca = T::mfma16x16x32(kj[s], ki[s], ca);
        cp = T::mfma16x16x32(kj[s], qi[s], cp);
      }
      f32x4 dec;
      float fa, fp;
      decay(I, J, dec, fa, fp);
      lds_store_b64(bT[J] + 16 * 128 * I, pack4<T>(-(fa * dec * ca)));                 // A: row 16 I + m, piece 4 J + g
      lds_store_b64(bT[J] + (kOffP - kOffA) + 16 * 128 * I, pack4<T>(fp * dec * cp));  // P
    };
    // P^T of the diagonal block I: operands K_I, Q_I
    auto diag_p_job = [&](int I) {
      f32x4 cp = f32x4{0.f, 0.f, 0.f, 0.f};
      u32x4 ki[4], qi[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        ki[s] = lds_load_b128<0>(bK[s] + 16 * 256 * I);
        qi[s] = lds_load_b128<0>(bQ[s] + 16 * 256 * I);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) cp = T::mfma16x16x32(ki[s], qi[s], cp);
      f32x4 dec;
      float fa, fp;
      decay(I, I, dec, fa, fp);
      f32x4 pv;
#pragma unroll
      for (int r = 0; r < 4; ++r) pv[r] = 4 * g + r <= m ? fp * dec[r] * cp[r] : 0.f;
      lds_store_b64(bT[I] + (kOffP - kOffA) + 16 * 128 * I, pack4<T>(pv));
    };
    // the diagonal block `wave` of A in float32 (row m, columns 4 g .. +3)
    {
      const int b = wave;
      f32x4 ca = f32x4{0.f, 0.f, 0.f, 0.f};
      u32x4 kb[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) kb[s] = lds_load_b128<0>(bK[s] + 16 * 256 * b);
#pragma unroll
      for (int s = 0; s < 4; ++s) ca = T::mfma16x16x32(kb[s], kb[s], ca);
      f32x4 dec, av;
      float fa, fp;
      decay(b, b, dec, fa, fp);
#pragma unroll
      for (int r = 0; r < 4; ++r) av[r] = 4 * g + r < m ? fa * dec[r] * ca[r] : 0.f;
      stf4(LBD + 4 * (256 * b + 16 * m + 4 * g), av);
    }
    lds_sync();
    if (wave == 0) {
      const int b = g, c = m;
      const uint32_t base = LBD + 4 * 256 * b;
      float x[16];
      // row by row, each row's reads issued three rows ahead (the scheduling
      // barrier keeps them there); two partial sums per row shorten the
      // dependent chain
      constexpr int kAhead = 3;
      f32x4 av[16][4];
      auto read_row = [&](int i) {
#pragma unroll
        for (int jc = 0; jc < 4; ++jc)
          if (4 * jc < i) av[i][jc] = ldf4(base + 4 * (16 * i + 4 * jc));
      };
#pragma unroll
      for (int i = 1; i <= kAhead; ++i) read_row(i);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i + kAhead < 16) read_row(i + kAhead);
        __builtin_amdgcn_sched_barrier(0);
        float acc0 = i == c ? 1.f : 0.f, acc1 = 0.f;
#pragma unroll
        for (int j = 0; j < i; ++j) {
          if (j & 1)
            acc1 -= av[i][j >> 2][j & 3] * x[j];
          else
            acc0 -= av[i][j >> 2][j & 3] * x[j];
        }
        x[i] = i < c ? 0.f : acc0 + acc1;
      }
      // column c of T_bb is row c of its transpose: four 8-byte pieces
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        lds_store_b64(t64(LA, 16 * b + c, 4 * b + q4), pack4<T>(f32x4{x[4 * q4], x[4 * q4 + 1], x[4 * q4 + 2], x[4 * q4 + 3]}));
    } else if (wave == 1) {
      pair_job(1, 0);
      pair_job(2, 0);
      diag_p_job(0);
      diag_p_job(1);
    } else if (wave == 2) {
      pair_job(2, 1);
      pair_job(3, 0);
      diag_p_job(2);
    } else {
      pair_job(3, 1);
      pair_job(3, 2);
      diag_p_job(3);
    }
    // This wave's V and gate copies (issued with the chunk's inputs; nothing
    // else is in flight here) complete before this barrier, so that Z, after
    // the products below (which write no LDS), reads every wave's V rows
    // without a barrier of its own.
    wait_vmcnt<0>();
    lds_sync();
    // The next chunk's q and k lines into L2 now, about half a chunk before
    // their fetch: from memory the fetch's latency outlasted the rest of the
    // chunk.  Issued after the wait above, nothing waits for these copies
    // before the fetch they precede is consumed.
    if (c0 + kC < t1) warm(c0 + kC, tid);

    // Y = K S^T, O = Q S^T by 16-row blocks mb and column halves hf (row
    // 16 mb + 4 g + r, column 32 w + 16 hf + m); B operand of k-step s: the
    // packed state blocks 2 s and 2 s + 1.
    f32x4 Y[4][2], O[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) Y[mb][hf] = O[mb][hf] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Rolling operand pipeline: block mb's K and Q operands of k-step s + 1
    // are read as soon as its products of k-step s are issued, so each read
    // has twelve products to land in; the scheduling barriers keep the
    // compiler from moving the reads down to their uses.
    u32x4 kr[4], qr[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      kr[mb] = lds_load_b128<0>(bK[0] + 16 * 256 * mb);
      qr[mb] = lds_load_b128<0>(bQ[0] + 16 * 256 * mb);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // the state packed once for both products
      const u32x4 sb[2] = {pack8<T>(S[2 * s][0], S[2 * s + 1][0]), pack8<T>(S[2 * s][1], S[2 * s + 1][1])};
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          Y[mb][hf] = T::mfma16x16x32(kr[mb], sb[hf], Y[mb][hf]);
          O[mb][hf] = T::mfma16x16x32(qr[mb], sb[hf], O[mb][hf]);
        }
        if (s < 3) {
          kr[mb] = lds_load_b128<0>(bK[s + 1] + 16 * 256 * mb);
          qr[mb] = lds_load_b128<0>(bQ[s + 1] + 16 * 256 * mb);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // ---- Z = diag(beta) (V - diag(exp(G)) Y) for rows 16 mb + 4 g + r,
    // then D by substitution over the blocks, per half of the columns.
    f32x4 D[4][2];
    {
      f32x4 Bt[4], Et[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        Bt[mb] = ldf4(LB + 4 * (16 * mb + 4 * g));
        Et[mb] = ldf4(LEG + 4 * (16 * mb + 4 * g)) * ldf4(LRK + 4 * (16 * mb + 4 * g));  // Y's rows: raw keys
      }
      // V rows 16 mb + 4 g .. +3 at column 32 w + 16 hf + m, by transposing
      // reads, all issued together (the scheduling barrier keeps the compiler
      // from spreading them out to their uses, one round trip each)
      u32x2 vw[4][2];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) vw[mb][hf] = lds_load_tr16<0>(bV[hf] + 16 * 256 * mb);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const f32x4 vf = unpack2x2<T>(vw[mb][hf][0], vw[mb][hf][1]);
#pragma unroll
          for (int r = 0; r < 4; ++r) Y[mb][hf][r] = Bt[mb][r] * (vf[r] - Et[mb][r] * Y[mb][hf][r]);
        }
      u32x2 Tb[4], Am[6];
      // T_jj is stored transposed: a transposing read gives lane (g, m) row m,
      // columns 4 g .. +3 (lane 4 rho + p addresses row 4 g + rho, piece p)
#pragma unroll
      for (int j = 0; j < 4; ++j) Tb[j] = lds_load_tr16<0>(t64(LA, 16 * j + 4 * g + (m >> 2), 4 * j + (m & 3)));
      // -A_jm: row 16 j + m, piece 4 mm + g
      Am[0] = lds_load_b64(bT[0] + 16 * 128 * 1);
      Am[1] = lds_load_b64(bT[0] + 16 * 128 * 2);
      Am[2] = lds_load_b64(bT[1] + 16 * 128 * 2);
      Am[3] = lds_load_b64(bT[0] + 16 * 128 * 3);
      Am[4] = lds_load_b64(bT[1] + 16 * 128 * 3);
      Am[5] = lds_load_b64(bT[2] + 16 * 128 * 3);
      const f32x4 z4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        D[0][hf] = T::mfma16x16x16(Tb[0], pack4<T>(Y[0][hf]), z4);
        const u32x2 d0 = pack4<T>(D[0][hf]);
        f32x4 w1 = T::mfma16x16x16(Am[0], d0, Y[1][hf]);
        f32x4 w2 = T::mfma16x16x16(Am[1], d0, Y[2][hf]);
        f32x4 w3 = T::mfma16x16x16(Am[3], d0, Y[3][hf]);
        D[1][hf] = T::mfma16x16x16(Tb[1], pack4<T>(w1), z4);
        const u32x2 d1 = pack4<T>(D[1][hf]);
        w2 = T::mfma16x16x16(Am[2], d1, w2);
        w3 = T::mfma16x16x16(Am[4], d1, w3);
        D[2][hf] = T::mfma16x16x16(Tb[2], pack4<T>(w2), z4);
        w3 = T::mfma16x16x16(Am[5], pack4<T>(D[2][hf]), w3);
        D[3][hf] = T::mfma16x16x16(Tb[3], pack4<T>(w3), z4);
      }
    }
    // the next chunk's q and k, in flight while this one finishes (issued
    // here, not at the top, so that their registers are not live beside the
    // products and the solve above)
    if (c0 + kC < t1) fetch(c0 + kC, tid);
    // D as the B operands of P D and of the state update (with the factors
    // exp(G_C - G) of its rows).
    u32x4 bd[2][2], bt[2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      // with 1 / |k_t|: the state update reads the raw keys
      const f32x4 flo = ldf4(LEC + 4 * (32 * s + 4 * g)) * ldf4(LRK + 4 * (32 * s + 4 * g));
      const f32x4 fhi = ldf4(LEC + 4 * (32 * s + 16 + 4 * g)) * ldf4(LRK + 4 * (32 * s + 16 + 4 * g));
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        bd[s][hf] = pack8<T>(D[2 * s][hf], D[2 * s + 1][hf]);
        bt[s][hf] = pack8<T>(D[2 * s][hf] * flo, D[2 * s + 1][hf] * fhi);
      }
    }
    // ---- O = diag(exp(G)) Q S^T + P D, stored as 16-bit values.
    {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const f32x4 e4 = ldf4(LEG + 4 * (16 * mb + 4 * g)) * ldf4(LRQ + 4 * (16 * mb + 4 * g));
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int r = 0; r < 4; ++r) O[mb][hf][r] *= e4[r];
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int s = 0; s <= (mb >> 1); ++s) {
          // P: row 16 mb + m, pieces 8 s + g and 8 s + 4 + g
          const u32x4 pa = cat(lds_load_b64(bT[2 * s] + (kOffP - kOffA) + 16 * 128 * mb),
                               lds_load_b64(bT[2 * s + 1] + (kOffP - kOffA) + 16 * 128 * mb));
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) O[mb][hf] = T::mfma16x16x32(pa, bd[s][hf], O[mb][hf]);
        }
      const auto ro = make_rsrc(a.out + static_cast<int64_t>(c0) * a.o_rs + hv * kD * 2,
                                static_cast<uint32_t>((ck - 1) * a.o_rs + kD * 2));
      // row t = 16 mb + 4 g + r: the lane's part in the vector offset, the
      // rest (uniform) in the scalar one; rows past the sequence fall outside
      // the descriptor
      const int ors = static_cast<int>(a.o_rs);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int voff = 4 * g * ors + 2 * (32 * wv + 16 * hf + m);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            __builtin_amdgcn_raw_buffer_store_b16(T::from_float(O[mb][hf][r]), ro, voff, (16 * mb + r) * ors, 0);
      }
    }
    // ---- S^T <- exp(G_C) S^T + K^T diag(exp(G_C - G)) D, this wave's columns.
    {
      const float eC = ldf(LEG + 4 * (ck - 1));
#pragma unroll
      for (int kb = 0; kb < 8; ++kb) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) S[kb][hf] *= eC;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const u32x4 ka = kt_op(bKT[kb >> 1], kb & 1, s);
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) S[kb][hf] = T::mfma16x16x32(ka, bt[s][hf], S[kb][hf]);
        }
      }
    }
    lds_sync();  // the next chunk overwrites K, Q, V, A, P; every read of this chunk's is done
  }
  if (has) {
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) *state_at(kb, hf) = S[kb][hf];
  }
}

}  // namespace

// Launches the chunked prefill over GdnArgs-style arguments (see
// nq_gdn_prefill in gdn_decode.hip, which validates them).
int launch_gdn_chunk_prefill(const void *q, int64_t q_rs, const void *k, int64_t k_rs, const void *v, int64_t v_rs,
                             const void *a, int64_t a_rs, const void *b, int64_t b_rs, const float *A_log,
                             const float *dt_bias, const int32_t *cu, int num_seqs, float *state,
                             const int32_t *idx, int64_t num_slots, int from_slot, void *out, int64_t o_rs, int H,
                             int HV, int dtype, hipStream_t s) {
  ChunkArgs c{};
  c.q = static_cast<const uint8_t *>(q);
  c.k = static_cast<const uint8_t *>(k);
  c.v = static_cast<const uint8_t *>(v);
  c.q_rs = q_rs;
  c.k_rs = k_rs;
  c.v_rs = v_rs;
  c.a = static_cast<const uint8_t *>(a);
  c.b = static_cast<const uint8_t *>(b);
  c.a_rs = a_rs;
  c.b_rs = b_rs;
  c.A_log = A_log;
  c.dt_bias = dt_bias;
  c.state = state;
  c.idx = idx;
  c.num_slots = num_slots;
  c.out = static_cast<uint8_t *>(out);
  c.o_rs = o_rs;
  c.cu = cu;
  c.H = H;
  c.HV = HV;
  c.num_seqs = num_seqs;
  c.from_slot = from_slot;
  c.eps = 1e-6f;
  c.scale = 1.0f / sqrtf(static_cast<float>(kD));
  dim3 grid(HV, num_seqs);
  if (dtype == NQ_BF16)
    gdn_chunk_kernel<BF16><<<grid, kThreads, kLds, s>>>(c);
  else
    gdn_chunk_kernel<F16><<<grid, kThreads, kLds, s>>>(c);
  return check_launch("gdn_prefill");
}

}  // namespace nq
