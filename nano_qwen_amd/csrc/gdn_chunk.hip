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
// arithmetic.  (W = T diag(beta exp(G)) K of the reference is never formed:
// W S^T = (T diag(..)) (K S^T).)
//
// One 8-wave workgroup (two waves per SIMD) per (sequence, value head) walks
// the sequence's chunks.  The state lives in MFMA accumulators (wave w owns
// value rows 32 (w / 2) .. +31 against key columns 64 (w % 2) .. +63), in
// float32 across the whole sequence, with a 16-bit copy in LDS for the
// products that read it; every product runs on v_mfma_f32_32x32x16 with
// 16-bit operands and float32 accumulation, as the reference's kernels do
// (their tl.dot operands are the input dtype).  The 64x64 triangular inverse
// runs in float32: its four 16x16 diagonal blocks on the VALU of waves 0-3
// while waves 4-7 form K S^T and Q S^T, which do not depend on it, then the
// off-diagonal blocks as float32 products (v_mfma_f32_16x16x4f32).
//
// LDS tiles are row-major with 16-byte chunks XOR-swizzled per row: tiles
// read only as row operands (ds_read_b128) use swz_r, tiles also read down
// their columns (ds_read_b64_tr_b16) use swz_c.
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kC = 64;       // tokens per chunk
constexpr int kD = 128;      // K = V
constexpr int kThreads = 512;  // 8 waves, two per SIMD

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
constexpr int kTile = kC * kD * 2;           // 64 x 128 16-bit values
constexpr int kOffK = 0;                     // K (unit keys), swz_c
constexpr int kOffQ = kOffK + kTile;         // Q (scaled unit queries), swz_r; then the output tile
constexpr int kOffV = kOffQ + kTile;         // V, swz_c; then D^T ([V][T], 128 x 64, swz_6)
constexpr int kOffS = kOffV + kTile;         // S^T, 16-bit [K][V], swz_c
constexpr int kTfStride = 68;                // floats per row of the fp32 64x64 matrix
constexpr int kOffT = kOffS + kD * kD * 2;   // A, then T (fp32 64 x 68)
constexpr int kOffTw = kOffT + kC * kTfStride * 4;
constexpr int kOffTu = kOffTw + kC * kC * 2;  // 64 x 64 16-bit, swz_6
constexpr int kOffP = kOffTu + kC * kC * 2;  // P^T [j][i], swz_6
constexpr int kGates = 4 * kC * 4;            // G, beta, exp(G), exp(G_C - G): 64 fp32 each
constexpr int kOffG = kOffP + kC * kC * 2;    // two gate sets: this chunk's and the next one's
constexpr int kOffM = kOffG + 2 * kGates;     // 4 x 16 x 16 fp32: block products of the inverse
constexpr int kOffY = kOffM + 4 * 256 * 4;    // Y^T = S K^T, [V][T] 128 x 64 16-bit, swz_6
constexpr int kLds = kOffY + kTile;
static_assert(kLds <= 160 * 1024, "LDS");

// Chunk swizzles of the 128-column tiles (16 chunks a row) and of the
// 64-column tiles (8 chunks a row, two rows per 256 bytes).
__device__ inline int swz_r(int row) { return row & 15; }
__device__ inline int swz_c(int row) { return ((row & 7) << 1) | ((row >> 3) & 1); }
__device__ inline int swz_6(int row) { return (row >> 1) & 7; }

__device__ inline uint32_t lds_addr(const uint8_t *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t *)(p)));
}
__device__ inline uint32_t a128(uint32_t base, int row, int chunk, bool colwise) {
  return base + row * 256 + ((chunk ^ (colwise ? swz_c(row) : swz_r(row))) << 4);
}
__device__ inline uint32_t a64(uint32_t base, int row, int chunk) { return base + row * 128 + ((chunk ^ swz_6(row)) << 4); }
__device__ inline void st16(uint32_t addr, uint16_t v) {
  *reinterpret_cast<__attribute__((address_space(3))) uint16_t *>(static_cast<uintptr_t>(addr)) = v;
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

// Row operand of a 32x32x16 product from a 128-column tile: lane l takes
// row r0 + l % 32, columns 16 s + 8 (l / 32) .. +7 (k-step s).
__device__ inline u32x4 row_op(uint32_t base, int r0, int s, int lane, bool colwise) {
  return lds_load_b128<0>(a128(base, r0 + (lane & 31), 2 * s + (lane >> 5), colwise));
}
__device__ inline u32x4 row_op64(uint32_t base, int r0, int s, int lane) {
  return lds_load_b128<0>(a64(base, r0 + (lane & 31), 2 * s + (lane >> 5)));
}
// Column operand from a 128-column swz_c tile: lane l takes rows
// 16 s + 8 (l / 32) .. +7 of column c0 + l % 32, by two transposing reads
// (in a 16-lane group, lane i addresses row + (i >> 2), 8-byte piece i & 3 of
// the group's 32 bytes, and receives the group's column i).
__device__ inline u32x4 col_op(uint32_t base, int c0, int s, int lane) {
  const int i = lane & 15, grp = lane >> 4;
  const int row = 16 * s + 8 * (lane >> 5) + (i >> 2);
  const int chunk = (c0 >> 3) + 2 * (grp & 1) + ((i & 3) >> 1);
  const uint32_t lo_a = a128(base, row, chunk, true) + 8 * (i & 1);
  const uint32_t hi_a = a128(base, row + 4, chunk, true) + 8 * (i & 1);
  const u32x2 lo = lds_load_tr16<0>(lo_a), hi = lds_load_tr16<0>(hi_a);
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// The same from a 64-column tile (swz_6).
__device__ inline u32x4 col_op64(uint32_t base, int c0, int s, int lane) {
  const int i = lane & 15, grp = lane >> 4;
  const int row = 16 * s + 8 * (lane >> 5) + (i >> 2);
  const int chunk = (c0 >> 3) + 2 * (grp & 1) + ((i & 3) >> 1);
  const uint32_t lo_a = a64(base, row, chunk) + 8 * (i & 1);
  const uint32_t hi_a = a64(base, row + 4, chunk) + 8 * (i & 1);
  const u32x2 lo = lds_load_tr16<0>(lo_a), hi = lds_load_tr16<0>(hi_a);
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// Accumulator element r of lane l: row (r & 3) + 4 (l / 32) + 8 (r / 4), column l % 32.
__device__ inline int acc_row(int r, int lane) { return (r & 3) + 4 * (lane >> 5) + 8 * (r >> 2); }

__device__ inline float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }

template <int CTRL, int ROW_MASK>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}
// Sum over the 8 lanes of an aligned group (xor 1, xor 2 within quads, then
// the mirrored quad); every lane of the group gets the same bits.
__device__ inline float sum8(float v) {
  v += dpp_f<0xb1, 0xf>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4e, 0xf>(v);   // quad_perm [2, 3, 0, 1]
  return v + dpp_f<0x141, 0xf>(v);  // row_half_mirror
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

// acc + X Y for 16x16 float32 blocks in LDS (row strides xs, ys floats) on
// v_mfma_f32_16x16x4f32: k-slice q takes X[l % 16][4q + l / 16] and
// Y[4q + l / 16][l % 16]; element r of lane l of the result is row
// 4 (l / 16) + r, column l % 16.
__device__ inline f32x4 prod16(uint32_t x, int xs, uint32_t y, int ys, f32x4 acc, int lane) {
  float av[4], bv[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    av[q] = ldf(x + 4 * ((lane & 15) * xs + 4 * q + (lane >> 4)));
    bv[q] = ldf(y + 4 * ((4 * q + (lane >> 4)) * ys + (lane & 15)));
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[q], bv[q], acc, 0, 0, 0);
  return acc;
}
__device__ inline void store16x16(uint32_t base, int stride, const f32x4 &v, float sign, int lane) {
#pragma unroll
  for (int r = 0; r < 4; ++r) stf(base + 4 * ((4 * (lane >> 4) + r) * stride + (lane & 15)), sign * v[r]);
}

__device__ inline void lds_store_b64(uint32_t addr, const u32x2 &v) {
  *reinterpret_cast<__attribute__((address_space(3))) u32x2 *>(static_cast<uintptr_t>(addr)) = v;
}
// 16-bit copy of a 32x32 accumulator block, transposed: element
// (m0 + acc_row(r, l), n0 + l % 32) goes to tile row n0 + l % 32, column
// m0 + acc_row(r, l).  Each lane's runs of 4 consecutive M rows become
// 8-byte writes.  The tile has 128 columns (swz_c) or 64 (swz_6).
template <class T>
__device__ inline void st_acc_t(uint32_t tile, bool c128, int m0, int n0, const f32x16 &acc, int lane) {
  const int row = n0 + (lane & 31);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = m0 + 8 * q + 4 * (lane >> 5);
    const u32x2 w = u32x2{T::pack2(acc[4 * q], acc[4 * q + 1]), T::pack2(acc[4 * q + 2], acc[4 * q + 3])};
    const uint32_t ca = c128 ? a128(tile, row, col >> 3, true) : a64(tile, row, col >> 3);
    lds_store_b64(ca + 2 * (col & 7), w);
  }
}
// 16-bit copy of a wave's state blocks (value rows 32 vb .. +31, key
// columns 32 kb0 .. +63) into the S^T tile ([K][V], swz_c).
template <class T>
__device__ inline void write_state(uint32_t s_base, const f32x16 (&S)[2], int vb, int kb0, int lane) {
#pragma unroll
  for (int j = 0; j < 2; ++j) st_acc_t<T>(s_base, true, 32 * vb, 32 * (kb0 + j), S[j], lane);
}

// Workgroup barrier after this wave's LDS writes complete, without the
// fence of __syncthreads(), which would also wait for the next chunk's
// global loads in flight and the output stores.
__device__ inline void lds_sync() {
  wait_lgkmcnt0();
  raw_barrier();
}

template <class T>
__global__ __launch_bounds__(kThreads) void gdn_chunk_kernel(const ChunkArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t L = lds_addr(smem);
  const uint32_t LK = L + kOffK, LQ = L + kOffQ, LV = L + kOffV, LS = L + kOffS, LT = L + kOffT, LTw = L + kOffTw,
                 LTu = L + kOffTu, LP = L + kOffP, LM = L + kOffM, LY = L + kOffY;
  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);  // uniform: branches on it are scalar
  const int hv = blockIdx.x;
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
      if (lane == 0) *reinterpret_cast<__attribute__((address_space(3))) int *>(static_cast<uintptr_t>(L + kOffM)) =
          static_cast<int>(__builtin_ctzll(hit));
    }
    lds_sync();
    n = __builtin_amdgcn_readfirstlane(
        *reinterpret_cast<const __attribute__((address_space(3))) int *>(static_cast<uintptr_t>(L + kOffM)));
    lds_sync();  // read by every wave before the region is reused
  }
  const int h = hv / (a.HV / a.H);
  const int t0 = a.cu[n], t1 = a.cu[n + 1];
  const int slot = a.idx[n];
  const bool has = slot >= 0 && slot < a.num_slots;
  float *st = has ? a.state + (static_cast<int64_t>(slot) * a.HV + hv) * kD * kD : nullptr;
  const float neg_a = -expf(a.A_log[hv]), dtb = a.dt_bias[hv];

  // This wave's state blocks: value rows 32 vb .. +31, key columns 32 (kb0 + j) .. +31.
  const int vb = wave >> 1, kb0 = 2 * (wave & 1);
  f32x16 S[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      S[j][r] = (has && a.from_slot) ? st[(32 * vb + acc_row(r, tid0 & 63)) * kD + 32 * (kb0 + j) + (tid0 & 31)]
                                     : 0.f;

  if (t1 > t0) write_state<T>(LS, S, vb, kb0, tid0 & 63);
  // Inputs of a chunk, fetched one chunk ahead: row tid / 8 (columns
  // 16 (tid % 8) .. +15) of q, k, v, and (wave 0) lane's gate inputs.
  u32x4 qv[2], kv[2], vv[2];
  uint32_t gab = 0;  // a (low half) and b (high half) of token lane
  // Through buffer descriptors over the chunk's rows of this head: rows past
  // the sequence are out of range and read as zeros.
  auto fetch = [&](int c0, int tid) {
    const int r = tid >> 3, e = tid & 7;
    const int rows = min(kC, t1 - c0);
    const auto rq = make_rsrc(a.q + static_cast<int64_t>(c0) * a.q_rs + h * kD * 2,
                              static_cast<uint32_t>((rows - 1) * a.q_rs + kD * 2));
    const auto rk = make_rsrc(a.k + static_cast<int64_t>(c0) * a.k_rs + h * kD * 2,
                              static_cast<uint32_t>((rows - 1) * a.k_rs + kD * 2));
    const auto rv = make_rsrc(a.v + static_cast<int64_t>(c0) * a.v_rs + hv * kD * 2,
                              static_cast<uint32_t>((rows - 1) * a.v_rs + kD * 2));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col2 = (16 * e + 8 * j) * 2;
      qv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, r * static_cast<int>(a.q_rs) + col2, 0, 0));
      kv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, r * static_cast<int>(a.k_rs) + col2, 0, 0));
      vv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, r * static_cast<int>(a.v_rs) + col2, 0, 0));
    }
    if (tid < 64) {
      const int64_t tg = c0 + tid;
      gab = tid < t1 - c0 ? (static_cast<uint32_t>(reinterpret_cast<const uint16_t *>(a.a + tg * a.a_rs)[hv]) |
                             (static_cast<uint32_t>(reinterpret_cast<const uint16_t *>(a.b + tg * a.b_rs)[hv]) << 16))
                          : 0u;
    }
  };
  // Gates of the chunk whose inputs gab holds (wave 0; lane = token): G, the
  // in-chunk inclusive sum of the log decays, beta, exp(G) and exp(G_C - G)
  // into gate set `set`.
  auto gates = [&](int ck, int set) {
    const int lane = tid0 & 63;
    const uint32_t g0 = L + kOffG + set * kGates;
    float g = 0.f, beta = 0.f;
    if (lane < ck) {
      const float ga = T::to_float(static_cast<uint16_t>(gab & 0xffffu));
      const float gb = T::to_float(static_cast<uint16_t>(gab >> 16));
      g = neg_a * softplus(ga + dtb);
      beta = 1.0f / (1.0f + expf(-gb));
    }
    g = wave_scan(g);
    // G_C = G of the chunk's last token (tokens past the sequence add 0)
    const float gc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, g), 63));
    stf(g0 + 4 * lane, g);
    stf(g0 + 4 * (kC + lane), beta);
    stf(g0 + 4 * (2 * kC + lane), __expf(g));
    stf(g0 + 4 * (3 * kC + lane), __expf(gc - g));
  };
  if (t1 > t0) {
    fetch(t0, tid0);
    if (wave == 0) gates(min(kC, t1 - t0), 0);
  }
  for (int c0 = t0; c0 < t1; c0 += kC) {
    // this chunk's gate set (the next chunk's is written during this one)
    const int gset = ((c0 - t0) / kC) & 1;
    const uint32_t LG = L + kOffG + gset * kGates, LB = LG + kC * 4, LEG = LB + kC * 4, LEC = LEG + kC * 4;
    const int ck = min(kC, t1 - c0);
    // The thread index from an instruction the compiler cannot hoist: the
    // hundreds of LDS addresses derived from it are recomputed per chunk
    // instead of each holding a register across the loop.
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wv = tid >> 6;  // the wave index for addresses (branches use the uniform `wave`)
    // ---- unit keys, scaled unit queries (float32 norms, rounded to 16
    // bits) and values into LDS; gates and their inclusive sum G.
    {
      const int r = tid >> 3, e = tid & 7;
      float fq[16], fk[16];
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x4 q0 = unpack2x2<T>(qv[j][0], qv[j][1]), q1 = unpack2x2<T>(qv[j][2], qv[j][3]);
        const f32x4 k0 = unpack2x2<T>(kv[j][0], kv[j][1]), k1 = unpack2x2<T>(kv[j][2], kv[j][3]);
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          fq[8 * j + x] = q0[x];
          fq[8 * j + 4 + x] = q1[x];
          fk[8 * j + x] = k0[x];
          fk[8 * j + 4 + x] = k1[x];
        }
      }
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        sq += fq[x] * fq[x];
        sk += fk[x] * fk[x];
      }
      sq = sum8(sq);
      sk = sum8(sk);
      const float rq = a.scale * __builtin_amdgcn_rsqf(sq + a.eps), rk = __builtin_amdgcn_rsqf(sk + a.eps);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        u32x4 wq, wk;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          wq[x] = T::pack2(fq[8 * j + 2 * x] * rq, fq[8 * j + 2 * x + 1] * rq);
          wk[x] = T::pack2(fk[8 * j + 2 * x] * rk, fk[8 * j + 2 * x + 1] * rk);
        }
        const int chunk = 2 * e + j;
        lds_store_b128(a128(LQ, r, chunk, false), wq);
        lds_store_b128(a128(LK, r, chunk, true), wk);
        lds_store_b128(a128(LV, r, chunk, true), vv[j]);
      }
    }
    if (c0 + kC < t1) fetch(c0 + kC, tid);  // in flight while this chunk computes
    lds_sync();

    // ---- waves 0-3: K K^T -> A (fp32); waves 4-7: Q K^T -> P (16-bit);
    // block (bm, bn) = ((w / 2) % 2, w % 2).  Each wave's LDS reads are
    // issued together ahead of their uses, so their latencies overlap.
    {
      const int bm = (wv >> 1) & 1, bn = wv & 1;
      f32x16 acc = f32x16{};
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {  // two halves of the 8 k-steps
        u32x4 kb[4], ab[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          kb[s4] = row_op(LK, 32 * bn, 4 * h2 + s4, lane, true);
          ab[s4] = wave < 4 ? row_op(LK, 32 * bm, 4 * h2 + s4, lane, true) : row_op(LQ, 32 * bm, 4 * h2 + s4, lane, false);
        }
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) acc = T::mfma32x32x16(ab[s4], kb[s4], acc);
      }
      // rows i = 32 bm + acc_row(r): four runs of 4 consecutive rows
      const int j = 32 * bn + (lane & 31);
      const int i0 = 32 * bm + 4 * (lane >> 5);
      const float Gj = ldf(LG + 4 * j);
      f32x4 Gi[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) Gi[q] = ldf4(LG + 4 * (i0 + 8 * q));
      if (wave < 4) {
        f32x4 Bi[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) Bi[q] = ldf4(LB + 4 * (i0 + 8 * q));
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = i0 + (r & 3) + 8 * (r >> 2);
          const float dec = __expf(j <= i ? Gi[r >> 2][r & 3] - Gj : 0.f);
          stf(LT + 4 * (i * kTfStride + j), j < i ? Bi[r >> 2][r & 3] * dec * acc[r] : 0.f);
        }
      } else {
        // P^T ([j][i], 8-byte writes), read back by columns as P D's row operand
        f32x16 pv;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = i0 + (r & 3) + 8 * (r >> 2);
          const float dec = __expf(j <= i ? Gi[r >> 2][r & 3] - Gj : 0.f);
          pv[r] = j <= i ? dec * acc[r] : 0.f;
        }
        st_acc_t<T>(LP, false, 32 * bm, 32 * bn, pv, lane);
      }
    }
    lds_sync();

    // ---- T = (I + A)^-1 in float32, by halves: T_A and T_B, the inverses of
    // the two diagonal 32x32 halves, and the lower-left half
    // X = -T_B A_BA T_A.  Waves 0 and 1 invert the diagonal 16x16 blocks
    // 2w and 2w + 1 by forward substitution (lane = block and column), then
    // the block between them, T_{2w+1,2w} = -T_{2w+1,2w+1} A_{2w+1,2w} T_{2w,2w};
    // waves 4-7 meanwhile form Y = K S^T (to LDS) and O = diag(exp(G)) Q S^T
    // for value columns 32 (w - 4) .. +31.  An off-diagonal block T_{i,j} is
    // stored at block position (j, i), the unused upper triangle, so A's
    // lower blocks stay intact.
    f32x16 O[2];
    auto blk = [&](int r, int c) { return LT + 4 * (16 * r * kTfStride + 16 * c); };
    if (wave < 2) {
      if (lane < 32) {
        const int b0 = 16 * (2 * wv + (lane >> 4)), c = lane & 15;
        float x[16];
        // four rows at a time: their A values are read together, then
        // consumed; two partial sums per row shorten the dependent chain
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 av[4][4];
#pragma unroll
          for (int ii = 0; ii < 4; ++ii)
#pragma unroll
            for (int jc = 0; jc <= g; ++jc) av[ii][jc] = ldf4(LT + 4 * ((b0 + 4 * g + ii) * kTfStride + b0 + 4 * jc));
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = 4 * g + ii;
            float acc0 = i == c ? 1.f : 0.f, acc1 = 0.f;
#pragma unroll
            for (int j = 0; j < i; ++j) {
              if (j & 1)
                acc1 -= av[ii][j >> 2][j & 3] * x[j];
              else
                acc0 -= av[ii][j >> 2][j & 3] * x[j];
            }
            x[i] = i < c ? 0.f : acc0 + acc1;
          }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) stf(LT + 4 * ((b0 + i) * kTfStride + b0 + c), x[i]);
      }
      // the wave's own LDS writes and reads, in order
      const int d = 2 * wv;
      const uint32_t lm = LM + 4 * 256 * wv;
      store16x16(lm, 16, prod16(blk(d + 1, d), kTfStride, blk(d, d), kTfStride, f32x4{0, 0, 0, 0}, lane), 1.f, lane);
      store16x16(blk(d, d + 1), kTfStride, prod16(blk(d + 1, d + 1), kTfStride, lm, 16, f32x4{0, 0, 0, 0}, lane), -1.f,
                 lane);
    } else if (wave >= 4) {
      const int bn = wv - 4;
      f32x16 Y[2] = {f32x16{}, f32x16{}};
      O[0] = f32x16{};
      O[1] = f32x16{};
      // operands of two k-steps at a time, read ahead of their products
#pragma unroll
      for (int s = 0; s < kD / 16; s += 2) {
        u32x4 sb[2], kr[2][2], qr[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          sb[u] = col_op(LS, 32 * bn, s + u, lane);  // S^T operand: keys of column v of the [K][V] tile
#pragma unroll
          for (int bm = 0; bm < 2; ++bm) {
            kr[u][bm] = row_op(LK, 32 * bm, s + u, lane, true);
            qr[u][bm] = row_op(LQ, 32 * bm, s + u, lane, false);
          }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int bm = 0; bm < 2; ++bm) {
            Y[bm] = T::mfma32x32x16(kr[u][bm], sb[u], Y[bm]);
            O[bm] = T::mfma32x32x16(qr[u][bm], sb[u], O[bm]);
          }
      }
      // exp(G) of the rows: runs of 4 consecutive tokens at 8q + 4 (l / 32)
      f32x4 eg[2][4];
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
#pragma unroll
        for (int q = 0; q < 4; ++q) eg[bm][q] = ldf4(LEG + 4 * (32 * bm + 8 * q + 4 * (lane >> 5)));
#pragma unroll
      for (int bm = 0; bm < 2; ++bm) {
        st_acc_t<T>(LY, false, 32 * bm, 32 * bn, Y[bm], lane);  // Y^T: [V][T]
#pragma unroll
        for (int r = 0; r < 16; ++r) O[bm][r] *= eg[bm][r >> 2][r & 3];
      }
    }
    lds_sync();
    // Lower-left half: waves 0-3 each own block (p, q) = (2 + w / 2, w % 2),
    // Y_pq = sum_r A_{p,r} T_{r,q} (r = q, 1), then X_pq = -sum_r T_{p,r} Y_{r,q}
    // (r = 2 .. p).
    if (wave < 4) {
      const int p = 2 + (wv >> 1), q = wv & 1;
      f32x4 y = prod16(blk(p, 1), kTfStride, q == 1 ? blk(1, 1) : blk(0, 1), kTfStride, f32x4{0, 0, 0, 0}, lane);
      if (q == 0) y = prod16(blk(p, 0), kTfStride, blk(0, 0), kTfStride, y, lane);
      store16x16(LM + 4 * 256 * wv, 16, y, 1.f, lane);
    }
    lds_sync();
    if (wave < 4) {
      const int p = 2 + (wv >> 1), q = wv & 1;
      // Y_{2,q} is block q of LM, Y_{3,q} block 2 + q
      f32x4 x = prod16(p == 2 ? blk(2, 2) : blk(2, 3), kTfStride, LM + 4 * 256 * q, 16, f32x4{0, 0, 0, 0}, lane);
      if (p == 3) x = prod16(blk(3, 3), kTfStride, LM + 4 * 256 * (2 + q), 16, x, lane);
      store16x16(blk(q, p), kTfStride, x, -1.f, lane);
    }
    lds_sync();
    // Tw = -T diag(beta exp(G)), Tu = T diag(beta): row tid / 8, columns 8 (tid % 8) .. +7,
    // which lie in one block of T: a diagonal block in place (zero above its
    // diagonal), a lower one at the transposed block position, an upper one
    // zero.
    {
      const int i = tid >> 3, j0 = 8 * (tid & 7);
      const int bi_ = i >> 4, bj_ = j0 >> 4;
      const uint32_t src = bj_ == bi_ ? LT + 4 * (i * kTfStride + j0)
                                      : LT + 4 * ((16 * bj_ + (i & 15)) * kTfStride + 16 * bi_ + (j0 & 15));
      f32x4 t4[2] = {ldf4(src), ldf4(src + 16)};
      if (bj_ > bi_) t4[0] = t4[1] = f32x4{0, 0, 0, 0};
      const f32x4 b4[2] = {ldf4(LB + 4 * j0), ldf4(LB + 4 * j0 + 16)};
      const f32x4 e4[2] = {ldf4(LEG + 4 * j0), ldf4(LEG + 4 * j0 + 16)};
      u32x4 ww, wu;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        float tw[2], tu[2];
#pragma unroll
        for (int z = 0; z < 2; ++z) {
          const int e = 2 * x + z;
          const float tb = t4[e >> 2][e & 3] * b4[e >> 2][e & 3];
          tu[z] = tb;
          tw[z] = -tb * e4[e >> 2][e & 3];
        }
        ww[x] = T::pack2(tw[0], tw[1]);
        wu[x] = T::pack2(tu[0], tu[1]);
      }
      lds_store_b128(a64(LTw, i, j0 >> 3), ww);
      lds_store_b128(a64(LTu, i, j0 >> 3), wu);
    }
    lds_sync();

    // ---- D = Tu V + Tw Y: block (bm, bn) = (w / 4, w % 4); D takes V's place.
    {
      const int bm = wv >> 2, bn = wv & 3;
      f32x16 Dv = f32x16{};
      u32x4 tu[4], tw[4], vc[4], yc[4];
#pragma unroll
      for (int s = 0; s < kC / 16; ++s) {
        tu[s] = row_op64(LTu, 32 * bm, s, lane);
        vc[s] = col_op(LV, 32 * bn, s, lane);
        tw[s] = row_op64(LTw, 32 * bm, s, lane);
        yc[s] = row_op64(LY, 32 * bn, s, lane);
      }
#pragma unroll
      for (int s = 0; s < kC / 16; ++s) {
        Dv = T::mfma32x32x16(tu[s], vc[s], Dv);
        Dv = T::mfma32x32x16(tw[s], yc[s], Dv);
      }
      lds_sync();  // V read by every wave
      st_acc_t<T>(LV, false, 32 * bm, 32 * bn, Dv, lane);  // D^T: [V][T]
    }
    lds_sync();

    // ---- waves 4-7: O += P D, stored as 16-bit values straight from the
    // accumulators (rows past the sequence fall outside the descriptor).
    if (wave >= 4) {
      const int bn = wv - 4;
      u32x4 db[4], pr[4][2];
#pragma unroll
      for (int s = 0; s < kC / 16; ++s) {
        db[s] = row_op64(LV, 32 * bn, s, lane);
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) pr[s][bm] = col_op64(LP, 32 * bm, s, lane);
      }
#pragma unroll
      for (int s = 0; s < kC / 16; ++s)
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) O[bm] = T::mfma32x32x16(pr[s][bm], db[s], O[bm]);
      const auto ro = make_rsrc(a.out + static_cast<int64_t>(c0) * a.o_rs + hv * kD * 2,
                                static_cast<uint32_t>((ck - 1) * a.o_rs + kD * 2));
      // row t = 32 bm + (r & 3) + 8 (r >> 2) + 4 (l / 32): the lane's part in the
      // vector offset, the rest (uniform) in the scalar one
      const int ors = static_cast<int>(a.o_rs);
      const int voff = 4 * (lane >> 5) * ors + 2 * (32 * bn + (lane & 31));
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          __builtin_amdgcn_raw_buffer_store_b16(T::from_float(O[bm][r]), ro, voff,
                                                (32 * bm + (r & 3) + 8 * (r >> 2)) * ors, 0);
    }
    // ---- S <- exp(G_C) S + (diag(exp(G_C - G)) D)^T K, this wave's blocks.
    {
      const float eC = ldf(LEG + 4 * (kC - 1));
#pragma unroll
      for (int j = 0; j < 2; ++j) S[j] *= eC;
      // two k-steps at a time: operands and factors read ahead of the products
#pragma unroll
      for (int s = 0; s < kC / 16; s += 2) {
        u32x4 d[2], kc[2][2];
        f32x4 f[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          // A operand: value row 32 vb + l % 32, tokens 16 (s + u) + 8 (l / 32) .. +7, scaled.
          d[u] = row_op64(LV, 32 * vb, s + u, lane);
          const int tb = 16 * (s + u) + 8 * (lane >> 5);
          f[u][0] = ldf4(LEC + 4 * tb);
          f[u][1] = ldf4(LEC + 4 * (tb + 4));
#pragma unroll
          for (int j = 0; j < 2; ++j) kc[u][j] = col_op(LK, 32 * (kb0 + j), s + u, lane);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          u32x4 da;
#pragma unroll
          for (int x = 0; x < 4; ++x)
            da[x] = T::pack2(T::to_float(d[u][x] & 0xffffu) * f[u][x >> 1][2 * (x & 1)],
                             T::to_float(d[u][x] >> 16) * f[u][x >> 1][2 * (x & 1) + 1]);
#pragma unroll
          for (int j = 0; j < 2; ++j) S[j] = T::mfma32x32x16(da, kc[u][j], S[j]);
        }
      }
    }
    // wave 0: the next chunk's gates (its inputs arrived with the prefetch),
    // into the other gate set, while waves 4-7 finish the output
    if (wave == 0 && c0 + kC < t1) gates(min(kC, t1 - c0 - kC), gset ^ 1);
    // The S^T tile was last read by the Y and Q S^T products, barriers ago.
    write_state<T>(LS, S, vb, kb0, lane);
    lds_sync();  // the next chunk overwrites K, Q, V; every read of K and D of this chunk is done
  }
  if (has) {
    const int lane = tid0 & 63;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) st[(32 * vb + acc_row(r, lane)) * kD + 32 * (kb0 + j) + (lane & 31)] = S[j][r];
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
