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
  int H, HV, from_slot;
  float eps, scale;
};

// LDS layout (bytes).
constexpr int kTile = kC * kD * 2;           // 64 x 128 16-bit values
constexpr int kOffK = 0;                     // K (unit keys), swz_c
constexpr int kOffQ = kOffK + kTile;         // Q (scaled unit queries), swz_r; then the output tile
constexpr int kOffV = kOffQ + kTile;         // V, swz_c; then D
constexpr int kOffS = kOffV + kTile;         // S, 16-bit [V][K], swz_r
constexpr int kTfStride = 68;                // floats per row of the fp32 64x64 matrix
constexpr int kOffT = kOffS + kD * kD * 2;   // A, then T (fp32 64 x 68)
constexpr int kOffTw = kOffT + kC * kTfStride * 4;
constexpr int kOffTu = kOffTw + kC * kC * 2;  // 64 x 64 16-bit, swz_6
constexpr int kOffP = kOffTu + kC * kC * 2;
constexpr int kOffG = kOffP + kC * kC * 2;    // G[64], beta[64] (fp32)
constexpr int kOffM = kOffG + 2 * kC * 4;     // 3 x 16 x 16 fp32: one product M per block column of the inverse
constexpr int kOffY = kOffM + 3 * 256 * 4;    // Y = K S^T, 64 x 128 16-bit, swz_c
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

// Accumulator element r of lane l: row (r & 3) + 4 (l / 32) + 8 (r / 4), column l % 32.
__device__ inline int acc_row(int r, int lane) { return (r & 3) + 4 * (lane >> 5) + 8 * (r >> 2); }

__device__ inline float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }

template <class T>
__device__ inline f32x4 unpack2x2(uint32_t w0, uint32_t w1) {
  return f32x4{T::to_float(w0 & 0xffffu), T::to_float(w0 >> 16), T::to_float(w1 & 0xffffu), T::to_float(w1 >> 16)};
}

// 16-bit copy of a wave's state blocks (value rows 32 vb .. +31, key
// columns 32 kb0 .. +63) into the S tile.
template <class T>
__device__ inline void write_state(uint32_t s_base, const f32x16 (&S)[2], int vb, int kb0, int lane) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int v = 32 * vb + acc_row(r, lane), kc = 32 * (kb0 + j) + (lane & 31);
      st16(a128(s_base, v, kc >> 3, false) + 2 * (kc & 7), T::from_float(S[j][r]));
    }
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
                 LTu = L + kOffTu, LP = L + kOffP, LG = L + kOffG, LB = L + kOffG + kC * 4, LM = L + kOffM,
                 LY = L + kOffY;
  const int tid0 = threadIdx.x, wave = tid0 >> 6;
  const int hv = blockIdx.x, n = blockIdx.y;
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
  auto fetch = [&](int c0, int tid) {
    const int r = tid >> 3, e = tid & 7;
    const bool ok = r < t1 - c0;
    const int64_t t = c0 + r;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = 16 * e + 8 * j;
      qv[j] = ok ? *reinterpret_cast<const u32x4 *>(a.q + t * a.q_rs + (h * kD + col) * 2) : u32x4{0, 0, 0, 0};
      kv[j] = ok ? *reinterpret_cast<const u32x4 *>(a.k + t * a.k_rs + (h * kD + col) * 2) : u32x4{0, 0, 0, 0};
      vv[j] = ok ? *reinterpret_cast<const u32x4 *>(a.v + t * a.v_rs + (hv * kD + col) * 2) : u32x4{0, 0, 0, 0};
    }
    if (tid < 64) {
      const int64_t tg = c0 + tid;
      gab = tid < t1 - c0 ? (static_cast<uint32_t>(reinterpret_cast<const uint16_t *>(a.a + tg * a.a_rs)[hv]) |
                             (static_cast<uint32_t>(reinterpret_cast<const uint16_t *>(a.b + tg * a.b_rs)[hv]) << 16))
                          : 0u;
    }
  };
  if (t1 > t0) fetch(t0, tid0);
  for (int c0 = t0; c0 < t1; c0 += kC) {
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
#pragma unroll
      for (int off = 1; off < 8; off <<= 1) {
        sq += __shfl_xor(sq, off, 64);
        sk += __shfl_xor(sk, off, 64);
      }
      const float rq = a.scale / sqrtf(sq + a.eps), rk = 1.0f / sqrtf(sk + a.eps);
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
    if (wave == 0) {
      float g = 0.f, beta = 0.f;
      if (lane < ck) {
        const float ga = T::to_float(static_cast<uint16_t>(gab & 0xffffu));
        const float gb = T::to_float(static_cast<uint16_t>(gab >> 16));
        g = neg_a * softplus(ga + dtb);
        beta = 1.0f / (1.0f + expf(-gb));
      }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(g, off, 64);
        if (lane >= off) g += y;
      }
      stf(LG + 4 * lane, g);
      stf(LB + 4 * lane, beta);
    }
    if (c0 + kC < t1) fetch(c0 + kC, tid);  // in flight while this chunk computes
    lds_sync();

    // ---- waves 0-3: K K^T -> A (fp32); waves 4-7: Q K^T -> P (16-bit);
    // block (bm, bn) = ((w / 2) % 2, w % 2).
    {
      const int bm = (wave >> 1) & 1, bn = wave & 1;
      const bool qk = wave >= 4;
      f32x16 acc = f32x16{};
#pragma unroll
      for (int s = 0; s < kD / 16; ++s) {
        const u32x4 kb = row_op(LK, 32 * bn, s, lane, true);
        const u32x4 ab = qk ? row_op(LQ, 32 * bm, s, lane, false) : row_op(LK, 32 * bm, s, lane, true);
        acc = T::mfma32x32x16(ab, kb, acc);
      }
      const int j = 32 * bn + (lane & 31);
      const float Gj = ldf(LG + 4 * j);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * bm + acc_row(r, lane);
        const float Gi = ldf(LG + 4 * i);
        const float dec = __expf(j <= i ? Gi - Gj : 0.f);
        if (qk)
          st16(a64(LP, i, j >> 3) + 2 * (j & 7), T::from_float(j <= i ? dec * acc[r] : 0.f));
        else
          stf(LT + 4 * (i * kTfStride + j), j < i ? ldf(LB + 4 * i) * dec * acc[r] : 0.f);
      }
    }
    lds_sync();

    // ---- waves 0-3: the four 16x16 diagonal blocks of T = (I + A)^-1 by
    // forward substitution (lane = column); waves 4-7: Y = K S^T (to LDS)
    // and O = diag(exp(G)) Q S^T for value columns 32 (w - 4) .. +31.
    f32x16 O[2];
    if (wave < 4) {
      if (lane < 16) {
        const int b0 = 16 * wv, c = lane;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float acc = i == c ? 1.f : 0.f;
#pragma unroll
          for (int j4 = 0; j4 < i; j4 += 4) {
            const f32x4 av = ldf4(LT + 4 * ((b0 + i) * kTfStride + b0 + j4));
#pragma unroll
            for (int j = j4; j < j4 + 4 && j < i; ++j) acc -= av[j - j4] * x[j];
          }
          x[i] = i < c ? 0.f : acc;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) stf(LT + 4 * ((b0 + i) * kTfStride + b0 + c), x[i]);
      }
    } else {
      const int bn = wave - 4;
      f32x16 Y[2] = {f32x16{}, f32x16{}};
      O[0] = f32x16{};
      O[1] = f32x16{};
#pragma unroll
      for (int s = 0; s < kD / 16; ++s) {
        const u32x4 sb = row_op(LS, 32 * bn, s, lane, false);  // S^T operand: row v, columns K
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) {
          Y[bm] = T::mfma32x32x16(row_op(LK, 32 * bm, s, lane, true), sb, Y[bm]);
          O[bm] = T::mfma32x32x16(row_op(LQ, 32 * bm, s, lane, false), sb, O[bm]);
        }
      }
      const int v = 32 * bn + (lane & 31);
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * bm + acc_row(r, lane);
          st16(a128(LY, t, v >> 3, true) + 2 * (v & 7), T::from_float(Y[bm][r]));
          O[bm][r] *= __expf(ldf(LG + 4 * t));
        }
    }
    lds_sync();
    // Off-diagonal blocks of T, one block column per wave (waves 0-2):
    // wave bj forms T_{bi,bj} = -T_{bi,bi} sum_{kb = bj}^{bi - 1} A_{bi,kb} T_{kb,bj}
    // for bi = bj + 1 .. 3 as float32 products (v_mfma_f32_16x16x4f32).
    // Every operand is a diagonal block, a block of A or an earlier block of
    // the wave's own column, so the block rows need no barrier.  T_{bi,bj} is
    // stored at block position (bj, bi) of the array (its unused upper
    // triangle): A's lower blocks, operands of the other columns, stay intact.
    if (wave < 3) {
      const int bj = wv;
      auto blk = [&](int r, int c) { return LT + 4 * (16 * r * kTfStride + 16 * c); };
      // acc + X Y for 16x16 float32 blocks X, Y (row strides xs, ys floats):
      // k-slice q takes X[l % 16][4q + l / 16] and Y[4q + l / 16][l % 16].
      auto prod = [&](uint32_t x, int xs, uint32_t y, int ys, f32x4 acc) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float av = ldf(x + 4 * ((lane & 15) * xs + 4 * q + (lane >> 4)));
          const float bv = ldf(y + 4 * ((4 * q + (lane >> 4)) * ys + (lane & 15)));
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
        }
        return acc;
      };
      const uint32_t lm = LM + 4 * 256 * bj;
#pragma unroll
      for (int bi = 1; bi < 4; ++bi) {
        if (bi <= bj) continue;
        f32x4 m = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int kb = 0; kb < bi; ++kb)
          if (kb >= bj) m = prod(blk(bi, kb), kTfStride, kb == bj ? blk(bj, bj) : blk(bj, kb), kTfStride, m);
        // M (accumulator element r of lane l: row 4 (l / 16) + r, column
        // l % 16) through LDS into operand layout; the wave's own write and
        // read, in order.
#pragma unroll
        for (int r = 0; r < 4; ++r) stf(lm + 4 * ((4 * (lane >> 4) + r) * 16 + (lane & 15)), m[r]);
        const f32x4 t = prod(blk(bi, bi), kTfStride, lm, 16, f32x4{0, 0, 0, 0});
#pragma unroll
        for (int r = 0; r < 4; ++r) stf(blk(bj, bi) + 4 * ((4 * (lane >> 4) + r) * kTfStride + (lane & 15)), -t[r]);
      }
    }
    lds_sync();
    // Tw = -T diag(beta exp(G)), Tu = T diag(beta): row tid / 8, columns 8 (tid % 8) .. +7.
    {
      const int i = tid >> 3, j0 = 8 * (tid & 7);
      u32x4 ww, wu;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        float tw[2], tu[2];
#pragma unroll
        for (int z = 0; z < 2; ++z) {
          const int j = j0 + 2 * x + z;
          // T[i][j]: a diagonal block in place, an off-diagonal one at the
          // transposed block position
          const int bi_ = i >> 4, bj_ = j >> 4;
          const float tij = j > i ? 0.f
                                  : ldf(bj_ == bi_ ? LT + 4 * (i * kTfStride + j)
                                                   : LT + 4 * ((16 * bj_ + (i & 15)) * kTfStride + 16 * bi_ + (j & 15)));
          const float bj = ldf(LB + 4 * j);
          tu[z] = tij * bj;
          tw[z] = -tij * bj * __expf(ldf(LG + 4 * j));
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
      const int bm = wave >> 2, bn = wave & 3;
      f32x16 Dv = f32x16{};
#pragma unroll
      for (int s = 0; s < kC / 16; ++s) {
        Dv = T::mfma32x32x16(row_op64(LTu, 32 * bm, s, lane), col_op(LV, 32 * bn, s, lane), Dv);
        Dv = T::mfma32x32x16(row_op64(LTw, 32 * bm, s, lane), col_op(LY, 32 * bn, s, lane), Dv);
      }
      lds_sync();  // V read by every wave
      const int v = 32 * bn + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * bm + acc_row(r, lane);
        st16(a128(LV, t, v >> 3, true) + 2 * (v & 7), T::from_float(Dv[r]));
      }
    }
    lds_sync();

    // ---- waves 4-7: O += P D, 16-bit output tile where Q was.
    if (wave >= 4) {
      const int bn = wave - 4;
#pragma unroll
      for (int s = 0; s < kC / 16; ++s) {
        const u32x4 db = col_op(LV, 32 * bn, s, lane);
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) O[bm] = T::mfma32x32x16(row_op64(LP, 32 * bm, s, lane), db, O[bm]);
      }
      const int v = 32 * bn + (lane & 31);
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * bm + acc_row(r, lane);
          st16(a128(LQ, t, v >> 3, false) + 2 * (v & 7), T::from_float(O[bm][r]));
        }
    }
    // ---- S <- exp(G_C) S + (diag(exp(G_C - G)) D)^T K, this wave's blocks.
    {
      const float GC = ldf(LG + 4 * (kC - 1));
      const float eC = __expf(GC);
#pragma unroll
      for (int j = 0; j < 2; ++j) S[j] *= eC;
#pragma unroll
      for (int s = 0; s < kC / 16; ++s) {
        // A operand: value row 32 vb + l % 32, tokens 16 s + 8 (l / 32) .. +7, scaled.
        const u32x4 d = col_op(LV, 32 * vb, s, lane);
        const int tb = 16 * s + 8 * (lane >> 5);
        u32x4 da;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const float f0 = __expf(GC - ldf(LG + 4 * (tb + 2 * x))), f1 = __expf(GC - ldf(LG + 4 * (tb + 2 * x + 1)));
          da[x] = T::pack2(T::to_float(d[x] & 0xffffu) * f0, T::to_float(d[x] >> 16) * f1);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) S[j] = T::mfma32x32x16(da, col_op(LK, 32 * (kb0 + j), s, lane), S[j]);
      }
    }
    lds_sync();  // every read of S, K and D of this chunk is done; the output tile is complete
    {
      const int r = tid >> 3, e = tid & 7;
      if (r < ck) {
        uint8_t *o = a.out + static_cast<int64_t>(c0 + r) * a.o_rs + hv * kD * 2;
#pragma unroll
        for (int j = 0; j < 2; ++j)
          *reinterpret_cast<u32x4 *>(o + (16 * e + 8 * j) * 2) = lds_load_b128<0>(a128(LQ, r, 2 * e + j, false));
      }
    }
    write_state<T>(LS, S, vb, kb0, lane);
    lds_sync();  // the next chunk overwrites K, Q, V
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
