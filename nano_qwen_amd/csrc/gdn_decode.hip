// Gated DeltaNet decode step over a pool of recurrent states (gfx950).
//
// Reference: decode_gated_delta_rule (layers/gated_delta_net.py:85-122),
// which calls FlashInfer's gated_delta_rule_decode_pretranspose once per
// sequence (models/qwen3_5.py:226-240 loops over the batch), after reading
// and before writing the sequence's state slot (layers/gated_delta_net.py:
// 168-173, 250-262).  Per sequence b and value head hv (key head
// h = hv / (HV / H)), with the state S [V, K] ("K-last") of slot
// state_indices[b]:
//   q, k  <- x / sqrt(sum(x^2) + 1e-6)            (fp32, use_qk_l2norm)
//   g      = -exp(A_log[hv]) * softplus(a + dt_bias[hv])
//   beta   = sigmoid(b)
//   S     <- exp(g) * S
//   u      = beta * (v - S k)
//   S     <- S + u k^T
//   o      = S (q * K^-1/2)
// Here one launch covers the whole batch and updates the pool in place.
//
// Prefill (nq_gdn_prefill) runs the chunked form in gdn_chunk.hip.
//
// One one-wave workgroup per (sequence, value head, slice of 2 NL state
// rows; NL = 4), K = V = 128: no workgroup barrier,
// many small workgroups, few registers.  The wave owning rows
// 2NL w .. 2NL w + 2NL - 1 reads with load i of lane l the 16 bytes at row
// 2NL w + 2i + l/32, columns 4(l%32) .. +3: every load instruction covers
// 1 KiB of contiguous state, so the 64 KiB state is read and written once,
// fully coalesced.  Each wave normalizes q and k itself from its lanes' 4
// columns (a 32-lane reduction).  A row's dot products (S k, S q) are spread
// over the 32 lanes of a half-wave and summed by a reduce-scatter
// (reduce_rows, DPP and permlane swaps); the per-row update factors go back
// to the lanes by lane reads.
#include "nq_device.hpp"

namespace nq {
// gdn_chunk.hip: the chunked (WY) prefill on MFMA.
int launch_gdn_chunk_prefill(const void *q, int64_t q_rs, const void *k, int64_t k_rs, const void *v, int64_t v_rs,
                             const void *a, int64_t a_rs, const void *b, int64_t b_rs, const float *A_log,
                             const float *dt_bias, const int32_t *cu, int num_seqs, float *state,
                             const int32_t *idx, int64_t num_slots, int from_slot, void *out, int64_t o_rs, int H,
                             int HV, int dtype, hipStream_t s);
namespace {

constexpr int kThreads = 64;
constexpr int kDim = 128;   // K = V

struct GdnArgs {
  const uint8_t *q, *k, *v;  // [B, H, K], [B, H, K], [B, HV, V] (rows of heads, dtype T)
  int64_t q_rs, k_rs, v_rs;  // bytes per token row
  const uint8_t *a, *b;      // [B, HV] (dtype T)
  int64_t a_rs, b_rs;        // bytes per token row
  const float *A_log;        // [HV]
  const float *dt_bias;      // [HV]
  float *state;              // [num_slots, HV, V, K]
  const int32_t *idx;        // [B]
  int64_t num_slots;
  uint8_t *out;              // [B, HV, V]
  int64_t o_rs;              // bytes per token row
  int H, HV;
  float eps, scale;
};

template <class T>
__device__ inline float elem(const uint8_t *p, int i) {
  return T::to_float(reinterpret_cast<const uint16_t *>(p)[i]);
}

__device__ inline float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }

// Cross-lane steps within a half-wave without the LDS crossbar: the value of
// the partner lane at step M, which differs from this lane in bit M (and,
// for M = 8 and 4, in the bits below it): l ^ 16 by a permlane swap, l ^ 15
// and l ^ 7 by DPP row_mirror and row_half_mirror, l ^ 2 and l ^ 1 by DPP
// quad permutes.  The five partners' XOR masks are independent, so a
// butterfly over them covers all 32 lanes once.
template <int CTRL>
__device__ inline float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int M>
__device__ inline float partner(float v, int lane) {
  if constexpr (M == 16) {
    // the swap returns {row 2r's value, row 2r + 1's value} of each row pair
    const auto r = __builtin_amdgcn_permlane16_swap(f2u(v), f2u(v), false, false);
    return u2f((lane & 16) ? r[0] : r[1]);
  } else if constexpr (M == 8) {
    return dpp_mov<0x140>(v);  // row_mirror
  } else if constexpr (M == 4) {
    return dpp_mov<0x141>(v);  // row_half_mirror
  } else if constexpr (M == 2) {
    return dpp_mov<0x4e>(v);  // quad_perm [2, 3, 0, 1]
  } else {
    return dpp_mov<0xb1>(v);  // quad_perm [1, 0, 3, 2]
  }
}
// Sum over the 32 lanes of a half-wave; every lane gets it.
__device__ inline float hsum32(float v, int lane) {
  v += partner<16>(v, lane);
  v += partner<8>(v, lane);
  v += partner<4>(v, lane);
  v += partner<2>(v, lane);
  return v + partner<1>(v, lane);
}

// Sum of p[i] over the 32 lanes of a half-wave, for N values i per lane
// (N = 4, 8 or 16): a reduce-scatter over lane bits 4, 3, ... (N/2 + N/4 + ...
// + 1 exchanges) leaves value i = (l >> (5 - log2 N)) & (N - 1) in lane l
// (each step keeps the half selected by the lane's bit M and adds the
// partner's other half), and the remaining steps complete the sum in those
// lanes.
template <int M, int C, int N>
__device__ inline void scatter_step(float (&p)[N], int lane) {
  if constexpr (C >= 2) {
    const bool hi = (lane & M) != 0;
#pragma unroll
    for (int j = 0; j < C / 2; ++j) {
      // Both elements are first fixed in registers: otherwise the compiler
      // turns the selects into an indexed read of p, a compare-and-select
      // chain over the whole array.
      float lo = p[j], up = p[j + C / 2];
      asm volatile("" : "+v"(lo), "+v"(up));
      const float keep = hi ? up : lo;
      const float send = hi ? lo : up;
      p[j] = keep + partner<M>(send, lane);
    }
    scatter_step<M / 2, C / 2, N>(p, lane);
  }
}
template <int M>
__device__ inline float finish_sum(float r, int lane) {
  if constexpr (M >= 1) return finish_sum<M / 2>(r + partner<M>(r, lane), lane);
  return r;
}
template <int N>
__device__ inline float reduce_rows(float (&p)[N], int lane) {
  scatter_step<16, N, N>(p, lane);
  return finish_sum<16 / N>(p[0], lane);
}

// A wave owns 2 * NL state rows (NL loads per lane); NL = 4: more, smaller
// waves hide the HBM latency better.
constexpr int kDecodeLoads = 4;
// Lane bits below the row index after reduce_rows<NL>.
template <int NL>
constexpr int kShOf = NL == 16 ? 1 : (NL == 8 ? 2 : 3);

// One token's inputs for one lane: its 4 columns of q and k, its row's v, and
// the two gate inputs (16-bit values).
struct TokIn {
  u32x2 q, k;
  uint32_t v, ga, gb;
};

template <class T>
__device__ inline TokIn load_tok(const GdnArgs &a, int64_t t, int h, int hv, int vrow, int c0) {
  TokIn in;
  in.q = *reinterpret_cast<const u32x2 *>(a.q + t * a.q_rs + (h * kDim + c0) * 2);
  in.k = *reinterpret_cast<const u32x2 *>(a.k + t * a.k_rs + (h * kDim + c0) * 2);
  in.v = reinterpret_cast<const uint16_t *>(a.v + t * a.v_rs + hv * kDim * 2)[vrow];
  in.ga = reinterpret_cast<const uint16_t *>(a.a + t * a.a_rs)[hv];
  in.gb = reinterpret_cast<const uint16_t *>(a.b + t * a.b_rs)[hv];
  return in;
}

template <class T>
__device__ inline f32x4 unpack4(const u32x2 &w) {
  return f32x4{T::to_float(w[0] & 0xffffu), T::to_float(w[0] >> 16), T::to_float(w[1] & 0xffffu),
               T::to_float(w[1] >> 16)};
}

// One token of the gated delta rule on the wave's kRowsW state rows (held in
// s), writing the token's output for those rows.  neg_a = -exp(A_log[hv]).
template <class T, int NL>
__device__ inline void gdn_token(f32x4 (&s)[NL], const TokIn &in, float neg_a, float dt_bias, float eps,
                                 float scale, int lane, int my_row, bool writer, uint16_t *orow) {
  // q and k: this lane's 4 columns, l2-normalized over the 32 lanes that
  // cover all 128 columns; q also carries the scale.
  f32x4 qc = unpack4<T>(in.q), kc = unpack4<T>(in.k);
  float sq = qc[0] * qc[0] + qc[1] * qc[1] + qc[2] * qc[2] + qc[3] * qc[3];
  float sk = kc[0] * kc[0] + kc[1] * kc[1] + kc[2] * kc[2] + kc[3] * kc[3];
  sq = hsum32(sq, lane);
  sk = hsum32(sk, lane);
  qc *= scale / sqrtf(sq + eps);
  kc *= 1.0f / sqrtf(sk + eps);
  const float decay = expf(neg_a * softplus(T::to_float(static_cast<uint16_t>(in.ga)) + dt_bias));
  const float beta = 1.0f / (1.0f + expf(-T::to_float(static_cast<uint16_t>(in.gb))));
  // u = beta * (v - (exp(g) S) k) for every row of the wave.
  float p[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    s[i] *= decay;
    p[i] = s[i][0] * kc[0] + s[i][1] * kc[1] + s[i][2] * kc[2] + s[i][3] * kc[3];
  }
  const float u = beta * (T::to_float(static_cast<uint16_t>(in.v)) - reduce_rows(p, lane));
  // S += u k^T, then o = S q.  Row 2 i + h's factor is held by every lane of
  // its group (h, i) (lane bits 5 and kSh ..): read from lane 32 h + (i << kSh).
  constexpr int kSh = kShOf<NL>;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const float u0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, u), i << kSh));
    const float u1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, u), 32 + (i << kSh)));
    const float ui = (lane >> 5) ? u1 : u0;
    s[i] += ui * kc;
    p[i] = s[i][0] * qc[0] + s[i][1] * qc[1] + s[i][2] * qc[2] + s[i][3] * qc[3];
  }
  const float o = reduce_rows(p, lane);
  if (writer) orow[my_row] = T::from_float(o);
}

// Decode: one token per sequence b (row b of q, k, v, a, b and out).
template <class T>
__global__ __launch_bounds__(kThreads) void gdn_decode_kernel(const GdnArgs a) {
  constexpr int NL = kDecodeLoads, kRowsW = 2 * NL, kSh = kShOf<NL>;
  // The slices of one state are neighbours in dispatch order, so the state's
  // 64 KiB is read and written as one run (5% faster than value-head order).
  const int w = blockIdx.x, hv = blockIdx.y, bi = blockIdx.z;
  const int lane = threadIdx.x;
  const int32_t slot = a.idx[bi];
  if (slot < 0 || slot >= a.num_slots) return;  // padded row: no state to advance
  const int h = hv / (a.HV / a.H);
  const int r0 = kRowsW * w + (lane >> 5);  // row of load 0; load i adds 2i
  const int c0 = 4 * (lane & 31);           // this lane's 4 columns
  const int my_row = 2 * ((lane >> kSh) & (NL - 1)) + (lane >> 5);  // row whose sums this lane ends with
  const bool writer = (lane & ((1 << kSh) - 1)) == 0;

  // The state loads first (coalesced), then the token's inputs.
  float *sp = a.state + ((static_cast<int64_t>(slot) * a.HV + hv) * kDim + r0) * kDim + c0;
  f32x4 s[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i)
    s[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(sp + 2 * i * kDim));
  const TokIn in = load_tok<T>(a, bi, h, hv, kRowsW * w + my_row, c0);
  uint16_t *orow = reinterpret_cast<uint16_t *>(a.out + bi * a.o_rs + hv * kDim * 2) + kRowsW * w;
  gdn_token<T, NL>(s, in, -expf(a.A_log[hv]), a.dt_bias[hv], a.eps, a.scale, lane, my_row, writer, orow);
#pragma unroll
  for (int i = 0; i < NL; ++i) __builtin_nontemporal_store(s[i], reinterpret_cast<f32x4 *>(sp + 2 * i * kDim));
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_gdn_decode(const void *q, int64_t q_row_stride, const void *k, int64_t k_row_stride,
                             const void *v, int64_t v_row_stride, const void *a, int64_t a_row_stride,
                             const void *b, int64_t b_row_stride, const float *A_log, const float *dt_bias,
                             float *state, const int32_t *state_indices, int64_t num_slots, void *out,
                             int64_t out_row_stride, int batch, int num_k_heads, int num_v_heads,
                             int head_k_dim, int head_v_dim, int dtype, void *stream) {
  if (batch < 0 || num_k_heads <= 0 || num_v_heads <= 0 || num_slots < 0)
    return fail(NQ_EINVAL, "gdn_decode: bad sizes (batch=%d heads=%d/%d)", batch, num_k_heads, num_v_heads);
  if (num_v_heads % num_k_heads != 0)
    return fail(NQ_EINVAL, "gdn_decode: value heads %d not a multiple of key heads %d", num_v_heads, num_k_heads);
  if (head_k_dim != kDim || head_v_dim != kDim)
    return fail(NQ_EUNSUPPORTED, "gdn_decode: head dims %d/%d (built: 128/128)", head_k_dim, head_v_dim);
  if (dtype != NQ_BF16 && dtype != NQ_F16) return fail(NQ_EUNSUPPORTED, "gdn_decode: dtype %d (f16/bf16)", dtype);
  if (batch == 0) return NQ_OK;
  if (!q || !k || !v || !a || !b || !A_log || !dt_bias || !state || !state_indices || !out)
    return fail(NQ_EINVAL, "gdn_decode: null pointer");
  if (!aligned(state, 16)) return fail(NQ_EINVAL, "gdn_decode: state must be 16-byte aligned");
  if (!aligned(q, 8) || !aligned(k, 8) || (q_row_stride * 2) % 8 || (k_row_stride * 2) % 8)
    return fail(NQ_EINVAL, "gdn_decode: q and k rows must be 8-byte aligned");
  if (batch > 65535 || num_v_heads > 65535) return fail(NQ_EINVAL, "gdn_decode: grid too large");
  GdnArgs g{};
  g.q = static_cast<const uint8_t *>(q);
  g.k = static_cast<const uint8_t *>(k);
  g.v = static_cast<const uint8_t *>(v);
  g.q_rs = q_row_stride * 2;
  g.k_rs = k_row_stride * 2;
  g.v_rs = v_row_stride * 2;
  g.a = static_cast<const uint8_t *>(a);
  g.b = static_cast<const uint8_t *>(b);
  g.a_rs = a_row_stride * 2;
  g.b_rs = b_row_stride * 2;
  g.A_log = A_log;
  g.dt_bias = dt_bias;
  g.state = state;
  g.idx = state_indices;
  g.num_slots = num_slots;
  g.out = static_cast<uint8_t *>(out);
  g.o_rs = out_row_stride * 2;
  g.H = num_k_heads;
  g.HV = num_v_heads;
  g.eps = 1e-6f;
  g.scale = 1.0f / sqrtf(static_cast<float>(head_k_dim));
  dim3 grid(kDim / (2 * kDecodeLoads), num_v_heads, batch);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == NQ_BF16) gdn_decode_kernel<BF16><<<grid, kThreads, 0, s>>>(g);
  else gdn_decode_kernel<F16><<<grid, kThreads, 0, s>>>(g);
  return check_launch("gdn_decode");
}

extern "C" int nq_gdn_prefill(const void *q, int64_t q_row_stride, const void *k, int64_t k_row_stride,
                              const void *v, int64_t v_row_stride, const void *a, int64_t a_row_stride,
                              const void *b, int64_t b_row_stride, const float *A_log, const float *dt_bias,
                              const int32_t *cu_seqlens, int num_seqs, float *state, const int32_t *state_indices,
                              int64_t num_slots, int initial_state_from_slot, void *out, int64_t out_row_stride,
                              int num_k_heads, int num_v_heads, int head_k_dim, int head_v_dim, int dtype,
                              void *stream) {
  if (num_seqs < 0 || num_k_heads <= 0 || num_v_heads <= 0 || num_slots < 0)
    return fail(NQ_EINVAL, "gdn_prefill: bad sizes (seqs=%d heads=%d/%d)", num_seqs, num_k_heads, num_v_heads);
  if (num_v_heads % num_k_heads != 0)
    return fail(NQ_EINVAL, "gdn_prefill: value heads %d not a multiple of key heads %d", num_v_heads, num_k_heads);
  if (head_k_dim != kDim || head_v_dim != kDim)
    return fail(NQ_EUNSUPPORTED, "gdn_prefill: head dims %d/%d (built: 128/128)", head_k_dim, head_v_dim);
  if (dtype != NQ_BF16 && dtype != NQ_F16) return fail(NQ_EUNSUPPORTED, "gdn_prefill: dtype %d (f16/bf16)", dtype);
  if (num_seqs == 0) return NQ_OK;
  if (!q || !k || !v || !a || !b || !A_log || !dt_bias || !cu_seqlens || !state || !state_indices || !out)
    return fail(NQ_EINVAL, "gdn_prefill: null pointer");
  if (!aligned(state, 16) || !aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16) ||
      (q_row_stride * 2) % 16 || (k_row_stride * 2) % 16 || (v_row_stride * 2) % 16 || (out_row_stride * 2) % 16)
    return fail(NQ_EINVAL, "gdn_prefill: state, q/k/v/out rows 16-byte alignment");
  if (num_seqs > 65535 || num_v_heads > 65535) return fail(NQ_EINVAL, "gdn_prefill: grid too large");
  return launch_gdn_chunk_prefill(q, q_row_stride * 2, k, k_row_stride * 2, v, v_row_stride * 2, a, a_row_stride * 2,
                                  b, b_row_stride * 2, A_log, dt_bias, cu_seqlens, num_seqs, state, state_indices,
                                  num_slots, initial_state_from_slot, out, out_row_stride * 2, num_k_heads, num_v_heads,
                                  dtype, static_cast<hipStream_t>(stream));
}
