// Qwen3.5 attention output gate, one in-place pass (gfx950).
//
// Reference: models/qwen3_5.py:140-142,
//   attn_output = attn_output.reshape(-1, q_size)
//   attn_output = attn_output * torch.sigmoid(gate.reshape(-1, q_size))
// two eager launches (sigmoid into a temporary, then the product into a new
// tensor) that read 3 and write 2 elements per output element; here one
// launch reads the output and the gate once and writes the output in place.  The
// decode kernel applies the same gate inside its own output store
// (nq_paged_decode_gated); this pass serves the prefill path.
//
// One lane per 8 consecutive elements of a row (16-byte accesses), rows
// addressed through (token, head) strides so the gate can stay the strided
// second half of q_proj's [N, Hq, 2*D] output.
#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kThreads = 256;

template <class T>
__global__ __launch_bounds__(kThreads) void output_gate_kernel(uint8_t *out, int64_t o_rs, int64_t o_hs,
                                                               const uint8_t *gate, int64_t g_rs, int64_t g_hs,
                                                               int heads, int chunks_per_row, int64_t total) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (c >= total) return;
  const int64_t per_tok = static_cast<int64_t>(heads) * chunks_per_row;
  const int64_t tok = c / per_tok;
  const int rem = static_cast<int>(c - tok * per_tok);
  const int h = rem / chunks_per_row;
  const int e = (rem - h * chunks_per_row) * 16;  // byte offset in the row
  uint8_t *op = out + tok * o_rs + h * o_hs + e;
  const u32x4 ov = load16(op);
  const u32x4 gv = load16(gate + tok * g_rs + h * g_hs + e);
  u32x4 w;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float o0 = T::to_float(static_cast<uint16_t>(ov[t] & 0xffffu));
    const float o1 = T::to_float(static_cast<uint16_t>(ov[t] >> 16));
    w[t] = T::pack2(gate_one<T>(o0, gv[t] & 0xffffu), gate_one<T>(o1, gv[t] >> 16));
  }
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(op));
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_output_gate(void *out, int64_t out_row_stride, int64_t out_head_stride, const void *gate,
                              int64_t gate_row_stride, int64_t gate_head_stride, int64_t num_tokens,
                              int num_heads, int head_dim, int dtype, void *stream) {
  if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 8 != 0)
    return fail(NQ_EINVAL, "output_gate: bad sizes (tokens=%lld heads=%d dim=%d)", (long long)num_tokens,
                num_heads, head_dim);
  if (dtype != NQ_BF16 && dtype != NQ_F16) return fail(NQ_EUNSUPPORTED, "output_gate: dtype %d (f16/bf16)", dtype);
  if (num_tokens == 0) return NQ_OK;
  if (!out || !gate) return fail(NQ_EINVAL, "output_gate: null pointer");
  if (!aligned(out, 16) || !aligned(gate, 16) || (out_row_stride * 2) % 16 || (out_head_stride * 2) % 16 ||
      (gate_row_stride * 2) % 16 || (gate_head_stride * 2) % 16)
    return fail(NQ_EINVAL, "output_gate: pointers and strides must be 16-byte aligned");
  const int cpr = head_dim / 8;
  const int64_t total = num_tokens * num_heads * cpr;
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffffLL) return fail(NQ_EINVAL, "output_gate: too large for one launch");
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t *o = static_cast<uint8_t *>(out);
  const uint8_t *g = static_cast<const uint8_t *>(gate);
  if (dtype == NQ_BF16)
    output_gate_kernel<BF16><<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(
        o, out_row_stride * 2, out_head_stride * 2, g, gate_row_stride * 2, gate_head_stride * 2, num_heads, cpr,
        total);
  else
    output_gate_kernel<F16><<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(
        o, out_row_stride * 2, out_head_stride * 2, g, gate_row_stride * 2, gate_head_stride * 2, num_heads, cpr,
        total);
  return check_launch("output_gate");
}
