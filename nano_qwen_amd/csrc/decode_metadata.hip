// Decode-step metadata on the device (replaces the Triton
// _prepare_decode_kernel of engine/decode_init.py:6-65).
//
// One lane per scheduled sequence, written as the closed form of
// engine/decode_init.py:29-36: the new token sits at position seq_len-1, the
// context (including it) is seq_len tokens, and its cache slot is offset
// (seq_len-1) % block_size of the sequence's last block.  input_ids gathers
// the last sampled token through the persistent batch-slot indirection.
#include "nq_device.hpp"

namespace nq {
namespace {

__global__ __launch_bounds__(256) void prepare_decode_kernel(
    const int64_t *__restrict__ sampled_token_ids, const int64_t *__restrict__ batch_slots,
    const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ last_block_ids,
    int64_t *__restrict__ input_ids, int64_t *__restrict__ positions, int32_t *__restrict__ context_lens,
    int32_t *__restrict__ slot_mapping, int num_seqs, int block_size) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= num_seqs) return;
  const int32_t len = seq_lens[i];
  const int32_t last = last_block_ids[i];
  if (sampled_token_ids != nullptr && input_ids != nullptr)
    input_ids[i] = sampled_token_ids[batch_slots[i]];
  positions[i] = static_cast<int64_t>(len) - 1;
  context_lens[i] = len;
  slot_mapping[i] = last * block_size + (len - 1) % block_size;
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_prepare_decode(const int64_t *sampled_token_ids, const int64_t *batch_slots,
                                 const int32_t *seq_lens, const int32_t *last_block_ids, int64_t *input_ids,
                                 int64_t *positions, int32_t *context_lens, int32_t *slot_mapping,
                                 int num_seqs, int block_size, void *stream) {
  if (num_seqs == 0) return NQ_OK;
  if (num_seqs < 0 || block_size <= 0) return fail(NQ_EINVAL, "prepare_decode: bad sizes");
  if (!seq_lens || !last_block_ids || !positions || !context_lens || !slot_mapping)
    return fail(NQ_EINVAL, "prepare_decode: null pointer");
  if ((sampled_token_ids == nullptr) != (input_ids == nullptr) || (sampled_token_ids && !batch_slots))
    return fail(NQ_EINVAL, "prepare_decode: sampled_token_ids, batch_slots and input_ids go together");
  const int threads = 256;
  const int blocks = (num_seqs + threads - 1) / threads;
  prepare_decode_kernel<<<blocks, threads, 0, static_cast<hipStream_t>(stream)>>>(
      sampled_token_ids, batch_slots, seq_lens, last_block_ids, input_ids, positions, context_lens,
      slot_mapping, num_seqs, block_size);
  return check_launch("prepare_decode");
}
