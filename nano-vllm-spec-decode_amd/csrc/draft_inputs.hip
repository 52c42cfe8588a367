// Inputs of one later draft step (nanovllm/engine/model_runner.py:443-452, run_draft steps j = 1 .. k-1) in
// one launch, in place of the reference's chain of small tensor operations (where, gather, two casts, a
// slice copy). One thread per sequence; every output element is written, so the buffers can be reused by
// a captured graph without clearing.
#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {
namespace {

__global__ __launch_bounds__(256) void draft_step_inputs(const int32_t* __restrict__ real_lens,
                                                         const int64_t* __restrict__ last_pos,
                                                         const int32_t* __restrict__ block_tables, int32_t width,
                                                         int32_t block_size, const int64_t* __restrict__ tokens,
                                                         int32_t num_tokens, int32_t step, int32_t num_seqs,
                                                         int64_t* __restrict__ input_ids,
                                                         int64_t* __restrict__ positions,
                                                         int32_t* __restrict__ slot_mapping,
                                                         int32_t* __restrict__ context_lens) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= num_seqs) return;
  const bool real = real_lens[b] > 0;
  const int64_t pos = real ? last_pos[b] + step : 0;
  // torch's floor division and remainder (block_size > 0): the table column and the offset in the block.
  int64_t col = pos / block_size, off = pos % block_size;
  if (off < 0) {
    off += block_size;
    col -= 1;
  }
  int64_t slot = -1;
  if (real && col >= 0 && col < width) slot = (int64_t)block_tables[(int64_t)b * width + col] * block_size + off;
  positions[b] = pos;
  slot_mapping[b] = (int32_t)slot;
  context_lens[b] = real ? (int32_t)(pos + 1) : 0;
  input_ids[b] = b < num_tokens ? tokens[b] : 0;
}

}  // namespace
}  // namespace sd

using namespace sd;

extern "C" int sd_draft_step_inputs(const int32_t* real_lens, const int64_t* last_positions,
                                    const int32_t* block_tables, int32_t table_width, int32_t block_size,
                                    const int64_t* tokens, int32_t num_tokens, int32_t step, int32_t num_seqs,
                                    int64_t* input_ids, int64_t* positions, int32_t* slot_mapping,
                                    int32_t* context_lens, void* stream) {
  const char* who = "sd_draft_step_inputs";
  if (num_seqs < 0 || num_tokens < 0 || num_tokens > num_seqs || table_width <= 0 || block_size <= 0)
    return fail(kBadArgument, "%s: bad sizes (seqs %d, tokens %d, table width %d, block_size %d)", who, num_seqs,
                num_tokens, table_width, block_size);
  if (num_seqs == 0) return kOk;
  if (!real_lens || !last_positions || !block_tables || (num_tokens > 0 && !tokens) || !input_ids || !positions ||
      !slot_mapping || !context_lens)
    return fail(kBadArgument, "%s: null pointer", who);
  const int threads = 256;
  hipLaunchKernelGGL(draft_step_inputs, dim3((num_seqs + threads - 1) / threads), dim3(threads), 0,
                     (hipStream_t)stream, real_lens, last_positions, block_tables, table_width, block_size, tokens,
                     num_tokens, step, num_seqs, input_ids, positions, slot_mapping, context_lens);
  return check_launch(who);
}
