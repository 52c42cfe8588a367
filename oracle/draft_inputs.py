"""Oracle for the draft loop's per-step input building. Test infrastructure only.

Restates nanovllm/engine/model_runner.py:443-452 (ModelRunner.run_draft, steps j = 1 .. k-1) on the CPU with
the same PyTorch operations: a sequence is real when the first draft step's context length is > 0; its
step-j position is last_pos + j (last_pos = position N-1 of the first step, :444), the slot is looked up
through the block table, the context length is position + 1; padding sequences get position 0, slot -1 and
context length 0; input_ids is zero except rows [0, S), which take the last sampled tokens (:440, :452).
"""
import torch


def draft_step_inputs(real_lens: torch.Tensor, last_pos: torch.Tensor, block_tables: torch.Tensor,
                      block_size: int, tokens: torch.Tensor, j: int):
    """(input_ids int64 [B], positions int64 [B], slot_mapping int32 [B], context_lens int32 [B]) of draft
    step j (model_runner.py:446-452). real_lens int32 [B] (the first step's context_lens), last_pos int64 [B],
    block_tables int32 [B, W], tokens int64 [S] (S <= B)."""
    real = real_lens > 0
    pos = torch.where(real, last_pos + j, 0)
    block = block_tables.gather(1, (pos // block_size).unsqueeze(1)).squeeze(1)
    slot_mapping = torch.where(real, block * block_size + pos % block_size, -1).to(torch.int32)
    context_lens = torch.where(real, pos + 1, 0).to(torch.int32)
    input_ids = torch.zeros(real_lens.size(0), dtype=torch.int64)
    input_ids[:tokens.size(0)] = tokens
    return input_ids, pos, slot_mapping, context_lens
