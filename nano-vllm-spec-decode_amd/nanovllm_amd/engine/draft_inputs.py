"""Inputs of the draft model's later steps, built on the GPU in one launch.

Counterpart of the loop body of ModelRunner.run_draft (nanovllm/engine/model_runner.py:443-452): for draft step
j = 1 .. k-1 the reference derives positions, slot_mapping and context_lens from the first step's Context
with torch.where / gather / casts and copies the last sampled tokens into input_ids (about ten small
launches per step). ``draft_step_inputs`` does the same in one HIP kernel (sd_draft_step_inputs) into
caller-owned buffers, so a step's inputs can be rebuilt inside a captured graph.

Use in run_draft's loop:

    real_lens, tables = context.context_lens, context.block_tables    # the first draft step's Context
    last_pos = positions.view(B, 2)[:, 1]
    bufs = DraftStepBuffers(B, device)
    for j in range(1, k):
        input_ids, pos, slot_mapping, context_lens = draft_step_inputs(real_lens, last_pos, tables, block_size,
                                                                       tokens[-1], j, bufs)
        set_context(False, slot_mapping=slot_mapping, context_lens=context_lens, block_tables=tables)
        ...
"""
from __future__ import annotations

import torch

from nanovllm_amd import _lib


class DraftStepBuffers:
    """Output buffers of one batch shape (B sequences, padding included)."""

    def __init__(self, num_seqs: int, device) -> None:
        self.input_ids = torch.zeros(num_seqs, dtype=torch.int64, device=device)
        self.positions = torch.zeros(num_seqs, dtype=torch.int64, device=device)
        self.slot_mapping = torch.zeros(num_seqs, dtype=torch.int32, device=device)
        self.context_lens = torch.zeros(num_seqs, dtype=torch.int32, device=device)


def draft_step_inputs(real_lens: torch.Tensor, last_pos: torch.Tensor, block_tables: torch.Tensor,
                      block_size: int, tokens: torch.Tensor, j: int, out: DraftStepBuffers | None = None):
    """(input_ids int64 [B], positions int64 [B], slot_mapping int32 [B], context_lens int32 [B]) of draft step
    j, as model_runner.py:446-452 computes them. real_lens int32 [B] (> 0: a real sequence), last_pos int64
    [B], block_tables int32 [B, W], tokens int64 [S] with S <= B (the last sampled draft tokens)."""
    B = real_lens.numel()
    if not (real_lens.dtype == torch.int32 and last_pos.dtype == torch.int64 and block_tables.dtype == torch.int32
            and tokens.dtype == torch.int64):
        raise ValueError("draft_step_inputs: int32 real_lens / block_tables, int64 last_pos / tokens required")
    if last_pos.numel() != B or block_tables.dim() != 2 or block_tables.size(0) != B or tokens.numel() > B:
        raise ValueError("draft_step_inputs: shape mismatch")
    real_lens, last_pos, tokens = real_lens.contiguous(), last_pos.contiguous(), tokens.contiguous()
    block_tables = block_tables.contiguous()
    if out is None:
        out = DraftStepBuffers(B, real_lens.device)
    lib = _lib.load()
    _lib.check(lib.sd_draft_step_inputs(real_lens.data_ptr(), last_pos.data_ptr(), block_tables.data_ptr(),
                                        block_tables.size(1), block_size,
                                        tokens.data_ptr() if tokens.numel() else None, tokens.numel(), j, B,
                                        out.input_ids.data_ptr(), out.positions.data_ptr(),
                                        out.slot_mapping.data_ptr(), out.context_lens.data_ptr(),
                                        _lib.stream_of(real_lens.device)), "sd_draft_step_inputs")
    return out.input_ids, out.positions, out.slot_mapping, out.context_lens
