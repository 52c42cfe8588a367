"""Per-step attention metadata, read by Attention.forward.

Same fields, defaults and functions as the reference's module-global context
(nanovllm/utils/context.py:5-28), so a model runner that sets it for the reference's Attention sets it for
this one unchanged.
"""
from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None     # int32 [nseq+1], device
    cu_seqlens_k: torch.Tensor | None = None     # int32 [nseq+1], device
    max_seqlen_q: int = 0                        # host int
    max_seqlen_k: int = 0                        # host int
    slot_mapping: torch.Tensor | None = None     # int32 [N], -1 = do not store
    context_lens: torch.Tensor | None = None     # int32 [B] (decode), 0 = padding sequence
    block_tables: torch.Tensor | None = None     # int32 [B, W], -1 padded
    logits_indices: torch.Tensor | None = None   # int64, rows the LM head computes (mixed batching)


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0, slot_mapping=None,
                context_lens=None, block_tables=None, logits_indices=None) -> None:
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, slot_mapping, context_lens,
                       block_tables, logits_indices)


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()
