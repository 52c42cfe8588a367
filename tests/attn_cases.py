"""Seeded synthetic inputs of the attention tests (shared with bench.py through nanovllm_amd.engine.synthetic:
paged KV caches with randomly permuted block tables, queries; Qwen3 shapes, block size 256) and the error
statistics the tolerance checks print."""
import torch

from nanovllm_amd.engine.synthetic import BLOCK, paged_cache, queries  # noqa: F401


def error_stats(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    diff = (got.float().cpu() - ref.float().cpu()).abs()
    return diff.max().item(), diff.mean().item()
