"""Seeded synthetic inputs of the attention tests (shared with bench.py through nanovllm_amd.engine.synthetic:
paged KV caches with randomly permuted block tables, queries; Qwen3 shapes, block size 256) and the error
statistics the tolerance checks print."""
import torch

from nanovllm_amd.engine.synthetic import BLOCK, paged_cache, queries  # noqa: F401


def error_stats(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    diff = (got.float().cpu() - ref.float().cpu()).abs()
    return diff.max().item(), diff.mean().item()


def sub_cache(k_cache: torch.Tensor, v_cache: torch.Tensor, tables: torch.Tensor, rows: list[int]):
    """The blocks that sequences `rows` use, gathered into small CPU caches, with their tables renumbered
    (negative entries kept): the oracle on a sample of a large batch without copying the whole cache."""
    t = tables[rows].cpu()
    used = sorted({int(b) for b in t.flatten().tolist() if b >= 0})
    index = {b: i for i, b in enumerate(used)}
    ids = torch.tensor(used, dtype=torch.long, device=k_cache.device)
    sub_t = t.clone()
    for i in range(t.size(0)):
        for j in range(t.size(1)):
            if t[i, j] >= 0:
                sub_t[i, j] = index[int(t[i, j])]
    return k_cache[ids].cpu(), v_cache[ids].cpu(), sub_t
