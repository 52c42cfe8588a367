"""Seeded synthetic inputs shared by the attention tests and bench.py: paged KV caches with randomly
permuted block tables, as in the decode / verify and mixed-step workloads (Qwen3 shapes, block size 256)."""
import math

import torch

BLOCK = 256


def paged_cache(device, ctx, Hkv, D, W=None, bs=BLOCK, extra_blocks=4, seed=0, tail=-1):
    """Caches [NB, bs, Hkv, D] ~ N(0,1) bf16 and an int32 block table [B, W] whose used entries are a random
    permutation of the free blocks; entries past ceil(ctx/bs) hold `tail` (-1, or a stale id)."""
    g = torch.Generator(device=device).manual_seed(seed)
    nblk = [max(1, math.ceil(c / bs)) for c in ctx]
    NB = sum(nblk) + extra_blocks
    W = W or max(nblk)
    perm = torch.randperm(NB, device=device, generator=g).to(torch.int32)
    tables = torch.full((len(ctx), W), tail, dtype=torch.int32, device=device)
    at = 0
    for b, nb in enumerate(nblk):
        tables[b, :nb] = perm[at:at + nb]
        at += nb
    kc = torch.randn(NB, bs, Hkv, D, device=device, generator=g).to(torch.bfloat16)
    vc = torch.randn(NB, bs, Hkv, D, device=device, generator=g).to(torch.bfloat16)
    return kc, vc, tables


def queries(device, tokens, Hq, D, seed=1):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(tokens, Hq, D, device=device, generator=g).to(torch.bfloat16)


def error_stats(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    diff = (got.float().cpu() - ref.float().cpu()).abs()
    return diff.max().item(), diff.mean().item()
