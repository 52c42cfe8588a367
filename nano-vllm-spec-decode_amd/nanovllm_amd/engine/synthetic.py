"""Synthetic workloads of the attention hot path, shared by the benchmark and the tests: seeded paged KV caches
with randomly permuted block tables (block size 256, as the reference's), queries, and the request mix of a
2048-token-budget mixed step at Qwen3-8B shapes (decode requests checking k guesses, then prefill chunks
after a cached prefix), as the scheduler's schedule_mixed would hand it to the model runner
(nanovllm/engine/model_runner.py:487-535).
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np
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
    """[tokens, Hq, D] ~ N(0,1) bf16."""
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(tokens, Hq, D, device=device, generator=g).to(torch.bfloat16)


def mixed_step_lengths(seed: int, num_decode: int = 48, k: int = 4, num_chunks: int = 3, budget: int = 2048):
    """(lq, lk): per sequence, query rows and keys. num_decode decode requests come first, each with 1 + k verify
    rows and a context drawn lognormal (median 600, sigma 0.6, at most 4096 keys including the new rows); then
    num_chunks prefill chunks whose lengths are lognormal (median 220, sigma 0.5, at least 16, within what is
    left of the budget) after a cached prefix uniform in [0, 512]."""
    rnd = np.random.default_rng(seed)
    dec_ctx = np.minimum(np.exp(rnd.normal(math.log(600), 0.6, num_decode)).astype(int) + k + 1, 4096).tolist()
    left = budget - num_decode * (1 + k)
    chunks = []
    for _ in range(num_chunks):
        L = int(min(max(np.exp(rnd.normal(math.log(220), 0.5)), 16), left))
        left -= L
        prefix = int(rnd.integers(0, 513))
        chunks.append((L, prefix + L))
    lq = [1 + k] * num_decode + [a for a, _ in chunks]
    lk = dec_ctx + [b for _, b in chunks]
    return lq, lk


def requests(lq, lk, tables, num_decode: int, k: int, block_size: int):
    """Sequence objects with the fields mixed_batch reads (nanovllm_amd.engine.metadata), for num_decode decode
    requests (lk = num_tokens + k, one token cached short of num_tokens, k guesses) followed by prefill chunks
    (lk = cached + scheduled); block tables from the rows of `tables` (a [seqs, W] int tensor or array)."""
    seqs = []
    for s, (a, c) in enumerate(zip(lq, lk)):
        blocks = [int(x) for x in tables[s, :math.ceil(c / block_size)].tolist()]
        if s < num_decode:
            n = c - k
            seqs.append(SimpleNamespace(token_ids=[7] * n, last_token=7, num_tokens=n, num_cached_tokens=n - 1,
                                        num_scheduled_tokens=1, is_prefill=False, block_table=blocks,
                                        draft_token_ids=[3] * k))
        else:
            seqs.append(SimpleNamespace(token_ids=[5] * (c + 1), last_token=5, num_tokens=c + 1,
                                        num_cached_tokens=c - a, num_scheduled_tokens=a, is_prefill=True,
                                        block_table=blocks, draft_token_ids=[]))
    return seqs
