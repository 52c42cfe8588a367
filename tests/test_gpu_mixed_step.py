"""The mixed-step graph runtime on the GPU: a 2048-token-budget mixed step (48 verify requests with k = 4 and
3 prefill chunks, Qwen3-8B shapes, 3 layers) replayed from one HIP graph per bucket gives bitwise the
outputs and KV caches of the eager per-layer calls on the unpadded metadata; the padding rows come out as
zeros; a second step with another layout in the same bucket replays the same graph."""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from nanovllm_amd.engine.mixed_step import MixedStepRunner
from nanovllm_amd.layers.attention import store_kvcache, varlen_attention
from attn_cases import BLOCK, paged_cache, queries
from test_gpu_varlen import mixed_step

pytestmark = pytest.mark.gpu

HQ, HKV, D, K = 32, 8, 128, 4
LAYERS = 3


def _requests(lq, lk, tables, nd):
    """Sequence objects (the fields mixed_batch reads) for nd decode requests then prefill chunks."""
    seqs = []
    for s, (a, c) in enumerate(zip(lq, lk)):
        blocks = [int(x) for x in tables[s, :math.ceil(c / BLOCK)].tolist()]
        if s < nd:   # decode: Lk = num_tokens + k
            n = c - K
            seqs.append(SimpleNamespace(token_ids=[7] * n, last_token=7, num_tokens=n, num_cached_tokens=n - 1,
                                        num_scheduled_tokens=1, is_prefill=False, block_table=blocks,
                                        draft_token_ids=[3] * K))
        else:        # prefill chunk: Lk = cached + scheduled
            seqs.append(SimpleNamespace(token_ids=[5] * (c + 1), last_token=5, num_tokens=c + 1,
                                        num_cached_tokens=c - a, num_scheduled_tokens=a, is_prefill=True,
                                        block_table=blocks, draft_token_ids=[]))
    return seqs


def _eager(layout, q, k, v, caches, W):
    """Per layer: store then varlen attention on the unpadded metadata (the Python entry points)."""
    n, dev = layout["n"], q.device
    cu_q = torch.tensor(layout["cu_seqlens_q"], dtype=torch.int32, device=dev)
    cu_k = torch.tensor(layout["cu_seqlens_k"], dtype=torch.int32, device=dev)
    slots = torch.tensor(layout["slot_mapping"], dtype=torch.int32, device=dev)
    S = len(layout["cu_seqlens_q"]) - 1
    tables = torch.tensor(layout["meta"][2 * (layout["S"] + 1) + layout["N"]:], dtype=torch.int32,
                          device=dev).view(layout["S"], W)[:S].contiguous()
    out = None
    for kc, vc in caches:
        store_kvcache(k[:n], v[:n], kc, vc, slots)
        out = varlen_attention(q[:n], kc, vc, cu_q, cu_k, layout["max_seqlen_q"], layout["max_seqlen_k"],
                               D ** -0.5, tables)
    return out


def test_mixed_step_graph_replays_bitwise(device):
    lq, lk = mixed_step(0)
    nd = 48
    W = math.ceil(max(lk) / BLOCK)
    kc, vc, tables = paged_cache(device, lk, HKV, D, W=W, seed=5)
    graph_caches = [(kc.clone(), vc.clone()) for _ in range(LAYERS)]
    eager_caches = [(kc.clone(), vc.clone()) for _ in range(LAYERS)]
    del kc, vc
    layers = [SimpleNamespace(k_cache=a, v_cache=b) for a, b in graph_caches]
    runner = MixedStepRunner(layers, HQ, HKV, D, D ** -0.5, block_size=BLOCK, max_num_batched_tokens=2048,
                             max_num_seqs=64, table_width=W)
    rng = np.random.default_rng(3)
    tb = tables.cpu()
    steps = [(lq, lk)]
    # a second layout in the same bucket: the same query counts, shorter contexts and cached prefixes
    lk2 = [max(c - int(rng.integers(0, 200)), a + (K if s < nd else 0) + 1) for s, (a, c) in enumerate(zip(lq, lk))]
    steps.append((lq, lk2))
    for i, (sq, sk) in enumerate(steps):
        layout = runner.prepare(_requests(sq, sk, tb, nd), K)
        n, N = layout["n"], layout["N"]
        print(f"step {i}: {n} tokens in bucket ({N}, {layout['S']})", flush=True)
        q = queries(device, N, HQ, D, seed=10 + i)
        k = queries(device, N, HKV, D, seed=20 + i)
        v = queries(device, N, HKV, D, seed=30 + i)
        runner.bufs["q"][:N] = q
        runner.bufs["k"][:N] = k
        runner.bufs["v"][:N] = v
        out = runner.run(layout).clone()
        ref = _eager(layout, q, k, v, eager_caches, W)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"step {i}: graph output differs from the eager calls"
        assert not runner.bufs["o"][n:N].any(), "padding rows must be zero"
        for l, ((gk, gv), (ek, ev)) in enumerate(zip(graph_caches, eager_caches)):
            assert torch.equal(gk, ek) and torch.equal(gv, ev), f"step {i} layer {l}: caches differ"
    assert len(runner.graphs) == 1


def test_mixed_step_eager_body_matches_graph(device):
    """The runner's eager body (use_graph=False) and a replay of its graph agree bitwise on the same step."""
    lq, lk = mixed_step(2)
    nd = 48
    W = math.ceil(max(lk) / BLOCK)
    kc, vc, tables = paged_cache(device, lk, HKV, D, W=W, seed=6)
    caches = [(kc.clone(), vc.clone()) for _ in range(2)]
    layers = [SimpleNamespace(k_cache=a, v_cache=b) for a, b in caches]
    runner = MixedStepRunner(layers, HQ, HKV, D, D ** -0.5, block_size=BLOCK, max_num_seqs=64, table_width=W)
    layout = runner.prepare(_requests(lq, lk, tables.cpu(), nd), K)
    N = layout["N"]
    runner.bufs["q"][:N] = queries(device, N, HQ, D, seed=40)
    runner.bufs["k"][:N] = queries(device, N, HKV, D, seed=41)
    runner.bufs["v"][:N] = queries(device, N, HKV, D, seed=42)
    eager = runner.run(layout, use_graph=False).clone()
    first = runner.run(layout).clone()        # records the graph (its warm-up runs the step)
    replay = runner.run(layout).clone()       # replays it
    torch.cuda.synchronize()
    assert torch.equal(eager, first) and torch.equal(eager, replay)


def test_mixed_step_with_fused_pre_attention(device):
    """pre_attn: every layer's q/k RMSNorm + rotary embedding + KV store run fused in the step's graph. Two
    steps in one bucket (the second a replay) give bitwise the outputs and caches of eager per-layer calls:
    qk_norm_rope_store on the unpadded rows, then the varlen attention."""
    from nanovllm_amd.layers.rotary_embedding import qk_norm_rope_store
    from oracle import qk_norm_rope as onr
    lq, lk = mixed_step(1)
    nd = 48
    W = math.ceil(max(lk) / BLOCK)
    kc, vc, tables = paged_cache(device, lk, HKV, D, W=W, seed=7)
    graph_caches = [(kc.clone(), vc.clone()) for _ in range(LAYERS)]
    eager_caches = [(kc.clone(), vc.clone()) for _ in range(LAYERS)]
    del kc, vc
    g = torch.Generator().manual_seed(8)
    weights = [tuple((1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16).to(device) for _ in range(2))
               for _ in range(LAYERS)]
    cs = onr.rope_cache(D, 16384, 1e6).to(device)
    layers = [SimpleNamespace(k_cache=a, v_cache=b) for a, b in graph_caches]
    runner = MixedStepRunner(layers, HQ, HKV, D, D ** -0.5, block_size=BLOCK, max_num_seqs=64, table_width=W,
                             pre_attn=(cs, weights, 1e-6))
    tb = tables.cpu()
    for i in range(2):
        layout = runner.prepare(_requests(lq, lk, tb, nd), K)
        n, N, S = layout["n"], layout["N"], layout["S"]
        qkv = queries(device, N, HQ + 2 * HKV, D, seed=50 + i).view(N, -1)
        runner.bufs["qkv"][:N] = qkv
        out = runner.run(layout).clone()
        # eager reference on the unpadded rows
        pos = torch.tensor(layout["positions"], dtype=torch.int64, device=device)
        slots = torch.tensor(layout["slot_mapping"], dtype=torch.int32, device=device)
        cu_q = torch.tensor(layout["cu_seqlens_q"], dtype=torch.int32, device=device)
        cu_k = torch.tensor(layout["cu_seqlens_k"], dtype=torch.int32, device=device)
        Sr = len(layout["cu_seqlens_q"]) - 1
        tab = torch.tensor(layout["meta"][2 * (S + 1) + N:], dtype=torch.int32, device=device).view(S, W)[:Sr]
        x = qkv[:n]
        ref = None
        for (ek, ev), (qw, kw) in zip(eager_caches, weights):
            q, _ = qk_norm_rope_store(pos, x[:, :HQ * D].view(n, HQ, D), x[:, HQ * D:(HQ + HKV) * D].view(n, HKV, D),
                                      x[:, (HQ + HKV) * D:].view(n, HKV, D), qw, kw, 1e-6, cs, ek, ev, slots,
                                      write_k=False)
            ref = varlen_attention(q, ek, ev, cu_q, cu_k, layout["max_seqlen_q"], layout["max_seqlen_k"], D ** -0.5,
                                   tab.contiguous())
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"step {i}: fused pre-attention step differs from the eager calls"
        for l, ((gk, gv), (ek, ev)) in enumerate(zip(graph_caches, eager_caches)):
            assert torch.equal(gk, ek) and torch.equal(gv, ev), f"step {i} layer {l}: caches differ"
    assert len(runner.graphs) == 1
