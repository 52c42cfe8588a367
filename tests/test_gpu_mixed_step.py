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
from nanovllm_amd.engine.synthetic import mixed_step_lengths as mixed_step, requests

pytestmark = pytest.mark.gpu

HQ, HKV, D, K = 32, 8, 128, 4
LAYERS = 3


def _requests(lq, lk, tables, nd):
    return requests(lq, lk, tables, nd, K, BLOCK)


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


class _RecordingSegment:
    """Segment i writes seeded q / k / v rows for layer i (per token, no metadata); with `record` set it also
    keeps copies of what it wrote and of bufs["o"] (layer i-1's attention output) for the oracle."""

    def __init__(self, device, n_layers, seed):
        self.L, self.record, self.seen = n_layers, False, {}
        self.qkv = [(queries(device, 2048, HQ, D, seed=seed + 3 * i), queries(device, 2048, HKV, D, seed=seed + 3 * i + 1),
                     queries(device, 2048, HKV, D, seed=seed + 3 * i + 2)) for i in range(n_layers)]

    def __call__(self, i, n, bufs):
        if self.record and i > 0:
            self.seen[("o", i - 1)] = bufs["o"][:n].clone()
        if i == self.L:
            return
        for name, src in zip("qkv", self.qkv[i]):
            bufs[name][:n].copy_(src[:n])
            if self.record:
                self.seen[(name, i)] = src[:n].clone()


def _oracle_layers(layout, seg, caches_cpu, W):
    """Per layer: oracle store of the layer's k / v rows, then oracle varlen attention of its q rows."""
    from oracle import attention as oatt
    from oracle import kvcache as okv
    n, S = layout["n"], layout["S"]
    Sr = len(layout["cu_seqlens_q"]) - 1
    cu_q = torch.tensor(layout["cu_seqlens_q"], dtype=torch.int32)
    cu_k = torch.tensor(layout["cu_seqlens_k"], dtype=torch.int32)
    slots = torch.tensor(layout["slot_mapping"], dtype=torch.int32)
    tab = torch.tensor(layout["meta"][2 * (S + 1) + layout["N"]:], dtype=torch.int32).view(S, W)[:Sr]
    outs = []
    for i, (kc, vc) in enumerate(caches_cpu):
        q, k, v = (seg.seen[(x, i)].cpu()[:n] for x in "qkv")
        okv.store_kvcache(k, v, kc, vc, slots)
        outs.append(oatt.varlen_attention(q, kc, vc, cu_q, cu_k, D ** -0.5, tab))
    return outs


@pytest.mark.parametrize("case", ["config5", "one_chunk_one_verify", "decode_only_two"])
def test_mixed_step_runner_vs_oracle(device, case):
    """MixedStepRunner with a segment callback, eager: every layer's attention output against the oracle's
    varlen attention (max-abs 2e-2, mean-abs 2e-3) and the KV caches against the oracle's store, bitwise;
    then the same step replayed from the bucket's graph equals the eager run bitwise. The small cases run in
    small buckets, whose residue work lists are short."""
    from attn_cases import error_stats
    if case == "config5":
        lq, lk = mixed_step(4)
        nd = 48
    elif case == "one_chunk_one_verify":
        lq, lk, nd = [K + 1, 37], [700, 37 + 300], 1
    else:
        lq, lk, nd = [K + 1, K + 1], [1000, 260], 2
    W = math.ceil(max(lk) / BLOCK)
    kc, vc, tables = paged_cache(device, lk, HKV, D, W=W, seed=9)
    caches = [(kc.clone(), vc.clone()) for _ in range(LAYERS)]
    caches_cpu = [(kc.cpu(), vc.cpu()) for _ in range(LAYERS)]
    layers = [SimpleNamespace(k_cache=a, v_cache=b) for a, b in caches]
    seg = _RecordingSegment(device, LAYERS, seed=60)
    runner = MixedStepRunner(layers, HQ, HKV, D, D ** -0.5, block_size=BLOCK, max_num_batched_tokens=2048,
                             max_num_seqs=64, table_width=W, segment=seg)
    layout = runner.prepare(_requests(lq, lk, tables.cpu(), nd), K)
    n, N = layout["n"], layout["N"]
    print(f"{case}: {n} tokens, {len(lq)} sequences in bucket ({N}, {layout['S']})", flush=True)
    seg.record = True
    eager = runner.run(layout, use_graph=False).clone()
    seg.record = False
    torch.cuda.synchronize()
    refs = _oracle_layers(layout, seg, caches_cpu, W)
    for i, ref in enumerate(refs):
        got = seg.seen[("o", i)][:n]
        mx, mean = error_stats(got, ref)
        print(f"  layer {i}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
        assert mx <= 2e-2 and mean <= 2e-3, (case, i, mx, mean)
    assert torch.equal(eager, seg.seen[("o", LAYERS - 1)][:n])
    for i, ((gk, gv), (ok, ov)) in enumerate(zip(caches, caches_cpu)):
        assert torch.equal(gk.cpu(), ok) and torch.equal(gv.cpu(), ov), f"layer {i}: caches differ from the oracle"
    first = runner.run(layout).clone()     # records the graph (its warm-up runs the step again: same stores)
    replay = runner.run(layout).clone()
    torch.cuda.synchronize()
    assert torch.equal(first, eager) and torch.equal(replay, eager)
    for i, ((gk, gv), (ok, ov)) in enumerate(zip(caches, caches_cpu)):
        assert torch.equal(gk.cpu(), ok) and torch.equal(gv.cpu(), ov), f"layer {i}: caches changed on replay"


def test_mixed_step_qwen3_segments_graph_equals_eager(device):
    """The piecewise step with model segments: a random-init Qwen3-8B-shaped stack (3 layers) recorded into
    the step's graph with the fused pre-attention kernel. The graph replay equals the same body run eagerly,
    bitwise, in the hidden states and in every layer's KV cache; a second step with other token ids in the
    same bucket replays the graph and again equals its eager run."""
    from nanovllm_amd.engine.qwen3_segments import Qwen3Segments
    lq, lk = mixed_step(5)
    nd = 48
    W = math.ceil(max(lk) / BLOCK)
    kc, vc, tables = paged_cache(device, lk, HKV, D, W=W, seed=11)
    graph_caches = [(kc.clone(), vc.clone()) for _ in range(LAYERS)]
    eager_caches = [(kc.clone(), vc.clone()) for _ in range(LAYERS)]
    del kc, vc
    seg = Qwen3Segments(num_layers=LAYERS, device=device, seed=3)
    mk = lambda caches: MixedStepRunner([SimpleNamespace(k_cache=a, v_cache=b) for a, b in caches], HQ, HKV, D,
                                        D ** -0.5, block_size=BLOCK, max_num_seqs=64, table_width=W, segment=seg,
                                        pre_attn=seg.pre_attn())
    graph_runner, eager_runner = mk(graph_caches), mk(eager_caches)
    layout = graph_runner.prepare(_requests(lq, lk, tables.cpu(), nd), K)
    n, N = layout["n"], layout["N"]
    g = torch.Generator(device=device).manual_seed(12)
    for step in range(2):
        ids = torch.randint(0, 151936, (N,), device=device, generator=g)
        ids[n:] = 0
        seg.input_ids[:N] = ids
        graph_runner.run(layout)
        hg = seg.hidden_out[:n].clone()
        seg.input_ids[:N] = ids
        eager_runner.run(layout, use_graph=False)
        he = seg.hidden_out[:n].clone()
        torch.cuda.synchronize()
        print(f"step {step}: {n} tokens, hidden |mean| {he.float().abs().mean().item():.3f}", flush=True)
        assert torch.isfinite(he.float()).all()
        assert torch.equal(hg, he), f"step {step}: graph hidden states differ from the eager body"
        for i, ((a, b), (c, d)) in enumerate(zip(graph_caches, eager_caches)):
            assert torch.equal(a, c) and torch.equal(b, d), f"step {step} layer {i}: caches differ"
    assert len(graph_runner.graphs) == 1
