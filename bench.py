"""Benchmark of the MI355X spec-decode attention hot path (one GPU).

Headline (value): speculative-verify paged attention at Qwen3-8B shapes — 32 query / 8 KV heads, head_dim
128, bf16 KV cache in 256-token blocks, B = 64 sequences, k = 4 guesses (5 causal queries each), context
4096 — as algorithmic HBM TB/s: the bytes one call must move (every KV byte of every sequence, the queries,
the outputs, the block-table entries and context lengths) divided by the measured time. One step = one call
(one layer). Inputs are resident in HBM before the timed region. `roofline.traffic` is the HBM bytes per
launch that rocprofv3's FETCH_SIZE + WRITE_SIZE counters measured for this launch (committed summary under
profiles/), null if that summary is absent.

Also reported (same JSON line):
* the verify attention with context lengths uniform in [1024, 8192], and at B in {1, 16, 64} x k in {1, 4, 8};
* the KV-cache scatter (2048 rows, 10% padding slots);
* the fused q/k RMSNorm + RoPE + KV store over 2048 tokens, next to the reference's eager operations;
* one draft step's inputs for 64 sequences, next to the reference's tensor operations;
* the rejection sampler (S 64, K 4, V 151936, T 0 and T 1 with draft logits);
* the unfused path in front of it: the LM head as the library GEMM into bf16 logits, then the T 0 verifier;
* a 2048-token mixed prefill+decode attention step over 36 layers, replayed as one HIP graph by the mixed-step
  runtime (tok/s), its roofline fractions, the prefill kernel at GPU-filling sizes, and the whole step of a
  random-init Qwen3-8B-shaped model (36 layers run piecewise in the step's graph, then the LM head and the
  verifier);
* whole-model verify (k = 4) and plain decode steps of the same model at B in {1, 16, 64} x context {256,
  1024} (one HIP graph per step, then the LM head and the greedy decision), with the library GEMMs and with
  the row-invariant projections and norms;
* a CPU baseline: the oracle (PyTorch CPU restatement) timed on the headline workload for about 10 s on 16
  host threads.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10]
    python bench.py --only qk_norm_rope_store      (one secondary workload alone, for profiling)
"""
import argparse
import json
import math
import os
import sys
import time
import types

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "nano-vllm-spec-decode_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
HQ, HKV, D, BLOCK = 32, 8, 128, 256


def decode_bytes(ctx, n):
    """Algorithmic bytes of one verify-attention call: K and V of every visible key (Hkv*D*2 B each), the
    queries and outputs (Hq*D*2 B per row each), block-table entries and the context length."""
    per_key = 2 * HKV * D * 2
    per_row = 2 * HQ * D * 2
    return sum(per_key * c + per_row * n + 4 * math.ceil(c / BLOCK) + 4 for c in ctx)


def timed(fn, steps, warmup):
    """Runs fn warmup times, then `steps` back-to-back times between two synchronizations (the wall clock of
    that region gives seconds per step), then `steps` more times with an event pair around each call on the
    current stream (the stream every kernel of this package launches on) for the per-launch durations.
    Returns (seconds per step, [per-call event seconds])."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    ev = [s.elapsed_time(e) / 1e3 for s, e in zip(starts, ends)]
    return wall, ev


def graph_timed(fn, reps=20, replays=5):
    """Per-call GPU time of fn without host launch overhead: fn is captured `reps` times into one CUDA/HIP
    graph (after an eager warm-up call) and the graph is replayed between events. Returns seconds per call."""
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (reps * replays)


def bench_verify_attention(dev, steps, warmup, B=64, k=4, ctx_len=4096, W=33):
    import torch
    from nanovllm_amd.engine.synthetic import paged_cache, queries
    from nanovllm_amd.layers.attention import paged_decode_attention
    n = k + 1
    ctx = [ctx_len] * B
    kc, vc, tables = paged_cache(dev, ctx, HKV, D, W=W, seed=0)
    q = queries(dev, B * n, HQ, D, seed=1).view(B, n, HQ, D)
    lens = torch.tensor(ctx, dtype=torch.int32, device=dev)
    out = torch.empty(B * n, HQ, D, dtype=torch.bfloat16, device=dev)
    fn = lambda: paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5, out=out)
    wall, ev = timed(fn, steps, warmup)
    nbytes = decode_bytes(ctx, n)
    return dict(bytes=nbytes, wall_s=wall, event_s=sum(ev) / len(ev), inputs=(q, kc, vc, lens, tables))


def bench_verify_uniform(dev, B=64, k=4, lo=1024, hi=8192, W=33):
    """Spec-verify attention with context lengths uniform in [lo, hi] (seeded), through the path
    Attention.forward takes (sequences dispatched longest first, order planned once per step), graph-timed
    over calls that each read the next of 3 cache copies; also the same call unplanned (index order)."""
    import types
    import numpy as np
    import torch
    from nanovllm_amd.engine.synthetic import paged_cache, queries
    from nanovllm_amd.layers.attention import paged_decode_attention
    n = k + 1
    ctx = np.random.default_rng(0).integers(lo, hi + 1, B).tolist()
    kc, vc, tables = paged_cache(dev, ctx, HKV, D, W=W, seed=0)
    caches = [(kc, vc)] + [(kc.clone(), vc.clone()) for _ in range(2)]
    q = queries(dev, B * n, HQ, D, seed=1).view(B, n, HQ, D)
    lens = torch.tensor(ctx, dtype=torch.int32, device=dev)
    out = torch.empty(B * n, HQ, D, dtype=torch.bfloat16, device=dev)
    nbytes = decode_bytes(ctx, n)
    res = {}
    for name, owner in (("planned", types.SimpleNamespace()), ("unplanned", None)):
        turn = [0]

        def call():
            a, b = caches[turn[0] % 3]
            turn[0] += 1
            paged_decode_attention(q, a, b, lens, tables, D ** -0.5, out=out, plan_owner=owner)
        t = graph_timed(call, reps=12)
        res[name] = dict(us=round(t * 1e6, 2), GBs=round(nbytes / t / 1e9, 1), frac=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4))
    res["bytes"] = nbytes
    res["contexts"] = f"uniform [{lo}, {hi}], seed 0, B={B}, k={k}"
    return res


def bench_verify_sweep(dev, ctx_len=4096, W=33):
    """The batch / guess-count points of the verify workload at ctx 4096: B in {1, 16, 64}, k in {1, 2, 4, 8},
    through Attention.forward's path (planned order), graph-timed over calls that each read the next of
    enough cache copies to exceed the 256 MB last-level cache."""
    import types
    import torch
    from nanovllm_amd.engine.synthetic import paged_cache, queries
    from nanovllm_amd.layers.attention import paged_decode_attention
    res = {}
    for B in (64, 16, 1):  # the largest caches first, from a released allocator cache
        torch.cuda.empty_cache()
        ctx = [ctx_len] * B
        kc, vc, tables = paged_cache(dev, ctx, HKV, D, W=W, seed=0)
        copies = [(kc, vc)] + [(kc.clone(), vc.clone()) for _ in range(max(1, 300 // (17 * B)))]
        lens = torch.tensor(ctx, dtype=torch.int32, device=dev)
        for k in (1, 2, 4, 8):
            n = k + 1
            q = queries(dev, B * n, HQ, D, seed=1).view(B, n, HQ, D)
            out = torch.empty(B * n, HQ, D, dtype=torch.bfloat16, device=dev)
            owner, turn = types.SimpleNamespace(), [0]

            def call():
                a, b = copies[turn[0] % len(copies)]
                turn[0] += 1
                paged_decode_attention(q, a, b, lens, tables, D ** -0.5, out=out, plan_owner=owner)
            t = graph_timed(call, reps=len(copies) * max(1, 12 // len(copies)))  # at least 12 calls a replay
            nbytes = decode_bytes(ctx, n)
            res[f"B{B}_k{k}"] = dict(us=round(t * 1e6, 2), frac=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4))
        del kc, vc, tables, copies
        torch.cuda.empty_cache()
    res["contexts"] = f"{ctx_len} for every sequence"
    return res


def bench_store(dev, steps, warmup, N=2048, NB=4096):
    import torch
    from nanovllm_amd.layers.attention import store_kvcache
    g = torch.Generator(device=dev).manual_seed(3)
    key = torch.randn(N, HKV, D, device=dev, generator=g).to(torch.bfloat16)
    value = torch.randn(N, HKV, D, device=dev, generator=g).to(torch.bfloat16)
    slots = torch.randperm(NB * BLOCK, device=dev, generator=g)[:N].to(torch.int32)
    npad = N // 10
    slots[torch.randperm(N, device=dev, generator=g)[:npad]] = -1
    kc = torch.zeros(NB, BLOCK, HKV, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    t = graph_timed(lambda: store_kvcache(key, value, kc, vc, slots))
    nbytes = (N - npad) * 4 * HKV * D * 2 + 4 * N
    return dict(us=t * 1e6, GBs=nbytes / t / 1e9, bytes=nbytes, timing="graph replay of 20 calls")


def norm_rope_bytes(N, write_k):
    """Algorithmic bytes of one sd_qk_norm_rope_store call over N tokens with every slot valid: the qkv row,
    the position, the fp32 cos / sin row and the slot per token; q out (and k out), the k / v cache rows."""
    per_tok = (HQ + 2 * HKV) * D * 2 + 8 + D * 4 + 4 + HQ * D * 2 + (HKV * D * 2 if write_k else 0) + 2 * HKV * D * 2
    return N * per_tok + 2 * D * 2


def bench_qk_norm_rope(dev, N=2048, NB=4096, copies=12, max_pos=40960):
    """Fused q/k RMSNorm + RoPE + KV store over one step's 2048 tokens (Qwen3-8B: 32 q / 8 kv heads, rope base
    1e6), k read back from the cache only (mixed / decode steps), graph-timed over calls that each read the
    next of `copies` qkv buffers (more bytes than the 256 MB last-level cache). Also the reference's
    sequence of eager operations on this GPU (two RMSNorms, the rotation, the store) for comparison."""
    import torch
    from nanovllm_amd.layers.attention import store_kvcache
    from nanovllm_amd.layers.rotary_embedding import RotaryEmbedding, qk_norm_rope_store
    g = torch.Generator(device=dev).manual_seed(5)
    W = (HQ + 2 * HKV) * D
    qkvs = [torch.randn(N, W, device=dev, generator=g).to(torch.bfloat16) for _ in range(copies)]
    pos = torch.randint(0, 4096, (N,), device=dev, generator=g)
    slots = torch.randperm(NB * BLOCK, device=dev, generator=g)[:N].to(torch.int32)
    rope = RotaryEmbedding(D, D, max_pos, 1e6).to(dev)
    cs = rope.cos_sin_cache
    qw = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16)
    kc = torch.zeros(NB, BLOCK, HKV, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q_out = torch.empty(N, HQ, D, dtype=torch.bfloat16, device=dev)
    turn = [0]

    def split():
        x = qkvs[turn[0] % copies]
        turn[0] += 1
        return (x[:, :HQ * D].view(N, HQ, D), x[:, HQ * D:(HQ + HKV) * D].view(N, HKV, D),
                x[:, (HQ + HKV) * D:].view(N, HKV, D))

    def fused():
        q, k, v = split()
        qk_norm_rope_store(pos, q, k, v, qw, kw, 1e-6, cs, kc, vc, slots, q_out=q_out, write_k=False)

    def eager_norm(x, w):
        xf = x.float()
        var = xf.pow(2).mean(dim=-1, keepdim=True)
        xf.mul_(torch.rsqrt(var + 1e-6))
        return xf.to(torch.bfloat16).mul_(w)

    cs3 = cs.view(max_pos, 1, D)

    def eager_rot(x, cos, sin):
        x1, x2 = torch.chunk(x.float(), 2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

    def unfused():
        q, k, v = split()
        q, k = eager_norm(q, qw), eager_norm(k, kw)
        cos, sin = cs3[pos].chunk(2, dim=-1)
        q, k = eager_rot(q, cos, sin), eager_rot(k, cos, sin)
        store_kvcache(k, v, kc, vc, slots)

    nbytes = norm_rope_bytes(N, write_k=False)
    t = graph_timed(fused, reps=24)
    te = graph_timed(unfused, reps=4)
    return dict(us=round(t * 1e6, 2), GBs=round(nbytes / t / 1e9, 1), frac=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                bytes=nbytes, tokens=N, eager_reference_ops_us=round(te * 1e6, 1),
                timing=f"graph replay of 24 calls over {copies} qkv buffers")


def bench_draft_inputs(dev, B=64, W=33):
    """One later draft step's inputs for 64 sequences (sd_draft_step_inputs, one launch) against the
    reference's tensor operations for the same step on this GPU (model_runner.py:446-452), both graph-timed."""
    import torch
    from nanovllm_amd.engine.draft_inputs import DraftStepBuffers, draft_step_inputs
    g = torch.Generator(device=dev).manual_seed(6)
    real_lens = torch.randint(1024, 8192, (B,), device=dev, generator=g).to(torch.int32)
    last_pos = real_lens.long() - 1
    tables = torch.randperm(4096, device=dev, generator=g)[:B * W].view(B, W).to(torch.int32)
    tokens = torch.randint(0, 151936, (B,), device=dev, generator=g)
    bufs = DraftStepBuffers(B, dev)
    input_ids = torch.zeros(B, dtype=torch.int64, device=dev)

    def reference_ops():
        real = real_lens > 0
        pos = torch.where(real, last_pos + 1, 0)
        block = tables.gather(1, (pos // BLOCK).unsqueeze(1)).squeeze(1)
        slot = torch.where(real, block * BLOCK + pos % BLOCK, -1).to(torch.int32)
        lens = torch.where(real, pos + 1, 0).to(torch.int32)
        input_ids[:B] = tokens
        return pos, slot, lens

    t = graph_timed(lambda: draft_step_inputs(real_lens, last_pos, tables, BLOCK, tokens, 1, bufs), reps=20)
    tr = graph_timed(reference_ops, reps=20)
    return dict(us=round(t * 1e6, 2), reference_ops_us=round(tr * 1e6, 2), seqs=B,
                timing="graph replay of 20 calls (one launch against the reference's ten operations)")


def bench_sampler(dev, steps, warmup, S=64, K=4, V=151936):
    """The verifier through its C ABI (graph-timed): T 0 as the engine calls it when every row is greedy (no
    temperatures, no noise: the argmax pass and the decision), and T 1 with draft logits and injected noise."""
    import torch
    from nanovllm_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev).manual_seed(4)
    logits = torch.randn(S * (K + 1), V, device=dev, generator=g) * 3
    dlog = torch.randn(S, K, V, device=dev, generator=g) * 3
    drafts = dlog.argmax(-1)
    nd = torch.full((S,), K, device=dev)
    u = torch.rand(S, K, device=dev, generator=g)
    e = torch.empty(S, V, device=dev).exponential_(1, generator=g)
    acc = torch.empty(S, dtype=torch.int64, device=dev)
    nxt = torch.empty(S, dtype=torch.int64, device=dev)
    res = {}
    for T, with_draft in ((0.0, False), (1.0, True)):
        temps = torch.full((S,), T, device=dev)
        ws = torch.empty(lib.sd_verify_workspace_size(S, K, V, int(with_draft)), dtype=torch.uint8, device=dev)

        def call():
            _lib.check(lib.sd_verify_drafts(
                logits.data_ptr(), _lib.DTYPE_F32, V, drafts.data_ptr(), nd.data_ptr(),
                temps.data_ptr() if T else None, dlog.data_ptr() if with_draft else None, _lib.DTYPE_F32,
                V if with_draft else 0, u.data_ptr() if T else None, e.data_ptr() if T else None, S, K, V,
                acc.data_ptr(), nxt.data_ptr(), ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream),
                "sd_verify_drafts")
        t = graph_timed(call, reps=10, replays=20)
        nbytes = S * (K + 1) * V * 4 + ((S * K * V * 4 + 2 * S * V * 4 + S * V * 4) if T else 0)
        res[f"T{int(T)}"] = dict(us=round(t * 1e6, 2), GBs=round(nbytes / t / 1e9, 1),
                                 frac=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4), bytes=nbytes,
                                 timing="20 graph replays of 10 calls")
    return res


def bench_lm_head_verify(dev, S=64, K=4, V=151936, H=4096):
    """The unfused path in front of the verifier: the LM head as the library GEMM (F.linear, as
    embed_head.py:63 computes it) over the S(K+1) verify rows into bf16 logits, then sd_verify_drafts at
    T = 0 on them. Reports each part and what fusing the verify statistics into the GEMM could save at most:
    the logits' write and re-read at the HBM rate the verifier reaches."""
    import torch
    import torch.nn.functional as F
    from nanovllm_amd.layers.sampler import verify_drafts
    g = torch.Generator(device=dev).manual_seed(9)
    h = (torch.randn(S * (K + 1), H, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    w = (torch.randn(V, H, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    logits = torch.empty(S * (K + 1), V, device=dev, dtype=torch.bfloat16)
    drafts = torch.randint(0, V, (S, K), device=dev, generator=g)
    nd = torch.full((S,), K, device=dev)
    temps = torch.zeros(S, device=dev)
    u = torch.rand(S, K, device=dev, generator=g)
    e = torch.empty(S, V, device=dev).exponential_(1, generator=g)
    t_gemm = graph_timed(lambda: F.linear(h, w), reps=5)
    logits.copy_(F.linear(h, w))
    t_verify = graph_timed(lambda: verify_drafts(logits, drafts, nd, temps, None, uniforms=u, exp_noise=e), reps=10)
    t_both = graph_timed(lambda: verify_drafts(F.linear(h, w), drafts, nd, temps, None, uniforms=u, exp_noise=e),
                         reps=5)
    flops = 2.0 * S * (K + 1) * H * V
    w_bytes = V * H * 2
    logit_bytes = S * (K + 1) * V * 2
    verify_rate = logit_bytes / t_verify
    # the fused path: sd_lm_head_verify, greedy (the GEMM's epilogue takes the argmax; no logits written)
    from nanovllm_amd import _lib
    lib = _lib.load()
    acc = torch.empty(S, dtype=torch.int64, device=dev)
    nxt = torch.empty(S, dtype=torch.int64, device=dev)
    ws = torch.empty(lib.sd_lm_head_verify_workspace_size(S, K, V, H, 0), dtype=torch.uint8, device=dev)
    from nanovllm_amd.layers.lm_head import pack_weight
    wp = pack_weight(w)

    def fused():
        _lib.check(lib.sd_lm_head_verify(h.data_ptr(), H, S * (K + 1), None, wp.data_ptr(), V, H, drafts.data_ptr(),
                                         nd.data_ptr(), None, None, 0, 0, None, None, S, K, None, 0, acc.data_ptr(),
                                         nxt.data_ptr(), ws.data_ptr(), ws.numel(),
                                         torch.cuda.current_stream().cuda_stream), "sd_lm_head_verify")
    t_fused = graph_timed(fused, reps=5)
    return dict(
        shape=f"[{S * (K + 1)}, {H}] x [{H}, {V}] bf16",
        gemm_us=round(t_gemm * 1e6, 2), gemm_tflops=round(flops / t_gemm / 1e12, 1),
        gemm_mfma_frac=round(flops / t_gemm / 2.5e15, 4), gemm_weight_TBs=round(w_bytes / t_gemm / 1e12, 3),
        verify_us=round(t_verify * 1e6, 2), gemm_then_verify_us=round(t_both * 1e6, 2),
        fused_us=round(t_fused * 1e6, 2), fused_tflops=round(flops / t_fused / 1e12, 1),
        fused_mfma_frac=round(flops / t_fused / 2.5e15, 4), fused_weight_TBs=round(w_bytes / t_fused / 1e12, 3),
        timing="graph replays; logits bf16 as the engine's LM head writes them; fused = sd_lm_head_verify "
               "(hand-written MFMA GEMM with the argmax in its epilogue, T = 0, no logits written)")


def bench_mixed_attention(dev, steps, warmup, layers=36):
    """Attention phase of a 2048-token-budget mixed step (48 verify requests with k = 4 and 3 prefill chunks,
    lognormal lengths, Qwen3-8B shapes): per layer, store this step's KV then varlen paged attention, for 36
    layers. Timed as one HIP-graph replay per step through the mixed-step runtime (plan + 36 x (store +
    attention), metadata refreshed by one host-to-device copy per step), as eager per-layer calls, and as the
    runtime's step with each layer's q/k RMSNorm + RoPE + KV store fused in front of the attention."""
    import numpy as np
    import torch
    from types import SimpleNamespace
    from nanovllm_amd.engine.synthetic import paged_cache, queries
    from nanovllm_amd.engine.mixed_step import MixedStepRunner
    from nanovllm_amd.layers.attention import store_kvcache, varlen_attention
    from nanovllm_amd.engine.synthetic import mixed_step_lengths, requests
    K = 4
    lq, lk = mixed_step_lengths(0)
    nd = 48
    W = math.ceil(max(lk) / BLOCK)
    kc, vc, tables = paged_cache(dev, lk, HKV, D, W=W, seed=5)
    caches = [(kc, vc)] + [(torch.empty_like(kc).copy_(kc), torch.empty_like(vc).copy_(vc)) for _ in range(layers - 1)]
    runner = MixedStepRunner([SimpleNamespace(k_cache=a, v_cache=b) for a, b in caches], HQ, HKV, D, D ** -0.5,
                             block_size=BLOCK, max_num_batched_tokens=2048, max_num_seqs=64, table_width=W)
    layout = runner.prepare(requests(lq, lk, tables.cpu(), nd, K, BLOCK), K)
    Nq, N = layout["n"], layout["N"]
    runner.bufs["q"][:N] = queries(dev, N, HQ, D, seed=6)
    runner.bufs["k"][:N] = queries(dev, N, HKV, D, seed=7)
    runner.bufs["v"][:N] = queries(dev, N, HKV, D, seed=8)
    wall, ev = timed(lambda: runner.run(layout), steps, warmup)
    t = sum(ev) / len(ev)
    # the replay alone, its metadata already on the device (as the eager calls below have theirs)
    graph = runner.graphs[(N, layout["S"])]
    _, replay_ev = timed(graph.replay, steps, warmup)
    t_replay = sum(replay_ev) / len(replay_ev)

    # eager: the same step as 36 x (store_kvcache + varlen_attention) Python calls (plan reused per step)
    q, knew, vnew = runner.bufs["q"][:Nq], runner.bufs["k"][:Nq], runner.bufs["v"][:Nq]
    slots = torch.tensor(layout["slot_mapping"], dtype=torch.int32, device=dev)
    cu_q = torch.tensor(layout["cu_seqlens_q"], dtype=torch.int32, device=dev)
    cu_k = torch.tensor(layout["cu_seqlens_k"], dtype=torch.int32, device=dev)
    out = torch.empty(Nq, HQ, D, dtype=torch.bfloat16, device=dev)

    def eager_step():
        owner = SimpleNamespace()  # the step's context: layer 1 plans the work lists, the others reuse them
        for kcl, vcl in caches:
            store_kvcache(knew, vnew, kcl, vcl, slots)
            varlen_attention(q, kcl, vcl, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables, out=out, plan_owner=owner)

    _, eager_ev = timed(eager_step, steps, warmup)
    t_eager = sum(eager_ev) / len(eager_ev)

    # the same step with each layer's q/k RMSNorm + RoPE + KV store fused in front of its attention (the
    # runner's pre_attn: qkv rows in, per-layer norm weights, Qwen3-8B rope base 1e6)
    from nanovllm_amd.layers.rotary_embedding import RotaryEmbedding
    g = torch.Generator(device=dev).manual_seed(9)
    weights = [tuple((1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16) for _ in range(2))
               for _ in range(layers)]
    rope = RotaryEmbedding(D, D, 40960, 1e6).to(dev)
    fused = MixedStepRunner([SimpleNamespace(k_cache=a, v_cache=b) for a, b in caches], HQ, HKV, D, D ** -0.5,
                            block_size=BLOCK, max_num_batched_tokens=2048, max_num_seqs=64, table_width=W,
                            pre_attn=(rope.cos_sin_cache, weights, 1e-6))
    fused.bufs["qkv"][:N] = queries(dev, N, HQ + 2 * HKV, D, seed=9).view(N, -1)
    _, fused_ev = timed(lambda: fused.run(layout), steps, warmup)
    t_fused = sum(fused_ev) / len(fused_ev)
    flops = sum(4 * HQ * D * (a * (b - a) + a * (a + 1) / 2) for a, b in zip(lq[nd:], lk[nd:]))
    dec_bytes = decode_bytes(lk[:nd], 5)
    # One layer's attention kernel (work lists planned beforehand), whole step and its prefill chunks alone,
    # each call on the next layer's caches.
    layer_s = planned_varlen_time(q, caches, lq, lk, tables)
    pre = slice(sum(lq[:nd]), Nq)
    prefill_s = planned_varlen_time(q[pre], caches, lq[nd:], lk[nd:], tables[nd:].contiguous())
    return dict(ms=round(t * 1e3, 4), tok_s=round(Nq / t, 1),
                timing="one HIP-graph replay per step after the step's metadata copy (host to device)",
                replay_ms=round(t_replay * 1e3, 4), replay_tok_s=round(Nq / t_replay, 1),
                eager_ms=round(t_eager * 1e3, 4), eager_tok_s=round(Nq / t_eager, 1),
                eager_timing="36 x (store + attention) Python calls on metadata already on the device",
                with_qk_norm_rope_ms=round(t_fused * 1e3, 4), with_qk_norm_rope_tok_s=round(Nq / t_fused, 1),
                query_tokens=Nq, bucket_tokens=N, bucket_seqs=layout["S"], decode_seqs=nd,
                prefill_chunks=len(lq) - nd, prefill_flops_per_layer=flops, decode_bytes_per_layer=dec_bytes,
                layer_attention_us=round(layer_s * 1e6, 2),
                prefill_only_us=round(prefill_s * 1e6, 2),
                prefill_only_tflops=round(flops / prefill_s / 1e12, 1),
                prefill_mfma_frac=round(flops / prefill_s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                layer_prefill_mfma_frac=round(flops / layer_s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4))


def bench_prefill(dev):
    """The prefill q-block kernel on its own at sizes that fill the GPU (Qwen3-8B shapes, paged KV): 16
    chunks of 1024 queries after a 1024-token cached prefix, and one fresh 2048-token prompt. FLOPs are the
    causal attention's 4*Hq*D*(Lq*P + Lq(Lq+1)/2) per chunk."""
    from nanovllm_amd.engine.synthetic import paged_cache, queries
    res = {}
    for name, lq, lk in (("16x1024_after_1024", [1024] * 16, [2048] * 16), ("1x2048", [2048], [2048])):
        kc, vc, tables = paged_cache(dev, lk, HKV, D, W=math.ceil(max(lk) / BLOCK), seed=21)
        q = queries(dev, sum(lq), HQ, D, seed=22)
        t = planned_varlen_time(q, [(kc, vc)], lq, lk, tables)
        flops = sum(4 * HQ * D * (a * (b - a) + a * (a + 1) / 2) for a, b in zip(lq, lk))
        res[name] = dict(us=round(t * 1e6, 2), tflops=round(flops / t / 1e12, 1),
                         mfma_frac=round(flops / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4))
        del kc, vc, tables, q
    return res


def bench_mixed_step_full(dev, layers=36, steps=5, warmup=2, row_invariant=False):
    """The whole config-5 step: a random-init Qwen3-8B-shaped model (36 layers, hidden 4096, 32 q / 8 kv heads,
    MLP 12288, vocab 151936, bf16) run piecewise by the mixed-step runtime in one HIP graph per bucket
    (embedding, per layer: input norm + qkv GEMM, fused q/k norm + RoPE + KV store, varlen attention,
    o_proj + post norm + MLP; final norm), then, eagerly as the reference's run_mixed does, the LM head on the
    decode requests' verify rows and the greedy verifier (sd_lm_head_verify: one call, no logits written).
    Reports the model step alone (graph replay) and the whole step, as query tokens per second. row_invariant:
    the projections and norms through sd_linear / sd_rms_norm instead of the library's."""
    import torch
    from types import SimpleNamespace
    from nanovllm_amd import _lib
    from nanovllm_amd.engine.mixed_step import MixedStepRunner
    from nanovllm_amd.engine.qwen3_segments import Qwen3Segments
    from nanovllm_amd.engine.synthetic import mixed_step_lengths, paged_cache, requests
    K = 4
    lq, lk = mixed_step_lengths(0)
    nd = 48
    W = math.ceil(max(lk) / BLOCK)
    kc, vc, tables = paged_cache(dev, lk, HKV, D, W=W, seed=5)
    caches = [(kc, vc)] + [(kc.clone(), vc.clone()) for _ in range(layers - 1)]
    seg = Qwen3Segments(num_layers=layers, device=dev, seed=1, row_invariant=row_invariant)
    runner = MixedStepRunner([SimpleNamespace(k_cache=a, v_cache=b) for a, b in caches], HQ, HKV, D, D ** -0.5,
                             block_size=BLOCK, max_num_batched_tokens=2048, max_num_seqs=64, table_width=W,
                             segment=seg, pre_attn=seg.pre_attn())
    layout = runner.prepare(requests(lq, lk, tables.cpu(), nd, K, BLOCK), K)
    n, N = layout["n"], layout["N"]
    g = torch.Generator(device=dev).manual_seed(2)
    seg.input_ids[:N] = torch.randint(0, 151936, (N,), device=dev, generator=g)
    seg.input_ids[n:N] = 0
    lib = _lib.load()
    idx = torch.tensor(layout["logits_indices"], dtype=torch.int64, device=dev)
    drafts = torch.randint(0, 151936, (nd, K), device=dev, generator=g)
    ndr = torch.full((nd,), K, dtype=torch.int64, device=dev)
    acc = torch.empty(nd, dtype=torch.int64, device=dev)
    nxt = torch.empty(nd, dtype=torch.int64, device=dev)
    V = 151936
    from nanovllm_amd.layers.lm_head import pack_weight
    wp = pack_weight(seg.lm_head)   # once per model
    H = seg.hidden
    ws = torch.empty(lib.sd_lm_head_verify_workspace_size(nd, K, V, H, 0), dtype=torch.uint8, device=dev)

    def model_step():
        runner.run(layout)

    def whole_step():
        # the step, then the LM head over the decode requests' verify rows and the greedy verifier in one call
        runner.run(layout)
        h = seg.hidden_out
        _lib.check(lib.sd_lm_head_verify(h.data_ptr(), h.stride(0), h.size(0), idx.data_ptr(), wp.data_ptr(), V, H,
                                         drafts.data_ptr(), ndr.data_ptr(), None, None, 0, 0, None, None, nd, K, None,
                                         0, acc.data_ptr(), nxt.data_ptr(), ws.data_ptr(), ws.numel(),
                                         torch.cuda.current_stream().cuda_stream), "sd_lm_head_verify")

    wall_m, _ = timed(model_step, steps, warmup)
    wall_w, _ = timed(whole_step, steps, warmup)
    gemm_flops = 2 * N * layers * (4096 * 6144 + 4096 * 4096 + 4096 * 24576 + 12288 * 4096)
    res = dict(model_step_ms=round(wall_m * 1e3, 3), model_step_tok_s=round(n / wall_m, 1),
               whole_step_ms=round(wall_w * 1e3, 3), whole_step_tok_s=round(n / wall_w, 1),
               query_tokens=n, bucket_tokens=N, logits_rows=len(layout["logits_indices"]),
               layer_gemm_tflops_per_step=round(gemm_flops / 1e12, 2),
               timing="wall clock of back-to-back steps between synchronizations (the step's metadata copy, "
                      "one graph replay, then sd_lm_head_verify eagerly)")
    del caches, kc, vc, seg, runner, wp
    torch.cuda.empty_cache()
    return res


def bench_decode_step_full(dev, layers=36, steps=5, warmup=2, k=4):
    """Whole-model verify steps (1 + k rows per sequence: DecodeStepRunner graph replay, then sd_lm_head_verify)
    against plain decode steps (one row: graph replay, then the LM head and the greedy sampler through the same
    GEMM, K = 0) of a random-init Qwen3-8B-shaped model (36 layers), at B in {1, 16, 64} x context {256, 1024}:
    the grid of the reference's step-cost runs (nanovllm/engine/model_runner.py:591-634 measure_step_costs; A100,
    Qwen3-8B: B=64 ctx 1024 42.80 vs 18.17 ms). Each step: its metadata copy, the graph replay, the LM head
    call; wall clock between synchronizations. Then the same grid with the row-invariant projections and norms
    (greedy spec == plain bitwise), on a second copy of the model."""
    import torch
    from types import SimpleNamespace
    from nanovllm_amd.engine.decode_step import DecodeStepRunner
    from nanovllm_amd.engine.qwen3_segments import Qwen3Segments
    from nanovllm_amd.layers.lm_head import LMHeadVerifier, lm_head_sample, lm_head_verify
    Bmax, ctxs, batches = 64, (256, 1024), (1, 16, 64)
    W = math.ceil((max(ctxs) + k + 1) / BLOCK)
    NB = Bmax * W
    caches = [SimpleNamespace(k_cache=torch.zeros(NB, BLOCK, HKV, D, dtype=torch.bfloat16, device=dev),
                              v_cache=torch.zeros(NB, BLOCK, HKV, D, dtype=torch.bfloat16, device=dev))
              for _ in range(layers)]
    g = torch.Generator(device=dev).manual_seed(3)

    def seqs_for(B, ctx):
        return [SimpleNamespace(token_ids=[100 + i] * ctx, last_token=100 + i, num_tokens=ctx,
                                block_table=list(range(i * W, (i + 1) * W)), draft_token_ids=[7] * k)
                for i in range(B)]

    def measure(model, head, B, ctx):
        runner = measure.runners[id(model)]
        seqs = seqs_for(B, ctx)
        zeros = torch.zeros(B, device=dev)
        drafts = torch.full((B, k), 7, dtype=torch.int64, device=dev)
        nd = torch.full((B,), k, dtype=torch.int64, device=dev)
        out = {}
        for name, n in (("verify", 1 + k), ("plain", 1)):
            layout = runner.prepare(seqs, n, with_drafts=n > 1)

            def step():
                h = runner.run(layout)
                if n > 1:
                    lm_head_verify(h, head, drafts, nd, zeros)
                else:
                    lm_head_sample(h, head, zeros)
            wall, _ = timed(step, steps, warmup)
            out[f"{name}_ms"] = round(wall * 1e3, 3)
        out["verify_over_plain"] = round(out["verify_ms"] / out["plain_ms"], 3)
        return out
    measure.runners = {}

    res = {}
    for mode in ("library", "row_invariant"):
        model = Qwen3Segments(num_layers=layers, device=dev, seed=1, max_tokens=Bmax * (1 + k),
                              row_invariant=mode == "row_invariant")
        head = LMHeadVerifier(model.lm_head)
        measure.runners[id(model)] = DecodeStepRunner(caches, model, HQ, HKV, D, D ** -0.5, BLOCK, table_width=W,
                                                      max_batch=Bmax, query_tokens=(1, 1 + k))
        res[mode] = {f"B{B}_ctx{c}": measure(model, head, B, c) for c in ctxs for B in batches}
        del measure.runners[id(model)], model, head
        torch.cuda.empty_cache()
    res["reference_a100_ms"] = {"B1_ctx1024": [12.05, 11.35], "B16_ctx1024": [16.81, 12.99],
                                "B64_ctx1024": [42.80, 18.17], "B64_ctx256": [33.01, 13.88],
                                "note": "[verify, plain] whole-step ms on A100 (CUDA graphs, Qwen3-8B weights), "
                                        "other hardware: context only"}
    res["timing"] = ("wall clock of back-to-back steps between synchronizations: metadata copy, one graph replay "
                     "of the 36-layer model, the LM head with the greedy decision (k = 4 verify / plain)")
    del caches
    torch.cuda.empty_cache()
    return res


def planned_varlen_time(q, caches, lq, lk, tables):
    """Seconds per sd_varlen_attention_planned call (the attention kernel alone; the work lists are planned
    once outside the timed graph, as the per-layer loop of a step does). The calls cycle through `caches`
    (one (k, v) pair per layer), so that a layer's KV is not still in the 256 MB last-level cache from the
    call before, as in a real step."""
    import numpy as np
    import torch
    from nanovllm_amd import _lib
    dev = q.device
    lib = _lib.load()
    Nq, nseq = sum(lq), len(lq)
    cu_q = torch.tensor([0] + np.cumsum(lq).tolist(), dtype=torch.int32, device=dev)
    cu_k = torch.tensor([0] + np.cumsum(lk).tolist(), dtype=torch.int32, device=dev)
    out = torch.empty(Nq, HQ, D, dtype=torch.bfloat16, device=dev)
    qr = q.contiguous()
    nbytes = lib.sd_varlen_workspace_size(nseq, Nq, max(lk), HQ, HKV, D)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    stream = lambda: torch.cuda.current_stream().cuda_stream
    _lib.check(lib.sd_varlen_plan(cu_q.data_ptr(), cu_k.data_ptr(), nseq, Nq, max(lq), HQ, HKV, ws.data_ptr(), nbytes,
                                  stream()), "sd_varlen_plan")
    turn = [0]

    def call():
        kc, vc = caches[turn[0] % len(caches)]
        turn[0] += 1
        _lib.check(lib.sd_varlen_attention_planned(
            qr.data_ptr(), qr.stride(0), kc.data_ptr(), HKV * D, vc.data_ptr(), HKV * D, 0, kc.size(0), BLOCK,
            tables.data_ptr(), tables.size(1), cu_q.data_ptr(), cu_k.data_ptr(), nseq, Nq, max(lq), max(lk), HQ,
            HKV, D, D ** -0.5, out.data_ptr(), out.stride(0), ws.data_ptr(), nbytes, stream()),
            "sd_varlen_attention_planned")
    return graph_timed(call, reps=len(caches))


def cpu_baseline(inputs, min_seconds=10.0, max_reps=8):
    """The oracle (fp32 PyTorch CPU restatement of the reference semantics) on the headline workload: all
    64 sequences, repeated until at least `min_seconds` of CPU work have been timed (at most `max_reps`
    runs, after one untimed 2-sequence warm-up), on 16 host threads; returns GB/s of algorithmic bytes."""
    import torch
    from oracle import attention as oatt
    q, kc, vc, lens, tables = inputs
    # at most 16 host threads: the CPU share of one GPU on a shared 8-GPU host, whatever os.cpu_count() says
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    qs, ls, ts = q.cpu(), lens.cpu(), tables.cpu()
    kcs, vcs = kc.cpu(), vc.cpu()
    oatt.paged_decode_attention(qs[:2], kcs, vcs, ls[:2], ts[:2], D ** -0.5)
    reps, total = 0, 0.0
    while reps < max_reps and (total < min_seconds or reps < 2):
        t0 = time.perf_counter()
        oatt.paged_decode_attention(qs, kcs, vcs, ls, ts, D ** -0.5)
        total += time.perf_counter() - t0
        reps += 1
    t = total / reps
    nbytes = decode_bytes(ls.tolist(), q.size(1))
    threads = torch.get_num_threads()
    visible = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return dict(value=round(nbytes / t / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                cpu_model=cpu_model(), cpu=cpu_info(), os_cpu_count=os.cpu_count(), affinity_cpus=visible,
                threads_note=(f"{threads} intra-op threads = every one of the {visible} CPUs this process may run "
                              f"on" if threads >= (visible or 0) else
                              f"{threads} intra-op threads of the {visible} CPUs this process may run on (capped at "
                              f"16, the host-CPU share of one GPU)"),
                sample=f"the full headline call (64 sequences, ctx 4096, k=4) through the oracle's "
                       f"paged_decode_attention, {reps} runs, {total:.1f} s total, {t * 1e3:.0f} ms per call",
                secondary=cpu_secondary())


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_info() -> dict:
    """What /proc/cpuinfo and sysfs say of the first CPU (a virtualised host may report only a bare model name):
    vendor, family / model / stepping, clock, cache, SIMD extensions the oracle's PyTorch kernels can use, and
    the NUMA node count."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
    except OSError:
        return {}
    flags = set(info.get("flags", "").split())
    nodes = [d for d in os.listdir("/sys/devices/system/node") if d.startswith("node")] \
        if os.path.isdir("/sys/devices/system/node") else []
    out = {k: info[k] for k in ("vendor_id", "cpu family", "model", "stepping", "cpu MHz", "cache size",
                                "siblings", "cpu cores") if k in info}
    out["simd"] = [f for f in ("avx2", "avx512f", "avx512_bf16", "avx512_vnni", "amx_bf16") if f in flags]
    out["numa_nodes"] = len(nodes)
    try:
        import torch
        out["torch_cpu_capability"] = torch.backends.cpu.get_cpu_capability()
    except Exception:
        pass
    return out


def cpu_secondary(reps=3):
    """The oracle on the secondary workloads' shapes (same threads), milliseconds per call: the KV scatter of
    2048 rows, the fused q/k norm + RoPE + store over 2048 tokens and one draft step's inputs for 64 sequences
    (best of `reps`); the verifier at S 64, K 4, V 151936 (T 0, and T 1 with draft logits) and one layer of
    the mixed step's attention (one run each)."""
    import numpy as np
    import torch
    from oracle import attention as oatt
    from oracle import draft_inputs as odi
    from oracle import kvcache as okv
    from oracle import qk_norm_rope as onr
    from oracle import sampler as osmp
    from nanovllm_amd.engine.synthetic import mixed_step_lengths
    g = torch.Generator().manual_seed(7)
    N, NB, W = 2048, 512, 33
    qkv = torch.randn(N, (HQ + 2 * HKV) * D, generator=g).to(torch.bfloat16)
    q = qkv[:, :HQ * D].view(N, HQ, D)
    k = qkv[:, HQ * D:(HQ + HKV) * D].view(N, HKV, D)
    v = qkv[:, (HQ + HKV) * D:].view(N, HKV, D)
    pos = torch.randint(0, 4096, (N,), generator=g)
    cs = onr.rope_cache(D, 40960, 1e6)
    w = torch.ones(D, dtype=torch.bfloat16)
    slots = torch.randperm(NB * BLOCK, generator=g)[:N].to(torch.int32)
    kc = torch.zeros(NB, BLOCK, HKV, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    real = torch.randint(1024, 8192, (64,), generator=g).to(torch.int32)
    last = real.long() - 1
    tables = torch.randperm(4096, generator=g)[:64 * W].view(64, W).to(torch.int32)
    toks = torch.randint(0, 151936, (64,), generator=g)
    out = {}

    def clock(name, fn, n):
        best = float("inf")
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            best = min(best, time.perf_counter() - t0)
        out[name] = round(best * 1e3, 3)

    clock("kv_store_2048_rows_ms", lambda: okv.store_kvcache(k, v, kc, vc, slots), reps)
    clock("qk_norm_rope_store_2048_tokens_ms",
          lambda: onr.qk_norm_rope_store(q, k, v, pos, w, w, 1e-6, cs, kc, vc, slots), reps)
    clock("draft_step_inputs_64_seqs_ms", lambda: odi.draft_step_inputs(real, last, tables, BLOCK, toks, 1), reps)
    del kc, vc, qkv, q, k, v
    S, K, V = 64, 4, 151936
    logits = torch.randn(S * (K + 1), V, generator=g) * 3
    dlog = torch.randn(S, K, V, generator=g) * 3
    drafts, nd = dlog.argmax(-1), torch.full((S,), K)
    u, e = torch.rand(S, K, generator=g), torch.empty(S, V).exponential_(1, generator=g)
    for T in (0.0, 1.0):
        clock(f"verify_T{int(T)}_ms", lambda: osmp.verify_drafts(logits, drafts, nd, torch.full((S,), T),
                                                                 dlog if T else None, uniforms=u, exp_noise=e), 1)
    del logits, dlog, e
    lq, lk = mixed_step_lengths(0)
    Wm = math.ceil(max(lk) / BLOCK)
    nblk = sum(math.ceil(c / BLOCK) for c in lk)
    kcm = torch.randn(nblk, BLOCK, HKV, D, generator=g).to(torch.bfloat16)
    vcm = torch.randn(nblk, BLOCK, HKV, D, generator=g).to(torch.bfloat16)
    tab = torch.full((len(lk), Wm), -1, dtype=torch.int32)
    b = 0
    for i, c in enumerate(lk):
        nb = math.ceil(c / BLOCK)
        tab[i, :nb] = torch.arange(b, b + nb)
        b += nb
    qm = torch.randn(sum(lq), HQ, D, generator=g).to(torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum(lq).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(lk).tolist(), dtype=torch.int32)
    clock("mixed_step_attention_one_layer_ms", lambda: oatt.varlen_attention(qm, kcm, vcm, cu_q, cu_k, D ** -0.5, tab), 1)
    return out


def pmc_traffic(path=os.path.join(ROOT, "profiles", "attn_fwd_verify_b64_k4_ctx4096.pmc.txt")):
    """HBM bytes per headline launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (each
    counter scaled by what it reads for a plain 1 GiB device copy); None when the summary is absent."""
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-extras", action="store_true", help="headline only (for profiling)")
    ap.add_argument("--no-cpu", action="store_true", help="leave out the CPU baseline (for profiling)")
    ap.add_argument("--only", choices=["qk_norm_rope_store", "draft_step_inputs", "kv_store", "lm_head_verify",
                                       "verify_sampler", "mixed_step_full", "mixed_step_attention", "prefill_kernel",
                                       "verify_attention_sweep", "decode_step_full"],
                    help="run one secondary workload alone and print its JSON (for profiling)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device copy (reference kernel for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (the hot path shards by sequence or "
              "KV head with no cross-GPU exchange). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only:
        fn = {"qk_norm_rope_store": lambda: bench_qk_norm_rope(dev), "draft_step_inputs": lambda: bench_draft_inputs(dev),
              "kv_store": lambda: bench_store(dev, args.steps, args.warmup),
              "lm_head_verify": lambda: bench_lm_head_verify(dev),
              "verify_sampler": lambda: bench_sampler(dev, args.steps, args.warmup),
              "mixed_step_full": lambda: [bench_mixed_step_full(dev), bench_mixed_step_full(dev, row_invariant=True)],
              "mixed_step_attention": lambda: bench_mixed_attention(dev, max(5, args.steps // 10), 2),
              "prefill_kernel": lambda: bench_prefill(dev),
              "verify_attention_sweep": lambda: bench_verify_sweep(dev),
              "decode_step_full": lambda: bench_decode_step_full(dev)}[args.only]
        print(json.dumps({args.only: fn()}), flush=True)
        return
    head = bench_verify_attention(dev, args.steps, args.warmup)
    t = head["event_s"]
    achieved = head["bytes"] / t / 1e9
    value_tbs = head["bytes"] / head["wall_s"] / 1e12
    result = {
        "metric": "spec-verify attn TB/s (% HBM peak) Qwen3-8B k=4 B=64; mixed-step tok/s",
        "value": round(value_tbs, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["wall_s"] * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) bf16 KV cache and queries, randomly permuted block tables)",
        "config": {"workload": "spec-verify paged attention, Qwen3-8B shapes (32 q / 8 kv heads, head_dim 128), "
                               "B=64, k=4 (5 causal queries), ctx 4096, block 256, table width 33",
                   "batch": 64, "k": 4, "context": 4096, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": pmc_traffic(),
                     "kernel": "attn_fwd<RT=2, 8 waves> (one sd_paged_decode call: one launch, residues merged in LDS)",
                     "bytes_per_launch": head["bytes"], "us_per_launch": round(t * 1e6, 2),
                     "timing": "mean of per-launch HIP event pairs on the launch stream over the timed steps "
                               "(rocprofv3 kernel average: profiles/bench_workloads.kernel_stats.txt)"},
    }
    if not args.skip_extras:
        result["verify_attention_uniform_ctx"] = bench_verify_uniform(dev)
        result["verify_attention_sweep"] = bench_verify_sweep(dev)
        result["kv_store"] = bench_store(dev, args.steps, args.warmup)
        result["qk_norm_rope_store"] = bench_qk_norm_rope(dev)
        result["draft_step_inputs"] = bench_draft_inputs(dev)
        result["verify_sampler"] = bench_sampler(dev, max(10, args.steps // 2), args.warmup)
        result["lm_head_then_verify"] = bench_lm_head_verify(dev)
        mixed = bench_mixed_attention(dev, max(5, args.steps // 10), 2)
        result["mixed_step_attention"] = mixed
        layer_s = mixed["layer_attention_us"] / 1e6
        pre_tf = mixed["prefill_flops_per_layer"] / 1e12
        result["mixed_step_roofline"] = {
            "bound": "mfma (prefill rows) + hbm (decode rows)",
            "prefill_achieved_tflops": round(pre_tf / layer_s, 1), "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS,
            "prefill_frac_of_layer_time": round(pre_tf / layer_s / MFMA_BF16_PEAK_TFLOPS, 4),
            "decode_achieved_GBs": round(mixed["decode_bytes_per_layer"] / layer_s / 1e9, 1),
            "decode_frac_of_layer_time": round(mixed["decode_bytes_per_layer"] / layer_s / 1e9 / HBM_PEAK_GBS, 4),
            "combined_frac": round((pre_tf / MFMA_BF16_PEAK_TFLOPS
                                    + mixed["decode_bytes_per_layer"] / (HBM_PEAK_GBS * 1e9)) / layer_s, 4),
            "note": "one layer's attention launch (planned work lists, caches cycled over 36 layers); combined_frac "
                    "= (prefill FLOPs / MFMA peak + decode bytes / HBM peak) / layer time"}
        result["mixed_step_full_model"] = bench_mixed_step_full(dev)
        result["mixed_step_full_model_row_invariant"] = bench_mixed_step_full(dev, row_invariant=True)
        result["decode_step_full_model"] = bench_decode_step_full(dev)
        result["prefill_kernel"] = bench_prefill(dev)
    if not args.skip_extras and not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(head["inputs"])
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
