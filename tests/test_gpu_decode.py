"""Decode / speculative-verify attention on the GPU (HIP sd_paged_decode) against the fp32 oracle.

Tolerance (attention output, bf16): max-abs <= 2e-2 and mean-abs <= 2e-3 versus the fp32 oracle.
Bitwise properties: batch padding (check_padding.py style: B real rows alone == padded to the graph bucket
with context_len 0 sequences), spec == non-spec rows (a verify row equals the plain decode of the same
query at the same position), run-to-run repeatability, hipGraph capture at context_len 0 then replay.
"""
import random

import pytest
import torch

from nanovllm_amd.layers.attention import paged_decode_attention
from oracle import attention as oatt
from attn_cases import error_stats, paged_cache, queries, sub_cache

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _check(device, ctx, n, Hq, Hkv, D=128, W=None, seed=0, tail=-1):
    B = len(ctx)
    kc, vc, tables = paged_cache(device, ctx, Hkv, D, W=W, seed=seed, tail=tail)
    q = queries(device, B * n, Hq, D, seed=seed + 100).view(B, n, Hq, D)
    lens = torch.tensor(ctx, dtype=torch.int32, device=device)
    scale = D ** -0.5
    out = paged_decode_attention(q, kc, vc, lens, tables, scale)
    ref = oatt.paged_decode_attention(q.cpu(), kc.cpu(), vc.cpu(), lens.cpu(), tables.cpu(), scale)
    mx, mean = error_stats(out.view(B, n, Hq, D), ref)
    print(f"B={B} n={n} Hq={Hq} Hkv={Hkv} ctx[:4]={ctx[:4]}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)
    return out


def test_config1_qwen3_06b_shapes(device):
    """16 q / 8 kv heads, block 256, B 4, ctx {300, 512, 777, 1024}, k = 4 (5 causal queries)."""
    _check(device, [300, 512, 777, 1024], 5, 16, 8)


@pytest.mark.parametrize("B", [1, 16, 64])
@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_config3_qwen3_8b_verify(device, B, k):
    """32 q / 8 kv heads, contexts uniform in [1024, 8192], table width 33 = ceil((8192 + k) / 256)."""
    rnd = random.Random(B * 100 + k)
    ctx = [rnd.randint(1024, 8192) for _ in range(B)]
    _check(device, ctx, k + 1, 32, 8, W=33, seed=B + k)


def test_headline_ctx4096(device):
    _check(device, [4096] * 64, 5, 32, 8, W=33, seed=7)


def test_short_and_edge_contexts(device):
    """Contexts shorter than a tile, exactly at tile / block / split boundaries, and one past them."""
    ctx = [5, 31, 32, 33, 255, 256, 257, 511, 512, 513, 1023, 1024, 1025, 2047, 2048, 2049]
    _check(device, ctx, 5, 32, 8, W=9, seed=3)
    _check(device, ctx, 1, 32, 8, W=9, seed=4)
    _check(device, [9, 40, 600], 9, 16, 2, seed=5)        # g = 8, n = 9 -> 72 rows: two query groups


def test_padding_sequences_write_zeros_and_stale_tables(device):
    """context_len 0 rows produce zeros; table entries past the used blocks (-1 or stale ids) are never read."""
    ctx = [700, 0, 1500, 0]
    B, n, Hq, Hkv, D = 4, 5, 32, 8, 128
    kc, vc, tables = paged_cache(device, ctx, Hkv, D, W=12, seed=11, tail=10 ** 6)
    tables[1].fill_(-1)
    q = queries(device, B * n, Hq, D, seed=12).view(B, n, Hq, D)
    lens = torch.tensor(ctx, dtype=torch.int32, device=device)
    out = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5).view(B, n, Hq, D)
    assert torch.equal(out[1], torch.zeros_like(out[1])) and torch.equal(out[3], torch.zeros_like(out[3]))
    ref = oatt.paged_decode_attention(q.cpu(), kc.cpu(), vc.cpu(), lens.cpu(), tables.cpu(), D ** -0.5)
    mx, mean = error_stats(out, ref)
    assert mx <= MAX_ABS and mean <= MEAN_ABS


def test_batch_padding_invariance_bitwise(device):
    """Real rows alone vs padded to the graph bucket with empty sequences: bitwise equal (check_padding.py)."""
    Hq, Hkv, D, W, n = 32, 8, 128, 17, 5
    for b, p in [(3, 4), (5, 8), (10, 16), (24, 32), (40, 48)]:
        ctx = [300 + 97 * i for i in range(b)] + [0] * (p - b)
        kc, vc, tables = paged_cache(device, ctx, Hkv, D, W=W, seed=b)
        q = queries(device, p * n, Hq, D, seed=b + 1).view(p, n, Hq, D)
        lens = torch.tensor(ctx, dtype=torch.int32, device=device)
        alone = paged_decode_attention(q[:b], kc, vc, lens[:b], tables[:b], D ** -0.5)
        padded = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5)[:b * n]
        assert torch.equal(alone, padded), (b, p)


def test_spec_rows_equal_plain_decode_bitwise(device):
    """Verify row i (position L - n + i, sees L - n + i + 1 keys) == plain decode (n = 1) of the same query
    with context L - n + i + 1: the split layout and combine order depend only on the key positions."""
    Hq, Hkv, D, W = 32, 8, 128, 33
    ctx = [513, 1024, 1030, 4096, 700, 8000]
    for n in (2, 5, 9):
        B = len(ctx)
        kc, vc, tables = paged_cache(device, ctx, Hkv, D, W=W, seed=n)
        q = queries(device, B * n, Hq, D, seed=n + 1).view(B, n, Hq, D)
        lens = torch.tensor(ctx, dtype=torch.int32, device=device)
        spec = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5).view(B, n, Hq, D)
        for i in range(n):
            plain = paged_decode_attention(q[:, i:i + 1].contiguous(), kc, vc, lens - (n - 1 - i), tables, D ** -0.5)
            assert torch.equal(plain.view(B, Hq, D), spec[:, i]), (n, i)


@pytest.mark.parametrize("n", [2, 5, 9])
def test_batch_64_against_batches_of_16_bitwise(device, n):
    """B = 64 (eight-wave workgroups merging the residues in LDS; at n = 9 three row tiles, merged in two
    passes, with Q read from LDS) equals the same sequences in batches of 16 (four-wave workgroups, one per
    CU, partials merged by attn_combine; at n <= 5 two tiles in flight per wave) and plain decode of each
    row, bitwise."""
    Hq, Hkv, D, W = 32, 8, 128, 33
    rnd = random.Random(93 + n)
    ctx = [rnd.randint(1, 8192) for _ in range(64)]
    kc, vc, tables = paged_cache(device, ctx, Hkv, D, W=W, seed=93)
    q = queries(device, 64 * n, Hq, D, seed=94).view(64, n, Hq, D)
    lens = torch.tensor(ctx, dtype=torch.int32, device=device)
    full = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5)
    for b0 in range(0, 64, 16):
        part = paged_decode_attention(q[b0:b0 + 16], kc, vc, lens[b0:b0 + 16], tables[b0:b0 + 16], D ** -0.5)
        assert torch.equal(part, full[b0 * n:(b0 + 16) * n]), b0
    spec = full.view(64, n, Hq, D)
    for i in sorted({0, n // 2, n - 1}):
        plain = paged_decode_attention(q[:, i:i + 1].contiguous(), kc, vc, (lens - (n - 1 - i)).clamp_min(0), tables,
                                       D ** -0.5)
        ok = lens - (n - 1 - i) >= 1   # rows that see at least one key
        assert torch.equal(plain.view(64, Hq, D)[ok], spec[:, i][ok]), i


def test_repeatable_bitwise(device):
    ctx = [random.Random(3).randint(1024, 8192) for _ in range(16)]
    kc, vc, tables = paged_cache(device, ctx, 8, 128, W=33, seed=21)
    q = queries(device, 16 * 5, 32, 128, seed=22).view(16, 5, 32, 128)
    lens = torch.tensor(ctx, dtype=torch.int32, device=device)
    a = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5)
    b = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5)
    assert torch.equal(a, b)


@pytest.mark.parametrize("B", [16, 2])   # 2: the streaming kernel for few (sequence, head) pairs
def test_graph_capture_at_zero_lengths_then_replay(device, B):
    """Captured like capture_cudagraph (all context_lens 0, zero block tables), replayed with real metadata
    copied into the same buffers; every replay equals the eager result bitwise."""
    Hq, Hkv, D, W, n = 32, 8, 128, 33, 5
    rnd = random.Random(5)
    ctx_all = [[rnd.randint(1024, 8192) for _ in range(B)] for _ in range(3)]
    kc, vc, _ = paged_cache(device, [8192] * B, Hkv, D, W=W, seed=31, extra_blocks=64)
    q = torch.zeros(B, n, Hq, D, dtype=torch.bfloat16, device=device)
    lens = torch.zeros(B, dtype=torch.int32, device=device)
    tables = torch.zeros(B, W, dtype=torch.int32, device=device)
    out = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5)
    NB = kc.size(0)
    for it, ctx in enumerate(ctx_all):
        g = torch.Generator(device=device).manual_seed(40 + it)
        q.copy_(queries(device, B * n, Hq, D, seed=50 + it).view(B, n, Hq, D))
        lens.copy_(torch.tensor(ctx, dtype=torch.int32))
        tables.copy_(torch.randperm(NB, device=device, generator=g)[:B * W].view(B, W).to(torch.int32))
        graph.replay()
        eager = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), it


def test_planned_order_bitwise_and_stale_plan(device):
    """The planned call (sequences dispatched longest first) equals the unplanned call bitwise, for small
    and large batches (in-workgroup merge and partials + combine); a plan left from other context lengths of
    the same batch size changes nothing either."""
    from types import SimpleNamespace
    from nanovllm_amd.layers import attention as att
    rnd = random.Random(11)
    for B, n in ((64, 5), (16, 9), (3, 2)):
        ctx = [rnd.randint(1, 8192) for _ in range(B)]
        kc, vc, tables = paged_cache(device, ctx, 8, 128, W=33, seed=60 + B)
        q = queries(device, B * n, 32, 128, seed=61).view(B, n, 32, 128)
        lens = torch.tensor(ctx, dtype=torch.int32, device=device)
        ref = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5)
        owner = SimpleNamespace()
        planned = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5, plan_owner=owner)
        again = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5, plan_owner=owner)   # reused plan
        assert torch.equal(planned, ref) and torch.equal(again, ref), B
        # stale: plan for reversed lengths, then run with the real ones through the same owner and key
        rev = torch.tensor(ctx[::-1], dtype=torch.int32, device=device)
        lens.copy_(rev)
        paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5, plan_owner=owner)
        lens.copy_(torch.tensor(ctx, dtype=torch.int32, device=device))
        stale = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5, plan_owner=owner)
        assert any(plan[0] is owner for plan in att._decode_plans.values())
        assert torch.equal(stale, ref), B


@pytest.mark.parametrize("B,n", [(1, 1), (1, 5), (2, 9), (5, 13), (16, 5), (16, 13), (31, 1), (40, 13)])
def test_planned_few_pairs_equals_unplanned_bitwise(device, B, n):
    """Few (item, head) pairs (residue partials merged by attn_combine): the planned call (longest first)
    equals the unplanned one bitwise over several calls on one plan (the layers of a step, each on its own
    cache), with zero-length and one-key contexts among the sequences (stream kernel: B = 1, 2, 5; four-wave
    workgroups: B = 16, 31, 40; four row tiles: n = 13)."""
    from types import SimpleNamespace
    rnd = random.Random(B * 100 + n)
    ctx = [rnd.randint(1, 6000) for _ in range(B)]
    if B > 2:
        ctx[1], ctx[2] = 0, 1
    owner = SimpleNamespace()
    for layer in range(3):
        kc, vc, tables = paged_cache(device, ctx, 8, 128, W=24, seed=300 + layer)
        q = queries(device, B * n, 32, 128, seed=301 + layer).view(B, n, 32, 128)
        lens = torch.tensor(ctx, dtype=torch.int32, device=device)
        ref = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5)
        fused = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5, plan_owner=owner)
        torch.cuda.synchronize()
        print(f"B={B} n={n} layer {layer}: |out| {fused.float().abs().mean().item():.4f}", flush=True)
        assert torch.equal(fused, ref), (B, n, layer)
    if layer == 2 and B == 16 and n == 5:
        o = oatt.paged_decode_attention(q.cpu(), kc.cpu(), vc.cpu(), lens.cpu(), tables.cpu(), 128 ** -0.5)
        mx, mean = error_stats(fused.view(B, n, 32, 128), o)
        assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def test_planned_past_1024_sequences(device):
    """1100 sequences, more than the plan's 1024-thread sort (the dispatch order is then the index order, and
    the plan's scan takes two passes): the planned call equals the unplanned one bitwise, and a sample of
    sequences on both sides of index 1024 (one of them with no context) matches the oracle."""
    from types import SimpleNamespace
    B, n = 1100, 5
    rnd = random.Random(1100)
    ctx = [rnd.randint(n, 700) for _ in range(B)]
    ctx[3] = 0
    kc, vc, tables = paged_cache(device, ctx, 8, 128, seed=77)
    q = queries(device, B * n, 32, 128, seed=78).view(B, n, 32, 128)
    lens = torch.tensor(ctx, dtype=torch.int32, device=device)
    ref = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5)
    planned = paged_decode_attention(q, kc, vc, lens, tables, 128 ** -0.5, plan_owner=SimpleNamespace())
    torch.cuda.synchronize()
    assert torch.equal(planned, ref)
    sample = [0, 3, 511, 1023, 1024, 1099]
    skc, svc, st = sub_cache(kc, vc, tables, sample)
    o = oatt.paged_decode_attention(q[sample].cpu(), skc, svc, lens[sample].cpu(), st, 128 ** -0.5)
    mx, mean = error_stats(planned.view(B, n, 32, 128)[sample], o)
    print(f"B={B}: sample max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("B", [32, 8, 1])
def test_planned_graph_capture_replays(device, B):
    """Attention.forward's decode path (planned) captured at zero lengths, replayed with real metadata: the
    graph holds the plan and equals the eager result bitwise on every replay (B = 32: residues merged in
    the workgroup; 8 and 1: partials merged by attn_combine)."""
    from nanovllm_amd.utils.context import Context
    Hq, Hkv, D, W, n = 32, 8, 128, 33, 5
    rnd = random.Random(7)
    kc, vc, _ = paged_cache(device, [8192] * B, Hkv, D, W=W, seed=71, extra_blocks=64)
    q = torch.zeros(B, n, Hq, D, dtype=torch.bfloat16, device=device)
    lens = torch.zeros(B, dtype=torch.int32, device=device)
    tables = torch.zeros(B, W, dtype=torch.int32, device=device)
    ctx_obj = Context(False, context_lens=lens, block_tables=tables)
    out = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5, plan_owner=ctx_obj)   # warm-up
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5, plan_owner=ctx_obj)
    NB = kc.size(0)
    for it in range(3):
        ctx = [rnd.randint(1, 8192) for _ in range(B)]
        g = torch.Generator(device=device).manual_seed(80 + it)
        q.copy_(queries(device, B * n, Hq, D, seed=90 + it).view(B, n, Hq, D))
        lens.copy_(torch.tensor(ctx, dtype=torch.int32))
        tables.copy_(torch.randperm(NB, device=device, generator=g)[:B * W].view(B, W).to(torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        eager = paged_decode_attention(q, kc, vc, lens, tables, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), it
