"""Varlen prefill and mixed prefill+decode attention on the GPU (HIP sd_varlen_attention) against the
fp32 oracle (max-abs <= 2e-2, mean-abs <= 2e-3), plus the bitwise identity of a mixed step's decode rows
with the decode kernel's rows (so greedy tokens do not depend on whether a step was mixed)."""
import math
import random

import numpy as np
import pytest
import torch

from nanovllm_amd.engine.synthetic import mixed_step_lengths as mixed_step
from nanovllm_amd.layers.attention import paged_decode_attention, varlen_attention
from oracle import attention as oatt
from attn_cases import BLOCK, error_stats, paged_cache, queries, sub_cache

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _cu(lengths, device):
    return torch.tensor([0] + np.cumsum(lengths).tolist(), dtype=torch.int32, device=device)


def _check(out, ref, what):
    mx, mean = error_stats(out, ref)
    print(f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (what, mx, mean)


def test_prefill_fresh_rows_strided(device):
    """Plain prefill: no block table, k / v are strided views of a fused qkv tensor (row stride 6144)."""
    Hq, Hkv, D = 32, 8, 128
    lens = [1, 17, 64, 100, 300, 613]
    N = sum(lens)
    g = torch.Generator(device=device).manual_seed(0)
    qkv = torch.randn(N, (Hq + 2 * Hkv) * D, device=device, generator=g).to(torch.bfloat16)
    q = qkv[:, :Hq * D].view(N, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D)
    cu = _cu(lens, device)
    out = varlen_attention(q, k, v, cu, cu, max(lens), max(lens), D ** -0.5)
    ref = oatt.varlen_attention(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), D ** -0.5)
    _check(out, ref, "prefill fresh")


def test_prefix_cache_chunks(device):
    """Chunked prefill over the paged cache: Lq new rows after Lk - Lq cached keys."""
    Hq, Hkv, D = 32, 8, 128
    pairs = [(50, 306), (220, 732), (1, 1000), (5, 600), (256, 256), (129, 1153), (700, 2100)]
    lq = [a for a, _ in pairs]
    lk = [b for _, b in pairs]
    kc, vc, tables = paged_cache(device, lk, Hkv, D, seed=3)
    q = queries(device, sum(lq), Hq, D, seed=4)
    cu_q, cu_k = _cu(lq, device), _cu(lk, device)
    out = varlen_attention(q, kc, vc, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables)
    ref = oatt.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), cu_q.cpu(), cu_k.cpu(), D ** -0.5, tables.cpu())
    _check(out, ref, "prefix-cache chunks")


def test_mixed_step_vs_oracle_and_decode_rows_bitwise(device):
    Hq, Hkv, D, k = 32, 8, 128, 4
    lq, lk = mixed_step(0)
    kc, vc, tables = paged_cache(device, lk, Hkv, D, W=math.ceil(max(lk) / BLOCK), seed=5)
    q = queries(device, sum(lq), Hq, D, seed=6)
    cu_q, cu_k = _cu(lq, device), _cu(lk, device)
    out = varlen_attention(q, kc, vc, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables)
    ref = oatt.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), cu_q.cpu(), cu_k.cpu(), D ** -0.5, tables.cpu())
    _check(out, ref, f"mixed step ({sum(lq)} query tokens)")
    nd = 48
    dec = paged_decode_attention(q[:nd * (1 + k)].view(nd, 1 + k, Hq, D), kc, vc,
                                 torch.tensor(lk[:nd], dtype=torch.int32, device=device), tables[:nd], D ** -0.5)
    assert torch.equal(dec, out[:nd * (1 + k)])


def test_varlen_edge_lengths(device):
    """Zero-length queries, keys shorter than queries (rows that see nothing -> zeros), GQA 2 and 8."""
    D = 128
    for Hq, Hkv in ((16, 8), (16, 2)):
        lq = [0, 3, 40, 1, 17, 10]
        lk = [5, 3, 600, 1, 513, 4]
        kc, vc, tables = paged_cache(device, lk, Hkv, D, seed=Hq + Hkv)
        q = queries(device, sum(lq), Hq, D, seed=9)
        cu_q, cu_k = _cu(lq, device), _cu(lk, device)
        out = varlen_attention(q, kc, vc, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables)
        ref = oatt.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), cu_q.cpu(), cu_k.cpu(), D ** -0.5, tables.cpu())
        _check(out, ref, f"edge lengths Hq={Hq} Hkv={Hkv}")


def test_random_varlen_batches(device):
    rnd = random.Random(11)
    Hq, Hkv, D = 32, 8, 128
    for trial in range(3):
        n = rnd.randint(1, 12)
        lq = [rnd.choice([1, 5, rnd.randint(1, 300)]) for _ in range(n)]
        lk = [a + rnd.randint(0, 1500) for a in lq]
        kc, vc, tables = paged_cache(device, lk, Hkv, D, seed=20 + trial)
        q = queries(device, sum(lq), Hq, D, seed=30 + trial)
        cu_q, cu_k = _cu(lq, device), _cu(lk, device)
        out = varlen_attention(q, kc, vc, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables)
        ref = oatt.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), cu_q.cpu(), cu_k.cpu(), D ** -0.5, tables.cpu())
        _check(out, ref, f"random batch {trial}")


def test_plan_past_1024_sequences(device):
    """1100 sequences, more than the plan's 1024-thread sort (work lists in index order, built in two scan
    passes): verify rows, single decode rows and three prefill chunks after cached keys in one mixed launch.
    A sample on both sides of index 1024 against the oracle, and the first 1000 sequences' rows bitwise equal
    to a call with those 1000 alone (sorted dispatch order): the order only changes which workgroup computes
    an item."""
    Hq, Hkv, D = 32, 8, 128
    rnd = np.random.default_rng(5)
    B = 1100
    lq = rnd.choice([1, 5, 5, 5], B).tolist()
    for i in (7, 512, 1050):
        lq[i] = 40
    lk = [a + int(rnd.integers(0, 300)) for a in lq]
    kc, vc, tables = paged_cache(device, lk, Hkv, D, seed=41)
    q = queries(device, sum(lq), Hq, D, seed=42)
    cu_q, cu_k = _cu(lq, device), _cu(lk, device)
    out = varlen_attention(q, kc, vc, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables)
    first = 1000
    r1 = int(cu_q[first])
    alone = varlen_attention(q[:r1], kc, vc, cu_q[:first + 1], cu_k[:first + 1], max(lq[:first]), max(lk[:first]),
                             D ** -0.5, tables[:first])
    torch.cuda.synchronize()
    assert torch.equal(alone, out[:r1])
    cq = cu_q.cpu().tolist()
    for s in (0, 7, 512, 1023, 1024, 1050, 1099):
        skc, svc, st = sub_cache(kc, vc, tables, [s])
        ref = oatt.varlen_attention(q[cq[s]:cq[s + 1]].cpu(), skc, svc, torch.tensor([0, lq[s]]), torch.tensor([0, lk[s]]),
                                    D ** -0.5, st)
        _check(out[cq[s]:cq[s + 1]], ref, f"sequence {s}: {lq[s]} queries, {lk[s]} keys")


def test_prefill_rows_chunk_invariant_bitwise(device):
    """A prefill row's result depends only on its own keys: the same 700-token sequence prefilled as one
    chunk, as 300 + 400, or beside other sequences gives bitwise equal rows (sequences longer than 16 queries
    take the prefill kernel, whose reduction order is fixed by key positions)."""
    Hq, Hkv, D, L = 32, 8, 128, 700
    kc, vc, tables = paged_cache(device, [L], Hkv, D, seed=12)
    q = queries(device, L, Hq, D, seed=13)

    def run(lq, lk, qrows, tb):
        return varlen_attention(qrows, kc, vc, _cu(lq, device), _cu(lk, device), max(lq), max(lk), D ** -0.5, tb)

    whole = run([L], [L], q, tables)
    first = run([300], [300], q[:300], tables)
    second = run([400], [L], q[300:], tables)
    assert torch.equal(whole[:300], first)
    assert torch.equal(whole[300:], second)
    # beside a decode sequence and another chunk of the same sequence
    mixed = run([5, 400, 300], [L, L, 300], torch.cat([q[300:305], q[300:], q[:300]]), tables.repeat(3, 1))
    assert torch.equal(mixed[5:405], second) and torch.equal(mixed[405:], first)
    ref = oatt.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), _cu([L], "cpu"), _cu([L], "cpu"), D ** -0.5,
                                tables.cpu())
    _check(whole, ref, "700-token prefill")


@pytest.mark.parametrize("paged", [True, False])
def test_prefill_only_and_mixed_calls_agree_bitwise(device, paged):
    """A call with prefill chunks only and the same chunks beside a 5-query sequence (a mixed launch, whose
    residue items share the grid) give bitwise equal prefill rows: chunks of 1000 queries after 1100 cached
    keys (q-blocks across the causal diagonal), 37 and 300 queries (partial q-blocks), fresh or paged keys."""
    Hq, Hkv, D = 32, 8, 128
    lq, lk = [1000, 37, 300], [2100, 37, 300]
    if paged:
        kc, vc, tables = paged_cache(device, lk + [lk[0]], Hkv, D, seed=21)
        k = v = None
    else:
        g = torch.Generator(device=device).manual_seed(21)
        k = torch.randn(sum(lk) + lk[0], Hkv, D, device=device, generator=g).to(torch.bfloat16)
        v = torch.randn(sum(lk) + lk[0], Hkv, D, device=device, generator=g).to(torch.bfloat16)
    q = queries(device, sum(lq) + 5, Hq, D, seed=22)

    # sequence j's keys: table row j (paged), or rows off[j] .. off[j] + lk[j] of k / v; sequence 3 (the
    # 5-query one) has chunk 0's key count in its own rows
    lens = lk + [lk[0]]
    off = np.cumsum([0] + lens).tolist()

    def run(lq_, seqs, qrows):
        lk_ = [lens[j] for j in seqs]
        if paged:
            return varlen_attention(qrows, kc, vc, _cu(lq_, device), _cu(lk_, device), max(lq_), max(lk_),
                                    D ** -0.5, tables[seqs])
        keys = torch.cat([k[off[j]:off[j] + lens[j]] for j in seqs])
        vals = torch.cat([v[off[j]:off[j] + lens[j]] for j in seqs])
        return varlen_attention(qrows, keys, vals, _cu(lq_, device), _cu(lk_, device), max(lq_), max(lk_),
                                D ** -0.5)

    alone = run(lq, [0, 1, 2], q[:sum(lq)])
    mixed = run([5] + lq, [3, 0, 1, 2], torch.cat([q[sum(lq):], q[:sum(lq)]]))
    assert torch.equal(mixed[5:], alone)
    lq_cpu, lk_cpu = _cu(lq, "cpu"), _cu(lk, "cpu")
    if paged:
        ref = oatt.varlen_attention(q[:sum(lq)].cpu(), kc.cpu(), vc.cpu(), lq_cpu, lk_cpu, D ** -0.5,
                                    tables[[0, 1, 2]].cpu())
    else:
        ref = oatt.varlen_attention(q[:sum(lq)].cpu(), k[:sum(lk)].cpu(), v[:sum(lk)].cpu(), lq_cpu, lk_cpu,
                                    D ** -0.5)
    _check(alone, ref, f"prefill-only call ({'paged' if paged else 'fresh'} keys)")


def test_plan_reuse_across_layers(device):
    """The step's work lists are planned once per owner (the step's Context) and reused by later layers:
    bitwise equal to unplanned calls; a different owner replans, and so does the first owner afterwards
    because its plan was replaced in the workspace."""
    from nanovllm_amd.layers import attention as att
    from nanovllm_amd.utils.context import Context
    Hq, Hkv, D = 32, 8, 128
    lq, lk = mixed_step(3)
    kc, vc, tables = paged_cache(device, lk, Hkv, D, W=math.ceil(max(lk) / BLOCK), seed=14)
    q = queries(device, sum(lq), Hq, D, seed=15)
    cu_q, cu_k = _cu(lq, device), _cu(lk, device)
    args = (q, kc, vc, cu_q, cu_k, max(lq), max(lk), D ** -0.5, tables)
    ref = varlen_attention(*args)
    owner = Context(True, cu_q, cu_k, max(lq), max(lk))   # the step's Context (a slotted dataclass)
    plans0, reuses0 = att.plan_stats["plans"], att.plan_stats["reuses"]
    for _ in range(3):
        assert torch.equal(varlen_attention(*args, plan_owner=owner), ref)
    assert att.plan_stats["plans"] - plans0 == 1 and att.plan_stats["reuses"] - reuses0 == 2
    lq2, lk2 = [5] * 8 + [40], [300] * 8 + [90]
    kc2, vc2, tb2 = paged_cache(device, lk2, Hkv, D, seed=16)
    q2 = queries(device, sum(lq2), Hq, D, seed=17)
    other = Context(True)
    out2 = varlen_attention(q2, kc2, vc2, _cu(lq2, device), _cu(lk2, device), max(lq2), max(lk2), D ** -0.5, tb2,
                            plan_owner=other)
    assert torch.equal(out2, varlen_attention(q2, kc2, vc2, _cu(lq2, device), _cu(lk2, device), max(lq2),
                                              max(lk2), D ** -0.5, tb2))
    plans1 = att.plan_stats["plans"]
    assert torch.equal(varlen_attention(*args, plan_owner=owner), ref)
    assert att.plan_stats["plans"] == plans1 + 1
