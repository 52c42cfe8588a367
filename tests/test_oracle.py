"""Pins the CPU oracle (oracle/) independently of its own formulas (CPU only).

store_kvcache  brute-force per-row loop; -1 skip; strided value rows.
attention      textbook SDPA (float64, explicit boolean mask) over keys gathered token by token; planted
               values that expose a wrong causal offset, GQA head mapping or block-table lookup; varlen ==
               decode on the same sequences; fresh rows == paged cache; empty context -> zeros.
verify_drafts  the reference unit tests' known answers (tests/test_spec_unit.py:64-92), its zero-residual
               guard (:175-191) and TV-distance property (:137-172, including the deliberately wrong rule),
               and golden vectors written by the reference's own sampler.py (tests/golden/), at V = 512 and at
               the full 151,936-token vocabulary.
sample         closed form in float64 on tiny inputs; K = 0 verify equals sample.
"""
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import kvcache as okv
from oracle import sampler as osmp

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "verify_vectors.npz")
GOLDEN_FULL = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "verify_full_vocab.npz")


# ------------------------------------------------------------------ store_kvcache

def test_store_kvcache_bruteforce():
    g = torch.Generator().manual_seed(0)
    NB, bs, H, D, N = 6, 4, 2, 8, 13
    qkv = torch.randn(N, 3 * H * D, generator=g).to(torch.bfloat16)
    key = qkv[:, H * D:2 * H * D].view(N, H, D)            # strided views, like the qkv split
    value = qkv[:, 2 * H * D:].view(N, H, D)
    slots = torch.randperm(NB * bs, generator=g)[:N].to(torch.int32)
    slots[[2, 7, 11]] = -1
    kc = torch.zeros(NB, bs, H, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    okv.store_kvcache(key, value, kc, vc, slots)
    ek, ev = torch.zeros_like(kc), torch.zeros_like(vc)
    for i in range(N):
        s = int(slots[i])
        if s == -1:
            continue
        for h in range(H):
            for d in range(D):
                ek[s // bs, s % bs, h, d] = key[i, h, d]
                ev[s // bs, s % bs, h, d] = value[i, h, d]
    assert torch.equal(kc.view(torch.int16), ek.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), ev.view(torch.int16))
    assert int((kc != 0).any(-1).any(-1).sum()) == N - 3   # exactly the non-padding rows were written


# ------------------------------------------------------------------ attention

def _paged(g, B, ctx, Hkv, D, bs, extra_blocks=3, W=None):
    nblk = [math.ceil(c / bs) for c in ctx]
    NB = sum(nblk) + extra_blocks
    perm = torch.randperm(NB, generator=g)
    W = W or max(nblk)
    tables = torch.full((B, W), -1, dtype=torch.int32)
    at = 0
    for b in range(B):
        tables[b, :nblk[b]] = perm[at:at + nblk[b]].to(torch.int32)
        at += nblk[b]
    kc = torch.randn(NB, bs, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(NB, bs, Hkv, D, generator=g).to(torch.bfloat16)
    return kc, vc, tables


def _sdpa_reference(q, kc, vc, lens, tables, scale):
    """Per sequence / head: keys gathered one token at a time, float64 SDPA with a boolean mask."""
    B, n, Hq, D = q.shape
    Hkv, bs = kc.size(2), kc.size(1)
    out = torch.zeros(B, n, Hq, D, dtype=torch.float64)
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        keys = torch.stack([kc[int(tables[b, j // bs]), j % bs] for j in range(L)]).double()   # [L, Hkv, D]
        vals = torch.stack([vc[int(tables[b, j // bs]), j % bs] for j in range(L)]).double()
        for h in range(Hq):
            kvh = h // (Hq // Hkv)
            mask = torch.tensor([[j <= L - n + i for j in range(L)] for i in range(n)])
            out[b, :, h] = torch.nn.functional.scaled_dot_product_attention(
                q[b, :, h].double()[None], keys[:, kvh][None], vals[:, kvh][None], attn_mask=mask[None],
                scale=scale)[0]
    return out


def test_decode_matches_sdpa_config1_shapes():
    """Qwen3-0.6B shapes: 16 q / 8 kv heads, D 128, block 256, B 4, ctx {300,512,777,1024}, k=4 -> n=5."""
    g = torch.Generator().manual_seed(1)
    Hq, Hkv, D, bs, n = 16, 8, 128, 256, 5
    ctx = [300, 512, 777, 1024]
    kc, vc, tables = _paged(g, 4, ctx, Hkv, D, bs)
    q = torch.randn(4, n, Hq, D, generator=g).to(torch.bfloat16)
    lens = torch.tensor(ctx, dtype=torch.int32)
    scale = D ** -0.5
    got = oatt.paged_decode_attention(q, kc, vc, lens, tables, scale)
    ref = _sdpa_reference(q, kc, vc, lens, tables, scale)
    assert (got.double() - ref).abs().max().item() < 1e-5


def test_decode_planted_positions_and_heads():
    """Key j of kv head c carries score slope j; value = (j, c). A sharp softmax must return the last visible
    key (L - n + i) of the right kv head (h // g) through the right block: off-by-one causal offsets, h % Hkv
    head mappings and wrong page lookups all change the answer."""
    g = torch.Generator().manual_seed(2)
    Hq, Hkv, D, bs, n = 6, 2, 8, 4, 3
    ctx = [7, 10, 3]
    B = len(ctx)
    kc, vc, tables = _paged(g, B, ctx, Hkv, D, bs)
    kc.zero_()
    vc.zero_()
    for b in range(B):
        for j in range(ctx[b]):
            blk, off = int(tables[b, j // bs]), j % bs
            for c in range(Hkv):
                kc[blk, off, c, 0] = float(j)
                vc[blk, off, c, 1] = float(j)
                vc[blk, off, c, 2] = float(c)
    q = torch.zeros(B, n, Hq, D, dtype=torch.bfloat16)
    q[..., 0] = 64.0
    got = oatt.paged_decode_attention(q, kc, vc, torch.tensor(ctx, dtype=torch.int32), tables, 1.0)
    for b in range(B):
        for i in range(n):
            for h in range(Hq):
                assert got[b, i, h, 1].item() == pytest.approx(ctx[b] - n + i, abs=1e-3)
                assert got[b, i, h, 2].item() == pytest.approx(h // (Hq // Hkv), abs=1e-3)


def test_decode_zero_context_gives_zeros():
    g = torch.Generator().manual_seed(3)
    kc, vc, tables = _paged(g, 2, [5, 1], 2, 8, 4)
    q = torch.randn(2, 1, 4, 8, generator=g).to(torch.bfloat16)
    got = oatt.paged_decode_attention(q, kc, vc, torch.tensor([5, 0], dtype=torch.int32), tables, 0.3)
    assert torch.equal(got[1], torch.zeros_like(got[1]))
    assert got[0].abs().sum() > 0


def test_varlen_paged_equals_decode():
    g = torch.Generator().manual_seed(4)
    Hq, Hkv, D, bs, n = 8, 2, 16, 8, 4
    ctx = [9, 23, 4, 16]
    kc, vc, tables = _paged(g, 4, ctx, Hkv, D, bs)
    q = torch.randn(4, n, Hq, D, generator=g).to(torch.bfloat16)
    lens = torch.tensor(ctx, dtype=torch.int32)
    dec = oatt.paged_decode_attention(q, kc, vc, lens, tables, 0.25)
    cu_q = torch.arange(0, 4 * n + 1, n, dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(ctx).tolist(), dtype=torch.int32)
    var = oatt.varlen_attention(q.view(4 * n, Hq, D), kc, vc, cu_q, cu_k, 0.25, tables)
    assert torch.equal(var.view(4, n, Hq, D), dec)


def test_varlen_fresh_equals_paged():
    """Prefill without a block table (fresh k/v rows) equals the same keys read back from the paged cache."""
    g = torch.Generator().manual_seed(5)
    Hq, Hkv, D, bs = 4, 2, 16, 8
    lq, lk = [5, 12, 1], [5, 12, 1]
    Nk = sum(lk)
    k = torch.randn(Nk, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(Nk, Hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(sum(lq), Hq, D, generator=g).to(torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum(lq).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(lk).tolist(), dtype=torch.int32)
    kc, vc, tables = _paged(g, 3, lk, Hkv, D, bs)
    slots = []
    for s in range(3):
        slots += [int(tables[s, j // bs]) * bs + j % bs for j in range(lk[s])]
    okv.store_kvcache(k, v, kc, vc, torch.tensor(slots, dtype=torch.int32))
    fresh = oatt.varlen_attention(q, k, v, cu_q, cu_k, 0.5)
    paged = oatt.varlen_attention(q, kc, vc, cu_q, cu_k, 0.5, tables)
    assert torch.equal(fresh, paged)
    # a prefill query i of a fresh sequence sees exactly keys 0..i
    s0 = torch.nn.functional.scaled_dot_product_attention(
        q[:5].transpose(0, 1).double(), k[:5].repeat_interleave(2, 1).transpose(0, 1).double(),
        v[:5].repeat_interleave(2, 1).transpose(0, 1).double(), is_causal=True, scale=0.5).transpose(0, 1)
    assert (fresh[:5].double() - s0).abs().max() < 1e-5


# ------------------------------------------------------------------ verify_drafts

def _logits_with_top1(top1, V=10, seed=0):
    g = torch.Generator().manual_seed(seed)
    top1 = torch.tensor(top1)
    logits = torch.randn(*top1.shape, V, generator=g)
    logits.scatter_(-1, top1.unsqueeze(-1), 100.0)
    return logits.view(-1, V)


def test_verify_greedy_known_answers():
    """tests/test_spec_unit.py:72-92 of the reference, re-expressed."""
    drafts = torch.tensor([[3, 4, 5], [3, 9, 5], [1, 4, 5], [3, 4, 5]])
    top1 = [[3, 4, 5, 6]] * 4
    nd = torch.tensor([3, 3, 3, 1])
    a, t = osmp.verify_drafts(_logits_with_top1(top1), drafts, nd, torch.zeros(4))
    assert a.tolist() == [3, 1, 0, 1] and t.tolist() == [6, 4, 3, 4]
    a, t = osmp.verify_drafts(_logits_with_top1([[7], [2]]), torch.zeros(2, 0, dtype=torch.int64),
                              torch.zeros(2, dtype=torch.int64), torch.zeros(2))
    assert a.tolist() == [0, 0] and t.tolist() == [7, 2]
    temps = torch.tensor([0.0, 1.0, 0.0, 1.0])
    g = torch.Generator().manual_seed(1)
    for _ in range(20):
        u = torch.rand(4, 3, generator=g)
        e = torch.empty(4, 10).exponential_(1, generator=g)
        a, t = osmp.verify_drafts(_logits_with_top1(top1), drafts, nd, temps, uniforms=u, exp_noise=e)
        assert a[0] == 3 and t[0] == 6 and a[2] == 0 and t[2] == 3


def test_verify_zero_residual_guard():
    """p == q and every guess rejected (u = 1): the all-zero residual must not emit token 0 (sampler.py:98)."""
    g = torch.Generator().manual_seed(2)
    V, K, S = 6, 2, 4
    logits = torch.randn(S, K + 1, V, generator=g)
    logits[..., 0] = -float("inf")
    drafts = torch.full((S, K), 3)
    e = torch.empty(S, V).exponential_(1, generator=g)
    a, t = osmp.verify_drafts(logits.view(-1, V), drafts, torch.full((S,), K), torch.ones(S),
                              logits[:, :K].clone(), uniforms=torch.ones(S, K), exp_noise=e)
    assert a.tolist() == [0] * S and bool((t != 0).all())


def _run_trials(p_logits, T, draft_probs, n, verify, gen, pass_q=True):
    K, V = draft_probs.shape
    drafts = torch.multinomial(draft_probs, n, replacement=True, generator=gen).T.contiguous()
    logits = p_logits.unsqueeze(0).expand(n, -1, -1).reshape(n * (K + 1), -1)
    one_hot = bool((draft_probs.max(-1).values == 1).all())
    q = None if one_hot or not pass_q else (T * draft_probs.log()).unsqueeze(0).expand(n, -1, -1)
    u = torch.rand(n, K, generator=gen)
    e = torch.empty(n, V).exponential_(1, generator=gen)
    a, t = verify(logits, drafts, torch.full((n,), K), torch.full((n,), T), q, u, e, gen)
    out = torch.cat([drafts, torch.zeros(n, 1, dtype=torch.int64)], 1)
    out[torch.arange(n), a] = t
    return out, a + 1


def _max_tv(p_logits, T, out, lengths):
    V = p_logits.size(-1)
    worst = 0.0
    for j in range(p_logits.size(0)):
        mask = lengths > j
        m = int(mask.sum())
        if m < 20000:
            continue
        emp = torch.bincount(out[mask, j], minlength=V).double() / m
        p = torch.softmax(p_logits[j].double() / T, -1)
        worst = max(worst, 0.5 * (emp - p).abs().sum().item())
    return worst


def _oracle_rule(logits, drafts, nd, temps, q, u, e, gen):
    return osmp.verify_drafts(logits, drafts, nd, temps, q, uniforms=u, exp_noise=e)


def _wrong_rule(logits, drafts, nd, temps, q, u, e, gen):
    """Deliberately wrong (reference test_spec_unit.py:129-134): after a rejection sample from p itself."""
    n, K = drafts.shape
    a, _ = osmp.verify_drafts(logits, drafts, nd, temps, q, uniforms=u, exp_noise=e)
    last = logits.view(n, K + 1, -1)[torch.arange(n), a].float() / temps[:, None]
    return a, torch.multinomial(torch.softmax(last, -1), 1, generator=gen).squeeze(1)


def test_verify_distribution_tv():
    """Speculative sampling reproduces p token by token: worst TV < 0.02 over 200k trials (reference
    tests/test_spec_unit.py:137-172); the wrong rule must exceed 0.06 so the test has power."""
    g = torch.Generator().manual_seed(0)
    V, K, n, T = 8, 3, 200000, 0.7
    p_logits = torch.randn(K + 1, V, generator=g) * 1.5
    p = torch.softmax(p_logits / T, -1)
    guesses = (p - 0.3).abs().argmin(-1)[:K]
    one_hot = torch.nn.functional.one_hot(guesses, V).float()
    q = torch.softmax(p_logits[:K] / T + torch.randn(K, V, generator=g), -1)
    for draft_probs in (one_hot, q):
        out, lengths = _run_trials(p_logits, T, draft_probs, n, _oracle_rule, g)
        assert _max_tv(p_logits, T, out, lengths) < 0.02
        out, lengths = _run_trials(p_logits, T, draft_probs, n, _wrong_rule, g)
        assert _max_tv(p_logits, T, out, lengths) > 0.06


def _golden_cases():
    data = np.load(GOLDEN)
    names = sorted({k.split(".")[0] for k in data.files})
    return data, names


def golden_case(data, name):
    """Tensors of one golden case (bf16 stored as uint16 bits)."""
    def get(key, bf16=False):
        arr = data[f"{name}.{key}"]
        if bf16:
            return torch.from_numpy(arr.view(np.int16).copy()).view(torch.bfloat16)
        return torch.from_numpy(arr.copy())
    bf16 = int(data[f"{name}.dtype"]) == 0
    dl = data[f"{name}.draft_logits"]
    return dict(logits=get("logits", bf16), drafts=get("drafts"), num_drafts=get("num_drafts"), temps=get("temps"),
                draft_logits=None if dl.size == 0 else get("draft_logits", bf16), uniforms=get("uniforms"),
                noise=get("noise"), num_accepted=get("num_accepted"), next_token=get("next_token"))


def test_verify_golden_vectors_from_reference():
    data, names = _golden_cases()
    assert len(names) >= 7
    for name in names:
        c = golden_case(data, name)
        a, t = osmp.verify_drafts(c["logits"], c["drafts"], c["num_drafts"], c["temps"], c["draft_logits"],
                                  uniforms=c["uniforms"], exp_noise=c["noise"])
        assert a.tolist() == c["num_accepted"].tolist(), name
        assert t.tolist() == c["next_token"].tolist(), name


@pytest.mark.parametrize("name", ["t0_f32_ngram", "t1_f32_draft", "t1_bf16_draft_ragged", "t005_f32_draft_masked",
                                  "t01_bf16_ngram_masked", "mixed_f32_draft_ragged", "k0_f32_sample",
                                  "zero_residual_t1_f32", "t0_bf16_draft_ragged", "t1_f32_ngram_ragged"])
def test_verify_full_vocab_goldens_from_reference(name):
    """Full-vocabulary outputs of the reference's sampler.py (inputs regenerated from seeds)."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import verify_inputs
    data = np.load(GOLDEN_FULL)
    c = verify_inputs.make_case(name)
    assert verify_inputs.checksum(c) == str(data[f"{name}.checksum"])
    logits, drafts, nd, temps, dl, u, e = c
    a, t = osmp.verify_drafts(logits, drafts, nd, temps, dl, uniforms=u, exp_noise=e)
    assert a.tolist() == data[f"{name}.num_accepted"].tolist()
    assert t.tolist() == data[f"{name}.next_token"].tolist()


# ------------------------------------------------------------------ sample

def test_sample_closed_form():
    g = torch.Generator().manual_seed(7)
    S, V = 16, 50
    logits = torch.randn(S, V, generator=g) * 2
    temps = torch.tensor([0.0, 1.0, 0.5, 2.0] * 4)
    e = torch.empty(S, V).exponential_(1, generator=g)
    got = osmp.sample(logits, temps, e)
    for s in range(S):
        if temps[s] == 0:
            assert got[s] == int(torch.argmax(logits[s]))
        else:
            x = logits[s].double() / float(temps[s])
            p = torch.exp(x - x.max())
            p = p / p.sum()
            assert got[s] == int(torch.argmax(p / e[s].double().clamp_min(1e-10)))
    a, t = osmp.verify_drafts(logits, torch.zeros(S, 0, dtype=torch.int64), torch.zeros(S, dtype=torch.int64), temps,
                              uniforms=torch.zeros(S, 0), exp_noise=e)
    assert torch.equal(t, got) and a.tolist() == [0] * S


# ------------------------------------------------------------------ draft-step inputs

def test_draft_step_inputs_bruteforce():
    """Per-sequence loop in plain Python (model_runner.py:446-452 read one sequence at a time): padding
    sequences (context length 0) get position 0, slot -1, length 0; block boundaries cross to the next
    table entry; rows past S keep input id 0."""
    from oracle import draft_inputs as odi
    g = torch.Generator().manual_seed(9)
    B, S, W, bs = 12, 9, 5, 16
    tables = torch.randperm(100, generator=g)[:B * W].view(B, W).to(torch.int32)
    real_lens = torch.tensor([5, 17, 0, 31, 1, 64, 16, 0, 33, 2, 47, 0], dtype=torch.int32)
    last_pos = torch.tensor([3, 15, 7, 30, 0, 60, 14, 0, 31, 0, 45, 2], dtype=torch.int64)
    tokens = torch.randint(0, 1000, (S,), generator=g)
    for j in (1, 2, 3):
        ids, pos, slots, lens = odi.draft_step_inputs(real_lens, last_pos, tables, bs, tokens, j)
        assert ids.dtype == torch.int64 and pos.dtype == torch.int64
        assert slots.dtype == torch.int32 and lens.dtype == torch.int32
        for b in range(B):
            if int(real_lens[b]) > 0:
                p = int(last_pos[b]) + j
                assert int(pos[b]) == p and int(lens[b]) == p + 1
                assert int(slots[b]) == int(tables[b, p // bs]) * bs + p % bs
            else:
                assert int(pos[b]) == 0 and int(slots[b]) == -1 and int(lens[b]) == 0
            assert int(ids[b]) == (int(tokens[b]) if b < S else 0)
    # position 15 + 1 = 16 is the first slot of the second block
    _, pos, slots, _ = odi.draft_step_inputs(real_lens, last_pos, tables, bs, tokens, 1)
    assert int(pos[1]) == 16 and int(slots[1]) == int(tables[1, 1]) * bs
