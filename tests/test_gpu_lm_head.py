"""LM head + verifier in one call (HIP sd_lm_head_verify) on the GPU.

Bar: the logits are the bf16 rounding of the fp32 dot products (within one bf16 unit of float64 dot products
rounded to bf16, the library GEMM's contract); accepted counts and tokens equal the oracle's verify_drafts on
those same logits, exactly (greedy rows decided in the GEMM's epilogue without storing the logits, and sampled
rows through the stored logits), including the logits_indices gather, a vocabulary that is not a multiple of
the 256-row tile and more token rows than one workgroup holds.
"""
import pytest
import torch

from nanovllm_amd.layers.lm_head import LMHeadVerifier, lm_head_mixed, lm_head_sample, lm_head_verify
from oracle import sampler as osmp

pytestmark = pytest.mark.gpu


def _inputs(device, seed, S, K, V, H, N=None, gather=False):
    g = torch.Generator(device=device).manual_seed(seed)
    N = N or S * (K + 1)
    hidden = torch.randn(N, H, device=device, generator=g).to(torch.bfloat16)
    weight = (torch.randn(V, H, device=device, generator=g) * H ** -0.5 * 3).to(torch.bfloat16)
    idx = torch.randperm(N, device=device, generator=g)[:S * (K + 1)] if gather else None
    return hidden, weight, idx


def _ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    a = x.abs().float().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def _check_logits(hidden, weight, idx, logits, rows):
    """Rows `rows` of our logits against float64 dot products: within one bf16 unit of the value plus the
    fp32 accumulation bound H * 2^-24 * sum |h_k w_k| (which matters only where the sum cancels), and at least
    99.9 % equal to the float64 dot product rounded to bf16."""
    h = hidden.cpu().double() if idx is None else hidden.cpu().double()[idx.cpu()]
    w = weight.cpu().double()
    ref = (h[rows] @ w.T)
    mag = (h[rows].abs() @ w.abs().T)
    ours = logits.cpu()[rows].double()
    err = (ours - ref).abs()
    bound = _ulp_bf16(ref.float()).double() + h.size(1) * 2.0 ** -24 * mag
    worst = (err / bound).max().item()
    exact = (ours.float() == ref.float().to(torch.bfloat16).float()).float().mean().item()
    print(f"logits vs float64: worst {worst:.3f} of the bound, {exact * 100:.3f} % equal to the rounded float64",
          flush=True)
    assert worst <= 1.0 and exact >= 0.999


@pytest.mark.parametrize("S,K,V,H,gather", [(4, 3, 1000, 256, False), (3, 2, 777, 128, True), (70, 4, 2053, 192, True),
                                            (64, 4, 151936, 4096, False)])
def test_lm_head_verify_greedy_and_sampled(device, S, K, V, H, gather):
    hidden, weight, idx = _inputs(device, 7, S, K, V, H, N=S * (K + 1) + 5 if gather else None, gather=gather)
    head = LMHeadVerifier(weight)
    g = torch.Generator().manual_seed(8)
    logits_out = torch.empty(S * (K + 1), V, dtype=torch.bfloat16, device=device)
    zeros = torch.zeros(S, device=device)
    drafts = torch.randint(0, V, (S, K), generator=g).to(device)
    nd = torch.randint(0, K + 1, (S,), generator=g).to(device)
    # greedy, logits stored: gives the logits every check below uses
    a_st, t_st = lm_head_verify(hidden, head, drafts, nd, zeros, logits_indices=idx, logits_out=logits_out)
    logits = logits_out.cpu()
    rows = list(range(0, S * (K + 1), max(1, S * (K + 1) // 8)))
    _check_logits(hidden, weight, idx, logits, rows)
    # guesses that agree with the argmax for a part of the slots, so accept runs of every length occur
    top = logits.float().view(S, K + 1, V)[:, :K].argmax(-1)
    drafts = torch.where(torch.rand(S, K, generator=g) < 0.6, top, drafts.cpu()).to(device)
    a_ref, t_ref = osmp.verify_drafts(logits, drafts.cpu(), nd.cpu(), zeros.cpu())
    a0, t0 = lm_head_verify(hidden, head, drafts, nd, zeros, logits_indices=idx)          # fused, no logits
    assert a0.cpu().tolist() == a_ref.tolist() and t0.cpu().tolist() == t_ref.tolist()
    # sampled rows (mixed temperatures): through the stored logits
    temps = torch.tensor([0.0, 1.0, 0.7, 0.1] * S)[:S]
    u = torch.rand(S, K, generator=g)
    e = torch.empty(S, V).exponential_(1, generator=g)
    a1, t1 = lm_head_verify(hidden, head, drafts, nd, temps.to(device), logits_indices=idx, uniforms=u.to(device),
                            exp_noise=e.to(device))
    a_ref1, t_ref1 = osmp.verify_drafts(logits, drafts.cpu(), nd.cpu(), temps, uniforms=u, exp_noise=e)
    assert a1.cpu().tolist() == a_ref1.tolist() and t1.cpu().tolist() == t_ref1.tolist()
    print(f"S={S} K={K} V={V} H={H}: accepted {a0.cpu().tolist()[:8]}..., sampled {a1.cpu().tolist()[:8]}...",
          flush=True)


def test_lm_head_verify_against_library_gemm_logits(device):
    """At Qwen3-8B's LM head shape the logits equal the library GEMM's (F.linear, bf16) up to one bf16 unit."""
    S, K, V, H = 64, 4, 151936, 4096
    hidden, weight, _ = _inputs(device, 9, S, K, V, H)
    out = torch.empty(S * (K + 1), V, dtype=torch.bfloat16, device=device)
    lm_head_verify(hidden, LMHeadVerifier(weight), torch.zeros(S, K, dtype=torch.int64, device=device),
                   torch.zeros(S, dtype=torch.int64, device=device), torch.zeros(S, device=device), logits_out=out)
    lib = torch.nn.functional.linear(hidden, weight)
    same = (out == lib).float().mean().item()
    # both round an fp32 sum to bf16: they may differ by one bf16 unit where the sums straddle a rounding point,
    # and by more only where the sum cancels (|logit| far below the terms' magnitude)
    diff = (out.float() - lib.float()).abs()
    big = diff > _ulp_bf16(torch.maximum(out.float().abs(), lib.float().abs())) + 1e-3
    print(f"vs F.linear: {same * 100:.3f} % identical, {int(big.sum())} entries differ by more than one bf16 unit "
          f"+ 1e-3", flush=True)
    assert same >= 0.99 and int(big.sum()) == 0


def test_lm_head_verify_repeatable(device):
    """Two calls at Qwen3-8B's shape give bitwise equal logits and decisions: the vocabulary tiles of the GEMM's
    last round are computed in ranges of H whose fp32 sums are added in a fixed order."""
    S, K, V, H = 64, 4, 151936, 4096
    hidden, weight, _ = _inputs(device, 11, S, K, V, H)
    head = LMHeadVerifier(weight)
    drafts = torch.randint(0, V, (S, K), generator=torch.Generator().manual_seed(3)).to(device)
    nd = torch.full((S,), K, dtype=torch.int64, device=device)
    zeros = torch.zeros(S, device=device)
    outs = []
    for _ in range(2):
        out = torch.empty(S * (K + 1), V, dtype=torch.bfloat16, device=device)
        a, t = lm_head_verify(hidden, head, drafts, nd, zeros, logits_out=out)
        outs.append((out, a.cpu(), t.cpu()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])
    # the last 82 tiles (vocabulary rows from 131072 on) meet the same bar as the others
    _check_logits(hidden, weight[131072:], None, outs[0][0].cpu()[:, 131072:].contiguous(), [0, 100, 319])


def test_lm_head_logits_independent_of_row_count(device):
    """The same hidden rows give bitwise-equal logits and argmax in calls of M = 16, 64, 320, 325 and 640 token
    rows at Qwen3-8B's head shape (plain decode of 16 and 64 sequences, verify of 64, 65 and 128 sequences with
    k = 4): which vocabulary tiles are split along H, and into how many ranges, follows from (V, H) alone, and
    every row of workgroups applies it. Greedy speculative and plain decoding therefore see the same logits
    (the reference's padding check covers GEMMs too: scripts/check_padding.py:46-52)."""
    V, H, P = 151936, 4096, 16
    g = torch.Generator(device=device).manual_seed(21)
    hidden = torch.randn(700, H, device=device, generator=g).to(torch.bfloat16)
    weight = (torch.randn(V, H, device=device, generator=g) * H ** -0.5 * 3).to(torch.bfloat16)
    head = LMHeadVerifier(weight)
    first = None
    for S, K in [(16, 0), (64, 0), (64, 4), (65, 4), (128, 4)]:
        M = S * (K + 1)
        # the P probe rows first, then other rows in a shuffled order
        idx = torch.cat([torch.arange(P, device=device),
                         P + torch.randperm(700 - P, device=device, generator=g)[:M - P]])
        out = torch.empty(M, V, dtype=torch.bfloat16, device=device)
        zeros = torch.zeros(S, device=device)
        _, nxt = lm_head_verify(hidden, head, torch.zeros(S, K, dtype=torch.int64, device=device),
                                torch.zeros(S, dtype=torch.int64, device=device), zeros, logits_indices=idx,
                                logits_out=out)
        probe = out[:P].clone()
        if first is None:
            first = probe
            # K = 0: the next tokens are the rows' first argmax
            assert torch.equal(nxt.cpu(), probe.float().cpu().argmax(-1))
        same = torch.equal(probe, first)
        print(f"M={M}: probe rows {'bitwise equal' if same else 'DIFFER'} to M=16's", flush=True)
        assert same
        # the greedy path that never stores the logits agrees with the stored ones
        rows = torch.arange(0, M, K + 1, device=device)
        t = lm_head_sample(hidden, head, zeros, logits_indices=idx[rows])
        assert torch.equal(t.cpu(), out[rows].float().cpu().argmax(-1))


def test_lm_head_mixed_matches_separate_calls(device):
    """lm_head_mixed (verify rows of D decode requests plus P finished prefill chunks in one GEMM) gives the
    decisions of lm_head_verify on the decode rows and lm_head_sample on the prefill rows, greedy and sampled."""
    D, k, P, V, H = 48, 4, 3, 3000, 512
    N = D * (1 + k) + 700
    hidden, weight, _ = _inputs(device, 31, D, k, V, H, N=N)
    head = LMHeadVerifier(weight)
    g = torch.Generator().manual_seed(32)
    idx = torch.randperm(N, generator=g)[:D * (1 + k) + P].to(device)
    drafts = torch.randint(0, V, (D, k), generator=g).to(device)
    nd = torch.randint(0, k + 1, (D,), generator=g).to(device)
    for temps_d, temps_p in [(torch.zeros(D), torch.zeros(P)),
                             (torch.tensor([0.0, 1.0, 0.5] * 16), torch.tensor([0.0, 0.8, 1.0]))]:
        u = torch.rand(D + P, k, generator=g).to(device)
        e = torch.empty(D + P, V).exponential_(1, generator=g).to(device)
        a, t, f = lm_head_mixed(hidden, head, idx, D, drafts, nd, temps_d.to(device), temps_p.to(device),
                                uniforms=u, exp_noise=e)
        a_ref, t_ref = lm_head_verify(hidden, head, drafts, nd, temps_d.to(device),
                                      logits_indices=idx[:D * (1 + k)], uniforms=u[:D], exp_noise=e[:D])
        f_ref = lm_head_sample(hidden, head, temps_p.to(device), logits_indices=idx[D * (1 + k):],
                               exp_noise=e[D:])
        assert a.cpu().tolist() == a_ref.cpu().tolist() and t.cpu().tolist() == t_ref.cpu().tolist()
        assert f.cpu().tolist() == f_ref.cpu().tolist()
    # k = 0 (nothing to verify: one row per decode request)
    a, t, f = lm_head_mixed(hidden, head, idx[:D + P], D, None, None, torch.zeros(D, device=device),
                            torch.zeros(P, device=device))
    ref = lm_head_sample(hidden, head, torch.zeros(D + P, device=device), logits_indices=idx[:D + P])
    assert a.cpu().tolist() == [0] * D and (t.cpu().tolist() + f.cpu().tolist()) == ref.cpu().tolist()


def test_lm_head_bad_logits_index_marks_its_sequence(device):
    """An index outside the hidden rows makes its sequence's accepted count and token -1 (the reference's
    gather raises); the other sequences are decided as with valid indices, greedy and sampled."""
    S, K, V, H = 6, 3, 1000, 256
    N = S * (K + 1) + 4
    hidden, weight, idx = _inputs(device, 41, S, K, V, H, N=N, gather=True)
    head = LMHeadVerifier(weight)
    g = torch.Generator().manual_seed(42)
    drafts = torch.randint(0, V, (S, K), generator=g).to(device)
    nd = torch.full((S,), K, dtype=torch.int64, device=device)
    bad = idx.clone()
    bad[1 * (K + 1) + 2] = N          # sequence 1: past the table
    bad[4 * (K + 1)] = -3             # sequence 4: negative
    for temps in (torch.zeros(S), torch.tensor([0.0, 1.0, 0.5, 0.0, 1.0, 0.7])):
        u = torch.rand(S, K, generator=g).to(device)
        e = torch.empty(S, V).exponential_(1, generator=g).to(device)
        a_ok, t_ok = lm_head_verify(hidden, head, drafts, nd, temps.to(device), logits_indices=idx, uniforms=u,
                                    exp_noise=e)
        a, t = lm_head_verify(hidden, head, drafts, nd, temps.to(device), logits_indices=bad, uniforms=u, exp_noise=e)
        a, t, a_ok, t_ok = a.cpu(), t.cpu(), a_ok.cpu(), t_ok.cpu()
        for s in range(S):
            if s in (1, 4):
                assert a[s] == -1 and t[s] == -1
            else:
                assert a[s] == a_ok[s] and t[s] == t_ok[s]
