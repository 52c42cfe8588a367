"""LM head + verifier in one call (HIP sd_lm_head_verify) on the GPU.

Bar: the logits are the bf16 rounding of the fp32 dot products (within one bf16 unit of float64 dot products
rounded to bf16, the library GEMM's contract); accepted counts and tokens equal the oracle's verify_drafts on
those same logits, exactly (greedy rows decided in the GEMM's epilogue without storing the logits, and sampled
rows through the stored logits), including the logits_indices gather, a vocabulary that is not a multiple of
the 256-row tile and more token rows than one workgroup holds.
"""
import pytest
import torch

from nanovllm_amd.layers.lm_head import LMHeadVerifier, lm_head_verify
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
