"""Rejection sampler / token sampler on the GPU (HIP sd_verify_drafts, sd_sample).

Bar: accepted counts and emitted tokens identical to the reference rule given the same uniforms and
exponential noise. Checked against
  (1) golden outputs of the reference's own sampler.py: the small vectors (V = 512) and the full-vocabulary
      cases (64 sequences, 4 slots, 151,936 tokens; T 0 / 0.05 / 0.1 / 0.5-2; fp32 and bf16; n-gram and
      draft-model guesses; ragged num_drafts; -inf masks), exactly, with no tolerance;
  (2) the oracle on further seeded full-vocabulary batches, exactly, except decisions that the oracle itself
      takes within 4 fp32 ulps of flipping (see _near_boundary); their count is printed and must be zero or
      one per batch;
  (3) the reference unit tests' known answers, zero-residual guard and total-variation property.
"""
import math
import os
import sys

import numpy as np
import pytest
import torch

from nanovllm_amd.layers.sampler import Sampler, verify_drafts
from oracle import sampler as osmp
from test_oracle import _logits_with_top1, _max_tv, golden_case

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import verify_inputs  # noqa: E402

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "verify_vectors.npz")
GOLDEN_FULL = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "verify_full_vocab.npz")
ULPS = 4


def test_golden_vectors_exact(device):
    data = np.load(GOLDEN)
    names = sorted({k.split(".")[0] for k in data.files})
    for name in names:
        c = golden_case(data, name)
        dl = c["draft_logits"]
        a, t = verify_drafts(c["logits"].to(device), c["drafts"].to(device), c["num_drafts"].to(device),
                             c["temps"].to(device), None if dl is None else dl.to(device),
                             uniforms=c["uniforms"].to(device), exp_noise=c["noise"].to(device))
        assert a.cpu().tolist() == c["num_accepted"].tolist(), name
        assert t.cpu().tolist() == c["next_token"].tolist(), name


@pytest.mark.parametrize("name", list(verify_inputs.CASES))
def test_golden_full_vocab_exact(device, name):
    """The reference's sampler.py outputs at the full vocabulary, regenerated inputs, no tolerance."""
    data = np.load(GOLDEN_FULL)
    logits, drafts, nd, temps, dl, u, e = verify_inputs.make_case(name)
    assert verify_inputs.checksum((logits, drafts, nd, temps, dl, u, e)) == str(data[f"{name}.checksum"]), \
        "regenerated inputs differ from the ones the golden outputs were written for"
    a, t = verify_drafts(logits.to(device), drafts.to(device), nd.to(device), temps.to(device),
                         None if dl is None else dl.to(device), uniforms=u.to(device), exp_noise=e.to(device))
    a, t = a.cpu(), t.cpu()
    ra, rt = torch.from_numpy(data[f"{name}.num_accepted"]), torch.from_numpy(data[f"{name}.next_token"])
    bad = ((a != ra) | (t != rt)).nonzero().flatten().tolist()
    print(f"{name}: {drafts.size(0)} sequences, mismatches {len(bad)} {bad}", flush=True)
    assert not bad


def _config4(seed, T, dtype, with_draft, S=64, K=4, V=151936, ragged=False, offset=0.0, masked=False):
    """Target and draft logits ~ N(offset, 3); 5% of rows get the draft's argmax planted in the target;
    optionally 30 % of the entries of every fourth row and the first 40,000 of every seventh row -inf."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(S, K + 1, V, generator=g) * 3 + offset
    draft_logits = torch.randn(S, K, V, generator=g) * 3 + offset
    if T == 0:
        drafts = draft_logits.argmax(-1)
    else:
        drafts = torch.multinomial(torch.softmax(draft_logits.view(-1, V) / T, -1), 1, generator=g).view(S, K)
    plant = torch.rand(S, K, generator=g) < 0.05
    for s, j in plant.nonzero().tolist():
        logits[s, j, drafts[s, j]] = logits[s, j].max() + 1.0
    # make a few guesses agree with the target's argmax so accept runs of every length occur
    agree = torch.rand(S, K, generator=g) < 0.6
    top = logits[:, :K].argmax(-1)
    drafts = torch.where(agree & (torch.rand(S, K, generator=g) < 0.5), top, drafts)
    if masked:
        rows = torch.rand(S, K + 1, generator=g) < 0.25
        keep = logits.gather(-1, torch.cat([drafts, drafts[:, :1]], 1).unsqueeze(-1))
        logits[rows] = logits[rows].masked_fill(torch.rand(int(rows.sum()), V, generator=g) < 0.3, -math.inf)
        logits[::7, :, :40000] = -math.inf
        logits.scatter_(-1, torch.cat([drafts, drafts[:, :1]], 1).unsqueeze(-1), keep)   # guesses stay finite
    nd = torch.randint(0, K + 1, (S,), generator=g) if ragged else torch.full((S,), K)
    temps = torch.full((S,), float(T))
    u = torch.rand(S, K, generator=g)
    e = torch.empty(S, V).exponential_(1, generator=g)
    logits = logits.view(S * (K + 1), V).to(dtype)
    draft_logits = draft_logits.to(dtype) if with_draft else None
    return logits, drafts, nd, temps, draft_logits, u, e


def _ulp(x: float) -> float:
    return float(np.spacing(np.float32(abs(x)))) if math.isfinite(x) else math.inf


def _near_boundary(logits, drafts, nd, temps, dl, u, e):
    """Rows whose oracle decision lies within ULPS fp32 ulps of flipping, in the quantities it is computed
    from: an accept test u*q < p, where log p = x_d - logsumexp(x) (x = logits / T) is fp32 rounding away
    from its neighbours at the scale of x_d and of the logsumexp; or the top two of the final argmax of
    p / E (or of the residual max(p - q, 0) / E), within ULPS ulps of p (and q) at the top entries.
    Greedy rows are never flagged: their argmax compares raw logits and must match exactly."""
    S, K = drafts.shape
    V = logits.size(-1)
    lg = logits.view(S, K + 1, V).double()
    flagged = set()
    a_ref, _ = osmp.verify_drafts(logits, drafts, nd, temps, dl, uniforms=u, exp_noise=e)
    for s in range(S):
        T = float(temps[s])
        if T == 0:
            continue
        for j in range(min(int(a_ref[s]) + 1, int(nd[s]), K)):
            x = lg[s, j] / T
            lse = float(torch.logsumexp(x, 0))
            logp = float(x[drafts[s, j]]) - lse
            win = ULPS * (_ulp(lse) + _ulp(float(x[drafts[s, j]])))
            logq = 0.0
            if dl is not None:
                xd = dl.view(S, K, V)[s, j].double() / T
                lsq = float(torch.logsumexp(xd, 0))
                logq = float(xd[drafts[s, j]]) - lsq
                win += ULPS * (_ulp(lsq) + _ulp(float(xd[drafts[s, j]])))
            uu = float(u[s, j])
            if uu > 0 and abs(math.log(uu) + logq - logp) <= win + ULPS * 2.0 ** -23:
                flagged.add(s)
        a = int(a_ref[s])
        p = torch.softmax(lg[s, a] / T, 0)
        lse = float(torch.logsumexp(lg[s, a] / T, 0))
        E = e[s].double().clamp_min(1e-10)
        cands = [(p.clone(), None)]
        if K > 0 and a < int(nd[s]):
            j = min(a, K - 1)
            if dl is None:
                cands[0][0][drafts[s, j]] = 0
            else:
                q = torch.softmax(dl.view(S, K, V)[s, j].double() / T, 0)
                cands.append(((p - q).clamp_min(0), q))
        for c, q in cands:
            sc = c / E
            top2 = torch.topk(sc, 2)
            if float(top2.values[0]) <= 0:
                continue
            i0, i1 = int(top2.indices[0]), int(top2.indices[1])
            scale = max(float(p[i0] + (0 if q is None else q[i0])) / float(E[i0]),
                        float(p[i1] + (0 if q is None else q[i1])) / float(E[i1]))
            # a logsumexp rounding scales every p alike (no effect on the order), but not p against q
            win = ULPS * 2.0 ** -23 * scale * (1 if q is None else 1 + _ulp(lse) / 2.0 ** -23)
            if float(top2.values[0] - top2.values[1]) <= win:
                flagged.add(s)
    return flagged


CONFIG4 = [  # (seed, T, dtype, draft, ragged, offset, masked)
    (3, 0.0, torch.float32, False, False, 0.0, False),
    (4, 0.0, torch.bfloat16, True, True, 0.0, False),
    (13, 1.0, torch.float32, False, False, 0.0, False),
    (14, 1.0, torch.float32, True, True, 0.0, False),
    (15, 1.0, torch.bfloat16, True, False, 0.0, False),
    (16, 1.0, torch.bfloat16, False, True, 0.0, False),
    (21, 0.05, torch.float32, True, False, -8.0, True),
    (22, 0.1, torch.float32, False, True, -8.0, True),
    (23, 0.1, torch.bfloat16, True, True, -9.5, True),
    (24, 0.2, torch.float32, True, False, -6.0, True),
]


@pytest.mark.parametrize("seed,T,dtype,with_draft,ragged,offset,masked", CONFIG4)
def test_config4_full_vocab_vs_oracle(device, seed, T, dtype, with_draft, ragged, offset, masked):
    logits, drafts, nd, temps, dl, u, e = _config4(seed, T, dtype, with_draft, ragged=ragged, offset=offset,
                                                   masked=masked)
    a_ref, t_ref = osmp.verify_drafts(logits, drafts, nd, temps, dl, uniforms=u, exp_noise=e)
    a, t = verify_drafts(logits.to(device), drafts.to(device), nd.to(device), temps.to(device),
                         None if dl is None else dl.to(device), uniforms=u.to(device), exp_noise=e.to(device))
    a, t = a.cpu(), t.cpu()
    bad = ((a != a_ref) | (t != t_ref)).nonzero().flatten().tolist()
    flagged = _near_boundary(logits, drafts, nd, temps, dl, u, e) if bad else set()
    print(f"seed {seed} T={T} {dtype} draft={with_draft} ragged={ragged} offset={offset} masked={masked}: "
          f"accepted {a.tolist()[:12]}... mismatches {bad}, within {ULPS} ulps of a flip {sorted(flagged)}",
          flush=True)
    # exact: the kernel reproduces the reference's own outputs bit for bit (test_golden_full_vocab_exact), and
    # on these ten batches it agrees with the oracle on every row; a mismatch prints whether the row lies within
    # ULPS of a flip, to tell a rounding-order tie from a real error
    assert not bad, (bad, flagged)


def test_all_greedy_path_equals_general_path(device):
    """temperatures all 0: the two-launch argmax path (no noise given) equals the full path (noise given)."""
    for seed, dtype, draft in ((5, torch.float32, False), (6, torch.bfloat16, True)):
        logits, drafts, nd, temps, dl, u, e = _config4(seed, 0.0, dtype, draft, ragged=True)
        args = (logits.to(device), drafts.to(device), nd.to(device), temps.to(device),
                None if dl is None else dl.to(device))
        a0, t0 = verify_drafts(*args)
        a1, t1 = verify_drafts(*args, uniforms=u.to(device), exp_noise=e.to(device))
        a_ref, t_ref = osmp.verify_drafts(logits, drafts, nd, temps, dl, uniforms=u, exp_noise=e)
        assert a0.tolist() == a1.tolist() == a_ref.tolist()
        assert t0.tolist() == t1.tolist() == t_ref.tolist()


def test_low_temperature_extremes(device):
    """T down to 0.01 on logits near -10 (x = l / T far below -88, where exp underflows) and rows that are
    mostly -inf: exact against the oracle, no NaN paths."""
    g = torch.Generator().manual_seed(31)
    S, K, V = 16, 3, 4099
    logits = torch.randn(S, K + 1, V, generator=g) * 2 - 10
    logits[0, :, 1:] = -math.inf                       # a single finite entry
    logits[1, :, :V - 3] = -math.inf                   # the last three entries finite
    logits[2, 1] = -math.inf
    logits[2, 1, 7] = -12.0
    draft_logits = torch.randn(S, K, V, generator=g) * 2 - 10
    draft_logits[3, :, :2048] = -math.inf
    drafts = logits[:, :K].argmax(-1)
    drafts[4:8] = torch.randint(0, V, (4, K), generator=g)
    temps = torch.tensor([0.01, 0.05, 0.1, 0.02, 0.05, 0.1, 1.0, 0.0] * 2)
    nd = torch.full((S,), K)
    u = torch.rand(S, K, generator=g)
    e = torch.empty(S, V).exponential_(1, generator=g)
    for dl in (None, draft_logits):
        flat = logits.view(S * (K + 1), V)
        a_ref, t_ref = osmp.verify_drafts(flat, drafts, nd, temps, dl, uniforms=u, exp_noise=e)
        a, t = verify_drafts(flat.to(device), drafts.to(device), nd.to(device), temps.to(device),
                             None if dl is None else dl.to(device), uniforms=u.to(device), exp_noise=e.to(device))
        assert a.cpu().tolist() == a_ref.tolist()
        assert t.cpu().tolist() == t_ref.tolist()


def test_greedy_known_answers(device):
    drafts = torch.tensor([[3, 4, 5], [3, 9, 5], [1, 4, 5], [3, 4, 5]], device=device)
    nd = torch.tensor([3, 3, 3, 1], device=device)
    top1 = [[3, 4, 5, 6]] * 4
    a, t = verify_drafts(_logits_with_top1(top1).to(device), drafts, nd, torch.zeros(4, device=device))
    assert a.tolist() == [3, 1, 0, 1] and t.tolist() == [6, 4, 3, 4]
    a, t = verify_drafts(_logits_with_top1([[7], [2]]).to(device), torch.zeros(2, 0, dtype=torch.int64, device=device),
                         torch.zeros(2, dtype=torch.int64, device=device), torch.zeros(2, device=device))
    assert a.tolist() == [0, 0] and t.tolist() == [7, 2]
    temps = torch.tensor([0.0, 1.0, 0.0, 1.0], device=device)
    for _ in range(20):
        a, t = verify_drafts(_logits_with_top1(top1).to(device), drafts, nd, temps)
        assert a[0] == 3 and t[0] == 6 and a[2] == 0 and t[2] == 3


def test_zero_residual_guard(device):
    g = torch.Generator().manual_seed(2)
    V, K, S = 6, 2, 4
    logits = torch.randn(S, K + 1, V, generator=g)
    logits[..., 0] = -float("inf")
    drafts = torch.full((S, K), 3)
    a, t = verify_drafts(logits.view(-1, V).to(device), drafts.to(device), torch.full((S,), K, device=device),
                         torch.ones(S, device=device), logits[:, :K].clone().to(device),
                         uniforms=torch.ones(S, K, device=device))
    assert a.tolist() == [0] * S and bool((t != 0).all())


def test_distribution_tv_on_gpu(device):
    """Reference tests/test_spec_unit.py:137-172 on the GPU kernels (noise drawn on the device)."""
    g = torch.Generator().manual_seed(0)
    V, K, n, T = 8, 3, 200000, 0.7
    p_logits = torch.randn(K + 1, V, generator=g) * 1.5
    p = torch.softmax(p_logits / T, -1)
    guesses = (p - 0.3).abs().argmin(-1)[:K]
    one_hot = torch.nn.functional.one_hot(guesses, V).float()
    q = torch.softmax(p_logits[:K] / T + torch.randn(K, V, generator=g), -1)
    for draft_probs in (one_hot, q):
        drafts = torch.multinomial(draft_probs, n, replacement=True, generator=g).T.contiguous()
        logits = p_logits.unsqueeze(0).expand(n, -1, -1).reshape(n * (K + 1), -1)
        ql = None if draft_probs is one_hot else (T * draft_probs.log()).unsqueeze(0).expand(n, -1, -1).contiguous()
        a, t = verify_drafts(logits.to(device), drafts.to(device), torch.full((n,), K, device=device),
                             torch.full((n,), T, device=device), None if ql is None else ql.to(device))
        a, t = a.cpu(), t.cpu()
        out = torch.cat([drafts, torch.zeros(n, 1, dtype=torch.int64)], 1)
        out[torch.arange(n), a] = t
        assert _max_tv(p_logits, T, out, a + 1) < 0.02


def test_sampler_matches_oracle(device):
    g = torch.Generator().manual_seed(9)
    S, V = 32, 151936
    logits = torch.randn(S, V, generator=g) * 3
    temps = torch.tensor([0.0, 1.0, 0.7, 1.5] * 8)
    e = torch.empty(S, V).exponential_(1, generator=g)
    ref = osmp.sample(logits, temps, e)
    got = Sampler()(logits.to(device), temps.to(device), e.to(device)).cpu()
    assert torch.equal(got, ref)
    got16 = Sampler()(logits.to(torch.bfloat16).to(device), temps.to(device), e.to(device)).cpu()
    assert torch.equal(got16, osmp.sample(logits.to(torch.bfloat16), temps, e))


def test_verify_graph_replays_equal_eager(device):
    """verify_drafts captured in a HIP graph (T = 0, 1, 0.7 rows, draft logits, injected noise; the last
    resample workgroup of each sampled sequence picks its token on counters verify_decide zeroes) and replayed
    with new inputs and eager calls of another size in between: every replay equals the eager call on the same
    inputs."""
    S, K, V = 48, 4, 151936
    g = torch.Generator(device=device).manual_seed(21)
    logits = torch.empty(S * (K + 1), V, device=device)
    dl = torch.empty(S * K, V, device=device)
    drafts = torch.empty(S, K, dtype=torch.int64, device=device)
    nd = torch.empty(S, dtype=torch.int64, device=device)
    temps = torch.tensor([0.0, 1.0, 0.7] * (S // 3), device=device)
    u = torch.empty(S, K, device=device)
    e = torch.empty(S, V, device=device)

    def refill(seed):
        gg = torch.Generator(device=device).manual_seed(seed)
        logits.copy_(torch.randn(logits.shape, device=device, generator=gg) * 3)
        dl.copy_(logits.view(S, K + 1, V)[:, :K].reshape(S * K, V) + torch.randn(dl.shape, device=device, generator=gg))
        top = logits.view(S, K + 1, V)[:, :K].argmax(-1)
        drafts.copy_(torch.where(torch.rand(S, K, device=device, generator=gg) < 0.6, top,
                                 torch.randint(0, V, (S, K), device=device, generator=gg)))
        nd.copy_(torch.randint(0, K + 1, (S,), device=device, generator=gg))
        u.copy_(torch.rand(S, K, device=device, generator=gg))
        e.copy_(torch.empty(S, V, device=device).exponential_(1, generator=gg))

    refill(0)
    verify_drafts(logits, drafts, nd, temps, dl, uniforms=u, exp_noise=e)   # warm-up (workspace)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        acc, nxt = verify_drafts(logits, drafts, nd, temps, dl, uniforms=u, exp_noise=e)
    small = torch.randn(3 * (K + 1), V, generator=g, device=device)
    for rep in range(3):
        refill(100 + rep)
        graph.replay()
        torch.cuda.synchronize()
        got = (acc.clone(), nxt.clone())
        a0, t0 = verify_drafts(logits, drafts, nd, temps, dl, uniforms=u, exp_noise=e)
        torch.cuda.synchronize()
        assert torch.equal(got[0], a0) and torch.equal(got[1], t0), rep
        assert (t0 >= 0).all() and (t0 < V).all()
        # an eager call of another size on the same workspace between replays
        verify_drafts(small, drafts[:3], nd[:3], temps[:3], dl[:3 * K], uniforms=u[:3], exp_noise=e[:3])
