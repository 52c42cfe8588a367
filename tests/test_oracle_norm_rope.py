"""Pins oracle/qk_norm_rope.py independently of its own formulas (CPU only).

rope_cache    closed form: column 0 is cos(p) / sin(p) (inv_freq_0 = 1), every entry equals cos / sin of the
              float32 product p * base^(-2j/D) evaluated in float64, cos^2 + sin^2 = 1; a planted wrong
              frequency spacing fails.
rms_norm      float64 textbook x / sqrt(mean(x^2) + eps) * w within the two bf16 roundings; a constant row
              where eps dominates (eps inside the root, added to the mean); RMS of the output is 1; scale
              invariance with eps = 0 (bitwise); planted mistakes (sum instead of mean, eps outside the root).
apply_rotary  position 0 is the identity (bitwise); a unit vector in the first half turns to (cos, sin)
              (the rotation's direction); complex multiplication (x1 + i x2) e^(i theta) in float64 within one
              bf16 rounding; pair norms are kept; rotating by p then by -p gives x back; q.k after rotation
              depends only on the position difference; planted sign / pairing mistakes fail.
composition   q_norm -> rotary -> store on views of one qkv row, v stored unchanged, -1 slots skipped, and
              the no-norm (qkv bias) path.
"""
import math

import numpy as np
import torch

from oracle import qk_norm_rope as onr

D = 128


def _bf16(x):
    return torch.as_tensor(x).to(torch.bfloat16)


def _ulps_bf16(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 units in the last place (ordered integer view)."""
    def key(t):
        i = t.to(torch.bfloat16).view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -32768 - i, i)
    return (key(a) - key(b)).abs()


# ------------------------------------------------------------------ rope_cache

def test_rope_cache_closed_form():
    base, P = 1_000_000.0, 5000
    cs = onr.rope_cache(D, P, base)
    assert cs.shape == (P, D) and cs.dtype == torch.float32
    p = np.arange(P, dtype=np.float64)
    np.testing.assert_allclose(cs[:, 0].double().numpy(), np.cos(p), atol=4e-7)
    np.testing.assert_allclose(cs[:, D // 2].double().numpy(), np.sin(p), atol=4e-7)
    j = np.arange(D // 2)
    inv64 = base ** (-2.0 * j / D)
    inv32 = (1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.float) / D))).double().numpy()
    np.testing.assert_allclose(inv32, inv64, rtol=3e-7)
    ang = (np.float32(1) * p[:, None].astype(np.float32) * inv32[None, :].astype(np.float32)).astype(np.float64)
    np.testing.assert_allclose(cs[:, :D // 2].double().numpy(), np.cos(ang), atol=4e-7)
    np.testing.assert_allclose(cs[:, D // 2:].double().numpy(), np.sin(ang), atol=4e-7)
    c, s = cs[:, :D // 2].double(), cs[:, D // 2:].double()
    assert torch.allclose(c * c + s * s, torch.ones_like(c), atol=1e-6)
    # planted: frequencies spaced by j / D instead of 2j / D would move column 1 far from the closed form
    wrong = np.cos(p * base ** (-1.0 / D))
    assert np.abs(cs[:, 1].double().numpy() - wrong).max() > 0.5


# ------------------------------------------------------------------ rms_norm

def _textbook_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xd = x.double()
    return xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps) * w.double()


def test_rms_norm_textbook_within_two_roundings():
    g = torch.Generator().manual_seed(0)
    for sigma in (1e-3, 1.0, 37.0):
        x = (torch.randn(64, 8, D, generator=g) * sigma).to(torch.bfloat16)
        w = (1 + 0.5 * torch.randn(D, generator=g)).to(torch.bfloat16)
        got = onr.rms_norm(x, w, 1e-6)
        ref = _textbook_norm(x, w, 1e-6)
        assert got.dtype == torch.bfloat16
        # two bf16 roundings (after the normalisation, after the weight): at most 2^-8 relative each
        err = (got.double() - ref).abs()
        assert (err <= ref.abs() * (2 ** -7) + 1e-30).all(), float((err / ref.abs()).max())
        y = onr.rms_norm(x, torch.ones(D, dtype=torch.bfloat16), 0.0).double()
        rms = y.pow(2).mean(-1).sqrt()
        assert torch.allclose(rms, torch.ones_like(rms), atol=8e-3)


def test_rms_norm_eps_inside_root_and_added_to_mean():
    c, eps = 2.0 ** -10, 1e-6
    x = torch.full((1, D), c).to(torch.bfloat16)
    got = onr.rms_norm(x, torch.ones(D, dtype=torch.bfloat16), eps)
    want = c / math.sqrt(c * c + eps)                # 0.6986...
    assert float(got[0, 0]) == float(_bf16(want))
    # planted: eps outside the root (sqrt(mean) + eps) or the sum instead of the mean
    assert float(_bf16(c / (math.sqrt(c * c) + eps))) != float(got[0, 0])
    assert float(_bf16(c / math.sqrt(D * c * c + eps))) != float(got[0, 0])
    assert torch.equal(onr.rms_norm(torch.zeros(2, D, dtype=torch.bfloat16), torch.ones(D, dtype=torch.bfloat16),
                                    eps), torch.zeros(2, D, dtype=torch.bfloat16))


def test_rms_norm_scale_invariance_and_weight():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(32, D, generator=g).to(torch.bfloat16)
    one = torch.ones(D, dtype=torch.bfloat16)
    a = onr.rms_norm(x, one, 0.0)
    assert torch.equal(a, onr.rms_norm(x * 4, one, 0.0))          # powers of two scale exactly
    assert torch.equal(onr.rms_norm(x, one * 2, 0.0), a * 2)      # the weight multiplies the rounded value


def test_add_rms_norm_sum_rounding_and_zero_residual():
    """add_rms_norm: the new residual is bf16(x + r) (the float64 sum rounded, where the fp32 sum is exact), the
    output normalises the unrounded sum within the two roundings, a zero residual reduces it to rms_norm, and the
    operands commute."""
    g = torch.Generator().manual_seed(5)
    H = 4096
    x = torch.randn(16, H, generator=g).to(torch.bfloat16)
    r = (torch.randn(16, H, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(H, generator=g)).to(torch.bfloat16)
    out, res = onr.add_rms_norm(x, r, w, 1e-6)
    s = x.double() + r.double()
    assert torch.equal(res, s.to(torch.bfloat16))
    ref = s / torch.sqrt((s * s).mean(-1, keepdim=True) + 1e-6) * w.double()
    err = (out.double() - ref).abs()
    assert (err <= ref.abs() * (2 ** -7) + 1e-30).all()
    # planted: normalising the rounded residual instead of the fp32 sum changes some rows
    planted = onr.rms_norm(res, w, 1e-6)
    assert not torch.equal(planted, out)
    z_out, z_res = onr.add_rms_norm(x, torch.zeros_like(x), w, 1e-6)
    assert torch.equal(z_res, x) and torch.equal(z_out, onr.rms_norm(x, w, 1e-6))
    c_out, c_res = onr.add_rms_norm(r, x, w, 1e-6)
    assert torch.equal(c_out, out) and torch.equal(c_res, res)


# ------------------------------------------------------------------ rotary

def _rope_inputs(seed, N=40, H=4, P=9000):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, P, (N,), generator=g)
    return x, pos, onr.rope_cache(D, P, 10000.0)


def test_rotary_position_zero_is_identity():
    x, _, cs = _rope_inputs(2)
    y, _ = onr.rotary(torch.zeros(x.size(0), dtype=torch.int64), x, x[:, :1], cs)
    assert torch.equal(y, x)


def test_rotary_direction_on_unit_vectors():
    cs = onr.rope_cache(D, 100, 10000.0)
    for j in (0, 5, 63):
        x = torch.zeros(1, 1, D, dtype=torch.bfloat16)
        x[0, 0, j] = 1
        y, _ = onr.rotary(torch.tensor([37]), x, x, cs)
        c, s = float(cs[37, j]), float(cs[37, D // 2 + j])
        assert float(y[0, 0, j]) == float(_bf16(c)) and float(y[0, 0, D // 2 + j]) == float(_bf16(s))
        nz = y[0, 0].nonzero().flatten().tolist()
        assert set(nz) <= {j, D // 2 + j}


def test_rotary_is_complex_multiplication():
    x, pos, cs = _rope_inputs(3)
    y, _ = onr.rotary(pos, x, x[:, :1], cs)
    c = cs[pos, :D // 2].double()[:, None, :]
    s = cs[pos, D // 2:].double()[:, None, :]
    z = torch.complex(x[..., :D // 2].double(), x[..., D // 2:].double()) * torch.complex(c, s)
    ref = torch.cat((z.real, z.imag), dim=-1)
    # one fp32 evaluation then one bf16 rounding: within 1 bf16 ulp of the exact value
    assert int(_ulps_bf16(y, ref).max()) <= 1
    # planted: the other rotation sign, or interleaved (GPT-J) pairs instead of halves, is far off
    zc = torch.complex(x[..., :D // 2].double(), x[..., D // 2:].double()) * torch.complex(c, -s)
    assert (torch.cat((zc.real, zc.imag), -1) - y.double()).abs().max() > 0.5
    xi = torch.complex(x[..., 0::2].double(), x[..., 1::2].double()) * torch.complex(c, s)
    inter = torch.stack((xi.real, xi.imag), -1).flatten(-2)
    assert (inter - y.double()).abs().max() > 0.5


def test_rotary_keeps_pair_norms_and_inverts():
    x, pos, cs = _rope_inputs(4)
    y, _ = onr.rotary(pos, x, x[:, :1], cs)
    nx = x[..., :D // 2].double() ** 2 + x[..., D // 2:].double() ** 2
    ny = y[..., :D // 2].double() ** 2 + y[..., D // 2:].double() ** 2
    assert torch.allclose(ny, nx, rtol=2 ** -6, atol=1e-6)
    back = cs.clone()
    back[:, D // 2:] = -back[:, D // 2:]                       # rotation by -theta
    z, _ = onr.rotary(pos, y, y[:, :1], back)
    assert (z.double() - x.double()).abs().max() <= 2 ** -5 * x.double().abs().max()


def test_rotary_scores_depend_on_position_difference():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 1, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 1, D, generator=g).to(torch.bfloat16)
    cs = onr.rope_cache(D, 4096, 10000.0)
    scores = []
    for p in (0, 100, 1000, 3000):
        qr, kr = onr.rotary(torch.tensor([p + 17]), q, k, cs)
        _, kr0 = onr.rotary(torch.tensor([p]), q, k, cs)
        scores.append(float((qr.double() * kr0.double()).sum()))
    ref = scores[0]
    for s in scores[1:]:
        assert abs(s - ref) <= 0.05 * (1 + abs(ref)), scores


# ------------------------------------------------------------------ composition

def test_qk_norm_rope_store_composition():
    g = torch.Generator().manual_seed(6)
    N, Hq, Hkv, NB, bs = 11, 4, 2, 3, 8
    qkv = torch.randn(N, (Hq + 2 * Hkv) * D, generator=g).to(torch.bfloat16)
    q = qkv[:, :Hq * D].view(N, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D)
    pos = torch.randint(0, 600, (N,), generator=g)
    cs = onr.rope_cache(D, 600, 1e6)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    slots = torch.randperm(NB * bs, generator=g)[:N].to(torch.int32)
    slots[[1, 6]] = -1
    kc = torch.zeros(NB, bs, Hkv, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    qo, ko = onr.qk_norm_rope_store(q, k, v, pos, qw, kw, 1e-6, cs, kc, vc, slots)
    eq, ek = onr.rotary(pos, onr.rms_norm(q, qw, 1e-6), onr.rms_norm(k, kw, 1e-6), cs)
    assert torch.equal(qo, eq) and torch.equal(ko, ek)
    kflat, vflat = kc.view(-1, Hkv, D), vc.view(-1, Hkv, D)
    for i in range(N):
        s = int(slots[i])
        if s >= 0:
            assert torch.equal(kflat[s], ek[i]) and torch.equal(vflat[s], v[i])
    written = set(int(s) for s in slots if s >= 0)
    for s in range(NB * bs):
        if s not in written:
            assert not kflat[s].any() and not vflat[s].any()
    qn, kn = onr.qk_norm_rope_store(q, k, v, pos, None, None, 1e-6, cs)
    rq, rk = onr.rotary(pos, q, k, cs)
    assert torch.equal(qn, rq) and torch.equal(kn, rk)
