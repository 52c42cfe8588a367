"""Row-invariant linear layer (sd_linear) and RMSNorm (sd_rms_norm) on the GPU.

Bar: the linear layer's outputs are the bf16 rounding of fp32 dot products (within one bf16 unit of the float64
dot product plus the fp32 accumulation bound, at least 99.9 % equal to it rounded: the library GEMM's
contract); the norm's residual output is bit-exact against the oracle (layernorm.py:28-38) and its normalised
output differs from the oracle only by the order of the sum of squares (at least 99.5 % bit-exact, the rest
within one bf16 unit). Both give bitwise the same row whatever the number of rows in the call, which the
library GEMM (o_proj, gate_up_proj and down_proj shapes) and reductions do not.
"""
import pytest
import torch

from nanovllm_amd.layers.layernorm import RMSNorm, rms_norm
from nanovllm_amd.layers.linear import RowInvariantLinear
from oracle import qk_norm_rope as onr

pytestmark = pytest.mark.gpu

QWEN3_8B = [("qkv_proj", 4096, 6144), ("o_proj", 4096, 4096), ("gate_up_proj", 4096, 24576),
            ("down_proj", 12288, 4096)]


def _ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    a = x.abs().float().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def _check_rows(x, w, y, rows):
    xd, wd = x.cpu().double()[rows], w.cpu().double()
    ref = xd @ wd.T
    mag = xd.abs() @ wd.abs().T
    ours = y.cpu()[rows].double()
    bound = _ulp_bf16(ref.float()).double() + x.size(1) * 2.0 ** -24 * mag
    worst = ((ours - ref).abs() / bound).max().item()
    exact = (ours.float() == ref.float().to(torch.bfloat16).float()).float().mean().item()
    print(f"vs float64: worst {worst:.3f} of the bound, {exact * 100:.3f} % equal to the rounded float64", flush=True)
    assert worst <= 1.0 and exact >= 0.999


@pytest.mark.parametrize("M,N,K", [(5, 1000, 256), (70, 2053, 192), (330, 6144, 4096), (64, 4096, 12288),
                                   (1300, 4096, 12288), (700, 2053, 192)])
def test_linear_vs_float64(device, M, N, K):
    g = torch.Generator(device=device).manual_seed(M + N)
    x = torch.randn(M, K, device=device, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, device=device, generator=g) * K ** -0.5).to(torch.bfloat16)
    y = RowInvariantLinear(w)(x)
    _check_rows(x, w, y, list(range(0, M, max(1, M // 6))) + [M - 1])


# 300 tiles: 256 whole ones and a split last round (the physical split at every row count, as the LM head)
@pytest.mark.parametrize("name,K,N", QWEN3_8B + [("partly_split", 128, 76800)])
def test_linear_rows_independent_of_row_count(device, name, K, N):
    g = torch.Generator(device=device).manual_seed(K + N)
    x = torch.randn(2048, K, device=device, generator=g).to(torch.bfloat16)
    lin = RowInvariantLinear((torch.randn(N, K, device=device, generator=g) * K ** -0.5).to(torch.bfloat16))
    probes = [0, 1, 63, 127, 128, 319, 320, 1000, 1215, 2047]
    alone = {r: lin(x[r:r + 1]) for r in probes}    # each row in a call of its own
    for M in (2, 16, 64, 80, 320, 325, 1216, 2048):
        y = lin(x[:M])
        for r in probes:
            if r < M:
                assert torch.equal(y[r:r + 1], alone[r]), f"{name}: row {r} differs at {M} rows"
    # a strided input (a column slice of a wider buffer) gives the same rows
    wide = torch.zeros(64, K + 64, dtype=torch.bfloat16, device=device)
    wide[:, :K] = x[:64]
    assert torch.equal(lin(wide[:, :K]), lin(x[:64]))


def test_linear_vs_library_gemm(device):
    g = torch.Generator(device=device).manual_seed(3)
    x = torch.randn(320, 4096, device=device, generator=g).to(torch.bfloat16)
    w = (torch.randn(6144, 4096, device=device, generator=g) * 4096 ** -0.5).to(torch.bfloat16)
    ours, lib = RowInvariantLinear(w)(x), torch.nn.functional.linear(x, w)
    same = (ours == lib).float().mean().item()
    big = ((ours.float() - lib.float()).abs() > _ulp_bf16(torch.maximum(ours.float().abs(), lib.float().abs())) + 1e-3)
    print(f"vs F.linear: {same * 100:.3f} % identical", flush=True)
    assert same >= 0.99 and int(big.sum()) == 0


@pytest.mark.parametrize("H", [4096, 1024, 1000, 12288])
def test_rms_norm_vs_oracle(device, H):
    g = torch.Generator().manual_seed(H)
    x = (torch.randn(37, H, generator=g) * 2).to(torch.bfloat16)
    r = torch.randn(37, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    for residual in (None, r):
        if residual is None:
            got = rms_norm(x.to(device), w.to(device), 1e-6).cpu()
            want = onr.rms_norm(x, w, 1e-6)
        else:
            got, got_res = (t.cpu() for t in rms_norm(x.to(device), w.to(device), 1e-6, residual.to(device)))
            want, want_res = onr.add_rms_norm(x, residual, w, 1e-6)
            assert torch.equal(got_res, want_res)
        same = (got == want).float().mean().item()
        diff = (got.float() - want.float()).abs()
        assert same >= 0.995 and bool((diff <= _ulp_bf16(want.float())).all()), (same, float(diff.max()))


def test_rms_norm_rows_independent_of_row_count_and_in_place(device):
    H = 4096
    g = torch.Generator(device=device).manual_seed(9)
    x = torch.randn(2048, H, device=device, generator=g).to(torch.bfloat16)
    r = torch.randn(2048, H, device=device, generator=g).to(torch.bfloat16)
    norm = RMSNorm(H).to(device)
    norm.weight.data = (1 + 0.1 * torch.randn(H, device=device, generator=g)).to(torch.bfloat16)
    first, first_res = norm(x[:1], r[:1])
    for M in (16, 64, 320, 2048):
        out, res = norm(x[:M], r[:M])
        assert torch.equal(out[:1], first) and torch.equal(res[:1], first_res)
    # in place: out over x, the new residual over the old one (as a fused residual stream uses it)
    xi, ri = x[:64].clone(), r[:64].clone()
    want_out, want_res = norm(x[:64], r[:64])
    rms_norm(xi, norm.weight.data, norm.eps, ri, out=xi, residual_out=ri)
    assert torch.equal(xi, want_out) and torch.equal(ri, want_res)
