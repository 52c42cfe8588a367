"""Speculative-decoding verifier and token sampler on MI355X: drop-in for nanovllm/layers/sampler.py.

``verify_drafts`` keeps the reference's signature and result (sampler.py:28-103) and adds two optional
arguments, ``uniforms`` [S, K] and ``exp_noise`` [S, V] (fp32, device): the random numbers the reference
draws internally with torch.rand and exponential_. Given the same numbers, the accepted counts and tokens
are those of the reference rule. When omitted they are drawn here the same way, on the same device.
"""
import torch
from torch import nn

from nanovllm_amd import _lib

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def _rows(x: torch.Tensor, V: int) -> torch.Tensor:
    x = x.reshape(-1, V)
    if x.stride(1) != 1:
        x = x.contiguous()
    if x.dtype not in _DTYPES:
        x = x.float()
    return x


def _any_random(temperatures: torch.Tensor) -> bool:
    # the reference reads this on the host too (sampler.py:64)
    return not bool((temperatures == 0).all())


def verify_drafts(logits: torch.Tensor, draft_token_ids: torch.Tensor, num_drafts: torch.Tensor,
                  temperatures: torch.Tensor, draft_logits: torch.Tensor | None = None,
                  uniforms: torch.Tensor | None = None, exp_noise: torch.Tensor | None = None
                  ) -> tuple[torch.Tensor, torch.Tensor]:
    """(num_accepted [S] int64, next_token [S] int64); see nanovllm/layers/sampler.py:28-56 for the rule."""
    S, K = draft_token_ids.shape
    V = logits.size(-1)
    device = logits.device
    rows = _rows(logits, V)
    if rows.size(0) != S * (K + 1):
        raise ValueError(f"verify_drafts: logits has {rows.size(0)} rows, expected S*(K+1) = {S * (K + 1)}")
    drafts = draft_token_ids.to(torch.int64).contiguous()
    nd = num_drafts.to(torch.int64).contiguous()
    temps = temperatures.float().contiguous()
    drows = _rows(draft_logits, V) if draft_logits is not None and K > 0 else None
    if drows is not None and drows.size(0) != S * K:
        raise ValueError("verify_drafts: draft_logits must hold S*K rows")
    all_greedy = False
    if uniforms is None or exp_noise is None:
        if _any_random(temps):
            if uniforms is None and K > 0:
                uniforms = torch.rand(S, K, device=device, dtype=torch.float32)
            if exp_noise is None:
                exp_noise = torch.empty(S, V, device=device, dtype=torch.float32).exponential_(1)
        else:
            all_greedy = True    # the argmax pass alone decides every row
    if uniforms is not None:
        uniforms = uniforms.float().contiguous()
    if exp_noise is not None:
        exp_noise = exp_noise.float().contiguous()
    num_accepted = torch.empty(S, dtype=torch.int64, device=device)
    next_token = torch.empty(S, dtype=torch.int64, device=device)
    if S == 0:
        return num_accepted, next_token
    lib = _lib.load()
    nbytes = lib.sd_verify_workspace_size(S, K, V, int(drows is not None))
    ws = _lib.workspace(nbytes, device)
    rc = lib.sd_verify_drafts(rows.data_ptr(), _DTYPES[rows.dtype], rows.stride(0), drafts.data_ptr(), nd.data_ptr(),
                              None if all_greedy else temps.data_ptr(), _lib.ptr(drows),
                              _DTYPES[drows.dtype] if drows is not None else 0,
                              drows.stride(0) if drows is not None else 0, _lib.ptr(uniforms), _lib.ptr(exp_noise),
                              S, K, V, num_accepted.data_ptr(), next_token.data_ptr(), ws.data_ptr(), ws.numel(),
                              _lib.stream_of(device))
    _lib.check(rc, "sd_verify_drafts")
    return num_accepted, next_token


class Sampler(nn.Module):
    """Drop-in for nanovllm.layers.sampler.Sampler (sampler.py:5-16); exp_noise [S, V] optional."""

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor, exp_noise: torch.Tensor | None = None):
        S, V = logits.shape
        device = logits.device
        rows = _rows(logits, V)
        temps = temperatures.float().contiguous()
        if exp_noise is None and _any_random(temps):
            exp_noise = torch.empty(S, V, device=device, dtype=torch.float32).exponential_(1)
        if exp_noise is not None:
            exp_noise = exp_noise.float().contiguous()
        out = torch.empty(S, dtype=torch.int64, device=device)
        if S == 0:
            return out
        lib = _lib.load()
        nbytes = lib.sd_verify_workspace_size(S, 0, V, 0) + 8 * S
        ws = _lib.workspace(nbytes, device)
        rc = lib.sd_sample(rows.data_ptr(), _DTYPES[rows.dtype], rows.stride(0), temps.data_ptr(),
                           _lib.ptr(exp_noise), S, V, out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(device))
        _lib.check(rc, "sd_sample")
        return out
