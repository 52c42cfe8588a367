"""LM head + speculative verifier in one call (HIP sd_lm_head_verify): the MI355X counterpart of
``logits = model.compute_logits(hidden_states)`` followed by ``verify_drafts(logits, ...)``
(nanovllm/engine/model_runner.py:482-483; nanovllm/layers/embed_head.py:56-68; nanovllm/layers/sampler.py:28-103).

When every row is greedy the logits are never materialised: the GEMM's epilogue takes each row's first argmax.
With sampled rows the logits are written (bf16, as the library GEMM rounds them) and verified by the same passes
as ``verify_drafts``. The weight is read in a tile layout made once per weight (``pack_weight``; LMHeadVerifier
keeps it). Launches go on torch's current stream.

A token row's logits are bitwise the same whatever the call's row count, so every consumer of greedy logits
goes through this one GEMM: ``lm_head_verify`` (verify step, model_runner.py:481-483), ``lm_head_sample``
(plain decode and prefill: ``compute_logits`` + ``Sampler``, model_runner.py:402,412) and ``lm_head_mixed``
(the mixed step's verify rows and finished prefill chunks in one pass over the weight, model_runner.py:513-533).
Greedy speculative decoding then picks the tokens plain decoding picks.
"""
import torch

from nanovllm_amd import _lib
from nanovllm_amd.layers.sampler import _DTYPES, _any_random, _rows


def pack_weight(weight: torch.Tensor) -> torch.Tensor:
    """The LM head weight [V, H] bf16 in the kernel's tile layout (uint8 buffer, sd_lm_head_pack_weight)."""
    V, H = weight.shape
    if weight.dtype != torch.bfloat16 or not weight.is_contiguous():
        raise ValueError("pack_weight: contiguous bf16 [V, H] required")
    lib = _lib.load()
    out = torch.empty(lib.sd_lm_head_packed_weight_size(V, H), dtype=torch.uint8, device=weight.device)
    _lib.check(lib.sd_lm_head_pack_weight(weight.data_ptr(), V, H, out.data_ptr(), _lib.stream_of(weight.device)),
               "sd_lm_head_pack_weight")
    return out


class LMHeadVerifier:
    """An LM head weight packed once, for lm_head_verify calls (the weight must not change afterwards)."""

    def __init__(self, weight: torch.Tensor):
        self.vocab, self.hidden = weight.shape
        self.packed = pack_weight(weight)

    def __call__(self, hidden: torch.Tensor, *args, **kwargs):
        return lm_head_verify(hidden, self, *args, **kwargs)


def lm_head_verify(hidden: torch.Tensor, head: LMHeadVerifier, draft_token_ids: torch.Tensor,
                   num_drafts: torch.Tensor, temperatures: torch.Tensor, logits_indices: torch.Tensor | None = None,
                   draft_logits: torch.Tensor | None = None, uniforms: torch.Tensor | None = None,
                   exp_noise: torch.Tensor | None = None, logits_out: torch.Tensor | None = None
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """(num_accepted [S], next_token [S]) int64 for the S*(K+1) verify rows of hidden [N, H] bf16 (gathered by
    logits_indices when given, else its first S*(K+1) rows) under the LM head `head` (an LMHeadVerifier). Pass
    logits_out ([S*(K+1), V] bf16) to also get the logits; it is allocated here when a row is sampled."""
    S, K = draft_token_ids.shape
    V, H = head.vocab, head.hidden
    device = hidden.device
    if hidden.dtype != torch.bfloat16:
        raise ValueError("lm_head_verify: bf16 hidden states required")
    if hidden.dim() != 2 or hidden.size(1) != H or hidden.stride(1) != 1:
        raise ValueError("lm_head_verify: hidden [N, H] with unit column stride required")
    idx = logits_indices.to(torch.int64).contiguous() if logits_indices is not None else None
    if idx is not None and idx.numel() != S * (K + 1):
        raise ValueError("lm_head_verify: logits_indices must list S*(K+1) rows")
    drafts = draft_token_ids.to(torch.int64).contiguous()
    nd = num_drafts.to(torch.int64).contiguous()
    temps = temperatures.float().contiguous()
    drows = _rows(draft_logits, V) if draft_logits is not None and K > 0 else None
    sampled = _any_random(temps)   # host read, as the reference's (sampler.py:64)
    if sampled:
        if uniforms is None and K > 0:
            uniforms = torch.rand(S, K, device=device, dtype=torch.float32)
        if exp_noise is None:
            exp_noise = torch.empty(S, V, device=device, dtype=torch.float32).exponential_(1)
        if logits_out is None:
            logits_out = torch.empty(S * (K + 1), V, dtype=torch.bfloat16, device=device)
    if logits_out is not None and (logits_out.dtype != torch.bfloat16 or logits_out.stride(1) != 1
                                   or logits_out.shape != (S * (K + 1), V)):
        raise ValueError("lm_head_verify: logits_out must be bf16 [S*(K+1), V] with unit column stride")
    uniforms = uniforms.float().contiguous() if uniforms is not None else None
    exp_noise = exp_noise.float().contiguous() if exp_noise is not None else None
    num_accepted = torch.empty(S, dtype=torch.int64, device=device)
    next_token = torch.empty(S, dtype=torch.int64, device=device)
    if S == 0:
        return num_accepted, next_token
    lib = _lib.load()
    nbytes = lib.sd_lm_head_verify_workspace_size(S, K, V, H, int(drows is not None))
    ws = _lib.workspace(nbytes, device)
    rc = lib.sd_lm_head_verify(
        hidden.data_ptr(), hidden.stride(0), hidden.size(0), _lib.ptr(idx), head.packed.data_ptr(), V, H,
        drafts.data_ptr(),
        nd.data_ptr(), temps.data_ptr() if sampled else None, _lib.ptr(drows),
        _DTYPES[drows.dtype] if drows is not None else 0, drows.stride(0) if drows is not None else 0,
        _lib.ptr(uniforms) if sampled else None, _lib.ptr(exp_noise) if sampled else None, S, K, _lib.ptr(logits_out),
        logits_out.stride(0) if logits_out is not None else 0, num_accepted.data_ptr(), next_token.data_ptr(),
        ws.data_ptr(), ws.numel(), _lib.stream_of(device))
    _lib.check(rc, "sd_lm_head_verify")
    return num_accepted, next_token


def lm_head_sample(hidden: torch.Tensor, head: LMHeadVerifier, temperatures: torch.Tensor,
                   logits_indices: torch.Tensor | None = None, exp_noise: torch.Tensor | None = None,
                   logits_out: torch.Tensor | None = None) -> torch.Tensor:
    """next_token [S] int64 for S rows of hidden (gathered by logits_indices when given, else its first S rows):
    ``Sampler()(compute_logits(hidden), temperatures)`` (nanovllm/layers/sampler.py:7-16,
    nanovllm/layers/embed_head.py:56-68) through the same GEMM as lm_head_verify, as a verify call with no
    draft slots."""
    S = temperatures.numel()
    device = hidden.device
    empty = torch.zeros(S, 0, dtype=torch.int64, device=device)
    nd = torch.zeros(S, dtype=torch.int64, device=device)
    return lm_head_verify(hidden, head, empty, nd, temperatures, logits_indices=logits_indices, exp_noise=exp_noise,
                          logits_out=logits_out)[1]


def mixed_rows(logits_indices: torch.Tensor, num_decode: int, k: int) -> torch.Tensor:
    """The verify call's row list for a mixed step: the D(1+k) decode rows, then each finished prefill chunk's
    row once per slot of a (1+k)-row sequence that has no drafts (only its first row decides its token)."""
    idx = logits_indices.to(torch.int64)
    head = idx[:num_decode * (1 + k)]
    tail = idx[num_decode * (1 + k):]
    return torch.cat([head, tail.repeat_interleave(1 + k)])


def lm_head_mixed(hidden: torch.Tensor, head: LMHeadVerifier, logits_indices: torch.Tensor, num_decode: int,
                  draft_token_ids: torch.Tensor | None, num_drafts: torch.Tensor | None,
                  temperatures: torch.Tensor, prefill_temperatures: torch.Tensor,
                  uniforms: torch.Tensor | None = None, exp_noise: torch.Tensor | None = None
                  ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The token decisions of a mixed step (nanovllm/engine/model_runner.py:513-533) in one pass over the LM head
    weight: (num_accepted [D], next_token [D], first_token [P]) for the D decode requests (k = the width of
    draft_token_ids [D, k], or 0 when it is None) and the P finished prefill chunks whose rows logits_indices
    lists after the decode rows (mixed_batch, model_runner.py:58-61). temperatures [D] and
    prefill_temperatures [P] as the reference's; uniforms [D+P, k] / exp_noise [D+P, V] inject the noise of
    the D decode requests, then the P chunks."""
    device = hidden.device
    k = 0 if draft_token_ids is None else draft_token_ids.size(1)
    D = num_decode
    P = logits_indices.numel() - D * (1 + k)
    if P < 0:
        raise ValueError("lm_head_mixed: logits_indices lists fewer than num_decode * (1 + k) rows")
    drafts = torch.zeros(D + P, k, dtype=torch.int64, device=device)
    nd = torch.zeros(D + P, dtype=torch.int64, device=device)
    if k:
        drafts[:D] = draft_token_ids
        nd[:D] = num_drafts
    temps = torch.cat([temperatures.float().to(device), prefill_temperatures.float().to(device)])
    acc, nxt = lm_head_verify(hidden, head, drafts, nd, temps, logits_indices=mixed_rows(logits_indices, D, k),
                              uniforms=uniforms, exp_noise=exp_noise)
    return acc[:D], nxt[:D], nxt[D:]
