"""Rotary embedding and the fused per-token work in front of attention, on MI355X.

Drop-ins for nanovllm/layers/rotary_embedding.py (RotaryEmbedding, get_rope) plus ``qk_norm_rope_store``, which
does Qwen3Attention.pre_attn's q_norm / k_norm / rotary_emb (nanovllm/models/qwen3.py:89-96) and the KV store
that Attention.forward would do next (nanovllm/layers/attention.py:62-63) in one HIP kernel
(sd_qk_norm_rope_store), reading the qkv row once. Launches go on torch's current stream with no host sync,
so both can be captured in a hipGraph.
"""
from functools import lru_cache

import torch
from torch import nn

from nanovllm_amd import _lib


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _heads(x: torch.Tensor, name: str) -> torch.Tensor:
    """[tokens, heads, head_dim] view with unit element stride and head stride head_dim (no copy)."""
    _require(x.dim() == 3, f"{name}: expected [tokens, heads, head_dim]")
    _require(x.dtype == torch.bfloat16, f"{name}: bf16 required")
    _require(x.stride(2) == 1 and x.stride(1) == x.size(2), f"{name}: heads must be contiguous within a token")
    return x


def qk_norm_rope_store(positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor | None,
                       q_norm_weight: torch.Tensor | None, k_norm_weight: torch.Tensor | None, eps: float,
                       cos_sin_cache: torch.Tensor, k_cache: torch.Tensor | None = None,
                       v_cache: torch.Tensor | None = None, slot_mapping: torch.Tensor | None = None,
                       q_out: torch.Tensor | None = None, k_out: torch.Tensor | None = None,
                       write_k: bool = True):
    """q [N, Hq, D], k / v [N, Hkv, D] bf16 (views of the qkv split are fine) -> (q, k) after
    RMSNorm (weights None: none, the qkv-bias models of qwen3.py:93) and the rotary embedding.

    With k_cache / v_cache ([NB, block_size, Hkv, D], the Attention module's caches; None or empty: no store)
    and slot_mapping, the rotated k and v are also stored (slot -1 skipped); the caller then passes
    kv_stored=True to Attention.forward. q_out / k_out default to new tensors; pass q / k for in place.
    write_k=False skips k_out (decode steps read k from the cache only) and returns None for it."""
    q, k = _heads(q, "q"), _heads(k, "k")
    N, Hq, D = q.shape
    Hkv = k.size(1)
    dev = q.device
    _require(k.size(0) == N and k.size(2) == D, "k: shape mismatch with q")
    _require(positions.numel() == N and positions.dtype == torch.int64 and positions.is_contiguous(),
             "positions: int64 [N] required")
    cs = cos_sin_cache.reshape(cos_sin_cache.size(0), -1)
    _require(cs.dtype == torch.float32 and cs.is_contiguous() and cs.size(1) == D,
             "cos_sin_cache: fp32 [max_position, head_dim] required")
    if q_norm_weight is not None or k_norm_weight is not None:
        _require(q_norm_weight is not None and k_norm_weight is not None, "give both norm weights or neither")
        for w in (q_norm_weight, k_norm_weight):
            _require(w.dtype == torch.bfloat16 and w.is_contiguous() and w.numel() == D,
                     "norm weights: bf16 [head_dim] required")
    # empty caches (before the KV cache is allocated) store nothing, as attention.py:62 skips the store
    store = k_cache is not None and k_cache.numel() > 0 and v_cache is not None and v_cache.numel() > 0
    if store:
        _require(v is not None and slot_mapping is not None, "store needs v and slot_mapping")
        v = _heads(v, "v")
        _require(v.shape == k.shape, "v: shape mismatch with k")
        _require(k_cache.dtype == torch.bfloat16 and v_cache.dtype == torch.bfloat16 and k_cache.is_contiguous()
                 and v_cache.is_contiguous() and k_cache.shape == v_cache.shape and k_cache.size(-2) == Hkv
                 and k_cache.size(-1) == D, "caches: contiguous bf16 [NB, block_size, Hkv, D] required")
        _require(slot_mapping.dtype == torch.int32 and slot_mapping.is_contiguous() and slot_mapping.numel() == N,
                 "slot_mapping: int32 [N] required")
    if q_out is None:
        q_out = torch.empty(N, Hq, D, dtype=torch.bfloat16, device=dev)
    if write_k and k_out is None:
        k_out = torch.empty(N, Hkv, D, dtype=torch.bfloat16, device=dev)
    q_out = _heads(q_out, "q_out")
    if write_k:
        k_out = _heads(k_out, "k_out")
    else:
        k_out = None
    if N == 0:
        return q_out, k_out
    lib = _lib.load()

    def ptr(t):
        return t.data_ptr() if t is not None else None

    rc = lib.sd_qk_norm_rope_store(
        q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), ptr(v) if store else None,
        v.stride(0) if store else 0, positions.data_ptr(), ptr(q_norm_weight), ptr(k_norm_weight), eps,
        cs.data_ptr(), cs.size(0), q_out.data_ptr(), q_out.stride(0), ptr(k_out),
        k_out.stride(0) if k_out is not None else 0, ptr(k_cache) if store else None,
        ptr(v_cache) if store else None, k_cache.numel() // (Hkv * D) if store else 0,
        ptr(slot_mapping) if store else None, N, Hq, Hkv, D, _lib.stream_of(dev))
    _lib.check(rc, "sd_qk_norm_rope_store")
    return q_out, k_out


class RotaryEmbedding(nn.Module):
    """Drop-in for nanovllm.layers.rotary_embedding.RotaryEmbedding (rotary_embedding.py:17-48): the same
    cos_sin_cache buffer ([max_position, 1, head_size] fp32, cos then sin), forward(positions, query, key)
    -> (query, key) rotated by the HIP kernel."""

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int, base: float) -> None:
        super().__init__()
        self.head_size = head_size
        _require(rotary_dim == head_size, "rotary_dim must equal head_size")
        inv_freq = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float) / rotary_dim))
        t = torch.arange(max_position_embeddings, dtype=torch.float)
        freqs = torch.einsum("i,j -> ij", t, inv_freq)
        cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)
        self.register_buffer("cos_sin_cache", cache, persistent=False)

    def forward(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        N = positions.numel()
        q = query.view(N, -1, self.head_size)
        k = key.view(N, -1, self.head_size)
        qo, ko = qk_norm_rope_store(positions, q, k, None, None, None, 0.0, self.cos_sin_cache)
        return qo.view_as(query), ko.view_as(key)


@lru_cache(1)
def get_rope(head_size: int, rotary_dim: int, max_position: int, base: float) -> RotaryEmbedding:
    """rotary_embedding.py:51-59: one shared module per configuration."""
    return RotaryEmbedding(head_size, rotary_dim, max_position, base)
