"""Attention for the spec-decode engine on MI355X: drop-in for nanovllm/layers/attention.py.

Same module contract as the reference (attention.py:43-79): ``Attention(num_heads, head_dim, scale,
num_kv_heads)`` with ``k_cache`` / ``v_cache`` attributes set by the model runner (per-layer views
[NB, block_size, Hkv, D] of one cache tensor) and ``forward(q, k, v)`` reading the global Context. The work
runs in HIP kernels of libsd_attn.so on torch's current stream, with no host synchronization, so the decode
path can be captured in a hipGraph (torch.cuda.graph).
"""
import torch
from torch import nn

from nanovllm_amd import _lib
from nanovllm_amd.utils.context import get_context


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """Scatter this step's K/V rows into the paged caches; slot -1 rows are skipped
    (nanovllm/layers/attention.py:33-40 contract, same stride requirements)."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    _require(key.stride(-1) == 1 and value.stride(-1) == 1, "store_kvcache: last dim must be contiguous")
    _require(key.stride(1) == head_dim and value.stride(1) == head_dim, "store_kvcache: head stride must be head_dim")
    _require(k_cache.stride(1) == D and v_cache.stride(1) == D, "store_kvcache: cache slot stride must be Hkv*D")
    _require(slot_mapping.numel() == N, "store_kvcache: slot_mapping must have one entry per token")
    _require(key.dtype == torch.bfloat16 and value.dtype == torch.bfloat16 and k_cache.dtype == torch.bfloat16
             and v_cache.dtype == torch.bfloat16, "store_kvcache: bf16 tensors required")
    _require(slot_mapping.dtype == torch.int32 and slot_mapping.is_contiguous(), "store_kvcache: int32 slot_mapping")
    _require(k_cache.is_contiguous() and v_cache.is_contiguous(), "store_kvcache: caches must be contiguous")
    if N == 0:
        return
    lib = _lib.load()
    rc = lib.sd_store_kvcache(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_cache.data_ptr(),
                              v_cache.data_ptr(), k_cache.numel() // D, slot_mapping.data_ptr(), N, num_heads,
                              head_dim, _lib.stream_of(key.device))
    _lib.check(rc, "sd_store_kvcache")


def _as_rows(x: torch.Tensor, heads: int, head_dim: int) -> torch.Tensor:
    """[tokens, heads, head_dim] view with head stride head_dim and unit dim stride (copy only if needed)."""
    x = x.view(-1, heads, head_dim) if x.is_contiguous() else x.reshape(-1, heads, head_dim)
    if x.stride(2) != 1 or x.stride(1) != head_dim or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    return x


# Per decode workspace (keyed by its address, so per device): (owner, key) of the decode order it holds, set
# by the last sd_paged_decode_plan call into it.
_decode_plans: dict = {}


def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           context_lens: torch.Tensor, block_tables: torch.Tensor, scale: float,
                           out: torch.Tensor | None = None, plan_owner: object | None = None) -> torch.Tensor:
    """q [B, n, Hq, D] -> [B*n, Hq, D]: flash_attn_with_kvcache(causal=True) semantics (attention.py:71-78).

    plan_owner: an object that lives as long as this context_lens (the step's Context). The sequences are
    then dispatched longest first, in an order planned once per owner and batch shape and reused by later
    layers (the order never changes results). A plan made while a graph is captured is only reused within
    captures, one made eagerly only eagerly, so that every graph holds the plan it replays with."""
    B, n, Hq, hd = q.shape
    NB, bs, Hkv, _ = k_cache.shape
    _require(q.dtype == torch.bfloat16 and k_cache.dtype == torch.bfloat16, "paged_decode_attention: bf16 required")
    _require(context_lens.dtype == torch.int32 and block_tables.dtype == torch.int32, "int32 lens / block tables")
    _require(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    block_tables = block_tables if block_tables.is_contiguous() else block_tables.contiguous()
    qr = _as_rows(q, Hq, hd)
    if out is None:
        out = torch.empty(B * n, Hq, hd, dtype=q.dtype, device=q.device)
    W = block_tables.size(1)
    lib = _lib.load()
    nbytes = lib.sd_paged_decode_workspace_size(B, n, Hq, Hkv, hd, bs, W)
    ws = _lib.workspace(nbytes, q.device, tag="decode")
    stream = _lib.stream_of(q.device)
    fn = lib.sd_paged_decode
    if plan_owner is not None and B > 0:
        capturing = torch.cuda.is_current_stream_capturing()
        key = (context_lens.data_ptr(), B, n, Hq, Hkv, ws.data_ptr(), ws.numel(), capturing)
        cached = _decode_plans.get(ws.data_ptr())
        if not (cached is not None and cached[0] is plan_owner and cached[1] == key):
            _lib.check(lib.sd_paged_decode_plan(context_lens.data_ptr(), B, n, Hq, Hkv, ws.data_ptr(), ws.numel(),
                                                stream), "sd_paged_decode_plan")
            _decode_plans[ws.data_ptr()] = (plan_owner, key)
        fn = lib.sd_paged_decode_planned
    else:
        _decode_plans.pop(ws.data_ptr(), None)  # an unplanned call may write partials over the order
    rc = fn(qr.data_ptr(), qr.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), NB, bs, context_lens.data_ptr(),
            block_tables.data_ptr(), W, B, n, Hq, Hkv, hd, scale, out.data_ptr(), out.stride(0), ws.data_ptr(),
            ws.numel(), stream)
    _lib.check(rc, "sd_paged_decode")
    return out


# Per varlen workspace (keyed by its address, so per device): (owner, key) of the plan it holds, set by the
# last sd_varlen_plan call into it. The owner is held here (not tagged: the Context dataclass has slots), so
# its id cannot be reused meanwhile.
_varlen_plans: dict = {}
plan_stats = {"plans": 0, "reuses": 0}


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                     cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int, scale: float,
                     block_table: torch.Tensor | None = None, out: torch.Tensor | None = None,
                     plan_owner: object | None = None) -> torch.Tensor:
    """flash_attn_varlen_func(causal=True) semantics (attention.py:64-70). q [Nq, Hq, D]; k / v are fresh
    [Nk, Hkv, D] rows, or the paged caches [NB, bs, Hkv, D] when block_table is given.

    plan_owner: an object that lives exactly as long as this cu_seqlens_q / cu_seqlens_k (the step's Context).
    The work lists derived from them are then computed once and reused by every later call with the same
    owner and sizes, as long as no other plan has replaced them in the varlen workspace. Never reused while
    a graph is being captured."""
    Nq, Hq, hd = q.shape
    _require(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16,
             "varlen_attention: bf16 required")
    _require(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32, "int32 cu_seqlens")
    nseq = cu_seqlens_q.numel() - 1
    qr = _as_rows(q, Hq, hd)
    if out is None:
        out = torch.empty(Nq, Hq, hd, dtype=q.dtype, device=q.device)
    lib = _lib.load()
    if block_table is not None:
        NB, bs, Hkv, _ = k.shape
        _require(k.is_contiguous() and v.is_contiguous(), "paged caches must be contiguous")
        block_table = block_table if block_table.is_contiguous() else block_table.contiguous()
        _require(block_table.dtype == torch.int32, "int32 block table")
        kr, vr, W, total_k = k, v, block_table.size(1), 0
        ks = vs = Hkv * hd
    else:
        Hkv = k.size(-2)
        kr, vr = _as_rows(k, Hkv, hd), _as_rows(v, Hkv, hd)
        NB, bs, W, total_k = 0, 0, 0, kr.size(0)
        ks, vs = kr.stride(0), vr.stride(0)
    nbytes = lib.sd_varlen_workspace_size(nseq, Nq, max_seqlen_k, Hq, Hkv, hd)
    ws = _lib.workspace(nbytes, q.device, tag="varlen")
    stream = _lib.stream_of(q.device)
    fn = lib.sd_varlen_attention
    if plan_owner is not None and not torch.cuda.is_current_stream_capturing():
        key = (cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), nseq, Nq, max_seqlen_q, Hq, Hkv, ws.data_ptr(),
               ws.numel())
        cached = _varlen_plans.get(ws.data_ptr())
        if cached is not None and cached[0] is plan_owner and cached[1] == key:
            plan_stats["reuses"] += 1
        else:
            _lib.check(lib.sd_varlen_plan(cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), nseq, Nq, max_seqlen_q,
                                          Hq, Hkv, ws.data_ptr(), ws.numel(), stream), "sd_varlen_plan")
            _varlen_plans[ws.data_ptr()] = (plan_owner, key)
            plan_stats["plans"] += 1
        fn = lib.sd_varlen_attention_planned
    else:
        _varlen_plans.pop(ws.data_ptr(), None)  # the call below rewrites the work lists
    rc = fn(qr.data_ptr(), qr.stride(0), kr.data_ptr(), ks, vr.data_ptr(), vs, total_k, NB, bs, _lib.ptr(block_table), W,
            cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), nseq, Nq, max_seqlen_q, max_seqlen_k, Hq, Hkv, hd,
            scale, out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "sd_varlen_attention")
    return out


class Attention(nn.Module):
    """Drop-in for nanovllm.layers.attention.Attention (attention.py:43-79)."""

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_stored: bool = False) -> torch.Tensor:
        """kv_stored: this step's k / v rows are already in the caches (qk_norm_rope_store did the store), so
        the store of attention.py:62-63 is skipped; k / v are then only read by a prefill without block
        tables (and may be None otherwise)."""
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        if not kv_stored and k_cache.numel() and v_cache.numel():
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
        if context.is_prefill:
            if context.block_tables is not None:    # prefix cache / mixed batching: keys from the paged cache
                k, v = k_cache, v_cache
            return varlen_attention(q, k, v, context.cu_seqlens_q, context.cu_seqlens_k, context.max_seqlen_q,
                                    context.max_seqlen_k, self.scale, context.block_tables, plan_owner=context)
        # decode / verify: every sequence brings the same number of query tokens (1, or 1+k)
        num_seqs = context.context_lens.size(0)
        q = q.reshape(num_seqs, -1, self.num_heads, self.head_dim)
        return paged_decode_attention(q, k_cache, v_cache, context.context_lens, context.block_tables, self.scale,
                                      plan_owner=context)
