"""Oracle for paged decode / verify attention and varlen (prefill, mixed) attention.
Test infrastructure only.

Semantics restated from the reference call sites (flash-attn 2.8.3 itself is a
third-party CUDA library that is not vendored and not installed here):

* decode / verify, nanovllm/layers/attention.py:71-78: q is [B, n, Hq, D];
  context_lens[b] counts the cached keys INCLUDING the n new ones; causal is
  aligned to the bottom right (attention.py:74), so query i of n sees keys
  0 .. context_lens[b] - n + i. Key j of sequence b lives at
  cache[block_tables[b, j // bs], j % bs, h // (Hq/Hkv)].
* varlen, nanovllm/layers/attention.py:64-70: sequence s has
  Lq = cu_q[s+1]-cu_q[s] queries and Lk = cu_k[s+1]-cu_k[s] keys; query i sees
  keys j <= Lk - Lq + i. Keys come from the paged caches through
  block_tables[s] when block_tables is given (prefix cache / mixed batching,
  attention.py:65-66), else from rows cu_k[s] + j of the fresh k / v.

Softmax in fp32 with scale = head_dim ** -0.5 (nanovllm/models/qwen3.py:39).
A query row that sees no key returns zeros (a padding sequence with
context_len 0 must give finite output).
"""
import torch


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, limits: torch.Tensor, scale: float) -> torch.Tensor:
    """q [Lq, Hq, D], k/v [Lk, Hkv, D], limits [Lq] = number of visible keys per query -> fp32 [Lq, Hq, D]."""
    Lq, Hq, D = q.shape
    Lk, Hkv, _ = k.shape
    g = Hq // Hkv
    qf = q.float().transpose(0, 1)                                  # [Hq, Lq, D]
    kf = k.float().repeat_interleave(g, dim=1).transpose(0, 1)       # [Hq, Lk, D]  q head h -> kv head h // g
    vf = v.float().repeat_interleave(g, dim=1).transpose(0, 1)
    s = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * scale    # [Hq, Lq, Lk]
    visible = torch.arange(Lk)[None, :] < limits[:, None]           # [Lq, Lk]
    s = s.masked_fill(~visible[None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)                                 # rows that see nothing -> 0
    o = torch.matmul(p, vf)                                          # [Hq, Lq, D]
    return o.transpose(0, 1).contiguous()


def _gather_pages(cache: torch.Tensor, table_row: torch.Tensor, n: int) -> torch.Tensor:
    """First n keys of one sequence from a paged cache [NB, bs, Hkv, D] -> [n, Hkv, D]."""
    bs = cache.size(1)
    nblk = (n + bs - 1) // bs
    blocks = table_row[:nblk].long()
    return cache[blocks].reshape(nblk * bs, cache.size(2), cache.size(3))[:n]


def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           context_lens: torch.Tensor, block_tables: torch.Tensor, scale: float) -> torch.Tensor:
    """q [B, n, Hq, D] -> fp32 [B, n, Hq, D] (attention.py:71-78, bottom-right causal)."""
    B, n, Hq, D = q.shape
    out = torch.zeros(B, n, Hq, D, dtype=torch.float32)
    lens = context_lens.cpu().long()
    tables = block_tables.cpu()
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        k = _gather_pages(k_cache, tables[b], L)
        v = _gather_pages(v_cache, tables[b], L)
        limits = L - n + 1 + torch.arange(n)
        out[b] = _attend(q[b], k, v, limits.clamp(min=0), scale)
    return out


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                     cu_seqlens_k: torch.Tensor, scale: float, block_tables: torch.Tensor | None = None) -> torch.Tensor:
    """q [Nq, Hq, D]; k/v either fresh [Nk, Hkv, D] rows or paged caches [NB, bs, Hkv, D] when block_tables
    is given -> fp32 [Nq, Hq, D] (attention.py:64-70)."""
    Nq, Hq, D = q.shape
    out = torch.zeros(Nq, Hq, D, dtype=torch.float32)
    cq = cu_seqlens_q.cpu().long().tolist()
    ck = cu_seqlens_k.cpu().long().tolist()
    tables = block_tables.cpu() if block_tables is not None else None
    for s in range(len(cq) - 1):
        Lq, Lk = cq[s + 1] - cq[s], ck[s + 1] - ck[s]
        if Lq == 0:
            continue
        if tables is not None:
            ks = _gather_pages(k, tables[s], Lk)
            vs = _gather_pages(v, tables[s], Lk)
        else:
            ks, vs = k[ck[s]:ck[s + 1]], v[ck[s]:ck[s + 1]]
        limits = (Lk - Lq + 1 + torch.arange(Lq)).clamp(min=0)
        out[cq[s]:cq[s + 1]] = _attend(q[cq[s]:cq[s + 1]], ks, vs, limits, scale)
    return out
