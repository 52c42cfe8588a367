"""Mixed prefill+decode steps replayed from HIP graphs: the runtime around the attention hot path on a mixed
step (the caller of the KV store and the varlen attention; counterpart of the reference's mixed-step path,
nanovllm/engine/model_runner.py:487-589 run_mixed / run_piecewise, :605-627 buckets and buffers, :646-696
capture).

The reference records the model segments between attentions as CUDA graphs per total-token bucket and runs
every attention eagerly between the replays, because flash-attn's varlen launch depends on the step's
lengths. Here the varlen kernels' launch geometry depends only on (num_seqs, total_q, max_seqlen_q), so one
graph per (token bucket, sequence bucket) holds the whole step: the work-list plan (once per step), then per
layer the optional model segment, the KV-cache store and the attention. A step refreshes the metadata with one
host-to-device copy from pinned memory and replays that graph. Optionally each layer's q/k RMSNorm, rotary
embedding and KV store run fused in front of its attention (pre_attn).

Padding. A step of n tokens in S_real requests runs in bucket (N, S): N >= n tokens, S >= S_real + 1
sequences. Rows n..N-1 form one padding sequence with no keys (Lk = 0): the kernels write zeros for them and
their slots are -1, so nothing is stored. The other padding sequences are empty (Lq = Lk = 0) with all -1
block-table rows. Every real row's result is bitwise the same as in an unpadded eager call, because the
kernels' reduction order depends only on key positions.
"""
from __future__ import annotations

import torch

from nanovllm_amd import _lib
from nanovllm_amd.engine.metadata import mixed_batch
from nanovllm_amd.layers.rotary_embedding import qk_norm_rope_store


def token_buckets(max_num_batched_tokens: int, step: int = 16) -> list[int]:
    """Total token counts mixed steps are padded to: every `step` up to max_num_batched_tokens (the reference
    uses 64 up to min(budget, 512), model_runner.py:605-615; every kernel here is capturable, so the buckets
    go up to the whole budget). The step is 16 rather than 64: a bucket's padding rows and its work lists'
    upper bounds cost launch slots in every layer (the 2048-token mixed step of 1164 tokens and 51 requests:
    1.749 ms replayed in bucket (1216, 64), 1.729 ms in (1168, 56))."""
    return list(range(step, max_num_batched_tokens, step)) + [max_num_batched_tokens]


def seq_buckets(max_num_seqs: int, step: int = 8) -> list[int]:
    """Sequence counts (including the padding sequence): 2, 4, then every `step`, then max_num_seqs + 1."""
    out = [b for b in (2, 4) if b < max_num_seqs + 1 and b < step]
    out += list(range(step, max_num_seqs + 1, step))
    return out + [max_num_seqs + 1]


def _bucket(buckets: list[int], x: int) -> int:
    for b in buckets:
        if b >= x:
            return b
    raise ValueError(f"{x} exceeds the largest bucket {buckets[-1]}")


def mixed_step_layout(seqs, k: int, block_size: int, table_width: int, tok_buckets: list[int],
                      sq_buckets: list[int]) -> dict:
    """Host layout of a mixed step (decode requests first, then prefill chunks, as the reference orders them,
    model_runner.py:512), padded to its bucket: the mixed_batch fields plus n (real tokens), N / S (bucket
    tokens / sequences) and `meta`, the int32 metadata in staging order: cu_seqlens_q [S+1], cu_seqlens_k
    [S+1], slot_mapping [N], block_tables [S, table_width] (-1 padded); `positions_padded` lists the N rows'
    positions (0 for padding rows)."""
    b = mixed_batch(seqs, k, block_size)
    n, Sr = len(b["input_ids"]), len(seqs)
    N, S = _bucket(tok_buckets, n), _bucket(sq_buckets, Sr + 1)
    for seq in seqs:
        if len(seq.block_table) > table_width:
            raise ValueError(f"block table of {len(seq.block_table)} blocks exceeds the width {table_width}")
    positions = list(b["positions"]) + [0] * (N - n)
    cu_q = list(b["cu_seqlens_q"]) + [N] * (S - Sr)            # sequence Sr: the padding rows n..N-1
    cu_k = list(b["cu_seqlens_k"]) + [b["cu_seqlens_k"][-1]] * (S - Sr)  # no keys
    slots = list(b["slot_mapping"]) + [-1] * (N - n)
    tables = []
    for seq in seqs:
        tables += list(seq.block_table) + [-1] * (table_width - len(seq.block_table))
    tables += [-1] * ((S - Sr) * table_width)
    b.update(n=n, N=N, S=S, meta=cu_q + cu_k + slots + tables, positions_padded=positions)
    return b


class MixedStepRunner:
    """Runs mixed steps over `layers` (objects with `k_cache` / `v_cache`, the per-layer paged caches
    [NB, block_size, Hkv, D] bf16, e.g. nanovllm_amd.layers.attention.Attention modules).

    segment(i, n, bufs): optional; records the model work of segment i for n (padded) tokens, as the
    reference's run_segment does (model_runner.py:536-556): segment i reads bufs["o"] (layer i-1's attention
    output, i > 0) and writes bufs["q"], bufs["k"], bufs["v"] for layer i; segment len(layers) is the last.
    It must be per token (no reads of step metadata). Without it the step is attention only: bufs["q"],
    bufs["k"], bufs["v"] hold the step's rows (written by the caller) and every layer reads them.

    pre_attn: optional (cos_sin_cache, norm_weights, eps): every layer's attention is preceded by the fused
    q/k RMSNorm + rotary embedding + KV store (qk_norm_rope_store, the reference's q_norm / k_norm /
    rotary_emb of qwen3.py:89-96 and the store of attention.py:62-63): cos_sin_cache is the RotaryEmbedding
    buffer (fp32, [max_position, D] or [max_position, 1, D]), norm_weights a list of per-layer (q_norm, k_norm)
    weights (None: a model with a qkv bias, no norm), eps the RMSNorm epsilon. The segments then write
    bufs["qkv"] [N, (Hq + 2 Hkv) D] (the qkv projection's output) and the step's positions travel with its
    metadata.

    Buffers (fixed addresses, sized for the largest bucket): bufs["q"] / ["o"] [N, Hq, D], bufs["k"] / ["v"]
    [N, Hkv, D] bf16 (and bufs["qkv"] with pre_attn). After run(), bufs["o"][:n] is the last layer's attention
    output."""

    def __init__(self, layers, num_heads: int, num_kv_heads: int, head_dim: int, scale: float,
                 block_size: int = 256, max_num_batched_tokens: int = 2048, max_num_seqs: int = 256,
                 table_width: int = 16, token_step: int = 16, segment=None, device=None, pre_attn=None):
        self.layers = list(layers)
        self.Hq, self.Hkv, self.D, self.scale = num_heads, num_kv_heads, head_dim, scale
        self.block_size, self.W = block_size, table_width
        self.token_buckets = token_buckets(max_num_batched_tokens, token_step)
        self.seq_buckets = seq_buckets(max_num_seqs)
        self.segment = segment
        self.device = torch.device(device) if device is not None else self.layers[0].k_cache.device
        Nmax, Smax = self.token_buckets[-1], self.seq_buckets[-1]
        dev = self.device
        self.bufs = dict(
            q=torch.zeros(Nmax, num_heads, head_dim, dtype=torch.bfloat16, device=dev),
            k=torch.zeros(Nmax, num_kv_heads, head_dim, dtype=torch.bfloat16, device=dev),
            v=torch.zeros(Nmax, num_kv_heads, head_dim, dtype=torch.bfloat16, device=dev),
            o=torch.zeros(Nmax, num_heads, head_dim, dtype=torch.bfloat16, device=dev),
        )
        self.pre_attn = None
        if pre_attn is not None:
            cos_sin, weights, eps = pre_attn
            if weights is not None and len(weights) != len(self.layers):
                raise ValueError("pre_attn: one (q_norm, k_norm) pair per layer")
            self.pre_attn = (cos_sin.reshape(cos_sin.size(0), -1), weights, float(eps))
            self.bufs["qkv"] = torch.zeros(Nmax, (num_heads + 2 * num_kv_heads) * head_dim, dtype=torch.bfloat16,
                                           device=dev)
            self._pos = torch.zeros(Nmax, dtype=torch.int64, device=dev)
            self._pos_staging = torch.zeros(Nmax, dtype=torch.int64, pin_memory=True)
        meta_len = 2 * (Smax + 1) + Nmax + Smax * table_width
        self._meta = torch.zeros(meta_len, dtype=torch.int32, device=dev)
        self._staging = torch.zeros(meta_len, dtype=torch.int32, pin_memory=True)
        lib = _lib.load()
        # The varlen workspace is not monotone in the bucket (few work items need residue partials), so it is
        # sized for the largest need over every (token, sequence) bucket.
        self._ws_bytes = max(lib.sd_varlen_workspace_size(S, N, table_width * block_size, num_heads, num_kv_heads,
                                                          head_dim)
                             for N in self.token_buckets for S in self.seq_buckets)
        self._ws = torch.empty(max(self._ws_bytes, 256), dtype=torch.uint8, device=dev)
        self._copied = torch.cuda.Event()  # the last staging copy has been read (the buffer is free again)
        self._copied.record(torch.cuda.current_stream(self.device))
        self.graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}
        self._pool = None

    # ---- host side ----
    def _views(self, N: int, S: int):
        """Device views of one bucket's metadata: cu_seqlens_q [S+1], cu_seqlens_k [S+1], slot_mapping [N],
        block_tables [S, W] (the staging buffer has the same layout)."""
        m, W = self._meta, self.W
        o1, o2, o3 = S + 1, 2 * (S + 1), 2 * (S + 1) + N
        return m[:o1], m[o1:o2], m[o2:o3], m[o3:o3 + S * W].view(S, W)

    def prepare(self, seqs, k: int) -> dict:
        """Host layout of a mixed step, padded to its bucket (see mixed_step_layout)."""
        return mixed_step_layout(seqs, k, self.block_size, self.W, self.token_buckets, self.seq_buckets)

    def load(self, layout: dict) -> None:
        """Copies a prepared layout's metadata to the bucket's device views (one copy, current stream)."""
        meta = layout["meta"]
        self._copied.synchronize()  # the previous step's copies may still read the staging buffers
        self._staging[:len(meta)] = torch.tensor(meta, dtype=torch.int32)
        self._meta[:len(meta)].copy_(self._staging[:len(meta)], non_blocking=True)
        if self.pre_attn is not None:
            pos = layout["positions_padded"]
            self._pos_staging[:len(pos)] = torch.tensor(pos, dtype=torch.int64)
            self._pos[:len(pos)].copy_(self._pos_staging[:len(pos)], non_blocking=True)
        self._copied.record(torch.cuda.current_stream(self.device))

    # ---- device side ----
    def _body(self, N: int, S: int) -> None:
        """The step for bucket (N, S): plan, then per layer segment + store + attention."""
        lib = _lib.load()
        stream = _lib.stream_of(self.device)
        cu_q, cu_k, slots, tables = self._views(N, S)
        Hq, Hkv, D, W, bs = self.Hq, self.Hkv, self.D, self.W, self.block_size
        q, k, v, o = (self.bufs[x] for x in ("q", "k", "v", "o"))
        ws, nws = self._ws.data_ptr(), self._ws.numel()
        _lib.check(lib.sd_varlen_plan(cu_q.data_ptr(), cu_k.data_ptr(), S, N, N, Hq, Hkv, ws, nws, stream),
                   "sd_varlen_plan")
        for i, layer in enumerate(self.layers):
            if self.segment is not None:
                self.segment(i, N, self.bufs)
            kc, vc = layer.k_cache, layer.v_cache
            if self.pre_attn is not None:
                cos_sin, weights, eps = self.pre_attn
                qkv = self.bufs["qkv"][:N]
                qw, kw = weights[i] if weights is not None else (None, None)
                qk_norm_rope_store(self._pos[:N], qkv[:, :Hq * D].view(N, Hq, D),
                                   qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D), qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D),
                                   qw, kw, eps, cos_sin, kc, vc, slots, q_out=q[:N], write_k=False)
            else:
                _lib.check(lib.sd_store_kvcache(k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), kc.data_ptr(),
                                                vc.data_ptr(), kc.numel() // (Hkv * D), slots.data_ptr(), N, Hkv, D,
                                                stream), "sd_store_kvcache")
            _lib.check(lib.sd_varlen_attention_planned(
                q.data_ptr(), q.stride(0), kc.data_ptr(), Hkv * D, vc.data_ptr(), Hkv * D, 0, kc.size(0), bs,
                tables.data_ptr(), W, cu_q.data_ptr(), cu_k.data_ptr(), S, N, N, W * bs, Hq, Hkv, D, self.scale,
                o.data_ptr(), o.stride(0), ws, nws, stream), "sd_varlen_attention_planned")
        if self.segment is not None:
            self.segment(len(self.layers), N, self.bufs)

    def capture(self, N: int, S: int) -> torch.cuda.CUDAGraph:
        """Records the graph of bucket (N, S) (after one eager warm-up run of the same body on the metadata
        currently loaded; all graphs share one memory pool)."""
        self._body(N, S)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=self._pool):
            self._body(N, S)
        if self._pool is None:
            self._pool = g.pool()
        self.graphs[(N, S)] = g
        torch.cuda.synchronize(self.device)
        return g

    def run(self, layout: dict, use_graph: bool = True) -> torch.Tensor:
        """One mixed step on a prepared layout: loads its metadata and replays its bucket's graph (recorded
        on first use), or runs the same body eagerly. Returns bufs["o"][:n]."""
        N, S = layout["N"], layout["S"]
        self.load(layout)
        if not use_graph:
            self._body(N, S)
        else:
            g = self.graphs.get((N, S))
            if g is None:
                g = self.capture(N, S)   # its warm-up already ran this step once: replaying would store twice
            else:
                g.replay()
        return self.bufs["o"][:layout["n"]]
