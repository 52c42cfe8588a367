"""Whole-model decode and verify steps replayed from HIP graphs: the caller of the spec-verify attention on the
headline path (counterpart of ModelRunner.run / run_verify, nanovllm/engine/model_runner.py:399-414,465-485,
with prepare_decode :319-362, run_model :370-390 and capture_cudagraph :646-675).

Every sequence of a step brings n query tokens: n = 1 for plain decode, n = 1 + k to verify k guesses. A step
of B sequences is padded to the next batch bucket (1, 2, 4, 8, then multiples of 16, the reference's
batch_buckets) with empty sequences (token 0, position 0, slot -1, context length 0), and one graph per
(n, bucket) holds the whole model: per layer the model segment (norms and projections), the fused q/k RMSNorm +
rotary embedding + KV store, and the paged decode attention, then the final segment into the hidden states.
The decode attention's dispatch order is planned once per step inside the graph (it reads the context lengths
on the device). The LM head and the token decision run after the replay on the rows that need them, as the
reference runs compute_logits and the sampler outside its graphs: lm_head_sample for plain decode,
lm_head_verify for a verify step (nanovllm_amd.layers.lm_head).

Every kernel's launch geometry depends on (n, bucket) only, so a replay computes what the same body run eagerly
computes, bitwise; padding sequences write no KV and their rows are never read.
"""
from __future__ import annotations

import torch

from nanovllm_amd import _lib
from nanovllm_amd.engine.metadata import batch_buckets, decode_batch
from nanovllm_amd.layers.rotary_embedding import qk_norm_rope_store


def _bucket(buckets: list[int], x: int) -> int:
    for b in buckets:
        if b >= x:
            return b
    raise ValueError(f"batch of {x} exceeds the largest bucket {buckets[-1]}")


class DecodeStepRunner:
    """Decode / verify steps over `layers` (objects with the per-layer paged caches `k_cache` / `v_cache`,
    [NB, block_size, Hkv, D] bf16) and `model`, a segmented decoder such as Qwen3Segments: model(i, N, bufs)
    records segment i (it reads bufs["o"], the previous layer's attention output, and writes bufs["qkv"], layer
    i's qkv projection), model.pre_attn() gives (cos_sin_cache, per-layer (q_norm, k_norm), eps), model.input_ids
    takes the step's token ids and model.hidden_out[:N] holds the final hidden states after a step.

    table_width: the block tables' fixed width (the reference pads decode tables to max_num_blocks,
    model_runner.py:357-360); max_batch: the largest batch (the last bucket)."""

    def __init__(self, layers, model, num_heads: int, num_kv_heads: int, head_dim: int, scale: float,
                 block_size: int = 256, table_width: int = 16, max_batch: int = 64, query_tokens=(1, 5),
                 device=None):
        self.layers = list(layers)
        self.model = model
        self.Hq, self.Hkv, self.D, self.scale = num_heads, num_kv_heads, head_dim, scale
        self.block_size, self.W = block_size, table_width
        self.buckets = batch_buckets(max_batch)
        self.ns = sorted(set(query_tokens))
        self.device = torch.device(device) if device is not None else self.layers[0].k_cache.device
        cos_sin, weights, eps = model.pre_attn()
        if weights is not None and len(weights) != len(self.layers):
            raise ValueError("one (q_norm, k_norm) pair per layer")
        self.cos_sin, self.norm_weights, self.eps = cos_sin.reshape(cos_sin.size(0), -1), weights, float(eps)
        Bmax, Nmax = self.buckets[-1], self.buckets[-1] * self.ns[-1]
        if model.input_ids.numel() < Nmax:
            raise ValueError(f"the model's buffers hold {model.input_ids.numel()} tokens, a step needs {Nmax}")
        dev = self.device
        self.bufs = dict(
            q=torch.zeros(Nmax, num_heads, head_dim, dtype=torch.bfloat16, device=dev),
            o=torch.zeros(Nmax, num_heads, head_dim, dtype=torch.bfloat16, device=dev),
            qkv=torch.zeros(Nmax, (num_heads + 2 * num_kv_heads) * head_dim, dtype=torch.bfloat16, device=dev),
        )
        # metadata, staged through pinned memory in one copy per step: int64 [input_ids N | positions N],
        # int32 [slot_mapping N | context_lens B | block_tables B x W]
        self._i64 = torch.zeros(2 * Nmax, dtype=torch.int64, device=dev)
        self._i32 = torch.zeros(Nmax + Bmax + Bmax * table_width, dtype=torch.int32, device=dev)
        self._i64_staging = torch.zeros_like(self._i64, device="cpu").pin_memory()
        self._i32_staging = torch.zeros_like(self._i32, device="cpu").pin_memory()
        lib = _lib.load()
        self._ws_bytes = max(lib.sd_paged_decode_workspace_size(B, n, num_heads, num_kv_heads, head_dim, block_size,
                                                                table_width)
                             for n in self.ns for B in self.buckets)
        self._ws = torch.empty(max(self._ws_bytes, 256), dtype=torch.uint8, device=dev)
        self._copied = torch.cuda.Event()
        self._copied.record(torch.cuda.current_stream(dev))
        self.graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}
        self._pool = None

    # ---- host side ----
    def prepare(self, seqs, num_query_tokens: int, with_drafts: bool = True) -> dict:
        """Host layout of a step (decode_batch: each sequence's last token, its guesses when with_drafts, padded
        to num_query_tokens), the batch padded to its bucket; adds n, B (bucket) and the real batch size."""
        if num_query_tokens not in self.ns:
            raise ValueError(f"no graphs for {num_query_tokens} query tokens (have {self.ns})")
        for seq in seqs:
            if len(seq.block_table) > self.W:
                raise ValueError(f"block table of {len(seq.block_table)} blocks exceeds the width {self.W}")
        b = decode_batch(seqs, num_query_tokens, self.block_size, self.buckets, self.W, with_drafts=with_drafts)
        b.update(n=num_query_tokens, B=len(seqs) + b["num_padding"], real=len(seqs))
        return b

    def load(self, layout: dict) -> None:
        """Copies a prepared layout's metadata to the device buffers (one copy per dtype, current stream)."""
        n, B, W = layout["n"], layout["B"], self.W
        N = n * B
        self._copied.synchronize()  # the previous step's copies may still read the staging buffers
        i64 = torch.tensor(layout["input_ids"] + layout["positions"], dtype=torch.int64)
        tables = [x for row in layout["block_tables"] for x in row]
        i32 = torch.tensor(layout["slot_mapping"] + layout["context_lens"] + tables, dtype=torch.int32)
        assert i64.numel() == 2 * N and i32.numel() == N + B + B * W
        self._i64_staging[:i64.numel()] = i64
        self._i32_staging[:i32.numel()] = i32
        stream = torch.cuda.current_stream(self.device)
        self._i64[:i64.numel()].copy_(self._i64_staging[:i64.numel()], non_blocking=True)
        self._i32[:i32.numel()].copy_(self._i32_staging[:i32.numel()], non_blocking=True)
        self._copied.record(stream)

    def _views(self, n: int, B: int):
        N, W = n * B, self.W
        ids, pos = self._i64[:N], self._i64[N:2 * N]
        slots, lens = self._i32[:N], self._i32[N:N + B]
        tables = self._i32[N + B:N + B + B * W].view(B, W)
        return ids, pos, slots, lens, tables

    # ---- device side ----
    def _body(self, n: int, B: int) -> None:
        """The whole model for bucket (n, B): token ids into the model, per layer segment + fused
        pre-attention + decode attention, then the last segment."""
        lib = _lib.load()
        stream = _lib.stream_of(self.device)
        N = n * B
        ids, pos, slots, lens, tables = self._views(n, B)
        Hq, Hkv, D, W, bs = self.Hq, self.Hkv, self.D, self.W, self.block_size
        q, o, qkv = self.bufs["q"], self.bufs["o"], self.bufs["qkv"][:N]
        ws, nws = self._ws.data_ptr(), self._ws.numel()
        self.model.input_ids[:N].copy_(ids)
        _lib.check(lib.sd_paged_decode_plan(lens.data_ptr(), B, n, Hq, Hkv, ws, nws, stream), "sd_paged_decode_plan")
        for i, layer in enumerate(self.layers):
            self.model(i, N, self.bufs)
            kc, vc = layer.k_cache, layer.v_cache
            qw, kw = self.norm_weights[i] if self.norm_weights is not None else (None, None)
            qk_norm_rope_store(pos, qkv[:, :Hq * D].view(N, Hq, D), qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D),
                               qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D), qw, kw, self.eps, self.cos_sin, kc, vc,
                               slots, q_out=q[:N], write_k=False)
            _lib.check(lib.sd_paged_decode_planned(
                q.data_ptr(), q.stride(0), kc.data_ptr(), vc.data_ptr(), kc.size(0), bs, lens.data_ptr(),
                tables.data_ptr(), W, B, n, Hq, Hkv, D, self.scale, o.data_ptr(), o.stride(0), ws, nws, stream),
                "sd_paged_decode_planned")
        self.model(len(self.layers), N, self.bufs)

    def capture(self, n: int, B: int) -> torch.cuda.CUDAGraph:
        """Records the graph of bucket (n, B) after one eager warm-up run of the same body on the metadata
        currently loaded (all graphs share one memory pool, biggest first as the reference captures)."""
        self._body(n, B)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=self._pool):
            self._body(n, B)
        if self._pool is None:
            self._pool = g.pool()
        self.graphs[(n, B)] = g
        torch.cuda.synchronize(self.device)
        return g

    def run(self, layout: dict, use_graph: bool = True) -> torch.Tensor:
        """One step on a prepared layout: loads its metadata and replays its bucket's graph (recorded on first
        use), or runs the same body eagerly. Returns the hidden states of the real sequences' rows,
        model.hidden_out[:real * n] (valid until the next step)."""
        n, B = layout["n"], layout["B"]
        self.load(layout)
        if not use_graph:
            self._body(n, B)
        else:
            g = self.graphs.get((n, B))
            if g is None:
                self.capture(n, B)   # its warm-up already ran this step once; the replay would store the same KV
            else:
                g.replay()
        return self.model.hidden_out[:layout["real"] * n]
