"""The model work between attentions of a piecewise mixed step: a Qwen3-shaped decoder stack with random bf16
weights (no checkpoint is read; the shapes set the step's cost), split at its attentions as the reference's
run_segment splits Qwen3ForCausalLM (nanovllm/engine/model_runner.py:536-556; nanovllm/models/qwen3.py:83-100
Qwen3Attention.pre_attn / post_attn, :178-201 Qwen3DecoderLayer.pre_attn / post_attn, :103-129 Qwen3MLP).

It is the `segment` callback of MixedStepRunner, which records it into the step's graph between the attentions:
  segment 0       embedding, then layer 0's input RMSNorm and qkv projection;
  segment i       layer i-1 after its attention (o_proj, post-attention RMSNorm with the residual add, gate/up
                  projection, SiLU-and-multiply, down projection), then layer i's input RMSNorm (residual add)
                  and qkv projection;
  segment L       the last layer after its attention and the final RMSNorm, into `hidden`.
Each layer's q/k RMSNorm, rotary embedding and KV store run in the runner's fused pre-attention kernel
(pass pre_attn=segments.pre_attn()), so the segments write the qkv projection into bufs["qkv"]. Every op works
on each token alone (no step metadata), so one recording serves every step padded to the same token count.
The norms follow the reference's RMSNorm arithmetic (nanovllm/layers/layernorm.py:16-38: fp32 mean of squares,
rsqrt, cast, times the weight); the GEMMs are torch's (hipBLASLt).

row_invariant=True runs the projections through RowInvariantLinear (sd_linear) and the norms through
sd_rms_norm instead: every op then computes a token's row the same way whatever the step's token count, so a
token's hidden state, and the greedy token picked from it, do not depend on the batch. That is what makes
greedy speculative decoding (1 + k rows per sequence) pick exactly the tokens of plain decoding (one row); with
the library GEMMs and reductions, whose kernels change with the row count, near-ties can flip.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from nanovllm_amd.layers import layernorm
from nanovllm_amd.layers.linear import RowInvariantLinear
from nanovllm_amd.layers.rotary_embedding import RotaryEmbedding


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.rms_forward (nanovllm/layers/layernorm.py:16-26)."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return xf.to(x.dtype) * weight


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """RMSNorm.add_rms_forward (nanovllm/layers/layernorm.py:28-38): (norm(x + residual), x + residual)."""
    xf = x.float() + residual.float()
    res = xf.to(x.dtype)
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return xf.to(x.dtype) * weight, res


class Qwen3Segments:
    """Random-init Qwen3 decoder stack (defaults: Qwen3-8B shapes) as MixedStepRunner segments.

    Buffers (fixed addresses, max_tokens rows): input_ids int64 (the caller writes a step's token ids, 0 for
    padding rows, before the runner's run), residual and hidden bf16 [max_tokens, hidden]; after a step,
    hidden_out[:n] holds the final-norm hidden states, to which the caller applies the LM head `lm_head`
    (with the verifier: nanovllm_amd.layers.lm_head.LMHeadVerifier(seg.lm_head))."""

    def __init__(self, num_layers: int = 36, hidden: int = 4096, num_heads: int = 32, num_kv_heads: int = 8,
                 head_dim: int = 128, intermediate: int = 12288, vocab: int = 151936, eps: float = 1e-6,
                 rope_theta: float = 1e6, max_position: int = 40960, max_tokens: int = 2048, device=None,
                 seed: int = 0, row_invariant: bool = False):
        dev = torch.device(device if device is not None else "cuda")
        self.L, self.hidden, self.Hq, self.Hkv, self.D = num_layers, hidden, num_heads, num_kv_heads, head_dim
        self.eps, self.device = eps, dev
        g = torch.Generator(device=dev).manual_seed(seed)

        def lin(out_f, in_f):
            return (torch.randn(out_f, in_f, device=dev, generator=g) * in_f ** -0.5).to(torch.bfloat16)

        def norm_w(n):
            return (1 + 0.1 * torch.randn(n, device=dev, generator=g)).to(torch.bfloat16)

        qkv_out = (num_heads + 2 * num_kv_heads) * head_dim
        self.layers = [dict(in_norm=norm_w(hidden), qkv=lin(qkv_out, hidden), q_norm=norm_w(head_dim),
                            k_norm=norm_w(head_dim), o=lin(hidden, num_heads * head_dim), post_norm=norm_w(hidden),
                            gate_up=lin(2 * intermediate, hidden), down=lin(hidden, intermediate))
                       for _ in range(num_layers)]
        self.embed = torch.randn(vocab, hidden, device=dev, generator=g).to(torch.bfloat16)
        self.final_norm = norm_w(hidden)
        self.lm_head = lin(vocab, hidden)
        self.cos_sin = RotaryEmbedding(head_dim, head_dim, max_position, rope_theta).cos_sin_cache.to(dev)
        self.row_invariant = row_invariant
        if row_invariant:   # the projections' weights packed once into the row-invariant GEMM's layout
            for w in self.layers:
                w.update({f"{name}_lin": RowInvariantLinear(w[name]) for name in ("qkv", "o", "gate_up", "down")})
        self.input_ids = torch.zeros(max_tokens, dtype=torch.int64, device=dev)
        self.residual = torch.zeros(max_tokens, hidden, dtype=torch.bfloat16, device=dev)
        self.hidden_out = torch.zeros(max_tokens, hidden, dtype=torch.bfloat16, device=dev)

    def pre_attn(self):
        """MixedStepRunner's pre_attn argument: (cos_sin_cache, per-layer (q_norm, k_norm), eps)."""
        return self.cos_sin, [(w["q_norm"], w["k_norm"]) for w in self.layers], self.eps

    def _linear(self, x: torch.Tensor, w: dict, name: str, out: torch.Tensor | None = None) -> torch.Tensor:
        if self.row_invariant:
            return w[f"{name}_lin"](x, out=out)
        if out is None:
            return F.linear(x, w[name])
        return torch.mm(x, w[name].t(), out=out)

    def _norm(self, x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor | None = None):
        if self.row_invariant:
            return layernorm.rms_norm(x, weight, self.eps, residual)
        return rms_norm(x, weight, self.eps) if residual is None else add_rms_norm(x, residual, weight, self.eps)

    def _post_attn(self, w: dict, o: torch.Tensor, residual: torch.Tensor):
        """Qwen3DecoderLayer.post_attn (qwen3.py:192-201)."""
        h = self._linear(o, w, "o")
        h, residual = self._norm(h, w["post_norm"], residual)
        gate, up = self._linear(h, w, "gate_up").chunk(2, -1)
        return self._linear(F.silu(gate) * up, w, "down"), residual

    def __call__(self, i: int, n: int, bufs: dict) -> None:
        if i == 0:
            h = F.embedding(self.input_ids[:n], self.embed)
            x, residual = self._norm(h, self.layers[0]["in_norm"]), h
        else:
            h, residual = self._post_attn(self.layers[i - 1], bufs["o"][:n].view(n, -1), self.residual[:n])
            if i == self.L:
                self.hidden_out[:n] = self._norm(h, self.final_norm, residual)[0]
                return
            x, residual = self._norm(h, self.layers[i]["in_norm"], residual)
        self.residual[:n] = residual
        self._linear(x, self.layers[i], "qkv", out=bufs["qkv"][:n])
