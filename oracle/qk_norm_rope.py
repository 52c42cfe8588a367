"""Oracle for the per-token work in front of attention: q/k RMSNorm, rotary embedding and the KV store.
Test infrastructure only.

Restates, on the CPU with the reference's eager PyTorch operations (fp32 math, the same bf16 roundings):

* rope_cache        nanovllm/layers/rotary_embedding.py:28-34 (RotaryEmbedding.__init__: inv_freq,
                    freqs = t x inv_freq, cache = cat(cos, sin))
* rms_norm          nanovllm/layers/layernorm.py:16-26 (RMSNorm.rms_forward: fp32 mean of squares,
                    x * rsqrt(var + eps), cast to the input dtype, then times the bf16 weight)
* add_rms_norm      nanovllm/layers/layernorm.py:28-38 (RMSNorm.add_rms_forward: x + residual in fp32, the sum
                    rounded as the new residual, the fp32 sum normalised as rms_norm does)
* apply_rotary      nanovllm/layers/rotary_embedding.py:6-14 (neox halves: y1 = x1 cos - x2 sin,
                    y2 = x2 cos + x1 sin, fp32, cast back) and :37-48 (cos / sin rows picked by position)
* qk_norm_rope_store nanovllm/models/qwen3.py:83-97 (pre_attn: split, q_norm / k_norm unless the model has
                    a qkv bias, rotary_emb) followed by the KV store of nanovllm/layers/attention.py:33-40
                    as Attention.forward calls it (:62-63)

The reference runs rms_forward and the rotary forward under torch.compile; this oracle follows the
eager meaning of the same code (one rounding to bf16 after the normalisation, one after the weight,
one after the rotation). How each function is pinned is listed in tests/test_oracle.py.
"""
import torch

from oracle import kvcache as okv


def rope_cache(head_size: int, max_position: int, base: float) -> torch.Tensor:
    """[max_position, head_size] fp32: cos(p * inv_freq_j) for j < head_size/2, then sin(...)
    (rotary_embedding.py:28-34; the reference keeps a [max_position, 1, head_size] buffer)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float) / head_size))
    t = torch.arange(max_position, dtype=torch.float)
    freqs = t[:, None] * inv_freq[None, :]
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim with the reference's roundings (layernorm.py:16-26)."""
    orig = x.dtype
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return xf.to(orig) * weight


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """(normalised x + residual, x + residual rounded) with the reference's roundings (layernorm.py:28-38)."""
    orig = x.dtype
    xf = x.float() + residual.float()
    res = xf.to(orig)
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return xf.to(orig) * weight, res


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Neox-style rotation of the two halves of the last dim (rotary_embedding.py:6-14)."""
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(x.dtype)


def rotary(positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor, cos_sin: torch.Tensor):
    """RotaryEmbedding.forward (rotary_embedding.py:37-48): q [N, Hq, D], k [N, Hkv, D], cos_sin
    [max_position, D]."""
    cs = cos_sin[positions.long()].unsqueeze(1)
    cos, sin = cs.chunk(2, dim=-1)
    return apply_rotary(q, cos, sin), apply_rotary(k, cos, sin)


def qk_norm_rope_store(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
                       q_weight: torch.Tensor | None, k_weight: torch.Tensor | None, eps: float,
                       cos_sin: torch.Tensor, k_cache: torch.Tensor | None = None,
                       v_cache: torch.Tensor | None = None, slot_mapping: torch.Tensor | None = None):
    """pre_attn after the qkv split (qwen3.py:89-97), then the store (attention.py:33-40, -1 skipped).
    q [N, Hq, D], k / v [N, Hkv, D] bf16 (views of one qkv row are fine); weights None = no norm
    (qwen3.py:93). Returns (q, k) after norm + rotation; k_cache / v_cache ([NB, bs, Hkv, D]) are
    updated in place when given."""
    if q_weight is not None:
        q = rms_norm(q, q_weight, eps)
        k = rms_norm(k, k_weight, eps)
    q, k = rotary(positions, q, k, cos_sin)
    if k_cache is not None:
        okv.store_kvcache(k, v, k_cache, v_cache, slot_mapping)
    return q, k
