"""Row-invariant linear layer (HIP sd_linear): y = x @ W^T in bf16 with fp32 accumulation, as F.linear computes
the reference's projections (nanovllm/layers/linear.py; qkv_proj / o_proj / gate_up_proj / down_proj of
nanovllm/models/qwen3.py:47-63,115-126), with each output row a function of its input row alone.

The library GEMM picks its kernel, and with it the summation order, by the row count (on MI355X the o_proj
shape gives three different results for one row across 1..2048 rows). A decode step of B sequences and a
verify step of B(1+k) rows then compute different hidden states for the same token, and greedy speculative
decoding can pick other tokens than plain decoding. This layer runs the LM head's GEMM (the weight packed once
into its tile layout) without the argmax epilogue, so a row's result never depends on the batch.
"""
import torch

from nanovllm_amd import _lib
from nanovllm_amd.layers.lm_head import pack_weight


class RowInvariantLinear:
    """y = x @ weight^T for weight [out_features, in_features] bf16 (packed once; it must not change after)."""

    def __init__(self, weight: torch.Tensor):
        self.out_features, self.in_features = weight.shape
        if self.in_features % 32:
            raise ValueError("RowInvariantLinear: in_features must be a multiple of 32")
        self.packed = pack_weight(weight)

    def __call__(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        if x.dtype != torch.bfloat16 or x.dim() != 2 or x.size(1) != self.in_features or x.stride(1) != 1:
            raise ValueError("RowInvariantLinear: bf16 [rows, in_features] with unit column stride required")
        M = x.size(0)
        if out is None:
            out = torch.empty(M, self.out_features, dtype=torch.bfloat16, device=x.device)
        if out.dtype != torch.bfloat16 or out.shape != (M, self.out_features) or out.stride(1) != 1:
            raise ValueError("RowInvariantLinear: out must be bf16 [rows, out_features] with unit column stride")
        if M == 0:
            return out
        lib = _lib.load()
        ws = _lib.workspace(lib.sd_linear_workspace_size(M, self.out_features, self.in_features), x.device)
        _lib.check(lib.sd_linear(x.data_ptr(), x.stride(0), M, self.packed.data_ptr(), self.out_features,
                                 self.in_features, out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(),
                                 _lib.stream_of(x.device)), "sd_linear")
        return out
