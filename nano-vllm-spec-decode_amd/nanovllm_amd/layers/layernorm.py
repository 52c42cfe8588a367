"""RMSNorm (HIP sd_rms_norm): drop-in for nanovllm/layers/layernorm.py's RMSNorm (same constructor, `weight`
parameter and forward(x, residual=None)), with each row's result independent of the number of rows (a fixed
summation order over the row; the library reductions split a short batch's rows differently)."""
import torch
from torch import nn

from nanovllm_amd import _lib


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
             out: torch.Tensor | None = None, residual_out: torch.Tensor | None = None):
    """rms_forward(x) (layernorm.py:16-26), or add_rms_forward(x, residual) -> (out, new residual)
    (layernorm.py:28-38). x / residual bf16 [rows, hidden] with unit column stride."""
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("rms_norm: bf16 [rows, hidden] with unit column stride required")
    M, H = x.shape
    if weight.dtype != torch.bfloat16 or weight.shape != (H,) or not weight.is_contiguous():
        raise ValueError("rms_norm: contiguous bf16 weight [hidden] required")
    if out is None:
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    if residual is not None:
        if residual.dtype != torch.bfloat16 or residual.shape != (M, H) or residual.stride(1) != 1:
            raise ValueError("rms_norm: residual must be bf16 [rows, hidden] with unit column stride")
        if residual_out is None:
            residual_out = torch.empty_like(residual, memory_format=torch.contiguous_format)
    lib = _lib.load()
    _lib.check(lib.sd_rms_norm(x.data_ptr(), x.stride(0), _lib.ptr(residual),
                               residual.stride(0) if residual is not None else 0, weight.data_ptr(), float(eps), M, H,
                               out.data_ptr(), out.stride(0), _lib.ptr(residual_out),
                               residual_out.stride(0) if residual_out is not None else 0, _lib.stream_of(x.device)),
               "sd_rms_norm")
    return out if residual is None else (out, residual_out)


class RMSNorm(nn.Module):
    """nanovllm.layers.layernorm.RMSNorm (layernorm.py:5-49) over bf16 rows."""

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, dtype=torch.bfloat16))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if residual is None:
            return rms_norm(x2, self.weight.data, self.eps).view(shape)
        out, res = rms_norm(x2, self.weight.data, self.eps, residual.reshape(-1, shape[-1]))
        return out.view(shape), res.view(shape)
