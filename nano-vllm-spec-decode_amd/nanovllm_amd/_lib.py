"""ctypes binding of libsd_attn.so, the gfx950 HIP extension (C ABI declared in include/sd_attn.h).

torch is imported first so that the HIP runtime it ships (SONAME libamdhip64.so.7) is the one the
extension binds to: streams and device pointers handed over from torch are then valid in the extension.
There is no fallback: if the library is missing, every op raises.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SD_ATTN_LIB", os.path.join(_HERE, "libsd_attn.so"))

DTYPE_BF16 = 0
DTYPE_F32 = 1

_c_void_p, _i32, _i64, _f32, _size = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/sd_attn.h
SIGNATURES = {
    "sd_abi_version": (_i32, []),
    "sd_last_error": (ctypes.c_char_p, []),
    "sd_store_kvcache": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _i32, _i32,
                                _i32, _c_void_p]),
    "sd_qk_norm_rope_store": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p,
                                     _c_void_p, _f32, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _c_void_p,
                                     _c_void_p, _i64, _c_void_p, _i32, _i32, _i32, _i32, _c_void_p]),
    "sd_paged_decode_workspace_size": (_size, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "sd_paged_decode": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32, _i32,
                               _i32, _i32, _i32, _i32, _f32, _c_void_p, _i64, _c_void_p, _size, _c_void_p]),
    "sd_paged_decode_plan": (_i32, [_c_void_p, _i32, _i32, _i32, _i32, _c_void_p, _size, _c_void_p]),
    "sd_paged_decode_planned": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32,
                                       _i32, _i32, _i32, _i32, _i32, _f32, _c_void_p, _i64, _c_void_p, _size,
                                       _c_void_p]),
    "sd_varlen_workspace_size": (_size, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "sd_varlen_attention": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _i32, _c_void_p,
                                   _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                                   _c_void_p, _i64, _c_void_p, _size, _c_void_p]),
    "sd_varlen_plan": (_i32, [_c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32, _c_void_p, _size, _c_void_p]),
    "sd_varlen_attention_planned": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _i32,
                                           _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32, _i32,
                                           _i32, _f32, _c_void_p, _i64, _c_void_p, _size, _c_void_p]),
    "sd_verify_workspace_size": (_size, [_i32, _i32, _i32, _i32]),
    "sd_verify_drafts": (_i32, [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64,
                                _c_void_p, _c_void_p, _i32, _i32, _i32, _c_void_p, _c_void_p, _c_void_p, _size,
                                _c_void_p]),
    "sd_lm_head_packed_weight_size": (_size, [_i32, _i32]),
    "sd_lm_head_pack_weight": (_i32, [_c_void_p, _i32, _i32, _c_void_p, _c_void_p]),
    "sd_lm_head_verify_workspace_size": (_size, [_i32, _i32, _i32, _i32, _i32]),
    "sd_lm_head_verify": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32, _i32, _c_void_p, _c_void_p,
                                 _c_void_p, _c_void_p, _i32, _i64, _c_void_p, _c_void_p, _i32, _i32, _c_void_p, _i64,
                                 _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "sd_verify_drafts_noalloc": (_i32, [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32,
                                        _i64, _c_void_p, _c_void_p, _i32, _i32, _i32, _c_void_p, _c_void_p,
                                        _c_void_p]),
    "sd_draft_step_inputs": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i32, _i32, _c_void_p, _i32, _i32, _i32,
                                    _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "sd_linear_workspace_size": (_size, [_i32, _i32, _i32]),
    "sd_linear": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _i32, _i32, _c_void_p, _i64, _c_void_p, _size, _c_void_p]),
    "sd_rms_norm": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _f32, _i32, _i32, _c_void_p, _i64, _c_void_p,
                           _i64, _c_void_p]),
    "sd_sample": (_i32, [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _i32, _i32, _c_void_p, _c_void_p, _size,
                         _c_void_p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """The loaded extension; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP extension not built: {LIB_PATH} is missing "
                               "(run `python nano-vllm-spec-decode_amd/build_ext.py`)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().sd_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_workspaces: dict[tuple[torch.device, str], list[torch.Tensor]] = {}


def workspace(nbytes: int, device: torch.device, tag: str = "") -> torch.Tensor:
    """A scratch buffer of at least nbytes on `device`, shared by consecutive launches on the current stream
    (one buffer per `tag`). Grows by allocating a bigger buffer; older buffers are kept alive because
    captured graphs may still point at them."""
    bufs = _workspaces.setdefault((device, tag), [])
    if not bufs or bufs[-1].numel() < nbytes:
        size = max(nbytes, 2 * bufs[-1].numel() if bufs else 1 << 20)
        bufs.append(torch.empty(size, dtype=torch.uint8, device=device))
    return bufs[-1]
