"""ctypes binding of ``libtiq_hip.so`` (the C ABI declared in ``include/tiq.h``).

Every call passes raw device pointers of torch tensors and the current HIP
stream; torch's caching allocator owns all memory. A non-zero status raises
``RuntimeError`` naming the entry point. There is no CPU fallback: if the
library is missing or no ROCm GPU is visible, :func:`lib` raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_NAME = "libtiq_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

F32, BF16 = 0, 1

_i64, _i32, _vp, _sz, _f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float

#: (name, argtypes, restype) of every exported symbol
SIGNATURES: dict[str, tuple[list, object]] = {
    "tiq_version": ([], _i32),
    "tiq_stamp_begin": ([_vp, _i64], _i32),
    "tiq_stamp_end": ([_vp, _vp, _i64], _i64),
    "tiq_status_string": ([_i32], ctypes.c_char_p),
    "tiq_quantize_per_channel": ([_vp, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _vp], _i32),
    "tiq_quantize_per_tensor_workspace": ([_i64], _sz),
    "tiq_quantize_per_tensor": ([_vp, _i64, _i32, _vp, _vp, _vp, _sz, _vp], _i32),
    "tiq_pack_int4": ([_vp, _i64, _vp, _vp], _i32),
    "tiq_unpack_int4": ([_vp, _i64, _vp, _vp], _i32),
    "tiq_quantize_per_channel_int4_packed": ([_vp, _i64, _i64, _i32, _vp, _vp, _vp], _i32),
    "tiq_quantize_groupwise_int4": ([_vp, _i64, _i64, _i32, _vp, _vp, _vp], _i32),
    "tiq_dequantize_int8": ([_vp, _vp, _i32, _i64, _i64, _vp, _vp], _i32),
    "tiq_dequantize_int4": ([_vp, _vp, _i32, _i64, _i64, _vp, _vp], _i32),
    "tiq_dequantize_groupwise_int4": ([_vp, _vp, _i32, _i64, _i64, _vp, _vp], _i32),
    "tiq_linear_w8": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i64, _vp], _i32),
    "tiq_linear_w8_workspace": ([_i32, _i64, _i64], _sz),
    "tiq_linear_w8_ws": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i64, _vp, _sz, _vp], _i32),
    "tiq_gemv_w8": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i64, _vp], _i32),
    "tiq_gemm_w8": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i64, _vp], _i32),
    "tiq_gemm_w8_tile": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i64, _i32, _vp], _i32),
    "tiq_linear_w4": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i64, _vp], _i32),
    "tiq_linear_w4g": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _i64, _vp, _i32, _i64, _vp], _i32),
    "tiq_linear_w4_ws": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i64, _vp, _sz, _vp], _i32),
    "tiq_linear_w4g_ws": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _i64, _vp, _i32, _i64, _vp, _sz, _vp],
                          _i32),
    "tiq_linear_fused": ([_vp, _i32, _i64, _i64, _i64, _vp, _i32, _vp, _vp, _i32, _vp, _i64, _vp, _i32, _i64,
                          _vp, _vp, ctypes.c_float, _i32, _vp, _i64, _vp], _i32),
    "tiq_gemm_w8_workspace": ([_i32, _i64, _i64, _i64], _sz),
    "tiq_gemm_w8_ws": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i64, _vp, _sz, _vp], _i32),
    "tiq_decode_linear_workspace": ([_i32, _i64, _i64, _i64], _sz),
    "tiq_decode_planes_bytes": ([_i64, _i64], _sz),
    "tiq_tile_int8": ([_vp, _i64, _i64, _i64, _vp, _vp], _i32),
    "tiq_tile_f32_bytes": ([_i64, _i64], _sz),
    "tiq_tile_f32": ([_vp, _i64, _i64, _i64, _vp, _vp], _i32),
    "tiq_decode_linear": ([_vp, _i64, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _f32, _i32,
                           _vp, _i64, _vp, _vp, _f32, _vp, _vp, _sz, _vp], _i32),
    "tiq_decode_linear_noalloc": ([_vp, _i64, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _f32,
                                   _i32, _vp, _i64, _vp, _vp, _f32, _vp, _vp], _i32),
    "tiq_linear_fused_workspace": ([_i32, _i32, _i64, _i64, _i64], _sz),
    "tiq_linear_fused_ws": ([_vp, _i32, _i64, _i64, _i64, _vp, _i32, _vp, _vp, _i32, _vp, _i64, _vp, _i32, _i64,
                             _vp, _vp, ctypes.c_float, _i32, _vp, _i64, _vp, _sz, _vp], _i32),
    "tiq_decode_attention": ([_vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp], _i32),
    "tiq_decode_attention_planes": ([_vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp], _i32),
    "tiq_decode_qkv_attention_workspace": ([_i64, _i64, _i64], _sz),
    "tiq_decode_qkv_attention": ([_vp, _i64, _i64, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp,
                                  _i64, _vp, _vp, _sz, _vp], _i32),
    "tiq_embed_tokens": ([_vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp], _i32),
    "tiq_gelu_tanh": ([_vp, _vp, _i64, _vp], _i32),
    "tiq_linear_gelu_in_ws": ([_vp, _i64, _i64, _i64, _vp, _i32, _vp, _vp, _i32, _vp, _i64, _vp, _i64, _vp, _sz, _vp],
                              _i32),
    "tiq_prefill_attention": ([_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                               _i64, _i64, _vp, _i64, _i64, _i64, _vp], _i32),
    "tiq_argmax_rows_workspace": ([_i64], _sz),
    "tiq_argmax_rows": ([_vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _sz, _vp], _i32),
    "tiq_head_screen_workspace": ([_i64], _sz),
    "tiq_head_screen_prepare": ([_vp, _i64, _i64, _i64, _vp, _vp, _vp], _i32),
    "tiq_head_argmax_screened": ([_vp, _i64, _vp, _vp, _f32, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp,
                                  _vp, _sz, _vp], _i32),
    "tiq_head_screen_prepare_i8": ([_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp], _i32),
    "tiq_head_argmax_screened_i8": ([_vp, _i64, _vp, _vp, _f32, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64,
                                     _vp, _vp, _sz, _vp], _i32),
}

WF_INT8, WF_INT4, WF_INT4G, WF_F32, WF_INT8_TILED, WF_F32_TILED = 0, 1, 2, 3, 4, 5
ACT_NONE, ACT_GELU_TANH = 0, 1
#: status codes of tiq.h
OK, EINVAL, EBITS, EALIGN, EUNSUPPORTED, EWORKSPACE, ESCRATCH = 0, -1, -2, -3, -4, -5, -6

_LIB: ctypes.CDLL | None = None


class LibraryUnavailable(RuntimeError):
    """The HIP library is not built, or no ROCm GPU is visible."""


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load the shared library and declare its signatures (no GPU needed)."""
    p = Path(path) if path is not None else Path(os.environ.get("TIQ_LIB", LIB_PATH))
    if not p.exists():
        raise LibraryUnavailable(
            f"{p} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            f"or `make -C gpt2-harness_amd/csrc`"
        )
    lib = ctypes.CDLL(os.fspath(p))
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


def lib() -> ctypes.CDLL:
    """The loaded library; raises :class:`LibraryUnavailable` without a GPU."""
    global _LIB
    if _LIB is None:
        if not torch.cuda.is_available():
            raise LibraryUnavailable("gpt2_harness_amd needs a ROCm GPU; none is visible")
        _LIB = load()
    return _LIB


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().tiq_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{name} is on {t.device}; gpt2_harness_amd runs its kernels on the ROCm GPU "
            f"(move it with .to('cuda'))"
        )


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise TypeError(f"activations must be float32 or bfloat16, got {dt}")
