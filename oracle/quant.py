"""numpy restatement of the reference's quantize / pack arithmetic, plus a
loader for the C restatement in ``quant_oracle.c``.

TEST INFRASTRUCTURE ONLY: tests, the smoke check and the CPU-baseline leg of
the benchmark import this module as the checker. The shipped library never
does.

Each function follows ``src/transformer_internals/quantization.py`` of the
reference, line by line in meaning:

* :func:`quantize_tensor`      -- ``quantization.py:78-116``
* :func:`quantize_dequantize`  -- ``quantization.py:119-129``
* :func:`pack_int4`            -- ``quantization.py:132-149``
* :func:`unpack_int4`          -- ``quantization.py:152-158``

:func:`quantize_groupwise_int4` is the build's own group-wise int4 format
(no counterpart in the reference); its rules are written out in
``quant_oracle.c``.

Pinning: the known-answer rows in ``tests/golden/quant_known_answers.json``
(ties at exact half steps, zero / subnormal / outlier / negative-max rows,
a one-column row), the pack byte table of ``arange(-8, 8)``, and agreement of
this numpy restatement with the independent C restatement on seeded inputs.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

FLT_TINY = np.float32(np.finfo(np.float32).tiny)

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "_build" / "liboracle_quant.so"


def _check_bits(bits: int) -> tuple[int, int]:
    if bits < 2 or bits > 8:
        raise ValueError(f"bits must be in [2, 8], got {bits}")
    return 2 ** (bits - 1) - 1, -(2 ** (bits - 1))


def _amax_bits(a: np.ndarray, axis=None) -> np.ndarray:
    """``|a|.amax`` computed on the raw bits (NaN-propagating like torch)."""
    u = a.astype(np.float32, copy=False).view(np.uint32) & np.uint32(0x7FFFFFFF)
    return u.max(axis=axis, keepdims=axis is not None).view(np.float32)


def quantize_tensor(w: np.ndarray, bits: int, granularity: str = "per_channel"):
    """Return ``(q int8, scale float32)`` exactly as ``quantization.py:78-116``."""
    qmax, qmin = _check_bits(bits)
    w = np.ascontiguousarray(w, dtype=np.float32)
    if granularity == "per_channel":
        amax = _amax_bits(w, axis=1)
    elif granularity == "per_tensor":
        amax = _amax_bits(w).reshape(())
    else:
        raise ValueError(f"unknown granularity {granularity!r}")
    scale = np.maximum(amax / np.float32(qmax), FLT_TINY).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.rint(w / scale)
    q = np.clip(r, qmin, qmax).astype(np.int8)
    return q, scale


def quantize_dequantize(w: np.ndarray, bits: int, granularity: str = "per_channel"):
    q, scale = quantize_tensor(w, bits, granularity)
    return q.astype(np.float32) * scale


def pack_int4(q: np.ndarray) -> np.ndarray:
    flat = q.reshape(-1).astype(np.int16) + 8
    if flat.size % 2:
        flat = np.concatenate([flat, np.zeros(1, dtype=np.int16)])
    low, high = flat[0::2], flat[1::2]
    return ((high << 4) | low).astype(np.uint8)


def unpack_int4(packed: np.ndarray, numel: int) -> np.ndarray:
    p = packed.reshape(-1).astype(np.int16)
    low = (p & 0x0F) - 8
    high = ((p >> 4) & 0x0F) - 8
    return np.stack([low, high], axis=1).reshape(-1)[:numel].astype(np.int8)


def quantize_groupwise_int4(w: np.ndarray, group: int = 128):
    """Group-wise int4 codes + fp16 scales (the build's own format).

    Returns ``(packed uint8 (rows, ceil(cols/2)), scale float16 (rows, ngroups),
    codes int8 (rows, cols))``.
    """
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    ngroups = -(-cols // group)
    pad = ngroups * group - cols
    wp = np.pad(w, ((0, 0), (0, pad))) if pad else w
    g = wp.reshape(rows, ngroups, group)
    amax = _amax_bits(g, axis=2)[..., 0]
    with np.errstate(over="ignore"):
        s16 = (amax / np.float32(7)).astype(np.float16)  # numpy casts with RNE
    bits16 = s16.view(np.uint16).copy()
    bits16[bits16 == 0] = 1
    bits16[bits16 > 0x7BFF] = 0x7BFF
    s16 = bits16.view(np.float16)
    s32 = s16.astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.rint(g / s32[..., None])
    codes = np.clip(r, -8, 7).astype(np.int8).reshape(rows, ngroups * group)[:, :cols]
    biased = codes.astype(np.int16) + 8
    if cols % 2:
        biased = np.concatenate([biased, np.zeros((rows, 1), np.int16)], axis=1)
    packed = ((biased[:, 1::2] << 4) | biased[:, 0::2]).astype(np.uint8)
    return packed, s16, codes


def dequantize_groupwise_int4(packed: np.ndarray, scale16: np.ndarray, cols: int, group: int = 128):
    rows = packed.shape[0]
    lo = (packed & 0x0F).astype(np.int16) - 8
    hi = ((packed >> 4) & 0x0F).astype(np.int16) - 8
    codes = np.stack([lo, hi], axis=2).reshape(rows, -1)[:, :cols].astype(np.float32)
    s = np.repeat(scale16.astype(np.float32), group, axis=1)[:, :cols]
    return codes * s


# --------------------------------------------------------------- C oracle


class COracle:
    """ctypes binding of ``quant_oracle.c`` (built by ``oracle/Makefile``)."""

    def __init__(self, path: Path = LIB_PATH) -> None:
        if not path.exists():
            raise FileNotFoundError(f"{path} missing; run `make -C {_HERE}`")
        self.lib = ctypes.CDLL(os.fspath(path))
        i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        L = self.lib
        L.oracle_quantize_per_channel.argtypes = [vp, i64, i64, i32, vp, vp]
        L.oracle_quantize_per_tensor.argtypes = [vp, i64, i32, vp, vp]
        L.oracle_pack_int4.argtypes = [vp, i64, vp]
        L.oracle_unpack_int4.argtypes = [vp, i64, vp]
        L.oracle_quantize_groupwise_int4.argtypes = [vp, i64, i64, i32, vp, vp]
        L.oracle_f32_to_f16_rne.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16_rne.restype = ctypes.c_uint16

    @staticmethod
    def _p(a: np.ndarray) -> int:
        return a.ctypes.data

    def quantize_per_channel(self, w: np.ndarray, bits: int):
        w = np.ascontiguousarray(w, dtype=np.float32)
        rows, cols = w.shape
        q = np.empty((rows, cols), np.int8)
        s = np.empty((rows, 1), np.float32)
        if self.lib.oracle_quantize_per_channel(self._p(w), rows, cols, bits, self._p(q), self._p(s)):
            raise ValueError(f"bits must be in [2, 8], got {bits}")
        return q, s

    def quantize_per_tensor(self, w: np.ndarray, bits: int):
        w = np.ascontiguousarray(w, dtype=np.float32)
        q = np.empty(w.shape, np.int8)
        s = np.empty((), np.float32)
        if self.lib.oracle_quantize_per_tensor(self._p(w), w.size, bits, self._p(q), self._p(s)):
            raise ValueError(f"bits must be in [2, 8], got {bits}")
        return q, s

    def pack_int4(self, q: np.ndarray) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.int8)
        out = np.empty((q.size + 1) // 2, np.uint8)
        self.lib.oracle_pack_int4(self._p(q), q.size, self._p(out))
        return out

    def unpack_int4(self, packed: np.ndarray, numel: int) -> np.ndarray:
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        out = np.empty(numel, np.int8)
        self.lib.oracle_unpack_int4(self._p(packed), numel, self._p(out))
        return out

    def quantize_groupwise_int4(self, w: np.ndarray, group: int = 128):
        w = np.ascontiguousarray(w, dtype=np.float32)
        rows, cols = w.shape
        ngroups = -(-cols // group)
        packed = np.empty((rows, (cols + 1) // 2), np.uint8)
        s = np.empty((rows, ngroups), np.uint16)
        if self.lib.oracle_quantize_groupwise_int4(self._p(w), rows, cols, group, self._p(packed), self._p(s)):
            raise ValueError(f"group must be even and >= 2, got {group}")
        return packed, s.view(np.float16)

    def f32_to_f16_bits(self, x: float) -> int:
        return int(self.lib.oracle_f32_to_f16_rne(ctypes.c_float(x)))


_C_ORACLE: COracle | None = None


def c_oracle() -> COracle:
    global _C_ORACLE
    if _C_ORACLE is None:
        _C_ORACLE = COracle()
    return _C_ORACLE
