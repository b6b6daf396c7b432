"""``QuantLinear``: the module that takes the place of a quantized ``nn.Linear``.

In the reference, ``quantize_model`` writes ``W_hat = q.float() * scale`` back
into an ordinary fp32 ``nn.Linear`` (``quantization.py:193-197``) and every
forward pass runs fp32 ``F.linear`` over it (``model.py:254,319,352,355``).
Here the module keeps the integer codes themselves (int8, or the reference's
two-nibbles-per-byte layout for <= 4 bits, or the group-wise int4 layout) and
its forward pass calls the HIP kernels of ``libtiq_hip.so``, which read the
codes from HBM and dequantize them in registers.

The call contract of the slot is unchanged: ``module(x)`` with ``x`` of shape
``(..., in_features)`` returns ``(..., out_features)``. fp32 activations give an
fp32 result accumulated in fp32 (the decode path used for greedy parity);
bf16 activations give a bf16 result (fp32 accumulation), the W8A16 path.
``weight`` returns the dequantized ``W_hat`` the reference would hold.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib

FMT_W8, FMT_W4, FMT_W4G = "int8", "int4", "int4_groupwise"


class QuantLinear(nn.Module):
    """A Linear whose weight lives as integer codes plus scales.

    Args:
        codes: ``(N, K)`` int8 codes (``fmt='int8'``), the reference nibble
            layout ``(N * K / 2,)`` uint8 (``fmt='int4'``), or ``(N, ceil(K/2))``
            uint8 group-wise nibbles (``fmt='int4_groupwise'``).
        scale: ``(N,)`` fp32 per-row scales (``int8``/``int4``) or
            ``(N, ceil(K/group))`` fp16 group scales.
        bias: ``(N,)`` fp32 or ``None``.
        in_features / out_features: ``K`` / ``N``.
        bits, granularity: recorded for ``extra_repr`` and the stats.
        group_size: group width of the group-wise format.
    """

    def __init__(
        self,
        codes: torch.Tensor,
        scale: torch.Tensor,
        bias: torch.Tensor | None,
        in_features: int,
        out_features: int,
        bits: int,
        granularity: str,
        fmt: str,
        group_size: int = 0,
    ) -> None:
        super().__init__()
        _lib.require_gpu(codes, "codes")
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.bits = int(bits)
        self.granularity = granularity
        self.fmt = fmt
        self.group_size = int(group_size)
        self.register_buffer("codes", codes.contiguous())
        self.register_buffer("scale", scale.contiguous())
        if bias is not None:
            self.bias = nn.Parameter(bias.detach().to(torch.float32).contiguous(), requires_grad=False)
        else:
            self.register_parameter("bias", None)

    # --------------------------------------------------------------- forward
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _lib.require_gpu(x, "input")
        K, N = self.in_features, self.out_features
        if x.shape[-1] != K:
            raise ValueError(f"expected last dimension {K}, got {tuple(x.shape)}")
        if x.dtype not in (torch.float32, torch.bfloat16):
            x = x.float()
        lead = x.shape[:-1]
        x2 = x.reshape(-1, K)
        if x2.stride(-1) != 1 or (x2.size(0) > 1 and x2.stride(0) != K):
            x2 = x2.contiguous()
        M = x2.size(0)
        y = torch.empty((M, N), dtype=x.dtype, device=x.device)
        if M:
            linear_into(self, x2, y)
        return y.reshape(*lead, N)

    def forward_gelu_in(self, x: torch.Tensor) -> torch.Tensor | None:
        """``self(gelu_tanh(x))`` for fp32 GPU rows of a prefill (at least 128
        rows, ``K % 64 == 0``, no gradient wanted), the activation applied
        while the library splits ``x`` into the matrix cores' bf16 planes
        (``tiq_linear_gelu_in_ws``): bit for bit ``self(gelu_tanh(x))``
        without the activation's own pass. None where that entry point does
        not apply; the caller then takes the two steps."""
        K, N = self.in_features, self.out_features
        if (not x.is_cuda or x.dtype != torch.float32 or x.shape[-1] != K or K % 64
                or (torch.is_grad_enabled() and x.requires_grad)):
            return None
        lead = x.shape[:-1]
        x2 = x.reshape(-1, K)
        M = x2.size(0)
        if M < 128:
            return None
        if x2.stride(-1) != 1 or x2.stride(0) != K or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        L = _lib.lib()
        y = torch.empty((M, N), dtype=torch.float32, device=x.device)
        ws_bytes = int(L.tiq_gemm_w8_workspace(_lib.dtype_code(torch.float32), M, K, N))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        wf = {FMT_W8: _lib.WF_INT8, FMT_W4: _lib.WF_INT4}.get(self.fmt, _lib.WF_INT4G)
        s32 = None if self.fmt == FMT_W4G else self.scale.data_ptr()
        s16 = self.scale.data_ptr() if self.fmt == FMT_W4G else None
        rc = L.tiq_linear_gelu_in_ws(x2.data_ptr(), M, K, K, self.codes.data_ptr(), wf, s32, s16, self.group_size,
                                     _lib.ptr(self.bias), N, y.data_ptr(), N, ws.data_ptr(), ws_bytes,
                                     _lib.stream_of(x2))
        if rc == _lib.EUNSUPPORTED:
            return None
        _lib.check(rc, f"quantized linear over gelu_tanh ({self.fmt}, M={M}, K={K}, N={N})")
        return y.reshape(*lead, N)

    @property
    def weight(self) -> torch.Tensor:
        """The dequantized ``W_hat`` (fp32, ``(N, K)``), as the reference stores it."""
        return dequantize(self)

    def extra_repr(self) -> str:
        g = f", group_size={self.group_size}" if self.fmt == FMT_W4G else ""
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, bits={self.bits}, "
            f"granularity={self.granularity}, format={self.fmt}{g}, bias={self.bias is not None}"
        )


def linear_into(m: QuantLinear, x2: torch.Tensor, y: torch.Tensor) -> None:
    """``y = x2 @ W_hat^T + b`` into a preallocated ``(M, N)`` tensor."""
    L = _lib.lib()
    M, K = x2.shape
    N = m.out_features
    xd, yd = _lib.dtype_code(x2.dtype), _lib.dtype_code(y.dtype)
    st = _lib.stream_of(x2)
    b = _lib.ptr(m.bias)
    if m.fmt == FMT_W8:
        # fp32 activations over many rows (a prefill) take the matrix cores as
        # three exact bf16 planes, and a product with few output tiles is split
        # over K; the library sizes the workspace (0: none)
        ws_bytes = max(int(L.tiq_linear_w8_workspace(xd, M, K)), int(L.tiq_gemm_w8_workspace(xd, M, K, N)))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x2.device) if ws_bytes else None
        rc = L.tiq_linear_w8_ws(x2.data_ptr(), xd, M, K, x2.stride(0), m.codes.data_ptr(), m.scale.data_ptr(), b, N,
                                y.data_ptr(), yd, y.stride(0), None if ws is None else ws.data_ptr(), ws_bytes, st)
    else:
        # int4 formats: fp32 activations over many rows take the matrix cores
        # through the same three exact bf16 planes; with bf16 rows a product
        # with few output tiles splits over K (workspace 0: none)
        ws_bytes = max(int(L.tiq_linear_w8_workspace(xd, M, K)), int(L.tiq_gemm_w8_workspace(xd, M, K, N)))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x2.device) if ws_bytes else None
        wp = None if ws is None else ws.data_ptr()
        if m.fmt == FMT_W4:
            rc = L.tiq_linear_w4_ws(x2.data_ptr(), xd, M, K, x2.stride(0), m.codes.data_ptr(), m.scale.data_ptr(), b,
                                    N, y.data_ptr(), yd, y.stride(0), wp, ws_bytes, st)
        else:
            rc = L.tiq_linear_w4g_ws(x2.data_ptr(), xd, M, K, x2.stride(0), m.codes.data_ptr(), m.scale.data_ptr(),
                                     m.group_size, b, N, y.data_ptr(), yd, y.stride(0), wp, ws_bytes, st)
    _lib.check(rc, f"quantized linear ({m.fmt}, M={M}, K={K}, N={N})")


def dequantize(m: QuantLinear) -> torch.Tensor:
    L = _lib.lib()
    N, K = m.out_features, m.in_features
    out = torch.empty((N, K), dtype=torch.float32, device=m.codes.device)
    st = _lib.stream_of(out)
    if m.fmt == FMT_W8:
        rc = L.tiq_dequantize_int8(m.codes.data_ptr(), m.scale.data_ptr(), 1, N, K, out.data_ptr(), st)
    elif m.fmt == FMT_W4:
        rc = L.tiq_dequantize_int4(m.codes.data_ptr(), m.scale.data_ptr(), 1, N, K, out.data_ptr(), st)
    else:
        rc = L.tiq_dequantize_groupwise_int4(m.codes.data_ptr(), m.scale.data_ptr(), m.group_size, N, K,
                                             out.data_ptr(), st)
    _lib.check(rc, "dequantize")
    return out
