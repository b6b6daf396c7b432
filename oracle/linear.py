"""Dequantize-then-fp32-matmul: the reference's runtime arithmetic for a
quantized Linear.

TEST INFRASTRUCTURE ONLY (checker and timed CPU baseline).

The reference writes ``W_hat = (q.float() * scale)`` into an ``nn.Linear``
(``quantization.py:193-197``) and the forward pass is then the plain fp32
``F.linear`` at ``model.py:254,319,352,355``. :func:`linear_ref` is exactly
that, on CPU tensors. Parity of a GPU linear against it is judged with the
tolerance ``max|y - y_ref| <= 1e-3 * max|y_ref|``.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def dequantize(q, scale) -> torch.Tensor:
    """``q.float() * scale`` (``quantization.py:129,197``)."""
    q = torch.as_tensor(np.asarray(q)) if not isinstance(q, torch.Tensor) else q
    s = torch.as_tensor(np.asarray(scale)) if not isinstance(scale, torch.Tensor) else scale
    return q.to(torch.float32) * s.to(torch.float32)


def linear_ref(x: torch.Tensor, w_hat: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x.float(), W_hat, b)`` in fp32 on the CPU."""
    b = None if bias is None else bias.float().cpu()
    return F.linear(x.float().cpu(), w_hat.float().cpu(), b)


def within_tolerance(y: torch.Tensor, y_ref: torch.Tensor, rel: float = 1e-3) -> tuple[bool, float, float]:
    """The output contract: ``max|y - y_ref| <= rel * max|y_ref|``.

    Returns ``(ok, max_abs_err, bound)``.
    """
    y = y.float().cpu()
    y_ref = y_ref.float().cpu()
    err = float((y - y_ref).abs().max()) if y.numel() else 0.0
    bound = rel * float(y_ref.abs().max()) if y.numel() else 0.0
    return err <= bound, err, bound
