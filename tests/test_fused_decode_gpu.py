"""The fused decode-step kernels (C ABI) against torch fp32 computations of the
same reference ops, and the fused decoder end to end.

* ``tiq_linear_fused``: LayerNorm prologue (``model.py:413,422``), GELU(tanh)
  epilogue (``model.py:57-75``), residual add in place (``model.py:419,427``),
  fp32 weights (the tied ``lm_head``, ``model.py:585``) -- within the 1e-3
  output contract;
* ``tiq_decode_attention``: one query over the cache (``model.py:286-309`` at
  T = 1) -- within fp32 rounding of torch's softmax attention;
* ``tiq_embed_tokens`` exact; ``tiq_argmax_rows`` exact, first index on ties;
* a position outside the cache yields NaN outputs (no access out of bounds);
* greedy tokens of the fused decoder equal the reference's (GPT-2 small int8)
  and the eager path's (int4, group-wise int4).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import gpt2_harness_amd as g
from gpt2_harness_amd import _lib
from oracle import linear as OL
from oracle import model as OM

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


def _gelu(x):
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x.pow(3))))


# LayerNorm + Linear + GELU at up to 8 rows, int8 and reference-layout int4
# (the direct GEMV's one- and two-row wavefronts with the LayerNorm in
# registers at 1-4 rows; 16 columns a lane in both formats).
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("M", [1, 3, 4, 8])
@pytest.mark.parametrize("K,N", [(768, 2304), (1600, 6400), (3072, 768)])
def test_fused_ln_gelu_linear(dev, c_oracle, M, K, N, bits):
    gen = torch.Generator().manual_seed(M * 7 + K)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen) * 2 + 0.5
    lw = 1 + 0.1 * torch.randn(K, generator=gen)
    lb = 0.1 * torch.randn(K, generator=gen)
    b = 0.1 * torch.randn(N, generator=gen)
    q, s = c_oracle.quantize_per_channel(w.numpy(), bits)
    codes = q if bits == 8 else c_oracle.pack_int4(q)
    y = torch.empty(M, N, device=dev)
    # device copies stay referenced until the kernel has run
    xd, qd, sd, bd = x.to(dev), torch.from_numpy(codes).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev)
    lwd, lbd = lw.to(dev), lb.to(dev)
    wf = _lib.WF_INT8 if bits == 8 else _lib.WF_INT4
    rc = _lib.lib().tiq_linear_fused(xd.data_ptr(), 0, M, K, K, qd.data_ptr(), wf, sd.data_ptr(), None, 0,
                                     bd.data_ptr(), N, y.data_ptr(), 0, N, lwd.data_ptr(), lbd.data_ptr(), 1e-5,
                                     _lib.ACT_GELU_TANH, None, 0, _st())
    _lib.check(rc, "fused")
    ref = _gelu(OL.linear_ref(F.layer_norm(x, (K,), lw, lb, 1e-5), OL.dequantize(q, s), b))
    ok, err, bound = OL.within_tolerance(y, ref)
    assert ok, (err, bound)


# Batched decode rows (5..64) take the matrix-core kernel: activations split
# exactly into three bf16 planes, so the result is fp32-accurate -- checked
# against a float64 computation of the same ops: the kernel's error is within
# a small factor of torch fp32's own error on the same inputs.
def _f64_check(y, ref32, ref64):
    err = float((y.cpu().double() - ref64).abs().max())
    err32 = float((ref32.double() - ref64).abs().max())
    floor = 2.0 ** -24 * float(ref64.abs().max())
    assert err <= 8 * max(err32, floor), f"error {err:.3g} vs torch fp32 {err32:.3g}"


def _fused_ws(*args):
    """tiq_linear_fused_ws with a workspace of the queried size (args are
    those of tiq_linear_fused; the stream comes last)."""
    L = _lib.lib()
    M, K, w_format, N = args[2], args[3], args[6], args[11]
    n = int(L.tiq_linear_fused_workspace(args[1], w_format, M, K, N))
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
    rc = L.tiq_linear_fused_ws(*args[:-1], ws.data_ptr(), n, args[-1])
    torch.cuda.synchronize()
    return rc


@pytest.mark.parametrize("use_ws", [False, True])
@pytest.mark.parametrize("M", [5, 16, 32, 33, 64])
@pytest.mark.parametrize("K,N", [(1600, 4800), (768, 2304)])
def test_batched_ln_gelu_linear(dev, c_oracle, M, K, N, use_ws):
    gen = torch.Generator().manual_seed(M * 11 + K)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen) * 2 + 0.5
    lw = 1 + 0.1 * torch.randn(K, generator=gen)
    lb = 0.1 * torch.randn(K, generator=gen)
    b = 0.1 * torch.randn(N, generator=gen)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    y = torch.empty(M, N, device=dev)
    xd, qd, sd, bd = x.to(dev), torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev)
    lwd, lbd = lw.to(dev), lb.to(dev)
    args = (xd.data_ptr(), 0, M, K, K, qd.data_ptr(), _lib.WF_INT8, sd.data_ptr(), None, 0, bd.data_ptr(), N,
            y.data_ptr(), 0, N, lwd.data_ptr(), lbd.data_ptr(), 1e-5, _lib.ACT_GELU_TANH, None, 0, _st())
    rc = _fused_ws(*args) if use_ws else _lib.lib().tiq_linear_fused(*args)
    _lib.check(rc, "fused batched")
    torch.cuda.synchronize()
    w_hat = OL.dequantize(q, s)
    ref = _gelu(OL.linear_ref(F.layer_norm(x, (K,), lw, lb, 1e-5), w_hat, b))
    ok, err, bound = OL.within_tolerance(y, ref)
    assert ok, (err, bound)
    xn64 = F.layer_norm(x.double(), (K,), lw.double(), lb.double(), 1e-5)
    _f64_check(y, ref, _gelu(xn64 @ w_hat.double().T + b.double()))


@pytest.mark.parametrize("use_ws", [False, True])
@pytest.mark.parametrize("M", [8, 32])
@pytest.mark.parametrize("K,N", [(6400, 1600), (3072, 768)])
def test_batched_residual_in_place(dev, c_oracle, M, K, N, use_ws):
    """Long K (activations streamed through a register ring), residual
    added in place. Two calls in a row on one workspace, the second with
    fewer rows: nothing of the first call's planes reaches the second."""
    L = _lib.lib()
    gen = torch.Generator().manual_seed(M + K)
    w = torch.randn(N, K, generator=gen) * 0.02
    b = 0.1 * torch.randn(N, generator=gen)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    qd, sd, bd = torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev)
    w_hat = OL.dequantize(q, s)
    n_ws = int(L.tiq_linear_fused_workspace(0, _lib.WF_INT8, M, K, N))
    ws = torch.empty(max(n_ws, 1), dtype=torch.uint8, device=dev)
    for rows in (M, M - 3):
        h = torch.randn(rows, K, generator=gen)
        x0 = torch.randn(rows, N, generator=gen)
        x = x0.to(dev).clone()
        hd = h.to(dev)
        args = (hd.data_ptr(), 0, rows, K, K, qd.data_ptr(), _lib.WF_INT8, sd.data_ptr(), None, 0, bd.data_ptr(), N,
                x.data_ptr(), 0, N, None, None, 1e-5, 0, x.data_ptr(), N)
        if use_ws:
            rc = L.tiq_linear_fused_ws(*args, ws.data_ptr(), n_ws, _st())
        else:
            rc = L.tiq_linear_fused(*args, _st())
        _lib.check(rc, "fused batched residual")
        torch.cuda.synchronize()
        ref = x0 + OL.linear_ref(h, w_hat, b)
        assert (x.cpu() - ref).abs().max() <= 1e-3 * ref.abs().max()
        _f64_check(x, ref, x0.double() + h.double() @ w_hat.double().T + b.double())


@pytest.mark.parametrize("M", [5, 16, 64])
@pytest.mark.parametrize("K,N,act", [(768, 3072, 1), (3072, 768, 0)])
def test_batched_bf16_rows_gelu_residual(dev, c_oracle, M, K, N, act):
    """bf16 activation rows on the matrix-core kernel with the GELU epilogue
    or the residual added in place."""
    L = _lib.lib()
    gen = torch.Generator().manual_seed(M * 5 + K)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen).to(torch.bfloat16)
    b = 0.1 * torch.randn(N, generator=gen)
    r0 = torch.randn(M, N, generator=gen)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    xd, qd, sd, bd = x.to(dev), torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev)
    y = r0.to(dev).clone()
    res = y.data_ptr() if act == 0 else None
    rc = L.tiq_linear_fused(xd.data_ptr(), 1, M, K, K, qd.data_ptr(), _lib.WF_INT8, sd.data_ptr(), None, 0,
                            bd.data_ptr(), N, y.data_ptr(), 0, N, None, None, 1e-5, act, res, N if res else 0,
                            _st())
    _lib.check(rc, "fused bf16 rows")
    torch.cuda.synchronize()
    w_hat = OL.dequantize(q, s)
    lin32 = OL.linear_ref(x, w_hat, b)
    lin64 = x.double() @ w_hat.double().T + b.double()
    if act == 1:
        ref32, ref64 = _gelu(lin32), _gelu(lin64)
    else:
        ref32, ref64 = r0 + lin32, r0.double() + lin64
    ok, err, bound = OL.within_tolerance(y, ref32)
    assert ok, (err, bound)
    _f64_check(y, ref32, ref64)


@pytest.mark.parametrize("use_ws", [False, True])
@pytest.mark.parametrize("M", [6, 32])
def test_batched_fp32_head(dev, M, use_ws):
    """fp32 weights (the tied lm_head) with LayerNorm, N not a multiple of 32."""
    K, N = 768, 5003
    gen = torch.Generator().manual_seed(M)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen)
    lw = 1 + 0.1 * torch.randn(K, generator=gen)
    lb = 0.1 * torch.randn(K, generator=gen)
    y = torch.empty(M, N, device=dev)
    xd, wd, lwd, lbd = x.to(dev), w.to(dev), lw.to(dev), lb.to(dev)
    args = (xd.data_ptr(), 0, M, K, K, wd.data_ptr(), _lib.WF_F32, None, None, 0, None, N, y.data_ptr(), 0, N,
            lwd.data_ptr(), lbd.data_ptr(), 1e-5, 0, None, 0, _st())
    rc = _fused_ws(*args) if use_ws else _lib.lib().tiq_linear_fused(*args)
    _lib.check(rc, "fused batched fp32 head")
    torch.cuda.synchronize()
    ref = F.layer_norm(x, (K,), lw, lb, 1e-5) @ w.T
    ref64 = F.layer_norm(x.double(), (K,), lw.double(), lb.double(), 1e-5) @ w.double().T
    _f64_check(y, ref, ref64)


@pytest.mark.parametrize("M", [1, 2])
def test_fused_residual_in_place_and_int4(dev, c_oracle, M):
    K, N = 3072, 768
    gen = torch.Generator().manual_seed(3)
    w = torch.randn(N, K, generator=gen) * 0.02
    h = torch.randn(M, K, generator=gen)
    x0 = torch.randn(M, N, generator=gen)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 4)
    packed = torch.from_numpy(c_oracle.pack_int4(q)).to(dev)
    x = x0.to(dev).clone()
    hd, sd = h.to(dev), torch.from_numpy(s.reshape(-1)).to(dev)
    rc = _lib.lib().tiq_linear_fused(hd.data_ptr(), 0, M, K, K, packed.data_ptr(), _lib.WF_INT4, sd.data_ptr(), None,
                                     0, None, N, x.data_ptr(), 0, N, None, None, 1e-5, 0, x.data_ptr(), N, _st())
    _lib.check(rc, "fused residual")
    ref = x0 + OL.linear_ref(h, OL.dequantize(q, s))
    assert (x.cpu() - ref).abs().max() <= 1e-3 * ref.abs().max()


# Up to 4 rows without LayerNorm take the direct GEMV (one wavefront per
# weight row, every load issued up front); rows too long for its registers
# (6400 int8 columns at 4 rows) take the LDS-staged kernel. Each weight
# format, both activation dtypes, the GELU epilogue and the in-place residual.
@pytest.mark.parametrize("fmt", ["int8", "int4", "f32"])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 3, 4])
@pytest.mark.parametrize("K,N", [(1600, 1000), (6400, 700)])
def test_direct_gemv_formats(dev, c_oracle, fmt, x_dtype, M, K, N):
    L = _lib.lib()
    gen = torch.Generator().manual_seed(M * 13 + K + len(fmt))
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen).to(x_dtype)
    b = 0.1 * torch.randn(N, generator=gen)
    r0 = torch.randn(M, N, generator=gen)
    if fmt == "f32":
        wd, sd, wf, w_hat = w.to(dev), None, _lib.WF_F32, w
    else:
        q, s = c_oracle.quantize_per_channel(w.numpy(), 8 if fmt == "int8" else 4)
        wd = torch.from_numpy(q if fmt == "int8" else c_oracle.pack_int4(q)).to(dev)
        sd = torch.from_numpy(s.reshape(-1)).to(dev)
        wf, w_hat = (_lib.WF_INT8 if fmt == "int8" else _lib.WF_INT4), OL.dequantize(q, s)
    act = 1 if K == 1600 else 0       # GELU epilogue, or the residual in place
    y = r0.to(dev).clone()
    xd, bd = x.to(dev), b.to(dev)
    res = None if act else y.data_ptr()
    rc = L.tiq_linear_fused(xd.data_ptr(), _lib.dtype_code(x_dtype), M, K, K, wd.data_ptr(), wf,
                            None if sd is None else sd.data_ptr(), None, 0, bd.data_ptr(), N, y.data_ptr(), 0, N,
                            None, None, 1e-5, act, res, 0 if act else N, _st())
    _lib.check(rc, f"direct {fmt}")
    torch.cuda.synchronize()
    lin = OL.linear_ref(x, w_hat, b)
    ref = _gelu(lin) if act else r0 + lin
    ok, err, bound = OL.within_tolerance(y, ref)
    assert ok, (err, bound)


@pytest.mark.parametrize("fmt", ["int8", "int4"])
@pytest.mark.parametrize("M,N", [(1, 50257), (1, 8203), (2, 50257)])
def test_fused_code_head_with_ln(dev, c_oracle, fmt, M, N):
    """A head of int8 / int4 codes behind its LayerNorm (non-trivial weight
    and bias): at one row over 8192 rows the direct kernel with eight weight
    rows a wavefront (50257 and 8203 leave a partial last wavefront), at two
    the LDS-staged one."""
    K = 768
    gen = torch.Generator().manual_seed(N + M)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen)
    lw, lb = 1 + 0.1 * torch.randn(K, generator=gen), 0.1 * torch.randn(K, generator=gen)
    bits = 8 if fmt == "int8" else 4
    q, s = c_oracle.quantize_per_channel(w.numpy(), bits)
    wd = torch.from_numpy(q if bits == 8 else c_oracle.pack_int4(q)).to(dev)
    wf = _lib.WF_INT8 if bits == 8 else _lib.WF_INT4
    sd = torch.from_numpy(s.reshape(-1)).to(dev)
    y = torch.empty(M, N, device=dev)
    # device copies stay referenced until the kernel has run
    xd, lwd, lbd = x.to(dev), lw.to(dev), lb.to(dev)
    rc = _lib.lib().tiq_linear_fused(xd.data_ptr(), 0, M, K, K, wd.data_ptr(), wf, sd.data_ptr(), None, 0,
                                     None, N, y.data_ptr(), 0, N, lwd.data_ptr(), lbd.data_ptr(), 1e-5, 0, None, 0,
                                     _st())
    _lib.check(rc, "code head")
    torch.cuda.synchronize()
    ref = OL.linear_ref(F.layer_norm(x, (K,), lw, lb, 1e-5), OL.dequantize(q, s))
    ok, err, bound = OL.within_tolerance(y, ref)
    assert ok, (err, bound)


@pytest.mark.parametrize("M", [1, 2])
def test_fused_f32_head_with_ln(dev, M):
    """The tied fp32 head behind its LayerNorm: at one row the direct kernel
    (four weight rows a wavefront, 50257 = 4 x 12564 + 1 leaves a partial last
    wavefront), at two the LDS-staged one."""
    K, N = 768, 50257
    gen = torch.Generator().manual_seed(4)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen)
    y = torch.empty(M, N, device=dev)
    lw, lb = torch.ones(K), torch.zeros(K)
    xd, wd, lwd, lbd = x.to(dev), w.to(dev), lw.to(dev), lb.to(dev)
    rc = _lib.lib().tiq_linear_fused(xd.data_ptr(), 0, M, K, K, wd.data_ptr(), _lib.WF_F32, None, None, 0, None, N,
                                     y.data_ptr(), 0, N, lwd.data_ptr(), lbd.data_ptr(), 1e-5, 0, None, 0, _st())
    _lib.check(rc, "head")
    ref = F.linear(F.layer_norm(x, (K,), lw, lb, 1e-5), w)
    assert (y.cpu() - ref).abs().max() <= 1e-4 * ref.abs().max()


@pytest.mark.parametrize("B,H,Hkv,pos,T", [(1, 12, 12, 0, 256), (1, 12, 12, 127, 256), (3, 25, 25, 200, 256),
                                           (2, 8, 2, 63, 256), (1, 12, 12, 127, 128), (2, 4, 4, 99, 100),
                                           (2, 4, 4, 150, 200), (1, 4, 2, 700, 1024), (1, 3, 3, 1023, 1024),
                                           (32, 25, 25, 0, 256), (32, 25, 25, 130, 256), (32, 25, 25, 255, 256),
                                           (32, 25, 25, 256, 384), (32, 25, 25, 300, 384), (32, 25, 25, 383, 384),
                                           (16, 25, 25, 100, 128)])
def test_decode_attention(dev, B, H, Hkv, pos, T):
    """Slots past 128 / 256 (histories streamed chunk by chunk), caches whose
    length is not a multiple of the 128-slot chunk, grouped kv heads. Layers
    whose keys and values pass 32 MB (batch 32 at 25 heads: 105-157 MB; batch
    16 at 128 slots: 26 MB does not) take the kernel whose reads are sized by
    the filled slots instead of the whole cache."""
    hd = 64
    gen = torch.Generator().manual_seed(pos + H)
    qkv = torch.randn(B, (H + 2 * Hkv) * hd, generator=gen)
    kc = torch.randn(B, Hkv, T, hd, generator=gen)
    vc = torch.randn(B, Hkv, T, hd, generator=gen)
    kd, vd = kc.to(dev), vc.to(dev)
    p = torch.tensor([pos], device=dev)
    y = torch.empty(B, H * hd, device=dev)
    qkvd = qkv.to(dev)
    rc = _lib.lib().tiq_decode_attention(qkvd.data_ptr(), qkv.shape[1], B, H, Hkv, hd, kd.data_ptr(),
                                         vd.data_ptr(), T, p.data_ptr(), y.data_ptr(), H * hd, _st())
    _lib.check(rc, "attention")
    q = qkv[:, : H * hd].view(B, H, 1, hd)
    knew = qkv[:, H * hd : (H + Hkv) * hd].view(B, Hkv, hd)
    vnew = qkv[:, (H + Hkv) * hd :].view(B, Hkv, hd)
    kc[:, :, pos] = knew
    vc[:, :, pos] = vnew
    K = kc[:, :, : pos + 1].repeat_interleave(H // Hkv, dim=1)
    V = vc[:, :, : pos + 1].repeat_interleave(H // Hkv, dim=1)
    ref = (F.softmax((q @ K.transpose(-2, -1)) / math.sqrt(hd), dim=-1) @ V).view(B, H * hd)
    assert (y.cpu() - ref).abs().max() < 2e-5
    assert torch.equal(kd.cpu()[:, :, pos], knew) and torch.equal(vd.cpu()[:, :, pos], vnew)
    assert torch.equal(kd.cpu()[:, :, pos + 1 :], kc[:, :, pos + 1 :])


@pytest.mark.parametrize("B,H,pos,T", [(2, 4, 5, 64), (2, 4, 130, 256), (32, 25, 40, 256), (32, 25, 200, 256)])
def test_decode_attention_ignores_memory_past_pos(dev, B, H, pos, T):
    """Cache slots past pos hold NaN (memory never written): the output is the
    attention over slots 0..pos only, for the whole-cache kernel (small caches
    read every slot) and the filled-slot one (batch 32: the first 128 slots'
    keys are requested before pos is known)."""
    hd = 64
    gen = torch.Generator().manual_seed(B * 1000 + pos)
    qkv = torch.randn(B, 3 * H * hd, generator=gen)
    kc = torch.full((B, H, T, hd), float("nan"))
    vc = torch.full((B, H, T, hd), float("nan"))
    kc[:, :, :pos] = torch.randn(B, H, pos, hd, generator=gen)
    vc[:, :, :pos] = torch.randn(B, H, pos, hd, generator=gen)
    kd, vd = kc.to(dev), vc.to(dev)
    p = torch.tensor([pos], device=dev)
    y = torch.empty(B, H * hd, device=dev)
    rc = _lib.lib().tiq_decode_attention(qkv.to(dev).data_ptr(), 3 * H * hd, B, H, H, hd, kd.data_ptr(),
                                         vd.data_ptr(), T, p.data_ptr(), y.data_ptr(), H * hd, _st())
    _lib.check(rc, "attention")
    q = qkv[:, : H * hd].view(B, H, 1, hd)
    kc[:, :, pos] = qkv[:, H * hd : 2 * H * hd].view(B, H, hd)
    vc[:, :, pos] = qkv[:, 2 * H * hd :].view(B, H, hd)
    K, V = kc[:, :, : pos + 1], vc[:, :, : pos + 1]
    ref = (F.softmax((q @ K.transpose(-2, -1)) / math.sqrt(hd), dim=-1) @ V).view(B, H * hd)
    out = y.cpu()
    assert torch.isfinite(out).all()
    assert (out - ref).abs().max() < 2e-5


@pytest.mark.parametrize("B,H,T", [(1, 2, 16), (32, 25, 256)])
def test_out_of_range_position_gives_nan_without_writes(dev, B, H, T):
    """A position outside the cache writes nothing and flags every output row
    NaN, for the whole-cache kernel (small caches) and the filled-slot one
    (the 105 MB batch-32 layer)."""
    hd = 64
    qkv = torch.ones(B, 3 * H * hd, device=dev)
    kc = torch.zeros(B, H, T, hd, device=dev)
    vc = torch.zeros(B, H, T, hd, device=dev)
    y = torch.zeros(B, H * hd, device=dev)
    for bad in (T, T + 5, -1):
        p = torch.tensor([bad], device=dev)
        rc = _lib.lib().tiq_decode_attention(qkv.data_ptr(), qkv.shape[1], B, H, H, hd, kc.data_ptr(), vc.data_ptr(),
                                             T, p.data_ptr(), y.data_ptr(), H * hd, _st())
        assert rc == 0
        assert torch.isnan(y).all() and not kc.any() and not vc.any()
    x = torch.zeros(1, 8, device=dev)
    tok, p0 = torch.tensor([99], device=dev), torch.tensor([0], device=dev)
    wte, wpe = torch.ones(10, 8, device=dev), torch.ones(4, 8, device=dev)
    rc = _lib.lib().tiq_embed_tokens(tok.data_ptr(), p0.data_ptr(), wte.data_ptr(), 10, wpe.data_ptr(), 4, 1, 8,
                                     x.data_ptr(), _st())
    assert rc == 0 and torch.isnan(x).all()


def test_embed_and_argmax(dev):
    V, P, C, B = 97, 32, 64, 3
    gen = torch.Generator().manual_seed(5)
    wte, wpe = torch.randn(V, C, generator=gen), torch.randn(P, C, generator=gen)
    tok = torch.tensor([3, 96, 0])
    x = torch.empty(B, C, device=dev)
    tokd, p7, wted, wped = tok.to(dev), torch.tensor([7], device=dev), wte.to(dev), wpe.to(dev)
    rc = _lib.lib().tiq_embed_tokens(tokd.data_ptr(), p7.data_ptr(), wted.data_ptr(), V, wped.data_ptr(), P, B, C,
                                     x.data_ptr(), _st())
    _lib.check(rc, "embed")
    assert torch.equal(x.cpu(), wte[tok] + wpe[7])
    logits = torch.randn(B, 50257, generator=gen)
    logits[1, 100] = logits[1, 40000] = 50.0  # a tie: the first index wins
    out = torch.zeros(B, dtype=torch.long, device=dev)
    ids = torch.zeros(B, 16, dtype=torch.long, device=dev)
    ld, p4 = logits.to(dev), torch.tensor([4], device=dev)
    ws = torch.empty(int(_lib.lib().tiq_argmax_rows_workspace(B)), dtype=torch.uint8, device=dev)
    rc = _lib.lib().tiq_argmax_rows(ld.data_ptr(), B, 50257, 50257, out.data_ptr(), ids.data_ptr(), 16, p4.data_ptr(),
                                    ws.data_ptr(), ws.numel(), _st())
    _lib.check(rc, "argmax")
    assert torch.equal(out.cpu(), logits.argmax(-1)) and int(out[1]) == 100
    assert torch.equal(ids.cpu()[:, 5], logits.argmax(-1))
    assert int(p4) == 5  # the position advanced
    for cols in (1, 10, 63, 65, 1000):  # short rows: partial slices may be empty
        x = torch.randn(2, cols, generator=gen)
        xd = x.to(dev)
        rc = _lib.lib().tiq_argmax_rows(xd.data_ptr(), 2, cols, cols, out.data_ptr(), None, 0, None, ws.data_ptr(),
                                        ws.numel(), _st())
        _lib.check(rc, "argmax")
        assert torch.equal(out.cpu()[:2], x.argmax(-1)), cols


@pytest.mark.parametrize("rows", [16, 17, 40])
def test_argmax_many_rows_advances_position_once(dev, rows):
    """More rows than the final pass has wavefronts: each row's token lands in
    its id slot and the position advances exactly once."""
    gen = torch.Generator().manual_seed(rows)
    logits = torch.randn(rows, 5003, generator=gen)
    out = torch.zeros(rows, dtype=torch.long, device=dev)
    ids = torch.zeros(rows, 12, dtype=torch.long, device=dev)
    p = torch.tensor([9], device=dev)
    ws = torch.empty(int(_lib.lib().tiq_argmax_rows_workspace(rows)), dtype=torch.uint8, device=dev)
    rc = _lib.lib().tiq_argmax_rows(logits.to(dev).data_ptr(), rows, 5003, 5003, out.data_ptr(), ids.data_ptr(), 12,
                                    p.data_ptr(), ws.data_ptr(), ws.numel(), _st())
    _lib.check(rc, "argmax")
    ref = logits.argmax(-1)
    assert torch.equal(out.cpu(), ref) and torch.equal(ids.cpu()[:, 10], ref)
    assert int(p) == 10 and not ids.cpu()[:, :10].any() and not ids.cpu()[:, 11].any()


def _model(cfg, dev):
    torch.manual_seed(0)
    return g.GPT(cfg).to(dev).eval()


def test_fused_decoder_gpt2_small_matches_reference(reference_decode, dev):
    e = reference_decode["gpt2_small"]
    qm, _ = g.quantize_model(_model(g.GPTConfig(**e["config"]), dev), 8)
    gr = e["greedy_int8"]
    prompt = OM.benchmark_prompt(e["config"]["vocab_size"], *gr["prompt_shape"]).to(dev)
    dec = g.make_decoder(qm, 1, 128)
    assert isinstance(dec, g.FusedDecoder)
    out = g.generate_graph(qm, prompt, gr["new_tokens"], decoder=dec)
    assert out.cpu().tolist() == gr["ids"]
    again = g.generate_graph(qm, prompt, gr["new_tokens"], decoder=dec)  # graph reuse
    assert torch.equal(out, again)


@pytest.mark.parametrize("scheme", [(8, None), (4, None), (4, 64)])
def test_fused_decoder_matches_eager_mini(dev, scheme):
    bits, group = scheme
    cfg = g.GPTConfig(vocab_size=97, n_positions=96, n_layer=2, n_head=2, n_embd=128)
    qm, _ = g.quantize_model(_model(cfg, dev), bits, group_size=group)
    prompt = OM.benchmark_prompt(97, 2, 9).to(dev)
    want = g.generate(qm, prompt, 40)
    dec = g.make_decoder(qm, 2, 49)
    assert isinstance(dec, g.FusedDecoder)
    got = g.generate_graph(qm, prompt, 40, decoder=dec)
    assert torch.equal(got, want)


@pytest.mark.parametrize("B,T0", [(1, 1), (1, 64), (4, 16), (2, 31)])
@pytest.mark.parametrize("emb", [False, True])
def test_row_prefill_matches_forward_prefill(dev, B, T0, emb):
    """Prompts of up to 64 rows with int8 blocks: the fused decoder's own
    prefill (fused-epilogue Linears over the rows, the prefill attention,
    head and argmax kernels) against the model's forward prefill: the same
    first token, slot and position, the caches and the last rows' logits to
    fp32 rounding; with the fp32 tied head and with int8 head codes."""
    cfg = g.GPTConfig(vocab_size=97, n_positions=96, n_layer=2, n_head=2, n_embd=128)
    qm, _ = g.quantize_model(_model(cfg, dev), 8, include_embedding=emb)
    prompt = OM.benchmark_prompt(97, B, T0).to(dev)
    rows, fwd = g.FusedDecoder(qm, B, T0 + 4), g.FusedDecoder(qm, B, T0 + 4)
    assert rows.rows_prefill
    fwd.rows_prefill = False
    rows.start(prompt)
    fwd.start(prompt)
    with torch.no_grad():
        want = qm(prompt, last_only=True)["logits"][:, -1, :]
    torch.cuda.synchronize()
    assert torch.equal(rows.out, fwd.out) and torch.equal(rows.tok, fwd.tok) and torch.equal(rows.pos, fwd.pos)
    assert int(rows.pos) == T0 and torch.equal(rows.out[:, T0], want.argmax(-1))
    for i in range(cfg.n_layer):
        for a, b in ((rows.k[i], fwd.k[i]), (rows.v[i], fwd.v[i])):
            assert float((a - b).abs().max()) <= 1e-5 * float(b.abs().max()), i
    assert float((rows.logits - want).abs().max()) <= 1e-4 * float(want.abs().max())


def test_graph_replays_with_different_prompts(reference_decode, dev):
    """Captured prefill and decode graphs replayed for several prompts of the
    same length, with eager work in between, match eager generation each time."""
    cfg = g.GPTConfig(vocab_size=97, n_positions=96, n_layer=2, n_head=2, n_embd=128)
    qm, _ = g.quantize_model(_model(cfg, dev), 8)
    dec = g.make_decoder(qm, 2, 40)
    for seed in range(4):
        torch.manual_seed(seed)
        prompt = torch.randint(0, 97, (2, 8), device=dev)
        want = g.generate(qm, prompt, 30)
        got = g.generate_graph(qm, prompt, 30, decoder=dec)
        torch.cuda.synchronize()
        assert torch.equal(got, want), seed
    assert len(dec.prefill_graphs) == 1


# ---- tiq_decode_linear: batched decode linears with the K range split over
# workgroups, chained through operand planes ---------------------------------

def _dl(x, xp, M, K, wd, wf, sd, bd, N, y, ln=None, act=0, res=None, nln=None, planes=None, ws=None):
    L = _lib.lib()
    n_ws = int(L.tiq_decode_linear_workspace(wf, M, K, N))
    if ws is None:
        ws = torch.empty(max(n_ws, 1), dtype=torch.uint8, device="cuda")
    p = lambda t: None if t is None else t.data_ptr()
    rc = L.tiq_decode_linear(p(x), 0 if x is None else x.stride(0), p(xp), M, K, wd.data_ptr(), wf, p(sd), p(bd), N,
                             p(y), 0 if y is None else y.stride(0), p(None if ln is None else ln[0]),
                             p(None if ln is None else ln[1]), 1e-5, act, p(res), 0 if res is None else res.stride(0),
                             p(None if nln is None else nln[0]), p(None if nln is None else nln[1]), 1e-5, p(planes),
                             ws.data_ptr(), n_ws, _st())
    torch.cuda.synchronize()
    return rc


def _w8(c_oracle, N, K, gen, dev):
    w = torch.randn(N, K, generator=gen) * 0.02
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    return torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), OL.dequantize(q, s)


@pytest.mark.parametrize("M", [5, 32, 64])
@pytest.mark.parametrize("K,N", [(1600, 4800), (1600, 1600), (6400, 1600), (768, 2304)])
def test_decode_linear_ln_gelu(dev, c_oracle, M, K, N):
    """fp32 rows in, LayerNorm + GELU epilogue, fp32 out: split-K products and
    the fixed-order reduction, held to the float64 bar."""
    gen = torch.Generator().manual_seed(M * 3 + K + N)
    qd, sd, w_hat = _w8(c_oracle, N, K, gen, dev)
    x = torch.randn(M, K, generator=gen) * 2 + 0.5
    lw, lb = 1 + 0.1 * torch.randn(K, generator=gen), 0.1 * torch.randn(K, generator=gen)
    b = 0.1 * torch.randn(N, generator=gen)
    y = torch.empty(M, N, device=dev)
    rc = _dl(x.to(dev), None, M, K, qd, _lib.WF_INT8, sd, b.to(dev), N, y, ln=(lw.to(dev), lb.to(dev)),
             act=_lib.ACT_GELU_TANH)
    _lib.check(rc, "decode linear")
    ref = _gelu(OL.linear_ref(F.layer_norm(x, (K,), lw, lb, 1e-5), w_hat, b))
    xn64 = F.layer_norm(x.double(), (K,), lw.double(), lb.double(), 1e-5)
    _f64_check(y, ref, _gelu(xn64 @ w_hat.double().T + b.double()))


@pytest.mark.parametrize("M", [8, 32])
def test_decode_linear_chain_through_planes(dev, c_oracle, M):
    """The decode block's chain: (1) fp32 rows + LayerNorm -> y1 and the
    planes of LayerNorm2(y1); (2) those planes -> GELU, planes only (no fp32
    output); (3) those planes -> + bias + residual in place. Each stage is
    checked against float64 from the GPU's previous fp32 result."""
    C, H = 1600, 6400
    gen = torch.Generator().manual_seed(M)
    q1, s1, w1 = _w8(c_oracle, C, C, gen, dev)
    q2, s2, w2 = _w8(c_oracle, H, C, gen, dev)
    q3, s3, w3 = _w8(c_oracle, C, H, gen, dev)
    b1, b2, b3 = (0.1 * torch.randn(n, generator=gen) for n in (C, H, C))
    g1, e1, g2, e2 = (1 + 0.1 * torch.randn(C, generator=gen), 0.1 * torch.randn(C, generator=gen),
                      1 + 0.1 * torch.randn(C, generator=gen), 0.1 * torch.randn(C, generator=gen))
    x = torch.randn(M, C, generator=gen)
    r0 = torch.randn(M, C, generator=gen)
    L = _lib.lib()
    pa = torch.empty(int(L.tiq_decode_planes_bytes(M, C)), dtype=torch.uint8, device=dev)
    pb = torch.empty(int(L.tiq_decode_planes_bytes(M, H)), dtype=torch.uint8, device=dev)
    y1 = torch.empty(M, C, device=dev)
    _lib.check(_dl(x.to(dev), None, M, C, q1, _lib.WF_INT8, s1, b1.to(dev), C, y1, ln=(g1.to(dev), e1.to(dev)),
                   nln=(g2.to(dev), e2.to(dev)), planes=pa), "stage 1")
    ref = OL.linear_ref(F.layer_norm(x, (C,), g1, e1, 1e-5), w1, b1)
    _f64_check(y1, ref, F.layer_norm(x.double(), (C,), g1.double(), e1.double(), 1e-5) @ w1.double().T + b1.double())
    _lib.check(_dl(None, pa, M, C, q2, _lib.WF_INT8, s2, b2.to(dev), H, None, act=_lib.ACT_GELU_TANH, planes=pb),
               "stage 2")
    y3 = r0.to(dev).clone()
    _lib.check(_dl(None, pb, M, H, q3, _lib.WF_INT8, s3, b3.to(dev), C, y3, res=y3), "stage 3")
    h64 = _gelu(F.layer_norm(y1.cpu().double(), (C,), g2.double(), e2.double(), 1e-5) @ w2.double().T + b2.double())
    h32 = _gelu(OL.linear_ref(F.layer_norm(y1.cpu(), (C,), g2, e2, 1e-5), w2, b2))
    _f64_check(y3, r0 + OL.linear_ref(h32, w3, b3), r0.double() + h64 @ w3.double().T + b3.double())


@pytest.mark.parametrize("M", [5, 32, 40])
def test_decode_linear_product_writes_planes(dev, c_oracle, M):
    """One split, planes out without a LayerNorm (the c_fc of a block): the
    product kernel writes the fp32 rows and the planes itself. The planes are
    exactly the split of those rows: a projection from them equals the
    projection from the rows bit for bit."""
    C, H = 1600, 6400
    gen = torch.Generator().manual_seed(M + 7)
    q2, s2, w2 = _w8(c_oracle, H, C, gen, dev)
    q3, s3, _ = _w8(c_oracle, C, H, gen, dev)
    b2 = 0.1 * torch.randn(H, generator=gen)
    x = torch.randn(M, C, generator=gen)
    L = _lib.lib()
    pb = torch.empty(int(L.tiq_decode_planes_bytes(M, H)), dtype=torch.uint8, device=dev)
    h = torch.empty(M, H, device=dev)
    _lib.check(_dl(x.to(dev), None, M, C, q2, _lib.WF_INT8, s2, b2.to(dev), H, h, act=_lib.ACT_GELU_TANH, planes=pb),
               "gelu rows + planes")
    h64 = _gelu(x.double() @ w2.double().T + b2.double())
    _f64_check(h, _gelu(OL.linear_ref(x, w2, b2)), h64)
    a = torch.empty(M, C, device=dev)
    b = torch.empty(M, C, device=dev)
    _lib.check(_dl(None, pb, M, H, q3, _lib.WF_INT8, s3, None, C, a), "from planes")
    _lib.check(_dl(h, None, M, H, q3, _lib.WF_INT8, s3, None, C, b), "from rows")
    assert torch.equal(a, b)


@pytest.mark.parametrize("M", [6, 32])
def test_decode_linear_fp32_weights_and_errors(dev, M):
    """fp32 weights (the head) from planes, N not a multiple of 8 (one split,
    no reduction); argument errors; a second call with fewer rows on the same
    workspace."""
    K, N = 768, 5003
    L = _lib.lib()
    gen = torch.Generator().manual_seed(M + 1)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen)
    lw, lb = 1 + 0.1 * torch.randn(K, generator=gen), 0.1 * torch.randn(K, generator=gen)
    wd = w.to(dev)
    y = torch.empty(M, N, device=dev)
    _lib.check(_dl(x.to(dev), None, M, K, wd, _lib.WF_F32, None, None, N, y, ln=(lw.to(dev), lb.to(dev))), "head")
    ref = F.layer_norm(x, (K,), lw, lb, 1e-5) @ w.T
    _f64_check(y, ref, F.layer_norm(x.double(), (K,), lw.double(), lb.double(), 1e-5) @ w.double().T)
    # planes carry their LayerNorm: LayerNorm with planes input is an error
    pl = torch.zeros(int(L.tiq_decode_planes_bytes(M, K)), dtype=torch.uint8, device=dev)
    assert _dl(None, pl, M, K, wd, _lib.WF_F32, None, None, N, y, ln=(lw.to(dev), lb.to(dev))) == -1
    # a workspace too small for the input planes
    assert int(L.tiq_decode_planes_bytes(M, K)) > 256
    small = torch.empty(256, dtype=torch.uint8, device=dev)
    rc = L.tiq_decode_linear(x.to(dev).data_ptr(), K, None, M, K, wd.data_ptr(), _lib.WF_F32, None, None, N,
                             y.data_ptr(), N, None, None, 1e-5, 0, None, 0, None, None, 1e-5, None, small.data_ptr(),
                             small.numel(), _st())
    assert rc == -5
    # two calls in a row on one workspace, the second with fewer rows
    gen2 = torch.Generator().manual_seed(9)
    C, N2 = 1600, 4800
    w2 = torch.randn(N2, C, generator=gen2) * 0.02
    w2d = w2.to(dev)
    ws = torch.empty(int(L.tiq_decode_linear_workspace(_lib.WF_F32, 32, C, N2)), dtype=torch.uint8, device=dev)
    for rows in (32, 32 - 7):
        xx = torch.randn(rows, C, generator=gen2)
        yy = torch.empty(rows, N2, device=dev)
        _lib.check(_dl(xx.to(dev), None, rows, C, w2d, _lib.WF_F32, None, None, N2, yy, ws=ws), "reuse")
        _f64_check(yy, xx @ w2.T, xx.double() @ w2.double().T)


@pytest.mark.parametrize("B,H,pos", [(8, 25, 130), (32, 2, 20)])
def test_decode_attention_planes_feed_the_projection(dev, c_oracle, B, H, pos):
    """tiq_decode_attention_planes writes the same rows as tiq_decode_attention
    and, as planes, the input of tiq_decode_linear: the projection from them
    equals the projection from the fp32 rows bit for bit."""
    L = _lib.lib()
    hd, T = 64, 256
    C = H * hd
    gen = torch.Generator().manual_seed(B + H + pos)
    qkv = torch.randn(B, 3 * C, generator=gen).to(dev)
    kc = torch.randn(B, H, T, hd, generator=gen).to(dev)
    vc = torch.randn(B, H, T, hd, generator=gen).to(dev)
    kc2, vc2 = kc.clone(), vc.clone()
    p = torch.tensor([pos], device=dev)
    y1 = torch.empty(B, C, device=dev)
    y2 = torch.empty(B, C, device=dev)
    planes = torch.empty(int(L.tiq_decode_planes_bytes(B, C)), dtype=torch.uint8, device=dev)
    _lib.check(L.tiq_decode_attention(qkv.data_ptr(), 3 * C, B, H, H, hd, kc.data_ptr(), vc.data_ptr(), T,
                                      p.data_ptr(), y1.data_ptr(), C, _st()), "attention")
    _lib.check(L.tiq_decode_attention_planes(qkv.data_ptr(), 3 * C, B, H, H, hd, kc2.data_ptr(), vc2.data_ptr(), T,
                                             p.data_ptr(), y2.data_ptr(), C, planes.data_ptr(), _st()), "planes")
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(kc, kc2) and torch.equal(vc, vc2)
    qd, sd, _ = _w8(c_oracle, C, C, gen, dev)
    a = torch.empty(B, C, device=dev)
    b = torch.empty(B, C, device=dev)
    _lib.check(_dl(y1, None, B, C, qd, _lib.WF_INT8, sd, None, C, a), "from rows")
    _lib.check(_dl(None, planes, B, C, qd, _lib.WF_INT8, sd, None, C, b), "from planes")
    assert torch.equal(a, b)


@pytest.mark.parametrize("n", [1, 3, 4, 1000, 4096 * 6400 + 3])
def test_gelu_tanh_pass(dev, n):
    """The one-pass GELU against the formula in float64 (model.py:57-75), in
    place and out of place, with a ragged tail; large and tiny magnitudes."""
    gen = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=gen) * 4.0
    x[: min(n, 8)] = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 30.0, -30.0, 1e4, -1e4])[: min(n, 8)]
    ref = (0.5 * x.double() * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x.double() + 0.044715 * x.double() ** 3))))
    xd = x.to(dev)
    y = torch.empty_like(xd)
    L = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(L.tiq_gelu_tanh(xd.data_ptr(), y.data_ptr(), n, st), "gelu")
    inplace = xd.clone()
    _lib.check(L.tiq_gelu_tanh(inplace.data_ptr(), inplace.data_ptr(), n, st), "gelu in place")
    torch.cuda.synchronize()
    err = (y.cpu().double() - ref).abs()
    assert bool((err <= 4e-6 * ref.abs() + 1e-6).all()), float((err - 4e-6 * ref.abs()).max())
    assert torch.equal(y.cpu(), inplace.cpu())
    from gpt2_harness_amd.model import gelu_tanh

    assert torch.equal(gelu_tanh(xd).cpu(), y.cpu())
    torch_chain = 0.5 * xd * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (xd + 0.044715 * xd.pow(3))))
    assert torch.allclose(y, torch_chain, rtol=1e-5, atol=1e-6)


# ---- operand-tiled int8 codes (tiq_tile_int8, TIQ_WF_INT8_TILED) -----------

@pytest.mark.parametrize("N,K,ldw", [(64, 96, 96), (96, 64, 80), (4800, 1600, 1600)])
def test_tile_int8_layout(dev, N, K, ldw):
    """Byte 16 l + j of block t * (K / 32) + u is w[32 t + l % 32][32 u +
    16 (l / 32) + j]: the expected bytes are rearranged here on the CPU."""
    gen = torch.Generator().manual_seed(N + K + ldw)
    full = torch.randint(-127, 128, (N, ldw), generator=gen, dtype=torch.int8)
    w = full[:, :K]
    tiles = torch.empty(N * K, dtype=torch.int8, device=dev)
    _lib.check(_lib.lib().tiq_tile_int8(full.to(dev).data_ptr(), N, K, ldw, tiles.data_ptr(), _st()), "tile")
    torch.cuda.synchronize()
    # (t, r, u, h, j) -> (t, u, h, r, j)
    want = w.reshape(N // 32, 32, K // 32, 2, 16).permute(0, 2, 3, 1, 4).reshape(-1)
    assert torch.equal(tiles.cpu(), want)


def test_tile_int8_rejects_partial_tiles(dev):
    L = _lib.lib()
    w = torch.zeros(48, 64, dtype=torch.int8, device=dev)
    t = torch.empty_like(w)
    assert L.tiq_tile_int8(w.data_ptr(), 48, 64, 64, t.data_ptr(), _st()) == -4
    assert L.tiq_tile_int8(w.data_ptr(), 32, 48, 64, t.data_ptr(), _st()) == -4
    assert L.tiq_tile_int8(w.data_ptr(), 32, 64, 40, t.data_ptr(), _st()) == -1  # ldw < K
    # the decode linear refuses tiled codes with a partial row tile
    n_ws = int(L.tiq_decode_linear_workspace(_lib.WF_INT8_TILED, 8, 64, 48))
    ws = torch.empty(max(n_ws, 1), dtype=torch.uint8, device=dev)
    x = torch.zeros(8, 64, device=dev)
    y = torch.empty(8, 48, device=dev)
    s = torch.ones(48, device=dev)
    rc = L.tiq_decode_linear(x.data_ptr(), 64, None, 8, 64, w.data_ptr(), _lib.WF_INT8_TILED, s.data_ptr(), None, 48,
                             y.data_ptr(), 48, None, None, 1e-5, 0, None, 0, None, None, 1e-5, None, ws.data_ptr(),
                             n_ws, _st())
    assert rc == -4


@pytest.mark.parametrize("M", [5, 32, 64])
@pytest.mark.parametrize("K,N", [(1600, 4800), (1600, 1600), (6400, 1600), (768, 2304), (3072, 768)])
def test_decode_linear_tiled_equals_row_major(dev, c_oracle, M, K, N):
    """The tiled codes feed the same products in the same order: every output
    of the decode chain (fp32 rows with LayerNorm in, GELU, planes out; then
    planes in, residual in place, next LayerNorm planes out) is bit-identical
    to the row-major call's."""
    gen = torch.Generator().manual_seed(M * 7 + K + N)
    qd, sd, _ = _w8(c_oracle, N, K, gen, dev)
    tiles = torch.empty_like(qd)
    _lib.check(_lib.lib().tiq_tile_int8(qd.data_ptr(), N, K, qd.stride(0), tiles.data_ptr(), _st()), "tile")
    b = (0.1 * torch.randn(N, generator=gen)).to(dev)
    x = (torch.randn(M, K, generator=gen) * 2 + 0.5).to(dev)
    lw, lb = (1 + 0.1 * torch.randn(K, generator=gen)).to(dev), (0.1 * torch.randn(K, generator=gen)).to(dev)
    nw, nb = (1 + 0.1 * torch.randn(N, generator=gen)).to(dev), (0.1 * torch.randn(N, generator=gen)).to(dev)
    L = _lib.lib()
    outs = {}
    for wf, wd in ((_lib.WF_INT8, qd), (_lib.WF_INT8_TILED, tiles)):
        y = torch.empty(M, N, device=dev)
        pl = torch.zeros(int(L.tiq_decode_planes_bytes(M, N)), dtype=torch.uint8, device=dev)
        _lib.check(_dl(x, None, M, K, wd, wf, sd, b, N, y, ln=(lw, lb), act=_lib.ACT_GELU_TANH, planes=pl), "rows in")
        r = torch.randn(M, N, generator=torch.Generator().manual_seed(M)).to(dev)
        y2 = r.clone()
        pl2 = torch.zeros_like(pl)
        _lib.check(_dl(None, _split_planes(x, dev), M, K, wd, wf, sd, b, N, y2, res=y2, nln=(nw, nb), planes=pl2),
                   "planes in")
        outs[wf] = (y, pl, y2, pl2)
    for a, c in zip(outs[_lib.WF_INT8], outs[_lib.WF_INT8_TILED]):
        assert torch.equal(a, c)


def _split_planes(x, dev):
    """Operand planes of fp32 rows x, made by the library's own split (a decode
    linear with planes out and no product work kept: the planes of y = x come
    from the reduction with one slice)."""
    M, K = x.shape
    L = _lib.lib()
    pl = torch.zeros(int(L.tiq_decode_planes_bytes(M, K)), dtype=torch.uint8, device=dev)
    # identity weights: y = x exactly (int8 codes 1 on the diagonal, scale 1),
    # planes of y out
    eye = torch.eye(K, dtype=torch.int8, device=dev)
    one = torch.ones(K, device=dev)
    _lib.check(_dl(x, None, M, K, eye, _lib.WF_INT8, one, None, K, None, planes=pl), "identity planes")
    return pl


@pytest.mark.parametrize("B,C,H,Hkv,pos,T,tiled", [(32, 1600, 25, 25, 200, 256, True), (32, 1600, 25, 25, 255, 384, False),
                                                   (8, 768, 12, 12, 130, 256, False), (5, 1024, 16, 16, 0, 128, True),
                                                   (40, 512, 4, 2, 99, 100, False), (6, 256, 2, 2, 63, 64, True),
                                                   (64, 1280, 20, 20, 300, 512, True)])
def test_qkv_attention_slices_equal_projection_then_attention(dev, c_oracle, B, C, H, Hkv, pos, T, tiled):
    """tiq_decode_qkv_attention (c_attn as split-K slices, summed with scale
    and bias by the attention kernel) against the two-call chain
    (tiq_decode_linear to qkv rows, then tiq_decode_attention_planes), and
    both against float64: the new key / value in the caches, the head outputs
    and their planes, the untouched slots of the caches."""
    hd = 64
    N = (H + 2 * Hkv) * hd
    L = _lib.lib()
    gen = torch.Generator().manual_seed(B + C + pos)
    qd, sd, w_hat = _w8(c_oracle, N, C, gen, dev)
    wd, wf = qd, _lib.WF_INT8
    if tiled:
        wd = torch.empty_like(qd)
        _lib.check(L.tiq_tile_int8(qd.data_ptr(), N, C, qd.stride(0), wd.data_ptr(), _st()), "tile")
        wf = _lib.WF_INT8_TILED
    b = 0.1 * torch.randn(N, generator=gen)
    bd = b.to(dev)
    x = torch.randn(B, C, generator=gen)
    pl = _split_planes(x.to(dev), dev)
    kc = torch.randn(B, Hkv, T, hd, generator=gen)
    vc = torch.randn(B, Hkv, T, hd, generator=gen)
    p = torch.tensor([pos], device=dev)
    # the two-call chain
    qkv = torch.empty(B, N, device=dev)
    _lib.check(_dl(None, pl, B, C, wd, wf, sd, bd, N, qkv), "c_attn")
    ka, va = kc.to(dev), vc.to(dev)
    ya = torch.empty(B, H * hd, device=dev)
    pa = torch.zeros(int(L.tiq_decode_planes_bytes(B, H * hd)), dtype=torch.uint8, device=dev)
    _lib.check(L.tiq_decode_attention_planes(qkv.data_ptr(), N, B, H, Hkv, hd, ka.data_ptr(), va.data_ptr(), T,
                                             p.data_ptr(), ya.data_ptr(), H * hd, pa.data_ptr(), _st()), "attention")
    # one call
    n_ws = int(L.tiq_decode_qkv_attention_workspace(B, C, N))
    assert n_ws >= B * N * 4
    ws = torch.full((n_ws,), 0xff, dtype=torch.uint8, device=dev)  # NaN bytes: every slice must be written
    kb, vb = kc.to(dev), vc.to(dev)
    yb = torch.empty(B, H * hd, device=dev)
    pb = torch.zeros_like(pa)
    _lib.check(L.tiq_decode_qkv_attention(pl.data_ptr(), B, C, wd.data_ptr(), wf, sd.data_ptr(), bd.data_ptr(), H,
                                          Hkv, hd, kb.data_ptr(), vb.data_ptr(), T, p.data_ptr(), yb.data_ptr(),
                                          H * hd, pb.data_ptr(), ws.data_ptr(), n_ws, _st()), "qkv attention")
    torch.cuda.synchronize()
    # float64 from the same inputs
    qkv64 = x.double() @ w_hat.double().T + b.double()
    q64 = qkv64[:, : H * hd].view(B, H, 1, hd)
    k64 = qkv64[:, H * hd : (H + Hkv) * hd].view(B, Hkv, hd)
    v64 = qkv64[:, (H + Hkv) * hd :].view(B, Hkv, hd)
    qkv32 = OL.linear_ref(x, w_hat, b)
    for got in (kb.cpu()[:, :, pos], ka.cpu()[:, :, pos]):
        _f64_check(got, qkv32[:, H * hd : (H + Hkv) * hd].view(B, Hkv, hd), k64)
    _f64_check(vb.cpu()[:, :, pos], qkv32[:, (H + Hkv) * hd :].view(B, Hkv, hd), v64)
    for c, d in ((kb, kc), (vb, vc)):  # every other slot as it was
        got = c.cpu()
        assert torch.equal(got[:, :, :pos], d[:, :, :pos]) and torch.equal(got[:, :, pos + 1 :], d[:, :, pos + 1 :])
    K64 = torch.cat([kc[:, :, :pos].double(), k64[:, :, None]], 2).repeat_interleave(H // Hkv, dim=1)
    V64 = torch.cat([vc[:, :, :pos].double(), v64[:, :, None]], 2).repeat_interleave(H // Hkv, dim=1)
    y64 = (F.softmax((q64 @ K64.transpose(-2, -1)) / math.sqrt(hd), dim=-1) @ V64).view(B, H * hd)
    err_b = float((yb.cpu().double() - y64).abs().max())
    err_a = float((ya.cpu().double() - y64).abs().max())
    assert err_b <= max(2 * err_a, 2e-6), (err_b, err_a)
    assert (yb - ya).abs().max().item() < 1e-5
    # the planes are exactly the split of the output rows
    qo, so, _ = _w8(c_oracle, C, H * hd, gen, dev)
    r1, r2 = torch.empty(B, C, device=dev), torch.empty(B, C, device=dev)
    _lib.check(_dl(None, pb, B, H * hd, qo, _lib.WF_INT8, so, None, C, r1), "from planes")
    _lib.check(_dl(yb, None, B, H * hd, qo, _lib.WF_INT8, so, None, C, r2), "from rows")
    assert torch.equal(r1, r2)


def test_qkv_attention_arguments(dev):
    """Refused shapes and arguments return before any launch: K not a multiple
    of 32, more than 64 rows, head_dim other than 64, a workspace short of the
    query; the query is 0 for an unsupported shape."""
    L = _lib.lib()
    assert L.tiq_decode_qkv_attention_workspace(65, 1600, 4800) == 0
    assert L.tiq_decode_qkv_attention_workspace(32, 1601, 4800) == 0
    assert L.tiq_decode_qkv_attention_workspace(32, 1600, 4800) > 0
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    f = buf.data_ptr()
    p = torch.zeros(1, dtype=torch.int64, device=dev)
    args = lambda B, C, hd, ws_bytes, wf=_lib.WF_INT8: (f, B, C, f, wf, f, None, 2, 2, hd, f, f, 16, p.data_ptr(), f,
                                                         128, None, f, ws_bytes, _st())
    assert L.tiq_decode_qkv_attention(*args(4, 100, 64, 1 << 16)) == L.tiq_decode_qkv_attention(*args(4, 100, 64, 0))
    assert L.tiq_decode_qkv_attention(*args(4, 100, 64, 1 << 16)) == -4  # TIQ_EUNSUPPORTED
    assert L.tiq_decode_qkv_attention(*args(65, 128, 64, 1 << 16)) == -4
    assert L.tiq_decode_qkv_attention(*args(4, 128, 32, 1 << 16)) == -4
    assert L.tiq_decode_qkv_attention(*args(4, 128, 64, 16, _lib.WF_F32)) == -4
    assert L.tiq_decode_qkv_attention(*args(4, 128, 64, 16)) == -5  # TIQ_EWORKSPACE
    assert L.tiq_decode_qkv_attention(*args(0, 128, 64, 0)) == 0


@pytest.mark.parametrize("N,K,ldw", [(100, 64, 64), (64, 256, 260), (50257, 768, 768)])
def test_tile_f32_layout(dev, N, K, ldw):
    """tiq_tile_f32: block (t, u) of 4 KB holds rows 32 t .. 32 t + 31 and columns
    32 u .. 32 u + 31, chunk 64 q + l the 4 floats w[32 t + l % 32][32 u +
    16 (l / 32) + 4 q ..]; rows past N are zero; a padded leading dimension."""
    L = _lib.lib()
    gen = torch.Generator().manual_seed(N + K)
    w = torch.randn(N, ldw, generator=gen)
    n_bytes = int(L.tiq_tile_f32_bytes(N, K))
    T, U = (N + 31) // 32, K // 32
    assert n_bytes == T * 32 * K * 4
    t = torch.full((n_bytes // 4,), float("nan"), device=dev)
    _lib.check(L.tiq_tile_f32(w.to(dev).data_ptr(), N, K, ldw, t.data_ptr(), _st()), "tile f32")
    wp = torch.zeros(T * 32, K)
    wp[:N] = w[:, :K]
    want = wp.view(T, 32, U, 2, 4, 4).permute(0, 2, 4, 3, 1, 5).reshape(-1)
    assert torch.equal(t.cpu(), want)


def test_tile_f32_errors(dev):
    L = _lib.lib()
    w = torch.zeros(64, 64, device=dev)
    t = torch.zeros(64 * 64, device=dev)
    assert L.tiq_tile_f32(w.data_ptr(), 64, 48, 64, t.data_ptr(), _st()) == -4  # K % 32
    assert L.tiq_tile_f32(w.data_ptr(), 64, 64, 40, t.data_ptr(), _st()) == -1  # ldw < K
    assert L.tiq_tile_f32(w.data_ptr(), 64, 64, 66, t.data_ptr(), _st()) == -3  # rows not 16-byte aligned
    assert L.tiq_tile_f32_bytes(64, 48) == 0


@pytest.mark.parametrize("M", [5, 32, 40, 64])
@pytest.mark.parametrize("K,N", [(768, 50257), (1600, 5003), (256, 1000), (1600, 64)])
def test_decode_linear_f32_tiles(dev, M, K, N):
    """The fp32 head from operand planes with tiled weights (one workgroup per
    CU streaming the tiles): bit-identical to the row-major weights' one-split
    product where that path takes one split, and to float64 within the fp32
    bar everywhere; workspace 0; the refused fusions."""
    L = _lib.lib()
    gen = torch.Generator().manual_seed(M + K + N)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen)
    wd = w.to(dev)
    t = torch.empty(int(L.tiq_tile_f32_bytes(N, K)) // 4, device=dev)
    _lib.check(L.tiq_tile_f32(wd.data_ptr(), N, K, K, t.data_ptr(), _st()), "tile f32")
    pl = _split_planes(x.to(dev), dev)
    assert L.tiq_decode_linear_workspace(_lib.WF_F32_TILED, M, K, N) == 0
    yt = torch.full((M, N), float("nan"), device=dev)
    _lib.check(_dl(None, pl, M, K, t, _lib.WF_F32_TILED, None, None, N, yt), "tiled head")
    yr = torch.empty(M, N, device=dev)
    _lib.check(_dl(None, pl, M, K, wd, _lib.WF_F32, None, None, N, yr), "row-major head")
    if N % 8 != 0 or N > 8192:  # the row-major path takes one split there: same products, same order
        assert torch.equal(yt, yr)
    _f64_check(yt, x @ w.T, x.double() @ w.double().T)
    # refused: fp32 rows in, a bias, planes out
    assert _dl(x.to(dev), None, M, K, t, _lib.WF_F32_TILED, None, None, N, yt) == -4
    b = torch.zeros(N, device=dev)
    assert _dl(None, pl, M, K, t, _lib.WF_F32_TILED, None, b, N, yt) == -4
    if N % 32 == 0:
        po = torch.zeros(int(L.tiq_decode_planes_bytes(M, N)), dtype=torch.uint8, device=dev)
        assert _dl(None, pl, M, K, t, _lib.WF_F32_TILED, None, None, N, yt, planes=po) == -4


@pytest.mark.parametrize("B,C,H,T", [(8, 768, 12, 64), (32, 1600, 25, 256)])
def test_qkv_attention_out_of_range_position(dev, c_oracle, B, C, H, T):
    """A position outside the cache through the fused q, k, v call: NaN output
    rows and planes' rows, nothing written to either cache (both the whole-cache
    kernel and the filled-slot one, whose first keys go out before pos is read)."""
    hd = 64
    N = 3 * H * hd
    L = _lib.lib()
    gen = torch.Generator().manual_seed(C + T)
    qd, sd, _ = _w8(c_oracle, N, C, gen, dev)
    pl = _split_planes(torch.randn(B, C, generator=gen).to(dev), dev)
    kc = torch.randn(B, H, T, hd, generator=gen).to(dev)
    vc = torch.randn(B, H, T, hd, generator=gen).to(dev)
    k0, v0 = kc.clone(), vc.clone()
    n_ws = int(L.tiq_decode_qkv_attention_workspace(B, C, N))
    ws = torch.empty(n_ws, dtype=torch.uint8, device=dev)
    y = torch.zeros(B, H * hd, device=dev)
    for bad in (T, T + 3, -1):
        p = torch.tensor([bad], device=dev)
        _lib.check(L.tiq_decode_qkv_attention(pl.data_ptr(), B, C, qd.data_ptr(), _lib.WF_INT8, sd.data_ptr(), None,
                                              H, H, hd, kc.data_ptr(), vc.data_ptr(), T, p.data_ptr(), y.data_ptr(),
                                              H * hd, None, ws.data_ptr(), n_ws, _st()), "qkv attention")
        torch.cuda.synchronize()
        assert torch.isnan(y).all()
        assert torch.equal(kc, k0) and torch.equal(vc, v0)


@pytest.mark.parametrize("rows,cols", [(1, 50257), (2, 50257), (1, 57344), (2, 1025), (1, 60000), (2, 3)])
def test_argmax_few_rows(dev, rows, cols):
    """One or two rows (a single-sequence decode step), vocabulary-sized and
    short: first index of the maximum on ties, a NaN never chosen, index 0 for
    a row of -inf and NaN, the token in its id slot and the position advanced
    once."""
    L = _lib.lib()
    gen = torch.Generator().manual_seed(rows * 7 + cols)
    logits = torch.randn(rows, cols, generator=gen)
    hi = cols - 1
    logits[0, hi] = 9.0
    logits[0, min(hi, 1)] = 9.0  # tie with a lower index
    logits[0, min(hi, 2)] = float("nan")
    if rows > 1:
        logits[1].fill_(float("-inf"))
        logits[1, :: max(1, cols // 5)] = float("nan")
    want = []
    for r in range(rows):  # the rule: maximum over non-NaN values, first index; 0 if none above -inf
        row = logits[r].clone()
        row[torch.isnan(row)] = float("-inf")
        want.append(int(row.argmax()) if bool((row > float("-inf")).any()) else 0)
    out = torch.full((rows,), -1, dtype=torch.long, device=dev)
    ids = torch.zeros(rows, 8, dtype=torch.long, device=dev)
    p = torch.tensor([3], device=dev)
    ws = torch.empty(int(L.tiq_argmax_rows_workspace(rows)), dtype=torch.uint8, device=dev)
    _lib.check(L.tiq_argmax_rows(logits.to(dev).data_ptr(), rows, cols, cols, out.data_ptr(), ids.data_ptr(), 8,
                                 p.data_ptr(), ws.data_ptr(), ws.numel(), _st()), "argmax")
    torch.cuda.synchronize()
    assert out.cpu().tolist() == want
    assert ids.cpu()[:, 4].tolist() == want and int(p) == 4
    assert not ids.cpu()[:, :4].any() and not ids.cpu()[:, 5:].any()


def _attn64(q, k, v, first):
    """float64 causal attention of queries at first .. first + T - 1 over keys 0 .. S - 1."""
    T, S = q.shape[-2], k.shape[-2]
    s = (q.double() @ k.double().transpose(-2, -1)) / 8.0
    mask = torch.arange(S)[None, :] > (first + torch.arange(T))[:, None]
    return F.softmax(s.masked_fill(mask, float("-inf")), dim=-1) @ v.double()


@pytest.mark.parametrize("B,H,T,first,cap", [(2, 12, 64, 0, 0), (2, 12, 70, 0, 0), (1, 4, 1, 0, 0),
                                             (3, 4, 70, 30, 256), (32, 25, 128, 0, 256), (1, 2, 1, 100, 128),
                                             (2, 3, 200, 500, 1024)])
def test_prefill_attention(dev, B, H, T, first, cap):
    """tiq_prefill_attention against float64: q, k, v read in place as views of
    the projection's (B, T, 3C) rows (cap = 0) or, with a history of `first`
    positions, k and v from (B, H, cap, 64) cache buffers; the output written as
    (B, T, C) rows; T not a multiple of the 64-row tile; a single query."""
    hd, C = 64, H * 64
    gen = torch.Generator().manual_seed(B * 100 + T + first)
    qkv = torch.randn(B, T, 3 * C, generator=gen)
    q, k, v = qkv.view(B, T, 3, H, hd).permute(2, 0, 3, 1, 4).unbind(0)
    if cap:
        kc = torch.randn(B, H, cap, hd, generator=gen)
        vc = torch.randn(B, H, cap, hd, generator=gen)
        kc[:, :, first : first + T] = k
        vc[:, :, first : first + T] = v
        kd, vd = kc.to(dev)[:, :, : first + T], vc.to(dev)[:, :, : first + T]
        kr, vr = kc[:, :, : first + T], vc[:, :, : first + T]
    else:
        kd = vd = None
        kr, vr = k, v
    qkvd = qkv.to(dev)
    qd, kd2, vd2 = qkvd.view(B, T, 3, H, hd).permute(2, 0, 3, 1, 4).unbind(0)
    if kd is None:
        kd, vd = kd2, vd2
    y = torch.full((B, T, C), float("nan"), device=dev)
    _lib.check(_lib.lib().tiq_prefill_attention(
        qd.data_ptr(), qd.stride(0), qd.stride(1), qd.stride(2), kd.data_ptr(), kd.stride(0), kd.stride(1),
        kd.stride(2), vd.data_ptr(), vd.stride(0), vd.stride(1), vd.stride(2), B, H, T, first, hd, y.data_ptr(),
        y.stride(0), hd, y.stride(1), _st()), "prefill attention")
    ref = _attn64(q, kr, vr, first).transpose(1, 2).reshape(B, T, C)
    err = float((y.cpu().double() - ref).abs().max())
    assert err < 2e-5, err


def test_prefill_attention_arguments(dev):
    L = _lib.lib()
    buf = torch.zeros(4 * 3 * 64 * 64, device=dev)
    f = buf.data_ptr()
    args = lambda hd, st=64, p=f: (p, 0, 0, st, f, 0, 0, 64, f, 0, 0, 64, 1, 1, 4, 0, hd, f, 0, 0, 64, _st())
    assert L.tiq_prefill_attention(*args(32)) == -4
    assert L.tiq_prefill_attention(*args(64, 66)) == -3
    assert L.tiq_prefill_attention(*args(64, 64, f + 4)) == -3
    assert L.tiq_prefill_attention(*args(64)) == 0
