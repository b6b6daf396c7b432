"""A quantized Linear over gelu_tanh of fp32 prefill rows (tiq_linear_gelu_in_ws,
QuantLinear.forward_gelu_in, MLP.forward): the MLP's c_proj(gelu_tanh(c_fc(x)))
with the activation applied while the rows are split into bf16 planes.

The fused product must equal, bit for bit, the two-step path whose parts the
other GPU tests pin (tiq_gelu_tanh against the reference formula, the
three-plane GEMM against the oracle's linear), and must stay within fp32
tolerance of a float64 restatement of gelu_tanh(x) @ W_hat^T + b.
"""
from __future__ import annotations

import math

import pytest
import torch

import gpt2_harness_amd as g
from gpt2_harness_amd import _lib
from gpt2_harness_amd.model import MLP, gelu_tanh

pytestmark = pytest.mark.gpu


def _quantized(K, N, fmt, dev, seed):
    gen = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(K, N)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=gen) * 0.02)
        lin.bias.copy_(torch.randn(N, generator=gen) * 0.1)
    lin = lin.to(dev)
    if fmt == "int8":
        mod, _ = g.quantize_linear(lin, 8)
    elif fmt == "int4":
        mod, _ = g.quantize_linear(lin, 4)
    else:
        mod, _ = g.quantize_linear(lin, 4, group_size=128)
    return mod.to(dev)


def _gelu64(x):
    x = x.double()
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x.pow(3))))


@pytest.mark.parametrize("fmt", ["int8", "int4", "int4_groupwise"])
@pytest.mark.parametrize("K,N,M", [(3072, 768, 256), (6400, 1600, 129), (768, 2304, 300)])
def test_gelu_in_equals_two_steps(dev, fmt, K, N, M):
    mod = _quantized(K, N, fmt, dev, seed=K + N + M)
    gen = torch.Generator().manual_seed(M)
    x = (torch.randn(M, K, generator=gen) * 2.0).to(dev)
    with torch.no_grad():
        fused = mod.forward_gelu_in(x)
        two = mod(gelu_tanh(x))
    torch.cuda.synchronize()
    assert fused is not None
    assert torch.equal(fused, two), (fused - two).abs().max().item()
    ref = _gelu64(x.cpu()) @ mod.weight.double().cpu().t() + mod.bias.double().cpu()
    err = (fused.double().cpu() - ref).abs().max().item()
    assert err <= 2e-5 * max(1.0, ref.abs().max().item()), err


def test_gelu_in_leading_dimensions_and_input_untouched(dev):
    mod = _quantized(768, 3072, "int8", dev, seed=3)
    x = torch.randn(2, 128, 768, device=dev)
    x0 = x.clone()
    with torch.no_grad():
        y = mod.forward_gelu_in(x)
        ref = mod(gelu_tanh(x0))
    assert y.shape == (2, 128, 3072)
    assert torch.equal(x, x0)
    assert torch.equal(y, ref)


def test_gelu_in_declines_what_it_does_not_take(dev):
    mod = _quantized(768, 768, "int8", dev, seed=4)
    with torch.no_grad():
        assert mod.forward_gelu_in(torch.randn(64, 768, device=dev)) is None  # decode-sized rows
        assert mod.forward_gelu_in(torch.randn(256, 768, device=dev, dtype=torch.bfloat16)) is None
        assert mod.forward_gelu_in(torch.randn(256, 768)) is None  # host rows
    xg = torch.randn(256, 768, device=dev, requires_grad=True)
    assert mod.forward_gelu_in(xg) is None  # a gradient is wanted


def test_gelu_in_arguments(dev):
    mod = _quantized(768, 768, "int8", dev, seed=5)
    L = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    M, K, N = 256, 768, 768
    x = torch.randn(M, K, device=dev)
    y = torch.empty(M, N, device=dev)
    need = int(L.tiq_gemm_w8_workspace(_lib.dtype_code(torch.float32), M, K, N))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)

    def call(m=M, wf=_lib.WF_INT8, ws_bytes=need, ldx=K):
        return L.tiq_linear_gelu_in_ws(x.data_ptr(), m, K, ldx, mod.codes.data_ptr(), wf, mod.scale.data_ptr(), None,
                                       0, _lib.ptr(mod.bias), N, y.data_ptr(), N, ws.data_ptr(), ws_bytes, st)

    assert call() == _lib.OK
    assert call(m=100) == _lib.EUNSUPPORTED
    assert call(m=0) == _lib.OK
    assert call(wf=_lib.WF_F32) == _lib.EINVAL
    assert call(ldx=K - 1) == _lib.EINVAL
    planes = M * 3 * K * 2  # the bf16 planes of the rows; the rest holds split-K partials
    assert call(ws_bytes=planes - 256) == _lib.EWORKSPACE
    assert call(ws_bytes=planes) == _lib.OK  # the product then runs unsplit
    torch.cuda.synchronize()


@pytest.mark.parametrize("bits,group", [(8, None), (4, 128)])
def test_mlp_prefill_uses_gelu_in(dev, bits, group):
    cfg = g.gpt2_config("gpt2")
    torch.manual_seed(0)
    mlp = MLP(cfg).to(dev)
    for name in ("c_fc", "c_proj"):
        q, _ = g.quantize_linear(getattr(mlp, name), bits, group_size=group)
        setattr(mlp, name, q)
    mlp = mlp.to(dev).eval()
    x = torch.randn(2, 100, cfg.n_embd, device=dev)
    with torch.no_grad():
        assert mlp.c_proj.forward_gelu_in(mlp.c_fc(x)) is not None  # 200 rows: the fused entry applies
        y = mlp(x)
        ref = mlp.c_proj(gelu_tanh(mlp.c_fc(x)))
    assert torch.equal(y, ref)
