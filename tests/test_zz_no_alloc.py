"""tiq_decode_linear_noalloc, the allocation-free batched decode linear.

It runs the kernels of tiq_decode_linear with a fixed device array as the
workspace, so its results must equal tiq_decode_linear's (given a workspace
the caller allocated) bit for bit -- fp32 rows and operand planes alike --
over two calls in a row, the second smaller than the first (the array keeps
the first call's contents); a request whose workspace would pass the array
is refused before anything is launched, with its output left untouched.
"""

from __future__ import annotations

import pytest
import torch

from gpt2_harness_amd import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20
TIQ_ESCRATCH = -6


def _st():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _case(dev, M, K, N, seed, gelu=False):
    """fp32 rows through LayerNorm into an int8 linear with bias (and GELU),
    writing y and the next linear's LayerNorm'd operand planes."""
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=gen) * 0.02
    amax = w.abs().amax(dim=1, keepdim=True)
    s = amax / 127
    q = torch.round(w / s).clamp(-127, 127).to(torch.int8)
    L = _lib.lib()
    c = {
        "M": M, "K": K, "N": N, "act": _lib.ACT_GELU_TANH if gelu else _lib.ACT_NONE,
        "x": torch.randn(M, K, generator=gen).to(dev),
        "q": q.to(dev), "s": s.reshape(-1).contiguous().to(dev),
        "b": (0.1 * torch.randn(N, generator=gen)).to(dev),
        "ln": ((1 + 0.1 * torch.randn(K, generator=gen)).to(dev), (0.1 * torch.randn(K, generator=gen)).to(dev)),
        "nln": ((1 + 0.1 * torch.randn(N, generator=gen)).to(dev), (0.1 * torch.randn(N, generator=gen)).to(dev)),
        "planes_bytes": int(L.tiq_decode_planes_bytes(M, N)),
        "ws_bytes": int(L.tiq_decode_linear_workspace(_lib.WF_INT8, M, K, N)),
    }
    return c


def _outputs(c, dev):
    y = torch.full((c["M"], c["N"]), 7.0, device=dev)
    planes = torch.full((c["planes_bytes"],), 0x5A, dtype=torch.uint8, device=dev)
    return y, planes


def _call(L, c, y, planes, ws=None):
    """tiq_decode_linear with a caller workspace (ws given) or the
    allocation-free entry (ws None)."""
    args = [_ptr(c["x"]), c["x"].stride(0), None, c["M"], c["K"], c["q"].data_ptr(), _lib.WF_INT8, c["s"].data_ptr(),
            c["b"].data_ptr(), c["N"], y.data_ptr(), y.stride(0), c["ln"][0].data_ptr(), c["ln"][1].data_ptr(), 1e-5,
            c["act"], None, 0, c["nln"][0].data_ptr(), c["nln"][1].data_ptr(), 1e-5, planes.data_ptr()]
    if ws is None:
        return L.tiq_decode_linear_noalloc(*args, _st())
    return L.tiq_decode_linear(*args, ws.data_ptr(), ws.numel(), _st())


def test_noalloc_equals_workspace_entry_on_two_calls(dev):
    L = _lib.lib()
    # GPT-2-XL mlp.c_proj shape (K split four ways: operand planes and fp32
    # partial slices in the scratch), then a smaller c_attn-shaped call
    big = _case(dev, 32, 6400, 1600, seed=1)
    small = _case(dev, 8, 1600, 4800, seed=2, gelu=True)
    assert 0 < small["ws_bytes"] < big["ws_bytes"] <= SCRATCH_BYTES
    got = []
    for c in (big, small):  # two calls in a row on the shared array
        y, planes = _outputs(c, dev)
        _lib.check(_call(L, c, y, planes), "tiq_decode_linear_noalloc")
        got.append((y, planes))
    torch.cuda.synchronize()
    for c, (y, planes) in zip((big, small), got):
        ws = torch.empty(c["ws_bytes"], dtype=torch.uint8, device=dev)
        y_ref, planes_ref = _outputs(c, dev)
        _lib.check(_call(L, c, y_ref, planes_ref, ws), "tiq_decode_linear")
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        assert torch.equal(y, y_ref), f"M={c['M']} K={c['K']} N={c['N']}: fp32 rows differ"
        assert torch.equal(planes, planes_ref), f"M={c['M']} K={c['K']} N={c['N']}: operand planes differ"


def test_noalloc_fp32_head_shape(dev):
    """The tied fp32 head of GPT-2-XL at 64 rows (row-major TIQ_WF_F32, no
    scale or bias): 13.5 MB of its 16 MiB scratch -- operand planes and one
    partial slice -- equal to the workspace entry bit for bit."""
    L = _lib.lib()
    M, K, N = 64, 1600, 50257
    need = int(L.tiq_decode_linear_workspace(_lib.WF_F32, M, K, N))
    assert 13_000_000 < need <= SCRATCH_BYTES
    gen = torch.Generator(device=dev).manual_seed(5)
    w = torch.randn(N, K, generator=gen, device=dev) * 0.02
    x = torch.randn(M, K, generator=gen, device=dev)
    ln = (1 + 0.1 * torch.randn(K, generator=gen, device=dev), 0.1 * torch.randn(K, generator=gen, device=dev))

    def call(y, ws):
        args = [x.data_ptr(), x.stride(0), None, M, K, w.data_ptr(), _lib.WF_F32, None, None, N, y.data_ptr(),
                y.stride(0), ln[0].data_ptr(), ln[1].data_ptr(), 1e-5, _lib.ACT_NONE, None, 0, None, None, 1e-5,
                None]
        if ws is None:
            return L.tiq_decode_linear_noalloc(*args, _st())
        return L.tiq_decode_linear(*args, ws.data_ptr(), ws.numel(), _st())

    y = torch.full((M, N), 7.0, device=dev)
    _lib.check(call(y, None), "tiq_decode_linear_noalloc (fp32 head)")
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    y_ref = torch.full((M, N), 7.0, device=dev)
    _lib.check(call(y_ref, ws), "tiq_decode_linear (fp32 head)")
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert torch.equal(y, y_ref)
    # and the head's result is the LayerNorm'd rows times the weights (fp32)
    ref = torch.nn.functional.layer_norm(x.double(), (K,), ln[0].double(), ln[1].double(), 1e-5) @ w.double().T
    assert (y.double() - ref).abs().max().item() <= 1e-3 * ref.abs().max().item()


def test_noalloc_refuses_beyond_its_scratch(dev):
    """64 rows of K = 12800 into N = 8192 need 21.7 MB (planes plus eight
    partial slices): refused before any launch. The buffers are full size
    all the same."""
    L = _lib.lib()
    M, K, N = 64, 12800, 8192
    need = int(L.tiq_decode_linear_workspace(_lib.WF_INT8, M, K, N))
    assert need > SCRATCH_BYTES
    c = {
        "M": M, "K": K, "N": N, "act": _lib.ACT_NONE,
        "x": torch.zeros(M, K, device=dev), "q": torch.zeros(N, K, dtype=torch.int8, device=dev),
        "s": torch.ones(N, device=dev), "b": torch.zeros(N, device=dev),
        "ln": (torch.ones(K, device=dev), torch.zeros(K, device=dev)),
        "nln": (torch.ones(N, device=dev), torch.zeros(N, device=dev)),
        "planes_bytes": int(L.tiq_decode_planes_bytes(M, N)),
    }
    y, planes = _outputs(c, dev)
    assert _call(L, c, y, planes) == TIQ_ESCRATCH
    assert b"fixed scratch" in L.tiq_status_string(TIQ_ESCRATCH)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all()) and bool((planes == 0x5A).all())
