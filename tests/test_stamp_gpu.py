"""Stamped measurement copies of the decode GEMV and the staged GEMM.

Between tiq_stamp_begin and tiq_stamp_end the direct GEMV kernel (int8
weights, bf16 in and out) and the staged prefill GEMM (int8, bf16 out) run a
copy that also writes each workgroup's entry and exit time. The copy must
compute exactly what the product kernel computes, hand out slots launch by
launch (first slot, workgroup count) in launch order, and leave entry <= exit
on both counters for every workgroup (four slots a workgroup: real-time entry
and exit, shader-clock entry and exit); with stamping off the product kernel
runs again.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import gpt2_harness_amd as g
from gpt2_harness_amd import _lib

pytestmark = pytest.mark.gpu


def _end(L):
    n = 64
    first, wgs = (ctypes.c_int64 * n)(), (ctypes.c_int64 * n)()
    k = int(L.tiq_stamp_end(first, wgs, n))
    return [(first[i], wgs[i]) for i in range(min(k, n))]


def _linear(L, x, q, s, N, y, ws=None):
    M, K = x.shape
    st = torch.cuda.current_stream().cuda_stream
    if ws is None:
        rc = L.tiq_linear_w8(x.data_ptr(), _lib.BF16, M, K, K, q.data_ptr(), s.data_ptr(), None, N, y.data_ptr(),
                             _lib.BF16, N, st)
    else:
        rc = L.tiq_gemm_w8_ws(x.data_ptr(), _lib.BF16, M, K, K, q.data_ptr(), s.data_ptr(), None, N, y.data_ptr(),
                              _lib.BF16, N, ws.data_ptr(), ws.numel(), st)
    _lib.check(rc, "linear")


@pytest.mark.parametrize("M,K,N", [(1, 768, 2304), (1, 3072, 768), (3, 1600, 6400), (4096, 1600, 1600)])
def test_stamped_copy_equals_product_kernel(dev, M, K, N):
    L = _lib.lib()
    gen = torch.Generator(device=dev).manual_seed(M + K + N)
    q, s = g.quantize_tensor(torch.randn(N, K, generator=gen, device=dev) * 0.02, 8)
    s = s.reshape(-1).contiguous()
    x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
    ws = None
    if M >= 128:
        n_ws = int(L.tiq_gemm_w8_workspace(_lib.BF16, M, K, N))
        ws = torch.empty(max(n_ws, 1), dtype=torch.uint8, device=dev)
    y_ref = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    _linear(L, x, q, s, N, y_ref, ws)
    buf = torch.zeros(1 << 20, dtype=torch.int64, device=dev)
    assert L.tiq_stamp_begin(buf.data_ptr(), buf.numel()) == 0
    try:
        y1 = torch.empty_like(y_ref)
        y2 = torch.empty_like(y_ref)
        _linear(L, x, q, s, N, y1, ws)
        _linear(L, x, q, s, N, y2, ws)
    finally:
        launches = _end(L)
    torch.cuda.synchronize()
    assert torch.equal(y1, y_ref) and torch.equal(y2, y_ref)
    assert len(launches) == 2, launches
    (f0, g0), (f1, g1) = launches
    assert f0 == 0 and g0 > 0 and f1 == 4 * g0 and g1 == g0
    t = buf[: 4 * (g0 + g1)].view(-1, 4).cpu()
    assert bool((t[:, 0] > 0).all()) and bool((t[:, 1] >= t[:, 0]).all())
    assert bool((t[:, 3] >= t[:, 2]).all())
    span = int(t[:, 1].max() - t[:, 0].min())  # 10 ns ticks: both launches within 10 ms
    assert 0 < span < 1_000_000
    # shader cycles over real time: a clock between 0.3 and 3 GHz
    ghz = float((t[:, 3] - t[:, 2]).sum()) / float((t[:, 1] - t[:, 0]).sum() * 10)
    assert 0.3 < ghz < 3.0, ghz
    assert int(buf[4 * (g0 + g1):].abs().sum()) == 0  # nothing past the handed-out slots
    # stamping off: no slots handed out, the product kernel again
    y3 = torch.empty_like(y_ref)
    _linear(L, x, q, s, N, y3, ws)
    assert _end(L) == []
    torch.cuda.synchronize()
    assert torch.equal(y3, y_ref)


def test_stamp_buffer_full_runs_unstamped(dev):
    """A launch that would pass the buffer's end runs the product kernel and
    takes no slots."""
    L = _lib.lib()
    M, K, N = 1, 768, 768
    q, s = g.quantize_tensor(torch.randn(N, K, device=dev) * 0.02, 8)
    s = s.reshape(-1).contiguous()
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    buf = torch.zeros(4 * N - 4, dtype=torch.int64, device=dev)  # one workgroup short
    assert L.tiq_stamp_begin(buf.data_ptr(), buf.numel()) == 0
    _linear(L, x, q, s, N, y)
    assert _end(L) == []
    torch.cuda.synchronize()
    assert int(buf.abs().sum()) == 0
    assert L.tiq_stamp_begin(None, 5) == _lib.EINVAL
