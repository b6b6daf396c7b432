"""Quantized linear kernels on the GPU against dequantize-then-fp32-matmul.

Contract: ``max|y - y_ref| <= 1e-3 * max|y_ref|`` with ``y_ref =
F.linear(x.float(), q.float() * scale, b)`` computed by the oracle on the CPU
from the same seeded inputs. Kernels write fp32 or bf16; a bf16 result must be
exactly the round-to-nearest-even of the fp32 result the same kernel computes
(so its only extra error is the storage rounding), and the fp32 result is held
to the 1e-3 bound. Entry points are called through the C ABI.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpt2_harness_amd import _lib
from oracle import linear as OL
from oracle import quant as OQ

pytestmark = pytest.mark.gpu

SMALL = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]   # (K, N) as in K x N
XL = [(1600, 4800), (1600, 1600), (1600, 6400), (6400, 1600)]
TOL = 1e-3


def _inputs(K, N, M, seed, x_dtype=torch.float32, bias=True):
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=gen) * 0.02
    x = torch.randn(M, K, generator=gen).to(x_dtype)
    b = torch.randn(N, generator=gen) * 0.1 if bias else None
    return w, x, b


def _call(entry, x, q, scale, b, N, y, *extra):
    L = _lib.lib()
    fn = getattr(L, entry)
    M, K = x.shape
    xd, yd = _lib.dtype_code(x.dtype), _lib.dtype_code(y.dtype)
    st = torch.cuda.current_stream().cuda_stream
    bp = None if b is None else b.data_ptr()
    if entry == "tiq_linear_w4g":
        group = extra[0]
        rc = fn(x.data_ptr(), xd, M, K, x.stride(0), q.data_ptr(), scale.data_ptr(), group, bp, N, y.data_ptr(), yd,
                y.stride(0), st)
    elif entry == "tiq_gemm_w8_tile":
        rc = fn(x.data_ptr(), xd, M, K, x.stride(0), q.data_ptr(), scale.data_ptr(), bp, N, y.data_ptr(), yd,
                y.stride(0), extra[0], st)
    else:
        rc = fn(x.data_ptr(), xd, M, K, x.stride(0), q.data_ptr(), scale.data_ptr(), bp, N, y.data_ptr(), yd,
                y.stride(0), st)
    _lib.check(rc, entry)
    torch.cuda.synchronize()


def _run_w8(entry, dev, c_oracle, K, N, M, x_dtype, seed=0, bias=True, *extra):
    w, x, b = _inputs(K, N, M, seed, x_dtype, bias)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    qd, sd = torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev)
    bd = None if b is None else b.to(dev)
    xd = x.to(dev)
    y32 = torch.empty(M, N, device=dev)
    ybf = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    _call(entry, xd, qd, sd, bd, N, y32, *extra)
    _call(entry, xd, qd, sd, bd, N, ybf, *extra)
    y_ref = OL.linear_ref(x, OL.dequantize(q, s), b)
    ok, err, bound = OL.within_tolerance(y32, y_ref, TOL)
    assert ok, f"{entry} M={M} K={K} N={N} {x_dtype}: max err {err:.3g} > {bound:.3g}"
    assert torch.equal(ybf.cpu(), y32.cpu().to(torch.bfloat16)), "bf16 output is not RNE of the fp32 output"


@pytest.mark.parametrize("KN", SMALL + XL)
@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_gemv_w8(dev, c_oracle, KN, M, x_dtype):
    _run_w8("tiq_gemv_w8", dev, c_oracle, *KN, M, x_dtype, seed=M)


@pytest.mark.parametrize("M", [2, 3, 5, 7, 8, 33])
def test_gemv_w8_odd_batches(dev, c_oracle, M):
    _run_w8("tiq_gemv_w8", dev, c_oracle, 768, 2304, M, torch.float32, seed=M, bias=M % 2 == 0)


@pytest.mark.parametrize("KN", XL)
@pytest.mark.parametrize("M", [256, 300])
def test_gemm_w8(dev, c_oracle, KN, M):
    _run_w8("tiq_gemm_w8", dev, c_oracle, *KN, M, torch.bfloat16, seed=M)


@pytest.mark.parametrize("KN", [(768, 2304), (3072, 768)])
@pytest.mark.parametrize("M", [16, 17, 64, 1024])
def test_gemm_w8_small_shapes(dev, c_oracle, KN, M):
    _run_w8("tiq_gemm_w8", dev, c_oracle, *KN, M, torch.bfloat16, seed=M, bias=False)


# Every GEMM tile configuration through tiq_gemm_w8_tile (10/11/12 the
# register-staged int8 kernel at 256x256 / 256x128 / 128x128 tiles, 13/14/15
# the same kernel with its wavefronts side by side along N at 224x256 /
# 160x256 / 224x128 (bf16 output; 128x128 for fp32 output), 16 its 128x128
# tile with four register staging sets, 17 128x128 side by side along N (bf16
# output), 1-4 the LDS-dequant kernel that also serves int4), on full,
# partial-row and partial-column tiles.
@pytest.mark.parametrize("tile", [10, 11, 12, 13, 14, 15, 16, 17, 1, 2, 3, 4])
@pytest.mark.parametrize("K,N,M", [(1600, 1600, 512), (1600, 4800, 300), (6400, 1600, 257), (768, 2304, 1024),
                                   (1600, 6400, 4096)])
def test_gemm_w8_tiles(dev, c_oracle, tile, K, N, M):
    _run_w8("tiq_gemm_w8_tile", dev, c_oracle, K, N, M, torch.bfloat16, tile + M, M % 2 == 0, tile)


def test_gemm_w8_tile_rejects_unknown_configuration(dev):
    L = _lib.lib()
    x = torch.zeros(256, 64, device=dev, dtype=torch.bfloat16)
    q = torch.zeros(64, 64, device=dev, dtype=torch.int8)
    s = torch.ones(64, device=dev)
    y = torch.empty(256, 64, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    for bad in (-1, 5, 9, 18):
        assert L.tiq_gemm_w8_tile(x.data_ptr(), 1, 256, 64, 64, q.data_ptr(), s.data_ptr(), None, 64, y.data_ptr(),
                                  0, 64, bad, st) == -1


# The prefill dispatch at its thresholds, through tiq_gemm_w8_ws with a
# workspace and tiq_gemm_w8 without: 47 / 48 tiles of 128 x 128 with a short
# K (split / unsplit on the side-by-side tile), 256 / 272 tiles (one round on
# the side-by-side tile / the cost model), 32 / 33 k64 steps (side-by-side /
# four staging sets), and 26 tiles at K = 6400 (split over 8). Every result
# within the oracle's bound, the bf16 output the rounding of the fp32 one, and
# the unsplit products of both entry points bit-identical.
@pytest.mark.parametrize("K,N,M", [(1600, 47 * 128, 128), (1600, 2048, 384), (1600, 2048, 2048), (1600, 2048, 2049),
                                   (2048, 1024, 256), (2112, 1024, 256), (6400, 1600, 256)])
def test_gemm_dispatch_thresholds(dev, c_oracle, K, N, M):
    L = _lib.lib()
    w, x, b = _inputs(K, N, M, M + N + K, torch.bfloat16)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    qd, sd, bd, xd = torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev), x.to(dev)
    n_ws = int(L.tiq_gemm_w8_workspace(_lib.BF16, M, K, N))
    ws = torch.empty(max(n_ws, 16), dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    outs = {}
    for with_ws in (True, False):
        for dt in (torch.float32, torch.bfloat16):
            y = torch.full((M, N), float("nan"), device=dev).to(dt)
            if with_ws:
                rc = L.tiq_gemm_w8_ws(xd.data_ptr(), _lib.BF16, M, K, K, qd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
                                      N, y.data_ptr(), _lib.dtype_code(dt), N, ws.data_ptr(), n_ws, st)
            else:
                rc = L.tiq_gemm_w8(xd.data_ptr(), _lib.BF16, M, K, K, qd.data_ptr(), sd.data_ptr(), bd.data_ptr(), N,
                                   y.data_ptr(), _lib.dtype_code(dt), N, st)
            _lib.check(rc, "gemm")
            outs[(with_ws, dt)] = y
    torch.cuda.synchronize()
    y_ref = OL.linear_ref(x, OL.dequantize(q, s), b)
    for with_ws in (True, False):
        y32 = outs[(with_ws, torch.float32)].cpu()
        ok, err, bound = OL.within_tolerance(y32, y_ref, TOL)
        assert ok, (with_ws, err, bound)
        assert torch.equal(outs[(with_ws, torch.bfloat16)].cpu(), y32.to(torch.bfloat16))
    tiles = ((M + 127) // 128) * ((N + 127) // 128)
    split = tiles * 2 < 512 and not (tiles >= 48 and K // 64 <= 32)
    if not split:  # the same unsplit kernel both ways
        assert torch.equal(outs[(True, torch.float32)].cpu(), outs[(False, torch.float32)].cpu())


# The 128x128 tile with four staging sets, and the one with its wavefronts
# side by side along N (bf16 output), sum the same products in the same order
# as the two-set 2 x 2 one: bit-identical outputs, fp32 and bf16, with a bias,
# for k-step counts that leave every remainder of the four-step loop (25, 12,
# 3, 1, 5 steps), partial tiles, and both fp32-output and bf16-output copies.
@pytest.mark.parametrize("K,N,M", [(1600, 1600, 256), (768, 2304, 1024), (192, 640, 200), (64, 256, 130),
                                   (320, 4800, 300)])
def test_gemm_w8_deep_staging_bit_identical(dev, K, N, M):
    L = _lib.lib()
    g = torch.Generator(device=dev).manual_seed(K + N + M)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    q = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    s = torch.rand(N, generator=g, device=dev) * 1e-3 + 1e-4
    b = torch.randn(N, generator=g, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    for ydt in (torch.float32, torch.bfloat16):
        ys = []
        for tile in (12, 16, 17):
            y = torch.full((M, N), float("nan"), device=dev).to(ydt)
            rc = L.tiq_gemm_w8_tile(x.data_ptr(), 1, M, K, K, q.data_ptr(), s.data_ptr(), b.data_ptr(), N,
                                    y.data_ptr(), _lib.dtype_code(ydt), N, tile, st)
            _lib.check(rc, f"tile {tile}")
            ys.append(y)
        torch.cuda.synchronize()
        assert not torch.isnan(ys[0].float()).any()
        iv = torch.int16 if ydt == torch.bfloat16 else torch.int32
        assert torch.equal(ys[0].cpu().view(iv), ys[1].cpu().view(iv))
        assert torch.equal(ys[0].cpu().view(iv), ys[2].cpu().view(iv))


# fp32 activations through the matrix cores (three exact bf16 planes): the
# contract bound, and fp32-level accuracy -- against a float64 product, the
# error is within a small factor of the fp32 oracle's own error (both differ
# from the exact result only by fp32 accumulation order).
@pytest.mark.parametrize("K,N,M", [(1600, 4800, 256), (6400, 1600, 300), (768, 3072, 1024), (3072, 768, 129)])
def test_linear_w8_fp32_matrix_cores(dev, c_oracle, K, N, M):
    L = _lib.lib()
    w, x, b = _inputs(K, N, M, seed=M + K)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    qd, sd = torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev)
    xd, bd = x.to(dev), b.to(dev)
    ws_bytes = int(L.tiq_linear_w8_workspace(_lib.F32, M, K))
    assert ws_bytes >= M * 3 * K * 2
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    y = torch.empty(M, N, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    # too small a workspace is refused before any work
    rc = L.tiq_linear_w8_ws(xd.data_ptr(), _lib.F32, M, K, K, qd.data_ptr(), sd.data_ptr(), bd.data_ptr(), N,
                            y.data_ptr(), _lib.F32, N, ws.data_ptr(), ws_bytes - 256, st)
    assert rc == -5
    _lib.check(L.tiq_linear_w8_ws(xd.data_ptr(), _lib.F32, M, K, K, qd.data_ptr(), sd.data_ptr(), bd.data_ptr(), N,
                                  y.data_ptr(), _lib.F32, N, ws.data_ptr(), ws_bytes, st), "tiq_linear_w8_ws")
    torch.cuda.synchronize()
    y_ref = OL.linear_ref(x, OL.dequantize(q, s), b)
    ok, err, bound = OL.within_tolerance(y, y_ref, TOL)
    assert ok, f"max err {err:.3g} > {bound:.3g}"
    w_hat = OL.dequantize(q, s)
    y64 = x.double() @ w_hat.double().T + b.double()
    err_gpu = float((y.cpu().double() - y64).abs().max())
    err_cpu = float((y_ref.double() - y64).abs().max())
    floor = 2.0 ** -24 * float(y64.abs().max())
    assert err_gpu <= 8 * max(err_cpu, floor), f"error {err_gpu:.3g} vs fp32 oracle {err_cpu:.3g}"


# bf16 activations at 4..16 rows take the 16-row matrix-core GEMV (9..16 rows
# on matrices under 1200 rows; fewer rows there stay on the direct GEMV), at
# 17..64 rows the batched matrix-core kernel (one bf16 plane: every int8 x bf16
# product is exact, fp32 accumulation); K beyond its register budget (6400)
# takes the GEMV. Besides the 1e-3 contract, the fp32 result is held to a
# small multiple of torch fp32's own error against a float64 computation of
# the same product.
@pytest.mark.parametrize("KN", SMALL + [(1600, 4800), (6400, 1600)])
@pytest.mark.parametrize("M", [5, 16, 33, 64])
def test_linear_w8_bf16_batched(dev, c_oracle, KN, M):
    K, N = KN
    _run_w8("tiq_linear_w8", dev, c_oracle, K, N, M, torch.bfloat16, seed=M + K, bias=M != 33)
    w, x, b = _inputs(K, N, M, M + K, torch.bfloat16, bias=M != 33)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    y = torch.empty(M, N, device=dev)
    bd = None if b is None else b.to(dev)
    _call("tiq_linear_w8", x.to(dev), torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), bd, N, y)
    w_hat = OL.dequantize(q, s)
    ref32 = OL.linear_ref(x, w_hat, b)
    ref64 = x.double() @ w_hat.double().T + (0 if b is None else b.double())
    err = float((y.cpu().double() - ref64).abs().max())
    err32 = float((ref32.double() - ref64).abs().max())
    assert err <= 8 * max(err32, 2.0 ** -24 * float(ref64.abs().max())), (err, err32)


# The 16-row matrix-core GEMV at its edges: weight-row blocks of 16, 8 and 4
# (N >= 2048, >= 1200, smaller) with a partial last block, K of one 64-column
# pair (4 wavefronts, three of them idle) up to 100 pairs (16 wavefronts of 7),
# runs that leave the last wavefronts without pairs (K = 1600: 25 pairs over
# 16 wavefronts of 2), 4 / 9 / 16 rows, fp32 and bf16 output.
@pytest.mark.parametrize("K,N", [(64, 40), (768, 1212), (1600, 2056), (3072, 1200), (6400, 768), (4160, 2048)])
@pytest.mark.parametrize("M", [4, 9, 16])
def test_rows16_edges(dev, c_oracle, K, N, M):
    _run_w8("tiq_linear_w8", dev, c_oracle, K, N, M, torch.bfloat16, seed=K + N + M, bias=M != 9)


@pytest.mark.parametrize("M,K,N", [(12, 768, 1212), (16, 1600, 4800), (4, 6400, 1600)])
def test_rows16_gelu_and_residual_in_place(dev, c_oracle, M, K, N):
    """GELU epilogue, then a residual added in place (y aliases it), bf16 rows."""
    L = _lib.lib()
    w, x, b = _inputs(K, N, M, M * 7 + K, torch.bfloat16)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    qd, sd, bd, xd = torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev), x.to(dev)
    st = torch.cuda.current_stream().cuda_stream
    w_hat = OL.dequantize(q, s)
    lin = OL.linear_ref(x, w_hat, b)
    y = torch.empty(M, N, device=dev)
    rc = L.tiq_linear_fused(xd.data_ptr(), 1, M, K, K, qd.data_ptr(), _lib.WF_INT8, sd.data_ptr(), None, 0,
                            bd.data_ptr(), N, y.data_ptr(), 0, N, None, None, 1e-5, 1, None, 0, st)
    _lib.check(rc, "rows16 gelu")
    torch.cuda.synchronize()
    gelu = 0.5 * lin * (1 + torch.tanh(0.7978845608028654 * (lin + 0.044715 * lin ** 3)))
    ok, err, bound = OL.within_tolerance(y, gelu, TOL)
    assert ok, (err, bound)
    r0 = torch.randn(M, N, generator=torch.Generator().manual_seed(M))
    yr = r0.to(dev)
    rc = L.tiq_linear_fused(xd.data_ptr(), 1, M, K, K, qd.data_ptr(), _lib.WF_INT8, sd.data_ptr(), None, 0,
                            bd.data_ptr(), N, yr.data_ptr(), 0, N, None, None, 1e-5, 0, yr.data_ptr(), N, st)
    _lib.check(rc, "rows16 residual")
    torch.cuda.synchronize()
    ok, err, bound = OL.within_tolerance(yr, r0 + lin, TOL)
    assert ok, (err, bound)


@pytest.mark.parametrize("pad", [64, 4])
def test_linear_w8_bf16_strided_rows(dev, c_oracle, pad):
    """Row stride K + 64 (16-byte rows: the 16-row matrix-core GEMV) and K + 4
    (8-byte rows: the GEMV), strided output; nothing written outside the
    outputs."""
    K, N, M = 768, 2304, 16
    w, x, b = _inputs(K, N, M, pad, torch.bfloat16)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    xs = torch.zeros(M, K + pad, device=dev, dtype=torch.bfloat16)
    xs[:, :K] = x.to(dev)
    ys = torch.full((M, N + 32), 7.0, device=dev)
    _call("tiq_linear_w8", xs[:, :K], torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev),
          b.to(dev), N, ys[:, :N])
    ok, err, bound = OL.within_tolerance(ys[:, :N], OL.linear_ref(x, OL.dequantize(q, s), b))
    assert ok, (err, bound)
    assert torch.all(ys[:, N:] == 7.0), "kernel wrote outside its output rows"


# Products with few output tiles split K over workgroups (fp32 partial slices
# in the workspace, summed in a fixed order): bf16 rows through tiq_gemm_w8_ws,
# fp32 rows through tiq_linear_w8_ws with a workspace sized by
# tiq_gemm_w8_workspace (three bf16 planes, then the split product). Two
# calls in a row on one workspace, the second with fewer rows.
@pytest.mark.parametrize("K,N,M", [(6400, 1600, 256), (1600, 1600, 256), (1600, 4800, 300), (6400, 1600, 1024),
                                   (768, 2304, 128)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_gemm_split_k(dev, c_oracle, K, N, M, x_dtype):
    L = _lib.lib()
    xd = _lib.dtype_code(x_dtype)
    n_ws = int(L.tiq_gemm_w8_workspace(xd, M, K, N))
    assert n_ws > 0
    ws = torch.empty(n_ws, dtype=torch.uint8, device=dev)
    entry = "tiq_gemm_w8_ws" if x_dtype == torch.bfloat16 else "tiq_linear_w8_ws"
    for rows in (M, M - 37):
        w, x, b = _inputs(K, N, rows, rows + K, x_dtype)
        q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
        qd, sd, bd, xg = torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev), x.to(dev)
        y32 = torch.empty(rows, N, device=dev)
        ybf = torch.empty(rows, N, device=dev, dtype=torch.bfloat16)
        for y in (y32, ybf):
            rc = getattr(L, entry)(xg.data_ptr(), xd, rows, K, K, qd.data_ptr(), sd.data_ptr(), bd.data_ptr(), N,
                                   y.data_ptr(), _lib.dtype_code(y.dtype), N, ws.data_ptr(), n_ws,
                                   torch.cuda.current_stream().cuda_stream)
            _lib.check(rc, entry)
        torch.cuda.synchronize()
        w_hat = OL.dequantize(q, s)
        ok, err, bound = OL.within_tolerance(y32, OL.linear_ref(x, w_hat, b), TOL)
        assert ok, (rows, err, bound)
        assert torch.equal(ybf.cpu(), y32.cpu().to(torch.bfloat16))
        if x_dtype == torch.float32:   # the exact planes: fp32-accurate
            ref64 = x.double() @ w_hat.double().T + b.double()
            err = float((y32.cpu().double() - ref64).abs().max())
            err32 = float((OL.linear_ref(x, w_hat, b).double() - ref64).abs().max())
            assert err <= 8 * max(err32, 2.0 ** -24 * float(ref64.abs().max())), (err, err32)


# Full-size prefill products through the workspace entry points (bf16 rows
# and the fp32 three-plane path, including 400 tiles of 256 x 256 on 256 CUs):
# each product run twice, both runs bit-identical, and the bf16 output the
# rounding of the fp32 one.
@pytest.mark.parametrize("K,N,M,x_dtype", [(1600, 6400, 4096, torch.bfloat16), (6400, 1600, 4096, torch.bfloat16),
                                           (1600, 4800, 1024, torch.float32), (1600, 1600, 4096, torch.float32)])
def test_gemm_large_shapes_deterministic(dev, c_oracle, K, N, M, x_dtype):
    L = _lib.lib()
    xd = _lib.dtype_code(x_dtype)
    n_ws = int(L.tiq_gemm_w8_workspace(xd, M, K, N))
    ws = torch.empty(max(n_ws, 16), dtype=torch.uint8, device=dev)
    entry = "tiq_gemm_w8_ws" if x_dtype == torch.bfloat16 else "tiq_linear_w8_ws"
    for rows in (M, M - 37):
        w, x, b = _inputs(K, N, rows, rows + K + 1, x_dtype)
        q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
        qd, sd, bd, xg = torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev), x.to(dev)
        ys = [torch.full((rows, N), float("nan"), device=dev) for _ in range(2)]
        ybf = torch.empty(rows, N, device=dev, dtype=torch.bfloat16)
        for y in (*ys, ybf):
            rc = getattr(L, entry)(xg.data_ptr(), xd, rows, K, K, qd.data_ptr(), sd.data_ptr(), bd.data_ptr(), N,
                                   y.data_ptr(), _lib.dtype_code(y.dtype), N, ws.data_ptr(), n_ws,
                                   torch.cuda.current_stream().cuda_stream)
            _lib.check(rc, entry)
        torch.cuda.synchronize()
        y32 = ys[0].cpu()
        assert torch.isfinite(y32).all()
        assert torch.equal(y32, ys[1].cpu()), "results differ between two runs"
        assert torch.equal(ybf.cpu(), y32.to(torch.bfloat16))
        w_hat = OL.dequantize(q, s)
        ok, err, bound = OL.within_tolerance(y32, OL.linear_ref(x, w_hat, b), TOL)
        assert ok, (rows, err, bound)
        if x_dtype == torch.float32:   # the exact planes: fp32-accurate
            ref64 = x.double() @ w_hat.double().T + b.double()
            err = float((y32.double() - ref64).abs().max())
            err32 = float((OL.linear_ref(x, w_hat, b).double() - ref64).abs().max())
            assert err <= 8 * max(err32, 2.0 ** -24 * float(ref64.abs().max())), (err, err32)


@pytest.mark.parametrize("M", [1, 16, 64, 256])
def test_linear_w8_dispatch(dev, c_oracle, M):
    _run_w8("tiq_linear_w8", dev, c_oracle, 1600, 4800, M, torch.bfloat16, seed=M)
    _run_w8("tiq_linear_w8", dev, c_oracle, 1600, 4800, M, torch.float32, seed=M)


@pytest.mark.parametrize("K,N", [(100, 37), (24, 5), (1600, 1)])
def test_generic_fallback_shapes(dev, c_oracle, K, N):
    """K not a multiple of 16 (and N = 1): the scalar fallback kernel."""
    _run_w8("tiq_linear_w8", dev, c_oracle, K, N, 3, torch.float32, seed=K)


def test_strided_activations_and_outputs(dev, c_oracle):
    K, N, M = 768, 2304, 4
    w, x, b = _inputs(K, N, M, 5)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 8)
    xs = torch.zeros(M, K + 64, device=dev)
    xs[:, :K] = x.to(dev)
    ys = torch.full((M, N + 32), 7.0, device=dev)
    _call("tiq_linear_w8", xs[:, :K], torch.from_numpy(q).to(dev), torch.from_numpy(s.reshape(-1)).to(dev),
          b.to(dev), N, ys[:, :N])
    ok, err, bound = OL.within_tolerance(ys[:, :N], OL.linear_ref(x, OL.dequantize(q, s), b))
    assert ok, (err, bound)
    assert torch.all(ys[:, N:] == 7.0), "kernel wrote outside its output rows"


# int4 in the reference's nibble layout: the GEMV at decode sizes, the staged
# MFMA GEMM (nibbles staged into bf16 tiles) at prefill sizes, every XL shape
# at M = 4096 and partial tiles; bf16 output exactly the RNE of the fp32 one.
@pytest.mark.parametrize("KN,M", [((768, 2304), 1), ((768, 2304), 4), ((1600, 6400), 1), ((6400, 1600), 4),
                                  ((768, 2304), 256), ((1600, 6400), 256), ((6400, 1600), 300),
                                  ((1600, 4800), 4096), ((1600, 1600), 4096), ((1600, 6400), 4096),
                                  ((6400, 1600), 4096), ((3072, 768), 1000)])
def test_linear_w4_reference_layout(dev, c_oracle, KN, M):
    K, N = KN
    w, x, b = _inputs(K, N, M, M + K, torch.bfloat16 if M >= 16 else torch.float32)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 4)
    packed = torch.from_numpy(c_oracle.pack_int4(q)).to(dev)
    sd, bd, xd = torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev), x.to(dev)
    y = torch.empty(M, N, device=dev)
    _call("tiq_linear_w4", xd, packed, sd, bd, N, y)
    ok, err, bound = OL.within_tolerance(y, OL.linear_ref(x, OL.dequantize(q, s), b))
    assert ok, (err, bound)
    if M >= 16:
        ybf = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        _call("tiq_linear_w4", xd, packed, sd, bd, N, ybf)
        assert torch.equal(ybf.cpu(), y.cpu().to(torch.bfloat16)), "bf16 output is not RNE of the fp32 output"


# fp32 rows against reference-layout int4 codes at 16..127 rows (a short
# prompt's prefill) with the workspace of tiq_gemm_w8_workspace: the three
# exact bf16 planes on the matrix cores, split over K (M >= 32, or >= 16 on
# N >= 2048); without a workspace the same call takes the GEMV path. Both
# within the oracle's bound, the planes also within 8x torch fp32's own error
# against float64, and the two paths agree to that tolerance.
@pytest.mark.parametrize("K,N,M", [(768, 2304, 16), (768, 768, 16), (768, 768, 33), (3072, 768, 64),
                                   (768, 3072, 127), (1600, 6400, 40)])
def test_linear_w4_fp32_few_rows_planes(dev, c_oracle, K, N, M):
    L = _lib.lib()
    w, x, b = _inputs(K, N, M, M * 3 + K)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 4)
    packed = torch.from_numpy(c_oracle.pack_int4(q)).to(dev)
    sd, bd, xd = torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev), x.to(dev)
    n_ws = int(L.tiq_gemm_w8_workspace(_lib.F32, M, K, N))
    planes = M >= 32 or N >= 2048
    assert (n_ws > 0) == planes
    ws = torch.empty(max(n_ws, 16), dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    ys = []
    for wsp, nb in ((ws.data_ptr(), n_ws), (None, 0)):
        y = torch.full((M, N), float("nan"), device=dev)
        rc = L.tiq_linear_w4_ws(xd.data_ptr(), _lib.F32, M, K, K, packed.data_ptr(), sd.data_ptr(), bd.data_ptr(), N,
                                y.data_ptr(), _lib.F32, N, wsp, nb, st)
        _lib.check(rc, "tiq_linear_w4_ws")
        ys.append(y)
    torch.cuda.synchronize()
    w_hat = OL.dequantize(q, s)
    ref32 = OL.linear_ref(x, w_hat, b)
    ref64 = x.double() @ w_hat.double().T + b.double()
    err32 = float((ref32.double() - ref64).abs().max())
    for y in ys:
        ok, err, bound = OL.within_tolerance(y, ref32, TOL)
        assert ok, (M, err, bound)
    if planes:
        err = float((ys[0].cpu().double() - ref64).abs().max())
        assert err <= 8 * max(err32, 2.0 ** -24 * float(ref64.abs().max())), (err, err32)


# int4 in the reference's nibble layout with bf16 rows and the GEMM workspace:
# products with few 128 x 128 tiles split over K (6400x1600 at M = 256: 26
# tiles, eight splits), the fp32 slices summed in order, scaled and biased
# after; the oracle's bound, the bf16 output the rounding of the fp32 one.
@pytest.mark.parametrize("K,N,M", [(6400, 1600, 256), (1600, 4800, 300), (768, 2304, 129)])
def test_linear_w4_split_k(dev, c_oracle, K, N, M):
    L = _lib.lib()
    w, x, b = _inputs(K, N, M, M + K + 7, torch.bfloat16)
    q, s = c_oracle.quantize_per_channel(w.numpy(), 4)
    packed = torch.from_numpy(c_oracle.pack_int4(q)).to(dev)
    sd, bd, xd = torch.from_numpy(s.reshape(-1)).to(dev), b.to(dev), x.to(dev)
    n_ws = int(L.tiq_gemm_w8_workspace(_lib.BF16, M, K, N))
    assert n_ws > 0, "the shape should plan a split"
    ws = torch.empty(n_ws, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    outs = {}
    for dt in (torch.float32, torch.bfloat16):
        y = torch.full((M, N), 7.0, device=dev, dtype=dt)
        rc = L.tiq_linear_w4_ws(xd.data_ptr(), _lib.BF16, M, K, K, packed.data_ptr(), sd.data_ptr(), bd.data_ptr(),
                                N, y.data_ptr(), _lib.dtype_code(dt), N, ws.data_ptr(), n_ws, st)
        _lib.check(rc, "tiq_linear_w4_ws")
        torch.cuda.synchronize()
        outs[dt] = y.cpu()
    ok, err, bound = OL.within_tolerance(outs[torch.float32], OL.linear_ref(x, OL.dequantize(q, s), b))
    assert ok, f"w4 split M={M} K={K} N={N}: max err {err:.3g} > {bound:.3g}"
    assert torch.equal(outs[torch.bfloat16], outs[torch.float32].to(torch.bfloat16)), "bf16 not RNE of fp32"


@pytest.mark.parametrize("KN", [(768, 2304), (1600, 4800), (6400, 1600)])
@pytest.mark.parametrize("M", [1, 4, 64])
def test_linear_w4_groupwise(dev, c_oracle, KN, M):
    K, N = KN
    w, x, b = _inputs(K, N, M, M + 2 * K)
    packed, s16 = c_oracle.quantize_groupwise_int4(w.numpy(), 128)
    y = torch.empty(M, N, device=dev)
    _call("tiq_linear_w4g", x.to(dev), torch.from_numpy(packed).to(dev),
          torch.from_numpy(s16.view(np.uint16).copy()).to(dev), b.to(dev), N, y, 128)
    w_hat = torch.from_numpy(OQ.dequantize_groupwise_int4(packed, s16, K, 128))
    ok, err, bound = OL.within_tolerance(y, OL.linear_ref(x, w_hat, b))
    assert ok, (err, bound)


def _run_w4g(dev, c_oracle, K, N, M, group, seed, bias=True):
    w, x, b = _inputs(K, N, M, seed, torch.bfloat16, bias)
    packed, s16 = c_oracle.quantize_groupwise_int4(w.numpy(), group)
    pd, sd = torch.from_numpy(packed).to(dev), torch.from_numpy(s16.view(np.uint16).copy()).to(dev)
    bd, xd = (None if b is None else b.to(dev)), x.to(dev)
    y32 = torch.empty(M, N, device=dev)
    ybf = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    _call("tiq_linear_w4g", xd, pd, sd, bd, N, y32, group)
    _call("tiq_linear_w4g", xd, pd, sd, bd, N, ybf, group)
    w_hat = torch.from_numpy(OQ.dequantize_groupwise_int4(packed, s16, K, group))
    ok, err, bound = OL.within_tolerance(y32, OL.linear_ref(x, w_hat, b))
    assert ok, f"w4g M={M} K={K} N={N} group={group}: max err {err:.3g} > {bound:.3g}"
    assert torch.equal(ybf.cpu(), y32.cpu().to(torch.bfloat16)), "bf16 output is not RNE of the fp32 output"


# Group-wise int4 at prefill sizes: the MFMA GEMM with one fp32 partial per
# 128-column group, the group's fp16 scale applied to it (K = 1600: twelve
# groups and a ragged 64-column one; K = 6400: fifty groups).
@pytest.mark.parametrize("KN", XL)
@pytest.mark.parametrize("M", [256, 1024, 4096])
def test_gemm_w4_groupwise_prefill(dev, c_oracle, KN, M):
    _run_w4g(dev, c_oracle, *KN, M, 128, seed=M + KN[0], bias=M != 1024)


# Group-wise int4 at the dispatch thresholds (groups of 128, K = 1600): 128-row
# tiles while 128 x 128 tiles fit one round (M = 1024: 256 tiles at N = 4096,
# 264 at N = 4224 take 224-row tiles), without the workspace and with it,
# where 96 tiles or more run unsplit (M = 384: 96 at N = 4096) and 93 split
# (N = 3968). Within the oracle's bound, the bf16 output the rounding of the
# fp32 one.
@pytest.mark.parametrize("N,M", [(4096, 1024), (4224, 1024), (4096, 384), (3968, 384)])
def test_gemm_w4_groupwise_dispatch_thresholds(dev, c_oracle, N, M):
    K = 1600
    _run_w4g(dev, c_oracle, K, N, M, 128, seed=N + M)
    L = _lib.lib()
    w, x, b = _inputs(K, N, M, N + M + 1, torch.bfloat16)
    packed, s16 = c_oracle.quantize_groupwise_int4(w.numpy(), 128)
    pd, sd = torch.from_numpy(packed).to(dev), torch.from_numpy(s16.view(np.uint16).copy()).to(dev)
    n_ws = int(L.tiq_gemm_w8_workspace(_lib.BF16, M, K, N))
    ws = torch.empty(max(n_ws, 16), dtype=torch.uint8, device=dev)
    y = torch.empty(M, N, device=dev)
    rc = L.tiq_linear_w4g_ws(x.to(dev).data_ptr(), _lib.BF16, M, K, K, pd.data_ptr(), sd.data_ptr(), 128,
                             b.to(dev).data_ptr(), N, y.data_ptr(), _lib.F32, N, ws.data_ptr(), n_ws,
                             torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "tiq_linear_w4g_ws")
    torch.cuda.synchronize()
    w_hat = torch.from_numpy(OQ.dequantize_groupwise_int4(packed, s16, K, 128))
    ok, err, bound = OL.within_tolerance(y.cpu(), OL.linear_ref(x, w_hat, b))
    assert ok, (err, bound)


# Group-wise int4 with bf16 rows and the GEMM workspace: products with few
# 128 x 128 tiles split over K, whole groups a split, the fp32 slices summed in
# order (6400x1600 at M = 256: 26 tiles, eight splits of 6-7 groups; group
# widths of one, three and sixteen k steps; partial tiles; 128-row tiles for
# groups of 128 at M = 256 .. 512, 224-row ones at M = 129). The result is held
# to the oracle's bound, and the bf16 output to the rounding of the fp32 one.
@pytest.mark.parametrize("K,N,M,group", [(6400, 1600, 256, 128), (1600, 4800, 256, 128), (1600, 1600, 1024, 128),
                                         (6400, 1600, 1024, 128), (1600, 4800, 300, 128), (768, 2304, 129, 128),
                                         (1600, 4800, 300, 64), (1600, 1600, 257, 192),
                                         (3072, 768, 129, 1024), (768, 2304, 512, 128), (1600, 6400, 384, 128)])
def test_gemm_w4_groupwise_split_k(dev, c_oracle, K, N, M, group):
    L = _lib.lib()
    w, x, b = _inputs(K, N, M, M + group + K, torch.bfloat16)
    packed, s16 = c_oracle.quantize_groupwise_int4(w.numpy(), group)
    pd, sd = torch.from_numpy(packed).to(dev), torch.from_numpy(s16.view(np.uint16).copy()).to(dev)
    bd, xd = b.to(dev), x.to(dev)
    n_ws = int(L.tiq_gemm_w8_workspace(_lib.BF16, M, K, N))
    assert n_ws > 0, "the shape should plan a split"
    ws = torch.empty(n_ws, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    outs = {}
    for dt in (torch.float32, torch.bfloat16):
        y = torch.full((M, N), 7.0, device=dev, dtype=dt)
        rc = L.tiq_linear_w4g_ws(xd.data_ptr(), _lib.BF16, M, K, K, pd.data_ptr(), sd.data_ptr(), group, bd.data_ptr(),
                                 N, y.data_ptr(), _lib.dtype_code(dt), N, ws.data_ptr(), n_ws, st)
        _lib.check(rc, "tiq_linear_w4g_ws")
        torch.cuda.synchronize()
        outs[dt] = y.cpu()
    w_hat = torch.from_numpy(OQ.dequantize_groupwise_int4(packed, s16, K, group))
    ok, err, bound = OL.within_tolerance(outs[torch.float32], OL.linear_ref(x, w_hat, b))
    assert ok, f"w4g split M={M} K={K} N={N} group={group}: max err {err:.3g} > {bound:.3g}"
    assert torch.equal(outs[torch.bfloat16], outs[torch.float32].to(torch.bfloat16)), "bf16 not RNE of fp32"


# other group widths (multiples of the 64-column k step, a last group of one
# step), partial row and column tiles, and a width the GEMM does not take
# (32: the vector-ALU kernel serves it); groups of 128 at K of one half group,
# one group and one and a half (the staged kernel), and with N % 32 != 0 (the
# LDS-dequant kernel takes it)
@pytest.mark.parametrize("K,N,M,group", [(1600, 4800, 300, 64), (1600, 1600, 257, 192), (768, 2304, 513, 256),
                                         (3072, 768, 129, 1024), (1600, 1000, 256, 32), (6400, 1600, 384, 6400),
                                         (64, 256, 130, 128), (128, 512, 224, 128), (192, 512, 200, 128),
                                         (1600, 1000, 256, 128)])
def test_gemm_w4_groupwise_widths_and_partial_tiles(dev, c_oracle, K, N, M, group):
    _run_w4g(dev, c_oracle, K, N, M, group, seed=M + group)


# fp32 activations with int4 weights (reference nibbles, group-wise g128) at
# prefill sizes: three exact bf16 planes through the LDS-dequant MFMA GEMM
# (the weight read at column k % K), the contract bound and fp32-level
# accuracy against float64 as for int8.
@pytest.mark.parametrize("fmt", ["int4", "int4_g128"])
@pytest.mark.parametrize("K,N,M", [(1600, 4800, 256), (6400, 1600, 300), (1600, 1600, 4096), (768, 3072, 128)])
def test_linear_w4_fp32_matrix_cores(dev, c_oracle, fmt, K, N, M):
    L = _lib.lib()
    w, x, b = _inputs(K, N, M, seed=M + K + 7)
    if fmt == "int4":
        q, s = c_oracle.quantize_per_channel(w.numpy(), 4)
        w_hat = OL.dequantize(q, s)
        codes, sc = torch.from_numpy(c_oracle.pack_int4(q)).to(dev), torch.from_numpy(s.reshape(-1)).to(dev)
    else:
        packed, s16 = c_oracle.quantize_groupwise_int4(w.numpy(), 128)
        w_hat = torch.from_numpy(OQ.dequantize_groupwise_int4(packed, s16, K, 128))
        codes, sc = torch.from_numpy(packed).to(dev), torch.from_numpy(s16.view(np.uint16).copy()).to(dev)
    xd, bd = x.to(dev), b.to(dev)
    ws_bytes = int(L.tiq_linear_w8_workspace(_lib.F32, M, K))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    y = torch.empty(M, N, device=dev)
    st = torch.cuda.current_stream().cuda_stream

    def call(nbytes):
        if fmt == "int4":
            return L.tiq_linear_w4_ws(xd.data_ptr(), _lib.F32, M, K, K, codes.data_ptr(), sc.data_ptr(),
                                      bd.data_ptr(), N, y.data_ptr(), _lib.F32, N, ws.data_ptr(), nbytes, st)
        return L.tiq_linear_w4g_ws(xd.data_ptr(), _lib.F32, M, K, K, codes.data_ptr(), sc.data_ptr(), 128,
                                   bd.data_ptr(), N, y.data_ptr(), _lib.F32, N, ws.data_ptr(), nbytes, st)

    assert call(ws_bytes - 256) == -5  # too small a workspace is refused before any work
    _lib.check(call(ws_bytes), f"tiq_linear_{fmt}_ws")
    torch.cuda.synchronize()
    y_ref = OL.linear_ref(x, w_hat, b)
    ok, err, bound = OL.within_tolerance(y, y_ref, TOL)
    assert ok, f"max err {err:.3g} > {bound:.3g}"
    y64 = x.double() @ w_hat.double().T + b.double()
    err_gpu = float((y.cpu().double() - y64).abs().max())
    err_cpu = float((y_ref.double() - y64).abs().max())
    floor = 2.0 ** -24 * float(y64.abs().max())
    assert err_gpu <= 8 * max(err_cpu, floor), f"error {err_gpu:.3g} vs fp32 oracle {err_cpu:.3g}"


def test_zero_rows_is_a_no_op(dev):
    L = _lib.lib()
    y = torch.full((1, 4), 3.0, device=dev)
    x = torch.zeros(1, 16, device=dev)
    q = torch.zeros(4, 16, dtype=torch.int8, device=dev)
    s = torch.ones(4, device=dev)
    rc = L.tiq_linear_w8(x.data_ptr(), 0, 0, 16, 16, q.data_ptr(), s.data_ptr(), None, 4, y.data_ptr(), 0, 4,
                         torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert torch.all(y == 3.0)


def test_bad_arguments_are_rejected(dev):
    L = _lib.lib()
    x = torch.zeros(2, 16, device=dev)
    q = torch.zeros(4, 16, dtype=torch.int8, device=dev)
    s = torch.ones(4, device=dev)
    y = torch.zeros(2, 4, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    # ldx smaller than K, bad dtype code, null weight pointer
    assert L.tiq_linear_w8(x.data_ptr(), 0, 2, 16, 8, q.data_ptr(), s.data_ptr(), None, 4, y.data_ptr(), 0, 4, st) == -1
    assert L.tiq_linear_w8(x.data_ptr(), 7, 2, 16, 16, q.data_ptr(), s.data_ptr(), None, 4, y.data_ptr(), 0, 4, st) == -1
    assert L.tiq_linear_w8(x.data_ptr(), 0, 2, 16, 16, None, s.data_ptr(), None, 4, y.data_ptr(), 0, 4, st) == -1
    # fp32 activations have no MFMA kernel: the explicit GEMM entry refuses them
    assert L.tiq_gemm_w8(x.data_ptr(), 0, 2, 16, 16, q.data_ptr(), s.data_ptr(), None, 4, y.data_ptr(), 0, 4, st) == -4
