"""Quantize / pack kernels on the GPU against the oracle: bit-exact.

Inputs are seeded on the CPU and copied to the device, so the kernel and the
oracle see the same bits. Shapes: the closed-form known-answer rows, GPT-2
small and GPT-2-XL Linear shapes with 0.1% outliers x20, odd / unaligned /
one-column / empty cases, and bit widths 2..8.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gpt2_harness_amd as g
from oracle import quant as OQ

pytestmark = pytest.mark.gpu

XL_SHAPES = [(4800, 1600), (1600, 1600), (6400, 1600), (1600, 6400)]  # (N, K) = (out, in)
SMALL_SHAPES = [(2304, 768), (768, 768), (3072, 768), (768, 3072)]


def weight(n: int, k: int, seed: int, outliers: float = 0.001) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=gen) * 0.02
    if outliers:
        idx = torch.randperm(n * k, generator=gen)[: max(1, int(outliers * n * k))]
        w.view(-1)[idx] *= 20.0
    return w


def _f32(bits) -> torch.Tensor:
    return torch.from_numpy(np.asarray(bits, dtype=np.uint32).view(np.float32).copy())


def _assert_codes(q_dev, s_dev, q_ref, s_ref):
    q = q_dev.cpu().numpy()
    s = s_dev.cpu().numpy().astype(np.float32)
    assert q.shape == q_ref.shape, (q.shape, q_ref.shape)
    bad = np.argwhere(q != q_ref)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[:3].tolist()}"
    assert np.array_equal(s.reshape(-1).view(np.uint32), s_ref.reshape(-1).view(np.uint32)), "scales differ"


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_known_answers_per_channel(known_answers, dev, bits):
    w = _f32(known_answers["input_bits"]).to(dev)
    exp = known_answers["per_channel"][str(bits)]
    q, s = g.quantize_tensor(w, bits)
    assert q.cpu().tolist() == exp["codes"]
    assert s.cpu().numpy().reshape(-1).view(np.uint32).tolist() == exp["scale_bits"]


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_known_answers_per_tensor(known_answers, dev, bits):
    w = _f32(known_answers["input_bits"]).to(dev)
    exp = known_answers["per_tensor"][str(bits)]
    q, s = g.quantize_tensor(w, bits, "per_tensor")
    assert q.reshape(-1).cpu().tolist() == exp["codes"]
    assert int(s.cpu().numpy().view(np.uint32)) == exp["scale_bits"] and s.shape == ()


def test_known_answers_one_column_and_groupwise(known_answers, dev):
    oc = known_answers["one_column"]
    q, s = g.quantize_tensor(_f32(oc["input_bits"]).to(dev), 8)
    assert q.cpu().tolist() == oc["codes"]
    assert s.cpu().numpy().reshape(-1).view(np.uint32).tolist() == oc["scale_bits"]
    gk = known_answers["groupwise_int4"]
    p, s16 = g.quantize_groupwise_int4(_f32(gk["input_bits"]).to(dev), gk["group"])
    assert p.cpu().tolist() == gk["packed"]
    assert s16.cpu().numpy().view(np.uint16).tolist() == gk["scale_f16_bits"]


@pytest.mark.parametrize("shape", XL_SHAPES + SMALL_SHAPES)
def test_int8_per_channel_bit_exact(dev, c_oracle, shape):
    w = weight(*shape, seed=shape[0] + shape[1])
    q, s = g.quantize_tensor(w.to(dev), 8)
    _assert_codes(q, s, *c_oracle.quantize_per_channel(w.numpy(), 8))


@pytest.mark.parametrize("shape", [(4800, 1600), (1600, 6400)])
@pytest.mark.parametrize("bits", [7, 5, 4, 3, 2])
def test_low_bit_per_channel_bit_exact(dev, c_oracle, shape, bits):
    w = weight(*shape, seed=bits)
    q, s = g.quantize_tensor(w.to(dev), bits)
    _assert_codes(q, s, *c_oracle.quantize_per_channel(w.numpy(), bits))


@pytest.mark.parametrize("shape", [(1600, 6400), (768, 768), (3, 5), (1, 1)])
@pytest.mark.parametrize("bits", [8, 4])
def test_per_tensor_bit_exact(dev, c_oracle, shape, bits):
    w = weight(*shape, seed=11)
    q, s = g.quantize_tensor(w.to(dev), bits, "per_tensor")
    _assert_codes(q, s, *c_oracle.quantize_per_tensor(w.numpy(), bits))


@pytest.mark.parametrize("shape", [(37, 9), (5, 1), (3, 10000), (129, 130)])
def test_generic_shapes_bit_exact(dev, c_oracle, shape):
    """Shapes off the vector path: odd columns, one column, rows longer than
    the register-resident limit, columns not a multiple of four."""
    w = weight(*shape, seed=5, outliers=0.01)
    q, s = g.quantize_tensor(w.to(dev), 8)
    _assert_codes(q, s, *c_oracle.quantize_per_channel(w.numpy(), 8))


def test_unaligned_view_bit_exact(dev, c_oracle):
    """A weight that starts 4 bytes past an allocation boundary (not 16-byte aligned)."""
    flat = weight(65, 257, seed=9).reshape(-1).to(dev)
    view = flat[1 : 1 + 64 * 256].view(64, 256)
    q, s = g.quantize_tensor(view, 8)
    _assert_codes(q, s, *c_oracle.quantize_per_channel(view.cpu().numpy(), 8))


def test_zero_and_subnormal_rows(dev, c_oracle):
    w = weight(8, 256, seed=2)
    w[1] = 0.0
    w[2] = torch.full((256,), 1e-40)
    w[3, :] = 0.0
    w[3, 5] = 8.5 * 2.0**-126
    q, s = g.quantize_tensor(w.to(dev), 8)
    _assert_codes(q, s, *c_oracle.quantize_per_channel(w.numpy(), 8))
    out = g.quantize_dequantize(w.to(dev), 8).cpu()
    assert torch.all(out[1] == 0) and torch.isfinite(out).all()


@pytest.mark.parametrize("shape", XL_SHAPES + [(7, 6), (5, 5), (3, 4)])
def test_int4_fused_packed_matches_pack_of_codes(dev, c_oracle, shape):
    """The fused quantize+pack path (QuantLinear storage) equals
    pack_int4(quantize_tensor(w, 4)) of the oracle, byte for byte."""
    w = weight(*shape, seed=3)
    lin = torch.nn.Linear(shape[1], shape[0]).to(dev)
    with torch.no_grad():
        lin.weight.copy_(w)
    mod, (q, s) = g.quantize_linear(lin, 4)
    q_ref, s_ref = c_oracle.quantize_per_channel(w.numpy(), 4)
    _assert_codes(q, s, q_ref, s_ref)
    if shape[1] % 2 == 0:
        assert mod.fmt == "int4"
        assert np.array_equal(mod.codes.cpu().numpy(), c_oracle.pack_int4(q_ref))
    else:
        assert mod.fmt == "int8"


@pytest.mark.parametrize("shape", [(7, 6), (5, 5), (1,), (3,), (4800, 1600)])
def test_pack_unpack_round_trip(dev, c_oracle, shape):
    gen = torch.Generator().manual_seed(0)
    q = torch.randint(-8, 8, shape, dtype=torch.int8, generator=gen)
    p = g.pack_int4(q.to(dev))
    assert p.dtype == torch.uint8 and p.numel() == (q.numel() + 1) // 2
    assert np.array_equal(p.cpu().numpy(), c_oracle.pack_int4(q.numpy()))
    assert torch.equal(g.unpack_int4(p, q.numel()).view(shape).cpu(), q)


def test_full_code_range(dev):
    q = torch.arange(-8, 8, dtype=torch.int8)
    p = g.pack_int4(q.to(dev))
    assert [hex(b) for b in p.cpu().tolist()] == ["0x10", "0x32", "0x54", "0x76", "0x98", "0xba", "0xdc", "0xfe"]
    assert torch.equal(g.unpack_int4(p, 16).cpu(), q)


@pytest.mark.parametrize("shape", XL_SHAPES + [(64, 200), (3, 130), (5, 7)])
def test_groupwise_int4_bit_exact(dev, c_oracle, shape):
    w = weight(*shape, seed=21)
    w[0, :] = 0.0  # zero groups store the smallest positive fp16
    p, s16 = g.quantize_groupwise_int4(w.to(dev), 128)
    p_ref, s_ref = c_oracle.quantize_groupwise_int4(w.numpy(), 128)
    assert np.array_equal(s16.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(p.cpu().numpy(), p_ref)


@pytest.mark.parametrize("group", [32, 64, 2])
def test_groupwise_other_group_sizes(dev, c_oracle, group):
    w = weight(48, 200, seed=group)
    p, s16 = g.quantize_groupwise_int4(w.to(dev), group)
    p_ref, s_ref = c_oracle.quantize_groupwise_int4(w.numpy(), group)
    assert np.array_equal(s16.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(p.cpu().numpy(), p_ref)


def _near_halves(s: float, kmin: int, kmax: int) -> np.ndarray:
    """Values whose quotient by the fp32 scale ``s`` is a half-integer
    k + 0.5 (kmin <= k < kmax) or within 1..3 ulps of one, both signs."""
    base = ((np.arange(kmin, kmax) + 0.5) * np.float64(s)).astype(np.float32)
    bits = base.view(np.int32)
    out = [base] + [(bits + d).view(np.float32) for d in (-3, -2, -1, 1, 2, 3)]
    return np.concatenate(out)


def _halfway_matrix(rows: int, cols: int, qmax: int, seed: int) -> np.ndarray:
    """Rows with |max| = amax (so s = fl(amax / qmax)) whose other entries sit
    on or next to the rounding boundaries of w / s."""
    rng = np.random.default_rng(seed)
    amaxes = [qmax * 2.0**-7, 1.0, 0.0173, 3.3e-3, 0.02 * 20, 1e-30]
    w = np.empty((rows, cols), np.float32)
    for r in range(rows):
        amax = np.float32(amaxes[r % len(amaxes)])
        s = np.float32(amax / np.float32(qmax))
        vals = _near_halves(float(s), -qmax, qmax)
        vals = vals[np.abs(vals) <= amax]
        w[r] = rng.choice(vals, cols)
        w[r, rng.integers(cols)] = amax
    return w


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("shape", [(4800, 1600), (37, 6400), (2049, 768)])
def test_per_channel_half_integer_quotients(dev, c_oracle, shape, bits):
    """Quotients on and within three ulps of k + 0.5: the kernel's product
    with the reciprocal is replaced by the exact division exactly there."""
    w = _halfway_matrix(*shape, qmax=(1 << (bits - 1)) - 1, seed=bits)
    q, s = g.quantize_tensor(torch.from_numpy(w).to(dev), bits)
    q_ref, s_ref = c_oracle.quantize_per_channel(w, bits)
    _assert_codes(q, s, q_ref, s_ref)
    if bits == 4:
        lin = torch.nn.Linear(shape[1], shape[0]).to(dev)
        with torch.no_grad():
            lin.weight.copy_(torch.from_numpy(w))
        mod, _ = g.quantize_linear(lin, 4)
        assert np.array_equal(mod.codes.cpu().numpy(), c_oracle.pack_int4(q_ref))


@pytest.mark.parametrize("shape", [(4800, 1600), (37, 6400), (2049, 768)])
def test_groupwise_half_integer_quotients(dev, c_oracle, shape):
    rng = np.random.default_rng(7)
    rows, cols = shape
    w = np.empty(shape, np.float32)
    scales = [2.0**-6, 0.0123, 3.1e-5, 1.5e-7, 60000.0]  # fp16 normal, subnormal, huge
    for r in range(rows):
        for g0 in range(0, cols, 128):
            s16 = np.float32(np.float16(scales[(r + g0 // 128) % len(scales)]))
            vals = _near_halves(float(s16), -8, 7)
            n = min(128, cols - g0)
            w[r, g0:g0 + n] = rng.choice(vals, n)
            w[r, g0 + rng.integers(n)] = np.float32(7.0) * s16
    p, sc = g.quantize_groupwise_int4(torch.from_numpy(w).to(dev), 128)
    p_ref, s_ref = c_oracle.quantize_groupwise_int4(w, 128)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(p.cpu().numpy(), p_ref)


@pytest.mark.parametrize("shape", [(4095, 1600), (2049, 768), (7, 1600), (9, 32768), (3, 32772), (1, 4)])
def test_rows_split_over_wavefronts(dev, c_oracle, shape):
    """One, two and four wavefronts per row, a last workgroup with fewer rows
    than it has room for, the longest register-resident row and one past it."""
    w = weight(*shape, seed=31)
    q, s = g.quantize_tensor(w.to(dev), 8)
    _assert_codes(q, s, *c_oracle.quantize_per_channel(w.numpy(), 8))
    p, s16 = g.quantize_groupwise_int4(w.to(dev), 128)
    p_ref, s_ref = c_oracle.quantize_groupwise_int4(w.numpy(), 128)
    assert np.array_equal(s16.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(p.cpu().numpy(), p_ref)


def test_dequantize_is_q_times_scale(dev, c_oracle):
    w = weight(300, 640, seed=4)
    q_ref, s_ref = c_oracle.quantize_per_channel(w.numpy(), 8)
    w_hat = g.quantize_dequantize(w.to(dev), 8).cpu().numpy()
    assert np.array_equal(w_hat, q_ref.astype(np.float32) * s_ref)
    p, s16 = g.quantize_groupwise_int4(w.to(dev), 128)
    lin = g.QuantLinear(p, s16, None, 640, 300, 4, "group128", "int4_groupwise", 128)
    want = OQ.dequantize_groupwise_int4(*c_oracle.quantize_groupwise_int4(w.numpy(), 128), 640, 128)
    assert np.array_equal(lin.weight.cpu().numpy(), want)


def test_empty_rows(dev):
    q, s = g.quantize_tensor(torch.empty(0, 16, device=dev), 8)
    assert q.shape == (0, 16) and s.shape == (0, 1)


def test_errors_match_reference_messages(dev):
    w = torch.zeros(4, 4, device=dev)
    with pytest.raises(ValueError, match=r"bits must be in \[2, 8\], got 1"):
        g.quantize_tensor(w, 1)
    with pytest.raises(ValueError, match="unknown granularity 'rows'"):
        g.quantize_tensor(w, 8, "rows")
