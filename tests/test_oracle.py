"""The oracle, pinned before it is trusted (CPU only).

* the numpy and C restatements against the closed-form known answers
  (exact rational arithmetic, ``golden/quant_known_answers.json``);
* the two restatements against each other on seeded inputs with outliers;
* the reference's own property tests (``tests/test_efficiency.py:24-104``)
  re-run on the oracle;
* a planted mistake (round-half-away instead of half-even, a multiply by the
  reciprocal instead of the divide) must fail the known answers;
* the model restatement against the reference's recorded seed-0 weight
  digests and greedy tokens (``golden/reference_decode.json``).
"""

from __future__ import annotations

import hashlib
import math

import numpy as np
import pytest
import torch

from oracle import linear as OL
from oracle import model as OM
from oracle import quant as OQ


def _f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


# ------------------------------------------------------------ known answers


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_numpy_oracle_per_channel_known_answers(known_answers, bits):
    w = _f32(known_answers["input_bits"])
    exp = known_answers["per_channel"][str(bits)]
    q, s = OQ.quantize_tensor(w, bits, "per_channel")
    assert q.tolist() == exp["codes"]
    assert s.reshape(-1).view(np.uint32).tolist() == exp["scale_bits"]


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_c_oracle_per_channel_known_answers(known_answers, c_oracle, bits):
    w = _f32(known_answers["input_bits"])
    exp = known_answers["per_channel"][str(bits)]
    q, s = c_oracle.quantize_per_channel(w, bits)
    assert q.tolist() == exp["codes"]
    assert s.reshape(-1).view(np.uint32).tolist() == exp["scale_bits"]


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_oracles_per_tensor_known_answers(known_answers, c_oracle, bits):
    w = _f32(known_answers["input_bits"])
    exp = known_answers["per_tensor"][str(bits)]
    q, s = OQ.quantize_tensor(w, bits, "per_tensor")
    assert q.reshape(-1).tolist() == exp["codes"] and int(s.view(np.uint32)) == exp["scale_bits"]
    q, s = c_oracle.quantize_per_tensor(w, bits)
    assert q.reshape(-1).tolist() == exp["codes"] and int(s.view(np.uint32)) == exp["scale_bits"]


def test_one_column_known_answers(known_answers, c_oracle):
    oc = known_answers["one_column"]
    w = _f32(oc["input_bits"])
    for q, s in (OQ.quantize_tensor(w, 8), c_oracle.quantize_per_channel(w, 8)):
        assert q.tolist() == oc["codes"]
        assert s.reshape(-1).view(np.uint32).tolist() == oc["scale_bits"]


def test_pack_known_answers(known_answers, c_oracle):
    pk = known_answers["pack_int4"]
    assert [hex(b) for b in pk["bytes"]] == ["0x10", "0x32", "0x54", "0x76", "0x98", "0xba", "0xdc", "0xfe"]
    for pack in (OQ.pack_int4, c_oracle.pack_int4):
        assert pack(np.array(pk["codes"], np.int8)).tolist() == pk["bytes"]
        assert pack(np.array(pk["odd_codes"], np.int8)).tolist() == pk["odd_bytes"]
    for unpack in (OQ.unpack_int4, c_oracle.unpack_int4):
        assert unpack(np.array(pk["bytes"], np.uint8), 16).tolist() == pk["codes"]
        assert unpack(np.array(pk["odd_bytes"], np.uint8), 3).tolist() == pk["odd_codes"]


def test_groupwise_known_answers(known_answers, c_oracle):
    gk = known_answers["groupwise_int4"]
    w = _f32(gk["input_bits"])
    p, s, codes = OQ.quantize_groupwise_int4(w, gk["group"])
    assert codes.tolist() == gk["codes"]
    assert s.view(np.uint16).tolist() == gk["scale_f16_bits"]
    assert p.tolist() == gk["packed"]
    p2, s2 = c_oracle.quantize_groupwise_int4(w, gk["group"])
    assert p2.tolist() == gk["packed"] and s2.view(np.uint16).tolist() == gk["scale_f16_bits"]


def test_planted_mistakes_fail_the_known_answers(known_answers):
    """A plausible wrong oracle must not pass: half-away rounding and a
    reciprocal multiply each change at least one code of the fixture."""
    w = _f32(known_answers["input_bits"])
    exp = np.array(known_answers["per_channel"]["8"]["codes"])
    amax = np.abs(w).max(axis=1, keepdims=True)
    s = np.maximum(amax / np.float32(127), np.float32(np.finfo(np.float32).tiny)).astype(np.float32)
    half_away = np.clip(np.sign(w / s) * np.floor(np.abs(w / s) + 0.5), -128, 127).astype(np.int8)
    assert not np.array_equal(half_away, exp)
    rcp = np.clip(np.rint(w * (np.float32(1) / s)), -128, 127).astype(np.int8)
    trap = known_answers["rows"].index("reciprocal_trap")
    assert not np.array_equal(rcp[trap], exp[trap])
    # and the oracle itself gets that row right
    assert OQ.quantize_tensor(w, 8)[0][trap].tolist() == exp[trap].tolist()


# ------------------------------------------------- numpy oracle vs C oracle


@pytest.mark.parametrize("shape", [(300, 257), (64, 1600), (33, 6400), (7, 1)])
@pytest.mark.parametrize("bits", [8, 4, 3])
def test_numpy_and_c_oracles_agree(c_oracle, shape, bits):
    rng = np.random.default_rng(hash((shape, bits)) & 0xFFFF)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    w[rng.random(shape) < 0.001] *= 20
    q1, s1 = OQ.quantize_tensor(w, bits)
    q2, s2 = c_oracle.quantize_per_channel(w, bits)
    assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    q1, s1 = OQ.quantize_tensor(w, bits, "per_tensor")
    q2, s2 = c_oracle.quantize_per_tensor(w, bits)
    assert np.array_equal(q1, q2) and s1.view(np.uint32) == s2.view(np.uint32)
    if bits == 4:
        assert np.array_equal(OQ.pack_int4(q1), c_oracle.pack_int4(q1))
    if shape[1] > 1:
        p1, g1, _ = OQ.quantize_groupwise_int4(w, 128)
        p2, g2 = c_oracle.quantize_groupwise_int4(w, 128)
        assert np.array_equal(p1, p2) and np.array_equal(g1.view(np.uint16), g2.view(np.uint16))


def test_fp16_rounding_matches_ieee(c_oracle):
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.standard_normal(3000).astype(np.float32) * s for s in (1e-7, 1e-5, 1, 3e4)])
    edge = np.float32([65504, 65519.99, 65520, 2.0**-25, 1.5 * 2.0**-25, 2.0**-24, 2.0**-14, 0.0, 3 * 2.0**-26])
    xs = np.concatenate([xs, edge])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([c_oracle.f32_to_f16_bits(float(v)) for v in xs], np.uint16)
    assert np.array_equal(want, got)


# ------------------------------------ the reference's property tests on the oracle


@pytest.mark.parametrize("bits", [8, 4])
def test_codes_stay_in_range(bits):
    w = np.random.default_rng(0).standard_normal((64, 32)).astype(np.float32) * 3
    q, s = OQ.quantize_tensor(w, bits)
    assert q.min() >= -(2 ** (bits - 1)) and q.max() <= 2 ** (bits - 1) - 1 and s.shape == (64, 1)


def test_error_bounded_by_half_step():
    w = np.random.default_rng(1).standard_normal((32, 16)).astype(np.float32)
    q, s = OQ.quantize_tensor(w, 8)
    assert np.all(np.abs(w - q.astype(np.float32) * s) <= s / 2 + 1e-6)


def test_more_bits_never_worse_and_per_channel_beats_per_tensor():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((64, 64)).astype(np.float32)
    errs = [np.abs(w - OQ.quantize_dequantize(w, b)).mean() for b in (4, 6, 8)]
    assert errs[0] > errs[1] > errs[2]
    w = (rng.standard_normal((16, 32)) * 0.01).astype(np.float32)
    w[3] *= 500.0
    pt = np.abs(w - OQ.quantize_dequantize(w, 4, "per_tensor"))
    pc = np.abs(w - OQ.quantize_dequantize(w, 4, "per_channel"))
    others = np.ones(16, bool)
    others[3] = False
    assert pc[others].mean() < pt[others].mean() / 5
    assert math.isclose(pc[3].mean(), pt[3].mean(), rel_tol=0.05)


def test_zero_row_and_bad_args():
    w = np.random.default_rng(4).standard_normal((4, 8)).astype(np.float32)
    w[2] = 0
    out = OQ.quantize_dequantize(w, 8)
    assert np.all(out[2] == 0) and np.isfinite(out).all()
    with pytest.raises(ValueError, match=r"bits must be in \[2, 8\], got 9"):
        OQ.quantize_tensor(w, 9)
    with pytest.raises(ValueError, match="unknown granularity 'per_row'"):
        OQ.quantize_tensor(w, 8, "per_row")


@pytest.mark.parametrize("shape", [(7, 6), (5, 5), (1,), (3,)])
def test_int4_round_trip(shape):
    q = np.random.default_rng(0).integers(-8, 8, shape).astype(np.int8)
    p = OQ.pack_int4(q)
    assert p.size == math.ceil(q.size / 2) and p.dtype == np.uint8
    assert np.array_equal(OQ.unpack_int4(p, q.size).reshape(shape), q)


def test_linear_ref_is_dequantize_then_matmul():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((48, 32)) * 0.02).astype(np.float32)
    q, s = OQ.quantize_tensor(w, 8)
    x = torch.from_numpy(rng.standard_normal((3, 32)).astype(np.float32))
    b = torch.from_numpy(rng.standard_normal(48).astype(np.float32))
    y = OL.linear_ref(x, OL.dequantize(q, s), b)
    w_hat = q.astype(np.float64) * s.astype(np.float64)
    y64 = x.double().numpy() @ w_hat.T + b.double().numpy()
    assert np.abs(y.numpy() - y64).max() < 1e-5
    ok, _, _ = OL.within_tolerance(y, torch.from_numpy(y64))
    assert ok
    assert not OL.within_tolerance(y * 1.01, torch.from_numpy(y64))[0]


# --------------------------------------------- model oracle vs the reference


def _shape(c) -> OM.Shape:
    return OM.Shape(c["vocab_size"], c["n_positions"], c["n_layer"], c["n_head"], c["n_embd"])


@pytest.mark.parametrize("label", ["tiny", "gpt2_small"])
def test_oracle_init_matches_reference_digests(reference_decode, label):
    e = reference_decode[label]
    p = OM.init_params(_shape(e["config"]), 0)
    for k, h in e["param_sha256"].items():
        assert hashlib.sha256(p[k].contiguous().numpy().tobytes()).hexdigest() == h, k


@pytest.mark.parametrize("bits", [8, 4])
def test_oracle_greedy_matches_reference_tiny(reference_decode, bits):
    e = reference_decode["tiny"]
    shp = _shape(e["config"])
    qp, _ = OM.quantize_params(OM.init_params(shp, 0), bits)
    g = e[f"greedy_int{bits}"]
    ids, margins = OM.generate_greedy(qp, shp, OM.benchmark_prompt(shp.vocab_size, *g["prompt_shape"]), g["new_tokens"])
    assert ids.tolist() == g["ids"]
    assert np.allclose(margins, g["margins"], atol=1e-5)


def test_oracle_greedy_matches_reference_gpt2_small(reference_decode):
    e = reference_decode["gpt2_small"]
    shp = _shape(e["config"])
    qp, codes = OM.quantize_params(OM.init_params(shp, 0), 8)
    assert len(codes) == e["stats_int8"]["n_quantized_tensors"] == 48
    assert sum(q.size for q, _ in codes.values()) == e["stats_int8"]["n_quantized_params"]
    g = e["greedy_int8"]
    ids, _ = OM.generate_greedy(qp, shp, OM.benchmark_prompt(shp.vocab_size, *g["prompt_shape"]), g["new_tokens"])
    assert ids.tolist() == g["ids"]
