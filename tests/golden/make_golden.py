"""Writes the golden fixtures under ``tests/golden/``.

Two independent sources, two output files:

``quant_known_answers.json`` (``--known-answers``)
    Hand-built rows whose expected codes and scales follow from the closed form
    of ``quantize_tensor`` (``quantization.py:78-116``) evaluated in exact
    rational arithmetic here, with an IEEE binary32 / binary16
    round-to-nearest-even written out on fractions. No numpy or C arithmetic
    enters an expected value, so the fixtures pin the oracle rather than
    restate it. Rows: exact half-step ties at a power-of-two scale, an all-zero
    row, a row whose amax/qmax falls below FLT_MIN (scale clamped), subnormal
    entries, an outlier row, a negative-maximum row, a one-column matrix,
    per-tensor, int4 codes, the ``pack_int4`` byte table and the group-wise
    int4 format with a ragged last group.

``reference_decode.json`` (``--reference``)
    Imports the reference's ``transformer_internals`` package from
    ``/root/reference/src`` in the development container (never on the GPU
    machine) to record what no closed form pins: digests of the seed-0 GPT-2
    small weights (``model.py:457-518`` init order), the greedy token ids and
    per-step top-1/top-2 logit margins of the int8 per-channel 64+64 decode
    (``quantization.py:161-216`` + ``sampling.py:100-181`` with the
    ``benchmark.py:167-170`` prompt), the ``quantize_model`` statistics, and
    the same for a tiny configuration used by fast tests.

Usage: ``python tests/golden/make_golden.py --known-answers --reference``
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import struct
import sys
from fractions import Fraction
from pathlib import Path

HERE = Path(__file__).resolve().parent
REFERENCE_SRC = Path("/root/reference/src")

# ------------------------------------------------ exact IEEE rounding helpers


def _rn_binary(x: Fraction, mant_bits: int, emin: int, emax: int) -> Fraction:
    """Round a rational to the nearest binary float with ``mant_bits`` of
    significand (implicit bit included), ties to even. Subnormals below
    ``2**emin`` keep the fixed quantum ``2**(emin - mant_bits + 1)``."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # fix the estimate so that 2**e <= a < 2**(e+1)
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - mant_bits + 1)
    n = a / quantum
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * quantum
    if r >= Fraction(2) ** (emax + 1):
        return Fraction(sign) * Fraction(10) ** 400  # stands for infinity
    return sign * r


def rn32(x: Fraction) -> Fraction:
    return _rn_binary(x, 24, -126, 127)


def rn16(x: Fraction) -> Fraction:
    return _rn_binary(x, 11, -14, 15)


def rint_half_even(x: Fraction) -> int:
    fl = x.numerator // x.denominator
    rem = x - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def f32_bits(x: Fraction | float) -> int:
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def f16_bits(x: Fraction) -> int:
    import numpy as np  # only to encode an already exact binary16 value

    return int(np.float16(float(x)).view(np.uint16))


FLT_MIN = Fraction(2) ** -126


def exact(v: float) -> Fraction:
    """A float32 value as an exact rational (inputs are float32 by construction)."""
    f = struct.unpack("<f", struct.pack("<f", v))[0]
    return Fraction(f)


def expected_row(row: list[Fraction], bits: int) -> tuple[list[int], Fraction]:
    qmax, qmin = 2 ** (bits - 1) - 1, -(2 ** (bits - 1))
    amax = max(abs(v) for v in row)
    scale = max(rn32(amax / qmax), FLT_MIN)
    codes = [min(max(rint_half_even(rn32(v / scale)), qmin), qmax) for v in row]
    return codes, scale


# ------------------------------------------------------ known-answer rows


def known_answer_rows() -> dict[str, list[float]]:
    s = 2.0**-7
    return {
        # amax = 127 * 2^-7 so scale = 2^-7 exactly: every k.5 entry is a tie
        "ties_pow2_scale": [127 * s, 0.5 * s, 1.5 * s, 2.5 * s, 3.5 * s, -0.5 * s, -1.5 * s,
                            -2.5 * s, 126.5 * s, -126.5 * s, 0.0, -127 * s],
        "zero_row": [0.0] * 12,
        # amax/127 < FLT_MIN: the scale is clamped to FLT_MIN = 2^-126
        "scale_clamped_to_flt_min": [8.5 * 2.0**-126, 7.5 * 2.0**-126, -3.5 * 2.0**-126,
                                     2.0**-130, 2.0**-140, -(2.0**-149), 0.0, 1.0 * 2.0**-126,
                                     -8.5 * 2.0**-126, 0.5 * 2.0**-126, 2.5 * 2.0**-126, 0.0],
        "subnormal_entries": [1.0, 2.0**-140, -(2.0**-149), 0.5, -0.25, 2.0**-127, 1e-3, -1e-3,
                              0.3, -0.7, 0.0, 2.0**-126],
        "outlier_row": [0.01, -0.02, 20.0, 0.03, -0.015, 0.0, 0.005, -19.5, 0.04, 0.002, -0.001,
                        0.5],
        "negative_max_row": [-0.75, 0.5, 0.25, -0.1, 0.7, -0.74, 0.0, 0.01, -0.5, 0.375, 0.125,
                             -0.0625],
    }


def _ulp_neighbours(x: Fraction, n: int) -> list[Fraction]:
    """``x`` (a binary32 value) and its ``n`` binary32 neighbours on each side."""
    b = f32_bits(x)
    out = []
    for d in range(-n, n + 1):
        v = struct.unpack("<f", struct.pack("<I", b + d))[0]
        out.append(Fraction(v))
    return out


def reciprocal_trap_row() -> list[float]:
    """Entries whose code differs between ``rint(w / s)`` (the reference) and
    ``rint(w * (1 / s))`` at the scale of amax = 0.75, found by exact search,
    so that an implementation multiplying by a reciprocal fails the fixture."""
    s = rn32(Fraction(3, 4) / 127)
    r = rn32(1 / s)
    row: list[float] = [0.75]
    for k in range(0, 127):
        for w in _ulp_neighbours(rn32((k + Fraction(1, 2)) * s), 4):
            if rint_half_even(rn32(w / s)) != rint_half_even(rn32(w * r)):
                row.append(float(w))
                break
        if len(row) == 12:
            break
    if len(row) < 12:
        raise RuntimeError("reciprocal search found too few entries")
    return row


def build_known_answers() -> dict:
    rows = known_answer_rows()
    rows["reciprocal_trap"] = reciprocal_trap_row()
    out: dict = {"description": "expected values derived in exact rational arithmetic",
                 "per_channel": {}, "per_tensor": {}, "one_column": {}, "pack_int4": {},
                 "groupwise_int4": {}}
    names = list(rows)
    matrix = [[exact(v) for v in rows[n]] for n in names]
    for bits in (8, 4, 2):
        codes, scales = [], []
        for r in matrix:
            c, sc = expected_row(r, bits)
            codes.append(c)
            scales.append(f32_bits(sc))
        out["per_channel"][str(bits)] = {"codes": codes, "scale_bits": scales}
        flat = [v for r in matrix for v in r]
        c, sc = expected_row(flat, bits)
        out["per_tensor"][str(bits)] = {"codes": c, "scale_bits": f32_bits(sc)}
    out["rows"] = names
    out["input_bits"] = [[f32_bits(v) for v in r] for r in matrix]
    one_col = [[0.3], [-2.0], [0.0], [2.0**-130]]
    oc_codes, oc_scales = [], []
    for r in one_col:
        c, sc = expected_row([exact(v) for v in r], 8)
        oc_codes.append(c)
        oc_scales.append(f32_bits(sc))
    out["one_column"] = {"input_bits": [[f32_bits(exact(v)) for v in r] for r in one_col],
                         "codes": oc_codes, "scale_bits": oc_scales}
    # pack_int4: arange(-8, 8) -> 0x10 0x32 ... 0xfe ; odd count pads high nibble 0
    out["pack_int4"] = {
        "codes": list(range(-8, 8)),
        "bytes": [((hi + 8) << 4) | (lo + 8) for lo, hi in zip(range(-8, 8, 2), range(-7, 8, 2))],
        "odd_codes": [3, -8, 7],
        "odd_bytes": [((-8 + 8) << 4) | (3 + 8), 7 + 8],
    }
    # group-wise int4, group 8 over 20 columns (ragged last group of 4)
    g = 8
    grow = [0.7, -0.35, 0.1, 0.0, 0.05, -0.7, 0.2, 0.3,          # amax 0.7
            0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0,              # zero group
            1e-9, -3e-9, 2e-9, 0.0]                               # scale underflows fp16
    grow2 = [3.0, 1.5, -1.5, 0.75, 2.25, -3.0, 0.0, 0.375,
             1e6, -2e6, 7.0, 0.0, 1.0, 2.0, 3.0, -4.0,            # saturated scale
             -1.0, 0.5, 0.25, 0.125]
    gcodes, gscales, gbytes = [], [], []
    for r in (grow, grow2):
        er = [exact(v) for v in r]
        rc, rs = [], []
        for c0 in range(0, len(er), g):
            grp = er[c0:c0 + g]
            amax = max(abs(v) for v in grp)
            s16 = rn16(rn32(amax / 7))
            if s16 == 0:
                s16 = Fraction(2) ** -24
            if s16 > 65504:
                s16 = Fraction(65504)
            rs.append(f16_bits(s16))
            rc += [min(max(rint_half_even(rn32(v / s16)), -8), 7) for v in grp]
        gcodes.append(rc)
        gscales.append(rs)
        gbytes.append([((rc[2 * j + 1] + 8) << 4) | (rc[2 * j] + 8) for j in range(len(rc) // 2)])
    out["groupwise_int4"] = {
        "group": g,
        "input_bits": [[f32_bits(exact(v)) for v in r] for r in (grow, grow2)],
        "codes": gcodes, "scale_f16_bits": gscales, "packed": gbytes,
    }
    return out


# ------------------------------------------------------- reference vectors


def _digest(t) -> str:
    return hashlib.sha256(t.detach().contiguous().numpy().tobytes()).hexdigest()


def build_reference_vectors() -> dict:
    sys.path.insert(0, str(REFERENCE_SRC))
    import torch

    from transformer_internals.config import GPTConfig  # type: ignore
    from transformer_internals.model import GPT, KVCache  # type: ignore
    from transformer_internals.quantization import quantize_model  # type: ignore

    torch.set_num_threads(8)

    def decode_with_margins(model, prompt, n):
        cache = KVCache.empty(model.config.n_layer)
        idx, margins = prompt, []
        with torch.no_grad():
            for step in range(n):
                inp = idx if step == 0 else idx[:, -1:]
                logits = model(inp, cache=cache)["logits"][:, -1, :]
                top2 = logits.topk(2, dim=-1).values
                margins.append(float((top2[:, 0] - top2[:, 1]).min()))
                idx = torch.cat([idx, logits.argmax(-1, keepdim=True)], dim=1)
        return idx, margins

    out: dict = {}
    for label, cfg, prompt_shape, new in (
        ("tiny", GPTConfig(vocab_size=97, n_positions=64, n_layer=3, n_head=4, n_embd=32), (2, 11), 40),
        ("gpt2_small", GPTConfig(), (1, 64), 64),
    ):
        torch.manual_seed(0)
        model = GPT(cfg).eval()
        sd = model.state_dict()
        keys = ["wte.weight", "wpe.weight", "h.0.attn.c_attn.weight", "h.0.attn.c_proj.weight",
                f"h.{cfg.n_layer - 1}.mlp.c_fc.weight", f"h.{cfg.n_layer - 1}.mlp.c_proj.weight",
                "h.0.attn.c_attn.bias"]
        entry: dict = {
            "config": {k: getattr(cfg, k) for k in ("vocab_size", "n_positions", "n_layer", "n_head", "n_embd")},
            "param_sha256": {k: _digest(sd[k]) for k in keys},
            "param_sum": {k: float(sd[k].double().sum()) for k in keys},
        }
        for bits in (8, 4):
            qm, stats = quantize_model(model, bits=bits, granularity="per_channel")
            entry[f"stats_int{bits}"] = stats
            torch.manual_seed(0)
            prompt = torch.randint(0, cfg.vocab_size, prompt_shape)
            ids, margins = decode_with_margins(qm, prompt, new)
            entry[f"greedy_int{bits}"] = {"prompt_shape": list(prompt_shape), "new_tokens": new,
                                          "ids": ids.tolist(), "margins": margins}
        out[label] = entry
    out["source"] = "reference transformer_internals imported from /root/reference/src"
    out["torch"] = torch.__version__
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--known-answers", action="store_true")
    ap.add_argument("--reference", action="store_true")
    args = ap.parse_args()
    if args.known_answers:
        (HERE / "quant_known_answers.json").write_text(json.dumps(build_known_answers(), indent=1))
        print("wrote quant_known_answers.json")
    if args.reference:
        (HERE / "reference_decode.json").write_text(json.dumps(build_reference_vectors(), indent=1))
        print("wrote reference_decode.json")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
