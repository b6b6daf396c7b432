"""The screened tied head (``tiq_head_argmax_screened`` and
``tiq_head_argmax_screened_i8``): the one-row decode step's ``lm_head``
(``model.py:585``) and argmax (``sampling.py:164-170``) computed from a bf16
copy, or an int8 copy with a scale a row, of the head, with only the rows whose
certified bound reaches their group's best recomputed from the fp32 weights.
Every test runs both copies.

The token must be the argmax of the fp32 logits -- checked against torch's
fp32 LayerNorm + matmul + argmax (with a float64 margin check where two logits
are within fp32 rounding of each other), on random heads and on rows built to
defeat the screening: every row identical (all rows recomputed, first index
wins), duplicated maxima far apart, two rows closer than bf16 can tell apart,
NaN rows (never selected) and rows of -inf logits.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gpt2_harness_amd import _lib

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


FMTS = ["bf16", "int8"]


def _prepare(w, fmt):
    """(copy, per-row scale or None, per-row bound coefficient)."""
    L = _lib.lib()
    V, C = w.shape
    coef = torch.empty(V, device=w.device)
    if fmt == "int8":
        wq = torch.empty(V, C, dtype=torch.int8, device=w.device)
        sc = torch.empty(V, device=w.device)
        _lib.check(L.tiq_head_screen_prepare_i8(w.data_ptr(), V, C, w.stride(0), wq.data_ptr(), sc.data_ptr(),
                                                coef.data_ptr(), _st()), "prepare i8")
        return wq, sc, coef
    wb = torch.empty(V, C, dtype=torch.int16, device=w.device)
    _lib.check(L.tiq_head_screen_prepare(w.data_ptr(), V, C, w.stride(0), wb.data_ptr(), coef.data_ptr(), _st()),
               "prepare")
    return wb, None, coef


def _copy64(prep):
    """The screened copy as float64 rows: bf16(w), or s q."""
    wc, sc, _ = prep
    if sc is None:
        return wc.view(torch.bfloat16).double()
    return wc.double() * sc.double()[:, None]


def _coef64(w, prep):
    """err + gamma (2 norm + err) in float64, gamma over C terms for the bf16
    copy and C + 1 for the int8 one (the scale's product)."""
    n = w.shape[1] + (0 if prep[1] is None else 1)
    err = (w.double() - _copy64(prep)).norm(dim=1)
    nrm = w.double().norm(dim=1)
    gamma = n * 2.0**-24 / (1 - n * 2.0**-24)
    return err + gamma * (2 * nrm + err)


def _screened(x, lw, lb, w, prep, pos=5, ld_ids=16):
    L = _lib.lib()
    V, C = w.shape
    wc, sc, coef = prep
    logits = torch.full((V,), float("nan"), device=w.device)
    out = torch.full((1,), -1, dtype=torch.long, device=w.device)
    ids = torch.zeros(1, ld_ids, dtype=torch.long, device=w.device)
    p = torch.tensor([pos], dtype=torch.long, device=w.device)
    ws = torch.empty(int(L.tiq_head_screen_workspace(V)), dtype=torch.uint8, device=w.device)
    if sc is None:
        rc = L.tiq_head_argmax_screened(x.data_ptr(), C, lw.data_ptr(), lb.data_ptr(), 1e-5, wc.data_ptr(),
                                        w.data_ptr(), w.stride(0), coef.data_ptr(), V, logits.data_ptr(),
                                        out.data_ptr(), ids.data_ptr(), ld_ids, p.data_ptr(), ws.data_ptr(),
                                        ws.numel(), _st())
    else:
        rc = L.tiq_head_argmax_screened_i8(x.data_ptr(), C, lw.data_ptr(), lb.data_ptr(), 1e-5, wc.data_ptr(),
                                           sc.data_ptr(), w.data_ptr(), w.stride(0), coef.data_ptr(), V,
                                           logits.data_ptr(), out.data_ptr(), ids.data_ptr(), ld_ids, p.data_ptr(),
                                           ws.data_ptr(), ws.numel(), _st())
    _lib.check(rc, "screened head")
    torch.cuda.synchronize()
    return int(out), ids.cpu(), int(p), logits


def _ref(x, lw, lb, w):
    xl = F.layer_norm(x.double(), (x.numel(),), lw.double(), lb.double(), 1e-5)
    y32 = F.layer_norm(x, (x.numel(),), lw, lb, 1e-5) @ w.T
    return y32, xl @ w.double().T


def _inputs(V, C, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randn(V, C, generator=g, device=dev) * 0.02
    x = torch.randn(C, generator=g, device=dev) * 3 + 0.5
    lw = 1 + 0.1 * torch.randn(C, generator=g, device=dev)
    lb = 0.1 * torch.randn(C, generator=g, device=dev)
    return x, lw, lb, w


def _check_token(tok, y32, y64):
    """tok is the argmax of the fp32 logits, or within fp32 rounding of it."""
    want = int(y32.argmax())
    if tok == want:
        return
    # a different row may win only where the two are equal within fp32 rounding
    assert abs(float(y64[tok]) - float(y64[want])) <= 1e-5 * float(y64.abs().max()), (tok, want)


@pytest.mark.parametrize("fmt", FMTS)
def test_prepare_bounds_hold(dev, fmt):
    x, lw, lb, w = _inputs(4099, 768, 1, dev)
    w[5] = 0.0  # a zero row: scale 0, codes 0, no error
    prep = _prepare(w, fmt)
    wc, sc, coef = prep
    if fmt == "bf16":
        assert torch.equal(wc.view(torch.bfloat16).cpu(), w.to(torch.bfloat16).cpu())  # nearest even, as torch
    else:
        # fp32 quotients correctly rounded (through float64, exact for fp32
        # operands), on the CPU: torch's GPU division by a scalar multiplies
        # by its reciprocal
        wd = w.cpu().double()
        s_ref = (wd.abs().amax(dim=1) / 127.0).float()
        assert torch.equal(sc.cpu(), s_ref)
        s_safe = torch.where(s_ref > 0, s_ref, torch.ones_like(s_ref)).double()
        quot = (wd / s_safe[:, None]).float()
        q = torch.where(s_ref[:, None] > 0, torch.round(quot).clamp(-127, 127), torch.zeros_like(quot))
        assert torch.equal(wc.cpu(), q.to(torch.int8))  # round half to even, clamped
        assert float(sc[5]) == 0.0 and not wc[5].any()
    c64 = _coef64(w, prep)
    assert bool((coef.double() >= c64).all())
    assert float((coef.double() - c64).max()) <= 1e-6 * float(c64.max())


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("V,C", [(50257, 768), (50257, 1024), (5003, 768), (5003, 64), (33, 128), (1, 16)])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_screened_argmax_matches_fp32(dev, fmt, V, C, seed):
    x, lw, lb, w = _inputs(V, C, seed, dev)
    prep = _prepare(w, fmt)
    tok, ids, pos, logits = _screened(x, lw, lb, w, prep, pos=5)
    y32, y64 = _ref(x, lw, lb, w)
    _check_token(tok, y32, y64)
    assert int(ids[0, 6]) == tok and pos == 6 and not ids[0, :6].any() and not ids[0, 7:].any()
    # the logits buffer holds the estimates from the copy: within the
    # certified bound ||x|| (err + gamma (2 norm + err)) of the exact products
    # (float64 here)
    xl = F.layer_norm(x.double(), (C,), lw.double(), lb.double(), 1e-5)
    bound = xl.norm() * _coef64(w, prep)
    assert bool(((logits.double() - y64).abs() <= bound * 1.01 + 1e-30).all())
    # the chosen row was recomputed from the fp32 weights
    assert float(logits[tok]) == pytest.approx(float(y64[tok]), rel=1e-5, abs=1e-6)


@pytest.mark.parametrize("fmt", FMTS)
def test_all_rows_equal_takes_first(dev, fmt):
    """Every row is a candidate of its group; the first index of the maximum wins."""
    x, lw, lb, w = _inputs(3000, 256, 3, dev)
    w[:] = w[7]
    tok, *_ = _screened(x, lw, lb, w, _prepare(w, fmt))
    assert tok == 0


@pytest.mark.parametrize("fmt", FMTS)
def test_duplicated_maximum_far_apart(dev, fmt):
    x, lw, lb, w = _inputs(50257, 768, 4, dev)
    y32, _ = _ref(x, lw, lb, w)
    best = int(y32.argmax())
    w[50000] = w[best]
    w[123] = w[best]
    tok, *_ = _screened(x, lw, lb, w, _prepare(w, fmt))
    assert tok == min(123, best)


@pytest.mark.parametrize("fmt", FMTS)
def test_rows_closer_than_bf16(dev, fmt):
    """Two rows whose bf16 copies (and int8 codes) are equal but whose fp32
    logits differ: the screening must recompute both and take the larger."""
    x, lw, lb, w = _inputs(8192, 768, 5, dev)
    y32, _ = _ref(x, lw, lb, w)
    best = int(y32.argmax())
    xl = F.layer_norm(x, (768,), lw, lb, 1e-5)
    twin = (best + 4000) % 8192
    # nudge one weight of the twin by far less than a bf16 step, toward a
    # larger logit: the column with the largest |x| whose bf16 stays the same
    for j in xl.abs().argsort(descending=True).tolist():
        w[twin] = w[best]
        w[twin, j] += torch.sign(xl[j]) * 1e-6
        if torch.equal(w[twin].to(torch.bfloat16), w[best].to(torch.bfloat16)):
            break
    assert torch.equal(w[twin].to(torch.bfloat16), w[best].to(torch.bfloat16))
    prep = _prepare(w, fmt)
    assert torch.equal(prep[0][twin], prep[0][best])
    tok, _, _, logits = _screened(x, lw, lb, w, prep)
    y32, y64 = _ref(x, lw, lb, w)
    assert float(y64[twin]) > float(y64[best])
    assert tok == twin


@pytest.mark.parametrize("fmt", FMTS)
def test_nan_rows_never_selected_and_all_neg_inf(dev, fmt):
    x, lw, lb, w = _inputs(4000, 256, 6, dev)
    y32, _ = _ref(x, lw, lb, w)
    best = int(y32.argmax())
    w[best] = float("nan")
    w[17] = float("nan")
    tok, *_ = _screened(x, lw, lb, w, _prepare(w, fmt))
    w2 = w.clone()
    w2[best] = 0.0
    w2[17] = 0.0
    y2, _ = _ref(x, lw, lb, w2)
    y2[best] = -float("inf")
    y2[17] = -float("inf")
    assert tok == int(y2.argmax())
    # every logit -inf or NaN: index 0, as tiq_argmax_rows
    w3 = torch.full_like(w, float("nan"))
    tok3, *_ = _screened(x, lw, lb, w3, _prepare(w3, fmt))
    assert tok3 == 0


def test_screened_arguments(dev):
    L = _lib.lib()
    x, lw, lb, w = _inputs(100, 1040, 7, dev)  # 1040 columns: more than a wavefront's 1024
    wb, _, coef = _prepare(w, "bf16")
    out = torch.zeros(1, dtype=torch.long, device=dev)
    ws = torch.empty(int(L.tiq_head_screen_workspace(100)), dtype=torch.uint8, device=dev)
    logits = torch.empty(100, device=dev)
    args = [x.data_ptr(), 1040, lw.data_ptr(), lb.data_ptr(), 1e-5, wb.data_ptr(), w.data_ptr(), 1040,
            coef.data_ptr(), 100, logits.data_ptr(), out.data_ptr(), None, 0, None, ws.data_ptr(), ws.numel(), _st()]
    assert L.tiq_head_argmax_screened(*args) == -4  # TIQ_EUNSUPPORTED
    args[1] = 1024
    args[16] = 0
    assert L.tiq_head_argmax_screened(*args) == -5  # TIQ_EWORKSPACE
    args[16] = ws.numel()
    args[9] = 0
    assert L.tiq_head_argmax_screened(*args) == -1  # TIQ_EINVAL


def test_screened_i8_arguments(dev):
    L = _lib.lib()
    x, lw, lb, w = _inputs(100, 1040, 8, dev)
    wq, sc, coef = _prepare(w, "int8")
    out = torch.zeros(1, dtype=torch.long, device=dev)
    ws = torch.empty(int(L.tiq_head_screen_workspace(100)), dtype=torch.uint8, device=dev)
    logits = torch.empty(100, device=dev)
    args = [x.data_ptr(), 1040, lw.data_ptr(), lb.data_ptr(), 1e-5, wq.data_ptr(), sc.data_ptr(), w.data_ptr(), 1040,
            coef.data_ptr(), 100, logits.data_ptr(), out.data_ptr(), None, 0, None, ws.data_ptr(), ws.numel(), _st()]
    assert L.tiq_head_argmax_screened_i8(*args) == -4  # TIQ_EUNSUPPORTED: more than 1024 columns
    args[1] = 1024
    args[17] = 0
    assert L.tiq_head_argmax_screened_i8(*args) == -5  # TIQ_EWORKSPACE
    args[17] = ws.numel()
    args[6] = None
    assert L.tiq_head_argmax_screened_i8(*args) == -1  # TIQ_EINVAL: no scales
    args[6] = sc.data_ptr()
    args[10] = 0
    assert L.tiq_head_argmax_screened_i8(*args) == -1  # TIQ_EINVAL: no rows
    assert L.tiq_head_screen_prepare_i8(w.data_ptr(), 100, 1040, 1000, wq.data_ptr(), sc.data_ptr(), coef.data_ptr(),
                                        _st()) == -1  # ldw < n_embd
