"""Host-side checks that need no GPU.

* the C-ABI library loads and exports every function ``include/tiq.h``
  declares, with the signatures the binding assumes;
* the Python API raises the reference's errors before touching a device, and
  refuses CPU tensors loudly (there is no CPU fallback);
* the host model mirrors the reference's init (seed-0 digests) and config
  validation; ``generate`` keeps its greedy / cache / context-limit semantics.
"""

from __future__ import annotations

import hashlib
import math
import re
from pathlib import Path

import pytest
import torch

import gpt2_harness_amd as g
from gpt2_harness_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions() -> list[str]:
    text = (ROOT / "include" / "tiq.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tiq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert len(declared) >= 16
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in tiq.h but not exported"
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signatures out of sync with tiq.h"
    assert lib.tiq_version() >= 100
    assert lib.tiq_status_string(-2) == b"bits must be in [2, 8]"
    assert lib.tiq_status_string(0) == b"ok"


def test_arguments_checked_before_any_launch():
    """Entry points validate arguments on the host and never launch on bad input
    (no GPU is needed to see the error codes)."""
    lib = _lib.load()
    assert lib.tiq_quantize_per_channel(None, 4, 4, 4, 9, None, 4, None, None) == -2
    assert lib.tiq_quantize_per_channel(None, 4, 4, 2, 8, None, 4, None, None) == -1
    assert lib.tiq_quantize_per_channel(None, 0, 4, 4, 8, None, 4, None, None) == 0
    assert lib.tiq_quantize_per_tensor(None, 16, 1, None, None, None, 0, None) == -2
    assert lib.tiq_quantize_groupwise_int4(None, 4, 4, 3, None, None, None) == -1
    assert lib.tiq_quantize_per_channel_int4_packed(None, 4, 5, 4, None, None, None) == -4
    assert lib.tiq_linear_w8(None, 0, 0, 16, 16, None, None, None, 4, None, 0, 4, None) == 0
    assert lib.tiq_linear_w8(None, 3, 1, 16, 16, None, None, None, 4, None, 0, 4, None) == -1
    assert lib.tiq_linear_w4g(None, 0, 1, 16, 16, None, None, 3, None, 4, None, 0, 4, None) == -1
    assert lib.tiq_quantize_per_tensor_workspace(1 << 20) >= 4
    assert lib.tiq_gelu_tanh(None, None, -1, None) == -1
    assert lib.tiq_gelu_tanh(None, None, 0, None) == 0
    assert lib.tiq_gelu_tanh(None, None, 8, None) == -1
    assert lib.tiq_gelu_tanh(4, 16, 8, None) == -3  # misaligned (never dereferenced)


def test_api_errors_match_reference_without_gpu():
    w = torch.zeros(4, 4)
    with pytest.raises(ValueError, match=r"bits must be in \[2, 8\], got 9"):
        g.quantize_tensor(w, 9)
    with pytest.raises(ValueError, match="unknown granularity 'per_row'"):
        g.quantize_tensor(w, 8, "per_row")
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        g.quantize_tensor(w, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        g.pack_int4(torch.zeros(4, dtype=torch.int8))


def test_config_validation_and_sizes():
    with pytest.raises(ValueError, match="must be divisible"):
        g.GPTConfig(n_embd=10, n_head=3)
    with pytest.raises(ValueError, match="unknown GPT-2 size"):
        g.gpt2_config("gpt2-huge")
    xl = g.gpt2_config("gpt2-xl")
    assert (xl.n_layer, xl.n_head, xl.n_embd) == (48, 25, 1600)
    assert g.GPTConfig().kv_cache_bytes_per_token(4) == 73_728
    assert xl.kv_cache_bytes_per_token(4) == 614_400


@pytest.mark.parametrize("label", ["tiny", "gpt2_small"])
def test_host_model_init_matches_reference(reference_decode, label):
    e = reference_decode[label]
    torch.manual_seed(0)
    sd = g.GPT(g.GPTConfig(**e["config"])).state_dict()
    for k, h in e["param_sha256"].items():
        assert hashlib.sha256(sd[k].contiguous().numpy().tobytes()).hexdigest() == h, k


def test_param_count_and_tying():
    torch.manual_seed(0)
    m = g.GPT(g.GPTConfig())
    assert sum(p.numel() for p in m.parameters()) == 124_439_808   # the tied matrix once
    assert m.lm_head.weight is m.wte.weight


def test_generate_semantics_on_cpu_float_model(reference_decode):
    """The decode loop itself (unquantized fp32 model on the CPU): cached ==
    uncached, context-limit stop, EOS stop, sampling refused."""
    torch.manual_seed(0)
    cfg = g.GPTConfig(vocab_size=64, n_positions=24, n_layer=2, n_head=4, n_embd=32)
    m = g.GPT(cfg).eval()
    p = torch.randint(0, 64, (2, 5))
    a = g.generate(m, p, 12, use_cache=True)
    b = g.generate(m, p, 12, use_cache=False)
    assert torch.equal(a, b)
    assert g.generate(m, p, 100).shape[1] == 24
    first = int(a[0, 5])
    out = g.generate(m, p[:1], 10, eos_token_id=first)
    assert out.shape[1] == 6
    with pytest.raises(NotImplementedError):
        g.generate(m, p, 3, do_sample=True)
    with pytest.raises(ValueError, match="exceeds n_positions"):
        m(torch.zeros(1, 25, dtype=torch.long))


def test_kv_cache_length_semantics():
    c = g.KVCache.empty(2)
    assert c.seq_len == 0 and c.length(1) == 0
    k = torch.zeros(1, 2, 3, 4)
    c.update(0, k, k)
    assert c.seq_len == 3 and c.length(1) == 0
    kk, _ = c.update(0, k[:, :, :1], k[:, :, :1])
    assert kk.shape[-2] == 4


def test_kv_cache_over_preallocated_buffers():
    """KVCache.over: appends land in the given buffers in place (no copy while
    they have room), the views cover the filled slots, and a buffer outgrown
    is replaced by a larger copy holding the same history."""
    kb = [torch.full((2, 3, 8, 4), -1.0) for _ in range(2)]
    vb = [torch.full((2, 3, 8, 4), -1.0) for _ in range(2)]
    c = g.KVCache.over(kb, vb)
    assert c.seq_len == 0 and c.length(1) == 0
    k = torch.arange(2 * 3 * 5 * 4, dtype=torch.float32).view(2, 3, 5, 4)
    kk, vv = c.update(1, k, -k)
    assert kk.data_ptr() == kb[1].data_ptr() and vv.data_ptr() == vb[1].data_ptr()
    assert torch.equal(kb[1][:, :, :5], k) and torch.equal(vb[1][:, :, :5], -k)
    assert bool((kb[1][:, :, 5:] == -1).all()) and bool((kb[0] == -1).all())
    assert c.length(1) == 5 and c.length(0) == 0
    kk, _ = c.update(1, k, k)  # 10 > 8 slots: grown
    assert kk.shape[-2] == 10 and kk.data_ptr() != kb[1].data_ptr()
    assert torch.equal(kk[:, :, :5], k) and torch.equal(kk[:, :, 5:], k)


def test_kv_cache_reference_constructor():
    """KVCache(keys=..., values=...) as the reference's dataclass is built
    (model.py:106-126): filled histories per layer (None: empty), lengths from
    them, appends continue the history; mismatched lists are refused."""
    k0 = torch.arange(2 * 3 * 4 * 4, dtype=torch.float32).view(2, 3, 4, 4)
    c = g.KVCache(keys=[k0, None], values=[-k0, None])
    assert c.seq_len == 4 and c.length(1) == 0
    assert torch.equal(c.keys[0], k0) and torch.equal(c.values[0], -k0) and c.keys[1] is None
    step = torch.ones(2, 3, 1, 4)
    kk, vv = c.update(0, step, -step)
    assert torch.equal(kk, torch.cat([k0, step], dim=2)) and torch.equal(vv, torch.cat([-k0, -step], dim=2))
    assert g.KVCache.empty(3).length(2) == 0
    with pytest.raises(ValueError):
        g.KVCache(keys=[k0], values=[])
    with pytest.raises(ValueError):
        g.KVCache(keys=[k0], values=[None])


def test_synthetic_token_stream_windows():
    """The perplexity windows: non-overlapping blocks of T predictions that
    share one id with the next (ids[wT : wT + T + 1]), y = x shifted by one,
    batch_size windows per batch, the limit honoured, seeded."""
    T, n = 16, 16 * 10 + 5
    ds = g.SyntheticTokenStream(50, n, T, seed=3)
    assert torch.equal(ds.tokens, g.SyntheticTokenStream(50, n, T, seed=3).tokens)
    assert not torch.equal(ds.tokens, g.SyntheticTokenStream(50, n, T, seed=4).tokens)
    batches = ds.sequential_batches("val", batch_size=4)
    assert [tuple(x.shape) for x, _ in batches] == [(4, T), (4, T), (2, T)]   # 10 windows
    flat_x = torch.cat([x for x, _ in batches]).reshape(-1)
    flat_y = torch.cat([y for _, y in batches]).reshape(-1)
    assert torch.equal(flat_x, ds.tokens[: 10 * T]) and torch.equal(flat_y, ds.tokens[1 : 10 * T + 1])
    assert len(ds.sequential_batches("val", batch_size=4, limit=2)) == 2
    assert int(ds.tokens.max()) < 50 and int(ds.tokens.min()) >= 0
    with pytest.raises(ValueError):
        g.SyntheticTokenStream(50, T + 1, T)
    with pytest.raises(ValueError):
        ds.sequential_batches("test", batch_size=4)


def test_last_only_logits_equal_the_last_row():
    """``last_only`` (used by the decoders' prefill) gives the last position's
    logits of the full forward; it refuses a loss, which needs every row."""
    torch.manual_seed(0)
    cfg = g.GPTConfig(vocab_size=64, n_positions=24, n_layer=2, n_head=4, n_embd=32)
    m = g.GPT(cfg).eval()
    idx = torch.randint(0, 64, (3, 10))
    with torch.no_grad():
        full = m(idx)["logits"]
        last = m(idx, last_only=True)["logits"]
    assert last.shape == (3, 1, 64)
    assert torch.allclose(last[:, 0], full[:, -1], atol=1e-6, rtol=1e-5)
    with pytest.raises(ValueError):
        m(idx, targets=idx, last_only=True)


@pytest.mark.parametrize("field,value", [("norm_position", "post"), ("pos_embedding", "sinusoidal"),
                                         ("activation", "relu"), ("n_kv_head", 2), ("use_sdpa", True),
                                         ("tie_weights", False)])
def test_model_refuses_layouts_outside_gpt2(field, value):
    """The host model is GPT-2's inference layout; the reference's ablation
    switches raise instead of silently computing something else."""
    cfg = g.GPTConfig(vocab_size=64, n_positions=16, n_layer=1, n_head=4, n_embd=32, **{field: value})
    with pytest.raises(NotImplementedError, match=field):
        g.GPT(cfg)


def test_kv_cache_growth_equals_concatenation():
    """Appends of 1..7 rows across several capacity doublings hold exactly the
    concatenated history, per layer, with per-layer lengths."""
    gen = torch.Generator().manual_seed(1)
    c = g.KVCache.empty(2)
    hist = []
    for t in (5, 1, 1, 7, 3, 1, 1, 6, 2):
        k = torch.randn(2, 3, t, 4, generator=gen)
        v = torch.randn(2, 3, t, 4, generator=gen)
        hist.append((k, v))
        kk, vv = c.update(0, k, v)
        assert torch.equal(kk, torch.cat([h[0] for h in hist], dim=2))
        assert torch.equal(vv, torch.cat([h[1] for h in hist], dim=2))
    assert c.seq_len == 27 and c.length(1) == 0
    assert torch.equal(c.keys[0], kk) and c.keys[1] is None


def test_time_call_and_bench_rows_on_cpu():
    calls = []
    t = g.time_call(lambda: calls.append(1), "cpu", repeats=4, warmup=2)
    assert len(calls) == 6 and set(t) == {"median_s", "min_s", "mean_s", "std_s"} and t["min_s"] >= 0
    torch.manual_seed(0)
    m = g.GPT(g.GPTConfig(vocab_size=64, n_positions=24, n_layer=1, n_head=4, n_embd=32))
    rows = g.benchmark_generation(m, [5, 20], new_tokens=6, device="cpu", repeats=1, warmup=0, mode="eager")
    assert [(r.use_cache, r.prompt_len) for r in rows] == [(True, 5), (False, 5)]   # 20 + 6 > 24: skipped
    d = rows[0].to_dict()
    assert list(d)[:10] == ["use_cache", "prompt_len", "new_tokens", "batch_size", "median_s", "min_s", "std_s",
                            "ms_per_token", "tokens_per_s", "device"]
    assert d["decoder"] == "eager" and d["tokens_per_s"] == pytest.approx(6 / d["median_s"])
    with pytest.raises(ValueError):
        g.benchmark_generation(m, [5], mode="sampled", device="cpu")


def test_paired_loss_delta():
    from gpt2_harness_amd.experiment import paired_loss_delta

    d = paired_loss_delta([2.0, 2.5, 3.0, 3.5], [1.9, 2.3, 2.9, 3.3])
    assert d["per_chunk"] == pytest.approx([0.1, 0.2, 0.1, 0.2])
    assert d["mean"] == pytest.approx(0.15) and d["stderr"] == pytest.approx(0.05 / 3 ** 0.5)   # sd 0.1/sqrt(3), n 4
    assert d["distinguishable"]
    assert not paired_loss_delta([1.0, 1.2], [1.1, 1.1])["distinguishable"]   # mean 0
    with pytest.raises(ValueError):
        paired_loss_delta([1.0], [1.0, 2.0])


def test_chunk_spread_statistics():
    """The spread of perplexity_with_error_bars: mean and sample standard
    deviation of the chunk losses and of exp(loss), and exp(mean loss)."""
    from gpt2_harness_amd.quantization import _chunk_spread

    d = _chunk_spread([1.0, 2.0, 4.0])
    mean = 7.0 / 3.0
    sd = math.sqrt(((1 - mean) ** 2 + (2 - mean) ** 2 + (4 - mean) ** 2) / 2)
    p = [math.exp(1.0), math.exp(2.0), math.exp(4.0)]
    pm = sum(p) / 3
    psd = math.sqrt(sum((v - pm) ** 2 for v in p) / 2)
    assert d["n_chunks"] == 3 and d["chunk_losses"] == [1.0, 2.0, 4.0]
    assert abs(d["loss_mean"] - mean) < 1e-12 and abs(d["loss_std"] - sd) < 1e-12
    assert abs(d["ppl_mean"] - pm) < 1e-9 and abs(d["ppl_std"] - psd) < 1e-9
    assert abs(d["ppl_of_mean_loss"] - math.exp(mean)) < 1e-9
    one = _chunk_spread([0.5])
    assert one["loss_std"] == 0.0 and one["ppl_std"] == 0.0 and one["ppl_mean"] == math.exp(0.5)


def test_greedy_agreement_reports_first_divergence():
    """bench.greedy_agreement: equal generations report the last-step logit
    difference; a token planted at step 5 of sequence 2 (and one later in
    sequence 0) is reported as the first divergence, with the oracle's gap
    there."""
    import bench

    gen = torch.Generator().manual_seed(0)
    want = torch.randint(0, 100, (3, 4 + 8), generator=gen)
    gaps = torch.rand(8, 3, generator=gen) + 0.5
    gaps[5, 2] = 0.001
    last = torch.randn(3, 100, generator=gen)
    a = bench.greedy_agreement(want.clone(), want, gaps, last + 1e-6, last, 4)
    assert a["tokens_match"] and a["steps"] == 8 and a["sequences"] == 3
    assert abs(a["last_step_max_abs_logit_diff"] - 1e-6) < 1e-7 and "first_divergence" not in a
    got = want.clone()
    got[2, 4 + 5] += 1
    got[0, 4 + 7] += 1
    b = bench.greedy_agreement(got, want, gaps, None, last, 4)
    assert not b["tokens_match"]
    assert b["first_divergence"] == {"step": 5, "sequence": 2, "oracle_top2_margin": float(gaps[5, 2]),
                                     "steps_all_equal": 5}
    assert abs(b["min_top2_margin"] - 0.001) < 1e-6
