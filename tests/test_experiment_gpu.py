"""The quantization experiment and generation timing on the GPU.

* ``run_quantization_table``: the five schemes of ``run_quantization.py:31-37``
  on seed-0 GPT-2 small over synthetic tokens, rows in the reference's
  ``QuantResult.to_dict`` layout with ``quality.paired_loss_delta``
  (``:88-101``) and a measured ``speed`` (``:56-63``); the size statistics of
  a row are those ``quantize_model`` reports for the same scheme, and coarser
  schemes cost more loss.
* ``benchmark_generation``: the graph-captured arm gives the eager loop's
  tokens and the rows carry the reference's fields.
* ``gelu_tanh`` keeps autograd: a model being trained differentiates through
  the torch ops, while no-grad fp32 tensors take the one-pass HIP kernel.
"""

from __future__ import annotations

import math

import pytest
import torch

import gpt2_harness_amd as g
from gpt2_harness_amd.model import gelu_tanh

pytestmark = pytest.mark.gpu

ROW_KEYS = {"label", "bits", "granularity", "include_embedding", "n_quantized_tensors", "n_quantized_params",
            "n_total_params", "fraction_quantized", "packed_bytes", "fp32_bytes", "compression_ratio", "quality",
            "speed"}


def test_quantization_table_gpt2_small(dev):
    torch.manual_seed(0)
    model = g.GPT(g.GPTConfig()).to(dev).eval()
    ds = g.SyntheticTokenStream(50257, 4 * 2 * 4 * 128 + 1, 128, seed=0)
    table = g.run_quantization_table(model, ds, n_chunks=4, batches_per_chunk=2, batch_size=4, device=dev)
    rows = {r["label"]: r for r in table["rows"]}
    assert list(rows) == [s[0] for s in g.SCHEMES]
    base = table["baseline"]
    assert base["n_chunks"] == 4 and len(base["chunk_losses"]) == 4
    assert base["bytes"] == 124_439_808 * 4   # fp32 parameters, the tied matrix once
    for label, bits, gran, emb in g.SCHEMES:
        r = rows[label]
        assert ROW_KEYS <= set(r), set(ROW_KEYS) - set(r)
        assert (r["bits"], r["granularity"], r["include_embedding"]) == (bits, gran, emb)
        assert r["n_quantized_tensors"] == 48 + int(emb)
        pd = r["quality"]["paired_loss_delta"]
        assert pd["n_chunks"] == 4
        assert pd["per_chunk"] == pytest.approx([a - b for a, b in zip(r["quality"]["chunk_losses"],
                                                                      base["chunk_losses"])])
        assert math.isfinite(pd["mean"]) and pd["stderr"] >= 0
        assert r["speed"]["tokens_per_s"] > 0 and r["speed"]["decoder"] == "FusedDecoder"
        assert r["packed_bytes"] < r["fp32_bytes"]
    d = {k: abs(rows[k]["quality"]["paired_loss_delta"]["mean"]) for k in rows}
    assert d["int8 per-channel"] < d["int4 per-tensor"]
    assert d["int8 per-channel"] < d["int4 per-channel"]
    assert rows["int4 per-channel"]["packed_bytes"] < rows["int8 per-channel"]["packed_bytes"]
    assert sum(bool(r.get("highlight")) for r in table["rows"]) <= 1
    assert table["meta"]["speed_measured"] and table["meta"]["n_chunks"] == 4


def test_benchmark_generation_graph_arm_matches_eager(reference_decode, dev):
    e = reference_decode["tiny"]
    torch.manual_seed(0)
    qm, _ = g.quantize_model(g.GPT(g.GPTConfig(**e["config"])).to(dev).eval(), 8)
    rows = g.benchmark_generation(qm, [8, 60], new_tokens=10, batch_size=2, device=dev, repeats=2, warmup=1)
    assert [(r.use_cache, r.prompt_len, r.extra["decoder"]) for r in rows] == [(True, 8, "GraphDecoder"),
                                                                            (False, 8, "eager")]
    for r in rows:
        assert r.tokens_per_s == pytest.approx(10 * 2 / r.median_s) and r.min_s <= r.median_s
    torch.manual_seed(0)
    prompt = torch.randint(0, e["config"]["vocab_size"], (2, 8)).to(dev)
    assert torch.equal(g.generate_graph(qm, prompt, 10), g.generate(qm, prompt, 10))


def test_gelu_tanh_gradient_through_mlp(dev):
    """An unquantized MLP in training: the output has a grad_fn and the
    gradients of c_fc / c_proj equal those of the torch-op chain; without
    grad the fp32 GPU tensor takes the HIP pass and gives the same values."""
    torch.manual_seed(0)
    mlp = g.model.MLP(g.GPTConfig(n_embd=64, n_head=4)).to(dev)
    x = torch.randn(3, 5, 64, device=dev, requires_grad=True)
    y = mlp(x)
    assert y.grad_fn is not None
    y.square().sum().backward()
    got = (x.grad.clone(), mlp.c_fc.weight.grad.clone(), mlp.c_proj.weight.grad.clone())
    for t in (x, mlp.c_fc.weight, mlp.c_proj.weight):
        t.grad = None
    h = mlp.c_fc(x)
    ref = mlp.c_proj(0.5 * h * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (h + 0.044715 * h.pow(3)))))
    ref.square().sum().backward()
    for a, b in zip(got, (x.grad, mlp.c_fc.weight.grad, mlp.c_proj.weight.grad)):
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-6)
    with torch.no_grad():
        z = torch.randn(1000, device=dev)
        assert torch.allclose(gelu_tanh(z), 0.5 * z * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi)
                                                                       * (z + 0.044715 * z.pow(3)))),
                              rtol=4e-6, atol=1e-7)
