"""The quantized model end to end on the GPU.

Greedy tokens must be identical to the reference's: the fixtures in
``golden/reference_decode.json`` were recorded from the reference package
itself (seed-0 init, ``quantize_model``, ``generate``), and the oracle's
restatement reproduces them bit for bit on the CPU (``test_oracle.py``).
The GPU path computes the four quantized Linears with the HIP kernels in fp32
(W8A32 / W4A32), everything else with fp32 torch ops.
"""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

import gpt2_harness_amd as g
from oracle import model as OM

pytestmark = pytest.mark.gpu


def _model(cfg_dict, dev):
    torch.manual_seed(0)
    return g.GPT(g.GPTConfig(**cfg_dict)).to(dev).eval()


@pytest.mark.parametrize("bits", [8, 4])
def test_tiny_greedy_matches_reference(reference_decode, dev, bits):
    e = reference_decode["tiny"]
    qm, stats = g.quantize_model(_model(e["config"], dev), bits)
    gr = e[f"greedy_int{bits}"]
    prompt = OM.benchmark_prompt(e["config"]["vocab_size"], *gr["prompt_shape"]).to(dev)
    out = g.generate(qm, prompt, gr["new_tokens"])
    assert out.cpu().tolist() == gr["ids"]
    ref = e[f"stats_int{bits}"]
    for k in ("bits", "granularity", "include_embedding", "n_quantized_tensors", "n_quantized_params",
              "n_total_params", "fp32_bytes"):
        assert stats[k] == ref[k], k


def test_gpt2_small_int8_greedy_matches_reference(reference_decode, dev):
    """The headline parity case: GPT-2 small, seed 0, int8 per-channel,
    64-token prompt, 64 greedy tokens."""
    e = reference_decode["gpt2_small"]
    model = _model(e["config"], dev)
    sd = model.state_dict()
    for k, h in e["param_sha256"].items():
        assert hashlib.sha256(sd[k].cpu().contiguous().numpy().tobytes()).hexdigest() == h, k
    qm, stats = g.quantize_model(model, 8)
    assert stats["n_quantized_tensors"] == 48 and stats["n_quantized_params"] == 84_934_656
    assert abs(stats["packed_bytes"] - e["stats_int8"]["packed_bytes"]) < 0.01 * e["stats_int8"]["packed_bytes"]
    gr = e["greedy_int8"]
    prompt = OM.benchmark_prompt(e["config"]["vocab_size"], *gr["prompt_shape"]).to(dev)
    out = g.generate(qm, prompt, gr["new_tokens"])
    assert out.cpu().tolist() == gr["ids"]


def test_quantlinear_weight_is_reference_w_hat(reference_decode, dev):
    e = reference_decode["tiny"]
    model = _model(e["config"], dev)
    original = model.h[0].mlp.c_fc.weight.detach().clone()
    qm, _ = g.quantize_model(model, 8)
    p = OM.init_params(OM.Shape(**{k: e["config"][k] for k in ("vocab_size", "n_positions", "n_layer", "n_head",
                                                                 "n_embd")}), 0)
    qp, _ = OM.quantize_params(p, 8)
    for name in ("h.0.attn.c_attn", "h.1.attn.c_proj", "h.2.mlp.c_fc", "h.2.mlp.c_proj"):
        got = qm.get_submodule(name).weight.cpu()
        assert torch.equal(got, qp[name + ".weight"]), name
    assert torch.equal(model.h[0].mlp.c_fc.weight, original), "quantize_model mutated its input"
    assert isinstance(qm.h[0].mlp.c_fc, g.QuantLinear)
    assert not torch.equal(qm.h[0].mlp.c_fc.weight, original)


@pytest.mark.parametrize("granularity", ["per_tensor", "per_channel"])
@pytest.mark.parametrize("bits", [8, 4, 6])
def test_tiny_greedy_matches_oracle_all_schemes(reference_decode, dev, granularity, bits):
    e = reference_decode["tiny"]
    c = e["config"]
    shp = OM.Shape(c["vocab_size"], c["n_positions"], c["n_layer"], c["n_head"], c["n_embd"])
    qp, _ = OM.quantize_params(OM.init_params(shp, 0), bits, granularity)
    prompt = OM.benchmark_prompt(shp.vocab_size, 2, 11)
    want, margins = OM.generate_greedy(qp, shp, prompt, 30)
    qm, _ = g.quantize_model(_model(c, dev), bits, granularity)
    got = g.generate(qm, prompt.to(dev), 30)
    assert got.cpu().tolist() == want.tolist(), f"min margin {min(margins):.3g}"


def test_cached_equals_uncached_on_gpu(reference_decode, dev):
    qm, _ = g.quantize_model(_model(reference_decode["tiny"]["config"], dev), 8)
    prompt = OM.benchmark_prompt(97, 2, 5).to(dev)
    a = g.generate(qm, prompt, 40, use_cache=True)
    b = g.generate(qm, prompt, 40, use_cache=False)
    assert torch.equal(a, b)


def test_logits_close_to_oracle(reference_decode, dev):
    e = reference_decode["tiny"]
    c = e["config"]
    shp = OM.Shape(c["vocab_size"], c["n_positions"], c["n_layer"], c["n_head"], c["n_embd"])
    qp, _ = OM.quantize_params(OM.init_params(shp, 0), 8)
    idx = OM.benchmark_prompt(shp.vocab_size, 2, 11)
    want = OM.forward(qp, shp, idx)
    qm, _ = g.quantize_model(_model(c, dev), 8)
    with torch.no_grad():
        got = qm(idx.to(dev))["logits"].cpu()
    assert (got - want).abs().max().item() <= 1e-4 * want.abs().max().item()


def test_include_embedding_writes_w_hat(reference_decode, dev):
    e = reference_decode["tiny"]
    model = _model(e["config"], dev)
    qm, stats = g.quantize_model(model, 8, include_embedding=True)
    assert stats["n_quantized_tensors"] == 4 * e["config"]["n_layer"] + 1
    w = model.wte.weight.detach().cpu().numpy()
    from oracle import quant as OQ

    assert np.array_equal(qm.wte.weight.detach().cpu().numpy(), OQ.quantize_dequantize(w, 8))
    # the tied head now reads the same codes: its W_hat is the embedding's
    assert isinstance(qm.lm_head, g.QuantLinear)
    assert torch.equal(qm.lm_head.weight, qm.wte.weight)
    assert model.lm_head.weight is model.wte.weight   # the source model keeps its tie


def test_groupwise_model_decodes(reference_decode, dev):
    qm, stats = g.quantize_model(_model(reference_decode["tiny"]["config"], dev), 4, group_size=32)
    assert stats["group_size"] == 32
    out = g.generate(qm, OM.benchmark_prompt(97, 1, 4).to(dev), 8)
    assert out.shape == (1, 12)


def test_cpu_model_is_refused(reference_decode):
    torch.manual_seed(0)
    model = g.GPT(g.GPTConfig(**reference_decode["tiny"]["config"]))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        g.quantize_model(model, 8)


@pytest.mark.parametrize("bits", [8, 4])
def test_graph_decode_matches_reference_tiny(reference_decode, dev, bits):
    """The captured decode step gives the reference's tokens, and a reused
    graph replays identically after eager work in between."""
    e = reference_decode["tiny"]
    qm, _ = g.quantize_model(_model(e["config"], dev), bits)
    gr = e[f"greedy_int{bits}"]
    prompt = OM.benchmark_prompt(e["config"]["vocab_size"], *gr["prompt_shape"]).to(dev)
    dec = g.GraphDecoder(qm, prompt.size(0), prompt.size(1) + gr["new_tokens"])
    first = g.generate_graph(qm, prompt, gr["new_tokens"], decoder=dec)
    assert first.cpu().tolist() == gr["ids"]
    eager = g.generate(qm, prompt, 5)  # eager work between replays
    torch.cuda.synchronize()
    again = g.generate_graph(qm, prompt, gr["new_tokens"], decoder=dec)
    assert torch.equal(first, again)
    assert eager.cpu().tolist() == [r[: prompt.size(1) + 5] for r in gr["ids"]]


@pytest.mark.parametrize("head_screen", ["int8", "bf16"])
def test_graph_decode_matches_reference_gpt2_small(reference_decode, dev, head_screen):
    """The captured fused decode (one sequence: the screened tied head from
    its int8 or its bf16 copy) gives the reference's 64 + 64 tokens."""
    e = reference_decode["gpt2_small"]
    qm, _ = g.quantize_model(_model(e["config"], dev), 8)
    gr = e["greedy_int8"]
    prompt = OM.benchmark_prompt(e["config"]["vocab_size"], *gr["prompt_shape"]).to(dev)
    dec = g.FusedDecoder(qm, prompt.size(0), prompt.size(1) + gr["new_tokens"], head_screen=head_screen)
    assert dec.screen and dec.screen_i8 == (head_screen == "int8")
    out = g.generate_graph(qm, prompt, gr["new_tokens"], decoder=dec)
    assert out.cpu().tolist() == gr["ids"]


@pytest.mark.parametrize("batch", [8, 32])
def test_batched_fused_decode_matches_oracle(reference_decode, dev, batch):
    """Batched greedy decode (the matrix-core decode linears at M = batch, the
    three-plane prefill at M = batch * T >= 128) against the oracle's fp32
    CPU generation of the same seed-0 model: identical token ids."""
    c = dict(vocab_size=97, n_positions=96, n_layer=2, n_head=2, n_embd=128)  # head_dim 64: the fused decoder
    shp = OM.Shape(c["vocab_size"], c["n_positions"], c["n_layer"], c["n_head"], c["n_embd"])
    qp, _ = OM.quantize_params(OM.init_params(shp, 0), 8)
    prompt = OM.benchmark_prompt(shp.vocab_size, batch, 16)
    want, margins = OM.generate_greedy(qp, shp, prompt, 20)
    qm, _ = g.quantize_model(_model(c, dev), 8)
    dec = g.make_decoder(qm, batch, 36)
    assert isinstance(dec, g.FusedDecoder)
    got = g.generate_graph(qm, prompt.to(dev), 20, decoder=dec)
    assert got.cpu().tolist() == want.tolist(), f"min margin {min(margins):.3g}"


MINI = dict(vocab_size=97, n_positions=96, n_layer=2, n_head=2, n_embd=128)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("batch", [1, 8])
def test_quantized_head_matches_oracle(dev, bits, batch):
    """include_embedding (the reference's SCHEMES row 5): wte holds the fp32
    W_hat for the lookup and the tied head runs on the same codes; eager
    generate and the captured fused decode give the oracle's tokens, whose
    head is the fp32 W_hat (quantization.py:189-197)."""
    shp = OM.Shape(MINI["vocab_size"], MINI["n_positions"], MINI["n_layer"], MINI["n_head"], MINI["n_embd"])
    qp, _ = OM.quantize_params(OM.init_params(shp, 0), bits, include_embedding=True)
    prompt = OM.benchmark_prompt(shp.vocab_size, batch, 16)
    want, margins = OM.generate_greedy(qp, shp, prompt, 20)
    qm, stats = g.quantize_model(_model(MINI, dev), bits, include_embedding=True)
    assert stats["n_quantized_tensors"] == 4 * MINI["n_layer"] + 1
    assert isinstance(qm.lm_head, g.QuantLinear)
    assert torch.equal(qm.lm_head.weight, qm.wte.weight)        # one W_hat, two storages
    assert torch.equal(qm.wte.weight.cpu(), qp["wte.weight"])    # the oracle's W_hat, bit for bit
    eager = g.generate(qm, prompt.to(dev), 20)
    assert eager.cpu().tolist() == want.tolist(), f"min margin {min(margins):.3g}"
    dec = g.make_decoder(qm, batch, 36)
    assert isinstance(dec, g.FusedDecoder)
    got = g.generate_graph(qm, prompt.to(dev), 20, decoder=dec)
    assert got.cpu().tolist() == want.tolist(), f"min margin {min(margins):.3g}"


def test_quantized_head_gpt2_small_matches_oracle(dev):
    """GPT-2 small int8 per-channel + embedding, 64-token prompt, 64 greedy
    tokens through the captured fused decode (int8 head GEMV over 50257
    rows) against the oracle's fp32 CPU generation."""
    shp = OM.GPT2_SMALL
    qp, _ = OM.quantize_params(OM.init_params(shp, 0), 8, include_embedding=True)
    prompt = OM.benchmark_prompt(shp.vocab_size, 1, 64)
    want, margins = OM.generate_greedy(qp, shp, prompt, 64)
    cfg = dict(vocab_size=shp.vocab_size, n_positions=shp.n_positions, n_layer=shp.n_layer, n_head=shp.n_head,
               n_embd=shp.n_embd)
    qm, _ = g.quantize_model(_model(cfg, dev), 8, include_embedding=True)
    got = g.generate_graph(qm, prompt.to(dev), 64)
    assert got.cpu().tolist() == want.tolist(), f"min margin {min(margins):.3g}"
