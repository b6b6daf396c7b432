"""The packed checkpoint (the reference's ``packed_size_bytes`` payload,
``quantization.py:219-259``) written by ``quantize_model(save_to=)`` and read
back by ``load_packed``, and perplexity on the GPU.

* the file holds exactly the reference's keys (``name.q``, ``name.scale``,
  ``name.shape`` for the quantized tensors, every other unique parameter in
  fp32) and its size is ``stats["packed_bytes"]``;
* a model of the same configuration with other weights, filled from the file,
  computes bit-identical logits to the quantized model it was saved from, and
  its greedy tokens are the reference's (GPT-2 small int8);
* ``perplexity_with_error_bars`` over the prefill-shaped Linears (M = 4 x 64)
  on the GPU agrees with the oracle's fp32 CPU forward of the same quantized
  model on the same synthetic windows.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import gpt2_harness_amd as g
from oracle import model as OM

pytestmark = pytest.mark.gpu

MINI = dict(vocab_size=97, n_positions=96, n_layer=2, n_head=2, n_embd=128)
TARGETS = ("attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj")


def _model(cfg, dev, seed=0):
    torch.manual_seed(seed)
    return g.GPT(g.GPTConfig(**cfg)).to(dev).eval()


SCHEMES = [
    dict(bits=8, granularity="per_channel"),
    dict(bits=8, granularity="per_tensor"),
    dict(bits=4, granularity="per_channel"),
    dict(bits=4, granularity="per_tensor"),
    dict(bits=3, granularity="per_channel"),
    dict(bits=8, granularity="per_channel", include_embedding=True),
    dict(bits=4, granularity="per_channel", group_size=32),
]


@pytest.mark.parametrize("scheme", SCHEMES, ids=lambda s: "-".join(str(v) for v in s.values()))
def test_packed_roundtrip(dev, tmp_path, scheme):
    path = tmp_path / "packed.pt"
    qm, stats = g.quantize_model(_model(MINI, dev), save_to=path, **scheme)
    assert stats["packed_bytes"] == path.stat().st_size
    payload = torch.load(path, map_location="cpu", weights_only=True)
    names = {n for n, _ in qm.named_modules() if n.endswith(TARGETS)}
    if scheme.get("include_embedding"):
        names.add("wte")
    for n in names:
        assert {f"{n}.q", f"{n}.scale", f"{n}.shape"} <= payload.keys(), n
        assert f"{n}.weight" not in payload
    bits, gran = scheme["bits"], scheme["granularity"]
    q = payload["h.0.mlp.c_fc.q"]
    if "group_size" in scheme:
        assert q.dtype == torch.uint8 and payload["h.0.mlp.c_fc.scale"].dtype == torch.float16
    elif bits == 4:
        assert q.dtype == torch.uint8 and q.numel() == 512 * 128 // 2   # pack_int4 of the row-major codes
    else:
        assert q.dtype == torch.int8 and tuple(q.shape) == (512, 128)
        assert payload["h.0.mlp.c_fc.scale"].shape == ((512, 1) if gran == "per_channel" else ())
    assert payload["h.0.mlp.c_fc.shape"].tolist() == [512, 128]
    # every non-quantized parameter in fp32, tied lm_head once
    assert payload["h.0.ln_1.weight"].dtype == torch.float32 and "lm_head.weight" not in payload

    fresh = g.load_packed(_model(MINI, dev, seed=1), path)
    for n in names - {"wte"}:
        a, b = qm.get_submodule(n), fresh.get_submodule(n)
        assert isinstance(b, g.QuantLinear) and a.fmt == b.fmt and a.bits == b.bits, n
        assert torch.equal(a.codes, b.codes) and torch.equal(a.scale, b.scale), n
    idx = torch.randint(0, MINI["vocab_size"], (3, 40), generator=torch.Generator().manual_seed(5)).to(dev)
    la, lb = qm(idx)["logits"], fresh(idx)["logits"]
    assert torch.equal(la, lb)


def test_packed_gpt2_small_greedy_matches_reference(reference_decode, dev, tmp_path):
    """A GPT-2 small skeleton with other weights, filled from the packed
    int8 file, decodes the reference's greedy tokens."""
    e = reference_decode["gpt2_small"]
    path = tmp_path / "gpt2_int8.pt"
    qm, stats = g.quantize_model(_model(e["config"], dev), 8, save_to=path)
    del qm
    assert abs(stats["packed_bytes"] - e["stats_int8"]["packed_bytes"]) < 0.01 * e["stats_int8"]["packed_bytes"]
    loaded = g.load_packed(_model(e["config"], dev, seed=3), path)
    gr = e["greedy_int8"]
    prompt = OM.benchmark_prompt(e["config"]["vocab_size"], *gr["prompt_shape"]).to(dev)
    out = g.generate(loaded, prompt, gr["new_tokens"])
    assert out.cpu().tolist() == gr["ids"]


def test_perplexity_on_gpu_matches_oracle(dev):
    """Per-chunk mean cross entropy of the int8 model on synthetic windows
    (4 chunks x 2 batches x 4 windows of 64 predictions: M = 256 prefill
    Linears on the matrix cores) against the oracle's CPU forward of the same
    seed-0 model with the same W_hat."""
    T = 64
    ds = g.SyntheticTokenStream(MINI["vocab_size"], 4 * 2 * 4 * T + 1, T, seed=11)
    qm, _ = g.quantize_model(_model(MINI, dev), 8)
    got = g.perplexity_with_error_bars(qm, ds, n_chunks=4, batches_per_chunk=2, batch_size=4, device=dev)
    shp = OM.Shape(MINI["vocab_size"], MINI["n_positions"], MINI["n_layer"], MINI["n_head"], MINI["n_embd"])
    qp, _ = OM.quantize_params(OM.init_params(shp, 0), 8)
    batches = ds.sequential_batches("val", batch_size=4, limit=8)
    want = []
    for c in range(0, 8, 2):
        tot, n = 0.0, 0
        for x, y in batches[c : c + 2]:
            logits = OM.forward(qp, shp, x)
            tot += float(F.cross_entropy(logits.reshape(-1, logits.size(-1)), y.reshape(-1), reduction="sum"))
            n += y.numel()
        want.append(tot / n)
    assert got["n_chunks"] == 4
    for a, b in zip(got["chunk_losses"], want):
        assert abs(a - b) <= 1e-5 * abs(b), (a, b)
    assert abs(got["ppl_of_mean_loss"] - math.exp(sum(want) / 4)) <= 1e-4 * got["ppl_of_mean_loss"]
