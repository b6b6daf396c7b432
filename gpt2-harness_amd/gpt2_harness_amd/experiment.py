"""The quantization experiment: quality, size and speed per scheme, on the GPU.

The reference's ``scripts/run_quantization.py`` (``:31-158``) scores an fp32
model and five quantization schemes on held-out perplexity with error bars,
records ``quantize_model``'s size statistics, and leaves ``speed`` empty (its
quantized weights are fp32 ``W_hat``, so there is nothing faster to time,
``results/quantization.json:280``). :func:`run_quantization_table` produces the
same table -- ``{"baseline", "rows", "meta"}`` with one
:class:`~gpt2_harness_amd.quantization.QuantResult` row per scheme -- with
every forward pass on the MI355X kernels and ``speed`` measured: the greedy
decode of :func:`~gpt2_harness_amd.benchmark.benchmark_generation` at the
reference's settings (64-token prompt, 16 new tokens, 2 repeats, 1 warmup,
cached arm only) through the graph-captured decoder.

Quality deltas are paired per chunk: every scheme is scored on the same
chunks as the fp32 baseline, so the chunk-to-chunk spread is common to both
arms and cancels; a shift is ``distinguishable`` when its mean exceeds twice
its standard error, and the highlighted row is the most compressed scheme
whose mean shift stays below :data:`PRACTICAL_NATS`.
"""

from __future__ import annotations

import math
import statistics
from typing import Any

import torch

from .benchmark import benchmark_generation, model_size_bytes
from .quantization import QuantResult, perplexity_with_error_bars, quantize_model

__all__ = ["PRACTICAL_NATS", "SCHEMES", "paired_loss_delta", "run_quantization_table"]

#: ``(label, bits, granularity, include_embedding)`` (``run_quantization.py:31-37``).
SCHEMES: tuple[tuple[str, int, str, bool], ...] = (
    ("int8 per-channel", 8, "per_channel", False),
    ("int8 per-tensor", 8, "per_tensor", False),
    ("int4 per-channel", 4, "per_channel", False),
    ("int4 per-tensor", 4, "per_tensor", False),
    ("int8 per-channel + embedding", 8, "per_channel", True),
)

#: A mean loss shift below this many nats (about 1% in perplexity) counts as
#: negligible for the highlight (``run_quantization.py:29``).
PRACTICAL_NATS = 0.01


def paired_loss_delta(losses: list[float], base: list[float]) -> dict[str, Any]:
    """Per-chunk ``loss - base_loss`` with its mean, spread and standard error."""
    if len(losses) != len(base):
        raise ValueError(f"{len(losses)} chunk losses against {len(base)} baseline chunks")
    d = [a - b for a, b in zip(losses, base)]
    n = len(d)
    mean = statistics.fmean(d) if d else 0.0
    sd = statistics.stdev(d) if n > 1 else 0.0
    se = sd / math.sqrt(n) if n else 0.0
    return {"mean": mean, "sd": sd, "stderr": se, "n_chunks": n, "per_chunk": d,
            "distinguishable": bool(se and abs(mean) > 2.0 * se)}


def _speed(model, device, enabled: bool) -> dict[str, Any]:
    if not enabled:
        return {}
    row = benchmark_generation(model, prompt_lens=[64], new_tokens=16, device=device, repeats=2, warmup=1,
                               both_arms=False)[0]
    # the speed's memory cost beside quantize_model's packed_bytes: weight
    # copies the decoder keeps on the device in addition to the model's codes
    return {"ms_per_token": row.ms_per_token, "tokens_per_s": row.tokens_per_s, "decoder": row.extra["decoder"],
            "decoder_extra_weight_bytes": row.extra.get("decoder_extra_weight_bytes", 0)}


@torch.no_grad()
def run_quantization_table(
    model,
    dataset,
    *,
    n_chunks: int = 8,
    batches_per_chunk: int = 2,
    batch_size: int = 4,
    speed: bool = True,
    device: str | torch.device = "cuda",
    schemes: tuple[tuple[str, int, str, bool], ...] = SCHEMES,
) -> dict[str, Any]:
    """Score the fp32 ``model`` and each scheme of ``schemes`` on ``dataset``.

    ``dataset`` provides ``sequential_batches(split, batch_size=, limit=)``
    (the reference's ``TokenDataset`` or
    :class:`~gpt2_harness_amd.quantization.SyntheticTokenStream`). Returns
    ``{"baseline": {...}, "rows": [QuantResult.to_dict(), ...], "meta": {...}}``.
    """
    device = torch.device(device)
    model = model.to(device).eval()
    scoring = dict(n_chunks=n_chunks, batches_per_chunk=batches_per_chunk, batch_size=batch_size, device=device)
    base = perplexity_with_error_bars(model, dataset, **scoring)
    baseline = {**base, "bytes": model_size_bytes(model), "speed": _speed(model, device, speed)}
    rows = []
    for label, bits, granularity, with_embedding in schemes:
        qm, stats = quantize_model(model, bits, granularity, include_embedding=with_embedding)
        quality = perplexity_with_error_bars(qm, dataset, **scoring)
        quality["paired_loss_delta"] = paired_loss_delta(quality["chunk_losses"], base["chunk_losses"])
        rows.append(QuantResult(label, bits, granularity, with_embedding, stats, quality,
                                _speed(qm, device, speed)).to_dict())
        del qm
    negligible = [r for r in rows if abs(r["quality"]["paired_loss_delta"]["mean"]) < PRACTICAL_NATS]
    if negligible:
        best = max(negligible, key=lambda r: r["compression_ratio"])["label"]
        for r in rows:
            r["highlight"] = r["label"] == best
    meta = {
        "device": str(device),
        "device_name": torch.cuda.get_device_name(device) if device.type == "cuda" else "cpu",
        "practical_threshold_nats": PRACTICAL_NATS,
        "n_chunks": n_chunks,
        "batches_per_chunk": batches_per_chunk,
        "batch_size": batch_size,
        "speed_measured": speed,
        "note": ("quantized Linears run on int8 / int4 codes in HBM through the HIP kernels; speed is greedy "
                 "decode through the graph-captured decoder (64-token prompt, 16 new tokens, median of 2)"),
    }
    return {"baseline": baseline, "rows": rows, "meta": meta}
