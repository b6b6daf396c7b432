"""Generation timing for the quantized path on the GPU.

The names, arguments and row fields are those of the reference's
``src/transformer_internals/benchmark.py`` (``:48-196``), so its result tables
read the same: :func:`time_call` (untimed warmup, then the median of timed
repeats), :func:`benchmark_generation` (prompt ``torch.manual_seed(0);
randint(0, vocab, (B, T))``, ``tokens_per_s = new_tokens * B / median``, prompt
lengths that would pass ``n_positions`` skipped) and :class:`BenchRow`.

What is timed is this library's: on the GPU each sample is bracketed by HIP
events recorded on the stream that does the work, and the cached arm runs the
graph-captured decoder (:class:`~gpt2_harness_amd.decode.FusedDecoder` or
:class:`~gpt2_harness_amd.decode.GraphDecoder`, prefill included) unless
``mode="eager"`` asks for the Python-level loop of :func:`generate`.
"""

from __future__ import annotations

import statistics
import time
from dataclasses import dataclass, field, fields
from typing import Any, Callable

import torch

from .decode import make_decoder
from .sampling import generate

__all__ = ["BenchRow", "benchmark_generation", "model_size_bytes", "synchronize", "time_call"]


def synchronize(device: torch.device | str) -> None:
    """Wait for the device's queued work (a no-op on the CPU)."""
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize(device)


def _samples(fn: Callable[[], Any], device: torch.device, repeats: int) -> list[float]:
    if device.type != "cuda":
        out = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            fn()
            out.append(time.perf_counter() - t0)
        return out
    pairs = []
    for _ in range(repeats):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        stop.record()
        pairs.append((start, stop))
    torch.cuda.synchronize(device)
    return [a.elapsed_time(b) / 1e3 for a, b in pairs]


def time_call(fn: Callable[[], Any], device: torch.device | str, repeats: int = 5,
              warmup: int = 2) -> dict[str, float]:
    """Seconds per call of ``fn``: median, min, mean and standard deviation
    over ``repeats`` calls after ``warmup`` untimed ones. ``fn`` must issue
    its device work on the current stream (or synchronise it)."""
    device = torch.device(device)
    for _ in range(warmup):
        fn()
    synchronize(device)
    s = _samples(fn, device, repeats)
    return {"median_s": statistics.median(s), "min_s": min(s), "mean_s": statistics.fmean(s),
            "std_s": statistics.stdev(s) if len(s) > 1 else 0.0}


@dataclass
class BenchRow:
    """One (prompt length, new tokens, cache arm) generation measurement."""

    use_cache: bool
    prompt_len: int
    new_tokens: int
    batch_size: int
    median_s: float
    min_s: float
    std_s: float
    ms_per_token: float
    tokens_per_s: float
    device: str
    extra: dict[str, Any] = field(default_factory=dict)

    def to_dict(self) -> dict[str, Any]:
        row = {f.name: getattr(self, f.name) for f in fields(self) if f.name != "extra"}
        row.update(self.extra)
        return row


@torch.no_grad()
def benchmark_generation(
    model,
    prompt_lens: list[int],
    new_tokens: int = 64,
    batch_size: int = 1,
    device: torch.device | str = "cuda",
    repeats: int = 3,
    warmup: int = 1,
    both_arms: bool = True,
    mode: str = "graph",
) -> list[BenchRow]:
    """Greedy generation throughput, one row per prompt length and cache arm.

    The cached arm runs ``mode`` (``"graph"``: one captured prefill and one
    captured decode step per token, decoder built once per prompt length;
    ``"eager"``: :func:`generate`); ``both_arms`` adds the uncached loop, which
    re-runs the whole window every token. The prompt is drawn on the CPU
    generator and moved to the device, so it equals the reference's CPU
    prompt.
    """
    if mode not in ("graph", "eager"):
        raise ValueError(f"mode must be 'graph' or 'eager', got {mode!r}")
    device = torch.device(device)
    model = model.to(device).eval()
    cfg = model.config
    rows: list[BenchRow] = []
    for T in prompt_lens:
        if T + new_tokens > cfg.n_positions:
            continue
        torch.manual_seed(0)
        prompt = torch.randint(0, cfg.vocab_size, (batch_size, T)).to(device)
        arms: list[tuple[bool, str, Callable[[], Any]]] = []
        extra_bytes = 0
        if mode == "graph":
            dec = make_decoder(model, batch_size, T + new_tokens)
            extra_bytes = int(getattr(dec, "extra_weight_bytes", 0))
            arms.append((True, type(dec).__name__, lambda d=dec, p=prompt: d.run(p, new_tokens)))
        else:
            arms.append((True, "eager", lambda p=prompt: generate(model, p, new_tokens)))
        if both_arms:
            arms.append((False, "eager", lambda p=prompt: generate(model, p, new_tokens, use_cache=False)))
        for use_cache, how, fn in arms:
            t = time_call(fn, device, repeats=repeats, warmup=warmup)
            rows.append(BenchRow(use_cache=use_cache, prompt_len=T, new_tokens=new_tokens, batch_size=batch_size,
                                 median_s=t["median_s"], min_s=t["min_s"], std_s=t["std_s"],
                                 ms_per_token=1e3 * t["median_s"] / new_tokens,
                                 tokens_per_s=new_tokens * batch_size / t["median_s"], device=str(device),
                                 extra={"decoder": how,
                                        "decoder_extra_weight_bytes": extra_bytes if use_cache else 0}))
    return rows


def model_size_bytes(model, count_tied_once: bool = True) -> int:
    """Bytes held by the model's parameters and buffers at their stored width
    (integer codes count one byte, nibble-packed codes half a byte each)."""
    seen: dict[int, torch.Tensor] = {}
    total = 0
    for t in list(model.parameters()) + list(model.buffers()):
        if count_tied_once:
            if id(t) in seen:
                continue
            seen[id(t)] = t
        total += t.numel() * t.element_size()
    return total
