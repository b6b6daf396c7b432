"""Timing helpers with the reference's methodology (``benchmark.py:48-196``):
warmup, device synchronisation around every sample, median of repeats, and
``benchmark_generation`` with the seeded prompt ``manual_seed(0);
randint(0, vocab, (B, T))`` and ``tokens_per_s = new_tokens * B / median``.
"""

from __future__ import annotations

import gc
import statistics
import time
from dataclasses import dataclass, field
from typing import Any

import torch

from .sampling import generate

__all__ = ["BenchRow", "benchmark_generation", "model_size_bytes", "synchronize", "time_call"]


def synchronize(device: torch.device | str) -> None:
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize()


def time_call(fn: Any, device: torch.device | str, repeats: int = 5, warmup: int = 2) -> dict[str, float]:
    for _ in range(warmup):
        fn()
    synchronize(device)
    samples: list[float] = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        synchronize(device)
        samples.append(time.perf_counter() - t0)
    return {
        "median_s": statistics.median(samples),
        "min_s": min(samples),
        "mean_s": statistics.fmean(samples),
        "std_s": statistics.stdev(samples) if len(samples) > 1 else 0.0,
    }


@dataclass
class BenchRow:
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
        return {
            "use_cache": self.use_cache, "prompt_len": self.prompt_len, "new_tokens": self.new_tokens,
            "batch_size": self.batch_size, "median_s": self.median_s, "min_s": self.min_s, "std_s": self.std_s,
            "ms_per_token": self.ms_per_token, "tokens_per_s": self.tokens_per_s, "device": self.device,
            **self.extra,
        }


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
) -> list[BenchRow]:
    device = torch.device(device)
    model = model.to(device).eval()
    rows: list[BenchRow] = []
    arms = [True, False] if both_arms else [True]
    for prompt_len in prompt_lens:
        if prompt_len + new_tokens > model.config.n_positions:
            continue
        torch.manual_seed(0)
        prompt = torch.randint(0, model.config.vocab_size, (batch_size, prompt_len), device=device)
        for use_cache in arms:
            stats = time_call(
                lambda p=prompt, uc=use_cache: generate(model, p, new_tokens, do_sample=False, use_cache=uc),
                device, repeats=repeats, warmup=warmup,
            )
            rows.append(BenchRow(
                use_cache=use_cache, prompt_len=prompt_len, new_tokens=new_tokens, batch_size=batch_size,
                median_s=stats["median_s"], min_s=stats["min_s"], std_s=stats["std_s"],
                ms_per_token=1000.0 * stats["median_s"] / new_tokens,
                tokens_per_s=new_tokens * batch_size / stats["median_s"], device=str(device),
            ))
            gc.collect()
    return rows


def model_size_bytes(model, count_tied_once: bool = True) -> int:
    """Bytes of parameters and buffers (integer codes count at their real width)."""
    tensors = list(model.parameters()) + list(model.buffers())
    if count_tied_once:
        tensors = list({id(t): t for t in tensors}.values())
    return sum(t.numel() * t.element_size() for t in tensors)
