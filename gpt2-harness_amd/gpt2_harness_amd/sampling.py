"""Greedy decode loop (``src/transformer_internals/sampling.py:100-181``).

Step 0 runs the whole prompt (prefill: the quantized Linears see M = B*T rows
and take the MFMA GEMM path for bf16 activations); every later step feeds
one token per sequence (decode: M = B, the GEMV path) and reads the rest from
the KV cache. Next token = ``argmax`` of the last position's logits;
generation stops at ``n_positions`` and, when ``eos_token_id`` is given, once
every row has emitted it. Sampling (temperature / top-k / top-p) is outside
this library's scope and raises.
"""

from __future__ import annotations

import torch

from .model import KVCache

__all__ = ["generate"]


@torch.no_grad()
def generate(
    model,
    idx: torch.Tensor,
    max_new_tokens: int,
    *,
    do_sample: bool = False,
    temperature: float = 1.0,
    top_k: int = 0,
    top_p: float = 1.0,
    eos_token_id: int | None = None,
    use_cache: bool = True,
    generator: torch.Generator | None = None,
) -> torch.Tensor:
    """Append up to ``max_new_tokens`` greedy tokens to ``idx`` ``(B, T)``."""
    if do_sample:
        raise NotImplementedError("gpt2_harness_amd implements greedy decoding only (do_sample=False)")
    was_training = model.training
    model.eval()
    try:
        n_pos = model.config.n_positions
        cache = KVCache.empty(model.config.n_layer) if use_cache else None
        finished = torch.zeros(idx.size(0), dtype=torch.bool, device=idx.device)
        for step in range(max_new_tokens):
            if idx.size(1) >= n_pos:
                break
            if cache is not None:
                step_input = idx if step == 0 else idx[:, -1:]
            else:
                step_input = idx[:, -n_pos:]
            logits = model(step_input, cache=cache)["logits"][:, -1, :]
            nxt = logits.argmax(dim=-1, keepdim=True)
            if eos_token_id is not None:
                nxt = torch.where(finished.unsqueeze(1), torch.full_like(nxt, eos_token_id), nxt)
                finished |= nxt.squeeze(1) == eos_token_id
            idx = torch.cat([idx, nxt], dim=1)
            if eos_token_id is not None and bool(finished.all()):
                break
        return idx
    finally:
        model.train(was_training)
