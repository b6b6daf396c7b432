"""Functional fp32 CPU restatement of the reference's GPT-2 forward, init and
greedy decode, with simulated quantization of the four target Linears.

TEST INFRASTRUCTURE ONLY: the checker for the GPU decode loop and the timed
CPU baseline of the benchmark. The shipped library never imports it.

Restated from the reference:

* init order and RNG consumption -- ``model.py:457-518`` (module construction
  draws, ``apply(_init_weights)`` in module order, the tied ``lm_head`` redraw
  of ``wte``, then residual scaling of both ``c_proj`` weights), with
  ``nn.Linear``/``nn.Embedding`` default ``reset_parameters`` draws at
  construction;
* forward -- ``model.py:528-599`` (pre-LN blocks ``:410-427``, attention
  ``:248-320`` with the absolute-position causal mask ``:286``, explicit
  softmax path ``:300-309``, MLP with ``gelu_tanh`` ``:57-75,351-355``, tied
  fp32 ``lm_head``);
* KV cache append by concatenation -- ``model.py:153-172``;
* greedy ``generate`` -- ``sampling.py:100-181`` (prefill at step 0, then one
  token per step, ``argmax``, stop at ``n_positions``);
* ``quantize_model`` -- ``quantization.py:161-216``: the four target weights
  become ``q.float() * scale`` with ``q, scale`` from the numpy restatement of
  ``quantize_tensor``;
* prompt seeding of ``benchmark_generation`` -- ``benchmark.py:167-170``.

Pinning: ``tests/golden/reference_decode.json`` holds digests of the seed-0
GPT-2 small weights and the greedy token ids of the 64+64 int8 decode, written
by importing the reference in the development container.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import quant as Q

TARGET_SUFFIXES = ("attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj")


@dataclass(frozen=True)
class Shape:
    vocab_size: int = 50257
    n_positions: int = 1024
    n_layer: int = 12
    n_head: int = 12
    n_embd: int = 768
    layer_norm_epsilon: float = 1e-5


GPT2_SMALL = Shape()
GPT2_XL = Shape(n_layer=48, n_head=25, n_embd=1600)


def _linear_ctor_draws(out_f: int, in_f: int, bias: bool) -> None:
    """RNG draws of ``nn.Linear.reset_parameters`` (values are discarded)."""
    w = torch.empty(out_f, in_f)
    torch.nn.init.kaiming_uniform_(w, a=math.sqrt(5))
    if bias:
        bound = 1.0 / math.sqrt(in_f) if in_f > 0 else 0.0
        torch.nn.init.uniform_(torch.empty(out_f), -bound, bound)


def init_params(cfg: Shape, seed: int | None = 0) -> dict[str, torch.Tensor]:
    """Parameters of ``GPT(cfg)`` after ``torch.manual_seed(seed)``."""
    if seed is not None:
        torch.manual_seed(seed)
    C, V, P, L = cfg.n_embd, cfg.vocab_size, cfg.n_positions, cfg.n_layer
    # --- construction (reset_parameters) draws, in registration order ---
    wte = torch.empty(V, C).normal_()
    wpe = torch.empty(P, C).normal_()
    for _ in range(L):
        _linear_ctor_draws(3 * C, C, True)   # attn.c_attn
        _linear_ctor_draws(C, C, True)       # attn.c_proj
        _linear_ctor_draws(4 * C, C, True)   # mlp.c_fc
        _linear_ctor_draws(C, 4 * C, True)   # mlp.c_proj
    _linear_ctor_draws(V, C, False)          # lm_head (then tied to wte)
    # --- apply(_init_weights): children before parents, registration order ---
    p: dict[str, torch.Tensor] = {}
    wte.normal_(0.0, 0.02)
    wpe.normal_(0.0, 0.02)
    for i in range(L):
        pre = f"h.{i}."
        p[pre + "ln_1.weight"], p[pre + "ln_1.bias"] = torch.ones(C), torch.zeros(C)
        for name, (o, n) in (("attn.c_attn", (3 * C, C)), ("attn.c_proj", (C, C))):
            p[pre + name + ".weight"] = torch.empty(o, n).normal_(0.0, 0.02)
            p[pre + name + ".bias"] = torch.zeros(o)
        p[pre + "ln_2.weight"], p[pre + "ln_2.bias"] = torch.ones(C), torch.zeros(C)
        for name, (o, n) in (("mlp.c_fc", (4 * C, C)), ("mlp.c_proj", (C, 4 * C))):
            p[pre + name + ".weight"] = torch.empty(o, n).normal_(0.0, 0.02)
            p[pre + name + ".bias"] = torch.zeros(o)
    p["ln_f.weight"], p["ln_f.bias"] = torch.ones(C), torch.zeros(C)
    wte.normal_(0.0, 0.02)  # lm_head is a Linear sharing wte's storage
    p["wte.weight"], p["wpe.weight"] = wte, wpe
    # --- _apply_residual_scaling ---
    std = 0.02 / math.sqrt(2 * L)
    for i in range(L):
        p[f"h.{i}.attn.c_proj.weight"].normal_(0.0, std)
        p[f"h.{i}.mlp.c_proj.weight"].normal_(0.0, std)
    return p


def quantize_params(p: dict[str, torch.Tensor], bits: int = 8, granularity: str = "per_channel",
                    include_embedding: bool = False, impl: str = "numpy"):
    """Simulated quantization of the target weights (``quantization.py:186-197``);
    with ``include_embedding`` also ``wte`` (``:189-192``), whose ``W_hat`` the
    tied head then uses (``forward`` reads ``wte.weight`` for both).

    ``impl="c"`` codes per-channel weights with the C restatement
    (``quant_oracle.c``, equal to the numpy one on every pinned case), one
    host thread per tensor, for models too large for the numpy passes.

    Returns ``(params_with_W_hat, codes)`` where ``codes[name] = (q, scale)``.
    """
    if impl not in ("numpy", "c"):
        raise ValueError(f"impl must be 'numpy' or 'c', got {impl!r}")
    out = dict(p)
    names = []
    for key in p:
        name = key[: -len(".weight")] if key.endswith(".weight") else None
        is_emb = include_embedding and name == "wte"
        if name is not None and (name.endswith(TARGET_SUFFIXES) or is_emb):
            names.append(name)

    def code(name):
        w = p[name + ".weight"].numpy()
        if impl == "c" and granularity == "per_channel":
            return Q.c_oracle().quantize_per_channel(w, bits)
        return Q.quantize_tensor(w, bits, granularity)

    if impl == "c":
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=min(16, len(names) or 1)) as pool:
            coded = list(pool.map(code, names))
    else:
        coded = [code(n) for n in names]
    codes = {}
    for name, (q, s) in zip(names, coded):
        codes[name] = (q, s)
        out[name + ".weight"] = torch.from_numpy(q).to(torch.float32) * torch.from_numpy(np.asarray(s))
    return out, codes


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x.pow(3))))


class Cache:
    def __init__(self, n_layer: int) -> None:
        self.k: list[torch.Tensor | None] = [None] * n_layer
        self.v: list[torch.Tensor | None] = [None] * n_layer

    def length(self, layer: int) -> int:
        k = self.k[layer]
        return 0 if k is None else int(k.shape[-2])


@torch.no_grad()
def forward(p, cfg: Shape, idx: torch.Tensor, cache: Cache | None = None, last_only: bool = False) -> torch.Tensor:
    """Logits ``(B, T, V)`` of ``GPT.forward`` (fp32, explicit attention);
    ``last_only`` applies ``ln_f`` and the head to the last position only
    (``(B, 1, V)``, the rows ``generate`` reads)."""
    B, T = idx.shape
    C, H = cfg.n_embd, cfg.n_head
    hd = C // H
    past = cache.length(0) if cache is not None else 0
    if past + T > cfg.n_positions:
        raise ValueError(
            f"sequence of length {past + T} exceeds n_positions={cfg.n_positions}; "
            f"learned position embeddings cannot extrapolate"
        )
    pos = torch.arange(past, past + T, dtype=torch.long)
    x = F.embedding(idx, p["wte.weight"]) + F.embedding(pos, p["wpe.weight"])
    tri = torch.tril(torch.ones(cfg.n_positions, cfg.n_positions, dtype=torch.bool))
    for i in range(cfg.n_layer):
        pre = f"h.{i}."
        lw = lambda n: p[pre + n]  # noqa: E731
        h = F.layer_norm(x, (C,), lw("ln_1.weight"), lw("ln_1.bias"), cfg.layer_norm_epsilon)
        layer_past = cache.length(i) if cache is not None else 0
        qkv = F.linear(h, lw("attn.c_attn.weight"), lw("attn.c_attn.bias"))
        q, k, v = qkv.split([C, C, C], dim=2)
        q = q.view(B, T, H, hd).transpose(1, 2)
        k = k.view(B, T, H, hd).transpose(1, 2)
        v = v.view(B, T, H, hd).transpose(1, 2)
        if cache is not None:
            if cache.k[i] is not None:
                k = torch.cat([cache.k[i], k], dim=-2)
                v = torch.cat([cache.v[i], v], dim=-2)
            cache.k[i], cache.v[i] = k, v
        Tt = k.shape[-2]
        mask = tri[layer_past : layer_past + T, :Tt]
        att = (q @ k.transpose(-2, -1)) / math.sqrt(hd)
        att = att.masked_fill(~mask.view(1, 1, T, Tt), float("-inf"))
        att = F.softmax(att, dim=-1)
        y = (att @ v).transpose(1, 2).contiguous().view(B, T, C)
        x = x + F.linear(y, lw("attn.c_proj.weight"), lw("attn.c_proj.bias"))
        h2 = F.layer_norm(x, (C,), lw("ln_2.weight"), lw("ln_2.bias"), cfg.layer_norm_epsilon)
        m = F.linear(gelu_tanh(F.linear(h2, lw("mlp.c_fc.weight"), lw("mlp.c_fc.bias"))),
                     lw("mlp.c_proj.weight"), lw("mlp.c_proj.bias"))
        x = x + m
    if last_only:
        x = x[:, -1:]
    x = F.layer_norm(x, (C,), p["ln_f.weight"], p["ln_f.bias"], cfg.layer_norm_epsilon)
    return F.linear(x, p["wte.weight"])


@torch.no_grad()
def generate_greedy(p, cfg: Shape, idx: torch.Tensor, max_new_tokens: int, detail: bool = False):
    """Greedy cached decode. Returns ``(ids (B, T+n), margins (n,))`` where a
    margin is the smallest top-1 minus top-2 logit gap over the batch; with
    ``detail`` also the per-sequence gaps ``(n, B)`` and the last step's
    logits ``(B, V)``."""
    cache = Cache(cfg.n_layer)
    margins, gaps, logits = [], [], None
    for step in range(max_new_tokens):
        if idx.size(1) >= cfg.n_positions:
            break
        step_input = idx if step == 0 else idx[:, -1:]
        logits = forward(p, cfg, step_input, cache, last_only=True)[:, -1, :]
        top2 = logits.topk(2, dim=-1).values
        gap = top2[:, 0] - top2[:, 1]
        margins.append(float(gap.min()))
        gaps.append(gap)
        nxt = logits.argmax(dim=-1, keepdim=True)
        idx = torch.cat([idx, nxt], dim=1)
    if detail:
        return idx, margins, torch.stack(gaps) if gaps else torch.empty(0, idx.size(0)), logits
    return idx, margins


def benchmark_prompt(vocab_size: int, batch: int, length: int) -> torch.Tensor:
    """The prompt of ``benchmark_generation`` (``benchmark.py:167-170``)."""
    torch.manual_seed(0)
    return torch.randint(0, vocab_size, (batch, length))
