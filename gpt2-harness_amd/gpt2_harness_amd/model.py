"""GPT-2 decoder whose four Linear slots take :class:`QuantLinear` modules.

This is the inference model of the quantized path: pre-LN GPT-2 blocks with
learned positions, the tanh GELU and a tied head. The reference's ablation
switches (post-LN, sinusoidal positions, other activations, grouped-query
heads, attention / neuron masks, activation taps) are not part of that path
and are refused at construction.

Three things are interface and therefore fixed:

* the module names (``wte``, ``wpe``, ``h.<i>.ln_1``, ``h.<i>.attn.c_attn``,
  ``h.<i>.attn.c_proj``, ``h.<i>.ln_2``, ``h.<i>.mlp.c_fc``,
  ``h.<i>.mlp.c_proj``, ``ln_f``, ``lm_head``): ``quantize_model`` finds its
  targets by these suffixes and checkpoints are keyed by them;
* the order of the random draws at construction and initialisation, which
  fixes the seed-0 weights every benchmark is quoted on
  (``src/transformer_internals/model.py:457-518``; see :meth:`GPT._seeded_init`);
* ``forward(idx, targets=None, cache=None)`` returning ``{"logits", "loss"}``
  and the ``KVCache`` calls made by the greedy loop
  (``sampling.py:100-181``, ``model.py:106-172``).

The arithmetic is GPT-2's (``model.py:57-75,227-320,351-355,528-599``); on the
GPU the quantized projections are the library's HIP kernels and the prefill's
GELU is one HIP pass.
"""

from __future__ import annotations

import math
from typing import Any

import torch
import torch.nn as nn
import torch.nn.functional as F

from .config import GPTConfig

__all__ = ["GPT", "MLP", "Block", "CausalSelfAttention", "KVCache", "gelu_tanh"]

_SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """GELU in GPT-2's tanh form, ``0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))``.

    An fp32 GPU tensor that needs no gradient goes through one HIP pass
    (``tiq_gelu_tanh``: one read and one write instead of the eight passes
    of the op chain). Anything else -- CPU tensors, other dtypes, or a tensor
    autograd must differentiate -- is computed with torch ops, which carry the
    gradient.
    """
    if x.is_cuda and x.dtype == torch.float32 and not (torch.is_grad_enabled() and x.requires_grad):
        from . import _lib

        src = x.contiguous()
        if src.data_ptr() % 16:
            src = src.clone()  # fresh allocations are 16-byte aligned
        out = torch.empty_like(src)
        _lib.check(_lib.lib().tiq_gelu_tanh(src.data_ptr(), out.data_ptr(), src.numel(), _lib.stream_of(src)),
                   "gelu_tanh")
        return out
    inner = _SQRT_2_OVER_PI * (x + 0.044715 * x.pow(3))
    return 0.5 * x * (1.0 + torch.tanh(inner))


class KVCache:
    """Per-layer key / value history for cached decoding.

    Each layer owns a buffer ``(B, heads, capacity, head_dim)`` that grows by
    doubling, so appending a step writes only the new rows (the reference's
    ``torch.cat`` copies the whole history every step, ``model.py:153-172``).
    ``length(layer)`` is that layer's own fill level -- inside one forward
    pass the earlier layers already hold the current step, so the causal
    offset of a layer must come from it, not from :attr:`seq_len`
    (``model.py:139-151``).
    """

    def __init__(self, keys: int | list[torch.Tensor | None], values: list[torch.Tensor | None] | None = None) -> None:
        """``KVCache(n_layer)``: an empty cache. ``KVCache(keys=[...],
        values=[...])`` (the reference's dataclass fields, ``model.py:106-126``):
        per layer a filled ``(B, heads, T, head_dim)`` history or ``None``;
        those tensors become the layers' buffers (full: the next append grows
        them by a copy)."""
        if isinstance(keys, int):
            if values is not None:
                raise ValueError("KVCache(n_layer) takes no values")
            self._k: list[torch.Tensor | None] = [None] * keys
            self._v: list[torch.Tensor | None] = [None] * keys
            self._len = [0] * keys
            return
        if values is None or len(keys) != len(values):
            raise ValueError("KVCache needs keys and values lists of the same length")
        for k, v in zip(keys, values):
            if (k is None) != (v is None) or (k is not None and k.shape != v.shape):
                raise ValueError("each layer's keys and values must both be None or tensors of one shape")
        self._k, self._v = list(keys), list(values)
        self._len = [0 if k is None else int(k.shape[-2]) for k in keys]

    @classmethod
    def empty(cls, n_layer: int) -> KVCache:
        return cls(n_layer)

    @classmethod
    def over(cls, keys: list[torch.Tensor], values: list[torch.Tensor]) -> KVCache:
        """An empty cache whose layer buffers are the given ``(B, heads,
        capacity, head_dim)`` tensors (a decoder's preallocated cache): a
        prefill appends into them in place (past ``capacity`` they grow by a
        copy, as an empty cache's do)."""
        cache = cls(len(keys))
        cache._k, cache._v = list(keys), list(values)  # buffers, 0 positions filled
        return cache

    @property
    def seq_len(self) -> int:
        """Positions already processed (layer 0's fill level): the absolute
        position of the tokens a forward pass is about to add."""
        return self._len[0]

    def length(self, layer: int) -> int:
        return self._len[layer]

    @property
    def keys(self) -> list[torch.Tensor | None]:
        """Each layer's filled history (views; append with :meth:`update`)."""
        return [None if b is None else b[:, :, :n] for b, n in zip(self._k, self._len)]

    @property
    def values(self) -> list[torch.Tensor | None]:
        return [None if b is None else b[:, :, :n] for b, n in zip(self._v, self._len)]

    def update(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Append ``k, v`` ``(B, heads, T_new, head_dim)`` to ``layer``; return
        views of the whole history ``(B, heads, length, head_dim)``."""
        n, t = self._len[layer], k.shape[-2]
        buf_k, buf_v = self._k[layer], self._v[layer]
        if buf_k is None or n + t > buf_k.shape[-2]:
            cap = max(16, 2 * (n + t))
            grown_k = k.new_empty(*k.shape[:-2], cap, k.shape[-1])
            grown_v = v.new_empty(*v.shape[:-2], cap, v.shape[-1])
            if buf_k is not None:
                grown_k[:, :, :n] = buf_k[:, :, :n]
                grown_v[:, :, :n] = buf_v[:, :, :n]
            self._k[layer], self._v[layer] = buf_k, buf_v = grown_k, grown_v
        buf_k[:, :, n : n + t] = k
        buf_v[:, :, n : n + t] = v
        self._len[layer] = n + t
        return buf_k[:, :, : n + t], buf_v[:, :, : n + t]


def _causal_softmax_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, first: int,
                              p_drop: float) -> torch.Tensor:
    """``softmax(q k^T / sqrt(hd) + mask) v`` for queries at absolute positions
    ``first .. first + T - 1`` over keys ``0 .. S - 1`` (``model.py:284-309``).

    Key ``j`` is visible to query ``i`` iff ``j <= first + i``; hidden scores
    are ``-inf``, so they get probability exactly 0. A query block that sees
    every key (one new token over the cache) needs no mask at all.
    """
    T, S = q.shape[-2], k.shape[-2]
    scores = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(q.shape[-1])
    if not (T == 1 and first + 1 == S):
        qpos = torch.arange(first, first + T, device=q.device).unsqueeze(1)
        kpos = torch.arange(S, device=q.device).unsqueeze(0)
        scores = scores.masked_fill(kpos > qpos, float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    if p_drop:
        probs = F.dropout(probs, p_drop, training=True)
    return torch.matmul(probs, v)


def _fused_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, first: int,
                     p_drop: float) -> torch.Tensor | None:
    """``_causal_softmax_attention`` as one HIP kernel (``tiq_prefill_attention``),
    its output as ``(B, T, heads * head_dim)`` rows, for fp32 GPU tensors with
    64-dim heads that need no gradient and no dropout; ``None`` otherwise. q, k
    and v are read in place through their strides (the projection's rows, a
    cache's buffers): no copies."""
    B, H, T, hd = q.shape
    ok = (q.is_cuda and hd == 64 and p_drop == 0.0 and k.shape[-2] == first + T
          and all(t.dtype == torch.float32 and t.stride(-1) == 1 for t in (q, k, v))
          and not (torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)))
    if not ok:
        return None
    from . import _lib

    y = torch.empty(B, T, H * hd, device=q.device, dtype=torch.float32)
    rc = _lib.lib().tiq_prefill_attention(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), B, H, T, first, hd, y.data_ptr(), y.stride(0), hd,
        y.stride(1), _lib.stream_of(q))
    if rc in (_lib.EALIGN, _lib.EUNSUPPORTED):
        return None  # strides or sizes the kernel does not take: the torch ops below
    _lib.check(rc, "prefill attention")
    return y


class CausalSelfAttention(nn.Module):
    """Fused ``c_attn`` (q, k, v side by side), heads of 64 columns, causal
    attention over the cache, ``c_proj``."""

    def __init__(self, config: GPTConfig, layer_idx: int = 0) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.n_head, self.head_dim, self.n_embd = config.n_head, config.head_dim, config.n_embd
        self.c_attn = nn.Linear(config.n_embd, 3 * config.n_embd, bias=config.attn_bias)
        self.c_proj = nn.Linear(config.n_embd, config.n_embd, bias=config.attn_bias)

    def forward(self, x: torch.Tensor, cache: KVCache | None = None) -> torch.Tensor:
        B, T, C = x.shape
        first = 0 if cache is None else cache.length(self.layer_idx)
        # (B, T, 3C) -> (3, B, heads, T, hd): q, k, v heads in one permute
        q, k, v = self.c_attn(x).view(B, T, 3, self.n_head, self.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
        if cache is not None:
            k, v = cache.update(self.layer_idx, k, v)
        p = self.config.dropout if self.training else 0.0
        y = _fused_attention(q, k, v, first, p)
        if y is not None:
            return self.c_proj(y)
        y = _causal_softmax_attention(q, k, v, first, p)
        return self.c_proj(y.transpose(1, 2).reshape(B, T, C))


class MLP(nn.Module):
    """``c_proj(gelu_tanh(c_fc(x)))``, 4x expansion."""

    def __init__(self, config: GPTConfig) -> None:
        super().__init__()
        self.c_fc = nn.Linear(config.n_embd, 4 * config.n_embd, bias=config.mlp_bias)
        self.c_proj = nn.Linear(4 * config.n_embd, config.n_embd, bias=config.mlp_bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = self.c_fc(x)
        fused = getattr(self.c_proj, "forward_gelu_in", None)  # a quantized c_proj over a prefill's rows
        y = fused(h) if fused is not None else None
        return y if y is not None else self.c_proj(gelu_tanh(h))


class Block(nn.Module):
    """Pre-LN block: ``x + attn(ln_1(x))``, then ``x + mlp(ln_2(x))``."""

    def __init__(self, config: GPTConfig, layer_idx: int = 0) -> None:
        super().__init__()
        self.p_drop = config.dropout
        # construction order = registration order = the order of the RNG draws
        self.ln_1 = nn.LayerNorm(config.n_embd, eps=config.layer_norm_epsilon)
        self.attn = CausalSelfAttention(config, layer_idx=layer_idx)
        self.ln_2 = nn.LayerNorm(config.n_embd, eps=config.layer_norm_epsilon)
        self.mlp = MLP(config)

    def _drop(self, t: torch.Tensor) -> torch.Tensor:
        return F.dropout(t, self.p_drop, training=True) if self.training and self.p_drop else t

    def forward(self, x: torch.Tensor, cache: KVCache | None = None) -> torch.Tensor:
        x = x + self._drop(self.attn(self.ln_1(x), cache))
        return x + self._drop(self.mlp(self.ln_2(x)))


def _refuse_unsupported(config: GPTConfig) -> None:
    """The layouts of the quantized path only: GPT-2 as released."""
    unsupported = {
        "norm_position": (config.norm_position, "pre"),
        "pos_embedding": (config.pos_embedding, "learned"),
        "activation": (config.activation, "gelu_tanh"),
        "n_kv_head": (config.kv_heads, config.n_head),
        "use_sdpa": (config.use_sdpa, False),
    }
    for field, (got, want) in unsupported.items():
        if got != want:
            raise NotImplementedError(
                f"{field}={got!r}: this model implements GPT-2's inference layout only ({field}={want!r})")


class GPT(nn.Module):
    """GPT-2 with a tied head (``lm_head.weight is wte.weight``)."""

    def __init__(self, config: GPTConfig) -> None:
        super().__init__()
        _refuse_unsupported(config)
        if not config.tie_weights:
            raise NotImplementedError("tie_weights=False: GPT-2's head is the embedding matrix")
        self.config = config
        self.wte = nn.Embedding(config.vocab_size, config.n_embd)
        self.wpe = nn.Embedding(config.n_positions, config.n_embd)
        self.h = nn.ModuleList(Block(config, layer_idx=i) for i in range(config.n_layer))
        self.ln_f = nn.LayerNorm(config.n_embd, eps=config.layer_norm_epsilon)
        self.lm_head = nn.Linear(config.n_embd, config.vocab_size, bias=False)
        self.lm_head.weight = self.wte.weight
        self._seeded_init()

    @torch.no_grad()
    def _seeded_init(self) -> None:
        """GPT-2's initialisation, drawn in the reference's order.

        Every Linear and Embedding weight ~ N(0, 0.02), biases 0, LayerNorm
        scale 1 and shift 0, visiting the leaf modules in registration order
        (so the tied ``lm_head``, last, redraws the embedding); then the two
        residual-writing projections of each block are redrawn with
        ``std = 0.02 / sqrt(2 * n_layer)``, attention's before the MLP's. With
        the construction draws of the ``nn`` modules before it, this sequence
        reproduces the reference's seed-0 weights bit for bit
        (``model.py:457-518``).
        """
        for mod in self.modules():
            if isinstance(mod, (nn.Linear, nn.Embedding)):
                mod.weight.normal_(0.0, 0.02)
                if getattr(mod, "bias", None) is not None:
                    mod.bias.zero_()
            elif isinstance(mod, nn.LayerNorm):
                mod.weight.fill_(1.0)
                mod.bias.zero_()
        if self.config.residual_scaled_init:
            std = 0.02 / math.sqrt(2 * self.config.n_layer)
            for block in self.h:
                block.attn.c_proj.weight.normal_(0.0, std)
                block.mlp.c_proj.weight.normal_(0.0, std)

    def position_embeddings(self, pos: torch.Tensor) -> torch.Tensor:
        return self.wpe(pos)

    def forward(
        self,
        idx: torch.Tensor,
        targets: torch.Tensor | None = None,
        cache: KVCache | None = None,
        last_only: bool = False,
    ) -> dict[str, Any]:
        """Logits ``(B, T, vocab)`` of ``idx`` ``(B, T)`` (``model.py:528-599``).

        With a ``cache``, ``idx`` holds only the new tokens, placed after the
        cached ones. ``targets`` adds the mean cross entropy (``-100``
        ignored) as ``loss``. ``last_only`` returns the last position's logits
        ``(B, 1, vocab)`` only -- all a prefill needs, and the head is the
        largest product of a long prompt.
        """
        T = idx.shape[1]
        first = 0 if cache is None else cache.seq_len
        if first + T > self.config.n_positions:
            raise ValueError(
                f"sequence of length {first + T} exceeds n_positions={self.config.n_positions}; "
                f"learned position embeddings cannot extrapolate"
            )
        if last_only and targets is not None:
            raise ValueError("last_only computes no loss: the loss needs every position's logits")
        pos = torch.arange(first, first + T, device=idx.device)
        x = self.wte(idx) + self.wpe(pos)
        if self.training and self.config.dropout:
            x = F.dropout(x, self.config.dropout, training=True)
        for block in self.h:
            x = block(x, cache)
        if last_only:
            x = x[:, -1:]
        logits = self.lm_head(self.ln_f(x))
        out: dict[str, Any] = {"logits": logits}
        if targets is not None:
            out["loss"] = F.cross_entropy(logits.flatten(0, 1), targets.reshape(-1), ignore_index=-100)
        return out
