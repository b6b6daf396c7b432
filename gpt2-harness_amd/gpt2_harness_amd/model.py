"""GPT-2 host model whose four Linear slots take :class:`QuantLinear` modules.

The module tree, parameter names and initialisation order are those of the
reference's ``GPT`` (``src/transformer_internals/model.py:445-518``) because
three things depend on them: the ``TARGET_SUFFIXES`` lookup of
``quantize_model`` (``attn.c_attn``, ``attn.c_proj``, ``mlp.c_fc``,
``mlp.c_proj``), state-dict compatibility with reference checkpoints, and the
seed-0 random weights the benchmarks are quoted on (module construction draws,
then ``_init_weights`` in module order -- the tied ``lm_head`` redraws ``wte``
-- then residual scaling of both ``c_proj`` weights).

The forward pass is the reference's arithmetic (``model.py:528-599``):
pre-LN blocks, fused ``c_attn`` split into q/k/v, explicit softmax attention
with the causal mask taken at absolute positions, ``gelu_tanh`` MLP, tied fp32
``lm_head``. Attention, LayerNorm and the head run as torch ops on the GPU;
the four projections per block are the HIP kernels once quantized.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn as nn
import torch.nn.functional as F

from .config import GPTConfig

__all__ = ["GPT", "MLP", "Block", "CausalSelfAttention", "KVCache", "gelu_tanh"]


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """``0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))`` (``model.py:57-75``).

    fp32 tensors on the GPU go through one HIP pass (``tiq_gelu_tanh``; the
    op chain below reads and writes the tensor eight times); other tensors
    (CPU, other dtypes) are computed with the torch ops of the reference.
    """
    if x.is_cuda and x.dtype == torch.float32:
        from . import _lib

        xc = x.contiguous()
        if xc.data_ptr() % 16:
            xc = xc.clone()  # a fresh allocation is 16-byte aligned
        y = torch.empty_like(xc)
        _lib.check(_lib.lib().tiq_gelu_tanh(xc.data_ptr(), y.data_ptr(), xc.numel(), _lib.stream_of(xc)),
                   "gelu_tanh")
        return y
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x.pow(3))))


def _sinusoid(n_positions: int, n_embd: int) -> torch.Tensor:
    pos = torch.arange(n_positions, dtype=torch.float32)[:, None]
    inv = torch.exp(torch.arange(0, n_embd, 2, dtype=torch.float32) * (-math.log(10000.0) / n_embd))
    pe = torch.zeros(n_positions, n_embd)
    pe[:, 0::2] = torch.sin(pos * inv)
    pe[:, 1::2] = torch.cos(pos * inv)[:, : n_embd // 2]
    return pe


@dataclass
class KVCache:
    """Per-layer key/value history, appended by concatenation (``model.py:106-172``).

    ``length(layer)`` -- not the model-level ``seq_len`` -- gives the causal
    offset inside a layer, since earlier layers already hold the current step.
    """

    keys: list[torch.Tensor | None]
    values: list[torch.Tensor | None]

    @classmethod
    def empty(cls, n_layer: int) -> KVCache:
        return cls(keys=[None] * n_layer, values=[None] * n_layer)

    @property
    def seq_len(self) -> int:
        return self.length(0)

    def length(self, layer: int) -> int:
        k = self.keys[layer]
        return 0 if k is None else int(k.shape[-2])

    def update(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        pk, pv = self.keys[layer], self.values[layer]
        if pk is not None and pv is not None:
            k = torch.cat([pk, k], dim=-2)
            v = torch.cat([pv, v], dim=-2)
        self.keys[layer], self.values[layer] = k, v
        return k, v


class CausalSelfAttention(nn.Module):
    def __init__(self, config: GPTConfig, layer_idx: int = 0) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.n_head, self.n_kv_head = config.n_head, config.kv_heads
        self.n_embd, self.head_dim = config.n_embd, config.head_dim
        self.kv_dim = self.n_kv_head * self.head_dim
        self.c_attn = nn.Linear(config.n_embd, config.n_embd + 2 * self.kv_dim, bias=config.attn_bias)
        self.c_proj = nn.Linear(config.n_embd, config.n_embd, bias=config.attn_bias)
        self.attn_dropout = nn.Dropout(config.dropout)
        self.resid_dropout = nn.Dropout(config.dropout)
        self.head_mask: torch.Tensor | None = None

    def forward(self, x: torch.Tensor, cache: KVCache | None = None, need_weights: bool = False):
        B, T, C = x.shape
        past = cache.length(self.layer_idx) if cache is not None else 0
        q, k, v = self.c_attn(x).split([self.n_embd, self.kv_dim, self.kv_dim], dim=2)
        q = q.view(B, T, self.n_head, self.head_dim).transpose(1, 2)
        k = k.view(B, T, self.n_kv_head, self.head_dim).transpose(1, 2)
        v = v.view(B, T, self.n_kv_head, self.head_dim).transpose(1, 2)
        if cache is not None:
            k, v = cache.update(self.layer_idx, k, v)
        total = k.shape[-2]
        if self.n_kv_head != self.n_head:
            g = self.n_head // self.n_kv_head
            k = k.repeat_interleave(g, dim=1)
            v = v.repeat_interleave(g, dim=1)
        # key j is visible to query i (absolute position past + i) iff j <= past + i
        qpos = torch.arange(past, past + T, device=x.device)[:, None]
        kpos = torch.arange(total, device=x.device)[None, :]
        allowed = kpos <= qpos
        probs = None
        if self.config.use_sdpa and not need_weights:
            y = F.scaled_dot_product_attention(q, k, v, attn_mask=allowed.view(1, 1, T, total),
                                               dropout_p=self.config.dropout if self.training else 0.0)
        else:
            kt = k.transpose(-2, -1)
            if kt.dtype == torch.bfloat16:
                kt = kt.contiguous()
            att = (q @ kt) / math.sqrt(self.head_dim)
            att = att.masked_fill(~allowed.view(1, 1, T, total), float("-inf"))
            att = F.softmax(att, dim=-1)
            probs = att if need_weights else None
            y = self.attn_dropout(att) @ v
        if self.head_mask is not None:
            y = y * self.head_mask.to(y.device, y.dtype).view(1, -1, 1, 1)
        y = y.transpose(1, 2).contiguous().view(B, T, C)
        return self.resid_dropout(self.c_proj(y)), probs


class MLP(nn.Module):
    def __init__(self, config: GPTConfig) -> None:
        super().__init__()
        self.config = config
        self.c_fc = nn.Linear(config.n_embd, 4 * config.n_embd, bias=config.mlp_bias)
        self.c_proj = nn.Linear(4 * config.n_embd, config.n_embd, bias=config.mlp_bias)
        self.dropout = nn.Dropout(config.dropout)
        self.neuron_mask: torch.Tensor | None = None

    def act(self, x: torch.Tensor) -> torch.Tensor:
        if self.config.activation == "gelu_tanh":
            return gelu_tanh(x)
        if self.config.activation == "gelu_exact":
            return F.gelu(x)
        return F.relu(x)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = self.act(self.c_fc(x))
        if self.neuron_mask is not None:
            h = h * self.neuron_mask.to(h.device, h.dtype)
        return self.dropout(self.c_proj(h))


class Block(nn.Module):
    def __init__(self, config: GPTConfig, layer_idx: int = 0) -> None:
        super().__init__()
        self.config = config
        self.ln_1 = nn.LayerNorm(config.n_embd, eps=config.layer_norm_epsilon)
        self.attn = CausalSelfAttention(config, layer_idx=layer_idx)
        self.ln_2 = nn.LayerNorm(config.n_embd, eps=config.layer_norm_epsilon)
        self.mlp = MLP(config)

    def forward(self, x: torch.Tensor, cache: KVCache | None = None, need_weights: bool = False):
        if self.config.norm_position == "pre":
            a, probs = self.attn(self.ln_1(x), cache=cache, need_weights=need_weights)
            x = x + a
            x = x + self.mlp(self.ln_2(x))
        else:
            a, probs = self.attn(x, cache=cache, need_weights=need_weights)
            x = self.ln_1(x + a)
            x = self.ln_2(x + self.mlp(x))
        return x, probs


class GPT(nn.Module):
    def __init__(self, config: GPTConfig) -> None:
        super().__init__()
        self.config = config
        self.wte = nn.Embedding(config.vocab_size, config.n_embd)
        if config.pos_embedding == "learned":
            self.wpe: nn.Embedding | None = nn.Embedding(config.n_positions, config.n_embd)
        else:
            self.wpe = None
            self.register_buffer("sinusoidal_pe", _sinusoid(config.n_positions, config.n_embd), persistent=False)
        self.drop = nn.Dropout(config.dropout)
        self.h = nn.ModuleList([Block(config, layer_idx=i) for i in range(config.n_layer)])
        self.ln_f = nn.LayerNorm(config.n_embd, eps=config.layer_norm_epsilon)
        self.lm_head = nn.Linear(config.n_embd, config.vocab_size, bias=False)
        if config.tie_weights:
            self.lm_head.weight = self.wte.weight
        self.apply(self._init_weights)
        if config.residual_scaled_init:
            std = 0.02 / math.sqrt(2 * config.n_layer)
            for block in self.h:
                nn.init.normal_(block.attn.c_proj.weight, mean=0.0, std=std)
                nn.init.normal_(block.mlp.c_proj.weight, mean=0.0, std=std)

    @staticmethod
    def _init_weights(module: nn.Module) -> None:
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
        elif isinstance(module, nn.LayerNorm):
            nn.init.ones_(module.weight)
            nn.init.zeros_(module.bias)

    def position_embeddings(self, pos: torch.Tensor) -> torch.Tensor:
        return self.wpe(pos) if self.wpe is not None else self.sinusoidal_pe[pos]

    def forward(
        self,
        idx: torch.Tensor,
        targets: torch.Tensor | None = None,
        cache: KVCache | None = None,
        need_weights: bool = False,
        collect_taps: bool = False,
        last_only: bool = False,
    ) -> dict[str, Any]:
        """``model.py:528-599``. ``last_only`` (an extension; the reference
        always computes every position) returns logits ``(B, 1, V)`` of the
        last position only, for a prefill that needs nothing else: the head
        is the largest product of a long prompt."""
        if collect_taps:
            raise NotImplementedError("activation taps belong to the verification tooling, not this library")
        _, T = idx.shape
        past = cache.seq_len if cache is not None else 0
        if past + T > self.config.n_positions:
            raise ValueError(
                f"sequence of length {past + T} exceeds n_positions={self.config.n_positions}; "
                f"learned position embeddings cannot extrapolate"
            )
        pos = torch.arange(past, past + T, dtype=torch.long, device=idx.device)
        x = self.drop(self.wte(idx) + self.position_embeddings(pos))
        attentions = []
        for block in self.h:
            x, probs = block(x, cache=cache, need_weights=need_weights)
            if probs is not None:
                attentions.append(probs)
        if last_only:
            if targets is not None:
                raise ValueError("last_only computes no loss: the loss needs every position's logits")
            x = x[:, -1:, :]
        logits = self.lm_head(self.ln_f(x))
        out: dict[str, Any] = {"logits": logits}
        if need_weights:
            out["attentions"] = attentions
        if targets is not None:
            out["loss"] = F.cross_entropy(logits.view(-1, logits.size(-1)), targets.reshape(-1), ignore_index=-100)
        return out

    def num_parameters(self, non_embedding: bool = False) -> int:
        n = sum(p.numel() for p in self.parameters())
        if non_embedding and self.wpe is not None:
            n -= self.wpe.weight.numel()
        return n
