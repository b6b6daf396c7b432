"""Graph-captured greedy decode on the GPU.

The reference's ``generate`` (``sampling.py:100-181``) runs one Python-level
forward pass per token over a ``torch.cat``-grown cache (``model.py:153-172``):
every op is a separate launch issued from the host. Here the prompt is
processed by the model's ordinary forward (prefill), and every later token by
one replay of a captured HIP graph that holds the whole decode step:

* the KV cache is preallocated, ``(B, kv_heads, T_max, head_dim)`` per layer,
  and the new key / value are written at the current position (a device
  tensor, so the graph does not change from step to step);
* attention runs over all ``T_max`` cache slots with the slots after the
  current position masked to ``-inf`` before the softmax, which gives them
  probability exactly 0 -- the reference's attention over the ``T_total``
  filled slots (``model.py:286-309``);
* the quantized Linears are the HIP kernels (launched on the capture stream);
* greedy ``argmax`` picks the next token, which is written to the output ids
  and fed to the next replay; the position advances inside the graph.

Token ids are the reference's; the logits agree with an eager forward to fp32
rounding (the matmuls see padded shapes).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = ["GraphDecoder", "generate_graph"]


class GraphDecoder:
    """Captures one decode step of ``model`` for ``batch`` sequences of up to
    ``max_len`` positions. ``model`` is a GPT with the reference's module
    layout (pre-LN or post-LN, learned or sinusoidal positions) on a GPU."""

    def __init__(self, model, batch: int, max_len: int) -> None:
        cfg = model.config
        if max_len > cfg.n_positions:
            raise ValueError(f"max_len={max_len} exceeds n_positions={cfg.n_positions}")
        self.model = model.eval()
        self.cfg = cfg
        self.B, self.T = batch, max_len
        dev = next(model.parameters()).device
        self.dev = dev
        H, Hkv, hd = cfg.n_head, cfg.kv_heads, cfg.head_dim
        self.H, self.Hkv, self.hd = H, Hkv, hd
        self.k = [torch.zeros(batch, Hkv, max_len, hd, device=dev) for _ in range(cfg.n_layer)]
        self.v = [torch.zeros(batch, Hkv, max_len, hd, device=dev) for _ in range(cfg.n_layer)]
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)        # position of the token being fed
        self.tok = torch.zeros(batch, 1, dtype=torch.long, device=dev)  # token being fed
        self.out = torch.zeros(batch, max_len, dtype=torch.long, device=dev)
        self.slots = torch.arange(max_len, device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None

    # ------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, idx: torch.Tensor) -> torch.Tensor:
        """Run the prompt through the model's own forward, filling the cache.
        Returns the last position's logits ``(B, V)``."""
        B, T0 = idx.shape
        if B != self.B or T0 > self.T:
            raise ValueError(f"prompt {tuple(idx.shape)} does not fit batch={self.B}, max_len={self.T}")
        from .model import KVCache

        cache = KVCache.empty(self.cfg.n_layer)
        logits = self.model(idx, cache=cache)["logits"][:, -1, :]
        for i in range(self.cfg.n_layer):
            self.k[i][:, :, :T0].copy_(cache.keys[i])
            self.v[i][:, :, :T0].copy_(cache.values[i])
        self.out[:, :T0].copy_(idx)
        return logits

    # ------------------------------------------------------------ one step
    def _step(self) -> None:
        m, cfg = self.model, self.cfg
        B, H, Hkv, hd, C = self.B, self.H, self.Hkv, self.hd, cfg.n_embd
        pos = self.pos
        x = m.wte(self.tok) + m.position_embeddings(pos.view(1, 1).expand(B, 1))
        visible = (self.slots <= pos).view(1, 1, 1, self.T)
        pre = cfg.norm_position == "pre"
        for i, block in enumerate(m.h):
            attn = block.attn
            h = block.ln_1(x) if pre else x
            q, k, v = attn.c_attn(h).split([C, Hkv * hd, Hkv * hd], dim=2)
            q = q.view(B, 1, H, hd).transpose(1, 2)
            k = k.view(B, 1, Hkv, hd).transpose(1, 2)
            v = v.view(B, 1, Hkv, hd).transpose(1, 2)
            self.k[i].index_copy_(2, pos, k)
            self.v[i].index_copy_(2, pos, v)
            K, V = self.k[i], self.v[i]
            if Hkv != H:
                K = K.repeat_interleave(H // Hkv, dim=1)
                V = V.repeat_interleave(H // Hkv, dim=1)
            att = (q @ K.transpose(-2, -1)) / math.sqrt(hd)
            att = att.masked_fill(~visible, float("-inf"))
            att = F.softmax(att, dim=-1)
            if attn.head_mask is not None:
                y = (att @ V) * attn.head_mask.to(att.device, att.dtype).view(1, -1, 1, 1)
            else:
                y = att @ V
            a = attn.c_proj(y.transpose(1, 2).contiguous().view(B, 1, C))
            if pre:
                x = x + a
                x = x + block.mlp(block.ln_2(x))
            else:
                x = block.ln_1(x + a)
                x = block.ln_2(x + block.mlp(x))
        logits = m.lm_head(m.ln_f(x))[:, -1, :]
        nxt = logits.argmax(dim=-1, keepdim=True)
        self.tok.copy_(nxt)
        self.pos.add_(1)
        self.out.index_copy_(1, pos, nxt)  # pos was advanced: writes slot of the new token

    @torch.no_grad()
    def capture(self) -> None:
        """Capture the decode step (after a warm-up run on a side stream)."""
        saved = (self.pos.clone(), self.tok.clone(), self.out.clone())
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            self._step()
        torch.cuda.current_stream(self.dev).wait_stream(s)
        self.pos.copy_(saved[0])
        self.tok.copy_(saved[1])
        self.out.copy_(saved[2])
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._step()
        self.graph = g

    @torch.no_grad()
    def run(self, idx: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        """Greedy decode: prefill, then ``max_new_tokens - 1`` graph replays."""
        B, T0 = idx.shape
        n = min(max_new_tokens, self.cfg.n_positions - T0, self.T - T0)
        if n <= 0:
            return idx
        logits = self.prefill(idx)
        first = logits.argmax(dim=-1, keepdim=True)
        self.out[:, T0 : T0 + 1].copy_(first)
        self.tok.copy_(first)
        self.pos.fill_(T0)
        if n > 1 and self.graph is None:
            self.capture()
        for _ in range(n - 1):
            self.graph.replay()
        return self.out[:, : T0 + n].clone()


@torch.no_grad()
def generate_graph(model, idx: torch.Tensor, max_new_tokens: int, decoder: GraphDecoder | None = None):
    """Greedy generation with a captured decode step; the same token ids as
    ``generate(model, idx, max_new_tokens)``. Pass a ``decoder`` built for
    this batch / length to reuse its captured graph across calls."""
    if decoder is None:
        decoder = GraphDecoder(model, idx.size(0), min(model.config.n_positions, idx.size(1) + max_new_tokens))
    return decoder.run(idx, max_new_tokens)
