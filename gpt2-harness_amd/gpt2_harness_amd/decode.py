"""Graph-captured greedy decode on the GPU.

The reference's ``generate`` (``sampling.py:100-181``) runs one Python-level
forward pass per token over a ``torch.cat``-grown cache (``model.py:153-172``):
every op is a separate launch issued from the host. Here the prompt is
processed by the model's ordinary forward (prefill; short prompts in the fused
decoder by the same ops over their rows with the epilogues fused into the
Linears), and every later token by
one replay of a captured HIP graph holding the whole decode step. The KV cache
is preallocated, ``(B, kv_heads, T_max, head_dim)`` per layer, and the fill
level is a device scalar, so the captured step is the same for every token.

Two step implementations:

* :class:`FusedDecoder` (used when the model fits: four quantized Linears per
  block, head_dim 64, an fp32 or quantized tied head): the library's decode kernels only -- an embedding kernel, then per
  block LayerNorm+``c_attn``, attention over the cache, ``c_proj``+residual,
  LayerNorm+``c_fc``+GELU, ``c_proj``+residual (5 launches), then
  LayerNorm+``lm_head`` (fp32, or int8 / int4 codes when the embedding was
  quantized) and ``argmax`` -- 5 * n_layer + 4 launches per token;
* :class:`GraphDecoder`: the model's own modules as torch ops with attention
  over all ``T_max`` slots, the slots after the current position masked to
  ``-inf`` (probability exactly 0), for models the fused step does not take
  (unquantized or partly quantized blocks, other head widths).

Greedy token ids are the reference's; logits agree with an eager forward to
fp32 rounding.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .qlinear import FMT_W4, FMT_W4G, FMT_W8, QuantLinear

__all__ = ["FusedDecoder", "GraphDecoder", "generate_graph", "make_decoder"]


class _DecoderBase:
    def __init__(self, model, batch: int, max_len: int) -> None:
        cfg = model.config
        if max_len > cfg.n_positions:
            raise ValueError(f"max_len={max_len} exceeds n_positions={cfg.n_positions}")
        self.model = model.eval()
        self.cfg = cfg
        self.B, self.T = batch, max_len
        dev = next(model.parameters()).device
        _lib.require_gpu(next(model.parameters()), "model parameters")
        self.dev = dev
        self.H, self.Hkv, self.hd = cfg.n_head, cfg.kv_heads, cfg.head_dim
        self.k = [torch.zeros(batch, self.Hkv, max_len, self.hd, device=dev) for _ in range(cfg.n_layer)]
        self.v = [torch.zeros(batch, self.Hkv, max_len, self.hd, device=dev) for _ in range(cfg.n_layer)]
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)        # position of the token being fed
        self.tok = torch.zeros(batch, 1, dtype=torch.long, device=dev)  # token being fed
        self.out = torch.zeros(batch, max_len, dtype=torch.long, device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None
        # captured prefills by prompt length: (graph, static prompt)
        self.prefill_graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}

    @torch.no_grad()
    def prefill(self, idx: torch.Tensor) -> torch.Tensor:
        """Run the prompt through the model's own forward, filling the cache.
        Returns the last position's logits ``(B, V)``."""
        B, T0 = idx.shape
        if B != self.B or T0 > self.T:
            raise ValueError(f"prompt {tuple(idx.shape)} does not fit batch={self.B}, max_len={self.T}")
        from .model import KVCache

        # the prompt's keys and values go straight into slots 0..T0-1 of the
        # preallocated cache (T0 <= its capacity: no growth, no copy after)
        cache = KVCache.over(self.k, self.v)
        logits = self.model(idx, cache=cache, last_only=True)["logits"][:, -1, :]
        self.out[:, :T0].copy_(idx)
        return logits

    def _step(self) -> None:  # pragma: no cover - provided by subclasses
        raise NotImplementedError

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

    def _start(self, idx: torch.Tensor) -> None:
        """Prefill, then set up the first generated token (position T0)."""
        T0 = idx.size(1)
        logits = self.prefill(idx)
        first = logits.argmax(dim=-1, keepdim=True)
        self.out[:, T0 : T0 + 1].copy_(first)
        self.tok.copy_(first)
        self.pos.fill_(T0)

    @torch.no_grad()
    def start(self, idx: torch.Tensor) -> None:
        """:meth:`_start` from a graph captured for this prompt length (the
        prompt is copied into the graph's static input first)."""
        T0 = idx.size(1)
        if T0 not in self.prefill_graphs:
            static = idx.clone()
            s = torch.cuda.Stream(device=self.dev)
            s.wait_stream(torch.cuda.current_stream(self.dev))
            with torch.cuda.stream(s):
                self._start(static)  # warm-up (also the result of this call)
            torch.cuda.current_stream(self.dev).wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._start(static)
            self.prefill_graphs[T0] = (g, static)
        g, static = self.prefill_graphs[T0]
        static.copy_(idx)
        g.replay()

    @torch.no_grad()
    def run(self, idx: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        """Greedy decode: prefill, then ``max_new_tokens - 1`` graph replays."""
        B, T0 = idx.shape
        n = min(max_new_tokens, self.cfg.n_positions - T0, self.T - T0)
        if n <= 0:
            return idx
        if B != self.B or T0 > self.T:
            raise ValueError(f"prompt {tuple(idx.shape)} does not fit batch={self.B}, max_len={self.T}")
        self.start(idx)
        if n > 1 and self.graph is None:
            self.capture()
        for _ in range(n - 1):
            self.graph.replay()
        return self.out[:, : T0 + n].clone()


class GraphDecoder(_DecoderBase):
    """Decode step from the model's own modules as torch ops."""

    def __init__(self, model, batch: int, max_len: int) -> None:
        super().__init__(model, batch, max_len)
        self.slots = torch.arange(max_len, device=self.dev)

    def _step(self) -> None:
        m, cfg = self.model, self.cfg
        B, H, hd, C = self.B, self.H, self.hd, cfg.n_embd
        pos = self.pos
        x = m.wte(self.tok) + m.wpe(pos.view(1, 1).expand(B, 1))
        hidden = (self.slots > pos).view(1, 1, 1, self.T)  # slots after the current position
        for i, block in enumerate(m.h):
            attn = block.attn
            q, k, v = attn.c_attn(block.ln_1(x)).view(B, 3, H, hd).unbind(1)
            self.k[i].index_copy_(2, pos, k.unsqueeze(2))
            self.v[i].index_copy_(2, pos, v.unsqueeze(2))
            scores = torch.matmul(q.unsqueeze(2), self.k[i].transpose(-2, -1)) / math.sqrt(hd)
            probs = torch.softmax(scores.masked_fill(hidden, float("-inf")), dim=-1)
            y = torch.matmul(probs, self.v[i])  # (B, H, 1, hd)
            x = x + attn.c_proj(y.view(B, 1, C))
            x = x + block.mlp(block.ln_2(x))
        logits = m.lm_head(m.ln_f(x))[:, -1, :]
        nxt = logits.argmax(dim=-1, keepdim=True)
        self.tok.copy_(nxt)
        self.pos.add_(1)
        self.out.index_copy_(1, pos, nxt)  # pos was advanced: the new token's slot


_WF = {FMT_W8: _lib.WF_INT8, FMT_W4: _lib.WF_INT4, FMT_W4G: _lib.WF_INT4G}


def fused_supported(model) -> str | None:
    """``None`` when :class:`FusedDecoder` can run ``model``, else the reason."""
    cfg = model.config
    if cfg.head_dim != 64 or cfg.n_positions > 1024:
        return "needs head_dim 64 and n_positions <= 1024"
    if cfg.n_embd % 32:
        return "needs n_embd % 32 == 0"
    for block in model.h:
        for lin in (block.attn.c_attn, block.attn.c_proj, block.mlp.c_fc, block.mlp.c_proj):
            if not isinstance(lin, QuantLinear):
                return "every target Linear must be quantized"
    head = model.lm_head
    if model.wte.weight.dtype != torch.float32 or head.bias is not None:
        return "needs an fp32 embedding and a bias-free lm_head"
    if not isinstance(head, QuantLinear) and head.weight.dtype != torch.float32:
        return "needs an fp32 or quantized lm_head"
    return None


def _layer_norm(ln, x: torch.Tensor) -> torch.Tensor:
    """The model's own LayerNorm module applied to rows (torch's kernel: at
    tens of rows it costs less as a launch of its own than inside every
    workgroup of the product that follows)."""
    return ln(x)


class FusedDecoder(_DecoderBase):
    """Decode step built from the library's fused decode kernels.

    ``head_screen`` (one sequence with the tied fp32 head): the copy of the head
    its screened argmax reads, ``"int8"`` (per-row int8 codes and scales, 1 byte
    a weight) or ``"bf16"`` (2 bytes a weight); either gives the argmax of the
    fp32 logits."""

    def __init__(self, model, batch: int, max_len: int, head_screen: str = "int8") -> None:
        if head_screen not in ("int8", "bf16"):
            raise ValueError(f"head_screen must be 'int8' or 'bf16', got {head_screen!r}")
        why = fused_supported(model)
        if why is not None:
            raise ValueError(f"fused decode unavailable: {why}")
        super().__init__(model, batch, max_len)
        cfg, dev, B = self.cfg, self.dev, batch
        C = cfg.n_embd
        self.x = torch.zeros(B, C, device=dev)
        self.qkv = torch.zeros(B, C + 2 * self.Hkv * self.hd, device=dev)
        self.att = torch.zeros(B, C, device=dev)
        self.hid = torch.zeros(B, model.h[0].mlp.c_fc.out_features, device=dev)
        self.logits = torch.zeros(B, cfg.vocab_size, device=dev)
        self.tok_flat = self.tok.view(-1)
        # the head: int8 / int4 codes when the embedding was quantized
        # (include_embedding), else the tied fp32 weight
        self.head_q = model.lm_head if isinstance(model.lm_head, QuantLinear) else None
        self.head_w = None if self.head_q is not None else model.lm_head.weight.detach().contiguous()
        self.L = _lib.lib()
        self.argmax_ws = torch.empty(int(self.L.tiq_argmax_rows_workspace(B)), dtype=torch.uint8, device=dev)
        # batched steps stage LayerNorm'd, split activations here (0 bytes: the
        # single-row GEMV path, which needs none)
        hidden = model.h[0].mlp.c_fc.out_features
        qkv = C + 2 * self.Hkv * self.hd
        ws = max(int(self.L.tiq_linear_fused_workspace(_lib.F32, _lib.WF_INT8, B, k, n))
                 for k, n in ((C, qkv), (C, C), (C, hidden), (hidden, C)))
        head_fmt = _lib.WF_F32 if self.head_q is None else _WF[self.head_q.fmt]
        ws = max(ws, int(self.L.tiq_linear_fused_workspace(_lib.F32, head_fmt, B, C, cfg.vocab_size)))
        self.lin_ws = torch.empty(max(ws, 1), dtype=torch.uint8, device=dev)
        self.lin_ws_bytes = ws
        # Batched rows (5..64) with int8 block Linears: each Linear splits its K
        # range over workgroups and hands the next one its LayerNorm'd operand
        # planes (tiq_decode_linear), so no separate LayerNorm / split launches
        lins = [l for b in model.h for l in (b.attn.c_attn, b.attn.c_proj, b.mlp.c_fc, b.mlp.c_proj)]
        head_ok = self.head_q is None or self.head_q.fmt == FMT_W8
        self.chain = 5 <= B <= 64 and head_ok and all(l.fmt == FMT_W8 for l in lins)
        self.rows_prefill = all(l.fmt == FMT_W8 for l in lins)
        # One sequence with the tied fp32 head: the decode step's head and
        # argmax read an int8 (or bf16) copy of the head and recompute from
        # the fp32 rows only those whose certified bound reaches the best of
        # their group (tiq_head_argmax_screened_i8 / tiq_head_argmax_screened):
        # the argmax of the fp32 logits
        self.screen = (B == 1 and self.head_q is None and C % 16 == 0 and C <= 1024)
        self.screen_i8 = head_screen == "int8"
        if self.screen:
            V, L = cfg.vocab_size, self.L
            st = torch.cuda.current_stream(dev).cuda_stream
            self.head_coef = torch.empty(V, device=dev)  # bound coefficient a row
            n = int(L.tiq_head_screen_workspace(V))
            self.screen_ws = torch.empty(n, dtype=torch.uint8, device=dev)
            if self.screen_i8:
                self.head_copy = torch.empty(V, C, dtype=torch.int8, device=dev)
                self.head_scale = torch.empty(V, device=dev)
                _lib.check(L.tiq_head_screen_prepare_i8(self.head_w.data_ptr(), V, C, self.head_w.stride(0),
                                                        self.head_copy.data_ptr(), self.head_scale.data_ptr(),
                                                        self.head_coef.data_ptr(), st), "head screen prepare")
            else:
                self.head_copy = torch.empty(V, C, dtype=torch.int16, device=dev)  # bf16 bits
                self.head_scale = None
                _lib.check(L.tiq_head_screen_prepare(self.head_w.data_ptr(), V, C, self.head_w.stride(0),
                                                     self.head_copy.data_ptr(), self.head_coef.data_ptr(), st),
                           "head screen prepare")
        if self.chain:
            L = self.L
            head_wf = _lib.WF_F32 if self.head_q is None else _lib.WF_INT8
            cws = max(int(L.tiq_decode_linear_workspace(_lib.WF_INT8, B, k, n))
                      for k, n in ((C, qkv), (C, C), (C, hidden), (hidden, C)))
            cws = max(cws, int(L.tiq_decode_linear_workspace(head_wf, B, C, cfg.vocab_size)))
            # c_attn's split-K slices summed by the attention kernel itself
            # (tiq_decode_qkv_attention; 0 bytes: this shape keeps the
            # separate product)
            self.qkv_slices = int(L.tiq_decode_qkv_attention_workspace(B, C, qkv)) > 0
            if self.qkv_slices:
                cws = max(cws, int(L.tiq_decode_qkv_attention_workspace(B, C, qkv)))
            self.chain_ws = torch.empty(max(cws, 1), dtype=torch.uint8, device=dev)
            self.chain_ws_bytes = cws
            pc, ph = int(L.tiq_decode_planes_bytes(B, C)), int(L.tiq_decode_planes_bytes(B, hidden))
            self.p_ln1 = torch.empty(pc, dtype=torch.uint8, device=dev)   # LayerNorm 1 (or ln_f) planes
            self.p_ln2 = torch.empty(pc, dtype=torch.uint8, device=dev)   # LayerNorm 2 planes
            self.p_hid = torch.empty(ph, dtype=torch.uint8, device=dev)   # GELU(c_fc) planes
            self.p_att = torch.empty(pc, dtype=torch.uint8, device=dev)   # attention output planes
            # the block Linears' codes once more, in the operand tiles the
            # batched products read as 1 KB consecutive loads (the row-major
            # codes stay for prefill): 1x the int8 weight bytes again
            self.tiles = {}
            for lin in lins:
                if lin.out_features % 32 or lin.in_features % 32:
                    continue  # whole 32 x 32 tiles only; these keep the row-major codes
                t = torch.empty_like(lin.codes)
                _lib.check(L.tiq_tile_int8(lin.codes.data_ptr(), lin.out_features, lin.in_features,
                                           lin.codes.stride(0), t.data_ptr(),
                                           torch.cuda.current_stream(dev).cuda_stream), "tile int8 codes")
                self.tiles[id(lin)] = t
            # the fp32 head (the tied embedding) in 4 KB operand tiles, which
            # the decode linear streams with one workgroup per CU (the
            # row-major weights stay for the embedding and the prefill)
            V = cfg.vocab_size
            if self.head_q is None and C % 32 == 0 and C >= 256:
                t = torch.empty(int(L.tiq_tile_f32_bytes(V, C)) // 4, dtype=torch.float32, device=dev)
                _lib.check(L.tiq_tile_f32(self.head_w.data_ptr(), V, C, self.head_w.stride(0), t.data_ptr(),
                                          torch.cuda.current_stream(dev).cuda_stream), "tile fp32 head")
                self.tiles[id(model.lm_head)] = t

    @property
    def extra_weight_bytes(self) -> int:
        """Device bytes of the weight copies this decoder holds beyond the
        model's own (the batched step's operand tiles of the int8 block codes
        and of the fp32 tied head; for one sequence with the fp32 tied head
        its int8 copy and two floats a row, or its bf16 copy and one float a
        row, for the screened argmax; 0 for two to four sequences, which read
        the model's row-major codes)."""
        extra = []
        if getattr(self, "screen", False):
            extra = [t for t in (self.head_copy, self.head_scale, self.head_coef) if t is not None]
        return sum(t.numel() * t.element_size() for t in [*getattr(self, "tiles", {}).values(), *extra])

    def _linear(self, lin: QuantLinear, x: torch.Tensor, y: torch.Tensor, ln=None, act: int = 0, res=None) -> None:
        M, K = x.shape
        st = torch.cuda.current_stream(self.dev).cuda_stream
        scale16 = lin.scale.data_ptr() if lin.fmt == FMT_W4G else None
        scale = None if lin.fmt == FMT_W4G else lin.scale.data_ptr()
        rc = self.L.tiq_linear_fused_ws(
            x.data_ptr(), _lib.F32, M, K, x.stride(0), lin.codes.data_ptr(), _WF[lin.fmt], scale, scale16,
            lin.group_size, _lib.ptr(lin.bias), lin.out_features, y.data_ptr(), _lib.F32, y.stride(0),
            None if ln is None else ln.weight.data_ptr(), None if ln is None else ln.bias.data_ptr(),
            float(ln.eps) if ln is not None else 1e-5, act, None if res is None else res.data_ptr(),
            0 if res is None else res.stride(0), self.lin_ws.data_ptr(), self.lin_ws_bytes, st)
        _lib.check(rc, "fused decode linear")

    # Prompts of at most this many rows (batch x length) are prefilled by the
    # block chain of fused Linears below rather than the model's forward.
    ROW_PREFILL_MAX = 64

    def _start(self, idx: torch.Tensor) -> None:
        """Prefill and the first generated token. A prompt of at most
        ``ROW_PREFILL_MAX`` rows (int8 blocks) runs the block's ops over all
        of its rows with the epilogues fused into the Linears: LayerNorm,
        ``c_attn``, the keys and values into the cache, causal attention over
        the prompt (``tiq_prefill_attention``, reading q, k, v in place from
        the projection's rows), ``c_proj`` + residual, LayerNorm, ``c_fc`` +
        GELU, ``c_proj`` + residual (9 launches a block against the forward's
        12: no separate residual adds or GELU pass); then LayerNorm + head on
        each sequence's last row and the argmax kernels. GPT-2 small, one
        64-token prompt: 0.94 against 1.04 ms, the same tokens. Longer
        prompts take the model's forward (``model.py:528-599``), and so do
        blocks with int4 codes, whose rows take the matrix cores through the
        forward's workspace."""
        B, T0 = idx.shape
        if B * T0 > self.ROW_PREFILL_MAX or not self.rows_prefill:
            super()._start(idx)
            return
        if B != self.B or T0 > self.T:
            raise ValueError(f"prompt {tuple(idx.shape)} does not fit batch={self.B}, max_len={self.T}")
        m, cfg, L = self.model, self.cfg, self.L
        C, R, H, hd = cfg.n_embd, B * T0, self.H, self.hd
        st = torch.cuda.current_stream(self.dev).cuda_stream
        bufs = getattr(self, "_row_bufs", {}).get(T0)
        if bufs is None:  # allocated by the uncaptured warm-up call of start()
            qkv_w = m.h[0].attn.c_attn.out_features
            bufs = (torch.empty(R, C, device=self.dev), torch.empty(R, qkv_w, device=self.dev),
                    torch.empty(R, C, device=self.dev), torch.empty(R, m.h[0].mlp.c_fc.out_features, device=self.dev))
            self._row_bufs = {**getattr(self, "_row_bufs", {}), T0: bufs}
        x, qkv, att, hid = bufs
        # the model's embedding: wte(idx) + wpe(0..T0-1) (model.py:564-568)
        torch.add(m.wte(idx), m.wpe.weight[:T0], out=x.view(B, T0, C))
        for i, block in enumerate(m.h):
            attn, mlp = block.attn, block.mlp
            self._linear_rows(attn.c_attn, _layer_norm(block.ln_1, x), qkv)
            kv = qkv.view(B, T0, 3, H, hd)
            self.k[i][:, :, :T0].copy_(kv[:, :, 1].transpose(1, 2))
            self.v[i][:, :, :T0].copy_(kv[:, :, 2].transpose(1, 2))
            rc = L.tiq_prefill_attention(
                qkv.data_ptr(), T0 * qkv.stride(0), hd, qkv.stride(0), qkv.data_ptr() + 4 * C, T0 * qkv.stride(0),
                hd, qkv.stride(0), qkv.data_ptr() + 8 * C, T0 * qkv.stride(0), hd, qkv.stride(0), B, H, T0, 0, hd,
                att.data_ptr(), T0 * C, hd, C, st)
            _lib.check(rc, "prefill attention")
            self._linear_rows(attn.c_proj, att, x, res=x)
            self._linear_rows(mlp.c_fc, _layer_norm(block.ln_2, x), hid, act=_lib.ACT_GELU_TANH)
            self._linear_rows(mlp.c_proj, hid, x, res=x)
        # LayerNorm + head on each sequence's last row (rows T0 - 1, 2 T0 - 1, ...)
        last = x.view(B, T0, C)[:, T0 - 1]
        ln = m.ln_f
        if self.head_q is not None:
            self._linear_rows(self.head_q, last, self.logits, ln=ln)
        else:
            rc = L.tiq_linear_fused_ws(last.data_ptr(), _lib.F32, B, C, last.stride(0), self.head_w.data_ptr(),
                                       _lib.WF_F32, None, None, 0, None, cfg.vocab_size, self.logits.data_ptr(),
                                       _lib.F32, cfg.vocab_size, ln.weight.data_ptr(), ln.bias.data_ptr(),
                                       float(ln.eps), 0, None, 0, self.lin_ws.data_ptr(), self.lin_ws_bytes, st)
            _lib.check(rc, "lm_head")
        self.out[:, :T0].copy_(idx)
        # the argmax records the first generated token at slot pos + 1 = T0
        # and in tok, and advances pos to T0
        self.pos.fill_(T0 - 1)
        _lib.check(L.tiq_argmax_rows(self.logits.data_ptr(), B, cfg.vocab_size, cfg.vocab_size,
                                     self.tok_flat.data_ptr(), self.out.data_ptr(), self.T, self.pos.data_ptr(),
                                     self.argmax_ws.data_ptr(), self.argmax_ws.numel(), st), "argmax")

    def _linear_rows(self, lin: QuantLinear, x: torch.Tensor, y: torch.Tensor, ln=None, act: int = 0,
                     res=None) -> None:
        """One tiq_linear_fused call over any number of fp32 rows (no
        workspace: the product splits its activations itself)."""
        M, K = x.shape
        st = torch.cuda.current_stream(self.dev).cuda_stream
        scale16 = lin.scale.data_ptr() if lin.fmt == FMT_W4G else None
        scale = None if lin.fmt == FMT_W4G else lin.scale.data_ptr()
        rc = self.L.tiq_linear_fused(
            x.data_ptr(), _lib.F32, M, K, x.stride(0), lin.codes.data_ptr(), _WF[lin.fmt], scale, scale16,
            lin.group_size, _lib.ptr(lin.bias), lin.out_features, y.data_ptr(), _lib.F32, y.stride(0),
            None if ln is None else ln.weight.data_ptr(), None if ln is None else ln.bias.data_ptr(),
            float(ln.eps) if ln is not None else 1e-5, act, None if res is None else res.data_ptr(),
            0 if res is None else res.stride(0), st)
        _lib.check(rc, "fused prefill linear")

    def _dl(self, lin, wf, y=None, x=None, planes_in=None, ln=None, act: int = 0, res=None, next_ln=None,
            planes_out=None) -> None:
        """One tiq_decode_linear: fp32 rows x (optionally LayerNorm'd) or the
        planes of the previous call in; y and / or the planes of next_ln(y) out."""
        st = torch.cuda.current_stream(self.dev).cuda_stream
        K = lin.in_features if hasattr(lin, "in_features") else self.cfg.n_embd
        N = lin.out_features if hasattr(lin, "out_features") else self.cfg.vocab_size
        w = lin.codes if isinstance(lin, QuantLinear) else self.head_w
        tiles = getattr(self, "tiles", {}).get(id(lin))
        if tiles is not None:
            w, wf = tiles, (_lib.WF_F32_TILED if wf == _lib.WF_F32 else _lib.WF_INT8_TILED)
        scale = lin.scale.data_ptr() if isinstance(lin, QuantLinear) else None
        bias = _lib.ptr(lin.bias) if isinstance(lin, QuantLinear) else None
        rc = self.L.tiq_decode_linear(
            _lib.ptr(x), 0 if x is None else x.stride(0), _lib.ptr(planes_in), self.B, K, w.data_ptr(), wf, scale,
            bias, N, _lib.ptr(y), 0 if y is None else y.stride(0), None if ln is None else ln.weight.data_ptr(),
            None if ln is None else ln.bias.data_ptr(), float(ln.eps) if ln is not None else 1e-5, act,
            _lib.ptr(res), 0 if res is None else res.stride(0), None if next_ln is None else next_ln.weight.data_ptr(),
            None if next_ln is None else next_ln.bias.data_ptr(), float(next_ln.eps) if next_ln is not None else 1e-5,
            _lib.ptr(planes_out), self.chain_ws.data_ptr(), self.chain_ws_bytes, st)
        _lib.check(rc, "decode linear")

    def _qkv_attention(self, i: int, lin) -> None:
        """c_attn on LayerNorm 1's planes as split-K slices, then the attention
        of block i summing them (tiq_decode_qkv_attention), its output rows and
        planes out."""
        st = torch.cuda.current_stream(self.dev).cuda_stream
        w, wf = lin.codes, _lib.WF_INT8
        tiles = self.tiles.get(id(lin))
        if tiles is not None:
            w, wf = tiles, _lib.WF_INT8_TILED
        rc = self.L.tiq_decode_qkv_attention(
            self.p_ln1.data_ptr(), self.B, lin.in_features, w.data_ptr(), wf, lin.scale.data_ptr(),
            _lib.ptr(lin.bias), self.H, self.Hkv, self.hd, self.k[i].data_ptr(), self.v[i].data_ptr(), self.T,
            self.pos.data_ptr(), self.att.data_ptr(), self.att.stride(0), self.p_att.data_ptr(),
            self.chain_ws.data_ptr(), self.chain_ws_bytes, st)
        _lib.check(rc, "decode q, k, v projection and attention")

    def _step_chain(self) -> None:
        m, cfg, L = self.model, self.cfg, self.L
        B, C = self.B, cfg.n_embd
        st = torch.cuda.current_stream(self.dev).cuda_stream
        W8 = _lib.WF_INT8
        _lib.check(L.tiq_embed_tokens(self.tok_flat.data_ptr(), self.pos.data_ptr(), m.wte.weight.data_ptr(),
                                      cfg.vocab_size, m.wpe.weight.data_ptr(), cfg.n_positions, B, C,
                                      self.x.data_ptr(), st), "embed")
        n = len(m.h)
        for i, block in enumerate(m.h):
            attn, mlp = block.attn, block.mlp
            if i > 0 and self.qkv_slices:  # LayerNorm 1's planes in, c_attn's slices summed by the attention
                self._qkv_attention(i, attn.c_attn)
            else:
                if i == 0:  # the embedding rows: LayerNorm 1 here
                    self._dl(attn.c_attn, W8, y=self.qkv, x=self.x, ln=block.ln_1)
                else:       # the previous block left LayerNorm 1's planes
                    self._dl(attn.c_attn, W8, y=self.qkv, planes_in=self.p_ln1)
                _lib.check(L.tiq_decode_attention_planes(self.qkv.data_ptr(), self.qkv.stride(0), B, self.H,
                                                         self.Hkv, self.hd, self.k[i].data_ptr(),
                                                         self.v[i].data_ptr(), self.T, self.pos.data_ptr(),
                                                         self.att.data_ptr(), self.att.stride(0),
                                                         self.p_att.data_ptr(), st), "decode attention")
            self._dl(attn.c_proj, W8, y=self.x, planes_in=self.p_att, res=self.x, next_ln=block.ln_2,
                     planes_out=self.p_ln2)
            self._dl(mlp.c_fc, W8, planes_in=self.p_ln2, act=_lib.ACT_GELU_TANH, planes_out=self.p_hid)
            nxt = m.h[i + 1].ln_1 if i + 1 < n else m.ln_f
            self._dl(mlp.c_proj, W8, y=self.x, planes_in=self.p_hid, res=self.x, next_ln=nxt, planes_out=self.p_ln1)
        head = self.head_q if self.head_q is not None else m.lm_head
        self._dl(head, W8 if self.head_q is not None else _lib.WF_F32, y=self.logits, planes_in=self.p_ln1)
        _lib.check(L.tiq_argmax_rows(self.logits.data_ptr(), B, cfg.vocab_size, cfg.vocab_size,
                                     self.tok_flat.data_ptr(), self.out.data_ptr(), self.T, self.pos.data_ptr(),
                                     self.argmax_ws.data_ptr(), self.argmax_ws.numel(), st), "argmax")

    def _step(self) -> None:
        if self.chain:
            self._step_chain()
            return
        m, cfg, L = self.model, self.cfg, self.L
        B, C = self.B, cfg.n_embd
        st = torch.cuda.current_stream(self.dev).cuda_stream
        _lib.check(L.tiq_embed_tokens(self.tok_flat.data_ptr(), self.pos.data_ptr(), m.wte.weight.data_ptr(),
                                      cfg.vocab_size, m.wpe.weight.data_ptr(), cfg.n_positions, B, C,
                                      self.x.data_ptr(), st), "embed")
        for i, block in enumerate(m.h):
            attn, mlp = block.attn, block.mlp
            self._linear(attn.c_attn, self.x, self.qkv, ln=block.ln_1)
            _lib.check(L.tiq_decode_attention(self.qkv.data_ptr(), self.qkv.stride(0), B, self.H, self.Hkv, self.hd,
                                              self.k[i].data_ptr(), self.v[i].data_ptr(), self.T,
                                              self.pos.data_ptr(), self.att.data_ptr(), self.att.stride(0), st),
                       "decode attention")
            self._linear(attn.c_proj, self.att, self.x, res=self.x)
            self._linear(mlp.c_fc, self.x, self.hid, ln=block.ln_2, act=_lib.ACT_GELU_TANH)
            self._linear(mlp.c_proj, self.hid, self.x, res=self.x)
        ln = m.ln_f
        if self.screen and self.screen_i8:  # head + argmax, which also records the token and advances pos
            _lib.check(L.tiq_head_argmax_screened_i8(
                self.x.data_ptr(), C, ln.weight.data_ptr(), ln.bias.data_ptr(), float(ln.eps),
                self.head_copy.data_ptr(), self.head_scale.data_ptr(), self.head_w.data_ptr(), self.head_w.stride(0),
                self.head_coef.data_ptr(), cfg.vocab_size, self.logits.data_ptr(), self.tok_flat.data_ptr(),
                self.out.data_ptr(), self.T, self.pos.data_ptr(), self.screen_ws.data_ptr(), self.screen_ws.numel(),
                st), "screened head")
            return
        if self.screen:
            _lib.check(L.tiq_head_argmax_screened(
                self.x.data_ptr(), C, ln.weight.data_ptr(), ln.bias.data_ptr(), float(ln.eps),
                self.head_copy.data_ptr(), self.head_w.data_ptr(), self.head_w.stride(0), self.head_coef.data_ptr(),
                cfg.vocab_size, self.logits.data_ptr(), self.tok_flat.data_ptr(),
                self.out.data_ptr(), self.T, self.pos.data_ptr(), self.screen_ws.data_ptr(), self.screen_ws.numel(),
                st), "screened head")
            return
        if self.head_q is not None:
            self._linear(self.head_q, self.x, self.logits, ln=ln)
        else:
            rc = L.tiq_linear_fused_ws(self.x.data_ptr(), _lib.F32, B, C, C, self.head_w.data_ptr(), _lib.WF_F32,
                                       None, None, 0, None, cfg.vocab_size, self.logits.data_ptr(), _lib.F32,
                                       cfg.vocab_size, ln.weight.data_ptr(), ln.bias.data_ptr(), float(ln.eps), 0,
                                       None, 0, self.lin_ws.data_ptr(), self.lin_ws_bytes, st)
            _lib.check(rc, "lm_head")
        # argmax also records the token at slot pos + 1 and advances pos
        _lib.check(L.tiq_argmax_rows(self.logits.data_ptr(), B, cfg.vocab_size, cfg.vocab_size,
                                     self.tok_flat.data_ptr(), self.out.data_ptr(), self.T, self.pos.data_ptr(),
                                     self.argmax_ws.data_ptr(), self.argmax_ws.numel(), st), "argmax")


def make_decoder(model, batch: int, max_len: int):
    """The fused decoder when the model fits it, else the torch-op one."""
    if fused_supported(model) is None:
        return FusedDecoder(model, batch, max_len)
    return GraphDecoder(model, batch, max_len)


@torch.no_grad()
def generate_graph(model, idx: torch.Tensor, max_new_tokens: int, decoder=None):
    """Greedy generation with a captured decode step; the same token ids as
    ``generate(model, idx, max_new_tokens)``. Pass a ``decoder`` built for
    this batch / length to reuse its captured graph across calls."""
    if decoder is None:
        decoder = make_decoder(model, idx.size(0), min(model.config.n_positions, idx.size(1) + max_new_tokens))
    return decoder.run(idx, max_new_tokens)
