"""Post-training weight quantization on the MI355X, behind the reference's API.

Same public names, argument meaning and error messages as the reference's
``src/transformer_internals/quantization.py`` (``:55-65``):

* :func:`quantize_tensor`     (``:78-116``)  -- HIP kernel, bit-identical codes
  and scales;
* :func:`quantize_dequantize` (``:119-129``);
* :func:`pack_int4` / :func:`unpack_int4` (``:132-158``) -- HIP kernels, the
  reference's byte layout;
* :func:`quantize_model`      (``:161-216``) -- returns a copy whose target
  Linears are :class:`~gpt2_harness_amd.qlinear.QuantLinear` modules holding
  the codes (int8, or nibble-packed for <= 4 bits), so the forward pass reads
  1 (or 0.5) byte per weight instead of the 4 bytes of the reference's
  simulated fp32 ``W_hat``; the stats dict has the reference's keys;
* :func:`packed_size_bytes`   (``:219-259``) -- same payload schema, written by
  :func:`save_packed`; :func:`load_packed` builds the quantized model straight
  from such a file (codes to :class:`QuantLinear`, no fp32 round trip);
* :func:`perplexity_with_error_bars` (``:262-319``, forward passes and cross
  entropy on the GPU) with :class:`SyntheticTokenStream` standing in for the
  corpus, and :class:`QuantResult`.

Everything runs on the GPU: tensors must live on a ROCm device, and the
functions raise when the HIP library is missing. Group-wise int4 with fp16
scales (``group_size=``) is an extension with no counterpart in the reference.
"""

from __future__ import annotations

import copy
import math
import statistics
import tempfile
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Literal

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .qlinear import FMT_W4, FMT_W4G, FMT_W8, QuantLinear

__all__ = [
    "TARGET_SUFFIXES",
    "QuantResult",
    "SyntheticTokenStream",
    "pack_int4",
    "packed_size_bytes",
    "perplexity_with_error_bars",
    "quantize_dequantize",
    "quantize_groupwise_int4",
    "quantize_linear",
    "quantize_model",
    "quantize_tensor",
    "load_packed",
    "save_packed",
    "unpack_int4",
]

Granularity = Literal["per_tensor", "per_channel"]

#: Module-name suffixes of the Linears that get quantized (``quantization.py:75``).
TARGET_SUFFIXES = ("attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj")


def _check_bits_granularity(bits: int, granularity: str) -> None:
    if bits < 2 or bits > 8:
        raise ValueError(f"bits must be in [2, 8], got {bits}")
    if granularity not in ("per_channel", "per_tensor"):
        raise ValueError(f"unknown granularity {granularity!r}")


def _fp32_on_gpu(w: torch.Tensor, name: str = "w") -> torch.Tensor:
    _lib.require_gpu(w, name)
    if w.dtype != torch.float32:
        raise TypeError(f"{name} must be float32 (the reference quantizes w.float()), got {w.dtype}")
    return w.contiguous()


def quantize_tensor(
    w: torch.Tensor, bits: int, granularity: Granularity = "per_channel"
) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric linear quantization of a weight matrix (one HIP kernel pass).

    Args:
        w: ``(out_features, in_features)`` fp32 weight on the GPU (any shape for
            ``per_tensor``).
        bits: Bit width in ``[2, 8]``.
        granularity: ``per_channel`` (one scale per row) or ``per_tensor``.

    Returns:
        ``(q, scale)``: int8 codes in ``[-2^(b-1), 2^(b-1)-1]`` shaped like ``w``
        and an fp32 scale of shape ``(rows, 1)`` or ``()``, bit-identical to the
        reference's ``quantize_tensor``.
    """
    _check_bits_granularity(bits, granularity)
    w = _fp32_on_gpu(w)
    L = _lib.lib()
    st = _lib.stream_of(w)
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    if granularity == "per_channel":
        if w.dim() != 2:
            raise ValueError(f"per_channel quantization expects a 2-D weight, got shape {tuple(w.shape)}")
        rows, cols = w.shape
        scale = torch.empty((rows, 1), dtype=torch.float32, device=w.device)
        if rows and cols:
            rc = L.tiq_quantize_per_channel(w.data_ptr(), rows, cols, cols, bits, q.data_ptr(), cols,
                                            scale.data_ptr(), st)
            _lib.check(rc, "quantize_tensor(per_channel)")
        return q, scale
    scale = torch.empty((), dtype=torch.float32, device=w.device)
    n = w.numel()
    if n == 0:
        raise RuntimeError("amax(): cannot reduce over an empty tensor")
    ws = torch.empty(int(L.tiq_quantize_per_tensor_workspace(n)), dtype=torch.uint8, device=w.device)
    rc = L.tiq_quantize_per_tensor(w.data_ptr(), n, bits, q.data_ptr(), scale.data_ptr(), ws.data_ptr(),
                                   ws.numel(), st)
    _lib.check(rc, "quantize_tensor(per_tensor)")
    return q, scale


def quantize_dequantize(
    w: torch.Tensor, bits: int, granularity: Granularity = "per_channel"
) -> torch.Tensor:
    """Round-trip through quantization; returns ``q.float() * scale``."""
    q, scale = quantize_tensor(w, bits, granularity)
    rows = q.shape[0] if q.dim() == 2 else 1
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    if q.numel():
        rc = _lib.lib().tiq_dequantize_int8(q.data_ptr(), scale.data_ptr(), int(granularity == "per_channel"),
                                            rows, q.numel() // rows, out.data_ptr(), _lib.stream_of(q))
        _lib.check(rc, "dequantize")
    return out.to(w.dtype)


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """Pack int4 codes two per byte (low nibble = even index, +8 bias)."""
    _lib.require_gpu(q, "q")
    flat = q.reshape(-1)
    if flat.dtype != torch.int8:
        flat = flat.to(torch.int8)
    flat = flat.contiguous()
    out = torch.empty((flat.numel() + 1) // 2, dtype=torch.uint8, device=q.device)
    rc = _lib.lib().tiq_pack_int4(flat.data_ptr(), flat.numel(), out.data_ptr(), _lib.stream_of(q))
    _lib.check(rc, "pack_int4")
    return out


def unpack_int4(packed: torch.Tensor, numel: int) -> torch.Tensor:
    """Inverse of :func:`pack_int4`."""
    _lib.require_gpu(packed, "packed")
    if numel > 2 * packed.numel():
        raise ValueError(f"numel={numel} exceeds the {2 * packed.numel()} codes held by packed")
    p = packed.reshape(-1).contiguous()
    out = torch.empty(numel, dtype=torch.int8, device=packed.device)
    rc = _lib.lib().tiq_unpack_int4(p.data_ptr(), numel, out.data_ptr(), _lib.stream_of(packed))
    _lib.check(rc, "unpack_int4")
    return out


def quantize_groupwise_int4(w: torch.Tensor, group_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Group-wise int4 codes with fp16 scales (no counterpart in the reference).

    Groups are ``group_size`` consecutive columns of a row (the last one
    ragged); ``scale = fp16(amax / 7)`` (0 -> smallest positive fp16, overflow
    -> 65504); codes ``clamp(rint(w / scale), -8, 7)`` packed per row, low
    nibble = even column, +8 bias.

    Returns ``(packed uint8 (rows, ceil(cols/2)), scale fp16 (rows, ceil(cols/group)))``.
    """
    w = _fp32_on_gpu(w)
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    if group_size < 2 or group_size % 2:
        raise ValueError(f"group_size must be even and >= 2, got {group_size}")
    rows, cols = w.shape
    packed = torch.empty((rows, (cols + 1) // 2), dtype=torch.uint8, device=w.device)
    scale = torch.empty((rows, -(-cols // group_size)), dtype=torch.float16, device=w.device)
    if rows and cols:
        rc = _lib.lib().tiq_quantize_groupwise_int4(w.data_ptr(), rows, cols, group_size, packed.data_ptr(),
                                                    scale.data_ptr(), _lib.stream_of(w))
        _lib.check(rc, "quantize_groupwise_int4")
    return packed, scale


def quantize_linear(
    linear: nn.Linear, bits: int, granularity: Granularity = "per_channel", group_size: int | None = None
) -> tuple[QuantLinear, tuple[torch.Tensor, torch.Tensor]]:
    """Build the :class:`QuantLinear` replacing ``linear``.

    Returns ``(module, (q, scale))`` where ``(q, scale)`` are the reference's
    ``quantize_tensor`` outputs (kept for :func:`packed_size_bytes`); for the
    group-wise format they are the packed nibbles and the fp16 scales.
    """
    _check_bits_granularity(bits, granularity)
    w = linear.weight.detach().float()
    N, K = w.shape
    bias = None if linear.bias is None else linear.bias.detach()
    if group_size is not None:
        if bits != 4:
            raise ValueError(f"group-wise quantization is int4 only, got bits={bits}")
        packed, s16 = quantize_groupwise_int4(w, group_size)
        mod = QuantLinear(packed, s16, bias, K, N, bits, f"group{group_size}", FMT_W4G, group_size)
        return mod, (packed, s16)
    q, scale = quantize_tensor(w, bits, granularity)
    return _quant_linear_from_codes(q, scale, bias, bits, granularity), (q, scale)


def _quant_linear_from_codes(q: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None, bits: int,
                             granularity: str) -> QuantLinear:
    """The storage :func:`quantize_linear` picks for ``(q, scale)`` of an
    ``(N, K)`` weight: nibbles for <= 4 bits and even K, int8 codes otherwise."""
    N, K = q.shape
    row_scale = scale.reshape(-1).expand(N).contiguous() if granularity == "per_tensor" else scale.reshape(N)
    if bits <= 4 and K % 2 == 0:
        return QuantLinear(pack_int4(q), row_scale, bias, K, N, bits, granularity, FMT_W4)
    return QuantLinear(q, row_scale, bias, K, N, bits, granularity, FMT_W8)


def _tied_head(model: nn.Module) -> bool:
    head, wte = getattr(model, "lm_head", None), getattr(model, "wte", None)
    return isinstance(head, nn.Linear) and isinstance(wte, nn.Embedding) and head.weight is wte.weight


def _set_submodule(root: nn.Module, name: str, new: nn.Module) -> None:
    parent_name, _, leaf = name.rpartition(".")
    parent = root.get_submodule(parent_name) if parent_name else root
    setattr(parent, leaf, new)


def quantize_model(
    model: nn.Module,
    bits: int,
    granularity: Granularity = "per_channel",
    include_embedding: bool = False,
    group_size: int | None = None,
    *,
    save_to: str | Path | None = None,
) -> tuple[nn.Module, dict[str, Any]]:
    """Return a copy of the model with its target Linears quantized.

    Args:
        model: Source model on the GPU. Not modified.
        bits: Bit width in ``[2, 8]``.
        granularity: ``per_channel`` or ``per_tensor``.
        include_embedding: Also quantize ``wte`` (and so the tied ``lm_head``):
            its ``W_hat`` is written back in fp32 as the reference does, for
            the embedding lookup; the tied ``lm_head`` becomes a
            :class:`QuantLinear` over the same codes, so the head reads 1 (or
            0.5) byte per weight and computes the same ``x @ W_hat^T``.
        group_size: Extension: group-wise int4 with fp16 scales for the
            target Linears (``bits`` must be 4).
        save_to: Extension: also keep the packed checkpoint whose size is
            ``packed_bytes`` at this path (read back by :func:`load_packed`).

    Returns:
        ``(quantized_model, stats)`` with the reference's stats keys.
    """
    _check_bits_granularity(bits, granularity)
    for p in model.parameters():
        _lib.require_gpu(p, "model parameters")
        break
    q_model = copy.deepcopy(model)
    quantized: list[str] = []
    n_quant_params = 0
    codes: dict[str, tuple[torch.Tensor, torch.Tensor]] = {}

    targets = []
    for name, module in q_model.named_modules():
        is_target = name.endswith(TARGET_SUFFIXES)
        is_emb = include_embedding and name == "wte"
        if not (is_target or is_emb) or not isinstance(module, (nn.Linear, nn.Embedding)):
            continue
        targets.append((name, module))

    with torch.no_grad():
        for name, module in targets:
            w = module.weight.data
            if isinstance(module, nn.Linear):
                new, code = quantize_linear(module, bits, granularity, group_size)
                _set_submodule(q_model, name, new)
            else:
                tied = _tied_head(q_model)
                q, scale = quantize_tensor(w.float(), bits, granularity)
                code = (q, scale)
                module.weight.data = quantize_dequantize(w.float(), bits, granularity).to(w.dtype)
                if tied:
                    q_model.lm_head = _quant_linear_from_codes(q, scale, None, bits, granularity)
            codes[name] = code
            quantized.append(name)
            n_quant_params += w.numel()

    total_params = sum(p.numel() for p in {id(p): p for p in model.parameters()}.values())
    stats = {
        "bits": bits,
        "granularity": granularity,
        "include_embedding": include_embedding,
        "n_quantized_tensors": len(quantized),
        "n_quantized_params": n_quant_params,
        "n_total_params": total_params,
        "fraction_quantized": n_quant_params / total_params,
        "packed_bytes": (packed_size_bytes(q_model, codes, bits, group_size=group_size) if save_to is None
                         else save_packed(q_model, codes, bits, save_to, group_size=group_size)),
        "fp32_bytes": total_params * 4,
    }
    stats["compression_ratio"] = stats["fp32_bytes"] / stats["packed_bytes"]
    if group_size is not None:
        stats["group_size"] = group_size
    return q_model, stats


def _packed_payload(
    model: nn.Module,
    codes: dict[str, tuple[torch.Tensor, torch.Tensor]],
    bits: int,
    group_size: int | None = None,
) -> dict[str, torch.Tensor]:
    """The reference's packed checkpoint payload (``quantization.py:239-250``).

    Keys: ``name.q`` (int8 codes, or ``pack_int4`` bytes at 4 bits),
    ``name.scale`` (fp32), ``name.shape`` (int32 ``[N, K]``), plus every other
    unique parameter in fp32. The group-wise format (no counterpart in the
    reference) stores its per-row nibbles, fp16 group scales, the true
    ``[N, K]`` and ``name.group`` (int32).
    """
    payload: dict[str, torch.Tensor] = {}
    for name, (q, scale) in codes.items():
        if group_size is not None and q.dtype == torch.uint8 and scale.dtype == torch.float16:
            K = int(model.get_submodule(name).in_features)
            payload[f"{name}.q"] = q.cpu()
            payload[f"{name}.scale"] = scale.cpu()
            payload[f"{name}.shape"] = torch.tensor([q.shape[0], K], dtype=torch.int32)
            payload[f"{name}.group"] = torch.tensor(group_size, dtype=torch.int32)
            continue
        payload[f"{name}.q"] = (pack_int4(q) if bits == 4 else q).cpu()
        payload[f"{name}.scale"] = scale.to(torch.float32).cpu()
        payload[f"{name}.shape"] = torch.tensor(list(q.shape), dtype=torch.int32)

    quantized_weight_names = {f"{n}.weight" for n in codes}
    seen: set[int] = set()
    for name, p in model.named_parameters():
        if name in quantized_weight_names or id(p) in seen:
            continue
        seen.add(id(p))
        payload[name] = p.detach().to(torch.float32).cpu()
    return payload


def save_packed(
    model: nn.Module,
    codes: dict[str, tuple[torch.Tensor, torch.Tensor]],
    bits: int,
    path: str | Path,
    group_size: int | None = None,
) -> int:
    """Write the packed checkpoint (the reference's payload schema, ``torch.save``)
    to ``path`` and return its size in bytes. ``codes`` is what
    :func:`quantize_model` records (``name -> (q, scale)``)."""
    torch.save(_packed_payload(model, codes, bits, group_size), Path(path))
    return Path(path).stat().st_size


def packed_size_bytes(
    model: nn.Module,
    codes: dict[str, tuple[torch.Tensor, torch.Tensor]],
    bits: int,
    group_size: int | None = None,
) -> int:
    """Serialise a packed checkpoint (reference payload schema) and return its
    real file size (``quantization.py:219-259``)."""
    with tempfile.NamedTemporaryFile(suffix=".pt", delete=False) as fh:
        tmp = Path(fh.name)
    try:
        return save_packed(model, codes, bits, tmp, group_size)
    finally:
        tmp.unlink(missing_ok=True)


def _bits_of_codes(q: torch.Tensor) -> int:
    """Smallest width in [2, 8] whose symmetric range holds every code."""
    lo, hi = int(q.min()), int(q.max())
    b = 2
    while b < 8 and (lo < -(1 << (b - 1)) or hi > (1 << (b - 1)) - 1):
        b += 1
    return b


@torch.no_grad()
def load_packed(model: nn.Module, source: str | Path | dict[str, torch.Tensor]) -> nn.Module:
    """Fill ``model`` from a packed checkpoint written by :func:`save_packed`.

    Every ``name.q`` entry becomes a :class:`QuantLinear` built straight from
    the stored codes and scales (no fp32 weight and no requantization on the
    way); a quantized embedding (``include_embedding``) gets the reference's
    fp32 ``W_hat``; every other stored parameter is copied in. ``model`` is a
    model of the same configuration on the GPU (its own weights are
    overwritten) and is returned. The file is read with ``weights_only=True``.
    """
    payload = source if isinstance(source, dict) else torch.load(Path(source), map_location="cpu",
                                                                 weights_only=True)
    dev = next(model.parameters()).device
    _lib.require_gpu(next(model.parameters()), "model parameters")
    names = [k[: -len(".q")] for k in payload if k.endswith(".q")]
    for name in names:
        q = payload[f"{name}.q"].to(dev)
        scale = payload[f"{name}.scale"].to(dev)
        N, K = (int(v) for v in payload[f"{name}.shape"].tolist())
        module = model.get_submodule(name)
        bias = payload.get(f"{name}.bias")
        bias = None if bias is None else bias.to(dev)
        if f"{name}.group" in payload:
            g = int(payload[f"{name}.group"])
            new = QuantLinear(q, scale, bias, K, N, 4, f"group{g}", FMT_W4G, g)
            _set_submodule(model, name, new)
            continue
        granularity = "per_tensor" if scale.dim() == 0 else "per_channel"
        if q.dtype == torch.uint8:  # pack_int4 of the row-major codes
            bits = 4
            c8 = unpack_int4(q, N * K).view(N, K)
        else:
            c8 = q.view(N, K)
            bits = _bits_of_codes(c8)
        if isinstance(module, nn.Embedding):
            tied = _tied_head(model)
            w_hat = torch.empty(N, K, device=dev)
            rc = _lib.lib().tiq_dequantize_int8(c8.data_ptr(), scale.data_ptr(), int(granularity == "per_channel"),
                                                N, K, w_hat.data_ptr(), _lib.stream_of(c8))
            _lib.check(rc, "dequantize")
            module.weight.data.copy_(w_hat)
            if tied:  # as quantize_model: the head over the same codes
                model.lm_head = _quant_linear_from_codes(c8, scale, None, bits, granularity)
            continue
        _set_submodule(model, name, _quant_linear_from_codes(c8, scale, bias, bits, granularity))
    quantized = set(names)
    for pname, p in model.named_parameters():
        owner = pname.rpartition(".")[0]
        if owner in quantized or pname not in payload:
            continue
        p.data.copy_(payload[pname].to(dev))
    return model


class SyntheticTokenStream:
    """A seeded uniform token stream with the reference's perplexity windows.

    Stands in for the reference's ``TokenDataset`` (``data.py:123-230``) where
    the corpus cannot be fetched: ``sequential_batches`` walks the split in
    non-overlapping windows of ``block_size`` predictions (a window holds
    ``block_size + 1`` ids, ``x = ids[:-1]``, ``y = ids[1:]``, windows ``w``
    starting at ``w * block_size``), ``batch_size`` windows per batch, a
    trailing short window dropped -- the shape of the reference's
    ``sequential_batches`` (``data.py:192-230``).
    """

    def __init__(self, vocab_size: int, n_tokens: int, block_size: int = 128, seed: int = 0) -> None:
        if n_tokens <= block_size + 1:
            raise ValueError(f"a stream of {n_tokens} tokens is too short for block_size={block_size}")
        gen = torch.Generator().manual_seed(seed)
        self.tokens = torch.randint(0, vocab_size, (n_tokens,), generator=gen, dtype=torch.int64)
        self.block_size = block_size

    def sequential_batches(self, split: str, batch_size: int, limit: int | None = None):
        if split not in ("train", "val"):
            raise ValueError(f"unknown split {split!r}")
        data, T = self.tokens, self.block_size
        n_windows = (len(data) - 1) // T
        out = []
        for start in range(0, n_windows, batch_size):
            rows = [data[w * T : w * T + T + 1] for w in range(start, min(start + batch_size, n_windows))]
            rows = [r for r in rows if len(r) == T + 1]
            if not rows:
                break
            block = torch.stack(rows)
            out.append((block[:, :-1].contiguous(), block[:, 1:].contiguous()))
            if limit is not None and len(out) >= limit:
                break
        return out


@torch.no_grad()
def perplexity_with_error_bars(
    model: nn.Module,
    dataset: Any,
    n_chunks: int = 8,
    batches_per_chunk: int = 2,
    batch_size: int = 4,
    device: str | torch.device = "cuda",
) -> dict[str, Any]:
    """Held-out perplexity with a spread over disjoint chunks (``quantization.py:262-319``).

    ``dataset`` is anything with ``sequential_batches(split, batch_size=, limit=)``
    returning ``(x, y)`` id tensors, as the reference's ``TokenDataset`` or
    :class:`SyntheticTokenStream`. The forward passes (prefill-shaped Linears,
    ``M = batch_size * block_size``) and the summed cross entropy run on the
    GPU; the chunk sums come back to the host once, after the last batch.
    """
    model = model.to(device).eval()
    batches = dataset.sequential_batches("val", batch_size=batch_size, limit=n_chunks * batches_per_chunk)
    # chunk c = batches [c * batches_per_chunk, (c + 1) * batches_per_chunk): its
    # loss is the token mean of the summed cross entropy; the per-chunk sums
    # stay on the device (fp64) and come back in one transfer at the end
    n_chunk = -(-len(batches) // batches_per_chunk)
    sums = torch.zeros(n_chunk, dtype=torch.float64, device=device)
    tokens = [0] * n_chunk
    for i, (x, y) in enumerate(batches):
        logits = model(x.to(device))["logits"].float()
        nll = F.cross_entropy(logits.flatten(0, -2), y.to(logits.device).flatten(), reduction="sum")
        sums[i // batches_per_chunk] += nll.double()
        tokens[i // batches_per_chunk] += y.numel()
    losses = [s / n for s, n in zip(sums.tolist(), tokens)]
    return _chunk_spread(losses)


def _chunk_spread(losses: list[float]) -> dict[str, Any]:
    """Mean and sample standard deviation of the chunk losses and of their
    perplexities (the keys of ``quantization.py:305-313``)."""
    def sd(v: list[float]) -> float:
        return statistics.stdev(v) if len(v) > 1 else 0.0

    ppls = [math.exp(v) for v in losses]
    mean = statistics.fmean(losses)
    return {"loss_mean": mean, "loss_std": sd(losses), "ppl_mean": statistics.fmean(ppls), "ppl_std": sd(ppls),
            "ppl_of_mean_loss": math.exp(mean), "n_chunks": len(losses), "chunk_losses": losses}


@dataclass
class QuantResult:
    """One row of the quantization table (``quantization.py:322-343``)."""

    label: str
    bits: int
    granularity: str
    include_embedding: bool
    stats: dict[str, Any]
    quality: dict[str, Any]
    speed: dict[str, Any]

    def to_dict(self) -> dict[str, Any]:
        return {
            "label": self.label,
            "bits": self.bits,
            "granularity": self.granularity,
            "include_embedding": self.include_embedding,
            **self.stats,
            "quality": self.quality,
            "speed": self.speed,
        }
