"""gpt2_harness_amd -- MI355X-native quantized inference for GPT-2.

The quantize-and-run API of gpt2-harness (``quantize_tensor``, ``pack_int4``,
``quantize_model``, ``generate`` ...) backed by hand-written HIP kernels for
gfx950 in ``libtiq_hip.so`` (C ABI in ``include/tiq.h``). Importing the
package does not touch the GPU; the first kernel call loads the library and
raises if it is missing or no ROCm GPU is visible.
"""

from .benchmark import BenchRow, benchmark_generation, model_size_bytes, time_call
from .config import GPT2_SIZES, GPTConfig, gpt2_config
from .decode import FusedDecoder, GraphDecoder, generate_graph, make_decoder
from .experiment import SCHEMES, run_quantization_table
from .model import GPT, KVCache
from .qlinear import QuantLinear
from .quantization import (
    TARGET_SUFFIXES,
    QuantResult,
    SyntheticTokenStream,
    load_packed,
    pack_int4,
    packed_size_bytes,
    perplexity_with_error_bars,
    quantize_dequantize,
    quantize_groupwise_int4,
    quantize_linear,
    quantize_model,
    quantize_tensor,
    save_packed,
    unpack_int4,
)
from .sampling import generate

__all__ = [
    "BenchRow",
    "GPT",
    "GPT2_SIZES",
    "FusedDecoder",
    "GPTConfig",
    "GraphDecoder",
    "KVCache",
    "QuantLinear",
    "QuantResult",
    "SCHEMES",
    "SyntheticTokenStream",
    "TARGET_SUFFIXES",
    "benchmark_generation",
    "generate",
    "generate_graph",
    "gpt2_config",
    "load_packed",
    "make_decoder",
    "model_size_bytes",
    "pack_int4",
    "packed_size_bytes",
    "perplexity_with_error_bars",
    "quantize_dequantize",
    "quantize_groupwise_int4",
    "quantize_linear",
    "quantize_model",
    "quantize_tensor",
    "run_quantization_table",
    "save_packed",
    "time_call",
    "unpack_int4",
]
