"""The oracle: CPU restatements of the reference's quantized-inference path.

TEST INFRASTRUCTURE ONLY. ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this package, and only as the
checker (or, for the CPU baseline, as the thing timed on the host). The
shipped library under ``gpt2-harness_amd/`` never imports, links or calls it.

* ``quant_oracle.c`` / :mod:`oracle.quant` -- ``quantize_tensor``,
  ``pack_int4``, ``unpack_int4`` (``quantization.py:78-158``) and the
  group-wise int4 format, in C and in numpy;
* :mod:`oracle.linear` -- dequantize-then-fp32-matmul (``model.py:254`` ...);
* :mod:`oracle.model` -- fp32 GPT-2 init / forward / greedy decode with
  simulated quantization (``model.py:57-599``, ``sampling.py:100-181``).
"""
