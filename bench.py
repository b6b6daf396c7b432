"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (``value``): W8A16 decode GEMV throughput at GPT-2 small Linear
shapes -- one step is the decode-time pass over all 48 quantized Linears of
GPT-2 small (12 layers x {c_attn 768x2304, attn.c_proj 768x768, c_fc
768x3072, mlp.c_proj 3072x768}, K x N) at M = 1 with bf16 activations, int8
per-channel weights and bf16 outputs. Weights are synthetic (N(0, 0.02),
quantized by this library) and rotated over 6 model copies (510 MB) so every
step reads them cold from HBM, past the 256 MB Infinity Cache. Algorithmic
bytes per launch = N*K + 4*N + 2*M*K + 2*M*N; value = bytes / wall time of
the K timed steps (HIP events on the launch stream; one step is one replay
of a captured HIP graph of the 48 launches).

``roofline`` also carries a 1 GiB device copy timed in the same run as the
measured-achievable HBM rate and the per-launch floor of a HIP graph (an
all-but-empty kernel, and this library's GEMV on a 4 KB matrix, back to back:
the fixed cost every decode GEMV launch pays); ``detail["platform_bf16_gemm"]`` is the
matching measured-achievable bf16 matrix-core rate (an 8192^3 platform GEMM).
``detail`` adds the other configurations:
M = 4 / 16 at the same shapes, GPT-2-XL layer shapes at M = 1 (per shape),
the int8->bf16 MFMA GEMM at GPT-2-XL shapes with M = 256 / 1024 / 4096, the
quantize kernels at GPT-2-XL shapes (a graph of calls over cold weight
copies), GPT-2 small int8 greedy decode (64-token prompt, 64 new tokens)
with its token parity against the reference fixture, and GPT-2-XL batch-32
greedy decode. ``cpu_baseline`` times the oracle's dequantize-then-
fp32-matmul (the reference's runtime arithmetic) on the host cores over a
bounded sample of the same GEMV workload; ``detail["cpu_oracle"]`` times the
oracle on bounded samples of the other configurations (greedy decode,
quantize, prefill F.linear, the GPT-2-XL batch-32 step extrapolated from a
2-layer model), each with its sample stated.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--quick]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "gpt2-harness_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "quantized-linear HBM GB/s (decode GEMV) + GPT-2 int8 decode tokens/sec, 1 GPU"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

SMALL_KN = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]
XL_KN = [(1600, 4800), (1600, 1600), (1600, 6400), (6400, 1600)]


def host_cores() -> int:
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if quota != "max":
            n = max(1, min(n, int(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    return n


def gemv_bytes(M: int, K: int, N: int, x_bytes: int = 2, y_bytes: int = 2) -> int:
    return N * K + 4 * N + x_bytes * M * K + y_bytes * M * N


class LinearSet:
    """Quantized weights of `copies` x `layers` Linears of the given shapes,
    with activation / output buffers, launched through the C ABI."""

    def __init__(self, kn, layers, copies, M, dev, seed=0, x_dtype=None, y_dtype=None):
        import torch

        import gpt2_harness_amd as g
        from gpt2_harness_amd import _lib

        self.torch, self.lib = torch, _lib.lib()
        self.M = M
        x_dtype = x_dtype or torch.bfloat16
        y_dtype = y_dtype or torch.bfloat16
        self.xd, self.yd = _lib.dtype_code(x_dtype), _lib.dtype_code(y_dtype)
        gen = torch.Generator(device=dev).manual_seed(seed)
        self.items = []  # per copy: list of (K, N, q, s, x, y)
        xs = {K: torch.randn(M, K, generator=gen, device=dev).to(x_dtype) for K, _ in kn}
        for _c in range(copies):
            items = []
            for _l in range(layers):
                for K, N in kn:
                    w = torch.randn(N, K, generator=gen, device=dev) * 0.02
                    q, s = g.quantize_tensor(w, 8)
                    del w
                    y = torch.empty(M, N, device=dev, dtype=y_dtype)
                    items.append((K, N, q, s.reshape(-1).contiguous(), xs[K], y))
            self.items.append(items)
        torch.cuda.synchronize()
        self.bytes_per_copy = sum(gemv_bytes(M, K, N, x_dtype.itemsize, y_dtype.itemsize)
                                  for K, N, *_ in self.items[0])
        self.launches_per_copy = len(self.items[0])

    def launch_copy(self, c: int, entry: str = "tiq_linear_w8") -> None:
        fn = getattr(self.lib, entry)
        st = self.torch.cuda.current_stream().cuda_stream
        for K, N, q, s, x, y in self.items[c]:
            rc = fn(x.data_ptr(), self.xd, self.M, K, K, q.data_ptr(), s.data_ptr(), None, N, y.data_ptr(), self.yd,
                    N, st)
            if rc:
                raise RuntimeError(f"{entry} failed with status {rc}")


def capture_graphs(ls: LinearSet, entry: str = "tiq_linear_w8"):
    """One HIP graph per weight copy. Copy 0 runs once eagerly first (module
    load); every other launch of the section is a graph replay."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ls.launch_copy(0, entry)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graphs = []
    for c in range(len(ls.items)):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            ls.launch_copy(c, entry)
        graphs.append(gr)
    return graphs


def replay_ms(graphs, steps: int, warmup: int) -> float:
    """Mean ms per replay over `steps` replays (rotating over the graphs),
    HIP events on the stream the graphs replay on."""
    import torch

    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def per_shape_graph_times(ls: LinearSet, reps: int, entry: str = "tiq_linear_w8"):
    """Per shape: a graph of that shape's launches over every layer and copy,
    timed alone (HIP events) after a 512 MiB buffer write has evicted the
    weights from the 256 MB Infinity Cache; returns ms per launch."""
    import torch

    flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    out = {}
    for K, N in dict.fromkeys((K, N) for K, N, *_ in ls.items[0]):
        fn = getattr(ls.lib, entry)
        gr = torch.cuda.CUDAGraph()
        launches = 0
        with torch.cuda.graph(gr):
            st = torch.cuda.current_stream().cuda_stream
            for items in ls.items:
                for k, n, q, s, x, y in items:
                    if (k, n) != (K, N):
                        continue
                    rc = fn(x.data_ptr(), ls.xd, ls.M, k, k, q.data_ptr(), s.data_ptr(), None, n, y.data_ptr(),
                            ls.yd, n, st)
                    if rc:
                        raise RuntimeError(f"{entry} failed with status {rc}")
                    launches += 1
        total = 0.0
        for _ in range(reps):
            flush.fill_(1)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            gr.replay()
            b.record()
            torch.cuda.synchronize()
            total += a.elapsed_time(b)
        out[(K, N)] = total / reps / launches
    del flush
    return out


class Stamps:
    """Kernel durations measured inside a timed run: between begin() and
    end() every stamped launch (tiq_stamp_begin) writes each workgroup's entry
    and exit on the GPU's 100 MHz real-time counter and on its shader-clock
    counter (four slots a workgroup); a launch's duration is its first
    workgroup's entry to its last workgroup's exit, its clock the shader
    cycles over the real time summed over its workgroups. Launches captured in
    a graph keep their slots, so after the timed replays the slots hold the
    last replay of each graph."""

    def __init__(self, dev, slots=1 << 23):
        import torch

        from gpt2_harness_amd import _lib

        self.lib, self.torch = _lib.lib(), torch
        self.buf = torch.zeros(slots, dtype=torch.int64, device=dev)
        self.launches: list[tuple[int, int]] = []

    def begin(self):
        rc = self.lib.tiq_stamp_begin(self.buf.data_ptr(), self.buf.numel())
        if rc:
            raise RuntimeError(f"tiq_stamp_begin status {rc}")

    def end(self):
        import ctypes

        n = 1 << 16
        first, wgs = (ctypes.c_int64 * n)(), (ctypes.c_int64 * n)()
        k = int(self.lib.tiq_stamp_end(first, wgs, n))
        self.launches = [(first[i], wgs[i]) for i in range(min(k, n))]
        return len(self.launches)

    def _slots(self):
        self.torch.cuda.synchronize()
        h = self.buf.cpu()
        return [h[s0: s0 + 4 * g].view(g, 4) for s0, g in self.launches]

    def durations_us(self):
        """Per stamped launch: (last exit - first entry) in us."""
        return [float(t[:, 1].max() - t[:, 0].min()) * 0.01 for t in self._slots()]

    def clocks_ghz(self):
        """Per stamped launch: shader cycles / real time over its workgroups, GHz."""
        return [float((t[:, 3] - t[:, 2]).sum()) / float((t[:, 1] - t[:, 0]).sum() * 10) for t in self._slots()]


def gemv_section(M, kn, layers, copies, steps, warmup, dev, seed, per_shape=True, stamped=False):
    ls = LinearSet(kn, layers, copies, M, dev, seed)
    ms = replay_ms(capture_graphs(ls), steps, warmup)
    gbs = ls.bytes_per_copy / (ms * 1e-3) / 1e9
    res = {"M": M, "ms_per_step": ms, "GB/s": gbs, "launches_per_step": ls.launches_per_copy,
           "bytes_per_step": ls.bytes_per_copy, "avg_launch_us": ms * 1e3 / ls.launches_per_copy}
    if stamped:
        # the same timed replays again with the stamped copies of the kernel:
        # each launch's own duration inside the replays (no per-dispatch
        # isolation as under a tracer), the replay time beside it
        st = Stamps(dev)
        ls.launch_copy(0)  # module load outside the stamps
        st.begin()
        try:
            graphs = capture_graphs(ls)
        finally:
            n = st.end()
        want = (copies + 1) * ls.launches_per_copy  # capture_graphs' eager first copy, then the graphs
        if n != want:
            raise RuntimeError(f"stamped launches {n}, expected {want}")
        ms_st = replay_ms(graphs, steps, warmup)
        d = st.durations_us()[ls.launches_per_copy:]  # the captured launches (the first ones ran eagerly)
        clk = statistics.fmean(st.clocks_ghz()[ls.launches_per_copy:])
        kus = statistics.fmean(d)
        res["stamped"] = {"kernel_us": kus, "kernel_us_min": min(d), "kernel_us_max": max(d), "launches": len(d),
                          "ms_per_step": ms_st, "kernel_sum_over_step": kus * ls.launches_per_copy / (ms_st * 1e3),
                          "clock_GHz": clk}
        res["kernel_us"] = kus
        res["kernel_GB/s"] = ls.bytes_per_copy / ls.launches_per_copy / (kus * 1e-6) / 1e9
        del graphs
    if per_shape:
        per = per_shape_graph_times(ls, 5)
        res["per_shape_graph"] = {f"{K}x{N}": {"us": per[(K, N)] * 1e3,
                                              "GB/s": gemv_bytes(M, K, N) / (per[(K, N)] * 1e-3) / 1e9}
                                  for K, N in kn}
    del ls
    return res


def hbm_stream_section(dev, reps=10):
    """Measured-achievable HBM rate beside the 8 TB/s datasheet figure:
    torch's device copy of 1 GiB (read + write counted), the median of `reps`
    launches between HIP events."""
    import torch

    n = 1 << 28
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        dst.copy_(src)
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b))
    del src, dst
    return {"copy": {"GB/s": 8 * n / (statistics.median(ts) * 1e-3) / 1e9, "bytes": 8 * n}}


def decode_linears_section(dev, layers=6, rounds=3):
    """The batched decode step's four Linears at GPT-2-XL widths, M = 32,
    called eagerly (no graph) exactly as the fused decoder's step calls them
    (tiq_decode_linear from the previous op's operand planes), on a
    ``layers``-layer XL-width model, ``rounds`` passes over its layers: a
    short program for counter runs of those kernels (``--only decode_lin``);
    the timed figures are decode_xl_section's."""
    import torch

    import gpt2_harness_amd as g
    from gpt2_harness_amd import _lib

    torch.manual_seed(0)
    cfg = g.gpt2_config("gpt2-xl", n_layer=layers)
    model = g.GPT(cfg).eval().to(dev)
    qm, _ = g.quantize_model(model, 8)
    del model
    B, T0 = 32, 128
    prompt = torch.randint(0, cfg.vocab_size, (B, T0)).to(dev)
    dec = g.FusedDecoder(qm, B, T0 + 8)
    dec.start(prompt)
    W8, gelu = _lib.WF_INT8, _lib.ACT_GELU_TANH
    blocks = list(qm.h)
    for _ in range(rounds):
        for i, b in enumerate(blocks):
            nb = blocks[i + 1].ln_1 if i + 1 < len(blocks) else qm.ln_f
            dec._dl(b.attn.c_attn, W8, y=dec.qkv, planes_in=dec.p_ln1)
            dec._dl(b.attn.c_proj, W8, y=dec.x, planes_in=dec.p_att, res=dec.x, next_ln=b.ln_2,
                    planes_out=dec.p_ln2)
            dec._dl(b.mlp.c_fc, W8, planes_in=dec.p_ln2, act=gelu, planes_out=dec.p_hid)
            dec._dl(b.mlp.c_proj, W8, y=dec.x, planes_in=dec.p_hid, res=dec.x, next_ln=nb,
                    planes_out=dec.p_ln1)
    torch.cuda.synchronize()
    return {"layers": layers, "rounds": rounds, "calls": 4 * layers * rounds, "batch": B}


def launch_floor_section(dev, launches=240, reps=5):
    """What one launch costs inside a HIP graph, the floor a decode GEMV sits
    on: back-to-back graph replays of `launches` launches of (a) a one-element
    torch fill (an all-but-empty kernel) and (b) this library's M = 1 GEMV on
    a 64 x 64 int8 matrix (its own argument path, one 4 KB read); HIP events
    around each replay, the median over `reps` replays, per launch."""
    import torch

    import gpt2_harness_amd as g
    from gpt2_harness_amd import _lib

    L = _lib.lib()
    t = torch.zeros(1, device=dev)
    q, sc = g.quantize_tensor(torch.randn(64, 64, device=dev) * 0.02, 8)
    sc = sc.reshape(-1).contiguous()
    x = torch.randn(1, 64, device=dev).to(torch.bfloat16)
    y = torch.empty(1, 64, device=dev, dtype=torch.bfloat16)

    def gemv():
        rc = L.tiq_linear_w8(x.data_ptr(), 1, 1, 64, 64, q.data_ptr(), sc.data_ptr(), None, 64, y.data_ptr(), 1, 64,
                             torch.cuda.current_stream().cuda_stream)
        if rc:
            raise RuntimeError(f"tiq_linear_w8 status {rc}")

    out = {}
    cases = (("torch_fill_1_element", lambda i: t.fill_(1.0)), ("tiq_linear_w8_64x64_M1", lambda i: gemv()))
    for name, fn in cases:
        s_cap = torch.cuda.Stream()
        with torch.cuda.stream(s_cap):
            fn(0)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=s_cap):
                for i in range(launches):
                    fn(i)
        gr.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            gr.replay()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e3 / launches)
        out[name] = {"us_per_launch": statistics.median(ts), "launches_per_graph": launches}
        del gr
    return out


def mfma_platform_section(dev, n=8192, reps=10):
    """Measured-achievable bf16 matrix-core rate beside the 2.5 PFLOP/s
    datasheet figure: the platform GEMM (torch.matmul -> hipBLASLt) on an
    n x n x n bf16 product, the median of `reps` launches between HIP events.
    Under a full-chip matrix load the MI355X clock settles well below its 2.4 GHz
    peak, so this, not the datasheet, is the ceiling the GEMM rows sit under."""
    import torch

    gen = torch.Generator(device=dev).manual_seed(3)
    a = torch.randn(n, n, generator=gen, device=dev).bfloat16()
    b = torch.randn(n, n, generator=gen, device=dev).bfloat16()
    c = torch.matmul(a, b)
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.matmul(a, b, out=c)
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    del a, b, c
    tf = 2 * n ** 3 / (statistics.median(ts) * 1e-3) / 1e12
    return {"shape": f"{n}x{n}x{n} bf16", "TFLOP/s": tf, "frac_bf16_peak": tf / BF16_PEAK_TFLOPS}


def gemm_section(M, kn, dev, reps=24, copies=8, fmt="int8", stamped=False):
    """int8 -> bf16 prefill GEMM (tiq_gemm_w8_ws; fmt="int4": the reference
    nibble layout, tiq_linear_w4; fmt="int4_g128": the group-wise int4 GEMM,
    tiq_linear_w4g_ws, group 128, split over K where the tiles are few) per
    shape: a captured HIP graph of one launch per `copies` independent
    (activation, weight, output) sets (at M = 4096 on 1600 x 6400 the eight
    sets hold 600 MB, past the 256 MB Infinity Cache), so no launch finds its
    operands left in the caches by the one before; the graph replayed between
    one HIP event pair, the median over `reps // copies` timings, per launch.
    In a graph neither side pays the host's launch cost (the platform GEMM's
    eager call costs 20 us a launch on the host, more than its kernel at
    M = 256). Beside it, as the measured-achievable reference (not this
    library's path), the platform's bf16 GEMM (torch.matmul -> hipBLASLt) on
    bf16 weights of the same shape, rotated the same way. The stamped pass
    (M = 4096) times `reps` eager launches instead, one stamp slot each."""
    import torch

    import gpt2_harness_amd as g
    from gpt2_harness_amd import _lib

    L = _lib.lib()
    out = {}
    gen = torch.Generator(device=dev).manual_seed(1)

    def timed(fns):
        for f in fns[:3]:
            f()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(reps):
            fns[i % len(fns)]()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / reps

    def timed_graph(fns):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            for f in fns:
                f()
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=s):
                for f in fns:
                    f()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(max(reps // len(fns), 3)):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            graph.replay()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e3 / len(fns))
        del graph
        return statistics.median(ts)

    for K, N in kn:
        n_ws = int(L.tiq_gemm_w8_workspace(1, M, K, N))  # split-K partials when the tiles are few
        ws = torch.empty(max(n_ws, 1), dtype=torch.uint8, device=dev)
        sets, lib_sets = [], []
        for _ in range(copies):
            w = torch.randn(N, K, generator=gen, device=dev) * 0.02
            if fmt == "int8":
                q, s = g.quantize_tensor(w, 8)
                s = s.reshape(-1).contiguous()
            elif fmt == "int4":
                q4, s = g.quantize_tensor(w, 4)
                q, s = g.pack_int4(q4), s.reshape(-1).contiguous()
            else:
                q, s = g.quantize_groupwise_int4(w, 128)
            x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
            sets.append((x, q, s, torch.empty(M, N, device=dev, dtype=torch.bfloat16)))
            lib_sets.append((x, w.to(torch.bfloat16), torch.empty(M, N, device=dev, dtype=torch.bfloat16)))
            del w

        def run(x, q, s, y):
            st = torch.cuda.current_stream().cuda_stream  # the capturing stream inside a graph
            if fmt == "int8":
                rc = L.tiq_gemm_w8_ws(x.data_ptr(), 1, M, K, K, q.data_ptr(), s.data_ptr(), None, N, y.data_ptr(), 1,
                                      N, ws.data_ptr(), n_ws, st)
            elif fmt == "int4":
                rc = L.tiq_linear_w4(x.data_ptr(), 1, M, K, K, q.data_ptr(), s.data_ptr(), None, N, y.data_ptr(), 1,
                                     N, st)
            else:
                rc = L.tiq_linear_w4g_ws(x.data_ptr(), 1, M, K, K, q.data_ptr(), s.data_ptr(), 128, None, N,
                                         y.data_ptr(), 1, N, ws.data_ptr(), n_ws, st)
            if rc:
                raise RuntimeError(f"{fmt} GEMM status {rc}")

        us = timed_graph([lambda a=a: run(*a) for a in sets])
        tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
        stamp = None
        if stamped and fmt == "int8":
            # the same timed launches again, the stamped copy of the staged
            # kernel: each launch's first-workgroup entry to last-workgroup exit
            stamps = Stamps(dev)
            stamps.begin()
            try:
                us_st = timed([lambda a=a: run(*a) for a in sets])
            finally:
                stamps.end()
            d = stamps.durations_us()[3:]  # after timed()'s three warm-up launches
            if len(d) == reps:  # one stamped kernel a launch (no split-K at this size)
                kus = statistics.fmean(d)
                clk = statistics.fmean(stamps.clocks_ghz()[3:])
                tf_k = 2.0 * M * N * K / (kus * 1e-6) / 1e12
                # the matrix cores' peak scales with the shader clock (datasheet: 2.4 GHz)
                stamp = {"kernel_us": kus, "TFLOP/s": tf_k, "launch_us": us_st, "clock_GHz": clk,
                         "frac_of_peak_at_clock": tf_k / (BF16_PEAK_TFLOPS * clk / 2.4)}
        us_lib = timed_graph([lambda x=x, wb=wb, yb=yb: torch.matmul(x, wb.T, out=yb) for x, wb, yb in lib_sets])
        tf_lib = 2.0 * M * N * K / (us_lib * 1e-6) / 1e12
        out[f"{K}x{N}"] = {"us": us, "TFLOP/s": tf, "frac_bf16_peak": tf / BF16_PEAK_TFLOPS,
                           "library_bf16_us": us_lib, "library_bf16_TFLOP/s": tf_lib,
                           "vs_library_bf16": tf / tf_lib}
        if stamp:
            out[f"{K}x{N}"]["stamped"] = stamp
        del sets, lib_sets
    return {"M": M, "weights": fmt, "copies": copies, "per_shape": out}


def quantize_section(dev, reps=5, copies=8):
    """Quantize kernels at GPT-2-XL shapes with data resident in HBM.

    One timed unit is a captured HIP graph of ``copies`` API calls, one per
    copy of the weight, so every call reads its fp32 weight cold from HBM
    (8 copies of the largest matrix, 328 MB, exceed the 256 MB Infinity
    Cache); per-call time = replay time / copies. ``api_us`` is the eager
    Python call (allocations, argument checks and launch included).
    """
    import torch

    import gpt2_harness_amd as g

    out = {}
    gen = torch.Generator(device=dev).manual_seed(2)
    for K, N in XL_KN:
        ws = []
        for _ in range(copies):
            w = torch.randn(N, K, generator=gen, device=dev) * 0.02
            n_out = max(1, N * K // 1000)
            idx = torch.randperm(N * K, generator=gen, device=dev)[:n_out]
            w.view(-1)[idx] *= 20.0
            ws.append(w)
        for label, fn, nbytes in (
            ("int8_per_channel", lambda w: g.quantize_tensor(w, 8), 5 * N * K + 4 * N),
            ("int4_g128", lambda w: g.quantize_groupwise_int4(w, 128),
             4 * N * K + N * K // 2 + 2 * N * -(-K // 128)),
        ):
            fn(ws[0])
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                fn(ws[0])
            torch.cuda.synchronize()
            api_us = (time.perf_counter() - t0) / reps * 1e6
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                fn(ws[0])
                torch.cuda.synchronize()
                with torch.cuda.graph(graph, stream=s):
                    keep = [fn(w) for w in ws]
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            ts = []
            for _ in range(reps):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                graph.replay()
                b.record()
                torch.cuda.synchronize()
                ts.append(a.elapsed_time(b) / copies)
            ms = statistics.median(ts)
            out[f"{label}_{K}x{N}"] = {"us": ms * 1e3, "GB/s": nbytes / (ms * 1e-3) / 1e9,
                                       "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                       "api_us": api_us}
            del graph, keep
        del ws
    return out


def decode_section(dev, repeats=3):
    import torch

    import gpt2_harness_amd as g

    golden = json.loads((ROOT / "tests" / "golden" / "reference_decode.json").read_text())["gpt2_small"]
    torch.manual_seed(0)
    model = g.GPT(g.GPTConfig()).to(dev).eval()
    qm, _ = g.quantize_model(model, 8)
    del model
    torch.manual_seed(0)
    prompt = torch.randint(0, 50257, (1, 64)).to(dev)
    want = golden["greedy_int8"]["ids"]
    res = {"model": "gpt2 (124M) seed 0, int8 per-channel", "prompt": 64, "new_tokens": 64}
    dec_t = g.GraphDecoder(qm, 1, 128)
    dec_f = g.FusedDecoder(qm, 1, 128)  # the screened head from the int8 copy
    dec_b = g.FusedDecoder(qm, 1, 128, head_screen="bf16")
    for label, fn in (("eager", lambda: g.generate(qm, prompt, 64)),
                      ("graph_torch_ops", lambda: g.generate_graph(qm, prompt, 64, decoder=dec_t)),
                      ("graph_fused", lambda: g.generate_graph(qm, prompt, 64, decoder=dec_f)),
                      ("graph_fused_bf16_screen", lambda: g.generate_graph(qm, prompt, 64, decoder=dec_b))):
        out = fn()
        match = out.cpu().tolist() == want
        ts = []
        for _ in range(repeats):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        med = statistics.median(ts)
        res[label] = {"tokens_per_s": 64 / med, "ms_per_token": 1e3 * med / 64, "tokens_match_reference": match}
    del dec_t, dec_f, dec_b, qm
    # the reference's fifth scheme: int8 per-channel + embedding; the tied
    # head (50257 x 768) runs on int8 codes (token parity: the GPU tests
    # against the oracle, no reference fixture holds these tokens)
    torch.manual_seed(0)
    model = g.GPT(g.GPTConfig()).to(dev).eval()
    qe, _ = g.quantize_model(model, 8, include_embedding=True)
    del model
    dec_e = g.FusedDecoder(qe, 1, 128)
    g.generate_graph(qe, prompt, 64, decoder=dec_e)
    ts = []
    for _ in range(repeats):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.generate_graph(qe, prompt, 64, decoder=dec_e)
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    med = statistics.median(ts)
    res["graph_fused_int8_embedding"] = {"tokens_per_s": 64 / med, "ms_per_token": 1e3 * med / 64}
    return res


def eval_section(dev):
    """GPT-2 small seed 0 int8 per-channel: the packed checkpoint written by
    quantize_model(save_to=) and read back into a fresh model by load_packed,
    then the reference's held-out evaluation shape (8 chunks x 2 batches x 4
    windows of 128 tokens: 16 forward passes with M = 512 prefill Linears)
    over synthetic tokens on the GPU."""
    import tempfile

    import torch

    import gpt2_harness_amd as g

    torch.manual_seed(0)
    model = g.GPT(g.GPTConfig()).to(dev).eval()
    res = {"model": "gpt2 (124M) seed 0, int8 per-channel"}
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "gpt2_int8.pt"
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        qm, stats = g.quantize_model(model, 8, save_to=path)
        torch.cuda.synchronize()
        t_quant = time.perf_counter() - t0
        del qm
        skeleton = g.GPT(g.GPTConfig()).to(dev).eval()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loaded = g.load_packed(skeleton, path)
        torch.cuda.synchronize()
        t_load = time.perf_counter() - t0
    del model
    res["packed_checkpoint"] = {"bytes": stats["packed_bytes"], "compression_ratio": stats["compression_ratio"],
                                "quantize_model_and_save_s": t_quant, "load_packed_s": t_load}
    ds = g.SyntheticTokenStream(50257, 8 * 2 * 4 * 128 + 1, 128, seed=0)
    g.perplexity_with_error_bars(loaded, ds, n_chunks=1, batches_per_chunk=1, device=dev)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ppl = g.perplexity_with_error_bars(loaded, ds, device=dev)
    torch.cuda.synchronize()
    t = time.perf_counter() - t0
    res["perplexity"] = {"forward_passes": 16, "tokens": 8 * 2 * 4 * 128, "seconds": t,
                         "tokens_per_s": 8 * 2 * 4 * 128 / t, "loss_mean": ppl["loss_mean"],
                         "loss_std": ppl["loss_std"], "ppl_of_mean_loss": ppl["ppl_of_mean_loss"]}
    return res


def greedy_agreement(got, want, gaps, gpu_last, oracle_last, prompt_len):
    """Token-for-token comparison of a GPU greedy generation with the oracle's:
    the first divergent (step, sequence) with the oracle's top-1 minus top-2
    logit gap there, the smallest gap over every step and sequence, and --
    when every token agrees -- the largest |logit difference| at the last step
    (the size of the fp32 summation-order differences the gaps are set
    against)."""
    import torch

    n = want.size(1) - prompt_len
    out = {"steps": n, "sequences": int(want.size(0)), "tokens_match": bool(torch.equal(got, want)),
           "min_top2_margin": float(gaps.min()) if gaps.numel() else None}
    diff = (got[:, prompt_len:] != want[:, prompt_len:]).nonzero()
    if diff.numel():
        step = int(diff[:, 1].min())
        seq = int(diff[diff[:, 1] == step][0, 0])
        out["first_divergence"] = {"step": step, "sequence": seq, "oracle_top2_margin": float(gaps[step, seq]),
                                   "steps_all_equal": step}
    elif gpu_last is not None and oracle_last is not None:
        out["last_step_max_abs_logit_diff"] = float((gpu_last.double() - oracle_last.double()).abs().max())
    return out


def decode_xl_section(dev, new_tokens=128, check_steps=None):
    """GPT-2-XL (48 layers, d 1600, 25 heads) seed 0, int8 per-channel, batch
    32, 128-token random prompts, greedy +new_tokens: end-to-end tokens/s
    (prefill + decode) and the per-Linear decode time / GB/s at M = 32.
    The step is the fused decoder's batched chain (tiq_decode_linear,
    tiq_decode_attention_planes), captured once and replayed per token.
    ``tokens_match_oracle``: every generated token (``check_steps``, all of
    them by default) of all 32 sequences against the oracle's fp32 CPU
    generation of the same seed-0 quantized model."""
    check_steps = new_tokens if check_steps is None else check_steps
    import torch

    import gpt2_harness_amd as g
    from gpt2_harness_amd import _lib
    from oracle import model as OM

    torch.manual_seed(0)
    cfg = g.gpt2_config("gpt2-xl")
    model = g.GPT(cfg).eval()
    p_cpu = {k: v.detach().clone() for k, v in model.state_dict().items() if k != "lm_head.weight"}
    model = model.to(dev)
    qm, _ = g.quantize_model(model, 8)
    del model
    torch.manual_seed(0)
    B, T0 = 32, 128
    prompt_cpu = torch.randint(0, cfg.vocab_size, (B, T0))
    prompt = prompt_cpu.to(dev)
    dec = g.FusedDecoder(qm, B, T0 + new_tokens)
    dec.start(prompt)
    dec.capture()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.start(prompt)
    torch.cuda.synchronize()
    t_pre = time.perf_counter() - t0
    t0 = time.perf_counter()
    for _ in range(new_tokens - 1):
        dec.graph.replay()
    torch.cuda.synchronize()
    t_dec = time.perf_counter() - t0
    got = dec.out[:, : T0 + check_steps].cpu()
    gpu_last = dec.logits.cpu() if check_steps == new_tokens else None  # the last replay's logits
    res = {"model": "gpt2-xl (1.56B) seed 0, int8 per-channel", "batch": B, "prompt": T0, "new_tokens": new_tokens,
           "prefill_ms": t_pre * 1e3, "decode_ms_per_step": t_dec * 1e3 / (new_tokens - 1),
           "tokens_per_s": B * new_tokens / (t_pre + t_dec),
           "decode_tokens_per_s": B * (new_tokens - 1) / t_dec}
    # per-Linear decode time at M = 32, each called as the decode step calls it
    # (tiq_decode_linear from the previous op's operand planes): a graph of the
    # 48 layers' calls of one Linear (their weights: 123-492 MB, past the 256 MB
    # Infinity Cache for all but attn.c_proj), replayed after a 512 MiB write has
    # evicted the caches, HIP events around each replay; GB/s by the decode GEMV
    # formula N K + 4 N + 2 M K + 2 M N
    per = {}
    W8, gelu = _lib.WF_INT8, _lib.ACT_GELU_TANH
    calls = (("c_attn", lambda b: b.attn.c_attn, lambda l, b, nb: dec._dl(l, W8, y=dec.qkv, planes_in=dec.p_ln1)),
             ("attn.c_proj", lambda b: b.attn.c_proj,
              lambda l, b, nb: dec._dl(l, W8, y=dec.x, planes_in=dec.p_att, res=dec.x, next_ln=b.ln_2,
                                       planes_out=dec.p_ln2)),
             ("c_fc", lambda b: b.mlp.c_fc,
              lambda l, b, nb: dec._dl(l, W8, planes_in=dec.p_ln2, act=gelu, planes_out=dec.p_hid)),
             ("mlp.c_proj", lambda b: b.mlp.c_proj,
              lambda l, b, nb: dec._dl(l, W8, y=dec.x, planes_in=dec.p_hid, res=dec.x, next_ln=nb,
                                       planes_out=dec.p_ln1)))
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    s_cap = torch.cuda.Stream()
    blocks = list(qm.h)
    for name, pick, fn in calls:
        lin0 = pick(blocks[0])
        K, N = lin0.in_features, lin0.out_features
        layer_calls = [(pick(b), b, blocks[i + 1].ln_1 if i + 1 < len(blocks) else qm.ln_f)
                       for i, b in enumerate(blocks)]
        with torch.cuda.stream(s_cap):
            fn(*layer_calls[0])
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=s_cap):
                for c in layer_calls:
                    fn(*c)
        gr.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(3):
            flush.fill_(1)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            gr.replay()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e3 / len(layer_calls))
        us = statistics.median(ts)
        nbytes = N * K + 4 * N + 2 * B * K + 2 * B * N
        per[f"{K}x{N}"] = {"linear": name, "us": us, "GB/s": nbytes / (us * 1e-6) / 1e9}
        del gr
    # the fp32 tied head at M = 32 from LayerNorm f's planes (4 N K bytes a
    # call, 322 MB: past the Infinity Cache), its weights as the decoder holds
    # them (4 KB operand tiles, streamed by one workgroup per CU) and row-major
    # (one workgroup per 32 rows): a graph of 10 calls, HIP events, median of 3
    head = {}
    V, C = cfg.vocab_size, cfg.n_embd
    tiles = dec.tiles.get(id(qm.lm_head))
    for label, wt, wf in (("tiled", tiles, _lib.WF_F32_TILED), ("row_major", dec.head_w, _lib.WF_F32)):
        if wt is None:
            continue
        st = s_cap.cuda_stream
        call = lambda: _lib.check(dec.L.tiq_decode_linear(
            None, 0, dec.p_ln1.data_ptr(), B, C, wt.data_ptr(), wf, None, None, V, dec.logits.data_ptr(), V, None,
            None, 1e-5, 0, None, 0, None, None, 1e-5, None, dec.chain_ws.data_ptr(), dec.chain_ws_bytes, st), "head")
        with torch.cuda.stream(s_cap):
            call()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=s_cap):
                for _ in range(10):
                    call()
        gr.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(3):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            gr.replay()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e3 / 10)
        us = statistics.median(ts)
        head[label] = {"us": us, "GB/s": 4 * V * C / (us * 1e-6) / 1e9}
        del gr
    del flush
    res["decode_linear_M32_cold"] = per
    res["lm_head_fp32_M32"] = head
    del dec, qm
    torch.cuda.empty_cache()
    # the oracle on the same seed-0 weights, first check_steps tokens
    threads = torch.get_num_threads()
    torch.set_num_threads(min(16, host_cores()))
    try:
        t0 = time.perf_counter()
        qp, _ = OM.quantize_params(p_cpu, 8, impl="c")
        del p_cpu
        want, margins, gaps, oracle_last = OM.generate_greedy(qp, OM.GPT2_XL, prompt_cpu, check_steps, detail=True)
        del qp
    finally:
        torch.set_num_threads(threads)
    agree = greedy_agreement(got, want, gaps, gpu_last, oracle_last, T0)
    res["tokens_match_oracle"] = agree["tokens_match"]
    res["oracle_check"] = {**agree, "oracle_s": time.perf_counter() - t0}
    return res


def schemes_section(dev):
    """The reference experiment's table (run_quantization.py:31-158) on seed-0
    GPT-2 small over synthetic tokens: fp32 baseline and the five schemes,
    perplexity over 8 chunks x 2 batches x 4 windows of 128 tokens, paired
    per-chunk loss deltas, quantize_model's size statistics, and speed = greedy
    decode (64-token prompt, 16 new tokens) through the captured decoder."""
    import torch

    import gpt2_harness_amd as g

    torch.manual_seed(0)
    model = g.GPT(g.GPTConfig()).to(dev).eval()
    ds = g.SyntheticTokenStream(50257, 8 * 2 * 4 * 128 + 1, 128, seed=0)
    table = g.run_quantization_table(model, ds, device=dev)
    del model
    keep = ("label", "packed_bytes", "compression_ratio", "highlight")
    rows = [{**{k: r[k] for k in keep if k in r}, "ppl": r["quality"]["ppl_of_mean_loss"],
             "paired_dloss": r["quality"]["paired_loss_delta"]["mean"],
             "paired_dloss_stderr": r["quality"]["paired_loss_delta"]["stderr"],
             "tokens_per_s": r["speed"]["tokens_per_s"]} for r in table["rows"]]
    b = table["baseline"]
    return {"baseline": {"ppl": b["ppl_of_mean_loss"], "bytes": b["bytes"], "tokens_per_s": b["speed"]["tokens_per_s"]},
            "rows": rows, "data": "synthetic uniform tokens (seed 0); random-init weights"}


def cpu_baseline(budget_s: float = 10.0):
    """The oracle's dequantize-then-fp32-matmul over the GEMV workload on the host."""
    import torch

    from oracle import linear as OL
    from oracle import quant as OQ

    cores = host_cores()
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(0)
    layers = []
    for _ in range(12):
        for K, N in SMALL_KN:
            w = (torch.randn(N, K, generator=gen) * 0.02).numpy()
            q, s = OQ.quantize_tensor(w, 8)
            layers.append((K, N, OL.dequantize(q, s)))
    xs = {K: torch.randn(1, K, generator=gen).to(torch.bfloat16) for K, _ in SMALL_KN}
    step_bytes = sum(gemv_bytes(1, K, N) for K, N, _ in layers)

    def step():
        for K, _N, w_hat in layers:
            OL.linear_ref(xs[K], w_hat)

    step()
    ts = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(ts) < 3:
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    med = statistics.median(ts)
    return {"value": step_bytes / med / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(ts)} steps of the same 48-Linear M=1 GEMV workload, oracle F.linear(x.float(), "
                      f"q.float()*scale) in fp32 on {cores} host threads; GB/s counts the same int8 "
                      f"algorithmic bytes as the GPU value (the CPU path reads 4-byte fp32 W_hat)",
            "ms_per_step": med * 1e3}


def cpu_configs():
    """The oracle (the reference's CPU quantized path restated) on bounded
    samples of the other configurations, on the same host threads."""
    import numpy as np
    import torch

    from oracle import linear as OL
    from oracle import model as OM
    from oracle import quant as OQ

    torch.set_num_threads(host_cores())
    out = {}

    def med(fn, reps=3):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    # GPT-2 small int8 greedy, batch 1, 64-token prompt
    p, _ = OM.quantize_params(OM.init_params(OM.GPT2_SMALL, 0), 8)
    idx = OM.benchmark_prompt(OM.GPT2_SMALL.vocab_size, 1, 64)
    new = 16
    t0 = time.perf_counter()
    OM.generate_greedy(p, OM.GPT2_SMALL, idx, new)
    dt = time.perf_counter() - t0
    out["gpt2_small_int8_greedy"] = {"tokens_per_s": new / dt, "sample": f"seed-0 GPT-2 small int8, prompt 64, "
                                     f"{new} new tokens (prefill included, as benchmark_generation counts)"}
    del p

    # quantize, GPT-2-XL shapes with 0.1% outliers x20
    gen = np.random.default_rng(0)
    q_res = {}
    for K, N in XL_KN:
        w = (gen.standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float32)
        flat = w.reshape(-1)
        pick = gen.choice(flat.size, flat.size // 1000, replace=False)
        flat[pick] *= 20
        t8 = med(lambda: OQ.quantize_tensor(w, 8), reps=1)
        t4 = med(lambda: OQ.quantize_groupwise_int4(w, 128), reps=1)
        q_res[f"int8_per_channel_{K}x{N}"] = {"GB/s": (5 * N * K + 4 * N) / t8 / 1e9}
        q_res[f"int4_g128_{K}x{N}"] = {"GB/s": (4 * N * K + N * K // 2 + 2 * N * -(-K // 128)) / t4 / 1e9}
    out["quantize_xl"] = q_res

    # prefill F.linear on W_hat, GPT-2-XL shapes
    g = torch.Generator().manual_seed(0)
    lin = {}
    w_hats = {}
    for K, N in XL_KN:
        q, s = OQ.quantize_tensor((torch.randn(N, K, generator=g) * 0.02).numpy(), 8)
        w_hats[(K, N)] = OL.dequantize(q, s)
    for M in (256, 1024):
        for K, N in XL_KN:
            x = torch.randn(M, K, generator=g).to(torch.bfloat16)
            t = med(lambda: OL.linear_ref(x, w_hats[(K, N)]), reps=2)
            lin[f"M{M}_{K}x{N}"] = {"TFLOP/s": 2 * M * N * K / t / 1e12}
    out["gemm_xl"] = lin
    del w_hats

    # GPT-2-XL batch 32: a 2-layer model at XL width, decode steps timed and the
    # per-layer part extrapolated to 48 layers (the head measured on its own)
    cfg2 = OM.Shape(n_layer=2, n_head=25, n_embd=1600)
    p2, _ = OM.quantize_params(OM.init_params(cfg2, 0), 8)
    B, T0, steps = 32, 128, 3
    idx = torch.randint(0, cfg2.vocab_size, (B, T0), generator=g)
    cache = OM.Cache(cfg2.n_layer)
    OM.forward(p2, cfg2, idx, cache)
    tok = idx[:, -1:]
    ts = []
    for _ in range(steps):
        t0 = time.perf_counter()
        logits = OM.forward(p2, cfg2, tok, cache)
        ts.append(time.perf_counter() - t0)
        tok = logits[:, -1:, :].argmax(-1)
    xh = torch.randn(B, 1600, generator=g)
    t_head = med(lambda: torch.nn.functional.linear(xh, p2["wte.weight"]), reps=3)
    t_layer = max(statistics.median(ts) - t_head, 0.0) / cfg2.n_layer
    t_step = 48 * t_layer + t_head
    out["gpt2_xl_int8_b32_decode"] = {"tokens_per_s": B / t_step, "ms_per_step": t_step * 1e3,
                                      "sample": f"extrapolated: {steps} decode steps of a 2-layer GPT-2-XL-width "
                                                f"model (seed 0, int8) at batch {B} after a {T0}-token prefill; "
                                                f"48 x the per-layer time plus the fp32 head"}
    return out


def sig(x, n: int = 4):
    """x with every float rounded to n significant digits (dicts and lists
    recursively), for a JSON line short enough to be kept whole."""
    import math

    if isinstance(x, float):
        return x if x == 0.0 or not math.isfinite(x) else float(f"{x:.{n}g}")
    if isinstance(x, dict):
        return {k: sig(v, n) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return [sig(v, n) for v in x]
    return x


def compact_detail(d: dict) -> dict:
    """The detail sections in tabular form: per-shape figures as lists in the
    order of ``shapes`` (K x N), derived fields (fractions of a stated peak,
    times implied by a rate) left out."""
    out: dict = {"shapes": {"small": [f"{K}x{N}" for K, N in SMALL_KN], "xl": [f"{K}x{N}" for K, N in XL_KN]}}
    gemm: dict = {}
    for key, v in d.items():
        if key.startswith("gemv_"):
            c = {"GB/s": v["GB/s"], "us_per_launch": v["avg_launch_us"]}
            if "per_shape_graph" in v:
                c["shape_us"] = [e["us"] for e in v["per_shape_graph"].values()]
            for k in ("launch_model_us", "frac_of_launch_model", "kernel_us", "kernel_GB/s", "stamped"):
                if k in v:
                    c[k] = v[k]
            out[key] = c
        elif key.startswith("gemm_xl"):
            per = v["per_shape"]
            gemm[key[len("gemm_xl_"):]] = {"TFLOP/s": [e["TFLOP/s"] for e in per.values()],
                                           "platform_bf16_TFLOP/s": [e["library_bf16_TFLOP/s"] for e in per.values()]}
            if all("stamped" in e for e in per.values()):
                gemm[key[len("gemm_xl_"):]]["kernel_us"] = [e["stamped"]["kernel_us"] for e in per.values()]
                gemm[key[len("gemm_xl_"):]]["launch_us"] = [e["us"] for e in per.values()]
        elif key == "quantize_xl":
            out[key] = {f"{lab}_GB/s": [v[f"{lab}_{K}x{N}"]["GB/s"] for K, N in XL_KN]
                        for lab in ("int8_per_channel", "int4_g128")}
        elif key == "cpu_oracle":
            c = {"gpt2_small_int8_greedy_tok/s": v["gpt2_small_int8_greedy"]["tokens_per_s"],
                 "gpt2_xl_int8_b32_tok/s": v["gpt2_xl_int8_b32_decode"]["tokens_per_s"]}
            for lab in ("int8_per_channel", "int4_g128"):
                c[f"quantize_{lab}_GB/s"] = [v["quantize_xl"][f"{lab}_{K}x{N}"]["GB/s"] for K, N in XL_KN]
            for M in (256, 1024):
                c[f"linear_M{M}_TFLOP/s"] = [v["gemm_xl"][f"M{M}_{K}x{N}"]["TFLOP/s"] for K, N in XL_KN]
            out[key] = c
        elif key == "schemes_gpt2_small":
            out[key] = {"baseline": v["baseline"],
                        "rows": [[r["label"], r["packed_bytes"], r["ppl"], r["paired_dloss"], r["paired_dloss_stderr"],
                                  r["tokens_per_s"]] for r in v["rows"]],
                        "row_fields": ["label", "packed_bytes", "ppl", "paired_dloss", "paired_dloss_stderr",
                                       "tokens_per_s"]}
        elif key == "decode_gpt2_xl_int8_b32":
            c = {k: v[k] for k in ("prefill_ms", "decode_ms_per_step", "tokens_per_s", "decode_tokens_per_s",
                                   "tokens_match_oracle", "oracle_check") if k in v}
            c["linear_M32_cold_us"] = [e["us"] for e in v["decode_linear_M32_cold"].values()]
            c["linear_M32_cold_GB/s"] = [e["GB/s"] for e in v["decode_linear_M32_cold"].values()]
            c["lm_head_fp32_M32_us"] = {k: e["us"] for k, e in v["lm_head_fp32_M32"].items()}
            out[key] = c
        elif key == "decode_gpt2_small_int8":
            out[key] = {k: ({kk: vv for kk, vv in e.items() if kk != "ms_per_token"} if isinstance(e, dict) else e)
                        for k, e in v.items() if k not in ("model", "prompt", "new_tokens")}
        elif key == "eval_gpt2_small_int8":
            out[key] = {"packed_bytes": v["packed_checkpoint"]["bytes"],
                        "load_packed_s": v["packed_checkpoint"]["load_packed_s"],
                        "ppl_tokens_per_s": v["perplexity"]["tokens_per_s"], "loss_mean": v["perplexity"]["loss_mean"]}
        elif key == "launch_floor":
            out[key] = {k: e["us_per_launch"] for k, e in v.items()}
        else:
            out[key] = v
    if gemm:
        out["gemm_xl"] = gemm
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline only (no detail sections, no CPU baseline)")
    ap.add_argument("--full-detail", default=None, metavar="PATH",
                    help="also write the uncompacted result line (every field of every section) to PATH")
    ap.add_argument("--only", choices=["headline", "gemv", "gemv_xl", "gemm", "gemm4096", "gemm_g128", "quantize", "decode", "decode_xl", "decode_lin", "eval", "schemes", "copy", "floor"],
                    default=None,
                    help="run one section alone (for profiling); 'copy' runs a plain 256 MiB device copy "
                         "used to calibrate the HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the benchmark runs the path on a single GPU)", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")

    if args.only == "copy":
        src = torch.randn(64 << 20, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "launches": 5}))
        return 0
    if args.only == "floor":
        print(json.dumps(launch_floor_section(dev)))
        return 0
    if args.only == "headline":  # the timed headline replays alone (what its kernel profile covers)
        h = gemv_section(1, SMALL_KN, 12, 6, args.steps, args.warmup, dev, seed=0, per_shape=False, stamped=True)
        print(json.dumps(h))
        return 0
    if args.only == "gemv_xl":  # the GPT-2-XL-shape replays alone (what their kernel profile covers)
        print(json.dumps(gemv_section(1, XL_KN, 12, 3, args.steps, args.warmup, dev, seed=7, per_shape=False,
                                      stamped=True)))
        return 0
    if args.only == "gemm":
        print(json.dumps({f"M{M}": gemm_section(M, XL_KN, dev) for M in (256, 1024, 4096)}))
        return 0
    if args.only == "gemm4096":
        print(json.dumps({"int8": gemm_section(4096, XL_KN, dev, stamped=True),
                          "int4": gemm_section(4096, XL_KN, dev, fmt="int4"),
                          "int4_g128": gemm_section(4096, XL_KN, dev, fmt="int4_g128"),
                          "platform_bf16_gemm": mfma_platform_section(dev)}))
        return 0
    if args.only == "gemm_g128":
        print(json.dumps({f"M{M}": gemm_section(M, XL_KN, dev, fmt="int4_g128") for M in (256, 1024, 4096)}))
        return 0
    if args.only == "quantize":
        print(json.dumps(quantize_section(dev)))
        return 0
    if args.only == "decode":
        print(json.dumps(decode_section(dev)))
        return 0
    if args.only == "decode_xl":
        print(json.dumps(decode_xl_section(dev)))
        return 0
    if args.only == "decode_lin":  # the batched decode Linears alone, for counter runs
        print(json.dumps(decode_linears_section(dev)))
        return 0
    if args.only == "eval":
        print(json.dumps(eval_section(dev)))
        return 0
    if args.only == "schemes":
        print(json.dumps(schemes_section(dev)))
        return 0

    head = gemv_section(1, SMALL_KN, 12, 6, args.steps, args.warmup, dev, seed=0, stamped=True)
    print(f"# headline gemv M=1: {head['GB/s']:.1f} GB/s, {head['ms_per_step']:.4f} ms/step", file=sys.stderr,
          flush=True)
    detail: dict = {}
    cpu = None
    if not args.quick and args.only in (None, "gemv"):
        for M in (4, 16):
            detail[f"gemv_small_M{M}"] = gemv_section(M, SMALL_KN, 12, 6, max(10, args.steps // 2), 2, dev, seed=M)
        detail["gemv_xl_M1"] = gemv_section(1, XL_KN, 12, 3, 10, 2, dev, seed=7, stamped=True)
        print("# gemv detail done", file=sys.stderr, flush=True)
    hbm = hbm_stream_section(dev)
    floor = launch_floor_section(dev)
    if not args.quick and args.only is None:
        for M in (256, 1024, 4096):
            detail[f"gemm_xl_M{M}"] = gemm_section(M, XL_KN, dev, stamped=M == 4096)
        for M in (256, 1024, 4096):
            detail[f"gemm_xl_g128_M{M}"] = gemm_section(M, XL_KN, dev, fmt="int4_g128")
        detail["gemm_xl_int4_M4096"] = gemm_section(4096, XL_KN, dev, fmt="int4")
        detail["platform_bf16_gemm"] = mfma_platform_section(dev)
        print("# gemm done", file=sys.stderr, flush=True)
        detail["quantize_xl"] = quantize_section(dev)
        detail["decode_gpt2_small_int8"] = decode_section(dev)
        print("# decode done", file=sys.stderr, flush=True)
        detail["decode_gpt2_xl_int8_b32"] = decode_xl_section(dev)
        print("# xl decode done", file=sys.stderr, flush=True)
        detail["eval_gpt2_small_int8"] = eval_section(dev)
        detail["schemes_gpt2_small"] = schemes_section(dev)
        print("# eval done", file=sys.stderr, flush=True)
        cpu = cpu_baseline()
        detail["cpu_oracle"] = cpu_configs()
        print("# cpu oracle done", file=sys.stderr, flush=True)

    traffic = None
    tfile = ROOT / "profiles" / "gemv_w8a16_gpt2small_m1.traffic.json"
    if tfile.exists():
        from gpt2_harness_amd import _lib

        t = json.loads(tfile.read_text())
        if t.get("tiq_version") == _lib.lib().tiq_version():
            traffic = t["traffic_bytes_per_launch"]
    launch_model_us = (floor["tiq_linear_w8_64x64_M1"]["us_per_launch"]
                       + head["bytes_per_step"] / head["launches_per_step"] / (hbm["copy"]["GB/s"] * 1e3))
    if "gemv_xl_M1" in detail:
        xl = detail["gemv_xl_M1"]
        xl_model = (floor["tiq_linear_w8_64x64_M1"]["us_per_launch"]
                    + xl["bytes_per_step"] / xl["launches_per_step"] / (hbm["copy"]["GB/s"] * 1e3))
        xl["launch_model_us"] = xl_model
        xl["frac_of_launch_model"] = xl_model / xl["avg_launch_us"]
    bytes_per_launch = head["bytes_per_step"] / head["launches_per_step"]
    # the kernel's own duration inside the timed replays (stamped copy,
    # first-workgroup entry to last-workgroup exit, mean over the launches of
    # the last replay of each graph); the launch time (step / launches, gaps
    # between kernels included) beside it
    kernel_us = head["kernel_us"]
    achieved = bytes_per_launch / (kernel_us * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": head["GB/s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights quantized int8 per-channel, N(0,1) bf16 activations)",
        "config": {
            "workload": "W8A16 decode GEMV over the 48 quantized Linears of GPT-2 small "
                        "(12 x K x N in 768x2304, 768x768, 768x3072, 3072x768), M=1, "
                        "weights rotated over 6 copies (510 MB) per step",
            "M": 1, "layers": 12, "weight_copies": 6,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": "gemv_direct_kernel (tiq_linear_w8, M=1)",
            "bytes_per_launch": bytes_per_launch,
            "kernel_us": kernel_us,
            "kernel_time": "in-kernel real-time stamps inside the timed graph replays (first entry to last exit)",
            "avg_launch_us": head["avg_launch_us"],
            "launch_GB/s": bytes_per_launch / (head["avg_launch_us"] * 1e-6) / 1e9,
            "measured_hbm_GBs": {k: v["GB/s"] for k, v in hbm.items()},
            "frac_of_measured_copy": achieved / hbm["copy"]["GB/s"],
            "graph_launch_floor_us": {k: v["us_per_launch"] for k, v in floor.items()},
            # what one launch of this size could cost at best: the library's
            # own minimal GEMV launch in a graph plus the bytes at the measured
            # copy rate; frac_of_launch_model = that / the measured launch
            "launch_model_us": launch_model_us,
            "frac_of_launch_model": launch_model_us / head["avg_launch_us"],
        },
        "cpu_baseline": cpu,
        "detail": {"gemv_small_M1": head, "hbm_measured": hbm, "launch_floor": floor, **detail},
    }
    if args.full_detail:
        Path(args.full_detail).write_text(json.dumps(line) + "\n")
    line["roofline"] = {k: v for k, v in line["roofline"].items() if k not in ("graph_launch_floor_us",)}
    if cpu is not None:
        line["cpu_baseline"] = {**cpu, "sample": "48-Linear M=1 GEMV steps, oracle fp32 F.linear on W_hat, "
                                                 "int8 algorithmic bytes counted"}
    line["detail"] = compact_detail(line["detail"])
    out = json.dumps(sig(line), separators=(",", ":"))
    print(f"# result line: {len(out)} bytes", file=sys.stderr, flush=True)
    print(out)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
