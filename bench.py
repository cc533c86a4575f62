"""Benchmark of the joyomni_ops hot path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W] [--only C1,C0,...]`

A "step" is one call of an op over one batch of synthetic input. The headline
workload (`value`) is benchmark config C1: per-token FP8 e4m3 quantization of a
bf16 [10530, 3072] activation. Every other benchmark config is timed the same
way and reported under "ops", as are the next-row workloads N3 (the gated
residual + LayerNorm + AdaLN with the per-token FP8 epilogue, C2 shape) and
N4 (the graph runner's 40-layer KV-pool commit at the deployment shape), and
the FP8 GEMMs G1-G6 (fp8_scaled_mm at Fp8Linear's deployment shapes: the
image stream's G1-G4, the text stream's G5-G6 at 256 prompt tokens), whose
lines add TFLOP/s against the 5.0 PFLOP/s dense fp8 matrix-core peak and the
time of torch._scaled_mm (hipBLASLt) on the same operands (both launched
eagerly in alternating blocks over the same rotating operand sets:
ab_eager_us_per_call, hipblaslt_us_per_call, hipblaslt_over_ours). R_* are the
reference-signature ops at the DiT block's deployment shapes (hidden 4096,
32 heads, 3120 tokens): table-mode QK norm + RoPE, LayerNorm with per-row
modulation, per-token quant of [3120, 4096] and [3120, 16384], and the
pre-RoPE K RMSNorm over [99840, 128] — on a contiguous copy (R_rms, the
reference caller's layout) and read straight from the packed qkv (R_kn, whose
line adds the time of the caller's copy-then-norm path), and the
K-cache-before-RoPE branch in one pass (R_qks: QK norm + RoPE in place on the
packed qkv plus the pre-RoPE K stage; its line adds the time of the two calls
the reference makes). T_* are the shapes of
the reference's own benchmark script (test_bench.py): rmsnorm and LayerNorm +
modulation at [4096, 4096], table-mode QK at [1, 1560, 32, 128], the FP8 GEMM
at 4096^3. R_gq is the MLP activation gelu(h, approximate="tanh") fused with the
down-projection's per-token FP8 quantization at [3120, 16384]; its line adds
the time of the two calls the reference makes (torch's GELU, then the quant).
B_img is the image stream of one DiT block at the deployment shape
(FP8 mode, attention output a fixed input) composed from the drop-in ops with
the reference's caller glue and through the fused callers: per-block time of
both (`reference_composition_us_per_call`, `us_per_call`).

Timing: max(W, 20) eager warmup calls, K eager calls (eager_us_per_call),
then max(K, 100) calls captured into one HIP graph. Five times: the graph is
replayed untimed and, enqueued right behind it (the GPU kept busy), replayed
again between HIP events recorded on the replay stream (the stream the kernels
run on). Per-call time = the median over the five timed replays of elapsed /
calls (min and max beside it), so that at least 500 calls are timed whatever
K is (`timed_calls` in each line). Each config's stream ceilings (S_*) are
timed right after it. The calls rotate over >= 4
input/output buffer sets totalling > 640 MB so the 256 MB Infinity Cache
cannot hold the working set. Inputs are resident in HBM before the timed
region. achieved GB/s = algorithmic bytes (compulsory reads + writes,
joyomni_ops.workloads.algorithmic_bytes) / per-call time.

S_* lines are bare row streams (csrc/bench/stream_ceiling.hip, built into
libjoyomni_stream.so, not part of the op library): for a config they move the
same bytes in the same launch shape as its kernel (workgroups, lanes per row,
16-byte chunks per lane, nontemporal accesses, scales) with no arithmetic
beyond the whole-row dependency every row kernel has. Their time is the
ceiling of that access shape on this GPU; the config's line carries
`stream_ceiling_us` and `frac_of_stream_ceiling` (ceiling time / kernel
time). Alternative shapes of the same bytes (S_*@LPRxCH) show whether another
launch shape would stream faster.

cpu_baseline: the CPU oracle's restatement of the reference formula of every
benchmark config (C0-C4), timed on the host's cores with the same inputs:
3 warmups, then at least 10 timed calls (more while under ~2 s), median
(`cpu_us_per_call` in each config's line; the headline one in cpu_baseline).

Prints ONE compact JSON line on stdout (under 4 KB: the headline with its
roofline and CPU baseline, and per line only us/call, roofline fraction,
stream ceiling and CPU time); progress and each line's full record go to
stderr, and the full record of the run to --detail (gpurun_out/bench_detail.json).
"""
from __future__ import annotations

import argparse
import collections
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "joyai-video-edit_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "µs/call + achieved HBM GB/s (% of ~8 TB/s) per op at 720p 3-frame chunk"
PEAK_GBPS = 8000.0
PEAK_FP8_TFLOPS = 5000.0
HEADLINE = "C1"
HEADLINE_KERNEL = "quant_rows_kernel<BF16, 64, 6, false>"
ROT_BYTES = 640e6


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def tensor_bytes(d: dict) -> int:
    return sum(t.numel() * t.element_size() for t in d.values())


def copy_probe(mb: int, steps: int, dev) -> dict:
    """Plain device copy of `mb` MiB (torch copy_), the calibration kernel for
    the FETCH_SIZE / WRITE_SIZE counters: it moves a known mb MiB each way."""
    import torch
    n = mb << 20
    sets = [(torch.empty(n, dtype=torch.uint8, device=dev), torch.empty(n, dtype=torch.uint8, device=dev))
            for _ in range(max(2, math.ceil(ROT_BYTES / (2 * n))))]
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        sets[i % len(sets)][1].copy_(sets[i % len(sets)][0])
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / steps
    return {"bytes_each_way": n, "us_per_call": round(us, 3), "gbps": round(2 * n / (us * 1e-6) / 1e9, 1)}


MIN_TIMED = 100   # calls per timed graph replay, whatever --steps is
TIMED_REPLAYS = 5  # timed replays per line; the line reports their median
MIN_WARMUP = 20   # eager warmup calls per line, whatever --warmup is


def time_launches(launch, n_sets: int, steps: int, warmup: int, dev,
                  use_graph: bool = True) -> dict:
    """Times launch(i, stream_handle) (call i uses buffer set i % n_sets).

    max(warmup, MIN_WARMUP) eager warmups; `steps` eager launches timed for
    eager_us_per_call; then max(steps, MIN_TIMED) launches captured into one
    HIP graph, replayed once untimed and once between HIP events on the replay
    stream. (One long graph rather than a short one replayed several times:
    the residual + LayerNorm kernels measured 1.5-2 us per call slower as 20-call
    graphs replayed five times than as one 100-call graph.)"""
    import torch
    warmup = max(warmup, MIN_WARMUP)
    stream = torch.cuda.Stream(dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for i in range(warmup):
            launch(i, stream.cuda_stream)
    torch.cuda.synchronize()

    # eager back-to-back launches (host launch path included)
    with torch.cuda.stream(stream):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            launch(i, stream.cuda_stream)
        e1.record(stream)
    torch.cuda.synchronize()
    eager_us = e0.elapsed_time(e1) * 1000.0 / steps
    if not use_graph:
        return {"us_per_call": eager_us, "eager_us_per_call": eager_us, "timed_calls": steps,
                "warmup_calls": warmup, "timing": "eager"}

    calls = max(steps, MIN_TIMED)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        h = torch.cuda.current_stream().cuda_stream
        for i in range(calls):
            launch(i, h)
    graph.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream(dev)
    per_call = []
    for _ in range(TIMED_REPLAYS):
        # An untimed replay is enqueued right before each timed one, so that the
        # timed calls run on a GPU that is already busy (steady state) rather
        # than one that has just idled through the host's synchronization.
        graph.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        graph.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        per_call.append(e0.elapsed_time(e1) * 1000.0 / calls)
    del graph
    return {"us_per_call": statistics.median(per_call), "eager_us_per_call": eager_us,
            "min_us_per_call": min(per_call), "max_us_per_call": max(per_call),
            "timed_calls": calls * TIMED_REPLAYS, "warmup_calls": warmup, "timing": "hip-graph"}


def _finish(res: dict, alg: int, n_sets: int, set_bytes: int) -> dict:
    us = res["us_per_call"]
    gbps = alg / (us * 1e-6) / 1e9
    out = {"us_per_call": round(us, 3), "eager_us_per_call": round(res["eager_us_per_call"], 3),
           "min_us_per_call": round(res.get("min_us_per_call", us), 3),
           "max_us_per_call": round(res.get("max_us_per_call", us), 3),
           "gbps": round(gbps, 1), "frac_of_peak": round(gbps / PEAK_GBPS, 4),
           "algorithmic_bytes": alg, "buffer_sets": n_sets,
           "rotated_mb": round(n_sets * set_bytes / 1e6, 1),
           "timed_calls": res["timed_calls"], "warmup_calls": res["warmup_calls"],
           "timing": res["timing"]}
    return out


def time_gpu(cfg, steps: int, warmup: int, dev, use_graph: bool = True) -> dict:
    import torch

    import joyomni_ops as jo
    from joyomni_ops import workloads as W

    host = W.make_inputs(cfg)
    set_bytes = tensor_bytes(host) + tensor_bytes(W.alloc_outputs(cfg, host))
    n_sets = max(4, math.ceil(ROT_BYTES / set_bytes))
    sets = []
    for _ in range(n_sets):
        t = {k: v.to(dev) for k, v in host.items()}
        t.update(W.alloc_outputs(cfg, t))
        sets.append(t)
    freqs = None
    if cfg.op in ("qk_grid", "qk_kvcache"):
        d = cfg.dims
        freqs = jo.rope_freqs(d["D"], d["rope_dims"], d["theta"])
    res = time_launches(lambda i, h: W.launch(cfg, sets[i % n_sets], h, freqs), n_sets, steps,
                        warmup, dev, use_graph)
    del sets
    torch.cuda.empty_cache()
    return _finish(res, W.algorithmic_bytes(cfg), n_sets, set_bytes)


# ---------------------------------------------------------------------------
# Stream ceilings. Each entry: the config it bounds, rows, lanes per row,
# chunks per lane, input streams, output streams, bytes stored per 16 read,
# fp32 scalars per row, in place, row-invariant inputs (the weight or
# modulation rows a kernel reads, through the cache, for every row), for input
# rows that come in groups (per-head rows of a strided view) the rows per
# group, the bytes between groups and the offset of the first row, and an
# extra output of 8 bytes per 16 read (an fp8 row next to a bf16 one), and
# whether the 16-byte row stores are written through (wt, as the in-place QK
# kernels store their rows) and whether workgroups take their rows in the
# XCD-grouped order of the per-token quantizer (xcd). The entry named S_<cfg> is the kernel's own access shape; entries named
# S_<cfg>@<what> are other shapes of the same bytes (@LPRxCH) or the shape
# without the cached row reads (@no-weight, @no-mod) or without the stride
# (@contiguous).
# ---------------------------------------------------------------------------
Stream = collections.namedtuple(
    "Stream", "cfg rows lpr ch nin nout outb nscal inplace nconst group gstride goff out8 wt xcd",
    defaults=(0, 0, 0, 0, 0, False, False))

_S = Stream
STREAMS = {
    "S_C0": _S("C0", 3510 * 6, 64, 2, 1, 1, 16, 0, True, wt=True),
    "S_C0@64x1": _S("C0", 3510 * 12, 64, 1, 1, 1, 16, 0, True, wt=True),
    "S_C0@64x3": _S("C0", 3510 * 4, 64, 3, 1, 1, 16, 0, True, wt=True),
    "S_C1": _S("C1", 10530, 64, 6, 1, 1, 8, 1, False, xcd=True),
    "S_C1@128x3": _S("C1", 10530, 128, 3, 1, 1, 8, 1, False),
    "S_C2": _S("C2", 10530, 128, 3, 2, 2, 16, 0, False, 2),
    "S_C2@no-mod": _S("C2", 10530, 128, 3, 2, 2, 16, 0, False),
    "S_C2@64x6": _S("C2", 10530, 64, 6, 2, 2, 16, 0, False),
    "S_C3": _S("C3", 10530 * 4, 64, 3, 1, 1, 16, 0, True),
    # x and residual in; residual and the fp8 row out, one scale per row;
    # broadcast gate, scale and shift rows
    "S_N3": _S("N3", 10530, 128, 3, 2, 1, 16, 1, False, 3, out8=1),
    "S_C4_4725_tok": _S("C4_4725_tok", 4725, 64, 6, 1, 1, 8, 1, False, 1),
    "S_C4_4725_tok@no-weight": _S("C4_4725_tok", 4725, 64, 6, 1, 1, 8, 1, False),
    "S_C4_4725_tok@128x3": _S("C4_4725_tok", 4725, 128, 3, 1, 1, 8, 1, False),
    "S_C4_4725_blk": _S("C4_4725_blk", 4725, 64, 6, 1, 1, 8, 24, False, 1),
    "S_C4_4725_blk@no-weight": _S("C4_4725_blk", 4725, 64, 6, 1, 1, 8, 24, False),
    "S_C4_10530_tok": _S("C4_10530_tok", 10530, 64, 6, 1, 1, 8, 1, False, 1),
    "S_C4_10530_tok@no-weight": _S("C4_10530_tok", 10530, 64, 6, 1, 1, 8, 1, False),
    "S_C4_10530_tok@128x3": _S("C4_10530_tok", 10530, 128, 3, 1, 1, 8, 1, False, 1),
    "S_C4_10530_blk": _S("C4_10530_blk", 10530, 64, 6, 1, 1, 8, 24, False, 1),
    "S_C4_10530_blk@no-weight": _S("C4_10530_blk", 10530, 64, 6, 1, 1, 8, 24, False),
    "S_C4_10530_blk@128x3": _S("C4_10530_blk", 10530, 128, 3, 1, 1, 8, 24, False, 1),
    "S_R_q4k": _S("R_q4k", 3120, 128, 4, 1, 1, 8, 1, False),
    "S_R_q4k@64x8": _S("R_q4k", 3120, 64, 8, 1, 1, 8, 1, False),
    "S_R_q16k": _S("R_q16k", 3120, 256, 8, 1, 1, 8, 1, False),
    "S_R_gq": _S("R_gq", 3120, 256, 8, 1, 1, 8, 1, False),
    "S_R_rms": _S("R_rms", 99840, 16, 1, 1, 1, 16, 0, False, 1),
    "S_R_rms@no-weight": _S("R_rms", 99840, 16, 1, 1, 1, 16, 0, False),
    # K slice of the packed qkv [1, 3120, 3, 32, 128]: 32 head rows of 256 B
    # per token, tokens 24576 B apart, starting 8192 B into the buffer
    "S_R_kn": _S("R_kn", 99840, 16, 1, 1, 1, 16, 0, False, 1, 32, 24576, 8192),
    "S_R_kn@contiguous": _S("R_kn", 99840, 16, 1, 1, 1, 16, 0, False, 1),
    "S_R_ln": _S("R_ln", 3120, 256, 2, 3, 1, 16, 0, False),
    "S_R_ln@64x8": _S("R_ln", 3120, 64, 8, 3, 1, 16, 0, False),
    "S_R_qk": _S("R_qk", 3120 * 8, 64, 2, 1, 1, 16, 0, True, wt=True),
    # q and k rows in place, and for the k rows the pre-RoPE stage as well:
    # on average one row read, one and a half written.
    "S_R_qks": _S("R_qks", 3120 * 8, 64, 2, 1, 1, 16, 0, True, out8=1, wt=True),
    "S_T_rms": _S("T_rms", 4096, 64, 8, 1, 1, 16, 0, False, 1),
    "S_T_rms@no-weight": _S("T_rms", 4096, 64, 8, 1, 1, 16, 0, False),
    "S_T_ln": _S("T_ln", 4096, 256, 2, 3, 1, 16, 0, False),
    "S_T_qk": _S("T_qk", 1560 * 8, 64, 2, 1, 1, 16, 0, True, wt=True),
}

_STREAM_LIB = None


def stream_lib():
    global _STREAM_LIB
    if _STREAM_LIB is None:
        import ctypes
        path = ROOT / "joyai-video-edit_amd" / "joyomni_ops" / "libjoyomni_stream.so"
        lib = ctypes.CDLL(str(path))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.jo_stream_rows.argtypes = [P, P, P, I64, I, I, I, I, I, I, I, I, I64, I64, I, P]
        lib.jo_stream_rows.restype = I
        _STREAM_LIB = lib
    return _STREAM_LIB


def stream_bytes(spec) -> int:
    """Bytes a stream moves per call: its rows in and out, the per-row
    scalars, and each row-invariant input once (as the kernels' algorithmic
    bytes count their weight row)."""
    row_in, row_out = spec.lpr * spec.ch * 16, spec.lpr * spec.ch * spec.outb
    return (spec.rows * (spec.nin * row_in + spec.nout * row_out + spec.out8 * row_in // 2
                         + spec.nscal * 4) + spec.nconst * row_in)


def time_stream(spec, steps: int, warmup: int, dev) -> dict:
    import torch
    row_in = spec.lpr * spec.ch * 16
    if spec.group:
        rin = spec.goff + (spec.rows // spec.group) * spec.gstride
    else:
        rin = spec.rows * row_in
    rout = spec.rows * spec.lpr * spec.ch * spec.outb
    rout8 = spec.rows * row_in // 2
    set_bytes = (spec.nin * rin + (0 if spec.inplace else spec.nout * rout)
                 + spec.out8 * rout8 + spec.nconst * row_in + spec.rows * spec.nscal * 4)
    n_sets = max(4, math.ceil(ROT_BYTES / set_bytes))
    sets = []
    for _ in range(n_sets):
        ins = [torch.randint(0, 255, (rin,), dtype=torch.uint8, device=dev)
               for _ in range(spec.nin)]
        consts = [torch.randint(0, 255, (row_in,), dtype=torch.uint8, device=dev)
                  for _ in range(spec.nconst)]
        outs = ins[:1] if spec.inplace else [torch.empty(rout, dtype=torch.uint8, device=dev)
                                             for _ in range(spec.nout)]
        outs += [torch.empty(rout8, dtype=torch.uint8, device=dev) for _ in range(spec.out8)]
        scal = torch.empty(max(1, spec.rows * spec.nscal), dtype=torch.float32, device=dev)
        sets.append((ins, consts, outs, scal))
    lib = stream_lib()

    import ctypes
    ptrs = []
    for ins, consts, outs, _ in sets:
        p = [t.data_ptr() + spec.goff for t in ins] + [t.data_ptr() for t in consts]
        ptrs.append(((ctypes.c_void_p * 5)(*p), (ctypes.c_void_p * 3)(*[t.data_ptr() for t in outs])))

    def launch(i, h):
        scal = sets[i % n_sets][3]
        pin, pout = ptrs[i % n_sets]
        rc = lib.jo_stream_rows(pin, pout, scal.data_ptr() if spec.nscal else None, spec.rows,
                                spec.lpr, spec.ch, spec.nin, spec.nout, spec.outb, spec.nscal,
                                spec.nconst, spec.out8, spec.group, spec.gstride,
                                int(spec.wt) | (int(spec.xcd) << 1), h)
        if rc != 0:
            raise RuntimeError(f"jo_stream_rows failed ({rc}) for {spec}")

    res = time_launches(launch, n_sets, steps, warmup, dev)
    del sets
    torch.cuda.empty_cache()
    out = _finish(res, stream_bytes(spec), n_sets, set_bytes)
    shape = (f"{spec.rows} rows, {spec.lpr} lanes x {spec.ch} chunks, "
             f"{spec.nin} in / {spec.nout} out")
    if spec.out8:
        shape += f" + an 8-byte-per-16 output"
    if spec.nconst:
        shape += f", {spec.nconst} cached row(s) read per row"
    if spec.group:
        shape += f", rows in groups of {spec.group} every {spec.gstride} B"
    out.update(shape=shape, kind="stream-ceiling")
    return out


def gemm_vs_hipblaslt(cfg, dev, rounds: int = 7, calls: int = 20):
    """This build's GEMM and torch._scaled_mm (hipBLASLt; row-wise scales and
    bias) on the same operands, both launched eagerly, rotating over the same
    >= 640 MB of operand sets, in alternating blocks of `calls` timed launches
    (each after one untimed launch, so that the switch from the other
    library's kernel is not timed) so that clock and power drift reach both
    alike. Returns the medians over `rounds` blocks of (ours, hipBLASLt)
    per-call times, or None if this torch build cannot run torch._scaled_mm."""
    if cfg.op != "gemm":
        return None
    import torch
    from joyomni_ops import workloads as W
    d = cfg.dims
    host = W.make_inputs(cfg)
    set_bytes = tensor_bytes(host) + tensor_bytes(W.alloc_outputs(cfg, host))
    n_sets = max(4, math.ceil(ROT_BYTES / set_bytes))
    sets = []
    for _ in range(n_sets):
        t = {k: v.to(dev) for k, v in host.items()}
        t.update(W.alloc_outputs(cfg, t))
        sets.append(t)
    cur = torch.cuda.current_stream(dev)

    def ours(i):
        W.launch(cfg, sets[i % n_sets], cur.cuda_stream)

    def lib(i):
        t = sets[i % n_sets]
        torch._scaled_mm(t["a"].view(torch.float8_e4m3fn), t["w"].view(torch.float8_e4m3fn).t(),
                         scale_a=t["sa"].view(d["M"], 1), scale_b=t["sb"].view(1, d["N"]),
                         out_dtype=torch.bfloat16, bias=t["bias"])

    try:
        for i in range(3):
            lib(i)
        torch.cuda.synchronize()
    except Exception as ex:  # noqa: BLE001 - report, do not fail the bench
        log(f"torch._scaled_mm unavailable: {str(ex)[:120]}")
        return None

    def block(fn, first):
        fn(first + calls)  # untimed: the first launch after the other library's
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        for i in range(calls):
            fn(first + i)
        e1.record(cur)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / calls

    t_ours, t_lib = [], []
    for r in range(rounds):
        t_ours.append(block(ours, r * calls))
        t_lib.append(block(lib, r * calls))
    del sets
    torch.cuda.empty_cache()
    return round(statistics.median(t_ours), 2), round(statistics.median(t_lib), 2)


def torch_reference_us(cfg, dev, iters: int = 10):
    """Per-call time of the reference's own code path where that path is plain
    torch, run eagerly on the same GPU: N4 is StreamingGraphRunner.run_commit
    (graph_runner.py:137-142) over apply_rotary_emb (rope.py:14-28). None for
    configs whose reference is a CUDA kernel (not runnable here)."""
    if cfg.op != "kv_commit":
        return None
    import torch
    from joyomni_ops import workloads as W

    def rotate_half(x):
        x_real, x_imag = x.float().reshape(*x.shape[:-1], -1, 2).unbind(-1)
        return torch.stack([-x_imag, x_real], dim=-1).flatten(-2)

    def apply_rotary_emb(x, cos, sin):
        c = cos.view(1, x.shape[1], 1, x.shape[-1])
        s = sin.view(1, x.shape[1], 1, x.shape[-1])
        return (x.float() * c + rotate_half(x.float()) * s).type_as(x)

    d = cfg.dims
    t = {k: v.to(dev) for k, v in W.make_inputs(cfg).items()}
    seg = slice(d["off"], d["off"] + d["T"])

    def run_commit():
        for li in range(d["L"]):
            roped = apply_rotary_emb(t["stage_k"][li], t["cos"], t["sin"])
            t["pool_k"][li, :, seg].copy_(roped)
            t["pool_v"][li, :, seg].copy_(t["stage_v"][li])

    for _ in range(2):
        run_commit()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        run_commit()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / iters
    del t
    torch.cuda.empty_cache()
    return round(us, 1)


def copy_then_rmsnorm_us(cfg, dev, iters: int = 20):
    """R_kn's path as the reference caller takes it (sgl_fused_ops.py:102-111):
    .contiguous() of the K slice, then the rmsnorm kernel (this build's, the
    reference's CUDA kernel not being runnable here), eager, per call."""
    if cfg.op != "rms_heads":
        return None
    import torch

    import joyomni_ops as jo
    from joyomni_ops import workloads as W
    d = cfg.dims
    sets = [{k: v.to(dev) for k, v in W.make_inputs(cfg).items()} for _ in range(4)]

    def call(t):
        k = t["qkv"][:, :, 1].contiguous().reshape(-1, d["D"])
        return jo.rmsnorm(k, t["weight"], d["eps"])

    for i in range(4):
        call(sets[i])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(iters):
        call(sets[i % 4])
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / iters
    del sets
    torch.cuda.empty_cache()
    return round(us, 1)


def unfused_kstage_us(cfg, dev, iters: int = 20):
    """R_qks's branch as the reference caller takes it (dit.py:360-370 over
    sgl_fused_ops.py:57-111): rmsnorm_qk_bf16 of the K slice (this build's op,
    reading the slice in place), then fused_qk_norm_rope_3d with its
    .contiguous() copies of q and k and the paired op, eager, per call."""
    if cfg.op != "qk_kstage":
        return None
    import torch

    from joyomni_ops import dit_ops
    from joyomni_ops import workloads as W
    sets = [{k: v.to(dev) for k, v in W.make_inputs(cfg).items()} for _ in range(4)]

    def call(t):
        qkv = t["qkv"]
        kc = dit_ops.rmsnorm_qk_bf16(qkv[:, :, 1], t["k_weight"], eps=1e-6)
        q, k = dit_ops.fused_qk_norm_rope_3d(qkv[:, :, 0], qkv[:, :, 1], t["q_weight"],
                                             t["k_weight"], (t["cos"], t["sin"]), eps=1e-6)
        return q, k, kc

    for i in range(4):
        call(sets[i])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(iters):
        call(sets[i % 4])
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / iters
    del sets
    torch.cuda.empty_cache()
    return round(us, 1)


def unfused_gelu_quant_us(cfg, dev, iters: int = 20):
    """R_gq as two calls, the reference's order (dit.py:433 then fp8_linear.py:166):
    torch.nn.functional.gelu(h, approximate="tanh") then sgl_per_token_quant_fp8
    (this build's op) on its bf16 output, eager, per call."""
    if cfg.op != "gelu_quant":
        return None
    import torch

    import joyomni_ops as jo
    from joyomni_ops import workloads as W
    sets = []
    for _ in range(4):
        t = {k: v.to(dev) for k, v in W.make_inputs(cfg).items()}
        t.update(W.alloc_outputs(cfg, t))
        sets.append(t)

    def call(t):
        jo.sgl_per_token_quant_fp8(torch.nn.functional.gelu(t["x"], approximate="tanh"),
                                   t["q"], t["s"])

    for i in range(4):
        call(sets[i])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(iters):
        call(sets[i % 4])
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / iters
    del sets
    torch.cuda.empty_cache()
    return round(us, 1)


def time_block(steps: int, warmup: int, dev, calls: int = 20) -> dict:
    """B_img: the image stream of one DiT block at the deployment shape (FP8
    mode, attention output a fixed input), composed from the drop-in ops with
    the reference's caller glue (workloads.block_reference) and through the
    fused callers (workloads.block_fused). Each composition: max(warmup, 3)
    eager calls, then `calls` blocks captured into one HIP graph, replayed once
    untimed and then timed, five times, interleaved with the other
    composition's replays; per-block time = median replay / calls."""
    import torch
    from joyomni_ops import workloads as W
    b = W.make_block(dev)
    img_f = b["img"].clone()
    runs = {"reference": lambda: W.block_reference(b, b["img"]),
            "fused": lambda: W.block_fused(b, img_f)}
    stream = torch.cuda.Stream(dev)
    graphs = {}
    for name, fn in runs.items():
        with torch.cuda.stream(stream):
            for _ in range(max(warmup, 3)):
                fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(calls):
                fn()
        g.replay()
        torch.cuda.synchronize()
        graphs[name] = g
    cur = torch.cuda.current_stream(dev)
    per = {name: [] for name in graphs}
    for _ in range(TIMED_REPLAYS):
        for name, g in graphs.items():
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(cur)
            g.replay()
            e1.record(cur)
            torch.cuda.synchronize()
            per[name].append(e0.elapsed_time(e1) * 1000.0 / calls)
    del graphs
    torch.cuda.empty_cache()
    ref_us = statistics.median(per["reference"])
    fused_us = statistics.median(per["fused"])
    flops = W.block_flops()
    d = W.BLOCK
    return {"us_per_call": round(fused_us, 3), "reference_composition_us_per_call": round(ref_us, 3),
            "reference_over_fused": round(ref_us / fused_us, 3),
            "min_us_per_call": round(min(per["fused"]), 3),
            "max_us_per_call": round(max(per["fused"]), 3),
            "gemm_flops": flops, "block_tflops": round(flops / (fused_us * 1e-6) / 1e12, 1),
            "timed_calls": calls * TIMED_REPLAYS, "timing": "hip-graph",
            "shape": f"img [{d['B']}, {d['L']}, {d['D']}], {d['H']} heads x {d['Dh']}, "
                     f"MLP {d['F']}; attention output a fixed input"}


def cpu_fn(cfg):
    """The oracle's restatement of the reference formula for a config (CPU tensors)."""
    from oracle import ops
    d = cfg.dims
    if cfg.op == "quant":
        return lambda t: ops.per_token_quant_fp8(t["x"])
    if cfg.op == "rms_quant":
        # the reference's torch RMSNorm formula (test_parity_light.py:31-32),
        # then the per-token / per-block quantization rule
        return lambda t: ops.rmsnorm_quant_fp8(t["x"], t["weight"], d["eps"], d["group"],
                                               v=ops.rmsnorm_f32(t["x"], t["weight"], d["eps"]))
    if cfg.op == "add_ln":
        return lambda t: ops.add_layernorm_scale_shift(t["x"], t["residual"], None, None, None,
                                                       t["scale"], t["shift"], d["eps"])
    if cfg.op == "kv_commit":
        return lambda t: ops.commit_kv(t["pool_k"], t["pool_v"], t["stage_k"], t["stage_v"],
                                       d["off"], t["cos"], t["sin"])
    if cfg.op == "add_ln_quant":
        return lambda t: ops.norm_scale_shift_quant_fp8(t["x"], t["residual"], t["gate"], None,
                                                        None, t["scale"], t["shift"], 0, d["eps"])
    B, L, H, D = d["B"], d["L"], d["H"], d["D"]
    frames = L // (d["grid"][0] * d["grid"][1])
    cos, sin = ops.half_tables(*ops.rope_grid_tables(frames, *d["grid"], d["t0"], d["rope_dims"],
                                                     d["theta"]))

    def qk(t):
        q = ops.qk_norm_rope_f32(t["q"].reshape(B, L, H, D), t["q_weight"], cos, sin, d["eps"])
        k = ops.qk_norm_rope_f32(t["k"].reshape(B, L, H, D), t["k_weight"], cos, sin, d["eps"])
        return q.to(t["q"].dtype), k.to(t["k"].dtype)
    return qk


def cpu_threads() -> int:
    """Threads for the CPU baseline: every CPU this process may run on, capped
    by OMP_NUM_THREADS where the host sets it (the GPU boxes give a process a
    16-CPU share of a larger machine and say so there)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


BENCH_CONFIGS = ("C0", "C1", "C2", "C3", "C4_4725_tok", "C4_4725_blk", "C4_10530_tok",
                    "C4_10530_blk")


def time_cpu(cfg, warmup: int, iters: int, seconds: float = 0.0) -> dict:
    """Median CPU time per call: at least `iters` calls and at least `seconds`
    of timed CPU work (capped at 1000 calls)."""
    import torch

    from joyomni_ops import workloads as W
    t = W.make_inputs(cfg)
    fn = cpu_fn(cfg)
    for _ in range(warmup):
        fn(t)
    ts = []
    while len(ts) < iters or (sum(ts) < seconds and len(ts) < 1000):
        t0 = time.perf_counter()
        fn(t)
        ts.append(time.perf_counter() - t0)
    iters = len(ts)
    us = statistics.median(ts) * 1e6
    alg = W.algorithmic_bytes(cfg)
    return {"us_per_call": round(us, 1), "gbps": round(alg / (us * 1e-6) / 1e9, 2),
            "threads": torch.get_num_threads(), "iters": iters, "seconds": round(sum(ts), 1)}


def cpu_model() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def load_traffic(kernel_key: str):
    """HBM bytes per launch of the headline kernel from the committed PMC summary."""
    p = ROOT / "profiles" / "pmc_traffic.json"
    if not p.exists():
        return None
    try:
        data = json.loads(p.read_text())
        return data.get(kernel_key, {}).get("traffic_bytes")
    except (ValueError, OSError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default="", help="comma-separated config names (C*, S_*, ...)")
    ap.add_argument("--no-streams", action="store_true", help="skip the S_* stream ceilings")
    ap.add_argument("--no-compare", action="store_true",
                    help="skip the reference-path timings (hipBLASLt, the torch commit loop, "
                         "the reference callers' unfused calls), e.g. for profiler runs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-iters", type=int, default=10, help="minimum timed CPU calls per config")
    ap.add_argument("--cpu-seconds", type=float, default=2.0,
                    help="keep timing a config's CPU calls while under this many seconds")
    ap.add_argument("--no-graph", action="store_true",
                    help="time eager launches only (for profiler counter runs)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="also run a plain copy of this many MiB (counter calibration)")
    ap.add_argument("--detail", default=str(ROOT / "gpurun_out" / "bench_detail.json"),
                    help="file for the full per-line record ('' for none); stdout carries the "
                         "compact summary line only")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested). The ops are row-independent and shard by "
              "tokens with no communication; run --gpus 1.", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    import joyomni_ops  # noqa: F401  (fails loudly if the libraries are missing)
    from joyomni_ops import workloads as W

    dev = torch.device("cuda", 0)
    if args.only:
        names = [n for n in args.only.split(",") if n]
    else:
        names = []
        for c in W.CONFIGS:
            names.append(c)
            if not args.no_streams:
                names += [sn for sn, spec in STREAMS.items() if spec.cfg == c]
    if HEADLINE not in names:
        names.insert(0, HEADLINE)
    results = {}
    for n in names:
        if n == "B_img":
            continue
        if n in STREAMS:
            log(f"{n}: timing bare stream")
            results[n] = time_stream(STREAMS[n], args.steps, args.warmup, dev)
            log(f"{n}: {results[n]}")
            continue
        cfg = W.CONFIGS[n]
        log(f"{n}: timing {'eager' if args.no_graph else 'graph-replayed'} calls")
        results[n] = time_gpu(cfg, args.steps, args.warmup, dev, use_graph=not args.no_graph)
        ref_us = None if args.no_compare else torch_reference_us(cfg, dev)
        if ref_us is not None:
            results[n]["torch_reference_us_per_call"] = ref_us
        caller_us = None if args.no_compare else copy_then_rmsnorm_us(cfg, dev)
        if caller_us is not None:
            results[n]["copy_then_rmsnorm_us_per_call"] = caller_us
        two_call_us = None if args.no_compare else (unfused_kstage_us(cfg, dev)
                                                    or unfused_gelu_quant_us(cfg, dev))
        if two_call_us is not None:
            results[n]["unfused_two_calls_us_per_call"] = two_call_us
        flops = W.algorithmic_flops(cfg)
        if flops is not None:
            gemm_roofline(results[n], flops)
            ab = None if args.no_compare else gemm_vs_hipblaslt(cfg, dev)
            if ab is not None:
                results[n]["ab_eager_us_per_call"] = ab[0]
                results[n]["hipblaslt_us_per_call"] = ab[1]
                results[n]["hipblaslt_tflops"] = round(flops / (ab[1] * 1e-6) / 1e12, 1)
                results[n]["hipblaslt_over_ours"] = round(ab[1] / ab[0], 3)
        log(f"{n}: {results[n]}")

    if "B_img" in names or not args.only:
        log("B_img: timing the block compositions")
        results["B_img"] = time_block(args.steps, args.warmup, dev)
        log(f"B_img: {results['B_img']}")

    # Each config's stream ceiling: its kernel's own shape, and the fastest shape.
    for sname, spec in STREAMS.items():
        cname = spec.cfg
        if sname not in results or cname not in results:
            continue
        r, s_us = results[cname], results[sname]["us_per_call"]
        if "@" not in sname:
            r["stream_ceiling"] = sname
            r["stream_ceiling_us"] = s_us
            r["frac_of_stream_ceiling"] = round(s_us / r["us_per_call"], 4)
        if s_us < r.get("best_stream_us", float("inf")):
            r["best_stream"] = sname
            r["best_stream_us"] = s_us
            r["frac_of_best_stream"] = round(s_us / r["us_per_call"], 4)

    copy = None
    if args.copy_mb:
        copy = copy_probe(args.copy_mb, args.steps, dev)
        log(f"copy {args.copy_mb} MiB: {copy}")

    cpu = None
    if not args.no_cpu:
        threads = cpu_threads()
        torch.set_num_threads(threads)
        for n in BENCH_CONFIGS:
            if n not in results:
                continue
            log(f"cpu baseline {n}: oracle restatement on the full input, {threads} threads")
            c = time_cpu(W.CONFIGS[n], 3, args.cpu_iters, args.cpu_seconds)
            results[n].update(cpu_us_per_call=c["us_per_call"], cpu_gbps=c["gbps"],
                              cpu_iters=c["iters"], cpu_threads=c["threads"],
                              gpu_over_cpu=round(c["us_per_call"] / results[n]["us_per_call"], 1))
            log(f"cpu {n}: {c}")
            if n == HEADLINE:
                cpu = c

    detail_path = Path(args.detail) if args.detail else None
    line = summary_line(results, cpu, args.steps, args.warmup, cpu_model(),
                        detail_path.name if detail_path else None)
    if detail_path is not None:
        # The whole per-line record (every field of every config and stream
        # ceiling) goes to a file; stdout carries the compact line only.
        full = dict(line, ops=results)
        if copy is not None:
            full["copy_probe"] = copy
        try:
            detail_path.parent.mkdir(parents=True, exist_ok=True)
            detail_path.write_text(json.dumps(full, indent=1))
            log(f"full record written to {detail_path}")
        except OSError as ex:
            log(f"could not write {detail_path}: {ex}")
    for n, r in results.items():
        log(f"line {n}: {json.dumps(r)}")
    print(json.dumps(line, separators=(",", ":")), flush=True)
    return 0


SUMMARY_MAX_BYTES = 4096


def _r(v, nd):
    return None if v is None else round(v, nd)


def compact_entry(name: str, r: dict) -> dict:
    """The few figures of one line that the summary carries: per-call time,
    fraction of the roofline (HBM, or the fp8 matrix-core peak for GEMMs whose
    flops outlast their bytes; GEMMs also carry TFLOP/s), the
    stream ceiling of the line's own access shape and the CPU baseline."""
    if r.get("kind") == "stream-ceiling":
        return {"us": _r(r["us_per_call"], 2), "frac": _r(r.get("frac_of_peak"), 3)}
    if name == "B_img":
        return {"us": _r(r["us_per_call"], 1), "ref_us": _r(r.get("reference_composition_us_per_call"), 1)}
    e = {"us": _r(r["us_per_call"], 2)}
    if "tflops" in r:
        e["tflops"] = _r(r.get("tflops"), 0)
        if r.get("bound") == "mfma":
            e["frac"] = _r(r.get("frac_of_fp8_peak"), 3)
        else:
            e.update(bound="hbm", frac=_r(r.get("frac_of_peak"), 3))
        if "hipblaslt_over_ours" in r:
            e["blt_x"] = _r(r["hipblaslt_over_ours"], 3)
        return e
    e["frac"] = _r(r.get("frac_of_peak"), 3)
    if "stream_ceiling_us" in r:
        e["S_us"] = _r(r["stream_ceiling_us"], 2)
        e["fS"] = _r(r.get("frac_of_stream_ceiling"), 3)
    if "cpu_us_per_call" in r:
        e["cpu_us"] = _r(r["cpu_us_per_call"], 0)
    for k, short in (("torch_reference_us_per_call", "ref_us"),
                     ("unfused_two_calls_us_per_call", "ref_us"),
                     ("copy_then_rmsnorm_us_per_call", "ref_us")):
        if k in r:
            e[short] = _r(r[k], 1)
    return e


def gemm_roofline(r, flops):
    """A GEMM line's roofline is whichever ideal time is longer: the fp8
    matrix cores' for the image stream's shapes, HBM's for the text stream's few
    rows, where streaming the weight once outlasts the flops (256 x 12288 x
    4096: 446 flop per byte against the ridge's 625, 5.0 PFLOP/s over 8 TB/s).
    Both fractions stay in the record."""
    tf = flops / (r["us_per_call"] * 1e-6) / 1e12
    mfma = flops / (PEAK_FP8_TFLOPS * 1e12) >= r["algorithmic_bytes"] / (PEAK_GBPS * 1e9)
    if mfma:
        r.pop("frac_of_peak", None)
    r.update(bound="mfma" if mfma else "hbm", algorithmic_flops=flops, tflops=round(tf, 1),
             frac_of_fp8_peak=round(tf / PEAK_FP8_TFLOPS, 4))
    return r


def summary_line(results: dict, cpu, steps: int, warmup: int, host_cpu: str = "",
                 detail: str | None = None) -> dict:
    """The one JSON line bench.py prints: the headline (C1) with its roofline
    and CPU baseline, and a compact entry for every other line that ran (the
    C0-C4 configs under "configs", the rest under "ops"). It is kept under
    SUMMARY_MAX_BYTES so that a reader that keeps only the tail of stdout
    still gets it whole; the full record goes to the detail file."""
    from joyomni_ops import workloads as W
    h = results[HEADLINE]
    cfg = W.CONFIGS[HEADLINE]
    configs = {n: compact_entry(n, results[n]) for n in BENCH_CONFIGS if n in results}
    ops = {n: compact_entry(n, r) for n, r in results.items()
           if n not in configs and not n.startswith("S_")}
    line = {
        "metric": METRIC,
        "value": h["gbps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "timed_calls": h["timed_calls"],
        "warmup_calls": h["warmup_calls"],
        "ms_per_step": round(h["us_per_call"] / 1000.0, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) bf16 with 0.5% x40 outliers)",
        "config": {"workload": "C1: per-token FP8 e4m3 quant, x bf16 [10530, 3072] -> fp8 + fp32 scales",
                   "M": cfg.dims["M"], "K": cfg.dims["K"], "us_per_call": h["us_per_call"]},
        "roofline": {"bound": "hbm", "kernel": HEADLINE_KERNEL, "achieved": h["gbps"],
                     "peak": PEAK_GBPS, "unit": "GB/s", "frac": h["frac_of_peak"],
                     "traffic": load_traffic(HEADLINE_KERNEL),
                     "algorithmic_bytes": h["algorithmic_bytes"]},
        "cpu_baseline": None if cpu is None else {
            "value": cpu["gbps"], "unit": "GB/s", "us_per_call": cpu["us_per_call"],
            "cores": cpu["threads"], "kind": "port",
            "sample": f"oracle per_token_quant_fp8 (torch CPU), full C1 input, median of "
                      f"{cpu['iters']} calls ({cpu['seconds']:.1f} s) after 3 warmups; "
                      f"{host_cpu[:48]}"},
        "configs": configs,
        "ops": ops,
        "keys": "us=us/call, frac=of 8 TB/s (GEMM: of 5 PF fp8), S_us=stream ceiling of the "
                "line's shape, fS=S_us/us, cpu_us=CPU oracle, ref_us=reference path, "
                "blt_x=hipBLASLt time/ours",
    }
    if detail:
        line["detail"] = detail
    return line


if __name__ == "__main__":
    sys.exit(main())
