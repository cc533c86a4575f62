"""CPU tests of bench.py's measurement tables: every stream ceiling (S_*) line
names a real config, uses a launch shape that csrc/bench/stream_ceiling.hip
instantiates, and — for the line that stands for a kernel's own access shape —
moves the config's algorithmic bytes; the stream library loads and rejects bad
sizes without touching a GPU."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
STREAM_SRC = ROOT / "joyai-video-edit_amd" / "csrc" / "bench" / "stream_ceiling.hip"


@pytest.fixture(scope="module")
def bench():
    import bench as b
    return b


def instantiated_shapes() -> set[tuple[int, ...]]:
    """(lpr, ch, nin, nout, outb, nconst, out8) of every TRY(...) in the dispatch list."""
    shapes = set()
    for m in re.finditer(r"TRY\(([\d,\s]+)\)", STREAM_SRC.read_text()):
        v = [int(t) for t in m.group(1).split(",")]
        shapes.add(tuple(v + [0] * (7 - len(v))))
    return shapes


def test_stream_shapes_are_instantiated(bench):
    shapes = instantiated_shapes()
    assert shapes, "no TRY(...) lines found"
    for name, s in bench.STREAMS.items():
        key = (s.lpr, s.ch, s.nin, s.nout, s.outb, s.nconst, s.out8)
        assert key in shapes, f"{name}: shape {key} is not instantiated in {STREAM_SRC.name}"
        assert s.nin + s.nconst <= 5 and s.nout + s.out8 <= 3, name
        assert not (s.inplace and s.nout != 1), name


def test_streams_name_configs_and_one_own_shape(bench):
    from joyomni_ops import workloads as W
    own = {}
    for name, s in bench.STREAMS.items():
        assert s.cfg in W.CONFIGS, name
        assert name.startswith("S_" + s.cfg), name
        if "@" not in name:
            assert s.cfg not in own, f"{s.cfg} has two own-shape streams"
            own[s.cfg] = name
    for cfg in ("C0", "C1", "C2", "C3", "C4_4725_tok", "C4_4725_blk", "C4_10530_tok",
                "C4_10530_blk"):
        assert cfg in own, f"benchmark config {cfg} has no stream ceiling"


def test_own_shape_streams_move_the_config_bytes(bench):
    """The S_<cfg> line moves the config's algorithmic bytes: exactly for the
    row ops (rows, scales and the weight row once), within 1% where the kernel
    also reads small per-token tables (QK: rotation tables, weights)."""
    from joyomni_ops import workloads as W
    for name, s in bench.STREAMS.items():
        if "@" in name:
            continue
        alg = W.algorithmic_bytes(W.CONFIGS[s.cfg])
        got = bench.stream_bytes(s)
        if s.cfg.startswith("C4") or s.cfg in ("C1", "C2", "N3", "R_q4k", "R_q16k", "R_rms", "R_kn",
                                               "T_rms"):
            assert got == alg, (name, got, alg)
        else:
            assert abs(got - alg) <= 0.01 * alg, (name, got, alg)


def test_grouped_stream_covers_the_strided_view(bench):
    """S_R_kn reads the K slice of a packed [1, 3120, 3, 32, 128] bf16 qkv: 32
    head rows of 256 bytes per token, tokens 3 * 32 * 128 * 2 bytes apart,
    starting one q slice (32 * 128 * 2 bytes) in."""
    s = bench.STREAMS["S_R_kn"]
    assert (s.group, s.gstride, s.goff) == (32, 3 * 32 * 128 * 2, 32 * 128 * 2)
    assert s.rows == 3120 * 32 and s.lpr * s.ch * 16 == 128 * 2


def test_stream_library_rejects_bad_sizes_without_a_gpu(bench):
    path = ROOT / "joyai-video-edit_amd" / "joyomni_ops" / "libjoyomni_stream.so"
    if not path.exists():
        pytest.skip("stream library not built (python joyai-video-edit_amd/build.py)")
    import torch  # noqa: F401  (shares torch's HIP runtime, as bench.py does)
    lib = bench.stream_lib()
    pin = (ctypes.c_void_p * 5)()
    pout = (ctypes.c_void_p * 3)()
    # rows <= 0, a group with no stride, too many streams, a shape that is not
    # instantiated
    assert lib.jo_stream_rows(pin, pout, None, 0, 64, 6, 1, 1, 8, 1, 0, 0, 0, 0, 0, None) == 1
    assert lib.jo_stream_rows(pin, pout, None, 10, 16, 1, 1, 1, 16, 0, 1, 0, 32, 0, 0, None) == 1
    assert lib.jo_stream_rows(pin, pout, None, 10, 64, 6, 3, 1, 8, 1, 3, 0, 0, 0, 0, None) == 1
    assert lib.jo_stream_rows(pin, pout, None, 10, 64, 5, 1, 1, 8, 1, 0, 0, 0, 0, 0, None) == 1
    # null stream pointers and a missing scale buffer
    assert lib.jo_stream_rows(pin, pout, None, 10, 64, 6, 1, 1, 8, 0, 0, 0, 0, 0, 0, None) == 1
    fake = (ctypes.c_void_p * 5)(*([16] * 5))
    fake_out = (ctypes.c_void_p * 3)(*([16] * 3))
    assert lib.jo_stream_rows(fake, fake_out, None, 10, 64, 6, 1, 1, 8, 1, 0, 0, 0, 0, 0, None) == 1
    # flags other than bit 0 (write-through stores) and bit 1 (XCD row order)
    assert lib.jo_stream_rows(fake, fake_out, None, 10, 64, 6, 1, 1, 8, 0, 0, 0, 0, 0, 4, None) == 1


def test_bench_refuses_more_than_one_gpu():
    """One GPU is what this build measures: --gpus 2 exits with a message
    naming the reason, before touching a GPU."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    out = r.stdout + r.stderr
    assert "one GPU" in out and "--gpus 2" in out, out


def _synthetic_results(bench):
    """A results dict with every line a default run produces, each carrying
    every field the timing code writes (long figures, as on the GPU)."""
    from joyomni_ops import workloads as W
    fake = {"us_per_call": 17.123456, "eager_us_per_call": 18.98765, "min_us_per_call": 17.0123,
            "max_us_per_call": 17.9876, "timed_calls": 500, "warmup_calls": 20,
            "timing": "hip-graph"}
    results = {}
    for n, cfg in W.CONFIGS.items():
        if n == "B_img":
            continue
        r = bench._finish(dict(fake), W.algorithmic_bytes(cfg), 13, 51_234_567)
        r.update(torch_reference_us_per_call=3988.123, unfused_two_calls_us_per_call=73.456,
                 copy_then_rmsnorm_us_per_call=20.234, cpu_us_per_call=153211.7,
                 cpu_gbps=0.63, cpu_iters=13, cpu_threads=16, gpu_over_cpu=8012.3,
                 stream_ceiling="S_" + n, stream_ceiling_us=17.3456,
                 frac_of_stream_ceiling=1.0081, best_stream="S_" + n + "@no-weight",
                 best_stream_us=17.1, frac_of_best_stream=0.998)
        if W.algorithmic_flops(cfg) is not None:
            r.pop("frac_of_peak", None)
            r.update(bound="mfma", algorithmic_flops=W.algorithmic_flops(cfg), tflops=2329.123,
                     frac_of_fp8_peak=0.4658, ab_eager_us_per_call=138.21,
                     hipblaslt_us_per_call=167.33, hipblaslt_tflops=1923.4,
                     hipblaslt_over_ours=1.2104)
        results[n] = r
    for n, s in bench.STREAMS.items():
        r = bench._finish(dict(fake), bench.stream_bytes(s), 13, 51_234_567)
        r.update(shape="x" * 90, kind="stream-ceiling")
        results[n] = r
    results["B_img"] = {"us_per_call": 633.123, "reference_composition_us_per_call": 779.456,
                        "reference_over_fused": 1.231, "min_us_per_call": 630.1,
                        "max_us_per_call": 640.2, "gemm_flops": 1_260_000_000_000,
                        "block_tflops": 1980.1, "timed_calls": 500, "timing": "hip-graph",
                        "shape": "y" * 100}
    return results


def test_summary_line_fits_the_driver_tail(bench):
    """The stdout line stays whole for a reader that keeps only the last 16 KB
    of stdout: a full-size results dict (every config, stream ceiling and
    comparison field) gives a line under 4 KB that still carries the headline,
    its roofline (with traffic), the CPU baseline and every C0-C4 config."""
    import json
    results = _synthetic_results(bench)
    cpu = {"gbps": 1.83, "us_per_call": 53100.2, "threads": 16, "iters": 38, "seconds": 2.1}
    line = bench.summary_line(results, cpu, 20, 5, "AMD EPYC 9575F 64-Core Processor" * 3,
                              "bench_detail.json")
    text = json.dumps(line, separators=(",", ":"))
    assert len(text.encode()) <= bench.SUMMARY_MAX_BYTES, len(text)
    back = json.loads(text)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
              "roofline", "cpu_baseline"):
        assert k in back, k
    assert back["value"] == results["C1"]["gbps"]
    rf = back["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    assert "traffic" in rf
    cb = back["cpu_baseline"]
    assert cb["kind"] == "port" and cb["cores"] == 16 and cb["unit"] == "GB/s"
    for n in bench.BENCH_CONFIGS:
        e = back["configs"][n]
        assert {"us", "frac", "S_us", "fS", "cpu_us"} <= set(e), (n, e)
    for n in ("N3", "N4", "G1", "G3", "G4", "R_qks", "T_ln", "B_img"):
        assert n in back["ops"], n
    assert not any(n.startswith("S_") for n in back["ops"])
    assert back["ops"]["G3"]["frac"] == 0.466 and back["ops"]["G3"]["blt_x"] == 1.21


def test_gemm_roofline_bound(bench):
    """A GEMM line is priced against whichever roofline takes longer: the fp8
    matrix cores for the image stream's shapes and 4096^3, HBM for the text
    stream's 256 rows (the weight bytes outlast the flops there); the summary
    entry carries the fraction of that bound."""
    from joyomni_ops import workloads as W
    want = {"G1": "mfma", "G2": "mfma", "G3": "mfma", "G4": "mfma", "T_gemm": "mfma",
            "G5": "hbm", "G6": "hbm"}
    for n, bound in want.items():
        cfg = W.CONFIGS[n]
        nbytes = W.algorithmic_bytes(cfg)
        r = {"us_per_call": 50.0, "algorithmic_bytes": nbytes,
             "frac_of_peak": nbytes / 50e-6 / 8e12}
        bench.gemm_roofline(r, W.algorithmic_flops(cfg))
        assert r["bound"] == bound, n
        assert abs(r["tflops"] - W.algorithmic_flops(cfg) / 50e-6 / 1e12) < 0.1
        e = bench.compact_entry(n, r)
        frac = r["frac_of_fp8_peak"] if bound == "mfma" else r["frac_of_peak"]
        assert e["frac"] == round(frac, 3) and e["tflops"] == round(r["tflops"]), (n, e)
        assert ("frac_of_peak" in r) == (bound == "hbm")
