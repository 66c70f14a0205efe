"""CPU: bench.py's reporting contract, without a GPU. `--gpus` above 1 exits
with a message (one GPU in this build); the component records are the short
form (one string per figure: time, rate, fraction of peak, traffic ratio,
cpu_baseline) and every leg keeps its headline figure; the rounding keeps
four significant digits."""
import json
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert p.returncode == 2
    line = json.loads(p.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def rl(v, peak, unit, traffic=None):
    return bench.roofline("hbm" if unit == "GB/s" else "mfma", v, peak, unit, traffic)


def cpu(v):
    return bench.cpu_baseline_obj(v, v / 10, "x/s", 16, "a sample of the workload")


def synthetic_report():
    gemm = {f"bf16_{s}": {"ms": 0.1, "tflops": 1.0, "hbm_gbs": 1.0, "roofline": rl(1200.0, 2500.0, "TFLOP/s", 5),
                          "cpu_baseline": cpu(0.5)}
            for s in ("1024x1024x1024", "4096x4096x4096", "8192x8192x8192")}
    gemm["bf16_16x4096x4096_packed"] = {"us": 12.9, "launches_per_product": 1.0,
                                        "roofline": rl(2600.0, 8000.0, "GB/s")}
    return {
        "lut": {a: {"gelem_s": 1400.0, "us": 11.6, "hbm_gbs": 5800.0} for a in ("gelu", "silu", "exp")},
        "lut_cpu": cpu(30.0),
        "copy": {"copy16_kernel": {"us": 10.9, "gbs": 6100.0, "roofline": rl(6100.0, 8000.0, "GB/s", 7)},
                 "hip_memcpy_d2d": {"us": 14.0, "gbs": 4800.0}},
        "kv": {"copy": {"us_per_step": 44.7, "launches_per_step": 2, "roofline": rl(6200.0, 8000.0, "GB/s")},
               "in_place": {"us_per_step": 5.2, "vs_launch_floor": 1.7, "roofline": rl(19.0, 8000.0, "GB/s")},
               "launch_floor_us_per_kernel": 1.55, "cpu_baseline": cpu(850.0)},
        "gemm": gemm,
        "w8a8": {"i8_decode": {"us": 90.0, "gmac_s": 6000.0, "roofline": rl(5900.0, 8000.0, "GB/s")},
                 "cpu_baseline": cpu(14.0)},
        "e2e": {"decode_tok_s": 8300.0, "decode_ms_per_step": 0.963, "prefill_tok_s": 401000.0,
                "prefill_ms": 10.2, "roofline": rl(2250.0, 8000.0, "GB/s"),
                "prefill_roofline": rl(794.0, 2500.0, "TFLOP/s"),
                "decode_walk": {"calls": 84, "fused_groups": 65}, "cpu_baseline": cpu(89.0)},
    }


def walk(o):
    if isinstance(o, dict):
        yield o
        for v in o.values():
            yield from walk(v)


def test_components_are_short_and_complete():
    comps = bench.compact_components(bench.rounded(synthetic_report()))
    assert set(comps) == {"key", "c1_lut_bf16_16M", "copy_64MiB", "c3_kv_append", "c2_gemm",
                          "w8a8_gemv", "c5_e2e_1b"}
    # tr: the committed counter pass of the LUT kernel over its 64 MiB
    assert comps["c1_lut_bf16_16M"]["gelu"] == "11.6us 1400Gelem/s 72.5%hbm tr1.02"
    assert comps["c1_lut_bf16_16M"]["cpu"] == "30x/s (3 1thr)"
    assert comps["copy_64MiB"] == "10.9us 76.2%hbm hipMemcpy 14us"
    assert comps["c2_gemm"]["bf16_8192^3"] == "100us 1200TF 48.0%mfma cpu 0.5"
    assert comps["c2_gemm"]["bf16_16x4096x4096_packed"] == "12.9us 2600GB/s 32.5%hbm 1 launch"
    assert comps["c3_kv_append"]["in_place"] == "5.2us/step 1.7x the 1.55us launch floor"
    assert comps["w8a8_gemv"]["i8_decode"] == "90us 6000GMAC/s 73.8%hbm"
    assert comps["c5_e2e_1b"]["decode"] == "0.963ms/step 8300tok/s 28.1%hbm"
    assert comps["c5_e2e_1b"]["prefill"] == "10.2ms 401000tok/s 31.8%mfma"
    # every leg a real run reports, at full length, stays well inside a 2000-character tail
    assert len(json.dumps(comps, separators=(",", ":"))) < 1500


def test_traffic_ratio_is_reported():
    rep = synthetic_report()
    rep["lut"]["gelu"]["hbm_gbs"] = 5800.0
    rl_ = rl(5800.0, 8000.0, "GB/s", 68185259)
    assert bench._tr(rl_, 2 * 16 * 2 ** 20 * 2) == " tr1.02"
    assert bench._tr(rl(1.0, 8000.0, "GB/s"), 100) == ""


def test_rounding_keeps_four_digits():
    assert bench.rounded({"a": [1.234567, 0.0, float("inf")], "b": 123456.7}) == {
        "a": [1.235, 0.0, float("inf")], "b": 123500.0}
