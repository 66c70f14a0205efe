"""Benchmark of the MI355X hot path on one GPU; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only attn,lut,copy,kv,gemm,w8a8,e2e]

Headline (`value`): int8-KV GQA decode attention
(B=32, H=32, Hkv=8, D=128, ragged L_b ~ U[512, 32768], bucket 32768, Q bf16,
cache filled by the int8 quantize+append op) in tokens/s = B / step time.
A step is one DecodeAttentionI8 dispatch over the whole batch, inputs
resident in HBM. The other configs are reported under "components":
LUT Gelem/s (config 1), GEMM TFLOP/s (config 2), KV append (config 3), the
end-to-end decoder through the `.holo` session (config 5, decode/prefill tok/s)
and the quantized-weight W8A8 GEMV (GMAC/s).
Every number comes from HIP events on the stream the kernels run on: per step
for the headline, and around a batch of back-to-back calls for the components
(queued_ms), whose kernels are short enough that per-call events would count
the host's dispatch latency. A component that rotates buffers (past the 256 MB
last-level cache) first calls once on every set, untimed (at least W calls),
so no timed call is a set's first touch; each GEMM shape also runs a quarter
second untimed first, so the clocks have ramped up after the host-side legs.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # dense bf16 MFMA
FP32_PEAK_TFLOPS = 157.3       # fp32 matrix
METRIC = "int8-KV decode attn tok/s & HBM GB/s; bf16 LUT Gelem/s; GEMM TFLOP/s"


def profiled_traffic(key):
    """HBM bytes per launch measured by rocprofv3 counters (profiles/traffic.txt)."""
    f = ROOT / "profiles" / "traffic.txt"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 3 and parts[0] == key:
            return int(parts[1]) + int(parts[2])
    return None


def roofline(bound, achieved, peak, unit, traffic=None, kernel=None):
    r = {"bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
         "frac": achieved / peak, "traffic": traffic}
    if kernel:
        r["kernel"] = kernel
    return r


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--only", default="attn,lut,copy,kv,gemm,w8a8,e2e")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--seed", type=int, default=1234)
    p.add_argument("--e2e-flags", type=int, default=0,
                   help="HOLO_SESSION_* load flags of config 5's decode session (A/B of the fusions)")
    return p.parse_args()


class Timer:
    """HIP events recorded on the backend's stream around each timed dispatch."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []

    def __enter__(self):
        s = self.torch.cuda.Event(enable_timing=True)
        s.record()
        self._s = s
        return self

    def __exit__(self, *exc):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs.append((self._s, e))

    def mean_ms(self):
        self.torch.cuda.synchronize()
        return sum(s.elapsed_time(e) for s, e in self.pairs) / max(1, len(self.pairs))


def queued_ms(torch, fn, n):
    """GPU time per call of n back-to-back calls, HIP events around the batch on
    the backend's stream. A spin kernel first keeps the GPU busy while the host
    queues the calls, so the host's dispatch cost (tens of microseconds through
    Python) is not counted as kernel time for the short kernels."""
    torch.cuda.synchronize()
    torch.cuda._sleep(int(n * 100e-6 * 2.0e9))     # about n x 100 us at ~2 GHz
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(n):
        fn(i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / n


def warm(torch, fn, seconds):
    """Untimed calls of fn(i) for at least `seconds` of wall time: a GPU that
    sat idle (behind a host-side leg) ramps its clocks back up before the
    timed calls, instead of during them."""
    t0, i = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def cpu_time(fn, min_seconds):
    """Seconds per call of fn() on the host, repeated until min_seconds pass."""
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            return dt / calls, calls, dt


def cpu_baseline_obj(value_multi, value_single, unit, threads, sample):
    """The cpu_baseline record: the multi-threaded leg is `value` (cores =
    its threads), the single-threaded leg beside it, and the host."""
    return {"value": value_multi, "unit": unit, "cores": threads, "kind": "port",
            "sample": sample, "single_thread": value_single}


def bf16_normal(torch, shape, gen, outlier_frac=0.0):
    x = torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32)
    if outlier_frac > 0:
        d = shape[-1]
        nout = max(1, math.ceil(outlier_frac * d))
        ch = torch.randperm(d, generator=gen, device="cuda")[:nout]
        x[..., ch] *= 20.0
    return x.to(torch.bfloat16)


# --------------------------------------------------------------- config 4 ----
def bench_attn(torch, be, args, rep):
    import numpy as np
    from hologram_amd import (DTYPE_BF16, BufferRef, DecodeAttentionI8Call, DeviceWorkspace,
                              KernelCall, KvQuantAppendCall)
    B, H, Hkv, D, bucket = 32, 32, 8, 128, 32768
    rng = np.random.default_rng(args.seed)
    lens = rng.integers(512, 32769, size=B).astype(np.uint32)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    planes = B * Hkv
    ws = DeviceWorkspace()
    kq = torch.empty(planes * bucket * D, dtype=torch.int8, device="cuda")
    vq = torch.empty_like(kq)
    ks = torch.empty(planes * bucket, dtype=torch.float32, device="cuda")
    vs = torch.empty_like(ks)
    pos0 = torch.zeros(1, dtype=torch.int32, device="cuda")
    # fill both caches through the int8 quantize+append op (config 3's scheme)
    for cq, cs in ((kq, ks), (vq, vs)):
        for p0 in range(0, planes, 32):       # 32 planes (256 MiB of bf16) per call
            src = bf16_normal(torch, (32, bucket, D), gen, 0.02)
            fill = DeviceWorkspace()
            fill.bind(0, src)
            fill.bind(1, pos0)
            fill.bind(2, cq)
            fill.bind(3, cs)
            off_q, off_s = p0 * bucket * D, p0 * bucket * 4
            call = KernelCall.KvQuantAppend(KvQuantAppendCall(
                BufferRef(0), BufferRef(1), BufferRef(2, off_q, 32 * bucket * D),
                BufferRef(3, off_s, 32 * bucket * 4), BufferRef(2, off_q, 32 * bucket * D),
                BufferRef(3, off_s, 32 * bucket * 4), 32, bucket, bucket, D, DTYPE_BF16))
            be.dispatch(call, fill)
            be.synchronize()
            del src
    nq = 4   # rotate fresh queries every step
    qs = [bf16_normal(torch, (B * H * D,), gen) for _ in range(nq)]
    out = torch.empty(B * H * D, dtype=torch.bfloat16, device="cuda")
    lens_t = torch.from_numpy(lens.astype(np.int32)).cuda()
    for s, t in enumerate([qs[0], kq, vq, ks, vs, lens_t, out]):
        ws.bind(s, t)
    for i in range(1, nq):
        ws.bind(7 + i, qs[i])
    calls = []
    for i in range(nq):
        qslot = 0 if i == 0 else 7 + i
        calls.append(KernelCall.DecodeAttentionI8(DecodeAttentionI8Call(
            BufferRef(qslot), *[BufferRef(s) for s in range(1, 7)], B, H, Hkv, bucket, D, 0,
            DTYPE_BF16)))
    for i in range(args.warmup):
        be.dispatch(calls[i % nq], ws)
    be.synchronize()
    # (1) each dispatch between its own pair of events, as the host issues
    # them one at a time (the wall clock of the K steps is taken here)
    timer = Timer(torch)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        with timer:
            be.dispatch(calls[i % nq], ws)
    be.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_each = timer.mean_ms()
    # (2) the headline: the same K steps queued back to back behind a spin
    # kernel, events around the batch, so no step waits on the host's Python
    # dispatch (a serving loop issues asynchronously)
    ms = queued_ms(torch, lambda i: be.dispatch(calls[i % nq], ws), args.steps)
    sum_l = int(lens.sum())
    kv_bytes = sum_l * Hkv * (2 * D + 8)          # int8 K and V rows + two f32 scales
    alg_bytes = kv_bytes + B * H * D * 2 * 2 + B * 4
    flops = 4.0 * D * H * sum_l
    res = {
        "tok_s": B / (ms / 1e3), "ms": ms, "ms_events_per_dispatch": ms_each,
        "wall_ms_per_step": wall * 1e3 / args.steps,
        "hbm_gbs": alg_bytes / (ms / 1e3) / 1e9, "alg_bytes": alg_bytes, "sum_len": sum_l,
        "gflops": flops / 1e9, "lens_seed": args.seed,
    }
    rep["attn"] = res
    if not args.no_cpu:
        rep["attn_cpu"] = cpu_attn(torch, kq, ks, vq, vs, qs[0], lens, B, H, Hkv, bucket, D)
    return res


def cpu_attn(torch, kq, ks, vq, vs, q, lens, B, H, Hkv, bucket, D, min_seconds=10.0):
    """The oracle-side C++ restatement of the reference CPU path (dequantize the
    realized rows, two-pass attention rows), all host threads, on the same batch,
    repeated until ~10 s of CPU work; tok/s = B * passes / seconds."""
    import numpy as np
    import oracle
    kq_h, vq_h = kq.cpu().numpy(), vq.cpu().numpy()
    ks_h, vs_h = ks.cpu().numpy(), vs.cpu().numpy()
    q_h = q.float().cpu().numpy().copy()
    l_h = lens.astype(np.uint32).copy()
    out = np.zeros(B * H * D, np.float32)
    th = oracle.host_threads()
    lib = oracle.lib()
    p = lambda a: a.ctypes.data
    run = lambda t: lambda: lib.cb_decode_attention_i8(
        p(q_h), p(kq_h), p(ks_h), p(vq_h), p(vs_h), p(l_h), p(out), B, H, Hkv, bucket, D,
        oracle.attn_scale(D), t)
    sec, passes, dt = cpu_time(run(th), min_seconds)
    sec1, passes1, dt1 = cpu_time(run(1), min_seconds / 2)
    return cpu_baseline_obj(B / sec, B / sec1, "tok/s", th,
                            f"full batch ({B} seq, {int(lens.sum())} keys): x{passes} "
                            f"{th}thr, x{passes1} 1thr")


# --------------------------------------------------------------- config 1 ----
def bench_lut(torch, be, args, rep):
    import numpy as np
    from hologram_amd import DTYPE_BF16, BufferRef, DeviceWorkspace, KernelCall, UnaryCall
    n = 16_777_216
    nbuf = 8                                   # 8 x (32 + 32) MiB = 512 MiB rotation
    ws = DeviceWorkspace()
    ins, outs = [], []
    for i in range(nbuf):
        x = torch.randint(0, 65536, (n,), dtype=torch.int32, device="cuda").to(torch.int16)
        ins.append(x)
        outs.append(torch.empty(n, dtype=torch.int16, device="cuda"))
        ws.bind(2 * i, ins[-1])
        ws.bind(2 * i + 1, outs[-1])
    res = {}
    for name in ("Gelu", "Silu", "Exp"):
        ctor = getattr(KernelCall, name)
        calls = [ctor(UnaryCall(BufferRef(2 * i), BufferRef(2 * i + 1), n, 16, DTYPE_BF16))
                 for i in range(nbuf)]
        for i in range(max(args.warmup, nbuf)):
            be.dispatch(calls[i % nbuf], ws)
        be.synchronize()
        ms = queued_ms(torch, lambda i: be.dispatch(calls[i % nbuf], ws), args.steps * 4)
        res[name.lower()] = {"gelem_s": n / (ms / 1e3) / 1e9, "us": ms * 1e3,
                             "hbm_gbs": 4 * n / (ms / 1e3) / 1e9}
    rep["lut"] = res
    if not args.no_cpu:
        import oracle
        tab = oracle.build_table(2, DTYPE_BF16)
        xs = ins[0].cpu().numpy().view(np.uint16)
        o = np.empty_like(xs)
        th = oracle.host_threads()
        run = lambda t: lambda: oracle.lib().cb_lut(tab.ctypes.data, xs.ctypes.data,
                                                    o.ctypes.data, n, t)
        sec, reps, _ = cpu_time(run(th), 6.0)
        sec1, reps1, _ = cpu_time(run(1), 3.0)
        rep["lut_cpu"] = cpu_baseline_obj(n / sec / 1e9, n / sec1 / 1e9, "Gelem/s", th,
                                          f"16M GELU gather: x{reps} {th}thr, x{reps1} 1thr")
    return res


# --------------------------------------------------------------- config 3 ----
def bench_kv(torch, be, args, rep):
    """Config 3: one step appends one new token per sequence to the K and to the
    V cache (two KvQuantAppend dispatches: 16 x 8 planes, bucket 4096, D 128,
    pos 4095). In place (the executor's move) a step writes 2 x 49,668 bytes;
    the honest-copy form (the reference kernel's contract) also copies both
    caches and their scales, 2 x (2 x 64 MiB + 2 x 2 MiB) + the new rows, with
    two sets of caches rotated (528 MiB). The empty-kernel launch floor is
    timed the same way beside the in-place figure."""
    import numpy as np
    from hologram_amd import DTYPE_BF16, BufferRef, DeviceWorkspace, KernelCall, KvQuantAppendCall
    planes, bucket, D = 16 * 8, 4096, 128
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 3)
    ws = DeviceWorkspace()
    nset = 2                                   # copy-form rotation: 2 x 264 MiB
    slot = iter(range(1000))
    bind = lambda t: (lambda s_: (ws.bind(s_, t), s_)[1])(next(slot))
    pos_s = bind(torch.tensor([4095], dtype=torch.int32, device="cuda"))
    caches = []                                # per set: (K q, K s, K out q, K out s, V ...)
    keep = []
    for _ in range(nset):
        c = []
        for _kv in range(2):
            cq = torch.randint(-127, 128, (planes * bucket * D,), dtype=torch.int8, device="cuda",
                               generator=gen)
            cs = torch.rand(planes * bucket, device="cuda", generator=gen)
            oq, os_ = torch.empty_like(cq), torch.empty_like(cs)
            keep += [cq, cs, oq, os_]
            c.append(tuple(bind(t) for t in (cq, cs, oq, os_)))
        caches.append(c)
    news = []
    for _ in range(4):
        t = bf16_normal(torch, (planes, 1, D), gen, 0.02)
        keep.append(t)
        news.append(bind(t))

    def step_calls(form, i):
        out = []
        for kv in range(2):
            cq, cs, oq, os_ = caches[i % nset][kv]
            tq, ts = (cq, cs) if form == "in_place" else (oq, os_)
            out.append(KernelCall.KvQuantAppend(KvQuantAppendCall(
                BufferRef(news[(2 * i + kv) % 4]), BufferRef(pos_s), BufferRef(cq), BufferRef(cs),
                BufferRef(tq), BufferRef(ts), planes, bucket, 1, D, DTYPE_BF16)))
        return out

    res = {}
    for form in ("in_place", "copy"):
        steps = [step_calls(form, i) for i in range(4)]
        run = lambda i: [be.dispatch(c, ws) for c in steps[i % 4]]
        for i in range(max(args.warmup, 4)):
            run(i)
        be.synchronize()
        ms = queued_ms(torch, run, args.steps * 4)
        if form == "in_place":
            alg = 2 * (planes * D * 2 + planes * D + planes * 4) + 4
        else:
            alg = 2 * (2 * (planes * bucket * D + planes * bucket * 4) + planes * D * 2)
        gbs = alg / (ms / 1e3) / 1e9
        res[form] = {"us_per_step": ms * 1e3, "dispatches_per_step": 2, "launches_per_step": 2,
                     "alg_bytes": alg,
                     "hbm_gbs": gbs,
                     "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s",
                                          profiled_traffic(f"kv_{form}_config3"))}
    # the launch floor: an empty kernel, queued back to back the same way
    floor_ms = queued_ms(torch, lambda i: torch.cuda._sleep(0), args.steps * 8)
    res["launch_floor_us_per_kernel"] = floor_ms * 1e3
    res["in_place"]["vs_launch_floor"] = (res["in_place"]["us_per_step"] / 2) / (floor_ms * 1e3)
    res["copy"]["rotation_bytes"] = nset * 2 * 2 * (planes * bucket * D + planes * bucket * 4)
    rep["kv"] = res
    if not args.no_cpu:
        import oracle
        th = oracle.host_threads()
        hq = [np.ascontiguousarray(keep[i].cpu().numpy()) for i in range(4)]
        nw = np.ascontiguousarray(keep[4 * nset * 2].cpu().view(torch.int16).numpy())
        lib = oracle.lib()
        p = lambda a: a.ctypes.data
        def copy_step(t):
            def f():
                for _ in range(2):   # K and V
                    lib.cb_kv_quant_append_copy(p(nw), DTYPE_BF16, 4095, p(hq[0]), p(hq[1]),
                                                p(hq[2]), p(hq[3]), planes, bucket, 1, D, t)
            return f
        sec, n1, _ = cpu_time(copy_step(th), 4.0)
        sec1, n2, _ = cpu_time(copy_step(1), 3.0)
        res["cpu_baseline"] = cpu_baseline_obj(
            1.0 / sec, 1.0 / sec1, "steps/s", th,
            f"copy-form step (K, V): x{n1} {th}thr, x{n2} 1thr")
        def move_step():
            for _ in range(2):
                lib.or_kv_quant_append(p(nw), DTYPE_BF16, 4095, p(hq[0]), p(hq[1]), planes, bucket,
                                       1, D)
        sec_m, n3, _ = cpu_time(move_step, 2.0)
        res["cpu_baseline"]["in_place_single_thread_steps_s"] = 1.0 / sec_m
    return res


# --------------------------------------------------------------- config 2 ----
def bench_gemm(torch, be, args, rep):
    """Config 2: bf16 and f32 C = A.B at 1024^3, 4096^3, 8192^3 and 16x4096x4096.
    Every shape rotates enough (A, B, C) sets to pass 512 MiB (at least two),
    so no call finds its operands in the 256 MB Infinity Cache. CPU legs: the
    reference engine restatement (cpu_baseline.c) on the host threads for
    every shape, and on one thread for 1024^3 and the few-row shape."""
    import numpy as np
    from hologram_amd import DTYPE_BF16, DTYPE_F32, BufferRef, DeviceWorkspace, KernelCall, MatMulCall
    shapes = [(1024, 1024, 1024), (4096, 4096, 4096), (8192, 8192, 8192), (16, 4096, 4096)]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 2)
    res = {}
    for dt, tdt, peak in ((DTYPE_BF16, torch.bfloat16, BF16_PEAK_TFLOPS),
                          (DTYPE_F32, torch.float32, FP32_PEAK_TFLOPS)):
        for (m, n, k) in shapes:
            es = 2 if dt == DTYPE_BF16 else 4
            set_bytes = (m * k + k * n + m * n) * es
            nbuf = max(2, -(-(512 << 20) // set_bytes) + 1)
            ws = DeviceWorkspace()
            calls, keep = [], []
            for i in range(nbuf):
                a = (torch.randn(m * k, generator=gen, device="cuda") / math.sqrt(k)).to(tdt)
                b = (torch.randn(k * n, generator=gen, device="cuda") / math.sqrt(k)).to(tdt)
                c = torch.empty(m * n, dtype=tdt, device="cuda")
                keep.append((a, b))
                ws.bind(3 * i, a)
                ws.bind(3 * i + 1, b)
                ws.bind(3 * i + 2, c)
                calls.append(KernelCall.MatMul(MatMulCall(BufferRef(3 * i), BufferRef(3 * i + 1),
                                                          BufferRef(3 * i + 2), m, k, n, dt)))
            for i in range(max(args.warmup, nbuf)):
                be.dispatch(calls[i % nbuf], ws)
            be.synchronize()
            warm(torch, lambda i: be.dispatch(calls[i % nbuf], ws), 0.25)
            steps = args.steps if m * n * k < 8192 ** 3 else max(3, args.steps // 4)
            ms = queued_ms(torch, lambda i: be.dispatch(calls[i % nbuf], ws), steps)
            tf = 2.0 * m * n * k / (ms / 1e3) / 1e12
            key = f"{'bf16' if dt == DTYPE_BF16 else 'f32'}_{m}x{n}x{k}"
            gbs = set_bytes / (ms / 1e3) / 1e9
            dname = "bf16" if dt == DTYPE_BF16 else "f32"
            tkey = f"gemm_{dname}_{m}c" if m == n == k else f"gemm_{dname}_{m}x{n}x{k}"
            if m <= 64:   # few rows: bandwidth-bound on B
                rl = roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s", profiled_traffic(tkey))
            else:
                rl = roofline("mfma", tf, peak, "TFLOP/s", profiled_traffic(tkey))
            res[key] = {"tflops": tf, "ms": ms, "hbm_gbs": gbs, "roofline": rl,
                        "rotation_bytes": nbuf * set_bytes}
            if dt == DTYPE_BF16 and m == n == k:
                # the vendor library on the same box and the same rotated
                # operands (torch.matmul -> hipBLASLt), for comparison only
                mats = [(keep[i][0].view(m, k), keep[i][1].view(k, n),
                         torch.empty(m, n, dtype=tdt, device="cuda")) for i in range(nbuf)]
                vend = lambda i: torch.matmul(mats[i % nbuf][0], mats[i % nbuf][1],
                                              out=mats[i % nbuf][2])
                warm(torch, vend, 0.25)
                vms = queued_ms(torch, vend, steps)
                res[key]["hipblaslt_tflops"] = 2.0 * m * n * k / (vms / 1e3) / 1e12
                del mats
            if not args.no_cpu:
                res[key]["cpu_baseline"] = cpu_gemm(keep[0], m, k, n, dt,
                                                    single=(m == 1024 or m <= 64))
            del ws, calls, keep
    res["bf16_16x4096x4096_packed"] = bench_fewrow_packed(torch, be, args, 16, 4096, 4096)
    rep["gemm"] = res
    return res


def bench_fewrow_packed(torch, be, args, m, k, n):
    """The few-row bf16 MatMul with its weight a constant of a compiled graph:
    the session packs the weight at load and runs the product as one launch
    (gemv_packed.hip) instead of split-K plus a reduce. One archive holds
    `nbuf` such products over different weights (rotated past the 256 MB
    Infinity Cache), each over its own A (a slice of 2x, computed in-graph by
    one Add), so no two products share a launch; the captured walk is replayed
    and the time per product is the replay's GPU time over nbuf (the one Add
    included)."""
    import numpy as np
    from hologram_amd import (DTYPE_BF16, BinaryCall, BufferRef, ConstantEntry, HipSession, HoloWriter,
                              KernelCall, MatMulCall, PortDescriptor)
    nbuf = max(2, -(-(512 << 20) // (k * n * 2)))
    rng = np.random.default_rng(args.seed + 9)
    r = lambda slot, elems: BufferRef(slot, 0, 2 * elems)
    w = HoloWriter()
    mk = m * k
    w.kernel_calls = [KernelCall.Add(BinaryCall(r(0, nbuf * mk), r(0, nbuf * mk), r(1, nbuf * mk),
                                                nbuf * mk, 16, DTYPE_BF16))]
    for i in range(nbuf):
        wt = (rng.standard_normal(k * n, dtype=np.float32) / np.float32(np.sqrt(k))).view(np.uint32) >> 16
        w.constants.append(ConstantEntry(2 + 2 * i, DTYPE_BF16, wt.astype(np.uint16).tobytes()))
        a_i = BufferRef(1, 2 * mk * i, 2 * mk)      # product i's own A: a slice of 2x
        w.kernel_calls.append(KernelCall.MatMul(MatMulCall(a_i, r(2 + 2 * i, k * n), r(3 + 2 * i, m * n),
                                                           m, k, n, DTYPE_BF16)))
        w.outputs.append(PortDescriptor(f"y{i}", 3 + 2 * i, m * n, DTYPE_BF16, [m, n]))
    w.inputs = [PortDescriptor("x", 0, nbuf * mk, DTYPE_BF16, [nbuf * m, k])]
    sess = HipSession(be, w.finish())
    packed = sess.packed[0]
    x = (rng.standard_normal(nbuf * m * k, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
    sess.write_input(0, x.tobytes())
    sess.capture()
    sess.synchronize()
    ext = torch.cuda.ExternalStream(sess.stream())
    reps = max(3, args.steps)
    for _ in range(2):
        sess.replay()
    sess.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    with torch.cuda.stream(ext):
        ev[0].record()
    for _ in range(reps):
        sess.replay()
    with torch.cuda.stream(ext):
        ev[1].record()
    sess.synchronize()
    us = ev[0].elapsed_time(ev[1]) * 1e3 / (reps * nbuf)
    gbs = (m * k + k * n + m * n) * 2 / (us / 1e6) / 1e9
    sess.close()
    # each packed group is one launch over one product's weights
    return {"us": us, "launches_per_product": packed / nbuf, "packed_groups": packed,
            "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s", None)}


def cpu_gemm(ab, m, k, n, dt, single):
    """The reference MatMul engines restated (4x16 AVX2/FMA tiles under the 64^3
    bisection; bf16: widen, f32 engine, truncate; few-row bf16 streamed) on
    the host threads, and on one thread when `single`; TFLOP/s."""
    import numpy as np
    import oracle
    from hologram_amd import DTYPE_BF16
    import torch
    a, b = (np.ascontiguousarray(x.cpu().view(torch.int16 if dt == DTYPE_BF16 else torch.float32)
                                 .numpy()) for x in ab)
    out = np.zeros(m * n, a.dtype)
    lib = oracle.lib()
    if dt == DTYPE_BF16:
        fn = lib.cb_matmul_bf16_gemv if m <= 8 else lib.cb_matmul_bf16
    else:
        fn = lib.cb_matmul_f32
    run = lambda t: lambda: fn(a.ctypes.data, b.ctypes.data, out.ctypes.data, m, k, n, t)
    th = oracle.host_threads()
    flops = 2.0 * m * n * k
    sec, reps, _ = cpu_time(run(th), 2.0)
    sec1, reps1 = (cpu_time(run(1), 2.0)[:2] if single else (None, 0))
    return cpu_baseline_obj(flops / sec / 1e12, flops / sec1 / 1e12 if sec1 else None, "TFLOP/s",
                            th, f"whole product x{reps} {th}thr"
                                + (f", x{reps1} 1thr" if single else ""))


# --------------------------------------------------------------- config 5 ----
class _DevBytes:
    """A device range as a torch uint8 tensor (CUDA array interface)."""

    def __init__(self, ptr, nbytes):
        self.__cuda_array_interface__ = {"shape": (nbytes,), "typestr": "|u1",
                                         "data": (ptr, False), "version": 2}


def bench_e2e(torch, be, args, rep):
    """Config 5: the Llama-style ~1B decoder run through HipSession as two `.holo`
    archives over the same weights and the same int8 caches (memo off: every
    walk computes). The prompt pass (build_prefill) takes each sequence's 512
    prompt tokens at once; the decode step (build_decode_step) then generates
    greedily, its walk captured once into a HIP graph and replayed per token,
    the next-token ids never leaving the device (ArgMax writes the buffer the
    next step's Gather reads). Batch 8, random prompts, 256 timed decode steps."""
    import numpy as np
    from hologram_amd import HipSession
    from hologram_amd.decoder_graph import (DecoderConfig, build_decode_step, build_prefill,
                                            init_weights, rope_tables, rope_tables_rows)
    cfg = DecoderConfig()
    prompt_len, gen_len = 512, 256
    B, H, Hkv, Dh, V = cfg.batch, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.vocab
    t0 = time.perf_counter()
    weights = init_weights(cfg, seed=args.seed + 5)
    dec_archive = build_decode_step(cfg, weights)
    pre_archive = build_prefill(cfg, weights, prompt_len)
    del weights
    t_build = time.perf_counter() - t0
    t0 = time.perf_counter()
    pre = HipSession(be, pre_archive)
    dec = HipSession(be, dec_archive, flags=args.e2e_flags)
    t_load = time.perf_counter() - t0
    archive_bytes = len(dec_archive)
    del pre_archive
    dev = lambda b: torch.frombuffer(bytearray(b), dtype=torch.uint8).cuda()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 6)

    # ---- prompt pass inputs, device-resident and bound in place
    prompt = torch.randint(0, V, (B, prompt_len), generator=gen, device="cuda", dtype=torch.int32)
    pos0 = torch.zeros(1, dtype=torch.int32, device="cuda")
    lens0 = torch.full((B,), prompt_len, dtype=torch.int32, device="cuda")
    rows = [dev(t) for t in rope_tables_rows(cfg, np.arange(prompt_len), H)]
    rows += [dev(t) for t in rope_tables_rows(cfg, np.arange(prompt_len), Hkv)]
    for i, t in enumerate([prompt, pos0, lens0] + rows):
        pre.bind_input(i, t)
    # the decode step reads and appends to the prompt pass's caches
    for c in range(4 * cfg.layers):
        dec.bind_input(7 + c, pre.output_ptr(2 + c))

    # ---- decode inputs: tokens live in the decode step's ArgMax output
    npos = prompt_len + gen_len + 1
    cq, sq = (dev(t).view(npos, -1) for t in rope_tables(cfg, np.arange(npos), H))
    ck, sk = (dev(t).view(npos, -1) for t in rope_tables(cfg, np.arange(npos), Hkv))
    pos_tab = torch.arange(npos, dtype=torch.int32, device="cuda").view(npos, 1)
    lens_tab = (torch.arange(npos, dtype=torch.int32, device="cuda") + 1).view(npos, 1).repeat(1, B)
    tptr, tbytes = dec.output_ptr(0)
    tok = torch.as_tensor(_DevBytes(tptr, tbytes), device="cuda").view(torch.int32)
    dec.bind_input(0, (tptr, tbytes))
    # the step's position, lengths and rotary rows, as one row per position of
    # one table: a step's inputs are one device copy into one staging row, the
    # session's six input ports bound to 256-byte aligned views of it
    parts = [pos_tab.view(torch.uint8).view(npos, -1), lens_tab.view(torch.uint8).view(npos, -1),
             cq.view(torch.uint8).view(npos, -1), sq.view(torch.uint8).view(npos, -1),
             ck.view(torch.uint8).view(npos, -1), sk.view(torch.uint8).view(npos, -1)]
    widths = [x.shape[1] for x in parts]
    offs = [0]
    for wdt in widths:
        offs.append(offs[-1] + (wdt + 255) // 256 * 256)
    table = torch.zeros((npos, offs[-1]), dtype=torch.uint8, device="cuda")
    for o, wdt, x in zip(offs, widths, parts):
        table[:, o:o + wdt] = x
    staging = torch.zeros(offs[-1], dtype=torch.uint8, device="cuda")
    for i, (o, wdt) in enumerate(zip(offs, widths)):
        dec.bind_input(1 + i, staging[o:o + wdt])
    ext_pre = torch.cuda.ExternalStream(pre.stream())
    ext = torch.cuda.ExternalStream(dec.stream())
    torch.cuda.synchronize()

    # ---- prompt pass: one eager walk, the capture, then one timed replay
    # (rewriting the same cache rows with the same values)
    pre.capture()
    pre.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    with torch.cuda.stream(ext_pre):
        ev[0].record()
    pre.replay()
    with torch.cuda.stream(ext_pre):
        ev[1].record()
    pre.synchronize()
    prefill_ms = ev[0].elapsed_time(ev[1])
    first = torch.as_tensor(_DevBytes(*pre.output_ptr(0)), device="cuda").view(torch.int32)

    def set_step(p):
        with torch.cuda.stream(ext):
            staging.copy_(table[p], non_blocking=True)

    # ---- decode: the prompt pass's greedy token at position 512 (the eager
    # step inside the capture), then 256 timed replays at 513 .. 768
    tok.copy_(first)
    set_step(prompt_len)
    torch.cuda.synchronize()
    dec.capture()
    dec.synchronize()
    with torch.cuda.stream(ext):
        ev[2].record()
    for p in range(prompt_len + 1, prompt_len + 1 + gen_len):
        set_step(p)
        dec.replay()
    with torch.cuda.stream(ext):
        ev[3].record()
    dec.synchronize()
    torch.cuda.synchronize()
    decode_ms = ev[2].elapsed_time(ev[3])
    last = tok.cpu().tolist()
    n_nodes, n_groups = dec.n_nodes, dec.n_groups
    pre_nodes = pre.n_nodes
    pre.close()
    dec.close()

    Dm, F, L = cfg.hidden, cfg.ffn, cfg.layers
    w_bytes = 2 * (L * (Dm * H * Dh + 2 * Dm * Hkv * Dh + H * Dh * Dm + 3 * Dm * F + 2 * Dm)
                   + Dm * V + Dm)
    mean_len = prompt_len + 1 + gen_len / 2
    kv_bytes = L * B * Hkv * mean_len * (2 * Dh + 8)
    step_ms = decode_ms / gen_len
    # prompt pass flops: every projection over B*T rows, causal attention
    # (QK and PV over the visible keys of each row), the LM head on the last rows
    R = B * prompt_len
    mm_flops = 2 * R * L * (Dm * H * Dh + 2 * Dm * Hkv * Dh + H * Dh * Dm + 3 * Dm * F)
    attn_flops = 4 * L * B * H * Dh * (prompt_len * (prompt_len + 1) / 2)
    pre_flops = mm_flops + attn_flops + 2 * B * Dm * V
    pre_tflops = pre_flops / (prefill_ms / 1e3) / 1e12
    res = {
        "decode_tok_s": B * gen_len / (decode_ms / 1e3),
        "prefill_tok_s": R / (prefill_ms / 1e3),
        "decode_ms_per_step": step_ms,
        "prefill_ms": prefill_ms,
        "decode_walk": {"calls": n_nodes, "fused_groups": n_groups},
        "prefill_walk_calls": pre_nodes,
        "alg_bytes_per_decode_step": int(w_bytes + kv_bytes),
        "hbm_gbs": (w_bytes + kv_bytes) / (step_ms / 1e3) / 1e9,
        "prefill_flops": int(pre_flops),
        "archive_bytes": archive_bytes, "build_s": t_build, "load_s": t_load,
        "last_tokens": last,
        "config": {"layers": L, "hidden": Dm, "heads": H, "kv_heads": Hkv,
                   "head_dim": Dh, "ffn": F, "vocab": V, "batch": B, "prompt": prompt_len,
                   "generate": gen_len, "bucket": cfg.bucket, "kv": "int8",
                   "weights": "bf16 ~ N(0, 0.02), seeded", "vocab_note": "32,000 assumed"},
        "roofline": roofline("hbm", (w_bytes + kv_bytes) / (step_ms / 1e3) / 1e9, HBM_PEAK_GBS,
                             "GB/s", kernel="decode step: weights + int8 KV"),
        "prefill_roofline": roofline("mfma", pre_tflops, BF16_PEAK_TFLOPS, "TFLOP/s",
                                     kernel="prompt pass"),
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_decode_step(cfg, dec_archive, int(mean_len))
    del dec_archive
    rep["e2e"] = res
    return res


def cpu_decode_step(cfg, archive, length):
    """One decode step of the same 16-layer archive walked on the host with the
    reference CPU engines (oracle/graph.py's cpu_baseline mode: streamed
    few-row bf16 MatMuls, two-pass attention rows, in-place int8 appends), at
    the timed run's mean context length; tok/s = batch / step time."""
    import numpy as np
    import oracle
    from oracle.graph import OracleSession
    from hologram_amd.decoder_graph import rope_tables
    th = oracle.host_threads()
    P, S, Dh = cfg.planes, cfg.bucket, cfg.head_dim
    walks = {}
    for t in (th, 1):
        o = OracleSession(archive, verify_footer=False, products="cpu_baseline", threads=t)
        cq, sq = rope_tables(cfg, np.array([length - 1]), cfg.heads)
        ck, sk = rope_tables(cfg, np.array([length - 1]), cfg.kv_heads)
        ins = [np.arange(cfg.batch, dtype=np.int32).tobytes(), np.uint32(length - 1).tobytes(),
               np.full(cfg.batch, length, np.uint32).tobytes(), cq, sq, ck, sk]
        for i, b in enumerate(ins):
            o.set_input(i, b)
        for layer in range(cfg.layers):
            for j, z in enumerate([P * S * Dh, P * S * 4] * 2):
                o.set_input(7 + 4 * layer + j, bytes(z))
        o.run()                                  # first walk: tables, first touches
        walks[t] = cpu_time(o.run, 6.0 if t == th else 3.0)
        del o
    (sec, n, _), (sec1, n1, _) = walks[th], walks[1]
    return cpu_baseline_obj(cfg.batch / sec, cfg.batch / sec1, "tok/s", th,
                            f"{cfg.layers}-layer decode step at ctx {length}: x{n} {th}thr, "
                            f"x{n1} 1thr")


# ------------------------------------------------------- copy ceiling ----
def bench_copy(torch, be, args, rep):
    """The plain-copy ceiling for the LUT's bytes: 32 MiB read + 32 MiB written
    per launch, 8 pairs rotated (512 MiB), through the backend's own copy
    kernel (a KvCacheWrite honest copy with no new rows, one copy16_kernel
    launch) and through torch's device copy (hipMemcpyAsync), timed like the
    LUT (queued_ms)."""
    from hologram_amd import BufferRef, DeviceWorkspace, KernelCall, KvCacheWriteCall
    nbytes, nbuf = 32 << 20, 8
    ws = DeviceWorkspace()
    src = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(nbuf)]
    dst = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(nbuf)]
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws.bind(2 * nbuf, pos)
    ws.bind(2 * nbuf + 1, torch.zeros(16, dtype=torch.uint8, device="cuda"))
    calls = []
    for i in range(nbuf):
        ws.bind(2 * i, src[i])
        ws.bind(2 * i + 1, dst[i])
        calls.append(KernelCall.KvCacheWrite(KvCacheWriteCall(
            BufferRef(2 * i), BufferRef(2 * nbuf + 1), BufferRef(2 * nbuf), BufferRef(2 * i + 1),
            1, nbytes // 16, 0, 16)))
    for i in range(max(args.warmup, nbuf)):
        be.dispatch(calls[i % nbuf], ws)
    be.synchronize()
    ms = queued_ms(torch, lambda i: be.dispatch(calls[i % nbuf], ws), args.steps * 4)
    ms_t = queued_ms(torch, lambda i: dst[i % nbuf].copy_(src[i % nbuf]), args.steps * 4)
    res = {"bytes_per_launch": 2 * nbytes,
           "copy16_kernel": {"us": ms * 1e3, "gbs": 2 * nbytes / (ms / 1e3) / 1e9},
           "hip_memcpy_d2d": {"us": ms_t * 1e3, "gbs": 2 * nbytes / (ms_t / 1e3) / 1e9}}
    res["copy16_kernel"]["roofline"] = roofline("hbm", res["copy16_kernel"]["gbs"], HBM_PEAK_GBS,
                                                "GB/s", profiled_traffic("copy16_64M"))
    rep["copy"] = res
    return res


# ------------------------------------------------- quantized-weight GEMV ----
def bench_w8a8(torch, be, args, rep):
    """MatMulDequant's output-major W8A8 GEMV (the decode projection over a
    quantized weight) at the reference's DRAM-streaming decode shape
    (crates/hologram-bench/examples/gemv_micro.rs: m=1, k=2048, n=262144;
    the i8 weight is 537 MB), for the i8 / i4 / e8cb tiers, and the i8 tier
    at m=16 over a 64 MB weight (BENCHMARKS.md's blocked-prefill table).
    GMAC/s = m*k*n per second; HBM bytes = weight + A + scales + output.
    Weights rotate over >= 512 MiB so the 256 MiB last-level cache holds none."""
    import numpy as np
    from hologram_amd import (DTYPE_E8CB, DTYPE_I4, DTYPE_I8, BufferRef, DeviceWorkspace,
                              KernelCall, MatMulDequantCall)
    res = {}
    cases = [("i8_decode", DTYPE_I8, 1, 2048, 262144), ("i4_decode", DTYPE_I4, 1, 2048, 262144),
             ("e8cb_decode", DTYPE_E8CB, 1, 2048, 262144), ("i8_m16_64MB", DTYPE_I8, 16, 2048, 32768)]
    for name, tier, m, k, n in cases:
        wbytes = {DTYPE_I8: k * n, DTYPE_I4: k * n // 2, DTYPE_E8CB: k * n // 8}[tier]
        nbuf = max(1, -(-(512 << 20) // wbytes))
        ws = DeviceWorkspace()
        gen = torch.Generator(device="cuda").manual_seed(args.seed)
        a = torch.randn(m * k, generator=gen, device="cuda", dtype=torch.float32)
        scales = torch.rand(n, generator=gen, device="cuda", dtype=torch.float32) * 0.01
        zps = torch.zeros(n, dtype=torch.int32, device="cuda")
        cb = torch.randint(-127, 128, (2048,), generator=gen, device="cuda",
                           dtype=torch.int32).to(torch.int8)
        out = torch.empty(m * n, dtype=torch.float32, device="cuda")
        for s_, t in ((0, a), (2, scales), (3, zps), (4, out), (5, cb)):
            ws.bind(s_, t)
        calls = []
        for i in range(nbuf):
            w = torch.randint(0, 256, (wbytes,), generator=gen, device="cuda",
                              dtype=torch.int32).to(torch.uint8)
            ws.bind(10 + i, w)
            calls.append(KernelCall.MatMulDequant(MatMulDequantCall(
                BufferRef(0), BufferRef(10 + i), BufferRef(2), BufferRef(3), BufferRef(4), m, k, n,
                channels=n, inner=1, quant_dtype=tier, bq_omajor=True, act_quant=1,
                codebook=BufferRef(5) if tier == DTYPE_E8CB else BufferRef(0xFFFFFFFF))))
        for i in range(max(args.warmup, nbuf)):
            be.dispatch(calls[i % nbuf], ws)
        be.synchronize()
        ms = queued_ms(torch, lambda i: be.dispatch(calls[i % nbuf], ws), args.steps * 2)
        be.synchronize()
        alg = wbytes + m * k * 4 + n * 4 + m * n * 4
        gbs = alg / (ms / 1e3) / 1e9
        res[name] = {"m": m, "k": k, "n": n, "us": ms * 1e3,
                     "gmac_s": m * k * n / (ms / 1e3) / 1e9,
                     "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s",
                                          profiled_traffic(f"w8a8_{name}"))}
        del calls, ws
        torch.cuda.empty_cache()
    res["reference_published"] = {"i8_decode_gmac_s": 14.4, "i4_decode_gmac_s": 13.1,
                                  "e8cb_decode_gmac_s": 27.0,
                                  "machine": "AMD EPYC 7763 4c/8t AVX2, single thread "
                                             "(BENCHMARKS.md:30-37)"}
    if not args.no_cpu:
        import oracle
        k, n = 2048, 262144 // 16               # a 1/16 column slice of the decode shape
        rng = np.random.default_rng(args.seed)
        a = rng.standard_normal(k).astype(np.float32)
        w = rng.integers(-128, 128, k * n).astype(np.int8)
        sc = rng.uniform(0, 0.01, n).astype(np.float32)
        sec, reps, _ = cpu_time(lambda: oracle.matmul_i8_pc_omajor(a, w, sc, 1, k, n), 3.0)
        g = k * n / sec / 1e9
        res["cpu_baseline"] = {"value": g, "unit": "GMAC/s", "cores": 1, "kind": "port",
                               "sample": f"i8 m=1 k={k} n={n} (1/16 of n): x{reps} 1thr"}
    rep["w8a8"] = res
    return res


def rounded(x, sig=4):
    """Floats rounded to `sig` significant digits, recursively, so the one
    JSON line stays short enough for a log tail to hold it whole."""
    if isinstance(x, float):
        if x != x or x in (float("inf"), float("-inf")) or x == 0.0:
            return x
        return float(f"{x:.{sig}g}")
    if isinstance(x, dict):
        return {k: rounded(v, sig) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return [rounded(v, sig) for v in x]
    return x


def _n(x):
    """Four significant digits, without an exponent for large figures."""
    return f"{x:.0f}" if abs(x) >= 1e4 else f"{x:.4g}"


def _pct(rl):
    return f"{100 * rl['frac']:.1f}%"


def _tr(rl, alg):
    """Profiled HBM bytes over algorithmic bytes, when a counter pass exists."""
    t = rl.get("traffic")
    return f" tr{t / alg:.2f}" if t and alg else ""


def _cpu(cb):
    st = cb.get("single_thread")
    return f"{_n(cb['value'])}{cb['unit']}" + (f" ({_n(st)} 1thr)" if st else "")


def compact_components(rep):
    """One short string per leg's figure: time per call, rate, the fraction of
    MI355X's peak for its bound (HBM 8 TB/s, or dense MFMA), the profiled
    traffic ratio (tr: HBM bytes / algorithmic bytes) and the cpu_baseline.
    The whole record stays about 1.5 KB and is printed last on the line, so a
    log tail of 2000 characters holds every leg."""
    comps = compact_full(rep)
    out = {"key": "us/call, rate, % of peak (hbm 8 TB/s; mfma bf16 2.5 / f32 0.157 PF), "
                  "tr = HBM/alg bytes, cpu = cpu_baseline (gemm: TF/s, 16 threads)"}
    if "c1_lut_bf16_16M" in comps:
        c = comps["c1_lut_bf16_16M"]
        d = {k: f"{v['us']:.4g}us {_n(v['gelem_s'])}Gelem/s {_pct(v['roofline'])}hbm"
                f"{_tr(v['roofline'], 2 * 16 * 2 ** 20 * 2)}"
             for k, v in c.items() if k != "cpu_baseline"}
        if "cpu_baseline" in c:
            d["cpu"] = _cpu(c["cpu_baseline"])
        out["c1_lut_bf16_16M"] = d
    if "copy_ceiling_64MiB" in comps:
        c = comps["copy_ceiling_64MiB"]
        out["copy_64MiB"] = (f"{c['us']:.4g}us {_pct(c['roofline'])}hbm "
                             f"hipMemcpy {c['hip_memcpy_us']:.4g}us")
    if "c3_kv_append" in comps:
        c = comps["c3_kv_append"]
        d = {"copy": f"{c['copy']['us_per_step']:.4g}us/step {_pct(c['copy']['roofline'])}hbm",
             "in_place": f"{c['in_place']['us_per_step']:.4g}us/step "
                         f"{c['in_place']['vs_launch_floor']:.3g}x the {c['launch_floor_us']:.3g}us launch floor"}
        if "cpu_baseline" in c:
            d["cpu"] = _cpu(c["cpu_baseline"])
        out["c3_kv_append"] = d
    if "c2_gemm" in comps:
        d = {}
        for k, v in comps["c2_gemm"].items():
            rl = v["roofline"]
            parts = [f"{v['us']:.4g}us", f"{rl['achieved']:.4g}{'TF' if rl['unit'] == 'TFLOP/s' else 'GB/s'}",
                     _pct(rl) + ("mfma" if rl["unit"] == "TFLOP/s" else "hbm")]
            if "hipblaslt_tflops" in v:
                parts.append(f"hipblaslt {v['hipblaslt_tflops']:.4g}TF")
            if "launches_per_product" in v:
                parts.append(f"{v['launches_per_product']:.3g} launch")
            if "cpu_baseline" in v:
                parts.append(f"cpu {_n(v['cpu_baseline']['value'])}")
            d[k.replace("1024x1024x1024", "1024^3").replace("4096x4096x4096", "4096^3")
               .replace("8192x8192x8192", "8192^3")] = " ".join(parts)
        out["c2_gemm"] = d
    if "w8a8_gemv" in comps:
        c = comps["w8a8_gemv"]
        d = {k: f"{v['us']:.4g}us {_n(v['gmac_s'])}GMAC/s {_pct(v['roofline'])}hbm"
             for k, v in c.items() if k != "cpu_baseline"}
        if "cpu_baseline" in c:
            d["cpu"] = _cpu(c["cpu_baseline"])
        out["w8a8_gemv"] = d
    if "c5_e2e_1b" in comps:
        c = comps["c5_e2e_1b"]
        d = {}
        if "decode_ms_per_step" in c:
            d["decode"] = (f"{c['decode_ms_per_step']:.4g}ms/step {_n(c['decode_tok_s'])}tok/s "
                           f"{_pct(c['roofline'])}hbm")
        if "prefill_ms" in c:
            d["prefill"] = (f"{c['prefill_ms']:.4g}ms {_n(c['prefill_tok_s'])}tok/s "
                            f"{_pct(c['prefill_roofline'])}mfma")
        if "decode_walk" in c:
            d["walk"] = f"{c['decode_walk']['calls']} calls, {c['decode_walk']['fused_groups']} fused"
        if "cpu_baseline" in c:
            d["cpu"] = _cpu(c["cpu_baseline"])
        out["c5_e2e_1b"] = d
    return out


def compact_full(rep):
    comps = {}
    if "lut" in rep:
        cp = rep.get("copy", {}).get("copy16_kernel", {}).get("us")
        lut = {}
        for k, v in rep["lut"].items():
            lut[k] = {"gelem_s": v["gelem_s"], "us": v["us"],
                      "roofline": roofline("hbm", v["hbm_gbs"], HBM_PEAK_GBS, "GB/s",
                                           profiled_traffic("lut_gather_bf16_16M"))}
            if cp:
                lut[k]["vs_copy"] = cp / v["us"]
        if "lut_cpu" in rep:
            lut["cpu_baseline"] = rep["lut_cpu"]
        comps["c1_lut_bf16_16M"] = lut
    if "copy" in rep:
        c = rep["copy"]
        comps["copy_ceiling_64MiB"] = {"us": c["copy16_kernel"]["us"],
                                       "roofline": c["copy16_kernel"]["roofline"],
                                       "hip_memcpy_us": c["hip_memcpy_d2d"]["us"]}
    if "kv" in rep:
        kv = rep["kv"]
        comps["c3_kv_append"] = {
            "copy": {k: kv["copy"][k] for k in ("us_per_step", "launches_per_step", "roofline")
                     if k in kv["copy"]},
            "in_place": {k: kv["in_place"][k] for k in ("us_per_step", "vs_launch_floor",
                                                        "roofline")},
            "launch_floor_us": kv["launch_floor_us_per_kernel"]}
        if "cpu_baseline" in kv:
            comps["c3_kv_append"]["cpu_baseline"] = kv["cpu_baseline"]
    if "gemm" in rep:
        g = {}
        for k, v in rep["gemm"].items():
            g[k] = {"us": v["ms"] * 1e3 if "ms" in v else v["us"], "roofline": v["roofline"]}
            if "launches_per_product" in v:
                g[k]["launches_per_product"] = v["launches_per_product"]
            if "hipblaslt_tflops" in v:
                g[k]["hipblaslt_tflops"] = v["hipblaslt_tflops"]
            if "cpu_baseline" in v:
                g[k]["cpu_baseline"] = v["cpu_baseline"]
        comps["c2_gemm"] = g
    if "w8a8" in rep:
        w = {k: {"us": v["us"], "gmac_s": v["gmac_s"], "roofline": v["roofline"]}
             for k, v in rep["w8a8"].items() if isinstance(v, dict) and "us" in v}
        if "cpu_baseline" in rep["w8a8"]:
            w["cpu_baseline"] = rep["w8a8"]["cpu_baseline"]
        comps["w8a8_gemv"] = w
    if "e2e" in rep:
        e = rep["e2e"]
        comps["c5_e2e_1b"] = {k: e[k] for k in (
            "decode_tok_s", "decode_ms_per_step", "prefill_tok_s", "prefill_ms", "roofline",
            "prefill_roofline", "decode_walk", "cpu_baseline") if k in e}
    return comps


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    from hologram_amd import HipBackend
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device"}))
        sys.exit(1)
    be = HipBackend(0, torch.cuda.current_stream().cuda_stream)
    only = set(args.only.split(","))
    rep = {}
    t_all = time.perf_counter()
    if "attn" in only:
        bench_attn(torch, be, args, rep)
        torch.cuda.empty_cache()
    if "lut" in only:
        bench_lut(torch, be, args, rep)
        torch.cuda.empty_cache()
    if "copy" in only:
        bench_copy(torch, be, args, rep)
        torch.cuda.empty_cache()
    if "kv" in only:
        bench_kv(torch, be, args, rep)
        torch.cuda.empty_cache()
    if "gemm" in only:
        bench_gemm(torch, be, args, rep)
        torch.cuda.empty_cache()
    if "w8a8" in only:
        bench_w8a8(torch, be, args, rep)
        torch.cuda.empty_cache()
    if "e2e" in only:
        bench_e2e(torch, be, args, rep)
    be.close()

    attn = rep.get("attn")
    line = {
        "metric": METRIC,
        "value": attn["tok_s"] if attn else None,
        "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": attn["ms"] if attn else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": ("int8 KV, bf16 Q/out, fp32 softmax; QK on int8 MFMA with Q as a 15-bit "
                  "integer per head (exact int8 halves), P x V on f16 MFMA"),
        "data": "synthetic (seeded N(0,1) K/V with 2% x20 outlier channels, quantized by the "
                "int8 append op; seeded ragged lengths)",
        "config": {"workload": "config 4: GQA decode attention over int8 KV", "batch": 32,
                   "heads": 32, "kv_heads": 8, "head_dim": 128, "bucket": 32768,
                   "len_dist": "U[512, 32768]", "sum_len": attn["sum_len"] if attn else None},
    }
    if attn:
        line["roofline"] = roofline("hbm", attn["hbm_gbs"], HBM_PEAK_GBS, "GB/s",
                                    profiled_traffic("decode_attn_i8_config4"),
                                    "attn_split_kernel+attn_merge_kernel")
        line["alg_bytes"] = attn["alg_bytes"]
    if "attn_cpu" in rep:
        line["cpu_baseline"] = rep["attn_cpu"]
    if not args.no_cpu:
        import oracle
        line["host"] = oracle.host_info()
    line["timing"] = ("headline and components: HIP events around back-to-back calls queued "
                      "behind a spin kernel (GPU time per call)")
    if attn:
        line["ms_events_per_dispatch"] = attn["ms_events_per_dispatch"]
        line["wall_ms_per_step"] = attn["wall_ms_per_step"]
    line["bench_wall_s"] = time.perf_counter() - t_all
    line = rounded(line)
    line["components"] = compact_components(rep)   # last: a log tail keeps every leg
    print(json.dumps(line, separators=(",", ":")))


if __name__ == "__main__":
    main()
