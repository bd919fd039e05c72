#!/usr/bin/env python3
"""Benchmark of the MI355X pytorch-rs hot path.

Headline: the fused pointwise chain
relu(exp(x*y + z) - 1.0) over three contiguous fp32 tensors of 2^28
elements, U(-4,4), seed 1, as ONE hipRTC-compiled kernel.  A step is one
launch over the whole batch with inputs resident in HBM.  `value` is GB/s of
algorithmic traffic (16 B per element: three reads and one write).

Also reported under "extra" (not the headline): the same chain unfused
(five eager kernels), relu(x + b) (config 0), (a + b) * c.mT (config 2),
fp32 matmul 4096^3 and batched 32x512^3 (config 3) in TFLOPS, and the MLP
forward+backward (config 4) when the host engine is built.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--quick]
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
sys.path.insert(0, str(ROOT / "pytorch-rs_amd"))

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
METRIC = "fused pointwise GB/s (% of HBM peak); fp32 matmul TFLOPS (% of MFMA peak)"
CHAIN_IR = "in f32\nin f32\nin f32\nmul %0 %1\nadd %3 %2\nexp %4\nconst 0x3f800000\nsub %5 %6\nrelu %7\nout %8\n"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def ensure_built() -> None:
    lib = ROOT / "pytorch-rs_amd" / "lib" / "libtrs_hip.so"
    if not lib.exists():
        log("native libraries missing; building")
        import __graft_entry__
        __graft_entry__.build()


def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline only (no extra configs, no CPU baseline)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--workload", choices=("fused_chain", "copy"), default="fused_chain",
                    help="copy: a plain 2^28-float copy kernel, the calibration run for rocprofv3 byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2

    ensure_built()
    import ctypes

    import numpy as np

    from trs_backend import abi
    from trs_backend.abi import DeviceArray, check, layout_of
    from trs_backend.configs import generate
    from trs_backend.timing import time_launches

    check(abi.lib.trs_init())
    name = ctypes.create_string_buffer(256)
    cus, clk = ctypes.c_int(), ctypes.c_int()
    check(abi.lib.trs_device_info(name, 256, ctypes.byref(cus), ctypes.byref(clk)))
    log(f"device {name.value.decode()} CUs={cus.value} clock={clk.value} kHz")

    n = 1 << 28
    if args.workload == "copy":
        return copy_calibration(n, args)
    t0 = time.time()
    x, y, z = (generate("fused_chain", k, threads=min(16, host_cores())) for k in ("x", "y", "z"))
    log(f"generated 3 x 2^28 inputs in {time.time() - t0:.1f}s")
    dx, dy, dz = (DeviceArray.from_numpy(a) for a in (x, y, z))
    dout = DeviceArray(n * 4)
    lay = layout_of((n,))
    lays = (abi.Layout * 3)(lay, lay, lay)
    ptrs = (ctypes.c_void_p * 3)(dx.addr, dy.addr, dz.addr)
    kid = ctypes.c_uint64()
    check(abi.lib.trs_fusion_compile(CHAIN_IR.encode(), len(CHAIN_IR), ctypes.byref(kid)))
    compile_ms = ctypes.c_double()
    check(abi.lib.trs_fusion_compile_ms(kid, ctypes.byref(compile_ms)))

    def fused_step():
        check(abi.lib.trs_fusion_launch(kid, 3, ptrs, lays, dout.ptr, ctypes.byref(lay)))

    from trs_backend.timing import Event, stream

    for _ in range(args.warmup):
        fused_step()
    check(abi.lib.trs_synchronize())
    s = stream()
    ev0, ev1 = Event(), Event()
    t0 = time.perf_counter()
    ev0.record(s)
    for _ in range(args.steps):
        fused_step()
    ev1.record(s)
    check(abi.lib.trs_synchronize())
    wall = time.perf_counter() - t0
    bytes_per_step = 16 * n
    value = bytes_per_step * args.steps / wall / 1e9
    # The dominant (only) kernel's average duration over the timed region,
    # from HIP events on the stream it runs on.
    kern_ms = ev0.elapsed_ms(ev1) / args.steps
    achieved = bytes_per_step / (kern_ms * 1e-3) / 1e9
    ev = time_launches(fused_step, reps=max(10, args.steps), warmup=0)
    log(f"fused chain: {value:.0f} GB/s wall, kernel {kern_ms * 1e3:.1f} us avg -> {achieved:.0f} GB/s")

    # Checksum of a strided sample of the output (materialised result).
    out_sample = dout.to_numpy(count=n)[:: 4099]
    checksum = float(np.sum(out_sample, dtype=np.float64))

    extra = {"fused_chain": {"kernel_us_avg_timed_region": kern_ms * 1e3,
                             "kernel_us_median_single_launch": statistics.median(ev) * 1e3,
                             "kernel_us_min": min(ev) * 1e3, "kernel_us_max": max(ev) * 1e3,
                             "hiprtc_compile_ms": compile_ms.value, "output_sample_checksum": checksum}}

    if not args.quick and not args.no_extra:
        # Unfused: the reference's five passes as eager kernels (48 B/element moved).
        t1, t2 = DeviceArray(n * 4), DeviceArray(n * 4)

        def unfused_step():
            check(abi.lib.trs_binary_f32(2, dx.ptr, ctypes.byref(lay), dy.ptr, ctypes.byref(lay), t1.ptr,
                                         ctypes.byref(lay)))
            check(abi.lib.trs_binary_f32(0, t1.ptr, ctypes.byref(lay), dz.ptr, ctypes.byref(lay), t2.ptr,
                                         ctypes.byref(lay)))
            check(abi.lib.trs_unary_f32(0, t2.ptr, ctypes.byref(lay), t1.ptr, ctypes.byref(lay)))
            check(abi.lib.trs_binary_scalar_f32(1, t1.ptr, ctypes.byref(lay), ctypes.c_float(1.0), t2.ptr,
                                                ctypes.byref(lay)))
            check(abi.lib.trs_unary_f32(1, t2.ptr, ctypes.byref(lay), dout.ptr, ctypes.byref(lay)))

        uev = time_launches(unfused_step, reps=5, warmup=1)
        u_ms = statistics.median(uev)
        extra["fused_chain"]["unfused_eager_ms"] = u_ms
        extra["fused_chain"]["unfused_GBps_algorithmic"] = bytes_per_step / (u_ms * 1e-3) / 1e9
        extra["fused_chain"]["unfused_GBps_moved"] = 48 * n / (u_ms * 1e-3) / 1e9
        extra["fused_chain"]["fusion_speedup"] = u_ms / statistics.median(ev)
        del t1, t2
        log(f"unfused chain: {u_ms:.3f} ms")
        try:
            from trs_backend import bench_configs
            extra.update(bench_configs.run_all(log))
        except Exception as exc:  # report, never hide
            extra["extra_error"] = repr(exc)
            log(f"extra configs failed: {exc!r}")

    cpu = None
    if not args.quick and not args.no_cpu_baseline:
        cpu = cpu_baseline(x, y, z, n, log)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (Philox4x32-10, seed 1, U(-4,4))",
        "config": {"workload": "fused_chain: relu(exp(x*y + z) - 1.0), x,y,z contiguous f32 [2^28], one fused kernel",
                   "elements": n, "bytes_per_step": bytes_per_step, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


def copy_calibration(n: int, args) -> int:
    """Plain contiguous copy of n floats (8 B/element moved): reference point for the PMC byte counters."""
    import ctypes
    import statistics

    import numpy as np

    from trs_backend import abi
    from trs_backend.abi import DeviceArray, check, layout_of
    from trs_backend.timing import time_launches

    src = DeviceArray.from_numpy(np.arange(n, dtype=np.float32))
    dst = DeviceArray(n * 4)
    lay = layout_of((n,))

    def step():
        check(abi.lib.trs_unary_f32(3, src.ptr, ctypes.byref(lay), dst.ptr, ctypes.byref(lay)))

    ev = time_launches(step, reps=max(10, args.steps), warmup=args.warmup)
    ms = statistics.mean(ev)
    gbs = 8 * n / (ms * 1e-3) / 1e9
    log(f"copy: {ms * 1e3:.1f} us avg -> {gbs:.0f} GB/s")
    print(json.dumps({"workload": "copy_calibration", "elements": n, "bytes_per_launch": 8 * n,
                      "kernel_us_avg": ms * 1e3, "GBps": gbs}), flush=True)
    return 0


def read_traffic():
    """HBM bytes per launch of the fused chain kernel, from the committed rocprofv3 PMC summary."""
    p = ROOT / "profiles" / "fused_chain_traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("traffic_bytes_per_launch")
    except Exception:
        return None


def cpu_baseline(x, y, z, n, log):
    """The reference's CPU path (oracle restatement, one thread) on a bounded sample."""
    try:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O
    except Exception as exc:
        log(f"cpu baseline unavailable: {exc!r}")
        return None
    sample = 1 << 25
    xs, ys, zs = x[:sample], y[:sample], z[:sample]
    t0 = time.perf_counter()
    reps = 0
    while True:
        t = O.binary_contig(O.MUL, xs, ys)
        t = O.binary_contig(O.ADD, t, zs)
        t = O.unary_contig(O.EXP, t)
        t = O.scalar_contig(O.S_SUB, t, 1.0)
        t = O.unary_contig(O.RELU, t)
        reps += 1
        el = time.perf_counter() - t0
        if el > 10.0 or reps >= 200:
            break
    gbs = 16 * sample * reps / el / 1e9
    log(f"cpu baseline: {gbs:.2f} GB/s over {reps} x 2^25 elements in {el:.1f}s")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"first 2^25 of the 2^28 elements, reference 5-pass chain (mul, add, exp, sub_scalar, relu), "
                      f"{reps} rep(s), {el:.1f}s, oracle built -O3 -march=x86-64 -ffp-contract=off"}


if __name__ == "__main__":
    sys.exit(main())
