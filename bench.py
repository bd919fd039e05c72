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
    ap.add_argument("--cpu-configs", action="store_true",
                    help="time the reference's CPU path (oracle, one thread) on every BASELINE config and exit")
    ap.add_argument("--workload", choices=("fused_chain", "copy", "transfer", "matmul", "config", "torch_ceilings"),
                    default="fused_chain",
                    help="copy: a plain 2^28-float copy kernel, the calibration run for rocprofv3 byte counters; "
                         "transfer: host<->device copy rates (pageable and page-locked host memory); "
                         "matmul: the 4096^3 fp32 GEMM alone, for rocprofv3 MFMA counters; "
                         "config: one of the extra configs alone (--config), for per-kernel profiles; "
                         "torch_ceilings: ROCm PyTorch's own kernels on configs 1 and 3's shapes, in a process "
                         "that never loads this library (independent same-box ceilings)")
    ap.add_argument("--config", choices=("relu_bias", "broadcast_strided", "reduce_vjp", "matmul", "matmul_shapes",
                                         "mlp"),
                    default="broadcast_strided", help="the extra config --workload config runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2

    if args.workload == "torch_ceilings":
        # Loaded by path: importing the trs_backend package would load libtrs_hip.so.
        import importlib.util
        spec = importlib.util.spec_from_file_location(
            "torch_ceilings", ROOT / "pytorch-rs_amd" / "trs_backend" / "torch_ceilings.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        return mod.main()
    ensure_built()
    if args.cpu_configs:
        return cpu_configs()
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
    if args.workload == "transfer":
        return transfer_rates()
    if args.workload == "matmul":
        return matmul_only(args)
    if args.workload == "config":
        from trs_backend import bench_configs
        print(json.dumps(getattr(bench_configs, args.config)(log)), flush=True)
        return 0
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

    # Peaks: the published figures, and the FP32 MFMA rate re-derived from this
    # device's CU count and engine clock (256 FLOP per clock per CU).
    derived_tflops = cus.value * clk.value * 1e3 * 256 / 1e12
    extra = {"peaks": {"hbm_GBps_published": HBM_PEAK_GBS, "fp32_mfma_TFLOPS_published": FP32_MFMA_PEAK_TFLOPS,
                       "fp32_mfma_TFLOPS_derived": round(derived_tflops, 1), "cu_count": cus.value,
                       "engine_clock_khz": clk.value},
             "fused_chain": {"kernel_us_avg_timed_region": kern_ms * 1e3,
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
        # Ceilings of the same launch shape: x*y + z (the same bytes, no exp)
        # and a plain 1 GiB copy (half the bytes), both flat one-shot kernels.
        kid_fma = ctypes.c_uint64()
        fma_ir = "in f32\nin f32\nin f32\nmul %0 %1\nadd %3 %2\nout %4\n"
        check(abi.lib.trs_fusion_compile(fma_ir.encode(), len(fma_ir), ctypes.byref(kid_fma)))
        from trs_backend.timing import time_region
        fma_ms = time_region(lambda: check(abi.lib.trs_fusion_launch(kid_fma, 3, ptrs, lays, dout.ptr, ctypes.byref(lay))),
                             reps=args.steps, warmup=2)
        copy_ms = time_region(lambda: check(abi.lib.trs_unary_f32(3, dx.ptr, ctypes.byref(lay), dout.ptr, ctypes.byref(lay))),
                              reps=args.steps, warmup=2)
        extra["fused_chain"]["same_bytes_no_exp_us"] = fma_ms * 1e3
        extra["fused_chain"]["same_bytes_no_exp_frac_hbm"] = bytes_per_step / (fma_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
        extra["fused_chain"]["copy_1GiB_us"] = copy_ms * 1e3
        extra["fused_chain"]["copy_1GiB_frac_hbm"] = 8 * n / (copy_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
        log(f"same-shape ceilings: x*y+z {fma_ms * 1e3:.1f} us, 1 GiB copy {copy_ms * 1e3:.1f} us")
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
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "traffic_source": "profiles/fused_chain_traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of "
                                       "this kernel, scaled by the same counters on a plain copy (not measured in "
                                       "this run)"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_configs() -> int:
    """The reference's single-threaded CPU path (oracle restatement) on every
    BASELINE config, each on a bounded sample scaled to the full size.  The
    matmuls use the reference's 4-row blocked loop (src/tensor.rs:3919-3966);
    the MLP runs at batch 64 and is scaled by 8192/64 (every GEMM is linear in
    the batch), plus the once-per-step .contiguous() of W1^T and W2^T."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    from trs_backend.configs import generate

    res = {}

    def timed(fn):
        t0 = time.perf_counter()
        out = fn()
        return time.perf_counter() - t0, out

    x, b = generate("relu_bias", "x"), generate("relu_bias", "b")
    t, _ = timed(lambda: O.unary_contig(O.RELU, O.row_broadcast(O.ADD, x, b, 4096, 4096)))
    res["relu_bias"] = {"seconds": t, "sample": "full [4096,4096]"}
    log(f"cpu relu_bias: {t:.3f} s")

    n = 1 << 25
    xs = [generate("fused_chain", k, count=n) for k in ("x", "y", "z")]
    t, _ = timed(lambda: O.unary_contig(O.RELU, O.scalar_contig(O.S_SUB, O.unary_contig(
        O.EXP, O.binary_contig(O.ADD, O.binary_contig(O.MUL, xs[0], xs[1]), xs[2])), 1.0)))
    res["fused_chain"] = {"seconds": t * 8, "sample": "2^25 of 2^28 elements, x8"}
    log(f"cpu fused_chain: {t * 8:.3f} s (scaled)")

    a = generate("broadcast_strided", "a")
    bb = generate("broadcast_strided", "b")
    c = generate("broadcast_strided", "c")
    osh = (64, 512, 1024)
    ocs = O.contiguous_strides(osh)

    def cfg2():
        s_ = O.binary(O.ADD, a, (64, 1, 1024), (1024, 1024, 1), 0, bb, (1, 512, 1024), (524288, 1024, 1), 0, osh, ocs)
        return O.binary(O.MUL, s_, osh, ocs, 0, c, osh, (524288, 1, 512), 0, osh, ocs)

    t, _ = timed(cfg2)
    res["broadcast_strided"] = {"seconds": t, "sample": "full [64,512,1024]"}
    log(f"cpu broadcast_strided: {t:.3f} s")

    A, B = generate("matmul", "A").reshape(4096, 4096), generate("matmul", "B").reshape(4096, 4096)
    t, _ = timed(lambda: O.matmul_row_blocked(A[:64], B))
    res["matmul_4096"] = {"seconds": t * 64, "sample": "64 of 4096 rows, x64",
                          "GFLOPS": 2 * 64 * 4096 * 4096 / t / 1e9}
    log(f"cpu matmul 4096^3: {t * 64:.1f} s (scaled)")
    Ab, Bb = generate("matmul", "Ab").reshape(32, 512, 512), generate("matmul", "Bb").reshape(32, 512, 512)
    t, _ = timed(lambda: [O.matmul_row_blocked(Ab[i], Bb[i]) for i in range(32)])
    res["matmul_batched_32x512"] = {"seconds": t, "sample": "full, 32 rank-2 calls"}
    log(f"cpu batched matmul: {t:.3f} s")

    bs = 64
    X = generate("mlp", "X", count=bs * 4096).reshape(bs, 4096)
    W1, W2 = generate("mlp", "W1").reshape(4096, 4096), generate("mlp", "W2").reshape(4096, 1024)
    mask = generate("mlp", "mask", count=bs * 4096).reshape(bs, 4096)
    s_ = np.float32(1 / 0.9)
    z1b, z2b = np.zeros(4096, np.float32), np.zeros(1024, np.float32)

    def transposes():
        w1t = O.unary(O.COPY, W1.ravel(), (4096, 4096), (1, 4096), 0, (4096, 1)).reshape(4096, 4096)
        w2t = O.unary(O.COPY, W2.ravel(), (1024, 4096), (1, 1024), 0, (4096, 1)).reshape(1024, 4096)
        return w1t, w2t

    t_tr, (w1t, w2t) = timed(transposes)

    def step():
        z1 = O.row_broadcast(O.ADD, O.matmul_row_blocked(X, W1).ravel(), z1b, bs, 4096)
        h = O.unary_contig(O.RELU, z1)
        d = O.mask_apply(h, mask.ravel(), s_).reshape(bs, 4096)
        out = O.row_broadcast(O.ADD, O.matmul_row_blocked(d, W2).ravel(), z2b, bs, 1024)
        O.sum_f32(out, (bs * 1024,))
        ones = np.ones((bs, 1024), np.float32)
        dd = O.matmul_row_blocked(ones, w2t)
        dt = O.unary(O.COPY, d.ravel(), (4096, bs), (1, 4096), 0, (bs, 1)).reshape(4096, bs)
        O.matmul_row_blocked(dt, ones)
        dh = O.mask_apply(O.scalar_contig(O.S_MUL, dd.ravel(), s_), mask.ravel(), np.float32(1.0))
        dz1 = O.relu_backward(z1, (bs, 4096), (4096, 1), 0, dh).reshape(bs, 4096)
        xt = O.unary(O.COPY, X.ravel(), (4096, bs), (1, 4096), 0, (bs, 1)).reshape(4096, bs)
        O.matmul_row_blocked(xt, dz1)
        O.matmul_row_blocked(dz1, w1t)

    t, _ = timed(step)
    res["mlp"] = {"seconds": t * (8192 // bs) + t_tr, "sample": f"batch {bs} of 8192, x{8192 // bs}, "
                  f"plus the W1^T/W2^T .contiguous() once ({t_tr:.2f} s)"}
    log(f"cpu mlp step: {res['mlp']['seconds']:.1f} s (scaled)")
    print(json.dumps({"cpu_configs": res, "threads": 1, "host_cpu": host_cpu_model(), "host_cores": host_cores(),
                      "libc": O.libc_version()}), flush=True)
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


def matmul_only(args) -> int:
    """The 4096^3 GEMM of the matmul config alone: `warmup` untimed launches,
    then `steps` launches between two HIP events on the library stream."""
    import ctypes

    from trs_backend import abi
    from trs_backend.abi import DeviceArray, check, layout_of
    from trs_backend.configs import generate
    from trs_backend.timing import time_region

    K = 4096
    dA, dB = DeviceArray.from_numpy(generate("matmul", "A")), DeviceArray.from_numpy(generate("matmul", "B"))
    dC = DeviceArray(K * K * 4)
    lay = layout_of((K, K))

    def mm():
        check(abi.lib.trs_matmul_f32(dA.ptr, ctypes.byref(lay), dB.ptr, ctypes.byref(lay), dC.ptr, ctypes.byref(lay)))

    ms = time_region(mm, reps=args.steps, warmup=args.warmup)
    tf = 2 * K ** 3 / (ms * 1e-3) / 1e12
    log(f"matmul 4096^3: {ms:.3f} ms avg over {args.steps} launches -> {tf:.1f} TFLOPS")
    print(json.dumps({"workload": "matmul_4096", "flop_per_launch": 2 * K ** 3, "ms_avg": ms, "TFLOPS": tf,
                      "frac_mfma_peak": tf / FP32_MFMA_PEAK_TFLOPS}), flush=True)
    return 0


def transfer_rates() -> int:
    """Host <-> device copy rates through trs_memcpy_h2d/d2h, for pageable numpy
    buffers (staged through the library's page-locked chunks above a few MiB)
    and for page-locked ones from trs_host_alloc (one DMA).  Median of five
    timed batches of back-to-back copies per size; every copy is checked."""
    import ctypes

    import numpy as np

    from trs_backend import abi
    from trs_backend.abi import DeviceArray, check

    def rate(fn, nbytes):
        fn()
        fn()
        reps = max(3, int(5e9 / nbytes))  # about 0.1 s per batch at 50 GB/s
        res = []
        for _ in range(5):
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            res.append(nbytes * reps / (time.perf_counter() - t0) / 1e9)
        return sorted(res)[2]

    rows = []
    for mib in (4, 16, 64, 256, 1024):
        nb = mib << 20
        src = np.random.default_rng(mib).integers(0, 256, nb, dtype=np.uint8)
        dev = DeviceArray(nb)
        out = np.empty(nb, np.uint8)
        h2d = rate(lambda: check(abi.lib.trs_memcpy_h2d(dev.ptr, ctypes.c_void_p(src.ctypes.data), nb)), nb)
        d2h = rate(lambda: check(abi.lib.trs_memcpy_d2h(ctypes.c_void_p(out.ctypes.data), dev.ptr, nb)), nb)
        if not np.array_equal(out, src):
            raise SystemExit(f"transfer of {mib} MiB through pageable memory changed the bytes")
        p = ctypes.c_void_p()
        check(abi.lib.trs_host_alloc(nb, ctypes.byref(p)))
        try:
            pin = np.ctypeslib.as_array((ctypes.c_uint8 * nb).from_address(p.value))
            pin[:] = src
            ph2d = rate(lambda: check(abi.lib.trs_memcpy_h2d(dev.ptr, p, nb)), nb)
            pin[:] = 0
            pd2h = rate(lambda: check(abi.lib.trs_memcpy_d2h(p, dev.ptr, nb)), nb)
            if not np.array_equal(pin, src):
                raise SystemExit(f"transfer of {mib} MiB through page-locked memory changed the bytes")
            del pin
        finally:
            check(abi.lib.trs_host_free(p))
        log(f"{mib:5d} MiB: pageable h2d {h2d:5.1f} d2h {d2h:5.1f} GB/s | page-locked h2d {ph2d:5.1f} "
            f"d2h {pd2h:5.1f} GB/s")
        rows.append({"MiB": mib, "pageable_h2d_GBps": round(h2d, 1), "pageable_d2h_GBps": round(d2h, 1),
                     "pinned_h2d_GBps": round(ph2d, 1), "pinned_d2h_GBps": round(pd2h, 1)})
    print(json.dumps({"workload": "host_transfer", "unit": "GB/s", "rows": rows}), flush=True)
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


def host_cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            return next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except Exception:
        return ""


def cpu_baseline(x, y, z, n, log):
    """The reference's CPU path (oracle restatement, one thread) on a bounded
    sample, with this process pinned to one core for the duration (restored
    afterwards; no re-launch)."""
    try:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O
    except Exception as exc:
        log(f"cpu baseline unavailable: {exc!r}")
        return None
    sample = 1 << 25
    xs, ys, zs = x[:sample], y[:sample], z[:sample]
    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[0]
    os.sched_setaffinity(0, {core})
    try:
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
    finally:
        os.sched_setaffinity(0, set(allowed))
    gbs = 16 * sample * reps / el / 1e9
    log(f"cpu baseline: {gbs:.2f} GB/s over {reps} x 2^25 elements in {el:.1f}s on core {core}")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "host_cpu": host_cpu_model(), "host_cores": len(allowed), "pinned_core": core,
            "sample": f"first 2^25 of the 2^28 elements, reference 5-pass chain (mul, add, exp, sub_scalar, relu), "
                      f"{reps} rep(s), {el:.1f}s, one thread pinned to core {core} of the {len(allowed)} this "
                      f"process may use, oracle built -O3 -march=x86-64 -ffp-contract=off"}


if __name__ == "__main__":
    sys.exit(main())
