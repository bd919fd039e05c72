"""Secondary benchmark configurations reported under bench.py's "extra".

Each returns device-time figures measured with HIP events on the library
stream: the average over a region of back-to-back launches (the rate used
for GB/s and TFLOPS) and the median, min and max of single launches (the
dispersion).  Inputs of a size the 256 MB Infinity Cache could hold are
rotated over enough buffer sets that the streamed inputs alone total at
least 512 MiB, so the GB/s figures reflect HBM: outputs written with
non-temporal stores do not displace cached inputs, and with three 64 MiB
sets a plain copy measured 0.98 of the HBM peak out of that cache.  Launch
arguments are built once per set.  Every output is read back and summed in
float64 as a checksum of the materialised result.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import abi
from .abi import DeviceArray, check, layout_of
from .configs import generate
from .timing import time_launches, time_region

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3


def _spread(times_ms: list[float], scale: float = 1e3, unit: str = "us") -> dict:
    """Median, min and max of single-launch times (ms in), in `unit`."""
    t = sorted(times_ms)
    return {f"{unit}_median_single_launch": t[len(t) // 2] * scale, f"{unit}_min": t[0] * scale,
            f"{unit}_max": t[-1] * scale, "launches": len(t)}


def _checksum(d: DeviceArray, count: int) -> float:
    return float(np.sum(d.to_numpy(count=count), dtype=np.float64))


def _fusion(ir: str) -> int:
    kid = ctypes.c_uint64()
    check(abi.lib.trs_fusion_compile(ir.encode(), len(ir), ctypes.byref(kid)))
    return kid.value


class _FusedCall:
    """A fused launch with its ctypes arguments built once."""

    def __init__(self, kid, devs, lays, out, lo):
        n = len(devs)
        self.args = (kid, n, (ctypes.c_void_p * n)(*[d.addr for d in devs]), (abi.Layout * n)(*lays), out.ptr,
                     ctypes.byref(lo))
        self.keep = (devs, lays, out, lo)

    def __call__(self):
        check(abi.lib.trs_fusion_launch(*self.args))


# Back-to-back launches per timed region for the short pointwise kernels: the
# region opens with one host launch latency before the queue fills, so it is
# sized to span milliseconds and that latency adds well under 1% per launch.
SHORT_KERNEL_REPS = 200


def relu_bias(log, reps: int = SHORT_KERNEL_REPS, sets: int = 8) -> dict:
    """Config 0: relu(x + b), x [4096,4096], b [4096] row-broadcast, seed 0."""
    R = C = 4096
    x = generate("relu_bias", "x")
    b = generate("relu_bias", "b")
    xs = [DeviceArray.from_numpy(x) for _ in range(sets)]
    outs = [DeviceArray(R * C * 4) for _ in range(sets)]
    tmp = [DeviceArray(R * C * 4) for _ in range(sets)]
    db = DeviceArray.from_numpy(b)
    lx, lb = layout_of((R, C)), layout_of((C,))
    algo = 2 * R * C * 4 + C * 4
    i = [0]

    def eager():
        k = i[0] % sets
        i[0] += 1
        check(abi.lib.trs_binary_f32(0, xs[k].ptr, ctypes.byref(lx), db.ptr, ctypes.byref(lb), tmp[k].ptr,
                                     ctypes.byref(lx)))
        check(abi.lib.trs_unary_f32(1, tmp[k].ptr, ctypes.byref(lx), outs[k].ptr, ctypes.byref(lx)))

    # The IR torch_rs.fuse emits for relu(x + b) at these layouts: the
    # broadcast row b is declared first (loaded before the streamed x), and
    # the add still computes x + b.
    kid = _fusion("in f32\nin f32\nadd %1 %0\nrelu %2\nout %3\n")
    calls = [_FusedCall(kid, [db, xs[k]], [lb, lx], outs[k], lx) for k in range(sets)]

    def fused():
        k = i[0] % sets
        i[0] += 1
        calls[k]()

    # The ceiling of this launch shape: a plain copy of x (the product's COPY
    # op, one float4 per lane, 16,384 blocks -- the rows kernel's grid) over
    # the same buffer sets.
    ln = layout_of((R * C,))

    def copy():
        k = i[0] % sets
        i[0] += 1
        check(abi.lib.trs_unary_f32(3, xs[k].ptr, ctypes.byref(ln), tmp[k].ptr, ctypes.byref(ln)))

    # The runtime's own device-to-device copy (hipMemcpyAsync) of the same bytes.
    def d2d():
        k = i[0] % sets
        i[0] += 1
        check(abi.lib.trs_memcpy_d2d(tmp[k].ptr, xs[k].ptr, R * C * 4))

    e = time_region(eager, reps)
    f = time_region(fused, reps)
    cp = time_region(copy, reps)
    dd = time_region(d2d, reps)
    spread = _spread(time_launches(fused, 20))
    log(f"relu_bias: eager {e * 1e3:.1f} us, fused {f * 1e3:.1f} us, same-shape copy {cp * 1e3:.1f} us, "
        f"hipMemcpyAsync d2d {dd * 1e3:.1f} us")
    return {"relu_bias": {"algorithmic_bytes": algo, "eager_us": e * 1e3, "fused_us": f * 1e3,
                          "eager_GBps": algo / (e * 1e-3) / 1e9, "fused_GBps": algo / (f * 1e-3) / 1e9,
                          "fused_frac_hbm": algo / (f * 1e-3) / 1e9 / HBM_PEAK_GBS, "fused_spread": spread,
                          "copy_same_shape_us": cp * 1e3, "copy_same_shape_frac_hbm": 2 * R * C * 4 / (cp * 1e-3) / 1e9 / HBM_PEAK_GBS,
                          "fused_time_over_copy": f / cp, "memcpy_d2d_same_shape_us": dd * 1e3,
                          "memcpy_d2d_same_shape_frac_hbm": 2 * R * C * 4 / (dd * 1e-3) / 1e9 / HBM_PEAK_GBS,
                          "buffer_sets": sets,
                          "output_checksum": _checksum(outs[(i[0] - 1) % sets], R * C)}}


def broadcast_strided(log, reps: int = SHORT_KERNEL_REPS, sets: int = 4) -> dict:
    """Config 2: (a + b) * c.mT, a [64,1,1024], b [1,512,1024], c [64,1024,512]."""
    B, M, N = 64, 512, 1024
    a = generate("broadcast_strided", "a")
    b = generate("broadcast_strided", "b")
    c = generate("broadcast_strided", "c")
    da, db = DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)
    dcs = [DeviceArray.from_numpy(c) for _ in range(sets)]
    outs = [DeviceArray(B * M * N * 4) for _ in range(sets)]
    tmps = [DeviceArray(B * M * N * 4) for _ in range(sets)]
    la, lb = layout_of((B, 1, N)), layout_of((1, M, N))
    lc = layout_of((B, M, N), (N * M, 1, M))
    lo = layout_of((B, M, N))
    algo = (B * N + M * N + B * N * M + B * M * N) * 4
    i = [0]

    def eager():
        k = i[0] % sets
        i[0] += 1
        check(abi.lib.trs_binary_f32(0, da.ptr, ctypes.byref(la), db.ptr, ctypes.byref(lb), tmps[k].ptr,
                                     ctypes.byref(lo)))
        check(abi.lib.trs_binary_f32(2, tmps[k].ptr, ctypes.byref(lo), dcs[k].ptr, ctypes.byref(lc), outs[k].ptr,
                                     ctypes.byref(lo)))

    kid = _fusion("in f32\nin f32\nin f32\nadd %0 %1\nmul %3 %2\nout %4\n")
    calls = [_FusedCall(kid, [da, db, dcs[k]], [la, lb, lc], outs[k], lo) for k in range(sets)]

    def fused():
        k = i[0] % sets
        i[0] += 1
        calls[k]()

    # c.mT copied to a contiguous tensor: the transposing kernel with no
    # broadcast operands, the access pattern's own cost.
    def transpose_copy():
        k = i[0] % sets
        i[0] += 1
        check(abi.lib.trs_unary_f32(3, dcs[k].ptr, ctypes.byref(lc), tmps[k].ptr, ctypes.byref(lo)))

    # The same 128 MiB read and written in order: c copied flat (the COPY op
    # on contiguous layouts), and through the runtime's hipMemcpyAsync.
    lflat = layout_of((B * M * N,))

    def flat_copy():
        k = i[0] % sets
        i[0] += 1
        check(abi.lib.trs_unary_f32(3, dcs[k].ptr, ctypes.byref(lflat), tmps[k].ptr, ctypes.byref(lflat)))

    def d2d():
        k = i[0] % sets
        i[0] += 1
        check(abi.lib.trs_memcpy_d2d(tmps[k].ptr, dcs[k].ptr, B * M * N * 4))

    e = time_region(eager, reps)
    f = time_region(fused, reps)
    tc = time_region(transpose_copy, reps)
    fc = time_region(flat_copy, reps)
    dd = time_region(d2d, reps)
    spread = _spread(time_launches(fused, 20))
    log(f"broadcast_strided: eager {e * 1e3:.1f} us, fused {f * 1e3:.1f} us, c.mT copy {tc * 1e3:.1f} us, "
        f"flat copy {fc * 1e3:.1f} us, hipMemcpyAsync d2d {dd * 1e3:.1f} us")
    return {"broadcast_strided": {"algorithmic_bytes": algo, "eager_us": e * 1e3, "fused_us": f * 1e3,
                                  "eager_GBps": algo / (e * 1e-3) / 1e9, "fused_GBps": algo / (f * 1e-3) / 1e9,
                                  "fused_frac_hbm": algo / (f * 1e-3) / 1e9 / HBM_PEAK_GBS, "fused_spread": spread,
                                  "transpose_copy_us": tc * 1e3,
                                  "transpose_copy_frac_hbm": 2 * B * M * N * 4 / (tc * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                  "flat_copy_us": fc * 1e3,
                                  "flat_copy_frac_hbm": 2 * B * M * N * 4 / (fc * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                  "memcpy_d2d_us": dd * 1e3,
                                  "memcpy_d2d_frac_hbm": 2 * B * M * N * 4 / (dd * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                  "buffer_sets": sets, "output_checksum": _checksum(outs[(i[0] - 1) % sets], B * M * N)}}


# MFMA-bound kernels reach steady clocks only after ~25 ms of sustained
# work on the MI355X (a 4096^3 GEMM runs ~14% slower in its first calls), so
# the GEMM figures are timed after a warm-up of that length.
GEMM_WARMUP_MS = 30.0


def matmul(log, reps: int = 20) -> dict:
    """Config 3: A @ B 4096^3 and batched [32,512,512]^2, fp32, N(0, 1/sqrt(K)), seed 3."""
    out = {}
    K = 4096
    A, Bm = generate("matmul", "A"), generate("matmul", "B")
    dA, dB, dC = DeviceArray.from_numpy(A), DeviceArray.from_numpy(Bm), DeviceArray(K * K * 4)
    l = layout_of((K, K))

    def mm():
        check(abi.lib.trs_matmul_f32(dA.ptr, ctypes.byref(l), dB.ptr, ctypes.byref(l), dC.ptr, ctypes.byref(l)))

    med = time_region(mm, reps, warmup=int(GEMM_WARMUP_MS / 1.0))
    t = time_launches(mm, reps)
    tf = 2 * K ** 3 / (med * 1e-3) / 1e12
    out["matmul_4096"] = {"ms_avg": med, "ms_min_single_launch": min(t), "TFLOPS": tf,
                          "frac_mfma_peak": tf / FP32_MFMA_PEAK_TFLOPS, "spread": _spread(t, 1.0, "ms"),
                          "output_checksum": _checksum(dC, K * K)}
    log(f"matmul 4096^3: {med:.3f} ms, {tf:.1f} TFLOPS")
    Ab, Bb = generate("matmul", "Ab"), generate("matmul", "Bb")
    dAb, dBb, dCb = DeviceArray.from_numpy(Ab), DeviceArray.from_numpy(Bb), DeviceArray(32 * 512 * 512 * 4)
    lb = layout_of((32, 512, 512))

    def bmm():
        check(abi.lib.trs_matmul_f32(dAb.ptr, ctypes.byref(lb), dBb.ptr, ctypes.byref(lb), dCb.ptr,
                                     ctypes.byref(lb)))

    med = time_region(bmm, reps * 3, warmup=int(GEMM_WARMUP_MS / 0.08))
    t = time_launches(bmm, reps * 3)
    tf = 2 * 32 * 512 ** 3 / (med * 1e-3) / 1e12
    out["matmul_batched_32x512"] = {"ms_avg": med, "ms_min_single_launch": min(t), "TFLOPS": tf,
                                    "frac_mfma_peak": tf / FP32_MFMA_PEAK_TFLOPS, "spread": _spread(t, 1.0, "ms"),
                                    "output_checksum": _checksum(dCb, 32 * 512 * 512)}
    log(f"batched matmul 32x512^3: {med:.3f} ms, {tf:.1f} TFLOPS")
    return out


# (name, M, K, N, A transposed, B transposed, bound): outputs with a short
# side (matrix-vector products and small-batch linear layers, x @ W or
# x @ W.mT), which stream the long operand once and are HBM-bound, shapes
# whose square tiles alone would leave CUs idle (K split over them), ragged
# squares, and tile counts whose last round leaves CUs idle (stream-K).
MATMUL_SHAPES = [
    ("matvec [1,4096]@[4096,4096]", 1, 4096, 4096, False, False, "hbm"),
    ("matvec [1,4096]@W.mT", 1, 4096, 4096, False, True, "hbm"),
    ("[8,4096]@[4096,4096]", 8, 4096, 4096, False, False, "hbm"),
    ("[32,4096]@W.mT", 32, 4096, 4096, False, True, "hbm"),
    ("[4096,4096]@[4096,1]", 4096, 4096, 1, False, False, "hbm"),
    ("matvec [1,16384]@W.mT", 1, 16384, 16384, False, True, "hbm"),
    ("[64,4096]@[4096,4096]", 64, 4096, 4096, False, False, "mfma"),
    ("1000^3", 1000, 1000, 1000, False, False, "mfma"),
    ("2047^3", 2047, 2047, 2047, False, False, "mfma"),
    ("4095^3", 4095, 4095, 4095, False, False, "mfma"),
    ("4097^3", 4097, 4097, 4097, False, False, "mfma"),
    # tile counts that leave CUs idle in whole rounds (stream-K)
    ("[512,4096]@[4096,4096]", 512, 4096, 4096, False, False, "mfma"),
    ("3072^3", 3072, 3072, 3072, False, False, "mfma"),
    ("5000^3", 5000, 5000, 5000, False, False, "mfma"),
    ("6144^3", 6144, 6144, 6144, False, False, "mfma"),
]


def matmul_shapes(log, reps: int = 100) -> dict:
    """The matmul beyond the square configs: each shape of MATMUL_SHAPES with
    its operands filled with constants (fp32 MFMA timing does not depend on
    the values) and rotated over enough sets that they total at least 512 MiB.
    Reports the average per call over a back-to-back region (the kernel and,
    for a split K, the pass that sums the slices), the rate against the
    shape's bound (algorithmic bytes, every operand read once and C written
    once, for HBM; 2*M*N*K for MFMA) and the plan trs_matmul_plan_f32 gives."""
    out = {}
    for name, M, K, N, ta, tb, bound in MATMUL_SHAPES:
        per_set = (M * K + K * N) * 4
        nsets = max(1, min(8, -(-(512 << 20) // per_set)))
        la = layout_of((M, K), (1, M) if ta else (K, 1))
        lb = layout_of((K, N), (1, K) if tb else (N, 1))
        lc = layout_of((M, N))
        sets = []
        for _ in range(nsets):
            a, b, c = DeviceArray(M * K * 4), DeviceArray(K * N * 4), DeviceArray(M * N * 4)
            check(abi.lib.trs_fill_f32(a.ptr, M * K, 0.5))
            check(abi.lib.trs_fill_f32(b.ptr, K * N, 0.25))
            sets.append((a.ptr, ctypes.byref(la), b.ptr, ctypes.byref(lb), c.ptr, ctypes.byref(lc), (a, b, c)))
        tm, tn, tk, sp, bl = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64()
        check(abi.lib.trs_matmul_plan_f32(*sets[0][:6], ctypes.byref(tm), ctypes.byref(tn), ctypes.byref(tk),
                                          ctypes.byref(sp), ctypes.byref(bl)))
        i = [0]

        def call():
            s = sets[i[0] % nsets]
            i[0] += 1
            check(abi.lib.trs_matmul_f32(*s[:6]))

        ms = time_region(call, reps, warmup=10)
        us = ms * 1e3
        entry = {"M": M, "K": K, "N": N, "a_transposed": ta, "b_transposed": tb, "us_avg": us,
                 "plan": {"tile": [tm.value, tn.value, tk.value], "splits": sp.value, "blocks": bl.value},
                 "input_sets": nsets, "bound": bound}
        if bound == "hbm":
            gbs = (M * K + K * N + M * N) * 4 / (us * 1e-6) / 1e9
            entry.update({"GBs": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS})
            rate = f"{gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.2f})"
        else:
            tf = 2 * M * N * K / (us * 1e-6) / 1e12
            entry.update({"TFLOPS": tf, "frac_mfma_peak": tf / FP32_MFMA_PEAK_TFLOPS})
            rate = f"{tf:.1f} TFLOPS ({tf / FP32_MFMA_PEAK_TFLOPS:.2f})"
        out[name] = entry
        log(f"matmul {name}: {us:.1f} us, {rate}, tile {tm.value}x{tn.value}x{tk.value} splits {sp.value}")
        del sets
    return out


def mlp(log, reps: int = 20) -> dict:
    """Config 4: 2-layer MLP forward+backward through the torch_rs API on the device."""
    from . import mlp_bench
    return {"mlp": mlp_bench.run(log, reps)}


def reduce_vjp(log, reps: int = 50) -> dict:
    """Broadcast-reduction VJPs, each a set of ordered chains of adds:
    the bias gradient [8192,4096] -> [4096] (trs_reduce_to_shape_f32, 4096
    chains of 8192) and config 2's operand a [64,1,1024] through the mul VJP
    against c.mT (trs_mul_backward_f32: up * other added along the 512 rows,
    65,536 chains).  GB/s counts the bytes read (up, and other) and written."""
    rng = np.random.default_rng(12)
    out = {}
    R, C = 8192, 4096
    # 4 inputs: 512 MiB rotated, twice the 256 MB MALL
    ups = [DeviceArray.from_numpy(rng.standard_normal(R * C).astype(np.float32)) for _ in range(4)]
    g = DeviceArray(C * 4)
    lo, ls = layout_of((R, C)), layout_of((C,))
    i = [0]

    def bias():
        k = i[0] % len(ups)
        i[0] += 1
        check(abi.lib.trs_reduce_to_shape_f32(ups[k].ptr, ctypes.byref(lo), ctypes.byref(ls), g.ptr))

    t = time_region(bias, reps)
    byts = R * C * 4 + C * 4
    out["bias_grad_8192x4096"] = {"us": t * 1e3, "bytes": byts, "GBps": byts / (t * 1e-3) / 1e9,
                                  "frac_hbm": byts / (t * 1e-3) / 1e9 / HBM_PEAK_GBS}
    log(f"reduce bias grad [8192,4096]->[4096]: {t * 1e3:.1f} us, {byts / (t * 1e-3) / 1e9:.0f} GB/s")
    del ups
    B, M, N = 64, 512, 1024
    # 3 (up, c) pairs: 768 MiB rotated, three times the 256 MB MALL
    ups = [DeviceArray.from_numpy(rng.standard_normal(B * M * N).astype(np.float32)) for _ in range(3)]
    cs = [DeviceArray.from_numpy(rng.standard_normal(B * M * N).astype(np.float32)) for _ in range(3)]
    ga = DeviceArray(B * N * 4)
    lout, lc, la = layout_of((B, M, N)), layout_of((B, M, N), (N * M, 1, M)), layout_of((B, 1, N))

    def mul_a():
        k = i[0] % len(cs)
        i[0] += 1
        check(abi.lib.trs_mul_backward_f32(ups[k].ptr, ctypes.byref(lout), cs[k].ptr, ctypes.byref(lc),
                                           ctypes.byref(la), ga.ptr))

    t = time_region(mul_a, reps)
    byts = 2 * B * M * N * 4 + B * N * 4
    out["mul_vjp_a_64x512x1024"] = {"us": t * 1e3, "bytes": byts, "GBps": byts / (t * 1e-3) / 1e9,
                                    "frac_hbm": byts / (t * 1e-3) / 1e9 / HBM_PEAK_GBS}
    log(f"mul VJP a [64,512,1024] x c.mT -> [64,1,1024]: {t * 1e3:.1f} us, {byts / (t * 1e-3) / 1e9:.0f} GB/s")
    return {"reduce_vjp": out}


def run_all(log) -> dict:
    res = {}
    for fn in (relu_bias, broadcast_strided, reduce_vjp, matmul, matmul_shapes, mlp):
        try:
            r = fn(log)
            res.update({fn.__name__: r} if fn is matmul_shapes else r)
        except Exception as exc:
            res[fn.__name__] = {"error": repr(exc)}
            log(f"{fn.__name__} failed: {exc!r}")
    return res
