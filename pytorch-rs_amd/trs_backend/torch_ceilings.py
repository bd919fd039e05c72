"""Independent same-box ceilings for the HBM-bound configs, timed with
ROCm PyTorch alone.

This module imports torch and nothing of this library: run it in a process
of its own (``python bench.py --workload torch_ceilings``) so that no kernel
of libtrs_hip.so is loaded or launched.  Every figure is the average device
time per call over a region of back-to-back calls bracketed by two
torch.cuda events on torch's current stream, with the inputs rotated over
the same number of buffer sets as the library's own bench lines (so every
timed call reads HBM, not the 256 MB Infinity Cache).

Shapes are BASELINE configs 1 and 3:
- relu_bias: x [4096,4096] + b [4096], then relu;
- broadcast_strided: (a [64,1,1024] + b [1,512,1024]) * c.mT, c [64,1024,512].
"""
from __future__ import annotations

import json
import sys

HBM_PEAK_GBS = 8000.0


def _region_ms(torch, fn, reps: int, warmup: int = 5) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / reps


def _rot(objs):
    i = [0]

    def nxt():
        k = i[0] % len(objs)
        i[0] += 1
        return objs[k]
    return nxt


def _entry(us: float, nbytes: int) -> dict:
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"us": us, "bytes": nbytes, "GBps": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


def relu_bias(torch, reps: int = 200, sets: int = 8) -> dict:
    R = C = 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    xs = [torch.randn(R, C, device="cuda", generator=g) for _ in range(sets)]
    outs = [torch.empty(R, C, device="cuda") for _ in range(sets)]
    b = torch.randn(C, device="cuda", generator=g)
    algo = 2 * R * C * 4 + C * 4
    flat = 2 * R * C * 4
    pairs = _rot(list(zip(xs, outs)))
    res = {}

    def run(name, fn, nbytes):
        res[name] = _entry(_region_ms(torch, fn, reps) * 1e3, nbytes)

    def relu_add():
        x, _ = pairs()
        return torch.relu(x + b)

    def add_out_relu_inplace():
        x, o = pairs()
        torch.add(x, b, out=o)
        torch.relu_(o)

    def add_out():
        x, o = pairs()
        torch.add(x, b, out=o)

    def copy_memcpy():
        x, o = pairs()
        o.copy_(x)

    def neg_out():
        x, o = pairs()
        torch.neg(x, out=o)

    run("relu(x + b), two kernels", relu_add, algo)
    run("add(x, b, out=o) + relu_(o), two kernels", add_out_relu_inplace, algo)
    run("add(x, b, out=o), one kernel: the fused op's bytes", add_out, algo)
    run("o.copy_(x), hipMemcpyAsync device to device", copy_memcpy, flat)
    run("neg(x, out=o), one elementwise kernel", neg_out, flat)
    return {"relu_bias": res, "buffer_sets": sets}


def broadcast_strided(torch, reps: int = 200, sets: int = 4) -> dict:
    B, M, N = 64, 512, 1024
    g = torch.Generator(device="cuda").manual_seed(2)
    a = torch.randn(B, 1, N, device="cuda", generator=g)
    b = torch.randn(1, M, N, device="cuda", generator=g)
    cs = [torch.randn(B, N, M, device="cuda", generator=g) for _ in range(sets)]
    outs = [torch.empty(B, M, N, device="cuda") for _ in range(sets)]
    algo = (B * N + M * N + 2 * B * M * N) * 4
    flat = 2 * B * M * N * 4
    pairs = _rot(list(zip(cs, outs)))
    res = {}

    def run(name, fn, nbytes):
        res[name] = _entry(_region_ms(torch, fn, reps) * 1e3, nbytes)

    s = torch.empty(B, M, N, device="cuda")

    def fused_expr():
        c, _ = pairs()
        return (a + b) * c.mT

    def mul_out_of_sum():
        c, o = pairs()
        torch.mul(s, c.mT, out=o)

    def mt_contiguous():
        c, _ = pairs()
        return c.mT.contiguous()

    def mt_copy_out():
        c, o = pairs()
        o.copy_(c.mT)

    def flat_copy():
        c, o = pairs()
        o.view(-1).copy_(c.view(-1))

    torch.add(a, b, out=s)
    run("(a + b) * c.mT, two kernels", fused_expr, algo)
    run("mul(s, c.mT, out=o), one kernel: a transposed operand plus a contiguous one", mul_out_of_sum,
        3 * B * M * N * 4)
    run("c.mT.contiguous(), transposed copy", mt_contiguous, flat)
    run("o.copy_(c.mT), transposed copy into an existing tensor", mt_copy_out, flat)
    run("o.copy_(c), flat 128 MiB copy (hipMemcpyAsync)", flat_copy, flat)
    return {"broadcast_strided": res, "buffer_sets": sets}


def flat_copy_1gib(torch, reps: int = 20) -> dict:
    n = 1 << 28
    src = torch.empty(n, device="cuda").fill_(1.0)
    dst = torch.empty(n, device="cuda")
    us = _region_ms(torch, lambda: dst.copy_(src), reps) * 1e3
    return {"copy_1GiB": _entry(us, 8 * n)}


def main() -> int:
    import torch
    if not torch.cuda.is_available():
        print("torch_ceilings needs a GPU", file=sys.stderr)
        return 2
    out = {"workload": "torch_ceilings", "torch": torch.__version__,
           "device": torch.cuda.get_device_name(0),
           "timing": "average per call over back-to-back calls between two torch.cuda events, inputs rotated"}
    out.update(relu_bias(torch))
    out.update(broadcast_strided(torch))
    out.update(flat_copy_1gib(torch))
    loaded = []
    try:
        with open("/proc/self/maps") as f:
            loaded = sorted({l.split()[-1] for l in f if "libtrs" in l})
    except OSError:
        pass
    out["libtrs_loaded"] = loaded
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
