"""2-layer MLP forward + backward through torch_rs.

X[8192,4096] ~ N(0,1); W1[4096,4096], W2[4096,1024] ~ U(-1/64, 1/64); zero
biases; relu; dropout p=0.1 applied with a seeded uint8 keep-mask and scale
f32(1/0.9); loss = sum(out); gradients for W1, W2 and X.  One step is the
whole forward + backward on device, timed with HIP events on the library
stream.  Work: six GEMMs, 1,030,792,151,040 FLOP per step.

The bias add, relu and dropout-apply after the first GEMM run as one fused
autograd node (torch_rs.fuse, the mask read as bytes); its gradient equals
the eager ops' bit for bit, which run() checks against the eager step.
"""
from __future__ import annotations

import numpy as np

from .configs import generate
from .timing import time_launches, time_region

GEMM_FLOP = 2 * (3 * 8192 * 4096 * 4096 + 3 * 8192 * 4096 * 1024)
FP32_MFMA_PEAK_TFLOPS = 157.3


def build(device: str = "cuda", fused: bool = True):
    import torch_rs

    F = torch_rs.nn.functional
    X = torch_rs.tensor(generate("mlp", "X").reshape(8192, 4096), device=device)
    W1 = torch_rs.tensor(generate("mlp", "W1").reshape(4096, 4096), device=device)
    W2 = torch_rs.tensor(generate("mlp", "W2").reshape(4096, 1024), device=device)
    mask = F.keep_mask(generate("mlp", "mask").reshape(8192, 4096), device)
    b1 = torch_rs.zeros(4096, device=device)
    b2 = torch_rs.zeros(1024, device=device)
    act = torch_rs.fuse(lambda z, b, m: ((z + b).relu() * m) * (1 / 0.9))

    def step():
        # Fresh leaves each step: the gradients of the step are new buffers
        # (zero_grad with set_to_none), not accumulated into the last step's.
        x, w1, w2 = X.with_requires_grad(True), W1.with_requires_grad(True), W2.with_requires_grad(True)
        if fused:
            d = act(x @ w1, b1, mask)
        else:
            d = F.dropout((x @ w1 + b1).relu(), 0.1, training=True, mask=mask)
        out = d @ w2 + b2
        loss = out.sum()
        loss.backward()
        return loss, x, w1, w2

    return step


def _bits(t) -> bytes:
    return t.numpy().tobytes()


def run(log, reps: int = 20) -> dict:
    step = build()
    eager_step = build(fused=False)
    holder = {}

    def timed():
        holder["last"] = step()

    med = time_region(timed, reps=reps, warmup=4)  # ~30 ms: steady MFMA clocks
    t = time_launches(timed, reps=reps, warmup=0)
    tf = GEMM_FLOP / (med * 1e-3) / 1e12
    loss = holder["last"][0].item()
    log(f"mlp fwd+bwd: {med:.3f} ms/step, {tf:.1f} TFLOPS on the GEMM work, loss {loss:.4f}")
    t = sorted(t)
    lf, x, w1, w2 = holder["last"]
    grad_sums = {name: float(np.sum(v.grad.numpy(), dtype=np.float64)) for name, v in
                 (("dX", x), ("dW1", w1), ("dW2", w2))}
    # The eager step: same loss and gradients, bit for bit, and its time.
    eager = {}
    med_eager = time_region(lambda: eager.__setitem__("last", eager_step()), reps=reps // 2, warmup=2)
    le, xe, w1e, w2e = eager["last"]
    same = _bits(lf) == _bits(le) and all(_bits(a.grad) == _bits(b.grad) for a, b in ((x, xe), (w1, w1e), (w2, w2e)))
    log(f"mlp eager activation: {med_eager:.3f} ms/step; fused and eager loss and gradients bit-identical: {same}")
    return {"ms_avg": med, "ms_min_single_step": t[0], "ms_median_single_step": t[len(t) // 2],
            "ms_max_single_step": t[-1], "gemm_flop_per_step": GEMM_FLOP, "TFLOPS": tf,
            "frac_mfma_peak": tf / FP32_MFMA_PEAK_TFLOPS, "loss": loss, "grad_checksums": grad_sums,
            "activation": "fused (bias add, relu, dropout-apply: one FusedBackward0 node)",
            "eager_activation_ms_avg": med_eager, "fused_equals_eager_bitwise": same}
