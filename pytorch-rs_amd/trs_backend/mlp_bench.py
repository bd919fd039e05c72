"""2-layer MLP forward + backward through torch_rs.

X[8192,4096] ~ N(0,1); W1[4096,4096], W2[4096,1024] ~ U(-1/64, 1/64); zero
biases; relu; dropout p=0.1 applied with a seeded uint8 keep-mask and scale
f32(1/0.9); loss = sum(out); gradients for W1, W2 and X.  One step is the
whole forward + backward on device, timed with HIP events on the library
stream.  Work: six GEMMs, 1,030,792,151,040 FLOP per step.
"""
from __future__ import annotations

import numpy as np

from .configs import generate
from .timing import time_launches, time_region

GEMM_FLOP = 2 * (3 * 8192 * 4096 * 4096 + 3 * 8192 * 4096 * 1024)
FP32_MFMA_PEAK_TFLOPS = 157.3


def build(device: str = "cuda"):
    import torch_rs

    F = torch_rs.nn.functional
    X = torch_rs.tensor(generate("mlp", "X").reshape(8192, 4096), device=device)
    W1 = torch_rs.tensor(generate("mlp", "W1").reshape(4096, 4096), device=device)
    W2 = torch_rs.tensor(generate("mlp", "W2").reshape(4096, 1024), device=device)
    mask = F.keep_mask(generate("mlp", "mask").reshape(8192, 4096), device)
    b1 = torch_rs.zeros(4096, device=device)
    b2 = torch_rs.zeros(1024, device=device)

    def step():
        # Fresh leaves each step: the gradients of the step are new buffers
        # (zero_grad with set_to_none), not accumulated into the last step's.
        x, w1, w2 = X.with_requires_grad(True), W1.with_requires_grad(True), W2.with_requires_grad(True)
        h = (x @ w1 + b1).relu()
        d = F.dropout(h, 0.1, training=True, mask=mask)
        out = d @ w2 + b2
        loss = out.sum()
        loss.backward()
        return loss, x, w1, w2

    return step


def run(log, reps: int = 20) -> dict:
    step = build()
    holder = {}

    def timed():
        holder["last"] = step()

    med = time_region(timed, reps=reps, warmup=4)  # ~30 ms: steady MFMA clocks
    t = time_launches(timed, reps=reps, warmup=0)
    tf = GEMM_FLOP / (med * 1e-3) / 1e12
    loss = holder["last"][0].item()
    log(f"mlp fwd+bwd: {med:.3f} ms/step, {tf:.1f} TFLOPS on the GEMM work, loss {loss:.4f}")
    t = sorted(t)
    _, x, w1, w2 = holder["last"]
    grad_sums = {name: float(np.sum(v.grad.numpy(), dtype=np.float64)) for name, v in
                 (("dX", x), ("dW1", w1), ("dW2", w2))}
    return {"ms_avg": med, "ms_min_single_step": t[0], "ms_median_single_step": t[len(t) // 2],
            "ms_max_single_step": t[-1], "gemm_flop_per_step": GEMM_FLOP, "TFLOPS": tf,
            "frac_mfma_peak": tf / FP32_MFMA_PEAK_TFLOPS, "loss": loss, "grad_checksums": grad_sums}
