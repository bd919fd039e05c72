"""The five BASELINE configurations as seeded synthetic input specs.

Each tensor is one Philox stream (key = {seed, stream index}) in the order the
configuration lists it.  N(0, 1/sqrt(K)) is read as standard deviation
1/sqrt(K).
"""
from __future__ import annotations

import math

# name -> list of (tensor name, shape, kind, params)
CONFIGS = {
    "relu_bias": {
        "seed": 0,
        "tensors": [("x", (4096, 4096), "normal", (0.0, 1.0)), ("b", (4096,), "normal", (0.0, 1.0))],
    },
    "fused_chain": {
        "seed": 1,
        "tensors": [(n, (1 << 28,), "uniform", (-4.0, 4.0)) for n in ("x", "y", "z")],
    },
    "broadcast_strided": {
        "seed": 2,
        "tensors": [("a", (64, 1, 1024), "normal", (0.0, 1.0)), ("b", (1, 512, 1024), "normal", (0.0, 1.0)),
                    ("c", (64, 1024, 512), "normal", (0.0, 1.0))],
    },
    "matmul": {
        "seed": 3,
        "tensors": [("A", (4096, 4096), "normal", (0.0, 1.0 / math.sqrt(4096))),
                    ("B", (4096, 4096), "normal", (0.0, 1.0 / math.sqrt(4096))),
                    ("Ab", (32, 512, 512), "normal", (0.0, 1.0 / math.sqrt(512))),
                    ("Bb", (32, 512, 512), "normal", (0.0, 1.0 / math.sqrt(512)))],
    },
    "mlp": {
        "seed": 4,
        "tensors": [("X", (8192, 4096), "normal", (0.0, 1.0)), ("W1", (4096, 4096), "uniform", (-1 / 64, 1 / 64)),
                    ("W2", (4096, 1024), "uniform", (-1 / 64, 1 / 64)), ("mask", (8192, 4096), "mask", (0.9,))],
    },
}


def numel(shape) -> int:
    n = 1
    for d in shape:
        n *= d
    return n


def generate(config: str, name: str, count: int | None = None, threads: int = 8):
    """Host array (flat) for one tensor of a config; `count` limits to a prefix."""
    from .abi import gen_mask, gen_normal, gen_uniform

    cfg = CONFIGS[config]
    for stream, (tname, shape, kind, params) in enumerate(cfg["tensors"]):
        if tname != name:
            continue
        n = numel(shape) if count is None else min(count, numel(shape))
        if kind == "normal":
            return gen_normal(cfg["seed"], stream, params[0], params[1], n, threads)
        if kind == "uniform":
            return gen_uniform(cfg["seed"], stream, params[0], params[1], n, threads)
        return gen_mask(cfg["seed"], stream, params[0], n, threads)
    raise KeyError(f"{config}.{name}")
