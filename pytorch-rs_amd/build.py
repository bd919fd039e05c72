"""Build the native libraries of the MI355X backend in-tree.

Outputs (git-ignored, shipped with the tree):
  pytorch-rs_amd/lib/libtrs_hip.so     HIP kernels + C ABI (include/trs_hip.h), gfx950 only
  pytorch-rs_amd/lib/libtrs_inputs.so  seeded synthetic inputs (host)
  pytorch-rs_amd/lib/_trs_native*.so   C++ host engine (Tensor/autograd) + Python binding
  oracle/liboracle.so                  CPU oracle (test infrastructure)

Usage: python pytorch-rs_amd/build.py [--if-stale] [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
GEN = CSRC / "_gen"
BUILD = PKG / "_build"
LIB = PKG / "lib"
INCLUDE = ROOT / "include"
ORACLE = ROOT / "oracle"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# -ffp-contract=off: one rounding per reference op (no FMA contraction).
# packed-fp32-ops disabled: never emit v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}", f"-I{CSRC}", f"-I{GEN}",
]
# The pointwise op families are separate translation units so they compile in
# parallel (one file held every instantiation and took about 3 minutes).
HIP_SOURCES = ["pw_binary.hip", "pw_binary_muldiv.hip", "pw_scalar.hip", "pw_unary.hip", "pw_mask.hip",
               "pointwise.hip", "runtime.hip", "transfer.hip", "gemm.hip", "gemm_skinny.hip", "fusion.hip"]
ENGINE_SOURCES = ["engine.cpp", "py_module.cpp"]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _stale(target: Path, deps: list[Path]) -> bool:
    if not target.exists():
        return True
    t = target.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def gen_embedded_source() -> Path:
    """pw_core.h as a C++ raw string literal for the hipRTC fusion compiler."""
    GEN.mkdir(parents=True, exist_ok=True)
    text = (CSRC / "pw_core.h").read_text()
    text = text.replace("#pragma once\n", "")
    delim = "TRSPWCORE"
    assert f"){delim}\"" not in text
    out = GEN / "pw_core_src.inc"
    body = f'R"{delim}({text}){delim}"\n'
    if not out.exists() or out.read_text() != body:
        out.write_text(body)
    return out


def build_hip(jobs: int, if_stale: bool) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB.mkdir(parents=True, exist_ok=True)
    gen_embedded_source()
    headers = [CSRC / h for h in ("pw_core.h", "pw_host.h", "pw_ops.h", "trs_internal.h", "gemm_skinny.h", "lds_dma.h")] + [INCLUDE / "trs_hip.h",
                                                                                 GEN / "pw_core_src.inc"]
    objs = []
    todo = []
    for src in HIP_SOURCES:
        obj = BUILD / (src + ".o")
        objs.append(obj)
        if not if_stale or _stale(obj, [CSRC / src] + headers):
            todo.append((CSRC / src, obj))
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)]) for s, o in todo]
        for f in futs:
            f.result()
    so = LIB / "libtrs_hip.so"
    if not if_stale or _stale(so, objs):
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(so), *map(str, objs),
              "-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"])
    return so


def build_inputs(if_stale: bool) -> Path:
    LIB.mkdir(parents=True, exist_ok=True)
    so = LIB / "libtrs_inputs.so"
    src = CSRC / "inputs.c"
    if not if_stale or _stale(so, [src]):
        _run(["gcc", "-O3", "-march=x86-64", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
              "-std=gnu11", "-Wall", "-o", str(so), str(src), "-lm", "-lpthread"])
    return so


def build_engine(if_stale: bool) -> Path | None:
    """C++ host engine + pybind11 module; links libtrs_hip.so through the C ABI only."""
    srcs = [CSRC / s for s in ENGINE_SOURCES]
    if not all(s.exists() for s in srcs):
        return None
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    so = LIB / f"_trs_native{suffix}"
    deps = srcs + [CSRC / "engine.h", INCLUDE / "trs_hip.h", LIB / "libtrs_hip.so"]
    if not if_stale or _stale(so, deps):
        _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-fvisibility=hidden",
              f"-I{INCLUDE}", f"-I{CSRC}", f"-I{pybind11.get_include()}",
              f"-I{sysconfig.get_paths()['include']}", "-o", str(so), *map(str, srcs),
              f"-L{LIB}", "-ltrs_hip", "-Wl,-rpath,$ORIGIN"])
    return so


def build_oracle(if_stale: bool) -> Path:
    so = ORACLE / "liboracle.so"
    if not if_stale or _stale(so, [ORACLE / "trs_oracle.c", ORACLE / "Makefile"]):
        if so.exists():
            so.unlink()
        _run(["make", "-s", "-C", str(ORACLE)])
    return so


def build_all(jobs: int = 8, if_stale: bool = False) -> None:
    build_hip(jobs, if_stale)
    build_inputs(if_stale)
    build_engine(if_stale)
    build_oracle(if_stale)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--if-stale", action="store_true", help="rebuild only what changed")
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 4))
    ap.add_argument("--clean", action="store_true")
    a = ap.parse_args()
    if a.clean:
        shutil.rmtree(BUILD, ignore_errors=True)
        shutil.rmtree(GEN, ignore_errors=True)
    build_all(a.jobs, a.if_stale)
    return 0


if __name__ == "__main__":
    sys.exit(main())
