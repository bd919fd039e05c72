"""Host-only checks of the C ABI library and the input generator (no GPU)."""
import ctypes
import hashlib
import re
from pathlib import Path

import numpy as np
import pytest

from helpers import golden
from trs_backend import abi
from trs_backend.configs import CONFIGS, generate

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    text = (ROOT / "include" / "trs_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(trs_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_entry_point():
    names = declared_functions()
    assert len(names) >= 30
    for name in names:
        assert hasattr(abi.lib, name), name
        assert name in abi._SIGNATURES, f"{name} has no ctypes signature"


def test_binding_declares_nothing_the_header_lacks():
    assert set(abi._SIGNATURES) <= set(declared_functions())


def test_layout_struct_matches_header_size():
    # int32 rank, int32 reserved, int64 shape[R], int64 stride[R], int64 offset
    # with R = TRS_MAX_RANK; the oracle's layout has the same binary form
    import oracle as O
    text = (ROOT / "include" / "trs_hip.h").read_text()
    max_rank = int(re.search(r"^#define TRS_MAX_RANK (\d+)", text, flags=re.M).group(1))
    assert max_rank == abi.MAX_RANK == O.MAX_RANK == 25
    assert ctypes.sizeof(abi.Layout) == 4 + 4 + 8 * max_rank + 8 * max_rank + 8
    assert ctypes.sizeof(O.OLayout) == ctypes.sizeof(abi.Layout)
    # trs_pw_plan_info: 10 int32 fields, an int64, then split and a reserved int32
    assert ctypes.sizeof(abi.PwPlanInfo) == 10 * 4 + 8 + 4 + 4


def test_philox_known_answer_vectors():
    # Random123 kat_vectors for philox4x32 with 10 rounds.
    assert abi.philox((0, 0, 0, 0), (0, 0)) == (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)
    assert abi.philox((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2) == (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)
    assert abi.philox((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0)) == (
        0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)


def test_generated_inputs_match_committed_hashes():
    ref = golden("input_sha256.json")
    for cfg, spec in CONFIGS.items():
        for name, *_ in spec["tensors"]:
            arr = generate(cfg, name, ref["prefix_elements"])
            assert hashlib.sha256(arr.tobytes()).hexdigest() == ref["hashes"][f"{cfg}.{name}"], f"{cfg}.{name}"


def test_generator_is_thread_count_independent_and_distributed():
    a = abi.gen_normal(4, 0, 0.0, 1.0, 300_001, threads=1)
    b = abi.gen_normal(4, 0, 0.0, 1.0, 300_001, threads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    u = abi.gen_uniform(1, 2, -4.0, 4.0, 200_000, threads=3)
    assert u.min() >= -4.0 and u.max() < 4.0 and abs(u.mean()) < 0.05
    m = abi.gen_mask(4, 3, 0.9, 200_000)
    assert set(np.unique(m)) <= {0, 1} and abs(m.mean() - 0.9) < 0.005


def _compile(ir: str):
    kid = ctypes.c_uint64()
    rc = abi.lib.trs_fusion_compile(ir.encode(), len(ir), ctypes.byref(kid))
    return rc, kid.value


def test_fusion_compiler_generates_and_compiles_on_the_host():
    ir = "in f32\nin f32\nin f32\nmul %0 %1\nadd %3 %2\nexp %4\nconst 0x3f800000\nsub %5 %6\nrelu %7\nout %8\n"
    rc, kid = _compile(ir)
    abi.check(rc)
    n = ctypes.c_size_t()
    abi.check(abi.lib.trs_fusion_source(kid, None, 0, ctypes.byref(n)))
    buf = ctypes.create_string_buffer(n.value)
    abi.check(abi.lib.trs_fusion_source(kid, buf, n.value, None))
    src = buf.value.decode()
    assert "v3 = v0 * v1" in src and "v4 = v3 + v2" in src
    assert "trs::exp_value(v4)" in src and "__uint_as_float(0x3f800000u)" in src
    assert "trs_fused_flat_c" in src and "trs_fused_rows_s" in src and "trs_fused_generic" in src
    ms = ctypes.c_double()
    abi.check(abi.lib.trs_fusion_compile_ms(kid, ctypes.byref(ms)))
    assert ms.value > 0
    # Same IR -> same cached program.
    rc2, kid2 = _compile(ir)
    assert rc2 == 0 and kid2 == kid


def test_fusion_compiler_multi_output_program():
    ir = "in f32\nin f32\nmul %0 %1\nexp %2\nrelub %0 %1\nout %2\nout %3\nout %4\nout %2\n"
    rc, kid = _compile(ir)
    abi.check(rc)
    n = ctypes.c_int()
    abi.check(abi.lib.trs_fusion_outputs(kid, ctypes.byref(n)))
    assert n.value == 4
    size = ctypes.c_size_t()
    abi.check(abi.lib.trs_fusion_source(kid, None, 0, ctypes.byref(size)))
    buf = ctypes.create_string_buffer(size.value)
    abi.check(abi.lib.trs_fusion_source(kid, buf, size.value, None))
    src = buf.value.decode()
    assert "static constexpr int NOUT = 4;" in src
    assert "r[0] = v2;" in src and "r[2] = v4;" in src and "r[3] = v2;" in src
    rc, one = _compile("in f32\nneg %0\nout %1\n")
    abi.check(rc)
    abi.check(abi.lib.trs_fusion_outputs(one, ctypes.byref(n)))
    assert n.value == 1


@pytest.mark.parametrize("ir,fragment", [
    ("in f32\nout %0\nrelu %0\n", "instruction after 'out'"),
    ("in f32\n" + "out %0\n" * 9, "more than 8 outputs"),
    ("in f32\nadd %0 %1\nout %1\n", "bad operand"),
    ("in f32\nfoo %0\nout %0\n", "unknown instruction"),
    ("in f32\nrelu %0\n", "no 'out'"),
    ("const 0x0\nout %0\n", "no inputs"),
    ("in f64\nout %0\n", "in f32"),
])
def test_fusion_compiler_rejects_bad_programs(ir, fragment):
    rc, _ = _compile(ir)
    assert rc == -9
    assert fragment in abi.lib.trs_last_error().decode()


_CACHE_CHILD = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
from trs_backend import abi
ir = sys.argv[2]
kid = ctypes.c_uint64()
abi.check(abi.lib.trs_fusion_compile(ir.encode(), len(ir), ctypes.byref(kid)))
hit, ms = ctypes.c_int(), ctypes.c_double()
abi.check(abi.lib.trs_fusion_from_disk_cache(kid, ctypes.byref(hit)))
abi.check(abi.lib.trs_fusion_compile_ms(kid, ctypes.byref(ms)))
print(hit.value, ms.value)
"""


def _compile_in_child(ir: str, cache_dir: str):
    import os
    import subprocess
    import sys
    env = dict(os.environ, TRS_FUSION_CACHE_DIR=cache_dir)
    pkg = str(Path(__file__).resolve().parent.parent / "pytorch-rs_amd")
    out = subprocess.run([sys.executable, "-c", _CACHE_CHILD, pkg, ir], env=env, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    hit, ms = out.stdout.split()
    return int(hit), float(ms)


def test_fusion_disk_cache_persists_across_processes_and_rejects_bad_files(tmp_path):
    ir = "in f32\nconst 0x40490fdb\nmul %0 %1\nneg %2\nout %3\n"
    cache = tmp_path / "fusion"
    hit, compile_ms = _compile_in_child(ir, str(cache))
    assert hit == 0
    files = list(cache.glob("*.co"))
    assert len(files) == 1 and not list(cache.glob("*.tmp.*"))
    hit, load_ms = _compile_in_child(ir, str(cache))
    assert hit == 1 and load_ms < compile_ms
    # A damaged file (wrong key bytes) is a miss and is replaced by a good one.
    data = bytearray(files[0].read_bytes())
    data[40] ^= 0xFF
    files[0].write_bytes(bytes(data))
    assert _compile_in_child(ir, str(cache))[0] == 0
    assert _compile_in_child(ir, str(cache))[0] == 1
    # A truncated file is a miss as well.
    files[0].write_bytes(files[0].read_bytes()[:-100])
    assert _compile_in_child(ir, str(cache))[0] == 0
    # An empty directory setting disables the cache.
    before = sorted(p.name for p in tmp_path.rglob("*"))
    assert _compile_in_child(ir, "")[0] == 0
    assert sorted(p.name for p in tmp_path.rglob("*")) == before


_C_HOST = r"""
#include <stdio.h>
#include "trs_hip.h"

int main(void) {
    int n = -1;
    int rc = trs_device_count(&n);
    /* No GPU in this container: a status code and a message, never a crash. */
    printf("%d %d %s\n", rc, n, rc ? trs_last_error() : "ok");
    trs_layout l = {.rank = 1, .shape = {4}, .stride = {1}, .offset = 0};
    rc = trs_binary_f32(99, NULL, &l, NULL, &l, NULL, &l);
    printf("%d\n", rc);
    return 0;
}
"""


def test_header_compiles_as_c_and_a_c_host_links_the_library(tmp_path):
    """include/trs_hip.h is plain C (C11): a C program compiles against it,
    links libtrs_hip.so and calls entry points; without a GPU they return
    status codes."""
    import subprocess
    from pathlib import Path
    repo = Path(__file__).resolve().parent.parent
    lib_dir = abi.LIB_DIR
    src = tmp_path / "host.c"
    src.write_text(_C_HOST)
    exe = tmp_path / "host"
    cc = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{repo / 'include'}", str(src), "-o", str(exe),
                         f"-L{lib_dir}", "-ltrs_hip", f"-Wl,-rpath,{lib_dir}"], capture_output=True, text=True)
    assert cc.returncode == 0, cc.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    first, second = out.stdout.splitlines()[:2]
    rc, n = (int(v) for v in first.split()[:2])
    # Either a device count, or (no GPU) a negative status with a message.
    assert (rc == 0 and n >= 0) or (rc < 0 and first.split(maxsplit=2)[2] != "ok")
    # An unknown op code is rejected before any device work.
    assert int(second) == abi.TRS_E_INVALID_ARGUMENT
