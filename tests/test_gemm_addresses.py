"""CPU address check of the 128x128 fp16 prefill GEMM (g2k_hgemm2_*).

tests/native/gemm_addr.cpp compiles the kernel's own index arithmetic
(gpt2-opencl-1.1_amd/csrc/g2_gemm_plan.h: tile of a work-group, K steps of
a slice, tile-load rows and chunks, LDS slots of the loads and of the
fragment reads, the output element of each accumulator value, and the
host's split-K choice) with g++ and walks every work-group, wave and lane of
a launch.  It checks that the loads stay inside the matrices, the K slice
and the LDS ring, that every fragment read finds the chunk its product
needs, that the outputs of a tile are each written once and the partial
slices stay inside their buffer, for every GEMM of the fp16 prefill (qkv,
proj, fc, fc2) at GPT-2 small to XL width and prompt lengths from 65 (the
first that takes this kernel) to 1023, with the slice count the host picks
on MI355X's 256 CUs.  Planted mistakes (the activation row clamp removed, a
narrower read swizzle, slices that drop the remainder steps) must be
caught.  No GPU is involved.
"""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gpt2-opencl-1.1_amd", "csrc")

WIDTHS = (768, 1024, 1280, 1600)
PROMPTS = (65, 100, 127, 128, 129, 200, 256, 300, 512, 640, 777, 1000, 1023)


def define(header, name):
    """An integer #define of one of the library's headers (the host's slice
    limits), so the check uses the values the library is built with."""
    text = open(os.path.join(CSRC, header)).read()
    m = re.search(r"^#define\s+%s\s+(\d+)" % name, text, re.M)
    assert m, f"{name} not defined in {header}"
    return int(m.group(1))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("gemm") / "gemm_addr")
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-I" + CSRC, "-o", out,
                    os.path.join(ROOT, "tests", "native", "gemm_addr.cpp")], check=True)
    return out


def gemms(E):
    """(N, K) of the prefill's four GEMMs: qkv, proj, fc, fc2 (ffn = 4 E)."""
    return [(3 * E, E), (E, E), (4 * E, E), (E, 4 * E)]


def run(checker, M, N, K, E, plant=0):
    maxk = define("g2_internal.h", "G2_PF_BIGSPLIT")
    cap = define("g2_internal.h", "G2_PF_MAXSPLIT") * define("g2_kargs.h", "G2_KV_MAX_SEQ") * E
    r = subprocess.run([checker, str(M), str(N), str(K), "256", str(maxk), str(cap), str(plant)],
                       capture_output=True, text=True, timeout=300)
    return r.returncode, (r.stdout + r.stderr).strip()


@pytest.mark.parametrize("E", WIDTHS)
def test_prefill_gemm_addresses(checker, E):
    jobs = [(P, N, K) for P in PROMPTS for N, K in gemms(E)]
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 2)) as ex:
        results = list(ex.map(lambda j: (j, run(checker, *j, E)), jobs))
    for (P, N, K), (rc, out) in results:
        assert rc == 0, f"width {E}, {P} rows, N {N}, K {K}: {out}"


def test_planted_unclamped_rows_are_caught(checker):
    rc, out = run(checker, 100, 4800, 1600, 1600, plant=1)
    assert rc == 1 and "out of bounds" in out, out


def test_planted_read_swizzle_is_caught(checker):
    rc, out = run(checker, 512, 4800, 1600, 1600, plant=2)
    assert rc == 1 and "needs chunk" in out, out


def test_planted_slice_remainder_is_caught(checker):
    rc, out = run(checker, 100, 4800, 1600, 1600, plant=3)
    assert rc == 1 and "slices end" in out, out
