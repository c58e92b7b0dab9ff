"""CPU address check of the persistent decode-step kernel's load plans.

tests/native/step_addr.cpp compiles the kernel's own index arithmetic
(gpt2-opencl-1.1_amd/csrc/g2_step_plan.h, which g2_step.hip uses for every
weight-row chunk, dot-product x chunk and KV-cache load) with g++ and walks
every work-group and thread of a launch through every phase, checking each
global address against its allocation (weights, biases, LayerNorm
parameters, embedding rows, KV cache loads and stores, exchange words,
logits) and each LDS index against the kernel's buffers.  It runs for every
model shape the library serves (GPT-2 small to XL, and the small test
shapes with fewer heads than XCDs), both weight element sizes and positions
at chunk boundaries, on MI355X's 256-CU grid (where every shape must be
admitted) and on other grid sizes (where the host's admission rule,
g2p_step_refusal in the same header, may refuse a shape instead).  Planted
mistakes (the per-lane chunk clamp removed; the dot products' x reads one
chunk off the padded input layout) must be caught.
No GPU is involved.
"""
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gpt2-opencl-1.1_amd", "csrc")

SHAPES = {  # L, E, NH, V, F
    "tiny": (2, 128, 2, 256, 512), "3-heads": (3, 192, 3, 1000, 768), "1-head": (1, 64, 1, 50257, 256),
    "small": (12, 768, 12, 50257, 3072), "medium": (24, 1024, 16, 50257, 4096),
    "large": (36, 1280, 20, 50257, 5120), "xl": (48, 1600, 25, 50257, 6400),
}


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("addr") / "step_addr")
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-I" + CSRC, "-o", out,
                    os.path.join(ROOT, "tests", "native", "step_addr.cpp")], check=True)
    return out


def run(checker, shape, ve, pos, nwg, plant=0):
    L, E, NH, V, F = SHAPES[shape]
    r = subprocess.run([checker, str(L), str(E), str(NH), str(V), str(F), str(ve), str(pos), str(nwg), str(plant)],
                       capture_output=True, text=True, timeout=600)
    return r.returncode, r.stdout.strip() + r.stderr.strip()


@pytest.mark.parametrize("shape", list(SHAPES))
def test_step_kernel_addresses_in_bounds(checker, shape):
    jobs = [(shape, ve, pos, nwg) for ve in (8, 4) for pos in (0, 1, 5, 63, 64, 511, 767, 1022, 1023)
            for nwg in (256,)] + [(shape, 8, 1023, nwg) for nwg in (80, 104, 304)]
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 2)) as ex:
        results = list(ex.map(lambda j: (j, run(checker, *j)), jobs))
    for (sh, ve, pos, nwg), (rc, out) in results:
        if nwg == 256:  # MI355X: every shape must be admitted
            assert rc == 0, f"{sh} chunk {ve} elements, position {pos}, {nwg} work-groups: {out}"
        else:  # other grids: refused by the host (and never launched) or in bounds
            assert rc in (0, 3), f"{sh} chunk {ve} elements, position {pos}, {nwg} work-groups: {out}"


def test_planted_x_layout_shift_is_caught(checker):
    """The dot products reading x one chunk off the padded positions the
    fetches write must be caught, for both weight sizes."""
    for ve in (8, 4):
        rc, out = run(checker, "xl", ve, 700, 256, plant=2)
        assert rc == 1 and "LDS x" in out, out


def test_planted_unclamped_chunk_is_caught(checker):
    rc, out = run(checker, "xl", 8, 1022, 256, plant=1)
    assert rc == 1 and "out of bounds" in out, out
    rc, out = run(checker, "tiny", 8, 5, 256, plant=1)
    assert rc == 1, out


def test_planted_row_plan_table_swap_is_caught(checker):
    """A row-plan table whose fc and fc2 entries are swapped must be caught
    (each entry is checked against the plan of its own matrix)."""
    for ve in (8, 4):
        rc, out = run(checker, "xl", ve, 700, 256, plant=3)
        assert rc == 1 and "row plan" in out, out
