"""CPU address check of the causal prompt attention on the fp16 matrix
cores (g2k_attn_prefill_h16).

tests/native/attn_addr.cpp compiles the kernel's own index arithmetic
(gpt2-opencl-1.1_amd/csrc/g2_attn_plan.h: the (head, query block) of a
work-group, the staged K/V-half rows and chunks of its lanes, the LDS
element of each fragment read, the query row of a lane) with g++ and walks
every work-group, key half, wave and lane of a launch: the staging loads
stay inside the K halves [S][E] and the transposed V halves [E][S] and
inside their LDS stage, every fragment read finds the chunk its product
needs, the query loads stay inside the prompt's rows and every output is
written once.  The idle work-groups' helper roles (g2a_help_plan) are walked
as the kernel takes them: every key block of every query block is taken
once, by the block's own work-group or its helper, and every helper slot is
written once, read once and inside the slot buffer.  Prompt lengths 1 to
1023 (the cache limit), GPT-2 small to XL head counts.  Planted mistakes (a
key block staged one block too far, a helper overlapping its block's own
key range, a narrower read swizzle) must be caught.  No GPU is involved.
"""
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gpt2-opencl-1.1_amd", "csrc")

HEADS = (1, 3, 12, 16, 20, 25)
PROMPTS = (1, 2, 63, 64, 65, 127, 128, 129, 200, 256, 511, 512, 513, 777, 960, 961, 1000, 1023)


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("attn") / "attn_addr")
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-I" + CSRC, "-o", out,
                    os.path.join(ROOT, "tests", "native", "attn_addr.cpp")], check=True)
    return out


def run(checker, P, NH, plant=0):
    r = subprocess.run([checker, str(P), str(NH), str(plant)], capture_output=True, text=True, timeout=300)
    return r.returncode, (r.stdout + r.stderr).strip()


def test_prompt_attention_addresses(checker):
    jobs = [(P, NH) for P in PROMPTS for NH in HEADS]
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 2)) as ex:
        results = list(ex.map(lambda j: (j, run(checker, *j)), jobs))
    for (P, NH), (rc, out) in results:
        assert rc == 0, f"P {P}, {NH} heads: {out}"


def test_planted_key_block_overrun_is_caught(checker):
    rc, out = run(checker, 1023, 25, plant=1)
    assert rc == 1 and "out of bounds" in out, out


def test_planted_helper_overlap_is_caught(checker):
    """A helper that also takes the first key block of its block's own
    work-group (the key ranges overlap) must be caught."""
    for P in (300, 512):
        rc, out = run(checker, P, 25, plant=3)
        assert rc == 1 and "taken 2 times" in out, out


def test_planted_read_swizzle_is_caught(checker):
    rc, out = run(checker, 512, 25, plant=2)
    assert rc == 1 and "needs chunk" in out, out
