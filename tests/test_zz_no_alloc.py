"""g2_attn_1q_noalloc (the entry point that allocates nothing) against
g2_attn_1q, through the C ABI: the same kernels with the chunk partials in a
static device array instead of a library buffer, so the outputs must be bit
for bit identical.  Two calls in a row, the second smaller (GPT-2 XL width
at 1000 positions, then GPT-2 small width at 100), so stale partials of the
first call in the shared array must not leak into the second; the CPU
oracle checks the first call's values too.  More heads than the array
holds is refused with G2_E_LIMIT."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu


def run_both(g2, NH, T, seed):
    D, S = NH * 64, 1024
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal(3 * D).astype(np.float32)
    kc = rng.standard_normal(D * S).astype(np.float32)
    vc = rng.standard_normal(S * D).astype(np.float32)
    scale = 1.0 / np.sqrt(64.0)
    d_qkv, d_k, d_v = g2.to_device(qkv), g2.to_device(kc), g2.to_device(vc)
    outs = []
    for fn in (g2.attn_1q, g2.attn_1q_noalloc):
        d_out = g2.DevBuf(D * 4)
        g2.check(g2._lib.g2_memset(d_out.ptr, 0, D * 4))
        fn(d_qkv, d_k, d_v, d_out, 0, T, D, NH, S, 0, scale)
        g2.sync()
        outs.append(d_out.download(np.float32, D))
    return outs, (qkv, kc, vc, D, S, scale)


def test_noalloc_matches_allocating_entry_point(g2):
    print("\n[noalloc] NH 25 T 1000, then NH 12 T 100", flush=True)
    (a1, b1), (qkv, kc, vc, D, S, scale) = run_both(g2, 25, 1000, 1)
    np.testing.assert_array_equal(b1, a1)
    sc = oracle.attn_scores_1q(qkv, kc, 0, 1000, D, 64, 25, S, scale)
    pr = oracle.attn_softmax_1q(sc, 1000, 25)
    ref = oracle.attn_out_1q(pr, vc, 1000, D, 64, 0, D)
    np.testing.assert_allclose(b1, ref, rtol=1e-4, atol=2e-5)
    (a2, b2), _ = run_both(g2, 12, 100, 2)
    np.testing.assert_array_equal(b2, a2)
    assert not np.array_equal(b2, b1[: b2.size])


def test_noalloc_refuses_beyond_its_scratch(g2):
    p = g2.to_device(np.zeros(4, np.float32))
    rc = g2._lib.g2_attn_1q_noalloc(p.ptr, p.ptr, p.ptr, p.ptr, 0, 10, 65 * 64, 65, 1024, 0, C.c_float(0.125))
    assert rc == g2.G2_E_LIMIT and "static scratch" in g2.last_error()
