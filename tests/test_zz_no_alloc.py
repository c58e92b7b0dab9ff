"""g2_attn_1q_noalloc (the entry point that allocates nothing) against
g2_attn_1q, through the C ABI: the same kernels with the chunk partials in a
static device array instead of a library buffer, so the outputs must be bit
for bit identical.  Two calls in a row, the second smaller (GPT-2 XL width
at 1000 positions, then GPT-2 small width at 100), both also checked
against the CPU oracle, so a merge that read the first call's stale
partials from the shared array (which both buffers still hold at the same
offsets) would fail the second call's oracle check.  More heads than the
array holds is refused with G2_E_LIMIT.

The documented use under HIP graph capture: one call captured on the
library stream (g2_stream) into a graph, the graph replayed three times,
with eager calls on other inputs between the replays (they overwrite the
static array), every replay checked bit for bit against the eager result of
the captured inputs."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu

SCALE = 1.0 / np.sqrt(64.0)


def inputs(NH, seed):
    D, S = NH * 64, 1024
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal(3 * D).astype(np.float32)
    kc = rng.standard_normal(D * S).astype(np.float32)
    vc = rng.standard_normal(S * D).astype(np.float32)
    return qkv, kc, vc, D, S


def oracle_out(qkv, kc, vc, T, D, NH, S):
    sc = oracle.attn_scores_1q(qkv, kc, 0, T, D, 64, NH, S, SCALE)
    pr = oracle.attn_softmax_1q(sc, T, NH)
    return oracle.attn_out_1q(pr, vc, T, D, 64, 0, D)


def run_both(g2, NH, T, seed):
    qkv, kc, vc, D, S = inputs(NH, seed)
    d_qkv, d_k, d_v = g2.to_device(qkv), g2.to_device(kc), g2.to_device(vc)
    outs = []
    for fn in (g2.attn_1q, g2.attn_1q_noalloc):
        d_out = g2.DevBuf(D * 4)
        g2.check(g2._lib.g2_memset(d_out.ptr, 0, D * 4))
        fn(d_qkv, d_k, d_v, d_out, 0, T, D, NH, S, 0, SCALE)
        g2.sync()
        outs.append(d_out.download(np.float32, D))
    return outs, oracle_out(qkv, kc, vc, T, D, NH, S)


def test_noalloc_matches_allocating_entry_point(g2):
    print("\n[noalloc] NH 25 T 1000, then NH 12 T 100", flush=True)
    (a1, b1), ref1 = run_both(g2, 25, 1000, 1)
    np.testing.assert_array_equal(b1, a1)
    np.testing.assert_allclose(b1, ref1, rtol=1e-4, atol=2e-5)
    (a2, b2), ref2 = run_both(g2, 12, 100, 2)
    np.testing.assert_array_equal(b2, a2)
    np.testing.assert_allclose(b2, ref2, rtol=1e-4, atol=2e-5)


def test_noalloc_refuses_beyond_its_scratch(g2):
    p = g2.to_device(np.zeros(4, np.float32))
    rc = g2._lib.g2_attn_1q_noalloc(p.ptr, p.ptr, p.ptr, p.ptr, 0, 10, 65 * 64, 65, 1024, 0, C.c_float(0.125))
    assert rc == g2.G2_E_LIMIT and "static scratch" in g2.last_error()


def _hip():
    hip = C.CDLL("libamdhip64.so")
    vp = C.c_void_p
    hip.hipStreamBeginCapture.argtypes = [vp, C.c_int]
    hip.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
    hip.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
    hip.hipGraphLaunch.argtypes = [vp, vp]
    hip.hipStreamSynchronize.argtypes = [vp]
    hip.hipGraphExecDestroy.argtypes = [vp]
    hip.hipGraphDestroy.argtypes = [vp]
    return hip


def test_noalloc_under_graph_capture(g2):
    hip = _hip()
    stream = g2._lib.g2_stream()
    assert stream, "g2_stream returned NULL after g2_init"
    NH, T = 25, 777
    qkv, kc, vc, D, S = inputs(NH, 3)
    d_qkv, d_k, d_v = g2.to_device(qkv), g2.to_device(kc), g2.to_device(vc)
    d_out = g2.DevBuf(D * 4)
    # eager result of the inputs the graph will hold
    g2.attn_1q_noalloc(d_qkv, d_k, d_v, d_out, 0, T, D, NH, S, 0, SCALE)
    g2.sync()
    eager = d_out.download(np.float32, D)
    np.testing.assert_allclose(eager, oracle_out(qkv, kc, vc, T, D, NH, S), rtol=1e-4, atol=2e-5)
    # other inputs for the eager calls between the replays
    q2, k2, v2, _, _ = inputs(NH, 4)
    e_qkv, e_k, e_v = g2.to_device(q2), g2.to_device(k2), g2.to_device(v2)
    e_out = g2.DevBuf(D * 4)

    graph, exe = C.c_void_p(), C.c_void_p()
    assert hip.hipStreamBeginCapture(stream, 1) == 0  # hipStreamCaptureModeThreadLocal
    rc = g2._lib.g2_attn_1q_noalloc(d_qkv.ptr, d_k.ptr, d_v.ptr, d_out.ptr, 0, T, D, NH, S, 0, C.c_float(SCALE))
    assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
    assert rc == 0, g2.last_error()
    assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
    try:
        for rep in range(3):
            print(f"[noalloc] graph replay {rep}", flush=True)
            g2.check(g2._lib.g2_memset(d_out.ptr, 0, D * 4))
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            np.testing.assert_array_equal(d_out.download(np.float32, D), eager, err_msg=f"replay {rep}")
            # eager work between replays: the static array now holds other partials
            g2.attn_1q_noalloc(e_qkv, e_k, e_v, e_out, 0, 1000 - 100 * rep, D, NH, S, 0, SCALE)
            g2.sync()
    finally:
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
