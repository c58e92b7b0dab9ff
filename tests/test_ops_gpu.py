"""GPU parity of every reference operator against the CPU oracle.

Shapes are the isolated operator sweep (matvec N x K in {2304x768, 768x768,
3072x768, 768x3072, 50257x768, 6400x1600, 50257x1600}, GEMM M in
{64,256,1024} over the same N x K, single-query attention over 25 heads of
dim 64 at KV length 1..1024), fp32 and fp16 weights, seeded N(0,1) inputs.
Integer/copy operators (embed, split_kv) must be bit-exact; arithmetic
operators must agree within the fp32 summation bound of tests/parity.py.
"""
import math

import numpy as np
import pytest

from oracle import oracle
from parity import EPS32, assert_close_bound, dot_bound

pytestmark = pytest.mark.gpu

MV_SHAPES = [(2304, 768), (768, 768), (3072, 768), (768, 3072), (50257, 768), (6400, 1600), (50257, 1600)]


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def f16_round(a):
    return a.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("N,K", MV_SHAPES)
def test_matvec_sweep(g2, N, K, f16):
    A = rnd(K, 1)
    B = rnd((K, N), 2)
    bias = rnd(N, 3)
    if f16:
        B = f16_round(B)
    dA, dB = g2.to_device(A), g2.to_device(g2.convert_f16(B) if f16 else B)
    dbias, dC = g2.to_device(bias), g2.DevBuf(N * 4)
    g2.matvec(dA, dB, dbias, None, dC, N, K, 0, f16=f16)
    got = dC.download(np.float32, N)
    ref = oracle.matvec(A, B, bias, None, N, K) if N % 4 == 0 else oracle.matvec_scalar(A, B, bias, None, N, K)
    assert_close_bound(got, ref, dot_bound(np.abs(A), np.abs(B), K), what=f"matvec {N}x{K}")


ROWS_SHAPES = MV_SHAPES + [(4800, 1600), (1600, 1600), (1600, 6400), (5, 8), (3, 1024), (77, 2048),
                           (1000, 4096), (64, 8192), (33, 5120), (50257, 1280)]


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("N,K", ROWS_SHAPES)
def test_matvec_rows(g2, N, K, f16):
    """The fused model's packed matvec: W = B^T stored [N,K], every lane
    shape (64 x 4, 256 x 4, 256 x 8 chunks) and the grid-stride path."""
    A, B, bias, res = rnd(K, 1), rnd((K, N), 2), rnd(N, 3), rnd(N, 4)
    if f16:
        B = f16_round(B)
    Wt = np.ascontiguousarray(B.T)
    dW = g2.to_device(g2.convert_f16(Wt) if f16 else Wt)
    dA, dbias = g2.to_device(A), g2.to_device(bias)
    dC = g2.DevBuf(N * 4)
    g2.matvec_rows(dA, dW, g2.F16 if f16 else g2.F32, dbias, None, dC, N, K)
    ref = oracle.matvec(A, B, bias, None, N, K) if N % 4 == 0 else oracle.matvec_scalar(A, B, bias, None, N, K)
    bound = dot_bound(np.abs(A), np.abs(B), K)
    assert_close_bound(dC.download(np.float32, N), ref, bound, what=f"rows {N}x{K}")
    dR = g2.to_device(res)
    g2.matvec_rows(dA, dW, g2.F16 if f16 else g2.F32, dbias, dR, dR, N, K)
    ref = oracle.matvec(A, B, bias, res, N, K) if N % 4 == 0 else oracle.matvec_scalar(A, B, bias, res, N, K)
    assert_close_bound(dR.download(np.float32, N), ref, bound, slack=2e-6, what=f"rows resid {N}x{K}")


def test_matvec_rows_rejects(g2):
    buf = g2.DevBuf(1 << 16)
    with pytest.raises(g2.G2Error):
        g2.matvec_rows(buf, buf, g2.F16, None, None, buf, 4, 12)  # K % 8
    with pytest.raises(g2.G2Error):
        g2.matvec_rows(buf, buf, g2.F32, None, None, buf, 4, 8196)  # K above 8192
    with pytest.raises(g2.G2Error):
        g2.matvec_rows(buf, buf, g2.F32, None, None, buf, 4, 8, apply_gelu=1)


@pytest.mark.parametrize("N,K", [(768, 768), (3072, 768), (7, 5), (13, 1000), (4, 1), (1, 33)])
@pytest.mark.parametrize("gelu", [0, 1])
def test_matvec_epilogues(g2, N, K, gelu):
    """bias + residual + GELU, residual aliasing C (in-place, main.c:1815)."""
    A, B, bias, res = rnd(K, 11), rnd((K, N), 12), rnd(N, 13), rnd(N, 14)
    dA, dB, dbias = g2.to_device(A), g2.to_device(B), g2.to_device(bias)
    dC = g2.to_device(res)
    g2.matvec(dA, dB, dbias, dC, dC, N, K, gelu)
    got = dC.download(np.float32, N)
    ref = oracle.matvec(A, B, bias, res, N, K, gelu) if N % 4 == 0 else oracle.matvec_scalar(A, B, bias, res, N, K, gelu)
    bound = dot_bound(np.abs(A), np.abs(B), K) * (1.2 if gelu else 1.0)
    assert_close_bound(got, ref, bound, slack=4e-6, what="matvec epilogue")


def test_matvec_null_bias(g2):
    N, K = 2304, 768
    A, B = rnd(K, 21), rnd((K, N), 22)
    dA, dB, dC = g2.to_device(A), g2.to_device(B), g2.DevBuf(N * 4)
    g2.matvec(dA, dB, None, None, dC, N, K)
    ref = oracle.matvec(A, B, None, None, N, K)
    assert_close_bound(dC.download(np.float32, N), ref, dot_bound(np.abs(A), np.abs(B), K), what="no bias")


def test_matvec_one_hot_exact(g2):
    """One-hot A picks a row of B: exact, plus bias (closed form)."""
    N, K = 3072, 768
    A = np.zeros(K, np.float32)
    A[317] = 1.0
    B, bias = rnd((K, N), 31), rnd(N, 32)
    dC = g2.DevBuf(N * 4)
    g2.matvec(g2.to_device(A), g2.to_device(B), g2.to_device(bias), None, dC, N, K)
    np.testing.assert_array_equal(dC.download(np.float32, N), B[317] + bias)


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("ks", [1, 2, 4, 8])
@pytest.mark.parametrize("N,K", [(768, 768), (768, 3072), (1600, 6400), (1600, 1600)])
def test_matvec_splitk(g2, N, K, ks, f16):
    """matvec4_sk partials (strided slices) and reduce_partial with the
    in-place residual, as decode's attn_proj/ffn2 use them."""
    A, B, bias, res = rnd(K, 41), rnd((K, N), 42), rnd(N, 43), rnd(N, 44)
    if f16:
        B = f16_round(B)
    dA, dB = g2.to_device(A), g2.to_device(g2.convert_f16(B) if f16 else B)
    dP = g2.DevBuf(ks * N * 4)
    g2.matvec_sk(dA, dB, dP, N, K, ks, f16=f16)
    got_p = dP.download(np.float32, ks * N).reshape(ks, N)
    ref_p = oracle.matvec4_sk(A, B, N, K, ks)
    for s in range(ks):
        sl = slice(s, K, ks)
        assert_close_bound(got_p[s], ref_p[s], dot_bound(np.abs(A[sl]), np.abs(B[sl]), len(A[sl])),
                           what=f"slice {s}")
    dC = g2.to_device(res)
    g2.reduce_partial(dP, g2.to_device(bias), dC, dC, N, ks, 0)
    ref = oracle.reduce_partial(ref_p, bias, res, N, ks)
    assert_close_bound(dC.download(np.float32, N), ref, dot_bound(np.abs(A), np.abs(B), K), slack=2e-6,
                       what="reduce")


GEMM_CASES = [(M, N, K) for M in (64, 256) for (N, K) in MV_SHAPES] + \
             [(1024, N, K) for (N, K) in MV_SHAPES if N < 50000] + [(1, 5, 3), (65, 67, 19), (3, 4800, 1600)]


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("M,N,K", GEMM_CASES)
def test_matmul(g2, M, N, K, f16):
    A, B, bias = rnd((M, K), 51), rnd((K, N), 52), rnd(N, 53)
    if f16:
        B = f16_round(B)
    dC = g2.DevBuf(M * N * 4)
    g2.matmul(g2.to_device(A), g2.to_device(g2.convert_f16(B) if f16 else B), g2.to_device(bias), dC, M, N, K,
              f16=f16)
    ref = oracle.matmul(A, B, bias, M, N, K)
    bound = dot_bound(np.abs(A).astype(np.float64), np.abs(B).astype(np.float64), K)
    assert_close_bound(dC.download(np.float32, M * N).reshape(M, N), ref, bound, what=f"matmul {M}x{N}x{K}")


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("K", [768, 1600])
def test_matmul_vocab_rows_sampled(g2, K, f16):
    """The 1024-row GEMM over the 50257-wide vocabulary (the operator
    sweep's largest case): every output row depends on its own A row only,
    so the GPU's full 1024 x 50257 product is checked row for row against
    the oracle run on a sample of 48 rows (first, last and spread rows,
    every column), which keeps the oracle to seconds."""
    M, N = 1024, 50257
    A, B, bias = rnd((M, K), 54), rnd((K, N), 55), rnd(N, 56)
    if f16:
        B = f16_round(B)
    dC = g2.DevBuf(M * N * 4)
    g2.matmul(g2.to_device(A), g2.to_device(g2.convert_f16(B) if f16 else B), g2.to_device(bias), dC, M, N, K,
              f16=f16)
    got = dC.download(np.float32, M * N).reshape(M, N)
    rows = np.unique(np.concatenate([[0, 1, 63, 64, 127, 128, 511, 512, 1022, 1023],
                                     np.random.default_rng(57).choice(M, 38, replace=False)]))
    ref = oracle.matmul(A[rows], B, bias, len(rows), N, K)
    bound = dot_bound(np.abs(A[rows]).astype(np.float64), np.abs(B).astype(np.float64), K)
    assert_close_bound(got[rows], ref, bound, what=f"matmul {M}x{N}x{K} sampled rows")
    assert np.isfinite(got).all()


def test_matmul_sweep_constant(g2):
    """The reference's tile-sweep known answer (main.c:750-753): A=B=0.01
    gives C = K*1e-4."""
    M, N, K = 64, 768, 3072
    A = np.full((M, K), 0.01, np.float32)
    B = np.full((K, N), 0.01, np.float32)
    dC = g2.DevBuf(M * N * 4)
    g2.matmul(g2.to_device(A), g2.to_device(B), None, dC, M, N, K)
    np.testing.assert_allclose(dC.download(np.float32, M * N), K * 1e-4, rtol=1e-4)


@pytest.mark.parametrize("E,rows", [(768, 1), (1600, 1), (1280, 7), (64, 3), (1000, 2)])
def test_layernorm(g2, E, rows):
    x = rnd((rows, E), 61) * 3 + 0.5
    g, b = rnd(E, 62), rnd(E, 63)
    dO = g2.DevBuf(rows * E * 4)
    g2.layernorm(g2.to_device(x), dO, g2.to_device(g), g2.to_device(b), E, rows)
    ref = oracle.layernorm(x, g, b, E, rows)
    np.testing.assert_allclose(dO.download(np.float32, rows * E).reshape(rows, E), ref, rtol=2e-5, atol=2e-5)


def test_layernorm_constant_row(g2):
    """A constant row normalises to beta (closed form)."""
    E = 768
    x = np.full((1, E), 3.25, np.float32)
    g, b = rnd(E, 64), rnd(E, 65)
    dO = g2.DevBuf(E * 4)
    g2.layernorm(g2.to_device(x), dO, g2.to_device(g), g2.to_device(b), E, 1)
    np.testing.assert_array_equal(dO.download(np.float32, E), b)


def test_add_gelu(g2):
    n = 100003
    a, b = rnd(n, 71), rnd(n, 72)
    da = g2.to_device(a)
    g2.add(da, g2.to_device(b), n)
    np.testing.assert_array_equal(da.download(np.float32, n), oracle.add_inplace(a, b))
    x = rnd(n, 73) * 4
    dx = g2.to_device(x)
    g2.gelu(dx, n)
    np.testing.assert_allclose(dx.download(np.float32, n), oracle.gelu(x), rtol=4e-6, atol=1e-6)


@pytest.mark.parametrize("E,seq,start", [(768, 1, 300), (1600, 64, 0), (1280, 5, 1019)])
def test_embed_exact(g2, E, seq, start):
    V = 50257
    wte, wpe = rnd((V, E), 81), rnd((1024, E), 82)
    ids = np.random.default_rng(83).integers(0, V, seq).astype(np.int32)
    dO = g2.DevBuf(seq * E * 4)
    g2.embed(g2.to_device(wte), g2.to_device(wpe), dO, E, seq, start, g2.to_device(ids))
    np.testing.assert_array_equal(dO.download(np.float32, seq * E).reshape(seq, E),
                                  oracle.embed(wte, wpe, E, seq, start, ids))


@pytest.mark.parametrize("D,T,start", [(768, 1, 500), (1600, 37, 0), (1024, 3, 1021)])
def test_split_kv_exact(g2, D, T, start):
    S = 1024
    qkv = rnd((T, 3 * D), 91)
    kc0, vc0 = rnd(D * S, 92), rnd(S * D, 93)
    dk, dv = g2.to_device(kc0), g2.to_device(vc0)
    g2.split_kv(g2.to_device(qkv), dk, dv, start, T, D, S)
    rk, rv = oracle.split_kv(qkv, kc0, vc0, start, T, D, S)
    np.testing.assert_array_equal(dk.download(np.float32, D * S), rk)
    np.testing.assert_array_equal(dv.download(np.float32, S * D), rv)


ATTN_T = [1, 2, 63, 64, 65, 255, 511, 777, 1023, 1024]


@pytest.mark.parametrize("T", ATTN_T)
@pytest.mark.parametrize("NH", [25, 12])
def test_attention_ops(g2, NH, T):
    """attn_scores_1q -> attn_softmax_1q -> attn_out_1q, and the fused
    attn_1q, against the oracle chain (25 heads x 64 = GPT-2 XL)."""
    DH, S = 64, 1024
    D = NH * DH
    qkv = rnd(3 * D, 101)
    kc = rnd(D * S, 102)
    vc = rnd(S * D, 103)
    scale = 1.0 / math.sqrt(DH)
    dqkv, dk, dv = g2.to_device(qkv), g2.to_device(kc), g2.to_device(vc)
    dS = g2.to_device(np.zeros(NH * S, np.float32))
    g2.attn_scores_1q(dqkv, dk, dS, 0, T, D, DH, NH, S, scale)
    ref_s = oracle.attn_scores_1q(qkv, kc, 0, T, D, DH, NH, S, scale)
    got_s = dS.download(np.float32, NH * S).reshape(NH, S)
    q_abs = np.abs(qkv[:D]).reshape(NH, DH)
    k_abs = np.abs(kc).reshape(NH, DH, S)
    bound = np.stack([2 * DH * EPS32 * scale * (q_abs[h] @ k_abs[h]) for h in range(NH)])
    assert_close_bound(got_s[:, :T], ref_s[:, :T], bound[:, :T], what="scores")
    g2.attn_softmax_1q(dS, T, NH)
    ref_p = oracle.attn_softmax_1q(ref_s, T, NH)
    got_p = dS.download(np.float32, NH * S).reshape(NH, S)
    np.testing.assert_allclose(got_p[:, :T], ref_p[:, :T], rtol=2e-5, atol=1e-7)
    np.testing.assert_allclose(got_p[:, :T].sum(axis=1), 1.0, rtol=1e-5)
    dO = g2.to_device(np.zeros(D, np.float32))
    g2.attn_out_1q(dS, dv, dO, T, D, DH, 0)
    ref_o = oracle.attn_out_1q(ref_p, vc, T, D, DH, 0, D)
    np.testing.assert_allclose(dO.download(np.float32, D), ref_o, rtol=1e-4, atol=2e-5)
    dF = g2.to_device(np.zeros(D, np.float32))
    g2.attn_1q(dqkv, dk, dv, dF, 0, T, D, NH, S, 0, scale)
    np.testing.assert_allclose(dF.download(np.float32, D), ref_o, rtol=1e-4, atol=2e-5)


def test_softmax_uniform(g2):
    """Equal scores give 1/T exactly enough (closed form)."""
    NH, S, T = 4, 1024, 640
    dS = g2.to_device(np.full(NH * S, 0.37, np.float32))
    g2.attn_softmax_1q(dS, T, NH)
    got = dS.download(np.float32, NH * S).reshape(NH, S)[:, :T]
    np.testing.assert_allclose(got, 1.0 / T, rtol=1e-6)


def test_attn_out_one_hot(g2):
    """One-hot probabilities select a V row exactly (closed form)."""
    NH, DH, S, T = 12, 64, 1024, 300
    D = NH * DH
    P = np.zeros((NH, S), np.float32)
    P[:, 123] = 1.0
    vc = rnd(S * D, 111)
    dO = g2.DevBuf(D * 4)
    g2.attn_out_1q(g2.to_device(P), g2.to_device(vc), dO, T, D, DH, 0)
    np.testing.assert_array_equal(dO.download(np.float32, D), vc.reshape(S, D)[123])


def test_error_paths(g2):
    """Invalid arguments come back as error codes, never as launches."""
    buf = g2.DevBuf(4096)
    with pytest.raises(g2.G2Error) as e:
        g2.matvec(None, buf, None, None, buf, 4, 4)
    assert e.value.code == g2.G2_E_ARG
    with pytest.raises(g2.G2Error):
        g2.matvec_sk(buf, buf, buf, 8, 8, 9)
    with pytest.raises(g2.G2Error):
        g2.matvec_sk(buf, buf, buf, 6, 8, 2)  # N % 4 != 0
    with pytest.raises(g2.G2Error):
        g2.attn_softmax_1q(buf, 1025, 1)
    with pytest.raises(g2.G2Error):
        g2.split_kv(buf, buf, buf, 1020, 8, 4, 1024)
    with pytest.raises(g2.G2Error):
        g2.attn_1q(buf, buf, buf, buf, 0, 10, 100, 2, 1024, 0, 0.125)  # head dim != 64
    with pytest.raises(g2.G2Error):
        g2.embed(buf, buf, buf, 8, 2, 1023, buf)
