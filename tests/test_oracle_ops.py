"""Pins of the CPU oracle's operators (CPU only).

The reference ships no tests or golden vectors, so each oracle function is
checked against what the mathematics fixes:
  - float64 library routines (numpy matmul, torch layer_norm / softmax /
    gelu(tanh)) within the fp32 summation bound, on non-square shapes so a
    transposed operand or a wrong index fails;
  - closed forms (constant inputs, one-hot operands, uniform scores);
  - brute force on tiny inputs: a literal emulation of the reference
    kernels' accumulation order (sequential k with fused multiply-add,
    four interleaved partial sums, strided split-K slices, 64-lane tree
    softmax), which must agree bit for bit.
"""
import math

import numpy as np
import pytest

from oracle import oracle
from parity import EPS32, assert_close_bound, dot_bound



def _torch():
    """torch, imported only inside the CPU tests that use it: a GPU test
    session then never loads torch's bundled HIP runtime beside the one
    libg2hip is linked against (two HIP runtimes in one process)."""
    import torch

    return torch

def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def f32(x):
    return float(np.float32(x))


def fma32(a, b, c):
    """fp32 fused multiply-add: a*b is exact in float64, one rounding after
    the add (double rounding is negligible for these tiny brute-force cases)."""
    return f32(float(a) * float(b) + float(c))


def gelu64(x):
    torch = _torch()
    x = torch.tensor(np.asarray(x, np.float64))
    return torch.nn.functional.gelu(x, approximate="tanh").numpy()


# ------------------------------------------------------------- matmul / matvec

@pytest.mark.parametrize("M,N,K", [(5, 7, 3), (64, 768, 3072), (33, 129, 65)])
def test_matmul_vs_float64(M, N, K):
    A, B, bias = rnd((M, K), 1), rnd((K, N), 2), rnd(N, 3)
    got = oracle.matmul(A, B, bias, M, N, K)
    ref = A.astype(np.float64) @ B.astype(np.float64) + bias
    assert_close_bound(got, ref, dot_bound(np.abs(A).astype(np.float64), np.abs(B).astype(np.float64), K) / 2,
                       what="matmul")


def test_matmul_sequential_fma_order():
    M, N, K = 3, 5, 9
    A, B, bias = rnd((M, K), 4), rnd((K, N), 5), rnd(N, 6)
    got = oracle.matmul(A, B, bias, M, N, K)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc = fma32(A[m, k], B[k, n], acc)
            assert got[m, n] == np.float32(f32(acc + float(bias[n])))


def test_matmul_sweep_known_answer():
    """main.c:750-753: A=B=0.01, M=64, N=E, K=F gives C = K*1e-4."""
    M, N, K = 64, 768, 3072
    got = oracle.matmul(np.full((M, K), 0.01, np.float32), np.full((K, N), 0.01, np.float32), None, M, N, K)
    np.testing.assert_allclose(got, K * 1e-4, rtol=1e-4)


@pytest.mark.parametrize("N,K", [(2304, 768), (50257, 768), (13, 1000), (768, 3072)])
@pytest.mark.parametrize("gelu", [0, 1])
def test_matvec_vs_float64(N, K, gelu):
    A, B, bias, res = rnd(K, 7), rnd((K, N), 8), rnd(N, 9), rnd(N, 10)
    got = oracle.matvec(A, B, bias, res, N, K, gelu)
    pre = A.astype(np.float64) @ B.astype(np.float64) + bias + res
    ref = gelu64(pre) if gelu else pre
    assert_close_bound(got, ref, dot_bound(np.abs(A), np.abs(B), K), slack=2e-6, what="matvec")


def test_matvec4_order_bit_exact():
    """matvec4 (math.cl:185-226): one accumulator per column, sequential k."""
    N, K = 8, 11
    A, B, bias, res = rnd(K, 11), rnd((K, N), 12), rnd(N, 13), rnd(N, 14)
    got = oracle.matvec(A, B, bias, res, N, K, 0)
    for n in range(N):
        s = 0.0
        for k in range(K):
            s = fma32(A[k], B[k, n], s)
        s = f32(f32(s + float(bias[n])) + float(res[n]))
        assert got[n] == np.float32(s)


def test_matvec_scalar_order_bit_exact():
    """matvec (math.cl:152-182): four interleaved sums, tail into s0,
    sum = s0+s1+s2+s3 left to right."""
    N, K = 5, 11
    A, B = rnd(K, 15), rnd((K, N), 16)
    got = oracle.matvec_scalar(A, B, None, None, N, K)
    for n in range(N):
        s = [0.0] * 4
        k = 0
        while k + 4 <= K:
            for j in range(4):
                s[j] = fma32(A[k + j], B[k + j, n], s[j])
            k += 4
        while k < K:
            s[0] = fma32(A[k], B[k, n], s[0])
            k += 1
        tot = f32(f32(f32(s[0] + s[1]) + s[2]) + s[3])
        assert got[n] == np.float32(tot)


def test_matvec_one_hot():
    N, K = 3072, 768
    A = np.zeros(K, np.float32)
    A[5] = 1.0
    B, bias = rnd((K, N), 17), rnd(N, 18)
    np.testing.assert_array_equal(oracle.matvec(A, B, bias, None, N, K), B[5] + bias)


@pytest.mark.parametrize("ks", [1, 2, 3, 8])
def test_splitk_slices_and_reduce(ks):
    N, K = 64, 100
    A, B, bias, res = rnd(K, 19), rnd((K, N), 20), rnd(N, 21), rnd(N, 22)
    part = oracle.matvec4_sk(A, B, N, K, ks)
    for s in range(ks):
        ref = A[s::ks].astype(np.float64) @ B[s::ks].astype(np.float64)
        assert_close_bound(part[s], ref, dot_bound(np.abs(A[s::ks]), np.abs(B[s::ks]), len(A[s::ks])) / 2,
                           what=f"slice {s}")
    out = oracle.reduce_partial(part, bias, res, N, ks, 0)
    exp = np.zeros(N, np.float32)
    for s in range(ks):
        exp = (exp + part[s]).astype(np.float32)
    exp = ((exp + bias).astype(np.float32) + res).astype(np.float32)
    np.testing.assert_array_equal(out, exp)


def test_splitk_slice_is_strided_not_contiguous():
    """Slice s holds rows k = s, s+ks, ... (math.cl:242): with A = e_k the
    row lands in slice k mod ks."""
    N, K, ks = 8, 12, 4
    B = rnd((K, N), 23)
    for k in range(K):
        A = np.zeros(K, np.float32)
        A[k] = 1.0
        part = oracle.matvec4_sk(A, B, N, K, ks)
        for s in range(ks):
            np.testing.assert_array_equal(part[s], B[k] if s == k % ks else 0.0)


# -------------------------------------------------------- layernorm / gelu / add

@pytest.mark.parametrize("E,rows", [(768, 3), (1600, 1), (7, 2)])
def test_layernorm_vs_torch(E, rows):
    torch = _torch()
    x = rnd((rows, E), 24) * 2 + 0.3
    g, b = rnd(E, 25), rnd(E, 26)
    got = oracle.layernorm(x, g, b, E, rows)
    ref = torch.nn.functional.layer_norm(torch.tensor(x, dtype=torch.float64), (E,),
                                         torch.tensor(g, dtype=torch.float64),
                                         torch.tensor(b, dtype=torch.float64), eps=1e-5).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_layernorm_closed_forms():
    E = 64
    g, b = rnd(E, 27), rnd(E, 28)
    np.testing.assert_array_equal(oracle.layernorm(np.full((1, E), 2.5, np.float32), g, b, E, 1)[0], b)
    x = np.where(np.arange(E) % 2 == 0, 3.0, -3.0).astype(np.float32)[None]
    out = oracle.layernorm(x, np.ones(E, np.float32), np.zeros(E, np.float32), E, 1)[0]
    np.testing.assert_allclose(out, np.sign(x[0]) * 3.0 / math.sqrt(9.0 + 1e-5), rtol=1e-6)


def test_gelu_vs_torch_and_limits():
    x = np.linspace(-8, 8, 10001).astype(np.float32)
    np.testing.assert_allclose(oracle.gelu(x), gelu64(x), rtol=2e-6, atol=2e-7)
    assert oracle.gelu(np.zeros(1, np.float32))[0] == 0.0
    np.testing.assert_allclose(oracle.gelu(np.array([30.0], np.float32)), 30.0)


def test_add_inplace():
    a, b = rnd(100, 29), rnd(100, 30)
    np.testing.assert_array_equal(oracle.add_inplace(a, b), (a + b).astype(np.float32))


# ---------------------------------------------------------------- embed / kv

def test_embed_indexing():
    V, E, S = 50, 6, 1024
    wte, wpe = rnd((V, E), 31), rnd((S, E), 32)
    ids = np.array([3, 49, 0, 7], np.int32)
    got = oracle.embed(wte, wpe, E, 4, 10, ids)
    np.testing.assert_array_equal(got, wte[ids] + wpe[10:14])


def test_split_kv_layout():
    D, S, T, start = 6, 1024, 3, 100
    qkv = rnd((T, 3 * D), 33)
    kc, vc = oracle.split_kv(qkv, np.zeros(D * S, np.float32), np.zeros(S * D, np.float32), start, T, D, S)
    kc, vc = kc.reshape(D, S), vc.reshape(S, D)
    np.testing.assert_array_equal(kc[:, start:start + T], qkv[:, D:2 * D].T)
    np.testing.assert_array_equal(vc[start:start + T], qkv[:, 2 * D:])
    assert not kc[:, :start].any() and not vc[start + T:].any()


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("T", [1, 5, 64, 300, 1024])
def test_attention_chain_vs_float64(T):
    torch = _torch()
    NH, DH, S = 3, 64, 1024
    D = NH * DH
    qkv, kc, vc = rnd(3 * D, 34), rnd(D * S, 35), rnd(S * D, 36)
    scale = 1.0 / math.sqrt(DH)
    sc = oracle.attn_scores_1q(qkv, kc, 0, T, D, DH, NH, S, scale)
    q = qkv[:D].astype(np.float64).reshape(NH, DH)
    K = kc.astype(np.float64).reshape(NH, DH, S)[:, :, :T]
    ref_s = np.einsum("hd,hdt->ht", q, K) * scale
    np.testing.assert_allclose(sc[:, :T], ref_s, rtol=1e-5, atol=1e-5)
    p = oracle.attn_softmax_1q(sc, T, NH)
    ref_p = torch.softmax(torch.tensor(ref_s), dim=-1).numpy()
    np.testing.assert_allclose(p[:, :T], ref_p, rtol=2e-5, atol=1e-7)
    out = oracle.attn_out_1q(p, vc, T, D, DH, 0, D)
    V = vc.astype(np.float64).reshape(S, NH, DH)[:T]
    ref_o = np.einsum("ht,thd->hd", ref_p, V).reshape(D)
    np.testing.assert_allclose(out, ref_o, rtol=1e-4, atol=1e-5)


def test_softmax_tree_bit_exact():
    """64-lane strided pass then a tree (math.cl:425-455), brute force."""
    NH, S, T, lws = 1, 1024, 150, 64
    sc = rnd((NH, S), 37)
    got = oracle.attn_softmax_1q(sc, T, NH)
    row = [float(v) for v in sc[0, :T]]
    mx = [-1e30] * lws
    for l in range(lws):
        for j in range(l, T, lws):
            if row[j] > mx[l]:
                mx[l] = row[j]
    s = lws // 2
    while s > 0:
        for l in range(s):
            mx[l] = mx[l] if mx[l] > mx[l + s] else mx[l + s]
        s //= 2
    m = mx[0]
    e = [f32(math.exp(f32(v - m))) for v in row]  # expf to within an ulp
    sm = [0.0] * lws
    for l in range(lws):
        for j in range(l, T, lws):
            sm[l] = f32(sm[l] + e[j])
    s = lws // 2
    while s > 0:
        for l in range(s):
            sm[l] = f32(sm[l] + sm[l + s])
        s //= 2
    inv = f32(1.0 / sm[0])
    exp = np.array([f32(v * inv) for v in e], np.float32)
    np.testing.assert_allclose(got[0, :T], exp, rtol=3e-7, atol=0)


def test_softmax_uniform_and_one_hot_out():
    NH, S, T, DH = 2, 1024, 37, 64
    p = oracle.attn_softmax_1q(np.full((NH, S), 0.5, np.float32), T, NH)
    np.testing.assert_allclose(p[:, :T], 1.0 / T, rtol=1e-6)
    P = np.zeros((NH, S), np.float32)
    P[:, 9] = 1.0
    vc = rnd(S * NH * DH, 38)
    out = oracle.attn_out_1q(P, vc, T, NH * DH, DH, 0, NH * DH)
    np.testing.assert_array_equal(out, vc.reshape(S, NH * DH)[9])
