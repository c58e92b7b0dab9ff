/*
 * g2_kernels.hip -- gfx950 device code of the GPT-2 forward pass.
 *
 * Built with `hipcc --genco --offload-arch=gfx950` into one code object that
 * the C99 host loads with hipModuleLoadData and launches with
 * hipModuleLaunchKernel.  Every kernel is extern "C" and takes one argument
 * block from g2_kargs.h by value.
 *
 * Two families:
 *  - reference operators (same argument meaning as the math.cl kernels):
 *    matmul, matvec, matvec split-K + reduce, layernorm, add, gelu, embed,
 *    split_kv, attention scores / softmax / weighted sum;
 *  - fused decode/prefill kernels over output-major packed weights:
 *    LayerNorm-prologue matvecs with bias/GELU/residual/KV-scatter/argmax
 *    epilogues, split single-query attention with an in-kernel merge, MFMA
 *    GEMMs with the same epilogues, and causal prompt attention.
 *
 * Wavefronts are 64 lanes; work-groups are 256 threads (4 waves) unless a
 * kernel says otherwise.  All accumulation is fp32; fp16 weights are widened
 * in registers.
 */
#include <hip/hip_runtime.h>
#include "g2_kargs.h"
#include "g2_step_plan.h"
#include "g2_gemm_plan.h"
#include "g2_attn_plan.h"

#define G2K extern "C" __global__ __launch_bounds__(256)

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

#define G2_MAXK 6400 /* largest K of a packed matvec (ffn of GPT-2 XL) */

/* ---------------------------------------------------------------- helpers */

/* tanh-approximate GELU, the formula of math.cl:21-23. */
__device__ __forceinline__ float gelu_f(float v)
{
    return 0.5f * v * (1.0f + tanhf(0.7978845608f * (v + 0.044715f * v * v * v)));
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

/* Sum over a 256-thread work-group; every thread gets the total.  The four
 * wave totals are added in wave order. */
__device__ __forceinline__ float block_sum(float v, float *red4)
{
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red4[wave] = v;
    __syncthreads();
    const float t = ((red4[0] + red4[1]) + red4[2]) + red4[3];
    __syncthreads();
    return t;
}

/* Loads/stores that other work-groups read after an agent-scope fence. */
__device__ __forceinline__ float ld_agent(const float *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int clampi(int v, int lo, int hi)
{
    return v < lo ? lo : (v > hi ? hi : v);
}

/* Element access for f32 / f16 weight storage. */
template <typename T> __device__ __forceinline__ float ldw(const T *p, size_t i);
template <> __device__ __forceinline__ float ldw<float>(const float *p, size_t i) { return p[i]; }
template <> __device__ __forceinline__ float ldw<_Float16>(const _Float16 *p, size_t i) { return (float)p[i]; }

/* ======================================================================
 * Reference operators
 * ==================================================================== */

/* ---- matvec, reference layout B[K,N] (launch_matvec, main.c:1554-1576) ---
 * Pass 1: grid (ceil(N/256), splits).  Each work-group owns 256 columns (4 per
 * lane) and a contiguous k-range of rows_per_split rows; wave w takes rows
 * k0+w, k0+w+4, ...; the four wave sums are added in wave order into
 * partial[split][n].  Pass 2 is g2k_reduce. */
template <typename WT, bool VEC>
__device__ void mvkn_impl(const g2_mvkn_args &a)
{
    __shared__ float red[4][256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = blockIdx.x * 256 + lane * 4;
    const int k0 = blockIdx.y * a.rows_per_split;
    const int k1 = min(a.K, k0 + a.rows_per_split);
    const WT *B = (const WT *)a.B;
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
    if (VEC && col + 3 < a.N) {
        int k = k0 + wave;
        for (; k + 12 < k1; k += 16) {
            float av[4];
            float bv[4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const size_t base = (size_t)(k + 4 * u) * a.N + col;
                av[u] = a.A[k + 4 * u];
                if constexpr (sizeof(WT) == 4) {
                    const f32x4 w = *(const f32x4 *)((const float *)B + base);
                    bv[u][0] = w.x; bv[u][1] = w.y; bv[u][2] = w.z; bv[u][3] = w.w;
                } else {
                    const f16x4 w = *(const f16x4 *)((const _Float16 *)B + base);
                    bv[u][0] = (float)w.x; bv[u][1] = (float)w.y;
                    bv[u][2] = (float)w.z; bv[u][3] = (float)w.w;
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                acc0 = fmaf(av[u], bv[u][0], acc0);
                acc1 = fmaf(av[u], bv[u][1], acc1);
                acc2 = fmaf(av[u], bv[u][2], acc2);
                acc3 = fmaf(av[u], bv[u][3], acc3);
            }
        }
        for (; k < k1; k += 4) {
            const size_t base = (size_t)k * a.N + col;
            const float av = a.A[k];
            acc0 = fmaf(av, ldw(B, base + 0), acc0);
            acc1 = fmaf(av, ldw(B, base + 1), acc1);
            acc2 = fmaf(av, ldw(B, base + 2), acc2);
            acc3 = fmaf(av, ldw(B, base + 3), acc3);
        }
    } else {
        for (int k = k0 + wave; k < k1; k += 4) {
            const size_t base = (size_t)k * a.N;
            const float av = a.A[k];
            if (col + 0 < a.N) acc0 = fmaf(av, ldw(B, base + col + 0), acc0);
            if (col + 1 < a.N) acc1 = fmaf(av, ldw(B, base + col + 1), acc1);
            if (col + 2 < a.N) acc2 = fmaf(av, ldw(B, base + col + 2), acc2);
            if (col + 3 < a.N) acc3 = fmaf(av, ldw(B, base + col + 3), acc3);
        }
    }
    red[wave][lane * 4 + 0] = acc0;
    red[wave][lane * 4 + 1] = acc1;
    red[wave][lane * 4 + 2] = acc2;
    red[wave][lane * 4 + 3] = acc3;
    __syncthreads();
    const int t = threadIdx.x, n = blockIdx.x * 256 + t;
    if (n < a.N)
        a.partial[(size_t)blockIdx.y * a.N + n] =
            ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
}

G2K void g2k_mvkn_f32(const g2_mvkn_args a) { mvkn_impl<float, true>(a); }
G2K void g2k_mvkn_f32_s(const g2_mvkn_args a) { mvkn_impl<float, false>(a); }
G2K void g2k_mvkn_f16(const g2_mvkn_args a) { mvkn_impl<_Float16, true>(a); }
G2K void g2k_mvkn_f16_s(const g2_mvkn_args a) { mvkn_impl<_Float16, false>(a); }

/* ---- matvec4_sk (math.cl:229-246): slice s sums k = s, s+kslice, ... ------
 * grid (ceil(N/4 / 256), kslice); one thread per (4 columns, slice). */
template <typename WT>
__device__ void mvsk_impl(const g2_mvsk_args &a)
{
    const int c4 = blockIdx.x * 256 + threadIdx.x;
    const int s = blockIdx.y;
    const int N4 = a.N >> 2;
    if (c4 >= N4 || s >= a.kslice) return;
    const WT *B = (const WT *)a.B;
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
    for (int k = s; k < a.K; k += a.kslice) {
        const size_t base = (size_t)k * a.N + (size_t)c4 * 4;
        const float av = a.A[k];
        acc0 = fmaf(av, ldw(B, base + 0), acc0);
        acc1 = fmaf(av, ldw(B, base + 1), acc1);
        acc2 = fmaf(av, ldw(B, base + 2), acc2);
        acc3 = fmaf(av, ldw(B, base + 3), acc3);
    }
    float *p = a.partial + (size_t)s * a.N + (size_t)c4 * 4;
    p[0] = acc0; p[1] = acc1; p[2] = acc2; p[3] = acc3;
}

G2K void g2k_mvsk_f32(const g2_mvsk_args a) { mvsk_impl<float>(a); }
G2K void g2k_mvsk_f16(const g2_mvsk_args a) { mvsk_impl<_Float16>(a); }

/* ---- reduce_partial (math.cl:249-280): slices added in order, then bias,
 * residual, GELU.  residual may alias C (each n is read then written by the
 * same thread). */
G2K void g2k_reduce(const g2_reduce_args a)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= a.N) return;
    float s = 0.f;
    for (int k = 0; k < a.nslice; ++k) s += a.partial[(size_t)k * a.N + n];
    if (a.bias) s += a.bias[n];
    if (a.residual) s += a.residual[n];
    if (a.apply_gelu) s = gelu_f(s);
    a.C[n] = s;
}

/* An fp32 value as the two fp16 halves the split-activation GEMMs take:
 * hi = fp16(v), lo = fp16(v - hi), both round-to-nearest-even. */
__device__ __forceinline__ void split_store(uint16_t *hi, uint16_t *lo, size_t i, float v)
{
    /* v is the rounded fp32 value, exactly what a consumer splitting the
     * stored fp32 sees: the register barrier keeps the producer's last
     * operation out of the conversions (a product would otherwise be
     * rounded to fp16 once, by v_fma_mixlo_f16, instead of to fp32 first),
     * and contract(off) keeps it out of v - hi */
#pragma clang fp contract(off)
    asm volatile("" : "+v"(v));
    const _Float16 h = (_Float16)v;
    const _Float16 l = (_Float16)(v - (float)h);
    hi[i] = __builtin_bit_cast(uint16_t, h);
    lo[i] = __builtin_bit_cast(uint16_t, l);
}

/* The halves of split_store as values: hi16(v) + lo16(v) represents v to
 * ~22 significant bits. */
__device__ __forceinline__ _Float16 hi16(float v) { return (_Float16)v; }
__device__ __forceinline__ _Float16 lo16(float v)
{
#pragma clang fp contract(off)
    return (_Float16)(v - (float)(_Float16)v);
}

/* Two fp32 values as packed fp16 halves, low word first: h holds hi16(a),
 * hi16(b) and l holds lo16(a), lo16(b), each half rounded to nearest even
 * from the fp32 value, two per packed v_cvt_pk_f16_f32 (measured equal to
 * the scalar conversion on 4M values down to fp16 subnormals). */
__device__ __forceinline__ void split2(float a, float b, unsigned &h, unsigned &l)
{
    /* a, b rounded to fp32 before the conversions, as in split_store */
#pragma clang fp contract(off)
    asm volatile("" : "+v"(a), "+v"(b));
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const f2 v = {a, b};
    const h2 hv = __builtin_convertvector(v, h2);
    const h2 lv = __builtin_convertvector(v - __builtin_convertvector(hv, f2), h2);
    h = __builtin_bit_cast(unsigned, hv);
    l = __builtin_bit_cast(unsigned, lv);
}

/* The qkv epilogue of output (m, n), v final: columns < E to q_out[m][n];
 * key columns E..2E-1 to the transposed K cache at position pos0 + m and,
 * when kh is set, as fp16 halves to kh/kl [position][E]; value columns
 * 2E..3E-1 to the V cache and as halves to vth/vtl [E][S] (transposed).
 * The halves are the staged operands of g2k_attn_prefill_h16. */
struct qkv_dst {
    float *q_out, *k_cache, *v_cache;
    uint16_t *kh, *kl, *vth, *vtl;
    int E, S, pos0;
};
template <typename ARGS>
__device__ __forceinline__ qkv_dst qkv_of(const ARGS &a)
{
    return qkv_dst{a.q_out, a.k_cache, a.v_cache, a.kh, a.kl, a.vth, a.vtl, a.E, a.S, a.pos0};
}

/* The qkv epilogue of rows mb..mb+3 (those < M) of column n, the four
 * values a lane holds in a 16x16 MFMA result tile: the transposed K cache
 * and the transposed V halves take the four consecutive positions with one
 * 16-byte (fp32) or two 8-byte (halves) stores when all four rows exist
 * and the first position is a multiple of 4. */
__device__ __forceinline__ void qkv_store4(const qkv_dst &d, int mb, int M, int n, const f32x4 &v)
{
    const int E = d.E, pos = d.pos0 + mb;
    const bool full = mb + 3 < M && (pos & 3) == 0;
    if (n < E) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (mb + q < M) d.q_out[(size_t)(mb + q) * E + n] = v[q];
    } else if (n < 2 * E) {
        float *kc = d.k_cache + (size_t)(n - E) * d.S + pos;
        if (full) {
            *(f32x4 *)kc = v;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (mb + q < M) kc[q] = v[q];
        }
        if (d.kh) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (mb + q < M) split_store(d.kh, d.kl, (size_t)(pos + q) * E + (n - E), v[q]);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (mb + q < M) d.v_cache[(size_t)(pos + q) * E + (n - 2 * E)] = v[q];
        if (d.kh) {
            const size_t o = (size_t)(n - 2 * E) * d.S + pos;
            if (full) {
                uint2 hv, lv;
                split2(v[0], v[1], hv.x, lv.x);
                split2(v[2], v[3], hv.y, lv.y);
                *(uint2 *)(d.vth + o) = hv;
                *(uint2 *)(d.vtl + o) = lv;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (mb + q < M) split_store(d.vth, d.vtl, o + q, v[q]);
            }
        }
    }
}

/* ---- layernorm (math.cl:283-311): one work-group per row, two-pass mean and
 * biased variance, eps 1e-5, out = (x-mean)*inv_std*gamma + beta.  SPLIT:
 * the row is written as fp16 halves (g2_lnsplit_args), same arithmetic. */
template <bool SPLIT, typename ARGS>
__device__ void layernorm_impl(const ARGS &a)
{
    __shared__ float red4[4];
    const int row = blockIdx.x;
    if (row >= a.rows) return;
    const float *x = a.x + (size_t)row * a.E;
    float s = 0.f;
    for (int i = threadIdx.x; i < a.E; i += 256) s += x[i];
    const float mean = block_sum(s, red4) / (float)a.E;
    float q = 0.f;
    for (int i = threadIdx.x; i < a.E; i += 256) {
        const float d = x[i] - mean;
        q = fmaf(d, d, q);
    }
    const float var = block_sum(q, red4) / (float)a.E;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    for (int i = threadIdx.x; i < a.E; i += 256) {
        const float y = fmaf((x[i] - mean) * inv, a.gamma[i], a.beta[i]);
        if constexpr (SPLIT) split_store(a.hi, a.lo, (size_t)row * a.E + i, y);
        else a.out[(size_t)row * a.E + i] = y;
    }
}

G2K void g2k_layernorm(const g2_ln_args a) { layernorm_impl<false>(a); }
G2K void g2k_layernorm_split(const g2_lnsplit_args a) { layernorm_impl<true>(a); }

/* ---- add_inplace (math.cl:314-322) and gelu (math.cl:325-330) ---------- */
G2K void g2k_add(const g2_ew_args a)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < a.n; i += gridDim.x * 256)
        a.a[i] += a.b[i];
}

G2K void g2k_gelu(const g2_ew_args a)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < a.n; i += gridDim.x * 256)
        a.a[i] = gelu_f(a.a[i]);
}

/* ---- embed (math.cl:333-350); grid (ceil(E/256), rows). With a state
 * pointer the single row takes its token and position from the device. */
template <typename T>
__device__ void embed_impl(const g2_embed_args &a)
{
    const int d = blockIdx.x * 256 + threadIdx.x;
    const int i = blockIdx.y;
    if (d >= a.E || i >= a.seq_len) return;
    int tok, pos;
    if (a.state) {
        tok = a.state[G2S_TOK];
        pos = clampi(a.state[G2S_POS], 0, G2_KV_MAX_SEQ - 1);
    } else {
        tok = a.ids[i];
        pos = a.start_pos + i;
    }
    tok = clampi(tok, 0, 0x7fffffff);
    const T *wte = (const T *)a.wte, *wpe = (const T *)a.wpe;
    a.out[(size_t)i * a.E + d] =
        ldw(wte, (size_t)tok * a.E + d) + ldw(wpe, (size_t)pos * a.E + d);
}

G2K void g2k_embed_f32(const g2_embed_args a) { embed_impl<float>(a); }
G2K void g2k_embed_f16(const g2_embed_args a) { embed_impl<_Float16>(a); }

/* ---- split_kv (math.cl:367-383) ---------------------------------------- */
G2K void g2k_split_kv(const g2_splitkv_args a)
{
    const long n = (long)blockIdx.x * 256 + threadIdx.x;
    if (n >= (long)a.T * a.D) return;
    const int i = (int)(n / a.D), d = (int)(n % a.D);
    const int pos = a.start_pos + i;
    a.k_cache[(size_t)d * a.S + pos] = a.qkv[(size_t)i * 3 * a.D + a.D + d];
    a.v_cache[(size_t)pos * a.D + d] = a.qkv[(size_t)i * 3 * a.D + 2 * a.D + d];
}

/* ---- attn_scores_1q (math.cl:388-412); grid (NH, ceil(T/256)) ---------- */
G2K void g2k_attn_scores(const g2_scores_args a)
{
    const int h = blockIdx.x, j = blockIdx.y * 256 + threadIdx.x;
    if (h >= a.NH || j >= a.T) return;
    const float *q = a.qkv + a.q_base + (size_t)h * a.DH;
    const float *kc = a.k_cache + (size_t)h * a.DH * a.S + j;
    float s = 0.f;
    for (int k = 0; k < a.DH; ++k) s = fmaf(q[k], kc[(size_t)k * a.S], s);
    a.scores[(size_t)h * a.S + j] = s * a.scale;
}

/* ---- attn_softmax_1q (math.cl:415-456): one work-group per head, in place,
 * row stride G2_MAX_SEQ. */
G2K void g2k_attn_softmax(const g2_softmax_args a)
{
    __shared__ float red4[4];
    const int h = blockIdx.x;
    if (h >= a.NH) return;
    float *row = a.scores + (size_t)h * G2_KV_MAX_SEQ;
    float mx = -1e30f;
    for (int j = threadIdx.x; j < a.T; j += 256) mx = fmaxf(mx, row[j]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
    __syncthreads();
    float s = 0.f;
    for (int j = threadIdx.x; j < a.T; j += 256) {
        const float e = expf(row[j] - m);
        row[j] = e;
        s += e;
    }
    const float inv = 1.0f / block_sum(s, red4);
    for (int j = threadIdx.x; j < a.T; j += 256) row[j] *= inv;
}

/* ---- attn_out_1q (math.cl:459-476): grid ceil(D/64), block 1024: lane d of
 * the block's 64 dims, 16 waves split j (j = wave, wave+16, ...). */
extern "C" __global__ __launch_bounds__(1024) void g2k_attn_out(const g2_attnout_args a)
{
    __shared__ float red[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = blockIdx.x * 64 + lane;
    float o = 0.f;
    if (d < a.D) {
        const float *srow = a.scores + (size_t)(d / a.DH) * G2_KV_MAX_SEQ;
        for (int j = wave; j < a.T; j += 16)
            o = fmaf(srow[j], a.v_cache[(size_t)j * a.D + d], o);
    }
    red[wave][lane] = o;
    __syncthreads();
    if (wave == 0 && d < a.D) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < 16; ++w) s += red[w][lane];
        a.out[a.out_base + d] = s;
    }
}

/* ======================================================================
 * MFMA GEMM (prefill and the reference matmul)
 *
 * Tile 64x64x16, 256 threads = 2x2 waves of 32x32, each wave a 2x2 grid of
 * v_mfma_f32_16x16x4f32.  A [M,K] fp32 row-major; B [K,N] (BKN) or [N,K]
 * (BNK), fp32 or fp16 (widened when staged to LDS).  LDS tiles hold
 * As[m][k] and Bs[n][k] so both fragments read 4 consecutive k per lane
 * group.  Epilogues as in g2_gemm_args.
 * MFMA 16x16x4 f32 operand layout: lane l supplies A[l%16][l/16] and
 * B[l/16][l%16]; the result lane l holds rows 4*(l/16)+r, column l%16.
 * ==================================================================== */
enum { GEPI_STORE = 0, GEPI_GELU = 1, GEPI_RESID = 2, GEPI_QKV = 3, GEPI_PARTIAL = 4, GEPI_GELU_SPLIT = 5 };

/* Bias (and for GEPI_RESID the old C) added to a wave's 32x32 tile in one
 * branch-free pass before its stores, every load issued before the first
 * add: a load's wait placed among the stores would also wait for every
 * store issued before it (stores count in the same counter), once per
 * element.  mb, nb: the tile's first row and column. */
template <int EPI>
__device__ __forceinline__ void epi_add(f32x4 (&acc)[2][2], const g2_gemm_args &a, int mb, int nb, int lane, int M,
                                        int N)
{
    if constexpr (EPI != GEPI_PARTIAL) {
        float bj[2] = {0.f, 0.f};
        if (a.bias) {
#pragma unroll
            for (int j = 0; j < 2; ++j) bj[j] = a.bias[min(nb + j * 16 + (lane & 15), N - 1)];
        }
        float rv[2][2][4];
        if constexpr (EPI == GEPI_RESID) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        rv[i][j][q] = a.C[(size_t)min(mb + i * 16 + 4 * (lane >> 4) + q, M - 1) * N +
                                          min(nb + j * 16 + (lane & 15), N - 1)];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc[i][j][q] += bj[j];
                    if constexpr (EPI == GEPI_RESID) acc[i][j][q] += rv[i][j][q];
                    asm volatile("" : "+v"(acc[i][j][q])); /* not sunk into the stores */
                }
    }
}

template <typename BT, bool BNK, int EPI>
__device__ void gemm_impl(const g2_gemm_args &a)
{
    constexpr int BM = 64, BN = 64, BK = 16, LDK = BK + 1;
    __shared__ float As[BM * LDK];
    __shared__ float Bs[BN * LDK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int M = a.M, N = a.N, K = a.K;
    const BT *B = (const BT *)a.B;
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < K; k0 += BK) {
        /* A tile: thread -> row tid/4, k (tid%4)*4 .. +3 */
        {
            const int r = tid >> 2, kq = (tid & 3) * 4;
            const int gm = m0 + r, gk = k0 + kq;
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (gm < M) {
                const float *ap = a.A + (size_t)gm * K + gk;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gk + e < K) v[e] = ap[e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) As[r * LDK + kq + e] = v[e];
        }
        /* B tile into Bs[n][k] */
        if (BNK) {
            const int r = tid >> 2, kq = (tid & 3) * 4;
            const int gn = n0 + r, gk = k0 + kq;
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (gn < N) {
                const size_t base = (size_t)gn * K + gk;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gk + e < K) v[e] = ldw(B, base + e);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) Bs[r * LDK + kq + e] = v[e];
        } else {
            const int kr = tid >> 4, nq = (tid & 15) * 4;
            const int gk = k0 + kr, gn = n0 + nq;
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (gk < K) {
                const size_t base = (size_t)gk * N + gn;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gn + e < N) v[e] = ldw(B, base + e);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) Bs[(nq + e) * LDK + kr] = v[e];
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            float af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = As[(wm * 32 + i * 16 + (lane & 15)) * LDK + kk + (lane >> 4)];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = Bs[(wn * 32 + j * 16 + (lane & 15)) * LDK + kk + (lane >> 4)];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    epi_add<EPI>(acc, a, m0 + wm * 32, n0 + wn * 32, lane, M, N);
    if constexpr (EPI == GEPI_QKV) {
        const qkv_dst d = qkv_of(a);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn * 32 + j * 16 + (lane & 15);
                if (n < N) qkv_store4(d, m0 + wm * 32 + i * 16 + 4 * (lane >> 4), M, n, acc[i][j]);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                const int n = n0 + wn * 32 + j * 16 + (lane & 15);
                if (m >= M || n >= N) continue;
                const float v = acc[i][j][r];
                if (EPI == GEPI_STORE) {
                    a.C[(size_t)m * N + n] = v;
                } else if (EPI == GEPI_GELU) {
                    a.C[(size_t)m * N + n] = gelu_f(v);
                } else if (EPI == GEPI_RESID) {
                    a.C[(size_t)m * N + n] = v;
                }
            }
}

#define G2_GEMM(name, BT, BNK, EPI) \
    G2K void name(const g2_gemm_args a) { gemm_impl<BT, BNK, EPI>(a); }

G2_GEMM(g2k_gemm_kn_f32, float, false, GEPI_STORE)
G2_GEMM(g2k_gemm_kn_f16, _Float16, false, GEPI_STORE)
G2_GEMM(g2k_gemm_nk_f32_store, float, true, GEPI_STORE)
G2_GEMM(g2k_gemm_nk_f16_store, _Float16, true, GEPI_STORE)
G2_GEMM(g2k_gemm_nk_f32_gelu, float, true, GEPI_GELU)
G2_GEMM(g2k_gemm_nk_f16_gelu, _Float16, true, GEPI_GELU)
G2_GEMM(g2k_gemm_nk_f32_resid, float, true, GEPI_RESID)
G2_GEMM(g2k_gemm_nk_f16_resid, _Float16, true, GEPI_RESID)
G2_GEMM(g2k_gemm_nk_f32_qkv, float, true, GEPI_QKV)
G2_GEMM(g2k_gemm_nk_f16_qkv, _Float16, true, GEPI_QKV)

/* ======================================================================
 * fp32-weight GEMM of the fused prefill, C = A . W^T with W [N,K] packed
 * output-major (fp32): 64x64 tiles, 4 waves of 32x32 (2x2 fragments of
 * v_mfma_f32_16x16x4f32), K in steps of 32 streamed global -> LDS with
 * global_load_lds_dwordx4 into a three-step ring (two steps in flight, one
 * barrier per step).  Rows of a staged tile are 128 bytes, chunk c of row r
 * at slot c ^ (r / 2 % 8), so the 16 rows of a fragment read fall on
 * distinct banks.  A lane reads the 4 consecutive k of one chunk with one
 * 16-byte read and feeds them to 4 successive products: in product s, the
 * instruction's k index j (lane / 16) stands for k = 16 kk + 4 j + s, for A
 * and W alike, so the 4 products of a chunk pass cover its 16 k once.
 * Split-K: gridDim.z slices of whole steps (slices differ by at most one),
 * each writing its partial tile to part[z][M][N]; g2k_splitk_epi then sums
 * the slices in order and applies the epilogue.  With one slice the
 * epilogue runs here.  Requires K % 32 == 0.
 * ==================================================================== */
namespace sg {
constexpr int BM = 64, BN = 64, BK = 32, NS = 3;
constexpr int TB = BM * BK * 4; /* bytes of one 64 x 32 fp32 tile */
constexpr int STAGE = 2 * TB;   /* A, W: 16 KB */
typedef __attribute__((address_space(3))) void lds_t;

/* The wave's products of one step from the stage at st. */
__device__ __forceinline__ void mma(f32x4 (&acc)[2][2], const unsigned char *st, int wm, int wn, int lane)
{
    const int fr = lane & 15, g = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        const int c = 4 * kk + g;
        f32x4 af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = wm * 32 + i * 16 + fr;
            af[i] = *(const f32x4 *)(st + row * 128 + ((c ^ ((row >> 1) & 7)) << 4));
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int row = wn * 32 + j * 16 + fr;
            bf[j] = *(const f32x4 *)(st + TB + row * 128 + ((c ^ ((row >> 1) & 7)) << 4));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][q], bf[j][q], acc[i][j], 0, 0, 0);
    }
}
} /* namespace sg */

template <int EPI>
__device__ void sgemm_impl(const g2_gemm_args &a)
{
    using namespace sg;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[NS * STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int M = a.M, N = a.N, K = a.K;
    const int nkt = K / BK, ks = gridDim.z;
    const int s0 = (int)(((long)nkt * blockIdx.z) / ks), s1 = (int)(((long)nkt * (blockIdx.z + 1)) / ks);
    const int nk = s1 - s0;
    /* this lane's load sources: wave w fills rows 16w..16w+15 of each tile
     * with two instructions of 8 rows (lane -> row l/8, slot l%8, holding
     * the chunk that the swizzle puts there); rows past M or N read the
     * last row (their results are not stored) */
    const float *as[2], *bs[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int row = 16 * wave + 8 * h + (lane >> 3);
        const int ch = (lane & 7) ^ ((row >> 1) & 7);
        as[h] = a.A + (size_t)min(m0 + row, M - 1) * K + s0 * BK + 4 * ch;
        bs[h] = (const float *)a.B + (size_t)min(n0 + row, N - 1) * K + s0 * BK + 4 * ch;
    }
    /* step t's loads into stage buffer b (steps past the last reload it) */
    auto issue = [&](int t, int b) {
        const int k = min(t, nk - 1) * BK;
        unsigned char *st = lds + b * STAGE + (16 * wave) * 128;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            __builtin_amdgcn_global_load_lds(as[h] + k, (lds_t *)(st + h * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(bs[h] + k, (lds_t *)(st + TB + h * 1024), 16, 0, 0);
        }
    };
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    issue(0, 0);
    issue(1, 1);
    int cur = 0;
    for (int t = 0; t < nk; ++t) {
        /* step t has landed (the 4 loads per wave of step t+1 may remain in
         * flight); every wave is done with the buffer of step t-1 */
        asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
        issue(t + 2, cur == 0 ? 2 : cur - 1);
        mma(acc, lds + cur * STAGE, wm, wn, lane);
        cur = cur == 2 ? 0 : cur + 1;
    }
    /* no load may land in LDS after the work-group has ended */
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    if constexpr (EPI == GEPI_PARTIAL) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                    const int n = n0 + wn * 32 + j * 16 + (lane & 15);
                    if (m < M && n < N) a.part[((size_t)blockIdx.z * M + m) * N + n] = acc[i][j][r];
                }
        return;
    }
    epi_add<EPI>(acc, a, m0 + wm * 32, n0 + wn * 32, lane, M, N);
    if constexpr (EPI == GEPI_QKV) {
        const qkv_dst d = qkv_of(a);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn * 32 + j * 16 + (lane & 15);
                if (n < N) qkv_store4(d, m0 + wm * 32 + i * 16 + 4 * (lane >> 4), M, n, acc[i][j]);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                const int n = n0 + wn * 32 + j * 16 + (lane & 15);
                if (m >= M || n >= N) continue;
                const float v = acc[i][j][r];
                if (EPI == GEPI_GELU) {
                    a.C[(size_t)m * N + n] = gelu_f(v);
                } else if (EPI == GEPI_RESID) {
                    a.C[(size_t)m * N + n] = v;
                }
            }
}

#define G2_SGEMM(name, EPI) \
    G2K void name(const g2_gemm_args a) { sgemm_impl<EPI>(a); }
G2_SGEMM(g2k_sgemm_gelu, GEPI_GELU)
G2_SGEMM(g2k_sgemm_resid, GEPI_RESID)
G2_SGEMM(g2k_sgemm_qkv, GEPI_QKV)
G2_SGEMM(g2k_sgemm_partial, GEPI_PARTIAL)

/* The split-K epilogue of g2k_sgemm_partial and g2k_hgemm2_partial: v =
 * (part[0][m][n] + ... + part[ks-1][m][n]) + bias[n], then by epi: gelu
 * (C = gelu(v)), resid (C = C + v, in place), qkv (the K/V cache scatter
 * of GEPI_QKV), gelu as fp16 halves (GEPI_GELU_SPLIT: Ch, Cl).  Four
 * consecutive columns per thread (16-byte loads; N % 4 == 0), except qkv:
 * four consecutive rows of one column per thread, so that the transposed
 * K cache and V halves (position-minor) take a lane's four positions with
 * one store, as the GEMM's own qkv epilogue does, and q, V and the K
 * halves (column-minor) are stored by consecutive lanes.  The ks slice
 * loads (ks <= G2_SKEPI_MAXKS) are all issued before the first add, so a
 * sum costs one memory latency rather than one per slice. */
/* Four consecutive slice sums at offset o: (part[0][o..o+3] + ... +
 * part[ks-1][o..o+3]) in order; the ks loads (ks <= G2_SKEPI_MAXKS) are all
 * issued before the first add, so the sum costs one memory latency rather
 * than one per slice. */
__device__ __forceinline__ void slice_loads4(const float *part, size_t MN, size_t o, int ks,
                                             f32x4 (&p)[G2_SKEPI_MAXKS])
{
#pragma unroll
    for (int z = 0; z < G2_SKEPI_MAXKS; ++z)
        p[z] = z < ks ? *(const f32x4 *)(part + (size_t)z * MN + o) : (f32x4){0.f, 0.f, 0.f, 0.f};
}
__device__ __forceinline__ f32x4 slice_sum4(const f32x4 (&p)[G2_SKEPI_MAXKS], int ks)
{
    f32x4 v = p[0];
#pragma unroll
    for (int z = 1; z < G2_SKEPI_MAXKS; ++z)
        if (z < ks) v += p[z];
    return v;
}

G2K void g2k_splitk_epi(const g2_skepi_args a)
{
    const size_t MN = (size_t)a.M * a.N;
    const int N4 = a.N >> 2;
    if (a.epi == GEPI_QKV) {
        const qkv_dst d = qkv_of(a);
        const size_t n4s = (size_t)((a.M + 3) >> 2) * a.N;
        for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4s; i += (size_t)gridDim.x * 256) {
            const int n = (int)(i % a.N), mb = 4 * (int)(i / a.N);
            float p[4][G2_SKEPI_MAXKS];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const size_t o = (size_t)min(mb + q, a.M - 1) * a.N + n;
#pragma unroll
                for (int z = 0; z < G2_SKEPI_MAXKS; ++z) p[q][z] = z < a.ks ? a.part[(size_t)z * MN + o] : 0.f;
            }
            const float b = a.bias ? a.bias[n] : 0.f;
            f32x4 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float x = p[q][0];
#pragma unroll
                for (int z = 1; z < G2_SKEPI_MAXKS; ++z)
                    if (z < a.ks) x += p[q][z];
                v[q] = a.bias ? x + b : x;
            }
            qkv_store4(d, mb, a.M, n, v);
        }
        return;
    }
    const size_t n4s = (size_t)a.M * N4;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4s; i += (size_t)gridDim.x * 256) {
        const int m = (int)(i / N4), n = (int)(i % N4) * 4;
        const size_t o = (size_t)m * a.N + n;
        f32x4 p[G2_SKEPI_MAXKS];
        slice_loads4(a.part, MN, o, a.ks, p);
        const f32x4 b = a.bias ? *(const f32x4 *)(a.bias + n) : (f32x4){0.f, 0.f, 0.f, 0.f};
        const f32x4 c = a.epi == GEPI_RESID ? *(const f32x4 *)(a.C + o) : (f32x4){0.f, 0.f, 0.f, 0.f};
        f32x4 v = slice_sum4(p, a.ks);
        if (a.bias) v += b;
        if (a.epi == GEPI_GELU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) a.C[o + e] = gelu_f(v[e]);
        } else if (a.epi == GEPI_RESID) {
            *(f32x4 *)(a.C + o) = c + v;
        } else if (a.epi == GEPI_GELU_SPLIT) {
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = gelu_f(v[e]);
            uint2 hv, lv;
            split2(y[0], y[1], hv.x, lv.x);
            split2(y[2], y[3], hv.y, lv.y);
            *(uint2 *)(a.Ch + o) = hv;
            *(uint2 *)(a.Cl + o) = lv;
        }
    }
}

/* ======================================================================
 * fp16 MFMA GEMM for the fused prefill with fp16 weights:
 * C[M,N] = A[M,K] . W[N,K]^T + bias with the epilogues of g2_gemm_args.
 *
 * A is fp32.  It enters the fp16 matrix cores as two halves, a_hi =
 * fp16(a) and a_lo = fp16(a - a_hi), so every product a*w is computed as
 * a_hi*w + a_lo*w with 22 significant bits of a and fp32 accumulation; the
 * weights are exact in fp16.  This keeps the fp32 activations of the
 * reference (main.c:1739-1790 runs its matmuls in fp32) at twice the cost
 * of a plain fp16 product, still far below the fp32 MFMA rate.
 *
 * Tile 64x64x64, 256 threads = 2x2 waves of 32x32, each wave a 2x2 grid of
 * v_mfma_f32_16x16x32_f16: lane l supplies A[l%16][8(l/16)..+7] and
 * W[l%16][8(l/16)..+7] (8 consecutive k), the result lane l holds rows
 * 4(l/16)+r, column l%16.  Requires N % 64 == 0 and K % 64 == 0 (the
 * fused path's matrices: multiples of the head dim); rows >= M are zero.
 * ==================================================================== */
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));

template <int EPI>
__device__ void hgemm_impl(const g2_gemm_args &a)
{
    constexpr int BM = 64, BN = 64, BK = 64, LD = BK + 8; /* halves per LDS row */
    __shared__ __attribute__((aligned(16))) _Float16 Ah[BM * LD];
    __shared__ __attribute__((aligned(16))) _Float16 Al[BM * LD];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int M = a.M, N = a.N, Kfull = a.K;
    /* split-K (GEPI_PARTIAL): this work-group's K slice */
    const int K = EPI == GEPI_PARTIAL ? Kfull / a.ksplit : Kfull;
    const int kz0 = EPI == GEPI_PARTIAL ? (int)blockIdx.z * K : 0;
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    /* staging: thread -> tile row r, 16 consecutive k from kq */
    const int r = tid >> 2, kq = (tid & 3) * 16;
    const bool arow = m0 + r < M;
    const float *ap = a.A + (size_t)min(m0 + r, M - 1) * Kfull + kz0 + kq;
    const _Float16 *wrow = (const _Float16 *)a.B + (size_t)(n0 + r) * Kfull + kz0 + kq;
    const int fr = lane & 15, fk = 8 * (lane >> 4);

    /* the next tile's global loads are issued before the current tile's
     * matrix products, so they overlap */
    f32x4 av[4];
    h16x8 bv[2];
#pragma unroll
    for (int q = 0; q < 4; ++q) av[q] = *(const f32x4 *)(ap + 4 * q);
#pragma unroll
    for (int q = 0; q < 2; ++q) bv[q] = *(const h16x8 *)(wrow + 8 * q);
    for (int k0 = 0; k0 < K; k0 += BK) {
        h16x8 hi[2], lo[2];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float x = arow ? av[e >> 2][e & 3] : 0.f;
            const _Float16 h = (_Float16)x;
            hi[e >> 3][e & 7] = h;
            lo[e >> 3][e & 7] = (_Float16)(x - (float)h);
        }
        __syncthreads(); /* the previous tile has been consumed */
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            *(h16x8 *)(Ah + r * LD + kq + 8 * q) = hi[q];
            *(h16x8 *)(Al + r * LD + kq + 8 * q) = lo[q];
            *(h16x8 *)(Bs + r * LD + kq + 8 * q) = bv[q];
        }
        __syncthreads();
        {
            const int kn = min(k0 + BK, K - BK); /* the last tile reloads itself */
#pragma unroll
            for (int q = 0; q < 4; ++q) av[q] = *(const f32x4 *)(ap + kn + 4 * q);
#pragma unroll
            for (int q = 0; q < 2; ++q) bv[q] = *(const h16x8 *)(wrow + kn + 8 * q);
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            h16x8 afh[2], afl[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = (wm * 32 + i * 16 + fr) * LD + kk + fk;
                afh[i] = *(const h16x8 *)(Ah + row);
                afl[i] = *(const h16x8 *)(Al + row);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[j] = *(const h16x8 *)(Bs + (wn * 32 + j * 16 + fr) * LD + kk + fk);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afh[i], bf[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afl[i], bf[j], acc[i][j], 0, 0, 0);
                }
        }
    }

    epi_add<EPI>(acc, a, m0 + wm * 32, n0 + wn * 32, lane, M, N);
    if constexpr (EPI == GEPI_QKV) {
        const qkv_dst d = qkv_of(a);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn * 32 + j * 16 + (lane & 15);
                if (n < N) qkv_store4(d, m0 + wm * 32 + i * 16 + 4 * (lane >> 4), M, n, acc[i][j]);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + q;
                const int n = n0 + wn * 32 + j * 16 + (lane & 15);
                if (m >= M || n >= N) continue;
                const float v = acc[i][j][q];
                if (EPI == GEPI_PARTIAL) {
                    a.part[(size_t)blockIdx.z * M * N + (size_t)m * N + n] = v;
                    continue;
                }
                if (EPI == GEPI_STORE) {
                    a.C[(size_t)m * N + n] = v;
                } else if (EPI == GEPI_GELU) {
                    a.C[(size_t)m * N + n] = gelu_f(v);
                } else if (EPI == GEPI_RESID) {
                    a.C[(size_t)m * N + n] = v;
                }
            }
}

G2K void g2k_hgemm_partial(const g2_gemm_args a) { hgemm_impl<GEPI_PARTIAL>(a); }

/* The split-K residual epilogue: slices summed in order, then + bias, then
 * added to C (the order of the single-pass resid epilogue, with the dot
 * product summed per slice). */
G2K void g2k_splitk_resid(const g2_skred_args a)
{
    const size_t MN = (size_t)a.M * a.N;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < MN; i += (size_t)gridDim.x * 256) {
        /* every slice load issued before the first add (ks <= G2_SKEPI_MAXKS) */
        float p[G2_SKEPI_MAXKS];
#pragma unroll
        for (int z = 0; z < G2_SKEPI_MAXKS; ++z) p[z] = z < a.ks ? a.part[(size_t)z * MN + i] : 0.f;
        float v = p[0];
#pragma unroll
        for (int z = 1; z < G2_SKEPI_MAXKS; ++z)
            if (z < a.ks) v += p[z];
        const int n = (int)(i % (size_t)a.N);
        if (a.bias) v += a.bias[n];
        a.C[i] = v + a.C[i];
    }
}

/* ======================================================================
 * The same GEMM for prompts of more than 64 rows, on 128x128 tiles:
 * 16 waves in 4x4, each 32x32 = 2x2 blocks of v_mfma_f32_16x16x32_f16
 * with the fragment layout above, K in steps of 64.  The activations
 * arrive already split into their fp16 halves (Ah, Al: written so by the
 * producing LayerNorm, attention or GELU epilogue), so a step's three
 * tiles (a_hi, a_lo, weights; 128 rows x 128 B each) are plain fp16.
 *
 * The tiles go from global memory straight into LDS (global_load_lds_
 * dwordx4: lane l of an instruction writes 16 bytes at LDS base + 16 l),
 * three steps in a ring, issued two steps ahead; a step waits for its own
 * loads only (vmcnt(3): the 3 loads per wave of the step after it may
 * still be in flight), then one barrier.  The barrier sits between a step's
 * two 32-k halves, so the LDS reads of each half run under the products of
 * the half before it (the second half's under the first's; the next
 * step's first half, once the barrier has seen it land, under the second),
 * instead of every wave reading and then multiplying in lock step.  The tile needs the 144 KB of LDS
 * of a CU, so the work-group is as wide as a work-group can be: the rate
 * at which one CU streams its tiles grew with the number of waves issuing
 * them (4, 8, 16 waves: 11.5, 10.0, 9.1 ms for the 512-token XL prefill).
 * Rows are XOR-swizzled in 16-byte chunks (chunk c of row r at slot c ^
 * (r / 2 % 8)) so the 16 rows of a fragment read fall on distinct banks.
 * Per 32-k half a wave issues its 4 a_hi products, then its 4 a_lo
 * products, which is the order of hgemm_impl for every output element.
 * Requires N % 64 == 0 and K % 64 == 0 (per split-K slice); rows >= M and
 * columns >= N are computed from clamped reads and not stored.
 * ==================================================================== */
namespace hg2 {
constexpr int BM = G2H_BM, BN = G2H_BN, BK = G2H_BK, NS = G2H_NS;
constexpr int TB = G2H_TB;       /* bytes of one 128 x 64 fp16 tile */
constexpr int STAGE = G2H_STAGE; /* a_hi, a_lo, weights: 48 KB */
typedef __attribute__((address_space(3))) void lds_t;

/* Wait until this wave's loads of the current step have landed (those of
 * the next step, 3 per wave, may remain), then wait for every wave. */
__device__ __forceinline__ void step_barrier() { asm volatile("s_waitcnt vmcnt(3)\n\ts_barrier" ::: "memory"); }

/* The fragments of one 32-k half of a step: the wave's a_hi, a_lo and
 * weight rows. */
struct frags {
    h16x8 ah[2], al[2], b[2];
};
__device__ __forceinline__ void read_half(frags &f, const unsigned char *st, int kk, int wm, int wn, int lane)
{
    const int slot = g2h_frag_slot(kk, lane);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const unsigned char *row = st + g2h_frag_row(wm, i, lane) * 128 + slot;
        f.ah[i] = *(const h16x8 *)row;
        f.al[i] = *(const h16x8 *)(row + TB);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) f.b[j] = *(const h16x8 *)(st + 2 * TB + g2h_frag_row(wn, j, lane) * 128 + slot);
}
__device__ __forceinline__ void mma_half(f32x4 (&acc)[2][2], const frags &f)
{
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.ah[i], f.b[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.al[i], f.b[j], acc[i][j], 0, 0, 0);
}
} /* namespace hg2 */

template <int EPI>
__device__ void hgemm2_impl(const g2_gemm_args &a)
{
    using namespace hg2;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[NS * STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3; /* 4 x 4 waves of 32 x 32 */
    const int M = a.M, N = a.N, Kfull = a.K;
    /* tile of this work-group (the XCD mapping of g2h_tile_of; the grid's
     * padding work-groups have no work) */
    const g2h_tile tl = g2h_tile_of((int)blockIdx.x, M, N);
    if (!tl.on) return;
    const int m0 = tl.m0, n0 = tl.n0;
    /* split-K (GEPI_PARTIAL): this work-group's K slice, steps [s0, s1) of
     * the Kfull / 64 */
    const int nkt = Kfull / BK;
    const int s0 = EPI == GEPI_PARTIAL ? g2h_slice_start(nkt, (int)blockIdx.z, a.ksplit) : 0;
    const int s1 = EPI == GEPI_PARTIAL ? g2h_slice_start(nkt, (int)blockIdx.z + 1, a.ksplit) : nkt;
    const int kz0 = s0 * BK, nk = s1 - s0;
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    /* this lane's load sources: wave w fills rows 8w..8w+7 of each tile
     * with one instruction (lane -> row l/8, slot l%8); each slot holds the
     * chunk that the swizzle puts there */
    const int row = g2h_load_row(wave, lane);
    const int ch = g2h_load_chunk(row, lane);
    const size_t ao = (size_t)min(m0 + row, M - 1) * Kfull + kz0 + 8 * ch;
    const _Float16 *hsrc = (const _Float16 *)a.Ah + ao, *lsrc = (const _Float16 *)a.Al + ao;
    const _Float16 *bsrc = (const _Float16 *)a.B + (size_t)min(n0 + row, N - 1) * Kfull + kz0 + 8 * ch;
    /* step t's loads into stage buffer b (steps past the last reload it) */
    auto issue = [&](int t, int b) {
        const int k = min(t, nk - 1) * BK;
        unsigned char *st = lds + g2h_load_lds(b, wave);
        __builtin_amdgcn_global_load_lds(hsrc + k, (lds_t *)st, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(lsrc + k, (lds_t *)(st + TB), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(bsrc + k, (lds_t *)(st + 2 * TB), 16, 0, 0);
    };

    /* the epilogue's bias values (two columns per lane), loaded before the
     * tiles so they land during the loop (the loop's waits count only the
     * tile loads issued after them) */
    float bj[2] = {0.f, 0.f};
    if (EPI != GEPI_PARTIAL && a.bias) {
#pragma unroll
        for (int j = 0; j < 2; ++j) bj[j] = a.bias[min(g2h_out_col(n0, wn, j, lane), N - 1)];
    }
    issue(0, 0);
    issue(1, 1);
    step_barrier(); /* step 0 has landed */
    issue(2, 2);
    frags f0, f1;
    read_half(f0, lds, 0, wm, wn, lane);
    int cur = 0;
    for (int t = 0; t < nk; ++t) {
        const unsigned char *st = lds + cur * STAGE;
        const int nx = cur == 2 ? 0 : cur + 1;
        /* second half's reads under the first half's products */
        read_half(f1, st, 32, wm, wn, lane);
        mma_half(acc, f0);
        /* step t + 1 has landed; every wave's reads of step t are done */
        __builtin_amdgcn_s_waitcnt(0x0073); /* vmcnt(3) lgkmcnt(0) */
        asm volatile("s_barrier" ::: "memory");
        /* unconditional: past the last step it reads a reloaded stage */
        read_half(f0, lds + nx * STAGE, 0, wm, wn, lane);
        issue(t + 3, cur);
        mma_half(acc, f1);
        cur = nx;
    }
    /* no load may land in LDS after the work-group has ended */
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    /* the residual epilogue's loads, all issued before the first use
     * (clamped into the matrix) */
    float rv[2][2][4];
    if constexpr (EPI == GEPI_RESID) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int m = min(g2h_out_row(m0, wm, i, lane, q), M - 1);
                    const int n = min(g2h_out_col(n0, wn, j, lane), N - 1);
                    rv[i][j][q] = a.C[(size_t)m * N + n];
                }
    }
    /* bias and residual added in one branch-free pass before the first
     * store: a load's wait placed among the stores would also wait for
     * every store before it (stores count in the same counter) */
    if constexpr (EPI != GEPI_PARTIAL) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc[i][j][q] += bj[j];
                    if constexpr (EPI == GEPI_RESID) acc[i][j][q] += rv[i][j][q];
                    /* keeps the add here (the compiler would sink it, and its
                     * wait, into the conditional store below) */
                    asm volatile("" : "+v"(acc[i][j][q]));
                }
    }
    if constexpr (EPI == GEPI_QKV) {
        const qkv_dst d = qkv_of(a);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = g2h_out_col(n0, wn, j, lane);
                if (n < N) qkv_store4(d, g2h_out_row(m0, wm, i, lane, 0), M, n, acc[i][j]);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = g2h_out_row(m0, wm, i, lane, q);
                const int n = g2h_out_col(n0, wn, j, lane);
                if (m >= M || n >= N) continue;
                const float v = acc[i][j][q];
                if (EPI == GEPI_PARTIAL) {
                    a.part[(size_t)blockIdx.z * M * N + (size_t)m * N + n] = v;
                    continue;
                }
                if (EPI == GEPI_GELU_SPLIT) {
                    split_store(a.Ch, a.Cl, (size_t)m * N + n, gelu_f(v));
                } else if (EPI == GEPI_RESID) {
                    a.C[(size_t)m * N + n] = v;
                }
            }
}

/* one work-group of 16 waves per CU (144 KB of LDS), 4 waves per SIMD */
#define G2K_HG2 extern "C" __global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4, 4)))
G2K_HG2 void g2k_hgemm2_gelu(const g2_gemm_args a) { hgemm2_impl<GEPI_GELU_SPLIT>(a); }
G2K_HG2 void g2k_hgemm2_resid(const g2_gemm_args a) { hgemm2_impl<GEPI_RESID>(a); }
G2K_HG2 void g2k_hgemm2_qkv(const g2_gemm_args a) { hgemm2_impl<GEPI_QKV>(a); }
G2K_HG2 void g2k_hgemm2_partial(const g2_gemm_args a) { hgemm2_impl<GEPI_PARTIAL>(a); }

/* The split-K residual epilogue fused with the LayerNorm that follows it
 * in the prefill (proj -> ln_2, fc2 -> the next layer's ln_1): one
 * work-group per row sums the slices, bias and residual as
 * g2k_splitk_resid does, keeps the row in registers, and normalises it
 * (two-pass mean and biased variance, eps 1e-5, as g2k_layernorm), writing
 * the next GEMM's operand: its fp16 halves (the fp16-weight GEMMs, at most
 * G2_SKLN_MAXKS slices) or fp32 (F32OUT: the fp32-weight GEMMs, at most
 * G2_SKLN_F32_MAXKS slices). */
template <int ZMAX, bool F32OUT>
__device__ __forceinline__ void splitk_resid_ln_impl(const g2_skred_args &a)
{
    /* thread t owns the 4-column groups t and t + 256 of the row (N % 4 ==
     * 0, N <= G2_SKLN_MAXN); every load of both groups -- the ks slices,
     * the residual, bias and LayerNorm parameters -- is issued before the
     * first sum (clamped into the row), so the row costs one memory latency
     * instead of one per group */
    constexpr int PG = G2_SKLN_MAXN / 1024; /* groups per thread */
    __shared__ float red4[4];
    const int m = blockIdx.x, N = a.N, NG = N >> 2;
    if (m >= a.M) return;
    const size_t MN = (size_t)a.M * N, row = (size_t)m * N;
    f32x4 pz[PG][ZMAX], cv[PG], bv[PG], gv[PG], ev[PG];
#pragma unroll
    for (int k = 0; k < PG; ++k) {
        const int g = min((int)threadIdx.x + 256 * k, NG - 1);
#pragma unroll
        for (int z = 0; z < ZMAX; ++z)
            pz[k][z] = z < a.ks ? *(const f32x4 *)(a.part + (size_t)z * MN + row + 4 * g)
                                : (f32x4){0.f, 0.f, 0.f, 0.f};
        cv[k] = *(const f32x4 *)(a.C + row + 4 * g);
        bv[k] = a.bias ? *(const f32x4 *)(a.bias + 4 * g) : (f32x4){0.f, 0.f, 0.f, 0.f};
        gv[k] = *(const f32x4 *)(a.ln_g + 4 * g);
        ev[k] = *(const f32x4 *)(a.ln_b + 4 * g);
    }
    f32x4 xv[PG];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < PG; ++k) {
        const int g = (int)threadIdx.x + 256 * k;
        /* slices in order, then bias, then the residual (the order of the
         * unfused splitk_resid) */
        f32x4 v = pz[k][0];
#pragma unroll
        for (int z = 1; z < ZMAX; ++z)
            if (z < a.ks) v += pz[k][z];
        v += bv[k];
        v += cv[k];
        xv[k] = v;
        if (g < NG) {
            *(f32x4 *)(a.C + row + 4 * g) = v;
            s += ((v.x + v.y) + v.z) + v.w;
        }
    }
    const float mean = block_sum(s, red4) / (float)N;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < PG; ++k)
        if ((int)threadIdx.x + 256 * k < NG) {
            const f32x4 d = xv[k] - mean;
            q = fmaf(d.x, d.x, q);
            q = fmaf(d.y, d.y, q);
            q = fmaf(d.z, d.z, q);
            q = fmaf(d.w, d.w, q);
        }
    const float var = block_sum(q, red4) / (float)N;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
    for (int k = 0; k < PG; ++k) {
        const int g = (int)threadIdx.x + 256 * k;
        if (g < NG) {
            /* the group's four outputs as one 8-byte store per half */
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = fmaf((xv[k][e] - mean) * inv, gv[k][e], ev[k][e]);
            if constexpr (F32OUT) {
                *(f32x4 *)(a.ln_out + row + 4 * g) = (f32x4){y[0], y[1], y[2], y[3]};
            } else {
                uint2 hv, lv;
                split2(y[0], y[1], hv.x, lv.x);
                split2(y[2], y[3], hv.y, lv.y);
                *(uint2 *)(a.hi + row + 4 * g) = hv;
                *(uint2 *)(a.lo + row + 4 * g) = lv;
            }
        }
    }
}
G2K void g2k_splitk_resid_ln(const g2_skred_args a) { splitk_resid_ln_impl<G2_SKLN_MAXKS, false>(a); }
G2K void g2k_splitk_resid_ln_f32(const g2_skred_args a) { splitk_resid_ln_impl<G2_SKLN_F32_MAXKS, true>(a); }

G2K void g2k_hgemm_store(const g2_gemm_args a) { hgemm_impl<GEPI_STORE>(a); }
G2K void g2k_hgemm_gelu(const g2_gemm_args a) { hgemm_impl<GEPI_GELU>(a); }
G2K void g2k_hgemm_resid(const g2_gemm_args a) { hgemm_impl<GEPI_RESID>(a); }
G2K void g2k_hgemm_qkv(const g2_gemm_args a) { hgemm_impl<GEPI_QKV>(a); }

/* Causal attention over a prompt (prefill), head dim 64, on the fp32
 * matrix cores (v_mfma_f32_16x16x4f32), keys and values from the transposed
 * K cache and the V cache: grid (NH, ceil(P/64)), 512 threads; waves w and
 * w + 4 own query rows
 * 16w..16w+15 of the block, the first over the even key blocks, the
 * second over the odd ones, each with its own online softmax, combined at
 * the end (the kernel lasts as long as its longest rows, whose key blocks
 * are thus shared by two waves).  Per 64-key block: S = Q K^T (4 tiles of
 * 16 keys, 16 k steps of 4 dims), scaled and causally masked, online softmax over the
 * block (row statistics reduced across the 16 lanes of a row group), P
 * re-laid through LDS into the operand layout, O += P V (4 tiles of 16
 * dims, 16 k steps of 4 keys).  fp32 throughout, as the reference.
 * Operand layout: lane l supplies A[l%16][k0 + l/16] and B[k0 + l/16][l%16];
 * the result lane l holds rows 4(l/16)+r, column l%16. */
template <int CTRL>
__device__ __forceinline__ float apf_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
/* max / sum over the 16 lanes of a DPP row (rotations 8, 4, 2, 1) */
__device__ __forceinline__ float row16_max(float v)
{
    v = fmaxf(v, apf_dpp<0x128>(v));
    v = fmaxf(v, apf_dpp<0x124>(v));
    v = fmaxf(v, apf_dpp<0x122>(v));
    return fmaxf(v, apf_dpp<0x121>(v));
}
__device__ __forceinline__ float row16_sum(float v)
{
    v += apf_dpp<0x128>(v);
    v += apf_dpp<0x124>(v);
    v += apf_dpp<0x122>(v);
    return v + apf_dpp<0x121>(v);
}

/* Work-group -> (head, 64-row query block) of the prompt attention
 * (g2a_block): the grid is 1-D, 8 * ceil(NH / 8) * nqb work-groups, and
 * work-group w runs on XCD w % 8 (consecutive work-groups go to consecutive
 * XCDs), so every query block of head h runs on XCD h % 8, whose L2 then
 * fetches that head's keys and values once for all of them; the longest
 * query blocks and the helpers are dispatched first.  Work-groups past the
 * last head have no work of their own. */
__device__ __forceinline__ void attnp_block(const g2_attnp_args &a, int &h, int &qb)
{
    g2a_block((int)blockIdx.x, a.P, a.NH, &h, &qb);
}

extern "C" __global__ __launch_bounds__(512) void g2k_attn_prefill_mfma(const g2_attnp_args a)
{
    /* The tiles are stored so that a lane's operands of all four 16-wide
     * tiles are 16 contiguous bytes (one ds_read_b128 for 4 products):
     * Kt[d][pk(k)] and Vs[k][pk(d)] with pk(c) = 4 (c % 16) + c / 16 (the
     * column 16 t + l of tile t at 4 l + t), and each wave's P as
     * [row][pp(k)], pp(k) = 16 (k % 4) + k / 4 (its 16 values of a k-step
     * group contiguous).  Row pitches of 68 floats spread the staging
     * writes over the banks. */
    constexpr int LD = 68, LDP = 68;
    __shared__ __attribute__((aligned(16))) float Kt[2][64 * LD]; /* per half [dim][pk(key)] */
    __shared__ __attribute__((aligned(16))) float Vs[2][64 * LD]; /* per half [key][pk(dim)] */
    __shared__ __attribute__((aligned(16))) float Ps[8][16 * LDP]; /* per wave [row][pp(key)] */
    int h, qb;
    attnp_block(a, h, qb);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    /* wave w: row group rg = w % 4 (query rows 16 rg..16 rg + 15 of the
     * block) over the key blocks of its half hs = w / 4 (kb = hs, hs + 2,
     * ...), so the blocks of the longest rows are shared by two waves */
    const int rg = wave & 3, hs = wave >> 2;
    if (h >= a.NH || qb * 64 >= a.P) return;
    const int E = a.E, P = a.P;
    /* Q operand: lane holds Q[row 16 rg + lr][dim 4s + lg], s < 16 */
    float qa[16];
    {
        const int i = min(qb * 64 + 16 * rg + lr, P - 1);
        const float *qp = a.q + (size_t)i * E + h * 64 + lg;
#pragma unroll
        for (int st = 0; st < 16; ++st) qa[st] = qp[4 * st];
    }
    f32x4 o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) { m[r] = -INFINITY; l[r] = 0.f; }
    const int i_base = qb * 64 + 16 * rg + 4 * lg;      /* query row of result r: i_base + r */
    const int sr = (tid & 255) >> 2, sq = (tid & 3) * 16; /* staging (per half): row, 16 columns */
    /* key block kb's staging loads (kb clamped to the last block: the loads
     * stay unconditional, see load_set in the step kernel) */
    f32x4 kv[4], vv[4];
    auto kvload = [&](int kb) {
        const int jb = min(kb, qb) * 64;
        const float *kp = a.k_cache + (size_t)(h * 64 + sr) * a.S + min(jb + sq, a.S - 16);
        const float *vp = a.v_cache + (size_t)min(jb + sr, a.S - 1) * E + h * 64 + sq;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            kv[q] = *(const f32x4 *)(kp + 4 * q);
            vv[q] = *(const f32x4 *)(vp + 4 * q);
        }
    };
    kvload(hs);
    const int nit = (qb + 2) >> 1; /* block pairs */
    for (int it = 0; it < nit; ++it) {
        const int kb = 2 * it + hs, j0 = kb * 64;
        __syncthreads(); /* the previous blocks have been consumed */
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = sq + 4 * q + e, pc = 4 * (c & 15) + (c >> 4);
                Kt[hs][sr * LD + pc] = kv[q][e];
                Vs[hs][sr * LD + pc] = vv[q][e];
            }
        __syncthreads();
        kvload(kb + 2); /* the next block streams in during this one's products */
        if (kb > qb) continue; /* the odd half of an odd block count (wave-uniform) */
        const float *Kb = Kt[hs], *Vb = Vs[hs];
        /* S = Q K^T: tile t covers keys 16t..16t+15; the four tiles'
         * product chains interleave (no product waits for the one before) */
        f32x4 sacc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) sacc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
        f32x4 kb4[16];
#pragma unroll
        for (int st = 0; st < 16; ++st) kb4[st] = *(const f32x4 *)(Kb + (4 * st + lg) * LD + 4 * lr);
#pragma unroll
        for (int st = 0; st < 16; ++st)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                sacc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[st], kb4[st][t], sacc[t], 0, 0, 0);
        /* scale, causal mask, online softmax per row */
        float alpha[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = i_base + r;
            float bm = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int j = j0 + 16 * t + lr;
                const float v = (i < P && j <= i) ? sacc[t][r] * a.scale : -INFINITY;
                sacc[t][r] = v;
                bm = fmaxf(bm, v);
            }
            bm = row16_max(bm);
            const float mn = fmaxf(m[r], bm);
            const float ms = mn == -INFINITY ? 0.f : mn;
            alpha[r] = expf(m[r] - ms);
            float ps = 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float p = expf(sacc[t][r] - ms);
                sacc[t][r] = p;
                ps += p;
            }
            l[r] = fmaf(l[r], alpha[r], row16_sum(ps));
            m[r] = mn;
        }
        /* P to LDS in [row][key], read back as the A operand */
        float *pw = Ps[wave];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int k = 16 * t + lr;
                pw[(4 * lg + r) * LDP + 16 * (k & 3) + (k >> 2)] = sacc[t][r];
            }
        __builtin_amdgcn_wave_barrier();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[t][r] *= alpha[r];
        f32x4 pa4[4], vb4[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) pa4[q] = *(const f32x4 *)(pw + lr * LDP + 16 * lg + 4 * q);
#pragma unroll
        for (int st = 0; st < 16; ++st) vb4[st] = *(const f32x4 *)(Vb + (4 * st + lg) * LD + 4 * lr);
#pragma unroll
        for (int st = 0; st < 16; ++st)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa4[st >> 2][st & 3], vb4[st][t], o[t], 0, 0, 0);
    }
    /* combine the halves: the odd half's (max, sum, o) through LDS (the
     * staging tiles are free), scaled to the common max */
    __syncthreads();
    float *xw = Kt[0] + (size_t)(rg * 64 + lane) * 24; /* 4 waves x 64 lanes x 24 floats <= 2 tiles */
    if (hs == 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            xw[r] = m[r];
            xw[4 + r] = l[r];
#pragma unroll
            for (int t = 0; t < 4; ++t) xw[8 + 4 * t + r] = o[t][r];
        }
    }
    __syncthreads();
    if (hs == 1) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float m1 = xw[r], l1 = xw[4 + r];
        const float mx = fmaxf(m[r], m1);
        const float f0 = m[r] == -INFINITY ? 0.f : expf(m[r] - mx);
        const float f1 = m1 == -INFINITY ? 0.f : expf(m1 - mx);
        l[r] = l[r] * f0 + l1 * f1;
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t][r] = o[t][r] * f0 + xw[8 + 4 * t + r] * f1;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = i_base + r;
        if (i >= P) continue;
        const float inv = 1.0f / l[r];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const size_t idx = (size_t)i * E + h * 64 + 16 * t + lr;
            if (a.out_hi) split_store(a.out_hi, a.out_lo, idx, o[t][r] * inv);
            else a.out[idx] = o[t][r] * inv;
        }
    }
}

/* Causal prompt attention on the fp16 matrix cores (same arguments, grid
 * and results as g2k_attn_prefill_mfma: per head and 64-query block, 8
 * waves, two per 16-row group, each taking every other 64-key block, their
 * online-softmax states combined at the end).  Every fp32 operand x is
 * split into fp16 halves hi = fp16(x), lo = fp16(x - hi) (split_store), and
 * each product of two split operands is hi.hi + hi.lo + lo.hi on
 * v_mfma_f32_16x16x32_f16 (fp32 accumulate; the dropped lo.lo term is below
 * fp32 rounding of the sum).
 *
 * The products are computed transposed, S^T = K Q^T and O^T = V^T P^T, so
 * that a lane holds one query row (lane % 16) throughout: the softmax's row
 * maximum and sum are in-lane over its 16 scores plus two cross-row lane
 * swaps, the rescale of O is one factor per lane, and P^T reaches the
 * second product by two permlane swaps instead of a round trip through LDS.
 * The online softmax works in base 2 (scores times log2 e, v_exp_f32), the
 * usual flash-attention form; the probabilities equal exp() of the
 * natural-base scores to fp32 rounding.
 *
 * Operand layouts (v_mfma_f32_16x16x32_f16: lane l supplies
 * A[l%16][8(l/16)..+7] and B[8(l/16)..+7][l%16]; D[4(l/16)+r][l%16]):
 *   K  A operand of S^T, staged as [key][dim] halves (8 consecutive dims of
 *      one key, one 16-byte LDS read), streamed by LDS DMA from the halves
 *      kh/kl the qkv epilogue wrote;
 *   Q  B operand of S^T, from global (8 consecutive dims of the lane's row);
 *   S^T, P^T  D tiles of 16 keys: lane 16g + row holds keys 4g..4g+3;
 *   V  A operand of O^T, staged as [dim][key] halves (8 consecutive keys of
 *      one dim), from the transposed halves vth/vtl;
 *   P^T  B operand of O^T (8 consecutive keys of the lane's row), made from
 *      two D tiles by a 32-lane and a 16-lane swap (pt_operand).
 * Staged K/V rows are 128 bytes (8 chunks of 8 halves), chunk c of row r at
 * slot c ^ (r / 2 % 8), so the 16 rows of an operand read fall on distinct
 * banks.  Each half stages its key blocks in a two-stage ring (the next
 * block's loads in flight during the products of the current one). */
__device__ __forceinline__ int kv_at(int row, int chunk) { return g2a_kv_at(row, chunk); }

/* max / sum over the four 16-lane rows of a wave (lanes l, l^16, l^32,
 * l^48), the same value in every lane */
__device__ __forceinline__ float xrow_max(float v)
{
    const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(s1[0]), __uint_as_float(s1[1]));
    const auto s2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s2[0]), __uint_as_float(s2[1]));
}
__device__ __forceinline__ float xrow_sum(float v)
{
    const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(s1[0]) + __uint_as_float(s1[1]);
    const auto s2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
}


/* The B operand P^T of a 32-key chunk (lane 16G + row: keys 8G..8G+7 of the
 * chunk, as hi and lo halves) from its two D tiles d0 (keys 0..15) and d1
 * (16..31), where lane 16g + row holds keys 4g..4g+3 of its tile.  Row
 * groups [a0 a1 a2 a3] of d0 and [b0 b1 b2 b3] of d1 become [a0 a1 b0 b1]
 * and [a2 a3 b2 b3] (32-lane swap), then [a0 a2 b0 b2] and [a1 a3 b1 b3]
 * (16-lane swap): keys 8G..8G+3 and 8G+4..8G+7. */
__device__ __forceinline__ void pt_operand(const f32x4 &d0, const f32x4 &d1, f16x8 &ph, f16x8 &pl)
{
    unsigned h[2][2], l[2][2]; /* [tile][key pair] */
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        split2(d0[2 * q], d0[2 * q + 1], h[0][q], l[0][q]);
        split2(d1[2 * q], d1[2 * q + 1], h[1][q], l[1][q]);
    }
    u32x4 oh, ol;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const auto a = __builtin_amdgcn_permlane32_swap(h[0][q], h[1][q], false, false);
        const auto b = __builtin_amdgcn_permlane16_swap(a[0], a[1], false, false);
        oh[q] = b[0];
        oh[2 + q] = b[1];
        const auto c = __builtin_amdgcn_permlane32_swap(l[0][q], l[1][q], false, false);
        const auto d = __builtin_amdgcn_permlane16_swap(c[0], c[1], false, false);
        ol[q] = d[0];
        ol[2 + q] = d[1];
    }
    ph = __builtin_bit_cast(f16x8, oh);
    pl = __builtin_bit_cast(f16x8, ol);
}

/* The softmax partial of a query block's row split between a helper and
 * the block's work-group (g2a_help_plan).  Both have combined their two key
 * halves into max mx, sum lx and unnormalised output o f0 + x f1 (x: the
 * other half's, in LDS at xw + 2).  The helper stores (mx, lx, 0, 0) and the
 * four output tiles into slot j (thread t's vectors at g2a_help_vec) and is
 * done; the block's work-group polls them (loads at the coherence point,
 * sc1, as relaxed agent-scope atomics are) until no float is G2V_EMPTY,
 * writes G2V_EMPTY back, and stores the merged row (helper's part first:
 * its keys come first) at out + idx.  Every float of a slot is written
 * once per launch by one store, so a float read non-empty is this
 * launch's; a stored value with G2V_EMPTY's bits (only a NaN could have
 * them) is stored as the canonical NaN.  The wait is bounded
 * (G2_ERR_ATTN_TIMEOUT in *err, after which the slots must be refilled). */
__device__ __forceinline__ void attn_help_merge(const g2_attnp_args &a, int j, bool helper, int t, float mx, float lx,
                                                const f32x4 (&o)[4], const float *xw, float f0, float f1, size_t idx)
{
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)a.help, (short)0,
                                                                        G2A_HELP_MAX_SLOTS * G2A_HELP_SLOT_BYTES, 0x00020000);
    f32x4 ox[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) ox[q][r] = o[q][r] * f0 + xw[2 + 4 * q + r] * f1;
    auto bits = [](float f) {
        const unsigned b = __float_as_uint(f);
        return b == G2V_EMPTY ? 0x7FC00000u : b;
    };
    if (helper) {
        const u32x4 v0 = {bits(mx), bits(lx), 0u, 0u};
        __builtin_amdgcn_raw_buffer_store_b128(v0, rs, g2a_help_vec(j, 0, t) * 16, 0, 16 /* sc1 */);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = {bits(ox[q].x), bits(ox[q].y), bits(ox[q].z), bits(ox[q].w)};
            __builtin_amdgcn_raw_buffer_store_b128(v, rs, g2a_help_vec(j, q + 1, t) * 16, 0, 16 /* sc1 */);
        }
        return;
    }
    auto empty = [](const u32x4 &v) {
        return v.x == G2V_EMPTY || v.y == G2V_EMPTY || v.z == G2V_EMPTY || v.w == G2V_EMPTY;
    };
    u32x4 v[5];
#pragma unroll
    for (int q = 0; q < 5; ++q) v[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, g2a_help_vec(j, q, t) * 16, 0, 16);
    bool bad = empty(v[0]) || empty(v[1]) || empty(v[2]) || empty(v[3]) || empty(v[4]);
    if (bad) {
        const unsigned long long t0 = wall_clock64();
        for (;;) {
            __builtin_amdgcn_s_sleep(2);
#pragma unroll
            for (int q = 0; q < 5; ++q)
                if (empty(v[q])) v[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, g2a_help_vec(j, q, t) * 16, 0, 16);
            bad = empty(v[0]) || empty(v[1]) || empty(v[2]) || empty(v[3]) || empty(v[4]);
            if (!bad) break;
            if (wall_clock64() - t0 > 20000000ull) { /* 200 ms of the 100 MHz clock */
                atomicOr(a.err, G2_ERR_ATTN_TIMEOUT);
                break;
            }
        }
    }
    const u32x4 e4 = {G2V_EMPTY, G2V_EMPTY, G2V_EMPTY, G2V_EMPTY};
#pragma unroll
    for (int q = 0; q < 5; ++q) __builtin_amdgcn_raw_buffer_store_b128(e4, rs, g2a_help_vec(j, q, t) * 16, 0, 16 /* sc1 */);
    const float mh = __uint_as_float(v[0].x), lh = __uint_as_float(v[0].y);
    const float mm = fmaxf(mh, mx);
    const float gh = mh == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mh - mm);
    const float gx = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mx - mm);
    const float inv = 1.0f / (lh * gh + lx * gx);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const f32x4 oh = __builtin_bit_cast(f32x4, v[q + 1]);
        f32x4 y;
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = (oh[r] * gh + ox[q][r] * gx) * inv;
        const size_t ix = idx + 16 * q;
        if (a.out_hi) {
            uint2 hv, lv;
            split2(y[0], y[1], hv.x, lv.x);
            split2(y[2], y[3], hv.y, lv.y);
            *(uint2 *)(a.out_hi + ix) = hv;
            *(uint2 *)(a.out_lo + ix) = lv;
        } else {
            *(f32x4 *)(a.out + ix) = y;
        }
    }
}

extern "C" __global__ __launch_bounds__(512) void g2k_attn_prefill_h16(const g2_attnp_args a)
{
    constexpr int TILE = 64 * 64; /* halves per staged array */
    constexpr int TB = 2 * TILE;  /* its bytes */
    /* stage b of half hs: Kh, Kl, Vh, Vl at (4 (2 hs + b) + 0..3) * TILE */
    __shared__ __attribute__((aligned(1024))) _Float16 kvs[16 * TILE];
    int h, qb;
    attnp_block(a, h, qb);
    const int tid = threadIdx.x;
    const int lane = tid & 63, lr = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); /* uniform: key half and row group in SGPRs */
    const int rg = wave & 3, hs = wave >> 2;
    /* key blocks [kb_lo, kb_hi] of query block qb: all of them, or with a
     * helper (g2a_help_plan) the helper's first 2 nh and the rest here;
     * `helper`: the slot this work-group fills as a helper, else -1 */
    const g2a_help hp = g2a_help_plan(a.P, a.NH);
    int helper = -1, kb_lo = 0, kb_hi = qb;
    if (h >= a.NH) {
        if (!a.help) return;
        helper = g2a_helper_index((int)blockIdx.x, a.P, a.NH, &hp);
        if (helper < 0) return;
        g2a_helped_block(helper, a.P, &hp, &h, &qb);
        kb_hi = 2 * hp.nh - 1;
    } else if (a.help && g2a_help_slot(h, qb, a.P, &hp) >= 0) {
        kb_lo = 2 * hp.nh;
    }
    if (qb * 64 >= a.P) return;
    /* scores in base-2 units (scaled by log2 e): the softmax's
     * exponentials are single v_exp_f32 instructions */
    const float scale2 = a.scale * 1.4426950408889634f;
    const int E = a.E, P = a.P, S = a.S;
    /* this lane's query row */
    const int i = g2a_query(qb, rg, lane);
    f16x8 qh[2], ql[2];
    {
        const float *qp = a.q + (size_t)min(i, P - 1) * E + h * 64 + 8 * lg;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const f32x4 x0 = *(const f32x4 *)(qp + 32 * s2), x1 = *(const f32x4 *)(qp + 32 * s2 + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qh[s2][e] = hi16(x0[e]); ql[s2][e] = lo16(x0[e]);
                qh[s2][4 + e] = hi16(x1[e]); ql[s2][4 + e] = lo16(x1[e]);
            }
        }
    }
    f32x4 o[4]; /* O^T: tile t = dims 16t..16t+15, lane 16g + row holds dims 16t + 4g..+3 */
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    /* Staging of key block kb into stage b by LDS DMA (global_load_lds_
     * dwordx4: lane l of an instruction writes 16 bytes at LDS base + 16 l),
     * from the halves the qkv epilogue wrote, with no conversion: wave w4 of
     * the half fills rows 16 w4..16 w4 + 15 of each array with two
     * instructions of 8 rows (lane -> row l/8, slot l%8, holding the chunk
     * that the swizzle puts there).  K rows are keys (8 dims per chunk, from
     * kh/kl [position][E]), V rows are dims (8 keys per chunk, from vth/vtl
     * [E][S]); every address is inside the arrays (positions j0 + 63 <= 1023
     * < S, dims < E). */
    const int w4 = wave & 3;
    typedef __attribute__((address_space(3))) void lds_t;
    /* per-lane element offsets of the two staging instructions within a
     * key block (the block's position part is added to the uniform bases) */
    unsigned kof[2], vof[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int rw = G2A_STAGE_ROW(w4, e, lane);
        const int c = G2A_STAGE_CHUNK(rw, lane);
        kof[e] = (unsigned)(rw * E + h * 64 + 8 * c);
        vof[e] = (unsigned)((h * 64 + rw) * S + 8 * c);
    }
    auto stage = [&](int kb, int b) {
        const int j0 = kb * 64;
        unsigned char *st = (unsigned char *)(kvs + g2a_array(hs, b, 0));
        const uint16_t *khb = a.kh + (size_t)j0 * E, *klb = a.kl + (size_t)j0 * E;
        const uint16_t *vhb = a.vth + j0, *vlb = a.vtl + j0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            unsigned char *dst = st + (16 * w4 + 8 * e) * 128;
            __builtin_amdgcn_global_load_lds(khb + kof[e], (lds_t *)dst, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(klb + kof[e], (lds_t *)(dst + TB), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vhb + vof[e], (lds_t *)(dst + 2 * TB), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vlb + vof[e], (lds_t *)(dst + 3 * TB), 16, 0, 0);
        }
    };
    const int nit = (kb_hi - kb_lo + 2) >> 1;
    if (kb_lo + hs <= kb_hi) stage(kb_lo + hs, 0); /* wave-uniform */
    for (int it = 0; it < nit; ++it) {
        const int kb = kb_lo + 2 * it + hs, j0 = kb * 64, b = it & 1;
        /* this wave's part of block kb has landed; every wave is past the
         * products of the block before, which read stage b ^ 1 */
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (kb + 2 <= kb_hi) stage(kb + 2, b ^ 1); /* wave-uniform */
        if (kb > kb_hi) continue;                   /* wave-uniform */
        const _Float16 *Kh = kvs + g2a_array(hs, b, 0), *Kl = Kh + TILE;
        const _Float16 *Vh = Kh + 2 * TILE, *Vl = Kh + 3 * TILE;
        /* S^T tiles: keys j0 + 16t + 4lg + r of row i */
        f32x4 sacc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) sacc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
        {
            f16x8 kh[4][2], kl[4][2];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const int at = kv_at(16 * t + lr, 4 * s2 + lg);
                    kh[t][s2] = *(const f16x8 *)(Kh + at);
                    kl[t][s2] = *(const f16x8 *)(Kl + at);
                }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    sacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[t][s2], ql[s2], sacc[t], 0, 0, 0);
                    sacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl[t][s2], qh[s2], sacc[t], 0, 0, 0);
                }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    sacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[t][s2], qh[s2], sacc[t], 0, 0, 0);
        }
        float bm = -INFINITY;
        /* wave-uniform: only the diagonal block has keys past a row (rows
         * past the prompt, in the last block, are masked there only: their
         * results are never stored) */
        if (kb == qb) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int j = j0 + 16 * t + 4 * lg + r;
                    const float v = (i < P && j <= i) ? sacc[t][r] * scale2 : -INFINITY;
                    sacc[t][r] = v;
                    bm = fmaxf(bm, v);
                }
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float v = sacc[t][r] * scale2;
                    sacc[t][r] = v;
                    bm = fmaxf(bm, v);
                }
        }
        bm = xrow_max(bm);
        const float mn = fmaxf(m, bm);
        const float ms = mn == -INFINITY ? 0.f : mn;
        const float alpha = __builtin_amdgcn_exp2f(m - ms);
        float ps = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = __builtin_amdgcn_exp2f(sacc[t][r] - ms);
                sacc[t][r] = pv;
                ps += pv;
            }
        l = fmaf(l, alpha, xrow_sum(ps));
        m = mn;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[t][r] *= alpha;
        f16x8 ph[2], pl[2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) pt_operand(sacc[2 * s2], sacc[2 * s2 + 1], ph[s2], pl[s2]);
        {
            f16x8 vh[4][2], vl[4][2];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const int at = kv_at(16 * t + lr, 4 * s2 + lg);
                    vh[t][s2] = *(const f16x8 *)(Vh + at);
                    vl[t][s2] = *(const f16x8 *)(Vl + at);
                }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[t][s2], pl[s2], o[t], 0, 0, 0);
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl[t][s2], ph[s2], o[t], 0, 0, 0);
                }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[t][s2], ph[s2], o[t], 0, 0, 0);
        }
    }
    __syncthreads();
    /* odd stride: the 64 lanes of a word access fall on distinct banks */
    float *xw = (float *)kvs + (size_t)(rg * 64 + lane) * 19;
    if (hs == 1) {
        xw[0] = m;
        xw[1] = l;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) xw[2 + 4 * t + r] = o[t][r];
    }
    __syncthreads();
    if (hs == 1 || i >= P) return;
    const float m1 = xw[0], l1 = xw[1];
    const float mx = fmaxf(m, m1);
    const float f0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mx);
    const float f1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mx);
    if (helper >= 0 || kb_lo > 0) {
        attn_help_merge(a, helper >= 0 ? helper : g2a_help_slot(h, qb, P, &hp), helper >= 0, tid, mx,
                        l * f0 + l1 * f1, o, xw, f0, f1, (size_t)i * E + h * 64 + 4 * lg);
        return;
    }
    const float inv = 1.0f / (l * f0 + l1 * f1);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        f32x4 y;
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = (o[t][r] * f0 + xw[2 + 4 * t + r] * f1) * inv;
        const size_t idx = (size_t)i * E + h * 64 + 16 * t + 4 * lg;
        if (a.out_hi) {
            /* the four dims as one 8-byte store per half */
            uint2 hv, lv;
            split2(y[0], y[1], hv.x, lv.x);
            split2(y[2], y[3], hv.y, lv.y);
            *(uint2 *)(a.out_hi + idx) = hv;
            *(uint2 *)(a.out_lo + idx) = lv;
        } else {
            *(f32x4 *)(a.out + idx) = y;
        }
    }
}

/* g2_lnfold_args: a row of W per wave, each lane summing k = lane, lane +
 * 64, ... in double, then the lanes in a fixed butterfly order. */
template <typename WT>
__device__ __forceinline__ void ln_fold_impl(const g2_lnfold_args &a)
{
    const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= a.N) return; /* wave-uniform */
    const WT *w = (const WT *)a.W + (size_t)r * a.K;
    double s1 = 0.0, s2 = 0.0;
    for (int k = lane; k < a.K; k += 64) {
        const double wv = (double)(float)w[k];
        s1 += wv * (double)a.gamma[k];
        s2 += wv * (double)a.beta[k];
    }
    for (int o = 32; o > 0; o >>= 1) {
        s1 += __shfl_xor(s1, o);
        s2 += __shfl_xor(s2, o);
    }
    if (lane == 0) {
        a.c1[r] = (float)s1;
        a.c2[r] = (float)(s2 + (a.bias ? (double)a.bias[r] : 0.0));
    }
}
G2K void g2k_ln_fold_f32(const g2_lnfold_args a) { ln_fold_impl<float>(a); }
G2K void g2k_ln_fold_f16(const g2_lnfold_args a) { ln_fold_impl<_Float16>(a); }

/* Fused decode kernels (packed matvecs, single-query attention). */
#include "g2_decode.hip"

/* The persistent decode step (one cooperative launch per token). */
#include "g2_step.hip"
