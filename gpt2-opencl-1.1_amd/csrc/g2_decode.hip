/*
 * g2_decode.hip -- fused decode kernels (included by g2_kernels.hip, which
 * provides the shared helpers and types).
 *
 *  - g2k_attn_part* / g2k_attn_merge: single-query attention, head dim 64,
 *    split over 64-position key chunks; the merge of the chunk partials is
 *    its own small launch, so no kernel needs a device-wide fence (on gfx950
 *    an agent-scope release/acquire writes back and invalidates the XCD's
 *    L2, which serialises when hundreds of work-groups issue it);
 *  - g2k_rows*: matvec over packed output-major weights W[N,K] with an
 *    optional LayerNorm prologue and a store / GELU / residual / KV-scatter /
 *    argmax-partial epilogue; g2k_argmax_merge finishes the greedy pick.
 *
 * Batch-1 decode moves every weight byte exactly once per token, so the
 * matvecs are built for memory-level parallelism: a group of SG lanes (one
 * wave, or the whole 256-thread work-group for long rows) owns R rows and
 * every lane issues R*CPT independent 16-byte weight loads at kernel entry,
 * right after the (L2-resident) activation loads, so the LayerNorm
 * statistics are computed while the weights stream in.
 */

/* ======================================================================
 * Single-query attention
 *
 * g2k_attn_part: grid (NH, max_chunks), 256 threads; work-group (h, c) takes
 * key positions [64c, 64c+64) of head h.
 *  scores: thread (pq = tid%16, dg = tid/16) reads 4 dims x 4 consecutive
 *    positions of the transposed K cache as four 16-byte loads; the 16 dim
 *    groups are summed in order through LDS;
 *  chunk softmax: wave 0 takes the max and sum over the 64 positions;
 *  weighted sum: thread (d4 = tid%16, jg = tid/16) reads 4 positions x 4
 *    dims of the V cache as four 16-byte loads; 16 position groups summed in
 *    order through LDS;
 *  the chunk's (max, sum, o[64]) goes to part[h][c].
 * g2k_attn_merge: grid NH, 64 threads: rescales the chunk partials by
 *  exp(max_c - max) and writes out[h*64 + d] = sum_c o_c w_c / sum_c l_c w_c.
 * VEC needs S%4 == 0, D%4 == 0 and 16-byte aligned caches; the scalar
 * variant serves other layouts.
 * ==================================================================== */
__device__ __forceinline__ int attn_T(const g2_attn1q_args &a)
{
    return clampi(a.T_fixed > 0 ? a.T_fixed : a.state[G2S_POS] + 1, 1, a.S);
}

template <bool VEC>
__device__ void attn_part_impl(const g2_attn1q_args &a)
{
    __shared__ float qs[64];
    __shared__ float red[16][65];
    __shared__ float pr[64];
    __shared__ float stat[2];
    const int h = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
    const int T = attn_T(a);
    const int nch = (T + 63) >> 6;
    if (h >= a.NH || c >= nch || nch > a.max_chunks) return;
    const int j0 = c * 64, S = a.S, D = a.D;
    if (tid < 64) qs[tid] = a.q[h * 64 + tid];
    __syncthreads();
    {
        const int pq = tid & 15, dg = tid >> 4, j = j0 + 4 * pq;
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        const float *kb = a.k_cache + (size_t)(h * 64 + 4 * dg) * S;
        if (VEC && j + 3 < S) {
            if (j < T) {
                f32x4 kv[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) kv[d] = *(const f32x4 *)(kb + (size_t)d * S + j);
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const float qv = qs[4 * dg + d];
                    s[0] = fmaf(qv, kv[d].x, s[0]);
                    s[1] = fmaf(qv, kv[d].y, s[1]);
                    s[2] = fmaf(qv, kv[d].z, s[2]);
                    s[3] = fmaf(qv, kv[d].w, s[3]);
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (j + e < T)
#pragma unroll
                    for (int d = 0; d < 4; ++d) s[e] = fmaf(qs[4 * dg + d], kb[(size_t)d * S + j + e], s[e]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) red[dg][4 * pq + e] = s[e];
    }
    __syncthreads();
    if (tid < 64) {
        const bool ok = j0 + tid < T;
        float s = 0.f;
#pragma unroll
        for (int g = 0; g < 16; ++g) s += red[g][tid];
        s *= a.scale;
        const float m = wave_max(ok ? s : -INFINITY);
        const float p = ok ? expf(s - m) : 0.f;
        const float l = wave_sum(p);
        pr[tid] = p;
        if (tid == 0) { stat[0] = m; stat[1] = l; }
    }
    __syncthreads();
    {
        const int d4 = tid & 15, jg = tid >> 4;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
        const float *vb = a.v_cache + h * 64 + 4 * d4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int jj = 4 * jg + e, j = j0 + jj;
            if (j < T) {
                const float p = pr[jj];
                if (VEC) {
                    const f32x4 vv = *(const f32x4 *)(vb + (size_t)j * D);
                    o[0] = fmaf(p, vv.x, o[0]);
                    o[1] = fmaf(p, vv.y, o[1]);
                    o[2] = fmaf(p, vv.z, o[2]);
                    o[3] = fmaf(p, vv.w, o[3]);
                } else {
#pragma unroll
                    for (int f = 0; f < 4; ++f) o[f] = fmaf(p, vb[(size_t)j * D + f], o[f]);
                }
            }
        }
#pragma unroll
        for (int f = 0; f < 4; ++f) red[jg][4 * d4 + f] = o[f];
    }
    __syncthreads();
    if (tid < 64) {
        float o = 0.f;
#pragma unroll
        for (int g = 0; g < 16; ++g) o += red[g][tid];
        float *pp = a.part + ((size_t)h * a.max_chunks + c) * 66;
        pp[2 + tid] = o;
        if (tid == 0) { pp[0] = stat[0]; pp[1] = stat[1]; }
    }
}

G2K void g2k_attn_part(const g2_attn1q_args a) { attn_part_impl<true>(a); }
G2K void g2k_attn_part_s(const g2_attn1q_args a) { attn_part_impl<false>(a); }

extern "C" __global__ __launch_bounds__(64) void g2k_attn_merge(const g2_attn1q_args a)
{
    __shared__ float cw[G2_KV_MAX_SEQ / 64];
    const int h = blockIdx.x, d = threadIdx.x;
    const int T = attn_T(a);
    const int nch = (T + 63) >> 6;
    if (h >= a.NH || nch > a.max_chunks) return;
    const float *hp = a.part + (size_t)h * a.max_chunks * 66;
    const float mc = d < nch ? hp[(size_t)d * 66] : -INFINITY;
    const float lc = d < nch ? hp[(size_t)d * 66 + 1] : 0.f;
    const float M = wave_max(mc);
    const float w = d < nch ? expf(mc - M) : 0.f;
    const float L = wave_sum(lc * w);
    if (d < nch) cw[d] = w;
    __syncthreads();
    float acc = 0.f;
    for (int c = 0; c < nch; ++c) acc = fmaf(hp[(size_t)c * 66 + 2 + d], cw[c], acc);
    a.out[h * 64 + d] = acc / L;
}

/* ======================================================================
 * Packed matvec rows
 * ==================================================================== */
enum { EPI_STORE = 0, EPI_GELU = 1, EPI_RESID = 2, EPI_QKV = 3, EPI_ARGMAX = 4 };

template <typename WT> struct chunk_t;
template <> struct chunk_t<float> { static constexpr int V = 4; };
template <> struct chunk_t<_Float16> { static constexpr int V = 8; };

/* One 16-byte chunk of weights times V input values. */
template <typename WT>
__device__ __forceinline__ float chunk_dot(const u32x4 &w, const float *x)
{
    if constexpr (sizeof(WT) == 4) {
        float s = __uint_as_float(w.x) * x[0];
        s = fmaf(__uint_as_float(w.y), x[1], s);
        s = fmaf(__uint_as_float(w.z), x[2], s);
        return fmaf(__uint_as_float(w.w), x[3], s);
    } else {
        const f16x8 h = __builtin_bit_cast(f16x8, w);
        float s = (float)h[0] * x[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) s = fmaf((float)h[i], x[i], s);
        return s;
    }
}

/* Sum of R values over a row group: one wave (SG 64) or the whole
 * work-group (SG 256, wave totals added in wave order through LDS). */
template <int SG, int R>
__device__ __forceinline__ void group_sum(float (&v)[R], float (*red)[4])
{
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = wave_sum(v[r]);
    if constexpr (SG == 256) {
        if ((threadIdx.x & 63) == 0)
#pragma unroll
            for (int r = 0; r < R; ++r) red[r][threadIdx.x >> 6] = v[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = ((red[r][0] + red[r][1]) + red[r][2]) + red[r][3];
        __syncthreads();
    }
}

__device__ __forceinline__ bool am_better(float v1, int i1, float v2, int i2)
{
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

/* WT: f32 or f16 weights; SG: lanes per row group (64 or 256); CPT: 16-byte
 * chunks per lane per row, so a row's K <= SG*CPT*V and the group's lanes
 * hold the whole input vector in registers; R: rows a group owns at once. */
template <typename WT, int EPI, bool LN, int SG, int CPT, int R>
__device__ void rows_impl(const g2_rows_args &a)
{
    constexpr int V = chunk_t<WT>::V;
    constexpr int G = 256 / SG;
    __shared__ float red[R > 2 ? R : 2][4];
    const int tid = threadIdx.x, gl = tid % SG;
    const int K = a.K, N = a.N, C = K / V;
    const u32x4 *W = (const u32x4 *)a.W;
    const int stride = gridDim.x * G * R;
    int row0 = (blockIdx.x * G + tid / SG) * R;

    /* 1. the lane's slice of the input vector (the group covers all of K) */
    float xv[CPT][V];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = gl + i * SG;
#pragma unroll
        for (int e = 0; e < V; e += 4) {
            f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
            if (c < C) v = *(const f32x4 *)(a.x + c * V + e);
            xv[i][e] = v.x; xv[i][e + 1] = v.y; xv[i][e + 2] = v.z; xv[i][e + 3] = v.w;
        }
    }
    /* 2. the weights of the group's first R rows */
    u32x4 w[R][CPT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = gl + i * SG, row = row0 + r;
            w[r][i] = (u32x4){0u, 0u, 0u, 0u};
            if (row < N && c < C) w[r][i] = __builtin_nontemporal_load(W + (size_t)row * C + c);
        }
    /* 3. LayerNorm while the weights stream in */
    if (LN) {
        float s[1] = {0.f};
#pragma unroll
        for (int i = 0; i < CPT; ++i)
#pragma unroll
            for (int e = 0; e < V; ++e) s[0] += xv[i][e];
        group_sum<SG, 1>(s, red);
        const float mean = s[0] / (float)K;
        float q[1] = {0.f};
#pragma unroll
        for (int i = 0; i < CPT; ++i)
            if (gl + i * SG < C)
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const float d = xv[i][e] - mean;
                    q[0] = fmaf(d, d, q[0]);
                }
        group_sum<SG, 1>(q, red);
        const float inv = 1.0f / sqrtf(q[0] / (float)K + 1e-5f);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = gl + i * SG;
            if (c < C)
#pragma unroll
                for (int e = 0; e < V; ++e)
                    xv[i][e] = fmaf((xv[i][e] - mean) * inv, a.ln_g[c * V + e], a.ln_b[c * V + e]);
        }
    }

    int pos = 0;
    if (EPI == EPI_QKV) pos = clampi(a.state[G2S_POS], 0, a.S - 1);
    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    int masked = -1;
    if (EPI == EPI_ARGMAX)
        masked = a.state[G2S_NGEN] < a.state[G2S_MIN_NEW] ? G2_EOS_ID : -1;

    for (; row0 < N; row0 += stride) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.f;
#pragma unroll
            for (int i = 0; i < CPT; ++i) acc[r] += chunk_dot<WT>(w[r][i], xv[i]);
        }
        /* next rows' weights go out before the reduction */
        const int nrow0 = row0 + stride;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                const int c = gl + i * SG, row = nrow0 + r;
                w[r][i] = (u32x4){0u, 0u, 0u, 0u};
                if (row < N && c < C) w[r][i] = __builtin_nontemporal_load(W + (size_t)row * C + c);
            }
        group_sum<SG, R>(acc, red);
        if (gl == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int n = row0 + r;
                if (n >= N) break;
                float v = acc[r];
                if (EPI == EPI_STORE) {
                    if (a.bias) v += a.bias[n];
                    a.y[n] = v;
                } else if (EPI == EPI_GELU) {
                    if (a.bias) v += a.bias[n];
                    a.y[n] = gelu_f(v);
                } else if (EPI == EPI_RESID) {
                    if (a.bias) v += a.bias[n];
                    a.y[n] = v + a.y[n];
                } else if (EPI == EPI_QKV) {
                    if (a.bias) v += a.bias[n];
                    const int E = a.E;
                    if (n < E) a.q_out[n] = v;
                    else if (n < 2 * E) a.k_cache[(size_t)(n - E) * a.S + pos] = v;
                    else a.v_cache[(size_t)pos * E + (n - 2 * E)] = v;
                } else {
                    a.y[n] = v;
                    const float mv = (n == masked) ? -1e30f : v;
                    if (am_better(mv, n, best_v, best_i)) { best_v = mv; best_i = n; }
                }
            }
        }
    }

    if constexpr (EPI == EPI_ARGMAX) {
        /* work-group partial (first-max); merged by g2k_argmax_merge */
        __shared__ float amv[256];
        __shared__ int ami[256];
        amv[tid] = best_v;
        ami[tid] = best_i;
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            if (tid < s && am_better(amv[tid + s], ami[tid + s], amv[tid], ami[tid])) {
                amv[tid] = amv[tid + s];
                ami[tid] = ami[tid + s];
            }
            __syncthreads();
        }
        if (tid == 0) {
            a.part[2 * blockIdx.x] = amv[0];
            a.part[2 * blockIdx.x + 1] = __int_as_float(ami[0]);
        }
    }
}

/* Greedy pick from the argmax partials of the lm_head work-groups (first
 * max wins ties); appends the id to state[G2S_IDS + NGEN] and sets TOK, and
 * with `advance` also POS+1 and NGEN+1.  One work-group. */
G2K void g2k_argmax_merge(const g2_amerge_args a)
{
    __shared__ float amv[256];
    __shared__ int ami[256];
    const int tid = threadIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int b = tid; b < a.n_parts; b += 256) {
        const float v = a.part[2 * b];
        const int i = __float_as_int(a.part[2 * b + 1]);
        if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    amv[tid] = bv;
    ami[tid] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s && am_better(amv[tid + s], ami[tid + s], amv[tid], ami[tid])) {
            amv[tid] = amv[tid + s];
            ami[tid] = ami[tid + s];
        }
        __syncthreads();
    }
    if (tid == 0) {
        const int tok = (ami[0] >= 0 && ami[0] < a.N) ? ami[0] : 0;
        const int ng = clampi(a.state[G2S_NGEN], 0, G2S_WORDS - G2S_IDS - 1);
        a.state[G2S_IDS + ng] = tok;
        a.state[G2S_TOK] = tok;
        if (a.advance) {
            a.state[G2S_NGEN] = ng + 1;
            a.state[G2S_POS] = a.state[G2S_POS] + 1;
        }
    }
}

/* Instantiations: per epilogue, the f32 and f16 twins of each lane shape, in
 * the order g2_internal.h lists them (SG lanes x CPT chunks x R rows):
 *   s64    64 x 4 x 1   rows of <= 256 chunks, short matrices (proj)
 *   s256r  256 x 1 x 2  rows of <= 256 chunks, long matrices (qkv, fc)
 *   s256   256 x 4 x 2  rows of <= 1024 chunks (fc2 of GPT-2 XL)
 *   s256x8 256 x 8 x 1  rows of <= 2048 chunks (fp32 ffn of large models)
 * chosen by measurement on the GPT-2 XL decode matrices. */
#define G2_ROWS_SET(ename, EPI, LN)                                                                                \
    G2K void g2k_rows_##ename##_f32_s64(const g2_rows_args a) { rows_impl<float, EPI, LN, 64, 4, 1>(a); }         \
    G2K void g2k_rows_##ename##_f16_s64(const g2_rows_args a) { rows_impl<_Float16, EPI, LN, 64, 4, 1>(a); }      \
    G2K void g2k_rows_##ename##_f32_s256r(const g2_rows_args a) { rows_impl<float, EPI, LN, 256, 1, 2>(a); }      \
    G2K void g2k_rows_##ename##_f16_s256r(const g2_rows_args a) { rows_impl<_Float16, EPI, LN, 256, 1, 2>(a); }   \
    G2K void g2k_rows_##ename##_f32_s256(const g2_rows_args a) { rows_impl<float, EPI, LN, 256, 4, 2>(a); }       \
    G2K void g2k_rows_##ename##_f16_s256(const g2_rows_args a) { rows_impl<_Float16, EPI, LN, 256, 4, 2>(a); }    \
    G2K void g2k_rows_##ename##_f32_s256x8(const g2_rows_args a) { rows_impl<float, EPI, LN, 256, 8, 1>(a); }     \
    G2K void g2k_rows_##ename##_f16_s256x8(const g2_rows_args a) { rows_impl<_Float16, EPI, LN, 256, 8, 1>(a); }

G2_ROWS_SET(store, EPI_STORE, false)
G2_ROWS_SET(ln_qkv, EPI_QKV, true)
G2_ROWS_SET(resid, EPI_RESID, false)
G2_ROWS_SET(ln_gelu, EPI_GELU, true)
G2_ROWS_SET(ln_argmax, EPI_ARGMAX, true)
