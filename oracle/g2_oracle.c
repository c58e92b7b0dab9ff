/*
 * g2_oracle.c -- CPU oracle for the GPT-2 per-token forward pass.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, the arithmetic of
 * the reference's OpenCL kernels (math.cl) and of its host orchestration
 * (main.c prefill/decode/sample_next_token).  Only the test suite, the smoke
 * check and the benchmark's CPU-baseline leg may load it, and only as the
 * checker / the timed CPU baseline.  The shipped library never calls it.
 *
 * Accumulation orders follow the reference kernels exactly:
 *   - dot products accumulate sequentially in k with a fused multiply-add
 *     (OpenCL C contracts a*b+c by default; the GPU compilers emit FMA);
 *   - matvec (scalar) keeps 4 interleaved partial sums (math.cl:165-177);
 *   - split-K slice s sums rows k = s, s+ks, ... (math.cl:242-243) and the
 *     reduce adds slices 0..ks-1 in order (math.cl:262-263);
 *   - layernorm is a serial two-pass over the row (math.cl:297-310);
 *   - softmax reduces with a 64-lane strided pass then a tree (math.cl:425-455).
 * Elementwise code is compiled with -ffp-contract=off so the only fused
 * operations are the explicit fmaf() calls.
 *
 * OpenMP parallelises over independent outputs only; the order of every
 * individual output's sum is the same for any thread count.
 *
 * Parity status per function: every function is pinned by the checks in
 * tests/test_oracle_ops.py and tests/test_oracle_model.py (library routines
 * in float64, closed forms, invariants and a transformers GPT-2 forward).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_EOS 50256

/* math.cl:21-23 (tanh-approximate GELU). */
static float gelu_f(float v)
{
    return 0.5f * v * (1.0f + tanhf(0.7978845608f * (v + 0.044715f * v * v * v)));
}

/* ---------------------------------------------------------------------
 * Operators (math.cl kernels and the runtime matmul of main.c:593-684)
 * ------------------------------------------------------------------- */

/* main.c:603-684 / math.cl:43-137: C[M,N] = A[M,K] B[K,N] (+bias[N]).
 * Every output accumulates sequentially in k (the tiles only change which
 * work-item owns an output), then adds the bias. */
void or_matmul(const float *A, const float *B, const float *bias, float *C,
               int M, int N, int K)
{
    const int NB = 256;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int m0 = 0; m0 < M; m0 += 4) {
        for (int n0 = 0; n0 < N; n0 += NB) {
            float acc[4][256];
            const int mm = (M - m0) < 4 ? (M - m0) : 4;
            const int nn = (N - n0) < NB ? (N - n0) : NB;
            for (int i = 0; i < mm; ++i)
                for (int j = 0; j < nn; ++j) acc[i][j] = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float *brow = B + (size_t)k * N + n0;
                for (int i = 0; i < mm; ++i) {
                    const float a = A[(size_t)(m0 + i) * K + k];
                    for (int j = 0; j < nn; ++j) acc[i][j] = fmaf(a, brow[j], acc[i][j]);
                }
            }
            for (int i = 0; i < mm; ++i)
                for (int j = 0; j < nn; ++j) {
                    float v = acc[i][j];
                    if (bias) v += bias[n0 + j];
                    C[(size_t)(m0 + i) * N + n0 + j] = v;
                }
        }
    }
}

/* math.cl:152-182: scalar matvec, one output per work-item, four interleaved
 * partial sums s0..s3 over k mod 4, tail into s0, sum = s0+s1+s2+s3. */
void or_matvec(const float *A, const float *B, const float *bias,
               const float *residual, float *C, int N, int K, int apply_gelu)
{
    #pragma omp parallel for schedule(static)
    for (int col = 0; col < N; ++col) {
        const float *Bcol = B + col;
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
        int k = 0;
        for (; k + 4 <= K; k += 4) {
            s0 = fmaf(A[k + 0], Bcol[(size_t)(k + 0) * N], s0);
            s1 = fmaf(A[k + 1], Bcol[(size_t)(k + 1) * N], s1);
            s2 = fmaf(A[k + 2], Bcol[(size_t)(k + 2) * N], s2);
            s3 = fmaf(A[k + 3], Bcol[(size_t)(k + 3) * N], s3);
        }
        for (; k < K; ++k) s0 = fmaf(A[k], Bcol[(size_t)k * N], s0);
        float sum = s0 + s1 + s2 + s3;
        if (bias) sum += bias[col];
        if (residual) sum += residual[col];
        if (apply_gelu) sum = gelu_f(sum);
        C[col] = sum;
    }
}

/* math.cl:185-226: matvec4, four columns per work-item, one accumulator per
 * column, sequential k; epilogue bias, residual, then GELU.  Requires N%4==0
 * (main.c:1560 routes other N to the scalar kernel). */
void or_matvec4(const float *A, const float *B, const float *bias,
                const float *residual, float *C, int N, int K, int apply_gelu)
{
    const int NB = 1024;
    #pragma omp parallel for schedule(static)
    for (int n0 = 0; n0 < N; n0 += NB) {
        float acc[1024];
        const int nn = (N - n0) < NB ? (N - n0) : NB;
        for (int j = 0; j < nn; ++j) acc[j] = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float a = A[k];
            const float *brow = B + (size_t)k * N + n0;
            for (int j = 0; j < nn; ++j) acc[j] = fmaf(a, brow[j], acc[j]);
        }
        for (int j = 0; j < nn; ++j) {
            float s = acc[j];
            if (bias) s += bias[n0 + j];
            if (residual) s += residual[n0 + j];
            if (apply_gelu) s = gelu_f(s);
            C[n0 + j] = s;
        }
    }
}

/* math.cl:229-246: split-K partials.  Slice s sums rows k = s, s+kslice, ...
 * partial is [kslice][N] floats (the reference's [kslice][N/4] float4). */
void or_matvec4_sk(const float *A, const float *B, float *partial,
                   int N, int K, int kslice)
{
    const int NB = 1024;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int s = 0; s < kslice; ++s) {
        for (int n0 = 0; n0 < N; n0 += NB) {
            float acc[1024];
            const int nn = (N - n0) < NB ? (N - n0) : NB;
            for (int j = 0; j < nn; ++j) acc[j] = 0.0f;
            for (int k = s; k < K; k += kslice) {
                const float a = A[k];
                const float *brow = B + (size_t)k * N + n0;
                for (int j = 0; j < nn; ++j) acc[j] = fmaf(a, brow[j], acc[j]);
            }
            for (int j = 0; j < nn; ++j) partial[(size_t)s * N + n0 + j] = acc[j];
        }
    }
}

/* math.cl:249-280: sum slices 0..kslice-1 in order, then bias, residual, GELU. */
void or_reduce_partial(const float *partial, const float *bias,
                       const float *residual, float *C, int N, int kslice,
                       int apply_gelu)
{
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        float s = 0.0f;
        for (int k = 0; k < kslice; ++k) s += partial[(size_t)k * N + n];
        if (bias) s += bias[n];
        if (residual) s += residual[n];
        if (apply_gelu) s = gelu_f(s);
        C[n] = s;
    }
}

/* math.cl:283-311: serial two-pass LayerNorm per row, biased variance,
 * eps 1e-5, out = (x-mean)*inv_std*gamma + beta. */
void or_layernorm(const float *x, float *out, const float *gamma,
                  const float *beta, int n_embd, int seq_len)
{
    #pragma omp parallel for schedule(static)
    for (int s = 0; s < seq_len; ++s) {
        const float *xi = x + (size_t)s * n_embd;
        float *xo = out + (size_t)s * n_embd;
        float mean = 0.0f;
        for (int i = 0; i < n_embd; ++i) mean += xi[i];
        mean /= (float)n_embd;
        float var = 0.0f;
        for (int i = 0; i < n_embd; ++i) {
            const float d = xi[i] - mean;
            var = fmaf(d, d, var);
        }
        var /= (float)n_embd;
        const float inv_std = 1.0f / sqrtf(var + 1e-5f);
        for (int i = 0; i < n_embd; ++i)
            xo[i] = fmaf((xi[i] - mean) * inv_std, gamma[i], beta[i]);
    }
}

/* math.cl:314-322 */
void or_add_inplace(float *a, const float *b, int n)
{
    for (int i = 0; i < n; ++i) a[i] += b[i];
}

/* math.cl:325-330 */
void or_gelu(float *x, int n)
{
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) x[i] = gelu_f(x[i]);
}

/* math.cl:333-350 */
void or_embed(const float *wte, const float *wpe, float *out, int n_embd,
              int seq_len, int start_pos, const int *ids)
{
    for (int i = 0; i < seq_len; ++i) {
        const int pos = start_pos + i, tok = ids[i];
        for (int d = 0; d < n_embd; ++d)
            out[(size_t)i * n_embd + d] =
                wte[(size_t)tok * n_embd + d] + wpe[(size_t)pos * n_embd + d];
    }
}

/* math.cl:367-383: K goes to the transposed cache kc[d*MAX_SEQ + pos],
 * V to vc[pos*D + d]. */
void or_split_kv(const float *qkv, float *k_cache, float *v_cache,
                 int start_pos, int T, int D, int max_seq)
{
    for (int i = 0; i < T; ++i) {
        const int pos = start_pos + i;
        for (int d = 0; d < D; ++d) {
            k_cache[(size_t)d * max_seq + pos] = qkv[(size_t)i * 3 * D + D + d];
            v_cache[(size_t)pos * D + d] = qkv[(size_t)i * 3 * D + 2 * D + d];
        }
    }
}

/* math.cl:388-412: scores[h*max_seq + j] = scale * sum_k q[h*DH+k] kc[(h*DH+k)*max_seq + j]. */
void or_attn_scores_1q(const float *qkv, const float *k_cache, float *scores,
                       int q_base, int T_kv, int D, int DH, int NH,
                       int max_seq, float scale)
{
    (void)D;
    const float *q_row = qkv + q_base;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int h = 0; h < NH; ++h) {
        for (int j = 0; j < T_kv; ++j) {
            const int off = h * DH;
            float s = 0.0f;
            for (int k = 0; k < DH; ++k)
                s = fmaf(q_row[off + k], k_cache[(size_t)(off + k) * max_seq + j], s);
            scores[(size_t)h * max_seq + j] = s * scale;
        }
    }
}

/* math.cl:415-456 with a work-group of `lws` items per head (main.c:1711
 * uses attn_lws = 64).  Row stride is `row_stride` (ATTN_MAX_SEQ_LEN=1024). */
void or_attn_softmax_1q(float *scores, int T_kv, int NH, int row_stride, int lws)
{
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < NH; ++h) {
        float scratch[256] = { 0 };
        float *row = scores + (size_t)h * row_stride;
        for (int lid = 0; lid < lws; ++lid) {
            float mx = -1e30f;
            for (int j = lid; j < T_kv; j += lws)
                if (row[j] > mx) mx = row[j];
            scratch[lid] = mx;
        }
        for (int s = lws >> 1; s > 0; s >>= 1)
            for (int lid = 0; lid < s; ++lid) {
                const float a = scratch[lid], b = scratch[lid + s];
                scratch[lid] = a > b ? a : b;
            }
        const float m = scratch[0];
        for (int lid = 0; lid < lws; ++lid) {
            float sum = 0.0f;
            for (int j = lid; j < T_kv; j += lws) {
                const float e = expf(row[j] - m);
                row[j] = e;
                sum += e;
            }
            scratch[lid] = sum;
        }
        for (int s = lws >> 1; s > 0; s >>= 1)
            for (int lid = 0; lid < s; ++lid) scratch[lid] += scratch[lid + s];
        const float inv = 1.0f / scratch[0];
        for (int j = 0; j < T_kv; ++j) row[j] *= inv;
    }
}

/* math.cl:459-476: out[out_base+d] = sum_j P[d/DH, j] * vc[j*D + d], sequential j. */
void or_attn_out_1q(const float *scores, const float *v_cache, float *out,
                    int T_kv, int D, int DH, int out_base, int row_stride)
{
    #pragma omp parallel for schedule(static)
    for (int d = 0; d < D; ++d) {
        const int h = d / DH;
        const float *srow = scores + (size_t)h * row_stride;
        float s = 0.0f;
        for (int j = 0; j < T_kv; ++j) s = fmaf(srow[j], v_cache[(size_t)j * D + d], s);
        out[out_base + d] = s;
    }
}

/* ---------------------------------------------------------------------
 * Model (main.c:1739-1833) and greedy selection (main.c:1872-1904)
 * ------------------------------------------------------------------- */

#define OR_MAX_SEQ 1024

typedef struct {
    int n_layer, n_embd, n_head, vocab, ffn, padded_vocab, kslice;
    /* weights in the reference's device layout: linear weights [in,out],
     * lm_head [E, padded_vocab] with zero pad columns (main.c:1252-1337) */
    const float *wte, *wpe, *lnf_w, *lnf_b;
    const float **ln1_w, **ln1_b, **qkv_w, **qkv_b, **proj_w, **proj_b;
    const float **ln2_w, **ln2_b, **fc_w, **fc_b, **fc2_w, **fc2_b;
    float *lm_head;
    /* workspaces (main.c:1451-1490) */
    float *hidden, *ln_out, *attn, *attn_proj, *ffn1, *ffn2, *qkv_new;
    float *qkv_full, *last_hidden, *logits, *partial, *scores;
    float **k_cache, **v_cache;
} or_model;

static void *xcalloc(size_t n, size_t sz)
{
    void *p = calloc(n, sz);
    if (!p) abort();
    return p;
}

/* Create a model over caller-owned weights.  `layers` holds 12 pointers per
 * layer in the order ln1_w, ln1_b, qkv_w, qkv_b, proj_w, proj_b, ln2_w,
 * ln2_b, fc_w, fc_b, fc2_w, fc2_b; linear weights are [in,out] row-major.
 * The tied lm_head is padded and transposed here as make_padded_lm_head does
 * (main.c:1302-1337). */
or_model *or_model_create(int n_layer, int n_embd, int n_head, int vocab,
                          int ffn, int kslice, const float *wte,
                          const float *wpe, const float *lnf_w,
                          const float *lnf_b, const float *const *layers)
{
    or_model *m = xcalloc(1, sizeof *m);
    m->n_layer = n_layer; m->n_embd = n_embd; m->n_head = n_head;
    m->vocab = vocab; m->ffn = ffn; m->kslice = kslice;
    m->padded_vocab = (vocab + 3) & ~3;                       /* main.c:326 */
    m->wte = wte; m->wpe = wpe; m->lnf_w = lnf_w; m->lnf_b = lnf_b;
    const float ***slots[12] = { &m->ln1_w, &m->ln1_b, &m->qkv_w, &m->qkv_b,
                                 &m->proj_w, &m->proj_b, &m->ln2_w, &m->ln2_b,
                                 &m->fc_w, &m->fc_b, &m->fc2_w, &m->fc2_b };
    for (int s = 0; s < 12; ++s) {
        *slots[s] = xcalloc((size_t)n_layer, sizeof(float *));
        for (int l = 0; l < n_layer; ++l) (*slots[s])[l] = layers[(size_t)l * 12 + s];
    }
    const size_t E = (size_t)n_embd, F = (size_t)ffn, T = 3 * E, S = OR_MAX_SEQ;
    const size_t V = (size_t)m->padded_vocab;
    m->lm_head = xcalloc(E * V, sizeof(float));
    #pragma omp parallel for schedule(static)
    for (int k = 0; k < (int)E; ++k)
        for (int n = 0; n < vocab; ++n)
            m->lm_head[(size_t)k * V + n] = wte[(size_t)n * E + k];
    m->hidden = xcalloc(S * E, sizeof(float));
    m->ln_out = xcalloc(S * E, sizeof(float));
    m->attn = xcalloc(S * E, sizeof(float));
    m->attn_proj = xcalloc(S * E, sizeof(float));
    m->ffn1 = xcalloc(S * F, sizeof(float));
    m->ffn2 = xcalloc(S * E, sizeof(float));
    m->qkv_new = xcalloc(T, sizeof(float));
    m->qkv_full = xcalloc(S * T, sizeof(float));
    m->last_hidden = xcalloc(E, sizeof(float));
    m->logits = xcalloc(V, sizeof(float));
    m->partial = xcalloc((size_t)8 * V, sizeof(float));
    m->scores = xcalloc((size_t)n_head * S, sizeof(float));
    m->k_cache = xcalloc((size_t)n_layer, sizeof(float *));
    m->v_cache = xcalloc((size_t)n_layer, sizeof(float *));
    for (int l = 0; l < n_layer; ++l) {
        m->k_cache[l] = xcalloc(E * S, sizeof(float));
        m->v_cache[l] = xcalloc(S * E, sizeof(float));
    }
    return m;
}

/* A separate lm_head [vocab, n_embd] instead of the tied wte (main.c:1374-1405:
 * lm_head.weight present in the file): padded and transposed the same way. */
void or_model_set_lm_head(or_model *m, const float *lm)
{
    const size_t E = (size_t)m->n_embd, V = (size_t)m->padded_vocab;
    memset(m->lm_head, 0, E * V * sizeof(float));
    #pragma omp parallel for schedule(static)
    for (int k = 0; k < (int)E; ++k)
        for (int n = 0; n < m->vocab; ++n)
            m->lm_head[(size_t)k * V + n] = lm[(size_t)n * E + k];
}

void or_model_destroy(or_model *m)
{
    if (!m) return;
    const float **slots[12] = { m->ln1_w, m->ln1_b, m->qkv_w, m->qkv_b,
                                m->proj_w, m->proj_b, m->ln2_w, m->ln2_b,
                                m->fc_w, m->fc_b, m->fc2_w, m->fc2_b };
    for (int s = 0; s < 12; ++s) free((void *)slots[s]);
    for (int l = 0; l < m->n_layer; ++l) { free(m->k_cache[l]); free(m->v_cache[l]); }
    free(m->k_cache); free(m->v_cache);
    free(m->lm_head); free(m->hidden); free(m->ln_out); free(m->attn);
    free(m->attn_proj); free(m->ffn1); free(m->ffn2); free(m->qkv_new);
    free(m->qkv_full); free(m->last_hidden); free(m->logits); free(m->partial);
    free(m->scores);
    free(m);
}

/* main.c:1554-1576: matvec4 when N%4==0, scalar matvec otherwise. */
static void launch_matvec(const float *A, const float *B, const float *bias,
                          const float *res, float *C, int N, int K, int gelu)
{
    if ((N & 3) == 0) or_matvec4(A, B, bias, res, C, N, K, gelu);
    else or_matvec(A, B, bias, res, C, N, K, gelu);
}

/* main.c:1578-1618: split-K with the pinned slice count; ks<=1 falls back. */
static void launch_matvec_splitk(or_model *m, const float *A, const float *B,
                                 const float *bias, const float *res, float *C,
                                 int N, int K, int gelu)
{
    const int ks = m->kslice;
    if ((N & 3) != 0 || ks <= 1 || ks > 8) {
        launch_matvec(A, B, bias, res, C, N, K, gelu);
        return;
    }
    or_matvec4_sk(A, B, m->partial, N, K, ks);
    or_reduce_partial(m->partial, bias, res, C, N, ks, gelu);
}

static void attention_row(or_model *m, const float *qkv, int l, int q_base,
                          int T_kv, float *out, int out_base)
{
    const int E = m->n_embd, DH = E / m->n_head;
    const float scale = 1.0f / sqrtf((float)DH);              /* main.c:1692 */
    or_attn_scores_1q(qkv, m->k_cache[l], m->scores, q_base, T_kv, E, DH,
                      m->n_head, OR_MAX_SEQ, scale);
    or_attn_softmax_1q(m->scores, T_kv, m->n_head, OR_MAX_SEQ, 64);
    or_attn_out_1q(m->scores, m->v_cache[l], out, T_kv, E, DH, out_base, OR_MAX_SEQ);
}

/* main.c:1739-1790 */
void or_prefill(or_model *m, const int *ids, int P)
{
    const int E = m->n_embd, T = 3 * E, F = m->ffn;
    or_embed(m->wte, m->wpe, m->hidden, E, P, 0, ids);
    for (int l = 0; l < m->n_layer; ++l) {
        or_layernorm(m->hidden, m->ln_out, m->ln1_w[l], m->ln1_b[l], E, P);
        or_matmul(m->ln_out, m->qkv_w[l], m->qkv_b[l], m->qkv_full, P, T, E);
        or_split_kv(m->qkv_full, m->k_cache[l], m->v_cache[l], 0, P, E, OR_MAX_SEQ);
        for (int i = 0; i < P; ++i)
            attention_row(m, m->qkv_full, l, i * 3 * E, i + 1, m->attn, i * E);
        or_matmul(m->attn, m->proj_w[l], m->proj_b[l], m->attn_proj, P, E, E);
        or_add_inplace(m->hidden, m->attn_proj, P * E);
        or_layernorm(m->hidden, m->ln_out, m->ln2_w[l], m->ln2_b[l], E, P);
        or_matmul(m->ln_out, m->fc_w[l], m->fc_b[l], m->ffn1, P, F, E);
        or_gelu(m->ffn1, P * F);
        or_matmul(m->ffn1, m->fc2_w[l], m->fc2_b[l], m->ffn2, P, E, F);
        or_add_inplace(m->hidden, m->ffn2, P * E);
    }
    or_layernorm(m->hidden, m->ln_out, m->lnf_w, m->lnf_b, E, P);
    memcpy(m->last_hidden, m->ln_out + (size_t)(P - 1) * E, (size_t)E * sizeof(float));
    launch_matvec(m->last_hidden, m->lm_head, NULL, NULL, m->logits,
                  m->padded_vocab, E, 0);
}

/* main.c:1792-1833 */
void or_decode(or_model *m, int tok, int pos)
{
    const int E = m->n_embd, T = 3 * E, F = m->ffn;
    or_embed(m->wte, m->wpe, m->hidden, E, 1, pos, &tok);
    for (int l = 0; l < m->n_layer; ++l) {
        or_layernorm(m->hidden, m->ln_out, m->ln1_w[l], m->ln1_b[l], E, 1);
        launch_matvec(m->ln_out, m->qkv_w[l], m->qkv_b[l], NULL, m->qkv_new, T, E, 0);
        or_split_kv(m->qkv_new, m->k_cache[l], m->v_cache[l], pos, 1, E, OR_MAX_SEQ);
        attention_row(m, m->qkv_new, l, 0, pos + 1, m->attn, 0);
        launch_matvec_splitk(m, m->attn, m->proj_w[l], m->proj_b[l], m->hidden,
                             m->hidden, E, E, 0);
        or_layernorm(m->hidden, m->ln_out, m->ln2_w[l], m->ln2_b[l], E, 1);
        launch_matvec(m->ln_out, m->fc_w[l], m->fc_b[l], NULL, m->ffn1, F, E, 1);
        launch_matvec_splitk(m, m->ffn1, m->fc2_w[l], m->fc2_b[l], m->hidden,
                             m->hidden, E, F, 0);
    }
    or_layernorm(m->hidden, m->ln_out, m->lnf_w, m->lnf_b, E, 1);
    launch_matvec(m->ln_out, m->lm_head, NULL, NULL, m->logits, m->padded_vocab, E, 0);
}

const float *or_logits(const or_model *m) { return m->logits; }

/* Overwrite layer l's caches (K transposed [E,1024], V [1024,E]); lets a
 * timing sample start decoding at a late position without a CPU prefill. */
void or_set_kv(or_model *m, int l, const float *k_cache, const float *v_cache)
{
    const size_t n = (size_t)m->n_embd * OR_MAX_SEQ;
    memcpy(m->k_cache[l], k_cache, n * sizeof(float));
    memcpy(m->v_cache[l], v_cache, n * sizeof(float));
}

#ifdef _OPENMP
#include <omp.h>
int or_num_threads(void) { return omp_get_max_threads(); }
#else
int or_num_threads(void) { return 1; }
#endif

/* main.c:1872-1904, greedy branch (temperature <= 0).  Works on a copy of
 * the first `vocab` logits: EOS mask, repetition penalty over distinct
 * context ids, then first-max argmax (lowest index wins ties). */
int or_greedy(const float *logits_in, int vocab, const int *ctx, int n_ctx,
              int forbid_eos, float rep_penalty, float *work)
{
    memcpy(work, logits_in, (size_t)vocab * sizeof(float));
    if (forbid_eos && OR_EOS < vocab) work[OR_EOS] = -1e30f;
    if (rep_penalty > 1.0f) {
        for (int i = 0; i < n_ctx; ++i) {
            const int tk = ctx[i];
            if (tk < 0 || tk >= vocab) continue;
            int dup = 0;
            for (int j = 0; j < i; ++j)
                if (ctx[j] == tk) { dup = 1; break; }
            if (dup) continue;
            if (work[tk] > 0.0f) work[tk] /= rep_penalty;
            else work[tk] *= rep_penalty;
        }
    }
    int best = 0;
    float bv = work[0];
    for (int i = 1; i < vocab; ++i)
        if (work[i] > bv) { bv = work[i]; best = i; }
    return best;
}

/* main.c:2106-2150 with temperature 0: prefill, first token from the prefill
 * logits, then decode until max_new tokens or seq_len 1024 or EOS.
 * min_new gives the EOS mask window (main.c:2110,2130).  Writes generated
 * ids to out_ids; if `logit_top2` is non-NULL it receives, per generated
 * token, the chosen logit and the runner-up after masking (the top-2 gap);
 * if `logits_out` is non-NULL and `logit_steps` > 0 it receives the padded
 * logits of the first `logit_steps` tokens.  Returns the number generated. */
int or_generate(or_model *m, const int *prompt, int P, int max_new, int min_new,
                float rep_penalty, int *out_ids, float *logit_top2,
                float *logits_out, int logit_steps)
{
    int *ids = xcalloc(OR_MAX_SEQ + 1, sizeof(int));
    float *work = xcalloc((size_t)m->padded_vocab, sizeof(float));
    memcpy(ids, prompt, (size_t)P * sizeof(int));
    int seq_len = P, generated = 0, next;
    or_prefill(m, ids, P);
    for (;;) {
        const int forbid = generated < min_new;
        next = or_greedy(m->logits, m->vocab, ids, seq_len, forbid, rep_penalty, work);
        if (logit_top2) {
            float second = -INFINITY;
            for (int i = 0; i < m->vocab; ++i)
                if (i != next && work[i] > second) second = work[i];
            logit_top2[2 * generated] = work[next];
            logit_top2[2 * generated + 1] = second;
        }
        if (logits_out && generated < logit_steps)
            memcpy(logits_out + (size_t)generated * m->padded_vocab, m->logits,
                   (size_t)m->padded_vocab * sizeof(float));
        ids[seq_len++] = next;
        out_ids[generated++] = next;
        if (generated >= max_new || next == OR_EOS || seq_len >= OR_MAX_SEQ) break;
        or_decode(m, ids[seq_len - 1], seq_len - 1);
    }
    free(ids);
    free(work);
    return generated;
}

/* Teacher-forced decode: run prefill on prompt[0..P) and then decode the
 * given forced tokens one by one, storing the padded logits after each
 * forward (n_forced + 1 rows: prefill, then each decode). */
void or_teacher_forced(or_model *m, const int *prompt, int P, const int *forced,
                       int n_forced, float *logits_out)
{
    const size_t V = (size_t)m->padded_vocab;
    or_prefill(m, prompt, P);
    memcpy(logits_out, m->logits, V * sizeof(float));
    for (int i = 0; i < n_forced; ++i) {
        or_decode(m, forced[i], P + i);
        memcpy(logits_out + (size_t)(i + 1) * V, m->logits, V * sizeof(float));
    }
}
