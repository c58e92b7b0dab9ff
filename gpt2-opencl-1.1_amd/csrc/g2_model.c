/*
 * g2_model.c -- GPT-2 model on one gfx950 GPU: weight upload and layout,
 * workspaces and KV caches, prefill/decode orchestration, greedy selection
 * and the replayed decode graph.  C99 host code over the HIP runtime C API.
 *
 * Two execution paths (g2hip.h):
 *  REFERENCE -- the reference's sequence of operator launches, restated from
 *    prefill()/decode() (main.c:1739-1833) over this library's reference
 *    operators, with the reference's device layouts: linear weights [in,out]
 *    (load_linear_weight, main.c:1252-1300), tied lm_head copied to a
 *    zero-padded [E, ceil4(V)] matrix (make_padded_lm_head, main.c:1302-1337),
 *    K cache transposed [E,1024], V cache [1024,E] (main.c:1481-1486).
 *  FUSED -- per layer and token five kernels: LayerNorm+qkv matvec with the
 *    K/V scatter, split single-query attention, proj matvec + residual,
 *    LayerNorm+fc matvec + GELU, fc2 matvec + residual; then LayerNorm +
 *    lm_head over wte + argmax.  Matrices are packed output-major [out,in]
 *    (f32 or f16) so each output row is one contiguous stream; the tied
 *    lm_head is wte itself ([V,E] is already output-major).  Token and
 *    position live in device memory, so one captured graph is replayed for
 *    every decode step.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g2_internal.h"
#include "g2_host.h"
#include "g2_step_plan.h"
#include "g2_gemm_plan.h"
#include "g2_attn_plan.h"

typedef struct {
    float *ln1_w, *ln1_b, *qkv_b, *proj_b, *ln2_w, *ln2_b, *fc_b, *fc2_b;
    void *qkv_w, *proj_w, *fc_w, *fc2_w;
    float *k_cache, *v_cache;
} g2_layer;

struct g2_model {
    g2_config cfg;
    int dtype, path, kslice, padded_vocab;
    size_t weight_bytes;
    void *wte, *wpe;
    void *lm_w; /* fused path lm_head [V,E] in the weight dtype (wte when tied) */
    float *lnf_w, *lnf_b;
    float *lm_head; /* reference path: padded [E, Vpad] */
    g2_layer *L;
    /* workspaces (main.c:1451-1490) */
    float *hidden, *ln_out, *attn, *attn_proj, *ffn1, *ffn2, *qkv_new, *qkv_full;
    float *last_hidden, *logits, *partial, *scores, *q;
    float *pf_part; /* split-K slices of the fp16 prefill GEMM */
    float *pf_help; /* helper slots of the prompt attention, G2V_EMPTY between launches */
    int help_ran;   /* a prompt attention with helpers ran since the last error check */
    uint16_t *pf_kv; /* the prompt's K and V as fp16 halves: kh, kl [S][E], vth, vtl [E][S] */
    int *ids_dev;
    /* fused path */
    int *state;
    float *att_part, *am_part;
    /* persistent step kernel: per-layer pointer table, exchange areas */
    g2_step_layer *step_layers;
    g2p_rows *step_shares; /* row plans [step_wgs][G2P_NSHARES] (g2p_shares) */
    unsigned long long *xbuf;
    size_t xbuf_bytes;
    float *xval;
    size_t xval_floats;
    float *lnfold; /* per layer qkv c1, c2 [3E], fc c1, c2 [F]; then lm c1, c2 [V] */
    int step_wgs;  /* grid of the step kernel, 0 if this model cannot use it */
    int step_on;   /* decode steps run the step kernel */
    int plain;     /* launches are plain, not cooperative (2-4: test modes of the
                      residency check, see g2_step_args.plain) */
    int step_ran;  /* a step kernel ran since the last error check */
    const char *step_why; /* why the step kernel cannot run this model */
    unsigned long long *trace; /* phase timestamps, when G2_STEP_TRACE names a file */
    size_t trace_words;
    hipGraphExec_t step_exec;
    int graph_state; /* 0 not built, 1 ready, -1 capture unsupported */
    hipEvent_t ev[3];
    int events_ok;
    float *host_logits;
};

/* ---------------------------------------------------------------- helpers */

static unsigned cdivu(long a, long b) { return (unsigned)((a + b - 1) / b); }

static int dev_alloc(g2_model *m, void **p, size_t bytes, int is_weight)
{
    int rc = g2i_device_alloc(p, bytes);
    if (!rc && is_weight) m->weight_bytes += bytes;
    return rc;
}

static int up(void *dst, const void *src, size_t bytes)
{
    int rc = g2i_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g2i_stream()), "upload");
    if (rc) return rc;
    return g2i_hip(hipStreamSynchronize(g2i_stream()), "upload sync");
}

/* Upload a host fp32 vector as a new device fp32 buffer. */
static int up_vec(g2_model *m, float **dst, const float *src, size_t n)
{
    int rc = dev_alloc(m, (void **)dst, n * sizeof(float), 1);
    if (!rc) rc = up(*dst, src, n * sizeof(float));
    return rc;
}

/* Upload a host fp32 array in the model's weight dtype. */
static int up_typed(g2_model *m, void **dst, const float *src, size_t n)
{
    int rc;
    if (m->dtype == G2_F32) {
        rc = dev_alloc(m, dst, n * sizeof(float), 1);
        if (!rc) rc = up(*dst, src, n * sizeof(float));
        return rc;
    }
    uint16_t *h = malloc(n * sizeof(uint16_t));
    if (!h) return g2i_err(G2_E_NOMEM, "host staging");
    g2i_f32_to_f16(h, src, n);
    rc = dev_alloc(m, dst, n * sizeof(uint16_t), 1);
    if (!rc) rc = up(*dst, h, n * sizeof(uint16_t));
    free(h);
    return rc;
}

/* A linear weight given in the Conv1D layout [in,out]: the reference path
 * keeps it (main.c:1252-1300 produces [in,out]); the fused path stores the
 * transpose [out,in] in the model dtype. */
static int up_linear(g2_model *m, void **dst, const float *w_in_out, int in, int out)
{
    if (m->path == G2_PATH_REFERENCE) return up_typed(m, dst, w_in_out, (size_t)in * out);
    float *t = malloc((size_t)in * out * sizeof(float));
    if (!t) return g2i_err(G2_E_NOMEM, "transpose staging");
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < out; ++o)
        for (int i = 0; i < in; ++i) t[(size_t)o * in + i] = w_in_out[(size_t)i * out + o];
    int rc = up_typed(m, dst, t, (size_t)in * out);
    free(t);
    return rc;
}

/* Reference path lm_head: [E, Vpad] with columns >= V zero (main.c:1302-1337). */
static int up_padded_lm_head(g2_model *m, const float *wte)
{
    const int E = m->cfg.n_embd, V = m->cfg.vocab_size, Vp = m->padded_vocab;
    float *t = calloc((size_t)E * Vp, sizeof(float));
    if (!t) return g2i_err(G2_E_NOMEM, "lm_head staging");
    #pragma omp parallel for schedule(static)
    for (int k = 0; k < E; ++k)
        for (int n = 0; n < V; ++n) t[(size_t)k * Vp + n] = wte[(size_t)n * E + k];
    int rc = dev_alloc(m, (void **)&m->lm_head, (size_t)E * Vp * sizeof(float), 1);
    if (!rc) rc = up(m->lm_head, t, (size_t)E * Vp * sizeof(float));
    free(t);
    return rc;
}

static int check_model_config(const g2_config *c, int dtype, int path)
{
    if (!c) return g2i_err(G2_E_ARG, "NULL config");
    if (dtype != G2_F32 && dtype != G2_F16) return g2i_err(G2_E_ARG, "weight dtype %d unknown", dtype);
    if (path != G2_PATH_REFERENCE && path != G2_PATH_FUSED) return g2i_err(G2_E_ARG, "path %d unknown", path);
    if (path == G2_PATH_REFERENCE && dtype != G2_F32)
        return g2i_err(G2_E_ARG, "the reference path stores fp32 weights only");
    if (c->n_layer <= 0 || c->n_embd <= 0 || c->n_head <= 0 || c->vocab_size <= 0 || c->ffn_dim <= 0)
        return g2i_err(G2_E_ARG, "non-positive model size");
    if (c->n_embd > G2_MAX_EMBED || c->n_layer > G2_MAX_LAYERS || c->n_head > G2_MAX_HEADS ||
        c->vocab_size > G2_MAX_VOCAB || c->ffn_dim > G2_MAX_FFN)
        return g2i_err(G2_E_LIMIT, "model exceeds compiled-in ceilings");
    if (c->n_embd % c->n_head) return g2i_err(G2_E_ARG, "n_embd not divisible by n_head");
    if (path == G2_PATH_FUSED) {
        if (c->n_embd != 64 * c->n_head) return g2i_err(G2_E_ARG, "fused path needs head dim 64");
        if (c->n_embd % 8 || c->ffn_dim % 8) return g2i_err(G2_E_ARG, "fused path needs n_embd, ffn multiples of 8");
        if (c->ffn_dim > G2_ROWS_MAXK) return g2i_err(G2_E_LIMIT, "ffn above %d", G2_ROWS_MAXK);
    }
    return G2_OK;
}

/* Exchange areas of the step kernel to their empty state: tags 0 (no step
 * has tag 0) and every value G2V_EMPTY. */
static int exchange_clear(g2_model *m)
{
    int rc = g2i_hip(hipMemsetAsync(m->xbuf, 0, m->xbuf_bytes, g2i_stream()), "exchange clear");
    if (!rc) rc = g2i_hip(hipMemsetD32Async((hipDeviceptr_t)m->xval, (int)G2V_EMPTY, m->xval_floats, g2i_stream()),
                          "exchange clear");
    return rc;
}

/* Whether the persistent step kernel can run this model: fused path, a
 * device grid and the kernel's own limits (g2p_step_refusal, shared with
 * the kernel's CPU address check).  On refusal `why` names the reason. */
static int step_supported(const g2_model *m, int nwg, const char **why)
{
    const g2_config *c = &m->cfg;
    if (m->path != G2_PATH_FUSED) { *why = "not the fused path"; return 0; }
    *why = g2p_step_refusal(c->n_embd, c->n_head, c->ffn_dim, c->vocab_size, m->dtype == G2_F16 ? 8 : 4, nwg);
    return *why == NULL;
}

/* Device tables of the step kernel (after the weights are uploaded). */
static int step_setup(g2_model *m)
{
    const int nwg = g2i_step_wgs();
    if (!step_supported(m, nwg, &m->step_why)) return G2_OK;
    const g2_config *c = &m->cfg;
    const int L = c->n_layer;
    const size_t E = (size_t)c->n_embd, F = (size_t)c->ffn_dim, V = (size_t)c->vocab_size;
    const size_t per_layer = 6 * E + 2 * F;
    int rc = dev_alloc(m, (void **)&m->lnfold, ((size_t)L * per_layer + 2 * V) * 4, 0);
    if (rc) return rc;
    g2_step_layer *t = calloc((size_t)L, sizeof *t);
    if (!t) return g2i_err(G2_E_NOMEM, "step layer table");
    const int ffold = m->dtype == G2_F16 ? G2F_LN_FOLD_F16 : G2F_LN_FOLD_F32;
    for (int l = 0; l < L && !rc; ++l) {
        const g2_layer *y = &m->L[l];
        float *f = m->lnfold + (size_t)l * per_layer;
        t[l].ln1_w = y->ln1_w; t[l].proj_b = y->proj_b; t[l].ln2_w = y->ln2_w; t[l].fc2_b = y->fc2_b;
        t[l].qkv_w = y->qkv_w; t[l].proj_w = y->proj_w; t[l].fc_w = y->fc_w; t[l].fc2_w = y->fc2_w;
        t[l].k_cache = y->k_cache; t[l].v_cache = y->v_cache;
        t[l].qkv_c1 = f; t[l].qkv_c2 = f + 3 * E; t[l].fc_c1 = f + 6 * E; t[l].fc_c2 = f + 6 * E + F;
        g2_lnfold_args q = { y->qkv_w, y->ln1_w, y->ln1_b, y->qkv_b, f, f + 3 * E, (int)(3 * E), (int)E };
        rc = g2i_launch(ffold, cdivu((long)(3 * E), 4), 1, 256, &q);
        g2_lnfold_args u = { y->fc_w, y->ln2_w, y->ln2_b, y->fc_b, f + 6 * E, f + 6 * E + F, (int)F, (int)E };
        if (!rc) rc = g2i_launch(ffold, cdivu((long)F, 4), 1, 256, &u);
    }
    if (!rc) {
        float *f = m->lnfold + (size_t)L * per_layer;
        g2_lnfold_args u = { m->lm_w, m->lnf_w, m->lnf_b, NULL, f, f + V, (int)V, (int)E };
        rc = g2i_launch(ffold, cdivu((long)V, 4), 1, 256, &u);
    }
    if (!rc) rc = dev_alloc(m, (void **)&m->step_layers, (size_t)L * sizeof *t, 0);
    if (!rc) rc = up(m->step_layers, t, (size_t)L * sizeof *t);
    free(t);
    /* every work-group's row plans, read by the kernel phase by phase */
    const size_t nsh = (size_t)nwg * G2P_NSHARES;
    g2p_rows *sh = rc ? NULL : calloc(nsh, sizeof *sh);
    if (!rc && !sh) rc = g2i_err(G2_E_NOMEM, "step row-plan table");
    for (int w = 0; w < nwg && !rc; ++w)
        g2p_shares(sh + (size_t)w * G2P_NSHARES, c->n_embd, c->n_head, c->ffn_dim, c->vocab_size,
                   m->dtype == G2_F16 ? 8 : 4, w, nwg);
    if (!rc) rc = dev_alloc(m, (void **)&m->step_shares, nsh * sizeof *sh, 0);
    if (!rc) rc = up(m->step_shares, sh, nsh * sizeof *sh);
    free(sh);
    /* A cooperative launch costs ~17 us more than a plain one between
     * back-to-back steps (1.4% of an XL token); the all-to-all kernel checks
     * residency itself, so it is launched plain unless G2_STEP_COOP=1. */
    const char *envc = getenv("G2_STEP_COOP"), *envw = getenv("G2_STEP_TEST_WITHHOLD");
    /* G2_STEP_TEST_WITHHOLD (tests of the residency check): 1 work-group 1
     * never arrives, 2 arrives 0.5 ms late, 3 arrives 2 ms late */
    const int tw = envw && envw[0] >= '1' && envw[0] <= '3' ? envw[0] - '0' : 0;
    m->plain = envc && envc[0] == '1' ? 0 : (tw ? 1 + tw : 1);
    m->xbuf_bytes = (size_t)G2X_TOTAL_WORDS(L, c->n_embd, c->n_head, nwg) * 8;
    m->xval_floats = (size_t)G2V_TOTAL_FLOATS(L, c->n_embd, c->ffn_dim);
    if (!rc) rc = dev_alloc(m, (void **)&m->xbuf, m->xbuf_bytes, 0);
    if (!rc) rc = dev_alloc(m, (void **)&m->xval, m->xval_floats * 4, 0);
    if (!rc) rc = exchange_clear(m);
    if (rc) return rc;
    m->step_wgs = nwg;
    const char *env = getenv("G2_STEP");
    m->step_on = !(env && env[0] == '0');
    const char *tr = getenv("G2_STEP_TRACE");
    if (tr && tr[0]) {
        m->trace_words = (size_t)nwg * G2_TRACE_STRIDE(L);
        rc = dev_alloc(m, (void **)&m->trace, m->trace_words * 8, 0);
        if (!rc) rc = g2i_hip(hipMemsetAsync(m->trace, 0, m->trace_words * 8, g2i_stream()), "trace clear");
    }
    return rc;
}

/* every float of the prompt attention's helper slots G2V_EMPTY (at
 * creation, and after a timed-out wait, which can leave a late partial
 * behind) */
static int help_fill(g2_model *m)
{
    return g2i_hip(hipMemsetD32Async((hipDeviceptr_t)m->pf_help, (int)G2V_EMPTY,
                                     (size_t)G2A_HELP_MAX_SLOTS * G2A_HELP_SLOT_BYTES / 4, g2i_stream()),
                   "attention helper slots fill");
}

/* After a prefill whose prompt attention had helpers: fail if a wait for a
 * helper's partial timed out (the prefill's outputs are then invalid),
 * after refilling the slots and clearing the bit. */
static int prefill_check(g2_model *m)
{
    if (!m->help_ran) return G2_OK;
    m->help_ran = 0;
    int err = 0;
    int rc = g2i_hip(hipMemcpyAsync(&err, m->state + G2S_ERR, sizeof err, hipMemcpyDeviceToHost, g2i_stream()),
                     "prefill check");
    if (!rc) rc = g2i_hip(hipStreamSynchronize(g2i_stream()), "prefill check sync");
    if (rc || !(err & G2_ERR_ATTN_TIMEOUT)) return rc;
    err &= ~G2_ERR_ATTN_TIMEOUT;
    rc = help_fill(m);
    if (!rc) rc = up(m->state + G2S_ERR, &err, sizeof err);
    return rc ? rc : g2i_err(G2_E_HIP, "prompt attention: a wait for a helper's partial timed out; "
                                       "the prefill's outputs are invalid");
}

static int alloc_workspaces(g2_model *m)
{
    const size_t E = (size_t)m->cfg.n_embd, F = (size_t)m->cfg.ffn_dim, T = 3 * E;
    const size_t S = G2_KV_MAX_SEQ, V = (size_t)m->padded_vocab, NH = (size_t)m->cfg.n_head;
    int rc = 0;
#define A(ptr, bytes) if (!rc) rc = dev_alloc(m, (void **)&(ptr), (bytes), 0)
    A(m->hidden, S * E * 4); A(m->ln_out, S * E * 4); A(m->attn, S * E * 4);
    A(m->attn_proj, S * E * 4); A(m->ffn1, S * F * 4); A(m->ffn2, S * E * 4);
    A(m->qkv_new, T * 4); A(m->qkv_full, S * T * 4); A(m->last_hidden, E * 4);
    A(m->logits, V * 4); A(m->ids_dev, S * 4); A(m->partial, 8 * V * 4);
    if (m->path == G2_PATH_FUSED && m->dtype == G2_F16) A(m->pf_part, (size_t)G2_PF_MAXSPLIT * S * E * 4);
    if (m->path == G2_PATH_FUSED && m->dtype == G2_F32) A(m->pf_part, (size_t)G2_SG_PART_FLOATS * 4);
    if (m->path == G2_PATH_FUSED) {
        A(m->pf_help, (size_t)G2A_HELP_MAX_SLOTS * G2A_HELP_SLOT_BYTES);
        if (!rc) rc = help_fill(m);
        /* zeroed once: entries past a prompt are finite (zero or an earlier
         * prompt's), so the masked keys of a block contribute 0 x finite */
        A(m->pf_kv, 4 * S * E * 2);
        if (!rc) rc = g2i_hip(hipMemsetAsync(m->pf_kv, 0, 4 * S * E * 2, g2i_stream()), "kv halves clear");
    }
    A(m->scores, NH * S * 4); A(m->q, S * E * 4);
    A(m->state, G2S_WORDS * 4);
    A(m->att_part, NH * G2_ATTN_MAX_CHUNKS * 66 * 4);
    A(m->am_part, 2 * 8192 * 4);
    for (int l = 0; l < m->cfg.n_layer && !rc; ++l) {
        A(m->L[l].k_cache, E * S * 4);
        A(m->L[l].v_cache, S * E * 4);
        if (!rc) rc = g2i_hip(hipMemsetAsync(m->L[l].k_cache, 0, E * S * 4, g2i_stream()), "kv clear");
        if (!rc) rc = g2i_hip(hipMemsetAsync(m->L[l].v_cache, 0, E * S * 4, g2i_stream()), "kv clear");
    }
#undef A
    if (!rc) rc = g2i_hip(hipMemsetAsync(m->state, 0, G2S_WORDS * 4, g2i_stream()), "state clear");
    if (!rc) rc = step_setup(m);
    if (!rc) rc = g2i_hip(hipStreamSynchronize(g2i_stream()), "workspace sync");
    if (!rc) {
        m->host_logits = malloc(V * sizeof(float));
        if (!m->host_logits) rc = g2i_err(G2_E_NOMEM, "host logits");
    }
    if (!rc) {
        m->events_ok = 1;
        for (int i = 0; i < 3; ++i)
            if (hipEventCreate(&m->ev[i]) != hipSuccess) m->events_ok = 0;
    }
    return rc;
}

static g2_model *model_new(const g2_config *cfg, int dtype, int path)
{
    g2_model *m = calloc(1, sizeof *m);
    if (!m) return NULL;
    m->cfg = *cfg;
    m->cfg.n_ctx = G2_KV_MAX_SEQ;
    m->dtype = dtype;
    m->path = path;
    m->kslice = 4; /* the reference's fallback slice count, main.c:1081 */
    m->padded_vocab = (cfg->vocab_size + 3) & ~3; /* main.c:326 */
    m->L = calloc((size_t)cfg->n_layer, sizeof *m->L);
    if (!m->L) { free(m); return NULL; }
    return m;
}

int g2_model_free(g2_model *m)
{
    if (!m) return G2_OK;
    if (g2i_ready()) hipStreamSynchronize(g2i_stream());
    if (m->graph_state == 1) hipGraphExecDestroy(m->step_exec);
    if (m->events_ok)
        for (int i = 0; i < 3; ++i) hipEventDestroy(m->ev[i]);
    if (m->lm_w && m->lm_w != m->wte) hipFree(m->lm_w);
    void *bufs[] = { m->wte, m->wpe, m->lnf_w, m->lnf_b, m->lm_head, m->hidden, m->ln_out,
                     m->attn, m->attn_proj, m->ffn1, m->ffn2, m->qkv_new, m->qkv_full,
                     m->last_hidden, m->logits, m->partial, m->scores, m->q, m->ids_dev,
                     m->state, m->att_part, m->am_part, m->step_layers, m->xbuf, m->xval, m->lnfold, m->trace, m->pf_part,
                     m->pf_kv, m->step_shares, m->pf_help };
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i)
        if (bufs[i]) hipFree(bufs[i]);
    for (int l = 0; l < m->cfg.n_layer; ++l) {
        g2_layer *y = &m->L[l];
        void *lb[] = { y->ln1_w, y->ln1_b, y->qkv_b, y->proj_b, y->ln2_w, y->ln2_b, y->fc_b,
                       y->fc2_b, y->qkv_w, y->proj_w, y->fc_w, y->fc2_w, y->k_cache, y->v_cache };
        for (size_t i = 0; i < sizeof lb / sizeof lb[0]; ++i)
            if (lb[i]) hipFree(lb[i]);
    }
    free(m->L);
    free(m->host_logits);
    free(m);
    return G2_OK;
}

/* Upload one layer from host Conv1D arrays (12 pointers, order of g2hip.h). */
static int up_layer(g2_model *m, int l, const float *const *w)
{
    const int E = m->cfg.n_embd, F = m->cfg.ffn_dim;
    g2_layer *y = &m->L[l];
    int rc = 0;
    if (!rc) rc = up_vec(m, &y->ln1_w, w[0], (size_t)E);
    if (!rc) rc = up_vec(m, &y->ln1_b, w[1], (size_t)E);
    if (!rc) rc = up_linear(m, &y->qkv_w, w[2], E, 3 * E);
    if (!rc) rc = up_vec(m, &y->qkv_b, w[3], (size_t)3 * E);
    if (!rc) rc = up_linear(m, &y->proj_w, w[4], E, E);
    if (!rc) rc = up_vec(m, &y->proj_b, w[5], (size_t)E);
    if (!rc) rc = up_vec(m, &y->ln2_w, w[6], (size_t)E);
    if (!rc) rc = up_vec(m, &y->ln2_b, w[7], (size_t)E);
    if (!rc) rc = up_linear(m, &y->fc_w, w[8], E, F);
    if (!rc) rc = up_vec(m, &y->fc_b, w[9], (size_t)F);
    if (!rc) rc = up_linear(m, &y->fc2_w, w[10], F, E);
    if (!rc) rc = up_vec(m, &y->fc2_b, w[11], (size_t)E);
    return rc;
}

/* wte/wpe/ln_f and the lm_head: `lm` is a separate [V,E] head or NULL when
 * tied to wte (main.c:1374-1386).  The reference path builds its padded
 * transposed copy; the fused path reads [V,E] rows directly. */
static int up_globals(g2_model *m, const float *wte, const float *wpe, const float *lnf_w,
                      const float *lnf_b, const float *lm)
{
    const int E = m->cfg.n_embd, V = m->cfg.vocab_size;
    int rc = up_typed(m, &m->wte, wte, (size_t)V * E);
    if (!rc) rc = up_typed(m, &m->wpe, wpe, (size_t)G2_KV_MAX_SEQ * E);
    if (!rc) rc = up_vec(m, &m->lnf_w, lnf_w, (size_t)E);
    if (!rc) rc = up_vec(m, &m->lnf_b, lnf_b, (size_t)E);
    if (!rc && m->path == G2_PATH_REFERENCE) rc = up_padded_lm_head(m, lm ? lm : wte);
    if (!rc && m->path == G2_PATH_FUSED) {
        if (lm) rc = up_typed(m, &m->lm_w, lm, (size_t)V * E);
        else m->lm_w = m->wte;
    }
    return rc;
}

int g2_model_from_host(const g2_config *cfg, const float *wte, const float *wpe,
                       const float *lnf_w, const float *lnf_b, const float *const *layers,
                       int weight_dtype, int path, g2_model **out)
{
    if (!out) return g2i_err(G2_E_ARG, "NULL out");
    *out = NULL;
    if (!g2i_ready()) return g2i_err(G2_E_STATE, "g2_init has not been called");
    int rc = check_model_config(cfg, weight_dtype, path);
    if (rc) return rc;
    if (!wte || !wpe || !lnf_w || !lnf_b || !layers) return g2i_err(G2_E_ARG, "NULL weight");
    for (int i = 0; i < cfg->n_layer * 12; ++i)
        if (!layers[i]) return g2i_err(G2_E_ARG, "NULL layer weight %d", i);
    g2_model *m = model_new(cfg, weight_dtype, path);
    if (!m) return g2i_err(G2_E_NOMEM, "model struct");
    rc = up_globals(m, wte, wpe, lnf_w, lnf_b, NULL);
    for (int l = 0; l < cfg->n_layer && !rc; ++l) rc = up_layer(m, l, layers + (size_t)l * 12);
    if (!rc) rc = alloc_workspaces(m);
    if (rc) { g2_model_free(m); return rc; }
    *out = m;
    return G2_OK;
}

int g2_model_synth(const g2_config *cfg, uint64_t seed, int weight_dtype, int path, g2_model **out)
{
    if (!out) return g2i_err(G2_E_ARG, "NULL out");
    *out = NULL;
    if (!g2i_ready()) return g2i_err(G2_E_STATE, "g2_init has not been called");
    int rc = check_model_config(cfg, weight_dtype, path);
    if (rc) return rc;
    const int E = cfg->n_embd, F = cfg->ffn_dim, V = cfg->vocab_size;
    g2_model *m = model_new(cfg, weight_dtype, path);
    if (!m) return g2i_err(G2_E_NOMEM, "model struct");
    const size_t big = (size_t)V * E > (size_t)E * F ? (size_t)V * E : (size_t)E * F;
    float *buf = malloc(big * sizeof(float));
    float *wpe = malloc((size_t)G2_KV_MAX_SEQ * E * sizeof(float));
    float *ones = malloc((size_t)(F > 3 * E ? F : 3 * E) * sizeof(float));
    float *zeros = calloc((size_t)(F > 3 * E ? F : 3 * E), sizeof(float));
    if (!buf || !wpe || !ones || !zeros) rc = g2i_err(G2_E_NOMEM, "synth staging");
    if (!rc) {
        for (int i = 0; i < (F > 3 * E ? F : 3 * E); ++i) ones[i] = 1.0f;
        g2_synth_normal(buf, (size_t)V * E, seed, g2_synth_tensor_id(-1, 1), 0.02f);
        g2_synth_normal(wpe, (size_t)G2_KV_MAX_SEQ * E, seed, g2_synth_tensor_id(-1, 2), 0.02f);
        rc = up_globals(m, buf, wpe, ones, zeros, NULL);
    }
    for (int l = 0; l < cfg->n_layer && !rc; ++l) {
        g2_layer *y = &m->L[l];
        const int dims[4][2] = { { E, 3 * E }, { E, E }, { E, F }, { F, E } };
        void **dst[4] = { &y->qkv_w, &y->proj_w, &y->fc_w, &y->fc2_w };
        for (int w = 0; w < 4 && !rc; ++w) {
            g2_synth_normal(buf, (size_t)dims[w][0] * dims[w][1], seed, g2_synth_tensor_id(l, w), 0.02f);
            rc = up_linear(m, dst[w], buf, dims[w][0], dims[w][1]);
        }
        if (!rc) rc = up_vec(m, &y->ln1_w, ones, (size_t)E);
        if (!rc) rc = up_vec(m, &y->ln1_b, zeros, (size_t)E);
        if (!rc) rc = up_vec(m, &y->qkv_b, zeros, (size_t)3 * E);
        if (!rc) rc = up_vec(m, &y->proj_b, zeros, (size_t)E);
        if (!rc) rc = up_vec(m, &y->ln2_w, ones, (size_t)E);
        if (!rc) rc = up_vec(m, &y->ln2_b, zeros, (size_t)E);
        if (!rc) rc = up_vec(m, &y->fc_b, zeros, (size_t)F);
        if (!rc) rc = up_vec(m, &y->fc2_b, zeros, (size_t)E);
    }
    free(buf); free(wpe); free(ones); free(zeros);
    if (!rc) rc = alloc_workspaces(m);
    if (rc) { g2_model_free(m); return rc; }
    *out = m;
    return G2_OK;
}

/* ------------------------------------------------------ safetensors load */

/* A matrix tensor returned in the Conv1D layout [in,out] whatever the file
 * holds (detect_weight_layout / load_linear_weight, main.c:1234-1300). */
static int read_linear(const g2h_st *st, const char *name, int in, int out, int conv1d, float *dst)
{
    const g2h_tensor *t = g2h_st_find(st, name);
    if (!t) return g2i_err(G2_E_FORMAT, "tensor '%s' not found", name);
    /* shapes compared as int64 (a dimension of 2^32 + n must not pass as n) */
    const int64_t r = t->ndim == 2 ? t->shape[0] : -1, c = t->ndim == 2 ? t->shape[1] : -1;
    const int64_t n = (int64_t)in * out;
    if (conv1d) {
        if (r != in || c != out || t->numel != n)
            return g2i_err(G2_E_FORMAT, "tensor '%s': expected [%d,%d], got [%lld,%lld]", name, in, out,
                           (long long)r, (long long)c);
        return g2h_st_read_f32(st, t, dst, n);
    }
    if (r != out || c != in || t->numel != n)
        return g2i_err(G2_E_FORMAT, "tensor '%s': expected [%d,%d], got [%lld,%lld]", name, out, in,
                       (long long)r, (long long)c);
    float *tmp = malloc((size_t)in * out * sizeof(float));
    if (!tmp) return g2i_err(G2_E_NOMEM, "staging %s", name);
    int rc = g2h_st_read_f32(st, t, tmp, n);
    if (!rc)
        for (int o = 0; o < out; ++o)
            for (int i = 0; i < in; ++i) dst[(size_t)i * out + o] = tmp[(size_t)o * in + i];
    free(tmp);
    return rc;
}

static int read_vec(const g2h_st *st, const char *name, int64_t n, float *dst)
{
    const g2h_tensor *t = g2h_st_find(st, name);
    if (!t) return g2i_err(G2_E_FORMAT, "tensor '%s' not found", name);
    if (t->numel != n) return g2i_err(G2_E_FORMAT, "tensor '%s': %lld elements, expected %lld", name, (long long)t->numel, (long long)n);
    return g2h_st_read_f32(st, t, dst, n);
}

int g2_model_load(const char *dir, int weight_dtype, int path, g2_model **out)
{
    if (!out || !dir) return g2i_err(G2_E_ARG, "NULL argument");
    *out = NULL;
    /* config and file structure are checked before the device is touched, so
     * malformed inputs are reported on a machine without a GPU */
    g2_config cfg;
    int rc = g2_config_load(dir, &cfg);
    if (rc) return rc;
    rc = check_model_config(&cfg, weight_dtype, path);
    if (rc) return rc;
    char p[1100];
    snprintf(p, sizeof p, "%s/model.safetensors", dir);
    g2h_st st;
    if ((rc = g2h_st_open(p, &st))) return rc;
    const int E = cfg.n_embd, F = cfg.ffn_dim, V = cfg.vocab_size;
    /* detect_weight_layout, main.c:1234-1250 */
    const g2h_tensor *probe = g2h_st_find(&st, "h.0.attn.c_attn.weight");
    int conv1d;
    if (!probe || probe->ndim != 2) { g2h_st_close(&st); return g2i_err(G2_E_FORMAT, "cannot find h.0.attn.c_attn.weight"); }
    if (probe->shape[0] == E && probe->shape[1] == 3 * E) conv1d = 1;
    else if (probe->shape[0] == 3 * E && probe->shape[1] == E) conv1d = 0;
    else { g2h_st_close(&st); return g2i_err(G2_E_FORMAT, "unexpected c_attn shape"); }
    for (int i = 0; i < st.n; ++i)
        if (st.t[i].dtype == G2H_ST_OTHER) {
            int code = g2i_err(G2_E_FORMAT, "tensor '%s' dtype=%s; F32, F16 and BF16 are supported",
                               st.t[i].name, st.t[i].dtype_name);
            g2h_st_close(&st);
            return code;
        }
    if (!g2i_ready()) { g2h_st_close(&st); return g2i_err(G2_E_STATE, "g2_init has not been called"); }

    g2_model *m = model_new(&cfg, weight_dtype, path);
    if (!m) { g2h_st_close(&st); return g2i_err(G2_E_NOMEM, "model struct"); }
    const size_t big = (size_t)V * E > (size_t)E * F ? (size_t)V * E : (size_t)E * F;
    float *wte = malloc((size_t)V * E * sizeof(float));
    float *wpe = malloc((size_t)G2_KV_MAX_SEQ * E * sizeof(float));
    float *lnf_w = malloc((size_t)E * sizeof(float)), *lnf_b = malloc((size_t)E * sizeof(float));
    float *buf = malloc(big * sizeof(float) + (size_t)(3 * E + F) * 2 * sizeof(float));
    if (!wte || !wpe || !lnf_w || !lnf_b || !buf) rc = g2i_err(G2_E_NOMEM, "staging");
    if (!rc) rc = read_vec(&st, "wte.weight", (int64_t)V * E, wte);
    if (!rc) {
        memset(wpe, 0, (size_t)G2_KV_MAX_SEQ * E * sizeof(float));
        const g2h_tensor *t = g2h_st_find(&st, "wpe.weight");
        if (!t) rc = g2i_err(G2_E_FORMAT, "tensor 'wpe.weight' not found");
        else if (t->numel % E || t->numel / E > G2_KV_MAX_SEQ) rc = g2i_err(G2_E_FORMAT, "wpe.weight has a bad shape");
        else rc = g2h_st_read_f32(&st, t, wpe, (int64_t)G2_KV_MAX_SEQ * E);
    }
    if (!rc) rc = read_vec(&st, "ln_f.weight", E, lnf_w);
    if (!rc) rc = read_vec(&st, "ln_f.bias", E, lnf_b);
    /* separate lm_head (main.c:1374-1414): [V,E] as is, [E,V] transposed;
     * absent means tied to wte */
    float *lmh = NULL;
    if (!rc) {
        const g2h_tensor *lm = g2h_st_find(&st, "lm_head.weight");
        if (lm) {
            lmh = malloc((size_t)V * E * sizeof(float));
            if (!lmh) rc = g2i_err(G2_E_NOMEM, "lm_head staging");
            else if (lm->ndim == 2 && lm->shape[0] == V && lm->shape[1] == E)
                rc = g2h_st_read_f32(&st, lm, lmh, (int64_t)V * E);
            else if (lm->ndim == 2 && lm->shape[0] == E && lm->shape[1] == V) {
                rc = g2h_st_read_f32(&st, lm, buf, (int64_t)V * E);
                if (!rc)
                    for (int v = 0; v < V; ++v)
                        for (int k = 0; k < E; ++k) lmh[(size_t)v * E + k] = buf[(size_t)k * V + v];
            } else rc = g2i_err(G2_E_FORMAT, "lm_head.weight: unexpected shape");
        }
    }
    if (!rc) rc = up_globals(m, wte, wpe, lnf_w, lnf_b, lmh);
    free(lmh);
    for (int l = 0; l < cfg.n_layer && !rc; ++l) {
        g2_layer *y = &m->L[l];
        char n[128];
        float *v = buf + big; /* small vectors live after the matrix staging */
#define VEC(field, suffix, len)                                                \
        if (!rc) { snprintf(n, sizeof n, "h.%d.%s", l, suffix);               \
                   rc = read_vec(&st, n, (len), v);                           \
                   if (!rc) rc = up_vec(m, &y->field, v, (size_t)(len)); }
#define MAT(field, suffix, in, outd)                                           \
        if (!rc) { snprintf(n, sizeof n, "h.%d.%s", l, suffix);               \
                   rc = read_linear(&st, n, (in), (outd), conv1d, buf);       \
                   if (!rc) rc = up_linear(m, &y->field, buf, (in), (outd)); }
        VEC(ln1_w, "ln_1.weight", E) VEC(ln1_b, "ln_1.bias", E)
        MAT(qkv_w, "attn.c_attn.weight", E, 3 * E) VEC(qkv_b, "attn.c_attn.bias", 3 * E)
        MAT(proj_w, "attn.c_proj.weight", E, E) VEC(proj_b, "attn.c_proj.bias", E)
        VEC(ln2_w, "ln_2.weight", E) VEC(ln2_b, "ln_2.bias", E)
        MAT(fc_w, "mlp.c_fc.weight", E, F) VEC(fc_b, "mlp.c_fc.bias", F)
        MAT(fc2_w, "mlp.c_proj.weight", F, E) VEC(fc2_b, "mlp.c_proj.bias", E)
#undef VEC
#undef MAT
    }
    free(wte); free(wpe); free(lnf_w); free(lnf_b); free(buf);
    g2h_st_close(&st);
    if (!rc) rc = alloc_workspaces(m);
    if (rc) { g2_model_free(m); return rc; }
    *out = m;
    return G2_OK;
}

int g2_model_config(const g2_model *m, g2_config *cfg)
{
    if (!m || !cfg) return g2i_err(G2_E_ARG, "NULL argument");
    *cfg = m->cfg;
    return G2_OK;
}

int g2_model_set_kslice(g2_model *m, int kslice)
{
    if (!m) return g2i_err(G2_E_ARG, "NULL model");
    if (kslice < 1 || kslice > 8) return g2i_err(G2_E_ARG, "kslice %d not in 1..8", kslice);
    m->kslice = kslice;
    return G2_OK;
}

size_t g2_model_weight_bytes(const g2_model *m) { return m ? m->weight_bytes : 0; }

int g2_model_set_step(g2_model *m, int on)
{
    if (!m) return g2i_err(G2_E_ARG, "NULL model");
    if (on && !m->step_wgs)
        return g2i_err(G2_E_ARG, "the persistent step kernel cannot run this model: %s (grid %d)",
                       m->step_why ? m->step_why : "not set up", g2i_step_wgs());
    m->step_on = on ? 1 : 0;
    return G2_OK;
}

int g2_model_uses_step(const g2_model *m)
{
    if (!m) return g2i_err(G2_E_ARG, "NULL model");
    return m->step_on ? 1 : 0;
}

static int step_fid(const g2_model *m);

const char *g2_model_step_kernel(const g2_model *m)
{
    if (!m || !m->step_on) return "";
    return g2i_kernel_name(step_fid(m));
}

int g2_model_uses_graph(const g2_model *m)
{
    if (!m) return g2i_err(G2_E_ARG, "NULL model");
    return m->graph_state == 1 ? 1 : (m->graph_state == -1 ? 0 : -1);
}

/* ------------------------------------------------ reference path (main.c) */

/* launch_matvec_splitk, main.c:1578-1618 with the pinned slice count. */
static int ref_matvec_splitk(g2_model *m, const float *A, const float *B, const float *bias,
                             const float *res, float *C, int N, int K)
{
    const int ks = m->kslice;
    if ((N & 3) || ks <= 1) return g2_matvec(A, B, bias, res, C, N, K, 0);
    int rc = g2_matvec_sk(A, B, m->partial, N, K, ks);
    if (!rc) rc = g2_reduce_partial(m->partial, bias, res, C, N, ks, 0);
    return rc;
}

static int ref_attention(g2_model *m, const float *qkv, int l, int q_base, int T_kv, float *out,
                         int out_base)
{
    const int E = m->cfg.n_embd, NH = m->cfg.n_head, DH = E / NH;
    const float scale = 1.0f / sqrtf((float)DH); /* main.c:1692 */
    int rc = g2_attn_scores_1q(qkv, m->L[l].k_cache, m->scores, q_base, T_kv, E, DH, NH,
                               G2_KV_MAX_SEQ, scale);
    if (!rc) rc = g2_attn_softmax_1q(m->scores, T_kv, NH);
    if (!rc) rc = g2_attn_out_1q(m->scores, m->L[l].v_cache, out, T_kv, E, DH, out_base);
    return rc;
}

static int ref_prefill(g2_model *m, int P)
{
    const int E = m->cfg.n_embd, T = 3 * E, F = m->cfg.ffn_dim;
    int rc = g2_embed((const float *)m->wte, (const float *)m->wpe, m->hidden, E, P, 0, m->ids_dev);
    for (int l = 0; l < m->cfg.n_layer && !rc; ++l) {
        g2_layer *y = &m->L[l];
        rc = g2_layernorm(m->hidden, m->ln_out, y->ln1_w, y->ln1_b, E, P);
        if (!rc) rc = g2_matmul(m->ln_out, y->qkv_w, y->qkv_b, m->qkv_full, P, T, E);
        if (!rc) rc = g2_split_kv(m->qkv_full, y->k_cache, y->v_cache, 0, P, E, G2_KV_MAX_SEQ);
        for (int i = 0; i < P && !rc; ++i)
            rc = ref_attention(m, m->qkv_full, l, i * 3 * E, i + 1, m->attn, i * E);
        if (!rc) rc = g2_matmul(m->attn, y->proj_w, y->proj_b, m->attn_proj, P, E, E);
        if (!rc) rc = g2_add(m->hidden, m->attn_proj, P * E);
        if (!rc) rc = g2_layernorm(m->hidden, m->ln_out, y->ln2_w, y->ln2_b, E, P);
        if (!rc) rc = g2_matmul(m->ln_out, y->fc_w, y->fc_b, m->ffn1, P, F, E);
        if (!rc) rc = g2_gelu(m->ffn1, P * F);
        if (!rc) rc = g2_matmul(m->ffn1, y->fc2_w, y->fc2_b, m->ffn2, P, E, F);
        if (!rc) rc = g2_add(m->hidden, m->ffn2, P * E);
    }
    if (!rc) rc = g2_layernorm(m->hidden, m->ln_out, m->lnf_w, m->lnf_b, E, P);
    if (!rc) rc = g2_copy(m->last_hidden, m->ln_out + (size_t)(P - 1) * E, (size_t)E * sizeof(float));
    if (!rc) rc = g2_matvec(m->last_hidden, m->lm_head, NULL, NULL, m->logits, m->padded_vocab, E, 0);
    return rc;
}

static int ref_decode(g2_model *m, int pos)
{
    const int E = m->cfg.n_embd, T = 3 * E, F = m->cfg.ffn_dim;
    int rc = g2_embed((const float *)m->wte, (const float *)m->wpe, m->hidden, E, 1, pos, m->ids_dev);
    for (int l = 0; l < m->cfg.n_layer && !rc; ++l) {
        g2_layer *y = &m->L[l];
        rc = g2_layernorm(m->hidden, m->ln_out, y->ln1_w, y->ln1_b, E, 1);
        if (!rc) rc = g2_matvec(m->ln_out, y->qkv_w, y->qkv_b, NULL, m->qkv_new, T, E, 0);
        if (!rc) rc = g2_split_kv(m->qkv_new, y->k_cache, y->v_cache, pos, 1, E, G2_KV_MAX_SEQ);
        if (!rc) rc = ref_attention(m, m->qkv_new, l, 0, pos + 1, m->attn, 0);
        if (!rc) rc = ref_matvec_splitk(m, m->attn, y->proj_w, y->proj_b, m->hidden, m->hidden, E, E);
        if (!rc) rc = g2_layernorm(m->hidden, m->ln_out, y->ln2_w, y->ln2_b, E, 1);
        if (!rc) rc = g2_matvec(m->ln_out, y->fc_w, y->fc_b, NULL, m->ffn1, F, E, 1);
        if (!rc) rc = ref_matvec_splitk(m, m->ffn1, y->fc2_w, y->fc2_b, m->hidden, m->hidden, E, F);
    }
    if (!rc) rc = g2_layernorm(m->hidden, m->ln_out, m->lnf_w, m->lnf_b, E, 1);
    if (!rc) rc = g2_matvec(m->ln_out, m->lm_head, NULL, NULL, m->logits, m->padded_vocab, E, 0);
    return rc;
}

/* ------------------------------------------------------------- fused path */


static int launch_rows(g2_model *m, int fid_f32_64, g2_rows_args *a)
{
    return g2i_rows_launch(fid_f32_64, m->dtype == G2_F16, a);
}

/* LayerNorm(ln_f) of row x, logits over the tied wte [V,E], argmax. */
static int fused_lm_head(g2_model *m, const float *x, int advance)
{
    g2_rows_args a;
    memset(&a, 0, sizeof a);
    a.W = m->lm_w; a.x = x; a.ln_g = m->lnf_w; a.ln_b = m->lnf_b; a.y = m->logits;
    a.state = m->state; a.part = m->am_part;
    a.N = m->cfg.vocab_size; a.K = m->cfg.n_embd; a.E = m->cfg.n_embd; a.S = G2_KV_MAX_SEQ;
    int rc = launch_rows(m, G2F_ROWS_LN_ARGMAX_F32_64, &a);
    g2_amerge_args g = { m->am_part, m->state, (int)g2i_rows_grid(a.N, a.K, m->dtype == G2_F16),
                         m->cfg.vocab_size, advance };
    if (!rc) rc = g2i_launch(G2F_ARGMAX_MERGE, 1, 1, 256, &g);
    return rc;
}

/* One decode forward at state[POS] with token state[TOK] (launches only). */
static int fused_step_launches(g2_model *m)
{
    const int E = m->cfg.n_embd, F = m->cfg.ffn_dim, NH = m->cfg.n_head;
    g2_embed_args e = { m->wte, m->wpe, m->hidden, NULL, m->state, E, 1, 0 };
    int rc = g2i_launch(m->dtype == G2_F16 ? G2F_EMBED_F16 : G2F_EMBED_F32, cdivu(E, 256), 1, 256, &e);
    for (int l = 0; l < m->cfg.n_layer && !rc; ++l) {
        g2_layer *y = &m->L[l];
        g2_rows_args a;
        memset(&a, 0, sizeof a);
        a.W = y->qkv_w; a.x = m->hidden; a.ln_g = y->ln1_w; a.ln_b = y->ln1_b; a.bias = y->qkv_b;
        a.q_out = m->q; a.k_cache = y->k_cache; a.v_cache = y->v_cache; a.state = m->state;
        a.N = 3 * E; a.K = E; a.E = E; a.S = G2_KV_MAX_SEQ;
        rc = launch_rows(m, G2F_ROWS_LN_QKV_F32_64, &a);
        if (rc) break;
        g2_attn1q_args t;
        memset(&t, 0, sizeof t);
        t.q = m->q; t.k_cache = y->k_cache; t.v_cache = y->v_cache; t.out = m->attn;
        t.state = m->state; t.part = m->att_part;
        t.T_fixed = 0; t.D = E; t.NH = NH; t.S = G2_KV_MAX_SEQ; t.max_chunks = G2_ATTN_MAX_CHUNKS;
        t.scale = 1.0f / sqrtf(64.0f);
        rc = g2i_attn_launch(&t, G2_ATTN_MAX_CHUNKS); /* chunks past the position exit at once */
        if (rc) break;
        memset(&a, 0, sizeof a);
        a.W = y->proj_w; a.x = m->attn; a.bias = y->proj_b; a.y = m->hidden;
        a.N = E; a.K = E;
        rc = launch_rows(m, G2F_ROWS_RESID_F32_64, &a);
        if (rc) break;
        memset(&a, 0, sizeof a);
        a.W = y->fc_w; a.x = m->hidden; a.ln_g = y->ln2_w; a.ln_b = y->ln2_b; a.bias = y->fc_b;
        a.y = m->ffn1; a.N = F; a.K = E;
        rc = launch_rows(m, G2F_ROWS_LN_GELU_F32_64, &a);
        if (rc) break;
        memset(&a, 0, sizeof a);
        a.W = y->fc2_w; a.x = m->ffn1; a.bias = y->fc2_b; a.y = m->hidden;
        a.N = E; a.K = F;
        rc = launch_rows(m, G2F_ROWS_RESID_F32_64, &a);
    }
    if (!rc) rc = fused_lm_head(m, m->hidden, 1);
    return rc;
}

/* The step kernel of a model: the tail form where every four-unit plan is
 * a tail plan. */
static int step_fid(const g2_model *m)
{
    const g2_config *c = &m->cfg;
    const int VE = m->dtype == G2_F16 ? 8 : 4, f16 = m->dtype == G2_F16;
    const int tail = g2p_step_tail(c->n_embd, c->ffn_dim, VE);
    /* the kernels compiled for a GPT-2 shape (g2p_step_shape), else the
     * ones that read the shape from their arguments */
    const int sh = g2p_step_shape(c->n_embd, c->ffn_dim, c->n_head, c->vocab_size, m->step_wgs);
    if (m->trace) /* the variants with the phase timestamps */
        return f16 ? (tail ? (sh == G2P_SHAPE_XL ? G2F_STEP_F16T_TR : G2F_STEP_F16TN_TR) : G2F_STEP_F16_TR)
                   : (tail ? G2F_STEP_F32T_TR : G2F_STEP_F32_TR);
    if (tail) return f16 ? (sh == G2P_SHAPE_XL ? G2F_STEP_F16T : G2F_STEP_F16TN) : G2F_STEP_F32T;
    if (f16) return sh == 3 ? G2F_STEP_F16_E1280 : G2F_STEP_F16;
    return sh == 1 ? G2F_STEP_F32_E768 : (sh == 2 ? G2F_STEP_F32_E1024 : (sh == 3 ? G2F_STEP_F32_E1280 : G2F_STEP_F32));
}

/* One decode forward at state[POS] as one cooperative launch of the
 * persistent step kernel. */
static int step_launch(g2_model *m)
{
    const g2_config *c = &m->cfg;
    g2_step_args a;
    memset(&a, 0, sizeof a);
    a.layers = m->step_layers; a.wte = m->wte; a.wpe = m->wpe; a.lm_w = m->lm_w;
    a.lnf_w = m->lnf_w; a.logits = m->logits; a.state = m->state;
    a.lm_c1 = m->lnfold + (size_t)c->n_layer * (6 * (size_t)c->n_embd + 2 * (size_t)c->ffn_dim);
    a.lm_c2 = a.lm_c1 + c->vocab_size;
    a.xbuf = m->xbuf;
    a.xval = m->xval;
    a.trace = m->trace;
    a.L = c->n_layer; a.E = c->n_embd; a.F = c->ffn_dim; a.NH = c->n_head; a.V = c->vocab_size;
    a.S = G2_KV_MAX_SEQ;
    a.scale = 1.0f / sqrtf(64.0f);
    m->step_ran = 1;
    a.xlayer = G2X_LAYER_WORDS(c->n_embd, c->n_head);
    a.shares = m->step_shares;
    a.nshares = m->step_wgs;
    const int fid = step_fid(m);
    if (m->plain) {
        a.plain = m->plain;
        return g2i_launch(fid, (unsigned)m->step_wgs, 1, G2_STEP_THREADS, &a);
    }
    return g2i_coop_launch(fid, (unsigned)m->step_wgs, G2_STEP_THREADS, &a);
}

static int fused_step(g2_model *m);

/* After step kernels ran, ngen_target = state[G2S_NGEN] once the run is
 * complete.  A plain launch that found its grid not resident did nothing
 * and made the later launches of the run skip: clear the flag and the
 * exchange area, switch this model to cooperative launches and run the
 * missing steps.  Fail if a step abandoned a hand-off (its outputs are
 * then invalid) and clear the exchange area for the next run. */
static int step_check(g2_model *m, int ngen_target)
{
    if (!m->step_ran) return G2_OK;
    m->step_ran = 0;
    int w[G2S_SEQ + 1];
    int rc = g2i_hip(hipMemcpyAsync(w, m->state, sizeof w, hipMemcpyDeviceToHost, g2i_stream()), "step check");
    if (!rc) rc = g2i_hip(hipStreamSynchronize(g2i_stream()), "step check sync");
    if (rc) return rc;
    const int err = w[G2S_ERR], zero = 0;
    if (err & G2_ERR_STEP_ARGS) {
        rc = up(m->state + G2S_ERR, &zero, sizeof zero);
        return rc ? rc : g2i_err(G2_E_HIP, "decode step kernel: launched with a grid its row-plan table "
                                           "was not built for; no step ran");
    }
    /* a timed-out hand-off (outputs invalid) is reported even if a later
     * launch of the call also found its grid not resident */
    if ((err & G2_ERR_STEP_NOT_RESIDENT) && !(err & G2_ERR_STEP_TIMEOUT)) {
        rc = exchange_clear(m);
        if (!rc) rc = up(m->state + G2S_ERR, &zero, sizeof zero);
        m->plain = 0;
        fprintf(stderr, "g2: decode step kernel: work-groups of a plain launch were not all resident; "
                        "resuming with cooperative launches\n");
        for (int s = w[G2S_NGEN]; s < ngen_target && !rc; ++s) rc = fused_step(m);
        return rc ? rc : step_check(m, ngen_target);
    }
    if (!(err & G2_ERR_STEP_TIMEOUT)) return G2_OK;
    rc = exchange_clear(m);
    if (!rc) rc = up(m->state + G2S_ERR, &zero, sizeof zero);
    if (rc) return rc;
    return g2i_err(G2_E_HIP, "decode step kernel: a hand-off between work-groups timed out; "
                             "the step's outputs are invalid");
}

/* With G2_STEP_TRACE=<file>: write the phase timestamps of the last step
 * (header: work-groups, layers, words per work-group; then the words). */
static int step_trace_dump(g2_model *m)
{
    if (!m->trace) return G2_OK;
    unsigned long long *h = malloc((m->trace_words + 3) * 8);
    if (!h) return g2i_err(G2_E_NOMEM, "trace staging");
    h[0] = (unsigned long long)m->step_wgs;
    h[1] = (unsigned long long)m->cfg.n_layer;
    h[2] = (unsigned long long)G2_TRACE_STRIDE(m->cfg.n_layer);
    int rc = g2i_hip(hipMemcpy(h + 3, m->trace, m->trace_words * 8, hipMemcpyDeviceToHost), "trace read");
    if (!rc) {
        FILE *f = fopen(getenv("G2_STEP_TRACE"), "wb");
        if (f) {
            fwrite(h, 8, m->trace_words + 3, f);
            fclose(f);
        }
    }
    free(h);
    return rc;
}

/* Run one decode step: the persistent step kernel, or the per-operator
 * kernels replaying the captured graph (captured on first use). */
static int fused_step(g2_model *m)
{
    if (m->step_on) return step_launch(m);
    if (m->graph_state == 0) {
        const char *env = getenv("G2_NO_GRAPH");
        if (env && env[0] && env[0] != '0') m->graph_state = -1;
    }
    if (m->graph_state == 0) {
        hipGraph_t g = NULL;
        int ok = hipStreamBeginCapture(g2i_stream(), hipStreamCaptureModeThreadLocal) == hipSuccess;
        if (ok) {
            const int lrc = fused_step_launches(m);
            const hipError_t ce = hipStreamEndCapture(g2i_stream(), &g);
            ok = lrc == 0 && ce == hipSuccess && g != NULL;
            if (ok) ok = hipGraphInstantiate(&m->step_exec, g, NULL, NULL, 0) == hipSuccess;
            if (g) hipGraphDestroy(g);
        }
        (void)hipGetLastError();
        m->graph_state = ok ? 1 : -1; /* -1: launch the kernels directly */
    }
    if (m->graph_state == 1) return g2i_hip(hipGraphLaunch(m->step_exec, g2i_stream()), "graph launch");
    return fused_step_launches(m);
}

static int set_state(g2_model *m, int pos, int tok, int min_new, int ngen)
{
    int h[4];
    h[G2S_POS] = pos; h[G2S_TOK] = tok; h[G2S_MIN_NEW] = min_new; h[G2S_NGEN] = ngen;
    return up(m->state, h, sizeof h);
}

/* g2k_splitk_epi over e's M x N outputs: one thread per 4 columns of a
 * row, or per 4 rows of a column (qkv) */
static int launch_splitk_epi(g2_skepi_args *e)
{
    if (e->ks > G2_SKEPI_MAXKS) return g2i_err(G2_E_LIMIT, "%d split-K slices (at most %d)", e->ks, G2_SKEPI_MAXKS);
    const unsigned n = cdivu((unsigned)(e->M * e->N / 4), 256);
    return g2i_launch(G2F_SPLITK_EPI, n < 2048 ? n : 2048, 1, 256, e);
}

/* C += A . W^T + bias (the residual matmuls of the fp16 prefill: proj, fc2)
 * as split-K slices when a single pass would leave the GPU under-filled.
 * big: the 128x128 kernel, which takes A as its fp16 halves Ah, Al and
 * whose work-groups (one per CU) should all run at once: its slice count
 * is the largest that keeps tiles x slices within the CU count, at most
 * G2_PF_BIGSPLIT and as the slice buffer holds; it splits the K steps into
 * slices that differ by at most one step. */
static int prefill_resid(g2_model *m, const float *A, const uint16_t *Ah, const uint16_t *Al, const void *W,
                         const float *bias, float *C, int P, int N, int K, int big, const float *ln_g,
                         const float *ln_b, uint16_t *hi, uint16_t *lo, int *ln_done)
{
    /* ln_g (with big): the LayerNorm that follows, fused into the slice
     * sum when there are slices (*ln_done = 1); otherwise left to the
     * caller */
    *ln_done = 0;
    const unsigned gx = cdivu(N, 64), gy = cdivu(P, 64);
    int ks = 1;
    for (int k = G2_PF_MAXSPLIT; k > 1; --k)
        if ((K / 64) % k == 0 && gx * gy * (unsigned)k <= 1024) { ks = k; break; }
    if (gx * gy >= 512) ks = 1;
    if (big) /* slices within the pf_part floats */
        ks = g2h_slices(P, N, K, g2i_cus(), G2_PF_BIGSPLIT, (long)G2_PF_MAXSPLIT * G2_KV_MAX_SEQ * m->cfg.n_embd);
    /* the 128x128 kernel: a 1-D grid (g2h_grid) per slice */
    const unsigned bx = big ? g2h_grid(P, N) : gx, by = big ? 1 : gy;
    g2_gemm_args g;
    memset(&g, 0, sizeof g);
    g.A = A; g.B = W; g.bias = bias; g.C = C; g.M = P; g.N = N; g.K = K;
    g.Ah = Ah; g.Al = Al;
    if (ks == 1) return g2i_launch(big ? G2F_HGEMM2_RESID : G2F_HGEMM_RESID, bx, by, big ? 1024 : 256, &g);
    g.part = m->pf_part; g.ksplit = ks;
    int rc = g2i_launch3(big ? G2F_HGEMM2_PARTIAL : G2F_HGEMM_PARTIAL, bx, by, (unsigned)ks, big ? 1024 : 256, &g);
    g2_skred_args r = { m->pf_part, bias, C, P, N, ks, ln_g, ln_b, hi, lo, NULL };
    if (!rc && ln_g && big && N <= G2_SKLN_MAXN && N % 4 == 0 && ks <= G2_SKLN_MAXKS) {
        *ln_done = 1;
        return g2i_launch(G2F_SPLITK_RESID_LN, (unsigned)P, 1, 256, &r);
    }
    if (!rc && ks > G2_SKEPI_MAXKS) rc = g2i_err(G2_E_LIMIT, "%d split-K slices (at most %d)", ks, G2_SKEPI_MAXKS);
    if (!rc) rc = g2i_launch(G2F_SPLITK_RESID, cdivu((unsigned)(P * N), 256) < 2048 ? cdivu((unsigned)(P * N), 256) : 2048,
                             1, 256, &r);
    return rc;
}

/* The fp32-weight prefill GEMM (g2k_sgemm_*, K % 32 == 0) with epilogue
 * epi (G2_SG_GELU, _RESID or _QKV as g2_gemm_args describes them).  A
 * prompt too short to fill the machine with 64x64 tiles gets split-K
 * slices (at most 8, each at least two K steps of 32), summed in order with
 * the bias and the epilogue by g2k_splitk_epi: as many as keep the
 * work-groups within 256, or within 512 for a K of 64 steps or more (fc2).
 * Measured at 64..512 rows and n_embd 768..1280, this picks the best or
 * within 10% of the best of 1..8 slices for every GEMM.  ks slices of at
 * most 64 ceil(M/64) x 64 ceil(N/64) floats each fit G2_SG_PART_FLOATS:
 * ks * tiles <= 512.  With ln_g (a residual epilogue followed by a
 * LayerNorm: proj -> ln_2, fc2 -> the next ln_1) the slice sum is fused
 * with that LayerNorm (g2k_splitk_resid_ln_f32, writing m->ln_out) and
 * *ln_done is set; otherwise the caller runs it. */
static int prefill_sgemm(g2_model *m, int epi, g2_gemm_args *g, const float *ln_g, const float *ln_b, int *ln_done)
{
    *ln_done = 0;
    const unsigned gx = cdivu(g->N, 64), gy = cdivu(g->M, 64), tiles = gx * gy;
    const int nk = g->K / 32;
    const unsigned target = nk >= 64 ? 512 : 256;
    int ks = tiles >= target ? 1 : (int)(target / tiles);
    if (ks > 8) ks = 8;
    if (ks > nk / 2) ks = nk / 2 > 1 ? nk / 2 : 1;
    if ((size_t)ks * g->M * g->N > G2_SG_PART_FLOATS) return g2i_err(G2_E_LIMIT, "split-K slices exceed the buffer");
    if (ks == 1)
        return g2i_launch(epi == G2_SG_GELU ? G2F_SGEMM_GELU : epi == G2_SG_RESID ? G2F_SGEMM_RESID : G2F_SGEMM_QKV,
                          gx, gy, 256, g);
    g->part = m->pf_part;
    int rc = g2i_launch3(G2F_SGEMM_PARTIAL, gx, gy, (unsigned)ks, 256, g);
    if (!rc && epi == G2_SG_RESID && ln_g && g->N <= G2_SKLN_MAXN && g->N % 4 == 0 && ks <= G2_SKLN_F32_MAXKS) {
        g2_skred_args r = { m->pf_part, g->bias, g->C, g->M, g->N, ks, ln_g, ln_b, NULL, NULL, m->ln_out };
        *ln_done = 1;
        return g2i_launch(G2F_SPLITK_RESID_LN_F32, (unsigned)g->M, 1, 256, &r);
    }
    g2_skepi_args e = { m->pf_part, g->bias, g->C, g->q_out, g->k_cache, g->v_cache, g->M, g->N, ks, epi,
                        g->E, g->S, g->pos0, g->kh, g->kl, g->vth, g->vtl, NULL, NULL };
    if (!rc) rc = launch_splitk_epi(&e);
    return rc;
}

/* The 128x128 fp16 GEMM (g2k_hgemm2_*, kernel fid) with its qkv or
 * GELU-split epilogue (epi G2_SG_QKV or G2_SG_GELU_SPLIT).  When its tiles
 * fill at most half the CUs (a 256-row prompt at GPT-2 large width: qkv 60,
 * fc 80 tiles), it runs as K slices (g2k_hgemm2_partial, as many as keep
 * tiles x slices within the CUs, at most G2_PF_BIGSPLIT and as the slice
 * buffer holds), summed in order with the bias and the epilogue by
 * g2k_splitk_epi; GPT-2 XL's 512 rows (qkv 152, fc 200 tiles) run whole. */
static int prefill_big_epi(g2_model *m, int fid, int epi, g2_gemm_args *g)
{
    const unsigned bx = g2h_grid(g->M, g->N);
    const int ks = g2h_slices(g->M, g->N, g->K, g2i_cus(), G2_PF_BIGSPLIT,
                              (long)G2_PF_MAXSPLIT * G2_KV_MAX_SEQ * m->cfg.n_embd); /* pf_part floats */
    if (ks == 1) return g2i_launch(fid, bx, 1, 1024, g);
    g->part = m->pf_part; g->ksplit = ks;
    int rc = g2i_launch3(G2F_HGEMM2_PARTIAL, bx, 1, (unsigned)ks, 1024, g);
    g2_skepi_args e = { m->pf_part, g->bias, g->C, g->q_out, g->k_cache, g->v_cache, g->M, g->N, ks, epi,
                        g->E, g->S, g->pos0, g->kh, g->kl, g->vth, g->vtl, g->Ch, g->Cl };
    if (!rc) rc = launch_splitk_epi(&e);
    return rc;
}

static int fused_prefill(g2_model *m, int P)
{
    const int E = m->cfg.n_embd, F = m->cfg.ffn_dim, NH = m->cfg.n_head;
    const int f16 = m->dtype == G2_F16;
    /* fp16 weights: the split-activation fp16 MFMA GEMM (n_embd and ffn are
     * multiples of 64 on the fused path); G2_PREFILL_F32MFMA=1 keeps the
     * fp32-MFMA GEMM for comparison */
    const char *pe = getenv("G2_PREFILL_F32MFMA");
    const int h = f16 && E % 64 == 0 && F % 64 == 0 && !(pe && pe[0] == '1');
    /* prompts of more than 64 rows: the 128x128 tiles (G2_PREFILL_GEMM64=1
     * keeps the 64x64 ones, whose results are identical) */
    const char *p64 = getenv("G2_PREFILL_GEMM64");
    const int big = h && P > 64 && !(p64 && p64[0] == '1');
    /* fp32 weights: the 64x64 fp32-MFMA GEMM with K steps of 32 streamed
     * through LDS, split-K for short prompts */
    const int sg = !f16 && E % 32 == 0 && F % 32 == 0;
    const int f_qkv = big ? G2F_HGEMM2_QKV : h ? G2F_HGEMM_QKV : (f16 ? G2F_GEMM_NK_F16_QKV : G2F_GEMM_NK_F32_QKV);
    const int f_resid = h ? G2F_HGEMM_RESID : (f16 ? G2F_GEMM_NK_F16_RESID : G2F_GEMM_NK_F32_RESID);
    const int f_gelu = big ? G2F_HGEMM2_GELU : h ? G2F_HGEMM_GELU : (f16 ? G2F_GEMM_NK_F16_GELU : G2F_GEMM_NK_F32_GELU);
    /* the 128x128 GEMMs take their activations as fp16 halves, written by
     * the producers into the fp32 buffers' memory: hi in the first half, lo
     * in the second, each [G2_KV_MAX_SEQ rows][width] */
    const size_t cap = G2_KV_MAX_SEQ;
    uint16_t *ln_h = (uint16_t *)m->ln_out, *ln_l = ln_h + cap * E;
    uint16_t *at_h = (uint16_t *)m->attn, *at_l = at_h + cap * E;
    uint16_t *ff_h = (uint16_t *)m->ffn1, *ff_l = ff_h + cap * F;
    /* the layer's K and V as fp16 halves, written by the qkv epilogue for
     * the prompt attention: kh, kl [cap][E], vth, vtl [E][cap] */
    uint16_t *kv_kh = m->pf_kv, *kv_kl = kv_kh + cap * E, *kv_vh = kv_kl + cap * E, *kv_vl = kv_vh + cap * E;
    g2_embed_args e = { m->wte, m->wpe, m->hidden, m->ids_dev, NULL, E, P, 0 };
    int rc = g2i_launch(f16 ? G2F_EMBED_F16 : G2F_EMBED_F32, cdivu(E, 256), (unsigned)P, 256, &e);
    int ln1_done = 0; /* the previous layer's fc2 sum already wrote this layer's ln_1 */
    int ln_unused = 0;
    const char *ea = getenv("G2_PREFILL_ATTN32");
    const int attn32 = ea && ea[0] == '1'; /* attention on the fp32 matrix cores (reference point) */
    const char *eh = getenv("G2_PREFILL_ATTN_HELP");
    const int help_off = eh && eh[0] == '0';
    for (int l = 0; l < m->cfg.n_layer && !rc; ++l) {
        g2_layer *y = &m->L[l];
        g2_lnsplit_args ls = { m->hidden, ln_h, ln_l, y->ln1_w, y->ln1_b, E, P };
        if (!ln1_done)
            rc = big ? g2i_launch(G2F_LAYERNORM_SPLIT, (unsigned)P, 1, 256, &ls)
                     : g2_layernorm(m->hidden, m->ln_out, y->ln1_w, y->ln1_b, E, P);
        g2_gemm_args g;
        memset(&g, 0, sizeof g);
        g.A = m->ln_out; g.Ah = ln_h; g.Al = ln_l; g.B = y->qkv_w; g.bias = y->qkv_b; g.q_out = m->q;
        g.k_cache = y->k_cache; g.v_cache = y->v_cache; g.M = P; g.N = 3 * E; g.K = E;
        g.E = E; g.S = G2_KV_MAX_SEQ; g.pos0 = 0;
        g.kh = kv_kh; g.kl = kv_kl; g.vth = kv_vh; g.vtl = kv_vl;
        if (!rc) rc = big ? prefill_big_epi(m, f_qkv, G2_SG_QKV, &g)
                      : sg  ? prefill_sgemm(m, G2_SG_QKV, &g, NULL, NULL, &ln_unused)
                            : g2i_launch(f_qkv, cdivu(3 * E, 64), cdivu(P, 64), 256, &g);
        g2_attnp_args t = { m->q, y->k_cache, y->v_cache, m->attn, P, E, NH, G2_KV_MAX_SEQ, 1.0f / sqrtf(64.0f),
                            big ? at_h : NULL, big ? at_l : NULL, kv_kh, kv_kl, kv_vh, kv_vl, NULL, NULL };
        /* the grid's idle work-groups help the longest query blocks
         * (g2a_help_plan; G2_PREFILL_ATTN_HELP=0 turns them off), when the
         * whole grid is resident at once (one work-group per CU), so a
         * block's helper is never dispatched behind the block's wait */
        if (!attn32 && !help_off && g2a_help_plan(P, NH).on && g2a_grid(P, NH) <= (unsigned)g2i_cus()) {
            t.help = m->pf_help;
            t.err = m->state + G2S_ERR;
            m->help_ran = 1;
        }
        /* 1-D grid: 8 XCDs x ceil(NH / 8) heads x query blocks (attnp_block) */
        if (!rc) rc = g2i_launch(attn32 ? G2F_ATTN_PREFILL_MFMA : G2F_ATTN_PREFILL_H16, 8 * cdivu(NH, 8) * cdivu(P, 64), 1,
                                 512, &t);
        memset(&g, 0, sizeof g);
        g.A = m->attn; g.B = y->proj_w; g.bias = y->proj_b; g.C = m->hidden; g.M = P; g.N = E; g.K = E;
        int ln2_done = 0;
        if (!rc) rc = h ? prefill_resid(m, m->attn, at_h, at_l, y->proj_w, y->proj_b, m->hidden, P, E, E, big,
                                        y->ln2_w, y->ln2_b, ln_h, ln_l, &ln2_done)
                      : sg ? prefill_sgemm(m, G2_SG_RESID, &g, y->ln2_w, y->ln2_b, &ln2_done)
                           : g2i_launch(f_resid, cdivu(E, 64), cdivu(P, 64), 256, &g);
        g2_lnsplit_args ls2 = { m->hidden, ln_h, ln_l, y->ln2_w, y->ln2_b, E, P };
        if (!rc && !ln2_done)
            rc = big ? g2i_launch(G2F_LAYERNORM_SPLIT, (unsigned)P, 1, 256, &ls2)
                     : g2_layernorm(m->hidden, m->ln_out, y->ln2_w, y->ln2_b, E, P);
        memset(&g, 0, sizeof g);
        g.A = m->ln_out; g.B = y->fc_w; g.bias = y->fc_b; g.C = m->ffn1; g.M = P; g.N = F; g.K = E;
        g.Ah = ln_h; g.Al = ln_l; g.Ch = ff_h; g.Cl = ff_l;
        if (!rc) rc = big ? prefill_big_epi(m, f_gelu, G2_SG_GELU_SPLIT, &g)
                      : sg  ? prefill_sgemm(m, G2_SG_GELU, &g, NULL, NULL, &ln_unused)
                            : g2i_launch(f_gelu, cdivu(F, 64), cdivu(P, 64), 256, &g);
        memset(&g, 0, sizeof g);
        g.A = m->ffn1; g.B = y->fc2_w; g.bias = y->fc2_b; g.C = m->hidden; g.M = P; g.N = E; g.K = F;
        const g2_layer *yn = l + 1 < m->cfg.n_layer ? &m->L[l + 1] : NULL;
        ln1_done = 0;
        if (!rc) rc = h ? prefill_resid(m, m->ffn1, ff_h, ff_l, y->fc2_w, y->fc2_b, m->hidden, P, E, F, big,
                                        yn ? yn->ln1_w : NULL, yn ? yn->ln1_b : NULL, ln_h, ln_l, &ln1_done)
                      : sg ? prefill_sgemm(m, G2_SG_RESID, &g, yn ? yn->ln1_w : NULL, yn ? yn->ln1_b : NULL,
                                           &ln1_done)
                           : g2i_launch(f_resid, cdivu(E, 64), cdivu(P, 64), 256, &g);
    }
    if (!rc) rc = fused_lm_head(m, m->hidden + (size_t)(P - 1) * E, 1);
    return rc;
}

/* --------------------------------------------------------------- public */

int g2_prefill(g2_model *m, const int *ids, int n)
{
    if (!m || !ids) return g2i_err(G2_E_ARG, "NULL argument");
    if (n < 1 || n > G2_KV_MAX_SEQ - 1) return g2i_err(G2_E_LIMIT, "prompt of %d ids (1..1023)", n);
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= m->cfg.vocab_size) return g2i_err(G2_E_ARG, "token id %d out of range", ids[i]);
    int rc = up(m->ids_dev, ids, (size_t)n * sizeof(int)); /* blocking, main.c:1745 */
    if (rc) return rc;
    if (m->path == G2_PATH_REFERENCE) return ref_prefill(m, n);
    rc = set_state(m, n - 1, ids[n - 1], 0, 0);
    if (!rc) rc = fused_prefill(m, n);
    if (!rc) rc = prefill_check(m);
    return rc;
}

int g2_decode(g2_model *m, int token, int pos)
{
    if (!m) return g2i_err(G2_E_ARG, "NULL model");
    if (pos < 0 || pos >= G2_KV_MAX_SEQ) return g2i_err(G2_E_LIMIT, "position %d outside 0..1023", pos);
    if (token < 0 || token >= m->cfg.vocab_size) return g2i_err(G2_E_ARG, "token id %d out of range", token);
    if (m->path == G2_PATH_REFERENCE) {
        int rc = up(m->ids_dev, &token, sizeof(int)); /* blocking, main.c:1798 */
        return rc ? rc : ref_decode(m, pos);
    }
    int rc = set_state(m, pos, token, 0, 0);
    if (!rc) rc = fused_step(m);
    return rc ? rc : step_check(m, 1);
}

int g2_read_logits(g2_model *m, float *host, int n)
{
    if (!m || !host) return g2i_err(G2_E_ARG, "NULL argument");
    if (n < 0 || n > m->cfg.vocab_size) return g2i_err(G2_E_ARG, "n %d outside 0..vocab", n);
    int rc = g2i_hip(hipMemcpyAsync(host, m->logits, (size_t)n * sizeof(float),
                                    hipMemcpyDeviceToHost, g2i_stream()), "read logits");
    return rc ? rc : g2i_hip(hipStreamSynchronize(g2i_stream()), "read logits sync");
}

int g2_read_kv(g2_model *m, int layer, float *k_host, float *v_host)
{
    if (!m) return g2i_err(G2_E_ARG, "NULL model");
    if (layer < 0 || layer >= m->cfg.n_layer) return g2i_err(G2_E_ARG, "layer %d out of range", layer);
    const size_t bytes = (size_t)m->cfg.n_embd * G2_KV_MAX_SEQ * sizeof(float);
    int rc = 0;
    if (k_host) rc = g2i_hip(hipMemcpyAsync(k_host, m->L[layer].k_cache, bytes, hipMemcpyDeviceToHost, g2i_stream()), "read k");
    if (!rc && v_host) rc = g2i_hip(hipMemcpyAsync(v_host, m->L[layer].v_cache, bytes, hipMemcpyDeviceToHost, g2i_stream()), "read v");
    return rc ? rc : g2i_hip(hipStreamSynchronize(g2i_stream()), "read kv sync");
}

/* sample_next_token, greedy branch (main.c:1872-1904). */
int g2_sample_greedy(g2_model *m, const int *ctx, int n_ctx, int forbid_eos, float rep_penalty)
{
    if (!m) return g2i_err(G2_E_ARG, "NULL model");
    const int V = m->cfg.vocab_size;
    float *lg = m->host_logits;
    int rc = g2_read_logits(m, lg, V);
    if (rc) return rc;
    if (forbid_eos && G2_EOS_TOKEN < V) lg[G2_EOS_TOKEN] = -1e30f;
    if (rep_penalty > 1.0f && ctx) {
        for (int i = 0; i < n_ctx; ++i) {
            const int tk = ctx[i];
            if (tk < 0 || tk >= V) continue;
            int dup = 0;
            for (int j = 0; j < i; ++j)
                if (ctx[j] == tk) { dup = 1; break; }
            if (dup) continue;
            if (lg[tk] > 0.0f) lg[tk] /= rep_penalty;
            else lg[tk] *= rep_penalty;
        }
    }
    int best = 0;
    float bv = lg[0];
    for (int i = 1; i < V; ++i)
        if (lg[i] > bv) { bv = lg[i]; best = i; }
    return best;
}

static double ev_ms(g2_model *m, int a, int b)
{
    float ms = 0.f;
    if (!m->events_ok || hipEventElapsedTime(&ms, m->ev[a], m->ev[b]) != hipSuccess) return -1.0;
    return (double)ms;
}

int g2_generate(g2_model *m, const int *prompt, int n_prompt, int max_new, int min_new,
                int *out_ids, double *timing)
{
    if (!m || !prompt || !out_ids) return g2i_err(G2_E_ARG, "NULL argument");
    if (n_prompt < 1 || n_prompt > G2_KV_MAX_SEQ - 1) return g2i_err(G2_E_LIMIT, "prompt of %d ids (1..1023)", n_prompt);
    if (max_new < 1) return g2i_err(G2_E_ARG, "max_new must be >= 1");
    /* generated = 1 + decode steps, decode steps end at seq_len 1024 (main.c:2126) */
    const int n_dec_max = G2_KV_MAX_SEQ - 1 - n_prompt;
    const int n_dec = max_new - 1 < n_dec_max ? max_new - 1 : n_dec_max;
    int rc;
    if (m->path == G2_PATH_REFERENCE) {
        int *ctx = malloc((size_t)(G2_KV_MAX_SEQ + 1) * sizeof(int));
        if (!ctx) return g2i_err(G2_E_NOMEM, "context");
        memcpy(ctx, prompt, (size_t)n_prompt * sizeof(int));
        int seq = n_prompt, gen = 0;
        if (m->events_ok) hipEventRecord(m->ev[0], g2i_stream());
        rc = g2_prefill(m, prompt, n_prompt);
        int next = rc ? rc : g2_sample_greedy(m, ctx, seq, 0 < min_new, 1.0f);
        if (m->events_ok) hipEventRecord(m->ev[1], g2i_stream());
        if (next < 0) { free(ctx); return next; }
        ctx[seq++] = next;
        out_ids[gen++] = next;
        while (gen < max_new && next != G2_EOS_TOKEN && seq < G2_KV_MAX_SEQ) {
            rc = g2_decode(m, ctx[seq - 1], seq - 1);
            next = rc ? rc : g2_sample_greedy(m, ctx, seq, gen < min_new, 1.0f);
            if (next < 0) { free(ctx); return next; }
            ctx[seq++] = next;
            out_ids[gen++] = next;
        }
        if (m->events_ok) {
            hipEventRecord(m->ev[2], g2i_stream());
            hipEventSynchronize(m->ev[2]);
        }
        if (timing) { timing[0] = ev_ms(m, 0, 1); timing[1] = ev_ms(m, 1, 2); }
        free(ctx);
        return gen;
    }
    for (int i = 0; i < n_prompt; ++i)
        if (prompt[i] < 0 || prompt[i] >= m->cfg.vocab_size) return g2i_err(G2_E_ARG, "token id %d out of range", prompt[i]);
    rc = up(m->ids_dev, prompt, (size_t)n_prompt * sizeof(int));
    if (!rc) rc = set_state(m, n_prompt - 1, prompt[n_prompt - 1], min_new, 0);
    if (rc) return rc;
    if (m->events_ok) hipEventRecord(m->ev[0], g2i_stream());
    rc = fused_prefill(m, n_prompt);
    if (m->events_ok) hipEventRecord(m->ev[1], g2i_stream());
    for (int s = 0; s < n_dec && !rc; ++s) rc = fused_step(m);
    if (m->events_ok) hipEventRecord(m->ev[2], g2i_stream());
    if (!rc) rc = prefill_check(m);
    if (!rc) rc = step_check(m, 1 + n_dec); /* the prefill's pick + n_dec steps */
    if (rc) return rc;
    int *st = malloc((size_t)G2S_WORDS * sizeof(int));
    if (!st) return g2i_err(G2_E_NOMEM, "state readback");
    rc = g2i_hip(hipMemcpyAsync(st, m->state, (size_t)G2S_WORDS * sizeof(int), hipMemcpyDeviceToHost,
                                g2i_stream()), "state readback");
    if (!rc) rc = g2i_hip(hipStreamSynchronize(g2i_stream()), "state sync");
    int gen = 0;
    if (!rc) {
        const int total = 1 + n_dec;
        for (int i = 0; i < total; ++i) {
            out_ids[gen++] = st[G2S_IDS + i];
            if (st[G2S_IDS + i] == G2_EOS_TOKEN) break; /* main.c:2135: stop at EOS */
        }
        if (timing) { timing[0] = ev_ms(m, 0, 1); timing[1] = ev_ms(m, 1, 2); }
    }
    free(st);
    return rc ? rc : gen;
}

int g2_decode_run(g2_model *m, int token, int start_pos, int n_steps, int forbid_eos,
                  int *out_ids, double *elapsed_ms)
{
    if (!m) return g2i_err(G2_E_ARG, "NULL model");
    if (m->path != G2_PATH_FUSED) return g2i_err(G2_E_ARG, "g2_decode_run needs the fused path");
    if (n_steps < 1 || start_pos < 0 || start_pos + n_steps > G2_KV_MAX_SEQ)
        return g2i_err(G2_E_LIMIT, "steps %d from position %d exceed 1024", n_steps, start_pos);
    if (token < 0 || token >= m->cfg.vocab_size) return g2i_err(G2_E_ARG, "token id %d out of range", token);
    int rc = set_state(m, start_pos, token, forbid_eos ? n_steps + 1 : 0, 0);
    if (rc) return rc;
    if (m->events_ok) hipEventRecord(m->ev[0], g2i_stream());
    for (int s = 0; s < n_steps && !rc; ++s) rc = fused_step(m);
    if (m->events_ok) hipEventRecord(m->ev[1], g2i_stream());
    if (!rc) rc = g2i_hip(hipStreamSynchronize(g2i_stream()), "decode run sync");
    if (!rc) rc = step_check(m, n_steps);
    if (!rc) rc = step_trace_dump(m);
    if (rc) return rc;
    if (elapsed_ms) *elapsed_ms = ev_ms(m, 0, 1);
    if (out_ids) {
        rc = g2i_hip(hipMemcpyAsync(out_ids, m->state + G2S_IDS, (size_t)n_steps * sizeof(int),
                                    hipMemcpyDeviceToHost, g2i_stream()), "ids readback");
        if (!rc) rc = g2i_hip(hipStreamSynchronize(g2i_stream()), "ids sync");
    }
    return rc;
}
