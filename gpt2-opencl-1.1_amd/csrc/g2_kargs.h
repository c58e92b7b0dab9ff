/*
 * g2_kargs.h -- kernel argument blocks shared by the C99 host (g2_shim.c,
 * g2_model.c) and the gfx950 device code (g2_kernels.hip).
 *
 * Every kernel takes exactly one of these structs by value, so a host launch
 * is hipModuleLaunchKernel(f, grid, block, 0, stream, {&args}, NULL).  Only
 * fixed-width scalars and pointers appear, so the layout is the same under
 * gcc (x86-64) and clang (amdgcn).
 */
#ifndef G2_KARGS_H
#define G2_KARGS_H

#include <stdint.h>

#define G2_KV_MAX_SEQ 1024   /* KV cache length and scores row stride (math.cl:18) */
#define G2_EOS_ID 50256      /* end-of-text id (main.c:58) */

/* Device-resident decode state (int32 words), read by the fused kernels so a
 * captured graph can be replayed token after token without host writes. */
enum {
    G2S_POS = 0,      /* position processed by the next decode forward       */
    G2S_TOK = 1,      /* token id at that position                           */
    G2S_MIN_NEW = 2,  /* EOS is masked while G2S_NGEN < G2S_MIN_NEW          */
    G2S_NGEN = 3,     /* tokens selected so far in this generation           */
    G2S_ERR = 4,      /* sticky error bits set by kernels (bounds clamps)    */
    G2S_SEQ = 5,      /* decode steps run by the persistent step kernel      */
    G2S_IDS = 16,     /* ids selected, G2S_IDS + k for the k-th selection    */
    G2S_WORDS = 16 + 1024
};

/* G2S_ERR bits */
#define G2_ERR_STEP_TIMEOUT 4 /* a step-kernel exchange wait ran out of time */
/* a plain (not cooperative) launch of the step kernel found its work-groups
 * not all resident and did nothing; later launches skip until it is cleared */
#define G2_ERR_STEP_NOT_RESIDENT 8
/* a step-kernel launch whose grid differs from its row-plan table did nothing */
#define G2_ERR_STEP_ARGS 16
/* a prompt-attention work-group waited too long for its helper's partial;
 * the prefill's outputs and the helper slots are invalid */
#define G2_ERR_ATTN_TIMEOUT 32

/* GEMM: C[M,N] = A[M,K] * op(B) with an epilogue.
 * B layout G2_BKN: [K,N] row-major (the reference's device layout);
 * B layout G2_BNK: [N,K] row-major (packed, output-major).
 * Epilogues: store (C = acc + bias), gelu (C = gelu(acc + bias)),
 * resid (C = C + (acc + bias), in place), qkv (columns < E to q_out[M,E],
 * E..2E-1 to k_cache[(n-E)*S + pos0+m], 2E..3E-1 to v_cache[(pos0+m)*E + n-2E]),
 * partial (the fp16 split-K GEMM: K slice z of ksplit equal slices to
 * part[z*M*N + m*N + n], no bias; g2k_splitk_resid adds the slices in
 * order, the bias and the residual). */
typedef struct {
    const float *A;
    const void *B;
    const float *bias;
    float *C;
    float *q_out;
    float *k_cache;
    float *v_cache;
    int M, N, K;
    int E, S, pos0;
    float *part;
    int ksplit;
    /* qkv epilogue, when non-NULL: the key columns also as fp16 halves to
     * kh, kl [S rows (positions)][E], the value columns as fp16 halves to
     * vth, vtl [E][S] (transposed): the staged operands of the prompt
     * attention (g2_attnp_args) */
    uint16_t *kh, *kl, *vth, *vtl;
    /* the 128x128 fp16 GEMM (g2k_hgemm2_*): A given as its fp16 halves
     * Ah = fp16(a), Al = fp16(a - Ah), [M,K] each (A unused); epilogue
     * gelu_split writes gelu(acc + bias) as halves to Ch, Cl [M,N] */
    const uint16_t *Ah, *Al;
    uint16_t *Ch, *Cl;
} g2_gemm_args;

/* C[m,n] = C[m,n] + ((sum over z < ks in order of part[z*M*N + m*N + n]) +
 * bias[n]) for m < M, n < N.  g2k_splitk_resid_ln (grid M, N <=
 * G2_SKLN_MAXN) then writes LayerNorm(C[m,:]; ln_g, ln_b) as fp16 halves
 * to hi, lo [M,N] (see g2_lnsplit_args); g2k_splitk_resid_ln_f32 writes it
 * as fp32 to ln_out [M,N] (the operand of the fp32-weight GEMM). */
typedef struct {
    const float *part;
    const float *bias;
    float *C;
    int M, N, ks;
    const float *ln_g, *ln_b;
    uint16_t *hi, *lo;
    float *ln_out;
} g2_skred_args;
#define G2_SKLN_MAXN 2048
#define G2_SKLN_MAXKS 8     /* slices g2k_splitk_resid_ln reads (ks <= this) */
#define G2_SKLN_F32_MAXKS 8 /* slices g2k_splitk_resid_ln_f32 reads */

/* The split-K epilogue of the prefill GEMMs (g2k_splitk_epi): v[m,n] =
 * (sum over z < ks in order of part[z][m][n]) + bias[n], then epi 1 gelu
 * (C = gelu(v)), 2 resid (C = C + v), 3 qkv (q_out / k_cache / v_cache and
 * the K/V halves as g2_gemm_args' qkv epilogue), 5 gelu as fp16 halves
 * (Ch, Cl = the halves of gelu(v), the operand of the next 128x128 GEMM).
 * N % 4 == 0, ks <= G2_SKEPI_MAXKS. */
typedef struct {
    const float *part;
    const float *bias;
    float *C;
    float *q_out, *k_cache, *v_cache;
    int M, N, ks, epi;
    int E, S, pos0;
    uint16_t *kh, *kl, *vth, *vtl; /* as in g2_gemm_args */
    uint16_t *Ch, *Cl;
} g2_skepi_args;
#define G2_SKEPI_MAXKS 8 /* slices g2k_splitk_epi reads */

/* Reference-layout matvec, first pass: partial[split*N + n] = sum over the
 * split's contiguous k-range of A[k] B[k*N + n]; grid (column tiles, splits). */
typedef struct {
    const float *A;
    const void *B;
    float *partial;
    int N, K, rows_per_split;
} g2_mvkn_args;

/* Split-K partials with the reference's strided slices (math.cl:229-246). */
typedef struct {
    const float *A;
    const void *B;
    float *partial;
    int N, K, kslice;
} g2_mvsk_args;

/* reduce_partial (math.cl:249-280), also the second pass of g2_matvec. */
typedef struct {
    const float *partial;
    const float *bias;
    const float *residual;
    float *C;
    int N, nslice, apply_gelu;
} g2_reduce_args;

typedef struct {
    const float *x;
    float *out;
    const float *gamma;
    const float *beta;
    int E, rows;
} g2_ln_args;

/* LayerNorm whose rows are written as fp16 halves hi = fp16(y), lo =
 * fp16(y - hi), [rows,E] each (the A operand of g2k_hgemm2_*). */
typedef struct {
    const float *x;
    uint16_t *hi, *lo;
    const float *gamma;
    const float *beta;
    int E, rows;
} g2_lnsplit_args;

typedef struct {
    float *a;
    const float *b;
    int n;
} g2_ew_args;

/* Embedding; wte/wpe are f32 or f16 by kernel variant.  If state != NULL the
 * single row uses state[G2S_TOK] at state[G2S_POS]; else ids[i] at start_pos+i. */
typedef struct {
    const void *wte;
    const void *wpe;
    float *out;
    const int *ids;
    const int *state;
    int E, seq_len, start_pos;
} g2_embed_args;

typedef struct {
    const float *qkv;
    float *k_cache;
    float *v_cache;
    int start_pos, T, D, S;
} g2_splitkv_args;

typedef struct {
    const float *qkv;
    const float *k_cache;
    float *scores;
    int q_base, T, D, DH, NH, S;
    float scale;
} g2_scores_args;

typedef struct {
    float *scores;
    int T, NH;
} g2_softmax_args;

typedef struct {
    const float *scores;
    const float *v_cache;
    float *out;
    int T, D, DH, out_base;
} g2_attnout_args;

/* Single-query attention, head dim 64, split over 64-position key chunks
 * (partials kernel) and merged by a second kernel.  T = T_fixed if > 0,
 * else state[G2S_POS] + 1.  part: [NH][max_chunks][2 + 64] floats. */
typedef struct {
    const float *q;
    const float *k_cache;
    const float *v_cache;
    float *out;
    const int *state;
    float *part;
    int T_fixed, D, NH, S, max_chunks;
    float scale;
} g2_attn1q_args;

/* Fused row-major matvec over packed weights W[N,K] (f32 or f16):
 * acc[n] = sum_k W[n*K + k] * xin[k], where xin is x, or LayerNorm(x) with
 * ln_g/ln_b when the LN variant is used.  Epilogue by kernel variant:
 * store y = acc + bias; gelu; resid y = y + (acc + bias);
 * qkv (q_out / k_cache / v_cache at state[G2S_POS]);
 * argmax: y = acc (logits) and each work-group's first-max (value, index)
 * to part[2b], with EOS masked while state[G2S_NGEN] < state[G2S_MIN_NEW]. */
typedef struct {
    const void *W;
    const float *x;
    const float *ln_g;
    const float *ln_b;
    const float *bias;
    float *y;
    float *q_out;
    float *k_cache;
    float *v_cache;
    int *state;
    float *part;
    int N, K, E, S;
} g2_rows_args;

/* Greedy pick over the lm_head work-groups' (value, index) partials. */
typedef struct {
    const float *part;
    int *state;
    int n_parts, N, advance;
} g2_amerge_args;

/* Persistent decode step (one cooperative launch per token, 512 threads per
 * work-group, one work-group per CU).  Per-layer weights come from a device
 * array of g2_step_layer.  Work-groups hand vectors to each other through
 * two exchange areas: `xbuf` of 64-bit words (value in the low half, the
 * step's tag in the high half), laid out by the G2X_* offsets below and
 * sized with G2X_TOTAL_WORDS, for q/k/v, the attention partials, the
 * argmax and the arrival words; and `xval` of plain floats, laid out by the
 * G2V_* offsets and sized with G2V_TOTAL_FLOATS, for the four vectors every
 * work-group reads whole (O, X1, H, X2). */
typedef struct {
    const float *ln1_w, *proj_b, *ln2_w, *fc2_b;
    const void *qkv_w, *proj_w, *fc_w, *fc2_w;
    float *k_cache, *v_cache;
    /* the LayerNorm folded into the matrix that follows it (g2k_ln_fold):
     * c1[r] = W[r,:] . gamma, c2[r] = W[r,:] . beta + bias[r] for qkv (ln_1,
     * qkv bias) and fc (ln_2, fc bias); the gains ln1_w, ln2_w scale x */
    const float *qkv_c1, *qkv_c2, *fc_c1, *fc_c2;
} g2_step_layer;

typedef struct {
    const g2_step_layer *layers;
    const void *wte;
    const void *wpe;
    const void *lm_w;
    const float *lnf_w;
    const float *lm_c1, *lm_c2; /* ln_f folded into the lm_head (no bias) */
    float *logits;
    int *state;
    unsigned long long *xbuf;
    float *xval;
    /* optional phase timestamps (100 MHz clock): work-group w writes
     * trace[w * G2_TRACE_STRIDE(L) + 24*l + k] for phase boundary k of layer
     * l, and 24*L + k for the lm_head and the pick; NULL: off */
    unsigned long long *trace;
    int L, E, F, NH, V, S;
    int xlayer; /* words per layer region */
    float scale;
    /* g2k_step_f16/f32 only: 0 cooperative launch; 1 plain launch, so the
     * kernel checks that all its work-groups are resident before its first
     * lasting write; tests of that check: 2 as 1 with work-group 1
     * withholding its arrival, 3 with it arriving 0.5 ms late (within the
     * limit), 4 with it arriving 2 ms late (after the others gave up) */
    int plain;
    /* the row plans of every work-group, [nshares][5] g2p_rows (qkv, proj,
     * fc, fc2, lm_head: g2p_shares in g2_step_plan.h), built by the host for
     * a grid of nshares work-groups; a launch of another grid size does
     * nothing but set G2_ERR_STEP_ARGS */
    const void *shares;
    int nshares;
} g2_step_args;

#define G2_TRACE_STRIDE(L) (24 * (L) + 8)

/* A LayerNorm folded into the matrix W[N,K] (output-major, f32 or f16 by
 * kernel variant) it feeds: c1[r] = sum_k W[r,k] gamma[k] and c2[r] =
 * sum_k W[r,k] beta[k] + bias[r] (bias may be NULL), each summed in double
 * in a fixed order and rounded once.  Then W . LayerNorm(x) + bias =
 * inv * (W . ((x - s) * gamma) - (mean - s) * c1) + c2 for any shift s,
 * inv = 1 / sqrt(var + eps).  Grid ceil(N / 4), 256 threads (a row per
 * wave). */
typedef struct {
    const void *W;
    const float *gamma, *beta, *bias;
    float *c1, *c2;
    int N, K;
} g2_lnfold_args;

#define G2_STEP_THREADS 512
#define G2_STEP_MAXE 1600   /* largest n_embd the step kernel holds in LDS */
#define G2_STEP_MAXF 6400   /* largest ffn width */
#define G2_STEP_MAXUNITS 512 /* (row, segment) units per work-group and phase */
#define G2_STEP_MAXCH 16    /* 64-position key chunks per head */
#define G2X_HEAD 64         /* words before the first layer region (word 0: abort) */
#define G2X_DECISION 1      /* header word: a plain launch's residency verdict */
/* Word offsets inside one layer region (E = n_embd, NH heads): QKV outputs
 * [3E], attention chunk partials [NH][G2_STEP_MAXCH][66]; regions are
 * padded to 32 words. */
#define G2X_ATT(E) (3 * (E))
#define G2X_LAYER_WORDS(E, NH) ((G2X_ATT(E) + (NH) * G2_STEP_MAXCH * 66 + 31) & ~31)
/* Total words: header, L layer regions, 2 argmax words per work-group, 32
 * spare words, 1 arrival word per work-group. */
#define G2X_TOTAL_WORDS(L, E, NH, nwg) ((long)G2X_HEAD + (long)(L) * G2X_LAYER_WORDS(E, NH) + 3L * (nwg) + 32)
/* Float offsets inside one value region (F = ffn): merged attention O [E],
 * X1 = x + proj [E], H = gelu(fc) [F, padded to 4], X2 = X1 + fc2 [E];
 * regions are padded to 64 floats.  Every vector starts at a multiple of 4
 * floats (E is a multiple of 64), so the step kernel reads them as 16-byte
 * quads.  Each layer has two regions: the step with tag t writes region
 * t & 1 and stores G2V_EMPTY into the same entries of the other region,
 * which the next step writes; a value is present once it differs from
 * G2V_EMPTY (a signalling NaN, which no arithmetic result equals). */
#define G2V_O(E) 0
#define G2V_X1(E) (E)
#define G2V_H(E) (2 * (E))
#define G2V_X2(E, F) (2 * (E) + (((F) + 3) & ~3))
#define G2V_REGION(E, F) ((G2V_X2(E, F) + (E) + 63) & ~63)
#define G2V_TOTAL_FLOATS(L, E, F) (2L * (L) * G2V_REGION(E, F))
#define G2V_EMPTY 0x7FA5A5A5u
/* after the layers: 2 argmax words per work-group, 32 spare words, then one
 * arrival word per work-group (plain launches) */
#define G2X_ARRIVE(L, xlayer, nwg) ((long)G2X_HEAD + (long)(L) * (xlayer) + 2L * (nwg) + 32)

/* Causal attention over a prompt block: rows i < P of q[P,E]; keys/values
 * j <= i, head dim 64: g2k_attn_prefill_mfma reads them from the transposed
 * K cache and the V cache, g2k_attn_prefill_h16 from the fp16 halves the
 * qkv epilogue wrote (kh, kl [S][E]; vth, vtl [E][S]).  Grid: 1-D, 8 *
 * ceil(NH / 8) * ceil(P / 64) work-groups of 512 threads, every query
 * block of head h on XCD h % 8. */
typedef struct {
    const float *q;
    const float *k_cache;
    const float *v_cache;
    float *out;
    int P, E, NH, S;
    float scale;
    /* non-NULL: the output is written as fp16 halves (see g2_lnsplit_args)
     * to out_hi, out_lo [P,E] instead of to out */
    uint16_t *out_hi, *out_lo;
    const uint16_t *kh, *kl, *vth, *vtl;
    /* g2k_attn_prefill_h16's helper slots (g2a_help_plan; NULL: no helpers),
     * G2A_HELP_MAX_SLOTS of G2A_HELP_SLOT_BYTES, every float G2V_EMPTY
     * between launches; err: the G2S_ERR word, which a timed-out wait for a
     * helper's partial marks */
    float *help;
    int *err;
} g2_attnp_args;

#endif /* G2_KARGS_H */
