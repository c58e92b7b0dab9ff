/*
 * g2hip.h -- C ABI of the MI355X (gfx950) GPT-2 forward-pass library.
 *
 * Plain C99: device buffers are `void *` / typed pointers into HBM, sizes are
 * ints or size_t, no HIP or C++ types appear in any signature.  Every
 * function returns 0 (G2_OK) on success or a negative G2_E_* code; the text
 * of the last error is in g2_last_error().  Nothing calls exit().
 *
 * Threading model (as the reference's single in-order queue, main.c:537):
 * one library-owned HIP stream, all launches asynchronous on it, blocking
 * calls are g2_upload/g2_download/g2_sync and the model's logits/token reads.
 *
 * Each operator names the reference launch helper whose argument meaning it
 * keeps (reference files main.c and math.cl).  A NULL bias/residual means
 * "absent" exactly as a NULL cl_mem does in the reference (math.cl:178-180);
 * residual == C is legal (in-place residual add, main.c:1815-1816).
 */
#ifndef G2HIP_H
#define G2HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    G2_OK = 0,
    G2_E_ARG = -1,     /* invalid argument: NULL buffer, bad shape, bad dtype   */
    G2_E_STATE = -2,   /* library not initialised / model not loaded            */
    G2_E_IO = -3,      /* file missing or short read                            */
    G2_E_FORMAT = -4,  /* malformed config.json / safetensors, missing tensor   */
    G2_E_LIMIT = -5,   /* exceeds a compiled-in ceiling (sizes, context 1024)   */
    G2_E_NOMEM = -6,   /* host or device allocation failed                      */
    G2_E_HIP = -7      /* HIP runtime error (text in g2_last_error)             */
};

/* Element type of weights (and of the KV cache in the fused model). */
enum { G2_F32 = 0, G2_F16 = 1 };

/* Model execution paths.
 * G2_PATH_REFERENCE: the reference's op sequence (main.c:1739-1833), one
 *   launch per reference operator, weights in the reference layout
 *   ([in,out] row-major, padded transposed lm_head), fp32 only.
 * G2_PATH_FUSED: the gfx950 path -- output-major packed weights (fp32 or fp16),
 *   LayerNorm fused into the following matvec, fused single-query attention,
 *   MFMA prefill GEMMs, device-side greedy selection, replayed HIP graph. */
enum { G2_PATH_REFERENCE = 0, G2_PATH_FUSED = 1 };

#define G2_MAX_SEQ 1024        /* MAX_SEQ_LEN, main.c:51; ATTN_MAX_SEQ_LEN, math.cl:18 */
#define G2_EOS_TOKEN 50256     /* EOS_TOKEN_ID, main.c:58 */

const char *g2_last_error(void);

/* ---- runtime (replaces init_opencl, main.c:528-587) ---------------------- */
int g2_init(int device);                 /* load the gfx950 code object, make the stream */
int g2_shutdown(void);                   /* release stream, module, library buffers       */
int g2_device_name(char *buf, int len, int *compute_units);
/* The library's HIP stream (a hipStream_t; no counterpart in the
 * reference, whose queue is main.c:537): every launch of the library goes to
 * it, so a caller may capture the library's calls into its own HIP graph
 * (hipStreamBeginCapture on this stream, the calls, hipStreamEndCapture).
 * NULL before g2_init. */
void *g2_stream(void);

/* ---- buffers (clCreateBuffer / clEnqueue{Write,Copy,Read}Buffer / clFinish) */
int g2_alloc(void **dptr, size_t bytes);                       /* main.c:1225, 1460-1486 */
int g2_free(void *dptr);                                       /* main.c:2193-2194       */
int g2_upload(void *dst, const void *src, size_t bytes);       /* blocking, main.c:1227  */
int g2_upload_rect(void *dst, size_t dst_pitch, const void *src,
                   size_t src_pitch, size_t width_bytes, size_t rows); /* main.c:1327 */
int g2_copy(void *dst, const void *src, size_t bytes);         /* async, main.c:1783     */
int g2_download(void *dst, const void *src, size_t bytes);     /* blocking, main.c:1878  */
int g2_memset(void *dst, int value, size_t bytes);             /* async fill             */
int g2_sync(void);                                             /* clFinish               */

/* ---- operators (main.c launch_* helpers; kernels math.cl) ----------------- */

/* launch_matmul, main.c:1518-1535 (kernel main.c:603-684):
 * C[M,N] = A[M,K] B[K,N] (+bias[N]); all row-major fp32. */
int g2_matmul(const float *A, const float *B, const float *bias, float *C,
              int M, int N, int K);
/* Same with B stored as IEEE half (fp16 weights, fp32 accumulation). */
int g2_matmul_f16(const float *A, const uint16_t *B, const float *bias, float *C,
                  int M, int N, int K);

/* launch_matvec, main.c:1554-1576 (matvec4 math.cl:185-226 / matvec
 * math.cl:152-182): C[n] = act(sum_k A[k] B[k*N+n] + bias[n] + residual[n]);
 * any N >= 1 (the reference's N%4 split between its two kernels is internal). */
int g2_matvec(const float *A, const float *B, const float *bias,
              const float *residual, float *C, int N, int K, int apply_gelu);
int g2_matvec_f16(const float *A, const uint16_t *B, const float *bias,
                  const float *residual, float *C, int N, int K, int apply_gelu);

/* launch_matvec_splitk first half, math.cl:229-246: partial[s*N + n] =
 * sum over k = s, s+kslice, ... of A[k] B[k*N+n]; 1 <= kslice <= 8, N%4 == 0. */
int g2_matvec_sk(const float *A, const float *B, float *partial,
                 int N, int K, int kslice);
int g2_matvec_sk_f16(const float *A, const uint16_t *B, float *partial,
                     int N, int K, int kslice);
/* reduce_partial, math.cl:249-280: C[n] = act(sum_s partial[s*N+n] + bias + residual). */
int g2_reduce_partial(const float *partial, const float *bias,
                      const float *residual, float *C, int N, int kslice,
                      int apply_gelu);

/* launch_layernorm, main.c:1620-1633 (math.cl:283-311): rows of n_embd, eps 1e-5. */
int g2_layernorm(const float *x, float *out, const float *gamma,
                 const float *beta, int n_embd, int seq_len);

/* launch_add, main.c:1635-1644 (math.cl:314-322): a[i] += b[i]. */
int g2_add(float *a, const float *b, int n);
/* launch_gelu, main.c:1646-1654 (math.cl:325-330): tanh-approximate GELU in place. */
int g2_gelu(float *x, int n);

/* launch_embed, main.c:1656-1669 (math.cl:333-350):
 * out[i*n_embd+d] = wte[ids[i]*n_embd+d] + wpe[(start_pos+i)*n_embd+d]; ids on device. */
int g2_embed(const float *wte, const float *wpe, float *out, int n_embd,
             int seq_len, int start_pos, const int *ids);

/* launch_split_kv, main.c:1671-1685 (math.cl:367-383): rows i<T of qkv[T,3D];
 * k_cache[d*max_seq + pos] = K, v_cache[pos*D + d] = V, pos = start_pos + i. */
int g2_split_kv(const float *qkv, float *k_cache, float *v_cache,
                int start_pos, int T, int D, int max_seq);

/* launch_attn_scores, main.c:1687-1706 (math.cl:388-412):
 * scores[h*max_seq + j] = scale * sum_{k<DH} q[q_base + h*DH + k] k_cache[(h*DH+k)*max_seq + j], j < T_kv. */
int g2_attn_scores_1q(const float *qkv, const float *k_cache, float *scores,
                      int q_base, int T_kv, int D, int DH, int NH, int max_seq,
                      float scale);
/* launch_attn_softmax, main.c:1708-1716 (math.cl:415-456): in-place softmax of
 * scores rows h < NH over j < T_kv; row stride G2_MAX_SEQ as in math.cl:423. */
int g2_attn_softmax_1q(float *scores, int T_kv, int NH);
/* launch_attn_out, main.c:1718-1733 (math.cl:459-476):
 * out[out_base + d] = sum_{j<T_kv} scores[(d/DH)*G2_MAX_SEQ + j] v_cache[j*D + d]. */
int g2_attn_out_1q(const float *scores, const float *v_cache, float *out,
                   int T_kv, int D, int DH, int out_base);
/* Fused scores -> softmax -> weighted sum for one query row (the three calls
 * above without the scores buffer); DH must be 64. */
int g2_attn_1q(const float *qkv, const float *k_cache, const float *v_cache,
               float *out, int q_base, int T_kv, int D, int NH, int max_seq,
               int out_base, float scale);
/* g2_attn_1q that allocates nothing (no counterpart in the reference): for
 * callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments and results as g2_attn_1q; its chunk partials go to a static
 * device array of 64 heads x 16 chunks x 66 floats (270 KB per GPU, held
 * until the process ends) instead of a library buffer.  More than 64 heads:
 * G2_E_LIMIT.  Every call on a GPU shares that array, so calls that overlap
 * on one GPU (other streams or threads of the process) race; calls on the
 * library stream run one after another. */
int g2_attn_1q_noalloc(const float *qkv, const float *k_cache, const float *v_cache,
                       float *out, int q_base, int T_kv, int D, int NH, int max_seq,
                       int out_base, float scale);

/* launch_matvec over the output-major weight layout the fused model uses:
 * y[n] = sum_k W[n*K + k] x[k] (+ bias[n]) (+ y[n] when residual == y);
 * W is [N,K] row-major fp32 or fp16 (w_dtype), i.e. the transpose of the
 * reference's B[K,N].  K must be a multiple of 4 (fp32) or 8 (fp16), at
 * most 8192 (fp32) / 16384 (fp16); x and W 16-byte aligned. apply_gelu must
 * be 0 (the GELU epilogue exists only fused with LayerNorm in the model). */
int g2_matvec_rows(const float *x, const void *W, int w_dtype, const float *bias,
                   const float *residual, float *y, int N, int K, int apply_gelu);

/* ---- configuration, weights, model (main.c:272-331, 1137-1512, 1739-1904) -- */

typedef struct {
    int n_layer, n_embd, n_head, n_ctx, vocab_size, ffn_dim;
} g2_config;

/* Ceilings of this library (the reference's are main.c:46-52; these admit GPT-2 XL). */
#define G2_MAX_EMBED 1600
#define G2_MAX_LAYERS 48
#define G2_MAX_HEADS 25
#define G2_MAX_VOCAB 50304
#define G2_MAX_FFN 6400

/* load_config, main.c:294-331: dir/config.json, missing file -> GPT-2 small
 * defaults, ffn = n_inner or 4*n_embd; G2_E_LIMIT above the ceilings. Host only. */
int g2_config_load(const char *dir, g2_config *cfg);
/* Same on a JSON string already in memory. Host only. */
int g2_config_parse(const char *json, g2_config *cfg);

/* Deterministic N(0, std) generator used for the synthetic random-init
 * weights (counter-based splitmix64 + Box-Muller in double, rounded to fp32).
 * Host only; identical output on any thread count. */
void g2_synth_normal(float *dst, size_t n, uint64_t seed, uint32_t tensor_id,
                     float std_dev);
/* Tensor ids used by g2_model_synth: wte 1, wpe 2, and for layer l
 * 16+8l (attn.c_attn.weight), 17+8l (attn.c_proj.weight),
 * 18+8l (mlp.c_fc.weight), 19+8l (mlp.c_proj.weight); all in the Conv1D
 * [in,out] storage order.  Biases are 0, LayerNorm gamma 1 and beta 0. */
uint32_t g2_synth_tensor_id(int layer, int which);

/* IEEE fp32 -> fp16 (binary16) with round-to-nearest-even; host only.  The
 * fp16 weight format stores exactly these values. */
void g2_convert_f16(uint16_t *dst, const float *src, size_t n);

typedef struct g2_model g2_model;

/* load_model, main.c:1339-1417: dir/config.json + dir/model.safetensors
 * (F32 or F16 tensors, Conv1D or Linear layout, tied or separate lm_head,
 * names with optional "transformer." / "model." prefix). weight_dtype picks
 * the device storage of the matrices (G2_F16 rounds to nearest even). */
int g2_model_load(const char *dir, int weight_dtype, int path, g2_model **out);
/* A model of the given shape with the synthetic random-init weights
 * (N(0,0.02) matrices via g2_synth_normal, zero biases, unit LayerNorm). */
int g2_model_synth(const g2_config *cfg, uint64_t seed, int weight_dtype,
                   int path, g2_model **out);
/* A model from caller-provided host weights in the Conv1D layout; `layers`
 * holds 12 pointers per layer: ln1_w ln1_b qkv_w qkv_b proj_w proj_b ln2_w
 * ln2_b fc_w fc_b fc2_w fc2_b (weights [in,out] row-major fp32). */
int g2_model_from_host(const g2_config *cfg, const float *wte, const float *wpe,
                       const float *lnf_w, const float *lnf_b,
                       const float *const *layers, int weight_dtype, int path,
                       g2_model **out);
int g2_model_free(g2_model *m);
int g2_model_config(const g2_model *m, g2_config *cfg);
/* Pinned split-K slice count of the reference path (default 4, main.c:1081). */
int g2_model_set_kslice(g2_model *m, int kslice);
/* Device bytes held by the model's weights (cf. "Model VRAM", main.c:1416). */
size_t g2_model_weight_bytes(const g2_model *m);
/* Fused path: 1 if decode steps replay a captured HIP graph, 0 if their
 * kernels are launched one by one (capture unavailable, or the environment
 * sets G2_NO_GRAPH=1, e.g. under a profiler), -1 before the first step. */
int g2_model_uses_graph(const g2_model *m);
/* Fused path decode engine.  By default (when the device supports
 * cooperative launch and the model fits the kernel: n_embd <= 1600, ffn <=
 * 6400) every decode forward is ONE launch of a persistent kernel that runs
 * all layers, the lm_head and the greedy pick (a plain launch that checks
 * in the kernel that its work-groups are resident, else resumes the call
 * with cooperative launches; G2_STEP_COOP=1 forces those); the variable
 * G2_STEP=0 or g2_model_set_step(m, 0) selects the per-operator kernels
 * instead.  Replaces the reference's per-op enqueue loop of decode()
 * (main.c:1792-1833) with no counterpart there.  set_step returns G2_E_ARG
 * if on=1 and the model cannot use the kernel; uses_step returns 1 (step
 * kernel) or 0 (per-operator kernels). */
int g2_model_set_step(g2_model *m, int on);
int g2_model_uses_step(const g2_model *m);
/* Name of the kernel one decode forward launches when the model decodes
 * with the persistent step kernel (g2k_step_f16 / _f32, or their tail forms
 * g2k_step_f16_tail / _f32_tail, which the host picks when every matrix row
 * plan ends 1..16 chunks into its last slot); "" for the per-operator
 * kernels or a NULL model.  No counterpart in the reference. */
const char *g2_model_step_kernel(const g2_model *m);

/* prefill, main.c:1739-1790: ids[0..n) at positions 0..n-1, 1 <= n <= 1023;
 * leaves the last row's logits on the device. */
int g2_prefill(g2_model *m, const int *ids, int n);
/* decode, main.c:1792-1833: one token at position pos (1 <= pos < 1024). */
int g2_decode(g2_model *m, int token, int pos);
/* Blocking read of the first n logits of the last forward (main.c:1878). */
int g2_read_logits(g2_model *m, float *host, int n);
/* Blocking read of layer `layer`'s KV cache in the reference layout
 * (main.c:1481-1486): k_host [n_embd, 1024] (transposed), v_host
 * [1024, n_embd]; either pointer may be NULL. */
int g2_read_kv(g2_model *m, int layer, float *k_host, float *v_host);
/* sample_next_token greedy branch, main.c:1872-1904 (temperature 0): EOS
 * mask when forbid_eos, repetition penalty over the distinct context ids
 * when rep_penalty > 1, first-max argmax. Returns the token id (>= 0) or a
 * negative error code. */
int g2_sample_greedy(g2_model *m, const int *ctx, int n_ctx, int forbid_eos,
                     float rep_penalty);

/* The generation loop of main.c:2106-2150 at temperature 0, repetition
 * penalty off: prefill, first token from the prefill logits, then decode
 * until max_new tokens, EOS, or 1024 positions; EOS is masked while fewer
 * than min_new tokens exist.  The fused path selects tokens on the device
 * and replays one captured HIP graph per token.  Returns the number of ids
 * written to out_ids (>= 1) or a negative error code.  If timing is
 * non-NULL it receives {prefill+first ms, decode ms} from HIP events. */
int g2_generate(g2_model *m, const int *prompt, int n_prompt, int max_new,
                int min_new, int *out_ids, double *timing);

/* Decode-only replay for measurement: with the KV cache already holding
 * positions < start_pos (from g2_prefill/g2_generate) and `token` the id at
 * start_pos, run n_steps greedy decode forwards (positions start_pos ..
 * start_pos+n_steps-1) with device-side selection, writing the chosen ids to
 * out_ids (may be NULL).  Fused path only.  elapsed_ms (may be NULL) gets
 * the HIP-event time of the whole run. */
int g2_decode_run(g2_model *m, int token, int start_pos, int n_steps,
                  int forbid_eos, int *out_ids, double *elapsed_ms);

/* ---- text prompts: GPT-2 byte-level BPE (replaces tokenizer.h / tokenizer.c)
 * Host-only; no device is needed.  Same behaviour as the reference's
 * tokenizer: ASCII-class pre-tokenisation, byte alphabet, ranked merges,
 * tokens missing from the vocabulary dropped. */
typedef struct g2_tokenizer g2_tokenizer;

/* vocab.json and merges.txt from the directory (gpt2_tokenizer_load,
 * tokenizer.h:11); G2_OK or an error code, *out NULL on failure. */
int g2_tok_load(const char *dir, g2_tokenizer **out);
void g2_tok_free(g2_tokenizer *t);                 /* gpt2_tokenizer_free, tokenizer.h:12 */
int g2_tok_vocab_size(const g2_tokenizer *t);      /* tokenizer.h:24: largest id + 1 */
/* UTF-8 text to at most max_ids ids (gpt2_encode, tokenizer.h:15): the count
 * written, or -1 on a NULL argument or max_ids <= 0. */
int g2_tok_encode(const g2_tokenizer *t, const char *text, int *ids, int max_ids);
/* ids to UTF-8, NUL-terminated, at most max_bytes - 1 bytes (gpt2_decode,
 * tokenizer.h:19): the bytes written, or -1 on a NULL argument or
 * max_bytes <= 0. */
int g2_tok_decode(const g2_tokenizer *t, const int *ids, int n, char *out, int max_bytes);

#ifdef __cplusplus
}
#endif

#endif /* G2HIP_H */
