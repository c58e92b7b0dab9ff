/*
 * g2_shim.c -- C99 HIP shim: runtime set-up, buffers and the reference
 * operator launchers.
 *
 * Replaces the reference's OpenCL context/queue/program code (main.c:528-587)
 * and its launch_* helpers (main.c:1518-1733).  The gfx950 code object is
 * linked into the library (g2_embed.S) and loaded with hipModuleLoadData;
 * kernels are resolved once with hipModuleGetFunction and launched with
 * hipModuleLaunchKernel on one library-owned stream (the in-order queue of
 * main.c:537).  Every entry point validates shapes and pointers on the host
 * and returns a G2_E_* code instead of launching an out-of-range kernel.
 */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g2_internal.h"

extern const unsigned char g2_hsaco_begin[];
extern const unsigned char g2_hsaco_end[];

#define G2_NAME_ENTRY(id, name) name,
static const char *const g2_kernel_names[G2F_COUNT] = { G2_KERNEL_LIST(G2_NAME_ENTRY) };
#undef G2_NAME_ENTRY

/* Library scratch: split-K partials of g2_matvec (at most 64 splits of
 * G2_MAX_VOCAB columns) and the attention chunk partials of g2_attn_1q. */
#define G2_MV_MAX_SPLITS 64
#define G2_SCRATCH_FLOATS ((size_t)G2_MV_MAX_SPLITS * 65536)
#define G2_ATTN_PART_FLOATS ((size_t)64 * G2_ATTN_MAX_CHUNKS * 66)

static struct {
    int ready, device, cus;
    int step_wgs; /* work-groups of a cooperative step launch (0: unsupported) */
    char name[256];
    hipModule_t module;
    hipStream_t stream;
    hipFunction_t fn[G2F_COUNT];
    float *scratch;
    float *attn_part;
    int noalloc_rc;         /* g2i_noalloc_setup result at g2_init */
    char noalloc_err[256];
} G;

static char g_errbuf[512] = "no error";

const char *g2_last_error(void) { return g_errbuf; }

int g2i_err(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_errbuf, sizeof g_errbuf, fmt, ap);
    va_end(ap);
    return code;
}

int g2i_hip(hipError_t e, const char *what)
{
    if (e == hipSuccess) return G2_OK;
    return g2i_err(e == hipErrorOutOfMemory ? G2_E_NOMEM : G2_E_HIP,
                   "HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
}

int g2i_ready(void) { return G.ready; }
hipStream_t g2i_stream(void) { return G.stream; }

int g2i_launch(int fid, unsigned gx, unsigned gy, unsigned bx, void *args)
{
    void *params[1] = { args };
    if (gx == 0 || gy == 0) return G2_OK;
    return g2i_hip(hipModuleLaunchKernel(G.fn[fid], gx, gy, 1, bx, 1, 1, 0,
                                         G.stream, params, NULL),
                   g2_kernel_names[fid]);
}

int g2i_launch3(int fid, unsigned gx, unsigned gy, unsigned gz, unsigned bx, void *args)
{
    void *params[1] = { args };
    if (gx == 0 || gy == 0 || gz == 0) return G2_OK;
    return g2i_hip(hipModuleLaunchKernel(G.fn[fid], gx, gy, gz, bx, 1, 1, 0,
                                         G.stream, params, NULL),
                   g2_kernel_names[fid]);
}

int g2i_coop_launch(int fid, unsigned gx, unsigned bx, void *args)
{
    void *params[1] = { args };
    return g2i_hip(hipModuleLaunchCooperativeKernel(G.fn[fid], gx, 1, 1, bx, 1, 1, 0, G.stream, params),
                   g2_kernel_names[fid]);
}

int g2i_step_wgs(void) { return G.step_wgs; }
void *g2_stream(void) { return G.ready ? (void *)G.stream : NULL; }
const char *g2i_kernel_name(int fid) { return fid >= 0 && fid < G2F_COUNT ? g2_kernel_names[fid] : ""; }
int g2i_cus(void) { return G.cus > 0 ? G.cus : 1; }

int g2i_device_alloc(void **p, size_t bytes)
{
    *p = NULL;
    if (bytes == 0) bytes = 256;
    return g2i_hip(hipMalloc(p, bytes), "hipMalloc");
}

#define NEED_READY() do { if (!G.ready) return g2i_err(G2_E_STATE, "g2_init has not been called"); } while (0)

/* Lane shape of the packed matvec for N rows of C = K/V 16-byte chunks
 * (measured on the GPT-2 XL decode matrices):
 *   0: 64 lanes x 4 chunks, 4 rows per work-group -- C <= 256, N <= 2048
 *   1: 256 lanes x 1 chunk x 2 rows                -- C <= 256, longer N
 *   2: 256 lanes x 4 chunks x 2 rows               -- C <= 1024
 *   3: 256 lanes x 8 chunks x 1 row                -- C <= 2048
 * Returns the shape and the rows a work-group takes at a time, or -1 if K
 * is not supported. */
static int rows_shape(int N, int K, int f16, int *rows_per_wg)
{
    const int V = f16 ? 8 : 4;
    if (K <= 0 || K % V) return -1;
    const int C = K / V;
    if (C <= 256 && N <= 2048) { *rows_per_wg = 4; return 0; }
    if (C <= 256) { *rows_per_wg = 2; return 1; }
    if (C <= 1024) { *rows_per_wg = 2; return 2; }
    if (C <= 2048) { *rows_per_wg = 1; return 3; }
    return -1;
}

unsigned g2i_rows_grid(int N, int K, int f16)
{
    int per;
    if (rows_shape(N, K, f16, &per) < 0 || N <= 0) return 0;
    const unsigned per_wg = (unsigned)per;
    unsigned g = ((unsigned)N + per_wg - 1) / per_wg;
    return g > G2_ROWS_MAX_GRID ? G2_ROWS_MAX_GRID : g;
}

int g2i_rows_launch(int fid_f32_64, int f16, g2_rows_args *a)
{
    int per;
    const int shape = rows_shape(a->N, a->K, f16, &per);
    if (shape < 0 || a->N <= 0)
        return g2i_err(G2_E_ARG, "packed matvec: K=%d must be a multiple of %d and at most %d",
                       a->K, f16 ? 8 : 4, (f16 ? 8 : 4) * 2048);
    return g2i_launch(fid_f32_64 + 2 * shape + (f16 ? 1 : 0), g2i_rows_grid(a->N, a->K, f16), 1, 256, a);
}

/* ------------------------------------------------------------------ runtime */

int g2_init(int device)
{
    int rc;
    if (G.ready) {
        if (device == G.device) return G2_OK;
        return g2i_err(G2_E_STATE, "already initialised on device %d", G.device);
    }
    int n = 0;
    if ((rc = g2i_hip(hipGetDeviceCount(&n), "hipGetDeviceCount"))) return rc;
    if (device < 0 || device >= n)
        return g2i_err(G2_E_ARG, "device %d out of range (%d devices)", device, n);
    if ((rc = g2i_hip(hipSetDevice(device), "hipSetDevice"))) return rc;
    hipDeviceProp_t prop;
    if ((rc = g2i_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"))) return rc;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return g2i_err(G2_E_HIP, "device %d is %s; this library is built for gfx950",
                       device, prop.gcnArchName);
    snprintf(G.name, sizeof G.name, "%s", prop.name);
    G.cus = prop.multiProcessorCount;
    if ((rc = g2i_hip(hipModuleLoadData(&G.module, g2_hsaco_begin), "hipModuleLoadData"))) return rc;
    for (int i = 0; i < G2F_COUNT; ++i) {
        rc = g2i_hip(hipModuleGetFunction(&G.fn[i], G.module, g2_kernel_names[i]),
                     g2_kernel_names[i]);
        if (rc) { hipModuleUnload(G.module); return rc; }
    }
    if ((rc = g2i_hip(hipStreamCreateWithFlags(&G.stream, hipStreamNonBlocking), "hipStreamCreate"))) {
        hipModuleUnload(G.module);
        return rc;
    }
    rc = g2i_hip(hipMalloc((void **)&G.scratch, G2_SCRATCH_FLOATS * sizeof(float)), "scratch");
    if (!rc) rc = g2i_hip(hipMalloc((void **)&G.attn_part, G2_ATTN_PART_FLOATS * sizeof(float)), "attn scratch");
    if (rc) {
        hipFree(G.scratch); hipFree(G.attn_part);
        hipStreamDestroy(G.stream); hipModuleUnload(G.module);
        memset(&G, 0, sizeof G);
        return rc;
    }
    /* The persistent step kernel runs one work-group per CU and needs all of
     * them co-resident: require cooperative launch support and an occupancy
     * of at least one work-group per CU for both weight types. */
    {
        enum { NSTEP = 14 };
        int coop = 0, nb[NSTEP];
        hipError_t ea = hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device);
        hipError_t eo[NSTEP];
        const int fids[NSTEP] = { G2F_STEP_F32, G2F_STEP_F16, G2F_STEP_F32T, G2F_STEP_F16T, G2F_STEP_F16TN,
                                  G2F_STEP_F32_E768, G2F_STEP_F32_E1024, G2F_STEP_F32_E1280, G2F_STEP_F16_E1280,
                                  G2F_STEP_F32_TR, G2F_STEP_F16_TR, G2F_STEP_F32T_TR, G2F_STEP_F16T_TR,
                                  G2F_STEP_F16TN_TR };
        int ok = ea == hipSuccess && coop;
        for (int i = 0; i < NSTEP; ++i) {
            nb[i] = -1;
            eo[i] = hipSuccess;
        }
        for (int i = 0; i < NSTEP; ++i) {
            eo[i] = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&nb[i], G.fn[fids[i]], G2_STEP_THREADS, 0);
            ok = ok && eo[i] == hipSuccess && nb[i] >= 1;
        }
        G.step_wgs = ok ? prop.multiProcessorCount : 0;
        if (!ok) {
            int rtv = 0;
            hipFuncAttributes fa;
            memset(&fa, 0, sizeof fa);
            (void)hipRuntimeGetVersion(&rtv);
            (void)hipFuncGetAttributes(&fa, (const void *)G.fn[G2F_STEP_F16]);
            fprintf(stderr, "g2hip: persistent step kernel unavailable (HIP runtime %d, cooperative launch %d, "
                            "err %d; work-groups per CU %d/%d/%d/%d, err %d/%d/%d/%d; kernel regs %d lds %zu max "
                            "threads %d); decode uses per-operator kernels\n",
                    rtv, coop, (int)ea, nb[0], nb[1], nb[2], nb[3], (int)eo[0], (int)eo[1], (int)eo[2], (int)eo[3],
                    fa.numRegs, fa.sharedSizeBytes, fa.maxThreadsPerBlock);
        }
        (void)hipGetLastError();
    }
    /* the allocation-free entry point's scratch: resolve its address on this
     * device now; a failure only disables that entry point */
    G.noalloc_rc = g2i_noalloc_setup(device);
    if (G.noalloc_rc) snprintf(G.noalloc_err, sizeof G.noalloc_err, "%s", g2_last_error());
    G.device = device;
    G.ready = 1;
    (void)g2_hsaco_end;
    return G2_OK;
}

int g2_shutdown(void)
{
    if (!G.ready) return G2_OK;
    hipStreamSynchronize(G.stream);
    hipFree(G.scratch);
    hipFree(G.attn_part);
    hipStreamDestroy(G.stream);
    hipModuleUnload(G.module);
    memset(&G, 0, sizeof G);
    return G2_OK;
}

int g2_device_name(char *buf, int len, int *compute_units)
{
    NEED_READY();
    if (buf && len > 0) snprintf(buf, (size_t)len, "%s", G.name);
    if (compute_units) *compute_units = G.cus;
    return G2_OK;
}

/* ------------------------------------------------------------------ buffers */

int g2_alloc(void **dptr, size_t bytes)
{
    NEED_READY();
    if (!dptr) return g2i_err(G2_E_ARG, "g2_alloc: NULL out pointer");
    return g2i_device_alloc(dptr, bytes);
}

int g2_free(void *dptr)
{
    NEED_READY();
    if (!dptr) return G2_OK;
    hipStreamSynchronize(G.stream);
    return g2i_hip(hipFree(dptr), "hipFree");
}

int g2_upload(void *dst, const void *src, size_t bytes)
{
    NEED_READY();
    if (!dst || !src) return g2i_err(G2_E_ARG, "g2_upload: NULL pointer");
    int rc = g2i_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, G.stream), "upload");
    if (rc) return rc;
    return g2i_hip(hipStreamSynchronize(G.stream), "upload sync");
}

int g2_upload_rect(void *dst, size_t dst_pitch, const void *src, size_t src_pitch,
                   size_t width_bytes, size_t rows)
{
    NEED_READY();
    if (!dst || !src || width_bytes > dst_pitch || width_bytes > src_pitch)
        return g2i_err(G2_E_ARG, "g2_upload_rect: bad arguments");
    int rc = g2i_hip(hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, width_bytes, rows,
                                      hipMemcpyHostToDevice, G.stream), "upload_rect");
    if (rc) return rc;
    return g2i_hip(hipStreamSynchronize(G.stream), "upload_rect sync");
}

int g2_copy(void *dst, const void *src, size_t bytes)
{
    NEED_READY();
    if (!dst || !src) return g2i_err(G2_E_ARG, "g2_copy: NULL pointer");
    return g2i_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, G.stream), "copy");
}

int g2_download(void *dst, const void *src, size_t bytes)
{
    NEED_READY();
    if (!dst || !src) return g2i_err(G2_E_ARG, "g2_download: NULL pointer");
    int rc = g2i_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, G.stream), "download");
    if (rc) return rc;
    return g2i_hip(hipStreamSynchronize(G.stream), "download sync");
}

int g2_memset(void *dst, int value, size_t bytes)
{
    NEED_READY();
    if (!dst) return g2i_err(G2_E_ARG, "g2_memset: NULL pointer");
    return g2i_hip(hipMemsetAsync(dst, value, bytes, G.stream), "memset");
}

int g2_sync(void)
{
    NEED_READY();
    return g2i_hip(hipStreamSynchronize(G.stream), "sync");
}

/* ---------------------------------------------------------------- operators */

static unsigned cdiv(long a, long b) { return (unsigned)((a + b - 1) / b); }
static int aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

static int gemm_kn(int fid, const float *A, const void *B, const float *bias, float *C,
                   int M, int N, int K)
{
    NEED_READY();
    if (!A || !B || !C) return g2i_err(G2_E_ARG, "g2_matmul: NULL buffer");
    if (M <= 0 || N <= 0 || K <= 0) return g2i_err(G2_E_ARG, "g2_matmul: M,N,K must be positive");
    g2_gemm_args a;
    memset(&a, 0, sizeof a);
    a.A = A; a.B = B; a.bias = bias; a.C = C; a.M = M; a.N = N; a.K = K;
    return g2i_launch(fid, cdiv(N, 64), cdiv(M, 64), 256, &a);
}

int g2_matmul(const float *A, const float *B, const float *bias, float *C, int M, int N, int K)
{
    return gemm_kn(G2F_GEMM_KN_F32, A, B, bias, C, M, N, K);
}

int g2_matmul_f16(const float *A, const uint16_t *B, const float *bias, float *C,
                  int M, int N, int K)
{
    return gemm_kn(G2F_GEMM_KN_F16, A, B, bias, C, M, N, K);
}

/* Split count for g2_matvec: about 2048 work-groups over the column tiles,
 * at least 8 rows per split, at most G2_MV_MAX_SPLITS. */
static int mv_splits(int N, int K, int *rows_per_split)
{
    const int tiles = (int)cdiv(N, 256);
    int s = (int)cdiv(2048, tiles);
    if (s > G2_MV_MAX_SPLITS) s = G2_MV_MAX_SPLITS;
    if (s > (K + 7) / 8) s = (K + 7) / 8;
    if (s < 1) s = 1;
    int rps = (int)cdiv(K, s);
    *rows_per_split = rps;
    return (int)cdiv(K, rps);
}

static int matvec_any(int f16, const float *A, const void *B, const float *bias,
                      const float *res, float *C, int N, int K, int gelu)
{
    NEED_READY();
    if (!A || !B || !C) return g2i_err(G2_E_ARG, "g2_matvec: NULL buffer");
    if (N <= 0 || K <= 0) return g2i_err(G2_E_ARG, "g2_matvec: N and K must be positive");
    if (N > 65536) return g2i_err(G2_E_LIMIT, "g2_matvec: N=%d above 65536", N);
    int rps;
    const int splits = mv_splits(N, K, &rps);
    const int vec = (N % 4) == 0 && aligned(B, f16 ? 8 : 16);
    const int fid = f16 ? (vec ? G2F_MVKN_F16 : G2F_MVKN_F16_S)
                        : (vec ? G2F_MVKN_F32 : G2F_MVKN_F32_S);
    g2_mvkn_args a = { A, B, G.scratch, N, K, rps };
    int rc = g2i_launch(fid, cdiv(N, 256), (unsigned)splits, 256, &a);
    if (rc) return rc;
    g2_reduce_args r = { G.scratch, bias, res, C, N, splits, gelu ? 1 : 0 };
    return g2i_launch(G2F_REDUCE, cdiv(N, 256), 1, 256, &r);
}

int g2_matvec(const float *A, const float *B, const float *bias, const float *residual,
              float *C, int N, int K, int apply_gelu)
{
    return matvec_any(0, A, B, bias, residual, C, N, K, apply_gelu);
}

int g2_matvec_f16(const float *A, const uint16_t *B, const float *bias,
                  const float *residual, float *C, int N, int K, int apply_gelu)
{
    return matvec_any(1, A, B, bias, residual, C, N, K, apply_gelu);
}

static int matvec_sk_any(int f16, const float *A, const void *B, float *partial,
                         int N, int K, int kslice)
{
    NEED_READY();
    if (!A || !B || !partial) return g2i_err(G2_E_ARG, "g2_matvec_sk: NULL buffer");
    if (N <= 0 || K <= 0 || (N & 3)) return g2i_err(G2_E_ARG, "g2_matvec_sk: N must be a positive multiple of 4");
    if (kslice < 1 || kslice > 8) return g2i_err(G2_E_ARG, "g2_matvec_sk: kslice %d not in 1..8", kslice);
    g2_mvsk_args a = { A, B, partial, N, K, kslice };
    return g2i_launch(f16 ? G2F_MVSK_F16 : G2F_MVSK_F32, cdiv(N / 4, 256), (unsigned)kslice, 256, &a);
}

int g2_matvec_sk(const float *A, const float *B, float *partial, int N, int K, int kslice)
{
    return matvec_sk_any(0, A, B, partial, N, K, kslice);
}

int g2_matvec_sk_f16(const float *A, const uint16_t *B, float *partial, int N, int K, int kslice)
{
    return matvec_sk_any(1, A, B, partial, N, K, kslice);
}

int g2_reduce_partial(const float *partial, const float *bias, const float *residual,
                      float *C, int N, int kslice, int apply_gelu)
{
    NEED_READY();
    if (!partial || !C) return g2i_err(G2_E_ARG, "g2_reduce_partial: NULL buffer");
    if (N <= 0 || kslice < 1 || kslice > 8) return g2i_err(G2_E_ARG, "g2_reduce_partial: bad N or kslice");
    g2_reduce_args r = { partial, bias, residual, C, N, kslice, apply_gelu ? 1 : 0 };
    return g2i_launch(G2F_REDUCE, cdiv(N, 256), 1, 256, &r);
}

int g2_layernorm(const float *x, float *out, const float *gamma, const float *beta,
                 int n_embd, int seq_len)
{
    NEED_READY();
    if (!x || !out || !gamma || !beta) return g2i_err(G2_E_ARG, "g2_layernorm: NULL buffer");
    if (n_embd <= 0 || seq_len <= 0) return g2i_err(G2_E_ARG, "g2_layernorm: bad sizes");
    g2_ln_args a = { x, out, gamma, beta, n_embd, seq_len };
    return g2i_launch(G2F_LAYERNORM, (unsigned)seq_len, 1, 256, &a);
}

static unsigned ew_grid(int n)
{
    unsigned g = cdiv(n, 256);
    return g > 4096 ? 4096 : g;
}

int g2_add(float *a, const float *b, int n)
{
    NEED_READY();
    if (!a || !b) return g2i_err(G2_E_ARG, "g2_add: NULL buffer");
    if (n < 0) return g2i_err(G2_E_ARG, "g2_add: negative n");
    g2_ew_args e = { a, b, n };
    return g2i_launch(G2F_ADD, ew_grid(n), 1, 256, &e);
}

int g2_gelu(float *x, int n)
{
    NEED_READY();
    if (!x) return g2i_err(G2_E_ARG, "g2_gelu: NULL buffer");
    if (n < 0) return g2i_err(G2_E_ARG, "g2_gelu: negative n");
    g2_ew_args e = { x, NULL, n };
    return g2i_launch(G2F_GELU, ew_grid(n), 1, 256, &e);
}

int g2_embed(const float *wte, const float *wpe, float *out, int n_embd, int seq_len,
             int start_pos, const int *ids)
{
    NEED_READY();
    if (!wte || !wpe || !out || !ids) return g2i_err(G2_E_ARG, "g2_embed: NULL buffer");
    if (n_embd <= 0 || seq_len <= 0 || start_pos < 0 || start_pos + seq_len > G2_MAX_SEQ)
        return g2i_err(G2_E_ARG, "g2_embed: bad sizes (seq_len %d start_pos %d)", seq_len, start_pos);
    g2_embed_args a = { wte, wpe, out, ids, NULL, n_embd, seq_len, start_pos };
    return g2i_launch(G2F_EMBED_F32, cdiv(n_embd, 256), (unsigned)seq_len, 256, &a);
}

int g2_split_kv(const float *qkv, float *k_cache, float *v_cache, int start_pos, int T,
                int D, int max_seq)
{
    NEED_READY();
    if (!qkv || !k_cache || !v_cache) return g2i_err(G2_E_ARG, "g2_split_kv: NULL buffer");
    if (T <= 0 || D <= 0 || start_pos < 0 || start_pos + T > max_seq)
        return g2i_err(G2_E_ARG, "g2_split_kv: positions %d..%d outside the cache of %d",
                       start_pos, start_pos + T - 1, max_seq);
    g2_splitkv_args a = { qkv, k_cache, v_cache, start_pos, T, D, max_seq };
    return g2i_launch(G2F_SPLIT_KV, cdiv((long)T * D, 256), 1, 256, &a);
}

int g2_attn_scores_1q(const float *qkv, const float *k_cache, float *scores, int q_base,
                      int T_kv, int D, int DH, int NH, int max_seq, float scale)
{
    NEED_READY();
    if (!qkv || !k_cache || !scores) return g2i_err(G2_E_ARG, "g2_attn_scores_1q: NULL buffer");
    if (T_kv <= 0 || T_kv > max_seq || max_seq > G2_MAX_SEQ || DH <= 0 || NH <= 0 ||
        NH * DH > D || q_base < 0)
        return g2i_err(G2_E_ARG, "g2_attn_scores_1q: bad sizes");
    g2_scores_args a = { qkv, k_cache, scores, q_base, T_kv, D, DH, NH, max_seq, scale };
    return g2i_launch(G2F_ATTN_SCORES, (unsigned)NH, cdiv(T_kv, 256), 256, &a);
}

int g2_attn_softmax_1q(float *scores, int T_kv, int NH)
{
    NEED_READY();
    if (!scores) return g2i_err(G2_E_ARG, "g2_attn_softmax_1q: NULL buffer");
    if (T_kv <= 0 || T_kv > G2_MAX_SEQ || NH <= 0) return g2i_err(G2_E_ARG, "g2_attn_softmax_1q: bad sizes");
    g2_softmax_args a = { scores, T_kv, NH };
    return g2i_launch(G2F_ATTN_SOFTMAX, (unsigned)NH, 1, 256, &a);
}

int g2_attn_out_1q(const float *scores, const float *v_cache, float *out, int T_kv, int D,
                   int DH, int out_base)
{
    NEED_READY();
    if (!scores || !v_cache || !out) return g2i_err(G2_E_ARG, "g2_attn_out_1q: NULL buffer");
    if (T_kv <= 0 || T_kv > G2_MAX_SEQ || D <= 0 || DH <= 0 || out_base < 0)
        return g2i_err(G2_E_ARG, "g2_attn_out_1q: bad sizes");
    g2_attnout_args a = { scores, v_cache, out, T_kv, D, DH, out_base };
    return g2i_launch(G2F_ATTN_OUT, cdiv(D, 64), 1, 1024, &a);
}

int g2_attn_1q(const float *qkv, const float *k_cache, const float *v_cache, float *out,
               int q_base, int T_kv, int D, int NH, int max_seq, int out_base, float scale)
{
    NEED_READY();
    if (!qkv || !k_cache || !v_cache || !out) return g2i_err(G2_E_ARG, "g2_attn_1q: NULL buffer");
    if (NH <= 0 || NH > 64 || NH * 64 != D)
        return g2i_err(G2_E_ARG, "g2_attn_1q: needs head dim 64 (D=%d NH=%d), NH <= 64", D, NH);
    if (T_kv <= 0 || T_kv > max_seq || max_seq > G2_MAX_SEQ || q_base < 0 || out_base < 0)
        return g2i_err(G2_E_ARG, "g2_attn_1q: bad sizes");
    g2_attn1q_args a;
    memset(&a, 0, sizeof a);
    a.q = qkv + q_base; a.k_cache = k_cache; a.v_cache = v_cache; a.out = out + out_base;
    a.part = G.attn_part;
    a.T_fixed = T_kv; a.D = D; a.NH = NH; a.S = max_seq; a.max_chunks = G2_ATTN_MAX_CHUNKS;
    a.scale = scale;
    return g2i_attn_launch(&a, cdiv(T_kv, G2_ATTN_CHUNK));
}

/* g2_attn_1q without allocation: the chunk partials go to the static device
 * scratch resolved at g2_init (g2_noalloc.hip), not to a library buffer.
 * Nothing is allocated or freed here; every partial the merge reads is
 * written by the same call, so no clearing is needed. */
int g2_attn_1q_noalloc(const float *qkv, const float *k_cache, const float *v_cache, float *out,
                       int q_base, int T_kv, int D, int NH, int max_seq, int out_base, float scale)
{
    NEED_READY();
    if (NH > 0 && (long)NH * G2_ATTN_MAX_CHUNKS * 66 > G2_NOALLOC_SCRATCH_FLOATS)
        return g2i_err(G2_E_LIMIT, "g2_attn_1q_noalloc: %d heads need %ld scratch floats, the static scratch "
                       "holds %d (64 heads)", NH, (long)NH * G2_ATTN_MAX_CHUNKS * 66, G2_NOALLOC_SCRATCH_FLOATS);
    if (G.noalloc_rc) return g2i_err(G2_E_HIP, "g2_attn_1q_noalloc: no static scratch: %s", G.noalloc_err);
    if (!qkv || !k_cache || !v_cache || !out) return g2i_err(G2_E_ARG, "g2_attn_1q_noalloc: NULL buffer");
    if (NH <= 0 || NH * 64 != D)
        return g2i_err(G2_E_ARG, "g2_attn_1q_noalloc: needs head dim 64 (D=%d NH=%d)", D, NH);
    if (T_kv <= 0 || T_kv > max_seq || max_seq > G2_MAX_SEQ || q_base < 0 || out_base < 0)
        return g2i_err(G2_E_ARG, "g2_attn_1q_noalloc: bad sizes");
    float *part = g2i_noalloc_scratch(G.device);
    if (!part) return g2i_err(G2_E_STATE, "g2_attn_1q_noalloc: static scratch not resolved on device %d", G.device);
    g2_attn1q_args a;
    memset(&a, 0, sizeof a);
    a.q = qkv + q_base; a.k_cache = k_cache; a.v_cache = v_cache; a.out = out + out_base;
    a.part = part;
    a.T_fixed = T_kv; a.D = D; a.NH = NH; a.S = max_seq; a.max_chunks = G2_ATTN_MAX_CHUNKS;
    a.scale = scale;
    return g2i_attn_launch(&a, cdiv(T_kv, G2_ATTN_CHUNK));
}

int g2i_attn_launch(g2_attn1q_args *a, unsigned chunks)
{
    const int vec = a->S % 4 == 0 && a->D % 4 == 0 && aligned(a->k_cache, 16) && aligned(a->v_cache, 16);
    int rc = g2i_launch(vec ? G2F_ATTN_PART : G2F_ATTN_PART_S, (unsigned)a->NH, chunks, 256, a);
    if (!rc) rc = g2i_launch(G2F_ATTN_MERGE, (unsigned)a->NH, 1, 64, a);
    return rc;
}

int g2_matvec_rows(const float *x, const void *W, int w_dtype, const float *bias,
                   const float *residual, float *y, int N, int K, int apply_gelu)
{
    NEED_READY();
    if (!x || !W || !y) return g2i_err(G2_E_ARG, "g2_matvec_rows: NULL buffer");
    if (w_dtype != G2_F32 && w_dtype != G2_F16) return g2i_err(G2_E_ARG, "g2_matvec_rows: bad dtype");
    if (N <= 0) return g2i_err(G2_E_ARG, "g2_matvec_rows: N must be positive");
    if (!aligned(x, 16) || !aligned(W, 16)) return g2i_err(G2_E_ARG, "g2_matvec_rows: x and W must be 16-byte aligned");
    if (apply_gelu) return g2i_err(G2_E_ARG, "g2_matvec_rows: GELU exists only fused with LayerNorm (model path)");
    if (residual && residual != y) return g2i_err(G2_E_ARG, "g2_matvec_rows: the residual must alias y");
    g2_rows_args a;
    memset(&a, 0, sizeof a);
    a.W = W; a.x = x; a.bias = bias; a.y = y; a.N = N; a.K = K;
    return g2i_rows_launch(residual ? G2F_ROWS_RESID_F32_64 : G2F_ROWS_STORE_F32_64, w_dtype == G2_F16, &a);
}
