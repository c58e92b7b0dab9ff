/*
 * g2_internal.h -- declarations shared by the C99 host files of libg2hip
 * (g2_shim.c, g2_model.c, g2_host.c).  Not part of the public ABI.
 */
#ifndef G2_INTERNAL_H
#define G2_INTERNAL_H

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "g2hip.h"
#include "g2_kargs.h"

/* Kernel table: index -> symbol name in the gfx950 code object. */
#define G2_KERNEL_LIST(X)                                                     \
    X(MVKN_F32, "g2k_mvkn_f32") X(MVKN_F32_S, "g2k_mvkn_f32_s")               \
    X(MVKN_F16, "g2k_mvkn_f16") X(MVKN_F16_S, "g2k_mvkn_f16_s")               \
    X(MVSK_F32, "g2k_mvsk_f32") X(MVSK_F16, "g2k_mvsk_f16")                   \
    X(REDUCE, "g2k_reduce") X(LAYERNORM, "g2k_layernorm")                     \
    X(ADD, "g2k_add") X(GELU, "g2k_gelu")                                     \
    X(EMBED_F32, "g2k_embed_f32") X(EMBED_F16, "g2k_embed_f16")               \
    X(SPLIT_KV, "g2k_split_kv") X(ATTN_SCORES, "g2k_attn_scores")             \
    X(ATTN_SOFTMAX, "g2k_attn_softmax") X(ATTN_OUT, "g2k_attn_out")           \
    X(ATTN_1Q, "g2k_attn_1q")                                                 \
    X(ROWS_F32_STORE, "g2k_rows_f32_store")                                   \
    X(ROWS_F16_STORE, "g2k_rows_f16_store")                                   \
    X(ROWS_F32_LN_STORE, "g2k_rows_f32_ln_store")                             \
    X(ROWS_F16_LN_STORE, "g2k_rows_f16_ln_store")                             \
    X(ROWS_F32_LN_QKV, "g2k_rows_f32_ln_qkv")                                 \
    X(ROWS_F16_LN_QKV, "g2k_rows_f16_ln_qkv")                                 \
    X(ROWS_F32_RESID, "g2k_rows_f32_resid")                                   \
    X(ROWS_F16_RESID, "g2k_rows_f16_resid")                                   \
    X(ROWS_F32_LN_GELU, "g2k_rows_f32_ln_gelu")                               \
    X(ROWS_F16_LN_GELU, "g2k_rows_f16_ln_gelu")                               \
    X(ROWS_F32_LN_ARGMAX, "g2k_rows_f32_ln_argmax")                           \
    X(ROWS_F16_LN_ARGMAX, "g2k_rows_f16_ln_argmax")                           \
    X(GEMM_KN_F32, "g2k_gemm_kn_f32") X(GEMM_KN_F16, "g2k_gemm_kn_f16")       \
    X(GEMM_NK_F32_STORE, "g2k_gemm_nk_f32_store")                             \
    X(GEMM_NK_F16_STORE, "g2k_gemm_nk_f16_store")                             \
    X(GEMM_NK_F32_GELU, "g2k_gemm_nk_f32_gelu")                               \
    X(GEMM_NK_F16_GELU, "g2k_gemm_nk_f16_gelu")                               \
    X(GEMM_NK_F32_RESID, "g2k_gemm_nk_f32_resid")                             \
    X(GEMM_NK_F16_RESID, "g2k_gemm_nk_f16_resid")                             \
    X(GEMM_NK_F32_QKV, "g2k_gemm_nk_f32_qkv")                                 \
    X(GEMM_NK_F16_QKV, "g2k_gemm_nk_f16_qkv")                                 \
    X(ATTN_PREFILL, "g2k_attn_prefill")

#define G2_ENUM_ENTRY(id, name) G2F_##id,
enum { G2_KERNEL_LIST(G2_ENUM_ENTRY) G2F_COUNT };
#undef G2_ENUM_ENTRY

/* Rows per work-group of the packed matvec kernels (4 waves x 2 rows). */
#define G2_ROWS_PER_WG 8
/* Largest K the packed matvec accepts (its LDS input vector). */
#define G2_ROWS_MAXK 6400
/* Key chunk of the single-query attention kernel and chunks per head. */
#define G2_ATTN_CHUNK 64
#define G2_ATTN_MAX_CHUNKS (G2_KV_MAX_SEQ / G2_ATTN_CHUNK)

/* error reporting */
int g2i_err(int code, const char *fmt, ...);
int g2i_hip(hipError_t e, const char *what);

/* runtime state owned by g2_shim.c */
int g2i_ready(void);
hipStream_t g2i_stream(void);
int g2i_launch(int fid, unsigned gx, unsigned gy, unsigned bx, void *args);
int g2i_device_alloc(void **p, size_t bytes);

/* host helpers (g2_host.c) */
void g2i_f32_to_f16(uint16_t *dst, const float *src, size_t n);

#endif /* G2_INTERNAL_H */
