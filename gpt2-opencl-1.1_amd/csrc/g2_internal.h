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

#ifdef __cplusplus
extern "C" {
#endif

/* Packed-matvec kernels of one epilogue: f32/f16 twins of the four lane
 * shapes (see g2_decode.hip and rows_shape in g2_shim.c). */
#define G2_ROWS_LIST(X, E, s)                                                 \
    X(ROWS_##E##_F32_64, "g2k_rows_" s "_f32_s64")                            \
    X(ROWS_##E##_F16_64, "g2k_rows_" s "_f16_s64")                            \
    X(ROWS_##E##_F32_256R, "g2k_rows_" s "_f32_s256r")                        \
    X(ROWS_##E##_F16_256R, "g2k_rows_" s "_f16_s256r")                        \
    X(ROWS_##E##_F32_256, "g2k_rows_" s "_f32_s256")                          \
    X(ROWS_##E##_F16_256, "g2k_rows_" s "_f16_s256")                          \
    X(ROWS_##E##_F32_256X8, "g2k_rows_" s "_f32_s256x8")                      \
    X(ROWS_##E##_F16_256X8, "g2k_rows_" s "_f16_s256x8")

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
    X(ATTN_PART, "g2k_attn_part") X(ATTN_PART_S, "g2k_attn_part_s")           \
    X(ATTN_MERGE, "g2k_attn_merge") X(ARGMAX_MERGE, "g2k_argmax_merge")       \
    G2_ROWS_LIST(X, STORE, "store") G2_ROWS_LIST(X, LN_QKV, "ln_qkv")         \
    G2_ROWS_LIST(X, RESID, "resid") G2_ROWS_LIST(X, LN_GELU, "ln_gelu")       \
    G2_ROWS_LIST(X, LN_ARGMAX, "ln_argmax")                                   \
    X(GEMM_KN_F32, "g2k_gemm_kn_f32") X(GEMM_KN_F16, "g2k_gemm_kn_f16")       \
    X(GEMM_NK_F32_STORE, "g2k_gemm_nk_f32_store")                             \
    X(GEMM_NK_F16_STORE, "g2k_gemm_nk_f16_store")                             \
    X(GEMM_NK_F32_GELU, "g2k_gemm_nk_f32_gelu")                               \
    X(GEMM_NK_F16_GELU, "g2k_gemm_nk_f16_gelu")                               \
    X(GEMM_NK_F32_RESID, "g2k_gemm_nk_f32_resid")                             \
    X(GEMM_NK_F16_RESID, "g2k_gemm_nk_f16_resid")                             \
    X(GEMM_NK_F32_QKV, "g2k_gemm_nk_f32_qkv")                                 \
    X(GEMM_NK_F16_QKV, "g2k_gemm_nk_f16_qkv")                                 \
    X(STEP_F32, "g2k_step_f32") X(STEP_F16, "g2k_step_f16")                   \
    X(STEP_F32T, "g2k_step_f32_tail") X(STEP_F16T, "g2k_step_f16_tail")       \
    X(STEP_F32_TR, "g2k_step_f32_trace") X(STEP_F16_TR, "g2k_step_f16_trace") \
    X(STEP_F32T_TR, "g2k_step_f32_tail_trace")                                \
    X(STEP_F16T_TR, "g2k_step_f16_tail_trace")                                \
    X(STEP_F16TN, "g2k_step_f16_tailn")                                       \
    X(STEP_F32_E768, "g2k_step_f32_e768")                                     \
    X(STEP_F32_E1024, "g2k_step_f32_e1024")                                   \
    X(STEP_F32_E1280, "g2k_step_f32_e1280")                                   \
    X(STEP_F16_E1280, "g2k_step_f16_e1280")                                   \
    X(STEP_F16TN_TR, "g2k_step_f16_tailn_trace")                              \
    X(HGEMM_STORE, "g2k_hgemm_store") X(HGEMM_GELU, "g2k_hgemm_gelu")         \
    X(HGEMM_RESID, "g2k_hgemm_resid") X(HGEMM_QKV, "g2k_hgemm_qkv")           \
    X(ATTN_PREFILL_MFMA, "g2k_attn_prefill_mfma")                             \
    X(ATTN_PREFILL_H16, "g2k_attn_prefill_h16")                               \
    X(HGEMM_PARTIAL, "g2k_hgemm_partial") X(SPLITK_RESID, "g2k_splitk_resid") \
    X(HGEMM2_GELU, "g2k_hgemm2_gelu") X(HGEMM2_RESID, "g2k_hgemm2_resid")     \
    X(HGEMM2_QKV, "g2k_hgemm2_qkv") X(HGEMM2_PARTIAL, "g2k_hgemm2_partial")   \
    X(LAYERNORM_SPLIT, "g2k_layernorm_split") X(SPLITK_RESID_LN, "g2k_splitk_resid_ln") X(SPLITK_RESID_LN_F32, "g2k_splitk_resid_ln_f32") \
    X(SGEMM_GELU, "g2k_sgemm_gelu") X(SGEMM_RESID, "g2k_sgemm_resid")         \
    X(SGEMM_QKV, "g2k_sgemm_qkv") X(SGEMM_PARTIAL, "g2k_sgemm_partial")       \
    X(SPLITK_EPI, "g2k_splitk_epi")                                           \
    X(LN_FOLD_F32, "g2k_ln_fold_f32") X(LN_FOLD_F16, "g2k_ln_fold_f16")

#define G2_ENUM_ENTRY(id, name) G2F_##id,
enum { G2_KERNEL_LIST(G2_ENUM_ENTRY) G2F_COUNT };
#undef G2_ENUM_ENTRY

/* Largest K of the fused model's packed matvecs (GPT-2 XL ffn). */
#define G2_ROWS_MAXK 6400
/* Cap on packed-matvec work-groups (4 per CU); longer matrices grid-stride. */
#define G2_ROWS_MAX_GRID 1024
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
int g2i_launch3(int fid, unsigned gx, unsigned gy, unsigned gz, unsigned bx, void *args);
/* the fp16 prefill's K slices: its slice buffer (pf_part) holds
 * G2_PF_MAXSPLIT x 1024 x n_embd floats; the 64x64 GEMM splits K in at most
 * G2_PF_MAXSPLIT slices, the 128x128 one in at most G2_PF_BIGSPLIT (and as
 * many as the buffer holds) */
#define G2_PF_MAXSPLIT 5
#define G2_PF_BIGSPLIT 8
/* the fp32-weight prefill GEMM's split-K slices (floats; 8 MiB) and its
 * epilogue codes (g2k_sgemm_*, g2k_splitk_epi) */
#define G2_SG_PART_FLOATS ((size_t)512 * 4096)
#define G2_SG_GELU 1
#define G2_SG_RESID 2
#define G2_SG_QKV 3
#define G2_SG_GELU_SPLIT 5 /* gelu, written as fp16 halves to Ch, Cl */
/* Cooperative launch (all gx work-groups co-resident) of a 1-D grid. */
int g2i_coop_launch(int fid, unsigned gx, unsigned bx, void *args);
/* Work-groups of the persistent step kernel's grid (0: not supported). */
int g2i_step_wgs(void);
/* The code-object name of kernel fid ("" out of range). */
const char *g2i_kernel_name(int fid);
/* compute units of the device (after g2_init) */
int g2i_cus(void);
int g2i_device_alloc(void **p, size_t bytes);
/* Launch a packed-matvec kernel: fid_f32_64 is the epilogue's first table
 * entry (f32, 64-lane shape); the lane shape and grid follow from K. */
int g2i_rows_launch(int fid_f32_64, int f16, g2_rows_args *a);
/* Work-groups g2i_rows_launch uses for N rows of K (0 if K is invalid). */
unsigned g2i_rows_grid(int N, int K, int f16);
/* Single-query attention: partials over `chunks` key chunks, then merge. */
int g2i_attn_launch(g2_attn1q_args *a, unsigned chunks);

/* host helpers (g2_host.c) */
void g2i_f32_to_f16(uint16_t *dst, const float *src, size_t n);

/* Static device scratch of g2_attn_1q_noalloc (g2_noalloc.hip): the chunk
 * partials of up to 64 heads x G2_ATTN_MAX_CHUNKS chunks, 66 floats each.
 * setup resolves its address on a device (the device current); scratch
 * returns it, or NULL before setup. */
#define G2_NOALLOC_SCRATCH_FLOATS (64 * G2_ATTN_MAX_CHUNKS * 66)
int g2i_noalloc_setup(int device);
float *g2i_noalloc_scratch(int device);

#ifdef __cplusplus
}
#endif

#endif /* G2_INTERNAL_H */
