/*
 * g2_attn_plan.h -- index arithmetic of the causal prompt attention on the
 * fp16 matrix cores (g2k_attn_prefill_h16, g2_kernels.hip; the grid mapping
 * also of g2k_attn_prefill_mfma): the (head, query block) of a work-group,
 * the K/V-half rows and 16-byte chunks its lanes stage into LDS, the LDS
 * element a fragment read takes and the query row of a lane.  Plain integer
 * functions, compiled into the kernel and into the CPU address check
 * (tests/native/attn_addr.cpp), so the check runs the kernel's own index
 * computations.
 */
#ifndef G2_ATTN_PLAN_H
#define G2_ATTN_PLAN_H

#if defined(__HIPCC__) || defined(__HIP__)
#define G2A_FN __host__ __device__ __forceinline__
#else
#define G2A_FN static inline
#endif

#define G2A_TILE (64 * 64) /* halves per staged array: 64 rows of 64 */
#define G2A_ARRAYS 16      /* 2 key halves x 2 stages x (Kh, Kl, Vh, Vl) */

/* Work-group w -> (head h, 64-row query block qb).  The grid is 1-D,
 * g2a_grid(P, NH) work-groups; work-group w runs on XCD w % 8 (consecutive
 * work-groups go to consecutive XCDs), so every query block of head h runs
 * on XCD h % 8, whose L2 then fetches that head's keys and values once for
 * all of them.  Work-groups with h >= NH have no work. */
G2A_FN void g2a_block(int w, int P, int *h, int *qb)
{
    const int nqb = (P + 63) / 64, k = w >> 3;
    *h = (w & 7) + 8 * (k / nqb);
    *qb = k % nqb;
}
G2A_FN unsigned g2a_grid(int P, int NH) { return 8u * (unsigned)((NH + 7) / 8) * (unsigned)((P + 63) / 64); }

/* The query row of a lane: row group rg (0..3) of the block, lane l holds
 * row 16 rg + l % 16. */
G2A_FN int g2a_query(int qb, int rg, int lane) { return qb * 64 + 16 * rg + (lane & 15); }

/* Staging of a 64-key block by LDS DMA (lane l of an instruction writes 16
 * bytes at its LDS base + 16 l): wave w4 (0..3) of a key half fills staged
 * rows 16 w4 .. 16 w4 + 15 of each array with instructions e = 0, 1 of 8
 * rows; lane -> row 16 w4 + 8 e + l / 8, slot l % 8, which holds the row's
 * chunk slot ^ (row / 2 % 8).  K rows are keys (8 dims per chunk), V rows
 * are dims (8 keys per chunk). */
/* (macros: the kernel's staging loop compiles them exactly as written in
 * place, which inlined functions did not, and the check uses the same text) */
#define G2A_STAGE_ROW(w4, e, lane) (16 * (w4) + 8 * (e) + ((lane) >> 3))
#define G2A_STAGE_CHUNK(row, lane) (((lane) & 7) ^ (((row) >> 1) & 7))
/* half-element offset of array x (0 Kh, 1 Kl, 2 Vh, 3 Vl) of stage b of key
 * half hs */
G2A_FN int g2a_array(int hs, int b, int x) { return 4 * (2 * hs + b) * G2A_TILE + x * G2A_TILE; }
/* half-element offset, within an array, of chunk c (8 halves) of staged
 * row r: the slot the staging swizzle put it in */
G2A_FN int g2a_kv_at(int r, int c) { return r * 64 + 8 * (c ^ ((r >> 1) & 7)); }

#endif
