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
 * all of them.  Work-groups with h >= NH have no work of their own (see the
 * helpers below).  Index k = the work-group's position on its XCD counts
 * down: the last head group (whose idle work-groups are the helpers) and,
 * within a head group, the last query blocks (the longest) are dispatched
 * first. */
G2A_FN unsigned g2a_grid(int P, int NH) { return 8u * (unsigned)((NH + 7) / 8) * (unsigned)((P + 63) / 64); }
G2A_FN int g2a_k(int w, int P, int NH) { return (int)(g2a_grid(P, NH) >> 3) - 1 - (w >> 3); }
G2A_FN void g2a_block(int w, int P, int NH, int *h, int *qb)
{
    const int nqb = (P + 63) / 64, k = g2a_k(w, P, NH);
    *h = (w & 7) + 8 * (k / nqb);
    *qb = k % nqb;
}

/* Helpers.  A query block qb takes (qb + 2) / 2 iterations (its key blocks
 * 0..qb, two at a time by the two key halves of the work-group), so the
 * last query blocks set the kernel's length.  When the head count is not a
 * multiple of 8 the grid has idle work-groups (h >= NH): (8 - NH % 8) per
 * query block index.  If they are enough, each of the longest query blocks
 * (those of the most iterations, n_long per head) gets one: the helper
 * runs key blocks [0, 2 nh) of it and leaves its softmax partial in slot
 * j; the block's own work-group runs key blocks [2 nh, qb] and merges the
 * partial.  nh = half the iterations, so both take about half as long,
 * below the next-longest blocks when there are at least 3 iterations.  A
 * block waits for its helper, which waits for nothing; the host uses
 * helpers only when the whole grid is resident at once (at most one
 * work-group per CU), so no helper is dispatched behind a waiting block. */
typedef struct {
    int on;     /* helpers in use */
    int nlong;  /* longest query blocks per head (the last one or two) */
    int nh;     /* iterations (pairs of key blocks) a helper runs */
    int nslots; /* helper slots = nlong * NH */
} g2a_help;

G2A_FN g2a_help g2a_help_plan(int P, int NH)
{
    g2a_help p;
    const int nqb = (P + 63) / 64;
    const int maxit = (nqb - 1 + 2) >> 1;
    p.nlong = nqb >= 2 && ((nqb - 2 + 2) >> 1) == maxit ? 2 : 1;
    p.nh = maxit >> 1;
    p.nslots = p.nlong * NH;
    const int idle = NH % 8 ? (8 - NH % 8) * nqb : 0;
    p.on = maxit >= 3 && p.nslots <= idle;
    return p;
}
/* helper index of idle work-group w (h >= NH), or -1 (past the helpers) */
G2A_FN int g2a_helper_index(int w, int P, int NH, const g2a_help *hp)
{
    const int nqb = (P + 63) / 64, x = w & 7, k = g2a_k(w, P, NH), g = (NH + 7) / 8 - 1, x0 = NH % 8;
    const int j = (k - g * nqb) * (8 - x0) + (x - x0);
    return hp->on && j < hp->nslots ? j : -1;
}
/* the (head, query block) helper j works for */
G2A_FN void g2a_helped_block(int j, int P, const g2a_help *hp, int *h, int *qb)
{
    const int nqb = (P + 63) / 64;
    *h = j / hp->nlong;
    *qb = nqb - hp->nlong + j % hp->nlong;
}
/* the helper slot of query block (h, qb), or -1 (no helper) */
G2A_FN int g2a_help_slot(int h, int qb, int P, const g2a_help *hp)
{
    const int nqb = (P + 63) / 64;
    return hp->on && qb >= nqb - hp->nlong ? h * hp->nlong + qb - (nqb - hp->nlong) : -1;
}
/* Slot j: 5 vectors of 4 floats per thread of the key half 0 (256
 * threads): vector 0 = (max, sum, 0, 0) of the thread's row, vectors 1..4 =
 * its unnormalised output tiles; vector q of thread t at (5 j + q) 256 + t
 * (16-byte units). */
#define G2A_HELP_SLOT_BYTES (5 * 256 * 16)
G2A_FN int g2a_help_vec(int j, int q, int t) { return (5 * j + q) * 256 + t; }
/* slots a buffer must hold for prompts of up to 1023 rows */
#define G2A_HELP_MAX_SLOTS (7 * 16)

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
