/*
 * g2_gemm_plan.h -- index arithmetic of the 128x128 fp16 prefill GEMM
 * (g2k_hgemm2_*, g2_kernels.hip) and the host's choice of its split-K
 * slices (g2_model.c): the tile a work-group computes, the K steps of its
 * slice, the rows and 16-byte chunks its lanes stream into LDS, the LDS
 * slots its fragment reads take and the output element each accumulator
 * value is.  Plain integer functions, compiled into the kernel, the host
 * and the CPU address check (tests/native/gemm_addr.cpp), so the check runs
 * the kernel's own index computations.
 */
#ifndef G2_GEMM_PLAN_H
#define G2_GEMM_PLAN_H

#if defined(__HIPCC__) || defined(__HIP__)
#define G2H_FN __host__ __device__ __forceinline__
#else
#define G2H_FN static inline
#endif

#define G2H_BM 128 /* tile rows (activations) */
#define G2H_BN 128 /* tile columns (weight rows) */
#define G2H_BK 64  /* K step, fp16 elements: a staged row is 128 bytes, 8 chunks */
#define G2H_NS 3   /* LDS stages (a three-step ring) */
#define G2H_TB (G2H_BM * G2H_BK * 2)  /* bytes of one staged 128 x 64 tile */
#define G2H_STAGE (3 * G2H_TB)        /* a_hi, a_lo, weights: 48 KB */
#define G2H_WAVES 16                  /* 4 x 4 waves of 32 x 32 outputs */

/* The tile of work-group w.  The grid is 1-D per K slice, g2h_grid(M, N)
 * work-groups; work-group w runs on XCD w % 8 (consecutive work-groups go
 * to consecutive XCDs), so w -> (column block 8 (s / nmb) + w % 8, row
 * block s % nmb), s = w / 8, puts all row blocks of a column block on one
 * XCD, whose L2 then fetches that weight block once.  Column blocks past
 * the last (the grid is padded to a multiple of 8) have no work (on = 0). */
typedef struct {
    int mb, nb, m0, n0, on;
} g2h_tile;

G2H_FN g2h_tile g2h_tile_of(int w, int M, int N)
{
    g2h_tile t;
    const int nmb = (M + G2H_BM - 1) / G2H_BM, nnb = (N + G2H_BN - 1) / G2H_BN;
    const int sw = w >> 3;
    t.nb = 8 * (sw / nmb) + (w & 7);
    t.mb = sw % nmb;
    t.on = t.nb < nnb;
    t.m0 = t.mb * G2H_BM;
    t.n0 = t.nb * G2H_BN;
    return t;
}

/* work-groups per K slice: 8 * ceil(column blocks / 8) * row blocks */
G2H_FN unsigned g2h_grid(int M, int N)
{
    const unsigned nnb = (unsigned)(N + G2H_BN - 1) / G2H_BN, nmb = (unsigned)(M + G2H_BM - 1) / G2H_BM;
    return 8u * ((nnb + 7u) / 8u) * nmb;
}

/* First K step of slice z of ks over nkt steps (slice z is [start(z),
 * start(z + 1)); slices differ by at most one step). */
G2H_FN int g2h_slice_start(int nkt, int z, int ks) { return (int)(((long)nkt * z) / ks); }

/* Tile loads: per step each wave fills rows 8 w .. 8 w + 7 of each staged
 * tile with one 16-byte-per-lane LDS-DMA instruction (lane l writes 16
 * bytes at the instruction's LDS base + 16 l): lane -> row l / 8 and LDS
 * slot l % 8, which holds the row's global chunk slot ^ (row / 2 % 8). */
G2H_FN int g2h_load_row(int wave, int lane) { return 8 * wave + (lane >> 3); }
G2H_FN int g2h_load_chunk(int row, int lane) { return (lane & 7) ^ ((row >> 1) & 7); }
/* byte offset of a wave's load destination in stage b (a_hi; a_lo at +
 * G2H_TB, the weights at + 2 G2H_TB) */
G2H_FN int g2h_load_lds(int b, int wave) { return b * G2H_STAGE + (8 * wave) * 128; }

/* Fragment reads of v_mfma_f32_16x16x32_f16 (lane l supplies row l % 16 of
 * a 16-row block, 8 consecutive k from 8 (l / 16)): at 32-k half kk (0 or
 * 32) of a step, the 16-byte slot of a row that holds global chunk (kk + 8
 * (l / 16)) / 8.  A fragment's 16 rows start at a multiple of 16, so a
 * row's (row / 2 % 8) is (l % 16) / 2 and the slot is the same for every
 * block a lane reads. */
G2H_FN int g2h_frag_slot(int kk, int lane) { return (((kk + 8 * (lane >> 4)) >> 3) ^ ((lane & 15) >> 1)) << 4; }
/* the row of block i (0, 1) of wave row wm (a_hi, a_lo; the weights take
 * wave column wn the same way) */
G2H_FN int g2h_frag_row(int w4, int i, int lane) { return w4 * 32 + i * 16 + (lane & 15); }

/* Output element of accumulator value q (0..3) of block (i, j) of wave
 * (wm, wn): row m0 + 32 wm + 16 i + 4 (l / 16) + q, column n0 + 32 wn + 16 j
 * + l % 16 (the v_mfma_f32_16x16x32_f16 result layout). */
G2H_FN int g2h_out_row(int m0, int wm, int i, int lane, int q) { return m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + q; }
G2H_FN int g2h_out_col(int n0, int wn, int j, int lane) { return n0 + wn * 32 + j * 16 + (lane & 15); }

/* The host's split-K choice: the largest slice count ks <= maxk with tiles
 * x ks within the CUs (all work-groups resident at once, one per CU: each
 * takes 144 KB of LDS), at least one K step per slice and ks M N floats
 * within the slice buffer (cap); 1 when none (the GEMM runs whole). */
G2H_FN int g2h_slices(int M, int N, int K, int cus, int maxk, long cap)
{
    const long tiles = (long)((N + G2H_BN - 1) / G2H_BN) * ((M + G2H_BM - 1) / G2H_BM);
    for (int k = maxk; k > 1; --k)
        if (tiles * k <= cus && k <= K / G2H_BK && (long)k * M * N <= cap) return k;
    return 1;
}

#endif
