/*
 * CPU check of the 128x128 fp16 prefill GEMM's index arithmetic
 * (g2k_hgemm2_*), which lives in gpt2-opencl-1.1_amd/csrc/g2_gemm_plan.h and
 * is compiled here unchanged.  For one GEMM shape (M rows, N columns, K)
 * it takes the host's slice count (g2h_slices with the given CU count,
 * slice cap and slice-buffer floats) and walks every work-group of the
 * launch (g2h_grid per slice), every wave and lane, checking:
 *   - the slices partition the K steps, each slice non-empty;
 *   - the working work-groups (g2h_tile_of) cover every tile exactly once;
 *   - every tile load (each step the kernel issues, past the last one
 *     included, as the kernel clamps it) reads inside A's and the weights'
 *     elements and inside the work-group's K slice, and writes inside the
 *     LDS ring;
 *   - the loads fill each staged row's 8 slots exactly once, and every
 *     fragment read finds the global row and 16-byte chunk the product
 *     needs (the XOR swizzle of the loads and of the reads agree);
 *   - the accumulator values map onto the tile's 128 x 128 outputs exactly
 *     once each, and partial-slice stores stay inside [ks][M][N].
 *
 * Usage: gemm_addr M N K CUS MAXK CAP [plant]
 *   plant=1 drops the row clamp of the activation loads, plant=2 reads the
 *   fragments with a 4-slot instead of an 8-slot swizzle, plant=3 ends each
 *   slice nkt / ks steps after its start, dropping the remainder (planted
 *   mistakes the check must catch).
 * Exit status 0: all checks pass; 1: a check failed (first failure
 * printed); 2: bad arguments.
 */
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "g2_gemm_plan.h"

static int plant = 0;
static long fails = 0;

#define FAIL(...)                                                                                                  \
    do {                                                                                                           \
        if (fails++ == 0) {                                                                                        \
            std::printf(__VA_ARGS__);                                                                              \
            std::printf("\n");                                                                                     \
        }                                                                                                          \
    } while (0)

/* slice z of ks: steps [*s0, *s1) */
static void slice(int nkt, int z, int ks, int *s0, int *s1)
{
    *s0 = g2h_slice_start(nkt, z, ks);
    *s1 = plant == 3 ? *s0 + nkt / ks : g2h_slice_start(nkt, z + 1, ks);
}

int main(int argc, char **argv)
{
    if (argc < 7) {
        std::fprintf(stderr, "usage: gemm_addr M N K CUS MAXK CAP [plant]\n");
        return 2;
    }
    const int M = std::atoi(argv[1]), N = std::atoi(argv[2]), K = std::atoi(argv[3]);
    const int cus = std::atoi(argv[4]), maxk = std::atoi(argv[5]);
    const long cap = std::atol(argv[6]);
    plant = argc > 7 ? std::atoi(argv[7]) : 0;
    if (M < 1 || N < 64 || N % 64 || K < 64 || K % 64) return 2;

    const int ks = g2h_slices(M, N, K, cus, maxk, cap);
    const int nkt = K / G2H_BK;
    const int nmb = (M + G2H_BM - 1) / G2H_BM, nnb = (N + G2H_BN - 1) / G2H_BN;
    const unsigned grid = g2h_grid(M, N);
    const long lds_bytes = (long)G2H_NS * G2H_STAGE;

    /* slices */
    int prev = 0;
    for (int z = 0; z < ks; ++z) {
        int s0, s1;
        slice(nkt, z, ks, &s0, &s1);
        if (s0 != prev) FAIL("slice %d starts at step %d, previous ended at %d", z, s0, prev);
        if (s1 <= s0) FAIL("slice %d of %d is empty (%d..%d)", z, ks, s0, s1);
        prev = s1;
    }
    if (prev != nkt) FAIL("slices end at step %d of %d", prev, nkt);
    if ((long)ks * M * N > cap && ks > 1) FAIL("%d slices of %d x %d exceed the %ld-float buffer", ks, M, N, cap);

    /* tiles */
    std::vector<int> seen((size_t)nmb * nnb, 0);
    for (unsigned w = 0; w < grid; ++w) {
        const g2h_tile t = g2h_tile_of((int)w, M, N);
        if (!t.on) continue;
        if (t.mb < 0 || t.mb >= nmb || t.nb < 0 || t.nb >= nnb) {
            FAIL("work-group %u: tile (%d, %d) outside %d x %d", w, t.mb, t.nb, nmb, nnb);
            continue;
        }
        seen[(size_t)t.mb * nnb + t.nb]++;
    }
    for (int mb = 0; mb < nmb; ++mb)
        for (int nb = 0; nb < nnb; ++nb)
            if (seen[(size_t)mb * nnb + nb] != 1)
                FAIL("tile (%d, %d) taken by %d work-groups", mb, nb, seen[(size_t)mb * nnb + nb]);

    /* loads, LDS placement and fragment reads: the staged rows of one tile
     * region (a_hi; a_lo and the weights use the same rows and slots) */
    const long a_elems = (long)M * K, b_elems = (long)N * K;
    std::vector<int> slot_row(G2H_BM * 8), slot_chunk(G2H_BM * 8), slot_hits(G2H_BM * 8);
    for (unsigned w = 0; w < grid; ++w) {
        const g2h_tile t = g2h_tile_of((int)w, M, N);
        if (!t.on) continue;
        for (int z = 0; z < ks; ++z) {
            int s0 = 0, s1 = nkt;
            if (ks > 1) slice(nkt, z, ks, &s0, &s1);
            const int nk = s1 - s0, kz0 = s0 * G2H_BK;
            std::fill(slot_hits.begin(), slot_hits.end(), 0);
            for (int wave = 0; wave < G2H_WAVES; ++wave)
                for (int lane = 0; lane < 64; ++lane) {
                    const int row = g2h_load_row(wave, lane), ch = g2h_load_chunk(row, lane);
                    const int arow = plant == 1 ? t.m0 + row : (t.m0 + row < M - 1 ? t.m0 + row : M - 1);
                    const int brow = t.n0 + row < N - 1 ? t.n0 + row : N - 1;
                    /* every step the kernel issues: 0 .. nk + 2, clamped to nk - 1 */
                    for (int s = 0; s <= nk + 2; ++s) {
                        const long k = (long)(s < nk - 1 ? s : nk - 1) * G2H_BK;
                        const long ao = (long)arow * K + kz0 + 8 * ch + k, bo = (long)brow * K + kz0 + 8 * ch + k;
                        if (ao < 0 || ao + 8 > a_elems)
                            FAIL("M %d N %d K %d slice %d wg %u wave %d lane %d step %d: activation load %ld out of bounds (%ld)",
                                 M, N, K, z, w, wave, lane, s, ao, a_elems);
                        if (bo < 0 || bo + 8 > b_elems)
                            FAIL("M %d N %d K %d slice %d wg %u wave %d lane %d step %d: weight load %ld out of bounds (%ld)",
                                 M, N, K, z, w, wave, lane, s, bo, b_elems);
                        const long kin = kz0 + 8 * ch + k - (long)s0 * G2H_BK;
                        if (kin < 0 || kin + 8 > (long)nk * G2H_BK)
                            FAIL("slice %d: load at k %ld outside the slice's %d steps", z, kin, nk);
                    }
                    for (int b = 0; b < G2H_NS; ++b) {
                        const long d = g2h_load_lds(b, wave) + 16L * lane;
                        if (d < 0 || d + 2 * G2H_TB + 16 > lds_bytes) FAIL("LDS load destination %ld out of the ring", d);
                    }
                    /* within a stage: byte offset row * 128 + 16 * slot */
                    const long off = g2h_load_lds(0, wave) + 16L * lane;
                    const int r = (int)(off / 128), slot = (int)(off % 128) / 16;
                    if (r != row) FAIL("lane %d of wave %d writes staged row %d, loads row %d", lane, wave, r, row);
                    slot_row[r * 8 + slot] = row;
                    slot_chunk[r * 8 + slot] = ch;
                    slot_hits[r * 8 + slot]++;
                }
            for (int i = 0; i < G2H_BM * 8; ++i)
                if (slot_hits[i] != 1) FAIL("staged row %d slot %d written %d times", i / 8, i % 8, slot_hits[i]);
            for (int wave = 0; wave < G2H_WAVES; ++wave) {
                const int wm = wave >> 2, wn = wave & 3;
                for (int lane = 0; lane < 64; ++lane)
                    for (int kk = 0; kk < G2H_BK; kk += 32) {
                        int slot = g2h_frag_slot(kk, lane);
                        if (plant == 2) slot = (((kk + 8 * (lane >> 4)) >> 3) ^ ((lane & 15) >> 1 & 3)) << 4;
                        const int want = (kk + 8 * (lane >> 4)) >> 3;
                        for (int i = 0; i < 2; ++i)
                            for (int side = 0; side < 2; ++side) {
                                const int r = g2h_frag_row(side ? wn : wm, i, lane);
                                const long off = (long)r * 128 + slot;
                                if (off < 0 || off + 16 > G2H_TB) {
                                    FAIL("fragment read %ld outside the staged tile", off);
                                    continue;
                                }
                                const int got = slot_chunk[r * 8 + slot / 16];
                                if (slot_row[r * 8 + slot / 16] != r || got != want)
                                    FAIL("wave %d lane %d k-half %d block %d: reads chunk %d of row %d, needs chunk %d of row %d",
                                         wave, lane, kk, i, got, slot_row[r * 8 + slot / 16], want, r);
                            }
                    }
            }
            if (fails) break;
        }
        if (fails) break;
    }

    /* outputs: each of a tile's 128 x 128 elements from exactly one
     * accumulator value; partial stores inside [ks][M][N] */
    if (!fails) {
        std::vector<int> hit(G2H_BM * G2H_BN);
        for (unsigned w = 0; w < grid && !fails; ++w) {
            const g2h_tile t = g2h_tile_of((int)w, M, N);
            if (!t.on) continue;
            std::fill(hit.begin(), hit.end(), 0);
            for (int wave = 0; wave < G2H_WAVES; ++wave)
                for (int lane = 0; lane < 64; ++lane)
                    for (int i = 0; i < 2; ++i)
                        for (int j = 0; j < 2; ++j)
                            for (int q = 0; q < 4; ++q) {
                                const int m = g2h_out_row(t.m0, wave >> 2, i, lane, q), n = g2h_out_col(t.n0, wave & 3, j, lane);
                                if (m < t.m0 || m >= t.m0 + G2H_BM || n < t.n0 || n >= t.n0 + G2H_BN) {
                                    FAIL("output (%d, %d) outside tile (%d, %d)", m, n, t.m0, t.n0);
                                    continue;
                                }
                                hit[(m - t.m0) * G2H_BN + (n - t.n0)]++;
                                if (m < M && n < N) {
                                    const long p = ((long)(ks - 1) * M + m) * N + n;
                                    if (p < 0 || p >= (long)ks * M * N) FAIL("partial store %ld out of [ks][M][N]", p);
                                }
                            }
            for (int e = 0; e < G2H_BM * G2H_BN; ++e)
                if (hit[e] != 1) {
                    FAIL("tile (%d, %d): output %d, %d written %d times", t.m0, t.n0, e / G2H_BN, e % G2H_BN, hit[e]);
                    break;
                }
        }
    }
    if (fails) {
        std::printf("M %d N %d K %d: %ld failed checks (%d slices)\n", M, N, K, fails, ks);
        return 1;
    }
    std::printf("M %d N %d K %d: %d slices, %u work-groups per slice: ok\n", M, N, K, ks, grid);
    return 0;
}
