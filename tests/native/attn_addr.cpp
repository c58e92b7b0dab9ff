/*
 * CPU check of the prompt attention's index arithmetic (g2k_attn_prefill_h16),
 * which lives in gpt2-opencl-1.1_amd/csrc/g2_attn_plan.h and is compiled
 * here unchanged.  For one prompt length P and head count NH (n_embd E =
 * 64 NH, cache length S = 1024) it walks every work-group of the launch
 * (g2a_grid), both key halves, every wave and lane, checking:
 *   - the working work-groups cover every (head, query block) exactly once;
 *   - every staging load of every key block a half takes reads inside the
 *     K halves [S][E] and the transposed V halves [E][S] (positions < S)
 *     and writes inside its own stage of the LDS arrays;
 *   - the staging fills each row's 8 slots exactly once, and every
 *     fragment read finds the row and 16-byte chunk its product needs;
 *   - the query loads stay inside the prompt's rows of q [P][E], and the
 *     outputs [P][E] are each written exactly once.
 *
 * Usage: attn_addr P NH [plant]
 *   plant=1 stages one key block too far, plant=3 lets a helper take one key
 *   block of its block's own work-group, plant=2 reads the fragments with a
 *   4-slot instead of an 8-slot swizzle (planted mistakes the check must
 *   catch).
 * Exit status 0: all checks pass; 1: a check failed (first failure
 * printed); 2: bad arguments.
 */
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "g2_attn_plan.h"

static int plant = 0;
static long fails = 0;

#define FAIL(...)                                                                                                  \
    do {                                                                                                           \
        if (fails++ == 0) {                                                                                        \
            std::printf(__VA_ARGS__);                                                                              \
            std::printf("\n");                                                                                     \
        }                                                                                                          \
    } while (0)

static int kv_at(int r, int c)
{
    return plant == 2 ? r * 64 + 8 * (c ^ ((r >> 1) & 3)) : g2a_kv_at(r, c);
}

int main(int argc, char **argv)
{
    if (argc < 3) {
        std::fprintf(stderr, "usage: attn_addr P NH [plant]\n");
        return 2;
    }
    const int P = std::atoi(argv[1]), NH = std::atoi(argv[2]);
    plant = argc > 3 ? std::atoi(argv[3]) : 0;
    const int S = 1024, E = 64 * NH;
    if (P < 1 || P > S - 1 || NH < 1) return 2;
    const int nqb = (P + 63) / 64;
    const unsigned grid = g2a_grid(P, NH);
    const long kv_elems = (long)S * E, lds_halves = (long)G2A_ARRAYS * G2A_TILE;

    /* work-groups */
    std::vector<int> seen((size_t)NH * nqb, 0);
    for (unsigned w = 0; w < grid; ++w) {
        int h, qb;
        g2a_block((int)w, P, NH, &h, &qb);
        if (h >= NH || qb * 64 >= P) continue;
        if (h < 0 || qb < 0 || qb >= nqb) {
            FAIL("work-group %u: head %d block %d outside the launch", w, h, qb);
            continue;
        }
        seen[(size_t)h * nqb + qb]++;
    }
    for (int h = 0; h < NH; ++h)
        for (int qb = 0; qb < nqb; ++qb)
            if (seen[(size_t)h * nqb + qb] != 1) FAIL("head %d block %d taken %d times", h, qb, seen[(size_t)h * nqb + qb]);

    /* staging, placement, fragment reads, queries and outputs; the idle
     * work-groups' helper roles (g2a_help_plan), as the kernel takes them */
    const g2a_help hp = g2a_help_plan(P, NH);
    std::vector<int> slot_chunk(64 * 8), slot_hits(64 * 8), out_hits((size_t)P * E, 0);
    std::vector<int> kcover((size_t)NH * nqb * nqb, 0), slot_w(hp.nslots + 1, 0), slot_r(hp.nslots + 1, 0);
    const long slot_bytes = (long)G2A_HELP_MAX_SLOTS * G2A_HELP_SLOT_BYTES;
    if (hp.on && hp.nslots > G2A_HELP_MAX_SLOTS) FAIL("%d helper slots, the buffer holds %d", hp.nslots, G2A_HELP_MAX_SLOTS);
    for (unsigned w = 0; w < grid && !fails; ++w) {
        int h, qb;
        g2a_block((int)w, P, NH, &h, &qb);
        int helper = -1, kb_lo = 0, kb_hi = qb;
        if (h >= NH) {
            if (!hp.on) continue;
            helper = g2a_helper_index((int)w, P, NH, &hp);
            if (helper < 0) continue;
            g2a_helped_block(helper, P, &hp, &h, &qb);
            kb_hi = 2 * hp.nh - 1 + (plant == 3 ? 1 : 0);
            if (helper >= hp.nslots || h < 0 || h >= NH || qb < 0 || qb >= nqb) {
                FAIL("work-group %u: helper %d of head %d block %d outside the launch", w, helper, h, qb);
                continue;
            }
        } else if (hp.on && g2a_help_slot(h, qb, P, &hp) >= 0) {
            kb_lo = 2 * hp.nh;
        }
        if (qb * 64 >= P) continue;
        for (int hs = 0; hs < 2; ++hs) {
            /* the key blocks this half stages: kb_lo + hs, + 2, ... <= kb_hi (stage it & 1) */
            for (int kb = kb_lo + hs, it = 0; kb <= kb_hi; kb += 2, ++it) {
                if (kb >= 0 && kb < nqb) kcover[((size_t)h * nqb + qb) * nqb + kb]++;
                const int b = it & 1, j0 = (kb + (plant == 1 ? 1 : 0)) * 64;
                std::fill(slot_hits.begin(), slot_hits.end(), 0);
                for (int w4 = 0; w4 < 4; ++w4)
                    for (int e = 0; e < 2; ++e)
                        for (int lane = 0; lane < 64; ++lane) {
                            const int rw = G2A_STAGE_ROW(w4, e, lane), c = G2A_STAGE_CHUNK(rw, lane);
                            const long ko = (long)(j0 + rw) * E + h * 64 + 8 * c, vo = (long)(h * 64 + rw) * S + j0 + 8 * c;
                            if (j0 + rw >= S || ko < 0 || ko + 8 > kv_elems)
                                FAIL("P %d NH %d head %d block %d key block %d lane %d: K load %ld out of bounds", P, NH, h, qb, kb, lane, ko);
                            if (j0 + 8 * c + 8 > S || vo < 0 || vo + 8 > kv_elems)
                                FAIL("P %d NH %d head %d block %d key block %d lane %d: V load %ld out of bounds", P, NH, h, qb, kb, lane, vo);
                            /* instruction base: staged row 16 w4 + 8 e, 64 halves per row */
                            const long base = (long)(16 * w4 + 8 * e) * 64 + 8L * lane;
                            for (int x = 0; x < 4; ++x) {
                                const long d = g2a_array(hs, b, x) + base;
                                if (d < g2a_array(hs, b, x) || d + 8 > g2a_array(hs, b, x) + G2A_TILE || d + 8 > lds_halves)
                                    FAIL("staging destination %ld outside array %d of stage %d half %d", d, x, b, hs);
                            }
                            const int r = (int)(base / 64), slot = (int)(base % 64) / 8;
                            if (r != rw) FAIL("lane %d writes staged row %d, loads row %d", lane, r, rw);
                            slot_chunk[r * 8 + slot] = c;
                            slot_hits[r * 8 + slot]++;
                        }
                for (int k = 0; k < 64 * 8; ++k)
                    if (slot_hits[k] != 1) FAIL("staged row %d slot %d written %d times", k / 8, k % 8, slot_hits[k]);
                for (int lane = 0; lane < 64; ++lane)
                    for (int t = 0; t < 4; ++t)
                        for (int s2 = 0; s2 < 2; ++s2) {
                            const int r = 16 * t + (lane & 15), c = 4 * s2 + (lane >> 4);
                            const int at = kv_at(r, c);
                            if (at < 0 || at + 8 > G2A_TILE) {
                                FAIL("fragment read %d outside the array", at);
                                continue;
                            }
                            if (at / 64 != r || slot_chunk[r * 8 + (at % 64) / 8] != c)
                                FAIL("lane %d tile %d: reads chunk %d of row %d, needs chunk %d of row %d", lane, t,
                                     slot_chunk[(at / 64) * 8 + (at % 64) / 8], at / 64, c, r);
                        }
            }
        }
        /* a helper's slot (stored by the first key half's threads), read by
         * the helped block's work-group */
        const int slot = helper >= 0 ? helper : (kb_lo > 0 ? g2a_help_slot(h, qb, P, &hp) : -1);
        if (slot >= 0) {
            if (slot > hp.nslots) FAIL("slot %d past %d", slot, hp.nslots);
            else (helper >= 0 ? slot_w : slot_r)[slot]++;
            for (int t = 0; t < 256; ++t)
                for (int q = 0; q < 5; ++q) {
                    const long o = (long)g2a_help_vec(slot, q, t) * 16;
                    if (o < 0 || o + 16 > slot_bytes) FAIL("helper slot %d vector %d of thread %d outside the slots", slot, q, t);
                }
        }
        /* queries and outputs (the first key half's waves store; a helper
         * stores none) */
        for (int rg = 0; rg < 4; ++rg)
            for (int lane = 0; lane < 64; ++lane) {
                const int i = g2a_query(qb, rg, lane), lg = lane >> 4;
                const long q0 = (long)(i < P - 1 ? i : P - 1) * E + h * 64 + 8 * lg;
                if (q0 < 0 || q0 + 36 + 4 > (long)P * E) FAIL("query load %ld outside q [P][E]", q0);
                if (i >= P || helper >= 0) continue;
                for (int t = 0; t < 4; ++t) {
                    const long idx = (long)i * E + h * 64 + 16 * t + 4 * lg;
                    if (idx < 0 || idx + 4 > (long)P * E) {
                        FAIL("output %ld outside [P][E]", idx);
                        continue;
                    }
                    for (int d = 0; d < 4; ++d) out_hits[idx + d]++;
                }
            }
    }
    if (!fails)
        for (long k = 0; k < (long)P * E; ++k)
            if (out_hits[k] != 1) {
                FAIL("output row %ld column %ld written %d times", k / E, k % E, out_hits[k]);
                break;
            }
    /* every key block 0..qb of every query block once (between a helper and
     * the block's own work-group), every helper slot written and read once */
    for (int h = 0; h < NH && !fails; ++h)
        for (int qb = 0; qb < nqb; ++qb)
            for (int kb = 0; kb < nqb; ++kb) {
                const int c = kcover[((size_t)h * nqb + qb) * nqb + kb];
                if (c != (kb <= qb ? 1 : 0)) {
                    FAIL("head %d block %d: key block %d taken %d times", h, qb, kb, c);
                    break;
                }
            }
    if (hp.on)
        for (int j = 0; j < hp.nslots; ++j)
            if (slot_w[j] != 1 || slot_r[j] != 1) FAIL("helper slot %d written %d, read %d times", j, slot_w[j], slot_r[j]);
    if (fails) {
        std::printf("P %d NH %d: %ld failed checks\n", P, NH, fails);
        return 1;
    }
    std::printf("P %d NH %d: %u work-groups, %d helpers: ok\n", P, NH, grid, hp.on ? hp.nslots : 0);
    return 0;
}
