/*
 * step_addr.cpp -- CPU address check of the persistent decode-step kernel
 * (gpt2-opencl-1.1_amd/csrc/g2_step.hip).  Test infrastructure, compiled
 * with g++ by tests/test_step_addresses.py.
 *
 * For one model shape, weight element size and position, every work-group
 * and thread of the launch (G2_STEP_THREADS threads, nwg work-groups) is
 * walked through the kernel's phases, and every global address it would
 * load or store is checked against the allocation it points into:
 *   weights   qkv [3E][K], proj [E][E], fc [F][E], fc2 [E][F], lm_head [V][E]
 *             (16-byte chunks from g2_step_plan.h, the kernel's own code),
 *             biases and LayerNorm parameters, the embedding rows;
 *   KV cache  the attention units' 16-byte loads of K [E][S] and V [S][E]
 *             and the current position's K/V stores;
 *   plans     the work-group's row plans in the host's table (g2p_shares):
 *             each entry read inside the table and equal to the plan of its
 *             matrix;
 *   exchange  every tagged word read or written: q/k/v, chunk partials,
 *             the argmax words, the arrival words; every plain value
 *             stored (merged O, X1, H, X2, in the region of either tag
 *             parity, and the emptied entry of the other region) and every
 *             16-byte quad of them fetched;
 *   LDS       the dot products' x reads and the partial-sum slots; every
 *             x read inside a segment must be where the fetch wrote that
 *             chunk's input values (g2p_x_slot), every read past it a zero
 *             slot no input value is written to, and the input quads the
 *             fetches write must fit the padded buffer.
 * Prints one line of counts; exits 1 if any access is out of bounds, 3 if
 * the host refuses the shape (g2p_step_refusal: it then never launches it).
 *
 * Usage: step_addr L E NH V F VE POS NWG [plant]
 *   VE: elements per 16-byte chunk (8 fp16, 4 fp32); plant=1 replaces the
 *   clamped chunk of g2p_unit_chunk by the unclamped one, plant=2 shifts the
 *   dot products' x reads by one chunk, plant=3 swaps the fc and fc2 entries
 *   of the row-plan table (planted mistakes the check must catch).
 */
#include <cstdio>
#include <cstdlib>

#include "g2_step_plan.h"

static long n_checked, n_bad;
static const char *first_bad;

static void chk(const char *what, long lo, long hi_excl, long lim)
{
    ++n_checked;
    if (lo < 0 || hi_excl > lim) {
        if (!n_bad) {
            first_bad = what;
            fprintf(stderr, "out of bounds: %s [%ld, %ld) of %ld\n", what, lo, hi_excl, lim);
        }
        ++n_bad;
    }
}

/* a row-plan table entry must be the plan of its matrix, field for field */
static void same_plan(const char *what, const g2p_rows &t, const g2p_rows &p)
{
    const bool eq = t.C == p.C && t.nseg == p.nseg && t.lseg == p.lseg && t.SL == p.SL && t.r0 == p.r0 &&
                    t.nrows == p.nrows && t.nunits == p.nunits && t.tail == p.tail;
    if (!eq && !n_bad) fprintf(stderr, "%s: table entry differs from the plan of its matrix\n", what);
    chk(what, 0, eq ? 0 : 1, 0);
}

static int plant = 0;
/* the kernel form the host launches for this shape (g2p_step_tail) */
static int tail_form = 0;

/* load_set<UM>(batch) of a work-group: every lane's 16-byte chunk loads */
static void load_set(const char *what, const g2p_rows &p, int UM, int batch, long N, long VE)
{
    const long chunks = N * p.C; /* 16-byte chunks in the matrix */
    for (int tid = 0; tid < G2_STEP_THREADS; ++tid) {
        const int wave = tid >> 6, lane = tid & 63;
        for (int j = 0; j < UM; ++j) {
            const g2p_unit un = g2p_unit_at(&p, UM, batch, wave, j);
            for (int i = 0; i < 4; ++i) {
                long c = g2p_unit_chunk(&un, lane, i);
                if (plant == 1 && un.uv) c = un.base + un.c0 + lane + 64 * i;
                if (i == 3 && UM == 4 && tail_form) { /* the packed slot 3 */
                    c = g2p_tail_chunk(&p, batch, wave, lane);
                    const g2p_unit ut = g2p_unit_at(&p, 4, batch, wave, lane >> 4);
                    if (plant == 1 && ut.uv) c = ut.base + ut.c0 + 3 * 64 + (lane & 15);
                }
                chk(what, c, c + 1, chunks);
            }
        }
    }
    (void)VE;
}

/* whether padded slot x holds an input value (k < K): the inverse of
 * g2p_x_slot (segment, plane, chunk, value) */
static bool x_is_data(const g2p_rows &p, int VE, long K, long x)
{
    const long seg = x / ((long)G2P_SEGC * VE), off = x % ((long)G2P_SEGC * VE);
    const long plane = VE == 8 ? off / (G2P_SEGC * 4) : 0, r = off % (G2P_SEGC * 4);
    const long c = r / 4, e = 4 * plane + r % 4;
    return c < p.SL && seg * p.SL * VE + c * VE + e < K;
}

/* dot_set's LDS reads of x (K floats written to a padded buffer of xcap
 * floats) and its partial-sum writes */
static void dot_set(const char *what, const g2p_rows &p, int UM, int batch, int VE, long K, long xcap)
{
    for (long k = 0; k < K; k += 4) {
        const long x = g2p_x_slot(&p, VE, (int)k);
        chk("LDS input quad", x, x + 4, xcap);
        for (int e = 0; e < 4; ++e)
            if (!x_is_data(p, VE, K, x + e)) chk("LDS input quad outside the data slots", 0, 1, 0);
        for (int e = 0; e < 4; ++e)
            if (g2p_x_slot(&p, VE, (int)k + e) != x + e) chk("LDS input quad not contiguous", 0, 1, 0);
    }
    for (int tid = 0; tid < G2_STEP_THREADS; ++tid) {
        const int wave = tid >> 6, lane = tid & 63;
        if (batch * G2P_NW * UM + wave >= p.nunits) continue;
        for (int i = 0; i < 4; ++i) {
            const bool packed = i == 3 && UM == 4 && tail_form;
            long x = (packed ? g2p_tail_x(&p, VE, wave, lane) : g2p_dot_x(&p, VE, wave, lane, i)) + (plant == 2 ? VE : 0);
            for (int e = 0; e < VE; e += 4) chk("LDS x", g2p_x_elem((int)x, VE, e), g2p_x_elem((int)x, VE, e) + 4, xcap);
            int cc = g2p_dot_chunk(&p, wave, lane, i);
            if (packed) { /* chunk 192 + lane % 16 of the wave's segment */
                const int c0 = (wave & (p.nseg - 1)) * p.SL, c1 = g2p_min(p.C, c0 + p.SL);
                cc = c0 + 3 * 64 + (lane & 15) < c1 ? c0 + 3 * 64 + (lane & 15) : -1;
            }
            if (cc >= 0) {
                chk(what, (long)cc * VE, (long)cc * VE + VE, K);
                if (x != g2p_x_slot(&p, VE, cc * VE)) chk("LDS x slot of a chunk (not where its values are)", 0, 1, 0);
                /* the weight chunk multiplied with it is the same column */
                for (int j = 0; j < UM; ++j) {
                    const g2p_unit un = g2p_unit_at(&p, UM, batch, wave, packed ? lane >> 4 : j);
                    if (!un.uv) continue;
                    const long wc = packed ? g2p_tail_chunk(&p, batch, wave, lane) : g2p_unit_chunk(&un, lane, i);
                    if (wc - un.base != cc) chk("weight column of a product (not its x column)", 0, 1, 0);
                    if (packed) break;
                }
            } else {
                for (int e = 0; e < VE; ++e)
                    if (x_is_data(p, VE, K, g2p_x_elem((int)x, VE, e))) chk("LDS x past the segment (not a zero slot)", 0, 1, 0);
            }
        }
        for (int j = 0; j < UM; ++j) {
            const int u = batch * G2P_NW * UM + wave + G2P_NW * j;
            if (u < p.nunits) chk("LDS partial sums", u, u + 1, G2_STEP_MAXUNITS);
        }
    }
}

/* a whole matrix share as matvec<UM> runs it (batch 0 preloaded, later
 * batches loaded on demand), its bias load and the row sums */
static void matrix(const char *what, const void *bias_tag, const g2p_rows &p, int N, int K, int VE, int UM,
                   long xcap = G2P_XE_FLOATS)
{
    chk("rows per work-group", 0, p.nrows, G2_STEP_THREADS);
    for (int b = 0; b == 0 || b * G2P_NW * UM < p.nunits; ++b) {
        load_set(what, p, UM, b, N, VE);
        dot_set(what, p, UM, b, VE, K, xcap);
    }
    if (bias_tag)
        for (int tid = 0; tid < G2_STEP_THREADS; ++tid) {
            const int r = g2p_min(p.r0 + tid, N - 1);
            chk("bias", r, r + 1, N);
        }
    for (int t = 0; t < p.nrows; ++t)
        for (int s = 0; s < p.nseg; ++s) chk("LDS partial sums", (long)t * p.nseg + s, (long)t * p.nseg + s + 1,
                                             G2_STEP_MAXUNITS);
}

int main(int argc, char **argv)
{
    if (argc < 9) return 2;
    const int L = atoi(argv[1]), E = atoi(argv[2]), NH = atoi(argv[3]), V = atoi(argv[4]), F = atoi(argv[5]);
    const int VE = atoi(argv[6]), pos = atoi(argv[7]), nwg = atoi(argv[8]);
    plant = argc > 9 ? atoi(argv[9]) : 0;
    tail_form = g2p_step_tail(E, F, VE);
    const int S = G2_KV_MAX_SEQ, NT = G2_STEP_THREADS;
    const long xlayer = G2X_LAYER_WORDS(E, NH);
    const long xtotal = G2X_TOTAL_WORDS(L, E, NH, nwg);
    const long att_end = G2X_ATT(E) + (long)NH * G2_STEP_MAXCH * 66; /* end of the partials */
    const long VR = G2V_REGION(E, F), vtotal = G2V_TOTAL_FLOATS(L, E, F);
    const int T = pos + 1, nch = (T + 63) / 64;
    if (nch > G2_STEP_MAXCH) {
        fprintf(stderr, "position beyond the cache\n");
        return 1;
    }
    /* the host never launches the kernel on a shape it refuses */
    const char *why = g2p_step_refusal(E, NH, F, V, VE, nwg);
    if (why) {
        printf("refused: %s\n", why);
        return 3;
    }
    /* value region of layer l for tag parity b, and the vector offsets in it;
     * each vector ends where the next one starts */
    auto vreg = [&](int l, int b) { return (2L * l + b) * VR; };
    const long vO = G2V_O(E), vX1 = G2V_X1(E), vH = G2V_H(E), vX2 = G2V_X2(E, F);
    for (int l = 0; l < L; ++l)
        for (int b = 0; b < 2; ++b) chk("value region", vreg(l, b), vreg(l, b) + VR, vtotal);
    /* a vector fetch by 16-byte quads: [base + 4q, base + 4q + 4) for 4q < n,
     * inside [.., end); the vector must start at a multiple of 4 floats and
     * have a length that is one */
    auto quads = [&](const char *what, long base, int n, long end) {
        if ((base & 3) || (n & 3)) chk("vector of value quads", 0, 1, 0);
        for (int w = 0; w < n; w += 4) chk(what, base + w, base + w + 4, end);
    };
    /* stores of values [lo, hi) of a vector at offset off (ending at offset
     * end) of layer l's region, for either tag parity; each also empties the
     * same entries of the other region */
    auto vstore = [&](const char *what, int l, long off, long lo, long hi, long end) {
        for (int b = 0; b < 2; ++b) chk(what, vreg(l, b) + off + lo, vreg(l, b) + off + hi, vreg(l, b) + end);
    };
    long proj_rows = 0; /* rows of proj over all work-groups and layers */
    for (long wg = 0; wg < nwg; ++wg) {
        /* the work-group's row plans as the kernel reads them from the host's
         * table (g2p_shares; entries wg * G2P_NSHARES + k of a [nwg][5]
         * table), each the plan of its own matrix */
        g2p_rows shp[G2P_NSHARES];
        g2p_shares(shp, E, NH, F, V, VE, wg, nwg);
        if (plant == 3) {
            const g2p_rows t = shp[G2P_SH_FC];
            shp[G2P_SH_FC] = shp[G2P_SH_FC2];
            shp[G2P_SH_FC2] = t;
        }
        for (int k = 0; k < G2P_NSHARES; ++k)
            chk("row-plan table read", wg * G2P_NSHARES + k, wg * G2P_NSHARES + k + 1, (long)nwg * G2P_NSHARES);
        same_plan("qkv row plan", shp[G2P_SH_QKV], g2p_rows_plan(3 * E, E, VE, wg, nwg));
        same_plan("proj row plan", shp[G2P_SH_PROJ], g2p_proj_plan(E, VE, NH, wg, nwg));
        same_plan("fc row plan", shp[G2P_SH_FC], g2p_rows_plan(F, E, VE, wg, nwg));
        same_plan("fc2 row plan", shp[G2P_SH_FC2], g2p_rows_plan(E, F, VE, wg, nwg));
        same_plan("lm_head row plan", shp[G2P_SH_LM], g2p_rows_plan(V, E, VE, wg, nwg));
        /* a kernel compiled for a GPT-2 shape (g2p_step_shape) computes each
         * plan from the shape's constant sizes and the 256-work-group grid
         * instead of reading the table: its plans must be the table's (which
         * this walk checks the addresses of) */
        if (const int sh = g2p_step_shape(E, F, NH, V, nwg)) {
            const int Es = G2P_SHAPE_E(sh), Fs = G2P_SHAPE_F(sh), NHs = G2P_SHAPE_NH(sh), Vs = G2P_SHAPE_V;
            const g2p_rows c[G2P_NSHARES] = {
                g2p_rows_plan(3 * Es, Es, VE, wg, G2P_SHAPE_WGS), g2p_proj_plan(Es, VE, NHs, wg, G2P_SHAPE_WGS),
                g2p_rows_plan(Fs, Es, VE, wg, G2P_SHAPE_WGS), g2p_rows_plan(Es, Fs, VE, wg, G2P_SHAPE_WGS),
                g2p_rows_plan(Vs, Es, VE, wg, G2P_SHAPE_WGS) };
            for (int k = 0; k < G2P_NSHARES; ++k) same_plan("plan computed by a shape-compiled kernel", c[k], shp[k]);
        }
        /* embedding of the token at pos, LayerNorm parameters */
        for (int tid = 0; tid < NT; ++tid) {
            for (int d = tid; d < E; d += NT) {
                chk("wte row", (long)(V - 1) * E + d, (long)(V - 1) * E + d + 1, (long)V * E);
                chk("wpe row", (long)pos * E + d, (long)pos * E + d + 1, (long)S * E);
            }
            /* gain and bias quads; the fused fetch's own quad and quad 0 are
             * among the vector quads checked per phase */
            const int q = g2p_min(tid, E / 4 - 1);
            chk("LayerNorm parameter quad", 4L * q, 4L * q + 4, E);
            if (4 * tid < E) chk("fetched quad in LDS", 4L * tid, 4L * tid + 4, G2_STEP_MAXE);
            chk("arrival word", G2X_ARRIVE(L, xlayer, nwg) + wg, G2X_ARRIVE(L, xlayer, nwg) + wg + 1, xtotal);
        }
        for (int l = 0; l < L; ++l) {
            const long R = G2X_HEAD + (long)l * xlayer;
            /* QKV: rows, K/V cache stores at pos, q/k/v words */
            const g2p_rows &pq = shp[G2P_SH_QKV];
            matrix("qkv weights", "b", pq, 3 * E, E, VE, 4);
            for (int tid = 0; tid < NT; ++tid) {
                const int rq = g2p_min(pq.r0 + tid, 3 * E - 1);
                chk("qkv LayerNorm fold sums", rq, rq + 1, 3L * E);
            }
            for (int t = 0; t < pq.nrows; ++t) {
                const int r = pq.r0 + t;
                chk("qkv word", R + r, R + r + 1, R + G2X_ATT(E));
                if (r >= 2 * E) chk("V cache store", (long)pos * E + (r - 2 * E), (long)pos * E + (r - 2 * E) + 1, (long)S * E);
                else if (r >= E) chk("K cache store", (long)(r - E) * S + pos, (long)(r - E) * S + pos + 1, (long)E * S);
            }
            if (l > 0)
                for (int b = 0; b < 2; ++b) quads("X2 fetch", vreg(l - 1, b) + vX2, E, vreg(l - 1, b) + VR);
            /* ATTN units */
            const int nunits = NH * nch, rounds = (nunits + 2 * nwg - 1) / (2 * nwg);
            for (int rd = 0; rd < rounds; ++rd)
                for (int tid = 0; tid < NT; ++tid) {
                    const int hf = tid >> 8, t = tid & 255;
                    const int u = g2p_attn_unit((int)wg, nwg, rd, hf);
                    const int on = u < nunits;
                    const int h = on ? u / nch : 0, ch = on ? u % nch : 0;
                    long koff, voff[4];
                    g2p_attn_offsets(t, on, h, ch, E, S, &koff, voff);
                    for (int d = 0; d < 4; ++d) chk("K cache load", koff + (long)d * S, koff + (long)d * S + 4, (long)E * S);
                    for (int e = 0; e < 4; ++e) chk("V cache load", voff[e], voff[e] + 4, (long)S * E);
                    if (on && t < 96) {
                        const int part = t >> 5, d = 2 * (t & 31);
                        const long w = (part == 0 ? 0 : (part == 1 ? E : 2 * E)) + h * 64 + d;
                        chk("q/k/v word pair of a unit", R + w, R + w + 2, R + G2X_ATT(E));
                        if ((R + w) & 1) chk("q/k/v word pair at an even word", 0, 1, 0);
                    }
                    if (on && t < 66) {
                        const long pw = R + G2X_ATT(E) + ((long)h * G2_STEP_MAXCH + ch) * 66 + t;
                        chk("chunk partial word", pw, pw + 1, R + att_end);
                    }
                }
            /* MERGE of head h by work-group h */
            for (int h = (int)wg; h < NH; h += nwg) {
                const long hp = R + G2X_ATT(E) + (long)h * G2_STEP_MAXCH * 66;
                chk("merge partial reads", hp, hp + (long)nch * 66, R + att_end);
                if ((hp & 1) || ((nch * 66) & 1)) chk("merge partials as word pairs", 0, 1, 0);
                vstore("O values", l, vO, h * 64, h * 64 + 64, vX1);
            }
            /* PROJ, FC, FC2 */
            /* proj: the work-groups merging no head */
            if (wg >= NH) {
                matrix("proj weights", "b", shp[G2P_SH_PROJ], E, E, VE, 1);
                for (int b = 0; b < 2; ++b) quads("O fetch", vreg(l, b) + vO, E, vreg(l, b) + vX1);
                const g2p_rows &pp = shp[G2P_SH_PROJ];
                vstore("X1 values", l, vX1, pp.r0, pp.r0 + pp.nrows, vH);
                proj_rows += pp.nrows;
            }
            for (int b = 0; b < 2; ++b) quads("X1 fetch", vreg(l, b) + vX1, E, vreg(l, b) + vH);
            const g2p_rows &pf = shp[G2P_SH_FC];
            matrix("fc weights", "b", pf, F, E, VE, 4);
            for (int tid = 0; tid < NT; ++tid) {
                const int rf = g2p_min(pf.r0 + tid, F - 1);
                chk("fc LayerNorm fold sums", rf, rf + 1, F);
            }
            vstore("H values", l, vH, pf.r0, pf.r0 + pf.nrows, vX2);
            for (int b = 0; b < 2; ++b) quads("H fetch", vreg(l, b) + vH, F, vreg(l, b) + vX2);
            const g2p_rows &p2 = shp[G2P_SH_FC2];
            matrix("fc2 weights", "b", p2, E, F, VE, 4, G2P_XF_FLOATS);
            vstore("X2 values", l, vX2, p2.r0, p2.r0 + p2.nrows, VR);

        }
        /* LM head: X2 of the last layer, rows, logits, argmax words */
        for (int b = 0; b < 2; ++b) quads("LM X2 fetch", vreg(L - 1, b) + vX2, E, vreg(L - 1, b) + VR);
        const g2p_rows &pl = shp[G2P_SH_LM];
        matrix("lm_head weights", nullptr, pl, V, E, VE, 4);
        chk("logits", pl.r0, pl.r0 + pl.nrows, V);
        for (int tid = 0; tid < NT; ++tid) {
            const int rl = g2p_min(pl.r0 + tid, V - 1);
            chk("lm_head LayerNorm fold sums", rl, rl + 1, V);
        }
        const long AM = G2X_HEAD + (long)L * xlayer;
        chk("argmax words", AM + 2 * wg, AM + 2 * wg + 2, G2X_ARRIVE(L, xlayer, nwg));
        if (AM & 1) chk("argmax words as word pairs", 0, 1, 0);
        if (nwg > NT) chk("argmax word pairs, one per thread", 0, 1, 0);
    }
    /* the proj rows of the non-merging work-groups cover every row once */
    if (proj_rows != (long)L * E) chk("proj rows covered once", 0, 1, 0);
    printf("checked %ld accesses, %ld out of bounds%s%s\n", n_checked, n_bad, n_bad ? "; first: " : "",
           n_bad ? first_bad : "");
    return n_bad ? 1 : 0;
}
