/*
 * g2_step_plan.h -- index arithmetic of the persistent decode-step kernel
 * (g2_step.hip): which rows and 16-byte chunks of each packed matrix a
 * work-group and lane load, and which KV-cache entries an attention unit
 * reads.  Plain integer functions, compiled both into the kernel and into
 * the CPU address check (tests/native/step_addr.cpp), so the check runs the
 * kernel's own address computations.
 */
#ifndef G2_STEP_PLAN_H
#define G2_STEP_PLAN_H

#include "g2_kargs.h"

#if defined(__HIPCC__) || defined(__HIP__)
#define G2P_FN __host__ __device__ __forceinline__
#else
#define G2P_FN static inline
#endif

#define G2P_NW (G2_STEP_THREADS / 64) /* waves per work-group */
#define G2P_SEGC 256                  /* chunks per (row, segment) unit: 64 lanes x 4 */

G2P_FN int g2p_min(int a, int b) { return a < b ? a : b; }

/* A work-group's share of one packed matrix W[N,K] (output-major, K / VE
 * 16-byte chunks per row of VE elements each): rows [r0, r0 + nrows), split
 * evenly over the nwg work-groups; each row in nseg (1, 2, 4 or 8: a divisor
 * of the wave count) segments of SL <= 256 chunks; a (row, segment) unit is
 * one wave's job, 64 lanes x up to 4 chunks. */
typedef struct {
    int C, nseg, lseg, SL, r0, nrows, nunits; /* nseg = 1 << lseg */
    /* the segments end 1..16 chunks into slot 3 (192 < SL <= 208): with four
     * units per wave, slot 3 of all four is packed into one register (lane l
     * holding chunk 192 + l % 16 of unit l / 16), see g2p_tail_chunk */
    int tail;
} g2p_rows;

G2P_FN g2p_rows g2p_rows_plan(int N, int K, int VE, long wg, long nwg)
{
    g2p_rows p;
    p.C = K / VE;
    const int need = (p.C + G2P_SEGC - 1) / G2P_SEGC;
    p.lseg = need <= 1 ? 0 : (need <= 2 ? 1 : (need <= 4 ? 2 : 3));
    p.nseg = 1 << p.lseg;
    p.SL = (p.C + p.nseg - 1) / p.nseg;
    p.r0 = (int)(((long)N * wg) / nwg);
    p.nrows = (int)(((long)N * (wg + 1)) / nwg) - p.r0;
    p.nunits = p.nrows * p.nseg;
    p.tail = p.SL > 3 * 64 && p.SL <= 3 * 64 + 16;
    return p;
}

/* The proj rows go to the work-groups that merge no attention head (wg >=
 * NH, of which the host admits at least one): a merging work-group issues
 * its fc rows after its merge, and its O fetch then completes only behind
 * them, so proj rows of its own would be the last X1 rows to arrive.  A
 * merging work-group gets no rows (nrows = nunits = 0). */
G2P_FN g2p_rows g2p_proj_plan(int E, int VE, int NH, long wg, long nwg)
{
    if (wg < NH) {
        g2p_rows p = g2p_rows_plan(E, E, VE, 0, nwg - NH);
        p.nrows = 0;
        p.nunits = 0;
        return p;
    }
    return g2p_rows_plan(E, E, VE, wg - NH, nwg - NH);
}

/* The row plans of work-group wg of nwg, in the order of the step kernel's
 * per-work-group table (qkv, proj, fc, fc2, lm_head).  The host builds the
 * table with this function; the kernel reads a plan from it when a phase
 * needs it, so no plan stays in scalar registers across the layers. */
enum { G2P_SH_QKV, G2P_SH_PROJ, G2P_SH_FC, G2P_SH_FC2, G2P_SH_LM, G2P_NSHARES };
G2P_FN void g2p_shares(g2p_rows *s, int E, int NH, int F, int V, int VE, long wg, long nwg)
{
    s[G2P_SH_QKV] = g2p_rows_plan(3 * E, E, VE, wg, nwg);
    s[G2P_SH_PROJ] = g2p_proj_plan(E, VE, NH, wg, nwg); /* none for a head-merging work-group */
    s[G2P_SH_FC] = g2p_rows_plan(F, E, VE, wg, nwg);
    s[G2P_SH_FC2] = g2p_rows_plan(E, F, VE, wg, nwg);
    s[G2P_SH_LM] = g2p_rows_plan(V, E, VE, wg, nwg);
}

/* Unit j of a register set of UM units per wave, for the batch `batch` of
 * the share, as loaded by wave `wave`: unit u = batch*NW*UM + wave + NW*j,
 * its row's first chunk (base = row * C) and its column chunks [c0, clast].
 * Every load is unconditional: a unit past the share (uv = 0) reads chunk 0
 * of the share's first row with every lane. */
typedef struct {
    long base;
    int c0, clast, uv;
} g2p_unit;

G2P_FN g2p_unit g2p_unit_at(const g2p_rows *p, int UM, int batch, int wave, int j)
{
    g2p_unit a;
    const int u = batch * G2P_NW * UM + wave + G2P_NW * j;
    a.uv = u < p->nunits;
    const int row = p->r0 + (a.uv ? u >> p->lseg : 0);
    a.c0 = (a.uv ? u & (p->nseg - 1) : 0) * p->SL;
    a.clast = g2p_min(p->C, a.c0 + p->SL) - 1;
    a.base = (long)row * p->C;
    return a;
}

/* The chunk (row * C + column chunk) that lane `lane` loads into slot i of
 * unit a: a lane past the segment's end reads the segment's last chunk
 * (which the same instruction fetches anyway). */
G2P_FN long g2p_unit_chunk(const g2p_unit *a, int lane, int i)
{
    return a->base + (a->uv ? g2p_min(a->c0 + lane + 64 * i, a->clast) : 0);
}

/* Packed slot 3 of a tail plan (four units per wave): the chunk lane
 * `lane` loads for it, chunk 192 + lane % 16 of the segment of unit lane /
 * 16, clamped into the segment like g2p_unit_chunk (a unit past the share
 * reads chunk 0 of the share's first row). */
G2P_FN long g2p_tail_chunk(const g2p_rows *p, int batch, int wave, int lane)
{
    const g2p_unit un = g2p_unit_at(p, 4, batch, wave, lane >> 4);
    return un.base + (un.uv ? g2p_min(un.c0 + 3 * 64 + (lane & 15), un.clast) : 0);
}

/* its x: chunk 192 + lane % 16 of the wave's segment (zero past the
 * segment's end, which cancels the clamped weight chunk) */
G2P_FN int g2p_tail_x(const g2p_rows *p, int VE, int wave, int lane)
{
    return (wave & (p->nseg - 1)) * (G2P_SEGC * VE) + 4 * (3 * 64 + (lane & 15));
}

/* The input chunk lane `lane` of wave `wave` multiplies in slot i of the
 * dot products (every unit of a wave has segment wave % nseg); -1 when the
 * slot lies past the segment (its x is zero).  The kernel reads x at
 * g2p_dot_x; the CPU address check uses this to confirm that the two agree
 * with where the fetches write the input (g2p_x_slot). */
G2P_FN int g2p_dot_chunk(const g2p_rows *p, int wave, int lane, int i)
{
    const int c0 = (wave & (p->nseg - 1)) * p->SL;
    const int c1 = g2p_min(p->C, c0 + p->SL);
    const int cc = c0 + lane + 64 * i;
    return cc < c1 ? cc : -1;
}

/* LDS layout of a matrix input for the dot products: the K input values
 * in the share's segments of SL chunks (VE values each), segment s at
 * floats [s * G2P_SEGC * VE, s * G2P_SEGC * VE + SL * VE) and zeros after it
 * up to the next segment, so a lane's x chunk (segment start + lane + 64 i,
 * i < 4) needs no bound: past the segment's end it reads zeros, which
 * cancel the clamped weight chunk loaded there.  K = n_embd inputs (qkv,
 * proj, fc, lm_head) and K = ffn inputs (fc2) have buffers of their own, so
 * neither layout's data lands in the other's zeros. */
#define G2P_XE_FLOATS 2048 /* K = n_embd: up to 2 segments of 256 chunks of 4, or 1 of 8 */
#define G2P_XF_FLOATS 8192 /* K = ffn: up to 8 segments of 256 chunks of 4, or 4 of 8 */

/* Within a segment, chunk c's values are 16-byte quads at 4 c: for VE = 4
 * the chunk itself, for VE = 8 its first four values in one plane of 256
 * quads and its last four at the same place of a second plane (so the 16-byte
 * reads of consecutive lanes, which take consecutive chunks, are
 * consecutive: no bank conflicts).  The position of value e (< VE) of the
 * chunk whose first value is at x: */
G2P_FN int g2p_x_elem(int x, int VE, int e)
{
    return VE == 8 ? x + (e >> 2) * (G2P_SEGC * 4) + (e & 3) : x + e;
}

/* the padded position of input value k */
G2P_FN int g2p_x_slot(const g2p_rows *p, int VE, int k)
{
    const int seg = p->SL * VE, off = k % seg;
    return (k / seg) * (G2P_SEGC * VE) + g2p_x_elem(4 * (off / VE), VE, off % VE);
}

/* the first x value lane `lane` of wave `wave` multiplies in slot i (the
 * others at g2p_x_elem) */
G2P_FN int g2p_dot_x(const g2p_rows *p, int VE, int wave, int lane, int i)
{
    return (wave & (p->nseg - 1)) * (G2P_SEGC * VE) + 4 * (lane + 64 * i);
}

/* Whether every four-unit plan of a model (qkv, fc and lm_head with K =
 * n_embd, fc2 with K = ffn; proj runs one unit per wave) is a tail plan, so
 * the step kernel's tail form applies to all of them. */
G2P_FN int g2p_step_tail(int E, int F, int VE)
{
    return g2p_rows_plan(1, E, VE, 0, 1).tail && g2p_rows_plan(1, F, VE, 0, 1).tail;
}

/* GPT-2 model shapes the step kernel is also compiled for, with the sizes
 * and the plans' per-matrix fields folded at compile time (id 1..4: small,
 * medium, large, XL: n_embd 768, 1024, 1280, 1600, ffn 4 n_embd, 64-dim
 * heads, vocabulary 50257); id 0: sizes read from the kernel arguments. */
#define G2P_SHAPE_E(id) ((id) == 1 ? 768 : (id) == 2 ? 1024 : (id) == 3 ? 1280 : (id) == 4 ? 1600 : 0)
#define G2P_SHAPE_F(id) (4 * G2P_SHAPE_E(id))
#define G2P_SHAPE_NH(id) (G2P_SHAPE_E(id) / 64)
#define G2P_SHAPE_V 50257
#define G2P_SHAPE_XL 4
/* ... and for a grid of 256 work-groups (one per CU of an MI355X): their
 * row plans are computed in the kernel from these constants */
#define G2P_SHAPE_WGS 256
G2P_FN int g2p_step_shape(int E, int F, int NH, int V, int nwg)
{
    if (nwg != G2P_SHAPE_WGS) return 0;
    for (int id = 1; id <= 4; ++id)
        if (E == G2P_SHAPE_E(id) && F == G2P_SHAPE_F(id) && NH == G2P_SHAPE_NH(id) && V == G2P_SHAPE_V) return id;
    return 0;
}

/* Attention unit (head h, 64-position chunk ch) by the 256 threads of one
 * half of a work-group, thread t: the K-cache floats it loads are
 * koff + d*S .. + 3 for d < 4 (transposed cache [E][S]: dims 4dg..4dg+3 of
 * the head at positions j0+4pq..+3), the V-cache floats voff[e] .. + 3 for
 * e < 4 (cache [S][E]: position j0+4jg+e, dims 4d4..+3).  A half without a
 * unit (on = 0) points every lane at the caches' first 16 bytes. */
G2P_FN void g2p_attn_offsets(int t, int on, int h, int ch, int E, int S, long *koff, long *voff)
{
    const int j0 = ch * 64;
    const int pq = t & 15, dg = t >> 4, jk = j0 + 4 * pq;
    const int d4 = t & 15, jg = t >> 4;
    *koff = on ? (long)(h * 64 + 4 * dg) * S + jk : 0;
    for (int e = 0; e < 4; ++e) {
        const int jj = j0 + 4 * jg + e;
        voff[e] = on ? (long)jj * E + h * 64 + 4 * d4 : 0;
    }
}

/* Whether the step kernel can run a model of n_embd E (NH heads of 64),
 * ffn F and vocabulary V with VE weight elements per 16-byte chunk on a grid
 * of nwg work-groups: E and F within its LDS buffers, whole chunks, and for
 * every matrix at most G2_STEP_MAXUNITS (row, segment) units per work-group
 * (hence at most that many rows: one epilogue thread per row) and at most 8
 * segments per row.  Returns NULL if it can, else the reason. */
G2P_FN const char *g2p_step_refusal(int E, int NH, int F, int V, int VE, int nwg)
{
    if (nwg <= 0 || nwg > G2_STEP_THREADS) return "no step grid";
    if (E > G2_STEP_MAXE || F > G2_STEP_MAXF) return "n_embd or ffn above the step kernel's ceilings";
    if (E % VE || F % VE || E != 64 * NH) return "sizes not multiples of the weight chunk or head dim not 64";
    if (nwg <= NH) return "no work-group left for the proj rows beside the head merges";
    /* rows, K and the work-groups sharing the rows (proj: those merging no head) */
    const int dims[5][3] = { { 3 * E, E, nwg }, { E, E, nwg - NH }, { F, E, nwg }, { E, F, nwg }, { V, E, nwg } };
    for (int i = 0; i < 5; ++i) {
        const int C = dims[i][1] / VE, need = (C + G2P_SEGC - 1) / G2P_SEGC;
        if (need > 8) return "a matrix row exceeds 8 segments";
        const int nseg = need <= 1 ? 1 : (need <= 2 ? 2 : (need <= 4 ? 4 : 8));
        if ((long)((dims[i][0] + dims[i][2] - 1) / dims[i][2]) * nseg > G2_STEP_MAXUNITS)
            return "a matrix exceeds the units per work-group";
        if ((long)nseg * G2P_SEGC * VE > (i == 3 ? G2P_XF_FLOATS : G2P_XE_FLOATS))
            return "a matrix input exceeds its padded LDS buffer";
    }
    return 0;
}

/* Attention unit u of a layer: work-group, half and round it runs in
 * (unit u -> work-group u % nwg, half (u / nwg) % 2, round u / (2 nwg)). */
G2P_FN int g2p_attn_unit(int wg, int nwg, int round, int half) { return wg + nwg * (2 * round + half); }

#endif /* G2_STEP_PLAN_H */
