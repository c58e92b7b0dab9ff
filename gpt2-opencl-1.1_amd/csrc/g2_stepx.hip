/*
 * g2_stepx.hip -- the decode step as one persistent cooperative kernel,
 * tensor-parallel over the 8 XCDs of gfx950 (included by g2_kernels.hip
 * after g2_step.hip, whose exchange, wait, LayerNorm and attention helpers
 * it uses).
 *
 * Why: an MI355X is 8 XCDs of 32 CUs, each with its own L2.  A hand-off
 * between work-groups of different XCDs must go through memory (~2 us
 * per hop with 256 participants); between work-groups of one XCD it can go
 * through that XCD's L2 (~0.7 us).  The per-operator layout of
 * g2k_step_* needs six all-to-all hand-offs per layer.  Here the XCDs work
 * like the devices of a tensor-parallel group:
 *
 *   XCD x owns heads [NH*x/8, NH*(x+1)/8) and ffn rows [F*x/8, F*(x+1)/8).
 *   QKV   rows of its heads (LayerNorm of the replicated x)      -> L2
 *   ATTN  (head, 64-position chunk) units of its heads            -> L2
 *   MERGE one work-group per head                                 -> L2
 *   PROJ  partial x'_x = Wp[:, its head columns] . o_x            -> memory
 *   RED1  x' = x + b + sum_x x'_x, rows split over the XCD, every
 *         XCD computing the same sums in the same order          -> L2
 *   FC    its ffn rows of gelu(LayerNorm(x') . Wfc + b)           -> L2
 *   FC2   partial x''_x = Wfc2[:, its ffn columns] . h_x          -> memory
 *   RED2  x'' = x' + b + sum_x x''_x                              -> L2
 * so only the two partial sums per layer cross XCDs, and each of those is a
 * reduce-scatter read of 8 x 50 words per work-group.
 *
 * Each work-group reads the XCD it runs on (XCC_ID).  The dispatcher deals
 * consecutive work-groups to consecutive XCDs, starting where the previous
 * launch stopped, so work-group w is on XCD (w + k) % 8 for some k and the
 * 32 work-groups of an XCD have distinct ranks w / 8 (the host checks this
 * with a probe launch before enabling the kernel; were it violated, some
 * rows would never be produced and the bounded waits would end the step
 * with G2_ERR_STEP_TIMEOUT).
 *
 * Words meant for the same XCD are written with plain stores (they stay in
 * that L2 until the kernel ends); words for other XCDs with agent-scope
 * stores.  Readers always use agent-scope loads, which see both.
 */

namespace g2step {

/* A work-group's rows of a packed W[N, K] restricted to the column slice
 * [k0, k0 + klen): local row indices [t0, t0 + nrows) of a row list mapped
 * to matrix rows by base + (i / blk) * bstride + i % blk; each row in nseg
 * segments of SL chunks, one (row, segment) unit per wave, CPL 16-byte
 * chunks per lane (1, 2 or 4, from the slice length). */
struct xplan {
    const u32x4 *W;
    int Crow, cbase, C, cpl, nseg, SL;
    int t0, nrows, nunits;
    int base, blk, bstride;
};

template <typename WT>
__device__ __forceinline__ xplan xmake(const void *W, int K, int k0, int klen, int rows, int part, int nparts,
                                       int base, int blk, int bstride)
{
    constexpr int VE = chunk_t<WT>::V;
    xplan p;
    p.W = (const u32x4 *)W;
    p.Crow = K / VE;
    p.cbase = k0 / VE;
    p.C = klen / VE;
    p.cpl = p.C <= 64 ? 1 : (p.C <= 128 ? 2 : 4);
    const int need = (p.C + 64 * p.cpl - 1) / (64 * p.cpl);
    p.nseg = need <= 1 ? 1 : (need <= 2 ? 2 : (need <= 4 ? 4 : 8));
    p.SL = (p.C + p.nseg - 1) / p.nseg;
    p.t0 = (int)(((long)rows * part) / nparts);
    p.nrows = (int)(((long)rows * (part + 1)) / nparts) - p.t0;
    p.nunits = p.nrows * p.nseg;
    p.base = base;
    p.blk = blk > 0 ? blk : 1;
    p.bstride = bstride;
    return p;
}

__device__ __forceinline__ int xrow(const xplan &p, int t)
{
    const int i = p.t0 + t;
    return p.base + (i / p.blk) * p.bstride + i % p.blk;
}

template <int UM, int CPL>
__device__ __forceinline__ void xload_t(int tid, u32x4 (&w)[UM * CPL], const xplan &p, int batch)
{
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int j = 0; j < UM; ++j) {
        const int u = batch * NW * UM + wave + NW * j;
        const bool uv = u < p.nunits;
        const int row = xrow(p, uv ? u / p.nseg : 0);
        const int c0 = (uv ? u % p.nseg : 0) * p.SL;
        const int c1 = min(p.C, c0 + p.SL);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            /* unconditional loads keep the compiler's waits exact; the chunk
             * is clamped into the row, also for an empty slice (an XCD
             * without heads has no proj columns: c1 = 0) */
            const int cc = uv ? min(c0 + lane + 64 * i, c1 - 1) : 0;
            const int ca = max(0, min(p.cbase + cc, p.Crow - 1));
            w[j * CPL + i] = __builtin_nontemporal_load(gl(p.W) + (size_t)row * p.Crow + ca);
        }
    }
}

template <typename WT, int UM, int CPL>
__device__ __forceinline__ void xdot_t(int tid, const u32x4 (&w)[UM * CPL], const xplan &p, int batch,
                                       const float *xin, float *part)
{
    constexpr int VE = chunk_t<WT>::V;
    const int wave = tid >> 6, lane = tid & 63;
    const int c0 = (wave % p.nseg) * p.SL;
    const int c1 = min(p.C, c0 + p.SL);
    if (batch * NW * UM + wave >= p.nunits) return; /* wave-uniform */
    float xv[CPL][VE];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int cc = c0 + lane + 64 * i;
#pragma unroll
        for (int e = 0; e < VE; e += 4) {
            f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
            if (cc < c1) v = *(const f32x4 *)(xin + cc * VE + e);
            xv[i][e] = v.x; xv[i][e + 1] = v.y; xv[i][e + 2] = v.z; xv[i][e + 3] = v.w;
        }
    }
#pragma unroll
    for (int j = 0; j < UM; ++j) {
        const int u = batch * NW * UM + wave + NW * j;
        if (u >= p.nunits) break; /* wave-uniform */
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) acc += chunk_dot<WT>(w[j * CPL + i], xv[i]);
        acc = wsum(acc);
        if (lane == 0) part[u] = acc;
    }
}

/* Issue batch `batch` of a plan into a register set of S chunk slots. */
template <int S>
__device__ __forceinline__ void xload(int tid, u32x4 (&w)[S], const xplan &p, int batch)
{
    if (p.cpl == 1) xload_t<S, 1>(tid, w, p, batch);
    else if (p.cpl == 2) xload_t<S / 2, 2>(tid, w, p, batch);
    else xload_t<S / 4, 4>(tid, w, p, batch);
}

/* All units of a plan: batch 0 from the preloaded set, later batches loaded
 * into the same set on demand.  Ends with a barrier. */
template <typename WT, int S, int UM, int CPL>
__device__ __forceinline__ void xmatvec_t(int tid, u32x4 (&w)[S], const xplan &p, const float *xin, float *part)
{
    xdot_t<WT, UM, CPL>(tid, w, p, 0, xin, part);
    for (int b = 1; b * NW * UM < p.nunits; ++b) {
        xload_t<UM, CPL>(tid, w, p, b);
        xdot_t<WT, UM, CPL>(tid, w, p, b, xin, part);
    }
    __syncthreads();
}

template <typename WT, int S>
__device__ __forceinline__ void xmatvec(int tid, u32x4 (&w)[S], const xplan &p, const float *xin, float *part)
{
    if (p.cpl == 1) xmatvec_t<WT, S, S, 1>(tid, w, p, xin, part);
    else if (p.cpl == 2) xmatvec_t<WT, S, S / 2, 2>(tid, w, p, xin, part);
    else xmatvec_t<WT, S, S / 4, 4>(tid, w, p, xin, part);
}

__device__ __forceinline__ float xrow_sum(const xplan &p, const float *part, int t)
{
    float v = part[t * p.nseg];
    for (int s = 1; s < p.nseg; ++s) v += part[t * p.nseg + s];
    return v;
}

/* Reduce-scatter read of the 8 XCD partials of rows [n0, n0+nr):
 * tmp[xs*nr + t] = P[xs*E + n0 + t] once tagged (nr*8 <= NT).  Ends with a
 * barrier. */
__device__ __forceinline__ void fetch_partials(int tid, const ctx &c, const u64 *P, int E, int n0, int nr,
                                               float *tmp)
{
    const int n = G2_NXCD * nr;
    if (nr > 0 && tid < n) {
        const int w = (tid / nr) * E + n0 + tid % nr;
        u64 v[1] = {ll_get(P + w)};
        settle(c, P, v, [&](int) { return w; });
        tmp[tid] = ll_val(v[0]);
    }
    __syncthreads();
}

#define XTRACE(k)                                                                      \
    do {                                                                               \
        if (a.trace && tid == 0)                                                       \
            a.trace[(size_t)wg * G2_TRACE_STRIDE(a.L) + 24 * l + (k)] = wall_clock64(); \
    } while (0)

template <typename WT>
__device__ __forceinline__ void stepx_impl(const g2_step_args &a)
{
    __shared__ __attribute__((aligned(16))) float xin[G2_STEP_MAXF];
    __shared__ __attribute__((aligned(16))) float xres[G2_STEP_MAXE];
    __shared__ float part[G2_STEP_MAXUNITS];
    __shared__ float red[2 * NW];
    __shared__ att_lds att[2];
    __shared__ float cw[G2_STEP_MAXCH];
    __shared__ float amv[NT];
    __shared__ int ami[NT];
    __shared__ volatile int dead;
    __shared__ volatile int flag;

    constexpr int NPE = (G2_STEP_MAXE + NT - 1) / NT;
    constexpr int NPM = (G2_STEP_MAXCH * 66 + NT - 1) / NT;
    constexpr int NPH = (G2_STEP_MAXF / G2_NXCD + NT - 1) / NT;
    const int wg = blockIdx.x, nwg = gridDim.x;
    /* the XCD this work-group runs on; the dispatcher deals consecutive
     * work-groups to consecutive XCDs (from a start that varies between
     * launches), so the work-groups of one XCD have distinct w / 8 */
    const int X = (__builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11)) & 15) % G2_NXCD;
    const int r = wg / G2_NXCD, G = nwg / G2_NXCD;
    const int E = a.E, F = a.F, NH = a.NH, S = a.S, V = a.V;
    const int HX = (NH + G2_NXCD - 1) / G2_NXCD, FX = (F + G2_NXCD - 1) / G2_NXCD;
    const int hb = NH * X / G2_NXCD, nh = NH * (X + 1) / G2_NXCD - hb;
    const int fb = F * X / G2_NXCD, nf = F * (X + 1) / G2_NXCD - fb;
    const int LW = G2XL_WORDS(HX, E, FX);
    const int pos = clampi(a.state[G2S_POS], 0, S - 1);
    const int tok = clampi(a.state[G2S_TOK], 0, V - 1);
    const int ngen = a.state[G2S_NGEN], min_new = a.state[G2S_MIN_NEW];
    const unsigned seq = (unsigned)a.state[G2S_SEQ];
    ctx c;
    c.tag = seq + 1u;
    c.abort_w = a.xbuf;
    c.state = a.state;
    c.dead = (lds_flag *)&dead;
    const int T = pos + 1, nch = (T + 63) >> 6;
    u64 *Xb = a.xbuf + G2X_HEAD;
    /* rows of E this work-group reduces (and every XCD's same-rank peer) */
    const int rn0 = (int)(((long)E * r) / G), rnr = (int)(((long)E * (r + 1)) / G) - rn0;
    att_regs ar[1];

    u32x4 wa[16], wp[8];
    const G2_CONST g2_step_layer *LT = (const G2_CONST g2_step_layer *)a.layers;
    {
        const int tid = fresh_tid();
        if (tid == 0) dead = 0;
        if (a.trace && tid == 0) a.trace[(size_t)wg * G2_TRACE_STRIDE(a.L) + 24 * a.L + 4] = X;
        xload<16>(tid, wa, xmake<WT>(LT[0].qkv_w, E, 0, E, 192 * nh, r, G, hb * 64, 64 * nh, E), 0);
        xload<8>(tid, wp, xmake<WT>(LT[0].proj_w, E, hb * 64, nh * 64, E, r, G, 0, E, 0), 0);
        for (int d = tid; d < E; d += NT)
            xres[d] = ldw((const WT *)a.wte, (size_t)tok * E + d) + ldw((const WT *)a.wpe, (size_t)pos * E + d);
        __syncthreads();
    }

    for (int l = 0; l < a.L; ++l) {
        const g2_step_layer y = LT[l];
        u64 *R = Xb + (size_t)l * a.xlayer;
        u64 *LR = R + (size_t)X * LW;             /* this XCD's local region */
        u64 *PP = R + (size_t)G2_NXCD * LW;       /* proj partials [8][E]    */
        u64 *P2 = PP + (size_t)G2_NXCD * E;       /* fc2 partials [8][E]     */

        /* ---- QKV of this XCD's heads */
        {
            const int tid = fresh_tid();
            XTRACE(0);
            const xplan p = xmake<WT>(y.qkv_w, E, 0, E, 192 * nh, r, G, hb * 64, 64 * nh, E);
            const ln_params<NPE> lp = ln_load<NPE>(tid, gl(y.ln1_w), gl(y.ln1_b), E);
            const float bias = gl(y.qkv_b)[xrow(p, min(tid, max(p.nrows - 1, 0)))];
            if (l > 0)
                fetch<NPE>(tid, c, Xb + (size_t)(l - 1) * a.xlayer + (size_t)X * LW + G2XL_X2(HX, E, FX), E, G,
                           xres, (lds_flag *)&flag);
            XTRACE(1);
            layernorm(tid, xres, xin, lp, E, red);
            XTRACE(11);
            xmatvec<WT, 16>(tid, wa, p, xin, part);
            XTRACE(12);
            if (tid < p.nrows) {
                const int row = xrow(p, tid);
                const float v = xrow_sum(p, part, tid) + bias;
                lx_put(LR + G2XL_QKV + p.t0 + tid, v, c.tag);
                if (row >= 2 * E) glw(y.v_cache)[(size_t)pos * E + (row - 2 * E)] = v;
                else if (row >= E) glw(y.k_cache)[(size_t)(row - E) * S + pos] = v;
            }
            XTRACE(2);
        }

        /* ---- ATTN: unit u = lh * nch + chunk, rank u % G, half */
        {
            const int tid = fresh_tid();
            const int nunits = nh * nch;
            const int rounds = (nunits + 2 * G - 1) / (2 * G);
            const int hf = tid >> 8;
            for (int rd = 0; rd < rounds; ++rd) {
                const int u = r + G * (2 * rd + hf);
                const bool on = u < nunits;
                const int lh = on ? u / nch : 0, ch = on ? u % nch : 0;
                attn_load(tid, y, ar[0], on, hb + lh, ch, pos, T, E, S);
                if (rd == 0) XTRACE(16);
                attn_chunk<true>(tid, c, a.scale, LR + G2XL_QKV, lh * 64, 64 * nh + lh * 64, 128 * nh + lh * 64,
                                 LR + G2XL_ATT(HX) + ((size_t)lh * G2_STEP_MAXCH + ch) * 66, att[hf], ar[0], on,
                                 ch, pos, T,
                                 a.trace && rd == 0 ? a.trace + (size_t)wg * G2_TRACE_STRIDE(a.L) + 24 * l + 19
                                                    : nullptr);
                __syncthreads();
            }
            XTRACE(3);
            if (r >= nh) xload<16>(tid, wa, xmake<WT>(y.fc_w, E, 0, E, nf, r, G, fb, nf, 0), 0);
        }

        /* ---- MERGE: local head lh by rank lh */
        for (int lh = r; lh < nh; lh += G) {
            const int tid = fresh_tid();
            fetch<NPM>(tid, c, LR + G2XL_ATT(HX) + (size_t)lh * G2_STEP_MAXCH * 66, nch * 66, nch, xin,
                       (lds_flag *)&flag);
            float Ls = 0.f;
            if (tid < 64) {
                const float mc = tid < nch ? xin[tid * 66] : -INFINITY;
                const float lc = tid < nch ? xin[tid * 66 + 1] : 0.f;
                const float M = wmax(mc);
                const float w = tid < nch ? expf(mc - M) : 0.f;
                Ls = wsum(lc * w);
                if (tid < nch) cw[tid] = w;
            }
            __syncthreads();
            if (tid < 64) {
                float acc = 0.f;
                for (int ch = 0; ch < nch; ++ch) acc = fmaf(xin[ch * 66 + 2 + tid], cw[ch], acc);
                lx_put(LR + G2XL_O(HX) + lh * 64 + tid, acc / Ls, c.tag);
            }
            __syncthreads();
        }
        {
            const int tid = fresh_tid();
            if (r < nh) xload<16>(tid, wa, xmake<WT>(y.fc_w, E, 0, E, nf, r, G, fb, nf, 0), 0);
            XTRACE(4);
        }

        /* ---- PROJ partial over this XCD's head columns */
        {
            const int tid = fresh_tid();
            const xplan p = xmake<WT>(y.proj_w, E, hb * 64, nh * 64, E, r, G, 0, E, 0);
            fetch<1>(tid, c, LR + G2XL_O(HX), 64 * nh, nh, xin, (lds_flag *)&flag);
            XTRACE(5);
            xmatvec<WT, 8>(tid, wp, p, xin, part);
            if (tid < p.nrows) ll_put(PP + (size_t)X * E + p.t0 + tid, xrow_sum(p, part, tid), c.tag);
            XTRACE(6);
            if (l + 1 < a.L) xload<8>(tid, wp, xmake<WT>(LT[l + 1].proj_w, E, hb * 64, nh * 64, E, r, G, 0, E, 0), 0);
        }

        /* ---- RED1: x' = (sum of partials + b) + x on this rank's rows */
        {
            const int tid = fresh_tid();
            const float bias = gl(y.proj_b)[min(rn0 + tid, E - 1)];
            fetch_partials(tid, c, PP, E, rn0, rnr, xin);
            XTRACE(17);
            if (tid < rnr) {
                float v = xin[tid];
#pragma unroll
                for (int xs = 1; xs < G2_NXCD; ++xs) v += xin[xs * rnr + tid];
                lx_put(LR + G2XL_X1(HX) + rn0 + tid, (v + bias) + xres[rn0 + tid], c.tag);
            }
            __syncthreads();
        }

        /* ---- FC rows of this XCD */
        {
            const int tid = fresh_tid();
            const xplan p = xmake<WT>(y.fc_w, E, 0, E, nf, r, G, fb, nf, 0);
            const ln_params<NPE> lp = ln_load<NPE>(tid, gl(y.ln2_w), gl(y.ln2_b), E);
            const float bias = gl(y.fc_b)[xrow(p, min(tid, max(p.nrows - 1, 0)))];
            fetch<NPE>(tid, c, LR + G2XL_X1(HX), E, G, xres, (lds_flag *)&flag);
            XTRACE(7);
            layernorm(tid, xres, xin, lp, E, red);
            XTRACE(13);
            xmatvec<WT, 16>(tid, wa, p, xin, part);
            XTRACE(14);
            if (tid < p.nrows) lx_put(LR + G2XL_H(HX, E) + p.t0 + tid, gelu_f(xrow_sum(p, part, tid) + bias), c.tag);
            XTRACE(8);
            xload<16>(tid, wa, xmake<WT>(y.fc2_w, F, fb, nf, E, r, G, 0, E, 0), 0);
            __syncthreads();
        }

        /* ---- FC2 partial over this XCD's ffn columns */
        {
            const int tid = fresh_tid();
            const xplan p = xmake<WT>(y.fc2_w, F, fb, nf, E, r, G, 0, E, 0);
            fetch<NPH>(tid, c, LR + G2XL_H(HX, E), nf, G, xin, (lds_flag *)&flag);
            XTRACE(9);
            xmatvec<WT, 16>(tid, wa, p, xin, part);
            XTRACE(15);
            if (tid < p.nrows) ll_put(P2 + (size_t)X * E + p.t0 + tid, xrow_sum(p, part, tid), c.tag);
            if (l + 1 < a.L)
                xload<16>(tid, wa, xmake<WT>(LT[l + 1].qkv_w, E, 0, E, 192 * nh, r, G, hb * 64, 64 * nh, E), 0);
            else
                xload<16>(tid, wa, xmake<WT>(a.lm_w, E, 0, E, V, wg, nwg, 0, V, 0), 0);
            XTRACE(10);
        }

        /* ---- RED2: x'' = (sum of partials + b) + x' */
        {
            const int tid = fresh_tid();
            const float bias = gl(y.fc2_b)[min(rn0 + tid, E - 1)];
            fetch_partials(tid, c, P2, E, rn0, rnr, xin);
            XTRACE(18);
            if (tid < rnr) {
                float v = xin[tid];
#pragma unroll
                for (int xs = 1; xs < G2_NXCD; ++xs) v += xin[xs * rnr + tid];
                lx_put(LR + G2XL_X2(HX, E, FX) + rn0 + tid, (v + bias) + xres[rn0 + tid], c.tag);
            }
            __syncthreads();
        }
    }

    /* ---- LM: logits over the head rows (all work-groups), first-max */
    const int tid = fresh_tid();
    const int l = a.L;
    const ln_params<NPE> lpf = ln_load<NPE>(tid, gl(a.lnf_w), gl(a.lnf_b), E);
    fetch<NPE>(tid, c, Xb + (size_t)(a.L - 1) * a.xlayer + (size_t)X * LW + G2XL_X2(HX, E, FX), E, G, xres,
               (lds_flag *)&flag);
    XTRACE(0);
    layernorm(tid, xres, xin, lpf, E, red);
    const xplan p = xmake<WT>(a.lm_w, E, 0, E, V, wg, nwg, 0, V, 0);
    xmatvec<WT, 16>(tid, wa, p, xin, part);
    const int masked = ngen < min_new ? G2_EOS_ID : -1;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (tid < p.nrows) {
        const int row = xrow(p, tid);
        const float v = xrow_sum(p, part, tid);
        glw(a.logits)[row] = v;
        bv = row == masked ? -1e30f : v;
        bi = row;
    }
    blk_argmax(tid, bv, bi, amv, ami);
    u64 *AM = Xb + (size_t)a.L * a.xlayer;
    if (tid == 0) {
        ll_put(AM + 2 * wg, amv[0], c.tag);
        ll_put(AM + 2 * wg + 1, __int_as_float(ami[0]), c.tag);
    }
    XTRACE(1);
    if (wg != 0) return;

    /* ---- greedy pick (g2k_argmax_merge with advance) */
    __syncthreads();
    fetch<2>(tid, c, AM, 2 * nwg, nwg, xin, (lds_flag *)&flag);
    bv = -INFINITY;
    bi = 0x7fffffff;
    for (int b = tid; b < nwg; b += NT) {
        const float v = xin[2 * b];
        const int i = __float_as_int(xin[2 * b + 1]);
        if (am_better2(v, i, bv, bi)) { bv = v; bi = i; }
    }
    blk_argmax(tid, bv, bi, amv, ami);
    if (tid == 0) {
        const int tk = (ami[0] >= 0 && ami[0] < V) ? ami[0] : 0;
        const int ng = clampi(ngen, 0, G2S_WORDS - G2S_IDS - 1);
        a.state[G2S_IDS + ng] = tk;
        a.state[G2S_TOK] = tk;
        a.state[G2S_NGEN] = ng + 1;
        a.state[G2S_POS] = pos + 1;
        a.state[G2S_SEQ] = (int)(seq + 1u);
    }
    XTRACE(2);
}

} /* namespace g2step */

extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_stepx_f32(const g2_step_args a)
{
    g2step::stepx_impl<float>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_stepx_f16(const g2_step_args a)
{
    g2step::stepx_impl<_Float16>(a);
}

/* Probe for the host (launched like the step kernels): work-group w writes
 * the XCC it runs on to xcc[w]. */
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_xcc_probe(int *xcc)
{
    if (threadIdx.x == 0) xcc[blockIdx.x] = __builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11)) & 15;
}
