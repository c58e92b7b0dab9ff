/*
 * g2_step4.hip -- the persistent decode step with loader waves (fp16
 * weights; included by g2_kernels.hip after g2_step.hip, whose exchange
 * protocol, helpers and exchange layout it shares).
 *
 * Why loader waves: a CU serves its vector memory requests roughly in
 * issue order and keeps only ~15 KB of them outstanding, and a wave that
 * issues a weight set stalls until most of it has landed.  In the
 * all-to-all step kernel the computing waves issue each matrix's rows as
 * one burst, so the burst either stalls the computation or queues in front
 * of the next exchange read.  Here waves 8..11 of each work-group do
 * nothing but stream the work-group's weight rows, in the order the
 * computation uses them, into a ring of 1 KB blocks in LDS (16-byte loads
 * into two register groups of LG blocks per loader, one group in flight
 * while the other is written to the ring); the eight computing waves read
 * the rows from LDS.
 *
 * Ring protocol (all in LDS): loader wave w streams blocks w, w + NL, ...
 * and publishes landed[w], how many of them are in LDS; computing wave w
 * publishes cons[w] (stream blocks it has finished reading); a loader
 * overwrites a slot only when every wave has passed it.  Each matrix share
 * (rows [r0, r0+nrows) of qkv, proj, fc, fc2 of every layer, then the
 * lm_head rows LMB at a time) is one ring segment starting on a block
 * boundary; both sides walk the same segment sequence.
 *
 * The loaders never take part in a barrier after the start, so the
 * computing waves synchronise through an LDS arrival counter (cw_bar)
 * instead of s_barrier.  Every wait -- for landed blocks, for ring space,
 * at a counter barrier -- is bounded like the exchange waits and gives up
 * through the same abort path.
 *
 * Measured on GPT-2 XL it is slower than the all-to-all kernel (the ring is
 * full more than half the time, so the weight stream is not what bounds a
 * layer; the hand-offs and the arithmetic between them are, and reading
 * the rows from LDS and the counter barriers lengthen the latter).  It is
 * kept as an opt-in form (G2_STEP4=1).
 */

namespace g2s4 {

using namespace g2step;

constexpr int NTH = G2_STEP4_THREADS;      /* 8 computing waves + the loaders */
constexpr int NL = (NTH - NT) / 64;        /* loader waves: loader w takes blocks b = w mod NL */
constexpr int RB = G2_STEP4_RING_BLOCKS;   /* ring blocks of 1 KB */
constexpr int RING = RB * 1024;
constexpr int LG = 8;                      /* blocks per load group of a loader wave */
constexpr int LMB = G2_STEP4_LM_ROWS;      /* lm_head rows per ring segment */

typedef G2_LDS void lds_v;
typedef G2_LDS int lds_i;
typedef const G2_LDS unsigned char lds_cb;

/* LDS control words of the ring and the counter barrier. */
struct ctl {
    int landed[4]; /* loader w: how many of its blocks (w, w+NL, ...) are in LDS */
    int bar;
    int pad[3];
    int cons[NW];
};

__device__ __forceinline__ int lds_get(const lds_i *p)
{
    return __hip_atomic_load(const_cast<lds_i *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

/* Barrier of the eight computing waves: one arrival per wave on a
 * monotonic LDS counter, then wait until the counter reaches the end of
 * this barrier's generation (a wave cannot arrive at the next barrier
 * before all eight arrived at this one).  LDS accesses of a wave complete
 * in order, so data a wave wrote before arriving is visible to every wave
 * that has seen the counter. */
struct cw_bar {
    lds_i *cnt;
    const ctx *c;
    __device__ __forceinline__ void operator()() const
    {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        int old = 0;
        if ((threadIdx.x & 63) == 0)
            old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        old = __builtin_amdgcn_readfirstlane(old);
        const int target = (old / NW + 1) * NW;
        /* the clock (a scalar memory read) is consulted only every 256
         * polls, so a normal wait never reads it */
        u64 t0 = 0;
        for (int n = 1; lds_get(cnt) < target; ++n) {
            __builtin_amdgcn_s_sleep(0);
            if ((n & 255) == 0) {
                const u64 now = wall_clock64();
                if (!t0) t0 = now;
                else if (now - t0 > WAIT_LIMIT) {
                    if (!*c->dead) give_up(*c);
                    break;
                }
            }
        }
        asm volatile("" ::: "memory");
    }
};

/* One ring segment: `bytes` from global `p`, first stream block b0. */
struct seg {
    const unsigned char *p;
    int bytes, b0;
    __device__ __forceinline__ int end() const { return b0 + ((bytes + 1023) >> 10); }
};

/* The next segment of the sequence: rows [row0, row0+nrows) of the
 * work-group's share of the matrix of plan p. */
__device__ __forceinline__ seg take(int &next_block, const plan &p, int row0, int nrows)
{
    seg s;
    s.p = (const unsigned char *)p.W + (size_t)(p.r0 + row0) * p.C * 16;
    s.bytes = nrows * p.C * 16;
    s.b0 = next_block;
    next_block = s.end();
    return s;
}

__device__ __forceinline__ int cons_min_asm(const G2_LDS ctl *k)
{
    const unsigned a = (unsigned)(size_t)&k->cons[0];
    f32x4 lo, hi;
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                 : "=v"(lo), "=v"(hi) : "v"(a) : "memory");
    int m = __float_as_int(lo.x);
    m = min(m, __float_as_int(lo.y)); m = min(m, __float_as_int(lo.z)); m = min(m, __float_as_int(lo.w));
    m = min(m, __float_as_int(hi.x)); m = min(m, __float_as_int(hi.y)); m = min(m, __float_as_int(hi.z));
    m = min(m, __float_as_int(hi.w));
    return __builtin_amdgcn_readfirstlane(m);
}

__device__ __forceinline__ int lds_get_asm(const lds_i *p)
{
    int v;
    const unsigned a = (unsigned)(size_t)p;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
    return __builtin_amdgcn_readfirstlane(v);
}

/* The loader: streams the segment sequence into the ring. */
struct loader_state {
    int n, lim; /* own blocks landed; ring limit */
    u64 waited; /* clock ticks spent waiting for ring space (trace only) */
    int nfull;  /* ring-full events (trace only) */
};

/* Wait until stream block b may be overwritten (every computing wave has
 * passed it); false if the step was abandoned. */
__device__ __forceinline__ bool ring_space(const ctx &c, const G2_LDS ctl *k, loader_state &st, int b)
{
    st.lim = cons_min_asm(k) + RB;
    if (b < st.lim) return true;
    const u64 t0 = wall_clock64();
    ++st.nfull;
    for (;;) {
        __builtin_amdgcn_s_sleep(1);
        st.lim = cons_min_asm(k) + RB;
        if (b < st.lim) {
            st.waited += wall_clock64() - t0;
            return true;
        }
        if (lds_get_asm((const lds_i *)c.dead)) return false;
        if (wall_clock64() - t0 > WAIT_LIMIT) {
            give_up(c);
            return false;
        }
    }
}

/* Writes a loaded group of n blocks into their ring slots and publishes
 * the loader's landed count (LDS stores of one wave complete in order, so
 * a wave that sees the count sees the blocks). */
__device__ __forceinline__ void grp_put(G2_LDS ctl *k, unsigned char G2_LDS *ring, const u32x4 (&X)[LG],
                                        const int (&sl)[LG], int &n, loader_state &st, int w)
{
    if (!n) return;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < LG; ++j)
        if (j < n) *(G2_LDS u32x4 *)(ring + sl[j] * 1024 + lane * 16) = X[j];
    st.n += n;
    n = 0;
    __hip_atomic_store(&k->landed[w], st.n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

/* Streams this loader's blocks of segment s (blocks w, w + NL, ... of the
 * stream) through two register groups of LG blocks: while one group's
 * loads are in flight the other is written to the ring. */
__device__ __forceinline__ bool stream(const ctx &c, G2_LDS ctl *k, unsigned char G2_LDS *ring, loader_state &st,
                                       const seg &s, int w)
{
    const int lane = threadIdx.x & 63;
    const int nb = (s.bytes + 1023) >> 10;
    int i = w - s.b0 % NL;
    i = i < 0 ? i + NL : i;
    u32x4 A[LG], B[LG];
    int sa[LG], sb[LG];
    int na = 0, nbb = 0;
    /* fill X with the next group (all LG loads unconditional, addresses
     * clamped to the group's last block), then put the pending group Y */
    auto step = [&](u32x4 (&X)[LG], int (&sx)[LG], int &nx, u32x4 (&Y)[LG], int (&sy)[LG], int &ny) -> int {
        const int cnt = i < nb ? min(LG, (nb - i + NL - 1) / NL) : 0;
        if (!cnt) return 0;
        const int blast = s.b0 + i + NL * (cnt - 1);
        if (blast >= st.lim) {
            grp_put(k, ring, Y, sy, ny, st, w); /* the computing waves may need it to free space */
            if (!ring_space(c, k, st, blast)) return -1;
        }
#pragma unroll
        for (int j = 0; j < LG; ++j) {
            const int ii = i + NL * min(j, cnt - 1);
            const int off = min(ii * 1024 + lane * 16, s.bytes - 16);
            X[j] = __builtin_nontemporal_load((const G2_GLOBAL u32x4 *)(s.p + off));
            sx[j] = (s.b0 + ii) % RB;
        }
        i += NL * cnt;
        nx = cnt;
        grp_put(k, ring, Y, sy, ny, st, w);
        return 1;
    };
    int r = 1;
    for (;;) {
        r = step(A, sa, na, B, sb, nbb);
        if (r <= 0) break;
        r = step(B, sb, nbb, A, sa, na);
        if (r <= 0) break;
    }
    grp_put(k, ring, A, sa, na, st, w);
    grp_put(k, ring, B, sb, nbb, st, w);
    return r >= 0;
}

template <typename WT>
__device__ __forceinline__ void loader(const g2_step_args &a, const ctx &c, G2_LDS ctl *k, unsigned char G2_LDS *ring)
{
    const G2_CONST g2_step_layer *LT = (const G2_CONST g2_step_layer *)a.layers;
    const int E = a.E, F = a.F;
    const int w = (threadIdx.x >> 6) - NW;
    loader_state st;
    st.n = 0; st.lim = RB; st.waited = 0; st.nfull = 0;
    const u64 t_start = wall_clock64();
    int nxt = 0;
    bool ok = true;
    for (int l = 0; l < a.L && ok; ++l) {
        const g2_step_layer y = LT[l];
        const plan pq = make_plan<WT>(y.qkv_w, 3 * E, E), pp = make_plan<WT>(y.proj_w, E, E);
        const plan pf = make_plan<WT>(y.fc_w, F, E), p2 = make_plan<WT>(y.fc2_w, E, F);
        ok = stream(c, k, ring, st, take(nxt, pq, 0, pq.nrows), w) && stream(c, k, ring, st, take(nxt, pp, 0, pp.nrows), w) &&
             stream(c, k, ring, st, take(nxt, pf, 0, pf.nrows), w) && stream(c, k, ring, st, take(nxt, p2, 0, p2.nrows), w);
    }
    const plan pl = make_plan<WT>(a.lm_w, a.V, E);
    for (int r = 0; r < pl.nrows && ok; r += LMB) ok = stream(c, k, ring, st, take(nxt, pl, r, min(LMB, pl.nrows - r)), w);
    __hip_atomic_store(&k->landed[w], 1 << 30, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); /* every block */
    if (a.trace && w == 0 && (threadIdx.x & 63) == 0) {
        u64 *tr = a.trace + (size_t)blockIdx.x * G2_TRACE_STRIDE(a.L) + 24 * a.L;
        tr[3] = t_start;
        tr[5] = wall_clock64();
        tr[6] = st.waited;
        tr[7] = (u64)st.nfull;
    }
}

/* Computing side: wait until the segment has landed. */
/* Whether every stream block below `need` is in LDS: loader w must have
 * landed its blocks w, w + NL, ... below need, ceil((need - w) / NL) of them. */
__device__ __forceinline__ bool all_landed(const G2_LDS ctl *k, int need)
{
    bool ok = true;
#pragma unroll
    for (int w = 0; w < NL; ++w) ok = ok && lds_get(&k->landed[w]) >= (need - w + NL - 1) / NL;
    return ok;
}

__device__ __forceinline__ void wait_landed(const ctx &c, const G2_LDS ctl *k, int need)
{
    u64 t0 = 0;
    for (int n = 1; !all_landed(k, need); ++n) {
        __builtin_amdgcn_s_sleep(1);
        if ((n & 255) == 0) {
            if (*c.dead) return;
            const u64 now = wall_clock64();
            if (!t0) t0 = now;
            else if (now - t0 > WAIT_LIMIT) {
                give_up(c);
                return;
            }
        }
    }
}

/* This wave has finished reading the ring up to stream block `end`. */
__device__ __forceinline__ void consume(G2_LDS ctl *k, int end)
{
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) __hip_atomic_store(&k->cons[wave], end, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

/* Dot products of rows [row0, row0+nrows) of the share of plan p, held by
 * ring segment s, with xin (LDS): the sum of unit (row r, segment g) goes
 * to part[(row0 + r) * nseg + g].  Units are dealt to waves as in the
 * all-to-all kernel (unit u to wave u % NW), four per wave per pass, their
 * sums reduced together.  Ends with this wave's consume of the segment. */
template <typename WT>
__device__ __forceinline__ void dot_ring(int tid, const ctx &c, G2_LDS ctl *k, lds_cb *ring, const plan &p, int row0,
                                         int nrows, const seg &s, const float *xin, float *part)
{
    constexpr int VE = chunk_t<WT>::V;
    const int wave = tid >> 6, lane = tid & 63;
    const int nunits = nrows * p.nseg;
    wait_landed(c, k, s.end());
    if (wave < nunits) {
        const int c0 = (wave % p.nseg) * p.SL;
        const int c1 = min(p.C, c0 + p.SL);
        float xv[4][VE];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int cc = c0 + lane + 64 * i;
#pragma unroll
            for (int e = 0; e < VE; e += 4) {
                f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
                if (cc < c1) v = *(const f32x4 *)(xin + cc * VE + e);
                xv[i][e] = v.x; xv[i][e + 1] = v.y; xv[i][e + 2] = v.z; xv[i][e + 3] = v.w;
            }
        }
        const int rbase = (s.b0 % RB) * 1024;
        for (int u0 = wave; u0 < nunits; u0 += 4 * NW) {
            float acc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int u = u0 + NW * j;
                const int r = u / p.nseg;
                acc[j] = 0.f;
                if (u >= nunits) continue; /* wave-uniform */
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    /* lanes past the segment end read its last chunk (x is 0 there) */
                    const int cc = min(c0 + lane + 64 * i, c1 - 1);
                    int o = rbase + (r * p.C + cc) * 16;
                    o = o >= RING ? o - RING : o;
                    const u32x4 w = *(const G2_LDS u32x4 *)(ring + o);
                    acc[j] += chunk_dot<WT>(w, xv[i]);
                }
            }
            const float v = wsum4(acc[0], acc[1], acc[2], acc[3]);
            if ((lane & 15) == 0) {
                const int j = (lane >> 4) == 0 ? 0 : ((lane >> 4) == 1 ? 2 : ((lane >> 4) == 2 ? 1 : 3));
                const int u = u0 + NW * j;
                if (u < nunits) part[row0 * p.nseg + u] = v;
            }
        }
    }
    consume(k, s.end());
}

#define TRACE4(k)                                                                      \
    do {                                                                               \
        if (a.trace && tid == 0)                                                       \
            a.trace[(size_t)wg * G2_TRACE_STRIDE(a.L) + 24 * l + (k)] = wall_clock64(); \
    } while (0)

template <typename WT>
__device__ __forceinline__ void step4_impl(const g2_step_args &a)
{
    __shared__ __attribute__((aligned(16))) unsigned char ring[RING];
    __shared__ __attribute__((aligned(16))) float xin[G2_STEP_MAXF];
    __shared__ __attribute__((aligned(16))) float xres[G2_STEP_MAXE];
    __shared__ float part[G2_STEP_MAXUNITS];
    __shared__ float red[2 * NW];
    __shared__ att_lds att[2];
    __shared__ float cw[G2_STEP_MAXCH];
    __shared__ float amv[NT];
    __shared__ int ami[NT];
    __shared__ __attribute__((aligned(16))) ctl K;
    __shared__ volatile int dead;
    __shared__ volatile int flag;

    constexpr int NPE = (G2_STEP_MAXE + NT - 1) / NT;
    constexpr int NPM = (G2_STEP_MAXCH * 66 + NT - 1) / NT;
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int E = a.E, F = a.F, NH = a.NH, S = a.S, V = a.V;
    const int pos = clampi(a.state[G2S_POS], 0, S - 1);
    const int tok = clampi(a.state[G2S_TOK], 0, V - 1);
    const int ngen = a.state[G2S_NGEN], min_new = a.state[G2S_MIN_NEW];
    const unsigned seq = (unsigned)a.state[G2S_SEQ];
    ctx c;
    c.tag = seq + 1u;
    c.abort_w = a.xbuf;
    c.state = a.state;
    c.dead = (lds_flag *)&dead;
    G2_LDS ctl *KP = (G2_LDS ctl *)&K;
    {
        const int tid = threadIdx.x;
        if (tid == 0) { dead = 0; K.bar = 0; }
        if (tid < 4) K.landed[tid] = 0;
        if (tid < NW) K.cons[tid] = 0;
        __syncthreads(); /* the only barrier the loader takes part in */
        if (tid >= NT) {
            loader<WT>(a, c, KP, (unsigned char G2_LDS *)ring);
            return;
        }
    }
    const cw_bar bar{&KP->bar, &c};
    lds_cb *rg = (lds_cb *)ring;
    const int T = pos + 1, nch = (T + 63) >> 6;
    u64 *X = a.xbuf + G2X_HEAD;
    att_regs ar[1];
    int nxt = 0; /* next stream block, as the loader counts */
    {
        const int tid = fresh_tid();
        for (int d = tid; d < E; d += NT)
            xres[d] = ldw((const WT *)a.wte, (size_t)tok * E + d) + ldw((const WT *)a.wpe, (size_t)pos * E + d);
        bar();
    }

    const G2_CONST g2_step_layer *LT = (const G2_CONST g2_step_layer *)a.layers;
    for (int l = 0; l < a.L; ++l) {
        const g2_step_layer y = LT[l];
        u64 *R = X + (size_t)l * a.xlayer;

        /* ---- QKV: LayerNorm(x) . Wqkv + b -> q, k, v (+ KV cache) */
        {
            const int tid = fresh_tid();
            TRACE4(0);
            const plan p = make_plan<WT>(y.qkv_w, 3 * E, E);
            const seg s = take(nxt, p, 0, p.nrows);
            const ln_params<NPE> lp = ln_load<NPE>(tid, gl(y.ln1_w), gl(y.ln1_b), E);
            const float bias = gl(y.qkv_b)[min(p.r0 + tid, 3 * E - 1)];
            if (l > 0)
                fetch<NPE, cw_bar, true>(tid, c, X + (size_t)(l - 1) * a.xlayer + G2X_X2(E, NH, F), E, nwg, xres, (lds_flag *)&flag, bar);
            TRACE4(1);
            layernorm(tid, xres, xin, lp, E, red, bar);
            TRACE4(11);
            dot_ring<WT>(tid, c, KP, rg, p, 0, p.nrows, s, xin, part);
            bar();
            TRACE4(12);
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                float v = row_sum(p, part, tid);
                v += bias;
                ll_put(R + r, v, c.tag);
                if (r >= 2 * E) glw(y.v_cache)[(size_t)pos * E + (r - 2 * E)] = v;
                else if (r >= E) glw(y.k_cache)[(size_t)(r - E) * S + pos] = v;
            }
            TRACE4(2);
        }

        /* ---- ATTN: unit u = h * nch + chunk, work-group u % nwg, half */
        {
            const int tid = fresh_tid();
            const int nunits = NH * nch;
            const int rounds = (nunits + 2 * nwg - 1) / (2 * nwg);
            const int hf = tid >> 8;
            for (int rd = 0; rd < rounds; ++rd) {
                const int u = wg + nwg * (2 * rd + hf);
                const bool on = u < nunits;
                const int h = on ? u / nch : 0, ch = on ? u % nch : 0;
                attn_load(tid, y, ar[0], on, h, ch, pos, T, E, S);
                attn_chunk<false>(tid, c, a.scale, R, h * 64, E + h * 64, 2 * E + h * 64,
                                  R + G2X_ATT(E) + ((size_t)h * G2_STEP_MAXCH + ch) * 66, att[hf], ar[0],
                                  on, ch, pos, T, nullptr, bar);
                bar();
            }
            TRACE4(3);
        }

        /* ---- MERGE: head h by work-group h (g2k_attn_merge) */
        for (int h = wg; h < NH; h += nwg) {
            const int tid = fresh_tid();
            const u64 *hp = R + G2X_ATT(E) + (size_t)h * G2_STEP_MAXCH * 66;
            fetch<NPM, cw_bar, true>(tid, c, hp, nch * 66, nch, xin, (lds_flag *)&flag, bar);
            float Ls = 0.f;
            if (tid < 64) {
                const float mc = tid < nch ? xin[tid * 66] : -INFINITY;
                const float lc = tid < nch ? xin[tid * 66 + 1] : 0.f;
                const float M = wmax(mc);
                const float w = tid < nch ? expf(mc - M) : 0.f;
                Ls = wsum(lc * w);
                if (tid < nch) cw[tid] = w;
            }
            bar();
            if (tid < 64) {
                float acc = 0.f;
                for (int ch = 0; ch < nch; ++ch) acc = fmaf(xin[ch * 66 + 2 + tid], cw[ch], acc);
                ll_put(R + G2X_O(E, NH) + h * 64 + tid, acc / Ls, c.tag);
            }
            bar();
        }
        {
            const int tid = fresh_tid();
            TRACE4(4);
        }

        /* ---- PROJ: X1 = x + (O . Wp + b) */
        {
            const int tid = fresh_tid();
            const plan p = make_plan<WT>(y.proj_w, E, E);
            const seg s = take(nxt, p, 0, p.nrows);
            const float bias = gl(y.proj_b)[min(p.r0 + tid, E - 1)];
            fetch<NPE, cw_bar, true>(tid, c, R + G2X_O(E, NH), E, NH, xin, (lds_flag *)&flag, bar);
            TRACE4(5);
            dot_ring<WT>(tid, c, KP, rg, p, 0, p.nrows, s, xin, part);
            bar();
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                float v = row_sum(p, part, tid);
                v += bias;
                ll_put(R + G2X_X1(E, NH) + r, v + xres[r], c.tag);
            }
            TRACE4(6);
            bar();
        }

        /* ---- FC: H = gelu(LayerNorm(X1) . Wfc + b) */
        {
            const int tid = fresh_tid();
            const plan p = make_plan<WT>(y.fc_w, F, E);
            const seg s = take(nxt, p, 0, p.nrows);
            const ln_params<NPE> lp = ln_load<NPE>(tid, gl(y.ln2_w), gl(y.ln2_b), E);
            const float bias = gl(y.fc_b)[min(p.r0 + tid, F - 1)];
            fetch<NPE, cw_bar, true>(tid, c, R + G2X_X1(E, NH), E, nwg, xres, (lds_flag *)&flag, bar);
            TRACE4(7);
            layernorm(tid, xres, xin, lp, E, red, bar);
            TRACE4(13);
            dot_ring<WT>(tid, c, KP, rg, p, 0, p.nrows, s, xin, part);
            bar();
            TRACE4(14);
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                float v = row_sum(p, part, tid);
                v += bias;
                ll_put(R + G2X_H(E, NH) + r, gelu_f(v), c.tag);
            }
            TRACE4(8);
            bar();
        }

        /* ---- FC2: X2 = X1 + (H . Wfc2 + b) */
        {
            const int tid = fresh_tid();
            const plan p = make_plan<WT>(y.fc2_w, E, F);
            const seg s = take(nxt, p, 0, p.nrows);
            const float bias = gl(y.fc2_b)[min(p.r0 + tid, E - 1)];
            fetch<PMAX, cw_bar, true>(tid, c, R + G2X_H(E, NH), F, nwg, xin, (lds_flag *)&flag, bar);
            TRACE4(9);
            dot_ring<WT>(tid, c, KP, rg, p, 0, p.nrows, s, xin, part);
            bar();
            TRACE4(15);
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                float v = row_sum(p, part, tid);
                v += bias;
                ll_put(R + G2X_X2(E, NH, F) + r, v + xres[r], c.tag);
            }
            TRACE4(10);
            bar();
        }
    }

    /* ---- LM: logits over the head rows (LMB rows per ring segment),
     * work-group first-max; then the greedy pick by work-group 0 */
    {
        const int tid = fresh_tid();
        const int l = a.L;
        const ln_params<NPE> lpf = ln_load<NPE>(tid, gl(a.lnf_w), gl(a.lnf_b), E);
        const plan p = make_plan<WT>(a.lm_w, V, E);
        fetch<NPE, cw_bar, true>(tid, c, X + (size_t)(a.L - 1) * a.xlayer + G2X_X2(E, NH, F), E, nwg, xres, (lds_flag *)&flag, bar);
        TRACE4(0);
        layernorm(tid, xres, xin, lpf, E, red, bar);
        for (int r = 0; r < p.nrows; r += LMB) {
            const int n = min(LMB, p.nrows - r);
            const seg s = take(nxt, p, r, n);
            dot_ring<WT>(tid, c, KP, rg, p, r, n, s, xin, part);
        }
        bar();
        const int masked = ngen < min_new ? G2_EOS_ID : -1;
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        if (tid < p.nrows) {
            const int r = p.r0 + tid;
            const float v = row_sum(p, part, tid);
            glw(a.logits)[r] = v;
            bv = r == masked ? -1e30f : v;
            bi = r;
        }
        blk_argmax(tid, bv, bi, amv, ami, bar);
        u64 *AM = X + (size_t)a.L * a.xlayer;
        if (tid == 0) {
            ll_put(AM + 2 * wg, amv[0], c.tag);
            ll_put(AM + 2 * wg + 1, __int_as_float(ami[0]), c.tag);
        }
        TRACE4(1);
        if (wg != 0) return;
        bar();
        fetch<2, cw_bar, true>(tid, c, AM, 2 * nwg, nwg, xin, (lds_flag *)&flag, bar);
        bv = -INFINITY;
        bi = 0x7fffffff;
        for (int b = tid; b < nwg; b += NT) {
            const float v = xin[2 * b];
            const int i = __float_as_int(xin[2 * b + 1]);
            if (am_better2(v, i, bv, bi)) { bv = v; bi = i; }
        }
        blk_argmax(tid, bv, bi, amv, ami, bar);
        if (tid == 0) {
            const int tk = (ami[0] >= 0 && ami[0] < V) ? ami[0] : 0;
            const int ng = clampi(ngen, 0, G2S_WORDS - G2S_IDS - 1);
            a.state[G2S_IDS + ng] = tk;
            a.state[G2S_TOK] = tk;
            a.state[G2S_NGEN] = ng + 1;
            a.state[G2S_POS] = pos + 1;
            a.state[G2S_SEQ] = (int)(seq + 1u);
        }
        TRACE4(2);
    }
}

#undef TRACE4

} /* namespace g2s4 */

extern "C" __global__ __launch_bounds__(G2_STEP4_THREADS) void g2k_step4_f16(const g2_step_args a)
{
    g2s4::step4_impl<_Float16>(a);
}
