/*
 * g2_step3.hip -- the decode step as one persistent cooperative kernel whose
 * work-groups split their waves into two roles (fp16 weights; included by
 * g2_kernels.hip after g2_step.hip, whose exchange, wait, attention and
 * lm_head helpers it uses).
 *
 * Why two roles: a wave's vector-memory counter completes in issue order, so
 * a wave with weight loads in flight cannot use the result of a later
 * exchange load before every one of those weights has arrived.  In the
 * single-role kernel (g2k_step_*) each hand-off therefore also waited for
 * the weights issued just before it (up to 20 MB over the chip, ~3 us), and
 * the weight stream could run only one matrix ahead.  Here:
 *
 *   wave 7, the exchange wave, issues no weight loads.  It reads every input
 *   vector from the exchange area into LDS, computes the LayerNorms, merges
 *   the attention partials of a head (work-groups < n_head) and sums the
 *   fc2 partials of its rows.  Its other loads are issued where they delay
 *   nothing: LayerNorm parameters go to LDS while the compute waves run a
 *   dot product, fc2 bias rows and its share of the cached keys and values
 *   just before a wait on the exchange, which takes longer anyway.
 *
 *   waves 0-6, the compute waves, hold the weights in three register sets,
 *   each reloaded as soon as it has been used:
 *     A  qkv rows of layer l -> fc2 block of layer l -> qkv rows of l + 1
 *     B  fc rows of layer l -> fc rows of layer l + 1
 *     D  proj rows of layer l -> proj rows of layer l + 1
 *   plus the cached keys and values of their attention chunks (loaded a
 *   layer ahead).  They never wait on the exchange area: they meet the
 *   exchange wave at work-group barriers.
 *
 * fc2 is split over K: a work-group multiplies its own gelu(fc) rows h_j by
 * the matching rows of the input-major fc2 matrix (W2T[F][E], a transposed
 * copy made at set-up) and publishes a partial product over all E outputs;
 * the exchange wave of the work-group owning output rows [n0, n0 + nr) adds
 * the nwg partials (32 per lane in work-group order, then across lanes in
 * a fixed order).  That replaces the hand-off of the F-wide h vector (every
 * work-group reading all F words) with one of 8 nwg contiguous words.
 *
 * Per layer (B = work-group barrier; every role passes the same barriers):
 *     exchange: X2 of the layer before (or the embedding) -> LayerNorm1
 *   B compute: qkv dot products
 *   B compute: q, k, v rows -> exchange, K/V cache; A <- fc2 block
 *     exchange: q, k, v of the work-group's attention chunks -> LDS
 *   B all: attention chunks -> partials (three barriers inside), B
 *     compute: keys/values of the next layer    exchange: merge, then O
 *   B compute: proj dot products
 *   B compute: X1 rows = x + proj + b -> exchange; D <- next proj
 *     exchange: X1 -> LayerNorm2
 *   B compute: fc dot products
 *   B compute: h rows = gelu(fc + b) -> LDS
 *   B compute: fc2 partial products -> LDS
 *   B compute: partial -> exchange; A <- next qkv, B <- next fc
 *     exchange: X2 rows = X1 + b + sum of partials -> exchange
 * then the lm_head and the greedy pick (lm_pick, all waves).
 */

namespace g2step {

constexpr int NWC = NW - 1;      /* compute waves */
constexpr int NTC = 64 * NWC;    /* compute threads */
constexpr int SA = 13, SB = 16, SD = 4;                   /* register set slots */
constexpr int UQ = 3, UF = 4, UP = 1;  /* row units per compute wave: qkv, fc, proj */
constexpr int XNE = (G2_STEP_MAXE + 63) / 64;             /* E-vector words per lane */
constexpr int XNP = 8 * G3_MAXWG / 64;                    /* fc2 partial words per lane */
constexpr int XNM = (G2_STEP_MAXCH * 66 + 63) / 64;       /* a head's attention partials */
constexpr int XNS = G3_MAXWG / 64;                        /* sentinel words per lane */
constexpr int RED2 = NTC * 8;                             /* fc2 partial staging floats */

/* The exchange wave's LDS writes are read by its other lanes: wait for
 * them to complete (and keep the compiler from moving accesses across). */
__device__ __forceinline__ void wave_lds_sync()
{
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

/* Exchange wave: v[i] = src[at(lane + 64 i)] for lane + 64 i < n, once it
 * carries this step's tag.  After one speculative read of every word, a
 * wave that found stale ones waits on nsent <= 256 sentinel words (word
 * n*k/nsent: the first word of producer k when n words are split evenly over
 * nsent producers; nsent 0: none) and then re-reads only its stale words, so
 * the wait costs one word per producer per round trip. */
template <int NPW, typename AT>
__device__ __forceinline__ void xw_fetch(int lane, const ctx &c, const u64 *src, int n, int nsent, AT at,
                                         u64 (&v)[NPW], u64 *tr = nullptr)
{
    const u64 filler = (u64)c.tag << 32;
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
        const int w = lane + 64 * i;
        v[i] = w < n ? ll_get(src + at(w)) : filler;
    }
    unsigned bad = 0;
#pragma unroll
    for (int i = 0; i < NPW; ++i) bad |= (unsigned)(ll_tag(v[i]) != c.tag);
    if (tr && lane == 0) tr[0] = wall_clock64();
    if (__builtin_amdgcn_ballot_w64(bad != 0u) == 0 || *c.dead) return;
    if (nsent > 0) {
        u64 sv[XNS];
#pragma unroll
        for (int k = 0; k < XNS; ++k) {
            const int s = lane + 64 * k;
            sv[k] = s < nsent ? ll_get(src + at((n * s) / nsent)) : filler;
        }
        settle(c, src, sv, [&](int k) {
            const int s = lane + 64 * k;
            return s < nsent ? at((n * s) / nsent) : -1;
        });
    }
    if (tr && lane == 0) tr[1] = wall_clock64();
    settle(c, src, v, [&](int i) {
        const int w = lane + 64 * i;
        return w < n ? at(w) : -1;
    });
}

/* Exchange wave: xin = LayerNorm(x) over the E entries x[i] = entry lane +
 * 64 i (mean, then biased variance of x - mean, eps 1e-5, (x - mean) *
 * inv_std * g + b: layernorm, math.cl:283-311); the raw entries go to xraw. */
__device__ __forceinline__ void xw_layernorm(int lane, const float (&x)[XNE], const float *lg, const float *lb,
                                             int E, float *xin, float *xraw)
{
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < XNE; ++i)
        if (lane + 64 * i < E) s += x[i];
    const float mean = wsum(s) / (float)E;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < XNE; ++i)
        if (lane + 64 * i < E) {
            const float d = x[i] - mean;
            q = fmaf(d, d, q);
        }
    const float inv = 1.0f / sqrtf(wsum(q) / (float)E + 1e-5f);
#pragma unroll
    for (int i = 0; i < XNE; ++i) {
        const int w = lane + 64 * i;
        if (w < E) {
            xraw[w] = x[i];
            xin[w] = fmaf((x[i] - mean) * inv, lg[w], lb[w]);
        }
    }
}

/* Exchange wave: fetch E words of a vector written by nsent producers and
 * LayerNorm it into xin (raw values to xraw). */
__device__ __forceinline__ void xw_vector_ln(int lane, const ctx &c, const u64 *src, int E, int nsent,
                                             const float *lg, const float *lb, float *xin, float *xraw,
                                             u64 *tr = nullptr)
{
    u64 v[XNE];
    xw_fetch(lane, c, src, E, nsent, [](int w) { return w; }, v, tr);
    float x[XNE];
#pragma unroll
    for (int i = 0; i < XNE; ++i) x[i] = ll_val(v[i]);
    xw_layernorm(lane, x, lg, lb, E, xin, xraw);
}

/* ------------------------------------------------------ compute waves */

/* A compute-wave share of a packed output-major W[N][K] (fp16, K = n_embd,
 * C = K/8 <= 256 16-byte chunks per row): rows [r0, r0 + nrows) of an even
 * split over the grid; share row t is unit t / 7 of wave t % 7, its 64
 * lanes taking chunks lane + 64 i (i < 4). */
struct cplan {
    const u32x4 *W;
    int C, r0, nrows;
};

__device__ __forceinline__ cplan cmake(const void *W, int N, int K)
{
    cplan p;
    p.W = (const u32x4 *)W;
    p.C = K / 8;
    const long nwg = gridDim.x, wg = blockIdx.x;
    p.r0 = (int)(((long)N * wg) / nwg);
    p.nrows = (int)(((long)N * (wg + 1)) / nwg) - p.r0;
    return p;
}

/* Loads are unconditional (every address clamped into the share, lanes
 * past the row end to its last chunk, which the same instruction already
 * fetches; units past the share to the wave's first row, an L2 hit): a load
 * under a lane condition makes the compiler wait for every load in flight
 * before the value is first used, which would serialize the weight stream. */
template <int UM, int S>
__device__ __forceinline__ void cload(int tid, u32x4 (&w)[S], const cplan &p, int N)
{
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int j = 0; j < UM; ++j) {
        const int t = wave + NWC * j;
        const int row = min(p.r0 + (t < p.nrows ? t : wave), N - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int cc = min(lane + 64 * i, p.C - 1);
            w[4 * j + i] = __builtin_nontemporal_load(gl(p.W) + (size_t)row * p.C + cc);
        }
    }
}

/* Dot products of the share with xin (LDS): part[t] for share row t. */
template <int UM, int S>
__device__ __forceinline__ void cdot(int tid, const u32x4 (&w)[S], const cplan &p, const float *xin,
                                     float *part)
{
    const int wave = tid >> 6, lane = tid & 63;
    if (wave >= p.nrows) return; /* wave-uniform */
    float acc[UM];
#pragma unroll
    for (int j = 0; j < UM; ++j) acc[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int cc = lane + 64 * i;
        float xv[8];
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
            f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
            if (cc < p.C) v = *(const f32x4 *)(xin + cc * 8 + e);
            xv[e] = v.x; xv[e + 1] = v.y; xv[e + 2] = v.z; xv[e + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < UM; ++j) acc[j] += chunk_dot<_Float16>(w[4 * j + i], xv);
    }
#pragma unroll
    for (int j = 0; j < UM; ++j) {
        const int t = wave + NWC * j;
        if (t >= p.nrows) break; /* wave-uniform */
        const float v = wsum(acc[j]);
        if (lane == 0) part[t] = v;
    }
}

/* The compute-wave share of the fc2 K-split: rows [f0, f0 + nf) of the
 * input-major W2T[F][E] (fp16; the work-group's fc rows).  Thread t <
 * JG * NC (NC = E/8 output chunks, JG = 448 / NC row groups) takes output
 * chunk c = t % NC and share rows [nf g / JG, nf (g + 1) / JG), g = t / NC. */
struct kplan {
    const u32x4 *W;
    int NC, JG, f0, c, g, j0, j1;
};

__device__ __forceinline__ kplan kmake(int tid, const void *W2T, int F, int E)
{
    kplan p;
    p.W = (const u32x4 *)W2T;
    p.NC = E / 8;
    p.JG = NTC / p.NC;
    const long nwg = gridDim.x, wg = blockIdx.x;
    p.f0 = (int)(((long)F * wg) / nwg);
    const int nf = (int)(((long)F * (wg + 1)) / nwg) - p.f0;
    p.g = tid / p.NC;
    p.c = p.g < p.JG ? tid - p.g * p.NC : 0;
    p.j0 = p.g < p.JG ? (nf * p.g) / p.JG : 0;
    p.j1 = p.g < p.JG ? (nf * (p.g + 1)) / p.JG : 0;
    return p;
}

/* Unconditional loads, as in cload: slots past the thread's rows reload
 * its last row (an L2 hit). */
template <int S>
__device__ __forceinline__ void kload(const kplan &p, u32x4 (&w)[S], int F)
{
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int row = min(p.f0 + min(p.j0 + s, max(p.j1 - 1, 0)), F - 1);
        w[s] = __builtin_nontemporal_load(gl(p.W) + (size_t)row * p.NC + p.c);
    }
}

/* red2[g*E + 8c + e] = sum over the thread's rows j (in order) of
 * W2T[f0 + j][8c + e] * hb[j]. */
template <int S>
__device__ __forceinline__ void kdot(const kplan &p, const u32x4 (&w)[S], const float *hb, float *red2, int E)
{
    if (p.g >= p.JG) return;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int j = p.j0 + s;
        if (j < p.j1) {
            const float hv = hb[j];
            const f16x8 h8 = __builtin_bit_cast(f16x8, w[s]);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf((float)h8[e], hv, acc[e]);
        }
    }
    f32x4 *o = (f32x4 *)(red2 + (size_t)p.g * E + 8 * p.c);
    o[0] = (f32x4){acc[0], acc[1], acc[2], acc[3]};
    o[1] = (f32x4){acc[4], acc[5], acc[6], acc[7]};
}

/* ---------------------------------------------------------- the kernel */

/* Phase timestamps, by thread 0 (compute) or lane 0 of the exchange wave. */
#define TRACE3(k, first)                                                               \
    do {                                                                               \
        if (a.trace && (first))                                                        \
            a.trace[(size_t)wg * G2_TRACE_STRIDE(a.L) + 24 * l + (k)] = wall_clock64(); \
    } while (0)

struct s3_lds {
    float xin[G2_STEP_MAXE] __attribute__((aligned(16)));
    float xr0[G2_STEP_MAXE];  /* x entering the layer (residual of proj) */
    float xr1[G2_STEP_MAXE];  /* X1 (residual of fc2) */
    float part[G2_STEP_MAXUNITS];
    float hb[4 * NWC];        /* gelu(fc) rows of the work-group */
    float red2[RED2] __attribute__((aligned(16)));
    float cw[G2_STEP_MAXCH];
    float lg1[G2_STEP_MAXE], lb1[G2_STEP_MAXE]; /* LayerNorm1 parameters */
    float lg2[G2_STEP_MAXE], lb2[G2_STEP_MAXE]; /* LayerNorm2 parameters */
    att_lds att[2];
};

/* Units of the attention: (head, chunk) u = h * nch + ch; round rd, half hf
 * of work-group wg takes u = wg + nwg * (2 rd + hf). */
__device__ __forceinline__ void unit_of(int u, int nunits, int nch, bool &on, int &h, int &ch)
{
    on = u < nunits;
    h = on ? u / nch : 0;
    ch = on ? u % nch : 0;
}

/* Compute waves (tid < 448). */
__device__ __forceinline__ void s3_compute(const g2_step_args &a, const ctx &c, s3_lds &S, int pos, int T,
                                           int nch)
{
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int E = a.E, F = a.F, NH = a.NH, SS = a.S;
    const int nunits = NH * nch;
    u64 *X = a.xbuf + G2X_HEAD;
    const G2_CONST g2_step_layer *LT = (const G2_CONST g2_step_layer *)a.layers;
    u32x4 A[SA], B[SB], D[SD];
    att_regs kv;
    float bq, bp, bf;
    {
        const int tid = fresh_tid();
        const g2_step_layer y = LT[0];
        const cplan pq = cmake(y.qkv_w, 3 * E, E), pp = cmake(y.proj_w, E, E), pf = cmake(y.fc_w, F, E);
        bq = gl(y.qkv_b)[min(pq.r0 + tid, 3 * E - 1)];
        bp = gl(y.proj_b)[min(pp.r0 + tid, E - 1)];
        bf = gl(y.fc_b)[min(pf.r0 + tid, F - 1)];
        cload<UQ>(tid, A, pq, 3 * E);
        __builtin_amdgcn_sched_barrier(0);
        cload<UF>(tid, B, pf, F);
        __builtin_amdgcn_sched_barrier(0);
        cload<UP>(tid, D, pp, E);
        __builtin_amdgcn_sched_barrier(0);
        bool on;
        int h, ch;
        unit_of(wg + nwg * (tid >> 8), nunits, nch, on, h, ch);
        attn_load(tid, y, kv, on, h, ch, pos, T, E, SS);
        /* Let the first layer's weights land here (the exchange wave is
         * still computing the embedding): with nothing in flight at the loop
         * entry, the compiler's wait counts inside the loop follow the
         * loop's own load order, not the prologue's register assignment. */
        __builtin_amdgcn_s_waitcnt(0);
    }
    for (int l = 0; l < a.L; ++l) {
        const g2_step_layer y = LT[l];
        u64 *R = X + (size_t)l * a.xlayer;
        /* the next layer's tables; the last layer reloads its own (a few
         * percent of one layer's weights), so every reload is unconditional
         * and the compiler's wait counts stay exact (a reload under a
         * condition leaves a path on which the loop's first use seems to wait
         * for the most recent loads) */
        const g2_step_layer z = LT[min(l + 1, a.L - 1)];

        /* ---- QKV */
        {
            const int tid = fresh_tid();
            const cplan p = cmake(y.qkv_w, 3 * E, E);
            __syncthreads(); /* xin = LayerNorm1(x) */
            cdot<UQ>(tid, A, p, S.xin, S.part);
            TRACE3(12, tid == 0);
            __syncthreads();
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                const float v = S.part[tid] + bq;
                ll_put(R + r, v, c.tag);
                if (r >= 2 * E) glw(y.v_cache)[(size_t)pos * E + (r - 2 * E)] = v;
                else if (r >= E) glw(y.k_cache)[(size_t)(r - E) * SS + pos] = v;
            }
            TRACE3(2, tid == 0);
            kload<SA>(kmake(tid, y.fc2_wt, F, E), A, F);
        }

        /* ---- ATTN: one (head, chunk) unit per half (at most 2 nwg units) */
        {
            const int tid = fresh_tid();
            const int hf = tid >> 8;
            bool on;
            int h, ch;
            unit_of(wg + nwg * hf, nunits, nch, on, h, ch);
            __syncthreads(); /* q, k, v in att[hf] */
            attn_compute<false>(tid, c, a.scale, R + G3X_ATT(E) + ((size_t)h * G2_STEP_MAXCH + ch) * 66, S.att[hf],
                                kv, on, ch, pos, T);
            __syncthreads();
            TRACE3(3, tid == 0);
            attn_load(tid, z, kv, on, h, ch, pos, T, E, SS);
        }

        /* ---- PROJ: X1 = x + (O . Wp + b) */
        {
            const int tid = fresh_tid();
            const cplan p = cmake(y.proj_w, E, E);
            __syncthreads(); /* xin = O */
            cdot<UP>(tid, D, p, S.xin, S.part);
            __syncthreads();
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                ll_put(R + G3X_X1(E, NH) + r, (S.part[tid] + bp) + S.xr0[r], c.tag);
            }
            TRACE3(6, tid == 0);
            cload<UP>(tid, D, cmake(z.proj_w, E, E), E);
        }

        /* ---- FC: h = gelu(LayerNorm2(X1) . Wfc + b), then the fc2 partial */
        {
            const int tid = fresh_tid();
            const cplan p = cmake(y.fc_w, F, E);
            __syncthreads(); /* xin = LayerNorm2(X1) */
            cdot<UF>(tid, B, p, S.xin, S.part);
            TRACE3(14, tid == 0);
            __syncthreads();
            if (tid < p.nrows) S.hb[tid] = gelu_f(S.part[tid] + bf);
            __syncthreads();
            const kplan k = kmake(tid, y.fc2_wt, F, E);
            kdot<SA>(k, A, S.hb, S.red2, E);
            TRACE3(15, tid == 0);
            __syncthreads();
            /* partial of row n -> its reader kk's block (row r of kk) */
            u64 *P2 = R + G3X_P2(E, NH);
            for (int n = tid; n < E; n += NTC) {
                float v = S.red2[n];
                for (int g = 1; g < k.JG; ++g) v += S.red2[(size_t)g * E + n];
                const int kk = ((n + 1) * nwg - 1) / E;
                const int r = n - (int)(((long)E * kk) / nwg);
                ll_put(P2 + ((size_t)kk * nwg + wg) * 8 + r, v, c.tag);
            }
            TRACE3(8, tid == 0);
            {
                const cplan pq = cmake(z.qkv_w, 3 * E, E), pp = cmake(z.proj_w, E, E), pf = cmake(z.fc_w, F, E);
                bq = gl(z.qkv_b)[min(pq.r0 + tid, 3 * E - 1)];
                bp = gl(z.proj_b)[min(pp.r0 + tid, E - 1)];
                bf = gl(z.fc_b)[min(pf.r0 + tid, F - 1)];
                /* qkv first: the next qkv dot then waits for A only */
                cload<UQ>(tid, A, pq, 3 * E);
                __builtin_amdgcn_sched_barrier(0);
                cload<UF>(tid, B, pf, F);
            }
        }
    }
}

/* Exchange wave: LayerNorm parameters of entries lane + 64 i, loaded into
 * registers (issued together; written to LDS later, once they have
 * arrived, by xw_ln_put). */
struct xw_lnp {
    float g[XNE], b[XNE];
};
__device__ __forceinline__ void xw_ln_issue(int lane, xw_lnp &p, const float *g, const float *b, int E)
{
#pragma unroll
    for (int i = 0; i < XNE; ++i) {
        const int w = min(lane + 64 * i, E - 1); /* unconditional, as in cload */
        p.g[i] = gl(g)[w];
        p.b[i] = gl(b)[w];
    }
}
__device__ __forceinline__ void xw_ln_put(int lane, const xw_lnp &p, int E, float *lg, float *lb)
{
#pragma unroll
    for (int i = 0; i < XNE; ++i) {
        const int w = lane + 64 * i;
        if (w < E) {
            lg[w] = p.g[i];
            lb[w] = p.b[i];
        }
    }
}

/* The exchange wave (tid 448..511).  Besides the exchange words it loads
 * only small things, each issued where the wait it precedes is longer:
 * its share of the cached keys and values right after LayerNorm1, the
 * LayerNorm parameters of the next two norms and its fc2 bias rows while
 * the compute waves run the qkv dot products (written to LDS after the
 * attention). */
__device__ __forceinline__ void s3_exchange(const g2_step_args &a, const ctx &c, s3_lds &S, int pos, int T,
                                            int nch, int tok)
{
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int E = a.E, NH = a.NH, SS = a.S;
    const int nunits = NH * nch;
    u64 *X = a.xbuf + G2X_HEAD;
    const G2_CONST g2_step_layer *LT = (const G2_CONST g2_step_layer *)a.layers;
    /* X2 rows this work-group sums */
    const int n0 = (int)(((long)E * wg) / nwg), nr = (int)(((long)E * (wg + 1)) / nwg) - n0;
    att_regs kv;
    {
        const int tid = fresh_tid(), lane = tid & 63;
        const g2_step_layer y = LT[0];
        xw_lnp p1;
        xw_ln_issue(lane, p1, y.ln1_w, y.ln1_b, E);
        /* embedding of the token at its position (embed, math.cl:333-350) */
        float x[XNE];
#pragma unroll
        for (int i = 0; i < XNE; ++i) {
            const int w = min(lane + 64 * i, E - 1);
            x[i] = ldw((const _Float16 *)a.wte, (size_t)tok * E + w) + ldw((const _Float16 *)a.wpe, (size_t)pos * E + w);
        }
        xw_ln_put(lane, p1, E, S.lg1, S.lb1);
        const int l = 0;
        TRACE3(1, lane == 0);
        wave_lds_sync();
        xw_layernorm(lane, x, S.lg1, S.lb1, E, S.xin, S.xr0);
        TRACE3(11, lane == 0);
    }
    for (int l = 0; l < a.L; ++l) {
        const g2_step_layer y = LT[l];
        const g2_step_layer z = LT[min(l + 1, a.L - 1)];
        u64 *R = X + (size_t)l * a.xlayer;
        const bool more = l + 1 < a.L;
        const int tid = fresh_tid(), lane = tid & 63;
        bool on0, on1;
        int h0, h1, ch;
        unit_of(wg, nunits, nch, on0, h0, ch);
        unit_of(wg + nwg, nunits, nch, on1, h1, ch);
        attn_load(tid, y, kv, on1, h1, ch, pos, T, E, SS);

        __syncthreads(); /* QKV: xin ready */
        xw_lnp p2, p1;
        xw_ln_issue(lane, p2, y.ln2_w, y.ln2_b, E);
        xw_ln_issue(lane, p1, z.ln1_w, z.ln1_b, E);
        const float b2 = gl(y.fc2_b)[min(n0 + lane, E - 1)]; /* used by lanes < nr */
        __syncthreads(); /* QKV: dot done */

        /* ---- ATTN: q, k, v of the two chunks, then the chunks */
        {
            u64 v[6];
            xw_fetch(lane, c, R, 6 * 64, 0, [&](int w) {
                const int i = w >> 6, hf = i / 3, part = i - 3 * hf;
                const int hh = hf ? h1 : h0;
                return ((hf ? on1 : on0) ? part * E + hh * 64 : 0) + (w & 63);
            }, v);
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                const int hf = i / 3, part = i - 3 * hf;
                float *dst = part == 0 ? S.att[hf].q : (part == 1 ? S.att[hf].kn : S.att[hf].vn);
                dst[lane] = ll_val(v[i]);
            }
            TRACE3(16, lane == 0);
            __syncthreads(); /* q, k, v in att[] */
            attn_compute<false>(tid, c, a.scale, R + G3X_ATT(E) + ((size_t)h1 * G2_STEP_MAXCH + ch) * 66,
                                S.att[1], kv, on1, ch, pos, T);
            __syncthreads();
        }
        /* LayerNorm2 of this layer and LayerNorm1 of the next (LayerNorm1 of
         * this layer is done) */
        xw_ln_put(lane, p2, E, S.lg2, S.lb2);
        if (more) xw_ln_put(lane, p1, E, S.lg1, S.lb1);

        /* ---- MERGE: head h by work-group h (g2k_attn_merge) */
        for (int h = wg; h < NH; h += nwg) {
            u64 v[XNM];
            xw_fetch(lane, c, R + G3X_ATT(E) + (size_t)h * G2_STEP_MAXCH * 66, nch * 66, nch,
                     [](int w) { return w; }, v);
#pragma unroll
            for (int i = 0; i < XNM; ++i) {
                const int w = lane + 64 * i;
                if (w < nch * 66) S.xin[w] = ll_val(v[i]);
            }
            wave_lds_sync();
            const float mc = lane < nch ? S.xin[lane * 66] : -INFINITY;
            const float lc = lane < nch ? S.xin[lane * 66 + 1] : 0.f;
            const float M = wmax(mc);
            const float w = lane < nch ? expf(mc - M) : 0.f;
            const float Ls = wsum(lc * w);
            if (lane < nch) S.cw[lane] = w;
            wave_lds_sync();
            float acc = 0.f;
            for (int ch = 0; ch < nch; ++ch) acc = fmaf(S.xin[ch * 66 + 2 + lane], S.cw[ch], acc);
            ll_put(R + G3X_O(E, NH) + h * 64 + lane, acc / Ls, c.tag);
            wave_lds_sync();
        }
        TRACE3(4, lane == 0);

        /* ---- O for the proj rows */
        {
            u64 v[XNE];
            xw_fetch(lane, c, R + G3X_O(E, NH), E, NH, [](int w) { return w; }, v);
#pragma unroll
            for (int i = 0; i < XNE; ++i) {
                const int w = lane + 64 * i;
                if (w < E) S.xin[w] = ll_val(v[i]);
            }
        }
        TRACE3(5, lane == 0);
        __syncthreads(); /* PROJ: xin = O */
        __syncthreads(); /* PROJ: dot done */

        /* ---- X1 -> LayerNorm2 */
        xw_vector_ln(lane, c, R + G3X_X1(E, NH), E, nwg, S.lg2, S.lb2, S.xin, S.xr1);
        TRACE3(7, lane == 0);
        __syncthreads(); /* FC: xin ready */
        __syncthreads(); /* FC: dot done */
        __syncthreads(); /* FC: h rows in LDS */
        __syncthreads(); /* FC2: partial in LDS */

        /* ---- X2 rows = X1 + (sum of partials + b): the reader-blocked
         * partials of this work-group, word 8 p + r (lane + 64 i: row r =
         * lane & 7, producer p = lane / 8 + 8 i) */
        if (nr > 0) {
            /* rows r >= nr are never written: their slots re-read row 0
             * (the lanes holding them write nothing) */
            u64 v[XNP];
            xw_fetch(lane, c, R + G3X_P2(E, NH) + (size_t)wg * nwg * 8, 8 * nwg, nwg,
                     [&](int w) { return (w & 7) < nr ? w : (w & ~7); }, v,
                     a.trace ? a.trace + (size_t)wg * G2_TRACE_STRIDE(a.L) + 24 * l + 17 : nullptr);
            TRACE3(9, lane == 0);
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < XNP; ++i) sum += ll_val(v[i]); /* producers in order; fillers are 0 */
            sum += dpp<0x128>(sum);      /* lane ^ 8 (row_ror 8) */
            sum += __shfl_xor(sum, 16);
            sum += __shfl_xor(sum, 32);
            if (lane < nr) ll_put(R + G3X_X2(E, NH) + n0 + lane, (sum + b2) + S.xr1[n0 + lane], c.tag);
            TRACE3(10, lane == 0);
        }

        /* ---- next layer's x -> LayerNorm1 */
        if (more) {
            const int l1 = l + 1;
            {
                const int l = l1;
                TRACE3(0, lane == 0);
            }
            xw_vector_ln(lane, c, R + G3X_X2(E, NH), E, nwg, S.lg1, S.lb1, S.xin, S.xr0,
                         a.trace ? a.trace + (size_t)wg * G2_TRACE_STRIDE(a.L) + 24 * l1 + 20 : nullptr);
            {
                const int l = l1;
                TRACE3(1, lane == 0);
            }
        }
    }
}

__device__ __forceinline__ void step3_impl(const g2_step_args &a)
{
    __shared__ s3_lds S;
    __shared__ float amv[NT];
    __shared__ int ami[NT];
    __shared__ float red[2 * NW];
    __shared__ volatile int dead;
    __shared__ volatile int flag;

    const int pos = clampi(a.state[G2S_POS], 0, a.S - 1);
    const int tok = clampi(a.state[G2S_TOK], 0, a.V - 1);
    const unsigned seq = (unsigned)a.state[G2S_SEQ];
    ctx c;
    c.tag = seq + 1u;
    c.abort_w = a.xbuf;
    c.state = a.state;
    c.dead = (lds_flag *)&dead;
    const int T = pos + 1, nch = (T + 63) >> 6;
    if (threadIdx.x == 0) dead = 0;
    __syncthreads();
    if ((threadIdx.x >> 6) == NW - 1) s3_exchange(a, c, S, pos, T, nch, tok);
    else s3_compute(a, c, S, pos, T, nch);
    __syncthreads();
    u64 *X = a.xbuf + G2X_HEAD;
    u32x4 wa[UMAX][4];
    lm_pick<_Float16>(a, c, X + (size_t)(a.L - 1) * a.xlayer + G3X_X2(a.E, a.NH), X + (size_t)a.L * a.xlayer, wa,
                      false, S.xr0, S.xin, S.part, red, amv, ami, (lds_flag *)&flag);
}

#undef TRACE3

} /* namespace g2step */

extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step3_f16(const g2_step_args a)
{
    g2step::step3_impl(a);
}
