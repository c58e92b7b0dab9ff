/*
 * g2_step.hip -- one GPT-2 decode forward as a single persistent cooperative
 * kernel (included by g2_kernels.hip, which provides the shared helpers).
 *
 * Why one kernel: on gfx950 every kernel boundary costs several
 * microseconds (wave start-up, drain, the end-of-kernel L2 write-back of the
 * 8 XCDs), and the multi-kernel decode crosses five of them per layer.  Here
 * one launch runs every layer: each work-group (one per CU) owns fixed rows
 * of every matrix, and work-groups hand the activation vectors to each other
 * through exchange areas.
 *
 * Exchange protocol, tagged words (q/k/v, attention partials, argmax): a
 * producer stores (tag << 32 | float bits) with a relaxed agent-scope
 * atomic store; a consumer loads the words with relaxed agent-scope atomic
 * loads (coherent across XCDs) until every tag equals this step's tag.
 * Each word carries its own validity, so no fence is needed (an agent-scope
 * release/acquire writes back or invalidates the XCD L2 and costs
 * microseconds).  Every word is written at most once per launch; the tag is
 * state[G2S_SEQ] + 1 and work-group 0 advances G2S_SEQ at the end of the
 * step, so words left by earlier steps never match.
 *
 * Plain values (the O, X1, H and X2 vectors, which every work-group of a
 * phase reads whole): half the bytes of tagged words.  Each layer has two
 * value regions; the step with tag t writes region t & 1 and empties the
 * same entries of the other region (G2V_EMPTY), which the next step
 * writes.  A consumer re-reads an entry until it is no longer empty.  After
 * a step that gave up a wait or did not run, the host empties both regions.
 *
 * The KV cache entries of the current position reach the attention through
 * the exchange area; the cache itself is read only at earlier positions,
 * which earlier launches wrote.
 *
 * Memory-level parallelism: a work-group's weight rows of a matrix are
 * loaded into registers as soon as the previous matrix held by the same
 * register set has been used (one set for qkv -> fc -> fc2 -> next qkv, a
 * small one for proj), so the weight stream runs while the work-group waits
 * for its next input vector.
 *
 * Phases per layer (input -> output, each a hand-off between work-groups):
 *   QKV   x (X2 of the layer before, or the embedding) -> LayerNorm ->
 *         qkv rows; writes q/k/v to the exchange and k/v to the KV cache
 *   ATTN  (head, 64-position chunk) units -> (max, sum, o[64]) partials
 *         (scores scaled by log2(e): the maxima are in base-2 units and the
 *         exponentials are single v_exp_f32 instructions)
 *   MERGE one work-group per head -> O
 *   PROJ  O -> proj rows + bias + x -> X1
 *   FC    X1 -> LayerNorm -> fc rows + bias -> GELU -> H
 *   FC2   H -> fc2 rows + bias + X1 -> X2
 * then LM (LayerNorm + logits over the tied head + per-work-group first-max)
 * and the greedy pick by work-group 0, which advances the device state.
 * Each LayerNorm is folded into the matrix that follows it (ln_fold_in):
 * the dot products start on (x - x[0]) * gain while the statistics are
 * reduced, and each row is corrected after them with the per-row sums
 * c1 = W . gain, c2 = W . bias_ln + bias computed once per model.
 *
 * Every wait is bounded in time: a wait that runs out (100 ms) sets
 * G2_ERR_STEP_TIMEOUT in the state and raises the abort word, after which
 * every wait of every work-group returns at once, so the grid always
 * drains.  No wait may depend on a work-group that has not started, so all
 * work-groups must be resident at once.  A cooperative launch guarantees
 * that; a plain launch (a.plain, ~17 us less between back-to-back steps)
 * is checked instead: each work-group posts an arrival word at its start
 * and, before its first lasting write, confirms that every work-group has
 * arrived and none gave up (grid_resident); otherwise the launch writes
 * nothing, sets G2_ERR_STEP_NOT_RESIDENT and the host resumes the run with
 * cooperative launches.
 */

namespace g2step {

constexpr int NT = G2_STEP_THREADS;                     /* 512 threads    */
constexpr int NW = NT / 64;                             /* 8 waves        */
constexpr int UMAX = 4;                                 /* units per wave, main set */
constexpr int UPROJ = 1;                                /* units per wave, proj set */
constexpr int SEGC = 256;                               /* chunks per unit: 64 lanes x 4 */
constexpr int QMAX = (G2_STEP_MAXF + 4 * NT - 1) / (4 * NT); /* value quads per thread */
constexpr unsigned long long WAIT_LIMIT = 10000000ull;  /* 100 ms of the 100 MHz clock */
constexpr unsigned long long ABORT_CHECK_AFTER = 200000ull; /* 2 ms */

typedef unsigned long long u64;

/* Pointers read from the per-layer table are generic; device memory
 * accessed through them must be addressed as global so the compiler emits
 * global (not flat) loads: flat loads also count against the LDS counter,
 * which would make every LDS access and barrier wait for the weight stream. */
#define G2_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const G2_GLOBAL T *gl(const T *p) { return (const G2_GLOBAL T *)p; }
template <typename T>
__device__ __forceinline__ G2_GLOBAL T *glw(T *p) { return (G2_GLOBAL T *)p; }
/* LDS flags likewise: through a generic pointer they become flat accesses,
 * which wait for every outstanding global load. */
#define G2_LDS __attribute__((address_space(3)))
/* The per-layer table is read-only for the whole launch: reading it through
 * the constant address space lets the compiler use scalar loads, so weight
 * addresses are a scalar base plus a lane offset (no vector-loaded pointer
 * whose wait would be merged into every weight load). */
#define G2_CONST __attribute__((address_space(4)))
typedef G2_LDS volatile int lds_flag;

__device__ __forceinline__ void ll_put(u64 *p, float v, unsigned tag)
{
    __hip_atomic_store(p, ((u64)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 ll_get(const u64 *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ll_tag(u64 w) { return (unsigned)(w >> 32); }
__device__ __forceinline__ float ll_val(u64 w) { return __uint_as_float((unsigned)w); }

/* Wave-wide sum / max through DPP lane moves (no LDS traffic): butterfly
 * within quads, rotations within 16-lane rows, then the four row results
 * combined in row order.  Every lane gets the result. */
template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_lane(float v, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ float wsum(float v)
{
    v += dpp<0xB1>(v);  /* quad_perm [1,0,3,2] */
    v += dpp<0x4E>(v);  /* quad_perm [2,3,0,1] */
    v += dpp<0x124>(v); /* row_ror:4 */
    v += dpp<0x128>(v); /* row_ror:8 */
    return ((row_lane(v, 0) + row_lane(v, 16)) + row_lane(v, 32)) + row_lane(v, 48);
}
__device__ __forceinline__ float wmax(float v)
{
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x124>(v));
    v = fmaxf(v, dpp<0x128>(v));
    return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 16)), fmaxf(row_lane(v, 32), row_lane(v, 48)));
}

/* Wave sums of four per-lane values at once (a transposed reduction):
 * lanes 32-63 of a are swapped with lanes 0-31 of b, and of c with d
 * (v_permlane32_swap), the pairs added; then odd rows of (a,b) with even
 * rows of (c,d) (v_permlane16_swap), added; then each 16-lane row summed by
 * rotations.  Returns, in every lane of row 0 / 1 / 2 / 3 (lanes 0-15,
 * 16-31, 32-47, 48-63), the total of a / c / b / d. */
__device__ __forceinline__ float wsum4(float a, float b, float c, float d)
{
    const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    const float ab = __uint_as_float(s1[0]) + __uint_as_float(s1[1]);
    const auto s2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(d), false, false);
    const float cd = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
    const auto s3 = __builtin_amdgcn_permlane16_swap(__float_as_uint(ab), __float_as_uint(cd), false, false);
    float v = __uint_as_float(s3[0]) + __uint_as_float(s3[1]);
    v += dpp<0x128>(v); /* row_ror:8 */
    v += dpp<0x124>(v); /* row_ror:4 */
    v += dpp<0x122>(v); /* row_ror:2 */
    return v + dpp<0x121>(v); /* row_ror:1 */
}

struct ctx {
    unsigned tag;
    u64 *abort_w;
    int *state;
    lds_flag *dead; /* this work-group stopped waiting */
};

/* A wait ran out of time: record it and release every work-group. */
__device__ __noinline__ void give_up(const ctx &c)
{
    atomicOr(c.state + G2S_ERR, G2_ERR_STEP_TIMEOUT);
    ll_put(c.abort_w, 0.f, c.tag);
    *c.dead = 1;
}

/* Two tagged words src[w], src[w + 1] (w even) with one 16-byte load, with
 * the cache policy of ll_get (sc1: read at the coherence point, as the
 * relaxed agent-scope loads are), through a buffer resource over the
 * vector; each 8-byte word of the pair is read whole.  The low halves (.x,
 * .z) are the values, the high halves (.y, .w) the tags: half the requests
 * of word-wise reads. */
__device__ __forceinline__ u32x4 ll_get2(__amdgpu_buffer_rsrc_t r, int w)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, w * 8, 0, 16 /* sc1 */);
}
__device__ __forceinline__ bool pair_stale(const u32x4 &v, unsigned tag) { return v.y != tag || v.w != tag; }

/* Bounded wait on word pairs already loaded into v[]: reload the pairs
 * whose tags are stale (with a short back-off) until all match, the abort
 * word is raised or time runs out.  Pair i starts at word idx(i) (< 0: an
 * unused slot, which holds a current filler). */
template <int NP2, typename IDX>
__device__ __forceinline__ void settle2(const ctx &c, __amdgpu_buffer_rsrc_t r, u32x4 (&v)[NP2], IDX idx)
{
    unsigned bad = 0;
#pragma unroll
    for (int i = 0; i < NP2; ++i) bad |= (unsigned)pair_stale(v[i], c.tag);
    if (!bad || *c.dead) return;
    const u64 t0 = wall_clock64();
    for (;;) {
        __builtin_amdgcn_s_sleep(4);
#pragma unroll
        for (int i = 0; i < NP2; ++i) {
            const int w = idx(i);
            if (w >= 0 && pair_stale(v[i], c.tag)) v[i] = ll_get2(r, w);
        }
        bad = 0;
#pragma unroll
        for (int i = 0; i < NP2; ++i) bad |= (unsigned)pair_stale(v[i], c.tag);
        if (!bad || *c.dead) return;
        /* the abort word is consulted only by waits that already took long */
        const u64 el = wall_clock64() - t0;
        if (el > ABORT_CHECK_AFTER) {
            if (ll_tag(ll_get(c.abort_w)) == c.tag) { *c.dead = 1; return; }
            if (el > WAIT_LIMIT) { give_up(c); return; }
        }
    }
}

/* All threads: dst[w] = value of src[w] for w < n once it carries the tag,
 * read by 16-byte word pairs (n <= 2*NT*NP2 <= 4*NT even, src at an even
 * word): thread tid takes pairs tid + NT*i (words 2p, 2p + 1) after one
 * speculative read and polls its own stale pairs, so a word is seen one
 * round trip after it lands.  Ends with a barrier. */
template <int NP2>
__device__ __forceinline__ void fetch2(int tid, const ctx &c, const u64 *src, int n, float *dst)
{
    static_assert(NP2 <= 2, "small vectors only");
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, n * 8, 0x00020000);
    const u32x4 filler = (u32x4){0u, c.tag, 0u, c.tag};
    u32x4 v[NP2];
#pragma unroll
    for (int i = 0; i < NP2; ++i) {
        const int w = 2 * (tid + NT * i);
        v[i] = w < n ? ll_get2(r, w) : filler;
    }
    settle2(c, r, v, [&](int i) { const int w = 2 * (tid + NT * i); return w < n ? w : -1; });
#pragma unroll
    for (int i = 0; i < NP2; ++i) {
        const int w = 2 * (tid + NT * i);
        if (w < n) {
            dst[w] = __uint_as_float(v[i].x);
            dst[w + 1] = __uint_as_float(v[i].z);
        }
    }
    __syncthreads();
}

/* Plain values (O, X1, H, X2): a producer stores the float of this step
 * into the region of the step's tag parity and G2V_EMPTY into the same entry
 * of the other region, which the next step fills; the kernel boundary
 * between steps makes those stores visible, so a consumer sees the
 * entries of its region either empty or holding this step's value.  Both
 * stores are relaxed agent-scope atomics, as ll_put's.  A result whose bits
 * equal G2V_EMPTY (only a NaN could) is stored as the canonical NaN. */
__device__ __forceinline__ void vput(float *cur, float *nxt, float v)
{
    unsigned b = __float_as_uint(v);
    b = b == G2V_EMPTY ? 0x7FC00000u : b;
    __hip_atomic_store((unsigned *)cur, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store((unsigned *)nxt, G2V_EMPTY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Values 4q .. 4q + 3 with one 16-byte load through a buffer resource over
 * the vector, with the cache policy of ll_get (sc1: read at the coherence
 * point, as the relaxed agent-scope loads are); each 4-byte value is read
 * whole.  Four values per request: a wave issues requests at a bounded
 * rate, and the 6400-value H vector is read by every work-group. */
__device__ __forceinline__ u32x4 vq_get(__amdgpu_buffer_rsrc_t r, int q)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, q * 16, 0, 16 /* sc1 */);
}
__device__ __forceinline__ bool quad_empty(const u32x4 &v)
{
    return v.x == G2V_EMPTY || v.y == G2V_EMPTY || v.z == G2V_EMPTY || v.w == G2V_EMPTY;
}

/* settle2 (above) for value quads, which are present once no value is
 * G2V_EMPTY: slot i holds quad idx(i) (< 0: an unused slot, which holds a
 * filler). */
template <int NQ, typename IDX>
__device__ __forceinline__ void settle4(const ctx &c, __amdgpu_buffer_rsrc_t r, u32x4 (&v)[NQ], IDX idx)
{
    unsigned bad = 0;
#pragma unroll
    for (int i = 0; i < NQ; ++i) bad |= (unsigned)quad_empty(v[i]);
    if (!bad || *c.dead) return;
    const u64 t0 = wall_clock64();
    for (;;) {
        __builtin_amdgcn_s_sleep(4);
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int q = idx(i);
            if (q >= 0 && quad_empty(v[i])) v[i] = vq_get(r, q);
        }
        bad = 0;
#pragma unroll
        for (int i = 0; i < NQ; ++i) bad |= (unsigned)quad_empty(v[i]);
        if (!bad || *c.dead) return;
        /* the abort word is consulted only by waits that already took long */
        const u64 el = wall_clock64() - t0;
        if (el > ABORT_CHECK_AFTER) {
            if (ll_tag(ll_get(c.abort_w)) == c.tag) { *c.dead = 1; return; }
            if (el > WAIT_LIMIT) { give_up(c); return; }
        }
    }
}

/* All threads: dst[w] = src[w] for w < n once no value is empty, for a
 * vector of plain values, n a multiple of 4 (n_embd is a multiple of 64,
 * the ffn width of the weight chunk), src 16-byte aligned: thread tid takes
 * quads tid + NT*i.  With one quad per thread each thread polls its own
 * empty quad.  Larger vectors must not flood the memory system (the
 * 6400-value H vector is read by every work-group), so a work-group that
 * found empty values first waits on the quads holding value n*k/nsent,
 * k < nsent (the first value of each producer when n is split evenly over
 * nsent producers), then re-reads its empty quads.  Quad tid + NT*i goes
 * to dst + dso[i] (LDS, 16-byte aligned: the padded position of its first
 * value).  Ends with a barrier; `flag` is an LDS word of the caller. */
template <int NQ>
__device__ __forceinline__ void fetch4(int tid, const ctx &c, const float *src, int n, int nsent, float *dst,
                                       const int (&dso)[NQ], lds_flag *flag)
{
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, n * 4, 0x00020000);
    const u32x4 filler = (u32x4){0u, 0u, 0u, 0u};
    u32x4 v[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int q = tid + NT * i;
        v[i] = 4 * q < n ? vq_get(r, q) : filler;
    }
    auto idx = [&](int i) { const int q = tid + NT * i; return 4 * q < n ? q : -1; };
    if constexpr (NQ <= 1) {
        (void)nsent;
        (void)flag;
        settle4(c, r, v, idx);
    } else {
        if (tid == 0) *flag = 0;
        __syncthreads();
        unsigned bad = 0;
#pragma unroll
        for (int i = 0; i < NQ; ++i) bad |= (unsigned)quad_empty(v[i]);
        if (bad) *flag = 1;
        __syncthreads();
        if (*flag && !*c.dead) {
            if (tid < nsent) {
                const int q = (int)(((long)n * tid) / nsent) >> 2;
                u32x4 sv[1] = {vq_get(r, q)};
                settle4(c, r, sv, [&](int) { return q; });
            }
            __syncthreads();
            settle4(c, r, v, idx);
        }
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int q = tid + NT * i;
        if (4 * q < n) *(u32x4 *)(dst + dso[i]) = v[i];
    }
    __syncthreads();
}

/* A vector of n <= 4*NT values with LayerNorm to follow: thread tid takes
 * quad tid (values 4tid .. 4tid + 3, present when 4tid < n) and keeps it in
 * registers; it also reads quad 0, whose first value is the shift of the
 * LayerNorm's sums, so no thread waits for another to learn it.  The quad
 * is also stored to dst[4tid..] (LDS) for the phase's residual; the
 * LayerNorm's first barrier makes it visible. */
__device__ __forceinline__ f32x4 fetch_q(int tid, const ctx &c, const float *src, int n, float *dst, float &x0)
{
    static_assert(G2_STEP_MAXE <= 4 * NT, "one quad per thread");
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, n * 4, 0x00020000);
    const bool on = 4 * tid < n;
    u32x4 v[2];
    v[0] = on ? vq_get(r, tid) : (u32x4){0u, 0u, 0u, 0u};
    v[1] = vq_get(r, 0);
    settle4(c, r, v, [&](int i) { return i == 1 ? 0 : (on ? tid : -1); });
    if (on) *(u32x4 *)(dst + 4 * tid) = v[0];
    x0 = __uint_as_float(v[1].x);
    return __builtin_bit_cast(f32x4, v[0]);
}

/* LayerNorm gain of the thread's quad (clamped: quads past E are never
 * stored), loaded at the start of a phase so its latency overlaps the input
 * wait; the bias is folded into the matrix's c2. */
__device__ __forceinline__ f32x4 ln_gload(int tid, const float *g, int E)
{
    return gl((const f32x4 *)g)[min(tid, E / 4 - 1)];
}

/* The LayerNorm folded into the matrix that follows it (layernorm,
 * math.cl:283-311: (x - mean) * inv_std * g + b with the biased variance,
 * eps 1e-5), by W . LN(x) + bias = inv * (W . ((x - x0) * g) - (mean - x0) *
 * c1) + c2 with c1 = W . g, c2 = W . b + bias (g2k_ln_fold), x0 = x[0].
 * ln_fold_in writes the matrix input (x - x0) * g of the thread's quad
 * (entries 4tid .. 4tid + 3 of x, held in registers) to xin at xo (their
 * padded position, g2p_x_slot) and each wave's
 * sums of d = x - x0 and d^2 to red (a shift that keeps the variance E[d^2]
 * - E[d]^2 free of cancellation when |mean| >> std); ends with a barrier,
 * after which the dot products may start while ln_fold_stats reads the
 * sums (wave totals added in wave order). */
__device__ __forceinline__ void ln_fold_in(int tid, const f32x4 &x, float x0, const f32x4 &g, int E, float *xin,
                                           int xo, float *red)
{
    const bool on = 4 * tid < E;
    float s = 0.f, q = 0.f;
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float d = on ? x[e] - x0 : 0.f;
        s += d;
        q = fmaf(d, d, q);
        o[e] = d * g[e];
    }
    if (on) *(f32x4 *)(xin + xo) = o;
    s = wsum(s);
    q = wsum(q);
    if ((tid & 63) == 0) {
        red[tid >> 6] = s;
        red[NW + (tid >> 6)] = q;
    }
    __syncthreads();
}
struct ln_st {
    float md, inv; /* mean - x0, 1 / sqrt(var + eps) */
};
__device__ __forceinline__ ln_st ln_fold_stats(const float *red, int E)
{
    float S = red[0], Q = red[NW];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        S += red[w];
        Q += red[NW + w];
    }
    ln_st st;
    const float rE = 1.0f / (float)E;
    st.md = S * rE;
    const float var = fmaxf(Q * rE - st.md * st.md, 0.f);
    st.inv = __builtin_amdgcn_rsqf(var + 1e-5f); /* v_rsq_f32 */
    return st;
}
/* row value of a folded LayerNorm from its dot product v with (x - x0) * g */
__device__ __forceinline__ float ln_fold_out(const ln_st &st, float v, float c1, float c2)
{
    return fmaf(st.inv, fmaf(-st.md, c1, v), c2);
}

/* A work-group's share of one packed matrix W[N,K] (output-major): rows
 * [r0, r0+nrows), each split into nseg (1, 2, 4 or 8: a divisor of the wave
 * count, so every unit of a wave has the segment wave % nseg) segments of
 * SL <= 256 16-byte chunks; a (row, segment) unit is one wave's job (64
 * lanes x up to 4 chunks).  With
 * a register set of UM units per wave, unit u belongs to wave u % NW, slot
 * (u / NW) % UM, batch u / (NW * UM). */
struct plan : g2p_rows {
    const u32x4 *W;
};

/* Row plan k (G2P_SH_QKV .. G2P_SH_LM) of this work-group, from the host's
 * per-work-group table (g2p_shares), read where a phase needs it: the table
 * address is made opaque to the compiler, so each use is one scalar load
 * instead of all five plans held in scalar registers across the layers. */
__device__ __forceinline__ g2p_rows row_plan(const g2_step_args &a, int k)
{
    const G2_CONST g2p_rows *p = (const G2_CONST g2p_rows *)a.shares + (size_t)blockIdx.x * G2P_NSHARES + k;
    asm volatile("" : "+s"(p));
    return *p;
}

/* row_plan with the fields that depend only on the matrix shape (chunks
 * per row, segments, segment length, tail) computed from the sizes of
 * shape SH, so the compiler folds them; the work-group's rows and units
 * still come from the table. */
template <typename WT, int SH>
__device__ __forceinline__ g2p_rows row_plan_x(const g2_step_args &a, int k)
{
    if constexpr (SH != 0) {
        /* computed from the shape's sizes and the 256-work-group grid (the
         * kernel refuses another), with the work-group index made opaque to
         * the compiler so the plan is recomputed where it is used */
        int w = (int)blockIdx.x;
        asm volatile("" : "+s"(w));
        constexpr int E = G2P_SHAPE_E(SH), F = G2P_SHAPE_F(SH), NH = G2P_SHAPE_NH(SH), V = G2P_SHAPE_V;
        constexpr int VE = chunk_t<WT>::V, NWG = G2P_SHAPE_WGS;
        if (k == G2P_SH_QKV) return g2p_rows_plan(3 * E, E, VE, w, NWG);
        if (k == G2P_SH_PROJ) return g2p_proj_plan(E, VE, NH, w, NWG);
        if (k == G2P_SH_FC) return g2p_rows_plan(F, E, VE, w, NWG);
        if (k == G2P_SH_FC2) return g2p_rows_plan(E, F, VE, w, NWG);
        return g2p_rows_plan(V, E, VE, w, NWG);
    } else {
        return row_plan(a, k);
    }
}

__device__ __forceinline__ plan make_plan(const void *W, const g2p_rows &r)
{
    plan p;
    static_cast<g2p_rows &>(p) = r;
    p.W = (const u32x4 *)W;
    return p;
}

/* Issue the loads of one batch (NW*UM units) into a register set.  The
 * loads are unconditional, every address clamped into the work-group's
 * share (lanes past a segment end to its last chunk, which the same
 * instruction fetches anyway; units past the share to its first row): a
 * load under a lane condition makes the compiler wait for every load in
 * flight before the value is first used.  Dot products ignore the clamped
 * chunks (their x is zero) and the units past the share. */
template <int UM, bool TAIL>
__device__ __forceinline__ void load_set(int tid, u32x4 (&w)[UM][4], const plan &p, int batch)
{
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    /* the tail form (every four-unit plan a tail plan) packs slot 3 of the
     * four units into w[0][3] */
    constexpr bool tail = TAIL && UM == 4;
#pragma unroll
    for (int j = 0; j < UM; ++j) {
        const g2p_unit un = g2p_unit_at(&p, UM, batch, wave, j);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (tail && i == 3) continue;
            /* a unit past the share reads one chunk with every lane (one line) */
            w[j][i] = __builtin_nontemporal_load(gl(p.W) + g2p_unit_chunk(&un, lane, i));
        }
    }
    if constexpr (tail) w[0][3] = __builtin_nontemporal_load(gl(p.W) + g2p_tail_chunk(&p, batch, wave, lane));
}

/* acc + (16-byte chunk of weights) . x, as one fma chain element by element */
template <typename WT>
__device__ __forceinline__ float chunk_fma(const u32x4 &w, const float *x, float acc)
{
    if constexpr (sizeof(WT) == 4) {
        acc = fmaf(__uint_as_float(w.x), x[0], acc);
        acc = fmaf(__uint_as_float(w.y), x[1], acc);
        acc = fmaf(__uint_as_float(w.z), x[2], acc);
        return fmaf(__uint_as_float(w.w), x[3], acc);
    } else {
        const f16x8 h = __builtin_bit_cast(f16x8, w);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf((float)h[e], x[e], acc);
        return acc;
    }
}

/* Dot products of a loaded batch with xin (LDS, the padded layout of
 * g2p_dot_x: a chunk past the segment holds zeros); unit sums to part[u].
 * Every unit of the wave covers the same chunks of x, so they are read from
 * LDS once, all at once and unconditionally (a read under a lane condition
 * would be waited for on its own).  The units' sums are independent fma
 * chains, interleaved chunk by chunk. */
template <typename WT, int UM, bool TAIL>
__device__ __forceinline__ void dot_set(int tid, const u32x4 (&w)[UM][4], const plan &p, int batch,
                                        const float *xin, float *part)
{
    constexpr int VE = chunk_t<WT>::V;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    if (batch * NW * UM + wave >= p.nunits) return; /* wave-uniform */
    float xv[4][VE];
    const int xo = g2p_dot_x(&p, VE, wave, lane, 0);
    /* slot 3 of a tail plan multiplies the packed chunks */
    const int x3 = (UM == 4 && TAIL) ? g2p_tail_x(&p, VE, wave, lane) : xo + 3 * 64 * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int e = 0; e < VE; e += 4) {
            const f32x4 v = *(const f32x4 *)(xin + g2p_x_elem(i == 3 ? x3 : xo + 64 * 4 * i, VE, e));
            xv[i][e] = v.x;
            xv[i][e + 1] = v.y;
            xv[i][e + 2] = v.z;
            xv[i][e + 3] = v.w;
        }
    }
    if constexpr (UM == 4) {
        /* the four units' sums in one transposed reduction: unit j's total
         * lands in row (0, 2, 1, 3)[j] of the wave.  Only the wave's units
         * inside the share are multiplied (nv of its four slots, a
         * wave-uniform count), so a share of fewer than 32 units costs its
         * waves no products for their empty slots. */
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        const int nv = (p.nunits - batch * NW * UM - wave + NW - 1) / NW; /* >= 1 here */
        /* a tail plan: slots 0-2 per unit, then the packed slot 3 (one
         * chain for all four units), each lane's sum added to its unit */
        auto prods = [&](auto nvc) {
            constexpr int NV = decltype(nvc)::value;
            if constexpr (TAIL) {
#pragma unroll
                for (int i = 0; i < 3; ++i)
#pragma unroll
                    for (int j = 0; j < NV; ++j) acc[j] = chunk_fma<WT>(w[j][i], xv[i], acc[j]);
                const float tl = chunk_fma<WT>(w[0][3], xv[3], 0.f);
                const int tj = lane >> 4;
#pragma unroll
                for (int j = 0; j < NV; ++j) acc[j] += tj == j ? tl : 0.f;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < NV; ++j) acc[j] = chunk_fma<WT>(w[j][i], xv[i], acc[j]);
            }
        };
        if (nv >= 4) prods(std::integral_constant<int, 4>{});
        else if (nv == 3) prods(std::integral_constant<int, 3>{});
        else if (nv == 2) prods(std::integral_constant<int, 2>{});
        else prods(std::integral_constant<int, 1>{});
        const float v = wsum4(acc[0], acc[1], acc[2], acc[3]);
        if ((lane & 15) == 0) {
            const int j = (lane >> 4) == 0 ? 0 : ((lane >> 4) == 1 ? 2 : ((lane >> 4) == 2 ? 1 : 3));
            const int u = batch * NW * UM + wave + NW * j;
            if (u < p.nunits) part[u] = v;
        }
    } else {
#pragma unroll
        for (int j = 0; j < UM; ++j) {
            const int u = batch * NW * UM + wave + NW * j;
            if (u >= p.nunits) break; /* wave-uniform */
            /* one chain per chunk, summed in chunk order */
            float a4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a4[i] = chunk_fma<WT>(w[j][i], xv[i], 0.f);
            float acc = ((a4[0] + a4[1]) + a4[2]) + a4[3];
            acc = wsum(acc);
            if (lane == 0) part[u] = acc;
        }
    }
}

/* The whole matrix share: batch 0 from the preloaded set, later batches
 * loaded on demand into the same set.  Ends with a barrier. */
template <typename WT, int UM, bool TAIL>
__device__ __forceinline__ void matvec(int tid, u32x4 (&w)[UM][4], const plan &p, const float *xin,
                                       float *part)
{
    dot_set<WT, UM, TAIL>(tid, w, p, 0, xin, part);
    for (int b = 1; b * NW * UM < p.nunits; ++b) {
        load_set<UM, TAIL>(tid, w, p, b);
        dot_set<WT, UM, TAIL>(tid, w, p, b, xin, part);
    }
    __syncthreads();
}

/* Row t's dot product from its segment sums (in segment order). */
__device__ __forceinline__ float row_sum(const plan &p, const float *part, int t)
{
    float v = part[t * p.nseg];
    for (int s = 1; s < p.nseg; ++s) v += part[t * p.nseg + s];
    return v;
}

/* Per-half LDS of the attention phase. */
struct att_lds {
    float q[64], kn[64], vn[64];
    float red[4][64]; /* per wave of the half: its 64 partial sums */
    float pr[64];
    float stat[2];
};

/* The first step of wsum4: in every lane of row 0 / 1 / 2 / 3 (lanes 0-15,
 * 16-31, 32-47, 48-63), the sum over the four rows of a / c / b / d at the
 * lane's position in its row (lane % 16). */
__device__ __forceinline__ float xsum4(float a, float b, float c, float d)
{
    const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    const float ab = __uint_as_float(s1[0]) + __uint_as_float(s1[1]);
    const auto s2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(d), false, false);
    const float cd = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
    const auto s3 = __builtin_amdgcn_permlane16_swap(__float_as_uint(ab), __float_as_uint(cd), false, false);
    return __uint_as_float(s3[0]) + __uint_as_float(s3[1]);
}

/* Cached keys and values of one 64-position chunk, loaded into registers
 * ahead of their use (they do not depend on this position's q), both
 * before the q/k/v wait: the keys (attn_load), then the values
 * (attn_load_v).
 * Scores: thread (pq = t%16, dg = t/16) of a half takes positions
 * j0+4pq..+3 and dims 4dg..+3 (four 16-byte loads of the transposed K
 * cache); weighted sum: thread (d4 = t%16, jg = t/16) takes dims 4d4..+3
 * and positions j0+4jg..+3 (four 16-byte loads of the V cache).  The
 * current position's entries are replaced by the exchanged k and v. */
struct att_regs {
    f32x4 kv[4], vv[4];
};

__device__ __forceinline__ void attn_load(int tid, const G2_CONST g2_step_layer *y, att_regs &r, bool on, int h,
                                          int ch, int pos, int T, int E, int S)
{
    const int t = tid & 255;
    const int j0 = ch * 64;
    const int pq = t & 15, dg = t >> 4, jk = j0 + 4 * pq;
    const int d4 = t & 15, jg = t >> 4;
    /* unconditional: every address is inside the caches (positions < S =
     * 1024, dims < E); values of positions >= T or of the current position
     * are never used.  Skipping loads under a lane mask would make the
     * compiler wait for all of the wave's earlier stores first.  A half
     * without a unit points every lane at the first 16 bytes of the caches,
     * so its loads cost one line each instead of 32 KB of memory traffic
     * queued in front of the work-group's later reads. */
    (void)T; (void)pos; (void)j0; (void)pq; (void)dg; (void)jk; (void)d4; (void)jg;
    long koff, voff[4];
    g2p_attn_offsets(t, on, h, ch, E, S, &koff, voff);
    const size_t kstr = on ? (size_t)(S / 4) : 0;
    const G2_GLOBAL f32x4 *kb = gl((const f32x4 *)(y->k_cache + koff));
#pragma unroll
    for (int d = 0; d < 4; ++d) r.kv[d] = kb[(size_t)d * kstr];
}
/* The values of the same chunk (needed only after the scores and the
 * softmax).  Issued behind the keys and ahead of the q/k/v wait: the q/k/v
 * reads then queue behind both, which costs nothing measurable at
 * E = 1600 and takes the value latency off the layer's attention chain at
 * E = 768..1280, where a work-group has few units. */
__device__ __forceinline__ void attn_load_v(int tid, const G2_CONST g2_step_layer *y, att_regs &r, bool on, int h,
                                            int ch, int E, int S)
{
    long koff, voff[4];
    g2p_attn_offsets(tid & 255, on, h, ch, E, S, &koff, voff);
#pragma unroll
    for (int e = 0; e < 4; ++e) r.vv[e] = *gl((const f32x4 *)(y->v_cache + voff[e]));
}

/* The attention of one 64-position chunk once L.q, L.kn and L.vn hold the
 * head's q, k and v at this position (by the 256 threads of one half; t =
 * thread in the half): the computation of g2k_attn_part, with the current
 * position's key and value taken from L; the chunk's (max, sum, o[64]) go
 * to pout[0..65].  `on` is false for a half without a unit; it still takes
 * part in the three barriers. */
__device__ __forceinline__ void attn_compute(int tid, const ctx &c, float scale, u64 *pout, att_lds &L,
                                             const att_regs &r, bool on, int ch, int pos, int T)
{
    const int t = tid & 255;
    const int j0 = ch * 64;
    const int pq = t & 15, dg = t >> 4, jk = j0 + 4 * pq;
    const int d4 = t & 15, jg = t >> 4;
    if (on) {
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        if (jk < T) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                f32x4 kv = r.kv[d];
                if (pos >= jk && pos < jk + 4) kv[pos - jk] = L.kn[4 * dg + d];
                const float qv = L.q[4 * dg + d];
                s[0] = fmaf(qv, kv.x, s[0]);
                s[1] = fmaf(qv, kv.y, s[1]);
                s[2] = fmaf(qv, kv.z, s[2]);
                s[3] = fmaf(qv, kv.w, s[3]);
            }
        }
        /* the wave's four dimension groups (lane rows) summed by lane
         * swaps: row r holds position 4 pq + (0, 2, 1, 3)[r] */
        const int rr = (t >> 4) & 3;
        L.red[t >> 6][4 * pq + (rr == 1 ? 2 : (rr == 2 ? 1 : rr))] = xsum4(s[0], s[1], s[2], s[3]);
    }
    __syncthreads();
    if (on && t < 64) {
        const bool ok = j0 + t < T;
        float s = ((L.red[0][t] + L.red[1][t]) + L.red[2][t]) + L.red[3][t];
        s *= scale; /* scale carries log2(e): scores in base-2 units */
        const float m = wmax(ok ? s : -INFINITY);
        const float p = ok ? __builtin_amdgcn_exp2f(s - m) : 0.f; /* v_exp_f32 */
        const float l = wsum(p);
        L.pr[t] = p;
        if (t == 0) { L.stat[0] = m; L.stat[1] = l; }
    }
    __syncthreads();
    if (on) {
        float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int jj = 4 * jg + e, j = j0 + jj;
            if (j < T) {
                const float p = L.pr[jj];
                f32x4 v = r.vv[e];
                if (j == pos) v = (f32x4){L.vn[4 * d4], L.vn[4 * d4 + 1], L.vn[4 * d4 + 2], L.vn[4 * d4 + 3]};
                o[0] = fmaf(p, v.x, o[0]);
                o[1] = fmaf(p, v.y, o[1]);
                o[2] = fmaf(p, v.z, o[2]);
                o[3] = fmaf(p, v.w, o[3]);
            }
        }
        /* the wave's four position groups summed the same way: row r
         * holds dimension 4 d4 + (0, 2, 1, 3)[r] */
        const int rr = (t >> 4) & 3;
        L.red[t >> 6][4 * d4 + (rr == 1 ? 2 : (rr == 2 ? 1 : rr))] = xsum4(o[0], o[1], o[2], o[3]);
    }
    __syncthreads();
    if (on && t < 64) {
        const float o = ((L.red[0][t] + L.red[1][t]) + L.red[2][t]) + L.red[3][t];
        ll_put(pout + 2 + t, o, c.tag);
        if (t == 0) {
            ll_put(pout, L.stat[0], c.tag);
            ll_put(pout + 1, L.stat[1], c.tag);
        }
    }
}


/* One 64-position chunk c of single-query attention for head h by the 256
 * threads of one half of the work-group (t = thread in the half): the
 * computation of g2k_attn_part, with the current position's key and value
 * taken from the exchange; the chunk's (max, sum, o[64]) go to pout[0..65].
 * `on` is false for a half without a unit; it still takes part in the
 * barriers. */
__device__ __forceinline__ void attn_chunk(int tid, const ctx &c, float scale, const u64 *src, int qo,
                                           int ko, int vo, u64 *pout, att_lds &L, const att_regs &r, bool on,
                                           int ch, int pos, int T)
{
    const int t = tid & 255;
    /* q, k and v of the head at this position: src[qo + d], src[ko + d],
     * src[vo + d], as word pairs (qo, ko, vo and the region are at even
     * words) */
    if (on && t < 96) {
        const int part = t >> 5, d = 2 * (t & 31);
        const int w = (part == 0 ? qo : (part == 1 ? ko : vo)) + d;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, (vo + 64) * 8, 0x00020000);
        u32x4 v[1] = {ll_get2(rs, w)};
        settle2(c, rs, v, [&](int) { return w; });
        float *dst = part == 0 ? L.q : (part == 1 ? L.kn : L.vn);
        dst[d] = __uint_as_float(v[0].x);
        dst[d + 1] = __uint_as_float(v[0].z);
    }
    __syncthreads();
    attn_compute(tid, c, scale, pout, L, r, on, ch, pos, T);
}

__device__ __forceinline__ bool am_better2(float v1, int i1, float v2, int i2)
{
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

/* First-max over the work-group's (bv, bi); result in amv[0], ami[0].  The
 * order (larger value, then smaller index) is total, so the butterfly within
 * each wave and the pass over the waves' results find the same element as any
 * other reduction order; two barriers instead of one per halving. */
__device__ __forceinline__ void blk_argmax(int tid, float bv, int bi, float *amv, int *ami)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(bv, o);
        const int i2 = __shfl_xor(bi, o);
        if (am_better2(v2, i2, bv, bi)) {
            bv = v2;
            bi = i2;
        }
    }
    if ((tid & 63) == 0) {
        amv[tid >> 6] = bv;
        ami[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NW; ++w)
            if (am_better2(amv[w], ami[w], bv, bi)) {
                bv = amv[w];
                bi = ami[w];
            }
        amv[0] = bv;
        ami[0] = bi;
    }
    __syncthreads();
}

/* Phase timestamps (only when the caller passed a trace buffer). */
/* Phase timestamps, compiled only into the traced kernel variants (TRACED):
 * the untraced ones carry no trace pointer or stamp code in their layer loop. */
#define TRACE(k)                                                                       \
    do {                                                                               \
        if (TRACED && a.trace && tid == 0)                                             \
            a.trace[(size_t)wg * G2_TRACE_STRIDE(a.L) + 24 * l + (k)] = wall_clock64(); \
    } while (0)

/* The thread index as a value the compiler cannot prove loop-invariant:
 * taken fresh in every phase, it keeps per-phase lane arithmetic from being
 * hoisted out of the layer loop (which would hold it in registers across
 * all 48 layers). */
__device__ __forceinline__ int fresh_tid()
{
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

/* Plain launches (not cooperative): before its first lasting write (the
 * K/V cache entries of layer 0), a work-group checks that every work-group
 * of the grid has posted its arrival word, i.e. is resident at the same
 * time.  The launch's verdict is one word decided once, by compare-and-swap
 * on the decision word (its high half the launch's tag): GO by the first
 * work-group that saw every arrival, ABORT by the first whose wait ran out
 * (RESIDENT_LIMIT).  Every work-group follows the stored verdict, so either
 * all of them go on or none writes anything.  GO is safe for a work-group
 * whose own wait ran out: a GO proves every work-group arrived, and none
 * leaves before the verdict, so all were resident together.  On ABORT the
 * work-groups set G2_ERR_STEP_NOT_RESIDENT, raise the abort word and exit;
 * a work-group that only got a CU when another exited finds the verdict
 * already stored.  Returns false for an aborted launch; all threads take
 * part and get the same answer. */
constexpr unsigned long long RESIDENT_LIMIT = 100000ull; /* 1 ms */
constexpr unsigned VERDICT_GO = 1u, VERDICT_ABORT = 2u;

__device__ __forceinline__ bool grid_resident(int tid, const ctx &c, const u64 *arr, u64 *decision, int nwg,
                                              lds_flag *flag)
{
    if (tid == 0) *flag = 0;
    __syncthreads();
    for (int w = tid; w < nwg; w += NT) {
        u64 v = ll_get(arr + w);
        const u64 t0 = wall_clock64();
        while (ll_tag(v) != c.tag) {
            if (wall_clock64() - t0 > RESIDENT_LIMIT) { *flag = 1; break; }
            __builtin_amdgcn_s_sleep(4);
            v = ll_get(arr + w);
        }
    }
    __syncthreads();
    if (tid == 0) {
        const unsigned mine = *flag ? VERDICT_ABORT : VERDICT_GO;
        u64 cur = ll_get(decision);
        while (ll_tag(cur) != c.tag) {
            const u64 want = ((u64)c.tag << 32) | mine;
            const u64 prev = atomicCAS((unsigned long long *)decision, cur, want);
            cur = prev == cur ? want : prev;
        }
        const bool go = (unsigned)cur == VERDICT_GO;
        if (!go) {
            atomicOr(c.state + G2S_ERR, G2_ERR_STEP_NOT_RESIDENT);
            ll_put(c.abort_w, 0.f, c.tag);
            *c.dead = 1;
        }
        *flag = go ? 0 : 1;
    }
    __syncthreads();
    return *flag == 0;
}

/* LM head and greedy pick, the end of every step kernel: X2 of the last
 * layer (xlast: E values from nwg producers) -> LayerNorm_f -> logits of the
 * work-group's head rows -> first-max per work-group (argmax words AM) ->
 * work-group 0 merges them (g2k_argmax_merge with advance) and advances the
 * device state.  All threads of the work-group take part. */
template <typename WT, bool TAIL, bool TRACED>
__device__ __forceinline__ void lm_pick(const g2_step_args &a, const ctx &c, const g2p_rows &plm, const float *xlast, u64 *AM,
                                        u32x4 (&wa)[UMAX][4], bool preloaded, float *xres, float *xe, int xeo,
                                        float *xsc, float *part, float *red, float *amv, int *ami, lds_flag *flag)
{
    /* ---- LM: logits over the head rows, work-group first-max */
    const int tid = fresh_tid();
    const int wg = blockIdx.x, nwg = gridDim.x, l = a.L;
    const int E = a.E, V = a.V;
    const int ngen = a.state[G2S_NGEN], min_new = a.state[G2S_MIN_NEW];
    const int pos = clampi(a.state[G2S_POS], 0, a.S - 1);
    const unsigned seq = (unsigned)a.state[G2S_SEQ];
    const f32x4 gf = ln_gload(tid, a.lnf_w, E);
    const plan p = make_plan(a.lm_w, plm);
    const int rl = min(p.r0 + tid, V - 1); /* used by tid < nrows */
    const float c1 = gl(a.lm_c1)[rl], c2 = gl(a.lm_c2)[rl];
    if (!preloaded) load_set<UMAX, TAIL>(tid, wa, p, 0);
    float x0;
    const f32x4 xq = fetch_q(tid, c, xlast, E, xres, x0);
    TRACE(0);
    ln_fold_in(tid, xq, x0, gf, E, xe, xeo, red);
    matvec<WT, UMAX, TAIL>(tid, wa, p, xe, part);
    const ln_st st = ln_fold_stats(red, E);
    const int masked = ngen < min_new ? G2_EOS_ID : -1;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (tid < p.nrows) {
        const int r = p.r0 + tid;
        const float v = ln_fold_out(st, row_sum(p, part, tid), c1, c2);
        glw(a.logits)[r] = v;
        bv = r == masked ? -1e30f : v;
        bi = r;
    }
    blk_argmax(tid, bv, bi, amv, ami);
    if (tid == 0) {
        ll_put(AM + 2 * wg, amv[0], c.tag);
        ll_put(AM + 2 * wg + 1, __int_as_float(ami[0]), c.tag);
    }
    TRACE(1);
    if (wg != 0) return;

    /* ---- greedy pick (g2k_argmax_merge with advance) */
    __syncthreads();
    fetch2<1>(tid, c, AM, 2 * nwg, xsc); /* nwg <= NT work-groups' word pairs */
    const u64 abort_seen = tid == 0 ? ll_get(c.abort_w) : 0; /* issued ahead of the merge */
    bv = -INFINITY;
    bi = 0x7fffffff;
    for (int b = tid; b < nwg; b += NT) {
        const float v = xsc[2 * b];
        const int i = __float_as_int(xsc[2 * b + 1]);
        if (am_better2(v, i, bv, bi)) { bv = v; bi = i; }
    }
    blk_argmax(tid, bv, bi, amv, ami);
    /* a launch that gave up a wait (its words may be stale) leaves the state
     * as it was; the host reports the failed step */
    if (tid == 0 && !*c.dead && ll_tag(abort_seen) != c.tag) {
        const int tk = (ami[0] >= 0 && ami[0] < V) ? ami[0] : 0;
        const int ng = clampi(ngen, 0, G2S_WORDS - G2S_IDS - 1);
        a.state[G2S_IDS + ng] = tk;
        a.state[G2S_TOK] = tk;
        a.state[G2S_NGEN] = ng + 1;
        a.state[G2S_POS] = pos + 1;
        a.state[G2S_SEQ] = (int)(seq + 1u);
    }
    TRACE(2);
}

template <typename WT, bool TAIL, bool TRACED, int SH>
__device__ __forceinline__ void step_impl(const g2_step_args &a)
{
    /* 16-byte alignment: the dot products read 16-byte chunks of these */
    /* matrix inputs in the padded layout (g2p_x_slot): K = n_embd, K = ffn */
    __shared__ __attribute__((aligned(16))) float xe[G2P_XE_FLOATS];
    __shared__ __attribute__((aligned(16))) float xf[G2P_XF_FLOATS];
    /* words fetched by the head merge and the pick */
    __shared__ __attribute__((aligned(16))) float xsc[G2_STEP_MAXCH * 66 > 2 * NT ? G2_STEP_MAXCH * 66 : 2 * NT];
    __shared__ __attribute__((aligned(16))) float xres[G2_STEP_MAXE];
    __shared__ float part[G2_STEP_MAXUNITS];
    __shared__ float red[2 * NW];
    __shared__ att_lds att[2];
    __shared__ float amv[NT];
    __shared__ int ami[NT];
    __shared__ volatile int dead;
    __shared__ volatile int flag;

    constexpr int NQE = (G2_STEP_MAXE + 4 * NT - 1) / (4 * NT);    /* its value quads      */
    constexpr int NPM2 = (G2_STEP_MAXCH * 66 + 2 * NT - 1) / (2 * NT); /* a head's partials, in pairs */
    const int wg = blockIdx.x, nwg = gridDim.x;
    /* SH: the sizes of the model shape this kernel is compiled for (the
     * host launches it only for that shape; a launch with others does
     * nothing but report it) */
    const int E = SH ? G2P_SHAPE_E(SH) : a.E, F = SH ? G2P_SHAPE_F(SH) : a.F, NH = SH ? G2P_SHAPE_NH(SH) : a.NH;
    const int S = SH ? G2_KV_MAX_SEQ : a.S, V = SH ? G2P_SHAPE_V : a.V;
    const int pos = clampi(a.state[G2S_POS], 0, S - 1);
    const int tok = clampi(a.state[G2S_TOK], 0, V - 1);
    const unsigned seq = (unsigned)a.state[G2S_SEQ];
    /* the row-plan table was built for another grid, or the shape is not
     * the one this kernel is compiled for: do nothing (every work-group
     * returns here) and report it */
    if (a.nshares != nwg || (SH && (a.E != E || a.F != F || a.NH != NH || a.S != S || a.V != V || nwg != G2P_SHAPE_WGS))) {
        if (wg == 0 && threadIdx.x == 0) atomicOr(a.state + G2S_ERR, G2_ERR_STEP_ARGS);
        return;
    }
    /* a plain launch earlier in this run found the grid not resident: skip
     * until the host has resumed the run */
    if (a.plain && (a.state[G2S_ERR] & G2_ERR_STEP_NOT_RESIDENT)) return;
    ctx c;
    c.tag = seq + 1u;
    c.abort_w = a.xbuf;
    c.state = a.state;
    c.dead = (lds_flag *)&dead;
    const int T = pos + 1, nch = (T + 63) >> 6;
    u64 *X = a.xbuf + G2X_HEAD;
    /* value regions of layer l: this step's at XV + 2*l*VR, the next step's
     * at XN + 2*l*VR */
    const size_t VR = G2V_REGION(E, F);
    float *XV = a.xval + (c.tag & 1u) * VR, *XN = a.xval + ((c.tag & 1u) ^ 1u) * VR;
    att_regs ar[1];

    /* register sets: wa carries qkv -> fc -> fc2 -> next qkv (each loaded as
     * soon as the previous matrix is consumed), wp the proj rows */
    u32x4 wa[UMAX][4], wp[UPROJ][4];
    /* padded positions of this thread's input quads: quad tid of a K =
     * n_embd input, quads tid + NT*i of the K = ffn input */
    constexpr int VE = chunk_t<WT>::V;
    int xeo[1], xfo[QMAX];
    {
        const g2p_rows pq = row_plan_x<WT, SH>(a, G2P_SH_QKV), p2 = row_plan_x<WT, SH>(a, G2P_SH_FC2);
        xeo[0] = g2p_x_slot(&pq, VE, 4 * min((int)threadIdx.x, E / 4 - 1));
#pragma unroll
        for (int i = 0; i < QMAX; ++i) xfo[i] = g2p_x_slot(&p2, VE, 4 * min((int)threadIdx.x + NT * i, F / 4 - 1));
    }
    {
        const G2_CONST g2_step_layer *LT0 = (const G2_CONST g2_step_layer *)a.layers;
        const int tid = fresh_tid();
        if (tid == 0) {
            dead = 0;
            /* test modes of a.plain (work-group 1 only): 2 never posts its
             * arrival, 3 posts it 0.5 ms late (within the limit), 4 posts it
             * 2 ms late (after the others gave up) */
            if (a.plain && wg == 1 && a.plain >= 3) {
                const u64 t0 = wall_clock64(), d = a.plain == 3 ? 50000ull : 200000ull;
                while (wall_clock64() - t0 < d) __builtin_amdgcn_s_sleep(8);
            }
            if (a.plain && !(a.plain == 2 && wg == 1))
                ll_put(a.xbuf + G2X_ARRIVE(a.L, a.xlayer, nwg) + wg, 0.f, c.tag);
        }
        load_set<UMAX, TAIL>(tid, wa, make_plan(LT0->qkv_w, row_plan_x<WT, SH>(a, G2P_SH_QKV)), 0);
        if (wg >= NH) load_set<UPROJ, TAIL>(tid, wp, make_plan(LT0->proj_w, row_plan_x<WT, SH>(a, G2P_SH_PROJ)), 0);
        /* the padded matrix inputs: zero everywhere (the fetches write only
         * the data positions) */
        for (int q = tid; q < G2P_XE_FLOATS / 4; q += NT) *(f32x4 *)(xe + 4 * q) = (f32x4){0.f, 0.f, 0.f, 0.f};
        for (int q = tid; q < G2P_XF_FLOATS / 4; q += NT) *(f32x4 *)(xf + 4 * q) = (f32x4){0.f, 0.f, 0.f, 0.f};
        /* embedding of the token at its position (embed, math.cl:333-350) */
        for (int d = tid; d < E; d += NT)
            xres[d] = ldw((const WT *)a.wte, (size_t)tok * E + d) + ldw((const WT *)a.wpe, (size_t)pos * E + d);
        __syncthreads();
    }

    const G2_CONST g2_step_layer *LT = (const G2_CONST g2_step_layer *)a.layers;
    for (int l = 0; l < a.L; ++l) {
        /* this layer's pointers, read from the layer table where a phase
         * uses them (the table address made opaque to the compiler, as for
         * the row plans) */
        auto layer = [&]() {
            const G2_CONST g2_step_layer *p = LT + l;
            asm volatile("" : "+s"(p));
            return p;
        };
        u64 *R = X + (size_t)l * a.xlayer;
        float *RV = XV + 2 * VR * l, *RN = XN + 2 * VR * l;

        /* ---- QKV: LayerNorm(x) . Wqkv + b -> q, k, v (+ KV cache), the
         * LayerNorm folded in */
        {
            const int tid = fresh_tid();
            TRACE(0);
            const G2_CONST g2_step_layer *y = layer();
            const plan p = make_plan(y->qkv_w, row_plan_x<WT, SH>(a, G2P_SH_QKV));
            const f32x4 g = ln_gload(tid, y->ln1_w, E);
            const int rq = min(p.r0 + tid, 3 * E - 1); /* used by tid < nrows */
            const float c1 = gl(y->qkv_c1)[rq], c2 = gl(y->qkv_c2)[rq];
            f32x4 xq;
            float x0;
            if (l > 0) {
                xq = fetch_q(tid, c, RV - 2 * VR + G2V_X2(E, F), E, xres, x0);
            } else { /* the embedding, in LDS since the prologue's barrier */
                xq = *(const f32x4 *)(xres + 4 * min(tid, E / 4 - 1));
                x0 = xres[0];
            }
            TRACE(1);
            ln_fold_in(tid, xq, x0, g, E, xe, xeo[0], red);
            TRACE(11);
            matvec<WT, UMAX, TAIL>(tid, wa, p, xe, part);
            const ln_st st = ln_fold_stats(red, E);
            TRACE(12);
            if (l == 0 && a.plain &&
                !grid_resident(tid, c, a.xbuf + G2X_ARRIVE(a.L, a.xlayer, nwg), a.xbuf + G2X_DECISION, nwg,
                               (lds_flag *)&flag))
                return;
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                const float v = ln_fold_out(st, row_sum(p, part, tid), c1, c2);
                ll_put(R + r, v, c.tag);
                if (r >= 2 * E) glw(y->v_cache)[(size_t)pos * E + (r - 2 * E)] = v;
                else if (r >= E) glw(y->k_cache)[(size_t)(r - E) * S + pos] = v;
            }
            TRACE(2);
        }

        /* ---- ATTN: unit u = h * nch + chunk, work-group u % nwg, half */
        {
            const int tid = fresh_tid();
            const G2_CONST g2_step_layer *y = layer();
            const int nunits = NH * nch;
            const int rounds = (nunits + 2 * nwg - 1) / (2 * nwg);
            const int hf = tid >> 8;
            for (int rd = 0; rd < rounds; ++rd) {
                const int u = g2p_attn_unit(wg, nwg, rd, hf);
                const bool on = u < nunits;
                const int h = on ? u / nch : 0, ch = on ? u % nch : 0;
                attn_load(tid, y, ar[0], on, h, ch, pos, T, E, S);
                attn_load_v(tid, y, ar[0], on, h, ch, E, S);
                attn_chunk(tid, c, a.scale * 1.4426950408889634f, R, h * 64, E + h * 64, 2 * E + h * 64,
                                  R + G2X_ATT(E) + ((size_t)h * G2_STEP_MAXCH + ch) * 66, att[hf], ar[0],
                                  on, ch, pos, T);
                __syncthreads();
            }
            TRACE(3);
            /* the fc rows stream from here on; a work-group that merges a head
             * issues them after its merge, so its merge waits behind nothing */
            if (wg >= NH) load_set<UMAX, TAIL>(tid, wa, make_plan(y->fc_w, row_plan_x<WT, SH>(a, G2P_SH_FC)), 0);
        }

        /* ---- MERGE: head h by work-group h (g2k_attn_merge) */
        for (int h = wg; h < NH; h += nwg) {
            const int tid = fresh_tid();
            const u64 *hp = R + G2X_ATT(E) + (size_t)h * G2_STEP_MAXCH * 66;
            fetch2<NPM2>(tid, c, hp, nch * 66, xsc); /* 66 words per chunk: even, at even words */
            /* wave 0 alone: lane ch holds chunk ch's weight, which every
             * lane reads by readlane (no LDS round trip, no barrier) */
            if (tid < 64) {
                const float mc = tid < nch ? xsc[tid * 66] : -INFINITY;
                const float lc = tid < nch ? xsc[tid * 66 + 1] : 0.f;
                const float M = wmax(mc);
                const float w = tid < nch ? __builtin_amdgcn_exp2f(mc - M) : 0.f; /* base-2 maxima */
                const float Ls = wsum(lc * w);
                float acc = 0.f;
                for (int ch = 0; ch < nch; ++ch) acc = fmaf(xsc[ch * 66 + 2 + tid], row_lane(w, ch), acc);
                vput(RV + G2V_O(E) + h * 64 + tid, RN + G2V_O(E) + h * 64 + tid, acc / Ls);
            }
            __syncthreads();
        }
        {
            const int tid = fresh_tid();
            TRACE(16);
            if (wg < NH) load_set<UMAX, TAIL>(tid, wa, make_plan(layer()->fc_w, row_plan_x<WT, SH>(a, G2P_SH_FC)), 0);
            TRACE(4);
        }

        /* ---- PROJ: X1 = x + (O . Wp + b), by the work-groups merging no head */
        if (wg < NH) {
            const int tid = fresh_tid();
            TRACE(5);
            TRACE(6);
        } else {
            const int tid = fresh_tid();
            const G2_CONST g2_step_layer *y = layer();
            const plan p = make_plan(y->proj_w, row_plan_x<WT, SH>(a, G2P_SH_PROJ));
            const float bias = gl(y->proj_b)[min(p.r0 + tid, E - 1)];
            fetch4<NQE>(tid, c, RV + G2V_O(E), E, NH, xe, xeo, (lds_flag *)&flag);
            TRACE(5);
            matvec<WT, UPROJ, TAIL>(tid, wp, p, xe, part);
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                float v = row_sum(p, part, tid);
                v += bias;
                vput(RV + G2V_X1(E) + r, RN + G2V_X1(E) + r, v + xres[r]);
            }
            TRACE(6);
            if (l + 1 < a.L) load_set<UPROJ, TAIL>(tid, wp, make_plan(LT[l + 1].proj_w, row_plan_x<WT, SH>(a, G2P_SH_PROJ)), 0);
            __syncthreads();
        }

        /* ---- FC: H = gelu(LayerNorm(X1) . Wfc + b), the LayerNorm folded in */
        {
            const int tid = fresh_tid();
            const G2_CONST g2_step_layer *y = layer();
            const plan p = make_plan(y->fc_w, row_plan_x<WT, SH>(a, G2P_SH_FC));
            const f32x4 g = ln_gload(tid, y->ln2_w, E);
            const int rf = min(p.r0 + tid, F - 1); /* used by tid < nrows */
            const float c1 = gl(y->fc_c1)[rf], c2 = gl(y->fc_c2)[rf];
            float x0;
            const f32x4 xq = fetch_q(tid, c, RV + G2V_X1(E), E, xres, x0);
            TRACE(7);
            ln_fold_in(tid, xq, x0, g, E, xe, xeo[0], red);
            TRACE(13);
            matvec<WT, UMAX, TAIL>(tid, wa, p, xe, part);
            const ln_st st = ln_fold_stats(red, E);
            TRACE(14);
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                const float v = ln_fold_out(st, row_sum(p, part, tid), c1, c2);
                vput(RV + G2V_H(E) + r, RN + G2V_H(E) + r, gelu_f(v));
            }
            TRACE(8);
            load_set<UMAX, TAIL>(tid, wa, make_plan(y->fc2_w, row_plan_x<WT, SH>(a, G2P_SH_FC2)), 0);
            __syncthreads();
        }

        /* ---- FC2: X2 = X1 + (H . Wfc2 + b) */
        {
            const int tid = fresh_tid();
            const G2_CONST g2_step_layer *y = layer();
            const plan p = make_plan(y->fc2_w, row_plan_x<WT, SH>(a, G2P_SH_FC2));
            const float bias = gl(y->fc2_b)[min(p.r0 + tid, E - 1)];
            fetch4<QMAX>(tid, c, RV + G2V_H(E), F, nwg, xf, xfo, (lds_flag *)&flag);
            TRACE(9);
            matvec<WT, UMAX, TAIL>(tid, wa, p, xf, part);
            TRACE(15);
            if (tid < p.nrows) {
                const int r = p.r0 + tid;
                float v = row_sum(p, part, tid);
                v += bias;
                vput(RV + G2V_X2(E, F) + r, RN + G2V_X2(E, F) + r, v + xres[r]);
            }
            TRACE(10);
            if (l + 1 < a.L) load_set<UMAX, TAIL>(tid, wa, make_plan(LT[l + 1].qkv_w, row_plan_x<WT, SH>(a, G2P_SH_QKV)), 0);
            else load_set<UMAX, TAIL>(tid, wa, make_plan(a.lm_w, row_plan_x<WT, SH>(a, G2P_SH_LM)), 0);
            __syncthreads();
        }
    }

    /* the first batch of lm_head rows was loaded by the last fc2 phase */
    lm_pick<WT, TAIL, TRACED>(a, c, row_plan_x<WT, SH>(a, G2P_SH_LM), XV + 2 * VR * (a.L - 1) + G2V_X2(E, F), X + (size_t)a.L * a.xlayer, wa, true,
                xres, xe, xeo[0], xsc, part, red, amv, ami, (lds_flag *)&flag);
}

} /* namespace g2step */

/* The plain form with the model shape from the arguments, and compiled for
 * the GPT-2 shapes of the benchmark configurations (g2p_step_shape: small,
 * medium and large with fp32 weights, large with fp16 weights). */
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f32(const g2_step_args a)
{
    g2step::step_impl<float, false, false, 0>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f16(const g2_step_args a)
{
    g2step::step_impl<_Float16, false, false, 0>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f32_e768(const g2_step_args a)
{
    g2step::step_impl<float, false, false, 1>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f32_e1024(const g2_step_args a)
{
    g2step::step_impl<float, false, false, 2>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f32_e1280(const g2_step_args a)
{
    g2step::step_impl<float, false, false, 3>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f16_e1280(const g2_step_args a)
{
    g2step::step_impl<_Float16, false, false, 3>(a);
}
/* The tail form, for models whose every four-unit plan is a tail plan
 * (g2p_step_tail: n_embd 1600, the rows of every matrix 200 chunks per
 * segment).  g2k_step_f16_tail is compiled for GPT-2 XL's shape;
 * g2k_step_f16_tailn and g2k_step_f32_tail take the shape from their
 * arguments. */
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f32_tail(const g2_step_args a)
{
    g2step::step_impl<float, true, false, 0>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f16_tail(const g2_step_args a)
{
    g2step::step_impl<_Float16, true, false, G2P_SHAPE_XL>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f16_tailn(const g2_step_args a)
{
    g2step::step_impl<_Float16, true, false, 0>(a);
}
/* The same with the phase timestamps of g2_step_args.trace (launched
 * instead of them when a trace buffer is set; shape from the arguments,
 * except the XL tail form). */
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f32_trace(const g2_step_args a)
{
    g2step::step_impl<float, false, true, 0>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f16_trace(const g2_step_args a)
{
    g2step::step_impl<_Float16, false, true, 0>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f32_tail_trace(const g2_step_args a)
{
    g2step::step_impl<float, true, true, 0>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f16_tail_trace(const g2_step_args a)
{
    g2step::step_impl<_Float16, true, true, G2P_SHAPE_XL>(a);
}
extern "C" __global__ __launch_bounds__(G2_STEP_THREADS) void g2k_step_f16_tailn_trace(const g2_step_args a)
{
    g2step::step_impl<_Float16, true, true, 0>(a);
}
