/*
 * g2_host.c -- host-only pieces of libg2hip: config.json parsing, the
 * synthetic weight generator, fp32 -> fp16 rounding and a safetensors
 * reader.  None of these touch the GPU, so they work on a machine without
 * one.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g2_internal.h"
#include "g2_host.h"

/* ------------------------------------------------------------ config.json */

/* Integer value of the first of `keys` present in `json`, as the reference's
 * substring scan does (main.c:272-292): find "key", skip to ':', atoi. */
static int json_int(const char *json, const char *const *keys, int nkeys, int defval)
{
    for (int i = 0; i < nkeys; ++i) {
        char pat[96];
        snprintf(pat, sizeof pat, "\"%s\"", keys[i]);
        const char *p = strstr(json, pat);
        if (!p) continue;
        p = strchr(p + strlen(pat), ':');
        if (!p) continue;
        ++p;
        while (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r') ++p;
        /* atoi's value, with out-of-range numbers clamped (they then fail the
         * ceilings instead of overflowing) */
        const long long v = strtoll(p, NULL, 10);
        return v > (1 << 28) ? (1 << 28) : (v < -(1 << 28) ? -(1 << 28) : (int)v);
    }
    return defval;
}

static int check_config(g2_config *c)
{
    if (c->n_layer <= 0 || c->n_embd <= 0 || c->n_head <= 0 || c->vocab_size <= 0 ||
        c->ffn_dim <= 0 || c->n_ctx <= 0)
        return g2i_err(G2_E_FORMAT, "config: non-positive size");
    if (c->n_embd > G2_MAX_EMBED || c->n_layer > G2_MAX_LAYERS || c->n_head > G2_MAX_HEADS ||
        c->vocab_size > G2_MAX_VOCAB || c->ffn_dim > G2_MAX_FFN || c->n_ctx > G2_MAX_SEQ)
        return g2i_err(G2_E_LIMIT, "config exceeds compiled-in ceilings");
    if (c->n_embd % c->n_head)
        return g2i_err(G2_E_FORMAT, "config: n_embd %d not divisible by n_head %d",
                       c->n_embd, c->n_head);
    return G2_OK;
}

/* load_config, main.c:294-331 */
int g2_config_parse(const char *json, g2_config *cfg)
{
    if (!json || !cfg) return g2i_err(G2_E_ARG, "g2_config_parse: NULL argument");
    static const char *const k_layer[] = { "n_layer" }, *const k_embd[] = { "n_embd" };
    static const char *const k_head[] = { "n_head" }, *const k_vocab[] = { "vocab_size" };
    static const char *const k_ctx[] = { "n_positions", "n_ctx" }, *const k_inner[] = { "n_inner" };
    cfg->n_layer = json_int(json, k_layer, 1, 12);
    cfg->n_embd = json_int(json, k_embd, 1, 768);
    cfg->n_head = json_int(json, k_head, 1, 12);
    cfg->n_ctx = json_int(json, k_ctx, 2, 1024);
    cfg->vocab_size = json_int(json, k_vocab, 1, 50257);
    const int inner = json_int(json, k_inner, 1, 0);
    cfg->ffn_dim = inner > 0 ? inner : 4 * cfg->n_embd;
    return check_config(cfg);
}

char *g2h_slurp(const char *path, size_t *size)
{
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    if (fseek(f, 0, SEEK_END) != 0) { fclose(f); return NULL; }
    long n = ftell(f);
    if (n < 0 || fseek(f, 0, SEEK_SET) != 0) { fclose(f); return NULL; }
    char *buf = malloc((size_t)n + 1);
    if (!buf) { fclose(f); return NULL; }
    if (fread(buf, 1, (size_t)n, f) != (size_t)n) { free(buf); fclose(f); return NULL; }
    fclose(f);
    buf[n] = 0;
    if (size) *size = (size_t)n;
    return buf;
}

int g2_config_load(const char *dir, g2_config *cfg)
{
    if (!dir || !cfg) return g2i_err(G2_E_ARG, "g2_config_load: NULL argument");
    char path[1024];
    snprintf(path, sizeof path, "%s/config.json", dir);
    char *json = g2h_slurp(path, NULL);
    if (!json) {
        /* main.c:299-305: a missing config.json means GPT-2 small */
        cfg->n_layer = 12; cfg->n_embd = 768; cfg->n_head = 12;
        cfg->n_ctx = 1024; cfg->vocab_size = 50257; cfg->ffn_dim = 3072;
        return G2_OK;
    }
    int rc = g2_config_parse(json, cfg);
    free(json);
    return rc;
}

/* ------------------------------------------------------ synthetic weights */

/* splitmix64 output function applied to a counter (stateless). */
static uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* Uniform in (0, 1] from the top 53 bits. */
static double unit53(uint64_t r) { return ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

/* Element 2p and 2p+1 come from the Box-Muller pair p:
 * u1 = unit53(mix64(key + 2p)), u2 = unit53(mix64(key + 2p + 1)),
 * z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = sqrt(-2 ln u1) sin(2 pi u2),
 * key = mix64(seed ^ (tensor_id * 0xD1B54A32D192ED03)). */
void g2_synth_normal(float *dst, size_t n, uint64_t seed, uint32_t tensor_id, float std_dev)
{
    if (!dst) return;
    const uint64_t key = mix64(seed ^ ((uint64_t)tensor_id * 0xD1B54A32D192ED03ULL));
    const long npair = (long)((n + 1) / 2);
    const double two_pi = 6.283185307179586476925286766559;
    #pragma omp parallel for schedule(static)
    for (long p = 0; p < npair; ++p) {
        const double u1 = unit53(mix64(key + 2 * (uint64_t)p));
        const double u2 = unit53(mix64(key + 2 * (uint64_t)p + 1));
        const double r = sqrt(-2.0 * log(u1));
        const double a = two_pi * u2;
        dst[2 * p] = (float)(std_dev * (r * cos(a)));
        if ((size_t)(2 * p + 1) < n) dst[2 * p + 1] = (float)(std_dev * (r * sin(a)));
    }
}

uint32_t g2_synth_tensor_id(int layer, int which)
{
    if (layer < 0) return (uint32_t)which;            /* 1 = wte, 2 = wpe */
    return (uint32_t)(16 + 8 * layer + which);        /* 0..3 per layer   */
}

/* -------------------------------------------------------- fp32 -> fp16 */

/* IEEE binary32 -> binary16, round to nearest even, subnormals, inf, nan. */
static uint16_t f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal */
        if (ax < 0x33000000u) return sign;                    /* < 2^-25 rounds to 0    */
        const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        const int e = (int)(ax >> 23);                        /* 102..112 */
        const int shift = 126 - e;                            /* 14..24   */
        uint32_t v = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (v & 1u))) ++v;
        return (uint16_t)(sign | v);
    }
    uint32_t v = ((ax >> 13) - (112u << 10));                 /* rebias exponent */
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) ++v;
    return (uint16_t)(sign | v);
}

void g2i_f32_to_f16(uint16_t *dst, const float *src, size_t n)
{
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < (long)n; ++i) dst[i] = f32_to_f16(src[i]);
}

void g2_convert_f16(uint16_t *dst, const float *src, size_t n)
{
    if (dst && src) g2i_f32_to_f16(dst, src, n);
}

float g2h_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = sign;
        else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-8f;
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------ safetensors */

/* Minimal reader for the safetensors container: 8-byte little-endian header
 * length, a JSON object mapping names to {"dtype", "shape", "data_offsets"}
 * (offsets relative to the end of the header), optional "__metadata__". */

static const char *skip_ws(const char *p, const char *end)
{
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    return p;
}

/* Parse a JSON string starting at p (which must be '"'); copies at most
 * cap-1 bytes into out; returns the position after the closing quote. */
static const char *parse_str(const char *p, const char *end, char *out, size_t cap)
{
    if (p >= end || *p != '"') return NULL;
    ++p;
    size_t n = 0;
    while (p < end && *p != '"') {
        char c = *p++;
        if (c == '\\') {
            if (p >= end) return NULL;
            c = *p++;
            if (c == 'u') { /* keep escapes opaque: tensor names are ASCII */
                if (end - p < 4) return NULL;
                p += 4;
                c = '?';
            }
        }
        if (n + 1 < cap) out[n++] = c;
    }
    if (p >= end) return NULL;
    out[n] = 0;
    return p + 1;
}

/* Skip any JSON value. */
static const char *skip_value(const char *p, const char *end)
{
    p = skip_ws(p, end);
    if (p >= end) return NULL;
    if (*p == '"') {
        char tmp[8];
        return parse_str(p, end, tmp, sizeof tmp);
    }
    if (*p == '{' || *p == '[') {
        int depth = 0;
        while (p < end) {
            if (*p == '"') {
                char tmp[8];
                p = parse_str(p, end, tmp, sizeof tmp);
                if (!p) return NULL;
                continue;
            }
            if (*p == '{' || *p == '[') ++depth;
            else if (*p == '}' || *p == ']') {
                --depth;
                if (depth == 0) return p + 1;
            }
            ++p;
        }
        return NULL;
    }
    while (p < end && *p != ',' && *p != '}' && *p != ']') ++p;
    return p;
}

static const char *parse_int_array(const char *p, const char *end, int64_t *vals, int cap, int *count)
{
    p = skip_ws(p, end);
    if (p >= end || *p != '[') return NULL;
    ++p;
    *count = 0;
    for (;;) {
        p = skip_ws(p, end);
        if (p < end && *p == ']') return p + 1;
        char *q;
        const long long v = strtoll(p, &q, 10);
        if (q == p) return NULL;
        if (*count < cap) vals[*count] = v;
        ++*count;
        p = skip_ws(q, end);
        if (p < end && *p == ',') { ++p; continue; }
        if (p < end && *p == ']') return p + 1;
        return NULL;
    }
}

static int dtype_code(const char *s, int *size)
{
    if (!strcmp(s, "F32")) { *size = 4; return G2H_ST_F32; }
    if (!strcmp(s, "F16")) { *size = 2; return G2H_ST_F16; }
    if (!strcmp(s, "BF16")) { *size = 2; return G2H_ST_BF16; }
    *size = 0;
    return G2H_ST_OTHER;
}

void g2h_st_close(g2h_st *st)
{
    if (!st) return;
    if (st->fp) fclose(st->fp);
    free(st->t);
    memset(st, 0, sizeof *st);
}

int g2h_st_open(const char *path, g2h_st *st)
{
    memset(st, 0, sizeof *st);
    st->fp = fopen(path, "rb");
    if (!st->fp) return g2i_err(G2_E_IO, "cannot open %s", path);
    unsigned char lb[8];
    if (fread(lb, 1, 8, st->fp) != 8) { g2h_st_close(st); return g2i_err(G2_E_IO, "%s: short header", path); }
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | lb[i];
    if (hlen == 0 || hlen > ((uint64_t)1 << 30)) {
        g2h_st_close(st);
        return g2i_err(G2_E_FORMAT, "%s: implausible header length", path);
    }
    char *h = malloc((size_t)hlen + 1);
    if (!h) { g2h_st_close(st); return g2i_err(G2_E_NOMEM, "header alloc"); }
    if (fread(h, 1, (size_t)hlen, st->fp) != (size_t)hlen) {
        free(h); g2h_st_close(st);
        return g2i_err(G2_E_IO, "%s: short header read", path);
    }
    h[hlen] = 0;
    st->data_start = 8 + (int64_t)hlen;
    /* every tensor's bytes must lie inside the file */
    int64_t fsize = -1;
    if (fseeko(st->fp, 0, SEEK_END) == 0) fsize = (int64_t)ftello(st->fp);
    if (fsize < st->data_start) {
        free(h); g2h_st_close(st);
        return g2i_err(G2_E_FORMAT, "%s: file shorter than its header", path);
    }
    const char *p = h, *end = h + hlen;
    int cap = 64;
    st->t = calloc((size_t)cap, sizeof *st->t);
    int rc = G2_OK;
    p = skip_ws(p, end);
    if (!st->t || p >= end || *p != '{') { rc = g2i_err(G2_E_FORMAT, "%s: header is not a JSON object", path); goto done; }
    ++p;
    for (;;) {
        p = skip_ws(p, end);
        if (p < end && *p == '}') break;
        char name[256];
        p = parse_str(p, end, name, sizeof name);
        if (!p) { rc = g2i_err(G2_E_FORMAT, "%s: bad key", path); goto done; }
        p = skip_ws(p, end);
        if (p >= end || *p != ':') { rc = g2i_err(G2_E_FORMAT, "%s: missing ':'", path); goto done; }
        p = skip_ws(p + 1, end);
        if (!strcmp(name, "__metadata__")) {
            p = skip_value(p, end);
            if (!p) { rc = g2i_err(G2_E_FORMAT, "%s: bad metadata", path); goto done; }
        } else {
            if (p >= end || *p != '{') { rc = g2i_err(G2_E_FORMAT, "%s: tensor entry not an object", path); goto done; }
            if (st->n == cap) {
                cap *= 2;
                void *nt = realloc(st->t, (size_t)cap * sizeof *st->t);
                if (!nt) { rc = g2i_err(G2_E_NOMEM, "header alloc"); goto done; }
                st->t = nt;
            }
            g2h_tensor *t = &st->t[st->n];
            memset(t, 0, sizeof *t);
            snprintf(t->name, sizeof t->name, "%s", name);
            t->dtype = -1;
            ++p;
            for (;;) {
                p = skip_ws(p, end);
                if (p < end && *p == '}') { ++p; break; }
                char key[32];
                p = parse_str(p, end, key, sizeof key);
                if (!p) { rc = g2i_err(G2_E_FORMAT, "%s: bad field", path); goto done; }
                p = skip_ws(p, end);
                if (p >= end || *p != ':') { rc = g2i_err(G2_E_FORMAT, "%s: missing ':'", path); goto done; }
                p = skip_ws(p + 1, end);
                if (!strcmp(key, "dtype")) {
                    char dt[16];
                    p = parse_str(p, end, dt, sizeof dt);
                    if (!p) { rc = g2i_err(G2_E_FORMAT, "%s: bad dtype", path); goto done; }
                    t->dtype = dtype_code(dt, &t->esize);
                    snprintf(t->dtype_name, sizeof t->dtype_name, "%s", dt);
                } else if (!strcmp(key, "shape")) {
                    p = parse_int_array(p, end, t->shape, 8, &t->ndim);
                    if (!p || t->ndim > 8) { rc = g2i_err(G2_E_FORMAT, "%s: bad shape", path); goto done; }
                } else if (!strcmp(key, "data_offsets")) {
                    int cnt = 0;
                    int64_t off[2] = { 0, 0 };
                    p = parse_int_array(p, end, off, 2, &cnt);
                    if (!p || cnt != 2) { rc = g2i_err(G2_E_FORMAT, "%s: bad data_offsets", path); goto done; }
                    t->begin = off[0];
                    t->end = off[1];
                } else {
                    p = skip_value(p, end);
                    if (!p) { rc = g2i_err(G2_E_FORMAT, "%s: bad value", path); goto done; }
                }
                p = skip_ws(p, end);
                if (p < end && *p == ',') ++p;
            }
            /* element count with every dimension and the product bounded (no
             * int64 overflow), byte range consistent with it and inside the file */
            const int64_t lim = (int64_t)1 << 40;
            int64_t nel = 1;
            int bad = t->dtype < 0;
            for (int i = 0; i < t->ndim && !bad; ++i) {
                if (t->shape[i] < 0 || t->shape[i] > lim) bad = 1;
                else if (t->shape[i] > 0 && nel > lim / t->shape[i]) bad = 1;
                else nel *= t->shape[i];
            }
            if (!bad && (t->begin < 0 || t->end < t->begin || t->end > fsize - st->data_start)) bad = 1;
            if (!bad && t->esize && nel * t->esize != t->end - t->begin) bad = 1;
            if (bad) {
                rc = g2i_err(G2_E_FORMAT, "%s: inconsistent entry for %s", path, t->name);
                goto done;
            }
            t->numel = nel;
            ++st->n;
        }
        p = skip_ws(p, end);
        if (p < end && *p == ',') { ++p; continue; }
        p = skip_ws(p, end);
        if (p < end && *p == '}') break;
        rc = g2i_err(G2_E_FORMAT, "%s: expected ',' or '}'", path);
        goto done;
    }
done:
    free(h);
    if (rc) g2h_st_close(st);
    return rc;
}

/* Name lookup with the reference's fallbacks "transformer." / "model."
 * (main.c:1194-1207). */
const g2h_tensor *g2h_st_find(const g2h_st *st, const char *name)
{
    static const char *const prefix[3] = { "", "transformer.", "model." };
    char buf[300];
    for (int k = 0; k < 3; ++k) {
        snprintf(buf, sizeof buf, "%s%s", prefix[k], name);
        for (int i = 0; i < st->n; ++i)
            if (!strcmp(st->t[i].name, buf)) return &st->t[i];
    }
    return NULL;
}

/* Read a tensor as fp32 (F32 copied, F16/BF16 widened) into dst, which
 * holds cap floats. */
int g2h_st_read_f32(const g2h_st *st, const g2h_tensor *t, float *dst, int64_t cap)
{
    if (t->dtype == G2H_ST_OTHER)
        return g2i_err(G2_E_FORMAT, "tensor %s has unsupported dtype %s", t->name, t->dtype_name);
    if (t->numel > cap || t->numel * t->esize != t->end - t->begin)
        return g2i_err(G2_E_FORMAT, "tensor %s: %lld elements do not fit the %lld expected", t->name,
                       (long long)t->numel, (long long)cap);
    const size_t bytes = (size_t)(t->end - t->begin);
    if (fseeko(st->fp, (off_t)(st->data_start + t->begin), SEEK_SET) != 0)
        return g2i_err(G2_E_IO, "seek to %s failed", t->name);
    if (t->dtype == G2H_ST_F32) {
        if (fread(dst, 1, bytes, st->fp) != bytes) return g2i_err(G2_E_IO, "short read of %s", t->name);
        return G2_OK;
    }
    uint16_t *tmp = malloc(bytes);
    if (!tmp) return g2i_err(G2_E_NOMEM, "staging %s", t->name);
    if (fread(tmp, 1, bytes, st->fp) != bytes) {
        free(tmp);
        return g2i_err(G2_E_IO, "short read of %s", t->name);
    }
    for (int64_t i = 0; i < t->numel; ++i) {
        if (t->dtype == G2H_ST_F16) {
            dst[i] = g2h_f16_to_f32(tmp[i]);
        } else {
            const uint32_t x = (uint32_t)tmp[i] << 16;
            memcpy(&dst[i], &x, 4);
        }
    }
    free(tmp);
    return G2_OK;
}
