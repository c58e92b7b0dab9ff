/*
 * g2_tokenizer.c -- GPT-2 byte-level BPE tokenizer for text prompts (the
 * reference's tokenizer.c API: load vocab.json + merges.txt from a model
 * directory, encode UTF-8 text to ids, decode ids to UTF-8), host C99.
 *
 * Behaviour follows the reference (tokenizer.c):
 *   - pre-tokenisation with ASCII character classes (tokenizer.c:476-550):
 *     contractions 's 't 'm 'd 're 've 'll; a space followed by a non-space
 *     starts a piece with the run of that character's class (letters a-z
 *     A-Z, digits, or "other": neither space, letter nor digit); letter,
 *     digit and other runs; every whitespace character not taken by the
 *     space rule is a piece of its own.  Bytes >= 0x80 are "other".
 *   - each piece's bytes map to the GPT-2 byte alphabet (tokenizer.c:
 *     332-343: bytes 33-126, 161-172, 174-255 to themselves, the other 68
 *     to 256, 257, ... in byte order), then BPE: while some adjacent pair
 *     has a merge rank, every occurrence of the lowest-ranked pair is
 *     merged, left to right (tokenizer.c:360-407); the final symbols that
 *     are vocabulary tokens are emitted, the others dropped (:409-417).
 *   - merges.txt: a first line starting with '#' is skipped; every other
 *     line with a space is "left right" (split at the first space, '\r'
 *     stripped) and gets the next rank; a pair listed twice keeps the later
 *     rank (:285-330).  vocab.json: an object of JSON strings to
 *     non-negative integers; an id listed twice keeps the later string.
 *   - decode: ids outside [0, vocab size) or without a string are skipped;
 *     each code point of a token maps back to its byte ('?' if none); the
 *     output stops at max_bytes - 1 bytes and is NUL-terminated (:552-579).
 *
 * Design (not the reference's): every string (the byte symbols, vocabulary
 * tokens, both sides of every merge and every merge result) is interned
 * once into a symbol table, so BPE runs on symbol ids and a merge is one
 * lookup of the 64-bit key (left id, right id) -> (rank, result id).
 */
#include "g2_internal.h"
#include "g2_host.h"

#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* open-addressing hash tables                                          */

static uint64_t hash_bytes(const unsigned char *p, int n)
{
    uint64_t h = 0x9E3779B97F4A7C15ull ^ (uint64_t)n;
    for (int i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x100000001B3ull;
        h ^= h >> 29;
    }
    return h;
}

static uint64_t mix64(uint64_t x)
{
    x ^= x >> 33;
    x *= 0xFF51AFD7ED558CCDull;
    x ^= x >> 33;
    x *= 0xC4CEB9FE1A85EC53ull;
    x ^= x >> 33;
    return x;
}

typedef struct {
    char *arena;      /* all symbol strings, back to back */
    size_t arena_len, arena_cap;
    size_t *off;      /* symbol -> offset in arena */
    int *len;         /* symbol -> byte length */
    int n, cap;       /* symbols */
    int *slot;        /* hash slot -> symbol + 1 (0: empty) */
    int nslots;       /* power of two */
} symtab;

typedef struct {
    uint64_t *key;    /* (left << 32 | right) + 1; 0: empty */
    int *rank, *out;
    int nslots, n;
} pairmap;

struct g2_tokenizer {
    symtab sy;
    pairmap mg;
    int byte_sym[256];   /* byte -> symbol of its alphabet character */
    int cp_byte[512];    /* alphabet code point -> byte, -1 if none */
    int *sym_vocab;      /* symbol -> vocabulary id, -1 if not a token */
    int sym_vocab_cap;
    int *vocab_sym;      /* vocabulary id -> symbol, -1 if none */
    int vocab_size;
};

static int sy_grow_slots(symtab *s)
{
    const int ns = s->nslots ? 2 * s->nslots : 1 << 16;
    int *sl = calloc((size_t)ns, sizeof(int));
    if (!sl) return -1;
    for (int i = 0; i < s->n; ++i) {
        uint64_t h = hash_bytes((const unsigned char *)s->arena + s->off[i], s->len[i]);
        int j = (int)(h & (uint64_t)(ns - 1));
        while (sl[j]) j = (j + 1) & (ns - 1);
        sl[j] = i + 1;
    }
    free(s->slot);
    s->slot = sl;
    s->nslots = ns;
    return 0;
}

/* Symbol id of the string (interned on first sight); -1 on allocation failure. */
static int sy_intern(symtab *s, const char *str, int n)
{
    if (!s->nslots && sy_grow_slots(s)) return -1;
    const uint64_t h = hash_bytes((const unsigned char *)str, n);
    int j = (int)(h & (uint64_t)(s->nslots - 1));
    while (s->slot[j]) {
        const int id = s->slot[j] - 1;
        if (s->len[id] == n && memcmp(s->arena + s->off[id], str, (size_t)n) == 0) return id;
        j = (j + 1) & (s->nslots - 1);
    }
    if (s->n == s->cap) {
        const int nc = s->cap ? 2 * s->cap : 4096;
        size_t *o = realloc(s->off, (size_t)nc * sizeof *o);
        if (!o) return -1;
        s->off = o;
        int *l = realloc(s->len, (size_t)nc * sizeof *l);
        if (!l) return -1;
        s->len = l;
        s->cap = nc;
    }
    if (s->arena_len + (size_t)n > s->arena_cap) {
        size_t nc = s->arena_cap ? 2 * s->arena_cap : 1 << 20;
        while (nc < s->arena_len + (size_t)n) nc *= 2;
        char *a = realloc(s->arena, nc);
        if (!a) return -1;
        s->arena = a;
        s->arena_cap = nc;
    }
    memcpy(s->arena + s->arena_len, str, (size_t)n);
    const int id = s->n++;
    s->off[id] = s->arena_len;
    s->len[id] = n;
    s->arena_len += (size_t)n;
    s->slot[j] = id + 1;
    if (2 * s->n > s->nslots && sy_grow_slots(s)) return -1;
    return id;
}

static int pm_grow(pairmap *m)
{
    const int ns = m->nslots ? 2 * m->nslots : 1 << 16;
    uint64_t *k = calloc((size_t)ns, sizeof *k);
    int *r = malloc((size_t)ns * sizeof *r), *o = malloc((size_t)ns * sizeof *o);
    if (!k || !r || !o) { free(k); free(r); free(o); return -1; }
    for (int i = 0; i < m->nslots; ++i) {
        if (!m->key[i]) continue;
        int j = (int)(mix64(m->key[i]) & (uint64_t)(ns - 1));
        while (k[j]) j = (j + 1) & (ns - 1);
        k[j] = m->key[i];
        r[j] = m->rank[i];
        o[j] = m->out[i];
    }
    free(m->key); free(m->rank); free(m->out);
    m->key = k; m->rank = r; m->out = o;
    m->nslots = ns;
    return 0;
}

/* Set (left, right) -> (rank, out), replacing an earlier entry of the pair. */
static int pm_put(pairmap *m, int left, int right, int rank, int out)
{
    if ((!m->nslots || 2 * (m->n + 1) > m->nslots) && pm_grow(m)) return -1;
    const uint64_t key = (((uint64_t)(uint32_t)left << 32) | (uint32_t)right) + 1;
    int j = (int)(mix64(key) & (uint64_t)(m->nslots - 1));
    while (m->key[j] && m->key[j] != key) j = (j + 1) & (m->nslots - 1);
    if (!m->key[j]) { m->key[j] = key; ++m->n; }
    m->rank[j] = rank;
    m->out[j] = out;
    return 0;
}

/* Rank of the pair (INT_MAX if none) and its merged symbol. */
static int pm_get(const pairmap *m, int left, int right, int *out)
{
    if (!m->nslots) return INT_MAX;
    const uint64_t key = (((uint64_t)(uint32_t)left << 32) | (uint32_t)right) + 1;
    int j = (int)(mix64(key) & (uint64_t)(m->nslots - 1));
    while (m->key[j]) {
        if (m->key[j] == key) { *out = m->out[j]; return m->rank[j]; }
        j = (j + 1) & (m->nslots - 1);
    }
    return INT_MAX;
}

/* ------------------------------------------------------------------ */
/* UTF-8 and file helpers                                               */

static int put_utf8(unsigned cp, char *o)
{
    if (cp < 0x80) { o[0] = (char)cp; return 1; }
    if (cp < 0x800) { o[0] = (char)(0xC0 | (cp >> 6)); o[1] = (char)(0x80 | (cp & 0x3F)); return 2; }
    if (cp < 0x10000) {
        o[0] = (char)(0xE0 | (cp >> 12)); o[1] = (char)(0x80 | ((cp >> 6) & 0x3F)); o[2] = (char)(0x80 | (cp & 0x3F));
        return 3;
    }
    o[0] = (char)(0xF0 | (cp >> 18)); o[1] = (char)(0x80 | ((cp >> 12) & 0x3F));
    o[2] = (char)(0x80 | ((cp >> 6) & 0x3F)); o[3] = (char)(0x80 | (cp & 0x3F));
    return 4;
}

/* Code point at s (the lead byte decides the length); 0 if the lead byte
 * is not a UTF-8 lead byte. */
static int get_utf8(const unsigned char *s, unsigned *cp)
{
    const unsigned c = s[0];
    if (c < 0x80) { *cp = c; return 1; }
    if ((c & 0xE0) == 0xC0) { *cp = ((c & 0x1F) << 6) | (s[1] & 0x3F); return 2; }
    if ((c & 0xF0) == 0xE0) { *cp = ((c & 0x0F) << 12) | ((s[1] & 0x3F) << 6) | (s[2] & 0x3F); return 3; }
    if ((c & 0xF8) == 0xF0) {
        *cp = ((c & 0x07) << 18) | ((s[1] & 0x3F) << 12) | ((s[2] & 0x3F) << 6) | (s[3] & 0x3F);
        return 4;
    }
    return 0;
}

static char *slurp(const char *path, size_t *n)
{
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    char *b = NULL;
    size_t cap = 0, len = 0;
    for (;;) {
        if (len + 65536 + 1 > cap) {
            cap = cap ? 2 * cap : 1 << 20;
            char *nb = realloc(b, cap);
            if (!nb) { free(b); fclose(f); return NULL; }
            b = nb;
        }
        const size_t r = fread(b + len, 1, 65536, f);
        len += r;
        if (r < 65536) break;
    }
    fclose(f);
    b[len] = 0;
    *n = len;
    return b;
}

static int hexval(int h)
{
    if (h >= '0' && h <= '9') return h - '0';
    if (h >= 'a' && h <= 'f') return h - 'a' + 10;
    if (h >= 'A' && h <= 'F') return h - 'A' + 10;
    return -1;
}

/* JSON string at *p (opening quote) into buf (capacity cap); the length,
 * or -1 if malformed or too long.  Advances *p past the closing quote. */
static int json_string(const char **p, const char *end, char *buf, int cap)
{
    const char *q = *p;
    if (q >= end || *q != '"') return -1;
    ++q;
    int n = 0;
    while (q < end && *q != '"') {
        char tmp[4];
        int tl = 1;
        if (*q != '\\') {
            tmp[0] = *q++;
        } else {
            if (++q >= end) return -1;
            const char e = *q++;
            switch (e) {
            case '"': tmp[0] = '"'; break;
            case '\\': tmp[0] = '\\'; break;
            case '/': tmp[0] = '/'; break;
            case 'b': tmp[0] = '\b'; break;
            case 'f': tmp[0] = '\f'; break;
            case 'n': tmp[0] = '\n'; break;
            case 'r': tmp[0] = '\r'; break;
            case 't': tmp[0] = '\t'; break;
            case 'u': {
                unsigned cp = 0;
                for (int i = 0; i < 4; ++i) {
                    const int v = q < end ? hexval(*q++) : -1;
                    if (v < 0) return -1;
                    cp = (cp << 4) | (unsigned)v;
                }
                if (cp >= 0xD800 && cp <= 0xDBFF && end - q >= 6 && q[0] == '\\' && q[1] == 'u') {
                    unsigned lo = 0;
                    int ok = 1;
                    for (int i = 2; i < 6 && ok; ++i) {
                        const int v = hexval(q[i]);
                        if (v < 0) ok = 0;
                        else lo = (lo << 4) | (unsigned)v;
                    }
                    if (ok && lo >= 0xDC00 && lo <= 0xDFFF) {
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        q += 6;
                    }
                }
                tl = put_utf8(cp, tmp);
                break;
            }
            default: return -1;
            }
        }
        if (n + tl > cap) return -1;
        memcpy(buf + n, tmp, (size_t)tl);
        n += tl;
    }
    if (q >= end) return -1;
    *p = q + 1;
    return n;
}

/* ------------------------------------------------------------------ */
/* loading                                                              */

static int set_vocab(g2_tokenizer *t, int sym, int id)
{
    if (sym >= t->sym_vocab_cap) {
        int nc = t->sym_vocab_cap ? t->sym_vocab_cap : 1 << 16;
        while (nc <= sym) nc *= 2;
        int *v = realloc(t->sym_vocab, (size_t)nc * sizeof *v);
        if (!v) return -1;
        for (int i = t->sym_vocab_cap; i < nc; ++i) v[i] = -1;
        t->sym_vocab = v;
        t->sym_vocab_cap = nc;
    }
    if (id >= t->vocab_size) {
        int *vs = realloc(t->vocab_sym, (size_t)(id + 1) * sizeof *vs);
        if (!vs) return -1;
        for (int i = t->vocab_size; i <= id; ++i) vs[i] = -1;
        t->vocab_sym = vs;
        t->vocab_size = id + 1;
    }
    /* a string listed twice keeps its later id; an id listed twice keeps
     * its later string (the earlier string stops decoding to it but still
     * encodes to it) */
    t->sym_vocab[sym] = id;
    t->vocab_sym[id] = sym;
    return 0;
}

static int load_vocab_json(g2_tokenizer *t, const char *path)
{
    size_t n = 0;
    char *b = slurp(path, &n);
    if (!b) return g2i_err(G2_E_IO, "cannot read %s", path);
    const char *p = b, *end = b + n;
    int rc = G2_OK;
    char *key = malloc(4096);
    if (!key) { free(b); return g2i_err(G2_E_NOMEM, "tokenizer"); }
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    if (p >= end || *p++ != '{') rc = g2i_err(G2_E_FORMAT, "%s: not a JSON object", path);
    while (!rc) {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r' || *p == ',')) ++p;
        if (p >= end || *p == '}') break;
        const int kl = json_string(&p, end, key, 4096);
        if (kl < 0) { rc = g2i_err(G2_E_FORMAT, "%s: bad token string", path); break; }
        while (p < end && (*p == ' ' || *p == '\t')) ++p;
        if (p >= end || *p++ != ':') { rc = g2i_err(G2_E_FORMAT, "%s: expected ':'", path); break; }
        while (p < end && (*p == ' ' || *p == '\t')) ++p;
        long id = 0;
        while (p < end && *p >= '0' && *p <= '9' && id <= INT_MAX / 16) id = id * 10 + (*p++ - '0');
        if (id > 16 * 1024 * 1024) { rc = g2i_err(G2_E_FORMAT, "%s: token id %ld", path, id); break; }
        const int sym = sy_intern(&t->sy, key, kl);
        if (sym < 0 || set_vocab(t, sym, (int)id)) rc = g2i_err(G2_E_NOMEM, "tokenizer vocabulary");
    }
    free(key);
    free(b);
    return rc;
}

static int load_merges_txt(g2_tokenizer *t, const char *path)
{
    size_t n = 0;
    char *b = slurp(path, &n);
    if (!b) return g2i_err(G2_E_IO, "cannot read %s", path);
    const char *p = b, *end = b + n;
    if (p < end && *p == '#') {
        while (p < end && *p != '\n') ++p;
        if (p < end) ++p;
    }
    int rank = 0, rc = G2_OK;
    char *cat = NULL;
    int catcap = 0;
    while (p < end && !rc) {
        const char *ls = p;
        while (p < end && *p != '\n') ++p;
        const char *le = p;
        if (p < end) ++p;
        while (le > ls && le[-1] == '\r') --le;
        const char *sp = le > ls ? memchr(ls, ' ', (size_t)(le - ls)) : NULL;
        if (!sp) continue;
        const int ll = (int)(sp - ls), rl = (int)(le - sp - 1);
        if (ll + rl > catcap) {
            catcap = 2 * (ll + rl) + 64;
            char *c = realloc(cat, (size_t)catcap);
            if (!c) { rc = g2i_err(G2_E_NOMEM, "tokenizer merges"); break; }
            cat = c;
        }
        memcpy(cat, ls, (size_t)ll);
        memcpy(cat + ll, sp + 1, (size_t)rl);
        const int a = sy_intern(&t->sy, ls, ll), c = sy_intern(&t->sy, sp + 1, rl);
        const int o = sy_intern(&t->sy, cat, ll + rl);
        if (a < 0 || c < 0 || o < 0 || pm_put(&t->mg, a, c, rank, o)) rc = g2i_err(G2_E_NOMEM, "tokenizer merges");
        ++rank;
    }
    free(cat);
    free(b);
    return rc;
}

void g2_tok_free(g2_tokenizer *t)
{
    if (!t) return;
    free(t->sy.arena); free(t->sy.off); free(t->sy.len); free(t->sy.slot);
    free(t->mg.key); free(t->mg.rank); free(t->mg.out);
    free(t->sym_vocab); free(t->vocab_sym);
    free(t);
}

int g2_tok_load(const char *dir, g2_tokenizer **out)
{
    if (!dir || !out) return g2i_err(G2_E_ARG, "NULL argument");
    *out = NULL;
    g2_tokenizer *t = calloc(1, sizeof *t);
    if (!t) return g2i_err(G2_E_NOMEM, "tokenizer");
    /* the byte alphabet: printable Latin-1 bytes are themselves, the rest
     * take code points 256, 257, ... in byte order */
    int next = 256, rc = G2_OK;
    for (int i = 0; i < 512; ++i) t->cp_byte[i] = -1;
    for (int byte = 0; byte < 256 && !rc; ++byte) {
        const int keep = (byte >= 33 && byte <= 126) || (byte >= 161 && byte <= 172) || byte >= 174;
        const int cp = keep ? byte : next++;
        char u[4];
        t->cp_byte[cp] = byte;
        t->byte_sym[byte] = sy_intern(&t->sy, u, put_utf8((unsigned)cp, u));
        if (t->byte_sym[byte] < 0) rc = g2i_err(G2_E_NOMEM, "tokenizer");
    }
    size_t dl = strlen(dir);
    char *path = malloc(dl + 16);
    if (!path && !rc) rc = g2i_err(G2_E_NOMEM, "tokenizer");
    if (!rc) {
        snprintf(path, dl + 16, "%s/vocab.json", dir);
        rc = load_vocab_json(t, path);
    }
    if (!rc) {
        snprintf(path, dl + 16, "%s/merges.txt", dir);
        rc = load_merges_txt(t, path);
    }
    free(path);
    if (rc) { g2_tok_free(t); return rc; }
    *out = t;
    return G2_OK;
}

int g2_tok_vocab_size(const g2_tokenizer *t) { return t ? t->vocab_size : 0; }

/* ------------------------------------------------------------------ */
/* encode / decode                                                      */

/* BPE of one piece of text; appends its tokens to ids[*n..max_ids). */
static void bpe_piece(const g2_tokenizer *t, const unsigned char *s, int len, int *sym, int *ids, int *n,
                      int max_ids)
{
    int k = len;
    for (int i = 0; i < len; ++i) sym[i] = t->byte_sym[s[i]];
    while (k > 1) {
        int best = INT_MAX, merged = -1;
        for (int i = 0; i + 1 < k; ++i) {
            int o;
            const int r = pm_get(&t->mg, sym[i], sym[i + 1], &o);
            if (r < best) { best = r; merged = o; }
        }
        if (best == INT_MAX) break;
        /* every occurrence of the lowest-ranked pair, left to right */
        int w = 0;
        for (int i = 0; i < k;) {
            int o;
            if (i + 1 < k && pm_get(&t->mg, sym[i], sym[i + 1], &o) == best) {
                sym[w++] = merged;
                i += 2;
            } else {
                sym[w++] = sym[i++];
            }
        }
        k = w;
    }
    for (int i = 0; i < k && *n < max_ids; ++i) {
        const int id = sym[i] < t->sym_vocab_cap ? t->sym_vocab[sym[i]] : -1;
        if (id >= 0) ids[(*n)++] = id;
    }
}

static int is_alpha(unsigned char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z'); }
static int is_num(unsigned char c) { return c >= '0' && c <= '9'; }
static int is_ws(unsigned char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\f' || c == '\v'; }
/* class of a non-space character: 1 letter, 2 digit, 3 other */
static int cclass(unsigned char c) { return is_alpha(c) ? 1 : (is_num(c) ? 2 : 3); }

int g2_tok_encode(const g2_tokenizer *t, const char *text, int *ids, int max_ids)
{
    if (!t || !text || !ids || max_ids <= 0) return -1;
    const unsigned char *s = (const unsigned char *)text;
    const int len = (int)strlen(text);
    int *sym = malloc(((size_t)len + 1) * sizeof *sym);
    if (!sym) return -1;
    int n = 0, i = 0;
    while (i < len && n < max_ids) {
        int j = i + 1;
        const unsigned char c = s[i];
        if (c == '\'' && i + 1 < len &&
            (s[i + 1] == 's' || s[i + 1] == 't' || s[i + 1] == 'm' || s[i + 1] == 'd')) {
            j = i + 2;
        } else if (c == '\'' && i + 2 < len &&
                   ((s[i + 1] == 'r' && s[i + 2] == 'e') || (s[i + 1] == 'v' && s[i + 2] == 'e') ||
                    (s[i + 1] == 'l' && s[i + 2] == 'l'))) {
            j = i + 3;
        } else if (c == ' ' && i + 1 < len && !is_ws(s[i + 1])) {
            const int k = cclass(s[i + 1]);
            j = i + 2;
            while (j < len && !is_ws(s[j]) && cclass(s[j]) == k) ++j;
        } else if (!is_ws(c)) {
            const int k = cclass(c);
            while (j < len && !is_ws(s[j]) && cclass(s[j]) == k) ++j;
        }
        bpe_piece(t, s + i, j - i, sym, ids, &n, max_ids);
        i = j;
    }
    free(sym);
    return n;
}

int g2_tok_decode(const g2_tokenizer *t, const int *ids, int n, char *out, int max_bytes)
{
    if (!t || !ids || !out || max_bytes <= 0) return -1;
    int w = 0;
    for (int i = 0; i < n; ++i) {
        if (ids[i] < 0 || ids[i] >= t->vocab_size || t->vocab_sym[ids[i]] < 0) continue;
        const int sm = t->vocab_sym[ids[i]];
        const unsigned char *s = (const unsigned char *)t->sy.arena + t->sy.off[sm];
        const int sl = t->sy.len[sm];
        for (int j = 0; j < sl;) {
            /* a sequence cut short by the end of the token reads zero bytes
             * past it (the reference's strings are NUL-terminated there) */
            unsigned char u[4] = {0, 0, 0, 0};
            memcpy(u, s + j, (size_t)(sl - j < 4 ? sl - j : 4));
            unsigned cp = 0;
            const int used = get_utf8(u, &cp);
            if (!used) break;
            int byte = cp < 512 ? t->cp_byte[cp] : -1;
            if (byte < 0) byte = '?';
            if (w >= max_bytes - 1) { out[w] = 0; return w; }
            out[w++] = (char)byte;
            j += used;
        }
    }
    out[w] = 0;
    return w;
}
