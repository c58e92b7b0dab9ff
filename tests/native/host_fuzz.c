/*
 * host_fuzz.c -- driver for the sanitizer build of the library's host-only
 * parsers (g2_host.c: the safetensors header reader and config.json scan).
 * Test infrastructure: tests/test_host_sanitize.py compiles it together with
 * g2_host.c under AddressSanitizer and UndefinedBehaviorSanitizer and runs it
 * over malformed inputs.
 *
 * Usage: host_fuzz st FILE...      open each safetensors file, read every
 *                                  tensor of at most 2^22 elements as fp32
 *        host_fuzz cfg FILE...     parse each file as a config.json string
 * One line per file: "<file> rc=<code> tensors=<n>" (or cfg values).
 */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g2_internal.h"
#include "g2_host.h"

/* The library's error hook (g2_shim.c holds the real one, which needs the
 * HIP runtime): keep the message for the line printed per file. */
static char msg[512];
int g2i_err(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    return code;
}

static int run_st(const char *path)
{
    g2h_st st;
    msg[0] = 0;
    int rc = g2h_st_open(path, &st);
    int n = 0, reads = 0;
    if (rc == G2_OK) {
        n = st.n;
        for (int i = 0; i < st.n; ++i) {
            const g2h_tensor *t = g2h_st_find(&st, st.t[i].name);
            if (!t || t->numel > ((int64_t)1 << 22) || t->dtype == G2H_ST_OTHER) continue;
            float *buf = malloc((size_t)(t->numel > 0 ? t->numel : 1) * sizeof(float));
            if (!buf) continue;
            if (g2h_st_read_f32(&st, t, buf, t->numel) == G2_OK) ++reads;
            /* a capacity one element short must be refused, never overrun */
            if (t->numel > 0 && g2h_st_read_f32(&st, t, buf, t->numel - 1) == G2_OK) {
                printf("%s overran capacity\n", path);
                exit(3);
            }
            free(buf);
        }
        g2h_st_close(&st);
    }
    printf("%s rc=%d tensors=%d reads=%d msg=%s\n", path, rc, n, reads, msg);
    return 0;
}

static int run_cfg(const char *path)
{
    size_t size = 0;
    char *json = g2h_slurp(path, &size);
    if (!json) { printf("%s rc=io\n", path); return 0; }
    g2_config c;
    memset(&c, 0, sizeof c);
    msg[0] = 0;
    const int rc = g2_config_parse(json, &c);
    printf("%s rc=%d L=%d E=%d H=%d V=%d F=%d\n", path, rc, c.n_layer, c.n_embd, c.n_head, c.vocab_size, c.ffn_dim);
    free(json);
    return 0;
}

int main(int argc, char **argv)
{
    if (argc < 3) return 2;
    for (int i = 2; i < argc; ++i) {
        if (!strcmp(argv[1], "st")) run_st(argv[i]);
        else run_cfg(argv[i]);
    }
    return 0;
}
