/*
 * g2_cli.c -- command-line driver (the reference's main(), main.c:1967-2200).
 *
 *   g2run (--model DIR | --synth small|medium|large|xl) [--seed S]
 *         [--format fp32|fp16] [--path fused|reference] [--tokenizer DIR]
 *         (--prompt TEXT | --ids 1,2,3 | --random-prompt P)
 *         [--max-tokens N] [--min-tokens N]
 *
 * Greedy decoding (temperature 0, repetition penalty off).  A text prompt is
 * encoded with vocab.json + merges.txt from --tokenizer (default: the
 * --model directory, which holds them as the reference's does, main.c:6,
 * 2057) to at most 1023 ids (main.c:2093); with a tokenizer loaded the
 * generated ids are also printed as text (main.c:1954).  Prints the ids and
 * a timing summary in the style of main.c:2162-2169.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g2hip.h"

static int preset(const char *name, g2_config *c)
{
    static const struct { const char *n; int L, E, H; } p[] = {
        { "small", 12, 768, 12 }, { "medium", 24, 1024, 16 },
        { "large", 36, 1280, 20 }, { "xl", 48, 1600, 25 } };
    for (size_t i = 0; i < sizeof p / sizeof p[0]; ++i)
        if (!strcmp(name, p[i].n)) {
            c->n_layer = p[i].L; c->n_embd = p[i].E; c->n_head = p[i].H;
            c->n_ctx = 1024; c->vocab_size = 50257; c->ffn_dim = 4 * p[i].E;
            return 0;
        }
    return -1;
}

static void die(const char *what, int rc)
{
    fprintf(stderr, "%s failed (%d): %s\n", what, rc, g2_last_error());
    exit(EXIT_FAILURE);
}

int main(int argc, char **argv)
{
    const char *model_dir = NULL, *synth = NULL, *ids_arg = NULL, *text = NULL, *tok_dir = NULL;
    unsigned long long seed = 0x67707432ULL;
    int dtype = G2_F32, path = G2_PATH_FUSED, random_prompt = 0, max_new = 32, min_new = 1;
    for (int i = 1; i < argc; ++i) {
        const char *a = argv[i];
        const char *v = i + 1 < argc ? argv[i + 1] : NULL;
        if (!strcmp(a, "--model") && v) { model_dir = v; ++i; }
        else if (!strcmp(a, "--synth") && v) { synth = v; ++i; }
        else if (!strcmp(a, "--seed") && v) { seed = strtoull(v, NULL, 0); ++i; }
        else if (!strcmp(a, "--format") && v) { dtype = !strcmp(v, "fp16") ? G2_F16 : G2_F32; ++i; }
        else if (!strcmp(a, "--path") && v) { path = !strcmp(v, "reference") ? G2_PATH_REFERENCE : G2_PATH_FUSED; ++i; }
        else if (!strcmp(a, "--ids") && v) { ids_arg = v; ++i; }
        else if (!strcmp(a, "--prompt") && v) { text = v; ++i; }
        else if (!strcmp(a, "--tokenizer") && v) { tok_dir = v; ++i; }
        else if (!strcmp(a, "--random-prompt") && v) { random_prompt = atoi(v); ++i; }
        else if (!strcmp(a, "--max-tokens") && v) { max_new = atoi(v); ++i; }
        else if (!strcmp(a, "--min-tokens") && v) { min_new = atoi(v); ++i; }
        else {
            fprintf(stderr, "usage: %s (--model DIR | --synth small|medium|large|xl) [--seed S] "
                            "[--format fp32|fp16] [--path fused|reference] [--tokenizer DIR] "
                            "(--prompt TEXT | --ids a,b,c | --random-prompt P) [--max-tokens N] "
                            "[--min-tokens N]\n", argv[0]);
            return EXIT_FAILURE;
        }
    }
    if ((!model_dir && !synth) || (!ids_arg && !text && random_prompt <= 0)) {
        fprintf(stderr, "need a model (--model/--synth) and a prompt (--prompt/--ids/--random-prompt)\n");
        return EXIT_FAILURE;
    }
    g2_tokenizer *tok = NULL;
    if (!tok_dir && model_dir && text) tok_dir = model_dir;
    if (tok_dir) {
        const int trc = g2_tok_load(tok_dir, &tok);
        if (trc) die("g2_tok_load", trc);
        printf("Tokenizer: %d tokens.\n", g2_tok_vocab_size(tok));
    }
    if (text && !tok) {
        fprintf(stderr, "--prompt needs vocab.json and merges.txt (--tokenizer DIR)\n");
        return EXIT_FAILURE;
    }
    int rc = g2_init(0);
    if (rc) die("g2_init", rc);
    char name[128];
    int cus = 0;
    g2_device_name(name, sizeof name, &cus);
    printf("Device: %s (%d CUs)\n", name, cus);

    g2_model *m = NULL;
    g2_config cfg;
    if (synth) {
        if (preset(synth, &cfg)) { fprintf(stderr, "unknown preset %s\n", synth); return EXIT_FAILURE; }
        rc = g2_model_synth(&cfg, seed, dtype, path, &m);
        if (rc) die("g2_model_synth", rc);
    } else {
        rc = g2_model_load(model_dir, dtype, path, &m);
        if (rc) die("g2_model_load", rc);
    }
    g2_model_config(m, &cfg);
    printf("Config: n_layer=%d n_embd=%d n_head=%d ffn=%d vocab=%d\n", cfg.n_layer, cfg.n_embd,
           cfg.n_head, cfg.ffn_dim, cfg.vocab_size);
    printf("Model VRAM: %.1f MiB\n", g2_model_weight_bytes(m) / 1048576.0);

    int prompt[G2_MAX_SEQ];
    int P = 0;
    if (text) {
        P = g2_tok_encode(tok, text, prompt, G2_MAX_SEQ - 1);
        if (P < 1) {
            fprintf(stderr, "the prompt encodes to no tokens\n");
            return EXIT_FAILURE;
        }
        printf("Prompt: %d tokens\n", P);
    } else if (ids_arg) {
        const char *s = ids_arg;
        while (*s && P < G2_MAX_SEQ - 1) {
            prompt[P++] = (int)strtol(s, (char **)&s, 10);
            while (*s == ',' || *s == ' ') ++s;
        }
    } else {
        unsigned long long x = seed ^ 0x5EEDULL;
        P = random_prompt < G2_MAX_SEQ - 1 ? random_prompt : G2_MAX_SEQ - 1;
        for (int i = 0; i < P; ++i) {
            x = x * 6364136223846793005ULL + 1442695040888963407ULL;
            prompt[i] = (int)((x >> 33) % (unsigned long long)cfg.vocab_size);
        }
    }
    int *out = malloc(sizeof(int) * G2_MAX_SEQ);
    double t[2] = { 0, 0 };
    const int n = g2_generate(m, prompt, P, max_new, min_new, out, t);
    if (n < 0) die("g2_generate", n);
    printf("Generated:");
    for (int i = 0; i < n; ++i) printf(" %d", out[i]);
    printf("\n");
    if (tok) {
        char *txt = malloc(16 * (size_t)G2_MAX_SEQ * 4 + 1);
        if (txt && g2_tok_decode(tok, out, n, txt, 16 * G2_MAX_SEQ * 4 + 1) >= 0) printf("Text: %s\n", txt);
        free(txt);
    }
    printf("Decode graph replay: %d\n", g2_model_uses_graph(m));
    fprintf(stderr,
            "Timing:\n"
            "  prefill+first : %9.3f ms (%d prompt tokens, %.1f tok/s)\n"
            "  decode (%3d steps): %9.3f ms (%.3f ms/token, %.1f tok/s)\n",
            t[0], P, t[0] > 0 ? P / (t[0] * 1e-3) : 0.0, n - 1, t[1],
            n > 1 ? t[1] / (n - 1) : 0.0, n > 1 && t[1] > 0 ? (n - 1) / (t[1] * 1e-3) : 0.0);
    free(out);
    g2_tok_free(tok);
    g2_model_free(m);
    g2_shutdown();
    return EXIT_SUCCESS;
}
