"""Writes the text-tokenizer fixture and its golden vectors (run in the
build container, where the reference's sources are):

  tests/golden/tok/vocab.json, merges.txt -- a small GPT-2-style byte-level
      BPE vocabulary trained here on a seeded synthetic corpus (the real
      GPT-2 files are not available offline), written with the quirks the
      loaders must handle: a '#version' first line, a blank line, a line
      without a space, CRLF endings, a merge listed twice (the later rank
      counts), JSON \\uXXXX escapes incl. a surrogate pair, an id gap, an id
      given to two strings and a string given two ids;
  tests/golden/tok/cases.json -- for each test text: the ids and the decoded
      bytes produced by the reference's own tokenizer (tokenizer.c built
      from its sources into oracle/_ref/libreftok.so by `make -C oracle
      ref`), plus decodes of hand-made id lists.

Usage: python3 tests/golden/make_tokenizer_fixture.py
"""
import ctypes as C
import json
import os
import random
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle.tokenizer import BYTE_CP, Tokenizer, _utf8  # noqa: E402

OUT = os.path.join(HERE, "tok")
N_MERGES = 400

WORDS = ("the of and to in is was he for it with as his on be at by had are but from or have an they "
         "which one you were her all she there would their we him been has when who will more no if out "
         "so said what up its about into than them can only other new some could time these two may then "
         "do first any my now such like our over man me even most made after also did many before must "
         "through back years where much your way well down should because each just those people Mr how "
         "too little state good very make world still own see men work long get here between both life "
         "being under never day same another know while last might us great old year off come since "
         "against go came right used take three GPU kernel memory tensor layer token decode prefill "
         "attention matrix cache HBM bandwidth").split()
EXTRA = ["don't", "we're", "I'll", "it's", "they've", "she'd", "I'm", "can't", "won't", "2024", "1024",
         "3.14", "x86", "gfx950", "e.g.", "U.S.", "--", "...", "!!", "?", "(see", "below)", "[1]", "#8",
         "café", "naïve", "über", "日本語", "🙂", "Ω", "—", "“quoted”"]


def corpus(seed=7, n=6000):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        w = rng.choice(WORDS) if rng.random() < 0.85 else rng.choice(EXTRA)
        if rng.random() < 0.08:
            w = w.capitalize()
        sep = " " if rng.random() < 0.9 else rng.choice([", ", ". ", "\n", "  ", "\t", "; "])
        out.append(w + sep)
    return "".join(out).encode("utf-8")


def train(data, n_merges):
    freq = {}
    for p in Tokenizer.pieces(data):
        freq[p] = freq.get(p, 0) + 1
    words = [[_utf8(BYTE_CP[b]) for b in p] for p in freq]
    counts = list(freq.values())
    merges = []
    for _ in range(n_merges):
        pairs = {}
        for w, c in zip(words, counts):
            for a, b in zip(w, w[1:]):
                pairs[(a, b)] = pairs.get((a, b), 0) + c
        if not pairs:
            break
        best = max(pairs.items(), key=lambda kv: (kv[1], tuple(-x for x in kv[0][0] + b"|" + kv[0][1])))[0]
        merges.append(best)
        a, b = best
        for k, w in enumerate(words):
            i, nw = 0, []
            while i < len(w):
                if i + 1 < len(w) and w[i] == a and w[i + 1] == b:
                    nw.append(a + b)
                    i += 2
                else:
                    nw.append(w[i])
                    i += 1
            words[k] = nw
    return merges


def jstr(b):
    """JSON string of token bytes with every non-ASCII code point escaped."""
    return json.dumps(b.decode("utf-8", "surrogatepass"), ensure_ascii=True)


def write_files():
    os.makedirs(OUT, exist_ok=True)
    merges = train(corpus(), N_MERGES)
    tokens = [_utf8(cp) for cp in BYTE_CP]
    for a, b in merges:
        if a + b not in tokens:
            tokens.append(a + b)
    entries = [(t, i) for i, t in enumerate(tokens)]
    nid = len(tokens)
    entries.append(("<|endoftext|>".encode(), nid + 1))          # id gap at nid
    entries.append(("😀".encode(), nid + 2))                     # surrogate-pair escape; decodes to '?'
    entries.append(("shared-id-first".encode(), nid + 3))
    entries.append(("shared-id-second".encode(), nid + 3))       # id given twice: the later string decodes
    entries.append((tokens[300], nid + 4))                       # a string given twice: the later id encodes
    with open(os.path.join(OUT, "vocab.json"), "w", newline="") as f:
        f.write("{" + ", ".join(f"{jstr(t)}: {i}" for t, i in entries) + "}\n")
    lines = [f"{a.decode('utf-8', 'surrogatepass')} {b.decode('utf-8', 'surrogatepass')}" for a, b in merges]
    # quirks: a blank line, a line without a space, CRLF endings, and the
    # 6th merge repeated near the end (its later rank applies)
    body = lines[:40] + [""] + lines[40:80] + ["nospacehere"] + lines[80:] + [lines[5]]
    text = "#version: 0.2\n" + "".join(l + ("\r\n" if k % 7 == 3 else "\n") for k, l in enumerate(body))
    with open(os.path.join(OUT, "merges.txt"), "wb") as f:
        f.write(text.encode("utf-8"))
    return nid


TEXTS = [
    "", " ", "  ", "hello", " hello", "hello world", "Hello, World!", "don't", "we're here", "I'll go",
    "'s", "''s", "' s", "it's 2024", "12345 678", "a1b2c3", "x  y", "tab\there", "new\nline", "trailing ",
    "  leading", "\r\n", "\n\n\nend", "mixed CASE words", "punct!!!", " ...", "café naïve", "日本語 text",
    "emoji 😀!", "can't won't shouldn't", "the kernel decode cache", "GPU memory bandwidth (see below)",
    "e.g. U.S. [1] #8", "\t\t tabs", "a'b 're 've 'll 'm 'd 't", "'", "x'", "9'9", "   nbsp",
    "“quoted” — dash", "Ω Ωmega", "   \t  ", "end.",
]


def reference():
    lib = C.CDLL(os.path.join(ROOT, "oracle", "_ref", "libreftok.so"))
    lib.gpt2_tokenizer_load.restype = C.c_void_p
    lib.gpt2_tokenizer_load.argtypes = [C.c_char_p]
    lib.gpt2_encode.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_int), C.c_int]
    lib.gpt2_decode.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.c_int, C.c_char_p, C.c_int]
    lib.gpt2_tokenizer_vocab_size.argtypes = [C.c_void_p]
    t = lib.gpt2_tokenizer_load(OUT.encode())
    assert t, "reference tokenizer failed to load the fixture"
    return lib, t


def ref_encode(lib, t, data, max_ids):
    buf = (C.c_int * max_ids)()
    n = lib.gpt2_encode(t, data, buf, max_ids)
    return list(buf[:n])


def ref_decode(lib, t, ids, max_bytes):
    arr = (C.c_int * max(len(ids), 1))(*ids)
    out = C.create_string_buffer(max_bytes)
    n = lib.gpt2_decode(t, arr, len(ids), out, max_bytes)
    return out.raw[:n]


def main():
    nid = write_files()
    lib, t = reference()
    rng = random.Random(11)
    texts = [s.encode("utf-8") for s in TEXTS]
    c = corpus(seed=23, n=400)
    for _ in range(30):
        a = rng.randrange(0, len(c) - 200)
        texts.append(c[a:a + rng.randrange(1, 200)].replace(b"\0", b""))
    cases = []
    for s in texts:
        for max_ids in (1023, 3):
            ids = ref_encode(lib, t, s, max_ids)
            cases.append({"text": s.hex(), "max_ids": max_ids, "ids": ids,
                          "decoded": ref_decode(lib, t, ids, 4096).hex()})
    decodes = []
    for ids, mb in [([nid + 2], 64), ([nid + 3], 64), ([nid], 64), ([-1, 5, 10**6], 64),
                    ([nid + 1, 300, nid + 4], 64), (list(range(0, 400, 7)), 10), ([], 8), ([65, 66], 1)]:
        decodes.append({"ids": ids, "max_bytes": mb, "bytes": ref_decode(lib, t, ids, mb).hex()})
    with open(os.path.join(OUT, "cases.json"), "w") as f:
        json.dump({"vocab_size": lib.gpt2_tokenizer_vocab_size(t), "encode": cases, "decode": decodes}, f,
                  indent=0)
    print(f"{len(cases)} encode cases, {len(decodes)} decode cases, vocab size "
          f"{lib.gpt2_tokenizer_vocab_size(t)}")


if __name__ == "__main__":
    main()
