"""Text tokenizer (g2_tok_*: the reference's tokenizer.c behind the C ABI),
host-only, so these run on the CPU.

Pinned by: golden vectors written by the reference's own tokenizer.c built
from its sources (tests/golden/make_tokenizer_fixture.py, fixture in
tests/golden/tok/), the same comparison live against that build when it is
present (oracle/_ref/libreftok.so, built by `make -C oracle ref` where the
reference sources are), the oracle restatement (oracle/tokenizer.py) on
random text, HF transformers' GPT2Tokenizer on text where the two
pre-tokenisers agree (the byte alphabet and the ranked-merge procedure), and
decode(encode(s)) == s.
"""
import ctypes as C
import json
import os
import random
import shutil

import numpy as np
import pytest

import g2hip as g2lib
from oracle import tokenizer as otok

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "tok")
REF_SO = os.path.join(os.path.dirname(HERE), "oracle", "_ref", "libreftok.so")
CASES = json.load(open(os.path.join(FIX, "cases.json")))

# characters that exercise every pre-tokeniser rule: letters, digits, the
# contraction letters, punctuation, every whitespace byte, non-ASCII text
ALPHABET = list("aZe tsmdrvlLT09'  \t\n\r\f\v.,!?-(\"\\/") + ["é", "日", "😀", "—", "Ġ", " "]


def fuzz(n, seed):
    rng = random.Random(seed)
    return ["".join(rng.choice(ALPHABET) for _ in range(rng.randrange(0, 40))) for _ in range(n)]


@pytest.fixture(scope="module")
def lib_tok():
    t = g2lib.Tokenizer(FIX)
    yield t
    t.free()


@pytest.fixture(scope="module")
def oracle_tok():
    return otok.Tokenizer(FIX)


def test_oracle_matches_reference_golden(oracle_tok):
    assert oracle_tok.vocab_size == CASES["vocab_size"]
    for c in CASES["encode"]:
        text = bytes.fromhex(c["text"])
        assert oracle_tok.encode(text, c["max_ids"]) == c["ids"], text
        assert oracle_tok.decode(c["ids"]) == bytes.fromhex(c["decoded"])
    for d in CASES["decode"]:
        assert oracle_tok.decode(d["ids"], d["max_bytes"]) == bytes.fromhex(d["bytes"]), d


def test_library_matches_reference_golden(lib_tok):
    assert lib_tok.vocab_size == CASES["vocab_size"]
    for c in CASES["encode"]:
        text = bytes.fromhex(c["text"])
        assert lib_tok.encode(text, c["max_ids"]).tolist() == c["ids"], text
        assert lib_tok.decode(c["ids"], 4096) == bytes.fromhex(c["decoded"])
    for d in CASES["decode"]:
        assert lib_tok.decode(d["ids"], d["max_bytes"]) == bytes.fromhex(d["bytes"]), d


def test_library_matches_oracle_on_random_text(lib_tok, oracle_tok):
    for s in fuzz(3000, 1):
        for max_ids in (1023, 4):
            ids = lib_tok.encode(s, max_ids).tolist()
            assert ids == oracle_tok.encode(s, max_ids), repr(s)
        assert lib_tok.decode(ids, 4096) == oracle_tok.decode(ids)
    rng = np.random.default_rng(2)
    for _ in range(300):
        ids = rng.integers(-3, CASES["vocab_size"] + 3, rng.integers(0, 12)).tolist()
        mb = int(rng.integers(1, 40))
        assert lib_tok.decode(ids, mb) == oracle_tok.decode(ids, mb), (ids, mb)


@pytest.mark.skipif(not os.path.exists(REF_SO), reason="the reference tokenizer is built only where its sources are")
def test_library_matches_reference_build_on_random_text(lib_tok):
    ref = C.CDLL(REF_SO)
    ref.gpt2_tokenizer_load.restype = C.c_void_p
    ref.gpt2_tokenizer_load.argtypes = [C.c_char_p]
    ref.gpt2_encode.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_int), C.c_int]
    ref.gpt2_decode.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.c_int, C.c_char_p, C.c_int]
    ref.gpt2_tokenizer_free.argtypes = [C.c_void_p]
    t = ref.gpt2_tokenizer_load(FIX.encode())
    assert t
    try:
        for s in fuzz(3000, 3):
            raw = s.encode()
            buf = (C.c_int * 1023)()
            n = ref.gpt2_encode(t, raw, buf, 1023)
            assert lib_tok.encode(raw).tolist() == list(buf[:n]), repr(s)
            out = C.create_string_buffer(4096)
            m = ref.gpt2_decode(t, buf, n, out, 4096)
            assert lib_tok.decode(list(buf[:n]), 4096) == out.raw[:m]
    finally:
        ref.gpt2_tokenizer_free(t)


def test_byte_alphabet_matches_gpt2():
    from transformers.convert_slow_tokenizer import bytes_to_unicode
    assert {b: chr(cp) for b, cp in enumerate(otok.BYTE_CP)} == bytes_to_unicode()


def test_merges_match_hf_gpt2_where_pretokenisers_agree(lib_tok, tmp_path):
    """ASCII words and punctuation separated by single spaces: the
    reference's pre-tokeniser and GPT-2's regex cut the same pieces, so the
    ids must equal HF's GPT2Tokenizer on the same files."""
    from transformers import GPT2Tokenizer
    shutil.copy(os.path.join(FIX, "vocab.json"), tmp_path / "vocab.json")
    # HF rejects the fixture's blank and space-less lines; without them (and
    # the CRs) the ranks are the ones the reference gives
    lines = open(os.path.join(FIX, "merges.txt"), "rb").read().split(b"\n")
    keep = [ln.rstrip(b"\r") for ln in lines[1:] if b" " in ln.rstrip(b"\r")]
    (tmp_path / "merges.txt").write_bytes(lines[0] + b"\n" + b"\n".join(keep) + b"\n")
    hf = GPT2Tokenizer(str(tmp_path / "vocab.json"), str(tmp_path / "merges.txt"))
    rng = random.Random(5)
    words = ["the", "kernel", "decode", "don't", "we're", "I'll", "it's", "2024", "x86", "GPU", "memory",
             "e.g.", "...", "!", "(see", "below)", "Mr", "cache", "3.14", "they've"]
    for _ in range(500):
        s = " ".join(rng.choice(words) for _ in range(rng.randrange(1, 12)))
        assert lib_tok.encode(s).tolist() == hf.encode(s), s


def test_round_trip(lib_tok):
    for s in fuzz(2000, 4):
        raw = s.encode()
        assert lib_tok.decode(lib_tok.encode(raw, 4096)) == raw, repr(s)


def test_errors(lib_tok, tmp_path):
    g2 = g2lib
    with pytest.raises(g2.G2Error):
        g2.Tokenizer(tmp_path)  # no vocab.json
    (tmp_path / "vocab.json").write_text('{"a": 0, ')
    with pytest.raises(g2.G2Error):
        g2.Tokenizer(tmp_path)  # no merges.txt
    (tmp_path / "merges.txt").write_text("#version: 0.2\n")
    (tmp_path / "vocab.json").write_text('{"a": 0, "\\q": 1}')
    with pytest.raises(g2.G2Error):
        g2.Tokenizer(tmp_path)  # bad escape
    with pytest.raises(g2.G2Error):
        lib_tok.encode("abc", 0)
    with pytest.raises(g2.G2Error):
        lib_tok.encode(b"a\0b")
    assert lib_tok.encode("").tolist() == []


@pytest.mark.gpu
def test_cli_text_prompt(g2):
    """g2run --prompt: the text is encoded with the fixture vocabulary, the
    model generates from those ids, and the output is printed as text.  The
    child runs while this process holds the GPU, so its cooperative launches
    are refused and it decodes with the per-operator kernels."""
    import subprocess
    exe = os.path.join(os.path.dirname(HERE), "gpt2-opencl-1.1_amd", "g2run")
    text = "the kernel decode cache"
    r = subprocess.run([exe, "--synth", "small", "--format", "fp16", "--tokenizer", FIX, "--prompt", text,
                        "--max-tokens", "4"], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    n = len(g2lib.Tokenizer(FIX).encode(text))
    assert f"Prompt: {n} tokens" in r.stdout
    assert "Text:" in r.stdout and "Generated:" in r.stdout
