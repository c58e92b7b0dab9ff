"""The library's host-only parsers under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only).

tests/native/host_fuzz.c is compiled with gpt2-opencl-1.1_amd/csrc/g2_host.c
(the safetensors header reader behind g2_model_load, the config.json scan
behind g2_config_load; load_model / load_config, main.c:294-331 and
main.c:1141-1232) with -fsanitize=address,undefined and run over malformed
files: truncated headers, shapes whose element count overflows int64 or
wraps a 32-bit int, byte ranges past the end of the file, negative
dimensions, unterminated strings, deep nesting, and seeded random mutations
of a well-formed file.  Every file must give an error code or a clean read;
any sanitizer report fails the test.
"""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gpt2-opencl-1.1_amd", "csrc")
G2_E_FORMAT, G2_E_IO, G2_E_LIMIT = -4, -3, -5


@pytest.fixture(scope="module")
def fuzz_bin(tmp_path_factory):
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    out = str(tmp_path_factory.mktemp("san") / "host_fuzz")
    cmd = ["gcc", "-std=c99", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-D_POSIX_C_SOURCE=200809L", "-D__HIP_PLATFORM_AMD__",
           "-I" + os.path.join(ROOT, "include"), "-I" + CSRC, "-I/opt/rocm/include", "-o", out,
           os.path.join(ROOT, "tests", "native", "host_fuzz.c"), os.path.join(CSRC, "g2_host.c"), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip(f"sanitizer build unavailable: {r.stderr[-500:]}")
    return out


def run(binary, mode, files):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=99",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=98")
    r = subprocess.run([binary, mode] + [str(f) for f in files], capture_output=True, text=True, env=env,
                       timeout=600)
    assert r.returncode == 0, f"sanitizer or driver failure (rc {r.returncode}):\n{r.stderr[-3000:]}"
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
    lines = {}
    for line in r.stdout.splitlines():
        name, rest = line.split(" ", 1)
        lines[os.path.basename(name)] = rest
    return lines


def st_bytes(hdr, data=b""):
    h = hdr if isinstance(hdr, bytes) else json.dumps(hdr).encode()
    return struct.pack("<Q", len(h)) + h + data


def rc_of(line):
    return int(line.split("rc=")[1].split()[0])


def test_safetensors_malformed_headers(fuzz_bin, tmp_path):
    good = np.arange(12, dtype=np.float32).tobytes()
    cases = {
        "ok": (st_bytes({"a": {"dtype": "F32", "shape": [3, 4], "data_offsets": [0, 48]}}, good), 0),
        "ok_f16_bf16": (st_bytes({"a": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]},
                                  "b": {"dtype": "BF16", "shape": [2], "data_offsets": [4, 8]},
                                  "__metadata__": {"format": "pt"}}, b"\0" * 8), 0),
        "empty_object": (st_bytes(b"{}"), 0),
        "short_len": (b"\x10\x00", G2_E_IO),
        "len_past_eof": (struct.pack("<Q", 1000) + b"{}", G2_E_IO),
        "zero_len": (struct.pack("<Q", 0), G2_E_FORMAT),
        "huge_len": (struct.pack("<Q", 1 << 40), G2_E_FORMAT),
        # [2^32 + 64, 192] with offsets that match the (huge) element count:
        # the bytes would lie far past the end of the file
        "wrap32": (st_bytes({"w": {"dtype": "F32", "shape": [(1 << 32) + 64, 192],
                                   "data_offsets": [0, ((1 << 32) + 64) * 192 * 4]}}, good), G2_E_FORMAT),
        "past_eof": (st_bytes({"w": {"dtype": "F32", "shape": [3, 4], "data_offsets": [0, 48]}}, good[:20]),
                     G2_E_FORMAT),
        "begin_past_eof": (st_bytes({"w": {"dtype": "F32", "shape": [1], "data_offsets": [4000, 4004]}}, good),
                           G2_E_FORMAT),
        "negative_dim": (st_bytes({"w": {"dtype": "F32", "shape": [-3, -4], "data_offsets": [0, 48]}}, good),
                         G2_E_FORMAT),
        "overflow_product": (st_bytes({"w": {"dtype": "F32", "shape": [1 << 40, 1 << 40, 1 << 40],
                                             "data_offsets": [0, 48]}}, good), G2_E_FORMAT),
        "int64_max_dim": (st_bytes({"w": {"dtype": "F32", "shape": [9223372036854775807], "data_offsets": [0, 48]}},
                                   good), G2_E_FORMAT),
        "mismatch": (st_bytes({"w": {"dtype": "F32", "shape": [3, 3], "data_offsets": [0, 48]}}, good), G2_E_FORMAT),
        "reversed": (st_bytes({"w": {"dtype": "F32", "shape": [3], "data_offsets": [12, 0]}}, good), G2_E_FORMAT),
        "nine_dims": (st_bytes({"w": {"dtype": "F32", "shape": [1] * 9, "data_offsets": [0, 4]}}, good), G2_E_FORMAT),
        "no_dtype": (st_bytes({"w": {"shape": [3], "data_offsets": [0, 12]}}, good), G2_E_FORMAT),
        "unterminated": (st_bytes(b'{"a": {"dtype": "F32", "shape": [2], "data_offsets": [0'), G2_E_FORMAT),
        "unterminated_str": (st_bytes(b'{"abc'), G2_E_FORMAT),
        "escape_at_end": (st_bytes(b'{"a\\'), G2_E_FORMAT),
        "unicode_escape_short": (st_bytes(b'{"a\\u12'), G2_E_FORMAT),
        "deep_metadata": (st_bytes(b'{"__metadata__": ' + b"[" * 5000 + b"]" * 5000 + b"}"), 0),
        "deep_unclosed": (st_bytes(b'{"__metadata__": ' + b"[" * 5000 + b"}"), G2_E_FORMAT),
        "not_object": (st_bytes(b"[1, 2]"), G2_E_FORMAT),
        "long_name": (st_bytes({"n" * 5000: {"dtype": "F32", "shape": [3], "data_offsets": [0, 12]}}, good), 0),
        "many_tensors": (st_bytes({f"t{i}": {"dtype": "F32", "shape": [1], "data_offsets": [4 * (i % 12), 4 * (i % 12) + 4]}
                                   for i in range(300)}, good), 0),
        "bad_number": (st_bytes(b'{"w": {"dtype": "F32", "shape": [x], "data_offsets": [0, 4]}}'), G2_E_FORMAT),
        "other_dtype": (st_bytes({"w": {"dtype": "I64", "shape": [3], "data_offsets": [0, 24]}}, good), 0),
    }
    files = []
    for name, (blob, _) in cases.items():
        p = tmp_path / name
        p.write_bytes(blob)
        files.append(p)
    out = run(fuzz_bin, "st", files)
    for name, (_, want) in cases.items():
        assert rc_of(out[name]) == want, f"{name}: {out[name]}"
    assert "reads=1" in out["ok"] and "reads=2" in out["ok_f16_bf16"]


def test_safetensors_random_mutations(fuzz_bin, tmp_path):
    """Seeded byte flips, truncations and splices of a well-formed file of a
    tiny model: every variant opens cleanly or fails with an error code."""
    rng = np.random.default_rng(1234)
    hdr, data, off = {}, b"", 0
    for i, shape in enumerate([(4, 8), (8,), (2, 3, 4), (16,)]):
        a = rng.standard_normal(shape).astype(np.float32).tobytes()
        hdr[f"h.{i}.w"] = {"dtype": "F32", "shape": list(shape), "data_offsets": [off, off + len(a)]}
        data += a
        off += len(a)
    base = bytearray(st_bytes(hdr, data))
    hlen = struct.unpack("<Q", bytes(base[:8]))[0]
    files = []
    for k in range(400):
        b = bytearray(base)
        kind = k % 4
        if kind == 0:  # flip bytes inside the header
            for _ in range(int(rng.integers(1, 6))):
                b[8 + int(rng.integers(0, hlen))] = int(rng.integers(0, 256))
        elif kind == 1:  # truncate anywhere
            b = b[: int(rng.integers(0, len(b)))]
        elif kind == 2:  # replace a digit run of the header with a large number
            text = b[8:8 + hlen].decode("latin1")
            digits = [i for i, c in enumerate(text) if c.isdigit()]
            i = digits[int(rng.integers(0, len(digits)))]
            big = str(int(rng.choice([2 ** 31, 2 ** 32 + 7, 2 ** 62, 2 ** 63 - 1, 10 ** 30])))
            text = text[:i] + big + text[i + 1:]
            h = text.encode("latin1")
            b = bytearray(struct.pack("<Q", len(h)) + h + bytes(base[8 + hlen:]))
        else:  # corrupt the length prefix
            b[:8] = struct.pack("<Q", int(rng.integers(0, 2 * len(b))))
        p = tmp_path / f"m{k}"
        p.write_bytes(bytes(b))
        files.append(p)
    out = run(fuzz_bin, "st", files)
    assert len(out) == len(files)
    assert any(rc_of(v) == 0 for v in out.values()) and any(rc_of(v) < 0 for v in out.values())


def test_config_scan_malformed(fuzz_bin, tmp_path):
    cases = {
        "empty": ("", 0),
        "huge": ('{"n_layer": 99999999999999999999, "n_embd": 768, "n_head": 12}', G2_E_LIMIT),
        "negative": ('{"n_embd": -2147483648}', G2_E_FORMAT),
        "inner_overflow": ('{"n_embd": 2147483647}', G2_E_LIMIT),
        "key_at_end": ('{"n_layer"', 0),
        "colon_at_end": ('{"n_layer":', G2_E_FORMAT),
        "garbage": ("\x01\x02\xff" * 100, 0),
        "xl": ('{"n_layer": 48, "n_embd": 1600, "n_head": 25}', 0),
    }
    files = []
    for name, (text, _) in cases.items():
        p = tmp_path / name
        p.write_bytes(text.encode("latin1"))
        files.append(p)
    out = run(fuzz_bin, "cfg", files)
    for name, (_, want) in cases.items():
        assert rc_of(out[name]) == want, f"{name}: {out[name]}"
    assert "L=48 E=1600 H=25" in out["xl"] and "F=6400" in out["xl"]
