"""Model files loaded onto the GPU (g2_model_load) against the oracle.

load_model (main.c:1339-1417) with detect_weight_layout / load_linear_weight
(main.c:1234-1300), the name fallbacks "transformer." / "model."
(main.c:1194-1207) and the tied or separate lm_head (main.c:1374-1405),
extended here to F16 and BF16 tensors (widened on the host).  A tiny GPT-2
with random biases and LayerNorm parameters is written as
config.json + model.safetensors in four forms:

  f32-conv1d   F32, Conv1D layout [in, out], names "transformer.h.0..."
  f32-linear   F32, Linear layout [out, in] (transposed on load), no prefix
  f16          every tensor F16, names "model.h.0...", separate lm_head [V, E]
  bf16         every tensor BF16, separate lm_head stored [E, V]

and loaded with fp32 or fp16 device weights on the fused path (and fp32 on
the reference path).  The oracle gets the values the file holds after the
same conversions (fp16 / bf16 widened exactly; fp16 device weights round
matrices and embeddings to fp16), so prefill and teacher-forced decode
logits must agree within 2e-3 and greedy ids must be identical (a parting
only at an oracle near tie below 1e-4).
"""
import json
import struct

import numpy as np
import pytest

from oracle import oracle
from parity import TIE_TOL, greedy_agree, masked_first_max, random_prompt

pytestmark = pytest.mark.gpu

SEED = 0x67707432
NAMES = ["ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias", "attn.c_proj.weight",
         "attn.c_proj.bias", "ln_2.weight", "ln_2.bias", "mlp.c_fc.weight", "mlp.c_fc.bias",
         "mlp.c_proj.weight", "mlp.c_proj.bias"]
MATRIX_SLOTS = {2, 4, 8, 10}


def bf16_round(a):
    """fp32 -> bf16 with round to nearest even, returned as the bf16 bit patterns."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_widen(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, numpy array of the stored element type)."""
    hdr, blobs, off = {}, [], 0
    for name, (dt, arr) in tensors.items():
        data = np.ascontiguousarray(arr).tobytes()
        hdr[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    h = json.dumps(hdr).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def make_model_dir(tmp_path, g2, cfg, form):
    """Writes the model in `form`; returns (directory, the fp32 weights the file holds)."""
    w = g2.synth_weights(cfg, SEED, affine=True)
    E, V = cfg.n_embd, cfg.vocab_size
    lm = None
    if form in ("f16", "bf16"):  # a separate head, unlike wte
        lm = (np.random.default_rng(3).standard_normal((V, E)) * 0.02).astype(np.float32)
    prefix = {"f32-conv1d": "transformer.", "f32-linear": "", "f16": "model.", "bf16": ""}[form]

    def enc(a):
        """(stored dtype, stored array, values the loader reads back as fp32)"""
        if form == "f16":
            h = a.astype(np.float16)
            return "F16", h, h.astype(np.float32)
        if form == "bf16":
            b = bf16_round(a)
            return "BF16", b, bf16_widen(b)
        return "F32", a.astype(np.float32), a.astype(np.float32)

    t, held = {}, {"layers": []}

    def put(name, a):
        dt, stored, back = enc(a)
        t[prefix + name] = (dt, stored)
        return back

    held["wte"] = put("wte.weight", w["wte"])
    held["wpe"] = put("wpe.weight", w["wpe"])
    held["lnf_w"] = put("ln_f.weight", w["lnf_w"])
    held["lnf_b"] = put("ln_f.bias", w["lnf_b"])
    for l, lw in enumerate(w["layers"]):
        vals = []
        for s, (n, a) in enumerate(zip(NAMES, lw)):
            if s in MATRIX_SLOTS and form == "f32-linear":
                vals.append(put(f"h.{l}.{n}", a.T.copy()).T.copy())  # stored [out, in]
            else:
                vals.append(put(f"h.{l}.{n}", a))
        held["layers"].append(tuple(vals))
    if lm is not None:
        if form == "bf16":
            held["lm_head"] = put("lm_head.weight", lm.T.copy()).T.copy()  # stored [E, V]
        else:
            held["lm_head"] = put("lm_head.weight", lm)
    d = tmp_path / form
    d.mkdir()
    (d / "config.json").write_text(json.dumps({"n_layer": cfg.n_layer, "n_embd": E, "n_head": cfg.n_head,
                                               "vocab_size": V, "n_positions": 1024}))
    write_safetensors(d / "model.safetensors", t)
    return str(d), held


def device_values(held, f16):
    """What an fp16-weight model computes with: matrices, embeddings and the
    head rounded to fp16, LayerNorm parameters and biases kept fp32."""
    if not f16:
        return held
    r = lambda a: a.astype(np.float16).astype(np.float32)
    out = {"wte": r(held["wte"]), "wpe": r(held["wpe"]), "lnf_w": held["lnf_w"], "lnf_b": held["lnf_b"],
           "layers": [tuple(r(a) if s in MATRIX_SLOTS else a for s, a in enumerate(lw)) for lw in held["layers"]]}
    if "lm_head" in held:
        out["lm_head"] = r(held["lm_head"])
    return out


LOADS = [("f32-conv1d", "f32", "fused"), ("f32-conv1d", "f32", "reference"), ("f32-linear", "f32", "fused"),
         ("f32-linear", "f16", "fused"), ("f16", "f16", "fused"), ("f16", "f32", "reference"),
         ("bf16", "f16", "fused"), ("bf16", "f32", "fused")]


@pytest.mark.parametrize("form,wdt,path", LOADS, ids=[f"{a}-{b}-{c}" for a, b, c in LOADS])
def test_load_file_matches_oracle(g2, tmp_path, form, wdt, path):
    cfg = g2.make_config(2, 128, 2, vocab_size=300)
    d, held = make_model_dir(tmp_path, g2, cfg, form)
    f16 = wdt == "f16"
    om = oracle.Model(cfg, device_values(held, f16), kslice=4)
    P, n_new = 37, 20
    prompt = random_prompt(P, cfg.vocab_size, 5)
    ref_ids, top2, _ = om.generate(prompt, n_new, min_new=n_new)
    ref_lg = om.teacher_forced(prompt, ref_ids[:-1])
    om.close()
    print(f"\n[load] {form} -> {wdt} {path}", flush=True)
    m = g2.Model.load(d, g2.F16 if f16 else g2.F32, g2.PATH_REFERENCE if path == "reference" else g2.PATH_FUSED)
    c = m.cfg
    assert (c.n_layer, c.n_embd, c.n_head, c.vocab_size, c.ffn_dim) == (2, 128, 2, 300, 512)
    ids, _ = m.generate(prompt, n_new, min_new=n_new)
    greedy_agree(ids, ref_ids, top2)
    gaps = top2[:, 0] - top2[:, 1]
    m.prefill(prompt)
    err = 0.0
    for k in range(n_new):
        if k > 0:
            m.decode(int(ref_ids[k - 1]), P + k - 1)
        lg = m.logits()
        err = max(err, float(np.abs(lg - ref_lg[k]).max()))
        assert masked_first_max(lg) == ref_ids[k] or gaps[k] < TIE_TOL
    print(f"[load] {form} -> {wdt} {path}: max logit error {err:.3e}", flush=True)
    assert err < 2e-3
    m.free()
