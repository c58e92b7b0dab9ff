#!/usr/bin/env python3
"""Writes the full-depth model fixtures: tests/golden/model/<config>.npz.

For every model configuration of the benchmark's workload list (GPT-2
small fp32 64+255, medium fp32 128+511, large fp32 and fp16-weight
256+511, XL fp16-weight 512+511: prompt tokens + decode forwards, EOS masked
on every step so the step count is fixed, stopping at 1024 positions), the
CPU oracle (oracle/g2_oracle.c: the reference kernels' arithmetic in their
accumulation order, composed as main.c prefill/decode/sample_next_token)
runs the greedy generation loop of main.c:2106-2150 on the synthetic
random-init weights (seed 0x67707432, matrices N(0, 0.02), LayerNorm gamma 1
beta 0, biases 0, tied lm_head; fp16 configurations use the fp16-rounded
values held as fp32, as the reference would see them) and a uniform-random
prompt.

Each fixture holds:
  prompt [P] int32, ids [n] int32 (the greedy tokens), top2 [n, 2] float32
  (chosen logit and runner-up after the EOS mask, per step),
  ck_steps [K] int32: checkpoint steps (0 = the prefill logits, k = the
    logits of decode forward k, at position P + k - 1),
  cols [K, C] int32 and vals [K, C] float32: at each checkpoint the 32
    largest logits and a fixed seeded sample of 2048 columns,
  meta: JSON with the configuration.

Usage: python tests/golden/make_model_fixtures.py [name ...]
(names: small medium large large16 xl; default all).  Takes a few minutes
per large configuration on an 8-core host; OMP_NUM_THREADS sets the oracle's
threads.
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "gpt2-opencl-1.1_amd"), ROOT]

SEED = 0x67707432
# name: (preset, fp16 weights, prompt tokens, decode forwards)
CONFIGS = {
    "small": ("small", False, 64, 255),
    "medium": ("medium", False, 128, 511),
    "large": ("large", False, 256, 511),
    "large16": ("large", True, 256, 511),
    "xl": ("xl", True, 512, 511),
}
N_CHECKPOINTS = 4
TOPK = 32
N_SAMPLE = 2048


def prompt_for(name, vocab):
    P = CONFIGS[name][2]
    return np.random.default_rng(SEED + 1000 + P).integers(0, vocab, P).astype(np.int32)


def checkpoints(n_dec):
    """Steps 0 (prefill), then decode forwards spread to the last one."""
    return sorted({0, max(1, n_dec // 3), max(1, 2 * n_dec // 3), n_dec})


def make(name):
    import g2hip
    from oracle import oracle

    preset, f16, P, n_dec = CONFIGS[name]
    cfg = g2hip.preset(preset)
    n_gen = n_dec + 1
    t0 = time.time()
    w = g2hip.synth_weights(cfg, SEED, f16_round=f16)
    om = oracle.Model(cfg, w, kslice=4)
    del w
    prompt = prompt_for(name, cfg.vocab_size)
    ids, top2, lg = om.generate(prompt, n_gen, min_new=n_gen, logit_steps=n_gen)
    om.close()
    assert len(ids) == n_gen, (name, len(ids))
    steps = checkpoints(n_dec)
    sample = np.sort(np.random.default_rng(SEED + 7).choice(cfg.vocab_size, N_SAMPLE, replace=False))
    cols, vals = [], []
    for k in steps:
        row = lg[k]
        top = np.argsort(-row, kind="stable")[:TOPK]
        c = np.concatenate([top, sample]).astype(np.int32)
        cols.append(c)
        vals.append(row[c].astype(np.float32))
    meta = {"name": name, "preset": preset, "n_layer": cfg.n_layer, "n_embd": cfg.n_embd, "n_head": cfg.n_head,
            "vocab_size": cfg.vocab_size, "ffn_dim": cfg.ffn_dim, "weights": "f16" if f16 else "f32",
            "seed": SEED, "prompt_len": P, "decode_forwards": n_dec, "kslice": 4,
            "oracle_threads": oracle.num_threads()}
    out = os.path.join(HERE, "model", f"{name}.npz")
    os.makedirs(os.path.dirname(out), exist_ok=True)
    np.savez_compressed(out, prompt=prompt, ids=ids.astype(np.int32), top2=top2.astype(np.float32),
                        ck_steps=np.array(steps, np.int32), cols=np.stack(cols), vals=np.stack(vals),
                        meta=np.array(json.dumps(meta)))
    gaps = top2[:, 0] - top2[:, 1]
    print(f"{name}: {n_gen} ids in {time.time() - t0:.0f}s, smallest top-2 gap {gaps.min():.3e} "
          f"(step {int(gaps.argmin())}) -> {out}", flush=True)


if __name__ == "__main__":
    for n in sys.argv[1:] or list(CONFIGS):
        make(n)
