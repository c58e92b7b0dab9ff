"""End-to-end GPU parity of the model paths against the CPU oracle.

Both execution paths (the reference operator sequence and the fused gfx950
path), fp32 and fp16 weights, on the same synthetic random-init weights and
random prompts.  Greedy ids must be identical (tests/parity.py allows a
parting only where the oracle's own top-2 gap is below 1e-4), and every
step teacher-forced along the oracle's ids must give the oracle's greedy
choice and logits within max-abs 2e-3 / rel 1e-3 of the oracle's, for
fp32 and fp16 weights alike (the oracle holds the same fp16-rounded
values).
"""
import numpy as np
import pytest

from oracle import oracle
from parity import TIE_TOL, greedy_agree, masked_first_max, random_prompt

pytestmark = pytest.mark.gpu

SEED = 0x67707432


def tiny_cfg(g2):
    return g2.make_config(2, 128, 2, vocab_size=256)


def check_logits(got, ref):
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=2e-3)


def run_parity(g2, cfg, path, dtype, P, n_new, seed=SEED, kslice=4):
    """Free-running greedy generation against the oracle's ids, then every
    step teacher-forced along the oracle's ids: logits within the parity
    bound and the greedy choice equal to the oracle's (near ties aside)."""
    f16 = dtype == g2.F16
    w = g2.synth_weights(cfg, seed, f16_round=f16)
    om = oracle.Model(cfg, w, kslice=kslice)
    prompt = random_prompt(P, cfg.vocab_size, seed + P)
    print(f"[model] L{cfg.n_layer} E{cfg.n_embd} V{cfg.vocab_size} path {path} dtype {dtype} P {P} new {n_new}",
          flush=True)
    ref_ids, top2, _ = om.generate(prompt, n_new, min_new=n_new)
    ref_lg = om.teacher_forced(prompt, ref_ids[:-1])
    gaps = top2[:, 0] - top2[:, 1]
    m = g2.Model.synth(cfg, seed, dtype, path)
    if path == g2.PATH_REFERENCE:
        m.set_kslice(kslice)
    ids, timing = m.generate(prompt, n_new, min_new=n_new)
    agree = greedy_agree(ids, ref_ids, top2)
    m.prefill(prompt)
    max_err = 0.0
    for k in range(len(ref_ids)):
        if k > 0:
            m.decode(int(ref_ids[k - 1]), P + k - 1)
        lg = m.logits()
        check_logits(lg, ref_lg[k])
        max_err = max(max_err, float(np.abs(lg - ref_lg[k]).max()))
        c = masked_first_max(lg)
        assert c == ref_ids[k] or gaps[k] < TIE_TOL, f"teacher-forced step {k}: {c} vs {ref_ids[k]}"
    print(f"[model] free-running ids agree for {agree} of {len(ref_ids)}; teacher-forced max logit error "
          f"{max_err:.3e}", flush=True)
    m.free()
    om.close()
    return ids, ref_ids, timing


@pytest.mark.parametrize("path", [0, 1], ids=["reference", "fused"])
def test_tiny_fp32(g2, path):
    ids, ref_ids, _ = run_parity(g2, tiny_cfg(g2), path, g2.F32, P=17, n_new=40)
    np.testing.assert_array_equal(ids, ref_ids)


def test_tiny_fp16_fused(g2):
    run_parity(g2, tiny_cfg(g2), g2.PATH_FUSED, g2.F16, P=17, n_new=40)


@pytest.mark.parametrize("path", [0, 1], ids=["reference", "fused"])
def test_small_fp32(g2, path):
    """GPT-2 small shape (12 layers, 768, 12 heads, vocab 50257); the full
    255-forward run is in test_full_depth_gpu.py."""
    run_parity(g2, g2.preset("small"), path, g2.F32, P=64, n_new=24)


def test_small_fp16_fused(g2):
    run_parity(g2, g2.preset("small"), g2.PATH_FUSED, g2.F16, P=64, n_new=24)


def test_prompt_edges(g2):
    """Prompt of 1 id, and a prompt filling the context (1023 ids: exactly
    one token, from the prefill logits, main.c:2126)."""
    cfg = tiny_cfg(g2)
    w = g2.synth_weights(cfg, SEED)
    om = oracle.Model(cfg, w)
    m = g2.Model.synth(cfg, SEED, g2.F32, g2.PATH_FUSED)
    for P, n_new in [(1, 5), (1023, 7), (1000, 30)]:
        prompt = random_prompt(P, cfg.vocab_size, P)
        ref_ids, top2, _ = om.generate(prompt, n_new)
        ids, _ = m.generate(prompt, n_new)
        assert len(ids) == min(n_new, 1024 - P)
        greedy_agree(ids, ref_ids, top2)


def test_eos_stop(g2):
    """With min_new < max_new the loop stops at EOS (main.c:2135).  A model
    whose lm_head row for EOS dominates makes EOS the greedy choice."""
    cfg = g2.make_config(1, 64, 1, vocab_size=50257)
    w = g2.synth_weights(cfg, 5)
    w["wte"] = w["wte"].copy()
    w["wte"][50256] *= 40.0
    om = oracle.Model(cfg, w)
    prompt = random_prompt(8, cfg.vocab_size, 3)
    ref_ids, top2, _ = om.generate(prompt, 20, min_new=3)
    m = g2.Model.from_host(cfg, w, g2.F32, g2.PATH_FUSED)
    ids, _ = m.generate(prompt, 20, min_new=3)
    np.testing.assert_array_equal(ids, ref_ids)
    assert ids[-1] == 50256 and len(ids) < 20


def test_host_sampler_rep_penalty(g2):
    """g2_sample_greedy with a repetition penalty matches the oracle's
    restatement of sample_next_token (main.c:1885-1903)."""
    cfg = tiny_cfg(g2)
    w = g2.synth_weights(cfg, SEED)
    om = oracle.Model(cfg, w)
    m = g2.Model.synth(cfg, SEED, g2.F32, g2.PATH_REFERENCE)
    prompt = random_prompt(30, cfg.vocab_size, 9)
    om.prefill(prompt)
    m.prefill(prompt)
    for rp in (1.0, 1.3, 3.0):
        assert m.sample_greedy(prompt, False, rp) == om.greedy(prompt, False, rp)


def test_prefill_matches_decode(g2):
    """Invariant: logits for position t from a prefill of t+1 ids equal those
    of a prefill of t ids followed by a decode of id t (fused path)."""
    cfg = g2.preset("small")
    m = g2.Model.synth(cfg, SEED, g2.F32, g2.PATH_FUSED)
    prompt = random_prompt(40, cfg.vocab_size, 1)
    m.prefill(prompt)
    a = m.logits()
    m.prefill(prompt[:-1])
    m.decode(prompt[-1], 39)
    b = m.logits()
    np.testing.assert_allclose(a, b, rtol=1e-3, atol=2e-3)
