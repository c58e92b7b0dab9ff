"""GPU parity of the persistent decode-step kernel (one launch per token
running every layer, the lm_head and the greedy pick).

The fused path decodes with them by default; these tests pin them against
the CPU oracle (greedy ids, teacher-forced per-step logits within 2e-3 for
both weight types, as for the other paths), against the per-operator
decode kernels of the same model, at GPT-2 XL width (n_embd 1600, 25 heads,
ffn 6400, vocab 50257) up to the last cache position, and for run-to-run
determinism (every reduction has a fixed order).
"""
import numpy as np
import pytest

from oracle import oracle
from parity import greedy_agree, random_prompt

pytestmark = pytest.mark.gpu

SEED = 0x67707432
def _check(got, ref):
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=2e-3)


def test_step_kernel_is_default(g2):
    for cfg in (g2.make_config(2, 128, 2, vocab_size=256), g2.preset("small"), g2.preset("xl")):
        m = g2.Model.synth(cfg, SEED, g2.F16, g2.PATH_FUSED)
        if not m.uses_step():
            m.set_step(True)  # raises with the reason
        assert m.uses_step(), f"E{cfg.n_embd}: the fused path should decode with the step kernel"
        print(f"[step] E{cfg.n_embd}: step kernel form {m.step_kind()}", flush=True)
        m.free()
    m = g2.Model.synth(g2.make_config(2, 128, 2, vocab_size=256), SEED, g2.F32, g2.PATH_REFERENCE)
    assert not m.uses_step()
    assert m.step_kernel() == ""
    with pytest.raises(g2.G2Error):
        m.set_step(True)
    m.free()


def test_step_kernel_names(g2):
    """The kernel a decode forward launches, as the library reports it
    (the name bench.py labels its roofline with and picks its traffic
    profile by): the tail form when every matrix row splits into segments
    of 193..208 16-byte chunks (GPT-2 XL: rows of n_embd 1600 or ffn 6400
    inputs split into segments of 200 chunks, in fp16 and in fp32), the
    plain form otherwise, none with the per-operator kernels.  The kernels
    of the benchmark configurations are compiled for their GPT-2 shapes
    (fp16 tail form for XL: g2k_step_f16_tail; plain form for small,
    medium and large in fp32 and large in fp16: g2k_step_<w>_e<n_embd>);
    other shapes (here XL width with a smaller vocabulary, and a small
    custom model) run the forms that read the shape from their arguments
    (g2k_step_f16_tailn, g2k_step_f32, g2k_step_f16)."""
    cases = [("xl", g2.F16, "g2k_step_f16_tail"), ("xl", g2.F32, "g2k_step_f32_tail"),
             ("large", g2.F16, "g2k_step_f16_e1280"), ("large", g2.F32, "g2k_step_f32_e1280"),
             ("small", g2.F32, "g2k_step_f32_e768"), ("medium", g2.F32, "g2k_step_f32_e1024"),
             ("small", g2.F16, "g2k_step_f16"),
             (g2.make_config(2, 1600, 25, vocab_size=4096), g2.F16, "g2k_step_f16_tailn"),
             (g2.make_config(2, 256, 4, vocab_size=1000), g2.F32, "g2k_step_f32"),
             (g2.make_config(2, 256, 4, vocab_size=1000), g2.F16, "g2k_step_f16")]
    for preset, dtype, name in cases:
        cfg = g2.preset(preset) if isinstance(preset, str) else preset
        m = g2.Model.synth(cfg, SEED, dtype, g2.PATH_FUSED)
        assert m.uses_step()
        assert m.step_kernel() == name, (preset, dtype, m.step_kernel())
        m.set_step(False)
        assert m.step_kernel() == ""
        m.free()


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_step_matches_operator_kernels(g2, dtype):
    """Same model, same prompt: the step kernel and the per-operator decode
    kernels give the same greedy ids and logits within the parity bound."""
    cfg = g2.preset("small")
    dt = g2.F16 if dtype == "f16" else g2.F32
    m = g2.Model.synth(cfg, SEED, dt, g2.PATH_FUSED)
    prompt = random_prompt(48, cfg.vocab_size, 11)
    print(f"[step] small {dtype}: step kernel vs operator kernels", flush=True)
    m.set_step(True)
    ids_s, _ = m.generate(prompt, 20)
    lg_s = m.logits()
    m.set_step(False)
    ids_k, _ = m.generate(prompt, 20)
    lg_k = m.logits()
    n = min(len(ids_s), len(ids_k))
    agree = int(np.argmax(ids_s[:n] != ids_k[:n])) if (ids_s[:n] != ids_k[:n]).any() else n
    if agree == n:
        _check(lg_s, lg_k)
    # the two may part only where the oracle sees a near tie
    w = g2.synth_weights(cfg, SEED, f16_round=dtype == "f16")
    om = oracle.Model(cfg, w)
    ref_ids, top2, _ = om.generate(prompt, 20)
    om.close()
    greedy_agree(ids_s, ref_ids, top2)
    greedy_agree(ids_k, ref_ids, top2)
    m.free()


def test_step_xl_width_to_end_of_context(g2):
    """Two layers at GPT-2 XL width (n_embd 1600, 25 heads, ffn 6400, vocab
    50257, fp16 weights): teacher-forced decode logits at positions
    1000..1022 (16 key chunks per head) against the oracle."""
    cfg = g2.make_config(2, 1600, 25, vocab_size=50257)
    assert cfg.ffn_dim == 6400
    w = g2.synth_weights(cfg, SEED, f16_round=True)
    om = oracle.Model(cfg, w, kslice=4)
    m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
    assert m.uses_step()
    P = 1000
    prompt = random_prompt(P, cfg.vocab_size, 77)
    print(f"[step] XL width L2, prompt {P}", flush=True)
    om.prefill(prompt)
    m.prefill(prompt)
    _check(m.logits(), om.logits())
    tok = om.greedy(prompt, False, 1.0)
    for k in range(1023 - P):
        pos = P + k
        om.decode(tok, pos)
        m.decode(tok, pos)
        _check(m.logits(), om.logits())
        tok = om.greedy([tok], False, 1.0)
    m.free()
    om.close()


def test_step_tail_form_other_shape(g2):
    """The tail form that reads the model shape from its arguments
    (g2k_step_f16_tailn: XL width, 4096-token vocabulary), two layers:
    prefill and teacher-forced decode logits at positions 300..315 against
    the oracle."""
    cfg = g2.make_config(2, 1600, 25, vocab_size=4096)
    w = g2.synth_weights(cfg, SEED, f16_round=True)
    om = oracle.Model(cfg, w, kslice=4)
    m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
    assert m.step_kernel() == "g2k_step_f16_tailn"
    P = 300
    prompt = random_prompt(P, cfg.vocab_size, 78)
    print(f"[step] tail form, vocab {cfg.vocab_size}, prompt {P}", flush=True)
    om.prefill(prompt)
    m.prefill(prompt)
    _check(m.logits(), om.logits())
    tok = om.greedy(prompt, False, 1.0)
    for k in range(16):
        om.decode(tok, P + k)
        m.decode(tok, P + k)
        _check(m.logits(), om.logits())
        tok = om.greedy([tok], False, 1.0)
    m.free()
    om.close()


def test_step_deterministic(g2):
    """Two identical runs produce bit-identical ids and logits."""
    cfg = g2.preset("small")
    m = g2.Model.synth(cfg, SEED, g2.F16, g2.PATH_FUSED)
    prompt = random_prompt(100, cfg.vocab_size, 5)
    outs = []
    for _ in range(2):
        ids, _ = m.generate(prompt, 64)
        outs.append((ids.copy(), m.logits().copy()))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    m.free()


def test_step_decode_run_matches_generate(g2):
    """decode_run (the bench's loop) continues a prefilled cache exactly as
    generate does."""
    cfg = g2.make_config(3, 256, 4, vocab_size=1000)
    m = g2.Model.synth(cfg, SEED, g2.F16, g2.PATH_FUSED)
    prompt = random_prompt(200, cfg.vocab_size, 8)
    ids, _ = m.generate(prompt, 40, min_new=40)
    run, _ = m.decode_run(int(ids[0]), len(prompt), 39)
    np.testing.assert_array_equal(run, ids[1:40])
    m.free()


@pytest.mark.parametrize("late", ["never", "0.5ms", "2ms"])
def test_step_plain_launch_not_resident_resumes(g2, monkeypatch, capfd, late):
    """The step kernel is launched plain (not cooperatively) and all its
    work-groups agree on one verdict, by compare-and-swap on a decision
    word, before their first lasting write: GO once one has seen every
    arrival word, ABORT once one has waited 1 ms.  Forced from the host
    (G2_STEP_TEST_WITHHOLD): work-group 1 never posts its arrival (every
    launch aborts), posts it 0.5 ms late (within the limit: no abort), or
    2 ms late (the others give up first; work-group 1 then finds ABORT
    stored).  After an abort nothing was written: the host resumes the run
    with cooperative launches.  In every mode generate, a second generate
    and a single decode give ids and logits bit-identical to cooperative
    launches only (G2_STEP_COOP=1) and to plain launches."""
    cfg = g2.make_config(3, 256, 4, vocab_size=1000)
    w = g2.synth_weights(cfg, SEED, f16_round=True)
    prompt = random_prompt(120, cfg.vocab_size, 31)
    mode = {"never": "1", "0.5ms": "2", "2ms": "3"}[late]
    outs = []
    for env in ({"G2_STEP_COOP": "1"}, {"G2_STEP_TEST_WITHHOLD": mode}, {}):
        for k in ("G2_STEP_COOP", "G2_STEP_TEST_WITHHOLD"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        print(f"[step] launch mode {env or 'plain'}", flush=True)
        run = []
        for _ in range(2):
            m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
            assert m.step_kind() == 1
            if not run:
                for _ in range(2):
                    ids, _ = m.generate(prompt, 30, min_new=30)
                    run += [ids.copy(), m.logits().copy()]
            else:
                m.prefill(prompt)
                m.decode(int(run[0][0]), len(prompt))
                run.append(m.logits().copy())
            m.free()
        err = capfd.readouterr().err
        resumed = err.count("resuming with cooperative launches")
        expect = 2 if ("G2_STEP_TEST_WITHHOLD" in env and late != "0.5ms") else 0
        assert resumed == expect, err
        outs.append(run)
    assert len(outs[0][0]) == 30
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            np.testing.assert_array_equal(a, b)
