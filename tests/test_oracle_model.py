"""Pins of the oracle's model composition (CPU only).

The oracle restates prefill()/decode()/sample_next_token (main.c:1739-1904).
Its composition is pinned against an independent implementation of the same
network -- transformers' GPT2LMHeadModel with gelu_new, eps 1e-5, tied
lm_head, loaded with the same weights from memory (no download) -- and by
invariants: split-K slice count independence, prefill/decode agreement,
first-max greedy semantics and the EOS mask.
"""
import numpy as np
import pytest

import g2hip
from oracle import oracle
from parity import random_prompt


NAMES = ["ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias", "attn.c_proj.weight",
         "attn.c_proj.bias", "ln_2.weight", "ln_2.bias", "mlp.c_fc.weight", "mlp.c_fc.bias",
         "mlp.c_proj.weight", "mlp.c_proj.bias"]



def _torch():
    """torch, imported only inside the CPU tests that use it: a GPU test
    session then never loads torch's bundled HIP runtime beside the one
    libg2hip is linked against (two HIP runtimes in one process)."""
    import torch

    return torch

def hf_model(cfg, w):
    transformers = pytest.importorskip("transformers")
    torch = _torch()
    tied = w.get("lm_head") is None
    hc = transformers.GPT2Config(vocab_size=cfg.vocab_size, n_positions=1024, n_embd=cfg.n_embd,
                                 n_layer=cfg.n_layer, n_head=cfg.n_head, n_inner=cfg.ffn_dim,
                                 activation_function="gelu_new", resid_pdrop=0.0, embd_pdrop=0.0,
                                 attn_pdrop=0.0, layer_norm_epsilon=1e-5, bos_token_id=0, eos_token_id=0,
                                 tie_word_embeddings=tied)
    m = transformers.GPT2LMHeadModel(hc).eval().double()
    sd = {"transformer.wte.weight": w["wte"], "transformer.wpe.weight": w["wpe"],
          "transformer.ln_f.weight": w["lnf_w"], "transformer.ln_f.bias": w["lnf_b"],
          "lm_head.weight": w["wte"] if tied else w["lm_head"]}
    for l, lw in enumerate(w["layers"]):
        for n, a in zip(NAMES, lw):
            sd[f"transformer.h.{l}.{n}"] = a
    m.load_state_dict({k: torch.tensor(np.asarray(v, np.float64)) for k, v in sd.items()}, strict=False)
    return m


def eos_dominant(w, E):
    """Weights whose EOS logit wins every step: ln_f beta = 10 e_0 and the
    EOS row of wte = 10 e_0 add 100 to the EOS logit, while the normalised
    hidden state moves it by at most 10*|h_0| and other logits stay O(1).
    The prompt never holds EOS, so the embedding lookup is unaffected."""
    w2 = dict(w)
    w2["wte"] = w["wte"].copy()
    w2["wte"][50256] = 0.0
    w2["wte"][50256, 0] = 10.0
    w2["lnf_b"] = np.zeros(E, np.float32)
    w2["lnf_b"][0] = 10.0
    return w2


def hf_logits(m, ids):
    torch = _torch()
    with torch.no_grad():
        return m(torch.tensor(np.asarray(ids, np.int64)[None])).logits[0].numpy()


@pytest.mark.parametrize("affine", [False, True], ids=["plain", "affine"])
@pytest.mark.parametrize("L,E,H,V", [(2, 128, 2, 256), (3, 192, 3, 1000)])
def test_prefill_decode_vs_transformers(L, E, H, V, affine):
    """affine: every bias and LayerNorm gamma/beta random (ln_1, ln_2, ln_f,
    c_attn, attn.c_proj, c_fc, mlp.c_proj: main.c:1752-1828 order), so each
    parameter's slot in the composition is pinned against transformers."""
    cfg = g2hip.make_config(L, E, H, vocab_size=V)
    w = g2hip.synth_weights(cfg, 11, affine=affine)
    om = oracle.Model(cfg, w)
    hf = hf_model(cfg, w)
    prompt = random_prompt(21, V, 2)
    om.prefill(prompt)
    ref = hf_logits(hf, prompt)
    np.testing.assert_allclose(om.logits(), ref[-1], rtol=1e-5, atol=2e-6)
    ids = list(prompt)
    for k in range(6):  # decode continues from the cache
        tok = (7 * k + 3) % V
        om.decode(tok, len(ids))
        ids.append(tok)
        np.testing.assert_allclose(om.logits(), hf_logits(hf, ids)[-1], rtol=1e-5, atol=2e-6)


def test_separate_lm_head_vs_transformers():
    """A file with its own lm_head.weight (main.c:1374-1405): the oracle's
    head replaces the tied wte; pinned against an untied transformers model."""
    cfg = g2hip.make_config(2, 128, 2, vocab_size=256)
    w = g2hip.synth_weights(cfg, 21, affine=True)
    w["lm_head"] = (np.random.default_rng(4).standard_normal((256, 128)) * 0.02).astype(np.float32)
    om = oracle.Model(cfg, w)
    hf = hf_model(cfg, w)
    assert hf.lm_head.weight.data_ptr() != hf.transformer.wte.weight.data_ptr()
    prompt = random_prompt(15, 256, 8)
    om.prefill(prompt)
    np.testing.assert_allclose(om.logits(), hf_logits(hf, prompt)[-1], rtol=1e-5, atol=2e-6)
    w_tied = dict(w)
    w_tied["lm_head"] = None
    om2 = oracle.Model(cfg, w_tied)
    om2.prefill(prompt)
    assert np.abs(om2.logits() - om.logits()).max() > 1e-2  # the separate head is really used


@pytest.mark.parametrize("affine", [False, True], ids=["plain", "affine"])
def test_generate_vs_transformers_greedy(affine):
    cfg = g2hip.make_config(2, 128, 2, vocab_size=512)
    w = g2hip.synth_weights(cfg, 12, affine=affine)
    om = oracle.Model(cfg, w)
    hf = hf_model(cfg, w)
    prompt = random_prompt(9, 512, 3)
    ids, top2, _ = om.generate(prompt, 12)
    seq = list(prompt)
    for k in range(12):
        lg = hf_logits(hf, seq)[-1]
        nxt = int(np.argmax(lg))
        assert ids[k] == nxt, f"step {k}"
        seq.append(nxt)


def test_kslice_independence_and_decode_consistency():
    """attn_proj/ffn2 split-K result is slice-count independent up to
    rounding, and prefill of t+1 ids matches prefill of t plus decode."""
    cfg = g2hip.make_config(2, 128, 2, vocab_size=300)
    w = g2hip.synth_weights(cfg, 13)
    prompt = random_prompt(30, 300, 4)
    outs = []
    for ks in (1, 2, 4, 8):
        om = oracle.Model(cfg, w, kslice=ks)
        om.prefill(prompt[:-1])
        om.decode(prompt[-1], len(prompt) - 1)
        outs.append(om.logits())
    for o in outs[1:]:
        np.testing.assert_allclose(o, outs[0], rtol=1e-5, atol=1e-6)
    om = oracle.Model(cfg, w)
    om.prefill(prompt)
    np.testing.assert_allclose(om.logits(), outs[0], rtol=1e-5, atol=1e-6)


def test_greedy_first_max_and_eos_mask():
    cfg = g2hip.make_config(1, 64, 1, vocab_size=50257)
    w = g2hip.synth_weights(cfg, 14)
    om = oracle.Model(cfg, w)
    om.prefill(np.array([1, 2, 3], np.int32))
    lg = om.logits()
    assert om.greedy([1, 2, 3]) == int(np.argmax(lg))  # np.argmax is first-max too
    w2 = eos_dominant(w, cfg.n_embd)
    om2 = oracle.Model(cfg, w2)
    om2.prefill(np.array([1, 2, 3], np.int32))
    assert om2.greedy([1, 2, 3]) == 50256
    masked = om2.greedy([1, 2, 3], forbid_eos=True)
    lg2 = om2.logits()
    lg2[50256] = -np.inf
    assert masked == int(np.argmax(lg2))


def test_rep_penalty_semantics():
    """main.c:1885-1896: distinct context ids, positive logits divided,
    negative multiplied, then argmax."""
    cfg = g2hip.make_config(1, 64, 1, vocab_size=100)
    w = g2hip.synth_weights(cfg, 15)
    om = oracle.Model(cfg, w)
    ctx = np.array([5, 9, 5, 40, 9, 77], np.int32)
    om.prefill(ctx)
    lg = om.logits().astype(np.float32)
    for pen in (1.0, 1.5, 4.0):
        adj = lg.copy()
        if pen > 1.0:
            for t in dict.fromkeys(ctx.tolist()):
                adj[t] = np.float32(adj[t] / np.float32(pen)) if adj[t] > 0 else np.float32(adj[t] * np.float32(pen))
        assert om.greedy(ctx, rep_penalty=pen) == int(np.argmax(adj))


def test_generation_protocol_lengths():
    """main.c:2106-2150: 1 token from prefill, decode until max tokens or
    1024 positions; EOS masked while fewer than min tokens exist."""
    cfg = g2hip.make_config(1, 64, 1, vocab_size=128)
    w = g2hip.synth_weights(cfg, 16)
    om = oracle.Model(cfg, w)
    ids, top2, _ = om.generate(random_prompt(1000, 128, 1), 50)
    assert len(ids) == 24  # 1024 - 1000 positions
    ids, _, _ = om.generate(random_prompt(1023, 128, 1), 5)
    assert len(ids) == 1
    ids, top2, _ = om.generate(random_prompt(10, 128, 2), 7)
    assert len(ids) == 7 and np.all(top2[:, 0] >= top2[:, 1])


SWAPS = [("ln1_b", "proj_b"), ("proj_b", "fc2_b"), ("ln1_w", "ln2_w"), ("ln1_b", "ln2_b"), ("ln2_b", "fc2_b")]


@pytest.mark.parametrize("a,b", SWAPS, ids=[f"{a}-{b}" for a, b in SWAPS])
def test_planted_slot_swap_fails_the_pin(a, b):
    """A mistake planted in the oracle's input: two same-sized parameter
    slots exchanged in one layer.  The transformers pin above must reject it
    (its tolerance is 1e-5), and so must the GPU model tests that use the
    same affine weights, whose logits tolerance is 2e-3: every planted swap
    moves some logit by more than that, at the first and the last layer."""
    cfg = g2hip.make_config(3, 192, 3, vocab_size=1000)
    w = g2hip.synth_weights(cfg, 11, affine=True)
    prompt = random_prompt(21, cfg.vocab_size, 2)
    hf = hf_model(cfg, w)
    ref = hf_logits(hf, prompt)[-1]
    for layer in (0, cfg.n_layer - 1):
        om = oracle.Model(cfg, g2hip.swap_slots(w, a, b, layer))
        om.prefill(prompt)
        d = float(np.abs(om.logits() - ref).max())
        om.close()
        assert d > 2e-3, f"swap {a}<->{b} in layer {layer} moved the logits by only {d:.2e}"
        with pytest.raises(AssertionError):
            np.testing.assert_allclose(om_logits_of(cfg, g2hip.swap_slots(w, a, b, layer), prompt), ref,
                                       rtol=1e-5, atol=2e-6)


def om_logits_of(cfg, w, prompt):
    om = oracle.Model(cfg, w)
    om.prefill(prompt)
    out = om.logits()
    om.close()
    return out
