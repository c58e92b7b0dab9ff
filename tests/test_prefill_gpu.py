"""GPU parity of the fused prefill with fp16 weights, whose matmuls run on
the fp16 matrix cores with the fp32 activations split into two fp16 halves
(g2k_hgemm_*): last-position logits against the CPU oracle (1e-4: the
oracle runs in fp32 on the same fp16-rounded weights) and against the
fp32-MFMA GEMM of the same library (G2_PREFILL_F32MFMA=1), which the split
must match to fp32-level accumulation differences, at GPT-2 XL width and
for ragged prompt lengths (not multiples of the 64-row tile) up to the
1023-position limit.  The lengths cover the 64x64 GEMM (P <= 64), the
128x128 GEMM with qkv and fc as K slices (100: 6 and 5 slices; 200, 256:
3 and 2) and run whole (1023 rows), with proj and fc2 as 2 to 8 slices
summed with the following LayerNorm.
"""
import numpy as np
import pytest

from oracle import oracle
from parity import TIE_TOL, random_prompt

pytestmark = pytest.mark.gpu

SEED = 0x67707432


@pytest.mark.parametrize("P", [1, 37, 64, 100, 200, 256, 1023])
def test_prefill_split_fp16_mfma(g2, monkeypatch, P):
    cfg = g2.make_config(2, 1600, 25, vocab_size=50257)
    w = g2.synth_weights(cfg, SEED, f16_round=True)
    prompt = random_prompt(P, cfg.vocab_size, 100 + P)
    print(f"[prefill] XL width L2, P {P}", flush=True)
    monkeypatch.delenv("G2_PREFILL_F32MFMA", raising=False)
    m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
    m.prefill(prompt)
    lg_h = m.logits().copy()
    m.free()
    monkeypatch.setenv("G2_PREFILL_F32MFMA", "1")
    m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
    m.prefill(prompt)
    lg_f = m.logits().copy()
    m.free()
    om = oracle.Model(cfg, w, kslice=4)
    om.prefill(prompt)
    ref = om.logits()
    om.close()
    np.testing.assert_allclose(lg_h, ref, rtol=0, atol=1e-4)
    np.testing.assert_allclose(lg_h, lg_f, rtol=1e-3, atol=2e-3)
    top2 = np.sort(ref)[-2:]
    assert int(np.argmax(lg_h)) == int(np.argmax(ref)) or top2[1] - top2[0] < TIE_TOL, \
        f"P {P}: gpu argmax {int(np.argmax(lg_h))}, oracle {int(np.argmax(ref))}, oracle top-2 gap {top2[1] - top2[0]:.3e}"


@pytest.mark.parametrize("P", [65, 200, 512, 1023])
def test_prefill_gemm_tiles_agree(g2, monkeypatch, P):
    """Prompts of more than 64 rows run the 128x128-tile GEMM (operands
    staged through LDS by asynchronous loads, activations split into their
    fp16 halves by the kernels that produce them); it sums every output in
    the order of the 64x64-tile GEMM (G2_PREFILL_GEMM64=1), which splits
    the stored fp32 activations itself.  The logits agree to fp32 rounding
    (1e-5; 2.4e-6 to 3.2e-6 measured at P 65 to 1023: the two forms split K
    into different slices and sum them in different kernels)."""
    cfg = g2.make_config(2, 1600, 25, vocab_size=50257)
    w = g2.synth_weights(cfg, SEED, f16_round=True)
    prompt = random_prompt(P, cfg.vocab_size, 200 + P)
    print(f"[prefill] XL width L2, P {P}: 128x128 vs 64x64 tiles", flush=True)
    out = []
    for v in ("0", "1"):
        monkeypatch.setenv("G2_PREFILL_GEMM64", v)
        m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
        m.prefill(prompt)
        out.append(m.logits().copy())
        m.free()
    np.testing.assert_allclose(out[0], out[1], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("P", [1, 63, 64, 65, 200, 512, 1023])
def test_prefill_attention_h16_matches_f32(g2, monkeypatch, P):
    """The prompt attention on the fp16 matrix cores (operands split into
    fp16 halves, three products per pair) against the same attention on the
    fp32 matrix cores (G2_PREFILL_ATTN32=1): the logits agree to fp32
    rounding of the attention output (1e-4); both runs are checked against
    the oracle elsewhere."""
    cfg = g2.make_config(2, 1600, 25, vocab_size=50257)
    w = g2.synth_weights(cfg, SEED, f16_round=True)
    prompt = random_prompt(P, cfg.vocab_size, 300 + P)
    print(f"[prefill] XL width L2, P {P}: attention fp16-split vs fp32 matrix cores", flush=True)
    out = []
    for v in ("0", "1"):
        monkeypatch.setenv("G2_PREFILL_ATTN32", v)
        m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
        m.prefill(prompt)
        out.append(m.logits().copy())
        m.free()
    np.testing.assert_allclose(out[0], out[1], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("E,NH,P", [(1600, 25, 300), (1600, 25, 512), (768, 12, 700), (1280, 20, 640)])
def test_prefill_attention_helpers(g2, monkeypatch, E, NH, P):
    """The prompt attention with the grid's idle work-groups computing the
    first key blocks of the longest query blocks (g2a_help_plan: 25 helpers
    at 300 rows and 50 at 512 for 25 heads, 12 at 700 rows for 12 heads,
    40 at 640 rows for 20 heads),
    their softmax partials merged by the blocks' own work-groups, against
    the same attention without helpers (G2_PREFILL_ATTN_HELP=0): the logits
    agree to fp32 rounding of the split softmax (1e-5).  A second prompt on
    the same model must give exactly what a fresh model gives (every helper
    slot was left empty by the first).  Both runs are checked against the
    oracle elsewhere (full depth at 512 rows)."""
    cfg = g2.make_config(2, E, NH, vocab_size=50257)
    w = g2.synth_weights(cfg, SEED, f16_round=True)
    prompt = random_prompt(P, cfg.vocab_size, 800 + P)
    prompt2 = random_prompt(P, cfg.vocab_size, 900 + P)
    print(f"[prefill] E {E} NH {NH} L2, P {P}: attention helpers vs none", flush=True)
    monkeypatch.setenv("G2_PREFILL_ATTN_HELP", "0")
    m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
    m.prefill(prompt)
    lg_n = m.logits().copy()
    m.free()
    monkeypatch.setenv("G2_PREFILL_ATTN_HELP", "1")
    m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
    m.prefill(prompt)
    lg_h = m.logits().copy()
    m.prefill(prompt2)
    lg_h2 = m.logits().copy()
    m.free()
    m = g2.Model.from_host(cfg, w, g2.F16, g2.PATH_FUSED)
    m.prefill(prompt2)
    lg_f2 = m.logits().copy()
    m.free()
    np.testing.assert_allclose(lg_h, lg_n, rtol=1e-5, atol=1e-5)
    assert np.array_equal(lg_h2, lg_f2), "second prompt differs from a fresh model's"
