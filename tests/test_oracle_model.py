"""Pins the oracle's decode-step ops and whole-model generation
(oracle/qd_oracle_model.c), the host side of the config-5 token-identity
check.

  * the fast GEMV rows equal the pinned qd_oracle_gemv (QD_ORDER_WAVE64) bit
    for bit, including a masked tail (K = 5504 = 10.75 x 512);
  * proj_residual, ffn_up_swiglu and lm_head_argmax equal their compositions
    of pinned pieces (rmsnorm, gemv, f2h) bit for bit;
  * SwiGLU is within one fp16 ulp of float64 w1 * silu(w2) and of the
    reference's expf form (swiglu.cuh:6-15);
  * argmax: lowest index on exact ties, -0 == +0, NaN never wins, and equal to
    numpy's first-maximum argmax otherwise;
  * the whole model: the last step's logits track an independent textbook
    float64 forward (tests/common.py) to within fp16 activation rounding, while
    planted mistakes (RoPE sign, gate/up swap) miss it by far more.
"""
import numpy as np
import pytest

import qdiy
from common import model_logits_fp64, model_tensors, normal_f16, ulp16
from oracle import oracle


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint16), np.asarray(b).view(np.uint16))


@pytest.mark.parametrize("K", [512, 2048, 5504, 72])
def test_proj_residual_is_gemv_then_residual(K):
    rng = np.random.default_rng(K)
    N = 96
    x = normal_f16(rng, K)
    W = normal_f16(rng, (N, K), 0.02)
    res = normal_f16(rng, N)
    got = oracle.proj_residual(x, W, res, N, K)
    y = oracle.gemv(x, W, N, K, 0, oracle.ORDER_WAVE64)
    want = (res.astype(np.float32) + y.astype(np.float32)).astype(np.float16)
    assert _same(got, want)


def test_swiglu_against_fp64_and_reference_form():
    rng = np.random.default_rng(1)
    g = normal_f16(rng, 20000, 2.0)
    u = normal_f16(rng, 20000, 3.0)
    got = np.array([oracle.swiglu(a, b) for a, b in zip(g, u)], np.float16).astype(np.float64)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    exact = gd * ud / (1.0 + np.exp(-ud))
    assert np.all(np.abs(got - exact) <= ulp16(exact))
    # the reference's form in fp32 with expf: w1 * (w2 / (1 + expf(-w2)))
    g32, u32 = g.astype(np.float32), u.astype(np.float32)
    ref = (g32 * (u32 / (np.float32(1) + np.exp(-u32)))).astype(np.float16).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp16(ref))
    assert np.mean(got == ref) > 0.98


def test_ffn_up_is_norm_gemvs_swiglu():
    rng = np.random.default_rng(2)
    H, I = 1024, 264
    x, nw = normal_f16(rng, H), normal_f16(rng, H)
    W1, W2 = normal_f16(rng, (I, H), 0.03), normal_f16(rng, (I, H), 0.03)
    got = oracle.ffn_up_swiglu(x, nw, W1, W2, H, I)
    xn = oracle.rmsnorm(x, nw, 1e-6, oracle.ORDER_WAVE64)
    g = oracle.gemv(xn, W1, I, H, 0, oracle.ORDER_WAVE64)
    u = oracle.gemv(xn, W2, I, H, 0, oracle.ORDER_WAVE64)
    want = np.array([oracle.swiglu(a, b) for a, b in zip(g, u)], np.float16)
    assert _same(got, want)


def test_lm_head_logits_and_argmax():
    rng = np.random.default_rng(3)
    H, V = 512, 3001
    x, nw = normal_f16(rng, H), normal_f16(rng, H)
    W = normal_f16(rng, (V, H), 0.05)
    tok, logits = oracle.lm_head_argmax(x, nw, W, V, H)
    xn = oracle.rmsnorm(x, nw, 1e-6, oracle.ORDER_WAVE64)
    assert _same(logits, oracle.gemv(xn, W, V, H, 0, oracle.ORDER_WAVE64))
    assert tok == int(np.argmax(logits.astype(np.float32)))


def test_argmax_ties_signed_zero_and_nan():
    H, V = 512, 64
    x = np.ones(H, np.float16)
    nw = np.ones(H, np.float16)
    W = np.zeros((V, H), np.float16)
    W[[7, 30, 41], 0] = 1.0                 # three equal maxima: lowest index wins
    assert oracle.lm_head_argmax(x, nw, W, V, H)[0] == 7
    W = np.zeros((V, H), np.float16)
    W[:, 0] = -1.0
    W[12, 0] = -0.0                         # -0 (row 12) ties +0 (rows 20, 21): lowest index
    W[20, 0] = 0.0
    W[21, 0] = 0.0
    assert oracle.lm_head_argmax(x, nw, W, V, H)[0] == 12
    W = np.zeros((V, H), np.float16)
    W[:, 0] = -2.0
    W[5, 0], W[5, 1] = np.inf, -np.inf      # inf + (-inf): a NaN logit never wins
    W[9, 0] = 1.0
    tok, logits = oracle.lm_head_argmax(x, nw, W, V, H)
    assert np.isnan(logits[5]) and tok == 9


TINY = dict(vocab_size=1000, hidden_size=512, num_layers=2, num_heads=4, intermediate_size=1368,
            max_seqlen=64)


def _tiny_image(seed=7, std=0.05):
    return qdiy.random_model_image(qdiy.model_cfg(**TINY), seed, std)


def test_random_image_format():
    cfg = qdiy.model_cfg(**TINY)
    img = _tiny_image()
    assert img.size == qdiy.model_image_bytes(cfg)
    m = model_tensors(img)
    assert m["cfg"] == dict(vocab=1000, hidden=512, layers=2, heads=4, inter=1368, max_seqlen=64)
    for L in m["layers"]:
        assert np.all(L["ln_1"] == 1.0) and np.all(L["ln_2"] == 1.0)
    assert np.all(m["ln_f"] == 1.0)
    w = m["layers"][1]["w1"].astype(np.float64)
    assert abs(w.mean()) < 1e-3 and abs(w.std() - 0.05) < 1e-3
    assert np.array_equal(img, _tiny_image())              # deterministic
    assert not np.array_equal(img, _tiny_image(seed=8))
    assert np.array_equal(img, qdiy.random_model_image(cfg, 7, 0.05, nthreads=1))


def test_generate_tracks_fp64_model_and_mistakes_do_not():
    img = _tiny_image()
    m = model_tensors(img)
    prompt = [11, 250, 999, 3, 42]
    plans = [oracle.split_plan(L, 3) if L >= 3 else oracle.fused_plan(L) for L in range(1, 65)]
    toks, logits = oracle.generate(img, prompt, 6, plans)
    assert len(toks) == 6
    hist = prompt + toks[:-1]                                # inputs of the 10 steps
    ref = model_logits_fp64(m, hist)
    scale = np.max(np.abs(ref))
    err = np.max(np.abs(logits.astype(np.float64) - ref))
    assert err <= 0.02 * scale, (err, scale)
    assert toks[-1] == int(np.argmax(logits.astype(np.float32)))
    for bad in ("rope_sign", "swap_gate_up"):
        wrong = model_logits_fp64(m, hist, mutate=bad)
        assert np.max(np.abs(wrong - ref)) > 10 * 0.02 * scale, bad


def test_generate_prompt_split_and_plans_do_not_change_tokens():
    """Steps after a prompt equal steps fed the same tokens one by one, and the
    thread count changes nothing."""
    img = _tiny_image(seed=9)
    plans = [oracle.fused_plan(L) for L in range(1, 65)]
    a, la = oracle.generate(img, [5, 6, 7], 5, plans, nthreads=1)
    b, lb = oracle.generate(img, [5, 6, 7], 5, plans, nthreads=8)
    assert a == b and _same(la, lb)
    c, lc = oracle.generate(img, [5, 6, 7] + a[:2], 3, plans)
    assert c == a[2:] and _same(lc, la)
