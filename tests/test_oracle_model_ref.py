"""Pins the reference-order model of the oracle (qd_oracle_model_new_order
with QD_ORDER_REF), the host side of the comparison of the GPU's greedy stream
with the reference kernels' own arithmetic (framework_src/qwen_infer.cu:614-737).

  * argmax_kernel's tie order (kernels/argmax.cuh:7-72), from its code: the
    first maximum within a thread's chunk of ceil(V/512) ids; in each xor
    butterfly a lane keeps its own value on a tie, so lane 0 ends with the tied
    lane that comes first in the butterfly's bit-reversed order (lane 16
    before lane 1), and the same between warps; NaN never wins; numpy's
    argmax when the maximum is unique;
  * SwiGLU as swiglu.cuh:11-13 computes it (w1 * (w2 / (1 + exp(-w2))), fp32):
    within one fp16 ulp of float64 and equal to numpy's fp32 form;
  * the model's wiring: one step equals the composition of the separately
    pinned reference-order pieces (rmsnorm and gemv with ORDER_REF, the QKV
    bias/RoPE/cache op, the engine's attention dispatch, the add_bias residual
    kernel) bit for bit, and it tracks the textbook float64 forward as the
    gfx950-order model does.
"""
import numpy as np

import qdiy
from common import model_logits_fp64, model_tensors, normal_f16, ulp16
from oracle import oracle

V = 151936
CHUNK = -(-V // 512)            # ids per argmax thread


def _logits(fill=-1.0):
    return np.full(V, fill, np.float16)


def test_argmax_ref_unique_maximum_is_numpy_argmax():
    rng = np.random.default_rng(4)
    for _ in range(5):
        lg = normal_f16(rng, V, 3.0)
        top = np.flatnonzero(lg == lg.max())
        if top.size == 1:
            assert oracle.argmax_ref(lg) == int(top[0])
    lg = _logits()
    lg[151935] = 2.0
    assert oracle.argmax_ref(lg) == 151935


def test_argmax_ref_tie_order_of_the_reference_kernel():
    lg = _logits()
    lg[[5, 7]] = 1.0                                   # one thread's chunk: first one
    assert oracle.argmax_ref(lg) == 5
    lg = _logits()
    a, b = 1 * CHUNK + 3, 16 * CHUNK + 1               # threads 1 and 16 of warp 0
    lg[[a, b]] = 1.0
    assert oracle.argmax_ref(lg) == b                  # lane 16 before lane 1
    lg = _logits()
    a, b = 32 * CHUNK, 64 * CHUNK                      # lane 0 of warps 1 and 2
    lg[[a, b]] = 1.0
    assert oracle.argmax_ref(lg) == b                  # warp 2 before warp 1
    lg = _logits()
    lg[[0, 16 * CHUNK]] = 1.0                          # thread 0 keeps its own
    assert oracle.argmax_ref(lg) == 0


def test_argmax_ref_nan_and_infinities():
    lg = _logits()
    lg[3] = np.nan
    lg[9] = 0.5
    assert oracle.argmax_ref(lg) == 9
    lg = np.full(V, -np.inf, np.float16)
    assert oracle.argmax_ref(lg) == -1                 # nothing exceeds the initial -inf
    lg[100] = np.inf
    assert oracle.argmax_ref(lg) == 100


def test_swiglu_ref_against_fp64_and_fp32_form():
    rng = np.random.default_rng(6)
    g = normal_f16(rng, 20000, 2.0)
    u = normal_f16(rng, 20000, 3.0)
    got = np.array([oracle.swiglu_ref(a, b) for a, b in zip(g, u)], np.float16)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    exact = gd * ud / (1.0 + np.exp(-ud))
    assert np.all(np.abs(got.astype(np.float64) - exact) <= ulp16(exact))
    g32, u32 = g.astype(np.float32), u.astype(np.float32)
    ref = (g32 * (u32 / (np.float32(1) + np.exp(-u32)))).astype(np.float16)
    assert np.mean(got.view(np.uint16) == ref.view(np.uint16)) > 0.999
    assert oracle.swiglu_ref(3.0, 0.0) == 0.0
    assert oracle.swiglu_ref(2.0, 30.0) == np.float16(60.0)        # silu(u) = u for large u
    assert abs(float(oracle.swiglu_ref(2.0, -30.0))) < 1e-9


TINY = dict(vocab_size=1000, hidden_size=512, num_layers=2, num_heads=4, intermediate_size=1368,
            max_seqlen=64)


def _step_from_pieces(m, kc, vc, token, pos):
    """One decode step of qwen_infer.cu:614-737 assembled from the pinned
    reference-order pieces; kc/vc [layers][max_seqlen * H] are updated."""
    c = m["cfg"]
    H, NH, I = c["hidden"], c["heads"], c["inter"]
    x = m["wte"][token].copy()
    for li, L in enumerate(m["layers"]):
        xn = oracle.rmsnorm(x, L["ln_1"], 1e-6, oracle.ORDER_REF)
        qkv = oracle.gemv(xn, L["qkv_w"], 3 * H, H, 0, oracle.ORDER_REF)
        oracle.qkv_bias_rope_cache(qkv, L["qkv_b"], kc[li], vc[li], pos, NH, 128, H, 128)
        attn = oracle.decode_attention(qkv[:H].reshape(NH, 128), kc[li], vc[li], pos + 1, NH, H, 128,
                                       oracle.ENGINE).reshape(-1)
        proj = oracle.gemv(attn, L["proj_w"], H, H, 0, oracle.ORDER_REF)
        x = (x.astype(np.float32) + proj.astype(np.float32)).astype(np.float16)    # bias.cuh:9
        xn = oracle.rmsnorm(x, L["ln_2"], 1e-6, oracle.ORDER_REF)
        g = oracle.gemv(xn, L["w1"], I, H, 0, oracle.ORDER_REF)
        u = oracle.gemv(xn, L["w2"], I, H, 0, oracle.ORDER_REF)
        act = np.array([oracle.swiglu_ref(a, b) for a, b in zip(g, u)], np.float16)
        down = oracle.gemv(act, L["w_down"], H, I, 0, oracle.ORDER_REF)
        x = (x.astype(np.float32) + down.astype(np.float32)).astype(np.float16)
    xn = oracle.rmsnorm(x, m["ln_f"], 1e-6, oracle.ORDER_REF)
    logits = oracle.gemv(xn, m["lm_head"], c["vocab"], H, 0, oracle.ORDER_REF)
    return oracle.argmax_ref(logits), logits


def test_reference_order_model_is_its_pieces_composed():
    img = qdiy.random_model_image(qdiy.model_cfg(**TINY), 7, 0.05)
    m = model_tensors(img)
    H, NL = m["cfg"]["hidden"], m["cfg"]["layers"]
    kc = np.zeros((NL, 64 * H), np.float16)
    vc = np.zeros((NL, 64 * H), np.float16)
    model = oracle.Model(img, 64, nthreads=4, order=oracle.ORDER_REF)
    try:
        tokens = [11, 250, 999, 3, 42, 7, 600]
        for pos, tok in enumerate(tokens):
            want_t, want_l = _step_from_pieces(m, kc, vc, tok, pos)
            got_t, got_l = model.forward(tok, pos)
            assert got_t == want_t, pos
            assert np.array_equal(got_l.view(np.uint16), want_l.view(np.uint16)), pos
    finally:
        model.close()


def test_reference_order_model_tracks_fp64():
    img = qdiy.random_model_image(qdiy.model_cfg(**TINY), 7, 0.05)
    m = model_tensors(img)
    hist = [11, 250, 999, 3, 42, 5, 6, 7, 8, 9]
    model = oracle.Model(img, 64, nthreads=4, order=oracle.ORDER_REF)
    try:
        for pos, tok in enumerate(hist[:-1]):
            model.forward(tok, pos, want_logits=False)
        _, logits = model.forward(hist[-1], len(hist) - 1)
    finally:
        model.close()
    ref = model_logits_fp64(m, hist)
    scale = np.max(np.abs(ref))
    assert np.max(np.abs(logits.astype(np.float64) - ref)) <= 0.02 * scale
