"""Pins the oracle's adjacent decode-step ops: RMSNorm (rmsnorm.cuh:6-57),
GEMV (hgemm_final.cuh:274-295) in both layouts, their two reduction orders, and
the fused attention front end (qwen_infer.cu:626-642).

  * the wave64 tree is pinned by inputs on which different summation trees give
    different fp32 results, with the expected value derived by hand;
  * the reference's sequential-k GEMV is pinned bit-exactly by numpy's
    sequential float32 cumulative sum (an independent implementation);
  * every order lands within fp32 accumulation + fp16 rounding of float64;
  * closed forms: constant x normalises to sign(x)*w; one-hot x picks a column.
"""
import numpy as np
import pytest

from common import normal_f16, ulp16
from oracle import oracle


def test_wave64_tree_structure():
    big = np.float32(2.0 ** 24)
    lanes = np.zeros(64, np.float32)
    lanes[0:4] = [big, 1.0, 1.0, -big]
    # ((2^24 + 1) + (1 - 2^24)) = 2^24 + (-(2^24 - 1)) = 1 in fp32 (2^24+1 rounds to 2^24);
    # a sequential left-to-right sum would give 0.
    assert oracle.wave64_sum(lanes) == np.float32(1.0)
    lanes = np.zeros(64, np.float32)
    lanes[0], lanes[16], lanes[32], lanes[48] = big, 1.0, 1.0, -big
    # rows pair as (row0 + row1) + (row2 + row3): (2^24 + 1) + (1 - 2^24) = 1
    assert oracle.wave64_sum(lanes) == np.float32(1.0)
    lanes = np.zeros(64, np.float32)
    lanes[0], lanes[32], lanes[16], lanes[48] = big, -big, 1.0, 1.0
    # (2^24 + 1) + (-2^24 + 1) = 2^24 - 2^24 + 1... = (2^24) + (1 - 2^24) = 1
    assert oracle.wave64_sum(lanes) == np.float32(1.0)
    ints = np.arange(64, dtype=np.float32)
    assert oracle.wave64_sum(ints) == np.float32(ints.sum())


@pytest.mark.parametrize("order", [oracle.ORDER_REF, oracle.ORDER_WAVE64])
def test_rmsnorm_close_to_fp64(order):
    rng = np.random.default_rng(5 + order)
    x = normal_f16(rng, 2048)
    w = normal_f16(rng, 2048)
    out = oracle.rmsnorm(x, w, 1e-6, order).astype(np.float64)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w.astype(np.float64)
    assert np.all(np.abs(out - want) <= ulp16(want) + 1e-6)


def test_rmsnorm_orders_agree_and_closed_form():
    rng = np.random.default_rng(9)
    x = normal_f16(rng, 2048)
    w = normal_f16(rng, 2048)
    a = oracle.rmsnorm(x, w, 1e-6, oracle.ORDER_REF).astype(np.float64)
    b = oracle.rmsnorm(x, w, 1e-6, oracle.ORDER_WAVE64).astype(np.float64)
    assert np.all(np.abs(a - b) <= ulp16(a))
    c = np.full(2048, np.float16(-0.75))
    ones = np.ones(2048, np.float16)
    for order in (oracle.ORDER_REF, oracle.ORDER_WAVE64):
        out = oracle.rmsnorm(c, w, 0.0, order)
        assert np.array_equal(out.view(np.uint16), (-w).view(np.uint16))   # x/|x| * w
        assert np.all(oracle.rmsnorm(c, ones, 0.0, order) == np.float16(-1.0))


def test_gemv_reference_order_is_sequential_fp32():
    rng = np.random.default_rng(11)
    K, N = 2048, 64
    x = normal_f16(rng, K)
    W = normal_f16(rng, (N, K), 0.02)
    got = oracle.gemv(x, W, N, K, layout=0, order=oracle.ORDER_REF)
    prods = (W.astype(np.float32) * x.astype(np.float32)[None, :])        # exact products
    seq = np.cumsum(prods, axis=1, dtype=np.float32)[:, -1]                # left-to-right
    assert np.array_equal(got.view(np.uint16), seq.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("K", [2048, 5504, 64])
@pytest.mark.parametrize("order", [oracle.ORDER_REF, oracle.ORDER_WAVE64])
def test_gemv_close_to_fp64_both_layouts(K, order):
    rng = np.random.default_rng(K + order)
    N = 96
    x = normal_f16(rng, K)
    W = normal_f16(rng, (N, K), 0.02)
    a = oracle.gemv(x, W, N, K, layout=0, order=order)
    b = oracle.gemv(x, np.ascontiguousarray(W.T), N, K, layout=1, order=order)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    exact = W.astype(np.float64) @ x.astype(np.float64)
    bound = 0.5 * ulp16(exact) + K * 2.0 ** -23 * (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(a.astype(np.float64) - exact) <= bound)


def test_gemv_one_hot_picks_column():
    rng = np.random.default_rng(12)
    K, N = 2048, 40
    W = normal_f16(rng, (N, K))
    x = np.zeros(K, np.float16)
    x[777] = 1.0
    for order in (oracle.ORDER_REF, oracle.ORDER_WAVE64):
        assert np.array_equal(oracle.gemv(x, W, N, K, 0, order).view(np.uint16), W[:, 777].view(np.uint16))


def test_qkv_front_is_norm_gemv_then_feeder():
    H, D = 16, 128
    hid = H * D
    rng = np.random.default_rng(13)
    x = normal_f16(rng, hid)
    nw = normal_f16(rng, hid)
    Wq = normal_f16(rng, (3 * hid, hid), 0.02)
    b = normal_f16(rng, 3 * hid, 0.02)
    S, pos = 8, 5
    for norm in (None, nw):
        qkv = np.zeros(3 * hid, np.float16)
        kc = np.zeros(S * hid, np.float16)
        vc = np.zeros(S * hid, np.float16)
        oracle.qkv_front(x, norm, Wq, b, qkv, kc, vc, pos, H)
        xn = x if norm is None else oracle.rmsnorm(x, nw, 1e-6, oracle.ORDER_WAVE64)
        want = oracle.gemv(xn, Wq, 3 * hid, hid, 0, oracle.ORDER_WAVE64)
        kc2 = np.zeros_like(kc)
        vc2 = np.zeros_like(vc)
        oracle.qkv_bias_rope_cache(want, b, kc2, vc2, pos, H)
        assert np.array_equal(qkv.view(np.uint16), want.view(np.uint16))
        assert np.array_equal(kc.view(np.uint16), kc2.view(np.uint16))
        assert np.array_equal(vc.view(np.uint16), vc2.view(np.uint16))
