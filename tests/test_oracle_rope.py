"""Pins the CPU oracle of bias + RoPE + KV-cache append
(kernels/bias.cuh:6-11, kernels/fused_qkv_rope_cache.cuh:6-55).

  * bias add: bit-exact against numpy's independent float32 add + RNE cast;
  * rotation arithmetic: bit-exact against numpy float32 q1*c - q2*s etc.
    (numpy never contracts) fed the oracle's cos/sin;
  * cos/sin: within 2 float32 ulps of float64 cos/sin of the same float32 theta,
    and theta within 1 ulp of pos * 10000^(-2i/128);
  * rotate-half structure: within 1 fp16 ulp (+theta error) of a float64
    rotation, pos=0 is the identity, pair norms are preserved;
  * cache append: only row `pos` changes, V is a bit copy, both layouts agree;
  * teeth: interleaved pairs, a sign flip or a /64 exponent all miss by far.
"""
import numpy as np
import pytest

from common import normal_f16, ulp16
from oracle import oracle

H, D = 16, 128
HID = H * D


def _run(qkv, bias, pos, max_seqlen=8, layout="engine", fill=0.0):
    if layout == "engine":
        rs, hs = HID, D
    else:
        rs, hs = D, max_seqlen * D
    kc = np.full(max_seqlen * HID, fill, np.float16)
    vc = np.full(max_seqlen * HID, fill, np.float16)
    out = qkv.copy()
    oracle.qkv_bias_rope_cache(out, bias, kc, vc, pos, H, D, rs, hs)
    return out, kc, vc, rs, hs


def _cs_table(pos):
    c = np.empty(64, np.float32)
    s = np.empty(64, np.float32)
    for i in range(64):
        c[i], s[i] = oracle.rope_cos_sin(pos, i)
    return c, s


def test_bias_add_bit_exact_vs_numpy():
    rng = np.random.default_rng(1)
    qkv = normal_f16(rng, 3 * HID)
    bias = normal_f16(rng, 3 * HID, 0.02)
    out, *_ = _run(qkv, bias, pos=0)
    want = (qkv.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
    # pos 0 rotation is the identity, so the whole buffer equals the biased input
    assert np.array_equal(out.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("pos", [0, 1, 3, 5, 2047, 32767])
def test_rotation_arithmetic_bit_exact(pos):
    rng = np.random.default_rng(pos + 10)
    qkv = normal_f16(rng, 3 * HID)
    out, kc, vc, rs, hs = _run(qkv, None, pos, max_seqlen=pos + 1)
    c, s = _cs_table(pos)
    f = qkv.astype(np.float32).reshape(3, H, 2, 64)
    q1, q2, k1, k2 = f[0, :, 0], f[0, :, 1], f[1, :, 0], f[1, :, 1]
    q1r = (q1 * c - q2 * s).astype(np.float16)
    q2r = (q2 * c + q1 * s).astype(np.float16)
    k1r = (k1 * c - k2 * s).astype(np.float16)
    k2r = (k2 * c + k1 * s).astype(np.float16)
    qw = np.stack([q1r, q2r], axis=1).reshape(HID)
    kw = np.stack([k1r, k2r], axis=1).reshape(HID)
    assert np.array_equal(out[:HID].view(np.uint16), qw.view(np.uint16))
    assert np.array_equal(out[HID:].view(np.uint16), qkv[HID:].view(np.uint16))  # K/V of qkv untouched
    row = slice(pos * HID, (pos + 1) * HID)
    assert np.array_equal(kc[row].view(np.uint16), kw.view(np.uint16))
    assert np.array_equal(vc[row].view(np.uint16), qkv[2 * HID:].view(np.uint16))


@pytest.mark.parametrize("pos", [1, 7, 100, 2047, 8191, 32767])
def test_cos_sin_close_to_fp64(pos):
    c, s = _cs_table(pos)
    i = np.arange(64)
    theta32 = (np.float32(pos) * (10000.0 ** (-2.0 * i / 128.0)).astype(np.float32)).astype(np.float32)
    th = np.array([np.float32(pos) * np.float32(10000.0 ** (-2.0 * k / 128.0)) for k in i], np.float64)
    # theta carries the float32 rounding of pos * powf(...)
    exact = pos * 10000.0 ** (-2.0 * i / 128.0)
    assert np.all(np.abs(th - exact) <= 2 * np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64) + 1e-30)
    ulp32 = lambda x: np.spacing(np.abs(x).astype(np.float32)).astype(np.float64)
    # cos/sin of the oracle's own float32 theta: compare against float64 of a
    # theta within 2 ulps (powf is not correctly rounded everywhere)
    for j in range(64):
        cands = np.float32(theta32[j]) + np.arange(-2, 3) * np.spacing(np.float32(theta32[j]))
        ok = any(abs(np.cos(np.float64(t)) - c[j]) <= 2 * ulp32(np.cos(np.float64(t))) + 1e-12 and
                 abs(np.sin(np.float64(t)) - s[j]) <= 2 * ulp32(np.sin(np.float64(t))) + 1e-12
                 for t in cands)
        assert ok, (pos, j, c[j], s[j])


@pytest.mark.parametrize("pos", [3, 5, 511, 2047])
def test_rotation_close_to_fp64(pos):
    rng = np.random.default_rng(pos)
    qkv = normal_f16(rng, 3 * HID)
    out, kc, *_ = _run(qkv, None, pos, max_seqlen=pos + 1)
    i = np.arange(64)
    th = pos * 10000.0 ** (-2.0 * i / 128.0)
    c, s = np.cos(th), np.sin(th)
    f = qkv.astype(np.float64).reshape(3, H, 2, 64)
    want_q = np.stack([f[0, :, 0] * c - f[0, :, 1] * s, f[0, :, 1] * c + f[0, :, 0] * s], 1).reshape(HID)
    want_k = np.stack([f[1, :, 0] * c - f[1, :, 1] * s, f[1, :, 1] * c + f[1, :, 0] * s], 1).reshape(HID)
    # theta's float32 rounding moves the angle by <= ulp32(theta); bound its effect
    dth = np.spacing(np.float32(th.max())).astype(np.float64) * 2
    mag = np.repeat(np.abs(f[:2]).sum(axis=2), 2, axis=1).reshape(2, HID)
    for got, want, m in ((out[:HID], want_q, mag[0]), (kc[pos * HID:(pos + 1) * HID], want_k, mag[1])):
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= 0.5 * ulp16(want) + dth * m + 1e-6)


def test_pos0_is_identity_and_norm_preserved():
    rng = np.random.default_rng(3)
    qkv = normal_f16(rng, 3 * HID)
    out, kc, vc, *_ = _run(qkv, None, 0, max_seqlen=2)
    assert np.array_equal(out.view(np.uint16), qkv.view(np.uint16))
    assert np.array_equal(kc[:HID].view(np.uint16), qkv[HID:2 * HID].view(np.uint16))
    out, kc, *_ = _run(qkv, None, 1000, max_seqlen=1001)
    a = qkv[:HID].astype(np.float64).reshape(H, 2, 64)
    b = out[:HID].astype(np.float64).reshape(H, 2, 64)
    na, nb = np.hypot(a[:, 0], a[:, 1]), np.hypot(b[:, 0], b[:, 1])
    assert np.all(np.abs(na - nb) <= 2 * ulp16(na) + 1e-6)


def test_only_row_pos_is_written_both_layouts():
    rng = np.random.default_rng(4)
    qkv = normal_f16(rng, 3 * HID)
    sentinel = np.float16(-7.5)
    out_e, kc_e, vc_e, *_ = _run(qkv, None, 5, max_seqlen=9, layout="engine", fill=sentinel)
    out_h, kc_h, vc_h, *_ = _run(qkv, None, 5, max_seqlen=9, layout="head_major", fill=sentinel)
    ke = kc_e.reshape(9, H, D)
    kh = kc_h.reshape(H, 9, D).transpose(1, 0, 2)
    ve = vc_e.reshape(9, H, D)
    vh = vc_h.reshape(H, 9, D).transpose(1, 0, 2)
    assert np.array_equal(ke.view(np.uint16), kh.view(np.uint16))
    assert np.array_equal(ve.view(np.uint16), vh.view(np.uint16))
    others = [r for r in range(9) if r != 5]
    assert np.all(ke[others] == sentinel) and np.all(ve[others] == sentinel)
    assert np.array_equal(out_e.view(np.uint16), out_h.view(np.uint16))


def test_rotation_has_teeth():
    pos = 2047
    rng = np.random.default_rng(8)
    qkv = normal_f16(rng, 3 * HID)
    out, *_ = _run(qkv, None, pos, max_seqlen=pos + 1)
    got = out[:HID].astype(np.float64).reshape(H, 128)
    q = qkv[:HID].astype(np.float64).reshape(H, 128)
    i = np.arange(64)

    def rot_half(freq_div, sign=1.0):
        th = pos * 10000.0 ** (-2.0 * i / freq_div)
        c, s = np.cos(th), sign * np.sin(th)
        return np.concatenate([q[:, :64] * c - q[:, 64:] * s, q[:, 64:] * c + q[:, :64] * s], 1)

    def interleaved():
        th = pos * 10000.0 ** (-2.0 * i / 128.0)
        c, s = np.cos(th), np.sin(th)
        e, o = q[:, 0::2], q[:, 1::2]
        r = np.empty_like(q)
        r[:, 0::2] = e * c - o * s
        r[:, 1::2] = o * c + e * s
        return r

    assert np.max(np.abs(rot_half(128.0) - got)) < 2e-3
    for name, m in {"sign": rot_half(128.0, -1.0), "exp64": rot_half(64.0),
                    "interleaved": interleaved()}.items():
        assert np.max(np.abs(m - got)) > 0.1, name


def test_rejects_invalid_arguments():
    qkv = np.zeros(3 * HID, np.float16)
    kc = np.zeros(HID, np.float16)
    with pytest.raises(ValueError):
        oracle.qkv_bias_rope_cache(qkv, None, kc, kc, -1, H)
