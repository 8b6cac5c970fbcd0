"""Pins the CPU oracle of the decode-attention path (flash_decode_q1_opt.cuh).

What pins it (no golden vectors ship with the reference; its tests draw from
libc rand() at run time, kernels/unit_tests/run_tests.cu:867):
  * float64 brute force (textbook softmax(Kq/sqrt(128))V, the procedure of
    run_tests.cu:576-600) within the binary16 rounding the restatement must do;
  * closed forms: L=1 -> V0; the bench's constant 0x3C inputs
    (bench_fd_opt.cu:134-136) -> every output 0x3C3C; constant V -> V;
    identical keys -> mean(V); one dominant key -> that V row;
  * invariants: fused == split == engine dispatch within rounding, layout
    independence (bit-exact), head independence (bit-exact);
  * teeth: plausible mistakes (missing scale, off-by-one row, sign flip, wrong
    head) miss the float64 reference by far more than the tolerance.
"""
import numpy as np
import pytest

from common import AttnCase, attn_fp64, ulp16, normal_f16
from oracle import oracle


def _tol_fused(ref):
    return 0.5 * ulp16(ref) + 1e-5


def _split_tol(case, h, ref, chunk=256):
    # partials are rounded to binary16 before the stage-2 merge (flash_decode_q1_opt.cuh:650)
    pmax = np.zeros(128)
    for c0 in range(0, case.L, chunk):
        pmax = np.maximum(pmax, np.abs(attn_fp64(case.q[h], case.Kh[h, c0:c0 + chunk],
                                                 case.Vh[h, c0:c0 + chunk])))
    return 0.5 * ulp16(ref) + 0.5 * ulp16(pmax) + 1e-5


@pytest.mark.parametrize("L", [1, 2, 31, 32, 33, 255, 256, 257, 512, 1000, 1024])
def test_fused_matches_fp64(L):
    case = AttnCase(L, H=4, seed=L)
    out = oracle.decode_attention(case.q, case.kc, case.vc, L, 4, case.row_stride,
                                  case.head_stride, oracle.FUSED).astype(np.float64)
    ref = case.fp64()
    assert np.all(np.abs(out - ref) <= _tol_fused(ref))


@pytest.mark.parametrize("L", [1, 255, 256, 257, 513, 1024, 3000, 8192])
def test_split_matches_fp64(L):
    case = AttnCase(L, H=2, seed=100 + L, kscale=0.5)
    out = oracle.decode_attention(case.q, case.kc, case.vc, L, 2, case.row_stride,
                                  case.head_stride, oracle.SPLIT).astype(np.float64)
    ref = case.fp64()
    for h in range(2):
        assert np.all(np.abs(out[h] - ref[h]) <= _split_tol(case, h, ref[h]))


def test_split_lse_and_partials_are_chunk_softmax():
    case = AttnCase(700, H=1, seed=7)
    out, part, lse = oracle.fd_split_head(case.q[0], case.kc, case.vc, 700, case.row_stride)
    assert part.shape == (3, 128) and lse.shape == (3,)
    for c in range(3):
        K = case.Kh[0, 256 * c:256 * c + 256].astype(np.float64)
        s = K @ case.q[0].astype(np.float64) / np.sqrt(128.0)
        want = np.log(np.exp(s - s.max()).sum()) + s.max()
        assert abs(lse[c] - want) <= 1e-5 * max(1.0, abs(want))
        pref = attn_fp64(case.q[0], case.Kh[0, 256 * c:256 * c + 256], case.Vh[0, 256 * c:256 * c + 256])
        assert np.all(np.abs(part[c].astype(np.float64) - pref) <= 0.5 * ulp16(pref) + 1e-5)


@pytest.mark.parametrize("variant", [oracle.ENGINE, oracle.FUSED, oracle.SPLIT])
def test_single_row_returns_v0_exactly(variant):
    case = AttnCase(1, H=3, seed=5)
    out = oracle.decode_attention(case.q, case.kc, case.vc, 1, 3, case.row_stride,
                                  case.head_stride, variant)
    assert np.array_equal(out.view(np.uint16), case.Vh[:, 0].view(np.uint16))


@pytest.mark.parametrize("variant,L", [(oracle.FUSED, 256), (oracle.FUSED, 1024),
                                       (oracle.SPLIT, 8192), (oracle.ENGINE, 256),
                                       (oracle.ENGINE, 4096)])
def test_bench_constant_0x3c_inputs(variant, L):
    # bench_fd_opt.cu fills Q/K/V bytes with 0x3C: every element is 0x3C3C = 1.0586
    fill = np.array([0x3C3C], np.uint16).view(np.float16)[0]
    case = AttnCase(L, H=2, fill=fill)
    out = oracle.decode_attention(case.q, case.kc, case.vc, L, 2, case.row_stride,
                                  case.head_stride, variant)
    assert np.all(out.view(np.uint16) == 0x3C3C)


def test_constant_v_returns_v():
    case = AttnCase(777, H=2, seed=9)
    case_v = case.Vh[:, :1, :].repeat(777, axis=1)
    case.Vh[:] = case_v
    case.vc[:] = np.ascontiguousarray(case.Vh.transpose(1, 0, 2)).reshape(-1)
    for variant in (oracle.SPLIT, oracle.ENGINE):
        out = oracle.decode_attention(case.q, case.kc, case.vc, 777, 2, case.row_stride,
                                      case.head_stride, variant).astype(np.float64)
        v0 = case.Vh[:, 0].astype(np.float64)
        assert np.all(np.abs(out - v0) <= ulp16(v0))


def test_identical_keys_give_mean_v():
    case = AttnCase(300, H=1, seed=11)
    case.Kh[:] = case.Kh[:, :1]
    case.kc[:] = np.ascontiguousarray(case.Kh.transpose(1, 0, 2)).reshape(-1)
    out = oracle.decode_attention(case.q, case.kc, case.vc, 300, 1, case.row_stride,
                                  case.head_stride, oracle.SPLIT)[0].astype(np.float64)
    Vd = case.Vh[0].astype(np.float64)
    mean = Vd.mean(axis=0)
    # stage-1 partials are the chunk means, rounded to binary16 before the merge
    pmax = np.maximum(np.abs(Vd[:256].mean(axis=0)), np.abs(Vd[256:].mean(axis=0)))
    assert np.all(np.abs(out - mean) <= 0.5 * ulp16(mean) + 0.5 * ulp16(pmax) + 1e-6)


def test_dominant_key_selects_its_row():
    case = AttnCase(1500, H=1, seed=12)
    j = 1234
    case.Kh[0, j] = (case.q[0].astype(np.float32) * 4).astype(np.float16)   # logit ~ 45 above the rest
    case.kc[:] = np.ascontiguousarray(case.Kh.transpose(1, 0, 2)).reshape(-1)
    out = oracle.decode_attention(case.q, case.kc, case.vc, 1500, 1, case.row_stride,
                                  case.head_stride, oracle.ENGINE)[0]
    vj = case.Vh[0, j].astype(np.float64)
    assert np.all(np.abs(out.astype(np.float64) - vj) <= ulp16(vj))


@pytest.mark.parametrize("L", [100, 256, 900])
def test_fused_and_split_agree(L):
    case = AttnCase(L, H=4, seed=20 + L)
    a = oracle.decode_attention(case.q, case.kc, case.vc, L, 4, case.row_stride,
                                case.head_stride, oracle.FUSED).astype(np.float64)
    b = oracle.decode_attention(case.q, case.kc, case.vc, L, 4, case.row_stride,
                                case.head_stride, oracle.SPLIT).astype(np.float64)
    assert np.max(np.abs(a - b)) <= 2e-3


@pytest.mark.parametrize("variant", [oracle.ENGINE, oracle.SPLIT])
def test_layout_independence_bit_exact(variant):
    eng = AttnCase(600, H=4, seed=33, layout="engine", max_seqlen=640)
    hm = AttnCase(600, H=4, seed=33, layout="head_major", max_seqlen=700)
    a = oracle.decode_attention(eng.q, eng.kc, eng.vc, 600, 4, eng.row_stride, eng.head_stride, variant)
    b = oracle.decode_attention(hm.q, hm.kc, hm.vc, 600, 4, hm.row_stride, hm.head_stride, variant)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_head_independence_bit_exact():
    case = AttnCase(520, H=4, seed=44)
    a = oracle.decode_attention(case.q, case.kc, case.vc, 520, 4, case.row_stride, case.head_stride)
    kc = case.kc.reshape(520, 4, 128).copy()
    kc[:, 2] = -kc[:, 2]
    b = oracle.decode_attention(case.q, kc.reshape(-1), case.vc, 520, 4, case.row_stride, case.head_stride)
    keep = [0, 1, 3]
    assert np.array_equal(a[keep].view(np.uint16), b[keep].view(np.uint16))
    assert not np.array_equal(a[2], b[2])


def test_rows_beyond_seqlen_are_ignored():
    case = AttnCase(400, H=2, seed=55, max_seqlen=512)
    a = oracle.decode_attention(case.q, case.kc, case.vc, 300, 2, case.row_stride, case.head_stride)
    kc = case.kc.reshape(512, 2, 128).copy()
    kc[300:] = np.float16(30.0)
    b = oracle.decode_attention(case.q, kc.reshape(-1), case.vc, 300, 2, case.row_stride, case.head_stride)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_threads_do_not_change_results():
    case = AttnCase(2000, H=4, seed=66)
    a = oracle.decode_attention(case.q, case.kc, case.vc, 2000, 4, case.row_stride, case.head_stride,
                                oracle.ENGINE, 1)
    b = oracle.decode_attention(case.q, case.kc, case.vc, 2000, 4, case.row_stride, case.head_stride,
                                oracle.ENGINE, 8)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_rejects_invalid_arguments():
    case = AttnCase(10, H=1, seed=1)
    with pytest.raises(ValueError):
        oracle.decode_attention(case.q, case.kc, case.vc, 0, 1, case.row_stride, case.head_stride)
    with pytest.raises(ValueError):   # fused single block holds at most 32 warps x 32 rows
        big = AttnCase(1025, H=1, seed=1)
        oracle.decode_attention(big.q, big.kc, big.vc, 1025, 1, big.row_stride, big.head_stride,
                                oracle.FUSED)


def test_fp64_check_has_teeth():
    """Each plausible mistake misses the oracle by >> the tolerance used above."""
    case = AttnCase(512, H=2, seed=77)
    out = oracle.decode_attention(case.q, case.kc, case.vc, 512, 2, case.row_stride,
                                  case.head_stride, oracle.FUSED).astype(np.float64)
    q, K, V = case.q[0], case.Kh[0], case.Vh[0]
    tol = np.max(_tol_fused(out[0]))

    def softmax_v(s, Vm):
        p = np.exp(s - s.max())
        return (p / p.sum()) @ Vm.astype(np.float64)

    Kd, qd = K.astype(np.float64), q.astype(np.float64)
    mutants = {
        "no_scale": softmax_v(Kd @ qd, V),
        "drop_last_row": softmax_v(Kd[:-1] @ qd / np.sqrt(128), V[:-1]),
        "sign_flip": softmax_v(-(Kd @ qd) / np.sqrt(128), V),
        "wrong_head_v": softmax_v(Kd @ qd / np.sqrt(128), case.Vh[1]),
        "scale_by_64": softmax_v(Kd @ qd / 8.0 / np.sqrt(2.0) / 2, V),
    }
    for name, m in mutants.items():
        assert np.max(np.abs(m - out[0])) > 5 * tol, name
