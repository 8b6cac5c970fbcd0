"""GPU parity of the batched projection qd_gemm_nt (the prefill GEMM) in both
modes, and of the engine's MFMA prefill mode.

Bars:
  * QD_GEMM_EXACT: every row bit-exact against the oracle's decode-order GEMV
    (and against its projection + residual), i.e. the same bits as the decode
    step computes token by token;
  * QD_GEMM_MFMA: fp16 x fp16 products are exact in fp32 and the matrix cores
    sum them in fp32 in their own order, so each output is within one fp16 ulp
    of the float64 sum plus the fp32 summation bound k * 2^-23 * sum|x w|
    (with a residual: plus one more fp16 rounding);
  * engine, MFMA prefill: the KV rows differ from exact prefill only by that
    summation order, so the next step's logits agree closely; decode steps
    themselves are unchanged.
"""
import numpy as np
import pytest
import torch

from common import model_kv_fp64, model_tensors, normal_f16, ulp16
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qdiy():
    import qdiy as m
    torch.cuda.set_device(0)
    m.load()
    return m


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint16), np.asarray(b).view(np.uint16))


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("m,n,k", [(1, 64, 64), (37, 100, 520), (127, 6144, 2048), (256, 2048, 5504),
                                   (45, 4104, 1544), (300, 4100, 2000)])
@pytest.mark.parametrize("with_res", [False, True])
def test_exact_mode_is_the_decode_gemv(qdiy, m, n, k, with_res):
    """Exact-mode rows against the oracle's decode GEMV, bit for bit.  From K = 1544 to
    2048 with n >= 4096 the four-rows-per-wave kernel runs: (45, 4104, 1544) has a last
    chunk of one lane, rows past n clamped in the last workgroup and odd token tiles;
    (300, 4100, 2000) more than 256 tokens.  (256, 2048, 5504) runs 64 tokens per
    workgroup in 4-token tiles.  The rows checked straddle the token tiles and the 32-
    and 64-token workgroups."""
    rng = np.random.default_rng(m * 1000 + n + k + with_res)
    x, W, R = normal_f16(rng, (m, k)), normal_f16(rng, (n, k), 0.02), normal_f16(rng, (m, n))
    y = torch.zeros(m * n, dtype=torch.float16, device="cuda")
    qdiy.gemm_nt(_dev(x.reshape(-1)), _dev(W.reshape(-1)), y, m, n, k,
                 residual=_dev(R.reshape(-1)) if with_res else None, mode=qdiy.GEMM_EXACT)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(m, n)
    rows = sorted({i for i in (0, 1, 7, 8, 31, 32, 63, 64, m // 2, m - 2, m - 1) if 0 <= i < m})
    for i in rows:
        if with_res:
            want = oracle.proj_residual(x[i], W.reshape(-1), R[i], n, k)
        else:
            want = oracle.gemv(x[i], W.reshape(-1), n, k, 0, oracle.ORDER_WAVE64)
        assert _same(got[i], want), f"row {i}"


@pytest.mark.parametrize("m,n,k", [(1, 64, 64), (37, 100, 512), (127, 6144, 2048), (256, 2048, 5504),
                                   (200, 5504, 2048),
                                   # from 128 rows: the 64 x 64 tile where a 128 x 128 grid would
                                   # leave most CUs idle (ragged m and n, a partial group of four
                                   # outputs at n = 130), the 128 x 128 ring tile, and the 192 x 256
                                   # ring tile where its grid covers the CUs (ragged rows of W at
                                   # n = 6000, ragged tokens at m = 1800)
                                   (600, 130, 512), (1024, 2048, 5504), (512, 6144, 2048),
                                   (2048, 6144, 2048), (2048, 6000, 2048), (1800, 6144, 1024),
                                   # the 192 x 256 tile with 1, 2, 3 and 17 K tiles of 64 (its two
                                   # stages never fill, fill once, or end on an odd tile)
                                   (2048, 6144, 64), (2048, 6144, 128), (2048, 6000, 192),
                                   (1800, 6144, 1088)])
@pytest.mark.parametrize("with_res", [False, True])
def test_mfma_mode_within_fp32_summation_bound(qdiy, m, n, k, with_res):
    rng = np.random.default_rng(7 * m + n + k + with_res)
    x, W, R = normal_f16(rng, (m, k)), normal_f16(rng, (n, k), 0.02), normal_f16(rng, (m, n))
    y = torch.full((m * n + 64,), 9.0, dtype=torch.float16, device="cuda")
    qdiy.gemm_nt(_dev(x.reshape(-1)), _dev(W.reshape(-1)), y, m, n, k,
                 residual=_dev(R.reshape(-1)) if with_res else None, mode=qdiy.GEMM_MFMA)
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    assert np.all(out[m * n:] == np.float16(9.0)), "write past the end of y"
    got = out[:m * n].reshape(m, n).astype(np.float64)
    x64, W64 = x.astype(np.float64), W.astype(np.float64)
    s = x64 @ W64.T
    bound = k * 2.0 ** -23 * (np.abs(x64) @ np.abs(W64).T)
    if with_res:
        h = s.astype(np.float16).astype(np.float64)
        want = R.astype(np.float64) + h
        tol = ulp16(want) + ulp16(h) + bound + ulp16(s)
    else:
        want, tol = s, ulp16(s) + bound
    assert np.all(np.abs(got - want) <= tol), float(np.max(np.abs(got - want) - tol))


@pytest.mark.parametrize("m,n,k,ldy", [(37, 100, 512, 100), (127, 1368, 2048, 1368),
                                        # from 128 rows: the 64 x 64 tile (n = 130, a strided
                                        # output), the 128 x 128 ring tile (a ragged last tile at
                                        # n = 1000; 512 x 5504), the 192 x 256 ring tile (2048 x
                                        # 5504: a last tile of 32 of its 96 outputs)
                                        (600, 130, 512, 136), (1000, 1000, 1024, 1000),
                                        (512, 5504, 2048, 5504), (2048, 5504, 2048, 5504),
                                        # the 192 x 256 tile over 3 K tiles, ragged tokens
                                        (1900, 5504, 192, 5504)])
def test_gemm_swiglu_within_bound(qdiy, m, n, k, ldy):
    """qd_gemm_swiglu: gate and up GEMMs on the matrix cores with the SwiGLU in the
    epilogue.  Each act is half(g * silu(u)) of g and u the fp16 roundings of
    fp32 sums; those may round to the neighbour of the float64 sum's fp16
    value when the fp32 sum lies within its summation bound of the boundary,
    so act is within the propagated bound of half(g64) * silu(half(u64)):
    |silu(u)| (ulp(g) + bound_g) + |g| 1.1 (ulp(u) + bound_u) + 2 ulp(act)."""
    rng = np.random.default_rng(31 * m + n + k)
    x = normal_f16(rng, (m, k))
    W1, W2 = normal_f16(rng, (n, k), 0.03), normal_f16(rng, (n, k), 0.03)
    act = torch.full((m * ldy + 64,), 9.0, dtype=torch.float16, device="cuda")
    qdiy.gemm_swiglu(_dev(x.reshape(-1)), _dev(W1.reshape(-1)), _dev(W2.reshape(-1)), act, m, n, k,
                     ldy=ldy)
    torch.cuda.synchronize()
    out = act.cpu().numpy()
    assert np.all(out[(m - 1) * ldy + n:] == np.float16(9.0)), "write past the last row"
    got = np.stack([out[i * ldy:i * ldy + n] for i in range(m)]).astype(np.float64)
    if ldy > n:
        gaps = np.stack([out[i * ldy + n:(i + 1) * ldy] for i in range(m - 1)])
        assert np.all(gaps == np.float16(9.0)), "write between rows"
    x64, W1d, W2d = x.astype(np.float64), W1.astype(np.float64), W2.astype(np.float64)
    g, u = x64 @ W1d.T, x64 @ W2d.T
    ax = np.abs(x64)
    bg, bu = k * 2.0 ** -23 * (ax @ np.abs(W1d).T), k * 2.0 ** -23 * (ax @ np.abs(W2d).T)
    gh = g.astype(np.float16).astype(np.float64)
    uh = u.astype(np.float16).astype(np.float64)
    silu = uh / (1.0 + np.exp(-uh))
    want = gh * silu
    tol = np.abs(silu) * (ulp16(gh) + bg) + np.abs(gh) * 1.1 * (ulp16(uh) + bu) + 2 * ulp16(want)
    err = np.abs(got - want)
    assert np.all(err <= tol), (float(np.max(err - tol)), np.unravel_index(np.argmax(err - tol), err.shape))
    # the bound is tight enough to see a swapped gate and up
    swapped = uh * (gh / (1.0 + np.exp(-gh)))
    assert np.mean(np.abs(swapped - got) > tol) > 0.5


@pytest.mark.parametrize("seed", range(16))
def test_mfma_random_shapes(qdiy, seed):
    """Seeded random m (both sides of the 128-row ring-tile threshold and of the
    64-token tile), n (ragged against 64), k (a multiple of 64 up to 6144, so the
    K-tile rings wrap several times or run short of their stages), row strides
    and the residual form of qd_gemm_nt, then qd_gemm_swiglu at the same m:
    every output within the bounds of the fixed-shape tests."""
    rng = np.random.default_rng(52000 + seed)
    m = int(rng.integers(1, 130)) if rng.random() < 0.6 else int(rng.integers(130, 700))
    n = int(rng.integers(1, 700))
    k = 64 * int(rng.integers(1, 97))
    ldy = n + int(rng.integers(0, 9))
    with_res = bool(rng.random() < 0.5)
    x, W, R = normal_f16(rng, (m, k)), normal_f16(rng, (n, k), 0.02), normal_f16(rng, (m, n))
    y = torch.full((m * ldy + 64,), 9.0, dtype=torch.float16, device="cuda")
    if with_res:
        yv = y[:m * ldy].view(m, ldy)
        yv[:, :n] = torch.from_numpy(R).cuda()
    qdiy.gemm_nt(_dev(x.reshape(-1)), _dev(W.reshape(-1)), y, m, n, k, residual=y if with_res else None,
                 mode=qdiy.GEMM_MFMA, ldy=ldy)
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    assert np.all(out[m * ldy:] == np.float16(9.0)), "write past the end of y"
    rows = out[:m * ldy].reshape(m, ldy)
    if ldy > n:
        assert np.all(rows[:, n:] == np.float16(9.0)), "write into a row's padding"
    got = rows[:, :n].astype(np.float64)
    x64, W64 = x.astype(np.float64), W.astype(np.float64)
    s = x64 @ W64.T
    bound = k * 2.0 ** -23 * (np.abs(x64) @ np.abs(W64).T)
    if with_res:
        h = s.astype(np.float16).astype(np.float64)
        want = R.astype(np.float64) + h
        tol = ulp16(want) + ulp16(h) + bound + ulp16(s)
    else:
        want, tol = s, ulp16(s) + bound
    assert np.all(np.abs(got - want) <= tol), (m, n, k, ldy, with_res, float(np.max(np.abs(got - want) - tol)))
    # gate and up with the SwiGLU epilogue at the same m (ldy = n)
    W1, W2 = normal_f16(rng, (n, k), 0.03), normal_f16(rng, (n, k), 0.03)
    act = torch.full((m * n + 64,), 9.0, dtype=torch.float16, device="cuda")
    qdiy.gemm_swiglu(_dev(x.reshape(-1)), _dev(W1.reshape(-1)), _dev(W2.reshape(-1)), act, m, n, k)
    torch.cuda.synchronize()
    a = act.cpu().numpy()
    assert np.all(a[m * n:] == np.float16(9.0)), "write past the last row"
    got = a[:m * n].reshape(m, n).astype(np.float64)
    W1d, W2d = W1.astype(np.float64), W2.astype(np.float64)
    g, u = x64 @ W1d.T, x64 @ W2d.T
    ax = np.abs(x64)
    bg, bu = k * 2.0 ** -23 * (ax @ np.abs(W1d).T), k * 2.0 ** -23 * (ax @ np.abs(W2d).T)
    gh, uh = g.astype(np.float16).astype(np.float64), u.astype(np.float16).astype(np.float64)
    silu = uh / (1.0 + np.exp(-uh))
    want = gh * silu
    tol = np.abs(silu) * (ulp16(gh) + bg) + np.abs(gh) * 1.1 * (ulp16(uh) + bu) + 2 * ulp16(want)
    assert np.all(np.abs(got - want) <= tol), (m, n, k, float(np.max(np.abs(got - want) - tol)))


def test_gemm_nt_rejects_bad_arguments(qdiy):
    x = torch.zeros(4 * 96, dtype=torch.float16, device="cuda")
    w = torch.zeros(16 * 96, dtype=torch.float16, device="cuda")
    y = torch.zeros(4 * 16, dtype=torch.float16, device="cuda")
    with pytest.raises(qdiy.QdError, match="multiple of 64"):
        qdiy.gemm_nt(x, w, y, 4, 16, 96, mode=qdiy.GEMM_MFMA)
    with pytest.raises(qdiy.QdError, match="unknown mode"):
        qdiy.gemm_nt(x, w, y, 4, 16, 96, mode=7)
    big = torch.zeros(4096, dtype=torch.float16, device="cuda")
    with pytest.raises(qdiy.QdError, match="overlaps"):
        qdiy.gemm_nt(big[:4 * 64], w, big[128:128 + 4 * 16], 4, 16, 64)
    qdiy.gemm_nt(x, w, y, 4, 16, 64, mode=qdiy.GEMM_MFMA, ldx=96)     # strided x is fine
    torch.cuda.synchronize()


def test_mfma_large_m_unaligned_output_and_in_place_residual(qdiy):
    """m >= 512 with y rows an odd number of elements apart (the 64 x 64 tile
    takes it: the ring tiles store 8 bytes at a time) and with the residual
    added in place: both within the fp32 summation bound."""
    m, n, k = 640, 96, 256
    rng = np.random.default_rng(3)
    x, W, R = normal_f16(rng, (m, k)), normal_f16(rng, (n, k), 0.02), normal_f16(rng, (m, n))
    x64, W64 = x.astype(np.float64), W.astype(np.float64)
    s = x64 @ W64.T
    bound = k * 2.0 ** -23 * (np.abs(x64) @ np.abs(W64).T)
    ldy = n + 1
    y = torch.zeros(m * ldy, dtype=torch.float16, device="cuda")
    qdiy.gemm_nt(_dev(x.reshape(-1)), _dev(W.reshape(-1)), y, m, n, k, mode=qdiy.GEMM_MFMA, ldy=ldy)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(m, ldy)[:, :n].astype(np.float64)
    assert np.all(np.abs(got - s) <= ulp16(s) + bound)
    yr = _dev(R.reshape(-1))
    qdiy.gemm_nt(_dev(x.reshape(-1)), _dev(W.reshape(-1)), yr, m, n, k, residual=yr, mode=qdiy.GEMM_MFMA)
    torch.cuda.synchronize()
    got = yr.cpu().numpy().reshape(m, n).astype(np.float64)
    h = s.astype(np.float16).astype(np.float64)
    want = R.astype(np.float64) + h
    assert np.all(np.abs(got - want) <= ulp16(want) + ulp16(h) + bound + ulp16(s))


@pytest.mark.parametrize("hidden,inter,n_prompt", [(512, 1368, 100), (512, 1368, 300), (2048, 5504, 300),
                                                  (512, 1408, 700)])
def test_engine_mfma_prefill(qdiy, hidden, inter, n_prompt):
    """MFMA prefill against exact prefill on the same prompt (with c_proj exact
    where inter is not a multiple of 64): the next step's logits agree to the
    fp32-order difference, and plain decode steps are bit-identical in both
    modes.  At hidden 2048 and 299 tokens the o_proj and c_proj products have
    48 tiles of 128 x 128 and run split over K on that tile (engine workspace,
    then the fold launch); gate/up is one launch with the SwiGLU epilogue."""
    cfg = qdiy.model_cfg(vocab_size=512, hidden_size=hidden, num_layers=2, num_heads=hidden // 128,
                         intermediate_size=inter, max_seqlen=n_prompt + 20)
    img = qdiy.random_model_image(cfg, 41 + hidden, 0.03, nthreads=8)
    prompt = [int(t) for t in np.random.default_rng(hidden).integers(0, 512, n_prompt)]
    res, kv = {}, {}
    with qdiy.Engine(image=img) as eng:
        for mode in (qdiy.GEMM_EXACT, qdiy.GEMM_MFMA):
            eng.set_prefill_mode(mode)
            eng.reset()
            pos = eng.prefill(prompt[:-1])
            kv[mode] = [eng.kv_rows(layer, 0, pos) for layer in range(cfg.num_layers)]
            eng.step(prompt[-1], pos)
            prefilled = eng.logits().astype(np.float64)
            eng.reset()
            eng.step(prompt[0], 0)                     # no prefill: decode kernels only
            res[mode] = (prefilled, eng.logits())
    exact, mfma = res[qdiy.GEMM_EXACT], res[qdiy.GEMM_MFMA]
    assert _same(exact[1], mfma[1]), "decode steps must not depend on the prefill mode"
    d = np.abs(exact[0] - mfma[0])
    assert float(np.max(d)) <= 0.02 * float(np.max(np.abs(exact[0]))) + 0.01, float(np.max(d))
    assert float(np.corrcoef(exact[0], mfma[0])[0, 1]) > 0.999
    # The KV rows the prefill leaves, against a float64 recomputation of the prompt.
    n = len(prompt) - 1
    m = model_tensors(img)
    ref_k, ref_v, term_k, term_v = model_kv_fp64(m, prompt[:-1], terms=True)
    bad_k, _ = model_kv_fp64(m, prompt[:-1], mutate="rope_sign")
    kv_terms = {"K": term_k, "V": term_v}
    for layer in range(cfg.num_layers):
        for mode in (qdiy.GEMM_EXACT, qdiy.GEMM_MFMA):
            k, v = kv[mode][layer]
            for name, got, ref in (("K", k, ref_k[layer]), ("V", v, ref_v[layer])):
                err = np.abs(got.astype(np.float64) - ref)
                scale = np.max(np.abs(ref), axis=1, keepdims=True)
                if layer == 0:
                    # fp16 roundings of the normalised input, the QKV sums, the bias add and
                    # the rotation, each within an ulp of values at most the row's scale
                    tol = 4 * ulp16(scale) + 2.0 ** -10 * kv_terms[name][layer]
                else:
                    # plus what the first layer's fp16 activations and attention carry over
                    tol = 0.01 * scale
                assert np.all(err <= tol), (layer, mode, name, float(np.max(err - tol)))
        if layer == 0:
            k0 = kv[qdiy.GEMM_MFMA][0][0].astype(np.float64)
            assert np.mean(np.abs(k0 - bad_k[0]) > 4 * ulp16(np.max(np.abs(bad_k[0])))) > 0.3


def test_engine_mfma_prefill_two_passes(qdiy):
    """A 2300-token prompt: the MFMA mode runs it as passes of 2048 and 251 tokens (the
    second pass's attention starts at position 2048, over the first pass's KV rows), the
    exact mode as passes of 256. The next step's logits agree as above, and switching the
    mode back and forth keeps both working."""
    cfg = qdiy.model_cfg(vocab_size=512, hidden_size=512, num_layers=2, num_heads=4,
                         intermediate_size=1408, max_seqlen=2400)
    img = qdiy.random_model_image(cfg, 77, 0.03, nthreads=8)
    prompt = [int(t) for t in np.random.default_rng(2300).integers(0, 512, 2300)]
    logits = {}
    with qdiy.Engine(image=img) as eng:
        for mode in (qdiy.GEMM_MFMA, qdiy.GEMM_EXACT, qdiy.GEMM_MFMA):
            eng.set_prefill_mode(mode)
            eng.reset()
            pos = eng.prefill(prompt[:-1])
            assert pos == len(prompt) - 1
            eng.step(prompt[-1], pos)
            got = eng.logits().astype(np.float64)
            if mode in logits:
                assert _same(logits[mode], got), "the same mode must repeat bit for bit"
            logits[mode] = got
    exact, mfma = logits[qdiy.GEMM_EXACT], logits[qdiy.GEMM_MFMA]
    assert np.all(np.isfinite(mfma))
    d = np.abs(exact - mfma)
    assert float(np.max(d)) <= 0.02 * float(np.max(np.abs(exact))) + 0.01, float(np.max(d))
    assert float(np.corrcoef(exact, mfma)[0, 1]) > 0.999
