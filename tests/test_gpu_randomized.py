"""Randomized GPU parity.

Seeded random shapes, cache layouts, strides, offsets and launch variants for
decode attention and the decode-step ops, each checked bit for bit against
the oracle's restatement of the kernels' arithmetic (the same bar as the
fixed-shape tests).  Attention is also checked within one binary16 ulp of
float64.  The seeds are fixed, so a failure names a reproducible case.
"""
import numpy as np
import pytest
import torch

from common import normal_f16, ulp16
from oracle import oracle

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture(scope="module")
def qdiy():
    import qdiy as m
    torch.cuda.set_device(0)
    m.load()
    return m


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint16), np.asarray(b).view(np.uint16))


def _odd(n, fill=0.0):
    """A device fp16 view of n elements starting one element (2 bytes) into its buffer."""
    return torch.full((n + 1,), float(fill), dtype=torch.float16, device="cuda")[1:]


def _attn_fp64(q, k, v, L, H, rs, hs):
    out = np.empty((H, D))
    rows = np.arange(L)[:, None] * rs + np.arange(D)[None, :]
    for h in range(H):
        Kh = k[rows + h * hs].astype(np.float64)
        Vh = v[rows + h * hs].astype(np.float64)
        s = Kh @ q[h].astype(np.float64) / np.sqrt(128.0)
        p = np.exp(s - s.max())
        out[h] = p @ Vh / p.sum()
    return out


@pytest.mark.parametrize("seed", range(60))
def test_attention_random_shapes(qdiy, seed):
    rng = np.random.default_rng(70000 + seed)
    H = int(rng.integers(1, 25))
    L = int(rng.integers(1, 300) if rng.random() < 0.5 else rng.integers(300, 3000))
    S = L + int(rng.integers(0, 40))
    layout = ("engine", "head_major", "padded")[int(rng.integers(0, 3))]
    if layout == "engine":
        rs, hs = H * D, D
    elif layout == "head_major":
        rs, hs = D, S * D
    else:                                   # heads and rows padded apart
        hs = D + 8 * int(rng.integers(0, 4))
        rs = (H - 1) * hs + D + 8 * int(rng.integers(0, 33))
    n = (S - 1) * rs + (H - 1) * hs + D
    kscale = float(rng.uniform(0.1, 3.0))
    q = normal_f16(rng, (H, D))
    k = normal_f16(rng, n, kscale)
    v = normal_f16(rng, n)
    if rng.random() < 0.3:                  # rows aligned with q: logit spikes
        every = int(rng.integers(2, 50))
        for j in range(0, L, every):
            for h in range(H):
                k[j * rs + h * hs:j * rs + h * hs + D] = q[h]
    variant = ("auto", "fused", "split")[int(rng.integers(0, 3))]
    splits = int(rng.integers(1, min(L, 256) + 1)) if variant == "split" else 0
    with qdiy.Context(num_heads=H, max_seqlen=S, kv_row_stride=rs, kv_head_stride=hs) as ctx:
        out = torch.empty(H * D, dtype=torch.float16, device="cuda")
        ctx.decode_attention(torch.from_numpy(q.reshape(-1)).cuda(), torch.from_numpy(k).cuda(),
                             torch.from_numpy(v).cuda(), out, L, variant, splits)
        torch.cuda.synchronize()
        plan = ctx.plan_detail(L, variant, splits)
    got = out.cpu().numpy().reshape(H, D)
    want = oracle.attention_planned(q, k, v, L, H, rs, hs, oracle.Plan(*plan.as_tuple()), nthreads=8)
    case = f"H={H} L={L} S={S} {layout} rs={rs} hs={hs} kscale={kscale:.2f} {variant}/{splits} plan={plan.as_tuple()}"
    assert _same(got, want), case
    ref = _attn_fp64(q, k, v, L, H, rs, hs)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= ulp16(ref) + 1e-5), case


@pytest.mark.parametrize("seed", range(16))
def test_attention_random_long_lengths(qdiy, seed):
    """The automatic plan beyond 3072 rows: interleaved blocks (32 rows of 2-row
    tiles with the next tile in flight up to 16384 rows, 64 rows of 4-row tiles
    beyond) merged in the scan kernel where the head count is a multiple of the
    dispatch period, contiguous splits and a merge kernel otherwise (12 heads);
    random lengths up to 40000 rows, layouts and logit spikes, bit-exact against
    the oracle's restatement of the plan the library reports."""
    rng = np.random.default_rng(90000 + seed)
    H = (8, 16, 24, 12)[int(rng.integers(0, 4))]
    L = int(rng.integers(3000, 40000))
    S = L + int(rng.integers(0, 40))
    layout = ("engine", "head_major", "padded")[int(rng.integers(0, 3))]
    if layout == "engine":
        rs, hs = H * D, D
    elif layout == "head_major":
        rs, hs = D, S * D
    else:
        hs = D + 8 * int(rng.integers(0, 4))
        rs = (H - 1) * hs + D + 8 * int(rng.integers(0, 33))
    n = (S - 1) * rs + (H - 1) * hs + D
    kscale = float(rng.uniform(0.1, 1.5))
    q = normal_f16(rng, (H, D))
    k = normal_f16(rng, n, kscale)
    v = normal_f16(rng, n)
    if rng.random() < 0.4:                  # rows aligned with q: logit spikes
        every = int(rng.integers(50, 500))
        for j in range(int(rng.integers(0, every)), L, every):
            for h in range(H):
                k[j * rs + h * hs:j * rs + h * hs + D] = q[h]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    with qdiy.Context(num_heads=H, max_seqlen=S, kv_row_stride=rs, kv_head_stride=hs) as ctx:
        out = torch.empty(H * D, dtype=torch.float16, device="cuda")
        ctx.decode_attention(torch.from_numpy(q.reshape(-1)).cuda(), torch.from_numpy(k).cuda(),
                             torch.from_numpy(v).cuda(), out, L)
        torch.cuda.synchronize()
        plan = ctx.plan_detail(L)
        period = ctx.xcd_period()
    case = f"H={H} L={L} S={S} {layout} rs={rs} hs={hs} kscale={kscale:.2f} plan={plan.as_tuple()}"
    print(case, flush=True)
    if L > 3072 and period >= 1 and H % period == 0 and plan.num_splits * H <= cus:
        assert plan.block_rows == (32 if L <= 16384 else 64) and plan.merge_in_kernel == 1, case
    elif L > 3072:
        assert plan.block_rows == 0 and plan.merge_in_kernel == 0, case
    got = out.cpu().numpy().reshape(H, D)
    want = oracle.attention_planned(q, k, v, L, H, rs, hs, oracle.Plan(*plan.as_tuple()), nthreads=8)
    assert _same(got, want), case
    ref = _attn_fp64(q, k, v, L, H, rs, hs)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= ulp16(ref) + 1e-5), case


@pytest.mark.parametrize("seed", range(20))
def test_proj_residual_random_shapes(qdiy, seed):
    rng = np.random.default_rng(71000 + seed)
    K = 8 * int(rng.integers(1, 1025))
    N = int(rng.integers(1, 3000))
    x, W, res = normal_f16(rng, K), normal_f16(rng, N * K, 0.02), normal_f16(rng, N)
    want = oracle.proj_residual(x, W, res, N, K)
    in_place = rng.random() < 0.5
    g_res = _odd(N) if rng.random() < 0.5 else torch.empty(N, dtype=torch.float16, device="cuda")
    g_res.copy_(torch.from_numpy(res))
    g_out = g_res if in_place else _odd(N)
    qdiy.proj_residual(torch.from_numpy(x).cuda(), torch.from_numpy(W).cuda(), g_res, g_out, N, K)
    torch.cuda.synchronize()
    assert _same(g_out.cpu().numpy(), want), f"N={N} K={K} in_place={in_place}"


@pytest.mark.parametrize("seed", range(20))
def test_ffn_up_random_shapes(qdiy, seed):
    rng = np.random.default_rng(72000 + seed)
    hid = 512 * int(rng.integers(1, 9))
    inter = int(rng.integers(1, 3000))
    x = normal_f16(rng, hid)
    nw = (1.0 + normal_f16(rng, hid, 0.1).astype(np.float32)).astype(np.float16)
    W1, W2 = normal_f16(rng, inter * hid, 0.02), normal_f16(rng, inter * hid, 0.02)
    want = oracle.ffn_up_swiglu(x, nw, W1, W2, hid, inter)
    act = _odd(inter) if rng.random() < 0.5 else torch.empty(inter, dtype=torch.float16, device="cuda")
    qdiy.ffn_up_swiglu(torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda(), torch.from_numpy(W1).cuda(),
                       torch.from_numpy(W2).cuda(), act, hid, inter)
    torch.cuda.synchronize()
    assert _same(act.cpu().numpy(), want), f"hidden={hid} inter={inter}"


@pytest.mark.parametrize("seed", range(20))
def test_lm_head_argmax_random_shapes(qdiy, seed):
    rng = np.random.default_rng(73000 + seed)
    hid = 512 * int(rng.integers(1, 9))
    V = int(rng.integers(1, 6000))
    x = normal_f16(rng, hid)
    nw = (1.0 + normal_f16(rng, hid, 0.1).astype(np.float32)).astype(np.float16)
    W = normal_f16(rng, V * hid, 0.02)
    if rng.random() < 0.3 and V > 1:         # plant an exact tie for the maximum
        r = int(rng.integers(1, V))
        W[r * hid:(r + 1) * hid] = W[0:hid]
    tok_want, logits_want = oracle.lm_head_argmax(x, nw, W, V, hid)
    logits = _odd(V) if rng.random() < 0.5 else torch.empty(V, dtype=torch.float16, device="cuda")
    ws = torch.empty(max(1, qdiy.lm_head_workspace_bytes(V) // 8), dtype=torch.int64, device="cuda")
    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    qdiy.lm_head_argmax(torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda(), torch.from_numpy(W).cuda(),
                        logits, V, hid, ws, tok)
    torch.cuda.synchronize()
    case = f"V={V} hidden={hid}"
    assert _same(logits.cpu().numpy(), logits_want), case
    assert int(tok.item()) == tok_want, case


@pytest.mark.parametrize("seed", range(20))
def test_qkv_front_random_shapes(qdiy, seed):
    rng = np.random.default_rng(74000 + seed)
    H = 4 * int(rng.integers(1, 9))          # hidden 512 .. 4096
    hid = H * D
    S = int(rng.integers(1, 200))
    pos = int(rng.integers(0, S))
    with_norm, with_bias = bool(rng.random() < 0.5), bool(rng.random() < 0.7)
    x, W = normal_f16(rng, hid), normal_f16(rng, 3 * hid * hid, 0.02).reshape(3 * hid, hid)
    b = normal_f16(rng, 3 * hid, 0.02)
    nw = (1.0 + normal_f16(rng, hid, 0.1).astype(np.float32)).astype(np.float16)
    o_qkv = np.zeros(3 * hid, np.float16)
    o_k = np.full(S * hid, np.float16(-2.5), np.float16)
    o_v = o_k.copy()
    oracle.qkv_front(x, nw if with_norm else None, W, b if with_bias else None, o_qkv, o_k, o_v, pos, H)
    g_b = None
    if with_bias:
        g_b = _odd(3 * hid) if rng.random() < 0.5 else torch.empty(3 * hid, dtype=torch.float16, device="cuda")
        g_b.copy_(torch.from_numpy(b))
    g_qkv = torch.zeros(3 * hid, dtype=torch.float16, device="cuda")
    g_k = torch.full((S * hid,), -2.5, dtype=torch.float16, device="cuda")
    g_v = g_k.clone()
    with qdiy.Context(num_heads=H, max_seqlen=S) as ctx:
        ctx.qkv_proj_rope_cache(torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda() if with_norm else None,
                                torch.from_numpy(W).cuda(), g_b, g_qkv, g_k, g_v, pos)
        torch.cuda.synchronize()
    case = f"H={H} S={S} pos={pos} norm={with_norm} bias={with_bias}"
    for name, w, g in zip(("qkv", "k_cache", "v_cache"), (o_qkv, o_k, o_v), (g_qkv, g_k, g_v)):
        assert _same(w, g.cpu().numpy()), f"{name}: {case}"


def _engine_plans(qdiy, cfg, n):
    """The engine's attention plans at lengths 1..n (its context has the same
    heads, cache layout and device, hence the same planner decisions)."""
    with qdiy.Context(num_heads=cfg.num_heads, max_seqlen=cfg.max_seqlen,
                      kv_row_stride=cfg.hidden_size, kv_head_stride=D) as ctx:
        return [oracle.Plan(*ctx.plan_detail(L).as_tuple()) for L in range(1, n + 1)]


@pytest.mark.parametrize("seed", range(6))
def test_engine_random_models(qdiy, seed):
    """Random model shapes and prompt lengths, some crossing the fused/split
    boundary (224 rows) and the 256-token prefill chunk: greedy tokens and the
    last step's logits equal the oracle's."""
    rng = np.random.default_rng(75000 + seed)
    heads = 4 * int(rng.integers(1, 3))
    n_prompt = int(rng.integers(1, 41) if rng.random() < 0.5 else rng.integers(200, 301))
    n_new = int(rng.integers(4, 13))
    cfg = qdiy.model_cfg(vocab_size=int(rng.integers(50, 3000)), hidden_size=heads * D,
                         num_layers=int(rng.integers(1, 3)), num_heads=heads,
                         intermediate_size=8 * int(rng.integers(16, 257)),
                         max_seqlen=n_prompt + n_new + int(rng.integers(0, 20)))
    img = qdiy.random_model_image(cfg, 1000 + seed, float(rng.uniform(0.02, 0.1)))
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, n_prompt)]
    with qdiy.Engine(image=img) as eng:
        got = eng.generate(prompt, n_new, stop_at_eos=False)
        got_logits = eng.logits()
    want, want_logits = oracle.generate(img, prompt, n_new, _engine_plans(qdiy, cfg, n_prompt + n_new))
    case = (f"heads={heads} layers={cfg.num_layers} inter={cfg.intermediate_size} "
            f"vocab={cfg.vocab_size} prompt={n_prompt} new={n_new}")
    assert got == want, case
    assert _same(got_logits, want_logits), case
