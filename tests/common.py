"""Shared input builders and fp64 references for the parity tests.

Inputs are drawn from numpy's PCG64 generator (portable across platforms for a
given numpy version) in float32 and rounded to fp16 with numpy's RNE cast.
"""
from __future__ import annotations

import numpy as np

D = 128


def normal_f16(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    x = rng.standard_normal(size=shape, dtype=np.float32)
    if scale != 1.0:
        x *= np.float32(scale)
    return x.astype(np.float16)


def ulp16(x) -> np.ndarray:
    """Spacing of binary16 at |x| (2^-24 in the subnormal range)."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.where(a < 2.0 ** -14, 2.0 ** -24, 2.0 ** (e - 10))


def attn_fp64(q: np.ndarray, K: np.ndarray, V: np.ndarray) -> np.ndarray:
    """Textbook q=1 attention in float64: softmax(K q / sqrt(128)) V."""
    s = K.astype(np.float64) @ q.astype(np.float64) / np.sqrt(128.0)
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ V.astype(np.float64)


class AttnCase:
    """Q [H,128] and K/V for H heads x L rows, stored in a cache layout.

    layout "engine": the reference engine's [pos][head*128] rows
    (qwen_infer.cu:75-76, row stride H*128, head stride 128), with
    max_seqlen >= L rows allocated.  layout "head_major": [head][max_seqlen][128]
    (row stride 128, head stride max_seqlen*128).
    """

    def __init__(self, L, H=16, seed=0, kscale=1.0, spike_every=0, layout="engine",
                 max_seqlen=None, fill=None):
        self.L, self.H = L, H
        self.max_seqlen = max_seqlen or L
        rng = np.random.default_rng(seed)
        if fill is not None:
            self.q = np.full((H, D), fill, np.float16)
            Kh = np.full((H, L, D), fill, np.float16)
            Vh = np.full((H, L, D), fill, np.float16)
        else:
            self.q = normal_f16(rng, (H, D))
            Kh = normal_f16(rng, (H, L, D), kscale)
            Vh = normal_f16(rng, (H, L, D))
        if spike_every:
            # adversarial logit spike: every spike_every-th key equals Q
            Kh[:, ::spike_every, :] = self.q[:, None, :]
        self.Kh, self.Vh = Kh, Vh
        self.layout = layout
        S = self.max_seqlen
        if layout == "engine":
            self.row_stride, self.head_stride = H * D, D
            kc = np.zeros((S, H, D), np.float16)
            vc = np.zeros((S, H, D), np.float16)
            kc[:L] = Kh.transpose(1, 0, 2)
            vc[:L] = Vh.transpose(1, 0, 2)
        elif layout == "head_major":
            self.row_stride, self.head_stride = D, S * D
            kc = np.zeros((H, S, D), np.float16)
            vc = np.zeros((H, S, D), np.float16)
            kc[:, :L] = Kh
            vc[:, :L] = Vh
        else:
            raise ValueError(layout)
        self.kc = np.ascontiguousarray(kc).reshape(-1)
        self.vc = np.ascontiguousarray(vc).reshape(-1)

    def fp64(self) -> np.ndarray:
        return np.stack([attn_fp64(self.q[h], self.Kh[h], self.Vh[h]) for h in range(self.H)])


# ----------------------------------------------------------------- .bin images

MODEL_MAGIC = 0x46445751


def model_tensors(image: np.ndarray) -> dict:
    """Views of every tensor of a .bin image (convert_weights.py:105-185):
    header (7 x uint32), wte, per-layer [ln_1, qkv_w, qkv_b, attn_proj_w,
    ln_2, ffn_w1, ffn_w2, ffn_proj_w], ln_f, lm_head."""
    hdr = np.frombuffer(image[:28].tobytes(), np.uint32)
    assert hdr[0] == MODEL_MAGIC
    V, H, NL, NH, I, S = (int(v) for v in hdr[1:])
    t = image[28:].view(np.float16)
    o = 0

    def take(*shape):
        nonlocal o
        n = int(np.prod(shape))
        a = t[o:o + n].reshape(shape)
        o += n
        return a

    m = {"cfg": dict(vocab=V, hidden=H, layers=NL, heads=NH, inter=I, max_seqlen=S)}
    m["wte"] = take(V, H)
    m["layers"] = []
    for _ in range(NL):
        m["layers"].append({"ln_1": take(H), "qkv_w": take(3 * H, H), "qkv_b": take(3 * H),
                            "proj_w": take(H, H), "ln_2": take(H), "w1": take(I, H),
                            "w2": take(I, H), "w_down": take(H, I)})
    m["ln_f"] = take(H)
    m["lm_head"] = take(V, H)
    assert o == t.size
    return m


def model_logits_fp64(m: dict, tokens, rope_base: float = 10000.0, mutate: str = "") -> np.ndarray:
    """Textbook float64 forward of the Qwen decoder over `tokens` (positions
    0..n-1, one at a time with a KV cache); returns the last token's logits.
    RMSNorm, fused QKV + bias, rotate-half RoPE on pairs (i, i+64), softmax
    attention per head, SwiGLU w1 * silu(w2), residual adds, final norm and
    lm_head.  `mutate` plants one mistake (for tests of the comparison)."""
    c = m["cfg"]
    H, NH, D = c["hidden"], c["heads"], 128
    f = lambda a: a.astype(np.float64)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + 1e-6) * f(w)

    inv = rope_base ** (-np.arange(64) * 2.0 / D)
    Ks = [[] for _ in range(c["layers"])]
    Vs = [[] for _ in range(c["layers"])]
    for pos, tok in enumerate(tokens):
        x = f(m["wte"][tok])
        th = pos * inv
        cs, sn = np.cos(th), np.sin(th)
        if mutate == "rope_sign":
            sn = -sn
        for l, L in enumerate(m["layers"]):
            qkv = f(L["qkv_w"]) @ rms(x, L["ln_1"]) + f(L["qkv_b"])
            q, k, v = (qkv[i * H:(i + 1) * H].reshape(NH, D) for i in range(3))

            def rot(a):
                a1, a2 = a[:, :64], a[:, 64:]
                return np.concatenate([a1 * cs - a2 * sn, a2 * cs + a1 * sn], axis=1)

            q, k = rot(q), rot(k)
            Ks[l].append(k)
            Vs[l].append(v)
            K, V = np.stack(Ks[l], 1), np.stack(Vs[l], 1)          # [NH, n, D]
            s = np.einsum("hd,hnd->hn", q, K) / np.sqrt(D)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            a = np.einsum("hn,hnd->hd", p, V).reshape(-1)
            x = x + f(L["proj_w"]) @ a
            xn = rms(x, L["ln_2"])
            g, u = f(L["w1"]) @ xn, f(L["w2"]) @ xn
            if mutate == "swap_gate_up":
                g, u = u, g
            x = x + f(L["w_down"]) @ (g * u / (1.0 + np.exp(-u)))
    return f(m["lm_head"]) @ rms(x, m["ln_f"])


def model_kv_fp64(m: dict, tokens, rope_base: float = 10000.0, mutate: str = "", terms: bool = False):
    """Float64 K (rotated) and V cache rows of every layer for `tokens` at
    positions 0..n-1, all positions at once with a causal mask (the same
    textbook forward as model_logits_fp64): lists over layers of [n][hidden].
    With terms=True also each element's sum of |addends| (|xn| |W| + |b|, the
    two rotated halves' added for K), for rounding bounds."""
    c = m["cfg"]
    H, NH, D = c["hidden"], c["heads"], 128
    f = lambda a: a.astype(np.float64)
    n = len(tokens)
    X = f(m["wte"][np.asarray(tokens)])                               # [n, H]

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6) * f(w)

    inv = rope_base ** (-np.arange(64) * 2.0 / D)
    th = np.arange(n)[:, None] * inv[None, :]
    cs, sn = np.cos(th)[:, None, :], np.sin(th)[:, None, :]           # [n, 1, 64]
    if mutate == "rope_sign":
        sn = -sn

    def rot(a):                                                       # [n, NH, D]
        a1, a2 = a[..., :64], a[..., 64:]
        return np.concatenate([a1 * cs - a2 * sn, a2 * cs + a1 * sn], axis=-1)

    Ks, Vs, TK, TV = [], [], [], []
    causal = np.triu(np.ones((n, n), bool), 1)
    for L in m["layers"]:
        xn = rms(X, L["ln_1"])
        W, b = f(L["qkv_w"]), f(L["qkv_b"])
        qkv = xn @ W.T + b
        q, k, v = (qkv[:, i * H:(i + 1) * H].reshape(n, NH, D) for i in range(3))
        q, k = rot(q), rot(k)
        Ks.append(k.reshape(n, H))
        Vs.append(v.reshape(n, H))
        if terms:
            t = np.abs(xn) @ np.abs(W).T + np.abs(b)
            tk = t[:, H:2 * H].reshape(n, NH, D)
            tk = np.concatenate([tk[..., :64] + tk[..., 64:]] * 2, axis=-1)
            TK.append(tk.reshape(n, H))
            TV.append(t[:, 2 * H:])
        s = np.einsum("ihd,jhd->hij", q, k) / np.sqrt(D)
        s[:, causal] = -np.inf
        p = np.exp(s - s.max(axis=2, keepdims=True))
        p /= p.sum(axis=2, keepdims=True)
        a = np.einsum("hij,jhd->ihd", p, v).reshape(n, H)
        X = X + a @ f(L["proj_w"]).T
        xn2 = rms(X, L["ln_2"])
        g, u = xn2 @ f(L["w1"]).T, xn2 @ f(L["w2"]).T
        X = X + (g * u / (1.0 + np.exp(-u))) @ f(L["w_down"]).T
    return (Ks, Vs, TK, TV) if terms else (Ks, Vs)
