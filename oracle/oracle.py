"""ctypes wrapper of the CPU oracle (oracle/libqd_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.  fp16 arrays are
numpy float16 (their uint16 bit patterns cross the C boundary unchanged).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqd_oracle.so")

ENGINE, FUSED, SPLIT = 0, 1, 2

_lib = None


class Plan(ctypes.Structure):
    """qd_oracle_plan: the launch plan of one decode-attention call."""
    _fields_ = [("variant", ctypes.c_int), ("num_splits", ctypes.c_int),
                ("rows_per_split", ctypes.c_int), ("rows_per_tile", ctypes.c_int),
                ("waves", ctypes.c_int), ("block_rows", ctypes.c_int)]

    def __repr__(self):
        return (f"Plan(variant={self.variant}, num_splits={self.num_splits}, rows_per_split="
                f"{self.rows_per_split}, rows_per_tile={self.rows_per_tile}, waves={self.waves}, "
                f"block_rows={self.block_rows})")


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        f32p = ctypes.POINTER(ctypes.c_float)
        ll = ctypes.c_longlong
        L.qd_oracle_h2f_array.argtypes = [u16p, f32p, ll]
        L.qd_oracle_f2h_array.argtypes = [f32p, u16p, ll]
        L.qd_oracle_fd_fused_head.argtypes = [u16p, u16p, u16p, u16p, ctypes.c_int, ll,
                                              ctypes.c_int, ctypes.c_int]
        L.qd_oracle_fd_split_head.argtypes = [u16p, u16p, u16p, u16p, ctypes.c_int, ll,
                                              ctypes.c_int, ctypes.c_int, u16p, f32p]
        L.qd_oracle_decode_attention.argtypes = [u16p, u16p, u16p, u16p, ctypes.c_int,
                                                 ctypes.c_int, ll, ll, ctypes.c_int,
                                                 ctypes.c_int]
        L.qd_oracle_decode_attention.restype = ctypes.c_int
        L.qd_oracle_qkv_bias_rope_cache.argtypes = [u16p, u16p, u16p, u16p, ctypes.c_int,
                                                    ctypes.c_int, ctypes.c_int, ll, ll,
                                                    ctypes.c_float]
        L.qd_oracle_qkv_bias_rope_cache.restype = ctypes.c_int
        L.qd_oracle_rope_cos_sin.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_float, f32p, f32p]
        L.qd_oracle_wave64_sum.argtypes = [f32p]
        L.qd_oracle_wave64_sum.restype = ctypes.c_float
        L.qd_oracle_rmsnorm.argtypes = [u16p, u16p, ctypes.c_int, ctypes.c_float, u16p, ctypes.c_int]
        L.qd_oracle_gemv.argtypes = [u16p, u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, u16p]
        L.qd_oracle_qkv_front.argtypes = [u16p, u16p, ctypes.c_float, u16p, u16p, u16p, u16p,
                                          u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ll, ll,
                                          ctypes.c_float, ctypes.c_int]
        L.qd_oracle_qkv_front.restype = ctypes.c_int
        L.qd_oracle_exp2_array.argtypes = [f32p, f32p, ll]
        vp, i = ctypes.c_void_p, ctypes.c_int
        L.qd_oracle_proj_residual.argtypes = [u16p, u16p, u16p, u16p, i, i, i]
        L.qd_oracle_swiglu.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        L.qd_oracle_swiglu.restype = ctypes.c_uint16
        L.qd_oracle_ffn_up_swiglu.argtypes = [u16p, u16p, ctypes.c_float, u16p, u16p, u16p, i, i, i]
        L.qd_oracle_lm_head_argmax.argtypes = [u16p, u16p, ctypes.c_float, u16p, u16p, i, i, i]
        L.qd_oracle_lm_head_argmax.restype = i
        L.qd_oracle_generate.argtypes = [vp, ll, ctypes.POINTER(i), i, i, i, ctypes.POINTER(Plan), i,
                                         ctypes.POINTER(i), ctypes.POINTER(i), u16p, i]
        L.qd_oracle_generate.restype = i
        L.qd_oracle_model_new.argtypes = [vp, ll, i, i]
        L.qd_oracle_model_new.restype = vp
        L.qd_oracle_model_new_order.argtypes = [vp, ll, i, i, i]
        L.qd_oracle_model_new_order.restype = vp
        L.qd_oracle_swiglu_ref.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        L.qd_oracle_swiglu_ref.restype = ctypes.c_uint16
        L.qd_oracle_argmax_ref.argtypes = [u16p, i]
        L.qd_oracle_argmax_ref.restype = i
        L.qd_oracle_model_free.argtypes = [vp]
        L.qd_oracle_model_forward.argtypes = [vp, i, i, ctypes.POINTER(Plan), i, u16p]
        L.qd_oracle_model_forward.restype = i
        L.qd_oracle_attention_planned.argtypes = [u16p, u16p, u16p, u16p, ctypes.c_int,
                                                  ctypes.c_int, ll, ll,
                                                  ctypes.POINTER(Plan), ctypes.c_int]
        L.qd_oracle_attention_planned.restype = ctypes.c_int
        _lib = L
    return _lib


def _u16(a: np.ndarray):
    assert a.dtype == np.float16 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def _f32(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def h2f(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.float16)
    out = np.empty(h.shape, np.float32)
    lib().qd_oracle_h2f_array(_u16(h), _f32(out), h.size)
    return out


def f2h(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.float16)
    lib().qd_oracle_f2h_array(_f32(f), _u16(out), f.size)
    return out


def fd_fused_head(q, k, v, seqlen, row_stride, rows_per_warp=32, num_warps=None):
    """One head of fd_v5_fused_kernel; k/v are flat fp16 arrays."""
    if num_warps is None:
        num_warps = min(32, (seqlen + rows_per_warp - 1) // rows_per_warp)
    out = np.zeros(128, np.float16)
    lib().qd_oracle_fd_fused_head(_u16(q), _u16(k), _u16(v), _u16(out), seqlen, row_stride,
                                  rows_per_warp, num_warps)
    return out


def fd_split_head(q, k, v, seqlen, row_stride, chunk=256, warps=8):
    """One head of split stage 1 + stage 2; returns (out, partial, lse)."""
    n = (seqlen + chunk - 1) // chunk
    out = np.zeros(128, np.float16)
    part = np.zeros((n, 128), np.float16)
    lse = np.zeros(n, np.float32)
    lib().qd_oracle_fd_split_head(_u16(q), _u16(k), _u16(v), _u16(out), seqlen, row_stride,
                                  chunk, warps, _u16(part), _f32(lse))
    return out, part, lse


def decode_attention(q, k, v, seqlen, num_heads, row_stride, head_stride,
                     variant=ENGINE, nthreads=1):
    """All heads: q [H,128] fp16, k/v flat fp16 caches; returns out [H,128]."""
    q = np.ascontiguousarray(q, dtype=np.float16)
    out = np.zeros((num_heads, 128), np.float16)
    rc = lib().qd_oracle_decode_attention(_u16(q), _u16(k), _u16(v), _u16(out), seqlen,
                                          num_heads, row_stride, head_stride, variant,
                                          nthreads)
    if rc != 0:
        raise ValueError("qd_oracle_decode_attention rejected its arguments")
    return out


def qkv_bias_rope_cache(qkv, bias, k_cache, v_cache, pos, num_heads, head_dim=128,
                        row_stride=None, head_stride=None, rope_base=10000.0):
    """In place on qkv / k_cache / v_cache (numpy fp16, flat)."""
    if row_stride is None:
        row_stride = num_heads * head_dim
    if head_stride is None:
        head_stride = head_dim
    rc = lib().qd_oracle_qkv_bias_rope_cache(_u16(qkv), None if bias is None else _u16(bias),
                                             _u16(k_cache), _u16(v_cache), pos, num_heads,
                                             head_dim, row_stride, head_stride, rope_base)
    if rc != 0:
        raise ValueError("qd_oracle_qkv_bias_rope_cache rejected its arguments")


def rope_cos_sin(pos, i, head_dim=128, rope_base=10000.0):
    c = ctypes.c_float()
    s = ctypes.c_float()
    lib().qd_oracle_rope_cos_sin(pos, i, head_dim, rope_base, ctypes.byref(c), ctypes.byref(s))
    return np.float32(c.value), np.float32(s.value)


ORDER_REF, ORDER_WAVE64 = 0, 1


def wave64_sum(lanes) -> np.float32:
    a = np.ascontiguousarray(lanes, dtype=np.float32)
    assert a.size == 64
    return np.float32(lib().qd_oracle_wave64_sum(_f32(a)))


def rmsnorm(x, w, eps=1e-6, order=ORDER_REF):
    x = np.ascontiguousarray(x, dtype=np.float16)
    w = np.ascontiguousarray(w, dtype=np.float16)
    out = np.zeros_like(x)
    lib().qd_oracle_rmsnorm(_u16(x), _u16(w), x.size, eps, _u16(out), order)
    return out


def gemv(x, W, N, K, layout=0, order=ORDER_REF):
    """out[n] = half(sum_k x[k] W(n,k)); layout 0: W[n*K+k], 1: W[k*N+n]."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    W = np.ascontiguousarray(W, dtype=np.float16)
    out = np.zeros(N, np.float16)
    lib().qd_oracle_gemv(_u16(x), _u16(W), N, K, layout, order, _u16(out))
    return out


def qkv_front(x, norm_w, w_qkv, bias, qkv_out, k_cache, v_cache, pos, num_heads,
              eps=1e-6, head_dim=128, row_stride=None, head_stride=None, rope_base=10000.0,
              order=ORDER_WAVE64):
    """RMSNorm (optional) + QKV GEMV + bias + RoPE + cache append, in place on the outputs."""
    if row_stride is None:
        row_stride = num_heads * head_dim
    if head_stride is None:
        head_stride = head_dim
    rc = lib().qd_oracle_qkv_front(_u16(x), None if norm_w is None else _u16(norm_w), eps,
                                   _u16(w_qkv), None if bias is None else _u16(bias),
                                   _u16(qkv_out), _u16(k_cache), _u16(v_cache), pos, num_heads,
                                   head_dim, row_stride, head_stride, rope_base, order)
    if rc != 0:
        raise ValueError("qd_oracle_qkv_front rejected its arguments")


def exp2(x) -> np.ndarray:
    """exp2_rep of the gfx950 kernels, elementwise on float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().qd_oracle_exp2_array(_f32(x), _f32(out), x.size)
    return out


def fused_plan(seqlen, rows_per_tile=4, waves=16) -> Plan:
    return Plan(0, 1, seqlen, rows_per_tile, waves)


def split_plan(seqlen, num_splits, rows_per_tile=None, waves=4) -> Plan:
    """A split plan laid out as the library's planner lays one out for an
    explicit split count: rows per split rounded up to a multiple of 4."""
    rows = -(-seqlen // num_splits)
    rows = (rows + 3) & ~3
    if rows_per_tile is None:
        rows_per_tile = 4 if rows >= 64 else 2
    return Plan(1, -(-seqlen // rows), rows, rows_per_tile, waves)


def interleaved_plan(seqlen, num_splits, rows_per_tile=2, waves=8) -> Plan:
    """A split plan whose rows form blocks of one load round (waves * 4 *
    rows_per_tile rows) dealt to the splits in turn; at most one split per
    block.  rows_per_split is split 0's row count (the largest)."""
    block = waves * 4 * rows_per_tile
    splits = max(1, min(num_splits, -(-seqlen // block)))
    full, rem = divmod(seqlen, block)
    nfull = (full - 1) // splits + 1 if full > 0 else 0
    rows0 = nfull * block + (rem if rem > 0 and full % splits == 0 else 0)
    return Plan(1, splits, rows0, rows_per_tile, waves, block)


def attention_planned(q, k, v, seqlen, num_heads, row_stride, head_stride, plan, nthreads=1):
    """The gfx950 kernels' arithmetic for all heads under `plan`; out [H,128]."""
    q = np.ascontiguousarray(q, dtype=np.float16)
    out = np.zeros((num_heads, 128), np.float16)
    rc = lib().qd_oracle_attention_planned(_u16(q), _u16(k), _u16(v), _u16(out), seqlen,
                                           num_heads, row_stride, head_stride,
                                           ctypes.byref(plan), nthreads)
    if rc != 0:
        raise ValueError(f"qd_oracle_attention_planned rejected its arguments ({plan})")
    return out


# ------------------------------------------------------- decode step, model

def proj_residual(x, W, residual, n_out, k_in, nthreads=4):
    """out[n] = half(residual[n] + half(W[n] . x)); W flat [n_out*k_in]."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    W = np.ascontiguousarray(W, dtype=np.float16)
    out = np.ascontiguousarray(residual, dtype=np.float16).copy()
    lib().qd_oracle_proj_residual(_u16(x), _u16(W), _u16(out), _u16(out), n_out, k_in, nthreads)
    return out


def swiglu(g, u) -> np.float16:
    r = lib().qd_oracle_swiglu(int(np.float16(g).view(np.uint16)), int(np.float16(u).view(np.uint16)))
    return np.uint16(r).view(np.float16)


def swiglu_ref(g, u) -> np.float16:
    """The reference's SwiGLU of two fp16 scalars (swiglu.cuh:11-13, expf)."""
    r = lib().qd_oracle_swiglu_ref(int(np.float16(g).view(np.uint16)), int(np.float16(u).view(np.uint16)))
    return np.uint16(r).view(np.float16)


def argmax_ref(logits) -> int:
    """argmax_kernel's token for fp16 logits, its tie order included."""
    lg = np.ascontiguousarray(logits, dtype=np.float16)
    return lib().qd_oracle_argmax_ref(_u16(lg), lg.size)


def ffn_up_swiglu(x, norm_w, W1, W2, hidden, inter, eps=1e-6, nthreads=4):
    x = np.ascontiguousarray(x, dtype=np.float16)
    norm_w = np.ascontiguousarray(norm_w, dtype=np.float16)
    W1 = np.ascontiguousarray(W1, dtype=np.float16)
    W2 = np.ascontiguousarray(W2, dtype=np.float16)
    act = np.zeros(inter, np.float16)
    lib().qd_oracle_ffn_up_swiglu(_u16(x), _u16(norm_w), eps, _u16(W1), _u16(W2), _u16(act),
                                  hidden, inter, nthreads)
    return act


def lm_head_argmax(x, norm_w, W, vocab, hidden, eps=1e-6, nthreads=4):
    """(token, logits[vocab] fp16)."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    norm_w = np.ascontiguousarray(norm_w, dtype=np.float16)
    W = np.ascontiguousarray(W, dtype=np.float16)
    logits = np.zeros(vocab, np.float16)
    t = lib().qd_oracle_lm_head_argmax(_u16(x), _u16(norm_w), eps, _u16(W), _u16(logits), vocab,
                                       hidden, nthreads)
    return t, logits


def generate(image, prompt, n_new, plans, stop_at_eos=False, nthreads=8):
    """Greedy tokens of the model in the .bin image (uint8 array); plans[L-1] is
    the attention plan at length L.  Returns (tokens, last_logits)."""
    img = np.ascontiguousarray(image).view(np.uint8)
    vocab = int(np.frombuffer(img[:28].tobytes(), np.uint32)[1])
    pr = (ctypes.c_int * len(prompt))(*prompt)
    pl = (Plan * len(plans))(*plans)
    out = (ctypes.c_int * max(1, n_new))()
    n = ctypes.c_int()
    logits = np.zeros(vocab, np.float16)
    rc = lib().qd_oracle_generate(img.ctypes.data_as(ctypes.c_void_p), img.size, pr, len(prompt),
                                  n_new, int(stop_at_eos), pl, len(plans), out, ctypes.byref(n),
                                  _u16(logits), nthreads)
    if rc != 0:
        raise ValueError("qd_oracle_generate rejected its arguments")
    return list(out[:n.value]), logits


class Model:
    """Stateful oracle model over a .bin image: forward(token, pos, plan).  order
    ORDER_WAVE64 restates this build's kernels (plan: the library's attention
    plan at length pos + 1); ORDER_REF the reference kernels' own arithmetic
    (the plan is not used)."""

    def __init__(self, image, max_pos, nthreads=8, order=None):
        self._img = np.ascontiguousarray(image).view(np.uint8)       # kept alive
        self.vocab = int(np.frombuffer(self._img[:28].tobytes(), np.uint32)[1])
        order = ORDER_WAVE64 if order is None else order
        self._h = lib().qd_oracle_model_new_order(self._img.ctypes.data_as(ctypes.c_void_p),
                                                  self._img.size, max_pos, nthreads, order)
        if not self._h:
            raise ValueError("qd_oracle_model_new rejected its arguments")

    def forward(self, token, pos, plan=None, want_logits=True):
        """Next token and logits (want_logits) or None."""
        logits = np.zeros(self.vocab, np.float16) if want_logits else None
        r = lib().qd_oracle_model_forward(self._h, int(token), pos,
                                          None if plan is None else ctypes.byref(plan),
                                          int(want_logits), _u16(logits) if want_logits else None)
        if r < 0:
            raise ValueError("qd_oracle_model_forward rejected its arguments")
        return (r, logits) if want_logits else None

    def close(self):
        if self._h:
            lib().qd_oracle_model_free(self._h)
            self._h = None

    def __del__(self):
        self.close()
