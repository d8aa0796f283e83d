"""TEST INFRASTRUCTURE ONLY: numpy/ctypes front end of the C++ CPU oracle (attn_oracle.cpp).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, as the checker or as the
timed CPU baseline. Nothing in the product (dgx-serving_amd/) imports it.

Every function follows the reference file:line named in attn_oracle.cpp. Pinning (which check fixes each
function) is listed in tests/test_oracle.py.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I, F, U16, U32, U64, S = (ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_uint16, ctypes.c_uint32,
                                     ctypes.c_uint64, ctypes.c_size_t)
        L.oracle_f32_to_f16.argtypes = [F]; L.oracle_f32_to_f16.restype = U16
        L.oracle_f16_to_f32.argtypes = [U16]; L.oracle_f16_to_f32.restype = F
        L.oracle_f32_to_bf16.argtypes = [F]; L.oracle_f32_to_bf16.restype = U16
        L.oracle_bf16_to_f32.argtypes = [U16]; L.oracle_bf16_to_f32.restype = F
        for n in ("oracle_round_f16", "oracle_round_bf16"):
            getattr(L, n).argtypes = [P, P, P, S]; getattr(L, n).restype = None
        for n in ("oracle_gen_lcg", "oracle_gen_lcg24", "oracle_gen_lcg16"):
            getattr(L, n).argtypes = [P, P, S]; getattr(L, n).restype = None
        L.oracle_gen_xorshift.argtypes = [P, P, S]; L.oracle_gen_xorshift.restype = None
        L.oracle_gen_normal.argtypes = [U64, U64, F, F, P, S]; L.oracle_gen_normal.restype = None
        L.oracle_gen_uniform_int.argtypes = [U64, I, I, P, I]; L.oracle_gen_uniform_int.restype = None
        L.oracle_tree_anc.argtypes = [P, I, P]; L.oracle_tree_anc.restype = I
        L.oracle_tree_kw.argtypes = [I, I, P, P]; L.oracle_tree_kw.restype = I
        L.oracle_tree_random.argtypes = [U64, I, I, I, P, P]; L.oracle_tree_random.restype = I
        L.oracle_attention.argtypes = [P, P, P, P, P, P, P, I, I, I, I, F, I, I, P, P, I]
        L.oracle_attention.restype = I
        L.oracle_attention_split.argtypes = [P, P, P, P, P, I, I, I, I, F, I, I, P, P]
        L.oracle_attention_split.restype = I
        L.oracle_norm_rope.argtypes = [P, P, I, I, F, P, P, P, I, P]
        L.oracle_norm_rope.restype = I
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ rounding
def round_f16(x):
    """RN-even fp32 -> f16 (values as fp32, bits as uint16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    vals = np.empty_like(x); bits = np.empty(x.shape, np.uint16)
    lib().oracle_round_f16(_p(x), _p(vals), _p(bits), x.size)
    return vals, bits


def round_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    vals = np.empty_like(x); bits = np.empty(x.shape, np.uint16)
    lib().oracle_round_bf16(_p(x), _p(vals), _p(bits), x.size)
    return vals, bits


def round_to(x, dtype):
    """Round to a storage dtype code (0 fp32, 1 f16, 2 bf16): returns (fp32 values, raw storage array)."""
    if dtype == 0:
        x = np.ascontiguousarray(x, dtype=np.float32)
        return x, x
    return round_f16(x) if dtype == 1 else round_bf16(x)


# ------------------------------------------------------------------ generators
def gen_lcg(seed, n):
    st = (ctypes.c_uint32 * 1)(seed); out = np.empty(n, np.float32)
    lib().oracle_gen_lcg(ctypes.cast(st, ctypes.c_void_p), _p(out), n)
    return out, st[0]


def gen_lcg24(seed, n):
    st = (ctypes.c_uint32 * 1)(seed); out = np.empty(n, np.float32)
    lib().oracle_gen_lcg24(ctypes.cast(st, ctypes.c_void_p), _p(out), n)
    return out, st[0]


def gen_lcg16(seed, n):
    st = (ctypes.c_uint32 * 1)(seed); out = np.empty(n, np.float32)
    lib().oracle_gen_lcg16(ctypes.cast(st, ctypes.c_void_p), _p(out), n)
    return out, st[0]


def gen_xorshift(seed, n):
    st = (ctypes.c_uint64 * 1)(seed); out = np.empty(n, np.float32)
    lib().oracle_gen_xorshift(ctypes.cast(st, ctypes.c_void_p), _p(out), n)
    return out, st[0]


def gen_normal(seed, n, mean=0.0, sd=1.0, offset=0):
    out = np.empty(n, np.float32)
    lib().oracle_gen_normal(seed, offset, mean, sd, _p(out), n)
    return out


def gen_uniform_int(seed, lo, hi, n):
    out = np.empty(n, np.int32)
    lib().oracle_gen_uniform_int(seed, lo, hi, _p(out), n)
    return out


# ------------------------------------------------------------------ trees
def tree_anc(parent):
    parent = np.ascontiguousarray(parent, dtype=np.int32)
    anc = np.empty(len(parent), np.uint32)
    rc = lib().oracle_tree_anc(_p(parent), len(parent), _p(anc))
    if rc:
        raise ValueError(f"bad tree ({rc})")
    return anc


def tree_kw(K, W):
    parent = np.empty(K + W, np.int32); depth = np.empty(K + W, np.int32)
    if lib().oracle_tree_kw(K, W, _p(parent), _p(depth)) < 0:
        raise ValueError("bad K/W")
    return parent, depth


def tree_random(seed, n, width=2, max_depth=7):
    parent = np.empty(n, np.int32); depth = np.empty(n, np.int32)
    if lib().oracle_tree_random(seed, n, width, max_depth, _p(parent), _p(depth)) < 0:
        raise ValueError("cannot build tree")
    return parent, depth


# ------------------------------------------------------------------ attention
def attention(q, k, v, kv_off, pos, NQ, NKV, HD, scale=0.0, window=0, anc=None, tree_base=None, mode=0, nthreads=0):
    """fp64 (mode 0) or fp32-host (mode 1) attention; returns (out [T,NQ,HD] f64, lse [T,NQ] f64)."""
    q = np.ascontiguousarray(q, np.float32); k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    kv_off = np.ascontiguousarray(kv_off, np.int64); pos = np.ascontiguousarray(pos, np.int32)
    T = len(pos)
    assert q.size == T * NQ * HD
    if anc is not None:
        anc = np.ascontiguousarray(anc, np.uint32); tree_base = np.ascontiguousarray(tree_base, np.int32)
    out = np.empty((T, NQ, HD), np.float64); lse = np.empty((T, NQ), np.float64)
    rc = lib().oracle_attention(_p(q), _p(k), _p(v), _p(kv_off), _p(pos), _p(anc), _p(tree_base), T, NQ, NKV, HD,
                                float(scale), int(window), int(mode), _p(out), _p(lse), int(nthreads))
    if rc:
        raise ValueError("oracle_attention: bad arguments")
    return out, lse


def attention_split(q, k, v, kv_off, pos, NQ, NKV, HD, C, scale=0.0, window=0):
    q = np.ascontiguousarray(q, np.float32); k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    kv_off = np.ascontiguousarray(kv_off, np.int64); pos = np.ascontiguousarray(pos, np.int32)
    T = len(pos)
    out = np.empty((T, NQ, HD), np.float64); lse = np.empty((T, NQ), np.float64)
    rc = lib().oracle_attention_split(_p(q), _p(k), _p(v), _p(kv_off), _p(pos), T, NQ, NKV, HD, float(scale),
                                      int(window), int(C), _p(out), _p(lse))
    if rc:
        raise ValueError("oracle_attention_split: bad arguments")
    return out, lse


def rope_tables(maxpos, hd, theta=10000.0):
    """cos/sin tables [maxpos, hd] in fp32 as the reference's gates build them (tests/test_norm_fused.cu:90-95):
    angle p * theta^(-2i/hd) for i < hd/2, written to entries i and hd/2 + i."""
    p = np.arange(maxpos, dtype=np.float32)[:, None]
    i = np.arange(hd // 2, dtype=np.float32)[None, :]
    a = (p * np.power(np.float32(theta), np.float32(-2.0) * i / np.float32(hd))).astype(np.float32)
    c, s = np.cos(a).astype(np.float32), np.sin(a).astype(np.float32)
    return np.concatenate([c, c], axis=1), np.concatenate([s, s], axis=1)


def norm_rope_rows(x, W, eps, cosT=None, sinT=None, pos=None, rope=True):
    """Per-head RMSNorm (+ rotate-half RoPE) of the rows x [rows, hd] in float64, restating norm_rope_store_kernel
    (kernels/norm_fused.cuh:84-126): y = x * (1 / sqrt(sum(x^2) / hd + eps)) * W (norm_par_sumsq / norm_par_mul,
    :34-52; W None: no scale), then for e < hd/2 with c = cosT[p, e], s = sinT[p, e] (:111-118):
    o_e = y_e c - y_{e+hd/2} s and o_{e+hd/2} = y_{e+hd/2} c + y_e s. pos[r] is row r's position."""
    x = np.asarray(x, np.float64)
    rows, hd = x.shape
    inv = 1.0 / np.sqrt((x * x).sum(axis=1, keepdims=True) / hd + eps)
    y = x * inv
    if W is not None:
        y = y * np.asarray(W, np.float64)[None, :]
    if not rope:
        return y
    h = hd // 2
    p = np.asarray(pos, np.int64)
    c = np.asarray(cosT, np.float64)[p, :h]
    s = np.asarray(sinT, np.float64)[p, :h]
    o = np.empty_like(y)
    o[:, :h] = y[:, :h] * c - y[:, h:] * s
    o[:, h:] = y[:, h:] * c + y[:, :h] * s
    return o
