"""CPU pinning of the oracle (oracle/attn_oracle.cpp) before it is trusted as the parity checker.

Each oracle function is pinned by something other than its own formula:
  * storage rounding      -> numpy's float16 cast and torch's bfloat16 cast (independent RN-even implementations),
                             incl. ties, subnormals, overflow, inf/nan
  * fp64 attention        -> torch.nn.functional.scaled_dot_product_attention in float64 on CPU (GQA by
                             repeat_interleave, causal / sliding window / tree masks as explicit boolean masks)
                             plus closed forms (one key, identical keys, window 1, zero query)
  * fp32 host attention   -> the fp64 oracle within 1e-5 (tests/test_kernels.cu:94-108 tolerance is 1e-4)
  * split-KV LSE combine  -> the unsplit oracle (associativity), for chunk sizes 1..512
  * tree ancestor masks   -> the known answers of tests/test_treeattn.cu:24,35 ({1,3,7,15} chain,
                             parent [-1,0,0,1] -> {1,3,5,11}) and the K7W2 tree of tools/bench_serve_spec.cu:186-200
  * generators            -> input synthesis only (both sides of every parity test read the same arrays); the
                             reference ships no golden values for them, so their equality with the reference's
                             streams is checked against an independent Python-integer evaluation
"""
import math

import numpy as np
import pytest
import torch

import oracle


# ------------------------------------------------------------------ rounding
def _special_floats():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0,
        rng.standard_normal(5000).astype(np.float32) * 1e-5,            # f16 subnormal range
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                  np.inf, -np.inf, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8,
                  3.4e38, 1e-40], np.float32),
    ])
    return vals


def test_round_f16_matches_numpy():
    x = _special_floats()
    vals, bits = oracle.round_f16(x)
    ref = x.astype(np.float16)
    assert np.array_equal(bits, ref.view(np.uint16))
    assert np.array_equal(vals, ref.astype(np.float32))
    _, nb = oracle.round_f16(np.array([np.nan], np.float32))
    assert (int(nb[0]) & 0x7c00) == 0x7c00 and (int(nb[0]) & 0x3ff) != 0


def test_round_bf16_matches_torch():
    x = _special_floats()
    vals, bits = oracle.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16)
    assert np.array_equal(bits, ref.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(vals, ref.float().numpy())


# ------------------------------------------------------------------ attention vs torch SDPA (float64)
def _sdpa(q, k, v, kv_off, pos, NQ, NKV, HD, scale=0.0, window=0, anc=None, tree_base=None):
    """Independent reference: torch SDPA per token over its own key span with an explicit mask."""
    T = len(pos)
    sc = float(np.float32(scale)) if scale > 0 else 1.0 / math.sqrt(HD)   # the C ABI takes a float scale
    out = np.zeros((T, NQ, HD)); lse = np.full((T, NQ), -np.inf)
    G = NQ // NKV
    for t in range(T):
        p = int(pos[t]); n = p + 1
        kk = torch.from_numpy(k[kv_off[t]:kv_off[t] + n * NKV * HD].reshape(n, NKV, HD).astype(np.float64))
        vv = torch.from_numpy(v[kv_off[t]:kv_off[t] + n * NKV * HD].reshape(n, NKV, HD).astype(np.float64))
        j = torch.arange(n)
        mask = torch.ones(n, dtype=torch.bool)
        if window > 0:
            mask &= j >= p - window + 1
        if anc is not None:
            tb = int(tree_base[t]); d = j - tb
            bit = ((int(anc[t]) >> d.clamp(0, 31)) & 1).bool() & (d < 32)
            mask &= (j < tb) | bit
        if not mask.any():
            continue
        qq = torch.from_numpy(q.reshape(T, NQ, HD)[t].astype(np.float64))            # [NQ, HD]
        kr = kk.permute(1, 0, 2).repeat_interleave(G, 0)                             # [NQ, n, HD]
        vr = vv.permute(1, 0, 2).repeat_interleave(G, 0)
        o = torch.nn.functional.scaled_dot_product_attention(qq[:, None, :], kr, vr, attn_mask=mask[None, None, :],
                                                             scale=sc)
        out[t] = o[:, 0, :].numpy()
        s = (kr @ qq[:, :, None])[:, :, 0] * sc
        lse[t] = torch.logsumexp(s.masked_fill(~mask[None, :], -math.inf), dim=1).numpy()
    return out, lse


def _rand_problem(seed, T, NQ, NKV, HD, L):
    q = oracle.gen_normal(seed, T * NQ * HD)
    k = oracle.gen_normal(seed + 1, L * NKV * HD, 0.0, 0.5)
    v = oracle.gen_normal(seed + 2, L * NKV * HD)
    return q, k, v


@pytest.mark.parametrize("NQ,NKV,HD", [(4, 4, 32), (6, 1, 64), (24, 4, 16), (8, 2, 128)])
@pytest.mark.parametrize("window", [0, 1, 7])
def test_attention_matches_sdpa(NQ, NKV, HD, window):
    L = 40
    q, k, v = _rand_problem(11 + HD, 5, NQ, NKV, HD, L)
    pos = np.array([0, 3, 17, 38, 39], np.int32)
    off = np.zeros(5, np.int64)
    out, lse = oracle.attention(q, k, v, off, pos, NQ, NKV, HD, window=window)
    ref, rlse = _sdpa(q, k, v, off, pos, NQ, NKV, HD, window=window)
    assert np.abs(out - ref).max() < 1e-12
    assert np.abs(lse - rlse).max() < 1e-12


def test_attention_scale_ragged_batch_matches_sdpa():
    NQ, NKV, HD, ML, B = 6, 2, 64, 50, 3
    q = oracle.gen_normal(5, B * NQ * HD)
    k = oracle.gen_normal(6, B * ML * NKV * HD)
    v = oracle.gen_normal(7, B * ML * NKV * HD)
    pos = np.array([4, 49, 20], np.int32)
    off = np.arange(B, dtype=np.int64) * ML * NKV * HD
    out, lse = oracle.attention(q, k, v, off, pos, NQ, NKV, HD, scale=0.3)
    ref, rlse = _sdpa(q, k, v, off, pos, NQ, NKV, HD, scale=0.3)
    assert np.abs(out - ref).max() < 1e-12 and np.abs(lse - rlse).max() < 1e-12


def test_tree_attention_matches_sdpa():
    NQ, NKV, HD, base = 4, 2, 32, 9
    parent, _ = oracle.tree_random(3, 12, 2, 7)
    anc = oracle.tree_anc(parent)
    T = len(parent)
    q, k, v = _rand_problem(21, T, NQ, NKV, HD, base + T)
    pos = base + np.arange(T, dtype=np.int32)
    tb = np.full(T, base, np.int32)
    off = np.zeros(T, np.int64)
    out, lse = oracle.attention(q, k, v, off, pos, NQ, NKV, HD, anc=anc, tree_base=tb)
    ref, rlse = _sdpa(q, k, v, off, pos, NQ, NKV, HD, anc=anc, tree_base=tb)
    assert np.abs(out - ref).max() < 1e-12 and np.abs(lse - rlse).max() < 1e-12
    # a tree node must differ from plain causal whenever a non-ancestor precedes it
    causal, _ = oracle.attention(q, k, v, off, pos, NQ, NKV, HD)
    assert np.abs(out[-1] - causal[-1]).max() > 1e-3


# ------------------------------------------------------------------ closed forms
def test_closed_forms():
    NQ, NKV, HD, L = 4, 2, 16, 30
    q, k, v = _rand_problem(31, 1, NQ, NKV, HD, L)
    kr = k.reshape(L, NKV, HD); vr = v.reshape(L, NKV, HD)
    sc = 1.0 / math.sqrt(HD)
    # one key: O = V0, LSE = s0
    out, lse = oracle.attention(q, k, v, [0], [0], NQ, NKV, HD)
    for h in range(NQ):
        assert np.allclose(out[0, h], vr[0, h // 2], atol=1e-12)
        assert abs(lse[0, h] - sc * float(np.dot(q.reshape(NQ, HD)[h].astype(np.float64), kr[0, h // 2]))) < 1e-12
    # window 1: O = V[pos]
    out, _ = oracle.attention(q, k, v, [0], [17], NQ, NKV, HD, window=1)
    assert np.allclose(out[0, 3], vr[17, 1], atol=1e-12)
    # identical keys: O = mean V, LSE = s + ln n
    kid = np.tile(kr[:1], (L, 1, 1)).reshape(-1)
    out, lse = oracle.attention(q, kid, v, [0], [L - 1], NQ, NKV, HD)
    s0 = sc * float(np.dot(q.reshape(NQ, HD)[0].astype(np.float64), kr[0, 0]))
    assert np.allclose(out[0, 0], vr[:, 0].astype(np.float64).mean(0), atol=1e-12)
    assert abs(lse[0, 0] - (s0 + math.log(L))) < 1e-12
    # zero query: uniform weights
    out, lse = oracle.attention(np.zeros_like(q), k, v, [0], [9], NQ, NKV, HD)
    assert np.allclose(out[0, 2], vr[:10, 1].astype(np.float64).mean(0), atol=1e-12)
    assert abs(lse[0, 2] - math.log(10)) < 1e-12


def test_fp32_host_mode_close_to_fp64():
    NQ, NKV, HD, L = 8, 2, 128, 300
    q, k, v = _rand_problem(41, 3, NQ, NKV, HD, L)
    pos = np.array([10, 150, 299], np.int32)
    a, la = oracle.attention(q, k, v, np.zeros(3, np.int64), pos, NQ, NKV, HD, mode=0)
    b, lb = oracle.attention(q, k, v, np.zeros(3, np.int64), pos, NQ, NKV, HD, mode=1)
    assert np.abs(a - b).max() < 1e-5 and np.abs(la - lb).max() < 1e-5
    assert np.abs(a - b).max() > 0            # mode 1 really computes in fp32


@pytest.mark.parametrize("C", [1, 16, 64, 512])
def test_split_combine_associative(C):
    NQ, NKV, HD, L = 6, 2, 32, 700
    q, k, v = _rand_problem(51, 4, NQ, NKV, HD, L)
    pos = np.array([0, 63, 64, 699], np.int32)
    for window in (0, 100):
        a, la = oracle.attention(q, k, v, np.zeros(4, np.int64), pos, NQ, NKV, HD, window=window)
        b, lb = oracle.attention_split(q, k, v, np.zeros(4, np.int64), pos, NQ, NKV, HD, C, window=window)
        assert np.abs(a - b).max() < 1e-12 and np.abs(la - lb).max() < 1e-12


def test_threads_do_not_change_results():
    NQ, NKV, HD, L = 8, 4, 64, 200
    q, k, v = _rand_problem(61, 6, NQ, NKV, HD, L)
    pos = np.arange(194, 200, dtype=np.int32)
    a, _ = oracle.attention(q, k, v, np.zeros(6, np.int64), pos, NQ, NKV, HD, nthreads=1)
    b, _ = oracle.attention(q, k, v, np.zeros(6, np.int64), pos, NQ, NKV, HD, nthreads=7)
    assert np.array_equal(a, b)


# ------------------------------------------------------------------ trees
def test_tree_known_answers():
    assert list(oracle.tree_anc(np.array([-1, 0, 1, 2]))) == [1, 3, 7, 15]          # chain == causal
    assert list(oracle.tree_anc(np.array([-1, 0, 0, 1]))) == [1, 3, 5, 11]          # tests/test_treeattn.cu:35
    parent, depth = oracle.tree_kw(7, 2)                                            # K7W2: Nn = K + W = 9
    assert list(parent) == [-1, 0, 0, 1, 3, 4, 5, 6, 7]
    assert list(depth) == [0, 1, 1, 2, 3, 4, 5, 6, 7]
    assert list(oracle.tree_anc(parent)) == [1, 3, 5, 11, 27, 59, 123, 251, 507]
    with pytest.raises(ValueError):
        oracle.tree_anc(np.zeros(33, np.int32))


def test_tree_random_shape():
    for seed in range(20):
        parent, depth = oracle.tree_random(seed, 8, 2, 7)
        assert parent[0] == -1 and all(0 <= parent[j] < j for j in range(1, 8))
        assert max(np.bincount(parent[1:], minlength=8)) <= 2 and depth.max() <= 7
        anc = oracle.tree_anc(parent)
        assert all((anc[j] >> j) & 1 and (anc[j] >> 0) & 1 for j in range(8))


# ------------------------------------------------------------------ generators
def test_generators_match_integer_evaluation():
    s = 123
    ref = []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        ref.append(np.float32(np.float32(s >> 8) / np.float32(8388608.0)) - np.float32(1.0))
    out, st = oracle.gen_lcg(123, 5)
    assert np.array_equal(out, np.array(ref, np.float32)) and st == s
    s = 77; ref = []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        ref.append(np.float32(((s >> 8) & 0xFFFF) / 65536.0) - np.float32(0.5))
    assert np.array_equal(oracle.gen_lcg16(77, 5)[0], np.array(ref, np.float32))
    x = 0x5eed1600; ref = []
    M = (1 << 64) - 1
    for _ in range(5):
        x ^= x >> 12; x ^= (x << 25) & M; x ^= x >> 27
        r = ((x * 2685821657736338717) & M) >> 40
        ref.append(np.float32(np.float32(r) / np.float32(16777216.0)) * np.float32(2.0) - np.float32(1.0))
    assert np.array_equal(oracle.gen_xorshift(0x5eed1600, 5)[0], np.array(ref, np.float32))


def test_normal_generator_statistics_and_slicing():
    x = oracle.gen_normal(9, 400000, 0.0, 0.5)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 0.5) < 5e-3
    assert np.array_equal(oracle.gen_normal(9, 100, 0.0, 0.5, offset=1000), x[1000:1100])
    u = oracle.gen_uniform_int(4, 256, 8192, 10000)
    assert u.min() >= 256 and u.max() <= 8192 and abs(u.mean() - 4224) < 80


# ---- per-head RMSNorm + RoPE (kernels/norm_fused.cuh:84-126): pinned by identities that do not restate it ----

def test_norm_rope_oracle_rms_identities():
    """RMS step: y = x * sqrt(hd) / sqrt(||x||^2 + hd*eps) (the 2-norm form), a constant row c maps to
    c / sqrt(c^2 + eps) per element, and W scales elementwise."""
    rng = np.random.default_rng(5)
    hd, eps = 64, 1e-6
    x = rng.standard_normal((5, hd)) * 3.0
    y = oracle.norm_rope_rows(x, None, eps, rope=False)
    ref = x * np.sqrt(hd) / np.sqrt(np.linalg.norm(x, axis=1, keepdims=True) ** 2 + hd * eps)
    assert np.allclose(y, ref, rtol=1e-13, atol=0)
    c = np.full((1, hd), -2.5)
    assert np.allclose(oracle.norm_rope_rows(c, None, eps, rope=False), -2.5 / np.sqrt(6.25 + eps), rtol=1e-14)
    W = rng.standard_normal(hd)
    assert np.allclose(oracle.norm_rope_rows(x, W, eps, rope=False), y * W[None, :], rtol=1e-14)


def test_norm_rope_oracle_rope_is_a_complex_rotation():
    """Rotate-half RoPE is the complex product (y_e + i y_{e+h}) * (c_e + i s_e): pins the signs and the index
    pairing; position 0 (angle 0) is the identity and every pair keeps its norm."""
    rng = np.random.default_rng(6)
    hd, eps, h = 32, 1e-6, 16
    cosT, sinT = oracle.rope_tables(40, hd)
    x = rng.standard_normal((7, hd))
    pos = np.array([0, 1, 5, 9, 17, 33, 39])
    y = oracle.norm_rope_rows(x, None, eps, rope=False)
    o = oracle.norm_rope_rows(x, None, eps, cosT, sinT, pos, rope=True)
    z = (y[:, :h] + 1j * y[:, h:]) * (cosT[pos, :h].astype(np.float64) + 1j * sinT[pos, :h].astype(np.float64))
    assert np.allclose(o[:, :h], z.real, rtol=0, atol=1e-13) and np.allclose(o[:, h:], z.imag, rtol=0, atol=1e-13)
    assert np.array_equal(o[0], y[0])                                  # cos 0 = 1, sin 0 = 0
    cs2 = cosT[pos, :h].astype(np.float64) ** 2 + sinT[pos, :h].astype(np.float64) ** 2
    assert np.allclose(o[:, :h] ** 2 + o[:, h:] ** 2, (y[:, :h] ** 2 + y[:, h:] ** 2) * cs2, rtol=1e-12)


def test_rope_tables_follow_the_reference_angles():
    """Table entries are cos/sin of p * 10000^(-2i/hd), duplicated into both halves (tests/test_norm_fused.cu:90-95)."""
    import math
    hd = 256
    cosT, sinT = oracle.rope_tables(4200, hd)
    for p, i in ((0, 0), (1, 0), (7, 3), (4100, 127), (4199, 64)):
        a = p * 10000.0 ** (-2.0 * i / hd)
        for t, f in ((cosT, math.cos), (sinT, math.sin)):
            assert abs(float(t[p, i]) - f(a)) < 2e-3 + 1e-6 * abs(a)   # fp32 angle rounding at large p
            assert t[p, i] == t[p, hd // 2 + i]


def test_norm_rope_c_restatement_matches_the_pinned_one():
    """The C restatement (oracle_norm_rope, which the C++ gate program checks against) agrees with the fp64 numpy
    restatement pinned above, with and without RoPE and the weight row, at hd 8 .. 512."""
    import ctypes
    L = oracle.lib()
    rng = np.random.default_rng(8)
    for hd in (8, 64, 256, 512):
        rows = 9
        x = (rng.standard_normal((rows, hd)) * 2).astype(np.float32)
        W = rng.standard_normal(hd).astype(np.float32)
        cosT, sinT = oracle.rope_tables(300, hd)
        pos = rng.integers(0, 300, size=rows).astype(np.int32)
        for w, rope in ((W, True), (None, True), (W, False), (None, False)):
            out = np.zeros((rows, hd), np.float64)
            p = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
            rc = L.oracle_norm_rope(p(x), p(w), rows, hd, 1e-6, p(cosT), p(sinT), p(pos), 1 if rope else 0, p(out))
            assert rc == 0
            ref = oracle.norm_rope_rows(x, w, 1e-6, cosT, sinT, pos, rope=rope)
            assert np.allclose(out, ref, rtol=1e-13, atol=1e-13), (hd, w is None, rope)
