"""Seeded inputs of the golden attention cases (shared by make_golden.py and the tests).

Each case rebuilds its inputs from the reference tests' generators (xorshift of tests/test_attn_decode_split.cu,
the LCG of tests/test_flash_v2.cu, a counter-based normal generator), rounded to the storage dtype, so a fixture
only needs the expected outputs plus a hash of the inputs. Sizes are small: the whole fixture file is < 1 MB.
"""
import hashlib

import numpy as np

import oracle


def _hash(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def case_config1():
    """B=1, Hq=16, Hkv=4, hd=128, L=512, f16 Q/K/V ~ N(0,1), scale 1/sqrt(128)."""
    NQ, NKV, HD, L, dt = 16, 4, 128, 512, 1
    q, qb = oracle.round_to(oracle.gen_normal(101, NQ * HD), dt)
    k, kb = oracle.round_to(oracle.gen_normal(202, L * NKV * HD), dt)
    v, vb = oracle.round_to(oracle.gen_normal(303, L * NKV * HD), dt)
    return dict(name="config1", kind="decode", NQ=NQ, NKV=NKV, HD=HD, dt=dt, window=0, scale=0.0,
                q=q, k=k, v=v, qb=qb, kb=kb, vb=vb, pos=np.array([L - 1], np.int32), ML=L,
                hash=_hash(qb, kb, vb))


def case_gate1_fp32_window():
    """Gate-1 style (tests/test_attn_decode_split.cu:58-90): xorshift K, V in [-1, 1), q * 0.25, scale 1.0, fp32
    cache, Gemma sliding shape (Hq=16, Hkv=8, hd=256, window 1024), one row at position 1499."""
    NQ, NKV, HD, L = 16, 8, 256, 1500
    k, st = oracle.gen_xorshift(0x5eed1500 + HD, L * NKV * HD)
    v, st = oracle.gen_xorshift(st, L * NKV * HD)
    q, _ = oracle.gen_xorshift(st, NQ * HD)
    q = q * np.float32(0.25)
    return dict(name="gate1_fp32_window", kind="decode", NQ=NQ, NKV=NKV, HD=HD, dt=0, window=1024, scale=1.0,
                q=q, k=k, v=v, qb=q, kb=k, vb=v, pos=np.array([L - 1], np.int32), ML=L, hash=_hash(q, k, v))


def case_window_batch_bf16():
    """Ragged bf16 batch decode under a 64-key window: three sequences of 1, 70 and 300 keys."""
    NQ, NKV, HD, ML, dt = 16, 8, 128, 300, 2
    lens = np.array([1, 70, 300], np.int32)
    B = len(lens)
    k = np.zeros((B, ML, NKV, HD), np.float32); v = np.zeros_like(k)
    for b in range(B):
        k[b, :lens[b]] = oracle.gen_normal(40 + b, lens[b] * NKV * HD, 0.0, 0.5).reshape(lens[b], NKV, HD)
        v[b, :lens[b]] = oracle.gen_normal(50 + b, lens[b] * NKV * HD, 0.0, 0.5).reshape(lens[b], NKV, HD)
    k, kb = oracle.round_to(k, dt); v, vb = oracle.round_to(v, dt)
    q, qb = oracle.round_to(oracle.gen_normal(60, B * NQ * HD), dt)
    return dict(name="window_batch_bf16", kind="batch", NQ=NQ, NKV=NKV, HD=HD, dt=dt, window=64, scale=0.0,
                q=q, k=k, v=v, qb=qb, kb=kb, vb=vb, pos=(lens - 1).astype(np.int32), ML=ML, Tq=1,
                hash=_hash(qb, kb, vb))


def case_tree_f16():
    """Tree verify: two sequences with 300 and 517 committed keys, 8 draft nodes each (seeded 2-wide trees), f16."""
    NQ, NKV, HD, Tq, dt = 24, 4, 128, 8, 1
    committed = np.array([300, 517], np.int32)
    B, ML = len(committed), 517 + Tq
    anc = np.stack([oracle.tree_anc(oracle.tree_random(1000 + b, Tq, 2, 7)[0]) for b in range(B)]).astype(np.uint32)
    k = np.zeros((B, ML, NKV, HD), np.float32); v = np.zeros_like(k)
    for b in range(B):
        n = committed[b] + Tq
        k[b, :n] = oracle.gen_normal(70 + b, n * NKV * HD, 0.0, 0.5).reshape(n, NKV, HD)
        v[b, :n] = oracle.gen_normal(80 + b, n * NKV * HD, 0.0, 0.5).reshape(n, NKV, HD)
    k, kb = oracle.round_to(k, dt); v, vb = oracle.round_to(v, dt)
    q, qb = oracle.round_to(oracle.gen_normal(90, B * Tq * NQ * HD), dt)
    return dict(name="tree_f16", kind="tree", NQ=NQ, NKV=NKV, HD=HD, dt=dt, window=0, scale=0.0,
                q=q, k=k, v=v, qb=qb, kb=kb, vb=vb, base_b=committed, anc=anc, Tq=Tq, ML=ML,
                hash=_hash(qb, kb, vb, anc))


def case_prefill_lcg_bf16():
    """Chunked prefill in the style of tests/test_flash_v2.cu: LCG inputs (seed 2101 + 17 hd + 43 sq + 59 base),
    bf16, 24 queries after a 40-key prefix, Hq=16, Hkv=8, hd=128, causal."""
    NQ, NKV, HD, Sq, base, dt = 16, 8, 128, 24, 40, 2
    seed = 2101 + 17 * HD + 43 * Sq + 59 * base
    vals, _ = oracle.gen_lcg(seed, Sq * NQ * HD + 2 * (base + Sq) * NKV * HD)
    q, qb = oracle.round_to(vals[:Sq * NQ * HD], dt)
    k, kb = oracle.round_to(vals[Sq * NQ * HD:Sq * NQ * HD + (base + Sq) * NKV * HD], dt)
    v, vb = oracle.round_to(vals[Sq * NQ * HD + (base + Sq) * NKV * HD:], dt)
    return dict(name="prefill_lcg_bf16", kind="prefill", NQ=NQ, NKV=NKV, HD=HD, dt=dt, window=0, scale=0.0,
                q=q, k=k, v=v, qb=qb, kb=kb, vb=vb, Sq=Sq, base=base, hash=_hash(qb, kb, vb))


CASES = [case_config1, case_gate1_fp32_window, case_window_batch_bf16, case_tree_f16, case_prefill_lcg_bf16]


def oracle_of(c):
    """The fp64 oracle's (O, LSE) of a case."""
    NQ, NKV, HD = c["NQ"], c["NKV"], c["HD"]
    if c["kind"] == "decode":
        return oracle.attention(c["q"], c["k"], c["v"], [0], c["pos"], NQ, NKV, HD, scale=c["scale"], window=c["window"])
    if c["kind"] == "batch":
        B = len(c["pos"])
        off = np.arange(B, dtype=np.int64) * c["ML"] * NKV * HD
        return oracle.attention(c["q"], c["k"], c["v"], off, c["pos"], NQ, NKV, HD, scale=c["scale"], window=c["window"])
    if c["kind"] == "tree":
        B, Tq = len(c["base_b"]), c["Tq"]
        pos = (c["base_b"][:, None] + np.arange(Tq)[None, :]).reshape(-1)
        off = np.repeat(np.arange(B, dtype=np.int64) * c["ML"] * NKV * HD, Tq)
        return oracle.attention(c["q"], c["k"], c["v"], off, pos, NQ, NKV, HD, anc=c["anc"].reshape(-1),
                                tree_base=np.repeat(c["base_b"], Tq))
    if c["kind"] == "prefill":
        Sq, base = c["Sq"], c["base"]
        return oracle.attention(c["q"], c["k"], c["v"], np.zeros(Sq, np.int64), base + np.arange(Sq), NQ, NKV, HD)
    raise ValueError(c["kind"])
