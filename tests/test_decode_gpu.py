"""GPU parity of the split-KV decode path (dgx_attn_decode_split / dgx_attn_batch) against the CPU oracle.

Re-expresses the reference gates of tests/test_attn_decode_split.cu (gate 1: error vs fp64 over KV lengths and
both Gemma layer shapes; gate 2: verify rows and batch rows bit-identical to S=1) and tests/test_fa2bs.cu
(determinism over repeats), plus BASELINE.json configs 1 and 2 at full size with the LSE check.
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import assert_close, dev, dev_bits, normal_cache, oracle_rows, TORCH_DT

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int32).cpu().numpy() if t.dtype == torch.float32 else t.view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("kvdt", [1, 2])
def test_config1_decode(kvdt):
    """B=1, Hq=16, Hkv=4, hd=128, L=512, N(0,1) inputs, scale 1/sqrt(128)."""
    NQ, NKV, HD, L = 16, 4, 128, 512
    qv, _ = oracle.round_to(oracle.gen_normal(101, NQ * HD), kvdt)
    kv, kd = normal_cache(202, 1, L, NKV, HD, [L], 1.0, kvdt)
    vv, vd = normal_cache(303, 1, L, NKV, HD, [L], 1.0, kvdt)
    ref, ref_lse = oracle_rows(qv, kv, vv, [0], [L - 1], NQ, NKV, HD)
    # drop-in: fp32 Q/O through launch_attn_decode_split semantics
    A.split_reserve(1, NQ, L, HD)
    O = torch.empty(NQ * HD, device="cuda"); lse = torch.empty(NQ, device="cuda")
    A.decode_split(dev(qv), kd, vd, O, 1, NQ, NKV, HD, L - 1, 1, None, L - 1, 0, A.split_ns_cap(L), lse=lse)
    torch.cuda.synchronize()
    assert_close(O.cpu().numpy().reshape(1, NQ, HD), ref, "config1 drop-in", lse.cpu().numpy().reshape(1, NQ), ref_lse)
    # native: 16-bit Q/O, one sequence
    Q16 = dev(qv, TORCH_DT[kvdt]); O16 = torch.empty(NQ * HD, device="cuda", dtype=TORCH_DT[kvdt])
    A.split_reserve(1, NQ, L, HD)
    A.attn_batch(Q16, kd, vd, O16, 1, 1, NQ, NKV, HD, None, 0, L - 1, chunk=A.split_chunk(), base=L - 1)
    torch.cuda.synchronize()
    assert_close(O16.float().cpu().numpy().reshape(1, NQ, HD), ref, "config1 native")


def _config2(seed=7, B=16, NQ=24, NKV=4, HD=256, max_len=8192, lo=256, kvdt=1):
    lens = oracle.gen_uniform_int(seed, lo, max_len, B)
    kv, kd = normal_cache(seed + 1, B, max_len, NKV, HD, lens, 0.5, kvdt)
    vv, vd = normal_cache(seed + 2, B, max_len, NKV, HD, lens, 0.5, kvdt)
    q = oracle.gen_normal(seed + 3, B * NQ * HD)
    return lens, q, kv, kd, vv, vd


@pytest.mark.parametrize("chunk", [512, 256])
def test_config2_batched_ragged(chunk):
    """BASELINE.json config 2 at full size: B=16, Hq=24, Hkv=4, hd=256, f16 KV [16,8192,4,256], L~U[256,8192]."""
    B, NQ, NKV, HD, ML = 16, 24, 4, 256, 8192
    lens, q, kv, kd, vv, vd = _config2()
    pos = (lens - 1).astype(np.int32)
    kv_off = np.arange(B, dtype=np.int64) * ML * NKV * HD
    ref, ref_lse = oracle_rows(q, kv, vv, kv_off, pos, NQ, NKV, HD)
    A.split_reserve(B, NQ, ML, HD)
    Q = dev(q); O = torch.empty(B * NQ * HD, device="cuda"); lse = torch.empty(B * NQ, device="cuda")
    A.attn_batch(Q, kd, vd, O, B, 1, NQ, NKV, HD, dev(pos), ML * NKV * HD, int(pos.max()), chunk=chunk, lse=lse)
    torch.cuda.synchronize()
    assert_close(O.cpu().numpy().reshape(B, NQ, HD), ref, f"config2 chunk={chunk}", lse.cpu().numpy().reshape(B, NQ), ref_lse)
    # 16-bit Q/O native form used by the benchmark
    Q16 = Q.half(); O16 = torch.empty(B * NQ * HD, device="cuda", dtype=torch.float16)
    A.attn_batch(Q16, kd, vd, O16, B, 1, NQ, NKV, HD, dev(pos), ML * NKV * HD, int(pos.max()), chunk=chunk)
    torch.cuda.synchronize()
    q16, _ = oracle.round_f16(q)
    ref16, _ = oracle_rows(q16, kv, vv, kv_off, pos, NQ, NKV, HD)
    assert_close(O16.float().cpu().numpy().reshape(B, NQ, HD), ref16, f"config2 f16 I/O chunk={chunk}")


def test_batch_rows_equal_single_bitwise():
    """Gate 2 (tests/test_attn_decode_split.cu:107-125): a batch row equals the S=1 launch on that slot."""
    B, NQ, NKV, HD, ML = 6, 24, 4, 256, 4096
    lens, q, kv, kd, vv, vd = _config2(seed=11, B=B, max_len=ML, lo=1)
    pos = (lens - 1).astype(np.int32)
    stride = ML * NKV * HD
    A.split_reserve(B, NQ, ML, HD)
    Q = dev(q); O = torch.empty(B * NQ * HD, device="cuda")
    A.decode_split(Q, kd, vd, O, B, NQ, NKV, HD, 0, 0, dev(pos), int(pos.max()), stride, A.split_ns_cap(ML))
    torch.cuda.synchronize()
    multi = _bits(O).reshape(B, -1)
    for b in range(B):
        O1 = torch.empty(NQ * HD, device="cuda")
        A.decode_split(Q[b * NQ * HD:], kd[b], vd[b], O1, 1, NQ, NKV, HD, int(pos[b]), 1, None, int(pos[b]), 0,
                       A.split_ns_cap(ML))
        torch.cuda.synchronize()
        assert np.array_equal(_bits(O1), multi[b]), f"slot {b} pos {pos[b]} differs from its single launch"


@pytest.mark.parametrize("shape", [(256, 16, 8, 1024), (512, 16, 1, 0), (256, 24, 4, 0)])
def test_verify_rows_equal_single_bitwise(shape):
    """Gate 2 (tests/test_attn_decode_split.cu:92-105): S consecutive rows on shared KV == S=1 at each position."""
    HD, NQ, NKV, window = shape
    ML = 2100
    kv, kd = normal_cache(21, 1, ML, NKV, HD, [ML], 1.0, 1)
    vv, vd = normal_cache(22, 1, ML, NKV, HD, [ML], 1.0, 1)
    A.split_reserve(16, NQ, ML, HD)
    for base, S in ((1000, 5), (1017, 16), (2040, 9)):
        q = oracle.gen_normal(base * 7 + S, S * NQ * HD, 0.0, 0.25)
        Q = dev(q); O = torch.empty(S * NQ * HD, device="cuda")
        A.decode_split(Q, kd, vd, O, S, NQ, NKV, HD, base, 1, None, base + S - 1, 0, A.split_ns_cap(ML), scale=1.0,
                       window=window)
        torch.cuda.synchronize()
        multi = _bits(O).reshape(S, -1)
        for r in range(S):
            O1 = torch.empty(NQ * HD, device="cuda")
            A.decode_split(Q[r * NQ * HD:], kd, vd, O1, 1, NQ, NKV, HD, base + r, 1, None, base + r, 0,
                           A.split_ns_cap(ML), scale=1.0, window=window)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(O1), multi[r]), f"verify row {r} base {base} S {S}"


@pytest.mark.parametrize("layer", [("sliding", 256, 16, 8, 1024), ("full", 512, 16, 1, 0)])
@pytest.mark.parametrize("kvdt", [0, 1, 2])
def test_gate1_lengths(layer, kvdt):
    """Gate 1 (tests/test_attn_decode_split.cu:58-90): xorshift K,V in [-1,1), q*0.25, scale 1.0, lengths up to
    32768. fp32 KV keeps the reference's fp32 bar (error / sum p|V| < 1e-5); f16/bf16 KV the north-star bar."""
    name, HD, NQ, NKV, window = layer
    maxd = 32768
    k, st = oracle.gen_xorshift(0x5eed1500 + HD, maxd * NKV * HD)
    v, st = oracle.gen_xorshift(st, maxd * NKV * HD)
    q, _ = oracle.gen_xorshift(st, NQ * HD)
    q = q * np.float32(0.25)
    kvals, kbits = oracle.round_to(k, kvdt)
    vvals, vbits = oracle.round_to(v, kvdt)
    kd, vd = dev_bits(kbits, kvdt), dev_bits(vbits, kvdt)
    Q = dev(q)
    A.split_reserve(1, NQ, maxd, HD)
    for d in (1, 31, 32, 33, 1023, 1024, 1025, 2048, 8192, 32768):
        pos = d - 1
        O = torch.empty(NQ * HD, device="cuda")
        A.decode_split(Q, kd, vd, O, 1, NQ, NKV, HD, pos, 1, None, pos, 0, A.split_ns_cap(d), scale=1.0, window=window)
        torch.cuda.synchronize()
        out = O.cpu().numpy().reshape(1, NQ, HD).astype(np.float64)
        ref, _ = oracle_rows(q, kvals, vvals, [0], [pos], NQ, NKV, HD, scale=1.0, window=window)
        if kvdt == 0:
            # error normalised by sum_j p_j |V_j,d| (fp64), as the reference gate does
            lo = max(0, pos - window + 1) if window > 0 else 0
            vv = vvals.reshape(maxd, NKV, HD)
            G = NQ // NKV
            worst = 0.0
            for h in range(NQ):
                kk = kvals.reshape(maxd, NKV, HD)[lo:pos + 1, h // G].astype(np.float64)
                s = kk @ q.reshape(NQ, HD)[h].astype(np.float64)
                p = np.exp(s - s.max()); p /= p.sum()
                den = p @ np.abs(vv[lo:pos + 1, h // G].astype(np.float64))
                worst = max(worst, float((np.abs(out[0, h] - ref[0, h]) / den).max()))
            assert worst < 1e-5, f"{name} d={d} fp32 normalised error {worst:.3e}"
        else:
            assert_close(out, ref, f"{name} d={d} kv={kvdt}")


def test_determinism_and_chunk_invariance():
    """30 repeats bitwise (tests/test_fa2bs.cu:45-49); chunks 64..512 agree within tolerance (LSE associativity)."""
    B, NQ, NKV, HD, ML = 4, 24, 4, 256, 4096
    lens, q, kv, kd, vv, vd = _config2(seed=31, B=B, max_len=ML, lo=700)
    pos = (lens - 1).astype(np.int32)
    A.split_reserve(B, NQ, ML, HD)
    # chunk 64 needs the most partials
    A.split_reserve(B * 8, NQ, ML, HD)
    Q = dev(q); P = dev(pos)
    outs = {}
    for chunk in (64, 128, 256, 512):
        O = torch.empty(B * NQ * HD, device="cuda")
        A.attn_batch(Q, kd, vd, O, B, 1, NQ, NKV, HD, P, ML * NKV * HD, int(pos.max()), chunk=chunk)
        torch.cuda.synchronize()
        outs[chunk] = O.clone()
        if chunk == 256:
            first = _bits(O)
            for _ in range(30):
                A.attn_batch(Q, kd, vd, O, B, 1, NQ, NKV, HD, P, ML * NKV * HD, int(pos.max()), chunk=chunk)
            torch.cuda.synchronize()
            assert np.array_equal(first, _bits(O)), "non-deterministic"
    for chunk in (64, 128, 512):
        d = (outs[chunk] - outs[256]).abs()
        assert float(d.max()) < 5e-3, f"chunk {chunk} vs 256: {float(d.max())}"
