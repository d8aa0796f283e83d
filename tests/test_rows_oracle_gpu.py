"""Oracle parity of the paths whose other tests compare the library with itself, plus BASELINE config 4b at its
full workload.

- Config 4b (sliding-window batched decode, the Gemma local layer as models/gemma4_batch.cu:173-174 calls it):
  B=8, context lengths U[1024, 32768] seeded, window 1024, Hq=16 Hkv=8 hd=256, bf16 KV and bf16 Q/O, through
  dgx_attn_batch at chunk 96 (the benchmark's), 128 and the library default, every row's O and LSE against the
  fp64 oracle. Keys outside each row's window hold K = 0 and V = 64: a kernel that attended any of them would
  move the output by far more than the tolerance.
- Per-slot K/V pointer tables (dgx_attn_batch_ex Kp/Vp; the per-slot caches of models/qwen35_batch.cu:165-167,
  333-335): decode and tree verify against the oracle over each slot's own cache.
- Ring-buffer caches (kv_cap; runtime/decode_state_gemma4.h:9-16): decode, verify runs and prefill against the
  oracle over the linear keys.
- Output gate (models/qwen35_decode.cu:166 launch_gate_sigmoid): against oracle O x sigmoid(gate) in fp64.
- Graph replay (models/gemma4_decode_graph.cuh): every replay with rewritten positions against the oracle.
- launch_attn_decode (tests/test_decode_kernels.cu:24-35 form, Sq > 1 and base > 0) at HD 128/256/512 against
  the fp32 host reference (oracle mode 1), before and after the flash scratch is reserved (scalar kernels, then
  the fp32 MFMA kernel).

Bars: max-abs <= 1e-2, mean-abs <= 1e-3, LSE <= 1e-4 relative (north star); fp32 launchers at the reference's
fp32 bar (max-abs <= 1e-4 against the fp32 host reference, tests/test_kernels.cu:94-108).
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import assert_close, dev, dev_bits, normal_cache, oracle_rows, TORCH_DT

pytestmark = pytest.mark.gpu


def _windows(seed, lens, NKV, HD, W, dt_code):
    """Per-sequence window keys (the last min(W, len) keys) as compact fp32 values + storage bits."""
    row = NKV * HD
    vals, bits = [], []
    for b, L in enumerate(lens):
        n = min(W, int(L))
        v, bt = oracle.round_to(oracle.gen_normal(seed, n * row, 0.0, 1.0, offset=b * W * row), dt_code)
        vals.append(v.reshape(n, NKV, HD)); bits.append(bt.reshape(n, NKV, HD))
    return vals, bits


@pytest.mark.parametrize("chunk", [96, 128, 0])
def test_config4b_sliding_decode_full_workload(chunk):
    B, NQ, NKV, HD, W, ML = 8, 16, 8, 256, 1024, 32768
    lens = oracle.gen_uniform_int(4242, 1024, ML, B)
    pos = (lens - 1).astype(np.int32)
    print(f"config4b chunk={chunk} lens={lens.tolist()}", flush=True)
    kv, kb = _windows(11, lens, NKV, HD, W, 2)
    vv, vb = _windows(12, lens, NKV, HD, W, 2)
    K = torch.zeros(B, ML, NKV, HD, device="cuda", dtype=torch.bfloat16)
    V = torch.full((B, ML, NKV, HD), 64.0, device="cuda", dtype=torch.bfloat16)
    for b in range(B):
        lo = int(pos[b]) - W + 1
        K[b, lo:pos[b] + 1] = dev_bits(kb[b], 2)
        V[b, lo:pos[b] + 1] = dev_bits(vb[b], 2)
    q, _ = oracle.round_bf16(oracle.gen_normal(13, B * NQ * HD))
    # oracle over the compact windows: row b sees its 1024 keys at positions 0..1023
    ref, ref_lse = oracle_rows(q, np.concatenate(kv), np.concatenate(vv), np.arange(B) * W * NKV * HD,
                               np.full(B, W - 1), NQ, NKV, HD, window=W)
    C = chunk if chunk else A.split_chunk()
    A.split_reserve(B * max(1, -(-A.split_chunk() // C)), NQ, ML, HD)     # the reservation counts default chunks
    Q = dev(q).bfloat16()
    O = torch.empty(B * NQ * HD, device="cuda", dtype=torch.bfloat16)
    lse = torch.empty(B * NQ, device="cuda")
    A.attn_batch(Q, K, V, O, B, 1, NQ, NKV, HD, dev(pos), ML * NKV * HD, int(pos.max()), chunk=C, window=W, lse=lse)
    torch.cuda.synchronize()
    assert_close(O.float().cpu().numpy().reshape(B, NQ, HD), ref, f"config4b chunk={C}",
                 lse.cpu().numpy().reshape(B, NQ), ref_lse)


def _slot_caches(seed, lens, NKV, HD, dt_code, extra=3):
    """Separate per-slot device caches (each its own allocation) with host values."""
    hv_k, hv_v, dk, dv = [], [], [], []
    for b, L in enumerate(lens):
        kv, kd = normal_cache(seed + 2 * b, 1, int(L) + extra, NKV, HD, [int(L) + extra], 0.5, dt_code)
        vv, vd = normal_cache(seed + 2 * b + 1, 1, int(L) + extra, NKV, HD, [int(L) + extra], 0.5, dt_code)
        hv_k.append(kv.reshape(-1)); hv_v.append(vv.reshape(-1)); dk.append(kd); dv.append(vd)
    return hv_k, hv_v, dk, dv


@pytest.mark.parametrize("kvdt", [1, 2])
@pytest.mark.parametrize("Tq,tree", [(1, False), (8, True)])
def test_slot_pointers_vs_oracle(kvdt, Tq, tree):
    B, NQ, NKV, HD = 6, 24, 4, 256
    rng = np.random.default_rng(70 + Tq + kvdt)
    committed = rng.integers(30, 3000, size=B).astype(np.int32)
    lens = committed + Tq
    hk, hv, dk, dv = _slot_caches(500 + Tq, lens, NKV, HD, kvdt)
    Kp = torch.tensor([t.data_ptr() for t in dk], device="cuda", dtype=torch.int64)
    Vp = torch.tensor([t.data_ptr() for t in dv], device="cuda", dtype=torch.int64)
    q, _ = oracle.round_to(oracle.gen_normal(33 + Tq, B * Tq * NQ * HD), kvdt)
    anc = ancd = None
    if tree:
        anc = np.concatenate([oracle.tree_anc(oracle.tree_random(90 + b, Tq, 2, 7)[0]) for b in range(B)]).astype(np.uint32)
        ancd = torch.from_numpy(anc.view(np.int32)).cuda()
    offs = np.cumsum([0] + [len(x) for x in hk[:-1]]).astype(np.int64)
    kv_off = np.repeat(offs, Tq)
    posn = (np.repeat(committed, Tq) + np.tile(np.arange(Tq), B)).astype(np.int32)
    tb = np.repeat(committed, Tq).astype(np.int32) if tree else None
    ref, ref_lse = oracle_rows(q, np.concatenate(hk), np.concatenate(hv), kv_off, posn, NQ, NKV, HD, anc=anc,
                               tree_base=tb)
    max_pos = int(lens.max()) - 1
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    Q = dev(q).to(TORCH_DT[kvdt]); O = torch.empty_like(Q); lse = torch.empty(B * Tq * NQ, device="cuda")
    A.attn_batch_ex(Q, O, B, Tq, NQ, NKV, HD, dev(committed), max_pos, Kp=Kp, Vp=Vp, kv_dtype=kvdt, chunk=256,
                    anc=ancd, lse=lse)
    torch.cuda.synchronize()
    assert_close(O.float().cpu().numpy().reshape(B * Tq, NQ, HD), ref, f"slot pointers Tq={Tq}",
                 lse.cpu().numpy().reshape(B * Tq, NQ), ref_lse)


def _ring(lin_vals, lin_dev, last, cap):
    """Ring of the latest cap keys of each linear sequence: device [B, cap, NKV, HD]; unused rows hold NaN
    (never attended: a kernel that mixed one in would produce NaN)."""
    B = lin_dev.shape[0]
    ring = torch.full((B, cap) + tuple(lin_dev.shape[2:]), float("nan"), device="cuda").to(lin_dev.dtype)
    for b in range(B):
        j = np.arange(max(0, int(last[b]) - cap + 1), int(last[b]) + 1)
        ring[b, torch.from_numpy(j % cap).cuda()] = lin_dev[b, torch.from_numpy(j).cuda()]
    return ring


@pytest.mark.parametrize("kvdt", [1, 2])
@pytest.mark.parametrize("Tq,cap", [(1, 1024), (3, 1088), (12, 1088)])
def test_ring_decode_verify_vs_oracle(kvdt, Tq, cap):
    B, NQ, NKV, HD, W = 5, 16, 8, 256, 1024
    committed = np.array([40, 1100, 2300, 4999, 1023], np.int32)
    L = int(committed.max()) + Tq
    lens = committed + Tq
    kvals, K = normal_cache(61, B, L, NKV, HD, lens, 0.5, kvdt)
    vvals, V = normal_cache(62, B, L, NKV, HD, lens, 0.5, kvdt)
    last = lens - 1
    Kr, Vr = _ring(kvals, K, last, cap), _ring(vvals, V, last, cap)
    q, _ = oracle.round_to(oracle.gen_normal(63 + Tq, B * Tq * NQ * HD), kvdt)
    posn = (np.repeat(committed, Tq) + np.tile(np.arange(Tq), B)).astype(np.int32)
    kv_off = np.repeat(np.arange(B) * L * NKV * HD, Tq)
    ref, ref_lse = oracle_rows(q, kvals.reshape(-1), vvals.reshape(-1), kv_off, posn, NQ, NKV, HD, window=W)
    max_pos = int(last.max())
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    Q = dev(q).to(TORCH_DT[kvdt]); O = torch.empty_like(Q); lse = torch.empty(B * Tq * NQ, device="cuda")
    A.attn_batch_ex(Q, O, B, Tq, NQ, NKV, HD, dev(committed), max_pos, K=Kr, V=Vr, kv_stride=cap * NKV * HD,
                    chunk=256, window=W, kv_cap=cap, lse=lse)
    torch.cuda.synchronize()
    assert_close(O.float().cpu().numpy().reshape(B * Tq, NQ, HD), ref, f"ring Tq={Tq} cap={cap}",
                 lse.cpu().numpy().reshape(B * Tq, NQ), ref_lse)


@pytest.mark.parametrize("HD", [128, 256])
def test_ring_prefill_vs_oracle(HD):
    NQ, NKV, W, Sq, base = 16, 8, 1024, 256, 3000
    cap = 1344
    L = base + Sq
    kvals, K = normal_cache(71, 1, L, NKV, HD, [L], 1.0, 2)
    vvals, V = normal_cache(72, 1, L, NKV, HD, [L], 1.0, 2)
    Kr, Vr = _ring(kvals, K, np.array([L - 1]), cap), _ring(vvals, V, np.array([L - 1]), cap)
    q, _ = oracle.round_bf16(oracle.gen_normal(73, Sq * NQ * HD))
    ref, ref_lse = oracle_rows(q, kvals.reshape(-1), vvals.reshape(-1), np.zeros(Sq, np.int64),
                               np.arange(base, base + Sq), NQ, NKV, HD, window=W)
    Q = dev(q).bfloat16(); O = torch.empty_like(Q); lse = torch.empty(Sq * NQ, device="cuda")
    A.attn_prefill(Q, Kr, Vr, O, 1, Sq, NQ, NKV, HD, base=base, window=W, kv_cap=cap, lse=lse)
    torch.cuda.synchronize()
    assert_close(O.float().cpu().numpy().reshape(Sq, NQ, HD), ref, f"ring prefill HD={HD}",
                 lse.cpu().numpy().reshape(Sq, NQ), ref_lse)


@pytest.mark.parametrize("gdt", [0, 1, 2])
def test_output_gate_vs_oracle(gdt):
    B, NQ, NKV, HD, ML = 4, 24, 4, 256, 2100
    lens = np.array([700, 1300, 64, 2049], np.int32)
    kvals, K = normal_cache(81, B, ML, NKV, HD, lens, 0.5, 1)
    vvals, V = normal_cache(82, B, ML, NKV, HD, lens, 0.5, 1)
    q, _ = oracle.round_f16(oracle.gen_normal(83, B * NQ * HD))
    graw = oracle.gen_normal(84, B * NQ * HD, 0.0, 3.0)
    gvals, gbits = oracle.round_to(graw, gdt)
    gate = dev_bits(gbits, gdt)
    pos = (lens - 1).astype(np.int32)
    ref, _ = oracle_rows(q, kvals.reshape(-1), vvals.reshape(-1), np.arange(B) * ML * NKV * HD, pos, NQ, NKV, HD)
    want = ref * (1.0 / (1.0 + np.exp(-gvals.astype(np.float64).reshape(B, NQ, HD))))
    A.split_reserve(B, NQ, ML, HD)
    O = torch.empty(B * NQ * HD, device="cuda")
    A.attn_batch_ex(dev(q), O, B, 1, NQ, NKV, HD, dev(pos), int(pos.max()), K=K, V=V, kv_stride=ML * NKV * HD,
                    gate=gate)
    torch.cuda.synchronize()
    assert_close(O.cpu().numpy().reshape(B, NQ, HD), want, f"gate dtype {gdt}")


def test_graph_replay_vs_oracle():
    B, NQ, NKV, HD, ML = 6, 24, 4, 256, 2048
    kvals, K = normal_cache(91, B, ML, NKV, HD, [ML] * B, 0.5, 1)
    vvals, V = normal_cache(92, B, ML, NKV, HD, [ML] * B, 0.5, 1)
    q, _ = oracle.round_f16(oracle.gen_normal(93, B * NQ * HD))
    Q = dev(q).half()
    posd = torch.full((B,), 100, dtype=torch.int32, device="cuda")
    O = torch.empty_like(Q)
    stride = ML * NKV * HD
    A.split_reserve(B, NQ, ML, HD)
    A.attn_batch(Q, K, V, O, B, 1, NQ, NKV, HD, posd, stride, ML - 1)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        A.attn_batch(Q, K, V, O, B, 1, NQ, NKV, HD, posd, stride, ML - 1)
    rng = np.random.default_rng(9)
    for step in range(3):
        p = rng.integers(0, ML, size=B).astype(np.int32)
        posd.copy_(torch.from_numpy(p).cuda())
        g.replay()
        torch.cuda.synchronize()
        ref, _ = oracle_rows(q, kvals.reshape(-1), vvals.reshape(-1), np.arange(B) * stride, p, NQ, NKV, HD)
        assert_close(O.float().cpu().numpy().reshape(B, NQ, HD), ref, f"graph replay {step} positions {p.tolist()}")


@pytest.mark.parametrize("HD", [128, 256, 512])
def test_attn_decode_verify_rows_vs_fp32_reference(HD):
    """launch_attn_decode with Sq = 6 tokens at base 37 (query i attends keys 0..37+i), LCG inputs as in
    tests/test_decode_kernels.cu; checked against the fp32 host reference before and after a flash-scratch
    reservation (scalar kernels, then the fp32 MFMA kernel where HD <= 256)."""
    Sq, NQ, NKV, base = 6, 4, 2, 37
    L = base + Sq
    q, st = oracle.gen_lcg(2024 + HD, Sq * NQ * HD)
    k, st = oracle.gen_lcg(st, L * NKV * HD)
    v, st = oracle.gen_lcg(st, L * NKV * HD)
    q, k = q * np.float32(0.2), k * np.float32(0.2)
    ref, _ = oracle.attention(q, k, v, np.zeros(Sq, np.int64), np.arange(base, base + Sq), NQ, NKV, HD, mode=1)
    Q, K, V = dev(q), dev(k), dev(v)
    for phase in ("unreserved", "reserved"):
        if phase == "reserved":
            A.flash_reserve_partials(Sq * NQ * 4, HD)
        O = torch.empty(Sq * NQ * HD, device="cuda")
        A.attn_decode(Q, K, V, O, Sq, NQ, NKV, HD, base)
        torch.cuda.synchronize()
        e = np.abs(O.cpu().numpy().reshape(Sq, NQ, HD) - ref).max()
        assert e <= 1e-4, f"attn_decode HD={HD} {phase}: max abs err {e:.3e}"
