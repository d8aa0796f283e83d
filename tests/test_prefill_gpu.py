"""GPU parity of the flash prefill path (dgx_flash_attn_v2 / dgx_attn_prefill / dgx_flash_attn) vs the oracle.

Re-expresses tests/test_flash_v2.cu (shapes, KV lengths Sq + {0, 1024, 8192}, sampled query tokens, 30-run
determinism, row-composition bit identity) and tests/test_flash_gemma.cu (scale / window variants), plus
BASELINE.json configs 3 (causal T=1024 and chunked 512 over a 4096 prefix) and 4a (sliding window T=4096).
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import assert_close, dev, dev_bits, oracle_rows, TORCH_DT

pytestmark = pytest.mark.gpu


def _inputs(seed, Sq, base, NQ, NKV, HD, dt, sd=1.0):
    q = oracle.gen_normal(seed, Sq * NQ * HD, 0.0, sd)
    qv, _ = oracle.round_to(q, dt)
    k, kb = oracle.round_to(oracle.gen_normal(seed + 1, (base + Sq) * NKV * HD, 0.0, sd), dt)
    v, vb = oracle.round_to(oracle.gen_normal(seed + 2, (base + Sq) * NKV * HD, 0.0, sd), dt)
    return q, qv, k, dev_bits(kb, dt), v, dev_bits(vb, dt)


def _sample_tokens(Sq, base, window, seed=77):
    if Sq <= 64:
        return np.arange(Sq)
    toks = {0, 1, 2, 15, 16, 17, Sq // 2, Sq - 3, Sq - 2, Sq - 1}
    for e in (1023, 1024, 1025):
        if 0 <= e - base < Sq:
            toks.add(e - base)
    rng = np.random.default_rng(seed + Sq)
    toks.update(int(x) for x in rng.integers(0, Sq, 24))
    return np.array(sorted(toks))


def _check(O, q, k, v, toks, Sq, base, NQ, NKV, HD, what, scale=0.0, window=0, lse=None):
    out = O.float().cpu().numpy().reshape(Sq, NQ, HD)[toks]
    qs = q.reshape(Sq, NQ, HD)[toks]
    ref, ref_lse = oracle_rows(qs, k, v, np.zeros(len(toks), np.int64), base + toks, NQ, NKV, HD, scale=scale,
                               window=window)
    l = None if lse is None else lse.cpu().numpy().reshape(Sq, NQ)[toks]
    return assert_close(out, ref, what, l, None if lse is None else ref_lse)


@pytest.mark.parametrize("kv_split", [0, 256, 512])
def test_config3_causal_prefill(kv_split):
    """B=1, T=1024, Hq=16, Hkv=8, hd=256, bf16 Q/K/V ~ N(0,1), causal, bf16 output."""
    Sq, NQ, NKV, HD = 1024, 16, 8, 256
    q, qv, k, kd, v, vd = _inputs(5, Sq, 0, NQ, NKV, HD, 2)
    Q = dev(qv, torch.bfloat16); O = torch.empty(Sq * NQ * HD, device="cuda", dtype=torch.bfloat16)
    lse = torch.empty(Sq * NQ, device="cuda")
    A.attn_prefill(Q, kd, vd, O, 1, Sq, NQ, NKV, HD, kv_split=kv_split, lse=lse)
    torch.cuda.synchronize()
    toks = np.arange(0, Sq, 3)
    _check(O, qv, k, v, toks, Sq, 0, NQ, NKV, HD, f"config3 split={kv_split}", lse=lse)


@pytest.mark.parametrize("kv_split", [1024, -1])
def test_config3_chunked_prefill(kv_split):
    """BASELINE.json config 3 chunked variant: 512 queries over a 4096-token cached prefix plus themselves, with an
    explicit key split and with the library's choice (-1)."""
    Sq, base, NQ, NKV, HD = 512, 4096, 16, 8, 256
    q, qv, k, kd, v, vd = _inputs(6, Sq, base, NQ, NKV, HD, 2)
    Q = dev(qv, torch.bfloat16); O = torch.empty(Sq * NQ * HD, device="cuda", dtype=torch.bfloat16)
    A.attn_prefill(Q, kd, vd, O, 1, Sq, NQ, NKV, HD, base=base, kv_split=kv_split)
    torch.cuda.synchronize()
    _check(O, qv, k, v, _sample_tokens(Sq, base, 0), Sq, base, NQ, NKV, HD, f"config3 chunked split {kv_split}")


def test_auto_split_leaves_full_grids_unsplit():
    """kv_split = -1 keeps a grid that fills the CUs unsplit: config 3 (256 equal workgroups) is bit-identical."""
    Sq, NQ, NKV, HD = 1024, 16, 8, 256
    q, qv, k, kd, v, vd = _inputs(3, Sq, 0, NQ, NKV, HD, 2)
    Q = dev(qv, torch.bfloat16)
    O0 = torch.empty(Sq * NQ * HD, device="cuda", dtype=torch.bfloat16); O1 = torch.empty_like(O0)
    A.attn_prefill(Q, kd, vd, O0, 1, Sq, NQ, NKV, HD, kv_split=0)
    A.attn_prefill(Q, kd, vd, O1, 1, Sq, NQ, NKV, HD, kv_split=-1)
    torch.cuda.synchronize()
    assert torch.equal(O0.view(torch.int16), O1.view(torch.int16))


def test_config4_sliding_prefill():
    """BASELINE.json config 4a: sliding window 1024, T=4096, Hq=16, Hkv=8, hd=256, bf16."""
    Sq, NQ, NKV, HD, W = 4096, 16, 8, 256, 1024
    q, qv, k, kd, v, vd = _inputs(8, Sq, 0, NQ, NKV, HD, 2)
    Q = dev(qv, torch.bfloat16); O = torch.empty(Sq * NQ * HD, device="cuda", dtype=torch.bfloat16)
    A.attn_prefill(Q, kd, vd, O, 1, Sq, NQ, NKV, HD, kv_split=0, window=W)
    torch.cuda.synchronize()
    _check(O, qv, k, v, _sample_tokens(Sq, 0, W), Sq, 0, NQ, NKV, HD, "config4 sliding", window=W)


@pytest.mark.parametrize("shape", [("sliding", 256, 16, 8, 1024), ("full", 512, 16, 1, 0), ("gqa6", 256, 24, 4, 0)])
@pytest.mark.parametrize("sq,base", [(1, 0), (6, 1024), (17, 0), (512, 1024), (1024, 0), (2048, 8192)])
def test_flash_v2_gate(shape, sq, base):
    """tests/test_flash_v2.cu gate: f16 cache (engine default), fp32 Q/O, normalised max error; 30-run
    determinism; the last rows launched alone equal the full launch bit for bit. The GQA-6 prompt of 1024 tokens
    runs on the wide 96-row tile (one round of workgroups) and its last rows alone on the 64-row one, so the
    bitwise check there also pins that the tile choice leaves a row's bits unchanged."""
    name, HD, NQ, NKV, window = shape
    uq = oracle.gen_lcg(2101 + HD * 17 + sq * 43 + base * 59, sq * NQ * HD)[0]
    q = uq
    k, kb = oracle.round_f16(oracle.gen_lcg(999 + sq, (base + sq) * NKV * HD)[0])
    v, vb = oracle.round_f16(oracle.gen_lcg(1999 + sq, (base + sq) * NKV * HD)[0])
    kd, vd = dev_bits(kb, 1), dev_bits(vb, 1)
    Q = dev(q); O = torch.empty(sq * NQ * HD, device="cuda")
    A.flash_attn_v2(Q, kd, vd, O, sq, NQ, NKV, HD, base, window=window)
    torch.cuda.synchronize()
    first = O.view(torch.int32).cpu().numpy().copy()
    toks = _sample_tokens(sq, base, window)
    out = O.cpu().numpy().reshape(sq, NQ, HD)[toks].astype(np.float64)
    ref, _ = oracle_rows(q.reshape(sq, NQ, HD)[toks], k, v, np.zeros(len(toks), np.int64), base + toks, NQ, NKV, HD,
                         window=window)
    nmax = np.abs(out - ref).max() / np.abs(ref).max()
    assert nmax < 1e-2, f"{name} sq={sq} base={base} normalised max error {nmax:.3e}"
    assert_close(out, ref, f"{name} sq={sq} base={base}")
    for _ in range(10):
        A.flash_attn_v2(Q, kd, vd, O, sq, NQ, NKV, HD, base, window=window)
    torch.cuda.synchronize()
    assert np.array_equal(first, O.view(torch.int32).cpu().numpy()), "non-deterministic"
    s1 = sq - 6 if sq > 6 else (sq - 1 if sq > 1 else 0)
    if s1 > 0:
        Ot = torch.empty((sq - s1) * NQ * HD, device="cuda")
        A.flash_attn_v2(Q[s1 * NQ * HD:], kd, vd, Ot, sq - s1, NQ, NKV, HD, base + s1, window=window)
        torch.cuda.synchronize()
        assert np.array_equal(first[s1 * NQ * HD:], Ot.view(torch.int32).cpu().numpy()), "row composition differs"


@pytest.mark.parametrize("sq,base,nq,nkv", [(1, 500, 24, 4), (16, 100, 24, 4), (40, 500, 24, 4), (16, 300, 16, 16),
                                           (7, 777, 16, 2), (8, 8192, 24, 4), (4, 32768, 24, 4)])
def test_fa2bs_gate(sq, base, nq, nkv):
    """tests/test_fa2bs.cu: launch_flash_attn on a bf16 cache, HD 256, incl. 32K-key accumulation."""
    HD = 256
    q, _ = oracle.round_bf16(oracle.gen_lcg24(777 + sq + base, sq * nq * HD)[0])
    k, kb = oracle.round_bf16(oracle.gen_lcg24(1777 + sq + base, (base + sq) * nkv * HD)[0])
    v, vb = oracle.round_bf16(oracle.gen_lcg24(2777 + sq + base, (base + sq) * nkv * HD)[0])
    Q = dev(q); O = torch.empty(sq * nq * HD, device="cuda")
    lse = torch.empty(sq * nq, device="cuda")
    A.flash_attn(Q, dev_bits(kb, 2), dev_bits(vb, 2), O, sq, nq, nkv, HD, base, lse=lse)
    torch.cuda.synchronize()
    ref, ref_lse = oracle_rows(q, k, v, np.zeros(sq, np.int64), base + np.arange(sq), nq, nkv, HD)
    assert_close(O.cpu().numpy().reshape(sq, nq, HD), ref, f"fa2bs sq={sq} base={base}",
                 lse.cpu().numpy().reshape(sq, nq), ref_lse)


@pytest.mark.parametrize("hd,nkv", [(256, 8), (512, 1), (512, 8), (256, 1)])
@pytest.mark.parametrize("window,scale", [(0, 0.0), (1024, 0.0625), (256, 0.0)])
@pytest.mark.parametrize("sq,base", [(37, 300), (512, 0), (16, 0)])
def test_flash_gemma_gate(hd, nkv, window, scale, sq, base):
    """tests/test_flash_gemma.cu accuracy sweep (subset): fp32 and bf16 caches, scale/window variants."""
    NQ = 16
    seed = 909 + hd * 17 + nkv * 31 + sq * 43 + base * 59
    vals, _ = oracle.gen_lcg(seed, sq * NQ * hd + 2 * (base + sq) * nkv * hd)
    q = vals[:sq * NQ * hd]
    kraw = vals[sq * NQ * hd: sq * NQ * hd + (base + sq) * nkv * hd]
    vraw = vals[sq * NQ * hd + (base + sq) * nkv * hd:]
    qr, _ = oracle.round_bf16(q)
    k, kb = oracle.round_bf16(kraw)
    v, vb = oracle.round_bf16(vraw)
    ref, _ = oracle_rows(qr, k, v, np.zeros(sq, np.int64), base + np.arange(sq), NQ, nkv, hd, scale=scale, window=window)
    for kvdt, kd, vd in ((2, dev_bits(kb, 2), dev_bits(vb, 2)), (0, dev(k), dev(v))):
        Q = dev(q); O = torch.empty(sq * NQ * hd, device="cuda")
        A.flash_attn(Q, kd, vd, O, sq, NQ, nkv, hd, base, scale=scale, window=window)
        torch.cuda.synchronize()
        out = O.cpu().numpy().reshape(sq, NQ, hd)
        den = np.abs(ref).max()
        e = np.abs(out - ref)
        assert e.max() / den < 1e-2 and e.mean() / den < 1e-3, f"kv={kvdt} {e.max() / den:.3e} {e.mean() / den:.3e}"
