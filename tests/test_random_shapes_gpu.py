"""Seeded random shapes through every path of the C ABI against the oracle: ragged batches of decode / verify /
tree rows (dgx_attn_batch), prefill and chunked prefill with and without key splits (dgx_attn_prefill), over head
dims, GQA group sizes, windows, storage dtypes and lengths that are not multiples of the 16/64-key tiles. Each case
draws its configuration from a fixed seed, so a failure names a reproducible case."""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import TORCH_DT, assert_close, dev, normal_cache, oracle_rows

pytestmark = pytest.mark.gpu


def _batch_cfg(seed, hds=(128, 256)):
    r = np.random.default_rng(seed)
    HD = int(r.choice(hds))
    NKV = int(r.choice([1, 2, 4, 8]))
    GRP = int(r.choice([1, 2, 4, 6, 8]))
    T = int(r.choice([1, 1, 2, 3, 5, 8, 12]))
    B = int(r.integers(1, 6))
    window = int(r.choice([0, 0, 0, 33, 256]))
    tree = T > 1 and bool(r.integers(0, 2)) and window == 0
    kvdt = int(r.choice([1, 2]))
    committed = r.integers(0, 1500, size=B).astype(np.int32)
    chunk = int(r.choice([0, 256, 512]))
    return dict(HD=HD, NKV=NKV, NQ=NKV * GRP, T=T, B=B, window=window, tree=tree, kvdt=kvdt, committed=committed,
                chunk=chunk)


@pytest.mark.parametrize("seed", range(32))
def test_random_batch(seed):
    # seeds 24.. draw HD 512 (the Gemma global-layer head size, served by split_kernel)
    c = _batch_cfg(1000 + seed) if seed < 24 else _batch_cfg(1000 + seed, hds=(512,))
    HD, NKV, NQ, T, B, kvdt = c["HD"], c["NKV"], c["NQ"], c["T"], c["B"], c["kvdt"]
    committed = c["committed"]
    ML = int(committed.max()) + T
    lens = committed + T
    kv, kd = normal_cache(seed + 1, B, ML, NKV, HD, lens, 0.5, kvdt)
    vv, vd = normal_cache(seed + 2, B, ML, NKV, HD, lens, 0.5, kvdt)
    q = oracle.gen_normal(seed + 3, B * T * NQ * HD)
    qr, _ = oracle.round_to(q, kvdt)
    anc = None
    if c["tree"]:
        anc = np.stack([oracle.tree_anc(oracle.tree_random(seed * 10 + b, T, 2, 7)[0]) for b in range(B)]).astype(np.uint32)
    max_pos = int((committed + T - 1).max())
    chunk = c["chunk"] or A.split_chunk()
    A.split_reserve(B * T * max(1, -(-A.split_chunk() // chunk)), NQ, max_pos + 1, HD)
    O = torch.empty(B * T * NQ * HD, device="cuda"); lse = torch.empty(B * T * NQ, device="cuda")
    A.attn_batch(dev(q), kd, vd, O, B, T, NQ, NKV, HD, dev(committed), ML * NKV * HD, max_pos, chunk=c["chunk"],
                 anc=None if anc is None else dev(anc.reshape(-1).view(np.int32)), window=c["window"], lse=lse)
    torch.cuda.synchronize()
    pos = (committed[:, None] + np.arange(T)[None, :]).reshape(-1)
    off = np.repeat(np.arange(B, dtype=np.int64) * ML * NKV * HD, T)
    ref, ref_lse = oracle_rows(qr, kv, vv, off, pos, NQ, NKV, HD, window=c["window"],
                               anc=None if anc is None else anc.reshape(-1),
                               tree_base=None if anc is None else np.repeat(committed, T))
    assert_close(O.cpu().numpy().reshape(B * T, NQ, HD), ref, f"case {seed} {c}", lse.cpu().numpy().reshape(-1, NQ),
                 ref_lse)


def _prefill_cfg(seed, hds=(128, 256)):
    r = np.random.default_rng(seed)
    HD = int(r.choice(hds))
    NKV = int(r.choice([1, 2, 4, 8]))
    GRP = int(r.choice([1, 2, 4]))
    Sq = int(r.integers(33, 400))
    base = int(r.choice([0, 0, 17, 600, 1500]))
    window = int(r.choice([0, 0, 100, 512]))
    kv_split = int(r.choice([0, 0, -1, 256, 512]))
    if window:
        kv_split = 0
    return dict(HD=HD, NKV=NKV, NQ=NKV * GRP, Sq=Sq, base=base, window=window, kv_split=kv_split)


@pytest.mark.parametrize("seed", range(22))
def test_random_prefill(seed):
    # seeds 16.. draw HD 512
    c = _prefill_cfg(2000 + seed) if seed < 16 else _prefill_cfg(2000 + seed, hds=(512,))
    HD, NKV, NQ, Sq, base = c["HD"], c["NKV"], c["NQ"], c["Sq"], c["base"]
    L = base + Sq
    kv, kd = normal_cache(seed + 11, 1, L, NKV, HD, [L], 1.0, 2)
    vv, vd = normal_cache(seed + 12, 1, L, NKV, HD, [L], 1.0, 2)
    q = oracle.gen_normal(seed + 13, Sq * NQ * HD)
    qr, _ = oracle.round_to(q, 2)
    Q = dev(qr, TORCH_DT[2]); O = torch.empty(Sq * NQ * HD, device="cuda", dtype=TORCH_DT[2])
    lse = torch.empty(Sq * NQ, device="cuda")
    A.attn_prefill(Q, kd.view(L, NKV, HD), vd.view(L, NKV, HD), O, 1, Sq, NQ, NKV, HD, base=base,
                   window=c["window"], kv_split=c["kv_split"], lse=lse)
    torch.cuda.synchronize()
    ref, ref_lse = oracle_rows(qr, kv, vv, np.zeros(Sq, np.int64), base + np.arange(Sq), NQ, NKV, HD,
                               window=c["window"])
    assert_close(O.float().cpu().numpy().reshape(Sq, NQ, HD), ref, f"case {seed} {c}",
                 lse.cpu().numpy().reshape(Sq, NQ), ref_lse)


@pytest.mark.parametrize("T,tree", [(1, False), (8, True), (3, False)])
def test_many_sequences(T, tree):
    """More than 64 sequences, so the device-side work enumeration (decode items, verify runs) and the combine's
    run scan cover several 64-lane blocks; short ragged lengths keep the oracle fast."""
    B, NQ, NKV, HD, kvdt = 100, 16, 2, 128, 1
    committed = np.random.default_rng(77 + T).integers(0, 700, size=B).astype(np.int32)
    ML = int(committed.max()) + T
    lens = committed + T
    kv, kd = normal_cache(91, B, ML, NKV, HD, lens, 0.5, kvdt)
    vv, vd = normal_cache(92, B, ML, NKV, HD, lens, 0.5, kvdt)
    q = oracle.gen_normal(93, B * T * NQ * HD)
    qr, _ = oracle.round_to(q, kvdt)
    anc = None
    if tree:
        anc = np.stack([oracle.tree_anc(oracle.tree_random(500 + b, T, 2, 7)[0]) for b in range(B)]).astype(np.uint32)
    max_pos = int((committed + T - 1).max())
    A.split_reserve(B * T * 2, NQ, max_pos + 1, HD)
    O = torch.empty(B * T * NQ * HD, device="cuda"); lse = torch.empty(B * T * NQ, device="cuda")
    A.attn_batch(dev(q), kd, vd, O, B, T, NQ, NKV, HD, dev(committed), ML * NKV * HD, max_pos, chunk=256,
                 anc=None if anc is None else dev(anc.reshape(-1).view(np.int32)), lse=lse)
    torch.cuda.synchronize()
    pos = (committed[:, None] + np.arange(T)[None, :]).reshape(-1)
    off = np.repeat(np.arange(B, dtype=np.int64) * ML * NKV * HD, T)
    ref, ref_lse = oracle_rows(qr, kv, vv, off, pos, NQ, NKV, HD, anc=None if anc is None else anc.reshape(-1),
                               tree_base=None if anc is None else np.repeat(committed, T))
    assert_close(O.cpu().numpy().reshape(B * T, NQ, HD), ref, f"B={B} T={T}", lse.cpu().numpy().reshape(-1, NQ),
                 ref_lse)


@pytest.mark.parametrize("chunk,T", [(384, 1), (224, 1), (384, 3)])
def test_chunks_off_powers_of_two(chunk, T):
    """Chunk sizes that are multiples of 32 but not powers of two (the streaming kernel's two key lanes then split
    a chunk into unequal tile counts, and chunk boundaries fall inside 64-key blocks)."""
    B, NQ, NKV, HD, kvdt = 6, 24, 4, 256, 1
    committed = np.array([0, 383, 384, 1000, 2047, 3001], np.int32)
    ML = int(committed.max()) + T
    lens = committed + T
    kv, kd = normal_cache(31, B, ML, NKV, HD, lens, 0.5, kvdt)
    vv, vd = normal_cache(32, B, ML, NKV, HD, lens, 0.5, kvdt)
    q = oracle.gen_normal(33, B * T * NQ * HD)
    qr, _ = oracle.round_to(q, kvdt)
    max_pos = int((committed + T - 1).max())
    A.split_reserve(B * T * -(-A.split_chunk() // chunk), NQ, max_pos + 1, HD)
    O = torch.empty(B * T * NQ * HD, device="cuda"); lse = torch.empty(B * T * NQ, device="cuda")
    A.attn_batch(dev(q), kd, vd, O, B, T, NQ, NKV, HD, dev(committed), ML * NKV * HD, max_pos, chunk=chunk, lse=lse)
    torch.cuda.synchronize()
    pos = (committed[:, None] + np.arange(T)[None, :]).reshape(-1)
    off = np.repeat(np.arange(B, dtype=np.int64) * ML * NKV * HD, T)
    ref, ref_lse = oracle_rows(qr, kv, vv, off, pos, NQ, NKV, HD)
    assert_close(O.cpu().numpy().reshape(B * T, NQ, HD), ref, f"chunk={chunk} T={T}", lse.cpu().numpy().reshape(-1, NQ),
                 ref_lse)
