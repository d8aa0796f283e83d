"""GPU parity of speculative tree-verify attention (ancestor bitmask) against the oracle.

Re-expresses tests/test_treeattn.cu (chain mask == causal bit for bit; a tree node equals the linear path of
its ancestors) and BASELINE.json config 5 (B=16 sequences x 8 tree nodes, committed context U[2048,16384],
Qwen3.5 full-attention shape, f16 KV) in one ragged launch.
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import assert_close, dev, dev_bits, normal_cache, oracle_rows

pytestmark = pytest.mark.gpu


def test_chain_equals_causal_and_branch_equals_linear():
    HD, NQ, NKV, base, Sq = 128, 4, 4, 2, 4
    vals, _ = oracle.gen_lcg16(77, Sq * NQ * HD + 2 * (base + Sq) * NKV * HD)
    q = vals[:Sq * NQ * HD]
    kraw = vals[Sq * NQ * HD:Sq * NQ * HD + (base + Sq) * NKV * HD]
    vraw = vals[Sq * NQ * HD + (base + Sq) * NKV * HD:]
    k, kb = oracle.round_bf16(kraw)
    v, vb = oracle.round_bf16(vraw)
    Q, Kd, Vd = dev(q), dev_bits(kb, 2), dev_bits(vb, 2)
    On = torch.empty(Sq * NQ * HD, device="cuda"); Oa = torch.empty_like(On)
    A.flash_attn(Q, Kd, Vd, On, Sq, NQ, NKV, HD, base)
    A.flash_attn(Q, Kd, Vd, Oa, Sq, NQ, NKV, HD, base, anc=dev(np.array([1, 3, 7, 15], np.int32)))
    torch.cuda.synchronize()
    assert torch.equal(On.view(torch.int32), Oa.view(torch.int32)), "chain mask differs from causal"
    # branch: parent = [-1, 0, 0, 1]; node 2 (second child of the root) sees prefix + root + itself
    anc = oracle.tree_anc(np.array([-1, 0, 0, 1]))
    assert list(anc) == [1, 3, 5, 11]
    Ot = torch.empty_like(On)
    A.flash_attn(Q, Kd, Vd, Ot, Sq, NQ, NKV, HD, base, anc=dev(anc.view(np.int32)))
    # linear reference: [prefix, R, C1], queries R and C1, causal
    row = NKV * HD
    k2 = np.concatenate([kb[:base * row], kb[base * row:(base + 1) * row], kb[(base + 2) * row:(base + 3) * row]])
    v2 = np.concatenate([vb[:base * row], vb[base * row:(base + 1) * row], vb[(base + 2) * row:(base + 3) * row]])
    q2 = np.concatenate([q[:NQ * HD], q[2 * NQ * HD:3 * NQ * HD]])
    O2 = torch.empty(2 * NQ * HD, device="cuda")
    A.flash_attn(dev(q2), dev_bits(k2, 2), dev_bits(v2, 2), O2, 2, NQ, NKV, HD, base)
    torch.cuda.synchronize()
    e = (Ot[2 * NQ * HD:3 * NQ * HD] - O2[NQ * HD:]).abs().max().item()
    assert e < 1e-6, f"tree node vs linear path: {e:.3e}"
    # and the whole tree against the oracle
    ref, _ = oracle_rows(q, k, v, np.zeros(Sq, np.int64), base + np.arange(Sq), NQ, NKV, HD, anc=anc,
                         tree_base=np.full(Sq, base))
    assert_close(Ot.cpu().numpy().reshape(Sq, NQ, HD), ref, "tree vs oracle")


@pytest.mark.parametrize("tree", ["random8", "kw9"])
def test_config5_batched_tree_verify(tree):
    """B=16, tree nodes per sequence (seeded 2-wide depth<=7 tree of 8 nodes, or the
    reference's K7W2 shape of 9 nodes), committed L ~ U[2048, 16384], Hq=24, Hkv=4, hd=256, f16 KV."""
    B, NQ, NKV, HD = 16, 24, 4, 256
    committed = oracle.gen_uniform_int(55, 2048, 16384, B)
    if tree == "random8":
        parents = [oracle.tree_random(1000 + b, 8, 2, 7)[0] for b in range(B)]
    else:
        parents = [oracle.tree_kw(7, 2)[0] for _ in range(B)]
    Tq = len(parents[0])
    anc = np.stack([oracle.tree_anc(p) for p in parents]).astype(np.uint32)
    ML = 16384 + Tq
    lens = committed + Tq
    kv, kd = normal_cache(61, B, ML, NKV, HD, lens, 0.5, 1)
    vv, vd = normal_cache(62, B, ML, NKV, HD, lens, 0.5, 1)
    q = oracle.gen_normal(63, B * Tq * NQ * HD)
    base_b = committed.astype(np.int32)
    max_pos = int((base_b + Tq - 1).max())
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    O = torch.empty(B * Tq * NQ * HD, device="cuda"); lse = torch.empty(B * Tq * NQ, device="cuda")
    A.attn_batch(dev(q), kd, vd, O, B, Tq, NQ, NKV, HD, dev(base_b), ML * NKV * HD, max_pos, chunk=512,
                 anc=dev(anc.reshape(-1).view(np.int32)), lse=lse)
    torch.cuda.synchronize()
    pos = (base_b[:, None] + np.arange(Tq)[None, :]).reshape(-1)
    kv_off = np.repeat(np.arange(B, dtype=np.int64) * ML * NKV * HD, Tq)
    ref, ref_lse = oracle_rows(q, kv, vv, kv_off, pos, NQ, NKV, HD, anc=anc.reshape(-1),
                               tree_base=np.repeat(base_b, Tq))
    assert_close(O.cpu().numpy().reshape(B * Tq, NQ, HD), ref, f"config5 {tree}", lse.cpu().numpy().reshape(-1, NQ),
                 ref_lse)


@pytest.mark.parametrize("kvdt", [1, 2])
@pytest.mark.parametrize("HD,NQ,NKV,Tq", [(128, 16, 2, 12), (128, 32, 4, 9), (256, 16, 4, 20)])
def test_ragged_tree_verify_shapes(kvdt, HD, NQ, NKV, Tq):
    """Tree verify at HD 128 and with more than 64 query rows per KV head (several token tiles per sequence), ragged
    committed lengths that are not multiples of the 16-key tile, f16 and bf16 caches, against the oracle."""
    B = 5
    committed = oracle.gen_uniform_int(71 + HD + Tq, 1, 3000, B)
    parents = [oracle.tree_random(300 + b, Tq, 3, 6)[0] for b in range(B)]
    anc = np.stack([oracle.tree_anc(p) for p in parents]).astype(np.uint32)
    ML = 3000 + Tq
    lens = committed + Tq
    kv, kd = normal_cache(81 + HD, B, ML, NKV, HD, lens, 0.5, kvdt)
    vv, vd = normal_cache(82 + HD, B, ML, NKV, HD, lens, 0.5, kvdt)
    q = oracle.gen_normal(83 + HD, B * Tq * NQ * HD)
    base_b = committed.astype(np.int32)
    max_pos = int((base_b + Tq - 1).max())
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    O = torch.empty(B * Tq * NQ * HD, device="cuda"); lse = torch.empty(B * Tq * NQ, device="cuda")
    A.attn_batch(dev(q), kd, vd, O, B, Tq, NQ, NKV, HD, dev(base_b), ML * NKV * HD, max_pos, chunk=512,
                 anc=dev(anc.reshape(-1).view(np.int32)), lse=lse)
    torch.cuda.synchronize()
    pos = (base_b[:, None] + np.arange(Tq)[None, :]).reshape(-1)
    kv_off = np.repeat(np.arange(B, dtype=np.int64) * ML * NKV * HD, Tq)
    qr, _ = oracle.round_to(q, kvdt)        # the kernel feeds Q to the MFMA in the cache's 16-bit type
    ref, ref_lse = oracle_rows(qr, kv, vv, kv_off, pos, NQ, NKV, HD, anc=anc.reshape(-1),
                               tree_base=np.repeat(base_b, Tq))
    assert_close(O.cpu().numpy().reshape(B * Tq, NQ, HD), ref, f"tree HD{HD} Tq{Tq} kv{kvdt}",
                 lse.cpu().numpy().reshape(-1, NQ), ref_lse)


def _run_batch(q, kd, vd, B, Tq, NQ, NKV, HD, ML, base_b, anc, chunk):
    max_pos = int((base_b + Tq - 1).max())
    O = torch.empty(B * Tq * NQ * HD, device="cuda"); lse = torch.empty(B * Tq * NQ, device="cuda")
    A.attn_batch(q, kd, vd, O, B, Tq, NQ, NKV, HD, dev(base_b), ML * NKV * HD, max_pos, chunk=chunk,
                 anc=None if anc is None else dev(anc.reshape(-1).view(np.int32)), lse=lse)
    torch.cuda.synchronize()
    return O.cpu().numpy().reshape(B, Tq, NQ, HD), lse.cpu().numpy().reshape(B, Tq, NQ)


@pytest.mark.parametrize("chunk", [0, 512, 640])
@pytest.mark.parametrize("shape", ["config5", "hd128_tiles", "verify_chain"])
def test_slot_alone_equals_slot_in_batch(shape, chunk):
    """A slot's verify rows are bit-identical whether it is launched alone or as one slot of a batch (the reference
    launches every slot on its own, models/qwen35_batch.cu:333-335): B = 16 trees of 8 nodes at config 5's heads,
    HD 128 with several token tiles per sequence, and a plain causal chain of 8 draft tokens."""
    assert A.verify_runs(-1) == 0, "the batch-invariant run mode is the default"
    if shape == "config5":
        B, NQ, NKV, HD, Tq, lo, hi = 16, 24, 4, 256, 8, 2048, 16384
    elif shape == "hd128_tiles":
        B, NQ, NKV, HD, Tq, lo, hi = 16, 16, 4, 128, 20, 1, 5000
    else:
        B, NQ, NKV, HD, Tq, lo, hi = 16, 16, 2, 256, 8, 300, 9000
    committed = oracle.gen_uniform_int(91 + HD + Tq, lo, hi, B).astype(np.int32)
    anc = None
    if shape != "verify_chain":
        parents = [oracle.tree_random(700 + b, Tq, 2, 7)[0] for b in range(B)]
        anc = np.stack([oracle.tree_anc(p) for p in parents]).astype(np.uint32)
    ML = hi + Tq
    lens = committed + Tq
    _, kd = normal_cache(92, B, ML, NKV, HD, lens, 0.5, 1)
    _, vd = normal_cache(93, B, ML, NKV, HD, lens, 0.5, 1)
    q = dev(oracle.gen_normal(94, B * Tq * NQ * HD))
    A.split_reserve(B * Tq, NQ, int(lens.max()), HD)
    Ob, Lb = _run_batch(q, kd, vd, B, Tq, NQ, NKV, HD, ML, committed, anc, chunk)
    row = ML * NKV * HD
    kf, vf = kd.reshape(-1), vd.reshape(-1)
    for b in range(B):
        qs = q[b * Tq * NQ * HD:(b + 1) * Tq * NQ * HD]
        Os, Ls = _run_batch(qs, kf[b * row:(b + 1) * row], vf[b * row:(b + 1) * row], 1, Tq, NQ, NKV, HD, ML,
                            committed[b:b + 1], None if anc is None else anc[b:b + 1], chunk)
        assert np.array_equal(Os[0].view(np.uint32), Ob[b].view(np.uint32)), f"{shape} chunk {chunk}: slot {b} O"
        assert np.array_equal(Ls[0].view(np.uint32), Lb[b].view(np.uint32)), f"{shape} chunk {chunk}: slot {b} lse"


def test_equal_runs_mode_against_oracle():
    """The other run mode (equal runs over the batch's key tiles) on config 5's tree verify, against the oracle."""
    prev = A.verify_runs(1)
    try:
        test_config5_batched_tree_verify("random8")
    finally:
        A.verify_runs(prev)


@pytest.mark.parametrize("runs", [0, 1])
def test_verify_more_than_64_pairs(runs):
    """72 sequences x 12 tokens (one token tile each: 72 (sequence, tile) pairs, past the 64 that the kernel keeps in
    lanes, so the run cuts come from scans over the positions), ragged lengths from 1 key, half of them trees, HD 128
    bf16, both run modes against the oracle; in the default mode three slots alone equal their rows in the batch."""
    B, NQ, NKV, HD, Tq = 72, 8, 4, 128, 12
    committed = oracle.gen_uniform_int(501, 0, 700, B).astype(np.int32)
    anc = np.stack([oracle.tree_anc(oracle.tree_random(900 + b, Tq, 3, 6)[0]) if b % 2 else
                    oracle.tree_anc(np.arange(-1, Tq - 1)) for b in range(B)]).astype(np.uint32)
    ML = 700 + Tq
    lens = committed + Tq
    kv, kd = normal_cache(502, B, ML, NKV, HD, lens, 0.5, 2)
    vv, vd = normal_cache(503, B, ML, NKV, HD, lens, 0.5, 2)
    q = oracle.gen_normal(504, B * Tq * NQ * HD)
    qr, _ = oracle.round_to(q, 2)
    A.split_reserve(B * Tq, NQ, int(lens.max()), HD)
    prev = A.verify_runs(runs)
    try:
        Ob, Lb = _run_batch(dev(qr), kd, vd, B, Tq, NQ, NKV, HD, ML, committed, anc, 256)
        if runs == 0:
            row = ML * NKV * HD
            kf, vf = kd.reshape(-1), vd.reshape(-1)
            qd = dev(qr)
            for b in (0, 35, 71):
                Os, Ls = _run_batch(qd[b * Tq * NQ * HD:(b + 1) * Tq * NQ * HD], kf[b * row:(b + 1) * row],
                                    vf[b * row:(b + 1) * row], 1, Tq, NQ, NKV, HD, ML, committed[b:b + 1],
                                    anc[b:b + 1], 256)
                assert np.array_equal(Os[0].view(np.uint32), Ob[b].view(np.uint32)), f"slot {b} O"
                assert np.array_equal(Ls[0].view(np.uint32), Lb[b].view(np.uint32)), f"slot {b} lse"
    finally:
        A.verify_runs(prev)
    pos = (committed[:, None] + np.arange(Tq)[None, :]).reshape(-1)
    kv_off = np.repeat(np.arange(B, dtype=np.int64) * ML * NKV * HD, Tq)
    ref, ref_lse = oracle_rows(qr, kv, vv, kv_off, pos, NQ, NKV, HD, anc=anc.reshape(-1),
                               tree_base=np.repeat(committed, Tq))
    assert_close(Ob.reshape(B * Tq, NQ, HD), ref, f"72 pairs runs {runs}", Lb.reshape(-1, NQ), ref_lse)
