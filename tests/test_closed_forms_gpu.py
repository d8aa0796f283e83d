"""Closed forms that fix the attention output without any reference implementation, on every kernel family.

* All keys of a head identical (or Q = 0): every attended key gets the same score, so O is the plain mean of the
  attended V rows and LSE = s + ln(n) with s the common score. With equal scores the softmax weights are exactly
  1 (2^0), so O is an fp32 sum of the stored V values divided by n.
* A one-key range (position 0, or window = 1): O = V[pos].
These pin the mask bookkeeping (which keys a row attends: causal, window, tree ancestors, ragged lengths, chunk and
tile boundaries) independently of the oracle.
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import TORCH_DT

pytestmark = pytest.mark.gpu

TOL = 2e-5          # fp32 sum of at most a few thousand stored values, divided by n


def _const_keys(B, ML, NKV, HD, kvdt, seed):
    """K with one random row per (sequence, KV head) repeated over all positions; V random. Stored-dtype values."""
    rng = np.random.default_rng(seed)
    k1 = rng.normal(0, 0.5, (B, 1, NKV, HD)).astype(np.float32)
    k = np.repeat(k1, ML, axis=1)
    v = rng.normal(0, 0.5, (B, ML, NKV, HD)).astype(np.float32)
    kr, kb = oracle.round_to(k, kvdt)
    vr, vb = oracle.round_to(v, kvdt)
    return kr, vr, _dev(kb, kvdt), _dev(vb, kvdt)


def _dev(bits, kvdt):
    if kvdt == 0:
        return torch.from_numpy(np.ascontiguousarray(bits, np.float32)).cuda()
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(TORCH_DT[kvdt])


def _expect_mean(vr, b, keys, NQ, NKV):
    """[NQ, HD] mean of V rows `keys` of sequence b, each q-head reading its KV head."""
    GRP = NQ // NKV
    m = vr[b, keys].astype(np.float64).mean(axis=0)                     # [NKV, HD]
    return np.repeat(m, GRP, axis=0)


def _lse_expect(q, kr, b, n, NQ, NKV, HD, scale):
    GRP = NQ // NKV
    k = kr[b, 0].astype(np.float64)                                     # [NKV, HD]
    s = np.array([scale * np.dot(q[h].astype(np.float64), k[h // GRP]) for h in range(NQ)])
    return s + np.log(n)


@pytest.mark.parametrize("kvdt", [1, 2])
def test_decode_constant_keys_and_one_key(kvdt):
    """Streaming decode kernel: ragged lengths incl. a one-key sequence and lengths off the 16/512 boundaries."""
    B, NQ, NKV, HD, ML = 5, 24, 4, 256, 2100
    lens = np.array([1, 17, 512, 513, 2100], np.int32)
    kr, vr, K, V = _const_keys(B, ML, NKV, HD, kvdt, 1)
    q = np.random.default_rng(2).normal(0, 1, (B, NQ, HD)).astype(np.float32)
    qr, _ = oracle.round_to(q, kvdt)                                    # the MFMA operand type
    A.split_reserve(B, NQ, ML, HD)
    O = torch.empty(B * NQ * HD, device="cuda"); lse = torch.empty(B * NQ, device="cuda")
    A.attn_batch(torch.from_numpy(q).cuda().reshape(-1), K, V, O, B, 1, NQ, NKV, HD,
                 torch.from_numpy(lens - 1).cuda(), ML * NKV * HD, int(lens.max()) - 1, lse=lse)
    torch.cuda.synchronize()
    O = O.cpu().numpy().reshape(B, NQ, HD); lse = lse.cpu().numpy().reshape(B, NQ)
    for b in range(B):
        exp = _expect_mean(vr, b, np.arange(lens[b]), NQ, NKV)
        assert np.abs(O[b] - exp).max() < TOL, f"seq {b} len {lens[b]}"
        le = _lse_expect(qr[b], kr, b, lens[b], NQ, NKV, HD, 1.0 / np.sqrt(HD))
        assert np.abs(lse[b] - le).max() < 1e-4 * np.abs(le).max() + 1e-5, f"seq {b} lse"
    assert np.array_equal(O[0], np.repeat(vr[0, 0], NQ // NKV, axis=0)), "one key: O = V[0] exactly"


@pytest.mark.parametrize("kvdt", [1, 2])
def test_tree_verify_constant_keys(kvdt):
    """verify_kernel: a tree row averages exactly the committed prefix plus its ancestors-or-self."""
    B, NQ, NKV, HD, Tq = 4, 24, 4, 256, 8
    committed = np.array([3, 700, 1500, 2047], np.int32)
    ML = 2048 + Tq
    kr, vr, K, V = _const_keys(B, ML, NKV, HD, kvdt, 3)
    parents = [oracle.tree_random(90 + b, Tq, 2, 7)[0] for b in range(B)]
    anc = np.stack([oracle.tree_anc(p) for p in parents]).astype(np.uint32)
    q = np.random.default_rng(4).normal(0, 1, (B * Tq, NQ, HD)).astype(np.float32)
    max_pos = int((committed + Tq - 1).max())
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    O = torch.empty(B * Tq * NQ * HD, device="cuda")
    A.attn_batch(torch.from_numpy(q).cuda().reshape(-1), K, V, O, B, Tq, NQ, NKV, HD, torch.from_numpy(committed).cuda(),
                 ML * NKV * HD, max_pos, chunk=512, anc=torch.from_numpy(anc.reshape(-1).view(np.int32)).cuda())
    torch.cuda.synchronize()
    O = O.cpu().numpy().reshape(B, Tq, NQ, HD)
    for b in range(B):
        for t in range(Tq):
            keys = list(range(committed[b])) + [committed[b] + j for j in range(Tq) if (anc[b, t] >> j) & 1]
            exp = _expect_mean(vr, b, np.array(keys), NQ, NKV)
            assert np.abs(O[b, t] - exp).max() < TOL, f"seq {b} node {t}"


def test_verify_q_zero_random_keys():
    """Q = 0: uniform weights over each row's causal range, whatever K holds (verify rows, sliding window)."""
    B, NQ, NKV, HD, Tq, W, kvdt = 3, 16, 2, 128, 12, 300, 2
    committed = np.array([5, 290, 1000], np.int32)
    ML = 1024 + Tq
    rng = np.random.default_rng(5)
    k = rng.normal(0, 1, (B, ML, NKV, HD)).astype(np.float32)
    v = rng.normal(0, 0.5, (B, ML, NKV, HD)).astype(np.float32)
    _, kb = oracle.round_to(k, kvdt)
    vr, vb = oracle.round_to(v, kvdt)
    max_pos = int((committed + Tq - 1).max())
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    Q = torch.zeros(B * Tq * NQ * HD, device="cuda"); O = torch.empty_like(Q)
    A.attn_batch(Q, _dev(kb, kvdt), _dev(vb, kvdt), O, B, Tq, NQ, NKV, HD, torch.from_numpy(committed).cuda(),
                 ML * NKV * HD, max_pos, chunk=256, window=W)
    torch.cuda.synchronize()
    O = O.cpu().numpy().reshape(B, Tq, NQ, HD)
    for b in range(B):
        for t in range(Tq):
            pos = committed[b] + t
            keys = np.arange(max(0, pos - W + 1), pos + 1)
            assert np.abs(O[b, t] - _expect_mean(vr, b, keys, NQ, NKV)).max() < TOL, f"seq {b} token {t}"


@pytest.mark.parametrize("HD,NQ,NKV", [(256, 16, 8), (128, 16, 4)])
def test_prefill_constant_keys_and_window_one(HD, NQ, NKV):
    """Prefill kernel: causal prefix means (constant keys) and O_t = V[t] under window = 1."""
    T, kvdt = 300, 2
    kr, vr, K, V = _const_keys(1, T, NKV, HD, kvdt, 6)
    q = np.random.default_rng(7).normal(0, 1, (T, NQ, HD)).astype(np.float32)
    Q = torch.from_numpy(q).cuda().reshape(-1)
    O = torch.empty(T * NQ * HD, device="cuda")
    A.attn_prefill(Q, K.view(T, NKV, HD), V.view(T, NKV, HD), O, 1, T, NQ, NKV, HD)
    torch.cuda.synchronize()
    O = O.cpu().numpy().reshape(T, NQ, HD)
    csum = np.cumsum(vr[0].astype(np.float64), axis=0) / np.arange(1, T + 1)[:, None, None]     # [T, NKV, HD]
    exp = np.repeat(csum, NQ // NKV, axis=1)
    assert np.abs(O - exp).max() < TOL, "causal prefix means"
    O1 = torch.empty_like(Q)
    A.attn_prefill(Q, K.view(T, NKV, HD), V.view(T, NKV, HD), O1, 1, T, NQ, NKV, HD, window=1)
    torch.cuda.synchronize()
    assert np.array_equal(O1.cpu().numpy().reshape(T, NQ, HD), np.repeat(vr[0], NQ // NKV, axis=1)), "window 1"


def test_fp32_decode_constant_keys():
    """fp32 caches (decode_f32_kernel): ragged batch means."""
    B, NQ, NKV, HD, ML = 4, 16, 2, 256, 1500
    lens = np.array([1, 100, 777, 1500], np.int32)
    kr, vr, K, V = _const_keys(B, ML, NKV, HD, 0, 8)
    q = np.random.default_rng(9).normal(0, 1, (B, NQ, HD)).astype(np.float32)
    O = torch.empty(B * NQ * HD, device="cuda")
    A.attn_decode_batch(torch.from_numpy(q).cuda().reshape(-1), K, V, O, B, NQ, NKV, HD, 0, ML * NKV * HD,
                        base_b=torch.from_numpy(lens - 1).cuda())
    torch.cuda.synchronize()
    O = O.cpu().numpy().reshape(B, NQ, HD)
    for b in range(B):
        assert np.abs(O[b] - _expect_mean(vr, b, np.arange(lens[b]), NQ, NKV)).max() < TOL, f"seq {b}"
