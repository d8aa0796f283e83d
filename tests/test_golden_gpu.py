"""The HIP kernels against the committed golden fixtures (tests/golden): decode (config 1, a gate-1 fp32 sliding
row, a ragged bf16 windowed batch), tree verify and chunked prefill, at the north-star tolerance (fp32 cache: the
1e-5 normalised bar of tests/test_attn_decode_split.cu:85-88)."""
import os

import numpy as np
import pytest
import torch

import dgx_attn as A
import cases
from helpers import TORCH_DT, assert_close, dev, dev_bits

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attn_golden.npz"))


def _expect(c):
    return FIX[c["name"] + ".o"].astype(np.float64), FIX[c["name"] + ".lse"].astype(np.float64)


def test_golden_config1():
    c = cases.case_config1()
    NQ, NKV, HD, L = c["NQ"], c["NKV"], c["HD"], c["ML"]
    eo, el = _expect(c)
    A.split_reserve(1, NQ, L, HD)
    O = torch.empty(NQ * HD, device="cuda"); lse = torch.empty(NQ, device="cuda")
    A.decode_split(dev(c["q"]), dev_bits(c["kb"], 1), dev_bits(c["vb"], 1), O, 1, NQ, NKV, HD, L - 1, 1, None, L - 1,
                   0, A.split_ns_cap(L), lse=lse)
    torch.cuda.synchronize()
    assert_close(O.cpu().numpy().reshape(eo.shape), eo, "config1", lse.cpu().numpy().reshape(el.shape), el)


def test_golden_gate1_fp32_window():
    c = cases.case_gate1_fp32_window()
    NQ, NKV, HD, L = c["NQ"], c["NKV"], c["HD"], c["ML"]
    eo, _ = _expect(c)
    A.split_reserve(1, NQ, L, HD)
    O = torch.empty(NQ * HD, device="cuda")
    A.decode_split(dev(c["q"]), dev(c["k"]), dev(c["v"]), O, 1, NQ, NKV, HD, L - 1, 1, None, L - 1, 0,
                   A.split_ns_cap(L), scale=1.0, window=1024)
    torch.cuda.synchronize()
    o = O.cpu().numpy().reshape(eo.shape).astype(np.float64)
    # error normalised by sum_j p_j |V_j,d| (fp64), as the reference's fp32 gate does
    pos, W, G = L - 1, c["window"], NQ // NKV
    lo = max(0, pos - W + 1)
    k = c["k"].reshape(L, NKV, HD).astype(np.float64); v = c["v"].reshape(L, NKV, HD).astype(np.float64)
    worst = 0.0
    for h in range(NQ):
        sc = k[lo:pos + 1, h // G] @ c["q"].reshape(NQ, HD)[h].astype(np.float64)
        p = np.exp(sc - sc.max()); p /= p.sum()
        den = p @ np.abs(v[lo:pos + 1, h // G])
        worst = max(worst, float((np.abs(o[0, h] - eo[0, h]) / den).max()))
    assert worst < 1e-5, f"fp32 normalised error {worst:.3e}"


def test_golden_window_batch_bf16():
    c = cases.case_window_batch_bf16()
    NQ, NKV, HD, ML = c["NQ"], c["NKV"], c["HD"], c["ML"]
    B = len(c["pos"])
    eo, el = _expect(c)
    A.split_reserve(B, NQ, ML, HD)
    dt = TORCH_DT[c["dt"]]
    Q = dev_bits(c["qb"], c["dt"]); O = torch.empty(B * NQ * HD, device="cuda", dtype=dt)
    lse = torch.empty(B * NQ, device="cuda")
    A.attn_batch(Q, dev_bits(c["kb"], c["dt"]), dev_bits(c["vb"], c["dt"]), O, B, 1, NQ, NKV, HD, dev(c["pos"]),
                 ML * NKV * HD, int(c["pos"].max()), window=c["window"], lse=lse)
    torch.cuda.synchronize()
    assert_close(O.float().cpu().numpy().reshape(eo.shape), eo, "window batch", lse.cpu().numpy().reshape(el.shape), el)


def test_golden_tree_f16():
    c = cases.case_tree_f16()
    NQ, NKV, HD, Tq, ML = c["NQ"], c["NKV"], c["HD"], c["Tq"], c["ML"]
    B = len(c["base_b"])
    eo, el = _expect(c)
    max_pos = int((c["base_b"] + Tq - 1).max())
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    dt = TORCH_DT[c["dt"]]
    Q = dev_bits(c["qb"], c["dt"]); O = torch.empty(B * Tq * NQ * HD, device="cuda", dtype=dt)
    lse = torch.empty(B * Tq * NQ, device="cuda")
    A.attn_batch(Q, dev_bits(c["kb"], c["dt"]), dev_bits(c["vb"], c["dt"]), O, B, Tq, NQ, NKV, HD, dev(c["base_b"]),
                 ML * NKV * HD, max_pos, chunk=512, anc=dev(c["anc"].reshape(-1).view(np.int32)), lse=lse)
    torch.cuda.synchronize()
    assert_close(O.float().cpu().numpy().reshape(eo.shape), eo, "tree", lse.cpu().numpy().reshape(el.shape), el)


def test_golden_prefill_lcg_bf16():
    c = cases.case_prefill_lcg_bf16()
    NQ, NKV, HD, Sq, base = c["NQ"], c["NKV"], c["HD"], c["Sq"], c["base"]
    eo, el = _expect(c)
    dt = TORCH_DT[c["dt"]]
    Q = dev_bits(c["qb"], c["dt"]); O = torch.empty(Sq * NQ * HD, device="cuda", dtype=dt)
    lse = torch.empty(Sq * NQ, device="cuda")
    K = dev_bits(c["kb"], c["dt"]).view(base + Sq, NKV, HD); V = dev_bits(c["vb"], c["dt"]).view(base + Sq, NKV, HD)
    A.attn_prefill(Q, K, V, O, 1, Sq, NQ, NKV, HD, base=base, lse=lse)
    torch.cuda.synchronize()
    assert_close(O.float().cpu().numpy().reshape(eo.shape), eo, "prefill", lse.cpu().numpy().reshape(el.shape), el)
