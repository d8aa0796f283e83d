"""GPU tests of dgx_attn_batch_ex, the one-launch ragged decode / tree-verify entry for the Qwen callers.

- Per-slot K/V base pointers (the per-slot loops at models/qwen35_batch.cu:165-167 and :333-335 read each slot's
  own cache): every row must be bit-identical to dgx_attn_batch over one contiguous [B, max_len, NKV, HD] copy of
  the same caches, for plain decode and for a draft tree with ancestor masks.
- Output gate (the reference's launch_gate_sigmoid(attn, gate) after attention, models/qwen35_decode.cu:166): the
  gated output equals the ungated output times sigmoid(gate) to fp32 rounding, for fp32 and 16-bit gates.
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import TORCH_DT

pytestmark = pytest.mark.gpu


def _slots(seed, B, lens, NKV, HD, dt):
    """Separate per-slot caches (each just long enough) and a contiguous copy of them."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    ML = int(max(lens))
    Kc = torch.zeros(B, ML, NKV, HD, device="cuda", dtype=dt); Vc = torch.zeros_like(Kc)
    ks, vs = [], []
    for b in range(B):
        k = (torch.randn(int(lens[b]) + 3, NKV, HD, device="cuda", generator=g) * 0.5).to(dt)
        v = (torch.randn(int(lens[b]) + 3, NKV, HD, device="cuda", generator=g) * 0.5).to(dt)
        ks.append(k); vs.append(v)
        Kc[b, :lens[b]] = k[:lens[b]]; Vc[b, :lens[b]] = v[:lens[b]]
    Kp = torch.tensor([k.data_ptr() for k in ks], device="cuda", dtype=torch.int64)
    Vp = torch.tensor([v.data_ptr() for v in vs], device="cuda", dtype=torch.int64)
    return ks, vs, Kp, Vp, Kc, Vc, ML


@pytest.mark.parametrize("kvdt", [1, 2])
@pytest.mark.parametrize("Tq,tree", [(1, False), (8, True), (2, False)])
def test_slot_pointers_equal_contiguous(kvdt, Tq, tree):
    B, NQ, NKV, HD = 6, 24, 4, 256
    dt = TORCH_DT[kvdt]
    rng = np.random.default_rng(40 + Tq)
    committed = rng.integers(30, 2500, size=B).astype(np.int32)
    lens = committed + Tq
    ks, vs, Kp, Vp, Kc, Vc, ML = _slots(7 + Tq, B, lens, NKV, HD, dt)
    Q = torch.randn(B * Tq * NQ * HD, device="cuda").to(dt)
    anc = None
    if tree:
        a = np.zeros((B, Tq), np.uint32)
        for b in range(B):
            par = [-1] + [int(rng.integers(0, j)) for j in range(1, Tq)]
            a[b] = oracle.tree_anc(np.array(par))
        anc = torch.from_numpy(a.reshape(-1).view(np.int32)).cuda()
    base_b = torch.from_numpy(committed).cuda()
    max_pos = int(lens.max()) - 1
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    O1 = torch.empty_like(Q); O2 = torch.empty_like(Q)
    A.attn_batch(Q, Kc, Vc, O1, B, Tq, NQ, NKV, HD, base_b, ML * NKV * HD, max_pos, chunk=256, anc=anc)
    A.attn_batch_ex(Q, O2, B, Tq, NQ, NKV, HD, base_b, max_pos, Kp=Kp, Vp=Vp, kv_dtype=kvdt, chunk=256, anc=anc)
    torch.cuda.synchronize()
    assert torch.equal(O1.view(torch.int16), O2.view(torch.int16)), "per-slot pointers differ from the contiguous cache"


@pytest.mark.parametrize("gdt", [0, 1, 2])
def test_output_gate(gdt):
    B, Tq, NQ, NKV, HD = 4, 1, 24, 4, 256
    lens = np.array([700, 1300, 64, 2049], np.int32)
    _, _, _, _, Kc, Vc, ML = _slots(3, B, lens, NKV, HD, torch.float16)
    Q = torch.randn(B * NQ * HD, device="cuda").half()
    gate = (torch.randn(B * NQ * HD, device="cuda") * 3.0).to(TORCH_DT[gdt])
    base_b = torch.from_numpy(lens - 1).cuda()
    max_pos = int(lens.max()) - 1
    A.split_reserve(B, NQ, max_pos + 1, HD)
    O = torch.empty(B * NQ * HD, device="cuda"); Og = torch.empty_like(O)
    Qf = Q.float()
    A.attn_batch_ex(Qf, O, B, Tq, NQ, NKV, HD, base_b, max_pos, K=Kc, V=Vc, kv_stride=ML * NKV * HD)
    A.attn_batch_ex(Qf, Og, B, Tq, NQ, NKV, HD, base_b, max_pos, K=Kc, V=Vc, kv_stride=ML * NKV * HD, gate=gate)
    torch.cuda.synchronize()
    g = gate.float().cpu().numpy().astype(np.float64)
    want = O.cpu().numpy().astype(np.float64) / (1.0 + np.exp(-g))
    got = Og.cpu().numpy().astype(np.float64)
    err = np.abs(got - want)
    assert (err <= 4e-6 * np.abs(want) + 1e-7).all(), f"gate: max err {err.max():.3e}"


def test_batch_ex_validation():
    Q = torch.zeros(24 * 256, device="cuda").half(); O = torch.empty_like(Q)
    ptrs = torch.zeros(1, device="cuda", dtype=torch.int64)
    with pytest.raises(A.HipError):                       # Kp without Vp
        A.attn_batch_ex(Q, O, 1, 1, 24, 4, 256, None, 10, Kp=ptrs, kv_dtype=1)
    with pytest.raises(A.HipError):                       # neither pointers nor caches
        A.attn_batch_ex(Q, O, 1, 1, 24, 4, 256, None, 10, kv_dtype=1)


@pytest.mark.parametrize("n,offset", [(24 * 256 * 4, 0), (1001, 0), (4099, 1)])
def test_standalone_gate_matches_fused_and_sigmoid(n, offset):
    """launch_gate_sigmoid after attention (models/qwen35_decode.cu:166): against fp64 y * sigmoid(g) within the fp32
    rounding bar of the fused gate, on aligned and unaligned arrays with tails; and, on an fp32 attention output, bit
    for bit equal to the gate fused into dgx_attn_batch_ex."""
    g0 = torch.Generator(device="cuda").manual_seed(n)
    yb = torch.randn(n + offset, device="cuda", generator=g0)
    gb = torch.randn(n + offset, device="cuda", generator=g0) * 4.0
    y, gate = yb[offset:], gb[offset:]
    y0 = y.cpu().numpy().astype(np.float64)
    A.gate_sigmoid(y, gate, n)
    torch.cuda.synchronize()
    want = y0 / (1.0 + np.exp(-gate.cpu().numpy().astype(np.float64)))
    err = np.abs(y.cpu().numpy().astype(np.float64) - want)
    assert (err <= 4e-6 * np.abs(want) + 1e-7).all(), f"max err {err.max():.3e}"
    if offset == 0 and n == 24 * 256 * 4:
        B, Tq, NQ, NKV, HD = 4, 1, 24, 4, 256
        lens = np.array([700, 1300, 64, 2049], np.int32)
        _, _, _, _, Kc, Vc, ML = _slots(3, B, lens, NKV, HD, torch.float16)
        Qf = torch.randn(B * NQ * HD, device="cuda", generator=g0)
        base_b = torch.from_numpy(lens - 1).cuda()
        A.split_reserve(B, NQ, int(lens.max()), HD)
        O = torch.empty(B * NQ * HD, device="cuda"); Og = torch.empty_like(O)
        A.attn_batch_ex(Qf, O, B, Tq, NQ, NKV, HD, base_b, int(lens.max()) - 1, K=Kc, V=Vc, kv_stride=ML * NKV * HD)
        A.attn_batch_ex(Qf, Og, B, Tq, NQ, NKV, HD, base_b, int(lens.max()) - 1, K=Kc, V=Vc, kv_stride=ML * NKV * HD,
                        gate=gate)
        A.gate_sigmoid(O, gate, B * NQ * HD)
        torch.cuda.synchronize()
        assert torch.equal(O.view(torch.int32), Og.view(torch.int32)), "separate gate differs from the fused one"
