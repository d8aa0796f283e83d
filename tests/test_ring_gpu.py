"""GPU tests of the sliding-window ring-buffer KV layout (kv_cap > 0: key j lives in cache row j % kv_cap, the
layout runtime/decode_state_gemma4.h:9-16 reserves as kv_cap).

A ring holding the latest kv_cap keys of each sequence must give bit for bit the output of the linear cache
under the same window, for decode, verify-length runs and prefill (the ring's only effect is key addressing).
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
from helpers import TORCH_DT

pytestmark = pytest.mark.gpu


def _ring_of(lin, last, cap):
    """[B, cap, NKV, HD] ring holding keys (last[b]-cap, last[b]] of the linear cache lin [B, L, NKV, HD]."""
    B = lin.shape[0]
    ring = torch.full((B, cap) + tuple(lin.shape[2:]), float("nan"), device="cuda").to(lin.dtype)
    for b in range(B):
        j = np.arange(max(0, int(last[b]) - cap + 1), int(last[b]) + 1)
        ring[b, torch.from_numpy(j % cap).cuda()] = lin[b, torch.from_numpy(j).cuda()]
    return ring


@pytest.mark.parametrize("kvdt", [1, 2])
@pytest.mark.parametrize("Tq,cap", [(1, 1088), (3, 1088), (1, 1024), (12, 1088)])
def test_ring_decode_equals_linear(kvdt, Tq, cap):
    """cap = window: the ring is exactly full, and the tile holding a row's first key also reads ring rows that
    hold newer keys (masked)."""
    B, NQ, NKV, HD, W = 5, 16, 8, 256, 1024
    dt = TORCH_DT[kvdt]
    committed = np.array([40, 1100, 2300, 4999, 1023], np.int32)
    L = int(committed.max()) + Tq
    g = torch.Generator(device="cuda").manual_seed(17)
    K = (torch.randn(B, L, NKV, HD, device="cuda", generator=g) * 0.5).to(dt); V = (torch.randn(B, L, NKV, HD, device="cuda", generator=g) * 0.5).to(dt)
    last = committed + Tq - 1
    Kr, Vr = _ring_of(K, last, cap), _ring_of(V, last, cap)
    Q = torch.randn(B * Tq * NQ * HD, device="cuda").to(dt)
    base_b = torch.from_numpy(committed).cuda()
    max_pos = int(last.max())
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    O1 = torch.empty_like(Q); O2 = torch.empty_like(Q)
    A.attn_batch(Q, K, V, O1, B, Tq, NQ, NKV, HD, base_b, L * NKV * HD, max_pos, chunk=256, window=W)
    A.attn_batch_ex(Q, O2, B, Tq, NQ, NKV, HD, base_b, max_pos, K=Kr, V=Vr, kv_stride=cap * NKV * HD, chunk=256,
                    window=W, kv_cap=cap)
    torch.cuda.synchronize()
    assert torch.equal(O1.view(torch.int16), O2.view(torch.int16)), "ring decode differs from the linear cache"


@pytest.mark.parametrize("HD", [128, 256])
def test_ring_prefill_equals_linear(HD):
    NQ, NKV, W, Sq, base = 16, 8, 1024, 256, 3000
    cap = 1344                                            # >= W + Sq - 1, multiple of 64
    L = base + Sq
    g = torch.Generator(device="cuda").manual_seed(23)
    K = torch.randn(1, L, NKV, HD, device="cuda", generator=g).bfloat16(); V = torch.randn(1, L, NKV, HD, device="cuda", generator=g).bfloat16()
    Kr, Vr = _ring_of(K, np.array([L - 1]), cap), _ring_of(V, np.array([L - 1]), cap)
    Q = torch.randn(Sq * NQ * HD, device="cuda").bfloat16()
    O1 = torch.empty_like(Q); O2 = torch.empty_like(Q)
    A.attn_prefill(Q, K, V, O1, 1, Sq, NQ, NKV, HD, base=base, window=W)
    A.attn_prefill(Q, Kr, Vr, O2, 1, Sq, NQ, NKV, HD, base=base, window=W, kv_cap=cap)
    torch.cuda.synchronize()
    assert torch.equal(O1.view(torch.int16), O2.view(torch.int16)), "ring prefill differs from the linear cache"


def test_ring_validation():
    Q = torch.zeros(16 * 128, device="cuda").half(); O = torch.empty_like(Q)
    K = torch.zeros(1, 1024, 8, 128, device="cuda").half()
    for cap, win in [(1000, 512), (1024, 0), (1024, 1025)]:   # not a multiple of 64, no window, window > ring
        with pytest.raises(A.HipError):
            A.attn_batch_ex(Q, O, 1, 1, 16, 8, 128, None, 2000, K=K, V=K, kv_stride=0, window=win, kv_cap=cap, base=2000)
