"""GPU test of dgx_attn_batch_noalloc, the allocation-free variant of dgx_attn_batch whose split partials live in
the library's fixed device array: on two calls in a row (the second with a smaller input) its outputs and LSE
must equal dgx_attn_batch's bit for bit (both run the same kernels), for ragged decode (the streaming decode
kernel) and for tree verify (the verify kernel); a call whose partials exceed the fixed array is rejected."""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle

pytestmark = pytest.mark.gpu


def _case(seed, B, Tq, NQ, NKV, HD, ML, lo, tree):
    g = torch.Generator(device="cuda").manual_seed(seed)
    K = (torch.randn(B, ML, NKV, HD, device="cuda", generator=g) * 0.5).half()
    V = (torch.randn(B, ML, NKV, HD, device="cuda", generator=g) * 0.5).half()
    Q = torch.randn(B * Tq * NQ * HD, device="cuda", generator=g).half()
    committed = np.random.default_rng(seed).integers(lo, ML - Tq, size=B, endpoint=True).astype(np.int32)
    anc = None
    if tree:
        a = np.stack([oracle.tree_anc(oracle.tree_random(seed + b, Tq, 2, 7)[0]) for b in range(B)]).astype(np.uint32)
        anc = torch.from_numpy(a.reshape(-1).view(np.int32)).cuda()
    return K, V, Q, torch.from_numpy(committed).cuda(), int(committed.max()) + Tq - 1, anc


def _compare(seed, B, Tq, NQ, NKV, HD, ML, lo, chunk, tree):
    print(f"noalloc case seed={seed} B={B} Tq={Tq} ML={ML} chunk={chunk} tree={tree}", flush=True)
    K, V, Q, base_b, max_pos, anc = _case(seed, B, Tq, NQ, NKV, HD, ML, lo, tree)
    stride = ML * NKV * HD
    O1, O2 = torch.empty_like(Q), torch.empty_like(Q)
    l1, l2 = torch.empty(B * Tq * NQ, device="cuda"), torch.empty(B * Tq * NQ, device="cuda")
    A.split_reserve(B * Tq * max(1, -(-A.split_chunk() // chunk)), NQ, max_pos + 1, HD)
    A.attn_batch(Q, K, V, O1, B, Tq, NQ, NKV, HD, base_b, stride, max_pos, chunk=chunk, anc=anc, lse=l1)
    A.attn_batch_noalloc(Q, K, V, O2, B, Tq, NQ, NKV, HD, base_b, stride, max_pos, chunk=chunk, anc=anc, lse=l2)
    torch.cuda.synchronize()
    assert torch.equal(O1.view(torch.int16), O2.view(torch.int16)), "noalloc output differs from dgx_attn_batch"
    assert torch.equal(l1.view(torch.int32), l2.view(torch.int32)), "noalloc LSE differs from dgx_attn_batch"


def test_noalloc_decode_two_calls():
    _compare(1, 16, 1, 24, 4, 256, 8192, 256, 512, False)     # BASELINE config 2 shape
    _compare(2, 3, 1, 24, 4, 256, 2048, 1, 256, False)        # smaller second call


def test_noalloc_tree_verify_two_calls():
    _compare(3, 8, 8, 24, 4, 256, 8192, 2048, 512, True)
    _compare(4, 2, 8, 24, 4, 256, 1024, 100, 512, True)


def test_noalloc_rejects_oversize():
    B, NQ, NKV, HD, ML = 64, 32, 4, 512, 65536
    Q = torch.zeros(B * NQ * HD, device="cuda").half(); O = torch.empty_like(Q)
    K = torch.zeros(1, 64, NKV, HD, device="cuda").half()
    pos = torch.zeros(B, dtype=torch.int32, device="cuda")
    with pytest.raises(A.HipError):                  # 64*32*512 partials x 514 floats >> 64 MiB
        A.attn_batch_noalloc(Q, K, K, O, B, 1, NQ, NKV, HD, pos, 0, ML - 1, chunk=128)
