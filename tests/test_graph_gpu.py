"""HIP graph capture of the attention launches (the reference's Gemma decode captures its attention launches into a
graph, models/gemma4_decode_graph.cuh; the scratch is reserved before capture and launches never allocate,
models/gemma4_decode.cu:318).

Positions are read on the device and the decode / verify grids are sized by max_pos (or by the resident
workgroups), so one graph captured at the cache capacity serves every later step: the position buffers are
rewritten in place between replays. Each replay must equal an eager call on the same inputs bit for bit, with
eager work and synchronisations between the replays.
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle

pytestmark = pytest.mark.gpu


def _cache(seed, B, ML, NKV, HD):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(B, ML, NKV, HD, device="cuda", generator=g) * 0.5).half()


def test_decode_graph_replays_with_new_positions():
    B, NQ, NKV, HD, ML = 6, 24, 4, 256, 2048
    K, V = _cache(1, B, ML, NKV, HD), _cache(2, B, ML, NKV, HD)
    Q = torch.randn(B * NQ * HD, device="cuda").half()
    pos = torch.full((B,), 100, dtype=torch.int32, device="cuda")
    Og = torch.empty_like(Q); Oe = torch.empty_like(Q)
    stride = ML * NKV * HD
    A.split_reserve(B, NQ, ML, HD)
    A.attn_batch(Q, K, V, Og, B, 1, NQ, NKV, HD, pos, stride, ML - 1)        # eager first call (warm-up)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        A.attn_batch(Q, K, V, Og, B, 1, NQ, NKV, HD, pos, stride, ML - 1)
    rng = np.random.default_rng(7)
    for step in range(4):
        p = rng.integers(0, ML, size=B).astype(np.int32)
        pos.copy_(torch.from_numpy(p).cuda())
        g.replay()
        A.attn_batch(Q, K, V, Oe, B, 1, NQ, NKV, HD, pos, stride, ML - 1)
        torch.cuda.synchronize()
        assert torch.equal(Og.view(torch.int16), Oe.view(torch.int16)), f"replay {step} positions {p.tolist()}"


def test_tree_verify_graph_replays_with_new_bases():
    B, NQ, NKV, HD, Tq, ML = 4, 24, 4, 256, 8, 4096
    K, V = _cache(3, B, ML, NKV, HD), _cache(4, B, ML, NKV, HD)
    Q = torch.randn(B * Tq * NQ * HD, device="cuda").half()
    anc = np.stack([oracle.tree_anc(oracle.tree_random(50 + b, Tq, 2, 7)[0]) for b in range(B)]).astype(np.uint32)
    ancd = torch.from_numpy(anc.reshape(-1).view(np.int32)).cuda()
    base_b = torch.full((B,), 64, dtype=torch.int32, device="cuda")
    max_pos = ML - 1
    Og = torch.empty_like(Q); Oe = torch.empty_like(Q)
    stride = ML * NKV * HD
    A.split_reserve(B * Tq, NQ, ML, HD)
    A.attn_batch(Q, K, V, Og, B, Tq, NQ, NKV, HD, base_b, stride, max_pos, chunk=512, anc=ancd)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        A.attn_batch(Q, K, V, Og, B, Tq, NQ, NKV, HD, base_b, stride, max_pos, chunk=512, anc=ancd)
    rng = np.random.default_rng(8)
    for step in range(4):
        b = rng.integers(0, ML - Tq + 1, size=B).astype(np.int32)
        base_b.copy_(torch.from_numpy(b).cuda())
        g.replay()
        A.attn_batch(Q, K, V, Oe, B, Tq, NQ, NKV, HD, base_b, stride, max_pos, chunk=512, anc=ancd)
        torch.cuda.synchronize()
        assert torch.equal(Og.view(torch.int16), Oe.view(torch.int16)), f"replay {step} bases {b.tolist()}"


def test_long_tree_flash_graph_after_reserve_partials():
    """A tree-masked flash run of 40 tokens (more than 32) goes to the split kernel; with its partials reserved
    through dgx_flash_attn_reserve_partials the captured call allocates nothing and replays like the eager one."""
    Sq, NQ, NKV, HD, base = 40, 16, 4, 256, 700
    L = base + Sq
    K, V = _cache(9, 1, L, NKV, HD)[0], _cache(10, 1, L, NKV, HD)[0]
    Q = torch.randn(Sq * NQ * HD, device="cuda")
    anc = np.array([(1 << (min(t, 31) + 1)) - 1 if t % 3 else (1 << min(t, 31)) | 1 for t in range(Sq)],
                   np.uint64).astype(np.uint32)
    ancd = torch.from_numpy(anc.view(np.int32)).cuda()
    A.flash_reserve_partials(Sq * NQ * ((base + Sq - 1) // 512 + 1), HD)
    Og = torch.empty(Sq * NQ * HD, device="cuda"); Oe = torch.empty_like(Og)
    A.flash_attn(Q, K, V, Og, Sq, NQ, NKV, HD, base, anc=ancd)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        A.flash_attn(Q, K, V, Og, Sq, NQ, NKV, HD, base, anc=ancd)
    for step in range(3):
        Q.copy_(torch.randn(Sq * NQ * HD, device="cuda"))
        g.replay()
        A.flash_attn(Q, K, V, Oe, Sq, NQ, NKV, HD, base, anc=ancd)
        torch.cuda.synchronize()
        assert torch.equal(Og.view(torch.int32), Oe.view(torch.int32)), f"replay {step}"


def test_prefill_graph_replays_with_new_queries():
    T, NQ, NKV, HD = 256, 16, 8, 256
    g0 = torch.Generator(device="cuda").manual_seed(5)
    K = torch.randn(T, NKV, HD, device="cuda", generator=g0).bfloat16()
    V = torch.randn(T, NKV, HD, device="cuda", generator=g0).bfloat16()
    Q = torch.randn(T * NQ * HD, device="cuda", generator=g0).bfloat16()
    Og = torch.empty_like(Q); Oe = torch.empty_like(Q)
    A.attn_prefill(Q, K, V, Og, 1, T, NQ, NKV, HD)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        A.attn_prefill(Q, K, V, Og, 1, T, NQ, NKV, HD)
    for step in range(3):
        Q.copy_(torch.randn(T * NQ * HD, device="cuda", generator=g0).bfloat16())
        g.replay()
        A.attn_prefill(Q, K, V, Oe, 1, T, NQ, NKV, HD)
        torch.cuda.synchronize()
        assert torch.equal(Og.view(torch.int16), Oe.view(torch.int16)), f"replay {step}"


def test_norm_rope_store_then_decode_graph_replays():
    """The Gemma decode step's producer and consumer in one captured graph (models/gemma4_decode.cu:340-354 then the
    split decode): k rows normed, rotated and stored into a bf16 cache at per-slot positions (pos_arr), then the
    batch decode over that cache. Positions are rewritten in place between replays; every replay equals the eager
    pair bit for bit (cache and output)."""
    B, NQ, NKV, HD, ML = 4, 16, 8, 256, 1024
    g0 = torch.Generator(device="cuda").manual_seed(11)
    Kc = (torch.randn(B * ML * NKV * HD, device="cuda", generator=g0) * 0.5).bfloat16()
    Vc = (torch.randn(B * ML * NKV * HD, device="cuda", generator=g0) * 0.5).bfloat16()
    Kce, Vce = Kc.clone(), Vc.clone()
    xk = torch.randn(B * NKV * HD, device="cuda", generator=g0)
    xv = torch.randn(B * NKV * HD, device="cuda", generator=g0)
    w = torch.randn(HD, device="cuda", generator=g0)
    cosT, sinT = oracle.rope_tables(ML, HD)
    C, S = torch.from_numpy(cosT).cuda(), torch.from_numpy(sinT).cuda()
    Q = torch.randn(B * NQ * HD, device="cuda", generator=g0).bfloat16()
    pos = torch.full((B,), 10, dtype=torch.int32, device="cuda")
    stride = ML * NKV * HD
    Og = torch.empty_like(Q); Oe = torch.empty_like(Q)
    A.split_reserve(B, NQ, ML, HD)

    def layer(Kt, Vt, O):
        A.norm_rope_store(xk, w, Kt, 2, B * NKV, NKV, HD, 1e-6, C, S, pos_arr=pos, slot_stride=stride,
                          row_stride=NKV * HD, rope=True)
        A.norm_rope_store(xv, None, Vt, 2, B * NKV, NKV, HD, 1e-6, pos_arr=pos, slot_stride=stride,
                          row_stride=NKV * HD, rope=False)
        A.attn_batch(Q, Kt, Vt, O, B, 1, NQ, NKV, HD, pos, stride, ML - 1)

    layer(Kc, Vc, Og)                                                    # eager first call (warm-up), on both
    layer(Kce, Vce, Oe)                                                  # caches so they stay alike
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer(Kc, Vc, Og)
    rng = np.random.default_rng(12)
    for step in range(4):
        p = rng.integers(0, ML, size=B).astype(np.int32)
        pos.copy_(torch.from_numpy(p).cuda())
        graph.replay()
        layer(Kce, Vce, Oe)
        torch.cuda.synchronize()
        assert torch.equal(Kc.view(torch.int16), Kce.view(torch.int16)), f"replay {step} cache positions {p.tolist()}"
        assert torch.equal(Vc.view(torch.int16), Vce.view(torch.int16)), f"replay {step} v cache"
        assert torch.equal(Og.view(torch.int16), Oe.view(torch.int16)), f"replay {step} output"
