"""GPU parity of the fp32 attention launchers of kernels/attention.cuh (dgx_attn, dgx_attn_decode,
dgx_attn_decode_batch): fp32 Q/K/V/O, fp32 arithmetic.

Re-expresses tests/test_kernels.cu:94-108 (launch_attn against the host fp32 reference, S=5 GQA causal, max abs
error <= 1e-4), tests/test_decode_kernels.cu:24-34 (launch_attn_decode == launch_attn on the same inputs,
1e-4) and tests/test_batch_kernels.cu:21-36 (launch_attn_decode_batch == B single launch_attn_decode calls,
1e-4), all with the reference's own LCG inputs, plus the config-2 decode shape on fp32 caches against the fp64
oracle at the reference's fp32 bar (error / sum_j p_j |V_j,d| < 1e-5, tests/test_attn_decode_split.cu:87).
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import dev

pytestmark = pytest.mark.gpu


def test_attn_prefill_vs_host_reference():
    S, NQ, NKV, HD = 5, 4, 2, 128
    q, st = oracle.gen_lcg(0x9e3779b9, S * NQ * HD)     # tests/test_kernels.cu frand stream order: Q, K, V
    k, st = oracle.gen_lcg(st, S * NKV * HD)
    v, st = oracle.gen_lcg(st, S * NKV * HD)
    q, k = q * np.float32(0.2), k * np.float32(0.2)
    O = torch.empty(S * NQ * HD, device="cuda")
    A.attn(dev(q), dev(k), dev(v), O, S, NQ, NKV, HD)
    torch.cuda.synchronize()
    ref, _ = oracle.attention(q, k, v, np.zeros(S, np.int64), np.arange(S), NQ, NKV, HD, mode=1)
    e = np.abs(O.cpu().numpy().reshape(S, NQ, HD) - ref).max()
    assert e <= 1e-4, f"attention max abs err {e:.3e}"


@pytest.mark.parametrize("S,HD", [(6, 128), (6, 256), (3, 512)])
def test_attn_decode_equals_prefill(S, HD):
    NQ, NKV = 4, 2
    q, st = oracle.gen_lcg(2024, S * NQ * HD)
    k, st = oracle.gen_lcg(st, S * NKV * HD)
    v, st = oracle.gen_lcg(st, S * NKV * HD)
    q, k = q * np.float32(0.2), k * np.float32(0.2)
    O1 = torch.empty(S * NQ * HD, device="cuda"); O2 = torch.empty_like(O1)
    A.attn(dev(q), dev(k), dev(v), O1, S, NQ, NKV, HD)
    A.attn_decode(dev(q), dev(k), dev(v), O2, S, NQ, NKV, HD, 0)   # query i attends 0..i
    torch.cuda.synchronize()
    e = (O1 - O2).abs().max().item()
    assert e <= 1e-4, f"attn_decode vs prefill {e:.3e}"


@pytest.mark.parametrize("HD,NQ,NKV", [(256, 8, 2), (128, 16, 4), (512, 8, 2)])
def test_attn_decode_batch_equals_single(HD, NQ, NKV):
    B, base, maxlen = 8, 20, 64
    kvs = maxlen * NKV * HD
    q, st = oracle.gen_lcg(99, B * NQ * HD)
    kc, st = oracle.gen_lcg(st, B * kvs)
    vc, st = oracle.gen_lcg(st, B * kvs)
    Q, K, V = dev(q), dev(kc), dev(vc)
    Ob = torch.empty(B * NQ * HD, device="cuda")
    A.attn_decode_batch(Q, K, V, Ob, B, NQ, NKV, HD, base, kvs)
    Os = torch.empty_like(Ob)
    for b in range(B):
        o1 = torch.empty(NQ * HD, device="cuda")
        A.attn_decode(Q[b * NQ * HD:], K[b * kvs:], V[b * kvs:], o1, 1, NQ, NKV, HD, base)
        Os[b * NQ * HD:(b + 1) * NQ * HD] = o1
    torch.cuda.synchronize()
    e = (Ob - Os).abs().max().item()
    assert e <= 1e-4, f"attn_decode_batch vs single {e:.3e}"
    ref, _ = oracle.attention(q, kc, vc, np.arange(B) * kvs, np.full(B, base), NQ, NKV, HD)
    e2 = np.abs(Ob.cpu().numpy().reshape(B, NQ, HD) - ref).max()
    assert e2 <= 1e-4, f"attn_decode_batch vs fp64 oracle {e2:.3e}"


def test_fp32_decode_config2_shape():
    """Qwen3.5 full-attention decode shape on fp32 caches, ragged positions (device base_b)."""
    B, NQ, NKV, HD, ML = 6, 24, 4, 256, 4096
    rng = np.random.default_rng(12)
    lens = rng.integers(200, ML, size=B, endpoint=True).astype(np.int32)
    row = NKV * HD
    k = oracle.gen_normal(1, B * ML * row, 0.0, 0.5); v = oracle.gen_normal(2, B * ML * row, 0.0, 0.5)
    q = oracle.gen_normal(3, B * NQ * HD)
    O = torch.empty(B * NQ * HD, device="cuda")
    A.attn_decode_batch(dev(q), dev(k), dev(v), O, B, NQ, NKV, HD, 0, ML * row, base_b=dev(lens - 1))
    torch.cuda.synchronize()
    out = O.cpu().numpy().reshape(B, NQ, HD).astype(np.float64)
    ref, _ = oracle.attention(q, k, v, np.arange(B) * ML * row, lens - 1, NQ, NKV, HD)
    G = NQ // NKV
    kk = k.reshape(B, ML, NKV, HD).astype(np.float64); vv = np.abs(v.reshape(B, ML, NKV, HD).astype(np.float64))
    worst = 0.0
    for b in range(B):
        n = int(lens[b])
        for h in range(NQ):
            s = kk[b, :n, h // G] @ q.reshape(B, NQ, HD)[b, h].astype(np.float64) / np.sqrt(HD)
            pr = np.exp(s - s.max()); pr /= pr.sum()
            den = pr @ vv[b, :n, h // G]
            worst = max(worst, float((np.abs(out[b, h] - ref[b, h]) / den).max()))
    assert worst < 1e-5, f"fp32 decode normalised error {worst:.3e}"
