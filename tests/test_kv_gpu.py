"""GPU parity of the KV-cache store paths against the CPU oracle's RN-even rounding.

dgx_kv_store re-expresses kv_store() / kv_store_kernel (kernels/kv_store.cuh:76-113): fp32 -> cache dtype with
round-to-nearest-even, fp32 copied. dgx_kv_append stores a ragged batch (B slots x T tokens at per-slot positions)
in one launch, replacing the per-slot loops of models/gemma4_batch.cu:160-171 and models/qwen35_batch.cu:159-162;
it must give exactly the bits of the per-slot dgx_kv_store loop and leave every other cache row untouched.
Bit-exact throughout (integer-exact storage conversion).
"""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import TORCH_DT

pytestmark = pytest.mark.gpu


def _raw(t):
    return t.view(torch.int32).cpu().numpy() if t.dtype == torch.float32 else t.view(torch.int16).cpu().numpy().view(np.uint16)


def _special(n, seed):
    """Values that exercise the rounding: normals, ties, subnormals of both 16-bit formats, overflow, inf/nan."""
    x = oracle.gen_normal(seed, n, 0.0, 3.0)
    k = min(n, 64)
    extra = np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, -1e-8, 6e-8, 3.0e38, -3.0e38,
                      np.inf, -np.inf, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8],
                     np.float32)
    x[:len(extra)] = extra
    x[len(extra):k] = np.float32(np.nan) if k > len(extra) else x[len(extra):k]
    return x.astype(np.float32)


@pytest.mark.parametrize("kvdt", [0, 1, 2])
def test_kv_store_matches_oracle_rounding(kvdt):
    n = 4096 + 37                                         # ragged tail past a 256-thread block
    x = _special(n, 11)
    src = torch.from_numpy(x).cuda()
    dst = torch.zeros(n + 8, device="cuda", dtype=TORCH_DT[kvdt])
    A.kv_store(src, dst, n, kvdt, 0)
    torch.cuda.synchronize()
    got = _raw(dst)[:n]
    _, want = oracle.round_to(x, kvdt)
    want = want.view(np.int32) if kvdt == 0 else want
    nanw = np.isnan(x)
    assert np.array_equal(got[~nanw], want[~nanw]), "kv_store differs from RN-even"
    assert np.array_equal(_raw(dst)[n:], np.zeros(8, got.dtype)), "kv_store wrote past n"


@pytest.mark.parametrize("kvdt", [0, 1, 2])
@pytest.mark.parametrize("B,T,NKV,HD", [(16, 1, 4, 256), (5, 3, 8, 128), (1, 8, 1, 512)])
def test_kv_append_equals_per_slot_store(kvdt, B, T, NKV, HD):
    row = NKV * HD
    ML = 64
    rng = np.random.default_rng(B * 100 + T)
    pos = rng.integers(0, ML - T + 1, size=B).astype(np.int32)
    k = _special(B * T * row, 21); v = _special(B * T * row, 22)[::-1].copy()
    Kc = torch.full((B, ML, NKV, HD), 7.0, device="cuda").to(TORCH_DT[kvdt])
    Vc = torch.full((B, ML, NKV, HD), -7.0, device="cuda").to(TORCH_DT[kvdt])
    K2, V2 = Kc.clone(), Vc.clone()
    kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    A.kv_append(kd, vd, Kc, Vc, kvdt, B, T, ML * row, row, torch.from_numpy(pos).cuda())
    esz = 4 if kvdt == 0 else 2
    for b in range(B):                                    # the reference's per-slot loop
        for t in range(T):
            off = (b * ML + int(pos[b]) + t) * row
            r = (b * T + t) * row
            A.kv_store(kd[r:], K2.view(-1)[off:], row, kvdt, 0)
            A.kv_store(vd[r:], V2.view(-1)[off:], row, kvdt, 1)
    torch.cuda.synchronize()
    assert np.array_equal(_raw(Kc), _raw(K2)) and np.array_equal(_raw(Vc), _raw(V2)), "append != per-slot store"
    # stored rows equal the oracle's rounding; every other row untouched
    _, kb = oracle.round_to(k, kvdt); _, vb = oracle.round_to(v, kvdt)
    kb = kb.view(np.int32) if kvdt == 0 else kb
    vb = vb.view(np.int32) if kvdt == 0 else vb
    gk, gv = _raw(Kc).reshape(B, ML, row), _raw(Vc).reshape(B, ML, row)
    fill_k, fill_v = _raw(torch.full((1,), 7.0).to(TORCH_DT[kvdt]))[0], _raw(torch.full((1,), -7.0).to(TORCH_DT[kvdt]))[0]
    for b in range(B):
        sel = np.zeros(ML, bool); sel[pos[b]:pos[b] + T] = True
        src_k = kb.reshape(B, T, row)[b]; src_v = vb.reshape(B, T, row)[b]
        nk, nv = np.isnan(k.reshape(B, T, row)[b]), np.isnan(v.reshape(B, T, row)[b])
        assert np.array_equal(gk[b, sel][~nk], src_k[~nk]) and np.array_equal(gv[b, sel][~nv], src_v[~nv])
        assert (gk[b, ~sel] == fill_k).all() and (gv[b, ~sel] == fill_v).all(), "append touched other rows"
    _ = esz


def test_kv_append_uniform_base_and_empty():
    B, T, row, ML = 3, 2, 64, 16
    x = oracle.gen_normal(5, B * T * row)
    kd = torch.from_numpy(x).cuda()
    Kc = torch.zeros(B * ML * row, device="cuda", dtype=torch.bfloat16); Vc = torch.zeros_like(Kc)
    A.kv_append(kd, kd, Kc, Vc, 2, 0, T, ML * row, row, None, 3)          # nothing to do
    A.kv_append(kd, kd, Kc, Vc, 2, B, T, ML * row, row, None, 5)          # all slots at position 5
    torch.cuda.synchronize()
    _, want = oracle.round_bf16(x)
    got = _raw(Kc).reshape(B, ML, row)
    assert np.array_equal(got[:, 5:5 + T].reshape(-1), want)
    assert np.array_equal(_raw(Vc), _raw(Kc))
    with pytest.raises(A.HipError):
        A.kv_append(kd, kd, Kc, Vc, 2, B, T, ML * row + 2, row, None, 0)  # stride not a multiple of 4


@pytest.mark.parametrize("n", [0, 1, 7, 4099])
def test_f32_to_bf16_matches_the_oracle_rounding(n):
    """launch_f32_to_bf16 (kernels/elementwise.cuh:85-95): RN-even fp32 -> bf16, bit for bit against the oracle's
    rounding, including ties, signed zeros, subnormals, infinities and overflow; nothing past n is written."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 10).astype(np.float32)
    special = np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1e-40, -1e-40, np.inf, -np.inf, 3.4e38],
                       np.float32)
    x[:min(n, len(special))] = special[:min(n, len(special))]
    src = torch.from_numpy(x).cuda()
    dst = torch.full((n + 8,), 0x1234, dtype=torch.int16, device="cuda")
    A.f32_to_bf16(src, dst, n)
    torch.cuda.synchronize()
    out = dst.cpu().numpy().view(np.uint16)
    _, bits = oracle.round_bf16(x)
    assert np.array_equal(out[:n], bits)
    assert (out[n:] == 0x1234).all()
