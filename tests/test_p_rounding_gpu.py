"""Rows that attend few keys with outputs of large magnitude: the probabilities enter the PV matrix product as
16-bit MFMA operands, and a bf16 operand alone carries them to 8 significant bits (relative error 2^-9, 4.5e-3 on
an output of magnitude 2.5 from a two-key row). The kernels split bf16 probabilities into a hi + lo pair, so the
kernel's own error stays far below the bar; what remains on a bf16 output is its final rounding (half a bf16 ulp:
3.9e-3 below |O| = 2, 7.8e-3 below 4, 1.56e-2 from 4 on, which the 1e-2 bar cannot hold at |O| >= 4).

The first case is the shape a random sweep found at max-abs 1.002e-2 with single bf16 probabilities
(HD 512, NQ = NKV = 8, 200 tokens from position 0, key split 512, bf16 output)."""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import TORCH_DT, assert_close, dev, errs, normal_cache, oracle_rows

pytestmark = pytest.mark.gpu

# The kernel's own error with an fp32 output (bf16 inputs exactly representable, fp32 accumulation): the P rounding
# it had before the hi + lo split reached 4.5e-3 here.
KERNEL_MAX_ABS = 1e-3


def _prefill(seed, HD, NQ, NKV, Sq, base, kv_split, kvdt, out_dt, vsd=1.0):
    L = base + Sq
    kv, kd = normal_cache(seed + 11, 1, L, NKV, HD, [L], 1.0, kvdt)
    vv, vd = normal_cache(seed + 12, 1, L, NKV, HD, [L], vsd, kvdt)
    q = oracle.gen_normal(seed + 13, Sq * NQ * HD)
    qr, _ = oracle.round_to(q, kvdt)
    Q = dev(qr, TORCH_DT[out_dt])
    O = torch.empty(Sq * NQ * HD, device="cuda", dtype=TORCH_DT[out_dt])
    lse = torch.empty(Sq * NQ, device="cuda")
    A.attn_prefill(Q, kd.view(L, NKV, HD), vd.view(L, NKV, HD), O, 1, Sq, NQ, NKV, HD, base=base, kv_split=kv_split,
                   lse=lse)
    torch.cuda.synchronize()
    ref, ref_lse = oracle_rows(qr, kv, vv, np.zeros(Sq, np.int64), base + np.arange(Sq), NQ, NKV, HD)
    return O.float().cpu().numpy().reshape(Sq, NQ, HD), ref, lse.cpu().numpy().reshape(Sq, NQ), ref_lse


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
@pytest.mark.parametrize("kv_split", [512, 0])
def test_sweep_case_hd512(seed, kv_split):
    """The sweep's shape, bf16 output, at the north-star bar; the same inputs with an fp32 output at 1e-3."""
    out, ref, lse, ref_lse = _prefill(2000 + seed, 512, 8, 8, 200, 0, kv_split, 2, 2)
    assert_close(out, ref, f"hd512 bf16 out seed {seed} split {kv_split}", lse, ref_lse)
    out, ref, lse, ref_lse = _prefill(2000 + seed, 512, 8, 8, 200, 0, kv_split, 2, 0)
    mx, _ = errs(out, ref)
    assert mx <= KERNEL_MAX_ABS, f"hd512 fp32 out seed {seed} split {kv_split}: kernel max-abs {mx:.3e}"


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("kvdt", [2, 1])
@pytest.mark.parametrize("HD", [128, 256])
def test_few_key_rows_prefill(seed, kvdt, HD):
    """The first tokens of a prompt (1..8 keys each) with V ~ N(0, 1.5^2): 16-bit output at the bar, fp32 output at
    the kernel bound."""
    out, ref, lse, ref_lse = _prefill(3000 + seed, HD, 8, 4, 64, 0, 0, kvdt, 0, vsd=1.5)
    mx, _ = errs(out, ref)
    assert mx <= KERNEL_MAX_ABS, f"fp32 out HD {HD} kv {kvdt} seed {seed}: kernel max-abs {mx:.3e}"
    # 16-bit output: keep |O| < 4 (V sd 1.0) so the output's own rounding fits the bar
    out, ref, lse, ref_lse = _prefill(3000 + seed, HD, 8, 4, 64, 0, 0, kvdt, kvdt, vsd=1.0)
    assert_close(out, ref, f"16-bit out HD {HD} kv {kvdt} seed {seed}", lse, ref_lse)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("kvdt", [2, 1])
@pytest.mark.parametrize("T,HD", [(1, 256), (4, 256), (1, 512), (8, 128)])
def test_few_key_rows_split(seed, kvdt, T, HD):
    """Decode / verify rows over 1..4 committed keys through dgx_attn_batch (decode_stream_kernel at T = 1 and
    HD <= 256, verify_kernel at T > 1, split_kernel at HD 512), fp32 output at the kernel bound."""
    B, NQ, NKV = 4, 8, 2
    committed = (np.arange(B) % 4).astype(np.int32)
    ML = int(committed.max()) + T
    lens = committed + T
    kv, kd = normal_cache(4000 + seed, B, ML, NKV, HD, lens, 1.0, kvdt)
    vv, vd = normal_cache(4100 + seed, B, ML, NKV, HD, lens, 1.5, kvdt)
    q = oracle.gen_normal(4200 + seed, B * T * NQ * HD)
    qr, _ = oracle.round_to(q, kvdt)
    max_pos = int((committed + T - 1).max())
    A.split_reserve(B * T * 2, NQ, max_pos + 1, HD)
    O = torch.empty(B * T * NQ * HD, device="cuda"); lse = torch.empty(B * T * NQ, device="cuda")
    A.attn_batch(dev(qr), kd, vd, O, B, T, NQ, NKV, HD, dev(committed), ML * NKV * HD, max_pos, lse=lse)
    torch.cuda.synchronize()
    pos = (committed[:, None] + np.arange(T)[None, :]).reshape(-1)
    off = np.repeat(np.arange(B, dtype=np.int64) * ML * NKV * HD, T)
    ref, ref_lse = oracle_rows(qr, kv, vv, off, pos, NQ, NKV, HD)
    out = O.cpu().numpy().reshape(B * T, NQ, HD)
    mx, _ = errs(out, ref)
    assert mx <= KERNEL_MAX_ABS, f"T {T} HD {HD} kv {kvdt} seed {seed}: kernel max-abs {mx:.3e}"
    assert_close(out, ref, f"T {T} HD {HD} kv {kvdt} seed {seed}", lse.cpu().numpy().reshape(-1, NQ), ref_lse)


def _half_ulp_bf16(x):
    """Half a bf16 ulp at |x| (8 significant bits): 2^(floor(log2|x|) - 8)."""
    x = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(x)) - 8)


# Cases of a 5,642-case random sweep (the configuration generator of test_random_shapes_gpu.py, seeds 100-2920)
# that miss the north-star numbers only where no bf16 output or relative LSE can meet them: rows with |O| >= 4,
# where the bf16 output itself is 1.56e-2 coarse, and rows whose LSE is within 1e-2 of zero.
SWEEP_LIMIT_CASES = [1529, 1869, 2278, 2647]


@pytest.mark.parametrize("s", SWEEP_LIMIT_CASES)
def test_sweep_cases_at_the_bf16_limit(s):
    """The kernel's fp32 result is within 1e-4 of the oracle everywhere; the bf16 output is within half a bf16 ulp
    of |O| (plus that 1e-4) of it, which exceeds 1e-2 only from |O| = 4 on; the LSE is within 1e-5 absolute (the
    relative bar is kept for |LSE| >= 1)."""
    import test_random_shapes_gpu as R
    c = R._prefill_cfg(2000 + s, hds=(128, 256, 512))
    HD, NKV, NQ, Sq, base = c["HD"], c["NKV"], c["NQ"], c["Sq"], c["base"]
    L = base + Sq
    kv, kd = normal_cache(s + 11, 1, L, NKV, HD, [L], 1.0, 2)
    vv, vd = normal_cache(s + 12, 1, L, NKV, HD, [L], 1.0, 2)
    q = oracle.gen_normal(s + 13, Sq * NQ * HD)
    qr, _ = oracle.round_to(q, 2)
    ref, ref_lse = oracle_rows(qr, kv, vv, np.zeros(Sq, np.int64), base + np.arange(Sq), NQ, NKV, HD,
                               window=c["window"])
    for odt in (0, 2):
        Q = dev(qr, TORCH_DT[odt])
        O = torch.empty(Sq * NQ * HD, device="cuda", dtype=TORCH_DT[odt])
        lse = torch.empty(Sq * NQ, device="cuda")
        A.attn_prefill(Q, kd.view(L, NKV, HD), vd.view(L, NKV, HD), O, 1, Sq, NQ, NKV, HD, base=base,
                       window=c["window"], kv_split=c["kv_split"], lse=lse)
        torch.cuda.synchronize()
        out = O.float().cpu().numpy().reshape(Sq, NQ, HD).astype(np.float64)
        d = np.abs(out - ref)
        if odt == 0:
            assert d.max() <= 1e-4, f"case {s} {c}: fp32-output kernel error {d.max():.3e}"
        else:
            over = d - (_half_ulp_bf16(np.abs(ref) + 1e-4) + 1e-4)
            assert over.max() <= 0, f"case {s} {c}: bf16 output beyond its rounding by {over.max():.3e}"
            assert d[np.abs(ref) < 4].max() <= 1e-2, f"case {s}: bf16 output error below |O| = 4"
        le = np.abs(lse.cpu().numpy().reshape(Sq, NQ).astype(np.float64) - ref_lse)
        assert le.max() <= 1e-5, f"case {s}: LSE abs error {le.max():.3e}"
        big = np.abs(ref_lse) >= 1
        assert (le[big] / np.abs(ref_lse[big])).max() <= 1e-4, f"case {s}: LSE rel error where |LSE| >= 1"
