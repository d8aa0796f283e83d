"""GPU parity of dgx_norm_rope_store (launch_norm_rope_store, kernels/norm_fused.cuh:84-133) against the fp64
oracle, in the three layouts the Gemma4 callers use: q into scratch (models/gemma4_decode.cu:340: slot stride
NQ*hd, row stride 0, positions base + s), k / v of a decode step into the cache (gemma4_decode.cu:353-354: slot
stride 0, row stride NKV*hd; v without scale and without RoPE) and a ragged batch with per-slot positions into
per-slot caches (models/gemma4_batch.cu:153). As the reference's gate (tests/test_norm_fused.cu) does, it also
checks that a row's bits do not depend on how many rows share the launch, and that nothing outside the written
rows changes."""
import numpy as np
import pytest
import torch

import dgx_attn as A
import oracle
from helpers import dev

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _inputs(seed, rows, hd, maxpos):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, hd)) * 2.0).astype(np.float32)
    x[np.arange(rows), np.arange(rows) % hd] *= 40.0                    # an outlier per row (the gate's pattern)
    w = rng.standard_normal(hd).astype(np.float32)
    cosT, sinT = oracle.rope_tables(maxpos, hd)
    return x, w, cosT, sinT


def _check(out, ref, ydt, what):
    """fp32: within a few fp32 roundings of the fp64 value (relative to the row's largest element); 16-bit: the
    stored value is the nearest-even rounding of a value within those roundings, so at most one unit in the last
    place away from the rounded fp64 value."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(out).all(), f"{what}: non-finite output"
    scale = np.abs(ref).max(axis=-1, keepdims=True)
    if ydt == 0:
        err = (np.abs(out - ref) / scale).max()
        assert err < 1e-5, f"{what}: normalised max error {err:.3e}"
    else:
        ulp = 2.0 ** -10 if ydt == 1 else 2.0 ** -7
        bound = ulp * np.maximum(np.abs(ref), 2.0 ** (-14 if ydt == 1 else -126)) + 4e-6 * scale
        bad = np.abs(out - ref) > bound
        assert not bad.any(), f"{what}: {int(bad.sum())} elements off by more than one 16-bit ulp"


@pytest.mark.parametrize("hd", [64, 128, 256, 512, 1024])
@pytest.mark.parametrize("ydt", [0, 1, 2])
def test_kv_append_layout_decode(hd, ydt):
    """k (norm + RoPE) and v (norm only) of Sq tokens at base .. base+Sq-1 into one sequence's cache."""
    nkv = 1 if hd >= 512 else 8
    Sq, base, L = 5, 4100, 4200
    rows = Sq * nkv
    x, w, cosT, sinT = _inputs(11 + hd + ydt, rows, hd, L)
    xv, _, _, _ = _inputs(91 + hd + ydt, rows, hd, L)
    dt = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}[ydt]
    sentinel = 7.0
    Kc = torch.full((L * nkv * hd,), sentinel, device="cuda", dtype=dt)
    Vc = torch.full((L * nkv * hd,), sentinel, device="cuda", dtype=dt)
    X, Wd, C, S = dev(x), dev(w), dev(cosT), dev(sinT)
    A.norm_rope_store(X, Wd, Kc, ydt, rows, nkv, hd, EPS, C, S, base=base, pos_step=1, slot_stride=0,
                      row_stride=nkv * hd, rope=True)
    A.norm_rope_store(dev(xv), None, Vc, ydt, rows, nkv, hd, EPS, C, S, base=base, pos_step=1, slot_stride=0,
                      row_stride=nkv * hd, rope=False)
    torch.cuda.synchronize()
    pos = base + np.arange(rows) // nkv
    kref = oracle.norm_rope_rows(x, w, EPS, cosT, sinT, pos, rope=True).reshape(Sq, nkv, hd)
    vref = oracle.norm_rope_rows(xv, None, EPS, rope=False).reshape(Sq, nkv, hd)
    k = Kc.float().cpu().numpy().reshape(L, nkv, hd)
    v = Vc.float().cpu().numpy().reshape(L, nkv, hd)
    _check(k[base:base + Sq], kref, ydt, f"k hd={hd} dt={ydt}")
    _check(v[base:base + Sq], vref, ydt, f"v hd={hd} dt={ydt}")
    for c in (k, v):
        assert (c[:base] == sentinel).all() and (c[base + Sq:] == sentinel).all(), "rows outside the step changed"


@pytest.mark.parametrize("hd", [256, 512])
def test_q_scratch_layout_and_row_identity(hd):
    """q rows into scratch (slot stride NQ*hd, row stride 0) for S = 1 .. 16 tokens: every launch matches the
    oracle and the last token's rows are bit-identical to a launch of that token alone."""
    NQ, base, L = 16, 4100, 4200
    x, w, cosT, sinT = _inputs(31 + hd, 16 * NQ, hd, L)
    X, Wd, C, S = dev(x.reshape(-1)), dev(w), dev(cosT), dev(sinT)            # flat: sliced by element offsets
    one = torch.empty(NQ * hd, device="cuda")
    A.norm_rope_store(X[15 * NQ * hd:], Wd, one, 0, NQ, NQ, hd, EPS, C, S, base=base + 15, pos_step=1,
                      slot_stride=NQ * hd, row_stride=0, rope=True)
    torch.cuda.synchronize()
    one_bits = one.view(torch.int32).cpu().numpy().copy()
    for Sn in (1, 5, 16):
        s0 = 16 - Sn
        Y = torch.empty(Sn * NQ * hd, device="cuda")
        A.norm_rope_store(X[s0 * NQ * hd:], Wd, Y, 0, Sn * NQ, NQ, hd, EPS, C, S, base=base + s0, pos_step=1,
                          slot_stride=NQ * hd, row_stride=0, rope=True)
        torch.cuda.synchronize()
        pos = base + s0 + np.arange(Sn * NQ) // NQ
        ref = oracle.norm_rope_rows(x[s0 * NQ:], w, EPS, cosT, sinT, pos, rope=True)
        out = Y.cpu().numpy().reshape(Sn * NQ, hd)
        _check(out, ref, 0, f"q hd={hd} S={Sn}")
        assert np.array_equal(Y.view(torch.int32).cpu().numpy()[-NQ * hd:], one_bits), "row identity"


@pytest.mark.parametrize("hd,nkv", [(256, 8), (512, 1)])
def test_ragged_batch_layout(hd, nkv):
    """A batch of B slots at ragged positions (pos_arr, pos_step 0) into per-slot caches (slot stride = capacity *
    NKV * hd, row stride NKV * hd), bf16, one launch."""
    B, cap = 8, 512
    rng = np.random.default_rng(hd)
    posv = rng.integers(0, cap, size=B).astype(np.int32)
    rows = B * nkv
    x, w, cosT, sinT = _inputs(51 + hd, rows, hd, cap)
    Kc = torch.zeros(B * cap * nkv * hd, device="cuda", dtype=torch.bfloat16)
    A.norm_rope_store(dev(x), dev(w), Kc, 2, rows, nkv, hd, EPS, dev(cosT), dev(sinT), base=0, pos_step=0,
                      pos_arr=dev(posv), slot_stride=cap * nkv * hd, row_stride=nkv * hd, rope=True)
    torch.cuda.synchronize()
    ref = oracle.norm_rope_rows(x, w, EPS, cosT, sinT, np.repeat(posv, nkv), rope=True).reshape(B, nkv, hd)
    k = Kc.float().cpu().numpy().reshape(B, cap, nkv, hd)
    _check(k[np.arange(B), posv], ref, 2, f"batch hd={hd}")
    written = np.zeros((B, cap), bool)
    written[np.arange(B), posv] = True
    assert (k[~written] == 0).all(), "rows other than the slots' positions changed"


@pytest.mark.parametrize("hd", [96, 100, 384, 768])
def test_head_dims_with_partners_through_lds(hd):
    """Head dims whose rotate-half partner is neither in the lane nor one lane swap away (any hd % 4 == 0, as the
    reference kernel takes them; at hd 100 a 4-element chunk straddles the halves): q rows in fp32 and k rows
    into a bf16 cache against the oracle."""
    NQ, S, base, L = 4, 3, 50, 64
    x, w, cosT, sinT = _inputs(61 + hd, S * NQ, hd, L)
    Y = torch.empty(S * NQ * hd, device="cuda")
    A.norm_rope_store(dev(x), dev(w), Y, 0, S * NQ, NQ, hd, EPS, dev(cosT), dev(sinT), base=base, pos_step=1,
                      slot_stride=NQ * hd, row_stride=0, rope=True)
    Kc = torch.zeros(L * NQ * hd, device="cuda", dtype=torch.bfloat16)
    A.norm_rope_store(dev(x), dev(w), Kc, 2, S * NQ, NQ, hd, EPS, dev(cosT), dev(sinT), base=base, pos_step=1,
                      slot_stride=0, row_stride=NQ * hd, rope=True)
    torch.cuda.synchronize()
    ref = oracle.norm_rope_rows(x, w, EPS, cosT, sinT, base + np.arange(S * NQ) // NQ, rope=True)
    _check(Y.cpu().numpy().reshape(S * NQ, hd), ref, 0, f"q hd={hd}")
    k = Kc.float().cpu().numpy().reshape(L, NQ * hd)
    _check(k[base:base + S].reshape(S * NQ, hd), ref, 2, f"k hd={hd}")
    assert (k[:base] == 0).all() and (k[base + S:] == 0).all()


def test_rejects_unsupported_shapes():
    X = torch.zeros(4 * 98, device="cuda")
    Y = torch.zeros(4 * 98, device="cuda")
    for rope in (True, False):                                          # whole 16-byte chunks: hd % 4 == 0
        with pytest.raises(A.HipError):
            A.norm_rope_store(X, None, Y, 0, 4, 4, 98, EPS, X, X, rope=rope)
    with pytest.raises(A.HipError):                                     # beyond the 1024-wide row buffer
        A.norm_rope_store(X, None, Y, 0, 1, 1, 1028, EPS, X, X, rope=True)
    A.norm_rope_store(X, None, Y, 0, 4, 4, 96, EPS, rope=False)         # plain norm: any hd % 4 == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("hd", [256, 512])
def test_norm_only_reference_accuracy_bar(hd):
    """Norm alone into fp32 at the reference gate's accuracy bar (tests/test_norm_fused.cu:32-56): relative error
    below 1e-6 on every element of magnitude at least 1e-3, against the fp64 oracle."""
    rows = 64
    x, w, _, _ = _inputs(71 + hd, rows, hd, 1)
    Y = torch.empty(rows * hd, device="cuda")
    A.norm_rope_store(dev(x), dev(w), Y, 0, rows, 1, hd, EPS, rope=False, slot_stride=hd, row_stride=0)
    torch.cuda.synchronize()
    ref = oracle.norm_rope_rows(x, w, EPS, rope=False)
    out = Y.cpu().numpy().astype(np.float64).reshape(rows, hd)
    big = np.abs(ref) >= 1e-3
    rel = np.abs(out - ref)[big] / np.abs(ref)[big]
    assert rel.max() < 1e-6, f"max relative error {rel.max():.3e}"


def test_all_tokens_at_one_position():
    """pos_step 0: every token of the launch takes position base (the rope_partial_batch form of the reference's
    gate, tests/test_norm_fused.cu:104-105)."""
    NQ, hd, S, base, L = 8, 256, 5, 777, 1024
    x, w, cosT, sinT = _inputs(81, S * NQ, hd, L)
    Y = torch.empty(S * NQ * hd, device="cuda")
    A.norm_rope_store(dev(x), dev(w), Y, 0, S * NQ, NQ, hd, EPS, dev(cosT), dev(sinT), base=base, pos_step=0,
                      slot_stride=NQ * hd, row_stride=0, rope=True)
    torch.cuda.synchronize()
    ref = oracle.norm_rope_rows(x, w, EPS, cosT, sinT, np.full(S * NQ, base), rope=True)
    _check(Y.cpu().numpy().reshape(S * NQ, hd), ref, 0, "pos_step 0")
