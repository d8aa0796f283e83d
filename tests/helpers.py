"""Shared helpers of the parity tests: seeded inputs, device upload, the CPU oracle call and error metrics.

Tolerances: max-abs <= 1e-2 and mean-abs <= 1e-3 on outputs against the fp64 /
fp32-accumulate reference, LSE within 1e-4 relative.
"""
import numpy as np
import torch

import oracle

MAX_ABS = 1e-2
MEAN_ABS = 1e-3
LSE_REL = 1e-4

TORCH_DT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def dev_bits(bits, dtype_code):
    """Upload raw storage (uint16 bits for f16/bf16, float32 for fp32) as a tensor of that dtype."""
    if dtype_code == 0:
        return torch.from_numpy(np.ascontiguousarray(bits, np.float32)).cuda()
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(TORCH_DT[dtype_code])


def normal_cache(seed, B, max_len, NKV, HD, lens, sd, dtype_code, offset=0):
    """[B, max_len, NKV, HD] cache: keys < lens[b] ~ N(0, sd^2) rounded to the storage dtype, the rest zero.
    Returns (fp32 values, device tensor)."""
    vals = np.zeros((B, max_len, NKV, HD), np.float32)
    row = NKV * HD
    for b in range(B):
        n = int(lens[b]) * row
        vals[b, :lens[b]] = oracle.gen_normal(seed, n, 0.0, sd, offset=offset + b * max_len * row).reshape(lens[b], NKV, HD)
    v, bits = oracle.round_to(vals, dtype_code)
    return v, dev_bits(bits, dtype_code)


def oracle_rows(q, kvals, vvals, kv_off, pos, NQ, NKV, HD, scale=0.0, window=0, anc=None, tree_base=None, mode=0):
    return oracle.attention(q, kvals, vvals, kv_off, pos, NQ, NKV, HD, scale=scale, window=window, anc=anc,
                            tree_base=tree_base, mode=mode)


def errs(out, ref):
    d = np.abs(np.asarray(out, np.float64) - np.asarray(ref, np.float64))
    return float(d.max()), float(d.mean())


def lse_rel(lse, ref):
    lse = np.asarray(lse, np.float64); ref = np.asarray(ref, np.float64)
    return float((np.abs(lse - ref) / np.maximum(np.abs(ref), 1e-30)).max())


def assert_close(out, ref, what, lse=None, lse_ref=None, max_abs=MAX_ABS, mean_abs=MEAN_ABS, lse_tol=LSE_REL):
    out = np.asarray(out, np.float64)
    assert np.isfinite(out).all(), f"{what}: non-finite output"
    mx, mn = errs(out, ref)
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max_abs={mx:.3e} mean_abs={mn:.3e}"
    if lse is not None:
        r = lse_rel(lse, lse_ref)
        assert r <= lse_tol, f"{what}: lse rel err {r:.3e}"
    return mx, mn
