"""Benchmark of the MI355X attention hot path (BASELINE.json metric).

Headline (`value`): batched split-KV decode at BASELINE.json config 2 - B=16, Hq=24, Hkv=4, hd=256, f16 KV cache
[16, 8192, 4, 256], ragged context lengths L_b ~ U[256, 8192] (seeded), split 512 + LSE combine, one query token
per sequence - as algorithmic HBM GB/s: bytes = sum_b L_b * Hkv * hd * 2 (K and V) * 2 B + |Q| + |O|.
Alongside: causal flash prefill at config 3 (T=1024, Hq=16, Hkv=8, hd=256, bf16) as TFLOP/s with
flops = 4 * hd * Hq * sum of attended keys, and the other BASELINE.json configs in µs per layer call.
A step is one layer call (the split kernel plus the LSE combine kernel for decode).

Timing: W untimed warm-up steps, then exactly K steps between torch.cuda.synchronize() calls, measured with
HIP events recorded on the stream the kernels are launched on (torch's current stream).
cpu_baseline: the oracle's fp32 host attention (restating tests/test_kernels.cu:94-108) on the same decode
inputs, timed on the host cores of this box.
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dgx-serving_amd"))
import dgx_attn as A  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def timed(fn, steps, warmup, kernel=False):
    """ms per step over `steps` calls (HIP events on the launch stream). kernel=True also returns the average
    duration of the library's main kernel, from a second pass of `steps` calls with HIP events around that
    kernel's launches (the extra event records between the kernels would inflate the first pass's clock)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    if kernel:
        ms = timed(fn, steps, 0)
        A.timing(True)
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    if not kernel:
        return e0.elapsed_time(e1) / steps        # ms per step
    kms, n = A.timing_read()
    A.timing(False)
    assert n == steps, f"timed {n} kernel launches for {steps} steps"
    return ms, kms


def decode_workload(seed=2026):
    B, NQ, NKV, HD, ML = 16, 24, 4, 256, 8192
    rng = np.random.default_rng(seed)
    lens = rng.integers(256, ML, size=B, endpoint=True).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(seed)
    K = (torch.randn(B, ML, NKV, HD, device="cuda", generator=g) * 0.5).half()
    V = (torch.randn(B, ML, NKV, HD, device="cuda", generator=g) * 0.5).half()
    Q = torch.randn(B * NQ * HD, device="cuda", generator=g).half()
    O = torch.empty_like(Q)
    pos = torch.from_numpy(lens - 1).cuda()
    return dict(B=B, NQ=NQ, NKV=NKV, HD=HD, ML=ML, lens=lens, K=K, V=V, Q=Q, O=O, pos=pos)


def run_decode(w, steps, warmup, chunk=512, copies=1):
    B, NQ, NKV, HD, ML = w["B"], w["NQ"], w["NKV"], w["HD"], w["ML"]
    max_pos = int(w["lens"].max()) - 1
    # the reservation is sized at the library's default chunk; smaller chunks need proportionally more partials
    A.split_reserve(B * max(1, -(-A.split_chunk() // chunk)), NQ, ML, HD)
    kvs = [(w["K"], w["V"])]
    for i in range(1, copies):
        kvs.append((torch.randn_like(w["K"]) * 0.5, torch.randn_like(w["V"]) * 0.5))
    it = [0]

    def fn():
        K, V = kvs[it[0] % len(kvs)]
        it[0] += 1
        A.attn_batch(w["Q"], K, V, w["O"], B, 1, NQ, NKV, HD, w["pos"], ML * NKV * HD, max_pos, chunk=chunk)
    ms, kms = timed(fn, steps, warmup, kernel=True)
    nbytes = int(w["lens"].sum()) * NKV * HD * 2 * 2 + 2 * B * NQ * HD * 2
    return ms, nbytes, kms


def run_prefill(steps, warmup, T=1024, NQ=16, NKV=8, HD=256, base=0, window=0, kv_split=0, seed=3):
    g = torch.Generator(device="cuda").manual_seed(seed)
    L = base + T
    K = torch.randn(L, NKV, HD, device="cuda", generator=g).bfloat16()
    V = torch.randn(L, NKV, HD, device="cuda", generator=g).bfloat16()
    Q = torch.randn(T * NQ * HD, device="cuda", generator=g).bfloat16()
    O = torch.empty_like(Q)
    fn = lambda: A.attn_prefill(Q, K, V, O, 1, T, NQ, NKV, HD, base=base, kv_split=kv_split, window=window)
    ms = timed(fn, steps, warmup)
    pos = base + np.arange(T, dtype=np.int64)
    lo = np.maximum(0, pos - window + 1) if window > 0 else np.zeros_like(pos)
    pairs = int((pos - lo + 1).sum())
    flops = 4.0 * HD * NQ * pairs
    return ms, flops


def run_tree(steps, warmup, seed=5, runs=None):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    B, NQ, NKV, HD, Tq = 16, 24, 4, 256, 8
    rng = np.random.default_rng(seed)
    committed = rng.integers(2048, 16384, size=B, endpoint=True).astype(np.int32)
    # 2-wide random tree of 8 nodes in BFS order, depth <= 7 (parents precede children)
    anc = np.zeros((B, Tq), np.uint32)
    for b in range(B):
        par = [-1]; kids = [0] * Tq
        for j in range(1, Tq):
            cand = [p for p in range(j) if kids[p] < 2]
            p = int(rng.choice(cand)); par.append(p); kids[p] += 1
        for j in range(Tq):
            m, x = 0, j
            while x >= 0:
                m |= 1 << x; x = par[x]
            anc[b, j] = m
    ML = 16384 + Tq
    g = torch.Generator(device="cuda").manual_seed(seed)
    K = (torch.randn(B, ML, NKV, HD, device="cuda", generator=g) * 0.5).half()
    V = (torch.randn(B, ML, NKV, HD, device="cuda", generator=g) * 0.5).half()
    Q = torch.randn(B * Tq * NQ * HD, device="cuda", generator=g).half()
    O = torch.empty_like(Q)
    base_b = torch.from_numpy(committed).cuda()
    ancd = torch.from_numpy(anc.reshape(-1).view(np.int32)).cuda()
    max_pos = int(committed.max()) + Tq - 1
    A.split_reserve(B * Tq, NQ, max_pos + 1, HD)
    # split chunk: a free parameter for tree verify (config 5 names none); with per-sequence chunk cuts 640 keys
    # measured fastest (256: 166, 384: 149, 512: 147-150, 640: 140, 768: 144, 1024: 154 us per call)
    chunk = int(os.environ.get("BENCH_TREE_CHUNK", "640"))
    # 0: per-sequence chunks (the library default, batch-invariant), 1: equal runs over the batch
    prev = A.verify_runs(int(os.environ.get("BENCH_VERIFY_RUNS", "0")) if runs is None else runs)
    fn = lambda: A.attn_batch(Q, K, V, O, B, Tq, NQ, NKV, HD, base_b, ML * NKV * HD, max_pos, chunk=chunk, anc=ancd)
    ms = timed(fn, steps, warmup)
    A.verify_runs(prev)
    nbytes = int((committed + Tq).sum()) * NKV * HD * 4 + 2 * Q.numel() * 2
    return ms, nbytes


def run_sliding_decode(steps, warmup, seed=9):
    B, NQ, NKV, HD, W = 8, 16, 8, 256, 1024
    rng = np.random.default_rng(seed)
    lens = rng.integers(1024, 32768, size=B, endpoint=True).astype(np.int32)
    ML = 32768
    g = torch.Generator(device="cuda").manual_seed(seed)
    K = torch.randn(B, ML, NKV, HD, device="cuda", generator=g).bfloat16()
    V = torch.randn(B, ML, NKV, HD, device="cuda", generator=g).bfloat16()
    Q = torch.randn(B * NQ * HD, device="cuda", generator=g).bfloat16()
    O = torch.empty_like(Q)
    pos = torch.from_numpy(lens - 1).cuda()
    chunk = int(os.environ.get("BENCH_SLIDING_CHUNK", "96"))
    A.split_reserve(B * max(1, -(-A.split_chunk() // chunk)), NQ, ML, HD)   # partials for the chunk
    # a 1K window spans few 256-key chunks: 96-key chunks measured fastest (18.6 us; 128: 19.5, 160: 19.7, 256: 24)
    fn = lambda: A.attn_batch(Q, K, V, O, B, 1, NQ, NKV, HD, pos, ML * NKV * HD, int(lens.max()) - 1, chunk=chunk,
                              window=W)
    ms = timed(fn, steps, warmup)
    nbytes = B * W * NKV * HD * 4 + 2 * Q.numel() * 2
    return ms, nbytes


def run_decode_fp32(steps, warmup, w):
    """The fp32-cache decode path (launch_attn_decode_batch semantics: fp32 Q/K/V/O, fp32 FMA) on the config-2
    shape and lengths. Returns (ms, algorithmic bytes)."""
    B, NQ, NKV, HD, ML = w["B"], w["NQ"], w["NKV"], w["HD"], w["ML"]
    K = w["K"].float(); V = w["V"].float()
    Q = w["Q"].float(); O = torch.empty_like(Q)
    A.flash_reserve_partials(B * NQ * (ML // 512 + 1), HD)     # the fp32 MFMA kernel's partials, before timing
    ms = timed(lambda: A.attn_decode_batch(Q, K, V, O, B, NQ, NKV, HD, 0, ML * NKV * HD, base_b=w["pos"]), steps,
               warmup)
    del K, V
    return ms, int(w["lens"].sum()) * NKV * HD * 4 * 2 + 2 * B * NQ * HD * 4


def run_kv_append(steps, warmup, B=16, T=1, NKV=4, HD=256, ML=8192, kvdt=1):
    """Ragged KV append of one decode step (Qwen3.5 shape): one dgx_kv_append launch vs the reference's per-slot
    loop of 2B kv_store launches. Returns (fused ms, loop ms, algorithmic bytes)."""
    row = NKV * HD
    g = torch.Generator(device="cuda").manual_seed(9)
    k = torch.randn(B * T * row, device="cuda", generator=g); v = torch.randn_like(k)
    dt = {1: torch.float16, 2: torch.bfloat16}[kvdt]
    Kc = torch.zeros(B * ML * row, device="cuda", dtype=dt); Vc = torch.zeros_like(Kc)
    pos_h = np.random.default_rng(9).integers(0, ML - T, size=B).astype(np.int32)
    pos = torch.from_numpy(pos_h).cuda()
    fused = timed(lambda: A.kv_append(k, v, Kc, Vc, kvdt, B, T, ML * row, row, pos), steps, warmup)

    def loop():
        for b in range(B):
            off = (b * ML + int(pos_h[b])) * row
            A.kv_store(k[b * T * row:], Kc[off:], T * row, kvdt, 0)
            A.kv_store(v[b * T * row:], Vc[off:], T * row, kvdt, 1)
    looped = timed(loop, steps, warmup)
    return fused, looped, B * T * row * (4 + 2) * 2


def run_norm_rope(steps, warmup, T=1024, NKV=8, HD=256):
    """Gemma4 k append of a T-token prompt chunk: per-head RMSNorm + RoPE + bf16 store into the cache (one
    dgx_norm_rope_store launch, launch_norm_rope_store's k call of models/gemma4_decode.cu:354). Returns (ms,
    algorithmic bytes: the fp32 rows and weights read, one cos and one sin half-row per token, the bf16 rows
    written)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    rows = T * NKV
    g = torch.Generator(device="cuda").manual_seed(11)
    X = torch.randn(rows * HD, device="cuda", generator=g)
    W = torch.randn(HD, device="cuda", generator=g)
    c, s_ = oracle.rope_tables(T, HD)
    C, S = torch.from_numpy(c).cuda(), torch.from_numpy(s_).cuda()
    Kc = torch.zeros(T * NKV * HD, device="cuda", dtype=torch.bfloat16)
    ms = timed(lambda: A.norm_rope_store(X, W, Kc, 2, rows, NKV, HD, 1e-6, C, S, base=0, pos_step=1, slot_stride=0,
                                         row_stride=NKV * HD, rope=True), steps, warmup)
    return ms, rows * HD * (4 + 2) + HD * 4 + T * HD * 4


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it, with its family / model / stepping numbers (some hosts report only
    a generic model name)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                info.setdefault(k, v)
    except OSError:
        return "unknown"
    ids = ", ".join(f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info)
    return f"{info.get('model name', 'unknown')} ({ids})" if ids else info.get("model name", "unknown")


def cpu_baseline(w):
    """Oracle fp32 host attention (restating tests/test_kernels.cu:94-108) over the full decode workload, on the
    GPU's inputs, at 1 thread, 8 threads (the reference harness's cap, tests/test_flash_gemma.cu:342) and every CPU
    this process may run on (its affinity set). `value` is the all-CPU rate and `cores` that thread count."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    B, NQ, NKV, HD, ML = w["B"], w["NQ"], w["NKV"], w["HD"], w["ML"]
    lens = w["lens"]
    Lmax = int(lens.max())
    K = w["K"][:, :Lmax].float().cpu().numpy()
    V = w["V"][:, :Lmax].float().cpu().numpy()
    q = w["Q"].float().cpu().numpy()
    kv_off = np.arange(B, dtype=np.int64) * Lmax * NKV * HD
    nbytes = int(lens.sum()) * NKV * HD * 4 + 2 * B * NQ * HD * 2
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    sweep = sorted({1, min(8, affinity), affinity})
    rates = {}
    for threads in sweep:
        t0 = time.perf_counter()
        oracle.attention(q, K, V, kv_off, lens - 1, NQ, NKV, HD, mode=1, nthreads=threads)
        dt = time.perf_counter() - t0
        rates[threads] = (nbytes / dt / 1e9, dt)
    vall, dtall = rates[affinity]
    out = dict(value=round(vall, 3), unit="GB/s", cores=affinity, kind="port")
    out.update({f"threads_{t}_gbs": round(rates[t][0], 3) for t in sweep})
    out.update(host_cpus=os.cpu_count(), affinity_cpus=affinity, cpu_model=_cpu_model(),
               sample=f"full decode workload (16 rows x 24 heads, sum L = {int(lens.sum())} keys), fp32 host "
                      f"attention (fp64 dot, fp32 softmax); ms per call at "
                      f"{'/'.join(str(t) for t in sweep)} threads: "
                      f"{'/'.join(f'{rates[t][1] * 1e3:.1f}' for t in sweep)}")
    return out


def run_global_decode(steps, warmup, seed=13):
    """Gemma4-12B global layer decode (tools/autotune/profiles/gemma4-12b.json: 16 q-heads, 1 KV head, head_dim
    512): B=8, ragged L~U[1024, 32768], bf16 KV and Q/O, no window, split 512. Returns (ms, bytes, kernel ms)."""
    B, NQ, NKV, HD, ML = 8, 16, 1, 512, 32768
    rng = np.random.default_rng(seed)
    lens = rng.integers(1024, ML, size=B, endpoint=True).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(seed)
    K = torch.randn(B, ML, NKV, HD, device="cuda", generator=g).bfloat16()
    V = torch.randn(B, ML, NKV, HD, device="cuda", generator=g).bfloat16()
    Q = torch.randn(B * NQ * HD, device="cuda", generator=g).bfloat16()
    O = torch.empty_like(Q)
    pos = torch.from_numpy(lens - 1).cuda()
    chunk = int(os.environ.get("BENCH_GLOBAL_CHUNK", "512"))    # 512 measured fastest (128-384: 93-103 us per call)
    A.split_reserve(B * max(1, -(-A.split_chunk() // chunk)), NQ, ML, HD)
    fn = lambda: A.attn_batch(Q, K, V, O, B, 1, NQ, NKV, HD, pos, ML * NKV * HD, int(lens.max()) - 1, chunk=chunk)
    ms, kms = timed(fn, steps, warmup, kernel=True)
    return ms, int(lens.sum()) * NKV * HD * 2 * 2 + 2 * Q.numel() * 2, kms


def traffic_from_profile():
    """HBM bytes per launch of the decode kernel from the committed rocprofv3 PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", "decode_stream_b16.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch="):
            return int(float(line.split("=", 1)[1]))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["decode", "prefill", "tree", "global", "norm", "sliding", "all"], default="all")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (scale reference for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (requested --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs the GPU"
    A.lib()
    out = {}
    if args.calib_copy:
        src = torch.empty(1 << 28, device="cuda", dtype=torch.float32).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    if args.only == "norm":                   # the norm + RoPE + cache store alone (profiling); not the headline line
        nms, nby = run_norm_rope(args.steps, args.warmup)
        print(json.dumps({"metric": "norm+RoPE+store GB/s (1024 tokens x 8 kv heads, hd 256, bf16 cache)",
                          "value": round(nby / (nms * 1e-3) / 1e9, 1), "unit": "GB/s", "us_per_call": round(nms * 1e3, 2),
                          "bytes": nby, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True}))
        return
    if args.only == "sliding":                # the sliding-window decode alone (profiling); not the headline line
        sms, sby = run_sliding_decode(args.steps, args.warmup)
        print(json.dumps({"metric": "sliding-window decode GB/s (B8 ragged <=32K, 1K window, hd 256, bf16)",
                          "value": round(sby / (sms * 1e-3) / 1e9, 1), "unit": "GB/s", "us_per_call": round(sms * 1e3, 2),
                          "bytes": sby, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True}))
        return
    if args.only == "tree":                   # the tree-verify workload alone (profiling); not the headline line
        tms, tby = run_tree(args.steps, args.warmup)
        print(json.dumps({"metric": "tree-verify attention GB/s (B16 x 8 draft tokens, L<=16K)",
                          "value": round(tby / (tms * 1e-3) / 1e9, 1), "unit": "GB/s", "us_per_call": round(tms * 1e3, 2),
                          "steps": args.steps, "warmup": args.warmup, "higher_is_better": True}))
        return
    if args.only == "global":                 # the Gemma4 global-layer shape alone (profiling); not the headline line
        gms, gby, gkms = run_global_decode(args.steps, args.warmup)
        pms2, pfl2 = run_prefill(args.steps, args.warmup, T=1024, NQ=16, NKV=1, HD=512)
        print(json.dumps({"metric": "Gemma4 global-layer attention (hd 512, 1 KV head)",
                          "decode_B8": dict(us=round(gms * 1e3, 2), gbs=round(gby / (gms * 1e-3) / 1e9, 1),
                                            kernel_us=round(gkms * 1e3, 2)),
                          "prefill_T1024": dict(us=round(pms2 * 1e3, 2), tflops=round(pfl2 / (pms2 * 1e-3) / 1e12, 2)),
                          "steps": args.steps, "warmup": args.warmup}))
        return
    w = decode_workload()
    ms, nbytes, kms = run_decode(w, args.steps, args.warmup, chunk=int(os.environ.get("BENCH_DECODE_CHUNK", "512")),
                           copies=int(os.environ.get("BENCH_DECODE_COPIES", "3")))
    gbs = nbytes / (ms * 1e-3) / 1e9
    kgbs = nbytes / (kms * 1e-3) / 1e9
    extra = {}
    if args.only in ("prefill", "all"):
        pms, pflops = run_prefill(args.steps, args.warmup, kv_split=int(os.environ.get("BENCH_PREFILL_SPLIT", "0")))
        ptf = pflops / (pms * 1e-3) / 1e12
        extra["prefill_causal_T1024"] = dict(us=round(pms * 1e3, 2), tflops=round(ptf, 2),
                                             frac_bf16_peak=round(ptf / BF16_PEAK_TFLOPS, 4))
    if args.only == "all":
        cms, cfl = run_prefill(args.steps, args.warmup, T=512, base=4096, kv_split=-1)   # library-chosen split (2 x 2304 keys on 256 CUs)
        extra["prefill_chunked_512_over_4096"] = dict(us=round(cms * 1e3, 2), tflops=round(cfl / (cms * 1e-3) / 1e12, 2))
        sms, sfl = run_prefill(max(args.steps // 4, 10), args.warmup, T=4096, window=1024, kv_split=0)
        extra["prefill_sliding_T4096_w1024"] = dict(us=round(sms * 1e3, 2), tflops=round(sfl / (sms * 1e-3) / 1e12, 2))
        # The same decode workload at a split of 384 keys: its ~776 chunk items fill the 256 CUs three deep, where
        # the 564 items of the 512 split leave 52 CUs a third item (the headline keeps the configured 512 split).
        ams, aby, akms = run_decode(w, args.steps, args.warmup, chunk=384, copies=3)
        extra["decode_split384"] = dict(us=round(ams * 1e3, 2), gbs=round(aby / (ams * 1e-3) / 1e9, 1),
                                        kernel_us=round(akms * 1e3, 2),
                                        kernel_frac_hbm=round(aby / (akms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        dms, dby = run_sliding_decode(args.steps, args.warmup)
        extra["decode_sliding_B8_w1024"] = dict(us=round(dms * 1e3, 2), gbs=round(dby / (dms * 1e-3) / 1e9, 1))
        fms, fby = run_decode_fp32(max(args.steps // 10, 5), 2, w)
        extra["decode_fp32_B16"] = dict(us=round(fms * 1e3, 2), gbs=round(fby / (fms * 1e-3) / 1e9, 1))
        ams, lms, aby = run_kv_append(args.steps, args.warmup)
        extra["kv_append_B16"] = dict(us=round(ams * 1e3, 2), per_slot_loop_us=round(lms * 1e3, 2),
                                      gbs=round(aby / (ams * 1e-3) / 1e9, 1))
        nms, nby = run_norm_rope(args.steps, args.warmup)
        extra["norm_rope_store_T1024"] = dict(us=round(nms * 1e3, 2), gbs=round(nby / (nms * 1e-3) / 1e9, 1))
        tms, tby = run_tree(args.steps, args.warmup)
        extra["tree_verify_B16x8"] = dict(us=round(tms * 1e3, 2), gbs=round(tby / (tms * 1e-3) / 1e9, 1),
                                          runs="per-sequence chunks (batch-invariant)")
        tms, tby = run_tree(args.steps, args.warmup, runs=1)
        extra["tree_verify_B16x8_equal_runs"] = dict(us=round(tms * 1e3, 2), gbs=round(tby / (tms * 1e-3) / 1e9, 1))
        gms, gby, gkms = run_global_decode(args.steps, args.warmup)
        extra["decode_global_hd512_B8"] = dict(us=round(gms * 1e3, 2), gbs=round(gby / (gms * 1e-3) / 1e9, 1),
                                               kernel_us=round(gkms * 1e3, 2),
                                               kernel_frac_hbm=round(gby / (gkms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        pms2, pfl2 = run_prefill(args.steps, args.warmup, T=1024, NQ=16, NKV=1, HD=512)
        extra["prefill_global_hd512_T1024"] = dict(us=round(pms2 * 1e3, 2), tflops=round(pfl2 / (pms2 * 1e-3) / 1e12, 2),
                                                   frac_bf16_peak=round(pfl2 / (pms2 * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4))
        qms, qfl = run_prefill(args.steps, args.warmup, T=1024, NQ=24, NKV=4, HD=256)   # Qwen3.5 full-attention shape
        extra["prefill_qwen35_gqa6_T1024"] = dict(us=round(qms * 1e3, 2), tflops=round(qfl / (qms * 1e-3) / 1e12, 2),
                                                  frac_bf16_peak=round(qfl / (qms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4))
    out = {
        "metric": "decode-attn HBM GB/s (B16 ragged <=8K) + prefill-attn TFLOP/s (T=1024)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "split-KV GQA decode, B=16 ragged L~U[256,8192], Hq=24 Hkv=4 hd=256 (Qwen3.5-27B "
                               "full-attention layer), f16 KV [16,8192,4,256], split 512 + LSE combine kernel, f16 Q/O",
                   "global_batch": 16, "seq_len": int(w["lens"].max()), "parallelism": "none (1 GPU)"},
        # Dominant kernel (the streaming decode kernel, without the LSE combine): algorithmic bytes over its
        # average duration, HIP events around its launches on the launch stream.
        "roofline": {"bound": "hbm", "achieved": round(kgbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kgbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(),
                     "kernel": "decode_stream_kernel", "algorithmic_bytes_per_launch": nbytes,
                     "kernel_us_per_launch": round(kms * 1e3, 2), "call_us_per_launch": round(ms * 1e3, 2)},
        "cpu_baseline": None if args.no_cpu else cpu_baseline(w),
    }
    if extra.get("prefill_causal_T1024"):
        pre = extra["prefill_causal_T1024"]
        out["prefill"] = {"bound": "mfma", "achieved": pre["tflops"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                          "frac": pre["frac_bf16_peak"], "us_per_launch": pre["us"],
                          "workload": "causal flash prefill T=1024, Hq=16 Hkv=8 hd=256, bf16 Q/K/V/O"}
    out["extra"] = extra
    print(json.dumps(out))


if __name__ == "__main__":
    main()
