"""ctypes binding of libdgx_attn.so (the C ABI in include/dgx_attn.h) over torch device tensors.

torch supplies device memory and the current HIP stream only; every computation runs in the library's HIP
kernels. Loading fails loudly when the library has not been built (there is no fallback path).
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdgx_attn.so")

FP32, F16, BF16 = 0, 1, 2
_DT = {torch.float32: FP32, torch.float16: F16, torch.bfloat16: BF16}

_lib = None


def lib():
    """Load libdgx_attn.so (raises if it is missing: build it with `make -C dgx-serving_amd`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() or make -C dgx-serving_amd")
        L = ctypes.CDLL(LIB_PATH)
        P, I, F, L64, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_long, ctypes.c_size_t
        sig = {
            "dgx_knobs_status": ([], I),
            "dgx_attn_verify_runs": ([I], I),
            "dgx_kv_dtype": ([], I),
            "dgx_kv_force_fp32": ([ctypes.c_char_p], None),
            "dgx_kv_elem": ([], S),
            "dgx_attn_split_chunk": ([], I),
            "dgx_attn_split_ns_cap": ([I], I),
            "dgx_attn_split_reserve": ([I, I, I, I], I),
            "dgx_attn_decode_split": ([P, P, P, I, P, P, I, I, I, I, I, I, P, I, L64, I, P, F, I], I),
            "dgx_flash_attn": ([P, P, P, I, P, P, I, I, I, I, I, P, P, F, I], I),
            "dgx_flash_attn_reserve": ([I, I, I, I], I),
            "dgx_flash_attn_reserve_partials": ([S, I], I),
            "dgx_flash_attn_v2": ([P, P, P, I, P, P, I, I, I, I, I, P, F, I, I], I),
            "dgx_attn": ([P, P, P, P, I, I, I, I, P, F, I], I),
            "dgx_attn_decode": ([P, P, P, P, I, I, I, I, I, P, F, I], I),
            "dgx_attn_decode_batch": ([P, P, P, P, I, I, I, I, I, L64, P, F, I, P], I),
            "dgx_kv_store": ([P, P, S, I, I, P], I),
            "dgx_f32_to_bf16": ([P, P, S, P], I),
            "dgx_gate_sigmoid": ([P, P, I, P], I),
            "dgx_kv_stats_enabled": ([], I),
            "dgx_flash_attn_hd512_lds": ([], S),
            "dgx_kv_stats": ([P], I),
            "dgx_kv_append": ([P, P, P, P, I, I, I, L64, I, P, I, P], I),
            "dgx_norm_rope_store": ([P, P, P, I, I, I, I, F, P, P, I, I, P, L64, L64, I, P], I),
            "dgx_attn_batch": ([P, I, P, P, I, P, I, P, I, I, I, I, I, P, I, L64, P, I, I, P, F, I], I),
            "dgx_attn_batch_noalloc": ([P, I, P, P, I, P, I, P, I, I, I, I, I, P, I, L64, P, I, I, P, F, I], I),
            "dgx_attn_batch_ex": ([P, I, P, P, P, P, I, P, I, P, P, I, I, I, I, I, I, P, I, L64, P, I, I, P, F, I, I], I),
            "dgx_attn_prefill_ex": ([P, I, P, P, I, P, I, P, I, I, I, I, I, P, I, L64, I, I, P, F, I, I], I),
            "dgx_attn_prefill": ([P, I, P, P, I, P, I, P, I, I, I, I, I, P, I, L64, I, I, P, F, I], I),
            "dgx_attn_version": ([], ctypes.c_char_p),
            "dgx_attn_timing": ([I], I),
            "dgx_attn_timing_read": ([P, P], I),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


class HipError(RuntimeError):
    pass


def _ck(code, what):
    if code != 0:
        raise HipError(f"{what} failed: hipError {code}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def kv_code(t):
    return _DT[t.dtype]


# ------------------------------------------------------------------ drop-in entry points
def knobs_status():
    """0 when the attention knobs (env and DGX_KNOBS_FILE) are valid, -1 otherwise (dgx_knobs_status)."""
    return lib().dgx_knobs_status()


def verify_runs(mode=-1):
    """Set how the batched verify kernel divides the keys (0: each sequence's absolute chunks, batch-invariant, the
    default; 1: equal runs over the batch); -1 queries. Returns the previous mode (dgx_attn_verify_runs)."""
    r = lib().dgx_attn_verify_runs(mode)
    if r < 0 and mode != -1:
        raise ValueError(f"verify_runs: mode {mode} is not 0, 1 or -1")
    return r


def split_chunk():
    return lib().dgx_attn_split_chunk()


def split_ns_cap(max_len):
    return lib().dgx_attn_split_ns_cap(max_len)


def split_reserve(rows, NQ, max_len, hd_max):
    _ck(lib().dgx_attn_split_reserve(rows, NQ, max_len, hd_max), "dgx_attn_split_reserve")


def decode_split(Q, K, V, O, rows, NQ, NKV, HD, base, pos_step, pos_arr, max_pos, kv_stride, ns_cap,
                 scale=0.0, window=0, lse=None):
    _ck(lib().dgx_attn_decode_split(_ptr(Q), _ptr(K), _ptr(V), kv_code(K), _ptr(O), _ptr(lse), rows, NQ, NKV, HD,
                                    base, pos_step, _ptr(pos_arr), max_pos, kv_stride, ns_cap, _stream(),
                                    float(scale), window), "dgx_attn_decode_split")


def flash_attn(Q, K, V, O, Sq, NQ, NKV, HD, base, anc=None, scale=0.0, window=0, lse=None):
    _ck(lib().dgx_flash_attn(_ptr(Q), _ptr(K), _ptr(V), kv_code(K), _ptr(O), _ptr(lse), Sq, NQ, NKV, HD, base,
                             _stream(), _ptr(anc), float(scale), window), "dgx_flash_attn")


def flash_attn_v2(Q, K, V, O, Sq, NQ, NKV, HD, base, scale=0.0, window=0, f16_mma=0, lse=None):
    _ck(lib().dgx_flash_attn_v2(_ptr(Q), _ptr(K), _ptr(V), kv_code(K), _ptr(O), _ptr(lse), Sq, NQ, NKV, HD, base,
                                _stream(), float(scale), window, f16_mma), "dgx_flash_attn_v2")


def flash_reserve(Sq, NQ, base, HD):
    _ck(lib().dgx_flash_attn_reserve(Sq, NQ, base, HD), "dgx_flash_attn_reserve")


def flash_reserve_partials(partials, hd_max):
    """Pre-size the flash scratch (also what lets the fp32 launchers take the fp32 MFMA kernel)."""
    _ck(lib().dgx_flash_attn_reserve_partials(partials, hd_max), "dgx_flash_attn_reserve_partials")


def attn(Q, K, V, O, S, NQ, NKV, HD, scale=0.0, window=0):
    _ck(lib().dgx_attn(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), S, NQ, NKV, HD, _stream(), float(scale), window), "dgx_attn")


def attn_decode(Q, K, V, O, Sq, NQ, NKV, HD, base, scale=0.0, window=0):
    _ck(lib().dgx_attn_decode(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), Sq, NQ, NKV, HD, base, _stream(), float(scale),
                              window), "dgx_attn_decode")


def attn_decode_batch(Q, K, V, O, B, NQ, NKV, HD, base, kv_stride, scale=0.0, window=0, base_b=None):
    _ck(lib().dgx_attn_decode_batch(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), B, NQ, NKV, HD, base, kv_stride, _stream(),
                                    float(scale), window, _ptr(base_b)), "dgx_attn_decode_batch")


def kv_store(src, dst, n, kv_dtype, which):
    _ck(lib().dgx_kv_store(_ptr(src), _ptr(dst), n, kv_dtype, which, _stream()), "dgx_kv_store")


def gate_sigmoid(y, gate, n):
    """launch_gate_sigmoid (kernels/elementwise.cuh:50-60): y *= sigmoid(gate) in place, fp32."""
    _ck(lib().dgx_gate_sigmoid(_ptr(y), _ptr(gate), n, _stream()), "dgx_gate_sigmoid")


def f32_to_bf16(src, dst, n):
    """launch_f32_to_bf16 (kernels/elementwise.cuh:85-95): RN-even fp32 -> bf16 of n elements."""
    _ck(lib().dgx_f32_to_bf16(_ptr(src), _ptr(dst), n, _stream()), "dgx_f32_to_bf16")


def kv_append(k_src, v_src, Kc, Vc, kv_dtype, nseq, T, kv_stride, row_elems, pos_b=None, base=0):
    _ck(lib().dgx_kv_append(_ptr(k_src), _ptr(v_src), _ptr(Kc), _ptr(Vc), kv_dtype, nseq, T, kv_stride, row_elems,
                            _ptr(pos_b), base, _stream()), "dgx_kv_append")


def norm_rope_store(X, W, Y, y_dtype, rows, NH, hd, eps, cosT=None, sinT=None, base=0, pos_step=0, pos_arr=None,
                    slot_stride=0, row_stride=0, rope=True):
    """Per-head RMSNorm (+ RoPE) (+ store) of launch_norm_rope_store (kernels/norm_fused.cuh:127-133)."""
    _ck(lib().dgx_norm_rope_store(_ptr(X), _ptr(W), _ptr(Y), y_dtype, rows, NH, hd, float(eps), _ptr(cosT), _ptr(sinT),
                                  base, pos_step, _ptr(pos_arr), slot_stride, row_stride, 1 if rope else 0, _stream()),
        "dgx_norm_rope_store")


def flash_attn_hd512_lds():
    """configure_flash_attn_hd512() (kernels/attention_flash.cuh:254-270): LDS bytes of the HD 512 flash path."""
    return int(lib().dgx_flash_attn_hd512_lds())


def kv_stats_enabled():
    """g4_kv_stats_enabled() (kernels/kv_store.cuh:87-90): whether G4_KV_STATS=1."""
    return bool(lib().dgx_kv_stats_enabled())


def kv_stats():
    out = (ctypes.c_uint * 4)()
    _ck(lib().dgx_kv_stats(out), "dgx_kv_stats")
    return list(out)


# ------------------------------------------------------------------ native entry points
def attn_batch(Q, K, V, O, B, Tq, NQ, NKV, HD, base_b, kv_stride, max_pos, chunk=0, anc=None, base=0,
               scale=0.0, window=0, lse=None):
    _ck(lib().dgx_attn_batch(_ptr(Q), _DT[Q.dtype], _ptr(K), _ptr(V), kv_code(K), _ptr(O), _DT[O.dtype], _ptr(lse),
                             B, Tq, NQ, NKV, HD, _ptr(base_b), base, kv_stride, _ptr(anc), max_pos, chunk, _stream(),
                             float(scale), window), "dgx_attn_batch")


def attn_batch_noalloc(Q, K, V, O, B, Tq, NQ, NKV, HD, base_b, kv_stride, max_pos, chunk=0, anc=None, base=0,
                       scale=0.0, window=0, lse=None):
    """dgx_attn_batch_noalloc: dgx_attn_batch with its partials in the library's fixed device array."""
    _ck(lib().dgx_attn_batch_noalloc(_ptr(Q), _DT[Q.dtype], _ptr(K), _ptr(V), kv_code(K), _ptr(O), _DT[O.dtype],
                                     _ptr(lse), B, Tq, NQ, NKV, HD, _ptr(base_b), base, kv_stride, _ptr(anc), max_pos,
                                     chunk, _stream(), float(scale), window), "dgx_attn_batch_noalloc")


def attn_batch_ex(Q, O, B, Tq, NQ, NKV, HD, base_b, max_pos, K=None, V=None, kv_stride=0, Kp=None, Vp=None,
                  kv_dtype=None, gate=None, chunk=0, anc=None, base=0, scale=0.0, window=0, lse=None, kv_cap=0):
    """dgx_attn_batch_ex: per-slot K/V base pointers (Kp, Vp: int64 device tensors of addresses) and/or an output
    gate multiplied in as sigmoid(gate)."""
    kvdt = kv_dtype if kv_dtype is not None else kv_code(K)
    _ck(lib().dgx_attn_batch_ex(_ptr(Q), _DT[Q.dtype], _ptr(K), _ptr(V), _ptr(Kp), _ptr(Vp), kvdt, _ptr(O),
                                _DT[O.dtype], _ptr(lse), _ptr(gate), _DT[gate.dtype] if gate is not None else 0,
                                B, Tq, NQ, NKV, HD, _ptr(base_b), base, kv_stride, _ptr(anc), max_pos, chunk,
                                _stream(), float(scale), window, kv_cap), "dgx_attn_batch_ex")


def attn_prefill(Q, K, V, O, nseq, Sq, NQ, NKV, HD, base=0, base_b=None, kv_stride=0, max_pos=None, kv_split=0,
                 scale=0.0, window=0, lse=None, kv_cap=0):
    if max_pos is None:
        max_pos = base + Sq - 1
    if kv_cap:
        _ck(lib().dgx_attn_prefill_ex(_ptr(Q), _DT[Q.dtype], _ptr(K), _ptr(V), kv_code(K), _ptr(O), _DT[O.dtype],
                                      _ptr(lse), nseq, Sq, NQ, NKV, HD, _ptr(base_b), base, kv_stride, max_pos,
                                      kv_split, _stream(), float(scale), window, kv_cap), "dgx_attn_prefill_ex")
        return
    _ck(lib().dgx_attn_prefill(_ptr(Q), _DT[Q.dtype], _ptr(K), _ptr(V), kv_code(K), _ptr(O), _DT[O.dtype], _ptr(lse),
                               nseq, Sq, NQ, NKV, HD, _ptr(base_b), base, kv_stride, max_pos, kv_split, _stream(),
                               float(scale), window), "dgx_attn_prefill")


def timing(on):
    """Bracket the main kernel of every decode/prefill launch with HIP events (dgx_attn_timing)."""
    _ck(lib().dgx_attn_timing(1 if on else 0), "dgx_attn_timing")


def timing_read():
    """(average kernel ms, launches) since the last read (dgx_attn_timing_read)."""
    ms, n = ctypes.c_float(), ctypes.c_int()
    _ck(lib().dgx_attn_timing_read(ctypes.addressof(ms), ctypes.addressof(n)), "dgx_attn_timing_read")
    return ms.value, n.value


def version():
    return lib().dgx_attn_version().decode()
