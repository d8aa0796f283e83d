"""CPU checks of the drop-in boundary: libdgx_attn.so loads and exports every entry point that include/dgx_attn.h
declares, the host-side knob logic follows the reference registry (runtime/knobs.h, kernels/kv_store.cuh:25-46,
kernels/attention_decode_split.cuh:26-37), argument validation rejects bad calls before any device work, and a
caller written against the reference's C++ launcher names (include/dgx_attn.hpp) compiles and links.
No test here launches a kernel."""
import ctypes
import os
import re
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "dgx-serving_amd", "libdgx_attn.so")
HDR = os.path.join(ROOT, "include", "dgx_attn.h")
HIP_INVALID_VALUE = 1


def _declared():
    txt = open(HDR).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(dgx_\w+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build the library first (__graft_entry__.build())"
    lib = ctypes.CDLL(LIB)
    names = _declared()
    assert len(names) >= 18
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_the_header():
    sys.path.insert(0, os.path.join(ROOT, "dgx-serving_amd"))
    import dgx_attn
    src = open(dgx_attn.__file__).read()
    missing = [n for n in _declared() if f'"{n}"' not in src]
    assert not missing, f"dgx_attn.py does not bind {missing}"


def _knobs(env):
    code = textwrap.dedent(f"""
        import ctypes
        L = ctypes.CDLL({LIB!r})
        print(L.dgx_kv_dtype(), L.dgx_attn_split_chunk(), L.dgx_attn_split_ns_cap(1000), L.dgx_kv_elem(),
              L.dgx_kv_stats_enabled(), L.dgx_knobs_status())
    """)
    e = {k: v for k, v in os.environ.items() if not k.startswith(("G4_", "DGX_KNOBS"))}
    e.update(env)
    out = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    return [int(x) for x in out.stdout.split()], out.stderr


def test_kv_dtype_and_chunk_knobs(tmp_path):
    assert _knobs({})[0] == [1, 256, 4, 2, 0, 0]                   # unset -> f16; MI355X chunk default 256
    assert _knobs({"G4_KV_STATS": "1"})[0][4] == 1                  # g4_kv_stats_enabled (kv_store.cuh:87-90)
    assert _knobs({"G4_ATTN_SPLIT": "0"})[0][0] == 0                # split off -> fp32 KV (kv_store.cuh:29-31)
    assert _knobs({"G4_KV_DTYPE": "bf16"})[0][0] == 2
    assert _knobs({"G4_KV_DTYPE": "fp32"})[0][:4] == [0, 256, 4, 4]
    v, err = _knobs({"G4_KV_DTYPE": "fp8"})
    assert v[0] == -1 and v[5] == -1 and "invalid G4_KV_DTYPE=fp8 (env)" in err
    assert _knobs({"G4_ATTN_CHUNK": "64"})[0][1:3] == [64, 16]
    for bad in ("100", "512"):                                      # the reference's set is 32/64/128/256
        v, err = _knobs({"G4_ATTN_CHUNK": bad})
        assert v[1] == -1 and "invalid G4_ATTN_CHUNK" in err
    recipe = tmp_path / "recipe.env"
    recipe.write_text("# recipe\nG4_KV_DTYPE = bf16  # comment\nG4_ATTN_CHUNK=128\n")
    assert _knobs({"DGX_KNOBS_FILE": str(recipe)})[0][:2] == [2, 128]
    # env beats the recipe (runtime/knobs.h precedence)
    assert _knobs({"DGX_KNOBS_FILE": str(recipe), "G4_KV_DTYPE": "f16"})[0][:2] == [1, 128]


@pytest.mark.parametrize("text,msg", [
    ("G4_KV_DTYPE=bf16\nnot a knob line\n", "recipe.env:2: expected NAME=VALUE"),
    ("=bf16\n", "recipe.env:1: expected NAME=VALUE"),
    ("G4_ATTN_CHUNKS=64\n", "unknown knob G4_ATTN_CHUNKS"),
    ("G4_FLASH_F16_MMA=2\n", "invalid G4_FLASH_F16_MMA=2 (recipe)"),
    ("G4_FLASH_MIN_S=0\n", "invalid G4_FLASH_MIN_S=0 (recipe)"),
    ("G4_ATTN_SPLIT=yes\n", "invalid G4_ATTN_SPLIT=yes (recipe)"),
])
def test_recipe_errors_fail_like_the_registry(tmp_path, text, msg):
    """runtime/knobs.h:241-275: malformed lines, unregistered names under the subsystem's prefixes and values out
    of their set make every knob query fail (the reference exits 2)."""
    recipe = tmp_path / "recipe.env"
    recipe.write_text(text)
    v, err = _knobs({"DGX_KNOBS_FILE": str(recipe)})
    assert v[0] == -1 and v[1] == -1 and v[5] == -1, v
    assert f"knobs: " in err and msg in err, err


def test_recipe_skips_other_subsystems_and_reads_every_attention_knob(tmp_path):
    recipe = tmp_path / "recipe.env"
    recipe.write_text("MMQ_TILE=4  # another subsystem's knob\nG4_MMQ_PREFILL=1\nG4_FLASH_MIN_S=17\n"
                      "G4_FLASH_V2=0\nG4_KV_STATS=1\n\n   # blank and comment lines\n")
    v, err = _knobs({"DGX_KNOBS_FILE": str(recipe)})
    assert v == [1, 256, 4, 2, 1, 0], (v, err)
    v, err = _knobs({"DGX_KNOBS_FILE": str(tmp_path / "missing.env")})
    assert v[5] == -1 and "cannot read DGX_KNOBS_FILE" in err


def test_unknown_env_knob_under_our_prefix_warns():
    """An environment name under the attention prefixes that is not registered only warns (runtime/knobs.h:273-283),
    with the closest registered name when it is within 3 edits; the configuration stays valid."""
    v, err = _knobs({"G4_ATTN_CHUNKS": "64"})
    assert v[5] == 0 and "unknown knob env G4_ATTN_CHUNKS (did you mean G4_ATTN_CHUNK?)" in err, err
    v, err = _knobs({"G4_KV_SOMETHING_ELSE": "1"})
    assert v[5] == 0 and "unknown knob env G4_KV_SOMETHING_ELSE" in err and "did you mean" not in err, err
    v, err = _knobs({"G4_MMQ_TILE": "4"})                     # another subsystem's prefix: silent
    assert v[5] == 0 and "warning" not in err, err


def test_force_fp32_overrides():
    code = textwrap.dedent(f"""
        import ctypes
        L = ctypes.CDLL({LIB!r})
        a = L.dgx_kv_dtype(); L.dgx_kv_force_fp32(b"moe"); print(a, L.dgx_kv_dtype(), L.dgx_kv_elem())
    """)
    e = dict(os.environ, G4_KV_DTYPE="bf16")
    out = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True, text=True, timeout=60)
    assert out.stdout.split() == ["2", "0", "4"] and "G4_KV_DTYPE ignored (moe)" in out.stderr


def test_argument_validation_without_device():
    L = ctypes.CDLL(LIB)
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    L.dgx_attn_decode_split.argtypes = [P, P, P, I, P, P, I, I, I, I, I, I, P, I, ctypes.c_long, I, P, F, I]
    L.dgx_flash_attn.argtypes = [P, P, P, I, P, P, I, I, I, I, I, P, P, F, I]
    L.dgx_attn_batch.argtypes = [P, I, P, P, I, P, I, P, I, I, I, I, I, P, I, ctypes.c_long, P, I, I, P, F, I]
    x = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    # rows == 0 is a no-op, as in the reference
    assert L.dgx_attn_decode_split(None, None, None, 1, None, None, 0, 24, 4, 256, 0, 1, None, 0, 0, 1, None, 0, 0) == 0
    # null pointers, NQ % NKV, unsupported HD, bad dtype
    assert L.dgx_attn_decode_split(None, x, x, 1, x, None, 1, 24, 4, 256, 0, 1, None, 0, 0, 1, None, 0, 0) == HIP_INVALID_VALUE
    assert L.dgx_attn_decode_split(x, x, x, 1, x, None, 1, 24, 5, 256, 0, 1, None, 0, 0, 1, None, 0, 0) == HIP_INVALID_VALUE
    assert L.dgx_attn_decode_split(x, x, x, 1, x, None, 1, 24, 4, 192, 0, 1, None, 0, 0, 1, None, 0, 0) == HIP_INVALID_VALUE
    assert L.dgx_attn_decode_split(x, x, x, 7, x, None, 1, 24, 4, 256, 0, 1, None, 0, 0, 1, None, 0, 0) == HIP_INVALID_VALUE
    assert L.dgx_flash_attn(x, x, x, 1, x, None, 4, 16, 8, 64, 0, None, None, 0, 0) == HIP_INVALID_VALUE
    assert L.dgx_flash_attn(x, x, x, 1, x, None, 4, 16, 8, 256, -1, None, None, 0, 0) == HIP_INVALID_VALUE
    # native batch: chunk must be a multiple of 32, fp32 caches are not served by the MFMA path
    assert L.dgx_attn_batch(x, 1, x, x, 1, x, 1, None, 2, 1, 24, 4, 256, x, 0, 100, None, 10, 48, None, 0, 0) == HIP_INVALID_VALUE
    assert L.dgx_attn_batch(x, 1, x, x, 0, x, 1, None, 2, 1, 24, 4, 256, x, 0, 100, None, 10, 64, None, 0, 0) == HIP_INVALID_VALUE
    # several sequences cannot share one cache without per-sequence positions
    assert L.dgx_attn_batch(x, 1, x, x, 1, x, 1, None, 2, 1, 24, 4, 256, None, 0, 0, None, 10, 64, None, 0, 0) == HIP_INVALID_VALUE


CALLER = r"""
// A reference-style caller: kernels/*.cuh includes replaced by dgx_attn.hpp, CUDA type names by HIP ones.
#include "dgx_attn.hpp"
#include <cstdio>
int main() {
    const float *q = nullptr; float *o = nullptr; const float *kc = nullptr;
    const __hip_bfloat16 *kb = nullptr; const __half *kh = nullptr;
    if (false) {   // compile-only: every launcher of the reference surface, with its defaults
        launch_attn(q, q, q, o, 5, 4, 2, 128);
        launch_attn_decode(q, kc, kc, o, 1, 16, 8, 256, 100);
        launch_attn_decode_batch(q, kc, kc, o, 4, 16, 8, 256, 0, 1000, 0, 1.f, 1024, nullptr);
        launch_attn_decode_split(q, kc, kc, o, 16, 24, 4, 256, 0, 0, nullptr, 8191, 1L << 20, attn_split_ns_cap(8192));
        launch_flash_attn(q, kb, kb, o, 8, 24, 4, 256, 2048, 0, nullptr);
        launch_flash_attn2bs<256, 16, 8>(q, kb, kb, o, 1, 24, 4, 300);
        launch_flash_attn_v2(q, kh, kh, o, 1024, 16, 8, 256, 0, 0, 0.f, 1024, true);
        reserve_flash_attn_scratch(1000, 256);
        kv_store(q, o, 16, 0);
        // kernels/norm_fused.cuh:127-133 as models/gemma4_decode.cu:353-354 call it (k with RoPE, v without scale)
        launch_norm_rope_store<__hip_bfloat16>(q, q, const_cast<__hip_bfloat16 *>(kb), 8, 8, 256, 1e-6f, q, q, 100, 1,
                                               nullptr, 0, 8L * 256, true);
        launch_norm_rope_store<float>(q, nullptr, o, 8, 8, 256, 1e-6f, q, q, 100, 1, nullptr, 0, 8L * 256, false);
        launch_f32_to_bf16(q, const_cast<__hip_bfloat16 *>(kb), 4096);
        launch_gate_sigmoid(o, q, 4096);
        if (g4_kv_stats_enabled()) printf("stats on\n");
        printf("%zu\n", configure_flash_attn_hd512<16, 8, __hip_bfloat16>());
        attn_smem_guard((const void *)attn_decode_kernel, (size_t)(256 + 4096) * sizeof(float), "attn_decode", 4096);
    }
    float *cache = reinterpret_cast<float *>(0x1000);
    printf("%d %d %d %zu %td\n", g4_kv_dtype(), attn_split_chunk(), attn_split_ns_cap(8192), g4_kv_elem(),
           reinterpret_cast<char *>(kv_at(cache, 10)) - reinterpret_cast<char *>(cache));
    return 0;
}
"""


def test_reference_style_caller_compiles_and_links(tmp_path):
    src = tmp_path / "caller.cpp"
    src.write_text(CALLER)
    exe = tmp_path / "caller"
    cmd = ["/opt/rocm/bin/amdclang++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include",
           str(src), "-o", str(exe), "-L", os.path.dirname(LIB), "-ldgx_attn", "-L", "/opt/rocm/lib", "-lamdhip64",
           f"-Wl,-rpath,{os.path.dirname(LIB)}:/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    e = {k: v for k, v in os.environ.items() if not k.startswith("G4_")}
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60, env=e)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["1", "256", "32", "2", "20"]
    # an invalid knob ends a reference-style caller with status 2 (runtime/knobs.h:240)
    bad = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60, env=dict(e, G4_ATTN_CHUNK="100"))
    assert bad.returncode == 2 and "invalid G4_ATTN_CHUNK=100" in bad.stderr, (bad.returncode, bad.stderr)
