"""Runs tests/cpp/ref_gates on the GPU: a plain C++ program that calls the library through include/dgx_attn.hpp
under the reference's own launcher names (launch_attn_decode_split, launch_flash_attn<bf16>,
launch_flash_attn_v2<bf16>, launch_attn_decode, attn_split_reserve, kv_at ...), as the reference's
tests/test_attn_decode_split.cu:58-125 main does, and checks every output against the CPU oracle (gate 1 over
lengths to 32768, the full gate-2 sweep of 5 bases x S=2..16 and 12 batch widths, a 40-node tree verify, chunked
prefill, the fp32 decode launcher and launch_norm_rope_store<float / __half / __hip_bfloat16>). The program is built by __graft_entry__.build()."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "ref_gates")


def _run(part, env):
    assert os.path.exists(EXE), "tests/cpp/ref_gates is not built (__graft_entry__.build())"
    e = {k: v for k, v in os.environ.items() if not k.startswith(("G4_", "DGX_KNOBS"))}
    e.update(env)
    r = subprocess.run([EXE, part], capture_output=True, text=True, timeout=600, env=e)
    print(r.stdout[-6000:])
    assert r.returncode == 0, f"ref_gates {part} {env}: rc={r.returncode}\n{r.stdout[-3000:]}\n{r.stderr[-2000:]}"
    assert "[ref_gates] PASS" in r.stdout


@pytest.mark.parametrize("kv", ["f16", "fp32", "bf16"])
def test_split_gates_through_cpp_launchers(kv):
    _run("split", {"G4_KV_DTYPE": kv})


def test_split_gates_reference_chunk():
    _run("split", {"G4_ATTN_CHUNK": "64"})                # the reference's default chunk


def test_tree_prefill_fp32_through_cpp_launchers():
    for part in ("tree", "prefill", "fp32"):
        _run(part, {})


def test_norm_rope_store_through_cpp_launcher():
    _run("norm", {})
