"""CPU checks of the C-ABI library: it loads, exports every entry point that
include/qe_kernels.h declares, and rejects bad shapes before touching a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header="qe_kernels.h"):
    text = open(os.path.join(ROOT, "include", header)).read()
    return sorted(set(re.findall(r"^(?:int|long|void|const char\*|const uint16_t\*)\s+(qe_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = _declared()
    assert "qe_launch_gemv_w4a8" in names and "qe_last_error" in names
    assert len(names) >= 16


def test_library_exports_every_declared_symbol():
    import qe_amd
    L = qe_amd.lib()
    for name in _declared():
        assert hasattr(L, name), f"libqe_amd.so does not export {name}"
    # and the Python binding covers every launcher
    launchers = [n for n in _declared() if n.startswith("qe_launch_")]
    assert sorted(launchers) == sorted(qe_amd.SIGNATURES)
    assert qe_amd.lib().qe_version().decode().startswith("qe_amd")
    for header in ("qe_engine.h", "qwenbin.h"):
        for name in _declared(header):
            assert hasattr(L, name), f"libqe_amd.so does not export {name}"
    assert "qe_qwenbin_inspect" in _declared("qwenbin.h")
    assert "qe_engine_create_from_qwenbin" in _declared("qe_engine.h")


@pytest.mark.parametrize("K", [0, 100, 129, -128])
def test_bad_k_rejected_on_host(K):
    """Precondition checks run before any HIP call (no GPU needed)."""
    import qe_amd
    L = qe_amd.lib()
    rc = L.qe_launch_gemv_w4a8(8, 8, 16, 16, 16, None, 16, 4, K, None)
    assert rc == 1
    assert "multiple of 128" in L.qe_last_error().decode()
    rc = L.qe_launch_gemm_prefill_w4a16(16, 16, 16, None, 16, 4, 4, K, None, 0)
    assert rc == 1


def test_gemm_workspace_calls_rejected_on_host():
    """The per-thread stream handle never holds a split-K workspace, a NULL or
    unaligned workspace is refused, and no workspace has been allocated: all
    decided before any HIP call."""
    import qe_amd
    L = qe_amd.lib()
    per_thread = 2  # hipStreamPerThread
    assert L.qe_gemm_reserve_workspace(per_thread) == 1
    assert "hipStreamPerThread" in L.qe_last_error().decode()
    assert L.qe_gemm_attach_workspace(None, None, 1 << 25) == 1
    assert L.qe_gemm_attach_workspace(None, 0x1000 + 16, 1 << 25) == 1
    assert L.qe_gemm_attach_workspace(None, 0x1000, 1 << 10) == 1
    assert qe_amd.gemm_workspace_allocations() == 0


def test_null_pointers_rejected_on_host():
    import qe_amd
    L = qe_amd.lib()
    assert L.qe_launch_gemv_w4a8(None, None, None, None, None, None, None, 4, 128, None) == 1
    assert L.qe_launch_quantize_fp16_to_q8_1(None, None, None, None, 128, None) == 1
    assert L.qe_launch_gemv_qkv_w4a8(None, 16, 16, 16, None, 128, 1, 1, 128) == 1
    assert "NULL" in L.qe_last_error().decode()


def test_engine_rejects_bad_config_on_host():
    import ctypes
    import qe_amd
    c = qe_amd.default_config()
    assert c.hidden_size == 1536 and c.num_layers == 28 and c.vocab_size == 151936
    c.head_dim = 64
    h = ctypes.c_void_p()
    assert qe_amd.lib().qe_engine_create(ctypes.byref(c), 1, ctypes.byref(h)) == 1
    assert "unsupported" in qe_amd.lib().qe_last_error().decode()


def test_cpp_mirror_header_compiles():
    """include/kernels.hpp (the reference-named C++ API) compiles every launcher
    call of the reference's decode and prefill loops (src/engine.cu:361-580),
    with the default arguments those calls rely on."""
    import shutil
    import subprocess
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    src = os.path.join(ROOT, "tests", "cpp", "engine_call_shapes.cpp")
    r = subprocess.run([hipcc, "-std=c++20", "-fsyntax-only", "-x", "hip", "--offload-arch=gfx950",
                        f"-I{ROOT}/include", src], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_cpp_mirror_covers_engine_launchers():
    """Every launcher that the reference declares in include/kernels.cuh and its
    engine calls has a namespace-qwen wrapper of the same name."""
    text = open(os.path.join(ROOT, "include", "kernels.hpp")).read()
    names = set(re.findall(r"^inline void (launch_\w+)\(", text, re.M))
    engine_calls = {
        "launch_embed_lookup_w4a16", "launch_rmsnorm_fp16", "launch_rmsnorm_q8_1", "launch_quantize_fp16_to_q8_1",
        "launch_gemv_w4a16", "launch_gemv_w4a8", "launch_gemv_qkv_w4a8", "launch_gemv_dual_gate_up_swiglu_w4a16",
        "launch_gemv_dual_gate_up_swiglu_w4a8", "launch_gemm_prefill_w4a16", "launch_gemm_prefill_qkv_w4a16",
        "launch_gemm_prefill_dual_gate_up_swiglu_w4a16", "launch_qkv_bias_rope_kv_append",
        "launch_attention_gqa_flash_decode", "launch_attention_gqa_prefill", "launch_sample_and_advance",
    }
    assert engine_calls <= names, engine_calls - names


def test_cpp_wrappers_throw(tmp_path):
    """A program linked against libqe_amd.so through kernels.hpp gets a
    std::runtime_error for a rejected launch (host-side check, no GPU)."""
    import shutil
    import subprocess
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    lib = os.path.join(ROOT, "qwen-engine_amd", "libqe_amd.so")
    if not os.path.exists(hipcc) or not os.path.exists(lib):
        pytest.skip("hipcc or the built library not available")
    exe = tmp_path / "throws"
    r = subprocess.run([hipcc, "-std=c++20", "-x", "hip", "--offload-arch=gfx950", f"-I{ROOT}/include",
                        os.path.join(ROOT, "tests", "cpp", "throws_on_bad_shape.cpp"), "-o", str(exe),
                        f"-L{os.path.dirname(lib)}", "-lqe_amd", f"-Wl,-rpath,{os.path.dirname(lib)}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr


def test_gemm_plan_policy():
    """The prefill GEMM planner (host code): K slices only where the tile grid
    leaves CUs idle, never more slices than whole 256-k quads allow with at
    least 4 steps each, the gemm_tile / gemm_slices overrides honoured, and
    no K slices when split-K is switched off."""
    import qe_amd
    shapes = [(M, N, K) for M in (1, 128, 512, 1024, 2048) for N, K in ((2048, 1536), (1536, 1536), (17920, 1536),
                                                                       (1536, 8960), (130, 384))]
    for tiled in (False, True):
        for M, N, K in shapes:
            tile, sl = qe_amd.gemm_prefill_plan(M, N, K, tiled)
            assert 1 <= tile <= 4 and sl >= 1
            KT = K // 64
            if sl > 1:
                assert sl <= (KT // 4 if K % 256 == 0 else KT) and KT // sl >= 4
                bm, bn = ((64, 64), (64, 128), (128, 64), (128, 128))[tile - 1]
                assert ((M + bm - 1) // bm) * ((N + bn - 1) // bn) < 2 * 256  # small grids only
    try:
        qe_amd.set_tuning("gemm_tile", 3)
        qe_amd.set_tuning("gemm_slices", 2)
        assert qe_amd.gemm_prefill_plan(128, 1536, 1536) == (3, 2)
        qe_amd.set_tuning("gemm_slices", 0)
        qe_amd.set_tuning("gemm_split_k", 0)
        assert qe_amd.gemm_prefill_plan(128, 1536, 8960)[1] == 1
    finally:
        qe_amd.set_tuning("gemm_tile", 0)
        qe_amd.set_tuning("gemm_slices", 0)
        qe_amd.set_tuning("gemm_split_k", 1)
