"""The C++ drop-in API on the GPU: qwen-engine_amd/cpp_api_gpu (built from
tests/cpp/cpp_api_gpu.cpp by the library's Makefile) includes kernels.hpp,
allocates with hipMalloc and calls the qwen:: launchers with the reference's
default arguments (include/kernels.cuh), as src/engine.cu does.  Its outputs
are checked against the CPU oracle."""
import os
import subprocess

import numpy as np
import pytest

from helpers import assert_fp16_close, ulp16

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "qwen-engine_amd", "cpp_api_gpu")


def test_cpp_api_matrix_path(orc, tmp_path):
    if not os.path.exists(EXE):
        pytest.fail("cpp_api_gpu is not built (make -C qwen-engine_amd)")
    K, N, M = 1536, 2048, 64
    x = orc.synth_f16_normal(1, K)
    gamma = (1 + 0.1 * orc.synth_f16_normal(2, K).astype(np.float32)).astype(np.float16)
    qw, sc = orc.synth_w4(3, N, K)
    A = orc.synth_f16_normal(4, M * K).reshape(M, K)
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        for a in (x, gamma, qw, sc, A):
            f.write(np.ascontiguousarray(a).tobytes())
    print("running cpp_api_gpu", flush=True)
    r = subprocess.run([EXE, str(fin), str(fout)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    raw = open(fout, "rb").read()
    off = 0

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(raw, dtype, count, off)
        off += a.nbytes
        return a

    q8, xs, s8 = take(np.int8, K), take(np.float32, K // 128), take(np.int32, K // 8)
    y8, y16, qkv = take(np.float16, N), take(np.float16, N), take(np.float16, 2048)
    gemm = take(np.float16, M * N).reshape(M, N)
    assert off == len(raw)
    # rmsnorm_q8_1: the norm is within one fp16 ulp of the oracle's, so q8 within one unit
    rq, _, _ = orc.quantize_q8_1(orc.rmsnorm_fp16(x, gamma))
    assert np.abs(q8.astype(int) - rq.astype(int)).max() <= 1
    assert np.array_equal(s8, -8 * q8.astype(np.int64).reshape(-1, 8).sum(1))
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert_fp16_close(y8, ex, bd, ref, what="C++ launch_gemv_w4a8")
    # the QKV view over the rows of the same matrix gives the same bits
    assert np.array_equal(qkv.view(np.uint16), y8.view(np.uint16))
    ref, ex, bd = orc.gemv_w4a16(qw, sc, x, N, K)
    assert_fp16_close(y16, ex, bd, ref, what="C++ launch_gemv_w4a16")
    ref, ex, bd = orc.gemm_w4a16(qw, sc, A[:8], 8, N, K)
    assert_fp16_close(gemm[:8], ex, bd, ref, what="C++ launch_gemm_prefill_w4a16")
    assert np.all(np.isfinite(gemm.astype(np.float32)))


def test_cpp_api_wrappers_match_c_abi():
    """Every other qwen:: launcher (embedding, RMSNorm, the quantizer, the
    SwiGLU GEMVs, the QKV and SwiGLU prefill GEMMs, bias + RoPE + KV append,
    prefill and decode attention with the Q8_1 epilogue, sampling) writes the
    same bytes as the qe_ function it wraps on the same inputs, so no wrapper
    passes an argument in the wrong place.  The qe_ functions themselves are
    checked against the oracle by the other GPU tests."""
    if not os.path.exists(EXE):
        pytest.fail("cpp_api_gpu is not built (make -C qwen-engine_amd)")
    print("running cpp_api_gpu --wrappers", flush=True)
    r = subprocess.run([EXE, "--wrappers"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "wrappers ok" in r.stdout, r.stdout + r.stderr
