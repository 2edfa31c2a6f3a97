"""The reference-named device primitives of include/quant_primitives.hpp on the
GPU: qwen-engine_amd/quant_primitives_gpu (built from
tests/cpp/quant_primitives_gpu.cpp by the library's Makefile) is device code
that calls quantize_group128_fp16_to_q8_1, compute_q8_sum8, dp4a_w4_q8_oct and
unpack_w4_to_half2_quad by the reference's names and parameter lists
(include/quant_primitives.cuh:13-115).  Every output is an integer or an exact
fp16 and is compared bit for bit with the CPU oracle."""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "qwen-engine_amd", "quant_primitives_gpu")


def _edge_vector():
    """Groups with a zero group, exact ties, subnormals, the fp16 extremes and
    constant groups (the quantizer edge cases), then random scales."""
    x = np.zeros(6 * 128, np.float16)
    g1 = x[128:256]
    g1[0] = 127.0
    g1[1:9] = [2.5, -2.5, 0.5, -0.5, 4.5, 126.5, -126.5, 1.5]
    x[256:384] = np.float16(6e-8)
    x[259] = -np.float16(6e-8)
    x[384:512] = np.linspace(-65504, 65504, 128).astype(np.float16)
    x[512:640] = np.float16(1e-3) * np.arange(128).astype(np.float16)
    x[640:768] = np.float16(-7.0)
    rng = np.random.default_rng(7)
    G = 250
    mag = (2.0 ** rng.uniform(-20, 15, G)).astype(np.float32)
    r = np.clip(rng.standard_normal((G, 128)).astype(np.float32) * mag[:, None], -65504, 65504)
    r = r.astype(np.float16).reshape(-1)
    return np.concatenate([x, r])


def test_reference_named_primitives_bit_exact(orc, tmp_path):
    if not os.path.exists(EXE):
        pytest.fail("quant_primitives_gpu is not built (make -C qwen-engine_amd)")
    x = _edge_vector()
    K = x.size
    N = 96
    qw, sc = orc.synth_w4(11, N, K)
    # a few rows of extreme nibbles: all 0, all 15, all 8 (dot = 0 exactly)
    qw[0, :] = 0
    qw[1, :] = 0xFFFFFFFF
    qw[2, :] = 0x88888888
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        f.write(np.array([K, N], np.int32).tobytes())
        for a in (x, qw, sc):
            f.write(np.ascontiguousarray(a).tobytes())
    print(f"running quant_primitives_gpu K={K} N={N}", flush=True)
    r = subprocess.run([EXE, str(fin), str(fout)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "quant_primitives ok" in r.stdout, r.stdout + r.stderr
    raw = open(fout, "rb").read()
    off = 0

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(raw, dtype, count, off)
        off += a.nbytes
        return a

    q8, xs, s8, s8b = take(np.int8, K), take(np.float32, K // 128), take(np.int32, K // 8), take(np.int32, K // 8)
    dots = take(np.int32, N * (K // 128)).reshape(N, K // 128)
    deq = take(np.uint16, N * K).reshape(N, K)
    assert off == len(raw)

    rq, rs, rs8 = orc.quantize_q8_1(x)
    assert np.array_equal(q8, rq), "quantize_group128_fp16_to_q8_1: q8"
    assert np.array_equal(xs.view(np.uint32), rs.view(np.uint32)), "quantize_group128_fp16_to_q8_1: scale"
    assert np.array_equal(s8, rs8), "quantize_group128_fp16_to_q8_1: sum8"
    assert q8[129:137].tolist() == [3, -3, 1, -1, 5, 127, -127, 2]  # half away from zero
    assert np.array_equal(s8b, rs8), "compute_q8_sum8"
    assert np.array_equal(dots, orc.group_dots(qw, rq, rs8, N, K)), "dp4a_w4_q8_oct"
    assert np.all(dots[2] == 0)
    assert np.array_equal(deq, orc.dequant_w4_f16(qw, sc, N, K).view(np.uint16)), "unpack_w4_to_half2_quad"
