"""numpy view of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The HIP library never
imports or calls this module.

fp16 arrays are passed as numpy float16 (bit patterns are what cross the
C interface).  Each wrapper names the C function it calls; the reference
citations live on the C definitions in oracle.cpp.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64


def build() -> str:
    """Compile the oracle with its Makefile (g++ only, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sigs = {
            "oracle_f16_to_f32_array": [_P, _P, _I64],
            "oracle_f32_to_f16_array": [_P, _P, _I64],
            "oracle_quantize_q8_1": [_P, _I, _P, _P, _P],
            "oracle_quantize_q8_1_f32": [_P, _I, _P, _P, _P],
            "oracle_quantize_q8_1_attn": [_P, _I, _I, _P, _P, _P, _P],
            "oracle_dequant_w4_f16": [_P, _P, _I, _I, _P],
            "oracle_group_dots": [_P, _P, _P, _I, _I, _P],
            "oracle_gemv_w4a8": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P],
            "oracle_gemv_swiglu_w4a8": [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P],
            "oracle_gemv_w4a16": [_P, _P, _P, _P, _P, _I, _I, _P, _P],
            "oracle_gemv_swiglu_w4a16": [_P, _P, _P, _P, _I, _I, _P, _P],
            "oracle_gemm_w4a16": [_P, _P, _P, _P, _P, _I, _I, _I, _P, _P],
            "oracle_gemm_swiglu_w4a16": [_P, _P, _P, _P, _I, _I, _I, _P, _P],
            "oracle_rmsnorm_fp16": [_P, _P, _P, _I, _I, ctypes.c_float],
            "oracle_argmax_f16": [_P, _I],
            "oracle_philox4x32_10": [_P, _P, _P],
            "oracle_gemv_swiglu_w4a8_mt": [_P, _P, _P, _P, _P, _P, _I, _I, _I],
            "oracle_suite3_inputs": [_I, _I, _P, _P, _P],
            "oracle_synth_w4": [ctypes.c_uint64, _I, _I, _P, _P],
            "oracle_synth_f16_normal": [ctypes.c_uint64, _I64, _P],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        L.oracle_argmax_f16.restype = ctypes.c_int32
        L.oracle_philox_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32]
        L.oracle_philox_uniform.restype = ctypes.c_float
        L.oracle_sample_f16.argtypes = [_P, _I, ctypes.c_float, ctypes.c_uint64, ctypes.c_uint32, _P]
        L.oracle_sample_f16.restype = ctypes.c_int32
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_unpack_w4.argtypes = [ctypes.c_uint32, _P]
        L.oracle_unpack_w4.restype = None
        L.oracle_pack_w4.argtypes = [_P]
        L.oracle_pack_w4.restype = ctypes.c_uint32
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# -- conversions -------------------------------------------------------------
def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.float16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.float16)
    lib().oracle_f32_to_f16_array(_p(f), _p(out), f.size)
    return out


# -- quantizers --------------------------------------------------------------
def quantize_q8_1(x: np.ndarray):
    """fp16[K] -> (q8 int8[K], scale f32[K/128], sum8 int32[K/8])."""
    x = _c(x, np.float16)
    K = x.size
    q8 = np.empty(K, np.int8)
    sc = np.empty(K // 128, np.float32)
    s8 = np.empty(K // 8, np.int32)
    lib().oracle_quantize_q8_1(_p(x), K, _p(q8), _p(sc), _p(s8))
    return q8, sc, s8


def quantize_q8_1_f32(x: np.ndarray):
    x = _c(x, np.float32)
    K = x.size
    q8 = np.empty(K, np.int8)
    sc = np.empty(K // 128, np.float32)
    s8 = np.empty(K // 8, np.int32)
    lib().oracle_quantize_q8_1_f32(_p(x), K, _p(q8), _p(sc), _p(s8))
    return q8, sc, s8


def quantize_q8_1_attn(acc: np.ndarray, head_dim: int = 128):
    acc = _c(acc, np.float32)
    nh = acc.size // head_dim
    out = np.empty(acc.size, np.float16)
    q8 = np.empty(acc.size, np.int8)
    sc = np.empty(nh, np.float32)
    s8 = np.empty(acc.size // 8, np.int32)
    lib().oracle_quantize_q8_1_attn(_p(acc), nh, head_dim, _p(out), _p(q8), _p(sc), _p(s8))
    return out, q8, sc, s8


# -- weights -----------------------------------------------------------------
def unpack_w4(word: int) -> list:
    q = np.zeros(8, np.int32)
    lib().oracle_unpack_w4(int(word) & 0xFFFFFFFF, _p(q))
    return q.tolist()


def pack_w4(q) -> int:
    q = np.ascontiguousarray(q, np.int32)
    return int(lib().oracle_pack_w4(_p(q)))


def dequant_w4_f16(qw: np.ndarray, scales: np.ndarray, N: int, K: int) -> np.ndarray:
    qw = _c(qw, np.uint32)
    scales = _c(scales, np.float16)
    out = np.empty((N, K), np.float16)
    lib().oracle_dequant_w4_f16(_p(qw), _p(scales), N, K, _p(out))
    return out


def group_dots(qw, q8, sum8, N, K):
    qw, q8, sum8 = _c(qw, np.uint32), _c(q8, np.int8), _c(sum8, np.int32)
    out = np.empty((N, K // 128), np.int32)
    lib().oracle_group_dots(_p(qw), _p(q8), _p(sum8), N, K, _p(out))
    return out


# -- GEMV ----------------------------------------------------------------------
def gemv_w4a8(qw, scales, q8, xs, sum8, N, K, residual=None):
    """Returns (y fp16[N], exact f64[N], abs_bound f64[N])."""
    qw, scales = _c(qw, np.uint32), _c(scales, np.float16)
    q8, xs, sum8 = _c(q8, np.int8), _c(xs, np.float32), _c(sum8, np.int32)
    residual = _c(residual, np.float16)
    y = np.empty(N, np.float16)
    ex = np.empty(N, np.float64)
    bd = np.empty(N, np.float64)
    lib().oracle_gemv_w4a8(_p(qw), _p(scales), _p(q8), _p(xs), _p(sum8), _p(residual),
                           _p(y), N, K, _p(ex), _p(bd))
    return y, ex, bd


def gemv_swiglu_w4a8(qw, scales, q8, xs, sum8, K, I):
    qw, scales = _c(qw, np.uint32), _c(scales, np.float16)
    q8, xs, sum8 = _c(q8, np.int8), _c(xs, np.float32), _c(sum8, np.int32)
    y = np.empty(I, np.float16)
    ex = np.empty(I, np.float64)
    bd = np.empty(I, np.float64)
    lib().oracle_gemv_swiglu_w4a8(_p(qw), _p(scales), _p(q8), _p(xs), _p(sum8), _p(y), K, I, _p(ex), _p(bd))
    return y, ex, bd


def gemv_w4a16(qw, scales, x, N, K, residual=None):
    qw, scales, x = _c(qw, np.uint32), _c(scales, np.float16), _c(x, np.float16)
    residual = _c(residual, np.float16)
    y = np.empty(N, np.float16)
    ex = np.empty(N, np.float64)
    bd = np.empty(N, np.float64)
    lib().oracle_gemv_w4a16(_p(qw), _p(scales), _p(x), _p(residual), _p(y), N, K, _p(ex), _p(bd))
    return y, ex, bd


def gemv_swiglu_w4a16(qw, scales, x, K, I):
    qw, scales, x = _c(qw, np.uint32), _c(scales, np.float16), _c(x, np.float16)
    y = np.empty(I, np.float16)
    ex = np.empty(I, np.float64)
    bd = np.empty(I, np.float64)
    lib().oracle_gemv_swiglu_w4a16(_p(qw), _p(scales), _p(x), _p(y), K, I, _p(ex), _p(bd))
    return y, ex, bd


# -- GEMM ----------------------------------------------------------------------
def gemm_w4a16(qw, scales, A, M, N, K, residual=None):
    qw, scales, A = _c(qw, np.uint32), _c(scales, np.float16), _c(A, np.float16)
    residual = _c(residual, np.float16)
    y = np.empty((M, N), np.float16)
    ex = np.empty((M, N), np.float64)
    bd = np.empty((M, N), np.float64)
    lib().oracle_gemm_w4a16(_p(qw), _p(scales), _p(A), _p(residual), _p(y), M, N, K, _p(ex), _p(bd))
    return y, ex, bd


def gemm_swiglu_w4a16(qw, scales, A, M, K, I):
    qw, scales, A = _c(qw, np.uint32), _c(scales, np.float16), _c(A, np.float16)
    y = np.empty((M, I), np.float16)
    ex = np.empty((M, I), np.float64)
    bd = np.empty((M, I), np.float64)
    lib().oracle_gemm_swiglu_w4a16(_p(qw), _p(scales), _p(A), _p(y), M, K, I, _p(ex), _p(bd))
    return y, ex, bd


# -- norm / argmax -------------------------------------------------------------
def rmsnorm_fp16(x, gamma, eps=1e-6):
    x, gamma = _c(x, np.float16), _c(gamma, np.float16)
    H = gamma.size
    T = x.size // H
    out = np.empty(x.shape, np.float16)
    lib().oracle_rmsnorm_fp16(_p(x), _p(gamma), _p(out), T, H, eps)
    return out


def argmax_f16(logits) -> int:
    logits = _c(logits, np.float16)
    return int(lib().oracle_argmax_f16(_p(logits), logits.size))


def gemv_swiglu_w4a8_mt(qw, scales, q8, xs, s8, K, I, threads):
    """fp16 outputs of gemv_swiglu_w4a8, rows split over host threads."""
    qw, scales = _c(qw, np.uint32), _c(scales, np.float16)
    q8, xs, s8 = _c(q8, np.int8), _c(xs, np.float32), _c(s8, np.int32)
    out = np.empty(I, np.float16)
    lib().oracle_gemv_swiglu_w4a8_mt(_p(qw), _p(scales), _p(q8), _p(xs), _p(s8), _p(out), K, I, threads)
    return out


def philox4x32_10(ctr, key):
    ctr = _c(np.asarray(ctr, np.uint32), np.uint32)
    key = _c(np.asarray(key, np.uint32), np.uint32)
    out = np.empty(4, np.uint32)
    lib().oracle_philox4x32_10(_p(ctr), _p(key), _p(out))
    return out


def philox_uniform(seed: int, subsequence: int, offset: int) -> float:
    return float(lib().oracle_philox_uniform(seed, subsequence, offset))


def sample_f16(logits, temperature: float, seed: int, seq_pos: int):
    """(token, compared values) of the reference's sample_and_advance."""
    logits = _c(logits, np.float16)
    vals = np.empty(logits.size, np.float32)
    tok = int(lib().oracle_sample_f16(_p(logits), logits.size, temperature, seed, seq_pos, _p(vals)))
    return tok, vals


# -- synthetic inputs ----------------------------------------------------------
def suite3_inputs(H: int, I: int):
    x = np.empty(H, np.float16)
    qw = np.empty(2 * I * H // 8, np.uint32)
    sc = np.empty(2 * I * H // 128, np.float16)
    lib().oracle_suite3_inputs(H, I, _p(x), _p(qw), _p(sc))
    return x, qw, sc


def synth_w4(seed: int, N: int, K: int):
    qw = np.empty((N, K // 8), np.uint32)
    sc = np.empty((N, K // 128), np.float16)
    lib().oracle_synth_w4(seed, N, K, _p(qw), _p(sc))
    return qw, sc


def synth_f16_normal(seed: int, n: int) -> np.ndarray:
    x = np.empty(n, np.float16)
    lib().oracle_synth_f16_normal(seed, n, _p(x))
    return x
