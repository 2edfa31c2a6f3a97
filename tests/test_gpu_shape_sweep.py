"""Seeded random shapes for the decode GEMVs and the prefill GEMM, against
the CPU oracle (tolerance of helpers.assert_fp16_close).  The fixed-shape
tests cover the Qwen2.5-1.5B projections and chosen edge cases; these cover
tails the hand-picked list may miss: row counts that end a segment, a block
or a grid-stride pass anywhere, K from one group up to the 16384 limit of the
fast GEMV, M tails of every GEMM tile, and (forced) every tile shape and K
slice count of the GEMM planner, in the .qwenbin and the tiled weight layouts.
"""
import numpy as np
import pytest
import torch

from helpers import assert_fp16_close, dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qe():
    import qe_amd
    qe_amd.lib()
    qe_amd.gemm_reserve_workspace()  # split-K partials of the default stream's GEMMs
    return qe_amd


def _gemv_shape(i):
    rng = np.random.default_rng(4000 + i)
    return int(rng.integers(1, 6000)), 128 * int(rng.integers(1, 129))


@pytest.mark.parametrize("i", range(16))
def test_gemv_random_shapes(qe, orc, i):
    N, K = _gemv_shape(i)
    print(f"gemv sweep {i}: N={N} K={K}", flush=True)
    qw, sc = orc.synth_w4(7000 + i, N, K)
    x = orc.synth_f16_normal(7100 + i, K)
    q8, xs, s8 = orc.quantize_q8_1(x)
    out = empty(N, torch.float16)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), None, out, N, K)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert_fp16_close(host(out), ex, bd, ref, what=f"gemv_w4a8 {N}x{K}")
    out16 = empty(N, torch.float16)
    qe.launch_gemv_w4a16(dev(qw), dev(sc), dev(x), None, out16, N, K)
    ref, ex, bd = orc.gemv_w4a16(qw, sc, x, N, K)
    assert_fp16_close(host(out16), ex, bd, ref, what=f"gemv_w4a16 {N}x{K}")


def _gemm_case(i):
    rng = np.random.default_rng(5000 + i)
    M = int(rng.integers(1, 400))
    N = int(rng.integers(1, 3000))
    K = 256 * int(rng.integers(1, 24)) if i % 2 == 0 else 128 * int(rng.integers(1, 48))
    tile = int(rng.integers(0, 5))      # 0: the planner's choice
    slices = int(rng.integers(0, 5))    # 0: the planner's choice
    return M, N, K, tile, slices


@pytest.mark.parametrize("i", range(16))
def test_gemm_random_shapes_and_plans(qe, orc, i):
    M, N, K, tile, slices = _gemm_case(i)
    print(f"gemm sweep {i}: M={M} N={N} K={K} tile={tile} slices={slices}", flush=True)
    qw, sc = orc.synth_w4(8000 + i, N, K)
    A = orc.synth_f16_normal(8100 + i, M * K).reshape(M, K)
    rows = sorted(set(list(range(min(M, 8))) + list(range(max(0, M - 8), M))))  # head and tail rows
    ref, ex, bd = orc.gemm_w4a16(qw, sc, A[rows], len(rows), N, K)
    layouts = ["qwenbin"] + (["tiled"] if K % 256 == 0 else [])
    try:
        qe.set_tuning("gemm_tile", tile)
        qe.set_tuning("gemm_slices", slices)
        for layout in layouts:
            out = empty((M, N), torch.float16)
            if layout == "tiled":
                tw, ts = qe.w4_tiled(dev(qw), dev(sc), N, K)
                qe.launch_gemm_prefill_w4a16_tiled(tw, ts, dev(A), None, out, M, N, K)
            else:
                qe.launch_gemm_prefill_w4a16(dev(qw), dev(sc), dev(A), None, out, M, N, K)
            got = host(out)
            assert_fp16_close(got[rows], ex, bd, ref, what=f"gemm {layout} {M}x{N}x{K} tile {tile} slices {slices}")
            assert np.all(np.isfinite(got.astype(np.float32)))
    finally:
        qe.set_tuning("gemm_tile", 0)
        qe.set_tuning("gemm_slices", 0)
