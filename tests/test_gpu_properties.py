"""Size-independent properties at the full BASELINE sizes, where the oracle
is too slow to run on every output.  Each holds bit for bit because of how
the integer and fp32 stages compose, so any indexing slip (a wrong row,
column, chunk or group) breaks it:

* homogeneity: x -> 2x doubles every output exactly (the Q8_1 quantizer gives
  the same q with a doubled scale; fp32 products and sums of values scaled by
  a power of two are exact; fp16 rounding commutes with doubling away from
  overflow and subnormals);
* permutation equivariance: permuting weight rows permutes the outputs (every
  row is computed by the same arithmetic, whichever block or lane gets it);
* row independence of the prefill GEMM: rows computed in separate launches
  equal rows computed together (same tile and slice plan).
"""
import numpy as np
import pytest
import torch

from helpers import dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qe():
    import qe_amd
    qe_amd.lib()
    qe_amd.gemm_reserve_workspace()  # split-K partials of the default stream's GEMMs
    return qe_amd


def _bits(t):
    return host(t).view(np.uint16)


def _q8(qe, x, K):
    q8, xs, s8 = empty(K, torch.int8), empty(K // 128, torch.float32), empty(K // 8, torch.int32)
    qe.launch_quantize_fp16_to_q8_1(x, q8, xs, s8, K)
    return q8, xs, s8


@pytest.mark.parametrize("N,K", [(151936, 1536), (1536, 8960), (17920, 1536)])
def test_gemv_w4a8_homogeneous_and_row_equivariant(qe, orc, N, K):
    """configs[2] (LM head), the down projection and gate+up at full size."""
    print(f"gemv properties N={N} K={K}", flush=True)
    qw, sc = orc.synth_w4(31 + N, N, K)
    x = torch.from_numpy(orc.synth_f16_normal(32, K)).cuda()
    y1, y2 = empty(N, torch.float16), empty(N, torch.float16)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), *_q8(qe, x, K), None, y1, N, K)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), *_q8(qe, x * 2, K), None, y2, N, K)
    a, b = host(y1).astype(np.float64), host(y2).astype(np.float64)
    ok = np.abs(a) >= 2.0 ** -13  # away from fp16 subnormals
    assert ok.mean() > 0.95
    assert np.array_equal(b[ok], 2 * a[ok])
    perm = np.random.default_rng(N).permutation(N)
    y3 = empty(N, torch.float16)
    qe.launch_gemv_w4a8(dev(np.ascontiguousarray(qw[perm])), dev(np.ascontiguousarray(sc[perm])),
                        *_q8(qe, x, K), None, y3, N, K)
    assert np.array_equal(_bits(y3), _bits(y1)[perm])


def test_gemv_w4a16_homogeneous_config0(qe, orc):
    """W4A16 1536 -> 8960 with the in-launch quantizer."""
    N, K = 8960, 1536
    qw, sc = orc.synth_w4(41, N, K)
    x = torch.from_numpy(orc.synth_f16_normal(42, K)).cuda()
    y1, y2 = empty(N, torch.float16), empty(N, torch.float16)
    qe.launch_gemv_w4a16(dev(qw), dev(sc), x, None, y1, N, K)
    qe.launch_gemv_w4a16(dev(qw), dev(sc), x * 2, None, y2, N, K)
    a, b = host(y1).astype(np.float64), host(y2).astype(np.float64)
    ok = np.abs(a) >= 2.0 ** -13
    assert ok.mean() > 0.95 and np.array_equal(b[ok], 2 * a[ok])


@pytest.mark.parametrize("tiled", [False, True])
def test_gemm_full_size_properties(qe, orc, tiled):
    """configs[3] gate+up shape at M = 1024 (plain GEMM): homogeneity in A,
    column permutation equivariance and row independence."""
    M, N, K = 1024, 17920, 1536
    print(f"gemm properties tiled={tiled}", flush=True)
    qw, sc = orc.synth_w4(51, N, K)
    A = torch.from_numpy(orc.synth_f16_normal(52, M * K).reshape(M, K)).cuda()

    def run(qw_, sc_, A_, m):
        out = empty((m, N), torch.float16)
        if tiled:
            tw, ts = qe.w4_tiled(dev(qw_), dev(sc_), N, K)
            qe.launch_gemm_prefill_w4a16_tiled(tw, ts, A_, None, out, m, N, K)
        else:
            qe.launch_gemm_prefill_w4a16(dev(qw_), dev(sc_), A_, None, out, m, N, K)
        return out

    y1 = run(qw, sc, A, M)
    y2 = run(qw, sc, A * 2, M)
    a, b = host(y1).astype(np.float64), host(y2).astype(np.float64)
    ok = np.abs(a) >= 2.0 ** -13
    assert ok.mean() > 0.95 and np.array_equal(b[ok], 2 * a[ok])
    perm = np.random.default_rng(53).permutation(N)
    y3 = run(np.ascontiguousarray(qw[perm]), np.ascontiguousarray(sc[perm]), A, M)
    assert np.array_equal(_bits(y3), _bits(y1)[:, perm])
    # rows in two launches with the plan of the whole launch (tile and slices forced)
    tile, slices = qe.gemm_prefill_plan(M, N, K, tiled)
    try:
        qe.set_tuning("gemm_tile", tile)
        qe.set_tuning("gemm_slices", slices)
        top = run(qw, sc, A[:384].contiguous(), 384)
        bottom = run(qw, sc, A[384:].contiguous(), M - 384)
    finally:
        qe.set_tuning("gemm_tile", 0)
        qe.set_tuning("gemm_slices", 0)
    assert np.array_equal(np.concatenate([_bits(top), _bits(bottom)]), _bits(y1))
