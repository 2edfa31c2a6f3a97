"""The allocation-free prefill GEMM entry point (qe_launch_gemm_prefill_w4a16_noalloc)
gives, through the C-ABI, the same bits as qe_launch_gemm_prefill_w4a16 on two
calls in a row (the second smaller: its scratch still holds the first call's
partials), with split-K plans on both, and rejects a shape beyond its limit."""
import ctypes

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


def _call(L, name, qw, sc, A, res, out, M, N, K):
    s = torch.cuda.current_stream().cuda_stream
    return getattr(L, name)(qw.data_ptr(), sc.data_ptr(), A.data_ptr(), None if res is None else res.data_ptr(),
                            out.data_ptr(), M, N, K, ctypes.c_void_p(s), 0)


def test_noalloc_matches_allocating_entry_point(qe, orc):
    L = qe.lib()
    # (M, N, K): gate-shaped and down-shaped prefill GEMMs whose plans split K,
    # then a smaller one, then one with a residual
    cases = [(128, 17920, 1536, False), (64, 1536, 8960, False), (16, 1536, 1536, True)]
    for M, N, K, with_res in cases:
        print(f"noalloc gemm M={M} N={N} K={K} residual={with_res}", flush=True)
        qw, sc = orc.synth_w4(M + N + K, N, K)
        A = orc.synth_f16_normal(M, M * K).reshape(M, K)
        R = orc.synth_f16_normal(M + 1, M * N).reshape(M, N) if with_res else None
        dq, ds, dA = dev(qw), dev(sc), dev(A)
        outs = []
        for name in ("qe_launch_gemm_prefill_w4a16", "qe_launch_gemm_prefill_w4a16_noalloc"):
            out = empty((M, N), torch.float16)
            res = dev(R) if with_res else None
            assert _call(L, name, dq, ds, dA, res, out, M, N, K) == 0, L.qe_last_error().decode()
            outs.append(host(out))
        assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16)), (M, N, K)
        assert np.all(np.isfinite(outs[1]))


def test_noalloc_rejects_beyond_limit(qe):
    L = qe.lib()
    t = empty(64, torch.int32)
    rc = L.qe_launch_gemm_prefill_w4a16_noalloc(t.data_ptr(), t.data_ptr(), t.data_ptr(), None, t.data_ptr(),
                                                4096, 4096, 128, None, 0)
    assert rc == 1
    assert "exceeds the scratch" in L.qe_last_error().decode()
