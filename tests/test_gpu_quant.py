"""GPU parity of the Q8_1 quantizers and RMSNorm (bit-exact integer stage).

Reference: launch_quantize_fp16_to_q8_1 / launch_rmsnorm_q8_1 /
launch_rmsnorm_fp16 (src/kernels/rmsnorm_rope.cu:75-314); rounding of the
CPU golden tests/test_kernels.cu:311-326.
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
    return qe_amd


def _run_quant(qe, x16):
    K = x16.size
    x = dev(x16)
    q8 = empty(K, torch.int8)
    sc = empty(K // 128, torch.float32)
    s8 = empty(K // 8, torch.int32)
    qe.launch_quantize_fp16_to_q8_1(x, q8, sc, s8, K)
    return host(q8), host(sc), host(s8)


@pytest.mark.parametrize("K", [128, 256, 1536, 8960, 16384])
def test_quantize_bit_exact(qe, orc, K):
    print(f"quantize K={K}", flush=True)
    rng = np.random.default_rng(K)
    x = rng.standard_normal(K).astype(np.float16)
    q8, sc, s8 = _run_quant(qe, x)
    rq, rs, rs8 = orc.quantize_q8_1(x)
    assert np.array_equal(q8, rq)
    assert np.array_equal(sc.view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(s8, rs8)


def test_quantize_edge_groups(qe, orc):
    # zero group, ties (x*inv_d = k + 0.5 exactly), subnormals, clamp, huge values
    x = np.zeros(6 * 128, np.float16)
    g1 = x[128:256]
    g1[0] = 127.0
    g1[1:9] = [2.5, -2.5, 0.5, -0.5, 4.5, 126.5, -126.5, 1.5]
    g2 = x[256:384]
    g2[:] = np.float16(6e-8)
    g2[3] = -np.float16(6e-8)
    x[384:512] = np.linspace(-65504, 65504, 128).astype(np.float16)
    x[512:640] = np.float16(1e-3) * np.arange(128).astype(np.float16)
    x[640:768] = np.float16(-7.0)
    q8, sc, s8 = _run_quant(qe, x)
    rq, rs, rs8 = orc.quantize_q8_1(x)
    assert np.array_equal(q8, rq) and np.array_equal(s8, rs8)
    assert np.array_equal(sc.view(np.uint32), rs.view(np.uint32))
    assert q8[129:137].tolist() == [3, -3, 1, -1, 5, 127, -127, 2]


def test_quantize_many_random_scales(qe, orc):
    # 4096 groups with scales spanning the fp16 range: hunts rounding differences
    rng = np.random.default_rng(99)
    G = 4096
    mag = (2.0 ** rng.uniform(-20, 15, G)).astype(np.float32)
    x = (rng.standard_normal((G, 128)).astype(np.float32) * mag[:, None]).astype(np.float16).reshape(-1)
    x = np.nan_to_num(x, posinf=65504, neginf=-65504).astype(np.float16)
    q8, sc, s8 = _run_quant(qe, x)
    rq, rs, rs8 = orc.quantize_q8_1(x)
    assert np.array_equal(q8, rq)
    assert np.array_equal(sc.view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(s8, rs8)


def test_quantize_rejects_bad_size(qe):
    x = empty(200, torch.float16)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        qe.launch_quantize_fp16_to_q8_1(x, empty(200, torch.int8), empty(2, torch.float32),
                                        empty(25, torch.int32), 200)


@pytest.mark.parametrize("H", [1536, 256, 8960])
def test_rmsnorm_q8_1(qe, orc, H):
    print(f"rmsnorm_q8_1 H={H}", flush=True)
    rng = np.random.default_rng(H + 1)
    x16 = (rng.standard_normal(H) * 3).astype(np.float16)
    g16 = (1 + 0.2 * rng.standard_normal(H)).astype(np.float16)
    x, g = dev(x16), dev(g16)
    out = empty(H, torch.float16)
    q8 = empty(H, torch.int8)
    sc = empty(H // 128, torch.float32)
    s8 = empty(H // 8, torch.int32)
    qe.launch_rmsnorm_q8_1(x, g, out, q8, sc, s8, hidden_size=H)
    n_gpu = host(out)
    n_ref = orc.rmsnorm_fp16(x16, g16)
    # fp part: the sum of squares is reduced in another order, so the fp16
    # output may differ by one ulp; the Q8_1 stage must be bit-exact on the
    # fp16 vector the kernel produced.
    d = np.abs(n_gpu.astype(np.float64) - n_ref.astype(np.float64))
    assert np.all(d <= ulp_or_zero(n_ref))
    rq, rs, rs8 = orc.quantize_q8_1(n_gpu)
    assert np.array_equal(host(q8), rq)
    assert np.array_equal(host(sc).view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(host(s8), rs8)
    # output pointer is optional
    q8b = empty(H, torch.int8)
    qe.launch_rmsnorm_q8_1(x, g, None, q8b, sc, s8, hidden_size=H)
    assert np.array_equal(host(q8b), host(q8))


def ulp_or_zero(ref16):
    from helpers import ulp16
    return ulp16(ref16.astype(np.float64))


def test_rmsnorm_fp16_rows(qe, orc):
    rng = np.random.default_rng(5)
    T, H = 37, 1536
    x16 = rng.standard_normal((T, H)).astype(np.float16)
    g16 = (1 + 0.2 * rng.standard_normal(H)).astype(np.float16)
    out = empty((T, H), torch.float16)
    qe.launch_rmsnorm_fp16(dev(x16), dev(g16), out, T, hidden_size=H)
    got = host(out)
    ref = orc.rmsnorm_fp16(x16, g16)
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(d <= ulp_or_zero(ref))
    assert np.mean(got == ref) > 0.99


@pytest.mark.parametrize("H", [128, 1536, 8960, 65536])
def test_rmsnorm_kernels_agree_bit_for_bit(qe, orc, H):
    """rmsnorm_fp16 (prefill), rmsnorm_q8_1 (decode) and the fused RMSNorm GEMV
    prologue sum the squares in one shared order: the same row gives the same
    normalized fp16 vector in all of them."""
    rng = np.random.default_rng(H)
    x16 = (rng.standard_normal((3, H)) * np.array([[0.01], [1.0], [40.0]])).astype(np.float16)
    g16 = (1 + 0.2 * rng.standard_normal(H)).astype(np.float16)
    rows = empty((3, H), torch.float16)
    qe.launch_rmsnorm_fp16(dev(x16), dev(g16), rows, 3, hidden_size=H)
    a = host(rows)
    for t in range(3):
        out = empty(H, torch.float16)
        q8, sc, s8 = empty(H, torch.int8), empty(H // 128, torch.float32), empty(H // 8, torch.int32)
        qe.launch_rmsnorm_q8_1(dev(x16[t]), dev(g16), out, q8, sc, s8, hidden_size=H)
        assert np.array_equal(host(out).view(np.uint16), a[t].view(np.uint16)), t
        if H <= 16384:
            norm = empty(H, torch.float16)
            qw, wsc = orc.synth_w4(H, 256, H)
            mlp = empty(128, torch.float16)
            qe.launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(dev(x16[t]), dev(g16), norm, dev(qw), dev(wsc), mlp, H,
                                                             128)
            assert np.array_equal(host(norm).view(np.uint16), a[t].view(np.uint16)), t
    ref = orc.rmsnorm_fp16(x16, g16)
    assert np.all(np.abs(a.astype(np.float64) - ref.astype(np.float64)) <= ulp_or_zero(ref))
