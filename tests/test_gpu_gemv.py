"""GPU parity of the decode GEMV family against the CPU oracle.

Reference: src/kernels/gemv_w4a16.cu (launchers :864-999), CPU golden
tests/test_kernels.cu:308-363.  Integer stage: the oracle's per-group dots
are exact; the fp16 outputs are compared with the tolerance of
helpers.assert_fp16_close (2 fp16 ulp / 1e-3 relative).
Shapes: BASELINE configs[0] (W4A16 1536->8960), configs[1] (QKV, O, gate+up
SwiGLU, down), configs[2] (LM head + argmax) and the reference's Suite 3
dimension sweep (test_kernels.cu:251-256).
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
    return qe_amd


def _act(orc, K, seed):
    x = orc.synth_f16_normal(seed, K)
    q8, xs, s8 = orc.quantize_q8_1(x)
    return x, q8, xs, s8


def _gemv_w4a8(qe, qw, sc, q8, xs, s8, N, K, residual=None, inplace=False):
    out = dev(residual) if inplace else empty(N, torch.float16)
    res = out if inplace else (dev(residual) if residual is not None else None)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), res, out, N, K)
    return host(out)


@pytest.mark.parametrize("N,K", [(1536, 1536), (1536, 8960), (8960, 1536), (64, 256), (1, 128), (37, 384),
                                 (1000, 2560), (300, 16384), (130, 16512), (77, 32768)])
def test_gemv_w4a8_shapes(qe, orc, N, K):
    print(f"gemv_w4a8 N={N} K={K}", flush=True)
    qw, sc = orc.synth_w4(N * 7 + K, N, K)
    _, q8, xs, s8 = _act(orc, K, K)
    got = _gemv_w4a8(qe, qw, sc, q8, xs, s8, N, K)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert_fp16_close(got, ex, bd, ref, what=f"gemv {N}x{K}")


@pytest.mark.parametrize("N,K", [(1536, 1536), (1536, 8960)])
def test_gemv_w4a8_residual_inplace(qe, orc, N, K):
    """O-proj / down-proj of the decode layer: residual == output
    (src/engine.cu:396-400, :426-430)."""
    qw, sc = orc.synth_w4(5 + K, N, K)
    _, q8, xs, s8 = _act(orc, K, 3)
    res = orc.synth_f16_normal(11, N)
    got = _gemv_w4a8(qe, qw, sc, q8, xs, s8, N, K, residual=res, inplace=True)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K, residual=res)
    assert_fp16_close(got, ex, bd, ref, what="residual in place")
    got2 = _gemv_w4a8(qe, qw, sc, q8, xs, s8, N, K, residual=res, inplace=False)
    assert np.array_equal(got2, got)


def test_gemv_uses_given_sum8(qe, orc):
    """sum8 is the dp4a seed (quant_primitives.cuh:28-32): a perturbed sum8
    changes the result exactly as in the oracle."""
    N, K = 256, 1536
    qw, sc = orc.synth_w4(1, N, K)
    _, q8, xs, s8 = _act(orc, K, 2)
    s8 = s8.copy()
    s8[::7] += 40
    got = _gemv_w4a8(qe, qw, sc, q8, xs, s8, N, K)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert_fp16_close(got, ex, bd, ref, what="perturbed sum8")


def test_gemv_unaligned_weights_take_generic_path(qe, orc):
    N, K = 200, 1536
    qw, sc = orc.synth_w4(21, N, K)
    _, q8, xs, s8 = _act(orc, K, 4)
    buf = dev(np.concatenate([np.zeros(1, np.uint32), qw.reshape(-1)]))
    w_ptr = buf.data_ptr() + 4  # 4-byte aligned, not 16-byte aligned
    out = empty(N, torch.float16)
    qe.launch_gemv_w4a8(w_ptr, dev(sc), dev(q8), dev(xs), dev(s8), None, out, N, K)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert_fp16_close(host(out), ex, bd, ref, what="unaligned")


def test_gemv_qkv(qe, orc):
    K, nq, nkv, hd = 1536, 12, 2, 128
    mats = [orc.synth_w4(100 + i, n, K) for i, n in enumerate((nq * hd, nkv * hd, nkv * hd))]
    _, q8, xs, s8 = _act(orc, K, 8)
    outs = [empty(n, torch.float16) for n in (nq * hd, nkv * hd, nkv * hd)]
    dw = [(dev(w), dev(s)) for w, s in mats]
    view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0], dw[2][1], outs[2])
    qe.launch_gemv_qkv_w4a8(view, dev(q8), dev(xs), dev(s8), in_features=K, num_q_heads=nq, num_kv_heads=nkv,
                            head_dim=hd)
    for (w, s), o, n in zip(mats, outs, (nq * hd, nkv * hd, nkv * hd)):
        ref, ex, bd = orc.gemv_w4a8(w, s, q8, xs, s8, n, K)
        assert_fp16_close(host(o), ex, bd, ref, what="qkv")


@pytest.mark.parametrize("I,K", [(8960, 1536), (512, 256), (1536, 8960)])
def test_gemv_swiglu_w4a8(qe, orc, I, K):
    qw, sc = orc.synth_w4(33 + I, 2 * I, K)
    _, q8, xs, s8 = _act(orc, K, 9)
    out = empty(I, torch.float16)
    qe.launch_gemv_dual_gate_up_swiglu_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), out, K, I)
    ref, ex, bd = orc.gemv_swiglu_w4a8(qw, sc, q8, xs, s8, K, I)
    assert_fp16_close(host(out), ex, bd, ref, what="swiglu w4a8")


@pytest.mark.parametrize("N,K", [(8960, 1536), (1536, 8960), (64, 128), (333, 2560), (50, 20480), (1001, 4096),
                                 (7, 16384), (20000, 1536), (13001, 8960)])
def test_gemv_w4a16(qe, orc, N, K):
    """W4A16 GEMV 1536->8960 with in-launch Q8_1 quantization."""
    print(f"gemv_w4a16 N={N} K={K}", flush=True)
    qw, sc = orc.synth_w4(77 + N, N, K)
    x = orc.synth_f16_normal(K + 1, K)
    res = orc.synth_f16_normal(K + 2, N)
    out = empty(N, torch.float16)
    qe.launch_gemv_w4a16(dev(qw), dev(sc), dev(x), dev(res), out, N, K)
    ref, ex, bd = orc.gemv_w4a16(qw, sc, x, N, K, residual=res)
    assert_fp16_close(host(out), ex, bd, ref, what="w4a16")


@pytest.mark.parametrize("H,I", [(1536, 8960), (2560, 10240), (5120, 27648), (256, 512)])
def test_suite3_swiglu_w4a16_sweep(qe, orc, H, I):
    """The reference's Synthetic Suite 3 (tests/test_kernels.cu:242-403):
    same generator, same entry point, its max|err| <= 5e-3 bar, and the
    oracle tolerance on top."""
    print(f"suite3 H={H} I={I}", flush=True)
    x, qw, sc = orc.suite3_inputs(H, I)
    out = empty(I, torch.float16)
    qe.launch_gemv_dual_gate_up_swiglu_w4a16(dev(qw), dev(sc), dev(x), out, H, I)
    got = host(out)
    ref, ex, bd = orc.gemv_swiglu_w4a16(qw, sc, x, H, I)
    assert np.abs(got.astype(np.float32) - ref.astype(np.float32)).max() <= 5e-3
    assert_fp16_close(got, ex, bd, ref, what="suite3")


def test_lm_head_and_argmax(qe, orc):
    """LM head 1536 -> 151936 then greedy argmax (bit-exact)."""
    N, K = 151936, 1536
    qw, sc = orc.synth_w4(2024, N, K)
    _, q8, xs, s8 = _act(orc, K, 12)
    logits = empty(N, torch.float16)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), None, logits, N, K)
    got = host(logits)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert_fp16_close(got, ex, bd, ref, what="lm head")
    val = empty(256, torch.float32)
    idx = empty(256, torch.int32)
    tok = empty(1, torch.int32)
    qe.launch_sample_and_advance(logits, val, idx, None, tok, vocab_size=N)
    assert int(host(tok)[0]) == orc.argmax_f16(got)


def test_gemv_rejects_bad_k(qe):
    with pytest.raises(RuntimeError, match="multiple of 128"):
        qe.launch_gemv_w4a8(empty(10, torch.int32), empty(10, torch.float16), empty(100, torch.int8),
                            empty(1, torch.float32), empty(13, torch.int32), None, empty(4, torch.float16), 4, 100)


@pytest.mark.parametrize("H", [1536, 256])
def test_fused_rmsnorm_qkv(qe, orc, H):
    """Fused RMSNorm + Q8_1 + QKV equals the reference's two-launch sequence
    (rmsnorm_q8_1 then gemv_qkv_w4a8, src/engine.cu:367-379)."""
    nq, nkv, hd = (12, 2, 128) if H == 1536 else (2, 1, 64)
    dims = (nq * hd, nkv * hd, nkv * hd)
    mats = [orc.synth_w4(600 + i, n, H) for i, n in enumerate(dims)]
    x16 = (orc.synth_f16_normal(5, H).astype(np.float32) * 3).astype(np.float16)
    g16 = (1 + 0.2 * orc.synth_f16_normal(6, H).astype(np.float32)).astype(np.float16)
    dw = [(dev(w), dev(s)) for w, s in mats]
    outs = [empty(n, torch.float16) for n in dims]
    norm = empty(H, torch.float16)
    view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0], dw[2][1], outs[2])
    qe.launch_rmsnorm_gemv_qkv_w4a16(dev(x16), dev(g16), norm, view, hidden_size=H, num_q_heads=nq,
                                     num_kv_heads=nkv, head_dim=hd)
    fused = [host(o) for o in outs]
    # two-launch path on the GPU
    q8, sc, s8 = empty(H, torch.int8), empty(H // 128, torch.float32), empty(H // 8, torch.int32)
    norm2 = empty(H, torch.float16)
    qe.launch_rmsnorm_q8_1(dev(x16), dev(g16), norm2, q8, sc, s8, hidden_size=H)
    outs2 = [empty(n, torch.float16) for n in dims]
    view2 = qe.make_qkv_view(dw[0][0], dw[0][1], outs2[0], dw[1][0], dw[1][1], outs2[1], dw[2][0], dw[2][1], outs2[2])
    qe.launch_gemv_qkv_w4a8(view2, q8, sc, s8, in_features=H, num_q_heads=nq, num_kv_heads=nkv, head_dim=hd)
    n_gpu = host(norm)
    # one summation order for the sum of squares in every RMSNorm kernel: the
    # fused prologue and rmsnorm_q8_1 give the same normalized vector, Q8_1
    # and projections, bit for bit
    assert np.array_equal(n_gpu.view(np.uint16), host(norm2).view(np.uint16))
    from helpers import ulp16
    n_ref = orc.rmsnorm_fp16(x16, g16)
    assert np.all(np.abs(n_gpu.astype(np.float64) - n_ref.astype(np.float64)) <= ulp16(n_ref))
    # oracle on the normalized vector the kernel produced
    rq, rs, rs8 = orc.quantize_q8_1(n_gpu)
    assert np.array_equal(host(q8), rq) and np.array_equal(host(s8), rs8)
    for (w, s), f, o2, n in zip(mats, fused, outs2, dims):
        ref, ex, bd = orc.gemv_w4a8(w, s, rq, rs, rs8, n, H)
        assert_fp16_close(f, ex, bd, ref, what="fused qkv")
        assert np.array_equal(f.view(np.uint16), host(o2).view(np.uint16))


@pytest.mark.parametrize("H,I", [(1536, 8960), (256, 300)])
def test_fused_rmsnorm_gate_up(qe, orc, H, I):
    qw, sc = orc.synth_w4(700 + I, 2 * I, H)
    x16 = (orc.synth_f16_normal(7, H).astype(np.float32) * 2).astype(np.float16)
    g16 = (1 + 0.2 * orc.synth_f16_normal(8, H).astype(np.float32)).astype(np.float16)
    out = empty(I, torch.float16)
    norm = empty(H, torch.float16)
    qe.launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(dev(x16), dev(g16), norm, dev(qw), dev(sc), out, H, I)
    n_gpu = host(norm)
    n_ref = orc.rmsnorm_fp16(x16, g16)
    from helpers import ulp16
    assert np.all(np.abs(n_gpu.astype(np.float64) - n_ref.astype(np.float64)) <= ulp16(n_ref))
    ref, ex, bd = orc.gemv_swiglu_w4a16(qw, sc, n_gpu, H, I)
    assert_fp16_close(host(out), ex, bd, ref, what="fused gate_up")
    # bit-identical to the reference's two launches (src/engine.cu:414-424)
    q8, xs, s8 = empty(H, torch.int8), empty(H // 128, torch.float32), empty(H // 8, torch.int32)
    norm2, out2 = empty(H, torch.float16), empty(I, torch.float16)
    qe.launch_rmsnorm_q8_1(dev(x16), dev(g16), norm2, q8, xs, s8, hidden_size=H)
    qe.launch_gemv_dual_gate_up_swiglu_w4a8(dev(qw), dev(sc), q8, xs, s8, out2, H, I)
    assert np.array_equal(n_gpu.view(np.uint16), host(norm2).view(np.uint16))
    assert np.array_equal(host(out).view(np.uint16), host(out2).view(np.uint16))


def test_gemv_w4a16_residual_inplace_down(qe, orc):
    """Down projection with the quantizer fused (W4A16 entry point) and the
    residual in place, as the fused decode layer issues it."""
    N, K = 1536, 8960
    qw, sc = orc.synth_w4(800, N, K)
    x = orc.synth_f16_normal(9, K)
    res = orc.synth_f16_normal(10, N)
    out = dev(res)
    qe.launch_gemv_w4a16(dev(qw), dev(sc), dev(x), out, out, N, K)
    ref, ex, bd = orc.gemv_w4a16(qw, sc, x, N, K, residual=res)
    assert_fp16_close(host(out), ex, bd, ref, what="down w4a16 inplace")


@pytest.mark.parametrize("N", [4096, 4097, 20000])
def test_gemv_two_rows_per_segment_tails(qe, orc, N):
    """Row counts >= 4096 use two rows per segment; odd counts exercise the
    clamped tail row."""
    K = 1536
    qw, sc = orc.synth_w4(900 + N, N, K)
    _, q8, xs, s8 = _act(orc, K, 13)
    got = _gemv_w4a8(qe, qw, sc, q8, xs, s8, N, K)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert_fp16_close(got, ex, bd, ref, what=f"rps2 N={N}")


@pytest.mark.parametrize("H,nq,nkv,pos", [(1536, 12, 2, 0), (1536, 12, 2, 777), (256, 2, 1, 4095)])
def test_fused_qkv_rope_kv_append_bit_identical(qe, orc, H, nq, nkv, pos):
    """RMSNorm + QKV GEMV with bias + RoPE + KV append in the epilogue equals,
    bit for bit, the two launches it replaces (rmsnorm_gemv_qkv_w4a16 then
    qkv_bias_rope_kv_append)."""
    hd, max_seq = 128, 4096
    dims = (nq * hd, nkv * hd, nkv * hd)
    mats = [orc.synth_w4(700 + i, n, H) for i, n in enumerate(dims)]
    x16 = (orc.synth_f16_normal(7, H).astype(np.float32) * 2).astype(np.float16)
    g16 = (1 + 0.2 * orc.synth_f16_normal(8, H).astype(np.float32)).astype(np.float16)
    rng = np.random.default_rng(pos)
    biases = [dev((rng.standard_normal(n) * 0.1).astype(np.float16)) for n in dims]
    dw = [(dev(w), dev(s)) for w, s in mats]
    raw = np.zeros(64, np.int32)
    raw[1] = pos
    ctl = dev(raw)
    results = []
    for fused in (True, False):
        outs = [empty(n, torch.float16) for n in dims]
        kc = torch.zeros((nkv, max_seq, hd), dtype=torch.float16, device="cuda")
        vc = torch.zeros((nkv, max_seq, hd), dtype=torch.float16, device="cuda")
        view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0], dw[2][1], outs[2])
        if fused:
            qe.launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16(dev(x16), dev(g16), None, view, biases[0], biases[1],
                                                            biases[2], kc, vc, ctl, hidden_size=H, num_q_heads=nq,
                                                            num_kv_heads=nkv, head_dim=hd, max_seq_len=max_seq)
        else:
            qe.launch_rmsnorm_gemv_qkv_w4a16(dev(x16), dev(g16), None, view, hidden_size=H, num_q_heads=nq,
                                             num_kv_heads=nkv, head_dim=hd)
            qe.launch_qkv_bias_rope_kv_append(outs[0], outs[1], outs[2], biases[0], biases[1], biases[2], kc, vc, ctl,
                                              1, num_q_heads=nq, num_kv_heads=nkv, head_dim=hd, max_seq_len=max_seq)
        results.append([host(o).view(np.uint16) for o in outs] + [host(kc).view(np.uint16), host(vc).view(np.uint16)])
    for a, b, name in zip(results[0], results[1], ("q", "k", "v", "k_cache", "v_cache")):
        assert np.array_equal(a, b), name
    assert np.any(results[0][3][:, pos] != 0)  # the cache row was written
