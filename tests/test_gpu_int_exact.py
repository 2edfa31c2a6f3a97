"""Bit-exact GPU parity of the integer stage (quant_primitives.cuh:28-32).

On the inputs of int_exact_inputs every fp32 operation of the path is exact,
so each fp16 output is the round-to-nearest-even of an exact value on both
the GPU and the CPU golden (tests/test_kernels.cu:328-363): the GPU must
reproduce the oracle bit for bit.  The sparse variant keeps outputs below
2048 units, so an int32 group dot that is off by one changes the output;
the dense variant uses full-range nibbles and activations with per-group
power-of-two scales, so a wrong scale index changes the output.
Entry points: gemv_w4a8 (O, down, gate-shape, residual in place), QKV,
gemv_w4a16 (in-launch Q8_1, configs[0] shape), SwiGLU (W4A8 and W4A16),
LM head + argmax (plain and fused sampling epilogue), and the prefill GEMMs
(fp16 MFMA and int8 MFMA, plain / QKV / SwiGLU).
"""
import numpy as np
import pytest
import torch

import int_exact_inputs as ie
from helpers import dev, empty, host

pytestmark = pytest.mark.gpu

SPARSE = dict(sparse=True, act_exps=(0,), w_exps=(0,))
DENSE = dict(sparse=False, act_exps=(0, 1), w_exps=(2, 3, 4))


@pytest.fixture(scope="module")
def qe():
    import qe_amd
    qe_amd.lib()
    qe_amd.gemm_reserve_workspace()  # split-K partials of the default stream's GEMMs
    return qe_amd


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def _case(orc, seed, N, K, kind):
    rng = np.random.default_rng(seed)
    x, main = ie.activation(rng, K, kind["sparse"], kind["act_exps"])
    qw, sc, _ = ie.weights(rng, N, K, main if kind["sparse"] else None, kind["w_exps"])
    q8, xs, s8 = orc.quantize_q8_1(x)
    return x, qw, sc, q8, xs, s8


def _check_exact(got, ref, ex, bd, kind, what):
    gran = 2.0 ** -(max(kind["act_exps"]) + max(kind["w_exps"]))
    assert ie.exact_in_fp32(bd, gran), f"{what}: input construction is not fp32-exact"
    assert np.array_equal(ref.astype(np.float64)[np.abs(ex) < 2048 * gran], ex[np.abs(ex) < 2048 * gran])
    if kind["sparse"]:
        assert ie.visible_fraction(ex, gran) > 0.8
    same = _bits(got) == _bits(ref)
    assert same.all(), (f"{what}: {np.count_nonzero(~same)} of {same.size} outputs differ, first at "
                        f"{np.argmax(~same)}: got {got.reshape(-1)[np.argmax(~same)]!r} "
                        f"want {ref.reshape(-1)[np.argmax(~same)]!r}")


KINDS = [pytest.param(SPARSE, id="sparse"), pytest.param(DENSE, id="dense")]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K", [(1536, 1536), (1536, 8960), (8960, 1536), (200, 16384), (37, 384)])
def test_gemv_w4a8_exact(qe, orc, N, K, kind):
    print(f"exact gemv_w4a8 N={N} K={K} sparse={kind['sparse']}", flush=True)
    x, qw, sc, q8, xs, s8 = _case(orc, N + K, N, K, kind)
    out = empty(N, torch.float16)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), None, out, N, K)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    _check_exact(host(out), ref, ex, bd, kind, f"gemv_w4a8 {N}x{K}")


@pytest.mark.parametrize("kind", KINDS)
def test_gemv_w4a8_residual_inplace_exact(qe, orc, kind):
    N, K = 1536, 8960
    x, qw, sc, q8, xs, s8 = _case(orc, 3, N, K, kind)
    res = np.random.default_rng(4).integers(-300, 300, N).astype(np.float16)
    out = dev(res)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), out, out, N, K)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K, residual=res)
    _check_exact(host(out), ref, ex, bd + np.abs(res), kind, "down + residual in place")


@pytest.mark.parametrize("kind", KINDS)
def test_gemv_qkv_exact(qe, orc, kind):
    K, dims = 1536, (1536, 256, 256)
    rng = np.random.default_rng(5)
    x, main = ie.activation(rng, K, kind["sparse"], kind["act_exps"])
    mats = [ie.weights(rng, n, K, main if kind["sparse"] else None, kind["w_exps"])[:2] for n in dims]
    q8, xs, s8 = orc.quantize_q8_1(x)
    outs = [empty(n, torch.float16) for n in dims]
    dw = [(dev(w), dev(s)) for w, s in mats]
    view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0], dw[2][1], outs[2])
    qe.launch_gemv_qkv_w4a8(view, dev(q8), dev(xs), dev(s8))
    for (w, s), o, n, name in zip(mats, outs, dims, "qkv"):
        ref, ex, bd = orc.gemv_w4a8(w, s, q8, xs, s8, n, K)
        _check_exact(host(o), ref, ex, bd, kind, f"qkv {name}")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K", [(8960, 1536), (1536, 8960), (333, 2560)])
def test_gemv_w4a16_exact(qe, orc, N, K, kind):
    """configs[0] shape with the in-launch quantizer: its Q8_1 of the fp16
    activation must be the oracle's for the outputs to match."""
    print(f"exact gemv_w4a16 N={N} K={K} sparse={kind['sparse']}", flush=True)
    x, qw, sc, q8, xs, s8 = _case(orc, 7 * N + K, N, K, kind)
    assert np.array_equal(q8.astype(np.float64) * np.repeat(xs, 128), x.astype(np.float64))
    out = empty(N, torch.float16)
    qe.launch_gemv_w4a16(dev(qw), dev(sc), dev(x), None, out, N, K)
    ref, ex, bd = orc.gemv_w4a16(qw, sc, x, N, K)
    _check_exact(host(out), ref, ex, bd, kind, f"gemv_w4a16 {N}x{K}")


@pytest.mark.parametrize("I,K", [(8960, 1536), (1536, 8960), (300, 256)])
def test_gemv_swiglu_exact(qe, orc, I, K):
    """Gate values >= 127 (silu(g) == g exactly) and |u| <= 12: every SwiGLU
    output is an exact fp16 integer, for the W4A8 and W4A16 entry points."""
    rng = np.random.default_rng(I + K)
    x, main = ie.activation(rng, K, True, (0,))
    qw, sc = ie.swiglu_weights(rng, I, K, x, main)
    q8, xs, s8 = orc.quantize_q8_1(x)
    ref, ex, bd = orc.gemv_swiglu_w4a8(qw, sc, q8, xs, s8, K, I)
    assert np.array_equal(ref.astype(np.float64), ex) and np.count_nonzero(ex) > I // 4
    for entry in ("w4a8", "w4a16"):
        out = empty(I, torch.float16)
        if entry == "w4a8":
            qe.launch_gemv_dual_gate_up_swiglu_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), out, K, I)
        else:
            qe.launch_gemv_dual_gate_up_swiglu_w4a16(dev(qw), dev(sc), dev(x), out, K, I)
        assert np.array_equal(_bits(host(out)), _bits(ref)), entry


@pytest.mark.parametrize("kind", KINDS)
def test_lm_head_argmax_exact(qe, orc, kind):
    """151936 integer-valued logits, bit-identical, and the greedy
    token (ties to the lowest index: integer logits tie often) through both
    the two-stage sampler and the LM head's fused sampling epilogue."""
    N, K = 151936, 1536
    x, qw, sc, q8, xs, s8 = _case(orc, 11, N, K, kind)
    logits = empty(N, torch.float16)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), None, logits, N, K)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    got = host(logits)
    _check_exact(got, ref, ex, bd, kind, "lm head")
    want = orc.argmax_f16(ref)
    val, idx, tok = empty(2048, torch.float32), empty(2048, torch.int32), empty(1, torch.int32)
    qe.launch_sample_and_advance(logits, val, idx, None, tok, vocab_size=N)
    assert int(host(tok)[0]) == want
    ctl = dev(np.zeros(64, np.int32))
    tok2, logits2 = empty(1, torch.int32), empty(N, torch.float16)
    qe.launch_gemv_lm_head_sample_w4a8(dev(qw), dev(sc), dev(q8), dev(xs), dev(s8), logits2, val, idx, ctl, tok2,
                                       vocab_size=N, in_features=K)
    assert np.array_equal(_bits(host(logits2)), _bits(ref))
    assert int(host(tok2)[0]) == want


def _rows(orc, M, K, seed, kind):
    rng = np.random.default_rng(seed)
    A = np.empty((M, K), np.float16)
    main = None
    for m in range(M):
        A[m], main = ie.activation(rng, K, kind["sparse"], kind["act_exps"], main)
    return rng, A, main


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,N,K", [(128, 1536, 1536), (64, 1536, 8960), (300, 130, 384), (129, 2048, 256)])
def test_gemm_w4a16_exact(qe, orc, M, N, K, kind):
    """fp16 MFMA prefill GEMM: fp16 A times fp16 dequantized weights with fp32
    accumulation is exact on these inputs, split-K slices included."""
    print(f"exact gemm M={M} N={N} K={K} sparse={kind['sparse']}", flush=True)
    rng, A, main = _rows(orc, M, K, M + N + K, kind)
    qw, sc, _ = ie.weights(rng, N, K, main if kind["sparse"] else None, kind["w_exps"])
    out = empty((M, N), torch.float16)
    qe.launch_gemm_prefill_w4a16(dev(qw), dev(sc), dev(A), None, out, M, N, K)
    ref, ex, bd = orc.gemm_w4a16(qw, sc, A, M, N, K)
    gran = 2.0 ** -(max(kind["act_exps"]) + max(kind["w_exps"]))
    assert ie.exact_in_fp32(bd, gran)
    assert np.array_equal(_bits(host(out)), _bits(ref))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,N,K", [(128, 1536, 1536), (64, 1536, 8960), (1024, 256, 1536), (37, 200, 256)])
def test_gemm_w4a8_exact(qe, orc, M, N, K, kind):
    """int8 MFMA prefill GEMM: every row equals the W4A8 GEMV oracle of the
    row's Q8_1 (quantized on the GPU by the bit-exact quantizer) bit for bit."""
    print(f"exact gemm_w4a8 M={M} N={N} K={K} sparse={kind['sparse']}", flush=True)
    rng, A, main = _rows(orc, M, K, 2 * M + N + K, kind)
    qw, sc, _ = ie.weights(rng, N, K, main if kind["sparse"] else None, kind["w_exps"])
    q8, xs, s8 = empty(M * K, torch.int8), empty(M * K // 128, torch.float32), empty(M * K // 8, torch.int32)
    qe.launch_quantize_fp16_to_q8_1(dev(A.reshape(-1)), q8, xs, s8, M * K)
    out = empty((M, N), torch.float16)
    qe.launch_gemm_prefill_w4a8(dev(qw), dev(sc), q8, xs, s8, None, out, M, N, K)
    got = host(out)
    rows = range(M) if M <= 130 else sorted({0, 1, M // 2, M - 1} | set(range(100, 116)))
    for m in rows:
        rq, rs, rs8 = orc.quantize_q8_1(A[m])
        ref, ex, bd = orc.gemv_w4a8(qw, sc, rq, rs, rs8, N, K)
        _check_exact(got[m], ref, ex, bd, kind, f"gemm_w4a8 row {m}")


def test_gemm_qkv_and_swiglu_exact(qe, orc):
    """QKV and gate/up SwiGLU prefill GEMMs (fp16 and int8 MFMA) on exact inputs."""
    M, H, I, dims = 96, 1536, 512, (1536, 256, 256)
    rng, A, main = _rows(orc, M, H, 77, SPARSE)
    mats = [ie.weights(rng, n, H, None, (0, 1))[:2] for n in dims]
    q8, xs, s8 = empty(M * H, torch.int8), empty(M * H // 128, torch.float32), empty(M * H // 8, torch.int32)
    qe.launch_quantize_fp16_to_q8_1(dev(A.reshape(-1)), q8, xs, s8, M * H)
    dw = [(dev(w), dev(s)) for w, s in mats]
    for entry in ("w4a16", "w4a8"):
        outs = [empty((M, n), torch.float16) for n in dims]
        view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0], dw[2][1],
                                outs[2])
        if entry == "w4a16":
            qe.launch_gemm_prefill_qkv_w4a16(view, dev(A), M)
        else:
            qe.launch_gemm_prefill_qkv_w4a8(view, q8, xs, s8, M)
        for (w, s), o, n in zip(mats, outs, dims):
            ref, ex, bd = orc.gemm_w4a16(w, s, A, M, n, H)
            assert ie.exact_in_fp32(bd, 0.5)
            assert np.array_equal(_bits(host(o)), _bits(ref)), f"{entry} qkv n={n}"
    # SwiGLU: the gate rows are built for one activation (gate values >= 127),
    # so every row of A is that activation
    x, main = ie.activation(rng, H, True, (0,))
    qgu, sgu = ie.swiglu_weights(rng, I, H, x, main)
    A2 = np.stack([x] * M)
    ref, ex, _ = orc.gemm_swiglu_w4a16(qgu, sgu, A2, M, H, I)
    assert np.array_equal(ref.astype(np.float64), ex)
    q8b, xsb, s8b = empty(M * H, torch.int8), empty(M * H // 128, torch.float32), empty(M * H // 8, torch.int32)
    qe.launch_quantize_fp16_to_q8_1(dev(A2.reshape(-1)), q8b, xsb, s8b, M * H)
    for entry in ("w4a16", "w4a8"):
        mlp = empty((M, I), torch.float16)
        if entry == "w4a16":
            qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a16(dev(qgu), dev(sgu), dev(A2), mlp, M, hidden_size=H,
                                                             intermediate_size=I)
        else:
            qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a8(dev(qgu), dev(sgu), q8b, xsb, s8b, mlp, M,
                                                            hidden_size=H, intermediate_size=I)
        assert np.array_equal(_bits(host(mlp)), _bits(ref)), f"{entry} swiglu"
