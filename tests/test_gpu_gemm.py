"""GPU parity of the prefill dequant-GEMM family (MFMA) against the oracle.

Reference: src/kernels/gemm_prefill.cu (kernels :319-610, launchers
:616-684).  fp16 A, fp16 dequantized W, fp32 accumulation, fp16 output;
residual added as fp16(fp16(acc) + res).  Tolerance: helpers.assert_fp16_close.
At the full BASELINE configs[3] sizes (M = 512, 1024) the oracle checks 16
full rows of each output (the double-precision oracle over all M rows would
take minutes on the CPU).
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


def _A(orc, M, K, seed):
    return orc.synth_f16_normal(seed, M * K).reshape(M, K)


@pytest.mark.parametrize("M,N,K", [(128, 1536, 1536), (128, 1536, 8960), (37, 200, 256), (1, 64, 128),
                                   (300, 130, 384), (16, 2048, 1536), (129, 257, 128)])
def test_gemm_plain(qe, orc, M, N, K):
    print(f"gemm M={M} N={N} K={K}", flush=True)
    qw, sc = orc.synth_w4(M + N + K, N, K)
    A = _A(orc, M, K, 5)
    out = empty((M, N), torch.float16)
    qe.launch_gemm_prefill_w4a16(dev(qw), dev(sc), dev(A), None, out, M, N, K)
    ref, ex, bd = orc.gemm_w4a16(qw, sc, A, M, N, K)
    assert_fp16_close(host(out), ex, bd, ref, what=f"gemm {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(128, 1536, 1536), (64, 1536, 8960), (50, 96, 256)])
def test_gemm_residual_inplace(qe, orc, M, N, K):
    """O-proj / down-proj of prefill: residual == output (src/engine.cu:500-524)."""
    qw, sc = orc.synth_w4(7 * N, N, K)
    A = _A(orc, M, K, 6)
    R = orc.synth_f16_normal(8, M * N).reshape(M, N)
    out = dev(R)
    qe.launch_gemm_prefill_w4a16(dev(qw), dev(sc), dev(A), out, out, M, N, K)
    got = host(out)
    ref, ex, bd = orc.gemm_w4a16(qw, sc, A, M, N, K, residual=R)
    _, acc, _ = orc.gemm_w4a16(qw, sc, A, M, N, K)
    # fp16(fp16(acc)+res) rounds twice: the first rounding (half an ulp of
    # acc, or a full ulp when the GPU's fp32 acc lands on the other side of a
    # rounding boundary) is added to the floor.
    from helpers import ulp16
    assert_fp16_close(got, ex, bd + ulp16(acc) * 2.0 ** 20, ref, what="gemm residual",
                      max_floor_frac=1.0)  # the floor carries the fp16 rounding of acc before the add


def test_gemm_qkv(qe, orc):
    M, K, nq, nkv, hd = 128, 1536, 12, 2, 128
    dims = (nq * hd, nkv * hd, nkv * hd)
    mats = [orc.synth_w4(300 + i, n, K) for i, n in enumerate(dims)]
    A = _A(orc, M, K, 9)
    outs = [empty((M, n), torch.float16) for n in dims]
    dw = [(dev(w), dev(s)) for w, s in mats]
    view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0], dw[2][1], outs[2])
    qe.launch_gemm_prefill_qkv_w4a16(view, dev(A), M, in_features=K, num_q_heads=nq, num_kv_heads=nkv, head_dim=hd)
    for (w, s), o, n in zip(mats, outs, dims):
        ref, ex, bd = orc.gemm_w4a16(w, s, A, M, n, K)
        assert_fp16_close(host(o), ex, bd, ref, what="gemm qkv")


def test_gemm_qkv_ragged_heads(qe, orc):
    """Head counts whose column ranges do not align with the tiles."""
    M, K, nq, nkv, hd = 70, 256, 3, 1, 40
    dims = (nq * hd, nkv * hd, nkv * hd)
    mats = [orc.synth_w4(400 + i, n, K) for i, n in enumerate(dims)]
    A = _A(orc, M, K, 10)
    outs = [empty((M, n), torch.float16) for n in dims]
    dw = [(dev(w), dev(s)) for w, s in mats]
    view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0], dw[2][1], outs[2])
    qe.launch_gemm_prefill_qkv_w4a16(view, dev(A), M, in_features=K, num_q_heads=nq, num_kv_heads=nkv, head_dim=hd)
    for (w, s), o, n in zip(mats, outs, dims):
        ref, ex, bd = orc.gemm_w4a16(w, s, A, M, n, K)
        assert_fp16_close(host(o), ex, bd, ref, what="gemm qkv ragged")


@pytest.mark.parametrize("M,I,K", [(128, 8960, 1536), (33, 100, 256)])
def test_gemm_swiglu(qe, orc, M, I, K):
    print(f"gemm swiglu M={M} I={I}", flush=True)
    qw, sc = orc.synth_w4(500 + I, 2 * I, K)
    A = _A(orc, M, K, 11)
    out = empty((M, I), torch.float16)
    qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a16(dev(qw), dev(sc), dev(A), out, M, hidden_size=K,
                                                     intermediate_size=I)
    ref, ex, bd = orc.gemm_swiglu_w4a16(qw, sc, A, M, K, I)
    assert_fp16_close(host(out), ex, bd, ref, what="gemm swiglu")


@pytest.mark.parametrize("K", [512, 640])  # the 256-k quad layout and the 64-k step layout
def test_gemm_every_tile_ragged(qe, orc, K):
    """Each block tile (64x64, 64x128, 128x64, 128x128) with one and two K
    slices, forced, on shapes whose rows and columns end inside a tile: plain
    with residual, QKV with head ranges off the tile grid, and SwiGLU (the
    epilogues' partial-fragment and column-tail paths)."""
    from helpers import ulp16
    M, N = 37, 200
    nq, nkv, hd = 3, 1, 40
    I = 100
    qw, sc = orc.synth_w4(600 + K, N, K)
    A = _A(orc, M, K, 12)
    R = orc.synth_f16_normal(13, M * N).reshape(M, N)
    dims = (nq * hd, nkv * hd, nkv * hd)
    mats = [orc.synth_w4(610 + i, n, K) for i, n in enumerate(dims)]
    gq, gs = orc.synth_w4(620 + K, 2 * I, K)
    ref_p, ex_p, bd_p = orc.gemm_w4a16(qw, sc, A, M, N, K, residual=R)
    _, acc_p, _ = orc.gemm_w4a16(qw, sc, A, M, N, K)
    refs_q = [orc.gemm_w4a16(w, s, A, M, n, K) for (w, s), n in zip(mats, dims)]
    ref_g, ex_g, bd_g = orc.gemm_swiglu_w4a16(gq, gs, A, M, K, I)
    dA = dev(A)
    dw = [(dev(w), dev(s)) for w, s in mats]
    try:
        for tile in (1, 2, 3, 4):
            for slices in (1, 2):
                what = f"tile {tile} slices {slices} K {K}"
                print(what, flush=True)
                qe.set_tuning("gemm_tile", tile)
                qe.set_tuning("gemm_slices", slices)
                out = dev(R)
                qe.launch_gemm_prefill_w4a16(dev(qw), dev(sc), dA, out, out, M, N, K)
                assert_fp16_close(host(out), ex_p, bd_p + ulp16(acc_p) * 2.0 ** 20, ref_p, what="plain " + what,
                                  max_floor_frac=1.0)  # the floor carries the fp16 rounding of acc
                outs = [empty((M, n), torch.float16) for n in dims]
                view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0],
                                        dw[2][1], outs[2])
                qe.launch_gemm_prefill_qkv_w4a16(view, dA, M, in_features=K, num_q_heads=nq, num_kv_heads=nkv,
                                                 head_dim=hd)
                for o, (ref, ex, bd) in zip(outs, refs_q):
                    assert_fp16_close(host(o), ex, bd, ref, what="qkv " + what)
                outg = empty((M, I), torch.float16)
                qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a16(dev(gq), dev(gs), dA, outg, M, hidden_size=K,
                                                                 intermediate_size=I)
                assert_fp16_close(host(outg), ex_g, bd_g, ref_g, what="swiglu " + what)
    finally:
        qe.set_tuning("gemm_tile", 0)
        qe.set_tuning("gemm_slices", 0)


@pytest.mark.parametrize("M", [512, 1024])
@pytest.mark.parametrize("N,K", [(2048, 1536), (1536, 1536), (17920, 1536), (1536, 8960)])
def test_gemm_full_configs(qe, orc, M, N, K):
    """configs[3] at full size against the oracle: 16 full output rows spread
    over every M tile (first, last, and rows in between), all N columns, with
    the path's plain tolerance; every output row is finite."""
    print(f"gemm full M={M} N={N} K={K}", flush=True)
    qw, sc = orc.synth_w4(N + K, N, K)
    A = _A(orc, M, K, M)
    out = empty((M, N), torch.float16)
    qe.launch_gemm_prefill_w4a16(dev(qw), dev(sc), dev(A), None, out, M, N, K)
    got = host(out)
    assert np.all(np.isfinite(got.astype(np.float32)))
    rows = sorted(set([0, 1, 63, 64, 127, 128, M // 2 - 1, M // 2, M // 2 + 37, M - 129, M - 128, M - 65,
                       M - 64, M - 2, M - 1, 200]))
    assert len(rows) == 16
    ref, ex, bd = orc.gemm_w4a16(qw, sc, A[rows], len(rows), N, K)
    assert_fp16_close(got[rows], ex, bd, ref, what=f"gemm full {M}x{N}x{K}")


def test_gemm_rejects_bad_k(qe):
    with pytest.raises(RuntimeError, match="multiple of 128"):
        qe.launch_gemm_prefill_w4a16(empty(10, torch.int32), empty(10, torch.float16), empty(100, torch.float16),
                                     None, empty(4, torch.float16), 1, 4, 100)


def test_gemm_split_k_deterministic_across_interleaved_launches(qe, orc):
    """Small-M shapes reduce K across blocks through the shared scratch: results
    are bit-identical launch after launch, with other split-K shapes in between."""
    shapes = [(40, 2048, 1536), (40, 1536, 8960), (40, 1536, 1536), (7, 512, 4096), (128, 1536, 8960)]
    data = []
    for (M, N, K) in shapes:
        qw, sc = orc.synth_w4(M * 3 + N + K, N, K)
        A = _A(orc, M, K, N)
        data.append((dev(qw), dev(sc), dev(A), empty((M, N), torch.float16), M, N, K, qw, sc, A))
    first = []
    for rep in range(12):
        for i, (dqw, dsc, dA, out, M, N, K, *_r) in enumerate(data):
            qe.launch_gemm_prefill_w4a16(dqw, dsc, dA, None, out, M, N, K)
            got = host(out)
            if rep == 0:
                first.append(got.copy())
            else:
                assert np.array_equal(got.view(np.uint16), first[i].view(np.uint16)), f"rep {rep} shape {i}"
    for i, (dqw, dsc, dA, out, M, N, K, qw, sc, A) in enumerate(data):
        ref, ex, bd = orc.gemm_w4a16(qw, sc, A, M, N, K)
        assert_fp16_close(first[i], ex, bd, ref, what=f"split-K shape {i}")


# ---- W4A8 prefill GEMM (int8 MFMA) ------------------------------------------------
def _q8_rows(qe, A):
    M, K = A.shape
    q8, xs, s8 = empty(M * K, torch.int8), empty(M * K // 128, torch.float32), empty(M * K // 8, torch.int32)
    qe.launch_quantize_fp16_to_q8_1(dev(A.reshape(-1)), q8, xs, s8, M * K)
    return q8, xs, s8


def _rows_ref(orc, qw, sc, q8, xs, s8, rows, N, K, residual=None):
    hq, hx, hs = host(q8).reshape(-1, K), host(xs).reshape(-1, K // 128), host(s8).reshape(-1, K // 8)
    out = []
    for m in rows:
        out.append(orc.gemv_w4a8(qw, sc, hq[m], hx[m], hs[m], N, K,
                                 residual=None if residual is None else residual[m]))
    return [np.stack(t) for t in zip(*out)]


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (37, 200, 256), (128, 1536, 1536), (300, 130, 384),
                                   (64, 1536, 8960), (129, 2048, 1536), (1024, 1536, 1536)])
def test_gemm_w4a8_rows_equal_w4a8_gemv(qe, orc, M, N, K):
    """Every output row of the int8-MFMA GEMM is the W4A8 GEMV of that row's
    Q8_1 (the activation quantized by the bit-exact quantizer)."""
    print(f"gemm_w4a8 M={M} N={N} K={K}", flush=True)
    qw, sc = orc.synth_w4(M + 3 * N + K, N, K)
    A = _A(orc, M, K, 15)
    q8, xs, s8 = _q8_rows(qe, A)
    out = empty((M, N), torch.float16)
    qe.launch_gemm_prefill_w4a8(dev(qw), dev(sc), q8, xs, s8, None, out, M, N, K)
    rows = list(range(M)) if M <= 130 else sorted(set([0, 1, M // 2, M - 2, M - 1] + list(range(60, 70))))
    ref, ex, bd = _rows_ref(orc, qw, sc, q8, xs, s8, rows, N, K)
    assert_fp16_close(host(out)[rows], ex, bd, ref, what=f"gemm_w4a8 {M}x{N}x{K}")


def test_gemm_w4a8_residual_qkv_swiglu(qe, orc):
    M, H, I = 96, 1536, 512
    A = _A(orc, M, H, 16)
    q8, xs, s8 = _q8_rows(qe, A)
    from helpers import ulp16
    # residual in place
    qw, sc = orc.synth_w4(90, H, H)
    R = orc.synth_f16_normal(91, M * H).reshape(M, H)
    out = dev(R)
    qe.launch_gemm_prefill_w4a8(dev(qw), dev(sc), q8, xs, s8, out, out, M, H, H)
    rows = list(range(0, M, 7))
    y16, acc, bd = _rows_ref(orc, qw, sc, q8, xs, s8, rows, H, H)
    # the GEMM epilogue: fp16(fp16(acc) + res), an fp16 add after rounding
    ref = (y16.astype(np.float16) + R[rows]).astype(np.float16)
    ex = acc + R[rows].astype(np.float64)
    assert_fp16_close(host(out)[rows], ex, bd + ulp16(acc) * 2.0 ** 20, ref, what="gemm_w4a8 residual",
                      max_floor_frac=1.0)  # the floor carries the fp16 rounding of acc before the add
    # QKV: three matrices, ragged boundaries handled per column
    dims = (1536, 256, 256)
    mats = [orc.synth_w4(92 + i, n, H) for i, n in enumerate(dims)]
    outs = [empty((M, n), torch.float16) for n in dims]
    dw = [(dev(w), dev(s)) for w, s in mats]
    view = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0], dw[1][0], dw[1][1], outs[1], dw[2][0], dw[2][1], outs[2])
    qe.launch_gemm_prefill_qkv_w4a8(view, q8, xs, s8, M)
    for (w, s), o, n in zip(mats, outs, dims):
        ref, ex, bd = _rows_ref(orc, w, s, q8, xs, s8, rows, n, H)
        assert_fp16_close(host(o)[rows], ex, bd, ref, what="gemm_w4a8 qkv")
    # gate/up SwiGLU
    qgu, sgu = orc.synth_w4(95, 2 * I, H)
    mlp = empty((M, I), torch.float16)
    qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a8(dev(qgu), dev(sgu), q8, xs, s8, mlp, M, hidden_size=H,
                                                    intermediate_size=I)
    hq, hx, hs = host(q8).reshape(M, H), host(xs).reshape(M, -1), host(s8).reshape(M, -1)
    for m in rows:
        ref, ex, bd = orc.gemv_swiglu_w4a8(qgu, sgu, hq[m], hx[m], hs[m], H, I)
        assert_fp16_close(host(mlp)[m], ex, bd, ref, what="gemm_w4a8 swiglu")


def test_gemm_split_k_streams_do_not_share_partials(qe, orc):
    """Two split-K GEMMs in flight on two streams at once give the results
    each gives alone: every stream has its own workspace for the partials."""
    M, H, I = 128, 1536, 8960
    qa, sa = orc.synth_w4(41, 2 * I, H)
    qb, sb = orc.synth_w4(42, H, I)
    A1, A2 = _A(orc, M, H, 43), _A(orc, M, I, 44)
    dqa, dsa, dqb, dsb, dA1, dA2 = dev(qa), dev(sa), dev(qb), dev(sb), dev(A1), dev(A2)
    alone = []
    for fn in (lambda o, s: qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a16(dqa, dsa, dA1, o, M, stream=s,
                                                                            hidden_size=H, intermediate_size=I),
               lambda o, s: qe.launch_gemm_prefill_w4a16(dqb, dsb, dA2, None, o, M, H, I, stream=s)):
        o = empty((M, I if len(alone) == 0 else H), torch.float16)
        fn(o, None)
        alone.append(host(o))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    qe.gemm_reserve_workspace(s1)
    qe.gemm_reserve_workspace(s2)
    for _ in range(3):
        o1, o2 = empty((M, I), torch.float16), empty((M, H), torch.float16)
        torch.cuda.synchronize()
        for rep in range(4):  # interleave the launches so the two streams overlap
            qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a16(dqa, dsa, dA1, o1, M, stream=s1, hidden_size=H,
                                                             intermediate_size=I)
            qe.launch_gemm_prefill_w4a16(dqb, dsb, dA2, None, o2, M, H, I, stream=s2)
        torch.cuda.synchronize()
        assert np.array_equal(host(o1).view(np.uint16), alone[0].view(np.uint16))
        assert np.array_equal(host(o2).view(np.uint16), alone[1].view(np.uint16))
    ref, ex, bd = orc.gemm_w4a16(qb, sb, A2[:8], 8, H, I)
    assert_fp16_close(alone[1][:8], ex, bd, ref, what="down M=128 rows 0..7")


def test_gemm_launch_never_allocates_and_plan_depends_only_on_the_stream(qe, orc):
    """A prefill GEMM on a fresh stream makes no hipMalloc (the library's
    workspace allocation counter does not move) and runs without K slices;
    captured into a graph on another fresh stream it gives the same bits.
    After qe_gemm_reserve_workspace (one allocation) the stream splits K, and
    eager and captured launches on it agree bit for bit again.  Every result
    is within the oracle tolerance."""
    M, N, K = 128, 1536, 8960
    assert qe.gemm_prefill_plan(M, N, K)[1] > 1  # this shape splits when it can
    qw, sc = orc.synth_w4(51, N, K)
    A = _A(orc, M, K, 52)
    dq, ds, dA = dev(qw), dev(sc), dev(A)
    ref, ex, bd = orc.gemm_w4a16(qw, sc, A[:16], 16, N, K)
    torch.cuda.synchronize()

    def eager(s):
        out = empty((M, N), torch.float16)
        torch.cuda.synchronize()
        qe.launch_gemm_prefill_w4a16(dq, ds, dA, None, out, M, N, K, stream=s)
        torch.cuda.synchronize()
        return host(out).copy()

    def captured(s):
        out = empty((M, N), torch.float16)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            qe.launch_gemm_prefill_w4a16(dq, ds, dA, None, out, M, N, K)
        outs = []
        for _ in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            outs.append(host(out).copy())
        assert all(np.array_equal(o.view(np.uint16), outs[0].view(np.uint16)) for o in outs)
        return outs[0]

    before = qe.gemm_workspace_allocations()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    unsplit = eager(s1)
    assert qe.gemm_workspace_allocations() == before, "a launch allocated"
    assert np.array_equal(captured(s2).view(np.uint16), unsplit.view(np.uint16))
    assert qe.gemm_workspace_allocations() == before, "a captured launch allocated"
    assert np.array_equal(eager(s1).view(np.uint16), unsplit.view(np.uint16))
    # the unsplit plan is the forced single-slice plan on a stream with a workspace
    qe.set_tuning("gemm_slices", 1)
    try:
        assert np.array_equal(eager(None).view(np.uint16), unsplit.view(np.uint16))
    finally:
        qe.set_tuning("gemm_slices", 0)
    assert_fp16_close(unsplit[:16], ex, bd, ref, what="gemm without workspace")
    qe.gemm_reserve_workspace(s1)
    assert qe.gemm_workspace_allocations() == before + 1
    qe.gemm_reserve_workspace(s1)  # idempotent
    assert qe.gemm_workspace_allocations() == before + 1
    split = eager(s1)
    assert np.array_equal(captured(s1).view(np.uint16), split.view(np.uint16))
    assert_fp16_close(split[:16], ex, bd, ref, what="gemm with workspace")
    # caller memory as the workspace gives the same plan and bits
    buf = torch.empty(32 << 20, dtype=torch.uint8, device="cuda")
    qe.gemm_attach_workspace(buf, buf.numel(), s2)
    assert np.array_equal(eager(s2).view(np.uint16), split.view(np.uint16))
    qe.gemm_release_workspace(s2)
    qe.gemm_release_workspace(s1)
    assert np.array_equal(eager(s1).view(np.uint16), unsplit.view(np.uint16))
    assert qe.gemm_workspace_allocations() == before + 1


# ---- tiled weight layout (load-time repack) ----------------------------------------
@pytest.mark.parametrize("M,N,K", [(128, 1536, 1536), (128, 17920, 1536), (64, 1536, 8960), (1024, 1536, 1536),
                                   (37, 1000, 768), (300, 130, 256), (1, 33, 512)])
def test_gemm_tiled_layout_bit_identical(qe, orc, M, N, K):
    """The GEMM on the tiled copy gives the bits of the GEMM on the .qwenbin
    layout for the same tile and K-slice plan (the same arithmetic), with and
    without a residual, and matches the oracle with its own plan."""
    print(f"gemm tiled M={M} N={N} K={K}", flush=True)
    qw, sc = orc.synth_w4(M + 5 * N + K, N, K)
    A = _A(orc, M, K, 61)
    R = orc.synth_f16_normal(62, M * N).reshape(M, N)
    dq, ds = dev(qw), dev(sc)
    tw, ts = qe.w4_tiled(dq, ds, N, K)
    pad = (N + 31) // 32 * 32
    assert tw.numel() == pad * K // 8 and ts.numel() == pad * K // 128
    for res, plan in ((None, (4, 1)), (R, (2, 2)), (None, (1, 3))):
        a, b = empty((M, N), torch.float16), empty((M, N), torch.float16)
        dres = dev(res) if res is not None else None
        with forced_plan(qe, *plan):
            qe.launch_gemm_prefill_w4a16(dq, ds, dev(A), dres, a, M, N, K)
            qe.launch_gemm_prefill_w4a16_tiled(tw, ts, dev(A), dres, b, M, N, K)
        assert np.array_equal(host(a).view(np.uint16), host(b).view(np.uint16)), plan
    rows = min(M, 16)
    ref, ex, bd = orc.gemm_w4a16(qw, sc, A[:rows], rows, N, K)
    qe.launch_gemm_prefill_w4a16_tiled(tw, ts, dev(A), None, b, M, N, K)
    assert_fp16_close(host(b)[:rows], ex, bd, ref, what="tiled gemm")


class forced_plan:
    """Forces the prefill GEMM tile (1..4) and K-slice count while active."""
    def __init__(self, qe, tile, slices):
        self.qe, self.tile, self.slices = qe, tile, slices

    def __enter__(self):
        self.qe.set_tuning("gemm_tile", self.tile)
        self.qe.set_tuning("gemm_slices", self.slices)

    def __exit__(self, *exc):
        self.qe.set_tuning("gemm_tile", 0)
        self.qe.set_tuning("gemm_slices", 0)


def test_gemm_tiled_qkv_and_swiglu_bit_identical(qe, orc):
    M, H, I = 160, 1536, 4096
    A = _A(orc, M, H, 63)
    for nq, nkv, hd in ((12, 2, 128), (4, 1, 64), (3, 3, 96)):
        dims = (nq * hd, nkv * hd, nkv * hd)
        mats = [orc.synth_w4(70 + i + nq, n, H) for i, n in enumerate(dims)]
        dw = [(dev(w), dev(s)) for w, s in mats]
        tw = [qe.w4_tiled(w, s, n, H) for (w, s), n in zip(dw, dims)]
        outs = [[empty((M, n), torch.float16) for n in dims] for _ in range(2)]
        v0 = qe.make_qkv_view(dw[0][0], dw[0][1], outs[0][0], dw[1][0], dw[1][1], outs[0][1], dw[2][0], dw[2][1],
                              outs[0][2])
        v1 = qe.make_qkv_view(tw[0][0], tw[0][1], outs[1][0], tw[1][0], tw[1][1], outs[1][1], tw[2][0], tw[2][1],
                              outs[1][2])
        with forced_plan(qe, 2, 2):
            qe.launch_gemm_prefill_qkv_w4a16(v0, dev(A), M, in_features=H, num_q_heads=nq, num_kv_heads=nkv,
                                             head_dim=hd)
            qe.launch_gemm_prefill_qkv_w4a16_tiled(v1, dev(A), M, in_features=H, num_q_heads=nq, num_kv_heads=nkv,
                                                   head_dim=hd)
        for a, b in zip(outs[0], outs[1]):
            assert np.array_equal(host(a).view(np.uint16), host(b).view(np.uint16)), (nq, nkv, hd)
    qgu, sgu = orc.synth_w4(80, 2 * I, H)
    dq, ds = dev(qgu), dev(sgu)
    tw, ts = qe.w4_tiled(dq, ds, 2 * I, H)
    a, b = empty((M, I), torch.float16), empty((M, I), torch.float16)
    with forced_plan(qe, 4, 1):
        qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a16(dq, ds, dev(A), a, M, hidden_size=H, intermediate_size=I)
        qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled(tw, ts, dev(A), b, M, hidden_size=H,
                                                               intermediate_size=I)
    assert np.array_equal(host(a).view(np.uint16), host(b).view(np.uint16))
    ref, ex, bd = orc.gemm_swiglu_w4a16(qgu, sgu, A[:8], 8, H, I)
    qe.launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled(tw, ts, dev(A), b, M, hidden_size=H, intermediate_size=I)
    assert_fp16_close(host(b)[:8], ex, bd, ref, what="tiled swiglu, own plan")
    with pytest.raises(RuntimeError, match="multiple of 256"):
        qe.launch_gemm_prefill_w4a16_tiled(tw, ts, dev(A), None, b, M, 64, 128)
