"""GPU checks of the decode-loop kernels around the matrix path and of the
engine built on it.

* embedding: bit-exact against the oracle's W4 dequantization
  (unpack_w4_to_half2_quad, quant_primitives.cuh:92-115);
* flash-decode combine + Q8_1 epilogue (attention_gqa.cu:263-310): bit-exact
  against the oracle when the combined value is exactly the partial (one
  active split with denominator 1);
* combine folded into the O projection: bit-identical to the stand-alone
  combine followed by the W4A8 GEMV (same arithmetic, one launch);
* RoPE / flash decode / prefill attention: float kernels, checked against a
  numpy float64 statement of the same math with a stated tolerance;
* engine: graph replay and eager launches produce the same tokens
  (tests/test_kernels.cu:635-684), same seed -> same tokens.
"""
import math

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


def _ctl(seq_pos=0, token=0):
    raw = np.zeros(64, np.int32)
    raw[0], raw[1] = token, seq_pos
    return dev(raw)


def test_embed_lookup_bit_exact(qe, orc):
    V, H = 1000, 1536
    qw, sc = orc.synth_w4(31, V, H)
    ids = np.array([0, 5, 999, 123, -1, 151936], np.int32)  # invalid ids read row 0
    out = empty((len(ids), H), torch.float16)
    qe.launch_embed_lookup_w4a16(dev(qw), dev(sc), dev(ids), out, None, len(ids), hidden_size=H)
    got = host(out)
    ref_rows = orc.dequant_w4_f16(qw, sc, V, H)
    for i, t in enumerate(ids):
        r = t if 0 <= t < V else 0
        assert np.array_equal(got[i].view(np.uint16), ref_rows[r].view(np.uint16))
    # token from the control block
    out1 = empty((1, H), torch.float16)
    qe.launch_embed_lookup_w4a16(dev(qw), dev(sc), None, out1, _ctl(token=777), 1, hidden_size=H)
    assert np.array_equal(host(out1)[0].view(np.uint16), ref_rows[777].view(np.uint16))


def test_flash_decode_combine_q8_epilogue_bit_exact(qe, orc):
    nq, S, D = 12, 16, 128
    rng = np.random.default_rng(3)
    part = (rng.standard_normal((nq, S, D)) * rng.uniform(0.01, 50, (nq, 1, 1))).astype(np.float32)
    part[3] = 0.0                                   # an all-zero head: d = 1e-8, q = 0
    part[4, 0, :] = 0.0
    part[4, 0, 0], part[4, 0, 1] = 127.0, 2.5       # rint tie: 2.5 -> 2 (half to even)
    lse = np.zeros((nq, S, 2), np.float32)
    lse[:, :, 0] = -np.inf
    lse[:, 0, 0] = rng.standard_normal(nq).astype(np.float32)
    lse[:, 0, 1] = 1.0                              # only split 0 active, denominator 1
    out = empty(nq * D, torch.float16)
    q8 = empty(nq * D, torch.int8)
    sc = empty(nq, torch.float32)
    s8 = empty(nq * D // 8, torch.int32)
    qe.launch_attention_gqa_flash_decode_combine(dev(part), dev(lse), out, nq, q8, sc, s8)
    acc = part[:, 0, :].reshape(-1)
    r_out, r_q8, r_sc, r_s8 = orc.quantize_q8_1_attn(acc)
    assert np.array_equal(host(out).view(np.uint16), r_out.view(np.uint16))
    assert np.array_equal(host(q8), r_q8)
    assert np.array_equal(host(sc).view(np.uint32), r_sc.view(np.uint32))
    assert np.array_equal(host(s8), r_s8)
    assert host(q8)[4 * D + 1] == 2


def _attn_ref(q, kc, vc, seq_len, group):
    nq, D = q.shape
    out = np.zeros((nq, D))
    for h in range(nq):
        kvh = h // group
        k = kc[kvh, :seq_len].astype(np.float64)
        v = vc[kvh, :seq_len].astype(np.float64)
        s = k @ q[h].astype(np.float64) / math.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v
    return out


@pytest.mark.parametrize("nq,nkv,seq_pos", [(12, 2, p) for p in (0, 5, 63, 64, 300, 1024, 1100, 4095)] +
                         [(8, 8, 300), (12, 4, 1100), (14, 2, 77), (16, 1, 2000)])
def test_flash_decode_attention(qe, orc, nq, nkv, seq_pos):
    """Stage 1 (one block per q head and split) + stage 2 against float64
    attention, for Qwen2.5-1.5B's 6:1 grouping and groups of 1, 3, 7, 16."""
    D, max_seq = 128, 4096
    rng = np.random.default_rng(seq_pos)
    q = rng.standard_normal((nq, D)).astype(np.float16)
    kc = rng.standard_normal((nkv, max_seq, D)).astype(np.float16)
    vc = rng.standard_normal((nkv, max_seq, D)).astype(np.float16)
    part = empty(nq * 16 * D, torch.float32)
    lse = empty(nq * 16 * 2, torch.float32)
    out = empty(nq * D, torch.float16)
    q8 = empty(nq * D, torch.int8)
    sc = empty(nq, torch.float32)
    s8 = empty(nq * D // 8, torch.int32)
    qe.launch_attention_gqa_flash_decode(dev(q), dev(kc), dev(vc), part, lse, out, _ctl(seq_pos), num_q_heads=nq,
                                         num_kv_heads=nkv, head_dim=D, max_seq_len=max_seq, out_q8=q8, out_scale=sc,
                                         out_sum8=s8)
    got = host(out).astype(np.float64).reshape(nq, D)
    ref = _attn_ref(q, kc, vc, min(seq_pos + 1, max_seq), nq // nkv)
    # fp32 online softmax vs float64: 2e-3 relative to the head's scale
    assert np.all(np.abs(got - ref) <= 2e-3 * np.abs(ref).max(axis=1, keepdims=True) + 1e-3)
    # Q8_1 epilogue consistent with the fp16 output: |q*d - out| <= d/2 (+ fp16 rounding)
    d = host(sc).astype(np.float64)
    qq = host(q8).astype(np.float64).reshape(nq, D)
    assert np.all(np.abs(qq * d[:, None] - got) <= d[:, None] * 0.5 + 1e-3 * np.abs(got) + 1e-6)
    assert np.array_equal(host(s8), -8 * host(q8).astype(np.int32).reshape(-1, 8).sum(1))


@pytest.mark.parametrize("nq,nkv,seq_pos,res", [(12, 2, 0, True), (12, 2, 300, True), (12, 2, 4095, False),
                                                 (16, 2, 77, True), (8, 1, 1000, False), (4, 4, 17, True),
                                                 (12, 2, 63, False), (12, 2, 64, True), (12, 2, 1500, True)])
def test_attention_combine_gemv_o_bit_identical(qe, orc, nq, nkv, seq_pos, res):
    """partials -> (combine + Q8_1 + O GEMV + residual) in one launch equals
    flash_decode (stage 1 + 2) -> gemv_w4a8 bit for bit; partial buffers start
    as NaN so empty splits are never read as numbers."""
    D, max_seq, H = 128, 4096, 1536
    K = nq * D
    rng = np.random.default_rng(seq_pos + nq)
    q = rng.standard_normal((nq, D)).astype(np.float16)
    kc = rng.standard_normal((nkv, max_seq, D)).astype(np.float16)
    vc = rng.standard_normal((nkv, max_seq, D)).astype(np.float16)
    qw, sc = orc.synth_w4(seq_pos + 5, H, K)
    residual = dev((rng.standard_normal(H)).astype(np.float16)) if res else None
    dq, dkc, dvc, dqw, dsc, ctl = dev(q), dev(kc), dev(vc), dev(qw), dev(sc), _ctl(seq_pos)
    nan = lambda n: torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")
    part, lse = nan(nq * 16 * D), nan(nq * 16 * 2)
    out, q8 = empty(K, torch.float16), empty(K, torch.int8)
    xs, s8 = empty(nq, torch.float32), empty(K // 8, torch.int32)
    qe.launch_attention_gqa_flash_decode(dq, dkc, dvc, part, lse, out, ctl, num_q_heads=nq, num_kv_heads=nkv,
                                         head_dim=D, max_seq_len=max_seq, out_q8=q8, out_scale=xs, out_sum8=s8)
    ref_y = empty(H, torch.float16)
    qe.launch_gemv_w4a8(dqw, dsc, q8, xs, s8, residual, ref_y, H, K)
    part2, lse2 = nan(nq * 16 * D), nan(nq * 16 * 2)
    qe.launch_attention_gqa_flash_decode_partials(dq, dkc, dvc, part2, lse2, ctl, num_q_heads=nq, num_kv_heads=nkv,
                                                  head_dim=D, max_seq_len=max_seq)
    lse_h, lse2_h = host(lse), host(lse2)
    assert np.array_equal(lse_h.view(np.uint32), lse2_h.view(np.uint32))
    live = (lse_h.reshape(nq, 16, 2)[:, :, 1] > 0)
    assert np.array_equal(host(part).reshape(nq, 16, D)[live].view(np.uint32),
                          host(part2).reshape(nq, 16, D)[live].view(np.uint32))
    y, attn = empty(H, torch.float16), empty(K, torch.float16)
    qe.launch_attention_combine_gemv_o_w4a8(part2, lse2, dqw, dsc, residual, y, attn, ctl, out_features=H,
                                            num_q_heads=nq, head_dim=D, max_seq_len=max_seq)
    assert np.array_equal(host(attn).view(np.uint16), host(out).view(np.uint16))
    assert np.array_equal(host(y).view(np.uint16), host(ref_y).view(np.uint16))
    # without the attention copy, in place on the residual (the engine's call)
    if res:
        r2 = residual.clone()
        qe.launch_attention_combine_gemv_o_w4a8(part2, lse2, dqw, dsc, r2, r2, None, None, out_features=H,
                                                num_q_heads=nq, head_dim=D)  # no control block: all 16 read
        assert np.array_equal(host(r2).view(np.uint16), host(ref_y).view(np.uint16))


def test_qkv_bias_rope_kv_append(qe):
    nq, nkv, D, max_seq, T, base = 12, 2, 128, 512, 5, 37
    rng = np.random.default_rng(1)
    q = rng.standard_normal((T, nq * D)).astype(np.float16)
    k = rng.standard_normal((T, nkv * D)).astype(np.float16)
    v = rng.standard_normal((T, nkv * D)).astype(np.float16)
    qb = (rng.standard_normal(nq * D) * 0.1).astype(np.float16)
    kb = (rng.standard_normal(nkv * D) * 0.1).astype(np.float16)
    vb = (rng.standard_normal(nkv * D) * 0.1).astype(np.float16)
    dq, dk, dv = dev(q), dev(k), dev(v)
    kc = torch.zeros((nkv, max_seq, D), dtype=torch.float16, device="cuda")
    vc = torch.zeros((nkv, max_seq, D), dtype=torch.float16, device="cuda")
    qe.launch_qkv_bias_rope_kv_append(dq, dk, dv, dev(qb), dev(kb), dev(vb), kc, vc, _ctl(base), T, num_q_heads=nq,
                                      num_kv_heads=nkv, head_dim=D, max_seq_len=max_seq)

    def rope(x, pos):  # x [heads, D] fp16 after bias
        x = x.astype(np.float64)
        i = np.arange(D // 2)
        inv = np.exp2(-2.0 * i / D * math.log2(1e6))
        a = pos * inv
        x0, x1 = x[:, :D // 2], x[:, D // 2:]
        return np.concatenate([x0 * np.cos(a) - x1 * np.sin(a), x0 * np.sin(a) + x1 * np.cos(a)], axis=1)

    gq, gk, gkc, gvc = host(dq), host(dk), host(kc), host(vc)
    for m in range(T):
        qm = (q[m] + qb).astype(np.float16).reshape(nq, D)
        km = (k[m] + kb).astype(np.float16).reshape(nkv, D)
        vm = (v[m] + vb).astype(np.float16).reshape(nkv, D)
        for got, ref in ((gq[m].reshape(nq, D), rope(qm, base + m)), (gk[m].reshape(nkv, D), rope(km, base + m))):
            assert np.all(np.abs(got.astype(np.float64) - ref) <= 2e-3 * np.abs(ref) + 2e-3)
        assert np.array_equal(gkc[:, base + m], gk[m].reshape(nkv, D))
        assert np.array_equal(gvc[:, base + m], vm)
    assert np.all(gkc[:, base + T:] == 0) and np.all(gkc[:, :base] == 0)


@pytest.mark.parametrize("T,base,nq,nkv", [(1, 0, 12, 2), (37, 0, 12, 2), (128, 0, 12, 2), (20, 100, 12, 2),
                                           (33, 31, 12, 2), (200, 300, 12, 2), (70, 5, 8, 1), (45, 0, 4, 4),
                                           (64, 17, 4, 2), (300, 0, 12, 2), (96, 10, 15, 5), (60, 452, 12, 2)])
def test_prefill_attention(qe, T, base, nq, nkv):
    D, max_seq = 128, 512
    rng = np.random.default_rng(T + base)
    q = rng.standard_normal((T, nq * D)).astype(np.float16)
    kc = rng.standard_normal((nkv, max_seq, D)).astype(np.float16)
    vc = rng.standard_normal((nkv, max_seq, D)).astype(np.float16)
    out = empty((T, nq * D), torch.float16)
    qe.launch_attention_gqa_prefill(dev(q), dev(kc), dev(vc), out, _ctl(base), T, num_q_heads=nq, num_kv_heads=nkv,
                                    head_dim=D, max_seq_len=max_seq, hidden_size=nq * D)
    got = host(out).astype(np.float64)
    for m in range(T):
        ref = _attn_ref(q[m].reshape(nq, D), kc, vc, base + m + 1, nq // nkv).reshape(-1)
        assert np.all(np.abs(got[m] - ref) <= 2e-3 * np.abs(ref).max() + 1e-3)


def _small_cfg(qe, fused=1):
    c = qe.default_config()
    c.num_layers, c.intermediate_size, c.vocab_size, c.max_seq_len, c.prefill_chunk = 2, 512, 4096, 256, 64
    c.fused_decode = fused
    return c


def test_engine_graph_matches_eager_and_is_deterministic(qe, orc):
    prompt = [(i % 1000) + 100 for i in range(40)]  # the reference bench's synthetic prompt (cli_bench.cpp:78-82)
    e = qe.Engine(_small_cfg(qe), seed=7)
    t0 = e.prefill(prompt)
    g = e.decode(12, use_graph=True)
    assert e.seq_pos == len(prompt) + 12
    e.reset()
    assert e.prefill(prompt) == t0
    eager = e.decode(12, use_graph=False)
    assert g == eager
    e2 = qe.Engine(_small_cfg(qe), seed=7)
    assert e2.prefill(prompt) == t0 and e2.decode(12) == g
    assert all(0 <= t < 4096 for t in g)
    assert np.isfinite(e2.logits().astype(np.float32)).all()
    assert g[-1] == orc.argmax_f16(e2.logits())  # fused LM head + sampling: token = argmax of its logits
    assert np.isfinite(e2.hidden_row0().astype(np.float32)).all()
    # the reference's launch sequence (src/engine.cu:361-450) gives the same
    # bits: same tokens, logits and hidden state after every fused launch
    e3 = qe.Engine(_small_cfg(qe, fused=0), seed=7)
    assert e3.prefill(prompt) == t0
    ref_seq = e3.decode(12)
    assert ref_seq == g
    assert np.array_equal(e3.logits().view(np.uint16), e2.logits().view(np.uint16))
    assert np.array_equal(e3.hidden_row0().view(np.uint16), e2.hidden_row0().view(np.uint16))
    for x in (e, e2, e3):
        x.close()


def test_engine_context_limits(qe):
    e = qe.Engine(_small_cfg(qe), seed=1)
    with pytest.raises(RuntimeError, match="context window"):
        e.prefill(list(range(256)))
    with pytest.raises(RuntimeError, match="outside"):
        e.prefill([5000])
    e.prefill(list(range(250)))
    e.decode(6)
    with pytest.raises(RuntimeError, match="context window"):
        e.decode(1)
    prof_ok = e.seq_pos == 256
    e.close()
    assert prof_ok


def test_engine_prefill_lm_head_matches_oracle(qe, orc):
    """After prefill, the engine's final RMSNorm+Q8_1 of the last row is bit-exact
    with the oracle applied to the engine's residual row, and its LM-head logits
    and greedy token match the oracle GEMV over the (tied) embedding."""
    H, V, n = 1536, 4096, 40
    prompt = [(i % 1000) + 100 for i in range(n)]
    engines = []
    for trial in range(2):  # a second engine after the first: no state leaks between engines
        e = qe.Engine(_small_cfg(qe), seed=7)
        tok = e.prefill(prompt)
        hid = e.read("hidden", np.float16, n * H).reshape(n, H)[n - 1]
        fnorm = e.read("final_norm", np.float16, H)
        q8 = e.read("q8", np.int8, H)
        sc = e.read("q8_scale", np.float32, H // 128)
        s8 = e.read("q8_sum8", np.int32, H // 8)
        ew = e.read("embed_w", np.uint32, V * H // 8)
        es = e.read("embed_s", np.float16, V * H // 128)
        logits = e.read("logits", np.float16, V)
        from helpers import ulp16
        nrm_ref = orc.rmsnorm_fp16(hid, fnorm)
        rq, rs, rs8 = orc.quantize_q8_1(nrm_ref)
        if not np.array_equal(q8, rq):  # the norm may differ by one fp16 ulp (sum order)
            assert np.abs(q8.astype(int) - rq.astype(int)).max() <= 1
        ref, ex, bd = orc.gemv_w4a8(ew, es, q8, sc, s8, V, H)
        from helpers import assert_fp16_close
        assert_fp16_close(logits, ex, bd, ref, what="engine lm head")
        assert tok == orc.argmax_f16(logits)
        engines.append((e, tok))
    assert engines[0][1] == engines[1][1]
    for e, _ in engines:
        e.close()


def test_engine_tiled_prefill_matches_qwenbin_layout(qe):
    """The engine's prefill on the tiled weight copies gives the same hidden
    rows, logits and tokens as on the .qwenbin layout for the same GEMM plan,
    over a multi-chunk prompt (chunk 64)."""
    prompt = [(i % 1000) + 100 for i in range(150)]
    outs = []
    for tiled in (1, 0):
        qe.set_tuning("engine_tiled_prefill", tiled)
        try:
            e = qe.Engine(_small_cfg(qe), seed=11)
        finally:
            qe.set_tuning("engine_tiled_prefill", 1)
        qe.set_tuning("gemm_tile", 2)
        qe.set_tuning("gemm_slices", 2)
        try:
            t = e.prefill(prompt)
        finally:
            qe.set_tuning("gemm_tile", 0)
            qe.set_tuning("gemm_slices", 0)
        hid = e.read("hidden", np.float16, 64 * 1536)
        outs.append((t, hid.view(np.uint16).copy(), e.logits().view(np.uint16).copy(), e.decode(4)))
        e.close()
    assert outs[0][0] == outs[1][0]
    assert np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(outs[0][2], outs[1][2])
    assert outs[0][3] == outs[1][3]


def test_engine_multi_chunk_prefill_equals_single_chunk(qe):
    """Prefill in 64-token chunks (later chunks attend to the KV the earlier
    ones wrote, positions rebased, src/engine.cu:529-590) against one 256-token
    chunk.  With one GEMM plan forced (a row's arithmetic then does not depend
    on M) the last residual row, the logits, the first token and the decode
    tokens after it are bit-identical; with each engine's own plan the last
    row differs from the forced result only by fp32 rounding (1 % of its
    largest element)."""
    n = 200
    prompt = [(i * 7919) % 4096 for i in range(n)]
    H = 1536

    def run(chunk, forced):
        cfg = _small_cfg(qe)
        cfg.prefill_chunk = chunk
        e = qe.Engine(cfg, seed=13)
        if forced:
            qe.set_tuning("gemm_tile", 4)
            qe.set_tuning("gemm_slices", 1)
        try:
            t = e.prefill(prompt)
        finally:
            qe.set_tuning("gemm_tile", 0)
            qe.set_tuning("gemm_slices", 0)
        rows = (n - 1) % chunk + 1  # rows of the last chunk in the hidden buffer
        last = e.read("hidden", np.float16, rows * H).reshape(rows, H)[rows - 1].copy()
        lg = e.logits().copy()
        dec = e.decode(8)
        e.close()
        return t, last, lg, dec

    f64, f256 = run(64, True), run(256, True)
    assert f64[0] == f256[0]
    assert np.array_equal(f64[1].view(np.uint16), f256[1].view(np.uint16))
    assert np.array_equal(f64[2].view(np.uint16), f256[2].view(np.uint16))
    assert f64[3] == f256[3]
    p64, p256 = run(64, False), run(256, False)
    from helpers import ulp16
    for got in (p64, p256):
        assert np.all(np.isfinite(got[1].astype(np.float32)))
        err = np.abs(got[1].astype(np.float64) - f64[1].astype(np.float64))
        scale = np.abs(f64[1].astype(np.float64)).max()
        assert err.max() <= 1e-2 * scale + 4 * ulp16(scale), err.max()


def test_engine_destroy_releases_its_gemm_workspace(qe):
    """Every engine registers 32 MiB of its arena as its stream's split-K
    workspace (at most 64 streams per device hold one) and drops the
    registration at destroy: 70 engines created and destroyed in turn all
    succeed, none allocates a library workspace, and the last one still
    prefills with split K (same first token as the first engine)."""
    before = qe.gemm_workspace_allocations()
    prompt = [(i % 1000) + 100 for i in range(100)]
    first = None
    for i in range(70):
        e = qe.Engine(_small_cfg(qe), seed=21)
        if i in (0, 69):
            t = e.prefill(prompt)
            first = t if first is None else first
            assert t == first
        e.close()
    assert qe.gemm_workspace_allocations() == before


@pytest.mark.parametrize("full", [False, True])
def test_engine_arena_buffers_do_not_overlap(qe, full):
    """Every buffer carved out of the engine's arena (weights, tiled copies,
    KV cache, activations, the Q8_1 scratch, partials, control block) starts
    on a 256-byte boundary, ends before the next one starts and inside the
    allocation - the layout property of the reference's scratch non-overlap
    test (tests/test_kernels.cu:687-705), for a small model and the full
    Qwen2.5-1.5B configuration."""
    cfg = qe.default_config() if full else _small_cfg(qe)
    e = qe.Engine(cfg, seed=3)
    spans, total = e.arena_spans()
    e.close()
    assert len(spans) > 20
    ends = 0
    for off, size in spans:  # allocation order = address order
        assert off % 256 == 0 and size > 0
        assert off >= ends, (off, ends)
        ends = off + size
    assert ends <= total
    if full:  # 28 layers x (2 norms, 3 biases, 6 matrices x (weights, scales) and their tiled copies)
        assert len(spans) >= 28 * (5 + 12 + 12)


def test_engine_profile_decode_stages(qe):
    """Per-stage timing of one eager decode step (the reference's
    profile_stages positivity check, tests/test_kernels.cu:708-719): every
    stage positive, the total their sum, one position consumed, and the next
    graph step still matches a fresh engine's."""
    prompt = [(i % 1000) + 100 for i in range(24)]
    e = qe.Engine(_small_cfg(qe), seed=5)
    e.prefill(prompt)
    prof = e.profile_decode()
    assert prof["gemv_ms"] > 0 and prof["attention_ms"] > 0 and prof["other_ms"] > 0
    assert abs(prof["total_ms"] - (prof["gemv_ms"] + prof["attention_ms"] + prof["other_ms"])) < 1e-3
    assert e.seq_pos == len(prompt) + 1
    after = e.decode(3)
    ref = qe.Engine(_small_cfg(qe), seed=5)
    ref.prefill(prompt)
    assert ref.decode(4)[1:] == after
    e.close()
    ref.close()
