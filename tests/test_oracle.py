"""Pins the CPU oracle (oracle/) against what the reference and mathematics fix.

The reference ships no golden vectors for this path (its `models/` holds only
`.gitkeep`); its own checks are the CPU golden in tests/test_kernels.cu:308-363,
the closed-form packing in tools/export_qwen25.py:42-76 and the kernel sources.
Each test below checks the oracle against an independent statement (numpy,
exhaustive enumeration, closed forms, invariants), chosen so that a dropped
term, a wrong rounding mode or a permuted nibble fails one of them.
"""
import numpy as np
import pytest


# ---------------------------------------------------------------- fp16 -----
def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h = bits.view(np.float16)
    got = orc.f16_to_f32(h)
    ref = h.astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(orc):
    rng = np.random.default_rng(1)
    # every fp16 value, every midpoint between neighbours, and random floats
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    f = h.astype(np.float32)
    f = f[np.isfinite(f)]
    fs = np.sort(np.unique(f))
    mids = ((fs[:-1].astype(np.float64) + fs[1:].astype(np.float64)) / 2).astype(np.float32)
    rnd = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1.0, 1e3, 6e4)
    ])
    edge = np.array([65504.0, 65519.99, 65520.0, 70000.0, -65520.0, 2.0 ** -24, 2.0 ** -25,
                     3 * 2.0 ** -26, 2.0 ** -26, 0.0, -0.0, np.inf, -np.inf], np.float32)
    allv = np.concatenate([f, mids, rnd, edge])
    got = orc.f32_to_f16(allv)
    ref = allv.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    assert np.isnan(orc.f32_to_f16(np.array([np.nan], np.float32))[0])


# ------------------------------------------------------------ packing ------
def _pack_like_exporter(q):
    """tools/export_qwen25.py:59-72 packing formula, for q[..., 8] in [0,15]."""
    q = q.astype(np.uint32)
    return (q[..., 0] | (q[..., 4] << 4) | (q[..., 1] << 8) | (q[..., 5] << 12)
            | (q[..., 2] << 16) | (q[..., 6] << 20) | (q[..., 3] << 24) | (q[..., 7] << 28))


def test_nibble_layout_exhaustive(orc):
    # every position x every value
    for pos in range(8):
        for v in range(16):
            q = np.full(8, 8, np.int64)
            q[pos] = v
            w = int(_pack_like_exporter(q[None])[0])
            assert orc.unpack_w4(w) == q.tolist()
            assert orc.pack_w4(q) == w
    rng = np.random.default_rng(2)
    for w in rng.integers(0, 2 ** 32, 500, dtype=np.uint64):
        q = orc.unpack_w4(int(w))
        assert int(_pack_like_exporter(np.array(q)[None])[0]) == int(w)


def _unpack_np(qw, N, K):
    """Independent numpy unpack: element 8w+j <- bits of the exporter layout."""
    qw = qw.reshape(N, K // 8).astype(np.uint32)
    shifts = np.array([0, 8, 16, 24, 4, 12, 20, 28], np.uint32)
    return ((qw[:, :, None] >> shifts[None, None, :]) & 0xF).reshape(N, K).astype(np.int64)


def test_dequant_matches_numpy_fp16(orc):
    rng = np.random.default_rng(3)
    N, K = 16, 256
    qw, sc = orc.synth_w4(7, N, K)
    q = _unpack_np(qw, N, K)
    s = np.repeat(sc.astype(np.float32), 128, axis=1)
    # (q-8) exact; product of 4-bit int and fp16 exact in fp32 -> one RNE to fp16
    ref = ((q - 8).astype(np.float32) * s).astype(np.float16)
    got = orc.dequant_w4_f16(qw, sc, N, K)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    # the 0x6400 bias trick of quant_primitives.cuh:101-113 is exact: 1024+q and 1032 are fp16
    for qq in range(16):
        assert float(np.float16(1024 + qq) - np.float16(1032)) == qq - 8


# ---------------------------------------------------------- quantizer ------
def _quant_np(x16):
    """numpy float32 statement of test_kernels.cu:311-326 (IEEE ops, half-away rounding)."""
    x = x16.astype(np.float32).reshape(-1, 128)
    mx = np.abs(x).max(axis=1)
    d = np.maximum(mx / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    inv = (np.float32(1.0) / d).astype(np.float32)
    v = (x * inv[:, None]).astype(np.float32)
    r = np.sign(v) * np.floor(np.abs(v) + 0.5)  # half away from zero
    q = np.clip(r, -127, 127).astype(np.int8).reshape(-1)
    s8 = -8 * q.astype(np.int32).reshape(-1, 8).sum(axis=1)
    return q, d, s8


def test_quantizer_matches_numpy_and_invariants(orc):
    rng = np.random.default_rng(4)
    for K in (128, 256, 1536, 8960):
        x = rng.standard_normal(K).astype(np.float16)
        q, d, s8 = orc.quantize_q8_1(x)
        rq, rd, rs8 = _quant_np(x)
        assert np.array_equal(q, rq)
        assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
        assert np.array_equal(s8, rs8)
        # invariants: |q| <= 127, the group max maps to +-127, |x - q*d| <= d/2 (+1 ulp)
        qg = q.reshape(-1, 128).astype(np.int32)
        assert np.abs(qg).max() <= 127
        assert np.all(np.abs(qg).max(axis=1) == 127)
        err = np.abs(x.astype(np.float64).reshape(-1, 128) - qg * d[:, None].astype(np.float64))
        assert np.all(err <= d[:, None] * 0.5000001)
        assert np.array_equal(s8, -8 * q.astype(np.int32).reshape(-1, 8).sum(1))


def test_quantizer_special_cases(orc):
    # all-zero group: d = 1e-8, q = 0, sum8 = 0
    q, d, s8 = orc.quantize_q8_1(np.zeros(128, np.float16))
    assert np.all(q == 0) and d[0] == np.float32(1e-8) and np.all(s8 == 0)
    # ties round half away from zero (std::round), not half-to-even:
    # max 127 -> d = 1, inv_d = 1 exactly, so x = 2.5 -> 3, -2.5 -> -3, 0.5 -> 1
    x = np.zeros(128, np.float16)
    x[0] = 127.0
    x[1], x[2], x[3], x[4] = 2.5, -2.5, 0.5, 4.5
    q, d, _ = orc.quantize_q8_1(x)
    assert d[0] == 1.0
    assert q[:5].tolist() == [127, 3, -3, 1, 5]
    # tiny values quantize against the 1e-8 floor, and clamp at 127
    x = np.zeros(128, np.float16)
    x[0] = np.float16(6e-8)  # smallest subnormal
    q, d, _ = orc.quantize_q8_1(x)
    assert d[0] == np.float32(1e-8) and q[0] == 6


def test_attn_epilogue_quantizer(orc):
    rng = np.random.default_rng(5)
    acc = rng.standard_normal(12 * 128).astype(np.float32)
    out, q, d, s8 = orc.quantize_q8_1_attn(acc)
    a = acc.reshape(12, 128)
    rd = np.maximum(np.abs(a).max(1) / np.float32(127), np.float32(1e-8)).astype(np.float32)
    rq = np.clip(np.rint((a / rd[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(q, rq.reshape(-1))
    assert np.array_equal(out, acc.astype(np.float16))
    assert np.array_equal(s8, -8 * q.astype(np.int32).reshape(-1, 8).sum(1))
    # ties to even here (the kernel's __float2int_rn): acc/d = 2.5 -> 2
    a = np.zeros(128, np.float32)
    a[0], a[1] = 127.0, 2.5
    _, q, _, _ = orc.quantize_q8_1_attn(a)
    assert q[1] == 2


# ------------------------------------------------------------ dot/GEMV -----
def test_group_dots_bruteforce(orc):
    rng = np.random.default_rng(6)
    N, K = 8, 384
    qw, sc = orc.synth_w4(9, N, K)
    x = rng.standard_normal(K).astype(np.float16)
    q8, xs, s8 = orc.quantize_q8_1(x)
    got = orc.group_dots(qw, q8, s8, N, K)
    w = _unpack_np(qw, N, K) - 8
    ref = (w * q8.astype(np.int64)[None, :]).reshape(N, K // 128, 128).sum(-1)
    assert np.array_equal(got, ref)
    # all weights 8 (zero point) -> zero dot regardless of x
    qw8 = np.full_like(qw, 0x88888888)
    assert np.all(orc.group_dots(qw8, q8, s8, N, K) == 0)
    # sum8 is used as given (dp4a seed), exactly as quant_primitives.cuh:28-32
    s8b = s8.copy()
    s8b[3] += 5
    d2 = orc.group_dots(qw, q8, s8b, N, K)
    assert np.all(d2[:, 0] - got[:, 0] == 5) and np.array_equal(d2[:, 1:], got[:, 1:])


def test_gemv_against_float64_matmul(orc):
    rng = np.random.default_rng(7)
    N, K = 96, 1536
    qw, sc = orc.synth_w4(11, N, K)
    x = rng.standard_normal(K).astype(np.float16)
    res = rng.standard_normal(N).astype(np.float16)
    q8, xs, s8 = orc.quantize_q8_1(x)
    y, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K, residual=res)
    w = (_unpack_np(qw, N, K) - 8).astype(np.float64)
    wsc = np.repeat(sc.astype(np.float64), 128, axis=1)
    xq = q8.astype(np.float64) * np.repeat(xs.astype(np.float64), 128)
    ref = (w * wsc) @ xq + res.astype(np.float64)
    # oracle rounds (w_s * x_s) to fp32 before use; that bounds the difference
    assert np.allclose(ex, ref, rtol=0, atol=1e-6 * bd.max())
    assert np.array_equal(y, ex.astype(np.float32).astype(np.float16))
    # W4A16 entry = quantize then W4A8
    y2, ex2, _ = orc.gemv_w4a16(qw, sc, x, N, K, residual=res)
    assert np.array_equal(y2, y) and np.array_equal(ex2, ex)


def test_gemv_one_hot_extracts_column(orc):
    N, K = 32, 256
    qw, sc = orc.synth_w4(13, N, K)
    sc = np.ones_like(sc)
    for col in (0, 5, 127, 128, 200, 255):
        x = np.zeros(K, np.float16)
        x[col] = 127.0  # -> q = 127 with d = 1 in its group, other group d = 1e-8, q = 0
        q8, xs, s8 = orc.quantize_q8_1(x)
        y, ex, _ = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
        expect = (_unpack_np(qw, N, K)[:, col] - 8) * 127.0
        assert np.array_equal(ex, expect.astype(np.float64))


def test_swiglu_gemv(orc):
    rng = np.random.default_rng(8)
    I, K = 40, 256
    qw, sc = orc.synth_w4(17, 2 * I, K)
    x = rng.standard_normal(K).astype(np.float16)
    y, ex, _ = orc.gemv_swiglu_w4a16(qw, sc, x, K, I)
    q8, xs, s8 = orc.quantize_q8_1(x)
    _, rows, _ = orc.gemv_w4a8(qw, sc, q8, xs, s8, 2 * I, K)
    g, u = rows[0::2], rows[1::2]
    ref = g / (1.0 + np.exp(-g)) * u
    assert np.allclose(ex, ref, rtol=1e-12, atol=0)
    assert np.array_equal(y, ex.astype(np.float32).astype(np.float16))


# ---------------------------------------------------------------- GEMM -----
def test_gemm_against_numpy(orc):
    rng = np.random.default_rng(9)
    M, N, K = 5, 24, 256
    qw, sc = orc.synth_w4(19, N, K)
    A = rng.standard_normal((M, K)).astype(np.float16)
    R = rng.standard_normal((M, N)).astype(np.float16)
    y, ex, bd = orc.gemm_w4a16(qw, sc, A, M, N, K)
    wdq = ((_unpack_np(qw, N, K) - 8).astype(np.float32) * np.repeat(sc.astype(np.float32), 128, 1)).astype(np.float16)
    ref = A.astype(np.float64) @ wdq.astype(np.float64).T
    assert np.allclose(ex, ref, rtol=1e-12, atol=1e-12)
    assert np.array_equal(y, ref.astype(np.float32).astype(np.float16))
    # residual epilogue: fp16(fp16(acc) + res)
    yr, _, _ = orc.gemm_w4a16(qw, sc, A, M, N, K, residual=R)
    assert np.array_equal(yr, (y.astype(np.float32) + R.astype(np.float32)).astype(np.float16))
    # swiglu over interleaved columns
    I = N // 2
    ys, exs, _ = orc.gemm_swiglu_w4a16(qw, sc, A, M, K, I)
    g, u = ref[:, 0::2], ref[:, 1::2]
    assert np.allclose(exs, g / (1 + np.exp(-g)) * u, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------- norm / argmax -----
def _f16(v):
    """Round a float64 value once to fp16 (round to nearest even)."""
    return float(np.float16(v))


def _rms_closed(x_i, mean_sq, gamma_i, eps=1e-6, divisor_fix=1.0, eps_outside=False,
                round_inv=True, one_rounding=False):
    """Closed form of one RMSNorm output for inputs whose mean square is known
    exactly (constant vectors, one-hot vectors), in float64 with one fp16
    rounding per fp16 operation of rmsnorm_rope.cu:214-227.  The keyword
    arguments produce the plausible misreadings the tests must reject."""
    m = mean_sq * divisor_fix
    inv = 1.0 / (np.sqrt(m) + eps) if eps_outside else 1.0 / np.sqrt(m + eps)
    h = _f16(inv) if round_inv else inv
    if one_rounding:
        return _f16(x_i * h * gamma_i)
    return _f16(_f16(x_i * h) * gamma_i)


def test_rmsnorm_constant_vector_closed_form(orc):
    """x = c (every element), gamma = g: mean(x^2) = c^2 exactly, so every
    output is fp16(fp16(c * fp16(1/sqrt(c^2 + eps))) * g)."""
    H = 1536
    cs = [3.0, -3.0, 0.5, 1.25, 0.0078125, 0.00390625, 7.0, 100.0, 0.2998046875,
          1.099609375, 0.7001953125, -2.19921875, 1.7001953125]
    gs = [1.0, 1.5, 0.7998046875, 3.0]
    caught = {"eps_outside": 0, "no_eps": 0, "unrounded_inv": 0, "one_rounding": 0}
    for c in cs:
        for g in gs:
            x = np.full((1, H), c, np.float16)
            gamma = np.full(H, g, np.float16)
            got = orc.rmsnorm_fp16(x, gamma).astype(np.float64)
            want = _rms_closed(c, c * c, g)
            assert np.all(got == want), (c, g, got[0, 0], want)
            caught["eps_outside"] += want != _rms_closed(c, c * c, g, eps_outside=True)
            caught["no_eps"] += want != _rms_closed(c, c * c, g, eps=0.0)
            caught["unrounded_inv"] += want != _rms_closed(c, c * c, g, round_inv=False)
            caught["one_rounding"] += want != _rms_closed(c, c * c, g, one_rounding=True)
    # the chosen inputs tell every misreading apart from the reference formula
    assert all(v > 0 for v in caught.values()), caught


def test_rmsnorm_one_hot_closed_form(orc):
    """x = a * e_i: mean(x^2) = a^2 / H, element i becomes
    fp16(fp16(a * fp16(1/sqrt(a^2/H + eps))) * gamma_i) ~ sign(a) sqrt(H) and
    every other element is exactly zero."""
    caught_divisor = 0
    for H in (128, 256, 1536, 8960):
        for a, i in ((1.0, 0), (-2.5, 7), (0.125, 127), (60000.0, 5), (0.0009765625, 3)):
            x = np.zeros((1, H), np.float16)
            x[0, i] = a
            gamma = np.full(H, 1.0, np.float16)
            gamma[i] = 0.5
            got = orc.rmsnorm_fp16(x, gamma)[0].astype(np.float64)
            want = _rms_closed(a, a * a / H, 0.5)
            assert got[i] == want, (H, a, got[i], want)
            assert np.count_nonzero(np.delete(got, i)) == 0
            if abs(a) >= 1.0:  # eps is negligible
                assert abs(abs(got[i]) - 0.5 * np.sqrt(H)) <= 0.01 * np.sqrt(H)
            caught_divisor += want != _rms_closed(a, a * a / H, 0.5, divisor_fix=H / (H - 1))
    assert caught_divisor > 0  # a divisor of H - 1 fails this test


def test_rmsnorm_symmetries(orc):
    """rmsnorm(-x) = -rmsnorm(x) bit for bit; doubling gamma doubles every
    output exactly (fp16 multiplication by 2 is exact away from overflow)."""
    rng = np.random.default_rng(10)
    for H in (128, 1536, 8960):
        x = rng.standard_normal((3, H)).astype(np.float16)
        g = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
        y = orc.rmsnorm_fp16(x, g)
        assert np.array_equal(orc.rmsnorm_fp16(-x, g).view(np.uint16), (-y).view(np.uint16))
        y2 = orc.rmsnorm_fp16(x, (g.astype(np.float32) * 2).astype(np.float16))
        normal = np.abs(y.astype(np.float32)) >= 2.0 ** -14  # subnormals round on a fixed grid
        assert normal.mean() > 0.99
        assert np.array_equal(y2[normal], (y.astype(np.float32) * 2).astype(np.float16)[normal])
        # rows are independent
        assert np.array_equal(orc.rmsnorm_fp16(x[1:2], g), y[1:2])
        # the output's RMS is |gamma|-weighted 1 within fp16 rounding
        rms = np.sqrt(np.mean((y.astype(np.float64) / g.astype(np.float64)) ** 2, axis=1))
        assert np.all(np.abs(rms - 1) < 2e-3)


def test_argmax_tie_break_and_nan(orc):
    rng = np.random.default_rng(11)
    v = rng.standard_normal(151936).astype(np.float16)
    assert orc.argmax_f16(v) == int(np.argmax(v))
    v[100] = v[90000] = np.float16(30.0)
    assert orc.argmax_f16(v) == 100  # lowest index wins a tie
    v[50] = np.nan
    assert orc.argmax_f16(v) == 100  # NaN never wins
    assert orc.argmax_f16(np.full(10, -np.inf, np.float16)) == 0
    assert orc.argmax_f16(np.full(10, np.nan, np.float16)) == 0


# ------------------------------------------------------ synthetic data -----
def test_suite3_generator_matches_mt19937_recipe(orc):
    """x follows std::mt19937(42+H) + uniform_real_distribution<float>
    (libstdc++ generate_canonical: one 32-bit draw / 2^32), as in
    tests/test_kernels.cu:265-272; numpy's legacy RandomState is the same MT19937."""
    H, I = 256, 512
    x, qw, sc = orc.suite3_inputs(H, I)
    rs = np.random.RandomState(42 + H)
    raw = rs.randint(0, 2 ** 32, size=H, dtype=np.uint32)
    sf = np.float32(1.0) / np.sqrt(np.float32(H))
    u = (raw.astype(np.float32) / np.float32(4294967296.0)).astype(np.float32)
    u = np.where(u >= 1, np.nextafter(np.float32(1), np.float32(0)), u)
    xr = (u * (sf - (-sf)) + (-sf)).astype(np.float32).astype(np.float16)
    assert np.array_equal(x, xr)
    q = _unpack_np(qw, 2 * I, H)
    assert q.min() == 2 and q.max() == 14
    counts = np.bincount(q.reshape(-1), minlength=16)[2:15]
    assert counts.min() > 0.9 * counts.mean()
    assert np.all(sc == np.float16(np.float32(0.05) * sf))


def test_suite3_nibbles_match_lemire_draws(orc):
    """The Suite 3 nibbles bit for bit: std::uniform_int_distribution<int>(2, 14)
    on a 32-bit mt19937 is, in libstdc++ 11 (bits/uniform_int_dist.h, _S_nd),
    Lemire's nearly divisionless method - q = 2 + (x * 13) >> 32 for each
    32-bit draw x, redrawing only when (x * 13) mod 2^32 < 2^32 mod 13 (never
    in these draws) - one draw per nibble after the H draws of x, nibbles
    q0..q7 of a word in draw order (tests/test_kernels.cu:288-300).  (A
    libstdc++ older than 11 divides instead and would give other nibbles.)"""
    for H, I in ((256, 512), (1536, 256)):
        _, qw, _ = orc.suite3_inputs(H, I)
        words = 2 * I * (H // 8)
        raw = np.random.RandomState(42 + H).randint(0, 2 ** 32, size=H + 8 * words, dtype=np.uint32)
        prod = raw[H:].astype(np.uint64) * np.uint64(13)
        assert np.all((prod & np.uint64(0xFFFFFFFF)) >= np.uint64((2 ** 32) % 13))  # no redraw happened
        qd = (2 + (prod >> np.uint64(32))).astype(np.uint32).reshape(words, 8)
        packed = (qd[:, 0] | (qd[:, 4] << 4) | (qd[:, 1] << 8) | (qd[:, 5] << 12) | (qd[:, 2] << 16) |
                  (qd[:, 6] << 20) | (qd[:, 3] << 24) | (qd[:, 7] << 28)).astype(np.uint32)
        assert np.array_equal(qw.reshape(-1), packed)


def test_synth_distributions(orc):
    qw, sc = orc.synth_w4(123, 256, 1536)
    q = _unpack_np(qw, 256, 1536)
    counts = np.bincount(q.reshape(-1), minlength=16)
    assert counts.min() > 0.95 * counts.mean()
    s = sc.astype(np.float64)
    assert s.min() >= 0 and abs(s.mean() - 0.02 * np.sqrt(2 / np.pi)) < 1e-3
    x = orc.synth_f16_normal(5, 200000).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


# --------------------------------------------------------- sampling -------
def test_philox4x32_10_known_answers(orc):
    """Philox-4x32-10 known-answer vectors of the Random123 distribution
    (Salmon et al., SC'11): counter, key -> output."""
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kat:
        assert list(orc.philox4x32_10(ctr, key)) == want


def test_philox_uniform_placement_and_range(orc):
    """sampling.cu:13-53: counter (subsequence, offset, 0, 0), key (seed lo,
    seed hi), u = clamp((float(w0) + 1) / 4294967298.0f, 1e-7, 1 - 1e-7)."""
    w0 = orc.philox4x32_10([0, 0, 0, 0], [0, 0])[0]
    want = np.float32((np.float32(w0) + np.float32(1.0)) / np.float32(4294967298.0))
    assert np.float32(orc.philox_uniform(0, 0, 0)) == want
    seed = 0x299F31D0A4093822
    w0 = orc.philox4x32_10([7, 11, 0, 0], [seed & 0xFFFFFFFF, seed >> 32])[0]
    want = np.float32((np.float32(w0) + np.float32(1.0)) / np.float32(4294967298.0))
    assert np.float32(orc.philox_uniform(seed, 7, 11)) == want
    us = np.array([orc.philox_uniform(1234, i, 5) for i in range(20000)], np.float64)
    assert us.min() >= np.float32(1e-7) and us.max() <= np.float32(1 - 1e-7)
    hist = np.histogram(us, bins=20, range=(0, 1))[0]
    chi2 = ((hist - 1000.0) ** 2 / 1000.0).sum()
    assert chi2 < 50  # 19 dof: p ~ 1e-4 at 43


def test_gumbel_sampling_follows_softmax(orc):
    """Gumbel-max: argmax(l/T - log(-log u)) is distributed as softmax(l/T).
    A sign or scale slip in the noise or temperature breaks the frequencies."""
    logits = np.array([1.0, 0.0, -1.0, 0.5], np.float16)
    T = 0.7
    counts = np.zeros(4)
    n = 6000
    for pos in range(n):
        tok, _ = orc.sample_f16(logits, T, 42, pos)
        counts[tok] += 1
    p = np.exp(logits.astype(np.float64) / T)
    p /= p.sum()
    chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
    assert chi2 < 20  # 3 dof
    # temperature <= 1e-5 is greedy
    tok, vals = orc.sample_f16(logits, 1e-6, 42, 3)
    assert tok == 0 and np.array_equal(vals, logits.astype(np.float32))


def test_multithreaded_swiglu_gemv_matches_scalar(orc):
    """The multi-core CPU baseline computes the same fp16 outputs as the scalar golden."""
    qw, sc = orc.synth_w4(17, 2 * 384, 1536)
    x = orc.synth_f16_normal(18, 1536)
    q8, xs, s8 = orc.quantize_q8_1(x)
    ref = orc.gemv_swiglu_w4a8(qw, sc, q8, xs, s8, 1536, 384)[0]
    for threads in (1, 3, 8):
        got = orc.gemv_swiglu_w4a8_mt(qw, sc, q8, xs, s8, 1536, 384, threads)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
