"""GPU parity of sample_and_advance (src/kernels/sampling.cu:60-232): greedy
argmax (lowest index on ties, NaN never wins), Gumbel-max temperature
sampling against the oracle's Philox restatement, control-block advance, and
the fused LM-head + sampling launches."""
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


def _argmax(qe, logits16, control=None):
    val = empty(256, torch.float32)
    idx = empty(256, torch.int32)
    tok = empty(1, torch.int32)
    qe.launch_sample_and_advance(dev(logits16), val, idx, control, tok, vocab_size=logits16.size)
    return int(host(tok)[0])


@pytest.mark.parametrize("n", [1, 100, 65536, 151936, 300000])
def test_argmax_random(qe, orc, n):
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n).astype(np.float16)
    assert _argmax(qe, v) == orc.argmax_f16(v) == int(np.argmax(v))


def test_argmax_ties_nan_inf(qe, orc):
    n = 151936
    v = np.full(n, -3.0, np.float16)
    for i in (151935, 70000, 5, 140000):
        v[i] = np.float16(9.0)  # four-way tie: lowest index wins
    v[3] = np.nan
    v[4] = np.inf if False else np.float16(8.0)
    assert _argmax(qe, v) == orc.argmax_f16(v) == 5
    # all NaN / -inf -> index 0 (the reference's initial best_idx)
    assert _argmax(qe, np.full(n, np.nan, np.float16)) == 0
    assert _argmax(qe, np.full(n, -np.inf, np.float16)) == 0
    # many equal maxima spread over blocks
    v = np.zeros(n, np.float16)
    assert _argmax(qe, v) == 0
    v[1:] = np.float16(1.0)
    assert _argmax(qe, v) == 1


def test_control_block_advance(qe):
    # DeviceControlBlock {token_id, seq_pos, temperature, reserved, rng_seed}, 256-byte aligned
    raw = np.zeros(64, np.int32)
    raw[1] = 41  # seq_pos
    seed = np.array([1337], np.uint64)
    raw[4:6] = seed.view(np.int32)
    ctl = dev(raw)
    v = np.zeros(1000, np.float16)
    v[777] = 5
    tok = _argmax(qe, v, control=ctl)
    out = host(ctl)
    assert tok == 777 and out[0] == 777 and out[1] == 42
    assert out[4:6].view(np.uint64)[0] == np.uint64(1337 + 0x9E3779B97F4A7C15)


def _ctl(seq_pos=0, temperature=0.0, seed=0):
    raw = np.zeros(64, np.int32)
    raw[1] = seq_pos
    raw[2:3] = np.array([temperature], np.float32).view(np.int32)
    raw[4:6] = np.array([seed], np.uint64).view(np.int32)
    return dev(raw)


def _near_tie(vals, a, b):
    return abs(float(vals[a]) - float(vals[b])) <= 1e-5 * max(1.0, abs(float(vals[a])))


@pytest.mark.parametrize("temperature,seed,pos", [(0.7, 1, 0), (1.0, 0x9E3779B97F4A7C15, 77), (0.05, 12345, 4000),
                                                  (2.5, 7, 1)])
def test_temperature_sampling_matches_oracle(qe, orc, temperature, seed, pos):
    rng = np.random.default_rng(seed % 1000 + pos)
    v = (rng.standard_normal(151936) * 3).astype(np.float16)
    val = empty(256, torch.float32)
    idx = empty(256, torch.int32)
    tok = empty(1, torch.int32)
    ctl = _ctl(pos, temperature, seed)
    qe.launch_sample_and_advance(dev(v), val, idx, ctl, tok, vocab_size=v.size)
    got = int(host(tok)[0])
    want, vals = orc.sample_f16(v, temperature, seed, pos)
    # logf may differ by an ulp between the device and the host: only a near tie may flip
    assert got == want or _near_tie(vals, got, want)
    out = host(ctl)
    assert out[0] == got and out[1] == pos + 1
    assert out[4:6].view(np.uint64)[0] == np.uint64((seed + 0x9E3779B97F4A7C15) % 2 ** 64)


def _lm_head_inputs(orc, V, K, seed):
    qw, sc = orc.synth_w4(seed, V, K)
    x = orc.synth_f16_normal(seed + 1, K)
    return qw, sc, x


@pytest.mark.parametrize("V,K", [(151936, 1536), (5000, 1536), (777, 256), (40000, 4096)])
def test_fused_lm_head_greedy(qe, orc, V, K):
    """Fused LM head + argmax: logits bit-identical to the plain W4A8 GEMV,
    token = argmax over those logits, control block advanced."""
    qw, sc, x = _lm_head_inputs(orc, V, K, 11 + V)
    q8, xs, s8 = (empty(K, torch.int8), empty(K // 128, torch.float32), empty(K // 8, torch.int32))
    qe.launch_quantize_fp16_to_q8_1(dev(x), q8, xs, s8, K)
    ref_logits = empty(V, torch.float16)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), q8, xs, s8, None, ref_logits, V, K)
    logits = empty(V, torch.float16)
    val = empty(qe.LM_HEAD_SAMPLE_PARTS, torch.float32)
    idx = empty(qe.LM_HEAD_SAMPLE_PARTS, torch.int32)
    tok = empty(1, torch.int32)
    ctl = _ctl(9)
    qe.launch_gemv_lm_head_sample_w4a8(dev(qw), dev(sc), q8, xs, s8, logits, val, idx, ctl, tok, vocab_size=V,
                                       in_features=K)
    lg = host(logits)
    assert np.array_equal(lg.view(np.uint16), host(ref_logits).view(np.uint16))
    assert int(host(tok)[0]) == orc.argmax_f16(lg)
    out = host(ctl)
    assert out[0] == int(host(tok)[0]) and out[1] == 10
    # without the logits buffer: same token
    tok2 = empty(1, torch.int32)
    qe.launch_gemv_lm_head_sample_w4a8(dev(qw), dev(sc), q8, xs, s8, None, val, idx, _ctl(9), tok2, vocab_size=V,
                                       in_features=K)
    assert int(host(tok2)[0]) == int(host(tok)[0])


def test_fused_rmsnorm_lm_head_temperature(qe, orc):
    """RMSNorm + LM head + Gumbel sampling in two launches: logits bit-identical
    to rmsnorm_q8_1 -> gemv_w4a8 (one summation order for every RMSNorm),
    token equal to the oracle's sample over those logits."""
    V, K = 151936, 1536
    qw, sc, x = _lm_head_inputs(orc, V, K, 5)
    gamma = (1.0 + 0.1 * np.random.default_rng(2).standard_normal(K)).astype(np.float16)
    q8, xs, s8 = (empty(K, torch.int8), empty(K // 128, torch.float32), empty(K // 8, torch.int32))
    qe.launch_rmsnorm_q8_1(dev(x), dev(gamma), None, q8, xs, s8, hidden_size=K)
    ref_logits = empty(V, torch.float16)
    qe.launch_gemv_w4a8(dev(qw), dev(sc), q8, xs, s8, None, ref_logits, V, K)
    for temperature, seed, pos in ((0.0, 0, 3), (0.8, 99, 3), (1.3, 2024, 500)):
        logits = empty(V, torch.float16)
        val = empty(qe.LM_HEAD_SAMPLE_PARTS, torch.float32)
        idx = empty(qe.LM_HEAD_SAMPLE_PARTS, torch.int32)
        tok = empty(1, torch.int32)
        qe.launch_rmsnorm_gemv_lm_head_sample_w4a16(dev(x), dev(gamma), None, dev(qw), dev(sc), logits, val, idx,
                                                    _ctl(pos, temperature, seed), tok, vocab_size=V,
                                                    hidden_size=K)
        lg = host(logits)
        assert np.array_equal(lg.view(np.uint16), host(ref_logits).view(np.uint16))
        got = int(host(tok)[0])
        want, vals = orc.sample_f16(lg, temperature, seed, pos)
        assert got == want or _near_tie(vals, got, want)
