"""GPU parity of greedy sample_and_advance (src/kernels/sampling.cu:60-232):
lowest index on ties, NaN never wins, control-block advance."""
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
