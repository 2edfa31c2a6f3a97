"""CPU checks of the exact-input construction used by test_gpu_int_exact:
the packing is the exporter's, the Q8_1 of the activations is exactly (2^-k,
integer q8), the oracle's outputs are fp32-exact, and the sparse variant makes
a one-unit change of a group dot visible in the fp16 output."""
import numpy as np
import pytest

import int_exact_inputs as ie


def test_pack_matches_oracle_unpack(orc):
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, (3, 64))
    w = ie.pack_nibbles(q)
    for n in range(3):
        for j in range(8):
            assert orc.unpack_w4(int(w[n, j])) == q[n, 8 * j:8 * j + 8].tolist()


@pytest.mark.parametrize("sparse,exps", [(True, (0,)), (False, (0, 1, 3))])
def test_activation_quantizes_exactly(orc, sparse, exps):
    rng = np.random.default_rng(1)
    x, main = ie.activation(rng, 8960, sparse, exps)
    q8, xs, s8 = orc.quantize_q8_1(x)
    assert np.all(np.isin(np.log2(xs), -np.asarray(exps, np.float64)))
    assert np.array_equal(q8.astype(np.float64) * np.repeat(xs, 128), x.astype(np.float64))
    assert np.all(np.abs(q8[main]) == 127)
    assert np.array_equal(s8, -8 * q8.astype(np.int64).reshape(-1, 8).sum(1))


@pytest.mark.parametrize("N,K", [(1536, 1536), (1536, 8960), (151936 // 64, 1536)])
def test_outputs_exact_and_sensitive(orc, N, K):
    rng = np.random.default_rng(N + K)
    # sparse: every output exact and an off-by-one group dot visible
    x, main = ie.activation(rng, K, True, (0,))
    qw, sc, q = ie.weights(rng, N, K, main, (0,))
    q8, xs, s8 = orc.quantize_q8_1(x)
    ref, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert ie.exact_in_fp32(bd, 1.0)
    assert ie.visible_fraction(ex, 1.0) > 0.9
    # an off-by-one nibble (one unit of weight times a +-1 activation) changes the fp16 output
    ones = np.nonzero(np.abs(q8) == 1)[0]
    k = int(ones[0])
    q2 = q.copy()
    q2[:, k] = np.where(q2[:, k] < 15, q2[:, k] + 1, q2[:, k] - 1)
    ref2, ex2, _ = orc.gemv_w4a8(ie.pack_nibbles(q2), sc, q8, xs, s8, N, K)
    assert np.all(np.abs(ex2 - ex) == 1)
    assert np.mean(ref2 != ref) > 0.9
    # dense: full-range values, still exact in fp32
    x, _ = ie.activation(rng, K, False, (0, 1))
    qw, sc, _ = ie.weights(rng, N, K, None, (2, 3, 4))
    q8, xs, s8 = orc.quantize_q8_1(x)
    _, ex, bd = orc.gemv_w4a8(qw, sc, q8, xs, s8, N, K)
    assert ie.exact_in_fp32(bd, 2.0 ** -5)
    assert np.all(np.abs(ex) < 65504)


def test_swiglu_construction_exact(orc):
    rng = np.random.default_rng(3)
    I, K = 1024, 1536
    x, main = ie.activation(rng, K, True, (0,))
    qw, sc = ie.swiglu_weights(rng, I, K, x, main)
    q8, xs, s8 = orc.quantize_q8_1(x)
    ref, ex, _ = orc.gemv_swiglu_w4a8(qw, sc, q8, xs, s8, K, I)
    assert np.array_equal(ref.astype(np.float64), ex)
    assert np.count_nonzero(ex) > I // 4 and np.all(np.abs(ex) < 2048)
