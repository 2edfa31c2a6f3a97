"""CPU tests of the .qwenbin v2 reader (qe_qwenbin_inspect, include/qwenbin.h):
fields read where the reference's format puts them, and malformed or
unsupported containers rejected on the host with the failing field named.
The containers come from tests/qwenbin_writer.py, an independent writer that
follows the reference exporter's struct formats."""
import os

import pytest

import qwenbin_writer as qw


@pytest.fixture(scope="module")
def qe():
    import qe_amd
    qe_amd.lib()
    return qe_amd


def test_header_and_table_fields(qe, tmp_path):
    m = qw.synth_model(L=3, H=256, I=384, nq=2, nkv=1, V=640, seed=1)
    p = tmp_path / "m.qwenbin"
    meta = qw.write(p, m, max_seq_len=2048, rope_theta=10000.0)
    info = qe.qwenbin_inspect(p)
    assert info["version"] == 2 and info["quant_type"] == 1 and info["tie_word_embeddings"] == 1
    assert (info["num_layers"], info["hidden_size"], info["intermediate_size"]) == (3, 256, 384)
    assert (info["num_q_heads"], info["num_kv_heads"], info["head_dim"], info["vocab_size"]) == (2, 1, 128, 640)
    assert info["max_seq_len"] == 2048 and info["rope_theta"] == 10000.0
    assert abs(info["rms_norm_eps"] - 1e-6) < 1e-12
    assert info["file_size"] == os.path.getsize(p) == meta["size"]
    assert info["weights_offset"] == meta["weights_offset"] == 4096 + ((3 * 216 + 255) // 256) * 256
    assert info["weights_bytes"] == meta["size"] - meta["weights_offset"]
    # untied LM head
    m2 = qw.synth_model(L=1, V=384, seed=2, untied=True)
    p2 = tmp_path / "u.qwenbin"
    qw.write(p2, m2)
    assert qe.qwenbin_inspect(p2)["tie_word_embeddings"] == 0


def _expect_fail(qe, path, code, text):
    import qe_amd
    with pytest.raises(RuntimeError) as ei:
        qe.qwenbin_inspect(path)
    msg = str(ei.value)
    assert text in msg, msg


@pytest.mark.parametrize("case,text", [
    ("magic", "bad magic"),
    ("version1", "version 1"),
    ("fp16", "quant_type 0"),
    ("deltanet", "type 1"),
    ("table", "truncated layer table"),
    ("weights_offset", "weights_offset"),
    ("down_outside", "down_proj"),
    ("gate_up_split", "separately"),
    ("misaligned_q", "not 16-byte aligned"),
    ("no_embed_scales", "embed_tokens"),
    ("head_dim", "dimensions outside"),
    ("eps", "rms_norm_eps"),
])
def test_malformed_containers_rejected(qe, tmp_path, case, text):
    m = qw.synth_model(L=2, seed=3)
    p = tmp_path / f"{case}.qwenbin"

    def mutate(h, d):
        if case == "magic":
            h[0] = 0x12345678
        elif case == "version1":
            h[1] = 1
        elif case == "fp16":
            h[10] = 0
        elif case == "deltanet":
            d[1][0] = 1
        elif case == "table":
            h[16] = 1 << 40
        elif case == "weights_offset":
            h[20] += 8
        elif case == "down_outside":
            d[1][16] = 1 << 40
        elif case == "gate_up_split":
            d[0][15] = d[0][14] + 256
        elif case == "misaligned_q":
            d[0][4] += 4
        elif case == "no_embed_scales":
            h[21] = 0
        elif case == "head_dim":
            h[7] = 64
        elif case == "eps":
            h[12] = 1e-5

    qw.write(p, m, mutate=mutate)
    _expect_fail(qe, p, None, text)


def test_truncated_and_missing_files(qe, tmp_path):
    m = qw.synth_model(L=1, seed=4)
    p = tmp_path / "t.qwenbin"
    meta = qw.write(p, m)
    data = open(p, "rb").read()
    open(p, "wb").write(data[: meta["size"] - 512])  # the last tensor runs past the end
    _expect_fail(qe, p, None, "outside the payload")
    open(p, "wb").write(data[:100])
    _expect_fail(qe, p, None, "too small")
    _expect_fail(qe, tmp_path / "absent.qwenbin", None, "cannot open")


def test_center_nibbles_maps_zero_to_eight_only():
    """The centered test weights: every nibble 0 becomes 8, every other nibble
    is kept, so uniform nibbles get mean exactly 8 (the zero point)."""
    import numpy as np
    import qwenbin_writer as qw
    w = np.random.default_rng(1).integers(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32)
    w[:16] = [0, 0xFFFFFFFF, 0x0F0F0F0F, 0xF0F0F0F0, 0x10000000, 1, 0x88888888, 0x01234567] * 2
    c = qw.center_nibbles(w)
    nib = lambda a: np.stack([(a >> (4 * j)) & 15 for j in range(8)])
    o, n = nib(w), nib(c)
    assert np.array_equal(n, np.where(o == 0, 8, o))
    assert c[0] == 0x88888888 and c[1] == 0xFFFFFFFF and c[2] == 0x8F8F8F8F
    assert abs(n.mean() - 8.0) < 0.02
