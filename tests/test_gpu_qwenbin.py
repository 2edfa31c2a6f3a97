"""GPU tests of the .qwenbin v2 loader (qe_engine_create_from_qwenbin, the
counterpart of QwenEngine::load_model_file + setup_arena,
src/engine.cu:85-348): every tensor lands where the container's offsets say,
an engine saved and reloaded decodes the same tokens with bit-identical
logits, and an untied LM head is used."""
import numpy as np
import pytest

import qwenbin_writer as qw

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qe():
    import qe_amd
    qe_amd.lib()
    return qe_amd


def _check_tensors(e, m):
    d = m["dims"]
    assert np.array_equal(e.read("embed_w", np.uint32, m["embed"][0].size), m["embed"][0].reshape(-1))
    assert np.array_equal(e.read("embed_s", np.uint16, m["embed"][1].size), m["embed"][1].view(np.uint16).reshape(-1))
    assert np.array_equal(e.read("final_norm", np.uint16, d["H"]), m["final_norm"].view(np.uint16))
    for l, t in enumerate(m["layers"]):
        for name, arr in (("ln1", t["ln1"]), ("ln2", t["ln2"]), ("q_w", t["q"][0]), ("q_s", t["q"][1]),
                          ("k_w", t["k"][0]), ("k_s", t["k"][1]), ("v_w", t["v"][0]), ("v_s", t["v"][1]),
                          ("o_w", t["o"][0]), ("o_s", t["o"][1]), ("gate_up_w", t["gu"][0]),
                          ("gate_up_s", t["gu"][1]), ("down_w", t["dn"][0]), ("down_s", t["dn"][1]),
                          ("q_bias", t["q_b"]), ("k_bias", t["k_b"]), ("v_bias", t["v_b"])):
            flat = arr.reshape(-1)
            dt = np.uint32 if flat.dtype == np.uint32 else np.uint16
            got = e.read(f"layer{l}.{name}", dt, flat.size)
            assert np.array_equal(got, flat.view(dt)), f"layer {l} {name}"


def test_loader_places_every_tensor(qe, tmp_path):
    m = qw.synth_model(L=2, H=256, I=256, nq=2, nkv=1, V=512, seed=5)
    p = tmp_path / "small.qwenbin"
    qw.write(p, m, max_seq_len=512)
    e = qe.Engine.from_qwenbin(p, prefill_chunk=64)
    _check_tensors(e, m)
    # the LM head is the embedding (tied)
    assert np.array_equal(e.read("lm_head_w", np.uint32, 64), m["embed"][0].reshape(-1)[:64])
    tok = e.prefill([3, 1, 4, 1, 5, 9, 2, 6])
    toks = e.decode(8)
    assert all(0 <= t < 512 for t in [tok] + toks)
    assert np.isfinite(e.logits().astype(np.float32)).all()
    assert e.seq_pos == 16
    e.close()


def test_untied_lm_head(qe, tmp_path):
    m = qw.synth_model(L=1, H=256, I=256, nq=2, nkv=1, V=384, seed=6, untied=True)
    p = tmp_path / "untied.qwenbin"
    qw.write(p, m)
    e = qe.Engine.from_qwenbin(p, max_seq_len=128, prefill_chunk=32)
    assert np.array_equal(e.read("lm_head_w", np.uint32, m["lm_head"][0].size), m["lm_head"][0].reshape(-1))
    assert np.array_equal(e.read("lm_head_s", np.uint16, m["lm_head"][1].size),
                          m["lm_head"][1].view(np.uint16).reshape(-1))
    assert not np.array_equal(e.read("lm_head_w", np.uint32, 64), e.read("embed_w", np.uint32, 64))
    e.prefill([7, 8, 9])
    e.decode(3)
    e.close()


def test_save_and_reload_round_trip(qe, tmp_path):
    """A random engine written as .qwenbin (the exporter's layout) and loaded
    back decodes the same greedy tokens with bit-identical logits."""
    c = qe.default_config()
    c.num_layers, c.intermediate_size, c.vocab_size, c.max_seq_len, c.prefill_chunk = 2, 512, 4096, 256, 64
    prompt = [(i % 1000) + 100 for i in range(40)]
    e1 = qe.Engine(c, seed=11)
    p = tmp_path / "rt.qwenbin"
    e1.save_qwenbin(p)
    info = qe.qwenbin_inspect(p)
    assert (info["num_layers"], info["hidden_size"], info["intermediate_size"], info["vocab_size"]) == (2, 1536, 512,
                                                                                                       4096)
    assert info["max_seq_len"] == 256 and info["tie_word_embeddings"] == 1
    t1 = e1.prefill(prompt)
    g1 = e1.decode(10)
    l1 = e1.logits()
    e2 = qe.Engine.from_qwenbin(p, prefill_chunk=64)
    assert e2.prefill(prompt) == t1
    assert e2.decode(10) == g1
    assert np.array_equal(e2.logits().view(np.uint16), l1.view(np.uint16))
    for e in (e1, e2):
        e.close()
