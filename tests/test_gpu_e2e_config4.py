"""configs[4] at full size: the 28-layer, 151936-vocab Qwen2.5-1.5B
architecture (random-init, W4A16 G128 everywhere), prompts of 128 ids -
seeded uniform ids in [0, 151936) as configs[4] states, and the reference
bench's synthetic ids ((i % 1000) + 100, src/cli_bench.cpp:78-82) - then
greedy decode of the configured 256 tokens (positions 128..383, so
flash-decode runs with up to 6 splits inside the engine).

Checks, on every decoded step:
  * the residual row stays finite;
  * the fused graph engine's residual row, logits and token equal the
    reference launch sequence's (eager) bit for bit;
and on every 32nd step and the last:
  * the final RMSNorm's Q8_1 (read from the engine with the reference launch
    sequence, which the fused engine matches bit for bit) is within one unit
    of the oracle's Q8_1 of the oracle RMSNorm of the engine's residual row
    (the two sum the squares in different orders);
  * the LM-head logits match the oracle GEMV over that Q8_1 to the path's
    tolerance, and the token is the lowest-index argmax of the logits;
Finally graph and eager decode of the fused engine give the same 256 tokens
(src/engine.cu:453-470 and tests/test_kernels.cu:635-684, the reference's
graph-vs-stream check).
"""
import numpy as np
import pytest

from helpers import assert_fp16_close

pytestmark = pytest.mark.gpu

STEPS = 256
CHECK_EVERY = 32


@pytest.fixture(scope="module")
def qe():
    import qe_amd
    qe_amd.lib()
    return qe_amd


def _run_decode(orc, fused, ref_eng, prompt, H, V):
    """Prefill + STEPS greedy tokens on both engines with the per-step checks
    of the module docstring; returns the graph tokens."""
    lm_w = fused.read("lm_head_w", np.uint32, V * H // 8).reshape(V, H // 8)
    lm_s = fused.read("lm_head_s", np.float16, V * H // 128).reshape(V, H // 128)
    fnorm = fused.read("final_norm", np.float16, H)
    t0 = fused.prefill(prompt)
    assert ref_eng.prefill(prompt) == t0
    graph_toks = []
    for step in range(STEPS):
        tok = fused.decode(1, use_graph=True)[0]
        tok_ref = ref_eng.decode(1, use_graph=False)[0]
        graph_toks.append(tok)
        hid = fused.hidden_row0()
        lg = fused.logits()
        assert np.all(np.isfinite(hid.astype(np.float32))), f"step {step}: residual not finite"
        assert np.array_equal(hid.view(np.uint16), ref_eng.hidden_row0().view(np.uint16)), step
        assert np.array_equal(lg.view(np.uint16), ref_eng.logits().view(np.uint16)), step
        assert tok == tok_ref
        assert tok == orc.argmax_f16(lg), step
        if step % CHECK_EVERY and step != STEPS - 1:
            continue
        q8 = ref_eng.read("q8", np.int8, H)
        xs = ref_eng.read("q8_scale", np.float32, H // 128)
        s8 = ref_eng.read("q8_sum8", np.int32, H // 8)
        rq, rs, rs8 = orc.quantize_q8_1(orc.rmsnorm_fp16(hid, fnorm))
        assert np.abs(q8.astype(np.int32) - rq.astype(np.int32)).max() <= 1, step
        assert np.array_equal(s8, -8 * q8.astype(np.int64).reshape(-1, 8).sum(1)), step
        ref, ex, bd = orc.gemv_w4a8(lm_w, lm_s, q8, xs, s8, V, H)
        assert_fp16_close(lg, ex, bd, ref, what=f"configs[4] LM head step {step}")
        print(f"step {step}: token {tok} max|h| {np.abs(hid.astype(np.float32)).max():.2f}", flush=True)
    fused.reset()
    assert fused.prefill(prompt) == t0
    assert fused.decode(STEPS, use_graph=False) == graph_toks
    return [t0] + graph_toks


@pytest.mark.parametrize("prompt_kind", ["uniform", "cli_bench"])
def test_config4_full_size_decode(qe, orc, prompt_kind):
    c = qe.default_config()
    assert (c.num_layers, c.hidden_size, c.intermediate_size, c.num_q_heads, c.num_kv_heads, c.head_dim,
            c.vocab_size, c.max_seq_len) == (28, 1536, 8960, 12, 2, 128, 151936, 4096)
    H, V = c.hidden_size, c.vocab_size
    if prompt_kind == "uniform":
        prompt = np.random.default_rng(4).integers(0, V, 128).tolist()
    else:
        prompt = [(i % 1000) + 100 for i in range(128)]
    print(f"configs[4] engines ({prompt_kind} prompt): fused graph, reference launch sequence", flush=True)
    fused = qe.Engine(qe.default_config(), seed=42)
    cu = qe.default_config()
    cu.fused_decode = 0
    ref_eng = qe.Engine(cu, seed=42)
    _run_decode(orc, fused, ref_eng, prompt, H, V)
    fused.close()
    ref_eng.close()


def test_config4_centered_weights_varied_trajectory(qe, orc, tmp_path):
    """configs[4] at full size from a .qwenbin whose layer weights have nibble
    mean 8 (no common-mode term, tests/qwenbin_writer.center_nibbles), loaded
    through qe_engine_create_from_qwenbin: the same per-step checks on a
    trajectory that is not one repeated token (greedy decode of a random model
    still settles into a short cycle: 5 distinct tokens), so the check covers attention
    over a changing context and the sampling of varying rows."""
    import qwenbin_writer as qw
    H, I, V = 1536, 8960, 151936
    print("writing a full-size centered .qwenbin", flush=True)
    m = qw.synth_model(L=28, H=H, I=I, nq=12, nkv=2, V=V, seed=5, centered=True)
    path = tmp_path / "centered.qwenbin"
    qw.write(path, m, max_seq_len=4096)
    del m
    fused = qe.Engine.from_qwenbin(str(path), prefill_chunk=1024, fused_decode=1)
    ref_eng = qe.Engine.from_qwenbin(str(path), prefill_chunk=1024, fused_decode=0)
    prompt = np.random.default_rng(6).integers(0, V, 128).tolist()
    toks = _run_decode(orc, fused, ref_eng, prompt, H, V)
    fused.close()
    ref_eng.close()
    distinct = len(set(toks))
    print(f"centered model: {distinct} distinct tokens of {len(toks)}", flush=True)
    assert distinct >= 4, toks  # seeded and deterministic: 5 distinct tokens
