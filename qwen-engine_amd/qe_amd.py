"""Python binding of libqe_amd.so (the C-ABI in include/qe_kernels.h).

The library is the product: this module only loads it with ctypes and
passes device pointers of torch tensors (torch provides HBM allocations and
streams).  There is no fallback: if the library is missing, `lib()` raises.

Function names mirror the reference's launchers (include/kernels.cuh) with
the same argument order; a non-zero status raises RuntimeError carrying
qe_last_error(), as the reference's CUDA_KERNEL_CHECK throws
std::runtime_error (include/tensor.cuh:11-23).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqe_amd.so")

_P = ctypes.c_void_p
_I = ctypes.c_int

# (name, argtypes) of every entry point declared in include/qe_kernels.h
SIGNATURES = {
    "qe_launch_quantize_fp16_to_q8_1": [_P, _P, _P, _P, _I, _P],
    "qe_launch_rmsnorm_q8_1": [_P, _P, _P, _P, _P, _P, _P, _I],
    "qe_launch_rmsnorm_fp16": [_P, _P, _P, _I, _P, _I],
    "qe_launch_gemv_w4a8": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _P],
    "qe_launch_gemv_qkv_w4a8": [_P, _P, _P, _P, _P, _I, _I, _I, _I],
    "qe_launch_gemv_dual_gate_up_swiglu_w4a8": [_P, _P, _P, _P, _P, _P, _I, _I, _P],
    "qe_launch_gemv_w4a16": [_P, _P, _P, _P, _P, _I, _I, _P],
    "qe_launch_gemv_dual_gate_up_swiglu_w4a16": [_P, _P, _P, _P, _I, _I, _P],
    "qe_launch_gemm_prefill_w4a16": [_P, _P, _P, _P, _P, _I, _I, _I, _P, _I],
    "qe_launch_gemm_prefill_w4a16_noalloc": [_P, _P, _P, _P, _P, _I, _I, _I, _P, _I],
    "qe_launch_gemm_prefill_w4a16_tiled": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "qe_launch_gemm_prefill_qkv_w4a16_tiled": [_P, _P, _I, _P, _I, _I, _I, _I],
    "qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled": [_P, _P, _P, _P, _I, _P, _I, _I],
    "qe_launch_gemm_prefill_qkv_w4a16": [_P, _P, _I, _P, _I, _I, _I, _I, _I],
    "qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16": [_P, _P, _P, _P, _I, _P, _I, _I],
    "qe_launch_sample_and_advance": [_P, _P, _P, _P, _P, _P, _I],
    "qe_launch_gemm_prefill_w4a8": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "qe_launch_gemm_prefill_qkv_w4a8": [_P, _P, _P, _P, _I, _P, _I, _I, _I, _I],
    "qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a8": [_P, _P, _P, _P, _P, _P, _I, _P, _I, _I],
    "qe_launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                                        _I, _I, ctypes.c_float],
    "qe_launch_gemv_lm_head_sample_w4a8": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P],
    "qe_launch_rmsnorm_gemv_lm_head_sample_w4a16": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P],
    "qe_launch_rmsnorm_gemv_qkv_w4a16": [_P, _P, _P, _P, _P, _I, _I, _I, _I],
    "qe_launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16": [_P, _P, _P, _P, _P, _P, _I, _I, _P],
    "qe_launch_embed_lookup_w4a16": [_P, _P, _P, _P, _P, _I, _P, _I],
    "qe_launch_qkv_bias_rope_kv_append": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I,
                                          ctypes.c_float],
    "qe_launch_attention_gqa_flash_decode": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P],
    "qe_launch_attention_gqa_flash_decode_combine": [_P, _P, _P, _P, _I, _P, _P, _P],
    "qe_launch_attention_gqa_flash_decode_partials": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I],
    "qe_launch_attention_combine_gemv_o_w4a8": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "qe_launch_attention_gqa_prefill": [_P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I],
}

OTHER_SIGNATURES = {
    "qe_stream_read": [_P, ctypes.c_size_t, _P, _P],
    "qe_set_tuning": [ctypes.c_char_p, _I],
    "qe_gemm_reserve_workspace": [_P],
    "qe_gemm_attach_workspace": [_P, _P, ctypes.c_size_t],
    "qe_gemm_release_workspace": [_P],
    "qe_w4_tiled_bytes": [_I, _I, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
    "qe_repack_w4_tiled": [_P, _P, _I, _I, _P, _P, _P],
    "qe_gemm_prefill_plan": [_I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)],
}

ENGINE_SIGNATURES = {
    "qe_engine_create": [_P, ctypes.c_uint64, _P],
    "qe_engine_reset": [_P],
    "qe_engine_prefill": [_P, _P, _I, _P],
    "qe_engine_decode": [_P, _I, _I, _P, _P],
    "qe_engine_profile_decode": [_P, _P],
    "qe_engine_seq_pos": [_P],
    "qe_engine_read_logits": [_P, _P, _I],
    "qe_engine_read_hidden": [_P, _P, _I],
    "qe_engine_read_buffer": [_P, ctypes.c_char_p, _P, ctypes.c_size_t],
    "qe_engine_arena_spans": [_P, _P, _P, _I, _P, _P],
    "qe_engine_create_from_qwenbin": [ctypes.c_char_p, _I, _I, _I, _P],
    "qe_engine_save_qwenbin": [_P, ctypes.c_char_p],
    "qe_qwenbin_inspect": [ctypes.c_char_p, _P],
}

_lib = None


class QKVView(ctypes.Structure):
    """qe_qkv_view / QKVProjectionView (include/kernels.cuh:23-27)."""
    _fields_ = [(n, _P) for n in ("q_weight", "q_scale", "d_q", "k_weight", "k_scale", "d_k",
                                   "v_weight", "v_scale", "d_v")]


def build(jobs: int = 8) -> str:
    """Compile libqe_amd.so in-tree for gfx950 (hipcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE, f"-j{jobs}"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libqe_amd.so not built at {LIB_PATH}; run __graft_entry__.build()")
        # torch bundles its own libamdhip64 (same SONAME, libamdhip64.so.7).
        # Loading torch first makes libqe_amd bind to that runtime, so the
        # process has one HIP runtime and torch's streams/pointers are valid here.
        import torch  # noqa: F401
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        for name, args in list(ENGINE_SIGNATURES.items()) + list(OTHER_SIGNATURES.items()):
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        for name in ("qe_engine_logits", "qe_engine_hidden"):
            getattr(L, name).argtypes = [_P]
            getattr(L, name).restype = ctypes.c_void_p
        L.qe_engine_destroy.argtypes = [_P]
        L.qe_engine_destroy.restype = None
        L.qe_engine_default_config.argtypes = [_P]
        L.qe_engine_default_config.restype = None
        L.qe_gemm_workspace_allocations.argtypes = []
        L.qe_gemm_workspace_allocations.restype = ctypes.c_long
        L.qe_last_error.restype = ctypes.c_char_p
        L.qe_version.restype = ctypes.c_char_p
        _lib = L
    return _lib


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _check(rc: int, name: str):
    if rc != 0:
        msg = lib().qe_last_error().decode()
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def _call(name, *args):
    _check(getattr(lib(), name)(*args), name)


# ---- launchers (reference names, tensor arguments) ---------------------------
def launch_quantize_fp16_to_q8_1(input_x, out_q8, out_scale, out_sum8, num_elements, stream=None):
    _call("qe_launch_quantize_fp16_to_q8_1", _ptr(input_x), _ptr(out_q8), _ptr(out_scale), _ptr(out_sum8),
          num_elements, _stream(stream))


def launch_rmsnorm_q8_1(input, gamma, output_fp16_opt, out_q8, out_scale, out_sum8, stream=None,
                        hidden_size=1536):
    _call("qe_launch_rmsnorm_q8_1", _ptr(input), _ptr(gamma), _ptr(output_fp16_opt), _ptr(out_q8),
          _ptr(out_scale), _ptr(out_sum8), _stream(stream), hidden_size)


def launch_rmsnorm_fp16(input, gamma, output, num_tokens, stream=None, hidden_size=1536):
    _call("qe_launch_rmsnorm_fp16", _ptr(input), _ptr(gamma), _ptr(output), num_tokens, _stream(stream),
          hidden_size)


def launch_gemv_w4a8(qweight, scales, input_q8, input_scale, input_sum8, residual, output_y,
                     out_features, in_features, stream=None):
    _call("qe_launch_gemv_w4a8", _ptr(qweight), _ptr(scales), _ptr(input_q8), _ptr(input_scale),
          _ptr(input_sum8), _ptr(residual), _ptr(output_y), out_features, in_features, _stream(stream))


def make_qkv_view(q_weight, q_scale, d_q, k_weight, k_scale, d_k, v_weight, v_scale, d_v) -> QKVView:
    return QKVView(*[_ptr(t) for t in (q_weight, q_scale, d_q, k_weight, k_scale, d_k, v_weight, v_scale, d_v)])


def launch_gemv_qkv_w4a8(view: QKVView, input_q8, input_scale, input_sum8, stream=None, in_features=1536,
                         num_q_heads=12, num_kv_heads=2, head_dim=128):
    _call("qe_launch_gemv_qkv_w4a8", ctypes.addressof(view), _ptr(input_q8), _ptr(input_scale),
          _ptr(input_sum8), _stream(stream), in_features, num_q_heads, num_kv_heads, head_dim)


def launch_gemv_dual_gate_up_swiglu_w4a8(gate_up_qweight, gate_up_scales, input_q8, input_scale, input_sum8,
                                         output_mlp, hidden_size, intermediate_size, stream=None):
    _call("qe_launch_gemv_dual_gate_up_swiglu_w4a8", _ptr(gate_up_qweight), _ptr(gate_up_scales),
          _ptr(input_q8), _ptr(input_scale), _ptr(input_sum8), _ptr(output_mlp), hidden_size,
          intermediate_size, _stream(stream))


def launch_gemv_w4a16(qweight, scales, input_x, residual, output_y, out_features, in_features, stream=None):
    _call("qe_launch_gemv_w4a16", _ptr(qweight), _ptr(scales), _ptr(input_x), _ptr(residual), _ptr(output_y),
          out_features, in_features, _stream(stream))


def launch_gemv_dual_gate_up_swiglu_w4a16(gate_up_qweight, gate_up_scales, input_x, output_mlp, hidden_size,
                                          intermediate_size, stream=None):
    _call("qe_launch_gemv_dual_gate_up_swiglu_w4a16", _ptr(gate_up_qweight), _ptr(gate_up_scales),
          _ptr(input_x), _ptr(output_mlp), hidden_size, intermediate_size, _stream(stream))


def launch_gemm_prefill_w4a16(qweight, scales, input_x, residual, output_y, M, N, K, stream=None, sm_count=0):
    _call("qe_launch_gemm_prefill_w4a16", _ptr(qweight), _ptr(scales), _ptr(input_x), _ptr(residual),
          _ptr(output_y), M, N, K, _stream(stream), sm_count)


def launch_gemm_prefill_w4a16_noalloc(qweight, scales, input_x, residual, output_y, M, N, K, stream=None,
                                      sm_count=0):
    _call("qe_launch_gemm_prefill_w4a16_noalloc", _ptr(qweight), _ptr(scales), _ptr(input_x), _ptr(residual),
          _ptr(output_y), M, N, K, _stream(stream), sm_count)


def w4_tiled(qweight, scales, N, K, stream=None):
    """Tiled copy (qe_repack_w4_tiled) of an N x K packed matrix: (weights int32, scales fp16) tensors."""
    import torch
    wb, sb = ctypes.c_size_t(), ctypes.c_size_t()
    _check(lib().qe_w4_tiled_bytes(N, K, ctypes.byref(wb), ctypes.byref(sb)), "qe_w4_tiled_bytes")
    w = torch.empty(wb.value // 4, dtype=torch.int32, device=qweight.device)
    s = torch.empty(sb.value // 2, dtype=torch.float16, device=qweight.device)
    _check(lib().qe_repack_w4_tiled(_ptr(qweight), _ptr(scales), N, K, _ptr(w), _ptr(s), _stream(stream)),
           "qe_repack_w4_tiled")
    return w, s


def launch_gemm_prefill_w4a16_tiled(tiled_weight, tiled_scales, input_x, residual, output_y, M, N, K, stream=None):
    _call("qe_launch_gemm_prefill_w4a16_tiled", _ptr(tiled_weight), _ptr(tiled_scales), _ptr(input_x),
          _ptr(residual), _ptr(output_y), M, N, K, _stream(stream))


def launch_gemm_prefill_qkv_w4a16_tiled(view: QKVView, input_x, M, stream=None, in_features=1536, num_q_heads=12,
                                        num_kv_heads=2, head_dim=128):
    _call("qe_launch_gemm_prefill_qkv_w4a16_tiled", ctypes.addressof(view), _ptr(input_x), M, _stream(stream),
          in_features, num_q_heads, num_kv_heads, head_dim)


def launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled(tiled_weight, tiled_scales, input_x, output_mlp, M,
                                                        stream=None, hidden_size=1536, intermediate_size=8960):
    _call("qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled", _ptr(tiled_weight), _ptr(tiled_scales),
          _ptr(input_x), _ptr(output_mlp), M, _stream(stream), hidden_size, intermediate_size)


def launch_gemm_prefill_qkv_w4a16(view: QKVView, input_x, M, stream=None, in_features=1536, num_q_heads=12,
                                  num_kv_heads=2, head_dim=128, sm_count=0):
    _call("qe_launch_gemm_prefill_qkv_w4a16", ctypes.addressof(view), _ptr(input_x), M, _stream(stream),
          in_features, num_q_heads, num_kv_heads, head_dim, sm_count)


def launch_gemm_prefill_dual_gate_up_swiglu_w4a16(gate_up_qweight, gate_up_scales, input_x, output_mlp, M,
                                                  stream=None, hidden_size=1536, intermediate_size=8960):
    _call("qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16", _ptr(gate_up_qweight), _ptr(gate_up_scales),
          _ptr(input_x), _ptr(output_mlp), M, _stream(stream), hidden_size, intermediate_size)


def launch_sample_and_advance(logits, sample_scratch_val, sample_scratch_idx, d_control, d_mapped_pinned_token,
                              stream=None, vocab_size=151936):
    _call("qe_launch_sample_and_advance", _ptr(logits), _ptr(sample_scratch_val), _ptr(sample_scratch_idx),
          _ptr(d_control), _ptr(d_mapped_pinned_token), _stream(stream), vocab_size)


LM_HEAD_SAMPLE_PARTS = 2048  # QE_LM_HEAD_SAMPLE_PARTS


def launch_gemm_prefill_w4a8(qweight, scales, input_q8, input_scale, input_sum8, residual, output_y, M, N, K,
                             stream=None):
    _call("qe_launch_gemm_prefill_w4a8", _ptr(qweight), _ptr(scales), _ptr(input_q8), _ptr(input_scale),
          _ptr(input_sum8), _ptr(residual), _ptr(output_y), M, N, K, _stream(stream))


def launch_gemm_prefill_qkv_w4a8(view: QKVView, input_q8, input_scale, input_sum8, M, stream=None, in_features=1536,
                                 num_q_heads=12, num_kv_heads=2, head_dim=128):
    _call("qe_launch_gemm_prefill_qkv_w4a8", ctypes.addressof(view), _ptr(input_q8), _ptr(input_scale),
          _ptr(input_sum8), M, _stream(stream), in_features, num_q_heads, num_kv_heads, head_dim)


def launch_gemm_prefill_dual_gate_up_swiglu_w4a8(gate_up_qweight, gate_up_scales, input_q8, input_scale,
                                                 input_sum8, output_mlp, M, stream=None, hidden_size=1536,
                                                 intermediate_size=8960):
    _call("qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a8", _ptr(gate_up_qweight), _ptr(gate_up_scales),
          _ptr(input_q8), _ptr(input_scale), _ptr(input_sum8), _ptr(output_mlp), M, _stream(stream), hidden_size,
          intermediate_size)


def launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16(input, gamma, output_fp16_opt, view: QKVView, q_bias, k_bias,
                                                 v_bias, layer_k_cache, layer_v_cache, d_control, stream=None,
                                                 hidden_size=1536, num_q_heads=12, num_kv_heads=2, head_dim=128,
                                                 max_seq_len=4096, rotary_dim=128, rope_theta=1000000.0):
    _call("qe_launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16", _ptr(input), _ptr(gamma), _ptr(output_fp16_opt),
          ctypes.addressof(view), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(layer_k_cache),
          _ptr(layer_v_cache), _ptr(d_control), _stream(stream), hidden_size, num_q_heads, num_kv_heads, head_dim,
          max_seq_len, rotary_dim, rope_theta)


# ---- fused decode entry points (no counterpart in the reference API) ---------
def launch_gemv_lm_head_sample_w4a8(qweight, scales, input_q8, input_scale, input_sum8, logits_opt,
                                    sample_scratch_val, sample_scratch_idx, d_control, d_mapped_pinned_token,
                                    vocab_size=151936, in_features=1536, stream=None):
    _call("qe_launch_gemv_lm_head_sample_w4a8", _ptr(qweight), _ptr(scales), _ptr(input_q8), _ptr(input_scale),
          _ptr(input_sum8), _ptr(logits_opt), _ptr(sample_scratch_val), _ptr(sample_scratch_idx), _ptr(d_control),
          _ptr(d_mapped_pinned_token), vocab_size, in_features, _stream(stream))


def launch_rmsnorm_gemv_lm_head_sample_w4a16(input, gamma, output_fp16_opt, qweight, scales, logits_opt,
                                             sample_scratch_val, sample_scratch_idx, d_control,
                                             d_mapped_pinned_token, vocab_size=151936, hidden_size=1536,
                                             stream=None):
    _call("qe_launch_rmsnorm_gemv_lm_head_sample_w4a16", _ptr(input), _ptr(gamma), _ptr(output_fp16_opt),
          _ptr(qweight), _ptr(scales), _ptr(logits_opt), _ptr(sample_scratch_val), _ptr(sample_scratch_idx),
          _ptr(d_control), _ptr(d_mapped_pinned_token), vocab_size, hidden_size, _stream(stream))


def launch_rmsnorm_gemv_qkv_w4a16(input, gamma, output_fp16_opt, view: QKVView, stream=None, hidden_size=1536,
                                  num_q_heads=12, num_kv_heads=2, head_dim=128):
    _call("qe_launch_rmsnorm_gemv_qkv_w4a16", _ptr(input), _ptr(gamma), _ptr(output_fp16_opt),
          ctypes.addressof(view), _stream(stream), hidden_size, num_q_heads, num_kv_heads, head_dim)


def launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(input, gamma, output_fp16_opt, gate_up_qweight, gate_up_scales,
                                                  output_mlp, hidden_size, intermediate_size, stream=None):
    _call("qe_launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16", _ptr(input), _ptr(gamma), _ptr(output_fp16_opt),
          _ptr(gate_up_qweight), _ptr(gate_up_scales), _ptr(output_mlp), hidden_size, intermediate_size,
          _stream(stream))


# ---- decode-loop kernels ---------------------------------------------------------
def launch_embed_lookup_w4a16(embed_qweight, embed_scales, d_token_ids, out_hidden, d_control, num_tokens,
                              stream=None, hidden_size=1536):
    _call("qe_launch_embed_lookup_w4a16", _ptr(embed_qweight), _ptr(embed_scales), _ptr(d_token_ids),
          _ptr(out_hidden), _ptr(d_control), num_tokens, _stream(stream), hidden_size)


def launch_qkv_bias_rope_kv_append(q, k, v, q_bias, k_bias, v_bias, layer_k_cache, layer_v_cache, d_control,
                                   num_tokens, stream=None, num_q_heads=12, num_kv_heads=2, head_dim=128,
                                   max_seq_len=4096, rotary_dim=0, rope_theta=1000000.0):
    _call("qe_launch_qkv_bias_rope_kv_append", _ptr(q), _ptr(k), _ptr(v), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias),
          _ptr(layer_k_cache), _ptr(layer_v_cache), _ptr(d_control), num_tokens, _stream(stream), num_q_heads,
          num_kv_heads, head_dim, max_seq_len, rotary_dim, rope_theta)


def launch_attention_gqa_flash_decode(q, layer_k_cache, layer_v_cache, splitk_partial_out, splitk_partial_lse,
                                      attn_out, d_control, stream=None, num_q_heads=12, num_kv_heads=2, head_dim=128,
                                      max_seq_len=4096, out_q8=None, out_scale=None, out_sum8=None):
    _call("qe_launch_attention_gqa_flash_decode", _ptr(q), _ptr(layer_k_cache), _ptr(layer_v_cache),
          _ptr(splitk_partial_out), _ptr(splitk_partial_lse), _ptr(attn_out), _ptr(d_control), _stream(stream),
          num_q_heads, num_kv_heads, head_dim, max_seq_len, _ptr(out_q8), _ptr(out_scale), _ptr(out_sum8))


def launch_attention_gqa_flash_decode_combine(splitk_partial_out, splitk_partial_lse, attn_out, num_q_heads,
                                              out_q8=None, out_scale=None, out_sum8=None, stream=None):
    _call("qe_launch_attention_gqa_flash_decode_combine", _ptr(splitk_partial_out), _ptr(splitk_partial_lse),
          _ptr(attn_out), _stream(stream), num_q_heads, _ptr(out_q8), _ptr(out_scale), _ptr(out_sum8))


def launch_attention_gqa_flash_decode_partials(q, layer_k_cache, layer_v_cache, splitk_partial_out,
                                               splitk_partial_lse, d_control, stream=None, num_q_heads=12,
                                               num_kv_heads=2, head_dim=128, max_seq_len=4096):
    _call("qe_launch_attention_gqa_flash_decode_partials", _ptr(q), _ptr(layer_k_cache), _ptr(layer_v_cache),
          _ptr(splitk_partial_out), _ptr(splitk_partial_lse), _ptr(d_control), _stream(stream), num_q_heads,
          num_kv_heads, head_dim, max_seq_len)


def launch_attention_combine_gemv_o_w4a8(splitk_partial_out, splitk_partial_lse, o_qweight, o_scales, residual,
                                         output_y, attn_out=None, d_control=None, out_features=1536, num_q_heads=12,
                                         head_dim=128, max_seq_len=4096, stream=None):
    _call("qe_launch_attention_combine_gemv_o_w4a8", _ptr(splitk_partial_out), _ptr(splitk_partial_lse),
          _ptr(o_qweight), _ptr(o_scales), _ptr(residual), _ptr(output_y), _ptr(attn_out), _ptr(d_control),
          out_features, num_q_heads, head_dim, max_seq_len, _stream(stream))


def launch_attention_gqa_prefill(q, layer_k_cache, layer_v_cache, attn_out, d_control, num_tokens, stream=None,
                                 num_q_heads=12, num_kv_heads=2, head_dim=128, max_seq_len=4096, hidden_size=1536):
    _call("qe_launch_attention_gqa_prefill", _ptr(q), _ptr(layer_k_cache), _ptr(layer_v_cache), _ptr(attn_out),
          _ptr(d_control), num_tokens, _stream(stream), num_q_heads, num_kv_heads, head_dim, max_seq_len,
          hidden_size)


# ---- engine ------------------------------------------------------------------------
class EngineConfig(ctypes.Structure):
    """qe_engine_config (include/qe_engine.h)."""
    _fields_ = [("num_layers", _I), ("hidden_size", _I), ("intermediate_size", _I), ("num_q_heads", _I),
                ("num_kv_heads", _I), ("head_dim", _I), ("vocab_size", _I), ("max_seq_len", _I),
                ("rope_theta", ctypes.c_float), ("prefill_chunk", _I), ("fused_decode", _I)]


def default_config() -> EngineConfig:
    c = EngineConfig()
    lib().qe_engine_default_config(ctypes.byref(c))
    return c


class QwenbinInfo(ctypes.Structure):
    """qe_qwenbin_info (include/qwenbin.h)."""
    _fields_ = [("version", ctypes.c_uint32), ("quant_type", ctypes.c_uint32),
                ("tie_word_embeddings", ctypes.c_uint32), ("hidden_size", _I), ("intermediate_size", _I),
                ("num_layers", _I), ("num_q_heads", _I), ("num_kv_heads", _I), ("head_dim", _I),
                ("vocab_size", _I), ("max_seq_len", _I), ("rms_norm_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("file_size", ctypes.c_uint64), ("weights_offset", ctypes.c_uint64),
                ("weights_bytes", ctypes.c_uint64)]


def qwenbin_inspect(path: str) -> dict:
    """qe_qwenbin_inspect: validate a .qwenbin v2 file (no GPU); raises RuntimeError on a bad file."""
    info = QwenbinInfo()
    _check(lib().qe_qwenbin_inspect(str(path).encode(), ctypes.byref(info)), "qe_qwenbin_inspect")
    return {n: getattr(info, n) for n, _ in QwenbinInfo._fields_}


class Engine:
    """Qwen2.5-style decode engine (include/qe_engine.h): random-init, or
    Engine.from_qwenbin(path) for a .qwenbin v2 file."""

    def __init__(self, cfg: EngineConfig | None = None, seed: int = 42, _handle=None):
        if _handle is not None:
            self._h = _handle
            self.cfg = EngineConfig()
            return
        self.cfg = cfg if cfg is not None else default_config()
        h = ctypes.c_void_p()
        _check(lib().qe_engine_create(ctypes.byref(self.cfg), seed, ctypes.byref(h)), "qe_engine_create")
        self._h = h

    @classmethod
    def from_qwenbin(cls, path: str, max_seq_len: int = 0, prefill_chunk: int = 0, fused_decode: int = 1):
        h = ctypes.c_void_p()
        _check(lib().qe_engine_create_from_qwenbin(str(path).encode(), max_seq_len, prefill_chunk, fused_decode,
                                                   ctypes.byref(h)), "qe_engine_create_from_qwenbin")
        e = cls(_handle=h)
        info = qwenbin_inspect(path)
        c = e.cfg
        for n in ("num_layers", "hidden_size", "intermediate_size", "num_q_heads", "num_kv_heads", "head_dim",
                  "vocab_size"):
            setattr(c, n, info[n])
        c.rope_theta = info["rope_theta"]
        fs = info["max_seq_len"] if 0 < info["max_seq_len"] <= 32768 else 4096
        c.max_seq_len = min(max_seq_len, fs) if max_seq_len > 0 else fs
        c.prefill_chunk = prefill_chunk if prefill_chunk > 0 else 1024
        c.fused_decode = fused_decode
        return e

    def save_qwenbin(self, path: str):
        _check(lib().qe_engine_save_qwenbin(self._h, str(path).encode()), "qe_engine_save_qwenbin")

    def close(self):
        if getattr(self, "_h", None):
            lib().qe_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        _check(lib().qe_engine_reset(self._h), "qe_engine_reset")

    def prefill(self, tokens) -> int:
        arr = (ctypes.c_int32 * len(tokens))(*tokens)
        out = ctypes.c_int32()
        _check(lib().qe_engine_prefill(self._h, arr, len(tokens), ctypes.byref(out)), "qe_engine_prefill")
        return out.value

    def decode(self, n: int, use_graph: bool = True, timed: bool = False):
        toks = (ctypes.c_int32 * max(n, 1))()
        ms = (ctypes.c_float * max(n, 1))() if timed else None
        _check(lib().qe_engine_decode(self._h, n, int(use_graph), toks, ms), "qe_engine_decode")
        return (list(toks)[:n], list(ms)[:n]) if timed else list(toks)[:n]

    def profile_decode(self):
        st = (ctypes.c_float * 4)()
        _check(lib().qe_engine_profile_decode(self._h, st), "qe_engine_profile_decode")
        return {"gemv_ms": st[0], "attention_ms": st[1], "other_ms": st[2], "total_ms": st[3]}

    def logits(self):
        """Copy of the last logits (numpy float16)."""
        import numpy as np
        out = np.empty(self.cfg.vocab_size, np.float16)
        _check(lib().qe_engine_read_logits(self._h, out.ctypes.data, out.size), "qe_engine_read_logits")
        return out

    def hidden_row0(self):
        import numpy as np
        out = np.empty(self.cfg.hidden_size, np.float16)
        _check(lib().qe_engine_read_hidden(self._h, out.ctypes.data, out.size), "qe_engine_read_hidden")
        return out

    def arena_spans(self):
        """[(offset, bytes)] of every buffer in the engine's arena, in allocation
        order, and the arena's size (qe_engine_arena_spans)."""
        n, total = ctypes.c_int(), ctypes.c_size_t()
        _check(lib().qe_engine_arena_spans(self._h, None, None, 0, ctypes.byref(n), ctypes.byref(total)),
               "qe_engine_arena_spans")
        offs, sizes = (ctypes.c_size_t * max(n.value, 1))(), (ctypes.c_size_t * max(n.value, 1))()
        _check(lib().qe_engine_arena_spans(self._h, offs, sizes, n.value, ctypes.byref(n), None),
               "qe_engine_arena_spans")
        return list(zip(offs[:n.value], sizes[:n.value])), total.value

    def read(self, name: str, dtype, count: int):
        """Copy of the first `count` elements of a named engine buffer."""
        import numpy as np
        out = np.empty(count, dtype)
        _check(lib().qe_engine_read_buffer(self._h, name.encode(), out.ctypes.data, out.nbytes),
               "qe_engine_read_buffer")
        return out

    @property
    def seq_pos(self) -> int:
        return lib().qe_engine_seq_pos(self._h)


def stream_read(data, nbytes: int, sink, stream=None):
    """Streaming-read kernel (qe_stream_read): bandwidth ceiling / counter calibration."""
    _call("qe_stream_read", _ptr(data), nbytes, _ptr(sink), _stream(stream))


def gemm_reserve_workspace(stream=None):
    """qe_gemm_reserve_workspace: a 32 MiB split-K workspace for the stream
    (the only allocation of the kernel API; prefill GEMMs on a stream
    without one run without K slices)."""
    _check(lib().qe_gemm_reserve_workspace(_stream(stream)), "qe_gemm_reserve_workspace")


def gemm_attach_workspace(buf, nbytes: int, stream=None):
    """qe_gemm_attach_workspace: caller memory as the stream's workspace."""
    _check(lib().qe_gemm_attach_workspace(_stream(stream), _ptr(buf), nbytes), "qe_gemm_attach_workspace")


def gemm_release_workspace(stream=None):
    _check(lib().qe_gemm_release_workspace(_stream(stream)), "qe_gemm_release_workspace")


def gemm_workspace_allocations() -> int:
    """hipMalloc calls made so far for GEMM workspaces (test hook)."""
    return int(lib().qe_gemm_workspace_allocations())


def gemm_prefill_plan(M, N, K, tiled=False):
    """(tile, slices) a prefill GEMM of this shape would use (qe_gemm_prefill_plan)."""
    t, sl = ctypes.c_int(), ctypes.c_int()
    _check(lib().qe_gemm_prefill_plan(M, N, K, int(tiled), ctypes.byref(t), ctypes.byref(sl)), "qe_gemm_prefill_plan")
    return t.value, sl.value


def set_tuning(key: str, value: int):
    """qe_set_tuning: process-wide switches ("gemm_split_k")."""
    _call("qe_set_tuning", key.encode(), int(value))
