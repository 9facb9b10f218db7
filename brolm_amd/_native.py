"""ctypes bindings of the two native libraries (include/brolm_hip.h, include/brolm_c.h).

There is no Python fallback: if the libraries are not built, loading raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIBDIR = Path(__file__).resolve().parent / "lib"

_hip = None
_lib = None

i32, i64, u64, f32, f64 = C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_double
vp, cp = C.c_void_p, C.c_char_p
P_i32 = C.POINTER(C.c_int32)
P_i64 = C.POINTER(C.c_int64)
P_f32 = C.POINTER(C.c_float)
P_u16 = C.POINTER(C.c_uint16)
P_u8 = C.POINTER(C.c_uint8)


class Qwen3ConfigC(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
                                        "num_attention_heads", "num_key_value_heads", "head_dim")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float),
        ("tie_word_embeddings", C.c_int), ("max_position_embeddings", C.c_int)]


class Mistral3TextConfigC(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
                                        "num_attention_heads", "num_key_value_heads", "head_dim")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float)] + [
        (n, C.c_int) for n in ("tie_word_embeddings", "max_position_embeddings", "has_sliding_window",
                               "sliding_window")]


class Mistral3ConfigC(C.Structure):
    _fields_ = [("text", Mistral3TextConfigC)] + [
        (n, C.c_int) for n in ("image_token_index", "spatial_merge_size", "multimodal_projector_bias")]


class Llm2VecConfigC(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
                                        "num_attention_heads", "num_key_value_heads", "head_dim")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float)]


class SynthSpecC(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab", "hidden", "intermediate", "layers", "n_q", "n_kv", "head_dim")] + [
        ("eps", C.c_float), ("theta", C.c_float), ("context", C.c_int), ("tied", C.c_int)] + [
        (n, C.c_int) for n in ("embed_type", "q_type", "k_type", "v_type", "o_type", "gate_type", "up_type",
                               "down_type", "output_type")] + [("stddev", C.c_float), ("seed", C.c_uint64),
                                                                ("more_bits_type", C.c_int)]


class DecodeDimsC(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("hidden", "intermediate", "n_q", "n_kv", "head_dim", "vocab", "cap")] + [
        ("eps", C.c_float)] + [(n, C.c_int) for n in ("qkv_type_q", "qkv_type_k", "qkv_type_v", "o_type",
                                                      "gate_type", "up_type", "down_type", "lm_type",
                                                      "no_qk_norm", "v_alt_type", "down_alt_type")]


# symbol -> (restype, argtypes); every symbol of include/brolm_hip.h
HIP_SYMBOLS = {
    "bx_last_error": (cp, []),
    "bx_abi_version": (C.c_int, []),
    "bx_device_ok": (C.c_int, []),
    "bx_profiler_attached": (C.c_int, []),
    "bx_repack_gguf_rows": (C.c_int, [C.c_int, vp, vp, i64, i64, vp]),
    "bx_unpack_carrier_rows": (C.c_int, [C.c_int, vp, vp, i64, i64, vp]),
    "bx_carrier_bytes": (i64, [C.c_int, i64, i64]),
    "bx_dequant_to_f16": (C.c_int, [C.c_int, vp, vp, i64, i64, vp]),
    "bx_dequant_to_f32": (C.c_int, [C.c_int, vp, vp, i64, i64, vp]),
    "bx_linear_f16": (C.c_int, [C.c_int, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_size_t, vp]),
    "bx_embedding_f16": (C.c_int, [vp, C.c_int, C.c_int, vp, C.c_int, vp, vp]),
    "bx_embedding_f32": (C.c_int, [vp, C.c_int, C.c_int, vp, C.c_int, vp, vp]),
    "bx_rms_norm": (C.c_int, [vp, C.c_int, vp, f32, vp, C.c_int, C.c_int, vp]),
    "bx_rope_f16": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, C.c_int, vp]),
    "bx_rope_table_host": (None, [P_f32, P_f32, C.c_int, C.c_int, f32]),
    "bx_kv_append_f16": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp, C.c_int, vp]),
    "bx_attention_workspace_bytes": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "bx_attention_decode_f16": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, f32, C.c_int,
                                          vp, vp, vp]),
    "bx_attention_gqa_f16": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp,
                                       vp]),
    "bx_sample_workspace_bytes": (C.c_size_t, [C.c_int]),
    "bx_sample_f16": (C.c_int, [vp, C.c_int, C.c_float, C.c_int, C.c_float, C.c_double, vp, vp, vp]),
    "bx_masked_mean_pool_f16": (C.c_int, [vp, vp, C.c_int, C.c_int, vp, vp]),
    "bx_attention_masked_f16": (C.c_int, [vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, vp]),
    "bx_scatter_row": (C.c_int, [vp, vp, vp, i64, C.c_int, vp]),
    "bx_silu_mul_f16": (C.c_int, [vp, vp, i64, vp]),
    "bx_silu_f16": (C.c_int, [vp, vp, i64, vp]),
    "bx_mul_f16": (C.c_int, [vp, vp, i64, vp]),
    "bx_add_inplace": (C.c_int, [vp, C.c_int, vp, i64, vp]),
    "bx_f32_to_f16": (C.c_int, [vp, vp, i64, vp]),
    "bx_decode_ws_bytes": (C.c_size_t, [C.POINTER(DecodeDimsC)]),
    "bx_decode_embed": (C.c_int, [C.POINTER(DecodeDimsC), vp, vp, vp, vp]),
    "bx_decode_layer_run": (C.c_int, [C.POINTER(DecodeDimsC), vp, vp, vp, vp, vp, vp]),
    "bx_decode_head": (C.c_int, [C.POINTER(DecodeDimsC), vp, vp, vp, vp, vp]),
    "bx_decode_advance": (C.c_int, [vp, vp, vp, vp, vp, vp]),
    "bx_persist_ws_bytes": (C.c_size_t, [C.POINTER(DecodeDimsC)]),
    "bx_persist_step": (C.c_int, [C.POINTER(DecodeDimsC), C.c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, C.c_uint32,
                                  vp]),
    "bx_persist_ws_init": (C.c_int, [C.POINTER(DecodeDimsC), vp, vp]),
    "bx_persist_status": (C.c_int, [vp, C.POINTER(C.c_uint32)]),
    "bx_persist_trace": (C.c_int, [vp, C.c_int]),
    "bx_argmax_workspace_bytes": (C.c_size_t, [i64]),
    "bx_argmax_f16": (C.c_int, [vp, i64, vp, vp, vp]),
    "bx_argmax_f16_noalloc": (C.c_int, [vp, i64, vp, vp]),
    "bx_linear_tiles_ok": (C.c_int, [C.c_int, C.c_int]),
    "bx_linear_workspace_bytes": (C.c_size_t, []),
    "bx_linear_workspace_init": (C.c_int, [vp, C.c_size_t, vp]),
    "bx_attention_varlen_f16": (C.c_int, [vp, vp, vp, C.c_int, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp,
                                          vp]),
    "bx_sample_feed_f16": (C.c_int, [vp, C.c_int, C.c_float, C.c_int, C.c_float, vp, vp, vp, vp, vp, vp]),
    "bx_rope_rows_f16": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp, vp, C.c_int, vp]),
    "bx_kv_append_rows_f16": (C.c_int, [vp, vp, C.c_int, C.c_int, vp, vp, vp, i64, vp]),
    "bx_linear_ss_floats": (C.c_size_t, [C.c_int]),
    "bx_linear_residual_ss_f16": (C.c_int, [C.c_int, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_size_t, vp]),
    "bx_linear_group_norm_f16": (C.c_int, [C.c_int, C.c_int, vp, vp, vp, vp, vp, C.c_float, vp, C.c_int, C.c_int,
                                           vp, C.c_size_t, vp]),
    "bx_linear_swiglu_norm_f16": (C.c_int, [C.c_int, vp, vp, vp, vp, C.c_float, vp, vp, C.c_int, C.c_int, C.c_int,
                                            vp, C.c_size_t, vp]),
    "bx_linear_group2_f16": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, vp, vp, C.c_int, C.c_int, vp, C.c_size_t, vp]),
    "bx_linear_group2_norm_f16": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, vp, vp, vp, C.c_float, vp,
                                            C.c_int, C.c_int, vp, C.c_size_t, vp]),
    "bx_batch_attention_workspace_bytes": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "bx_batch_attention_f16": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, C.c_float, vp, vp,
                                         C.c_int, vp, vp, C.c_int, vp, vp, i64, vp, vp, vp]),
    "bx_qk_rope_kv_rows_f16": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, C.c_float, vp, vp,
                                         vp, C.c_int, vp, vp, vp, i64, vp, vp]),
    "bx_linear_group_f16": (C.c_int, [C.c_int, C.c_int, C.POINTER(vp), C.POINTER(vp), C.POINTER(C.c_int), vp, C.c_int,
                                      C.c_int, vp, C.c_size_t, vp]),
    "bx_linear_residual_f16": (C.c_int, [C.c_int, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_size_t, vp]),
    "bx_linear_swiglu_f16": (C.c_int, [C.c_int, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_size_t, vp]),
}

# every symbol of include/brolm_c.h
C_SYMBOLS = {
    "brolm_last_error": (cp, []),
    "brolm_init": (C.c_int, []),
    "brolm_shutdown": (C.c_int, []),
    "brolm_synth_qwen3_write": (C.c_int, [C.POINTER(SynthSpecC), cp]),
    "brolm_synth_normal_bf16": (C.c_int, [u64, i64, f32, P_f32]),
    "brolm_synth_tensor_key": (u64, [u64, cp]),
    "brolm_synth_quantize": (C.c_int, [C.c_int, P_f32, i64, P_u8]),
    "brolm_qwen3_hf_to_ggml": (C.c_int, [cp, C.c_char_p, C.c_int]),
    "brolm_qwen3_config_from_gguf": (C.c_int, [cp, C.POINTER(Qwen3ConfigC)]),
    "brolm_gguf_tensor_count": (C.c_int, [cp, P_i64]),
    "brolm_gguf_tensor_info": (C.c_int, [cp, cp, C.POINTER(C.c_int), P_i64, C.POINTER(C.c_int), P_i64]),
    "brolm_qwen3_create": (vp, [C.POINTER(Qwen3ConfigC)]),
    "brolm_mistral3_config_from_gguf": (C.c_int, [cp, C.POINTER(Mistral3ConfigC)]),
    "brolm_mistral3_config_from_json": (C.c_int, [cp, C.POINTER(Mistral3ConfigC)]),
    "brolm_mistral3_hf_to_ggml": (C.c_int, [cp, C.c_char_p, C.c_int]),
    "brolm_synth_mistral3_write": (C.c_int, [C.POINTER(SynthSpecC), cp]),
    "brolm_mistral3_text_create": (vp, [C.POINTER(Mistral3TextConfigC)]),
    "brolm_llm2vec_config_from_json": (C.c_int, [cp, C.POINTER(Llm2VecConfigC)]),
    "brolm_llm2vec_create": (vp, [C.POINTER(Llm2VecConfigC)]),
    "brolm_decoder_forward_encode": (C.c_int, [vp, P_i32, C.c_int, P_f32]),
    "brolm_llm2vec_encode_pooled": (C.c_int, [vp, P_i32, C.c_int, P_f32, P_f32]),
    "brolm_qwen3_free": (None, [vp]),
    "brolm_qwen3_load_gguf": (C.c_int, [vp, cp]),
    "brolm_qwen3_allocate_cache": (C.c_int, [vp, C.c_int]),
    "brolm_qwen3_reset_cache": (C.c_int, [vp]),
    "brolm_qwen3_truncate_cache": (C.c_int, [vp, C.c_int]),
    "brolm_qwen3_cache_len": (C.c_int, [vp]),
    "brolm_qwen3_forward": (C.c_int, [vp, P_i32, C.c_int, P_f32, P_f32]),
    "brolm_qwen3_forward_last": (C.c_int, [vp, P_i32, C.c_int, P_f32]),
    "brolm_qwen3_decode_sampled": (C.c_int, [vp, C.c_int32, C.c_int, vp, C.c_float, C.c_int, C.c_float, P_i32,
                                             C.c_int]),
    "brolm_qwen3_allocate_batch": (C.c_int, [vp, C.c_int, C.c_int]),
    "brolm_qwen3_slot_len": (C.c_int, [vp, C.c_int]),
    "brolm_qwen3_truncate_slot": (C.c_int, [vp, C.c_int, C.c_int]),
    "brolm_qwen3_prefill_slot": (C.c_int, [vp, C.c_int, P_i32, C.c_int, P_f32]),
    "brolm_qwen3_forward_batch": (C.c_int, [vp, P_i32, P_i32, C.c_int, P_f32]),
    "brolm_qwen3_time_forward_batch": (C.c_double, [vp, P_i32, P_i32, C.c_int, C.c_int]),
    "brolm_qwen3_embed_tokens": (C.c_int, [vp, P_i32, C.c_int, P_u16]),
    "brolm_qwen3_forward_embeds": (C.c_int, [vp, P_u16, C.c_int, P_f32, P_f32]),
    "brolm_qwen3_generate": (C.c_int, [vp, P_i32, C.c_int, C.c_int, C.c_int, C.c_int, f32, C.c_int, f32, u64,
                                       C.c_int, C.c_int, P_i32]),
    "brolm_qwen3_decode_greedy": (C.c_int, [vp, i32, C.c_int, P_i32, C.c_int]),
    "brolm_qwen3_time_decode_steps": (f64, [vp, i32, C.c_int]),
    "brolm_qwen3_decode_weight_bytes": (i64, [vp]),
    "brolm_qwen3_decode_mode": (C.c_int, [vp]),
    "brolm_sample_token_device": (C.c_int, [vp, C.c_int, C.c_float, C.c_int, C.c_float, u64]),
    "brolm_sample_token": (C.c_int, [P_f32, C.c_int, f32, C.c_int, f32, u64]),
    "brolm_prompt_ids": (C.c_int, [u64, C.c_int, C.c_int, P_i32]),
    "brolm_tokenizer_load": (vp, [cp, cp, cp]),
    "brolm_tokenizer_from_gguf": (vp, [cp, cp]),
    "brolm_tokenizer_from_json": (vp, [cp, cp]),
    "brolm_tokenizer_free": (None, [vp]),
    "brolm_tokenizer_encode": (C.c_int, [vp, cp, i64, C.c_int, P_i32, C.c_int]),
    "brolm_tokenizer_decode": (i64, [vp, P_i32, C.c_int, C.c_char_p, i64]),
    "brolm_tokenizer_chat": (i64, [vp, C.POINTER(cp), C.POINTER(cp), C.c_int, C.c_int, C.c_char_p, i64]),
    "brolm_tokenizer_register_special": (C.c_int, [vp, cp, i32]),
    "brolm_tokenizer_info": (C.c_int, [vp, P_i64]),
    "brolm_qwen3_generate_text": (i64, [vp, vp, cp, C.c_int, C.c_int, f32, C.c_int, f32, u64, C.c_char_p, i64]),
    "brolm_profile_reset": (None, []),
    "brolm_profile_report": (None, []),
    "brolm_profile_enabled": (C.c_int, []),
    "brolm_gguf_tensor_data": (i64, [cp, cp, P_u8, i64]),
    "brolm_gguf_meta_int": (C.c_int, [cp, cp, C.POINTER(i64)]),
    "brolm_gguf_meta_f64": (C.c_int, [cp, cp, C.POINTER(f64)]),
    "brolm_gguf_meta_str": (i64, [cp, cp, C.c_char_p, i64]),
    "brolm_gguf_meta_array": (C.c_int, [cp, cp, C.POINTER(C.c_int), C.POINTER(i64)]),
    "brolm_gguf_parse_memory": (C.c_int, [P_u8, i64, C.POINTER(i64)]),
    "brolm_profile_stage": (C.c_int, [C.c_int, C.POINTER(u64), C.POINTER(u64)]),
}


def _bind(lib, table):
    for name, (res, args) in table.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def hip():
    """libbrolm_hip.so (kernels)."""
    global _hip
    if _hip is None:
        path = LIBDIR / "libbrolm_hip.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built; run `python -m brolm_amd.build`")
        lib = C.CDLL(str(path), mode=C.RTLD_GLOBAL)
        _bind(lib, HIP_SYMBOLS)
        _hip = lib
    return _hip


def lib():
    """libbrolm.so (C++ host stack)."""
    global _lib
    if _lib is None:
        hip()
        path = LIBDIR / "libbrolm.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built; run `python -m brolm_amd.build`")
        l = C.CDLL(str(path), mode=C.RTLD_GLOBAL)
        _bind(l, C_SYMBOLS)
        _lib = l
    return _lib


class NativeError(RuntimeError):
    pass


def check(rc: int, what: str = "") -> int:
    """Raise with the C++ message when a brolm_* call returned -1."""
    if rc < 0:
        raise NativeError(f"{what}: {lib().brolm_last_error().decode()}")
    return rc


def bx_check(rc: int, what: str = "") -> int:
    if rc != 0:
        raise NativeError(f"{what}: {hip().bx_last_error().decode()} (code {rc})")
    return rc
