"""ctypes binding of libqasr_hip.so (the C ABI declared in include/qasr_hip.h).

The library is built in-tree by ``__graft_entry__.build()``.  Loading fails
loudly when it is missing: there is no CPU fallback for anything in this
package.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqasr_hip.so")
SYNTH_PATH = os.path.join(_HERE, "libqasr_synth.so")

QASR_OK = 0
QASR_ERR_INVALID = -1
QASR_ERR_HIP = -2
QASR_ERR_NOMEM = -3
QASR_ROUND_HALF_AWAY = 0
QASR_TRUNC = 1

P = C.c_void_p
I64 = C.c_int64
I32 = C.c_int32
F32 = C.c_float


class QasrError(RuntimeError):
    """A qasr_hip call returned a non-zero status."""

    def __init__(self, code, msg):
        super().__init__(f"qasr_hip error {code}: {msg}")
        self.code = code


class DecConfig(C.Structure):
    _fields_ = [("n_layers", I32), ("hidden", I32), ("n_heads", I32), ("n_kv_heads", I32),
                ("head_dim", I32), ("intermediate", I32), ("vocab", I32),
                ("eps", F32), ("theta", F32)]


class DecLayer(C.Structure):
    _fields_ = [(n, P) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down",
                                  "q_norm", "k_norm", "input_norm", "post_attn_norm")]


class DecWeights(C.Structure):
    _fields_ = [("embed", P), ("norm", P), ("layers", C.POINTER(DecLayer))]


class EncConfig(C.Structure):
    _fields_ = [(n, I32) for n in ("d_model", "n_layers", "n_heads", "head_dim", "ffn_dim",
                                    "output_dim", "chunk_size", "n_window_infer", "conv_hidden")]


class EncLayer(C.Structure):
    _fields_ = [(n, P) for n in ("wq", "wk", "wv", "wo", "fc1", "fc2", "bq", "bk", "bv", "bo",
                                  "b1", "b2", "ln1_w", "ln1_b", "ln2_w", "ln2_b")]


class EncWeights(C.Structure):
    _fields_ = ([(n, P) for n in ("conv1_w", "conv2_w", "conv3_w", "conv_out_w",
                                   "conv1_b", "conv2_b", "conv3_b")]
                + [("layers", C.POINTER(EncLayer))]
                + [(n, P) for n in ("ln_post_w", "ln_post_b", "proj1_w", "proj2_w",
                                     "proj1_b", "proj2_b")])


class Prompt(C.Structure):
    _fields_ = [("prompt", P), ("n_prompt", I64), ("force", P), ("n_force", I64)]


class StreamConfig(C.Structure):
    _fields_ = [("chunk_sec", C.c_float), ("rollback", C.c_int32), ("unfixed_chunks", C.c_int32),
                ("max_new_tokens", C.c_int32), ("past_text_conditioning", C.c_int32),
                ("stop_tokens", C.c_int32 * 2)]


# name -> (restype, argtypes); every function returning int is status-checked
_SIGS = {
    "qasr_hip_create": (C.c_int, [C.c_int, C.POINTER(P)]),
    "qasr_hip_destroy": (None, [P]),
    "qasr_hip_last_error": (C.c_char_p, []),
    "qasr_hip_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "qasr_hip_synchronize": (C.c_int, [P]),
    "qasr_hip_stream": (P, [P]),
    "qasr_hip_malloc": (C.c_int, [P, C.c_size_t, C.POINTER(P)]),
    "qasr_hip_free": (C.c_int, [P, P]),
    "qasr_hip_upload": (C.c_int, [P, P, P, C.c_size_t]),
    "qasr_hip_download": (C.c_int, [P, P, P, C.c_size_t]),
    "qasr_hip_memset": (C.c_int, [P, P, C.c_int, C.c_size_t]),
    "qasr_hip_copy": (C.c_int, [P, P, P, C.c_size_t]),
    "qasr_hip_timer_start": (C.c_int, [P]),
    "qasr_hip_timer_stop": (C.c_int, [P, C.POINTER(F32)]),
    "qasr_hip_timer_hold": (C.c_int, [P, C.c_int]),
    "qasr_hip_pack_int8_rows": (C.c_int, [P, P, I64, I64, C.c_int, P, P]),
    "qasr_hip_quantize_act": (C.c_int, [P, P, I64, P, P]),
    "qasr_hip_linear_int8": (C.c_int, [P, P, P, P, P, P, I64, I64]),
    "qasr_hip_linear_int8_qkv": (C.c_int, [P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64]),
    "qasr_hip_linear_int8_swiglu": (C.c_int, [P, P, P, P, P, I64, I64]),
    "qasr_hip_linear_int8_addto": (C.c_int, [P, P, P, P, P, I64, I64]),
    "qasr_hip_argmax_int8": (C.c_int, [P, P, P, P, I64, I64, P]),
    "qasr_hip_rmsnorm_linear_int8_qkv": (C.c_int, [P, P, P, P, P, P, F32, P, P, P, P, P, P,
                                                   I64, I64, I64]),
    "qasr_hip_rmsnorm_linear_int8_swiglu": (C.c_int, [P, P, P, P, F32, P, P, I64, I64]),
    "qasr_hip_rmsnorm_argmax_int8": (C.c_int, [P, P, P, F32, P, P, I64, I64, P]),
    "qasr_hip_argmax_int8_noalloc": (C.c_int, [P, P, P, F32, P, P, I64, I64, P]),
    "qasr_hip_rms_norm": (C.c_int, [P, P, P, P, I64, I64, F32]),
    "qasr_hip_rms_norm_per_head": (C.c_int, [P, P, P, I64, I64, I64, F32]),
    "qasr_hip_apply_rope_neox": (C.c_int, [P, P, P, P, I64, I64, I64]),
    "qasr_hip_causal_attention": (C.c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, I64, F32,
                                            I64]),
    "qasr_hip_causal_attention_bf16kv": (C.c_int, [P, P, P, P, P, I64, I64, I64, I64, I64, F32, I64]),
    "qasr_hip_decoder_load": (C.c_int, [P, C.POINTER(DecConfig), C.POINTER(DecWeights), C.c_int,
                                        I64, C.c_int, C.POINTER(P)]),
    "qasr_hip_decoder_load_st": (C.c_int, [P, P, C.POINTER(DecConfig), C.c_int, I64, C.c_int, C.POINTER(P)]),
    "qasr_hip_decoder_free": (None, [P]),
    "qasr_hip_st_open": (C.c_int, [C.c_char_p, C.POINTER(P)]),
    "qasr_hip_st_open_file": (C.c_int, [C.c_char_p, C.POINTER(P)]),
    "qasr_hip_st_free": (None, [P]),
    "qasr_hip_st_count": (I64, [P]),
    "qasr_hip_st_shards": (I64, [P]),
    "qasr_hip_st_name": (C.c_char_p, [P, I64]),
    "qasr_hip_st_find": (C.c_int, [P, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(I64),
                                   C.POINTER(P), C.POINTER(I64)]),
    "qasr_hip_decoder_prefill": (C.c_int, [P, P, I64]),
    "qasr_hip_decoder_forward": (C.c_int, [P, P, I32, C.POINTER(I32)]),
    "qasr_hip_decoder_generate": (C.c_int, [P, P, I32, I32, P]),
    "qasr_hip_decoder_last_logit": (C.c_int, [P, P]),
    "qasr_hip_decoder_capacity": (I64, [P]),
    "qasr_hip_decoder_set_stamps": (C.c_int, [P, P, I64]),
    "qasr_hip_decoder_kv_upload_rows": (C.c_int, [P, I64, I64, P, P]),
    "qasr_hip_decoder_kv_download_rows": (C.c_int, [P, I64, I64, P, P]),
    "qasr_hip_decoder_set_len": (C.c_int, [P, I64]),
    "qasr_hip_decoder_len": (I64, [P]),
    "qasr_hip_decoder_packed": (C.c_int, [P, C.c_int, C.c_int, P, P]),
    "qasr_hip_decoder_kv_upload": (C.c_int, [P, P, P]),
    "qasr_hip_decoder_kv_download": (C.c_int, [P, P, P]),
    "qasr_hip_decoder_set_options": (C.c_int, [P, C.c_int, C.c_int]),
    "qasr_hip_decoder_set_fusion": (C.c_int, [P, C.c_int]),
    "qasr_hip_decoder_profile": (C.c_int, [P, I32, P, P, P]),
    "qasr_hip_linear_bf16w": (C.c_int, [P, P, P, P, P, I64, I64, I64, C.c_int]),
    "qasr_hip_gemm_w8_bf16": (C.c_int, [P, P, P, P, P, I64, I64, I64]),
    "qasr_hip_layer_norm": (C.c_int, [P, P, P, P, P, I64, I64, F32]),
    "qasr_hip_bidirectional_attention": (C.c_int, [P, P, P, P, P, I64, I64, I64, F32, I64]),
    "qasr_hip_encoder_load": (C.c_int, [P, C.POINTER(EncConfig), C.POINTER(EncWeights), C.POINTER(P)]),
    "qasr_hip_encoder_load_st": (C.c_int, [P, P, C.POINTER(EncConfig), C.POINTER(P)]),
    "qasr_hip_encoder_free": (None, [P]),
    "qasr_hip_encoder_tokens": (I64, [P, I64]),
    "qasr_hip_mel": (C.c_int, [P, P, I64, P, C.POINTER(I64)]),
    "qasr_hip_encoder_forward": (C.c_int, [P, P, I64, P, C.POINTER(I64)]),
    "qasr_hip_transcribe_forced": (C.c_int, [P, P, P, I64, I32, P, P]),
    "qasr_hip_transcribe": (C.c_int, [P, P, P, I64, I32, P, C.POINTER(I64), P]),
    "qasr_hip_text_tokens": (I64, [P, I64, P]),
    "qasr_hip_encoder_forward_batch": (C.c_int, [P, I32, P, P, P, P]),
    "qasr_hip_transcribe_prompt": (C.c_int, [P, P, P, I64, C.POINTER(Prompt), P, I64, I32, P, C.POINTER(I64), P]),
    "qasr_hip_text_tokens_from": (I64, [P, I64, C.c_int, P]),
    "qasr_hip_segment_splits": (I64, [P, I64, C.c_float, C.c_float, P, I64]),
    "qasr_hip_engine_last_segments": (C.c_int, [P, P, I64, C.POINTER(I64)]),
    "qasr_hip_engine_set_segment_sec": (None, [P, C.c_float]),
    "qasr_hip_engine_set_search_sec": (None, [P, C.c_float]),
    "qasr_hip_engine_set_language_tokens": (C.c_int, [P, P, I64]),
    "qasr_hip_engine_set_prompt_tokens": (C.c_int, [P, P, I64]),
    "qasr_hip_stream_set_prompt": (C.c_int, [P, C.POINTER(Prompt)]),
    "qasr_hip_engine_detect": (C.c_int, [P, C.POINTER(DecConfig), C.POINTER(EncConfig)]),
    "qasr_hip_engine_load": (C.c_int, [C.c_char_p, C.c_int, I64, C.POINTER(P)]),
    "qasr_hip_engine_free": (None, [P]),
    "qasr_hip_engine_config": (C.c_int, [P, C.POINTER(DecConfig), C.POINTER(EncConfig)]),
    "qasr_hip_engine_transcribe_pcm": (C.c_int, [P, P, I64, P, I64, C.POINTER(I64)]),
    "qasr_hip_engine_last_raw_tokens": (C.c_int, [P, P, I64, C.POINTER(I64)]),
    "qasr_hip_engine_stream_new": (C.c_int, [P, C.POINTER(P)]),
    "qasr_hip_engine_stream_free": (None, [P]),
    "qasr_hip_engine_stream_reset": (C.c_int, [P]),
    "qasr_hip_engine_stream_push": (C.c_int, [P, P, I64, C.c_int, P, I64, C.POINTER(I64)]),
    "qasr_hip_engine_stream_get_result": (C.c_int, [P, P, I64, C.POINTER(I64)]),
    "qasr_hip_engine_stream_set_chunk_sec": (None, [P, C.c_float]),
    "qasr_hip_engine_stream_set_rollback": (None, [P, I32]),
    "qasr_hip_engine_stream_set_unfixed_chunks": (None, [P, I32]),
    "qasr_hip_engine_stream_set_max_new_tokens": (None, [P, I32]),
    "qasr_hip_stream_default_config": (None, [C.POINTER(StreamConfig)]),
    "qasr_hip_stream_create": (C.c_int, [P, P, C.POINTER(StreamConfig), C.POINTER(P)]),
    "qasr_hip_stream_free": (None, [P]),
    "qasr_hip_stream_reset": (C.c_int, [P]),
    "qasr_hip_stream_push": (C.c_int, [P, P, I64, C.c_int, P, I64, C.POINTER(I64)]),
    "qasr_hip_stream_tokens": (C.c_int, [P, P, I64, C.POINTER(I64)]),
    "qasr_hip_stream_audio_cursor": (I64, [P]),
    "qasr_hip_stream_stats": (C.c_int, [P, P]),
    "qasr_hip_stream_batch_create": (C.c_int, [P, P, C.POINTER(StreamConfig), I32, I64, C.POINTER(P)]),
    "qasr_hip_stream_batch_free": (None, [P]),
    "qasr_hip_stream_batch_stream": (P, [P, I32]),
    "qasr_hip_stream_batch_times": (C.c_int, [P, P]),
    "qasr_hip_stream_batch_push": (C.c_int, [P, P, P, P, P, I64, P]),
    "qasr_hip_decoder_set_lm_head": (C.c_int, [P, P, I64]),
    "qasr_hip_decoder_logits_dim": (I64, [P]),
    "qasr_hip_decoder_head_rows": (I64, [P]),
    "qasr_hip_decoder_prefill_logits": (C.c_int, [P, P, I64, P]),
    "qasr_hip_decoder_prefill_argmax": (C.c_int, [P, P, I64, P, I64, P]),
    "qasr_hip_argmax_f32_rows": (C.c_int, [P, P, I64, I64, I64, P]),
    "qasr_hip_batch_create": (C.c_int, [P, I32, I64, I64, C.POINTER(P)]),
    "qasr_hip_batch_free": (None, [P]),
    "qasr_hip_batch_prefill": (C.c_int, [P, I32, P, I64]),
    "qasr_hip_batch_set_len": (C.c_int, [P, I32, I64]),
    "qasr_hip_batch_len": (I64, [P, I32]),
    "qasr_hip_batch_set_options": (C.c_int, [P, C.c_int, C.c_int]),
    "qasr_hip_batch_generate": (C.c_int, [P, P, I32, P]),
    "qasr_hip_batch_profile": (C.c_int, [P, P, I32, P, P]),
}

_lib = None


def lib():
    """Load libqasr_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first "
                               "(the HIP library is required; there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def declared_symbols():
    return sorted(_SIGS)


def check(rc):
    if rc != QASR_OK:
        msg = lib().qasr_hip_last_error()
        raise QasrError(rc, msg.decode() if msg else "")
    return rc
