"""ctypes binding of libprana_hip (include/prana_hip.h).

The library is loaded from prana_amd/_build/libprana_hip.so (built in-tree by
prana_amd/build.py). There is no fallback: if the library is missing or no GPU
is visible, calls fail with PranaError.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libprana_hip.so")

c_size = C.c_size_t
c_int = C.c_int
c_void_p = C.c_void_p
c_float = C.c_float
c_u64 = C.c_uint64
c_u32p = C.POINTER(C.c_uint32)
c_u64p = C.POINTER(C.c_uint64)


class PranaConfig(C.Structure):
    """prana_config (checkpoint.rs:32-56)."""

    _fields_ = [
        ("dim", c_size), ("hidden_dim", c_size), ("n_layers", c_size), ("n_heads", c_size),
        ("n_kv_heads", c_size), ("vocab_size", c_size), ("seq_len", c_size), ("head_dim", c_size),
        ("rope_theta", c_float), ("norm_eps", c_float), ("emb_scale", c_float),
        ("rope_neox", c_int), ("act", c_int),
    ]


class GenStats(C.Structure):
    _fields_ = [
        ("prompt_tokens", c_size), ("generated_tokens", c_size), ("proposed", c_size), ("accepted", c_size),
        ("seconds", C.c_double), ("prefill_seconds", C.c_double), ("decode_seconds", C.c_double),
    ]


class PranaError(RuntimeError):
    """A failed call: .code is the library's status (PRANA_ERR_*)."""

    def __init__(self, msg, code=None):
        super().__init__(msg)
        self.code = code


ERR_SHORT_BUFFER = -5


# name -> (restype, argtypes)
_SIGS = {
    "prana_last_error": (C.c_char_p, []),
    "prana_init": (c_int, [c_int]),
    "prana_device_alloc": (c_int, [c_size, C.POINTER(c_void_p)]),
    "prana_device_free": (c_int, [c_void_p]),
    "prana_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size]),
    "prana_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size]),
    "prana_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size]),
    "prana_memset_d": (c_int, [c_void_p, c_int, c_size]),
    "prana_synchronize": (c_int, []),
    "prana_mat_create": (c_int, [c_int, c_size, c_size, c_void_p, c_size, C.POINTER(c_void_p)]),
    "prana_mat_create_q8": (c_int, [c_size, c_size, c_void_p, c_void_p, C.POINTER(c_void_p)]),
    "prana_mat_destroy": (c_int, [c_void_p]),
    "prana_mat_info": (c_int, [c_void_p, C.POINTER(c_size), C.POINTER(c_size), C.POINTER(c_int), C.POINTER(c_size)]),
    "prana_quantize_acts": (c_int, [c_void_p, c_size, c_size, c_void_p, c_void_p, c_void_p, c_void_p]),
    "prana_quantize_q8": (c_int, [c_void_p, c_size, c_size, c_void_p, c_void_p, c_void_p]),
    "prana_matmul": (c_int, [c_void_p, c_void_p, c_size, c_void_p, c_void_p]),
    "prana_matmul_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_void_p, c_void_p]),
    "prana_matmul_block_sums": (c_int, [c_void_p, c_void_p, c_void_p, c_size, c_void_p, c_void_p]),
    "prana_embed_rows": (c_int, [c_void_p, c_void_p, c_size, c_float, c_void_p, c_void_p]),
    "prana_rmsnorm": (c_int, [c_void_p, c_void_p, c_size, c_size, c_float, c_void_p, c_void_p]),
    "prana_silu": (c_int, [c_void_p, c_size, c_void_p]),
    "prana_gelu_tanh": (c_int, [c_void_p, c_size, c_void_p]),
    "prana_silu_mul": (c_int, [c_void_p, c_void_p, c_size, c_void_p]),
    "prana_gelu_tanh_mul": (c_int, [c_void_p, c_void_p, c_size, c_void_p]),
    "prana_add_bias": (c_int, [c_void_p, c_void_p, c_size, c_size, c_void_p]),
    "prana_softmax": (c_int, [c_void_p, c_size, c_size, c_void_p, c_void_p]),
    "prana_rope_interleaved": (c_int, [c_void_p, c_size, c_size, c_size, c_size, c_float, c_void_p]),
    "prana_rope_neox": (c_int, [c_void_p, c_size, c_size, c_size, c_size, c_float, c_void_p]),
    "prana_kv_write_f16": (c_int, [c_void_p, c_size, c_size, c_void_p, c_size, c_void_p]),
    "prana_attention_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_size, c_size, c_size, c_size, c_void_p, c_void_p]),
    "prana_attention_verify": (c_int, [c_void_p, c_void_p, c_void_p, c_size, c_size, c_size, c_size, c_size, c_void_p,
                                       c_void_p]),
    "prana_attention_decode_splitk": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                                              c_size, c_void_p, c_void_p]),
    "prana_attention_decode_splitk_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_size,
                                                      c_size, c_size, c_void_p, c_void_p]),
    "prana_attention_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_size, c_size, c_size, c_size, c_void_p,
                                        c_void_p]),
    "prana_argmax": (c_int, [c_void_p, c_size, c_size, c_void_p, c_void_p]),
    "prana_f32_to_f16": (c_int, [c_void_p, c_size, c_void_p, c_void_p]),
    "prana_f16_to_f32": (c_int, [c_void_p, c_size, c_void_p, c_void_p]),
    "prana_expf": (c_int, [c_void_p, c_size, c_void_p, c_void_p]),
    "prana_tanhf": (c_int, [c_void_p, c_size, c_void_p, c_void_p]),
    "prana_model_create": (c_int, [C.POINTER(PranaConfig), C.POINTER(c_void_p)]),
    "prana_model_destroy": (c_int, [c_void_p]),
    "prana_model_set_tensor": (c_int, [c_void_p, C.c_char_p, c_int, c_u64p, c_int, c_void_p, c_size]),
    "prana_model_finalize": (c_int, [c_void_p]),
    "prana_model_stream_bytes": (c_int, [c_void_p, C.POINTER(c_size)]),
    "prana_cache_create": (c_int, [c_void_p, c_size, C.POINTER(c_void_p)]),
    "prana_cache_destroy": (c_int, [c_void_p]),
    "prana_cache_read": (c_int, [c_void_p, c_size, c_int, c_size, c_void_p]),
    "prana_forward": (c_int, [c_void_p, c_void_p, C.c_uint32, c_size, c_int, c_void_p]),
    "prana_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_size]),
    "prana_forward_batch": (c_int, [c_void_p, c_void_p, c_void_p, c_size, c_size, c_void_p]),
    "prana_decode": (c_int, [c_void_p, c_void_p, C.c_uint32, c_size, c_size, c_void_p]),
    "prana_decode_replay_enabled": (c_int, []),
    "prana_gemv_profile": (c_int, [c_int]),
    "prana_gemv_profile_read": (c_int, [C.POINTER(c_size), C.POINTER(C.c_double), C.POINTER(C.c_double), c_int]),
    "prana_gemv_profile_shapes": (c_int, [c_size, C.POINTER(c_size), C.POINTER(c_size), C.POINTER(C.c_double),
                                          C.POINTER(c_size)]),
    "prana_generate": (c_int, [c_void_p, c_void_p, c_size, c_size, c_void_p, c_size, c_void_p, C.POINTER(c_size),
                               C.POINTER(GenStats)]),
    "prana_generate_speculative": (c_int, [c_void_p, c_void_p, c_void_p, c_size, c_size, c_size, c_void_p, c_size,
                                           c_void_p, C.POINTER(c_size), C.POINTER(GenStats)]),
    "prana_ggml_nbytes": (c_size, [c_int, c_size]),
    # GGUF (host only, except prana_model_load_gguf)
    "prana_gguf_open": (c_int, [C.c_char_p, C.POINTER(c_void_p)]),
    "prana_gguf_open_bytes": (c_int, [c_void_p, c_size, C.POINTER(c_void_p)]),
    "prana_gguf_close": (c_int, [c_void_p]),
    "prana_gguf_counts": (c_int, [c_void_p, C.POINTER(C.c_uint32), C.POINTER(c_size), C.POINTER(c_size)]),
    "prana_gguf_tensor_name": (c_int, [c_void_p, c_size, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_gguf_tensor_info": (c_int, [c_void_p, C.c_char_p, C.POINTER(c_int), c_u64p, C.POINTER(c_int),
                                       C.POINTER(c_size)]),
    "prana_gguf_tensor_data": (c_int, [c_void_p, C.c_char_p, C.POINTER(c_void_p), C.POINTER(c_size)]),
    "prana_gguf_tensor_f32": (c_int, [c_void_p, C.c_char_p, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_gguf_meta_type": (c_int, [c_void_p, C.c_char_p, C.POINTER(c_int), C.POINTER(c_int)]),
    "prana_gguf_meta_u64": (c_int, [c_void_p, C.c_char_p, c_u64p]),
    "prana_gguf_meta_f32": (c_int, [c_void_p, C.c_char_p, C.POINTER(c_float)]),
    "prana_gguf_meta_str": (c_int, [c_void_p, C.c_char_p, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_gguf_meta_array_len": (c_int, [c_void_p, C.c_char_p, C.POINTER(c_size)]),
    "prana_gguf_meta_array_str": (c_int, [c_void_p, C.c_char_p, c_size, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_gguf_meta_array_f32": (c_int, [c_void_p, C.c_char_p, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_gguf_meta_array_i64": (c_int, [c_void_p, C.c_char_p, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_gguf_model_config": (c_int, [c_void_p, C.POINTER(PranaConfig)]),
    "prana_model_load_gguf": (c_int, [c_void_p, c_int, C.POINTER(c_void_p)]),
    "prana_model_config": (c_int, [c_void_p, C.POINTER(PranaConfig)]),
    # tokenizers
    "prana_tokenizer_from_gguf": (c_int, [c_void_p, C.POINTER(c_void_p)]),
    "prana_tokenizer_from_llama2c": (c_int, [c_void_p, c_size, c_size, C.POINTER(c_void_p)]),
    "prana_tokenizer_destroy": (c_int, [c_void_p]),
    "prana_tokenizer_info": (c_int, [c_void_p, C.POINTER(c_int), C.POINTER(c_size)]),
    "prana_tokenizer_encode": (c_int, [c_void_p, c_void_p, c_size, c_int, c_int, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_tokenizer_encode_prompt": (c_int, [c_void_p, c_void_p, c_size, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_tokenizer_decode": (c_int, [c_void_p, C.c_uint32, C.c_uint32, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_tokenizer_is_stop": (c_int, [c_void_p, C.c_uint32, C.POINTER(c_int)]),
    "prana_tokenizer_stop_ids": (c_int, [c_void_p, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_bpe_pre_tokenize": (c_int, [c_void_p, c_size, c_void_p, c_size, C.POINTER(c_size)]),
    # sampler
    "prana_sampler_create": (c_int, [c_float, c_u64, C.POINTER(c_void_p)]),
    "prana_sampler_destroy": (c_int, [c_void_p]),
    "prana_sampler_state": (c_int, [c_void_p, c_u64p]),
    "prana_sampler_next_f32": (c_int, [c_void_p, C.POINTER(c_float)]),
    "prana_sampler_sample": (c_int, [c_void_p, c_void_p, c_size, C.POINTER(C.c_uint32), c_void_p]),
    "prana_sample_pick": (c_int, [c_void_p, c_size, c_float, c_void_p, c_void_p]),
    "prana_generate_sampled": (c_int, [c_void_p, c_void_p, c_size, c_size, c_void_p, c_size, c_void_p, c_void_p,
                                       C.POINTER(c_size), C.POINTER(GenStats)]),
    # graph
    "prana_graph_create": (c_int, [C.POINTER(c_void_p)]),
    "prana_graph_destroy": (c_int, [c_void_p]),
    "prana_graph_input": (c_int, [c_void_p, c_size, C.POINTER(c_size)]),
    "prana_graph_matmul_f32": (c_int, [c_void_p, c_size, c_void_p, c_size, c_size, C.POINTER(c_size)]),
    "prana_graph_matmul_q8": (c_int, [c_void_p, c_size, c_size, c_size, c_void_p, c_void_p, C.POINTER(c_size)]),
    "prana_graph_rmsnorm": (c_int, [c_void_p, c_size, c_void_p, c_size, c_float, C.POINTER(c_size)]),
    "prana_graph_add": (c_int, [c_void_p, c_size, c_size, C.POINTER(c_size)]),
    "prana_graph_softmax": (c_int, [c_void_p, c_size, C.POINTER(c_size)]),
    "prana_graph_rope": (c_int, [c_void_p, c_size, c_size, c_size, c_float, C.POINTER(c_size)]),
    "prana_graph_attention": (c_int, [c_void_p, c_size, c_size, c_size, c_size, c_size, c_size, C.POINTER(c_size)]),
    "prana_graph_set_input": (c_int, [c_void_p, c_size, c_void_p, C.POINTER(c_size), c_int]),
    "prana_graph_set_input_device": (c_int, [c_void_p, c_size, c_void_p, C.POINTER(c_size), c_int]),
    "prana_graph_execute": (c_int, [c_void_p, C.POINTER(c_int), C.POINTER(c_size)]),
    "prana_graph_reset": (c_int, [c_void_p]),
    "prana_graph_shape": (c_int, [c_void_p, c_size, C.POINTER(c_size), C.POINTER(c_int)]),
    "prana_graph_output_f32": (c_int, [c_void_p, c_size, c_void_p, c_size, C.POINTER(c_size)]),
    "prana_graph_output_device": (c_int, [c_void_p, c_size, C.POINTER(c_void_p), C.POINTER(c_size)]),
}

# libprana_synth.so (prana_amd/synth/prana_synth.h): fixture encoders of the
# tests and the benchmark, host code only, kept out of the product library.
SYNTH_PATH = os.path.join(_HERE, "_build", "libprana_synth.so")
_SYNTH_SIGS = {
    "prana_synth_last_error": (C.c_char_p, []),
    "prana_quantize_tensor": (c_int, [c_int, c_void_p, c_size, c_size, c_void_p, c_size]),
    "prana_synth_normal": (c_int, [c_u64, c_float, c_void_p, c_size]),
    "prana_synth_tensor": (c_int, [c_int, c_size, c_size, c_u64, c_float, c_void_p, c_size]),
}
_synth = None

_lib = None


def load():
    """Load the in-tree library once and bind every symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise PranaError(f"{LIB_PATH} is missing: build it with `python prana_amd/build.py` "
                         "(or __graft_entry__.build())")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols():
    return list(_SIGS)


def load_synth():
    """Load the fixture-encoder library once and bind its symbols."""
    global _synth
    if _synth is not None:
        return _synth
    if not os.path.exists(SYNTH_PATH):
        raise PranaError(f"{SYNTH_PATH} is missing: build it with `python prana_amd/build.py`")
    lib = C.CDLL(SYNTH_PATH)
    for name, (res, args) in _SYNTH_SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _synth = lib
    return lib


def check_synth(rc):
    if rc != 0:
        msg = load_synth().prana_synth_last_error().decode(errors="replace")
        raise PranaError(f"prana_synth error {rc}: {msg}")
    return rc


def check(rc):
    if rc != 0:
        msg = load().prana_last_error().decode(errors="replace")
        raise PranaError(f"prana error {rc}: {msg}", rc)
    return rc
