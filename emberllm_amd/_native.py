"""ctypes prototypes of libember.so (include/ember.h, include/ehip.h,
include/ember_synth.h).

The library is built in-tree (``emberllm_amd/libember.so``) by the package
Makefile.  Loading fails loudly when it is missing: there is no fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("EMBER_LIB") or os.path.join(HERE, "libember.so")

DT_F32, DT_Q8_0, DT_Q4_0, DT_F16 = 0, 1, 2, 3
FLAG_TIED_EMBED, FLAG_QK_NORM, FLAG_THINKING = 1, 2, 4
ROPE_INTERLEAVED, ROPE_NEOX = 0, 1


class EmberHeader(ctypes.Structure):
    """Mirror of the packed 256-byte EmberHeader (src/ember.h:54-83)."""

    _pack_ = 1
    _fields_ = [
        ("magic", ctypes.c_char * 4), ("version", ctypes.c_uint32),
        ("header_bytes", ctypes.c_uint64),
        ("dim", ctypes.c_int32), ("hidden_dim", ctypes.c_int32),
        ("n_layers", ctypes.c_int32), ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32), ("max_seq_len", ctypes.c_int32),
        ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float),
        ("flags", ctypes.c_uint32), ("rope_style", ctypes.c_int32),
        ("bos_token_id", ctypes.c_int32), ("eos_token_id", ctypes.c_int32),
        ("eos_token_id2", ctypes.c_int32), ("n_tensors", ctypes.c_int32),
        ("tokenizer_type", ctypes.c_int32), ("default_top_k", ctypes.c_int32),
        ("default_temp", ctypes.c_float), ("default_top_p", ctypes.c_float),
        ("tokenizer_offset", ctypes.c_uint64), ("tokenizer_size", ctypes.c_uint64),
        ("tensor_table_offset", ctypes.c_uint64), ("tensor_table_size", ctypes.c_uint64),
        ("reserved", ctypes.c_uint8 * 128),
    ]


class EmberTensor(ctypes.Structure):
    """Mirror of the packed 88-byte EmberTensor (src/ember.h:85-92)."""

    _pack_ = 1
    _fields_ = [
        ("name", ctypes.c_char * 48), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int32 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64),
    ]


class EmberSampler(ctypes.Structure):
    """Mirror of EmberSampler (src/ember.h:141-155); its layout is ABI."""

    _fields_ = [
        ("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_int),
        ("min_p", ctypes.c_float), ("repeat_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float), ("frequency_penalty", ctypes.c_float),
        ("repeat_last_n", ctypes.c_int), ("rng_state", ctypes.c_uint64),
        ("history", ctypes.POINTER(ctypes.c_int)),
        ("hist_cap", ctypes.c_int), ("hist_len", ctypes.c_int), ("hist_pos", ctypes.c_int),
    ]


class EmberSynthConfig(ctypes.Structure):
    """Mirror of EmberSynthConfig (include/ember_synth.h)."""

    _fields_ = [
        ("dim", ctypes.c_int32), ("hidden_dim", ctypes.c_int32), ("n_layers", ctypes.c_int32),
        ("n_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32), ("max_seq_len", ctypes.c_int32),
        ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float),
        ("rope_style", ctypes.c_int32), ("qk_norm", ctypes.c_int32), ("qkv_bias", ctypes.c_int32),
        ("tied", ctypes.c_int32), ("dtype", ctypes.c_int32), ("threads", ctypes.c_int32),
        ("seed", ctypes.c_uint64), ("std", ctypes.c_float),
    ]


assert ctypes.sizeof(EmberHeader) == 256 and ctypes.sizeof(EmberTensor) == 88

_P = ctypes.c_void_p


class EhipQuantJob(ctypes.Structure):
    """ehip.h EhipQuantJob: rows x cols fp32 (host) -> Q8_0 / Q4_0 blocks (host)."""
    _fields_ = [("src", ctypes.c_void_p), ("rows", ctypes.c_int64), ("cols", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("dst", ctypes.c_void_p)]


assert ctypes.sizeof(EhipQuantJob) == 32
_FP = ctypes.POINTER(ctypes.c_float)
_IP = ctypes.POINTER(ctypes.c_int)

# every function of include/ember.h, include/ehip.h and include/ember_synth.h:
# name -> (restype, argtypes)
PROTOTYPES = {
    # ember.h
    "ember_model_load": (_P, [ctypes.c_char_p]),
    "ember_model_free": (None, [_P]),
    "ember_model_header": (ctypes.POINTER(EmberHeader), [_P]),
    "ember_model_tensor": (ctypes.POINTER(EmberTensor), [_P, ctypes.c_char_p]),
    "ember_model_data": (_P, [_P, _P]),
    "ember_state_new": (_P, [_P, ctypes.c_int]),
    "ember_state_new_ex": (_P, [_P, ctypes.c_int, ctypes.c_int]),
    "ember_state_free": (None, [_P]),
    "ember_forward": (_FP, [_P, _P, ctypes.c_int, ctypes.c_int]),
    "ember_prefill": (_FP, [_P, _P, _IP, ctypes.c_int, ctypes.c_int]),
    "ember_tokenizer_new": (_P, [_P]),
    "ember_tokenizer_free": (None, [_P]),
    "ember_encode": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_IP)]),
    "ember_decode": (ctypes.c_char_p, [_P, ctypes.c_int, ctypes.c_int]),
    "ember_sampler_init": (None, [ctypes.POINTER(EmberSampler), ctypes.c_float, ctypes.c_float,
                                  ctypes.c_int, ctypes.c_uint64]),
    "ember_sampler_set_penalties": (None, [ctypes.POINTER(EmberSampler), ctypes.c_float, ctypes.c_int,
                                           ctypes.c_float, ctypes.c_float, ctypes.c_float]),
    "ember_sampler_accept": (None, [ctypes.POINTER(EmberSampler), ctypes.c_int]),
    "ember_sampler_reset": (None, [ctypes.POINTER(EmberSampler)]),
    "ember_sampler_free": (None, [ctypes.POINTER(EmberSampler)]),
    "ember_sample": (ctypes.c_int, [ctypes.POINTER(EmberSampler), _FP, ctypes.c_int]),
    "ember_quantize_file": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]),
    "ember_threads_init": (None, [ctypes.c_int]),
    "ember_threads_shutdown": (None, []),
    "ember_nthreads": (ctypes.c_int, []),
    # ehip.h
    "ehip_last_error": (ctypes.c_char_p, []),
    "ehip_device_count": (ctypes.c_int, []),
    "ehip_model_upload": (_P, [_P, _P, _P, _P, _P, _P]),  # called from C only
    "ehip_model_free": (None, [_P]),
    "ehip_model_bytes": (ctypes.c_uint64, [_P]),
    "ehip_state_create": (_P, [_P, ctypes.c_int, ctypes.c_int]),
    "ehip_state_destroy": (None, [_P]),
    "ehip_forward": (_FP, [_P, ctypes.c_int, ctypes.c_int]),
    "ehip_prefill": (_FP, [_P, _IP, ctypes.c_int, ctypes.c_int]),
    "ehip_kv_read": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]),
    "ehip_kv_write": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]),
    "ehip_set_graph_mode": (ctypes.c_int, [_P, ctypes.c_int]),
    "ehip_decode_fusion": (ctypes.c_int, [_P]),
    "ehip_debug_buffer": (ctypes.c_int, [_P, ctypes.c_int, _P, ctypes.c_uint64]),
    "ehip_debug_capture": (ctypes.c_int, [_P, ctypes.c_int]),
    "ehip_debug_read": (ctypes.c_int, [_P, ctypes.c_int, _P, ctypes.c_uint64]),
    "ehip_debug_capture_prefill": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int]),
    "ehip_debug_read_prefill": (ctypes.c_int, [_P, ctypes.c_int, _P, ctypes.c_uint64, _IP, _IP]),
    "ehip_prefill_pass_tokens": (ctypes.c_int, [_P]),
    "ehip_time_decode": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, _FP]),
    "ehip_generate_greedy": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _IP, _FP]),
    "ehip_sample": (ctypes.c_int, [_P, _FP, ctypes.c_int, ctypes.POINTER(EmberSampler), _IP]),
    "ehip_generate_sampled": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.POINTER(EmberSampler), _IP, _FP]),
    "ehip_time_kernel": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _FP]),
    "ehip_measure_read_bw": (ctypes.c_int, [_P, ctypes.c_uint64, ctypes.c_int, _FP]),
    "ehip_libm_expf": (None, [_FP, _FP, ctypes.c_long]),
    "ehip_sample_noalloc": (ctypes.c_int, [_P, ctypes.c_int, ctypes.POINTER(EmberSampler), _P, _P, _P, _P, _P]),
    "ehip_noalloc_setup": (ctypes.c_int, []),
    "ehip_quantize_rows": (ctypes.c_int, [ctypes.POINTER(EhipQuantJob), ctypes.c_int]),
    # ember_synth.h
    "ember_synth_write": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(EmberSynthConfig)]),
    "ember_synth_fill_row": (None, [ctypes.c_uint64, ctypes.c_char_p, ctypes.c_int, ctypes.c_float,
                                    _FP, ctypes.c_int]),
    "ember_synth_row_state": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_char_p, ctypes.c_int]),
    # host helpers used by tests (declared in csrc/host/util.h and model.c)
    "ember_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
    "ember_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
    "ember_quant_q8_row": (None, [_FP, _P, ctypes.c_int]),
    "ember_quant_q4_row": (None, [_FP, _P, ctypes.c_int]),
    "ember_state_device": (_P, [_P]),
}

_lib = None


def lib():
    """Load libember.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `make -C emberllm_amd` "
                "(or __graft_entry__.build())")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def last_error():
    return (lib().ehip_last_error() or b"").decode()
