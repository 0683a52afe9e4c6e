"""ctypes binding of libq35.so (declarations in include/q35.h).

The library is loaded from the package directory (qwen-3.5_amd/libq35.so).  There is no
fallback: if the shared object is missing, every entry point raises, so a run can never silently
use another implementation.
"""
import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libq35.so")

Q35_OK, Q35_E_SHAPE, Q35_E_ALIGN, Q35_E_HIP, Q35_E_ARG, Q35_E_WS, Q35_E_NOMEM, Q35_E_RANGE = range(8)
Q35_KN, Q35_NK, Q35_KN_TILED, Q35_KN_PANEL, Q35_KN_MB = 0, 1, 2, 3, 4
Q35_LAUNCH_STREAM, Q35_LAUNCH_GRAPH, Q35_LAUNCH_PERSISTENT = 0, 1, 2
Q35_PREFILL_GEMM = 0x100
Q35_MB_PLAIN, Q35_MB_RMS, Q35_MB_GATED, Q35_MB_SWIGLU = 0, 1, 2, 3
ERROR_NAMES = {1: "Q35_E_SHAPE", 2: "Q35_E_ALIGN", 3: "Q35_E_HIP", 4: "Q35_E_ARG", 5: "Q35_E_WS", 6: "Q35_E_NOMEM",
               7: "Q35_E_RANGE"}

c_i32, c_i64, c_u64, c_f32, c_sz, c_vp = (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float,
                                          ctypes.c_size_t, ctypes.c_void_p)


class Q8F(ctypes.Structure):
    _fields_ = [("q", c_vp), ("scale", c_vp), ("rows", c_i32), ("cols", c_i32), ("layout", c_i32)]


class Dims(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("hidden", "ffn", "vocab", "n_layers", "full_interval", "lin_heads", "lin_dk",
                                     "lin_dv", "conv_k", "attn_heads", "kv_heads", "head_dim", "rot_dim")] + \
               [("eps", c_f32), ("theta", c_f32)]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class GdnWeights(ctypes.Structure):
    _fields_ = [("in_proj_qkv", Q8F), ("in_proj_z", Q8F), ("out_proj", Q8F), ("in_proj_b", c_vp), ("in_proj_a", c_vp),
                ("a_log", c_vp), ("dt_bias", c_vp), ("conv_w", c_vp), ("norm_w", c_vp)]


class AttnWeights(ctypes.Structure):
    _fields_ = [("q_proj", Q8F), ("k_proj", Q8F), ("v_proj", Q8F), ("o_proj", Q8F), ("q_norm", c_vp), ("k_norm", c_vp)]


class MlpWeights(ctypes.Structure):
    _fields_ = [("gate_proj", Q8F), ("up_proj", Q8F), ("down_proj", Q8F)]


# name -> (restype, argtypes); kept in the order of include/q35.h
PROTOTYPES = {
    "q35_last_error": (ctypes.c_char_p, []),
    "q35_dims_qwen35_2b": (Dims, []),
    "q35_q8_gemv": (ctypes.c_int, [c_vp, c_i32, Q8F, c_vp, c_vp, c_sz, c_vp]),
    "q35_q8_gemv_partial_sum": (ctypes.c_int, [c_vp, c_i32, Q8F, c_vp, c_vp, c_sz, c_vp]),
    "q35_q8_gemv_ws_bytes": (c_sz, [c_i32, Q8F]),
    "q35_q8_gemv_noalloc": (ctypes.c_int, [c_vp, c_i32, Q8F, c_vp, c_vp]),
    "q35_q8_lm_head": (ctypes.c_int, [c_vp, c_i32, Q8F, c_vp, c_vp]),
    "q35_q8_embedding_lookup": (ctypes.c_int, [Q8F, c_vp, c_i32, c_vp, c_vp]),
    "q35_gate_proj": (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp]),
    "q35_argmax": (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp, c_sz, c_vp]),
    "q35_argmax_ws_bytes": (c_sz, [c_i64]),
    "q35_gated_deltanet_decode": (ctypes.c_int, [ctypes.POINTER(Dims), ctypes.POINTER(GdnWeights), c_vp, c_i32, c_vp,
                                                 c_vp, c_vp, c_vp, c_sz, c_vp]),
    "q35_attention_decode": (ctypes.c_int, [ctypes.POINTER(Dims), ctypes.POINTER(AttnWeights), c_vp, c_i32, c_vp, c_vp,
                                            c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "q35_mlp_decode": (ctypes.c_int, [ctypes.POINTER(Dims), ctypes.POINTER(MlpWeights), c_vp, c_i32, c_vp, c_vp, c_sz,
                                      c_vp]),
    "q35_gated_delta_rule_decode": (ctypes.c_int, [c_vp, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32,
                                                   c_vp, c_sz, c_vp]),
    "q35_attention_core_decode": (ctypes.c_int, [ctypes.POINTER(Dims), c_vp, c_vp, c_vp, c_i32, c_i32, c_vp, c_vp,
                                                 c_vp, c_vp, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "q35_layer_ws_bytes": (c_sz, [ctypes.POINTER(Dims), c_i32, c_i32]),
    "q35_workspace_status": (ctypes.c_int, [c_vp, c_vp]),
    "q35_rope_tables": (ctypes.c_int, [ctypes.POINTER(Dims), c_i32, c_vp, c_vp]),
    "q35_q8_gemm": (ctypes.c_int, [c_vp, c_i32, c_i32, Q8F, c_vp, c_i32, c_i32, c_vp]),
    "q35_q8_gemm_ws_bytes": (ctypes.c_size_t, [c_i32, Q8F]),
    "q35_q8_gemv_mb_ws_bytes": (ctypes.c_size_t, [c_i32, Q8F]),
    "q35_q8_gemv_mb": (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp, c_i32, c_i32, ctypes.c_float, Q8F, c_vp,
                                      c_i32, c_i32, c_vp, ctypes.c_size_t, c_vp]),
    "q35_q8_gemm_ws": (ctypes.c_int, [c_vp, c_i32, c_i32, Q8F, c_vp, c_i32, c_i32, c_vp, ctypes.c_size_t, c_vp]),
    "q35_gate_proj_prompt": (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp]),
    "q35_gated_delta_rule_prefill": (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32,
                                                    c_i32, c_vp, c_sz, c_vp]),
    "q35_gated_delta_rule_prefill_ws_bytes": (c_sz, [c_i32, c_i32]),
    "q35_attention_core_prefill": (ctypes.c_int, [ctypes.POINTER(Dims), c_vp, c_i32, c_vp, c_vp, c_i32, c_i32, c_i32,
                                                  c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "q35_attention_prefill_ws_bytes": (c_sz, [ctypes.POINTER(Dims), c_i32]),
    "q35_model_create_synthetic": (ctypes.c_int, [ctypes.POINTER(Dims), c_u64, c_i32, ctypes.POINTER(c_vp)]),
    "q35_model_create_from_safetensors": (ctypes.c_int, [ctypes.POINTER(Dims), ctypes.c_char_p, c_i32,
                                                         ctypes.POINTER(c_vp)]),
    "q35_model_destroy": (ctypes.c_int, [c_vp]),
    "q35_model_reset": (ctypes.c_int, [c_vp, c_vp]),
    "q35_model_set_token": (ctypes.c_int, [c_vp, c_i32, c_vp]),
    "q35_model_step": (ctypes.c_int, [c_vp, c_i32, c_vp]),
    "q35_model_decode": (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp]),
    "q35_model_check": (ctypes.c_int, [c_vp, c_vp]),
    "q35_model_persistent_info": (ctypes.c_int, [c_vp, ctypes.POINTER(c_i32)]),
    "q35_model_generate": (ctypes.c_int, [c_vp, c_vp, c_i32, c_i32, c_vp, c_i32, c_i32,
                                          ctypes.POINTER(ctypes.c_double), c_vp]),
    "q35_model_generate_until": (ctypes.c_int, [c_vp, c_vp, c_i32, c_i32, c_vp, c_i32, c_vp, ctypes.POINTER(c_i32),
                                                c_i32, ctypes.POINTER(ctypes.c_double), c_vp]),
    "q35_model_prefill": (ctypes.c_int, [c_vp, c_vp, c_i32, c_vp]),
    "q35_model_decode_until": (ctypes.c_int, [c_vp, c_i32, c_vp, c_i32, c_vp, ctypes.POINTER(c_i32), c_i32,
                                              ctypes.POINTER(ctypes.c_double), c_vp]),
    "q35_model_position": (ctypes.c_int, [c_vp, ctypes.POINTER(c_i32)]),
    "q35_model_decode_stream": (ctypes.c_int, [c_vp, c_i32, c_vp, c_i32, c_vp]),
    "q35_model_stream_end": (ctypes.c_int, [c_vp, ctypes.POINTER(c_i32), c_vp]),
    "q35_model_token_stream": (c_vp, [c_vp]),
    "q35_model_tensor": (ctypes.c_int, [c_vp, ctypes.c_char_p, ctypes.POINTER(c_vp), ctypes.POINTER(c_sz)]),
    "q35_batch_create": (ctypes.c_int, [c_vp, c_i32, c_i32, ctypes.POINTER(c_vp)]),
    "q35_batch_destroy": (ctypes.c_int, [c_vp]),
    "q35_batch_reset": (ctypes.c_int, [c_vp, c_vp]),
    "q35_batch_step": (ctypes.c_int, [c_vp, c_i32, c_vp]),
    "q35_batch_decode": (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp]),
    "q35_batch_generate": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i32, c_vp, c_i32, ctypes.POINTER(ctypes.c_double), c_vp]),
    "q35_batch_position": (ctypes.c_int, [c_vp, c_vp]),
    "q35_batch_tensor": (ctypes.c_int, [c_vp, ctypes.c_char_p, ctypes.POINTER(c_vp), ctypes.POINTER(c_sz)]),
    "q35_synth_normal": (ctypes.c_int, [c_u64, c_u64, c_i64, c_i64, c_f32, c_vp]),
    "q35_synth_uniform": (ctypes.c_int, [c_u64, c_u64, c_i64, c_i64, c_f32, c_f32, c_vp]),
    "q35_synth_stream_id": (c_u64, [ctypes.c_char_p]),
    "q35_quantize_q8f": (ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_vp]),
    "q35_q8f_tiled_q_count": (c_i64, [ctypes.c_int32, ctypes.c_int32]),
    "q35_q8f_tiled_scale_count": (c_i64, [ctypes.c_int32, ctypes.c_int32]),
    "q35_q8f_pack_kn_tiled": (ctypes.c_int, [c_vp, c_vp, ctypes.c_int32, ctypes.c_int32, c_vp, c_vp]),
    "q35_q8f_pack_kn_panel": (ctypes.c_int, [c_vp, c_vp, ctypes.c_int32, ctypes.c_int32, c_vp, c_vp]),
    "q35_q8f_pack_mb": (ctypes.c_int, [Q8F, c_vp, c_vp, c_vp]),
    "q35_safetensors_tensor": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(Dims), ctypes.c_char_p, c_vp, c_i64]),
    "q35_synth_model_tensor": (ctypes.c_int, [ctypes.POINTER(Dims), c_u64, ctypes.c_char_p, c_vp, c_i64]),
}

_lib = None


class Q35Error(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code


def lib():
    """Load libq35.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != Q35_OK:
        raise Q35Error(rc, lib().q35_last_error().decode())
    return rc


def dims_2b():
    return lib().q35_dims_qwen35_2b()


def make_dims(**kw):
    d = dims_2b()
    for k, v in kw.items():
        setattr(d, k, v)
    return d
