"""ctypes binding of futon_amd/libfuton_hip.so (include/futon_hip.h,
include/futon_hip_ops.h and include/futon_host.h).  The library is the only compute path: if it is not
built, importing the model API raises; there is no CPU fallback."""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfuton_hip.so")

FH_OK = 0
FH_EINVAL = -22
FH_ENOMEM = -12
FH_EHIP = -5
FH_ECANCELED = -125
FH_ETOOLONG = -36
FH_ENODEV = -19

FH_POS_ABSOLUTE, FH_POS_ROPE = 0, 1
FH_ACT_GELU, FH_ACT_SWIGLU = 0, 1
FH_POOL_MEAN, FH_POOL_CLS = 0, 1
FH_DTYPE_F32, FH_DTYPE_F16 = 0, 1
FH_OP_F16, FH_OP_I8 = 0, 1
FH_OP_ACT_NONE, FH_OP_ACT_GELU, FH_OP_ACT_SWIGLU = 0, 1, 2

# Every symbol the public headers declare (checked by the CPU test suite).
EXPORTED = (
    "fh_model_create", "fh_model_destroy", "fh_encode", "fh_encode_device", "fh_encode_device_noalloc",
    "fh_noalloc_scratch_bytes", "fh_profile_enable",
    "fh_profile_reset", "fh_profile_read", "fh_debug_cancel_after", "fh_checkpoints_per_call",
    "fh_strerror", "fh_last_error", "fh_model_device_bytes",
    "fh_op_gemm", "fh_op_gemm_ring", "fh_op_gemm_ring_q8", "fh_op_gemm_ln", "fh_op_row_stats", "fh_op_ring_pack", "fh_op_mlp_pack", "fh_op_mlp", "fh_op_outproj_mlp", "fh_op_attention", "fh_op_layer_norm", "fh_op_quantize_rows", "fh_op_embed_ln",
    "fh_op_pool", "fh_route_flags",
    "fh_tokenizer_new", "fh_tokenizer_encode", "fh_tokenizer_vocab_size", "fh_tokenizer_free",
    "fh_pack_load", "fh_pack_config_load", "fh_pack_config", "fh_pack_model_id", "fh_pack_tensor_count",
    "fh_pack_create_model", "fh_pack_free", "fh_safetensors_check",
    "fh_provider_new", "fh_provider_embed", "fh_provider_embed_batch", "fh_provider_dimensions",
    "fh_provider_model_name", "fh_provider_is_available", "fh_provider_close", "fh_provider_free", "fh_futon_new",
)


# FH_ROUTE_* (include/futon_hip_ops.h)
FH_ROUTE_RING_QKV, FH_ROUTE_RING_OUT, FH_ROUTE_RING_FFN1, FH_ROUTE_RING_FC2 = 1, 2, 4, 8
FH_ROUTE_MLP, FH_ROUTE_MLP_QKV = 16, 32


class FhConfig(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int32), ("num_layers", ctypes.c_int32), ("num_heads", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32), ("vocab_size", ctypes.c_int32),
        ("type_vocab_size", ctypes.c_int32), ("max_seq_len", ctypes.c_int32),
        ("max_trained_positions", ctypes.c_int32), ("layer_norm_eps", ctypes.c_double),
        ("position_encoding", ctypes.c_int32), ("rope_theta", ctypes.c_double),
        ("activation", ctypes.c_int32), ("pooling", ctypes.c_int32), ("normalize", ctypes.c_int32),
        ("matryoshka", ctypes.c_int32), ("matryoshka_layernorm", ctypes.c_int32), ("q8", ctypes.c_int32),
    ]


class FhTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 4), ("data", ctypes.c_void_p)]


class FhTokenizerConfig(ctypes.Structure):
    _fields_ = [("do_lower_case", ctypes.c_int32), ("tokenize_chinese_chars", ctypes.c_int32),
                ("max_input_chars_per_word", ctypes.c_int32), ("cls_token", ctypes.c_char_p),
                ("sep_token", ctypes.c_char_p), ("unk_token", ctypes.c_char_p), ("pad_token", ctypes.c_char_p),
                ("mask_token", ctypes.c_char_p)]


class FutonError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


_lib = None


def load():
    """Loads the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run futon_amd/build.py (no CPU fallback exists)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32 = ctypes.c_void_p, ctypes.c_int32
    L.fh_model_create.restype = ctypes.c_int
    L.fh_model_create.argtypes = [ctypes.POINTER(FhConfig), ctypes.POINTER(FhTensor), i32, i32, ctypes.POINTER(vp)]
    L.fh_model_destroy.restype = None
    L.fh_model_destroy.argtypes = [vp]
    L.fh_encode.restype = ctypes.c_int
    L.fh_encode.argtypes = [vp, vp, vp, i32, i32, vp, vp]
    L.fh_encode_device.restype = ctypes.c_int
    L.fh_encode_device.argtypes = [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp]
    L.fh_encode_device_noalloc.restype = ctypes.c_int
    L.fh_encode_device_noalloc.argtypes = [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp]
    L.fh_noalloc_scratch_bytes.restype = ctypes.c_int64
    L.fh_noalloc_scratch_bytes.argtypes = []
    L.fh_profile_enable.argtypes = [vp, i32]
    L.fh_profile_reset.argtypes = [vp]
    L.fh_profile_read.argtypes = [vp, vp, vp, vp, vp, vp, i32]
    L.fh_debug_cancel_after.argtypes = [vp, i32]
    L.fh_checkpoints_per_call.argtypes = [vp]
    L.fh_strerror.restype = ctypes.c_char_p
    L.fh_strerror.argtypes = [ctypes.c_int]
    L.fh_last_error.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    L.fh_model_device_bytes.restype = ctypes.c_int64
    L.fh_model_device_bytes.argtypes = [vp]
    L.fh_op_gemm.argtypes = [i32, vp, vp, vp, vp, i32, vp, vp, vp, i32, i32, i32, i32, i32, vp]
    L.fh_op_gemm_ring.argtypes = [vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32, vp]
    L.fh_op_gemm_ring_q8.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp]
    L.fh_op_ring_pack.argtypes = [vp, vp, i32, i32, vp]
    L.fh_op_mlp_pack.argtypes = [i32, vp, vp, i32, i32, vp]
    L.fh_op_mlp.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_float, i32, i32, i32, vp]
    L.fh_op_outproj_mlp.argtypes = [vp] * 16 + [ctypes.c_float, vp, vp, vp, vp, i32, i32, i32, vp]
    L.fh_op_gemm_ln.argtypes = [i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp]
    L.fh_op_row_stats.argtypes = [vp, i32, i32, ctypes.c_float, vp, vp]
    L.fh_op_attention.argtypes = [vp, vp, i32, i32, i32, i32, vp, vp, vp, i32, i32, i32, vp]
    L.fh_op_layer_norm.argtypes = [vp, i32, i32, i32, vp, vp, ctypes.c_float, vp, vp, vp]
    L.fh_op_quantize_rows.argtypes = [vp, i32, i32, vp, vp, vp]
    L.fh_op_embed_ln.argtypes = [vp, vp, i32, i32, vp, vp, vp, vp, vp, ctypes.c_float, i32, vp, vp, vp]
    L.fh_op_pool.argtypes = [vp, vp, i32, i32, i32, i32, i32, i32, vp, vp]
    L.fh_route_flags.restype = i32
    L.fh_route_flags.argtypes = [i32, i32, i32, i32]
    cp, sz, pvp = ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(vp)
    L.fh_tokenizer_new.argtypes = [cp, ctypes.POINTER(FhTokenizerConfig), pvp]
    L.fh_tokenizer_encode.argtypes = [vp, cp, sz, i32, vp, i32, ctypes.POINTER(i32)]
    L.fh_tokenizer_vocab_size.restype = i32
    L.fh_tokenizer_vocab_size.argtypes = [vp]
    L.fh_tokenizer_free.restype = None
    L.fh_tokenizer_free.argtypes = [vp]
    L.fh_pack_load.argtypes = [cp, pvp]
    L.fh_pack_config_load.argtypes = [cp, ctypes.POINTER(FhConfig), ctypes.POINTER(i32)]
    L.fh_pack_config.argtypes = [vp, i32, ctypes.POINTER(FhConfig)]
    L.fh_pack_model_id.argtypes = [vp, cp, sz]
    L.fh_pack_tensor_count.restype = i32
    L.fh_pack_tensor_count.argtypes = [vp]
    L.fh_pack_create_model.argtypes = [vp, i32, i32, pvp]
    L.fh_pack_free.restype = None
    L.fh_pack_free.argtypes = [vp]
    L.fh_safetensors_check.argtypes = [cp, sz, ctypes.POINTER(i32)]
    L.fh_provider_new.argtypes = [cp, i32, i32, pvp]
    L.fh_provider_embed.argtypes = [vp, cp, sz, vp, vp]
    L.fh_provider_embed_batch.argtypes = [vp, vp, vp, i32, vp, vp]
    L.fh_provider_dimensions.restype = i32
    L.fh_provider_dimensions.argtypes = [vp]
    L.fh_provider_model_name.argtypes = [vp, cp, sz]
    L.fh_provider_is_available.restype = i32
    L.fh_provider_is_available.argtypes = [vp]
    L.fh_provider_close.argtypes = [vp]
    L.fh_provider_free.restype = None
    L.fh_provider_free.argtypes = [vp]
    L.fh_futon_new.argtypes = [cp, cp, cp, i32, i32, pvp]
    _lib = L
    return L


def last_error() -> str:
    buf = ctypes.create_string_buffer(2048)
    load().fh_last_error(buf, 2048)
    return buf.value.decode(errors="replace")


def check(rc: int, what: str = "") -> None:
    if rc != FH_OK:
        detail = last_error()
        name = load().fh_strerror(rc).decode()
        raise FutonError(rc, f"{what}: {name} ({rc}): {detail}" if what else f"{name} ({rc}): {detail}")
