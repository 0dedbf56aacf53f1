"""ctypes description of include/tenzor_hip.h (the C-ABI).

The structures mirror the C structs field for field; `bind()` attaches
argument and return types to every exported entry point.
"""
from __future__ import annotations

import ctypes as C

MAX_RANK = 8

# status codes
OK = 0
ERR_INVALID_ARGS = -1
ERR_OUT_OF_MEMORY = -2
ERR_DEVICE = -3
ERR_MISSING_WEIGHT = -4
ERR_WRONG_DTYPE = -5
ERR_UNSUPPORTED_DTYPE = -6
ERR_INVALID_FORMAT = -7
ERR_IO = -8
ERR_UNSUPPORTED_OP = -9
ERR_SHAPE = -10
ERR_TOO_LARGE = -11

ERROR_NAMES = {
    ERR_INVALID_ARGS: "InvalidArgs",
    ERR_OUT_OF_MEMORY: "OutOfMemory",
    ERR_DEVICE: "DeviceError",
    ERR_MISSING_WEIGHT: "MissingWeight",
    ERR_WRONG_DTYPE: "WrongDtype",
    ERR_UNSUPPORTED_DTYPE: "UnsupportedDtype",
    ERR_INVALID_FORMAT: "InvalidFormat",
    ERR_IO: "IoError",
    ERR_UNSUPPORTED_OP: "UnsupportedOp",
    ERR_SHAPE: "ShapeError",
    ERR_TOO_LARGE: "TooLarge",
}

# dtypes (safetensors DType order)
F16, BF16, F32, F64, I8, I16, I32, I64, U8, U16, U32, U64, BOOL = range(13)

# OpTag ordinals (expr.zig:19-91)
OP = {name: i for i, name in enumerate([
    "neg", "abs", "exp", "exp2", "log", "log2", "log10", "sqrt", "rsqrt", "sin", "cos", "tan",
    "tanh", "sinh", "cosh", "asin", "acos", "atan", "sigmoid", "relu", "leaky_relu", "gelu",
    "silu", "softplus", "ceil", "floor", "round", "sign",
    "add", "sub", "mul", "div", "pow", "max", "min", "mod", "atan2",
    "eq", "ne", "lt", "le", "gt", "ge",
    "matmul", "transpose",
    "sum", "prod", "reduce_max", "reduce_min", "mean", "variance",
    "reshape", "broadcast", "slice", "concat", "squeeze", "unsqueeze", "gather", "scatter",
])}

# NodeKind ordinals (expr.zig:137-149)
NODE_TENSOR, NODE_CONSTANT, NODE_UNARY, NODE_BINARY, NODE_MATMUL, NODE_REDUCE = 0, 1, 2, 3, 4, 5
NODE_RESHAPE, NODE_TRANSPOSE, NODE_SOFTMAX, NODE_LAYERNORM, NODE_GATHER = 6, 7, 8, 9, 10

# epilogues
EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RES_LN = 0, 1, 2


class Node(C.Structure):
    _fields_ = [
        ("kind", C.c_int32), ("op", C.c_int32), ("lhs", C.c_int32), ("rhs", C.c_int32),
        ("leaf", C.c_int32), ("axis", C.c_int32), ("keepdims", C.c_int32), ("ndim", C.c_int32),
        ("shape", C.c_int64 * MAX_RANK), ("value", C.c_double),
        ("aux", C.c_int32), ("pad_", C.c_int32), ("perm", C.c_int32 * MAX_RANK),
    ]


class Leaf(C.Structure):
    _fields_ = [("data", C.c_void_p), ("ndim", C.c_int32), ("dtype", C.c_int32), ("shape", C.c_int64 * MAX_RANK)]


class MatView(C.Structure):
    _fields_ = [("data", C.c_void_p), ("scale", C.c_void_p), ("dtype", C.c_int32), ("rows", C.c_int32),
                ("cols", C.c_int32), ("pad_", C.c_int32)]


class ArcticConfig(C.Structure):
    _fields_ = [("hidden_size", C.c_int32), ("num_hidden_layers", C.c_int32), ("num_attention_heads", C.c_int32),
                ("intermediate_size", C.c_int32), ("vocab_size", C.c_int32),
                ("max_position_embeddings", C.c_int32), ("type_vocab_size", C.c_int32),
                ("layer_norm_eps", C.c_float)]


class AttentionWeights(C.Structure):
    _fields_ = [("query_weight", MatView), ("query_bias", C.c_void_p),
                ("key_weight", MatView), ("key_bias", C.c_void_p),
                ("value_weight", MatView), ("value_bias", C.c_void_p),
                ("output_weight", MatView), ("output_bias", C.c_void_p),
                ("output_ln_gamma", C.c_void_p), ("output_ln_beta", C.c_void_p)]


class FfnWeights(C.Structure):
    _fields_ = [("intermediate_weight", MatView), ("intermediate_bias", C.c_void_p),
                ("output_weight", MatView), ("output_bias", C.c_void_p),
                ("output_ln_gamma", C.c_void_p), ("output_ln_beta", C.c_void_p)]


class LayerWeights(C.Structure):
    _fields_ = [("attention", AttentionWeights), ("ffn", FfnWeights)]


class ArcticWeights(C.Structure):
    _fields_ = [("config", ArcticConfig), ("word_embeddings", MatView), ("position_embeddings", MatView),
                ("token_type_embeddings", MatView), ("layer_norm_gamma", C.c_void_p),
                ("layer_norm_beta", C.c_void_p), ("layers", C.POINTER(LayerWeights))]


class IdsSlice(C.Structure):
    """tzh_ids_slice: one host sequence of a ragged batch."""
    _fields_ = [("ids", C.c_void_p), ("len", C.c_uint64)]


class TenzorEntry(C.Structure):
    """tzh_tenzor_entry: the 48-byte .tenzor index entry."""
    _fields_ = [("name_hash", C.c_uint64), ("dtype", C.c_uint8), ("ndim", C.c_uint8), ("pad_", C.c_uint8 * 2),
                ("shape", C.c_uint32 * 5), ("data_offset", C.c_uint64), ("data_size", C.c_uint64)]


vp = C.c_void_p
i32, i64, f32 = C.c_int32, C.c_int64, C.c_float
pp = C.POINTER(C.c_void_p)

# name -> (restype, argtypes); every entry is declared in include/tenzor_hip.h
PROTOTYPES = {
    "tzh_last_error": (C.c_char_p, []),
    "tzh_abi_version": (C.c_int, []),
    "tzh_init": (C.c_int, [C.c_int, vp, pp]),
    "tzh_destroy": (C.c_int, [vp]),
    "tzh_sync": (C.c_int, [vp]),
    "tzh_stream": (vp, [vp]),
    "tzh_ctx_scratch_info": (C.c_int, [vp, C.POINTER(i64), C.POINTER(i64)]),
    "tzh_malloc": (C.c_int, [vp, C.c_size_t, pp]),
    "tzh_free": (C.c_int, [vp, vp]),
    "tzh_memcpy_h2d": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "tzh_memcpy_d2h": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "tzh_eval_into": (C.c_int, [vp, C.POINTER(Node), i32, C.POINTER(Leaf), i32, i32, vp]),
    "tzh_matmul_w8a32": (C.c_int, [vp, vp, vp, vp, vp, vp, i64, i64, i64]),
    "tzh_matmul_w8a32_noalloc": (C.c_int, [vp, vp, vp, vp, vp, vp, i64, i64, i64]),
    "tzh_gemm_f32": (C.c_int, [vp, i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp, i64, i64, vp]),
    "tzh_matmul_nd": (C.c_int, [vp, i32, vp, vp, i32, vp, vp, i32, vp, vp, vp]),
    "tzh_linear_w8": (C.c_int, [vp, vp, i32, vp, vp, vp, vp, i32, i64, i64, i64, i32, vp, i32, vp, vp, f32]),
    "tzh_layernorm_last_dim": (C.c_int, [vp, vp, vp, vp, vp, i64, i64, f32]),
    "tzh_quantize_rows": (C.c_int, [vp, vp, i64, i64, vp, vp]),
    "tzh_quantize_rows_host": (C.c_int, [vp, i64, i64, vp, vp]),
    "tzh_quantize_safetensors": (C.c_int, [C.c_char_p, C.c_char_p, C.POINTER(i32)]),
    "tzh_arctic_upload": (C.c_int, [vp, C.POINTER(ArcticWeights), pp]),
    "tzh_arctic_load_safetensors": (C.c_int, [vp, C.c_char_p, C.POINTER(ArcticConfig), pp]),
    "tzh_arctic_free": (C.c_int, [vp]),
    "tzh_arctic_forward_batch": (C.c_int, [vp, vp, vp, vp, i32, i64]),
    "tzh_arctic_forward": (C.c_int, [vp, vp, vp, i64]),
    "tzh_arctic_forward_batch_host": (C.c_int, [vp, vp, vp, i32]),
    "tzh_arctic_forward_host": (C.c_int, [vp, vp, vp, i64]),
    "tzh_arctic_hidden": (C.c_int, [vp, vp, vp, vp, i32, i64, i32]),
    "tzh_attention_varlen": (C.c_int, [vp, vp, vp, i32, vp, i32, i32, i32]),
    "tzh_arctic_bad_id_count": (C.c_int, [vp, C.POINTER(i32)]),
    "tzh_arctic_last_launch_count": (C.c_int, [vp]),
    "tzh_arctic_set_timing": (C.c_int, [vp, i32]),
    "tzh_arctic_set_precision": (C.c_int, [vp, i32]),
    "tzh_arctic_precision": (C.c_int, [vp, C.POINTER(i32)]),
    "tzh_arctic_feed_forward": (C.c_int, [vp, i32, vp, vp, i64]),
    "tzh_arctic_set_ffn_fusion": (C.c_int, [vp, i32]),
    "tzh_arctic_launch_times": (C.c_int, [vp, C.POINTER(f32), C.POINTER(C.c_char_p), i32, C.POINTER(i32)]),
    "tzh_tenzor_name_hash": (C.c_uint64, [C.c_char_p, i64]),
    "tzh_tenzor_open": (C.c_int, [C.c_char_p, pp]),
    "tzh_tenzor_close": (C.c_int, [vp]),
    "tzh_tenzor_info": (C.c_int, [vp, C.POINTER(C.c_uint32), C.POINTER(C.c_void_p), C.POINTER(i64)]),
    "tzh_tenzor_get": (C.c_int, [vp, C.c_char_p, C.POINTER(TenzorEntry), C.POINTER(C.c_void_p)]),
    "tzh_tenzor_convert_safetensors": (C.c_int, [C.c_char_p, C.c_char_p]),
    "tzh_arctic_load_tenzor": (C.c_int, [vp, C.c_char_p, C.POINTER(ArcticConfig), pp]),
    "tzh_tokenizer_create": (C.c_int, [pp]),
    "tzh_tokenizer_free": (C.c_int, [vp]),
    "tzh_tokenizer_load_vocab": (C.c_int, [vp, C.c_char_p]),
    "tzh_tokenizer_load_vocab_bytes": (C.c_int, [vp, C.c_char_p, i64]),
    "tzh_tokenizer_put": (C.c_int, [vp, C.c_char_p, i64, C.c_uint32]),
    "tzh_tokenizer_encode": (C.c_int, [vp, C.c_char_p, i64, vp, i64, C.POINTER(i64)]),
    "tzh_tokenizer_encode_raw": (C.c_int, [vp, C.c_char_p, i64, vp, i64, C.POINTER(i64)]),
    "tzh_embed_chunk_count": (C.c_int, [i64, C.POINTER(i64)]),
    "tzh_arctic_embed_documents": (C.c_int, [vp, vp, C.POINTER(C.c_char_p), C.POINTER(i64), i32, vp, C.POINTER(i32)]),
    "tzh_arctic_embed_texts": (C.c_int, [vp, vp, C.POINTER(C.c_char_p), C.POINTER(i64), i32, vp, C.POINTER(i32)]),
}


def bind(lib: C.CDLL) -> C.CDLL:
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib
