"""ctypes binding of include/soso_hip.h and include/soso_hip_bench.h
(libsoso_hip.so, built in-tree).

The library is the product: if it is missing this module raises at import
time; there is no CPU fallback behind these calls.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsoso_hip.so")

DTYPE_F32 = 1
DTYPE_Q8_0 = 2
DTYPE_Q4_K = 3
DTYPE_Q6_K = 13

OK = 1
DECLINED = 0

DECODE_QK_NORM = 1    # SOSO_HIP_DECODE_QK_NORM
DECODE_ROPE_NEOX = 2  # SOSO_HIP_DECODE_ROPE_NEOX


class HipError(RuntimeError):
    pass


class Stats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "launches", "total_ns", "bytes_up", "bytes_down",
        "weight_bytes_resident", "weights_resident", "weights_declined",
        "decode_embed_up", "decode_control_up", "decode_logits_down", "decode_kv_down", "decode_steps")]


# soso_hip_cpu_moe_fn: (ctx, layer, xn, idx, wgt, top_k, out) -> 0 on success
CpuMoeFn = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.POINTER(C.c_float), C.POINTER(C.c_int32),
                       C.POINTER(C.c_float), C.c_size_t, C.POINTER(C.c_float))


class Op(C.Structure):
    _fields_ = [
        ("key", C.c_char_p), ("key_len", C.c_size_t),
        ("w", C.c_void_p), ("w_len", C.c_size_t), ("dtype", C.c_uint8),
        ("rows", C.c_size_t), ("cols", C.c_size_t),
        ("x", C.c_void_p), ("y", C.c_void_p),
    ]


class DecodeCfg(C.Structure):
    _fields_ = [
        ("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32), ("ctx_max", C.c_uint32),
        ("rope_theta", C.c_float), ("rms_eps", C.c_float), ("kv_f16", C.c_uint32),
    ]


class Expert(C.Structure):
    _fields_ = [
        ("keys", C.c_char_p * 3), ("key_lens", C.c_size_t * 3),
        ("w", C.c_void_p * 3), ("w_len", C.c_size_t * 3), ("dtype", C.c_uint8 * 3),
        ("tokens", C.c_void_p), ("targets", C.c_void_p), ("n_tokens", C.c_size_t),
        ("shared", C.c_int),
    ]


class MoeCapa(C.Structure):
    """soso_hip_moe_capa: GpuDispatch::moe_capa's MoeCapa (gpu.rs:294-335)."""
    _fields_ = [
        ("layer", C.c_uint32), ("pos0", C.c_size_t), ("n", C.c_size_t),
        ("hidden_dim", C.c_size_t), ("heads", C.c_size_t), ("kv_heads", C.c_size_t), ("head_dim", C.c_size_t),
        ("ffn", C.c_size_t), ("n_exp", C.c_size_t), ("top_k", C.c_size_t), ("ventana", C.c_size_t),
        ("ctx_max", C.c_size_t),
        ("eps", C.c_float), ("theta", C.c_float), ("escala", C.c_float), ("rope_mscale", C.c_float),
        ("qk_norm", C.c_int), ("continuar", C.c_int), ("encadenar", C.c_int),
        ("key_q", C.c_char_p), ("key_k", C.c_char_p), ("key_v", C.c_char_p), ("key_o", C.c_char_p),
        ("prefix", C.c_char_p),
        ("attn_norm", C.c_void_p), ("q_norm", C.c_void_p), ("k_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
        ("router", C.c_void_p), ("rope_factors", C.c_void_p),
    ]


_P = C.c_void_p
_S = C.c_size_t
_I = C.c_int
_U8 = C.c_uint8
_U64 = C.c_uint64

PROTOTYPES = {
    "soso_hip_create": (_I, [_I, _U64, C.POINTER(_P)]),
    "soso_hip_destroy": (None, [_P]),
    "soso_hip_available": (_I, [_P]),
    "soso_hip_dtype_supported": (_I, [_P, _U8]),
    "soso_hip_stats": (None, [_P, C.POINTER(Stats)]),
    "soso_hip_last_error": (C.c_char_p, [_P]),
    "soso_hip_matvec": (_I, [_P, C.c_char_p, _S, _P, _S, _U8, _S, _S, _P, _P]),
    "soso_hip_matmul": (_I, [_P, C.c_char_p, _S, _P, _S, _U8, _S, _S, _S, _P, _P]),
    "soso_hip_matvec_batch": (_I, [_P, _P, _S, _P]),
    "soso_hip_router_topk": (_I, [_P, C.c_char_p, _S, _P, _P, _S, _S, _S, _S, _P, _P]),
    "soso_hip_experts_block": (_I, [_P, _P, _S, _S, _S, _S, _P, _P, _S, _P, _P]),
    "soso_hip_moe_shared": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _S, _S, _S]),
    "soso_hip_moe_register": (_I, [_P, C.c_char_p, _S, C.c_char_p, _S, _P, _P, _S, _S, _S, _S]),
    "soso_hip_moe_ffn_dev": (_I, [_P, C.c_char_p, _S, _P, _S, _P, _P, _P]),
    "soso_hip_moe_ffn_dev_noalloc": (_I, [_P, C.c_char_p, _S, _P, _S, _P, _P, _P]),
    "soso_hip_gdn_block": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _S, _S, _S, _S, _S, C.c_float]),
    "soso_hip_gdn_block_dev": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _S, _S, _S, _S, _S, C.c_float]),
    "soso_hip_decode_create": (_I, [_P, C.c_char_p, _S, C.POINTER(DecodeCfg), _P, _P, _I]),
    "soso_hip_decode_create_moe": (_I, [_P, C.c_char_p, _S, C.POINTER(DecodeCfg), _P, _P, _P, _P, _I]),
    "soso_hip_decode_moe_routing_dev": (_I, [_P, C.c_char_p, _S, C.c_uint32, C.POINTER(_P), C.POINTER(_P)]),
    "soso_hip_decode_kv_dev": (_I, [_P, C.c_char_p, _S, C.c_uint32, C.POINTER(_P), C.POINTER(_P)]),
    "soso_hip_decode_kv_upload": (_I, [_P, C.c_char_p, _S, C.c_uint32, C.c_uint32, C.c_uint32, _P, _P, _I]),
    "soso_hip_decode_step_dev": (_I, [_P, C.c_char_p, _S, _P, C.c_uint32, _P, _P, _P]),
    "soso_hip_decode_create_ex": (_I, [_P, C.c_char_p, _S, C.POINTER(DecodeCfg), C.c_uint32, _P, _P, _P, _P, C.c_int]),
    "soso_hip_decode_token": (_I, [_P, C.c_char_p, _S, _P, C.c_uint32, CpuMoeFn, _P, _P, _P, _P]),
    "soso_hip_decode_destroy": (_I, [_P, C.c_char_p, _S]),
    "soso_hip_dev_alloc": (_I, [_P, _S, C.POINTER(_P)]),
    "soso_hip_dev_free": (_I, [_P, _P]),
    "soso_hip_h2d": (_I, [_P, _P, _P, _S]),
    "soso_hip_d2h": (_I, [_P, _P, _P, _S]),
    "soso_hip_sync": (_I, [_P]),
    "soso_hip_d2d": (_I, [_P, _P, _P, _S]),
    "soso_hip_weight_from_dev": (_I, [_P, C.c_char_p, _S, _P, _S, _U8, _S, _S]),
    "soso_hip_weight_synth": (_I, [_P, C.c_char_p, _S, _U8, _S, _S, _U64, _U64]),
    "soso_hip_synth_raw": (_I, [_P, _P, _U8, _S, _S, _U64, _U64]),
    "soso_hip_synth_normal": (_I, [_P, _P, _S, C.c_float, _U64, _U64]),
    "soso_hip_read_probe": (_I, [_P, _P, _S, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _P, _S]),
    "soso_hip_weight_drop": (_I, [_P, C.c_char_p, _S]),
    "soso_hip_matvec_dev": (_I, [_P, C.c_char_p, _S, _P, _P]),
    "soso_hip_matmul_dev": (_I, [_P, C.c_char_p, _S, _S, _P, _P]),
    "soso_hip_dequant_dev": (_I, [_P, C.c_char_p, _S, _P]),
    "soso_hip_argmax_dev": (_I, [_P, _P, _S, _P]),
    "soso_hip_timer_start": (_I, [_P]),
    "soso_hip_timer_stop": (_I, [_P, C.POINTER(C.c_float)]),
    "soso_hip_event_record": (_I, [_P, _I]),
    "soso_hip_event_elapsed": (_I, [_P, _I, _I, C.POINTER(C.c_float)]),
    "soso_hip_graph_begin": (_I, [_P]),
    "soso_hip_graph_end": (_I, [_P, C.POINTER(_I)]),
    "soso_hip_graph_launch": (_I, [_P, _I]),
    "soso_hip_graph_destroy": (_I, [_P, _I]),
    "soso_hip_moe_capa_run": (_I, [_P, C.POINTER(MoeCapa), _P]),
    "soso_hip_moe_capa_can": (_I, [_P, C.c_uint32]),
    "soso_hip_moe_capa_ready": (_I, [_P, C.c_uint32]),
    "soso_hip_moe_capa_pending": (_I, [_P, C.c_uint32, _S, _S]),
    "soso_hip_moe_capa_flush": (_I, [_P, _P]),
    "soso_hip_moe_capa_discard": (None, [_P, C.c_uint32]),
    "soso_hip_moe_capa_kv_dev": (_I, [_P, C.c_uint32, C.POINTER(_P), C.POINTER(_P)]),
    "soso_hip_moe_capa_routing_dev": (_I, [_P, C.c_uint32, C.POINTER(_P), C.POINTER(_P)]),
    "soso_hip_weight_upload": (_I, [_P, C.c_char_p, _S, _P, _S, _U8, _S, _S]),
    "soso_hip_weight_resident": (_I, [_P, C.c_char_p, _S]),
}

MOE_NOALLOC_SCRATCH_BYTES = 8 << 20  # SOSO_HIP_MOE_NOALLOC_SCRATCH_BYTES

_lib = None


def load(path=LIB_PATH):
    """Loads libsoso_hip.so and declares every entry point of soso_hip.h."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise HipError(f"{path} is missing: run __graft_entry__.build() (no CPU fallback exists)")
    lib = C.CDLL(path)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
