"""ctypes view of oracle/liboracle.so -- the CPU restatement of soso-llm-core.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker and the timed CPU baseline.  The
product library never loads it.  Function-level citations of the reference
are in oracle.c / oracle_avx2.c.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_q4k_decode.so")

DTYPE_F32, DTYPE_Q8_0, DTYPE_Q4_K, DTYPE_Q6_K = 1, 2, 3, 13
ELEMS = {DTYPE_Q8_0: 32, DTYPE_Q4_K: 256, DTYPE_Q6_K: 256}
BYTES = {DTYPE_Q8_0: 36, DTYPE_Q4_K: 144, DTYPE_Q6_K: 210}

_P, _S, _I, _U8, _U64, _F = C.c_void_p, C.c_size_t, C.c_int, C.c_uint8, C.c_uint64, C.c_float
_PROTO = {
    "or_f16_to_f32": (_F, [C.c_uint16]),
    "or_f32_to_f16": (C.c_uint16, [_F]),
    "or_f32_to_f16_n": (None, [_P, _S, _P]),
    "or_attention_heads_par": (_I, [_P, _P, _P, _S, _S, _S, _S, _P, _I]),
    "or_decode_layer": (_I, [_P, _P, _U8, _S, _S, _S, _S, _S, _P, _P, _S, _F, _F, _I, _I]),
    "or_row_bytes": (C.c_int64, [_U8, _S]),
    "or_dequant_q8_0_range": (_I, [_P, _S, _S, _P, _S]),
    "or_dequant_q4_k_range": (_I, [_P, _S, _S, _P, _S]),
    "or_dequant_q6_k": (_I, [_P, _S, _P, _S]),
    "or_q4k_scale_min": (None, [_P, _I, _P, _P]),
    "or_q4k_pack_scales": (None, [_P, _P, _P]),
    "or_q4k_dot_sub": (_F, [_P, _S, _I, _P, _S]),
    "or_q4k_dot_ref": (_F, [_P, _P]),
    "or_matvec_row": (_I, [_U8, _P, _S, _S, _P, _P]),
    "or_quantize_q8_0": (_S, [_P, _S, _P]),
    "or_quantize_q4_k": (_S, [_P, _S, _P]),
    "or_matvec_f32_scalar": (None, [_P, _S, _S, _P, _P]),
    "or_matvec_q8_0_scalar": (None, [_P, _S, _S, _P, _P]),
    "or_matvec_q4_k_scalar": (None, [_P, _S, _S, _P, _P]),
    "or_matvec_q6_k_scalar": (None, [_P, _S, _S, _P, _P]),
    "or_matvec_f64": (_I, [_U8, _P, _S, _S, _P, _P]),
    "or_have_avx2": (_I, []),
    "or_matvec_f32_avx2": (None, [_P, _S, _S, _P, _P]),
    "or_matvec_q8_0_avx2": (None, [_P, _S, _S, _P, _P]),
    "or_matvec_q4_k_avx2": (None, [_P, _S, _S, _P, _P]),
    "or_swiglu_avx2": (None, [_P, _P, _S]),
    "or_matvec_par": (_I, [_U8, _P, _S, _S, _P, _P, _I, _I]),
    "or_matmul_par": (_I, [_U8, _P, _S, _S, _S, _P, _P, _I, _I]),
    "or_softmax": (None, [_P, _S]),
    "or_topk_softmax": (_S, [_P, _S, _S, _P, _P]),
    "or_silu": (_F, [_F]),
    "or_swiglu": (None, [_P, _P, _S]),
    "or_rmsnorm": (None, [_P, _P, _S, _F]),
    "or_rope_heads": (None, [_P, _S, _S, _S, _F, _I]),
    "or_argmax": (C.c_uint32, [_P, _S]),
    "or_attention_f32": (None, [_P, _P, _P, _S, _S, _S, _S, _P]),
    "or_moe_ffn": (_I, [_P, _S, _S, _S, _S, _P, _P, _P, _U8, _U8, _P, _P, _P, _P, _I, _I]),
    "or_moe_shared": (_I, [_P, _S, _S, _P, _P, _P, _U8, _U8, _P, _S, _P]),
    "or_sigmoid": (_F, [_F]),
    "or_softplus": (_F, [_F]),
    "or_l2_normalize": (None, [_P, _S, _F]),
    "or_gdn_step": (None, [_P, _P, _P, _P, _S, _F, _F, _P]),
    "or_gdn_gates": (None, [_P, _P, _P, _P, _S, _S, _P, _P]),
    "or_gdn_block": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _S, _S, _S, _S, _S, _F]),
    "or_rng": (_U64, [_U64, _U64, _U64]),
    "or_normal": (_F, [_U64, _U64, _U64]),
    "or_synth_q4_k": (None, [_P, _S, _S, _U64, _U64]),
    "or_synth_q8_0": (None, [_P, _S, _S, _U64, _U64]),
    "or_synth_q6_k": (None, [_P, _S, _S, _U64, _U64]),
    "or_synth_normal": (None, [_P, _S, _F, _U64, _U64]),
    "or_now_seconds": (C.c_double, []),
    "or_stream_read": (C.c_double, [_P, _S, _I]),
}

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for n, (r, a) in _PROTO.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _lib = L
    return _lib


def ref_lib():
    """The reference's own C decode header, built by oracle/Makefile (or None)."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        L = C.CDLL(REF_PATH)
        L.ref_q4k_f16.restype, L.ref_q4k_f16.argtypes = _F, [C.c_ushort]
        L.ref_q4k_scale_min.restype, L.ref_q4k_scale_min.argtypes = None, [_P, _I, _P, _P]
        L.ref_q4k_dot_sub.restype, L.ref_q4k_dot_sub.argtypes = _F, [_P, _I, _P]
        L.ref_q4k_dot_block.restype, L.ref_q4k_dot_block.argtypes = _F, [_P, _P]
        L.ref_q80_dot_block.restype, L.ref_q80_dot_block.argtypes = _F, [_P, _P]
        _ref = L
    return _ref


def _p(a):
    return a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def row_bytes(dtype, cols):
    v = lib().or_row_bytes(dtype, cols)
    return None if v < 0 else v


def dequant(dtype, w, rows, cols):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(rows * cols, dtype=np.float32)
    if dtype == DTYPE_Q8_0:
        rc = lib().or_dequant_q8_0_range(_p(w), w.size, 0, _p(out), out.size)
    elif dtype == DTYPE_Q4_K:
        rc = lib().or_dequant_q4_k_range(_p(w), w.size, 0, _p(out), out.size)
    elif dtype == DTYPE_Q6_K:
        rc = lib().or_dequant_q6_k(_p(w), w.size, _p(out), out.size)
    else:
        raise ValueError(dtype)
    if rc != 0:
        raise ValueError("dequant rejected the input")
    return out.reshape(rows, cols)


def matvec(dtype, w, rows, cols, x, threads=1, avx2=False):
    """matvec_view_par over `threads` contiguous row strips."""
    w = np.ascontiguousarray(w, dtype=np.uint8) if dtype != DTYPE_F32 else f32(w)
    x = f32(x)
    out = np.empty(rows, dtype=np.float32)
    rc = lib().or_matvec_par(dtype, _p(w), rows, cols, _p(x), _p(out), threads, 1 if avx2 else 0)
    if rc != 0:
        raise ValueError("matvec rejected the shape")
    return out


def matmul(dtype, w, rows, cols, xs, threads=1, avx2=False):
    w = np.ascontiguousarray(w, dtype=np.uint8) if dtype != DTYPE_F32 else f32(w)
    xs = f32(xs)
    n = xs.size // cols
    out = np.empty(n * rows, dtype=np.float32)
    rc = lib().or_matmul_par(dtype, _p(w), rows, cols, n, _p(xs), _p(out), threads, 1 if avx2 else 0)
    if rc != 0:
        raise ValueError("matmul rejected the shape")
    return out.reshape(n, rows)


def matvec_f64(dtype, w, rows, cols, x):
    w = np.ascontiguousarray(w, dtype=np.uint8) if dtype != DTYPE_F32 else f32(w)
    x = f32(x)
    out = np.empty(rows, dtype=np.float64)
    if lib().or_matvec_f64(dtype, _p(w), rows, cols, _p(x), _p(out)) != 0:
        raise ValueError("matvec_f64 rejected the input")
    return out


def topk_softmax(logits, k):
    lg = f32(logits).copy()
    idx = np.empty(k, dtype=np.int32)
    w = np.empty(k, dtype=np.float32)
    kk = lib().or_topk_softmax(_p(lg), lg.size, k, _p(idx), _p(w))
    return idx[:kk], w[:kk]


def synth(dtype, rows, cols, seed, stream):
    if dtype == DTYPE_F32:
        out = np.empty(rows * cols, dtype=np.float32)
        lib().or_synth_normal(_p(out), out.size, 1.0, seed, stream)
        return out
    rb = row_bytes(dtype, cols)
    out = np.empty(rows * rb, dtype=np.uint8)
    fn = {DTYPE_Q4_K: lib().or_synth_q4_k, DTYPE_Q8_0: lib().or_synth_q8_0, DTYPE_Q6_K: lib().or_synth_q6_k}[dtype]
    fn(_p(out), rows, cols, seed, stream)
    return out


def f32_to_f16(v):
    """soso's f32 -> f16 bits (f16.rs:10-36) over an array, as uint16."""
    v = f32(v).ravel()
    out = np.empty(v.size, dtype=np.uint16)
    lib().or_f32_to_f16_n(_p(v), v.size, _p(out))
    return out


def f16_to_f32(bits):
    """soso's f16 -> f32 (dequant.rs:26-45) over an array of uint16 bits.  For
    every non-NaN pattern it equals IEEE widening (all 65536 patterns are
    compared in tests/test_oracle_golden.py), so numpy's conversion is used,
    with NaN made canonical as or_f16_to_f32 does."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = b.view(np.float16).astype(np.float32)
    out[np.isnan(out)] = np.float32(np.nan)
    return out


def normal(n, sigma, seed, stream):
    out = np.empty(n, dtype=np.float32)
    lib().or_synth_normal(_p(out), n, sigma, seed, stream)
    return out


def moe_ffn(router, n_exp, h, ffn, top_k, gate, up, down, dtype_gu, dtype_down, x, threads=1, avx2=False):
    """One token through the MoE FFN: returns (out[h], idx[top_k], w[top_k])."""
    router = f32(router)
    x = f32(x)
    arrs = [[np.ascontiguousarray(a, dtype=np.uint8) for a in grp] for grp in (gate, up, down)]
    ptrs = [(C.c_void_p * n_exp)(*[a.ctypes.data for a in grp]) for grp in arrs]
    out = np.empty(h, dtype=np.float32)
    idx = np.empty(top_k, dtype=np.int32)
    w = np.empty(top_k, dtype=np.float32)
    rc = lib().or_moe_ffn(_p(router), n_exp, h, ffn, top_k, ptrs[0], ptrs[1], ptrs[2], dtype_gu, dtype_down,
                          _p(x), _p(out), _p(idx), _p(w), threads, 1 if avx2 else 0)
    if rc != 0:
        raise ValueError("moe_ffn failed")
    return out, idx, w


def moe_shared(pg_w, h, ffn, gate, up, down, dtype_gu, dtype_down, xs, n):
    """The shared expert of an MoE block for n tokens: out [n * h]."""
    pg_w, xs = f32(pg_w), f32(xs)
    g, u, d = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down))
    out = np.empty(n * h, dtype=np.float32)
    if lib().or_moe_shared(_p(pg_w), h, ffn, _p(g), _p(u), _p(d), dtype_gu, dtype_down, _p(xs), n, _p(out)) != 0:
        raise ValueError("moe_shared failed")
    return out


def gdn_block(hist, conv, z, decay, beta, norm, state, n, n_k, n_v, d, kernel, eps):
    """GpuDispatch::gdn_bloque on the CPU: returns (out [n x n_v d], state');
    `state` is not modified."""
    st = np.array(state, dtype=np.float32, copy=True)
    out = np.empty(n * n_v * d, dtype=np.float32)
    hist, conv, z, decay, beta, norm = (f32(a) for a in (hist, conv, z, decay, beta, norm))
    rc = lib().or_gdn_block(_p(hist), _p(conv), _p(z), _p(decay), _p(beta), _p(norm), _p(st), _p(out), n, n_k, n_v,
                            d, kernel, np.float32(eps))
    if rc != 0:
        raise ValueError("gdn_block failed")
    return out, st


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    d = np.sqrt(np.sum((a - b) ** 2))
    n = np.sqrt(np.sum(b ** 2))
    return float(d / n) if n > 0 else float(d)
