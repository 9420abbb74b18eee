"""The oracle's one-call dense decode layer (or_decode_layer, the CPU baseline
of the device decode step) against the same layer composed step by step from
the oracle's pieces (rmsnorm gemm.rs:93-100, matvecs, rope_cabezas
gemm.rs:1452-1490, attention, swiglu gemm.rs:210-226, residuals;
LayerExecutor::forward_layer, layer.rs:1092-1389) -- the composition the GPU
decode test compares the device against.  Row strips and per-head tasks do not
change any result, so the threaded call must match bit for bit.
"""
import ctypes as C

import numpy as np
import pytest

Q4K = 3
HD = 128


def quant_q4k(orc, w):
    w = np.ascontiguousarray(w, np.float32).ravel()
    out = np.zeros(w.size // 256 * 144, np.uint8)
    orc.lib().or_quantize_q4_k(w.ctypes.data, w.size, out.ctypes.data)
    return out


def stepwise(orc, h, w, H, nh, nkv, F, kc, vc, pos, theta, eps):
    L = orc.lib()
    qd, kvd = nh * HD, nkv * HD
    xn = h.copy()
    L.or_rmsnorm(xn.ctypes.data, w[0].ctypes.data, H, np.float32(eps))
    q = orc.matvec(Q4K, w[1], qd, H, xn)
    k = orc.matvec(Q4K, w[2], kvd, H, xn)
    v = orc.matvec(Q4K, w[3], kvd, H, xn)
    L.or_rope_heads(q.ctypes.data, nh, HD, pos, np.float32(theta), 0)
    L.or_rope_heads(k.ctypes.data, nkv, HD, pos, np.float32(theta), 0)
    kc[pos], vc[pos] = k, v
    att = np.zeros(qd, np.float32)
    for hh in range(nh):
        qh = np.ascontiguousarray(q[hh * HD:(hh + 1) * HD])
        out = np.zeros(HD, np.float32)
        L.or_attention_f32(qh.ctypes.data, kc.ctypes.data, vc.ctypes.data, HD, kvd, hh // (nh // nkv), pos + 1,
                           out.ctypes.data)
        att[hh * HD:(hh + 1) * HD] = out
    h = h + orc.matvec(Q4K, w[4], H, qd, att)
    xn = h.copy()
    L.or_rmsnorm(xn.ctypes.data, w[5].ctypes.data, H, np.float32(eps))
    g = orc.matvec(Q4K, w[6], F, H, xn)
    u = orc.matvec(Q4K, w[7], F, H, xn)
    L.or_swiglu(u.ctypes.data, g.ctypes.data, F)
    return h + orc.matvec(Q4K, w[8], H, F, u)


@pytest.mark.parametrize("threads", [1, 4])
def test_decode_layer_matches_stepwise(orc, threads):
    H, nh, nkv, F, ctx, pos, theta, eps = 256, 4, 2, 512, 32, 17, 500000.0, 1e-5
    qd, kvd = nh * HD, nkv * HD
    s = iter(range(1, 100))
    mat = lambda r, c: quant_q4k(orc, orc.normal(r * c, 0.05, 5, next(s)))
    w = [(1.0 + orc.normal(H, 0.1, 5, next(s))).astype(np.float32), mat(qd, H), mat(kvd, H), mat(kvd, H),
         mat(H, qd), (1.0 + orc.normal(H, 0.1, 5, next(s))).astype(np.float32), mat(F, H), mat(F, H), mat(H, F)]
    kc = np.zeros((ctx, kvd), np.float32)
    vc = np.zeros((ctx, kvd), np.float32)
    kc[:pos] = orc.normal(pos * kvd, 1.0, 6, 1).reshape(pos, kvd)
    vc[:pos] = orc.normal(pos * kvd, 1.0, 6, 2).reshape(pos, kvd)
    h0 = orc.normal(H, 1.0, 7, 1)
    kr, vr = kc.copy(), vc.copy()
    ref = stepwise(orc, h0.copy(), w, H, nh, nkv, F, kr, vr, pos, theta, eps)
    h = h0.copy()
    ptrs = (C.c_void_p * 9)(*[a.ctypes.data for a in w])
    assert orc.lib().or_decode_layer(h.ctypes.data, C.cast(ptrs, C.c_void_p), Q4K, H, nh, nkv, HD, F,
                                     kc.ctypes.data, vc.ctypes.data, pos, np.float32(theta), np.float32(eps),
                                     threads, 0) == 0
    assert np.array_equal(h, ref)
    assert np.array_equal(kc[pos], kr[pos]) and np.array_equal(vc[pos], vr[pos])
