"""Pins the CPU oracle (oracle/) before anything is compared against it.

Every check here is independent of the oracle's own formulas: the
reference's golden vectors (tests/golden/reference_goldens.json), the
reference's own C decode header built into oracle/_ref, IEEE closed forms
(numpy float16), f64 brute force, and invariants stated by the reference's
tests.
"""
import json
import os

import numpy as np
import pytest

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_goldens.json")))
DT = {"q8": 2, "q4k": 3, "q6k": 13}


def blk(hexs):
    return np.frombuffer(bytes.fromhex(hexs), dtype=np.uint8).copy()


# ---------------------------------------------------------------- f16
def test_f16_reference_cases(orc):
    L = orc.lib()
    for bits, val in GOLD["f16_cases"]["cases"]:
        assert L.or_f16_to_f32(bits) == val
    assert np.isinf(L.or_f16_to_f32(0x7C00))
    assert np.isnan(L.or_f16_to_f32(0x7E00))


def test_f16_all_patterns_ieee(orc):
    """All 65536 halves against numpy's IEEE binary16; NaN -> canonical 0x7fc00000."""
    L = orc.lib()
    bits = np.arange(65536, dtype=np.uint32)
    ours = np.array([L.or_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    ieee = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ieee)
    assert np.array_equal(ours[~nan].view(np.uint32), ieee[~nan].view(np.uint32))
    assert np.all(ours[nan].view(np.uint32) == 0x7FC00000)


def test_f16_against_reference_c_twin(orc):
    """The reference's own C decoder (lxdde/ports/nouveau/q4k_decode.h)."""
    R = orc.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built (reference tree absent when building)")
    L = orc.lib()
    for b in range(65536):
        a, r = L.or_f16_to_f32(b), R.ref_q4k_f16(b)
        if np.isnan(r):
            assert np.isnan(a)
        else:
            assert np.float32(a).view(np.uint32) == np.float32(r).view(np.uint32), hex(b)


def test_f32_to_f16_rules(orc):
    L = orc.lib()
    # every finite half survives a round trip exactly
    for b in list(range(0, 0x7C00, 7)) + [0x7BFF, 0x0001, 0x03FF, 0x0400]:
        for s in (0, 0x8000):
            assert L.or_f32_to_f16(L.or_f16_to_f32(b | s)) == (b | s)
    # ties go UP (f16.rs:34-36), not to even: 1 + 2^-11 sits between 0x3c00 and 0x3c01
    assert L.or_f32_to_f16(np.float32(1.0 + 2.0 ** -11)) == 0x3C01
    assert L.or_f32_to_f16(np.float32(1.0 + 3 * 2.0 ** -11)) == 0x3C02
    # f16.rs:65-72 extremes
    assert L.or_f32_to_f16(0.0) == 0
    assert np.isinf(L.or_f16_to_f32(L.or_f32_to_f16(1e10)))
    assert L.or_f16_to_f32(L.or_f32_to_f16(1e-10)) == 0.0
    assert np.isnan(L.or_f16_to_f32(L.or_f32_to_f16(float("nan"))))
    # f16.rs:54-63 round trip within f16 precision
    for i in range(-1000, 1000):
        v = np.float32(i * 0.37)
        rt = L.or_f16_to_f32(L.or_f32_to_f16(v))
        assert abs(v - rt) <= abs(v) * 1e-3 + 1e-4


def test_f32_to_f16_against_ieee(orc):
    """soso's rounding differs from IEEE round-to-nearest-even only on exact
    ties, which it sends away from zero.  numpy's float16 conversion is the
    IEEE one: every non-tie input must agree with it, every tie must land one
    step further from zero than the even neighbour when that neighbour is the
    smaller magnitude.  Inputs cover every f32 exponent that reaches f16
    (subnormal flushes, the subnormal range, normals, overflow) with random
    and tie-shaped mantissas."""
    rng = np.random.default_rng(5)
    exps = np.arange(90, 150, dtype=np.uint32)  # 2^-37 .. 2^22
    mant = rng.integers(0, 1 << 23, size=(exps.size, 4000), dtype=np.uint32)
    # tie-shaped mantissas: the first dropped bit set, the rest zero, at every
    # shift a normal or subnormal half can have
    ties = []
    for sh in range(13, 25):
        m = rng.integers(0, 1 << 23, size=(exps.size, 50), dtype=np.uint32)
        keep = ~np.uint32((1 << sh) - 1) & np.uint32(0x7FFFFF)
        ties.append((m & keep) | np.uint32(1 << (sh - 1)) if sh <= 23 else m * 0)
    mant = np.concatenate([mant] + ties, axis=1)
    bits = (exps[:, None] << np.uint32(23)) | mant
    bits = np.concatenate([bits.ravel(), bits.ravel() | np.uint32(0x80000000)])
    v = bits.view(np.float32)
    ours = orc.f32_to_f16(v)
    with np.errstate(over="ignore", invalid="ignore"):
        return _check_ties(orc, bits, v, ours)


def _check_ties(orc, bits, v, ours):
    ieee = v.astype(np.float16).view(np.uint16)
    # exact ties: the input sits halfway between two adjacent halves
    lo = ieee.view(np.float16).astype(np.float64)
    nxt = (ieee.astype(np.int32) + 1).astype(np.uint16)
    prv = (ieee.astype(np.int32) - 1).astype(np.uint16)
    up = np.abs(nxt.view(np.float16).astype(np.float64))
    dn = np.abs(prv.view(np.float16).astype(np.float64))
    a = np.abs(v.astype(np.float64))
    finite = np.isfinite(ieee.view(np.float16))
    tie_up = finite & (np.abs(lo) < a) & (2 * a == np.abs(lo) + up)      # even neighbour below: soso goes up
    tie_dn = finite & (np.abs(lo) > a) & (2 * a == np.abs(lo) + dn)      # even neighbour above: both go up
    assert tie_up.sum() > 1000  # the tie-shaped inputs are there
    want = ieee.copy()
    want[tie_up] = nxt[tie_up]
    # ties between 0 and the smallest subnormal: numpy gives 0, soso 2^-24
    zero_tie = (ieee & 0x7FFF) == 0
    zero_tie &= a == 2.0 ** -25
    want[zero_tie] = ieee[zero_tie] | 1
    bad = np.flatnonzero(ours != want)
    assert bad.size == 0, [(hex(int(bits[i])), hex(int(ours[i])), hex(int(want[i]))) for i in bad[:8]]
    assert not tie_dn.any() or np.array_equal(ours[tie_dn], ieee[tie_dn])
    # NaN keeps its sign and becomes 0x7e00; overflow is infinity
    assert orc.f32_to_f16(np.array([np.nan], np.float32))[0] & 0x7FFF == 0x7E00
    assert list(orc.f32_to_f16(np.array([65520.0, -1e6], np.float32))) == [0x7C00, 0xFC00]


# ---------------------------------------------------------------- layout
def test_row_bytes_reference_cases(orc):
    for dtype, cols, want in GOLD["row_bytes"]["cases"]:
        assert orc.row_bytes(dtype, cols) == want, (dtype, cols)


# ---------------------------------------------------------------- Q4_K
def test_q4k_golden_scales_and_dot(orc):
    g = GOLD["q4k_golden"]
    b = blk(g["block_hex"])
    x = np.array(g["x"], dtype=np.float32)
    L = orc.lib()
    import ctypes as C
    for j, (sc_w, m_w) in enumerate(g["scale_min"]):
        sc, m = C.c_uint8(), C.c_uint8()
        L.or_q4k_scale_min(b[4:].ctypes.data, j, C.byref(sc), C.byref(m))
        assert (sc.value, m.value) == (sc_w, m_w)
    plano = orc.dequant(3, b, 1, 256)[0]
    ref_dot = np.float32(0.0)
    for i in range(256):
        ref_dot = np.float32(ref_dot + np.float32(plano[i] * x[i]))
    assert abs(ref_dot - g["dot"]) <= g["dot_tol"]
    porsub = L.or_q4k_dot_ref(b.ctypes.data, x.ctypes.data)
    assert abs(porsub - ref_dot) <= 1e-3 * max(abs(ref_dot), 1.0)


def test_q4k_against_reference_c_twin(orc):
    R = orc.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built")
    import ctypes as C
    L = orc.lib()
    rng = np.random.default_rng(7)
    for trial in range(300):
        b = rng.integers(0, 256, 144, dtype=np.uint8)
        # finite d/dmin halves
        b[1] &= 0x7B
        b[3] &= 0x7B
        x = rng.standard_normal(256).astype(np.float32)
        for j in range(8):
            s1, m1, s2, m2 = C.c_uint8(), C.c_uint8(), C.c_uint8(), C.c_uint8()
            L.or_q4k_scale_min(b[4:].ctypes.data, j, C.byref(s1), C.byref(m1))
            R.ref_q4k_scale_min(b[4:].ctypes.data, j, C.byref(s2), C.byref(m2))
            assert (s1.value, m1.value) == (s2.value, m2.value)
            a = L.or_q4k_dot_sub(b.ctypes.data, 144, j, x[32 * j:].ctypes.data, 32)
            r = R.ref_q4k_dot_sub(b.ctypes.data, j, x[32 * j:].ctypes.data)
            assert np.float32(a).view(np.uint32) == np.float32(r).view(np.uint32)
        a = L.or_q4k_dot_ref(b.ctypes.data, x.ctypes.data)
        r = R.ref_q4k_dot_block(b.ctypes.data, x.ctypes.data)
        assert np.float32(a).view(np.uint32) == np.float32(r).view(np.uint32)


def test_q4k_known_positions(orc):
    g = GOLD["q4k_known_positions"]
    sc = np.array(g["sc"], dtype=np.uint8)
    m = np.array(g["m"], dtype=np.uint8)
    packed = np.zeros(12, dtype=np.uint8)
    orc.lib().or_q4k_pack_scales(sc.ctypes.data, m.ctypes.data, packed.ctypes.data)
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = [0x00, 0x38]
    b[2:4] = [0x00, 0x34]
    b[4:16] = packed
    b[16:] = [(i % 16) | (((i * 7) % 16) << 4) for i in range(128)]
    out = orc.dequant(3, b, 1, 256)[0]
    for e, si, q, mi in g["positions"]:
        want = g["d"] * g["sc"][si] * q - g["dmin"] * g["m"][mi]
        assert abs(out[e] - want) < 1e-4, e


def test_q4k_scale_pack_roundtrip(orc):
    import ctypes as C
    L = orc.lib()
    rng = np.random.default_rng(1)
    for _ in range(200):
        sc = rng.integers(0, 64, 8, dtype=np.uint8)
        m = rng.integers(0, 64, 8, dtype=np.uint8)
        p = np.zeros(12, dtype=np.uint8)
        L.or_q4k_pack_scales(sc.ctypes.data, m.ctypes.data, p.ctypes.data)
        for j in range(8):
            a, b = C.c_uint8(), C.c_uint8()
            L.or_q4k_scale_min(p.ctypes.data, j, C.byref(a), C.byref(b))
            assert (a.value, b.value) == (sc[j], m[j])


def _np_dequant_q4k(raw):
    """Independent vectorised Q4_K decode from GGML's published layout."""
    b = raw.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = b[:, 4:16].astype(np.int32)
    sc = np.zeros((len(b), 8), np.int32)
    mn = np.zeros((len(b), 8), np.int32)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = b[:, 16:].reshape(-1, 4, 32).astype(np.int32)
    q = np.concatenate([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32)  # sub-block 2p = low, 2p+1 = high
    dd = (d[:, None] * sc.astype(np.float32))[:, :, None]
    mm = (dmin[:, None] * mn.astype(np.float32))[:, :, None]
    return (dd * q.astype(np.float32) - mm).astype(np.float32).reshape(-1)


def _np_dequant_q6k(raw):
    """Independent vectorised Q6_K decode (GGML dequantize_row_q6_K layout)."""
    b = raw.reshape(-1, 210)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    out = np.zeros((len(b), 256), np.float32)
    for h in range(2):
        ql = b[:, h * 64:h * 64 + 64].astype(np.int32)
        qh = b[:, 128 + h * 32:128 + h * 32 + 32].astype(np.int32)
        sc = b[:, 192 + h * 8:192 + h * 8 + 8].view(np.int8).astype(np.float32)
        l = np.arange(32)
        q1 = ((ql[:, l] & 15) | ((qh & 3) << 4)) - 32
        q2 = ((ql[:, l + 32] & 15) | (((qh >> 2) & 3) << 4)) - 32
        q3 = ((ql[:, l] >> 4) | (((qh >> 4) & 3) << 4)) - 32
        q4 = ((ql[:, l + 32] >> 4) | (((qh >> 6) & 3) << 4)) - 32
        is_ = l // 16
        for k, q in enumerate((q1, q2, q3, q4)):
            s = sc[:, is_ + 2 * k]
            out[:, h * 128 + 32 * k + l] = (d[:, None] * s).astype(np.float32) * q.astype(np.float32)
    return out.reshape(-1)


def test_q4k_dequant_independent(orc):
    raw = orc.synth(3, 64, 1024, 11, 3)
    a = orc.dequant(3, raw, 64, 1024).ravel()
    b = _np_dequant_q4k(raw)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q6k_known_answer(orc):
    b = blk(GOLD["q6k_known"]["block_hex"])
    out = orc.dequant(13, b, 1, 256)
    assert np.all(out == np.float32(GOLD["q6k_known"]["value"]))


def test_q6k_dequant_independent(orc):
    raw = orc.synth(13, 32, 1024, 5, 9)
    a = orc.dequant(13, raw, 32, 1024).ravel()
    b = _np_dequant_q6k(raw)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------- Q8_0
def test_q80_golden_dot(orc):
    g = GOLD["q80_golden"]
    b = blk(g["block_hex"])
    x = np.array(g["x"], dtype=np.float32)
    plano = orc.dequant(2, b, 1, 32)[0]
    dot = np.float32(0.0)
    for i in range(32):
        dot = np.float32(dot + np.float32(plano[i] * x[i]))
    assert abs(dot - g["dot"]) <= g["dot_tol"]
    # dequant is (q as i8) * scale, exactly
    q = b[4:].view(np.int8).astype(np.float32)
    assert np.array_equal(plano, q * np.float32(0.25))


def test_q80_quantize_roundtrip(orc):
    # crates/soso-llm-core/src/quant.rs:190-198
    src = ((np.arange(64) - 32) * 0.1).astype(np.float32)
    out = np.zeros(72, np.uint8)
    n = orc.lib().or_quantize_q8_0(src.ctypes.data, 64, out.ctypes.data)
    assert n == 72
    back = orc.dequant(2, out, 1, 64)[0]
    assert np.all(np.abs(src - back) < 0.05)


def test_q4k_quantize_roundtrip(orc):
    # crates/soso-llm-core/src/quant.rs:245-289
    i = np.arange(512)
    sub = (i // 32) % 8
    t = (i % 32) / 31.0
    src = np.select([sub == 0, sub == 1, sub == 2, sub == 3],
                    [t * 20 - 10, t * 1.5 + 0.5, -t * 2.0, np.full(512, 7.0)], (i % 13.0) - 6).astype(np.float32)
    out = np.zeros(288, np.uint8)
    assert orc.lib().or_quantize_q4_k(src.ctypes.data, 512, out.ctypes.data) == 288
    back = orc.dequant(3, out, 1, 512)[0]
    for sb in range(16):
        ch = src[sb * 32:(sb + 1) * 32]
        lo, hi = min(0.0, ch.min()), max(0.0, ch.max())
        tope = (hi - lo) / 15 * 1.5 + (hi - lo) * 0.02 + 1e-6
        assert np.all(np.abs(ch - back[sb * 32:(sb + 1) * 32]) <= tope)


# ---------------------------------------------------------------- matvec
@pytest.mark.parametrize("dtype,rows,cols", [(2, 37, 512), (3, 29, 1024), (13, 23, 768), (1, 31, 200)])
def test_matvec_scalar_vs_f64(orc, dtype, rows, cols):
    w = orc.synth(dtype, rows, cols, 3, 1)
    x = orc.normal(cols, 1.0, 3, 2)
    y = orc.matvec(dtype, w, rows, cols, x)
    y64 = orc.matvec_f64(dtype, w, rows, cols, x)
    assert orc.rel_l2(y, y64) < 2e-6


@pytest.mark.parametrize("dtype", [1, 2, 3])
def test_matvec_avx2_vs_scalar(orc, dtype):
    if not orc.lib().or_have_avx2():
        pytest.skip("no AVX2")
    rows, cols = 61, 2048
    w = orc.synth(dtype, rows, cols, 4, 1)
    x = orc.normal(cols, 1.0, 4, 2)
    a = orc.matvec(dtype, w, rows, cols, x, avx2=False)
    b = orc.matvec(dtype, w, rows, cols, x, avx2=True)
    # gemm.rs:1204-1209 tolerance, and the relative-L2 bar
    assert np.all(np.abs(a - b) <= 1e-3 + 1e-4 * np.abs(a))
    assert orc.rel_l2(b, a) < 1e-5


@pytest.mark.parametrize("dtype", [2, 3])
def test_matvec_row_matches_fused(orc, dtype):
    # crates/soso-llm-core/src/quant.rs:368-403
    import ctypes as C
    for cols in (256, 512, 2048):
        rows = 3
        w = orc.synth(dtype, rows, cols, 8, 1)
        x = orc.normal(cols, 1.0, 8, 2)
        fused = orc.matvec(dtype, w, rows, cols, x)
        rb = orc.row_bytes(dtype, cols)
        for r in range(rows):
            out = C.c_float()
            fila = np.ascontiguousarray(w[r * rb:(r + 1) * rb])
            assert orc.lib().or_matvec_row(dtype, fila.ctypes.data, rb, cols, x.ctypes.data, C.byref(out)) == 0
            assert abs(out.value - fused[r]) <= 1e-3 * max(abs(fused[r]), 1.0)


@pytest.mark.parametrize("avx2", [False, True])
def test_batched_is_bit_identical(orc, avx2):
    # crates/soso-llm-core/tests/gemm_batch.rs:64-112
    for dtype in (2, 3):
        for n in (1, 3, 8, 11):
            rows, cols = 17, 512
            w = orc.synth(dtype, rows, cols, 9, 1)
            xs = orc.normal(n * cols, 1.0, 9, 3).reshape(n, cols)
            batch = orc.matmul(dtype, w, rows, cols, xs, threads=3, avx2=avx2)
            for j in range(n):
                single = orc.matvec(dtype, w, rows, cols, xs[j], avx2=avx2)
                assert np.array_equal(batch[j].view(np.uint32), single.view(np.uint32))


def test_threads_do_not_change_results(orc):
    rows, cols = 101, 1024
    w = orc.synth(3, rows, cols, 2, 1)
    x = orc.normal(cols, 1.0, 2, 2)
    a = orc.matvec(3, w, rows, cols, x, threads=1, avx2=True)
    b = orc.matvec(3, w, rows, cols, x, threads=7, avx2=True)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- small ops
def test_topk_reference_case(orc):
    g = GOLD["topk"]
    idx, w = orc.topk_softmax(np.array(g["logits"], np.float32), g["k"])
    assert len(idx) == 2 and idx[0] == g["first"]
    assert abs(float(w.sum()) - 1.0) < 1e-5


def test_topk_ties_lowest_index_and_order(orc):
    lg = np.array([0.5, 2.0, 1.0, 2.0, 2.0, -1.0], np.float32)
    idx, w = orc.topk_softmax(lg, 4)
    assert list(idx) == [1, 3, 4, 2]
    assert np.all(np.diff(w) <= 0)
    # against an f64 softmax
    p = np.exp(lg.astype(np.float64) - lg.max())
    p /= p.sum()
    sel = p[idx] / p[idx].sum()
    assert np.allclose(w, sel, rtol=1e-6)


def test_argmax_last_maximum_wins(orc):
    L = orc.lib()
    for arr, want in (([1, 3, 3, 2], 2), ([5, 1, 5], 2), ([0.0], 0), ([-1, -2, -3], 0), ([2, 2, 2, 2], 3)):
        a = np.array(arr, np.float32)
        assert L.or_argmax(a.ctypes.data, a.size) == want


def test_argmax_nan_known_answers(orc):
    """Runtime::argmax (runtime.rs:2021-2028) is Iterator::max_by with
    partial_cmp(..).unwrap_or(Equal): max_by reduces with cmp::max_by, which
    keeps the running value only when it compares Greater and otherwise takes
    the next element; a NaN compares Equal both ways.  Indices worked out by
    hand from that rule."""
    L = orc.lib()
    nan = float("nan")
    for arr, want in (([1, nan, 0.5], 2),      # NaN takes over, then hands over to 0.5
                      ([5, 1, nan], 2),        # a NaN last wins
                      ([nan, 3, 2], 1),        # a NaN first is replaced by the next element
                      ([3, nan, 1, 2], 3),     # after the NaN the fold restarts at 1
                      ([9, nan, 1, 9], 3),
                      ([nan], 0), ([2, nan, nan], 2)):
        a = np.array(arr, np.float32)
        assert L.or_argmax(a.ctypes.data, a.size) == want, (arr, want)


def test_swiglu_avx2_close_to_libm(orc):
    L = orc.lib()
    if not L.or_have_avx2():
        pytest.skip("no AVX2")
    g = orc.normal(1003, 3.0, 1, 1)
    u = orc.normal(1003, 1.0, 1, 2)
    a, b = u.copy(), u.copy()
    L.or_swiglu(a.ctypes.data, g.ctypes.data, a.size)
    L.or_swiglu_avx2(b.ctypes.data, g.ctypes.data, b.size)
    ref = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    assert np.max(np.abs(a - ref) / (np.abs(ref) + 1e-30)) < 1e-6
    assert np.max(np.abs(b - ref) / (np.abs(ref) + 1e-30)) < 1e-5  # exp256: rel err < 2e-7 (simd_math.rs:10)


def test_rmsnorm_and_rope_closed_forms(orc):
    L = orc.lib()
    x = orc.normal(64, 2.0, 4, 4)
    w = orc.normal(64, 1.0, 4, 5)
    y = x.copy()
    L.or_rmsnorm(y.ctypes.data, w.ctypes.data, 64, np.float32(1e-5))
    ref = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-6)
    # rope at pos 0 is the identity; a pair rotates by pos*theta^(-2i/d)
    v = orc.normal(2 * 128, 1.0, 6, 6)
    z = v.copy()
    L.or_rope_heads(z.ctypes.data, 2, 128, 0, np.float32(500000.0), 0)
    assert np.array_equal(z, v)
    z = v.copy()
    L.or_rope_heads(z.ctypes.data, 2, 128, 7, np.float32(500000.0), 0)
    i = np.arange(64)
    ang = 7 * 500000.0 ** (-2 * i / 128)
    a, b = v[0:128:2].astype(np.float64), v[1:128:2].astype(np.float64)
    assert np.allclose(z[0:128:2], a * np.cos(ang) - b * np.sin(ang), atol=1e-5)
    assert np.allclose(z[1:128:2], a * np.sin(ang) + b * np.cos(ang), atol=1e-5)


@pytest.mark.parametrize("pos", [0, 1, 7, 4096])
def test_rope_neox_closed_form(orc, pos):
    """rope_cabezas' NeoX branch (crates/soso-llm-core/src/gemm.rs:1474-1479):
    pair i is (i, i + d/2), not (2i, 2i + 1), rotated by pos * theta^(-2i/d).
    Checked per head against a float64 rotation; pos 0 is the identity, and a
    mistake such as rotating interleaved pairs, swapping the sine's sign or
    taking the frequency of the wrong index fails the check."""
    L = orc.lib()
    hd, nh, theta = 128, 3, 1000000.0
    v = orc.normal(nh * hd, 1.0, 8, pos + 1)
    z = v.copy()
    L.or_rope_heads(z.ctypes.data, nh, hd, pos, np.float32(theta), 1)
    if pos == 0:
        assert np.array_equal(z, v)
        return
    half = hd // 2
    i = np.arange(half)
    ang = pos * np.float64(theta) ** (-2.0 * i / hd)
    # f32 angles at large pos: allow the angle's own rounding (|pos * freq| ulp)
    tol = 1e-5 + 4 * pos * np.finfo(np.float32).eps
    for h in range(nh):
        a = v[h * hd:h * hd + half].astype(np.float64)
        b = v[h * hd + half:(h + 1) * hd].astype(np.float64)
        assert np.allclose(z[h * hd:h * hd + half], a * np.cos(ang) - b * np.sin(ang), atol=tol), h
        assert np.allclose(z[h * hd + half:(h + 1) * hd], a * np.sin(ang) + b * np.cos(ang), atol=tol), h
    # the interleaved branch moves other elements: the two differ
    w = v.copy()
    L.or_rope_heads(w.ctypes.data, nh, hd, pos, np.float32(theta), 0)
    assert not np.allclose(w, z, atol=1e-3)
    # the rotation keeps each pair's norm
    za, zb = z[:half].astype(np.float64), z[half:hd].astype(np.float64)
    va, vb = v[:half].astype(np.float64), v[half:hd].astype(np.float64)
    assert np.allclose(za ** 2 + zb ** 2, va ** 2 + vb ** 2, rtol=1e-5)


def test_attention_matches_f64_softmax(orc):
    L = orc.lib()
    hd, kvd, n = 128, 1024, 300
    q = orc.normal(hd, 1.0, 7, 1)
    k = orc.normal(n * kvd, 1.0, 7, 2)
    v = orc.normal(n * kvd, 1.0, 7, 3)
    out = np.zeros(hd, np.float32)
    L.or_attention_f32(q.ctypes.data, k.ctypes.data, v.ctypes.data, hd, kvd, 3, n, out.ctypes.data)
    K = k.reshape(n, kvd)[:, 3 * hd:4 * hd].astype(np.float64)
    V = v.reshape(n, kvd)[:, 3 * hd:4 * hd].astype(np.float64)
    s = K @ q / np.sqrt(hd)
    p = np.exp(s - s.max())
    ref = (p / p.sum()) @ V
    assert orc.rel_l2(out, ref) < 1e-5


def test_moe_ffn_matches_independent_composition(orc):
    h, ffn, E, k = 512, 256, 16, 4
    router = orc.normal(E * h, 0.02, 2, 1)
    gate = [orc.synth(3, ffn, h, 2, 100 + e) for e in range(E)]
    up = [orc.synth(3, ffn, h, 2, 200 + e) for e in range(E)]
    down = [orc.synth(3, h, ffn, 2, 300 + e) for e in range(E)]
    x = orc.normal(h, 1.0, 2, 7)
    out, idx, w = orc.moe_ffn(router, E, h, ffn, k, gate, up, down, 3, 3, x)
    lg = router.reshape(E, h).astype(np.float64) @ x
    p = np.exp(lg - lg.max())
    p /= p.sum()
    order = np.argsort(-p, kind="stable")[:k]
    assert list(order) == list(idx)
    ref = np.zeros(h)
    ww = p[order] / p[order].sum()
    for j, e in enumerate(order):
        G = orc.dequant(3, gate[e], ffn, h).astype(np.float64) @ x
        U = orc.dequant(3, up[e], ffn, h).astype(np.float64) @ x
        a = G / (1 + np.exp(-G)) * U
        ref += ww[j] * (orc.dequant(3, down[e], h, ffn).astype(np.float64) @ a)
    assert orc.rel_l2(out, ref) < 2e-5


# ---------------------------------------------------------------- generator
def test_synth_normals_and_determinism(orc):
    a = orc.normal(200000, 1.0, 42, 1)
    assert abs(a.mean()) < 0.01 and abs(a.var() - 1.0) < 0.02
    assert np.array_equal(a, orc.normal(200000, 1.0, 42, 1))
    assert not np.array_equal(a, orc.normal(200000, 1.0, 42, 2))
    w = orc.synth(3, 4, 512, 1, 1).reshape(-1, 144)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and np.all(np.isfinite(d))
