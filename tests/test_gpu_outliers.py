"""Activation outliers on the paths that stage x for several tokens: the
matrix-core matmul (Q4_K, Q8_0) and the MoE expert kernels (single-token
self-ranked gate/up, down + ranking-order sum, batch-32 matrix-core experts).

Real hidden states carry a few channels 1e3-1e4 times the rest.  A staging
that gives a whole block one exponent would leave the other elements of the
block ~10 significant bits; where the large elements meet zero weights the
result is made of those small elements only and would be off by ~1e-3.
Every path must stay within relative L2 1e-5 of the CPU: the f64 brute force
for the matmuls, the oracle's f32 composition of the MoE FFN (whose own f32
arithmetic is exact here: the zero weights under the large elements make
their products, and the min terms of their super-blocks, exactly zero).

Reference: crates/sosomodel/src/dequant.rs:172-201 (the factorised Q4_K
dot), crates/soso-llm-core/src/layer.rs:1869-1934 (the MoE FFN).
"""
import numpy as np
import pytest

from test_gpu_matvec import outlier_x, zero_columns
from test_gpu_moe import Layer, moe_dev

pytestmark = pytest.mark.gpu

TOL = 1e-5
Q8, Q4K = 2, 3


def small_columns_q8(w, rows, cols, zc):
    """Q8_0 bytes with the codes of columns `zc` set to +-1 (64 times below
    the median code): the large elements then carry a small part of the sum."""
    w = w.copy()
    blk = w.reshape(rows, cols // 32, 36)
    for k, c in enumerate(zc):
        blk[:, c // 32, 4 + c % 32] = np.uint8(1 if k % 2 == 0 else 0xFF)
    return w


@pytest.mark.parametrize("dtype,rows,cols,n,weights", [
    (Q4K, 4096, 4096, 64, "zero"),
    (Q4K, 14336, 4096, 32, "zero"),
    (Q8, 4096, 4096, 64, "zero"),
    (Q8, 4096, 4096, 16, "small"),
    (Q4K, 1000, 4096, 37, "zero"),
])
def test_matmul_matrix_cores_outliers_under_zero_weights(gpu, orc, dtype, rows, cols, n, weights):
    """Every token has elements 1e3 and 1e4 times the rest in every 128
    elements (at token-dependent places), and the weights under the large
    elements are zero (or, for Q8_0, codes of +-1): per token, relative L2
    within 1e-5 of the f64 brute force."""
    w = orc.synth(dtype, rows, cols, 131, n)
    xs, zc = [], set()
    for t in range(n):
        at = (5 + (t % 3), 77 + 2 * (t % 5))
        x, oc = outlier_x(orc, cols, 132 + t, at=at)
        xs.append(x)
        zc.update(int(c) for c in oc)
    xs = np.stack(xs)
    zc = np.array(sorted(zc))
    w = zero_columns(dtype, w, rows, cols, zc) if weights == "zero" else small_columns_q8(w, rows, cols, zc)
    out = np.empty(n * rows, np.float32)
    key = f"outl.mm.{dtype}.{rows}.{cols}.{n}.{weights}"
    try:
        assert gpu.matmul(key, w, dtype, rows, cols, n, xs, out), gpu.last_error()
        out = out.reshape(n, rows)
        worst = 0.0
        for t in range(n):
            ref = orc.matvec_f64(dtype, w, rows, cols, xs[t])
            worst = max(worst, orc.rel_l2(out[t], ref))
        print(f"matmul outliers dtype {dtype} {rows}x{cols} n={n} {weights}: worst rel_l2 {worst:.3e}", flush=True)
        assert worst < TOL, worst
    finally:
        gpu.weight_drop(key)


@pytest.mark.parametrize("cols,n", [(4096, 16), (2048, 20)])
def test_matmul_matrix_cores_outlier_edges(gpu, orc, cols, n):
    """The edges of the outlier rule on the matrix cores: two whole 8-element
    chunks of a 128-block far above the rest (the list's capacity), a block
    that is zero but for a few elements, a constant token (no outliers) and
    a token with a single block of outliers; zero weights under the large
    elements."""
    rows = 512
    xs = orc.normal(n * cols, 1.0, 141, 1).reshape(n, cols).copy()
    zc = set()
    for t in range(n):
        x = xs[t]
        kind = t % 4
        if kind == 0:
            for b in range(cols // 128):
                x[b * 128 + 16:b * 128 + 24] = 5e4
                x[b * 128 + 96:b * 128 + 104] = -3e3
                zc.update(list(range(b * 128 + 16, b * 128 + 24)) + list(range(b * 128 + 96, b * 128 + 104)))
        elif kind == 1:
            x[:] = 0.0
            x[3::128] = 7.0
            x[64::512] = -1e5
            zc.update(range(64, cols, 512))
        elif kind == 2:
            x[:] = 0.75
        else:
            x[9 * 128 + 33] = -4e4
            zc.add(9 * 128 + 33)
    for dtype in (Q4K, Q8):
        w = zero_columns(dtype, orc.synth(dtype, rows, cols, 142, dtype), rows, cols, np.array(sorted(zc)))
        out = np.empty(n * rows, np.float32)
        key = f"outl.mm.edge.{dtype}.{cols}.{n}"
        try:
            assert gpu.matmul(key, w, dtype, rows, cols, n, xs, out), gpu.last_error()
            out = out.reshape(n, rows)
            for t in range(n):
                ref = orc.matvec_f64(dtype, w, rows, cols, xs[t])
                assert orc.rel_l2(out[t], ref) < TOL, (dtype, t, orc.rel_l2(out[t], ref))
        finally:
            gpu.weight_drop(key)


def _zero_gate_up_columns(layer, zc):
    layer.gate = [zero_columns(Q4K, w, layer.ffn, layer.h, zc) for w in layer.gate]
    layer.up = [zero_columns(Q4K, w, layer.ffn, layer.h, zc) for w in layer.up]


@pytest.mark.parametrize("n", [1, 32])
def test_moe_outliers_under_zero_weights(gpu, orc, n):
    """configs[3] (128 Q4_K experts of 768, hidden 2048, top-8) with every
    token's x carrying 1e3 / 1e4 elements in every 128, over zero gate/up
    weights: routing identical and outputs within 1e-5 of the CPU at batch 1
    (self-ranked single-token kernels) and batch 32 (matrix cores)."""
    n_exp, h, ffn, top_k = 128, 2048, 768, 8
    layer = Layer(orc, n_exp, h, ffn, top_k, 150 + n)
    # a router 1e4 times smaller keeps the logits of these large inputs
    # moderate, so the ranking is decided well above f32 rounding
    layer.router = (layer.router * np.float32(1e-4)).astype(np.float32)
    xs, zc = [], set()
    for t in range(n):
        x, oc = outlier_x(orc, h, 151 + t, at=(5 + (t % 3), 77 + (t % 7)))
        xs.append(x)
        zc.update(int(c) for c in oc)
    _zero_gate_up_columns(layer, np.array(sorted(zc)))
    xs = np.concatenate(xs)
    layer.upload(gpu)
    try:
        out, idx, wgt = moe_dev(gpu, layer, xs)
        worst = 0.0
        for t in range(n):
            ref, ri, rw = layer.cpu(orc, xs[t * h:(t + 1) * h])
            assert np.array_equal(idx[t], ri), (t, idx[t], ri)
            assert orc.rel_l2(wgt[t], rw) < TOL
            worst = max(worst, orc.rel_l2(out[t], ref))
        print(f"moe outliers n={n}: worst rel_l2 {worst:.3e}", flush=True)
        assert worst < TOL, worst
    finally:
        layer.drop(gpu)


@pytest.mark.parametrize("n", [1, 5, 32])
def test_moe_intermediate_outlier_under_zero_down_weights(gpu, orc, n):
    """A massive intermediate activation: for every expert, gate and up row
    r0 carry large weights exactly under the tokens' large x elements, so
    silu(g) * u at r0 is ten orders of magnitude above the other elements,
    and every expert's down column r0 is zero.  The down projection's
    staging (single-token down + sum, the grouped dot4 path at 5 tokens, the
    matrix cores at 32) must
    keep the other elements' precision: outputs within 1e-5 of the CPU."""
    n_exp, h, ffn, top_k = 64, 2048, 768, 8
    r0 = 300
    layer = Layer(orc, n_exp, h, ffn, top_k, 160 + n)
    layer.router = (layer.router * np.float32(1e-4)).astype(np.float32)
    # positive large elements at the same places in every token, so that g
    # and u at r0 are large and positive
    zc = np.array([b * 128 + a for b in range(h // 128) for a in (5, 77)])
    xs = []
    for t in range(n):
        x = orc.normal(h, 1.0, 161 + t, 1).copy()
        x[zc] = np.where(zc % 128 == 5, np.float32(1e3), np.float32(1e4))
        xs.append(x)
    _zero_gate_up_columns(layer, zc)
    # row r0 of gate and up: codes 15 under the large elements (sub-block
    # scale and d kept), so g and u at r0 are dominated by them
    stride = (h // 256) * 144
    for mats in (layer.gate, layer.up):
        for k, w in enumerate(mats):
            w = w.copy()
            row = w[r0 * stride:(r0 + 1) * stride].reshape(h // 256, 144)
            for c in zc:
                sb, pos = c // 256, c % 256
                pr, e = pos // 64, pos % 64
                byte = 16 + 32 * pr + (e & 31)
                row[sb, byte] |= np.uint8(0x0F if e < 32 else 0xF0)
            mats[k] = w
    layer.down = [zero_columns(Q4K, w, h, ffn, np.array([r0])) for w in layer.down]
    xs = np.concatenate(xs)
    layer.upload(gpu)
    try:
        out, idx, wgt = moe_dev(gpu, layer, xs)
        worst = 0.0
        for t in range(n):
            ref, ri, rw = layer.cpu(orc, xs[t * h:(t + 1) * h])
            assert np.array_equal(idx[t], ri), (t, idx[t], ri)
            worst = max(worst, orc.rel_l2(out[t], ref))
        print(f"moe intermediate outlier n={n}: worst rel_l2 {worst:.3e}", flush=True)
        assert worst < TOL, worst
    finally:
        layer.drop(gpu)
