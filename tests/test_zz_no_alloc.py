"""GPU test of soso_hip_moe_ffn_dev_noalloc, the MoE FFN entry point that
allocates nothing (its scratch is the library's fixed per-GPU array).

It has no counterpart in the reference; its results must equal those of
soso_hip_moe_ffn_dev (the same kernels on the same inputs), bit for bit, on
calls in a row whose token counts shrink, since the fixed array keeps the last
call's contents.
"""
import numpy as np
import pytest

from test_gpu_moe import Layer

pytestmark = pytest.mark.gpu

Q4K = 3
NOALLOC_BYTES = 8 << 20


def run(gpu, fn, layer, xd, n):
    od = gpu.dev_alloc(n * layer.h * 4)
    idd = gpu.dev_alloc(n * layer.top_k * 4)
    wd = gpu.dev_alloc(n * layer.top_k * 4)
    try:
        assert fn(layer.name, xd, n, od, idd, wd), gpu.last_error()
        gpu.sync()
        return (gpu.d2h(od, (n, layer.h), np.float32), gpu.d2h(idd, (n, layer.top_k), np.int32),
                gpu.d2h(wd, (n, layer.top_k), np.float32))
    finally:
        for p in (od, idd, wd):
            gpu.dev_free(p)


def test_noalloc_moe_equals_moe_ffn_dev(gpu, orc):
    n_exp, h, ffn, top_k = 32, 1024, 512, 4
    layer = Layer(orc, n_exp, h, ffn, top_k, 501)
    layer.upload(gpu)
    xs = orc.normal(40 * h, 1.0, 502, 1)
    xd = gpu.dev_alloc(xs.nbytes)
    try:
        gpu.h2d(xd, xs)
        # 40 tokens (the matrix-core experts), then 3 (down and the weighted
        # sum in one launch), then 1 (the self-ranking single-token kernels)
        for n in (40, 3, 1):
            print(f"noalloc moe: {n} tokens", flush=True)
            got = run(gpu, gpu.moe_ffn_dev_noalloc, layer, xd, n)
            want = run(gpu, gpu.moe_ffn_dev, layer, xd, n)
            assert np.array_equal(got[1], want[1]), n
            assert np.array_equal(got[2].view(np.uint32), want[2].view(np.uint32)), n
            assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32)), n
            ref, ri, _ = layer.cpu(orc, xs[:h])
            assert np.array_equal(got[1][0], ri) and orc.rel_l2(got[0][0], ref) < 1e-5
        # a token count the growable scratch never held, captured in a graph
        # (the allocating entry point would have to grow its scratch there)
        n = 7
        od = gpu.dev_alloc(n * h * 4)
        try:
            gpu.graph_begin()
            try:
                ok = gpu.moe_ffn_dev_noalloc(layer.name, xd, n, od)
            finally:
                gid = gpu.graph_end()
            try:
                assert ok, gpu.last_error()
                want = run(gpu, gpu.moe_ffn_dev, layer, xd, n)[0]
                for rep in range(2):
                    gpu.h2d(od, np.zeros(n * h, np.float32))
                    gpu.graph_launch(gid)
                    gpu.sync()
                    assert np.array_equal(gpu.d2h(od, (n, h), np.float32).view(np.uint32), want.view(np.uint32)), rep
            finally:
                gpu.graph_destroy(gid)
        finally:
            gpu.dev_free(od)
    finally:
        gpu.dev_free(xd)
        layer.drop(gpu)


def test_noalloc_moe_rejects_more_than_the_fixed_array(gpu, orc):
    """400 tokens at top-4 need 1600 * (512 + 1024) * 4 bytes of activations
    alone, more than the fixed array: a clear error, nothing launched."""
    from soso_amd.abi import HipError
    n_exp, h, ffn, top_k = 8, 1024, 512, 4
    layer = Layer(orc, n_exp, h, ffn, top_k, 503)
    layer.upload(gpu)
    n = 400
    assert n * top_k * (ffn + h) * 4 > NOALLOC_BYTES
    xd = gpu.dev_alloc(n * h * 4)
    od = gpu.dev_alloc(n * h * 4)
    try:
        with pytest.raises(HipError, match="fixed array"):
            gpu.moe_ffn_dev_noalloc(layer.name, xd, n, od)
    finally:
        gpu.dev_free(xd)
        gpu.dev_free(od)
        layer.drop(gpu)
