"""GPU parity of the Gated DeltaNet block (soso_hip_gdn_block /
soso_hip_gdn_block_dev; GpuDispatch::gdn_bloque, gpu.rs:577-599, computed as
bloque35.rs:372-465) against the oracle's restatement (or_gdn_block, pinned
in tests/test_oracle_gdn.py).

Bar: the block's output and the updated state within relative L2 1e-5 of the
oracle's (the device sums the state's columns in 16-row partial sums, the CPU
in row order); a block of n tokens equal, bit for bit, to the same tokens in
two calls with the conv history and the state carried; the device-pointer
entry equal, bit for bit, to the host one; other head dims and kernels
declined with the reason.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def make_block(orc, n, n_k, n_v, d, kernel, seed):
    C = 2 * n_k * d + n_v * d
    hist = orc.normal((kernel - 1 + n) * C, 1.0, seed, 1)
    conv = orc.normal(C * kernel, 0.5, seed, 2)
    z = orc.normal(n * n_v * d, 1.0, seed, 3)
    decay = np.exp(-np.abs(orc.normal(n * n_v, 0.3, seed, 4))).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-orc.normal(n * n_v, 1.0, seed, 5)))).astype(np.float32)
    norm = (1.0 + orc.normal(d, 0.1, seed, 6)).astype(np.float32)
    state = orc.normal(n_v * d * d, 0.05, seed, 7)
    return hist, conv, z, decay, beta, norm, state


@pytest.mark.parametrize("n,n_k,n_v,kernel", [
    (1, 16, 32, 4),   # one decode token of a Qwen3-Next-80B-A3B-like GDN layer (16 q/k heads, 32 value heads)
    (5, 2, 4, 4),     # a short block
    (33, 4, 8, 4),    # a prefill block
    (3, 2, 2, 1),     # no conv history (kernel 1)
    (2, 8, 8, 3),     # as many value heads as q/k heads
])
def test_gdn_block_matches_cpu(gpu, orc, n, n_k, n_v, kernel):
    d, eps = 128, 1e-6
    print(f"gdn block n={n} n_k={n_k} n_v={n_v} kernel={kernel}", flush=True)
    hist, conv, z, decay, beta, norm, state = make_block(orc, n, n_k, n_v, d, kernel, 600 + n)
    ref_out, ref_state = orc.gdn_block(hist, conv, z, decay, beta, norm, state, n, n_k, n_v, d, kernel, eps)
    st = state.copy()
    out = gpu.gdn_block(hist, conv, z, decay, beta, norm, st, n, n_k, n_v, d, kernel, eps)
    assert out is not False, gpu.last_error()
    e_out, e_st = orc.rel_l2(out, ref_out), orc.rel_l2(st, ref_state)
    print(f"  out rel_l2 {e_out:.2e}, state rel_l2 {e_st:.2e}", flush=True)
    assert e_out < 1e-5 and e_st < 1e-5, (e_out, e_st)


def test_gdn_block_split_and_device_entry(gpu, orc):
    """Five tokens at once = tokens 0-2 then 3-4 (conv history and state
    carried), bit for bit; soso_hip_gdn_block_dev on device copies of the
    same buffers gives the host entry's bits."""
    n, n_k, n_v, d, kernel, eps = 5, 2, 4, 128, 4, 1e-6
    C = 2 * n_k * d + n_v * d
    hist, conv, z, decay, beta, norm, state = make_block(orc, n, n_k, n_v, d, kernel, 640)
    st_all = state.copy()
    out_all = gpu.gdn_block(hist, conv, z, decay, beta, norm, st_all, n, n_k, n_v, d, kernel, eps)
    H = hist.reshape(kernel - 1 + n, C)
    st = state.copy()
    outs = []
    for t0, t1 in ((0, 3), (3, 5)):
        m = t1 - t0
        outs.append(gpu.gdn_block(H[t0:t1 + kernel - 1].ravel(), conv, z[t0 * n_v * d:t1 * n_v * d],
                                  decay[t0 * n_v:t1 * n_v], beta[t0 * n_v:t1 * n_v], norm, st, m, n_k, n_v, d,
                                  kernel, eps))
    assert np.array_equal(np.concatenate(outs), out_all)
    assert np.array_equal(st, st_all)
    bufs = [hist, conv, z, decay, beta, norm, state]
    ptrs = []
    try:
        for b in bufs:
            p = gpu.dev_alloc(b.nbytes)
            gpu.h2d(p, b)
            ptrs.append(p)
        od = gpu.dev_alloc(n * n_v * d * 4)
        ptrs.append(od)
        assert gpu.gdn_block_dev(*ptrs[:7], od, n, n_k, n_v, d, kernel, eps), gpu.last_error()
        gpu.sync()
        assert np.array_equal(gpu.d2h(od, (n * n_v * d,), np.float32), out_all)
        assert np.array_equal(gpu.d2h(ptrs[6], (n_v * d * d,), np.float32), st_all)
    finally:
        for p in ptrs:
            gpu.dev_free(p)


@pytest.mark.parametrize("d,kernel,why", [(64, 4, "head dim"), (128, 17, "kernel")])
def test_gdn_block_declines(gpu, orc, d, kernel, why):
    n, n_k, n_v, eps = 1, 1, 1, 1e-6
    C = 3 * d
    st = np.zeros(d * d, np.float32)
    out = gpu.gdn_block(np.zeros((kernel - 1 + n) * C, np.float32), np.zeros(C * kernel, np.float32),
                        np.zeros(d, np.float32), np.ones(1, np.float32), np.ones(1, np.float32),
                        np.ones(d, np.float32), st, n, n_k, n_v, d, kernel, eps)
    assert out is False and why in gpu.last_error(), gpu.last_error()
