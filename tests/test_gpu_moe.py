"""GPU parity of the MoE decode path through the C ABI.

Reference behaviour: topk_softmax (crates/soso-llm-core/src/gemm.rs:62-91)
with ties to the lowest index, experts combined in ranking order
(crates/soso-llm-core/src/layer.rs:1869-1934), GpuDispatch::router_topk and
expertos_bloque (crates/soso-llm-core/src/gpu.rs:461-494).  The oracle's
or_moe_ffn composes the same steps on the CPU.

Bar: the chosen expert indices identical, in the same ranking order; routing
weights and FFN outputs within relative L2 1e-5 (f32 accumulate).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-5
Q4K, Q8, F32 = 3, 2, 1


class Layer:
    """A seeded MoE FFN (router f32 ~ N(0, 0.02), experts Q4_K like configs[3])."""

    def __init__(self, orc, n_exp, h, ffn, top_k, seed, dt_down=Q4K):
        self.n_exp, self.h, self.ffn, self.top_k, self.dt_down = n_exp, h, ffn, top_k, dt_down
        self.router = orc.normal(n_exp * h, 0.02, seed, 1)
        self.gate = [orc.synth(Q4K, ffn, h, seed, 100 + e) for e in range(n_exp)]
        self.up = [orc.synth(Q4K, ffn, h, seed, 1000 + e) for e in range(n_exp)]
        self.down = [orc.synth(dt_down, h, ffn, seed, 2000 + e) for e in range(n_exp)]
        self.name = f"moe{seed}.{n_exp}.{h}.{ffn}.{top_k}.{dt_down}"

    def keys(self, e):
        return [f"{self.name}.E{e}.gate", f"{self.name}.E{e}.up", f"{self.name}.E{e}.down"]

    def cpu(self, orc, x):
        return orc.moe_ffn(self.router, self.n_exp, self.h, self.ffn, self.top_k, self.gate, self.up, self.down,
                           Q4K, self.dt_down, x)

    def upload(self, gpu):
        """Every matrix resident under its key, the router as an F32 weight."""
        for e in range(self.n_exp):
            for k, (w, dt, r, c) in zip(self.keys(e), ((self.gate[e], Q4K, self.ffn, self.h),
                                                       (self.up[e], Q4K, self.ffn, self.h),
                                                       (self.down[e], self.dt_down, self.h, self.ffn))):
                d = gpu.dev_alloc(w.size)
                try:
                    gpu.h2d(d, w)
                    gpu.weight_from_dev(k, d, w.size, dt, r, c)
                finally:
                    gpu.dev_free(d)
        d = gpu.dev_alloc(self.router.nbytes)
        try:
            gpu.h2d(d, self.router)
            gpu.weight_from_dev(self.name + ".router", d, self.router.nbytes, F32, self.n_exp, self.h)
        finally:
            gpu.dev_free(d)
        keys = [k for e in range(self.n_exp) for k in self.keys(e)]
        gpu.moe_register(self.name, self.name + ".router", keys, self.n_exp, self.h, self.ffn, self.top_k)

    def drop(self, gpu):
        for e in range(self.n_exp):
            for k in self.keys(e):
                gpu.weight_drop(k)
        gpu.weight_drop(self.name + ".router")


def moe_dev(gpu, layer, xs):
    n = xs.size // layer.h
    xd = gpu.dev_alloc(xs.nbytes)
    od = gpu.dev_alloc(n * layer.h * 4)
    idd = gpu.dev_alloc(n * layer.top_k * 4)
    wd = gpu.dev_alloc(n * layer.top_k * 4)
    try:
        gpu.h2d(xd, xs)
        gpu.moe_ffn_dev(layer.name, xd, n, od, idd, wd)
        gpu.sync()
        return (gpu.d2h(od, (n, layer.h), np.float32), gpu.d2h(idd, (n, layer.top_k), np.int32),
                gpu.d2h(wd, (n, layer.top_k), np.float32))
    finally:
        for p in (xd, od, idd, wd):
            gpu.dev_free(p)


@pytest.mark.parametrize("n_exp,h,top_k,n", [(128, 2048, 8, 1), (128, 2048, 8, 32), (16, 512, 4, 5), (40, 256, 1, 3)])
def test_router_topk_matches_cpu(gpu, orc, n_exp, h, top_k, n):
    w = orc.normal(n_exp * h, 0.02, 71, n_exp)
    xs = orc.normal(n * h, 1.0, 72, n)
    idx = np.full(n * top_k, -1, np.int32)
    wgt = np.zeros(n * top_k, np.float32)
    assert gpu.router_topk(f"router.{n_exp}.{h}", w, xs, n, h, n_exp, top_k, idx, wgt), gpu.last_error()
    for t in range(n):
        logits = orc.matvec(F32, w, n_exp, h, xs[t * h:(t + 1) * h])
        ci, cw = orc.topk_softmax(logits, top_k)
        assert np.array_equal(idx[t * top_k:(t + 1) * top_k], ci), (t, idx[t * top_k:(t + 1) * top_k], ci)
        assert orc.rel_l2(wgt[t * top_k:(t + 1) * top_k], cw) < TOL
        assert abs(float(np.sum(wgt[t * top_k:(t + 1) * top_k], dtype=np.float64)) - 1.0) < 1e-5


def test_router_topk_beyond_one_route_launch(gpu, orc):
    """600 tokens at top-8 (4800 slots) run as two route launches of at most
    4096 slots (the reference's router has no cap): every token's indices and
    weights match the CPU, the block edge (tokens 511, 512) included."""
    n_exp, h, top_k, n = 32, 256, 8, 600
    w = orc.normal(n_exp * h, 0.05, 74, 1)
    xs = orc.normal(n * h, 1.0, 75, 1)
    idx = np.full(n * top_k, -1, np.int32)
    wgt = np.zeros(n * top_k, np.float32)
    assert gpu.router_topk("router.many", w, xs, n, h, n_exp, top_k, idx, wgt), gpu.last_error()
    for t in range(n):
        logits = orc.matvec(F32, w, n_exp, h, xs[t * h:(t + 1) * h])
        ci, cw = orc.topk_softmax(logits, top_k)
        assert np.array_equal(idx[t * top_k:(t + 1) * top_k], ci), t
        assert orc.rel_l2(wgt[t * top_k:(t + 1) * top_k], cw) < TOL, t


def test_router_ties_lowest_index_first(gpu, orc):
    """Equal logits: the stable descending sort keeps the lower index first."""
    n_exp, h, top_k = 64, 64, 6
    w = np.zeros((n_exp, h), np.float32)
    for e in (3, 10, 17, 40, 41, 63):  # six experts with the same (largest) logit
        w[e, 0] = 1.0
    w[20, 0] = 0.5
    xs = np.zeros(h, np.float32)
    xs[0] = 2.0
    idx = np.zeros(top_k, np.int32)
    wgt = np.zeros(top_k, np.float32)
    assert gpu.router_topk("router.ties", w.ravel(), xs, 1, h, n_exp, top_k, idx, wgt)
    assert list(idx) == [3, 10, 17, 40, 41, 63]
    assert np.allclose(wgt, 1.0 / 6.0, rtol=1e-6)


@pytest.mark.parametrize("n_exp,h,ffn,top_k,n,dt_down", [
    (16, 2048, 768, 8, 1, Q4K),    # configs[3] expert shapes, fewer experts
    (128, 2048, 768, 8, 1, Q4K),   # configs[3] at batch 1: the expert kernel ranks the token itself
    (40, 256, 512, 1, 1, Q4K),     # one token, top-1
    (200, 512, 256, 5, 1, Q4K),    # one token, 200 experts (four logits per lane), top-5
    (12, 512, 256, 3, 1, Q8),      # one token with Q8_0 down projections: the general path
    (16, 2048, 768, 8, 32, Q4K),   # batch 32: 16 tokens per expert (four rounds), the matrix-core path
    (128, 2048, 768, 8, 32, Q4K),  # configs[3] at batch 32: about 2.3 tokens per expert, tile-major copies
    (128, 2048, 768, 8, 64, Q4K),  # 512 ranked slots: the most the expert kernels find by scanning the ranking
    (64, 512, 256, 8, 65, Q4K),    # 520 slots: one past the scan, the route sorts the slots
    (12, 512, 256, 3, 7, Q8),      # Q8_0 down projections (soso's converted Q6_K experts)
    (8, 512, 256, 4, 48, Q4K),     # 24 tokens per expert: six 4-token rounds on the matrix cores
    (6, 512, 256, 3, 16, Q8),      # matrix-core gate/up, dot4 Q8_0 down
    (20, 512, 512, 6, 4, Q4K),     # 4 tokens, top-6: down and the weighted sum in one launch
    (10, 256, 1024, 2, 3, Q4K),    # 3 tokens, top-2, wide ffn: down + sum in one launch
    (24, 512, 256, 8, 5, Q4K),     # 5 tokens: one past the fused launch, grouped down + combine
])
def test_moe_ffn_dev_matches_cpu(gpu, orc, n_exp, h, ffn, top_k, n, dt_down):
    layer = Layer(orc, n_exp, h, ffn, top_k, 40 + n, dt_down)
    layer.upload(gpu)
    try:
        xs = orc.normal(n * h, 1.0, 73, n)
        out, idx, wgt = moe_dev(gpu, layer, xs)
        for t in range(n):
            ref, ri, rw = layer.cpu(orc, xs[t * h:(t + 1) * h])
            assert np.array_equal(idx[t], ri), (t, idx[t], ri)
            assert orc.rel_l2(wgt[t], rw) < TOL
            assert orc.rel_l2(out[t], ref) < TOL, (t, orc.rel_l2(out[t], ref))
        # a second call with the same inputs gives the same bits (no state left behind)
        out2, idx2, _ = moe_dev(gpu, layer, xs)
        assert np.array_equal(out2.view(np.uint32), out.view(np.uint32)) and np.array_equal(idx2, idx)
    finally:
        layer.drop(gpu)


def test_moe_ffn_dev_beyond_one_route_launch(gpu, orc):
    """600 tokens at top-8: the call runs as blocks of 512 tokens (4096 route
    slots) and one of 88; tokens on both sides of the block edge and a sample
    of the rest match the CPU (indices identical, weights and outputs within
    1e-5)."""
    n_exp, h, ffn, top_k, n = 16, 512, 256, 8, 600
    layer = Layer(orc, n_exp, h, ffn, top_k, 47)
    layer.upload(gpu)
    try:
        xs = orc.normal(n * h, 1.0, 76, 1)
        out, idx, wgt = moe_dev(gpu, layer, xs)
        for t in sorted(set(range(0, n, 23)) | {510, 511, 512, 513, n - 1}):
            ref, ri, rw = layer.cpu(orc, xs[t * h:(t + 1) * h])
            assert np.array_equal(idx[t], ri), (t, idx[t], ri)
            assert orc.rel_l2(wgt[t], rw) < TOL, t
            assert orc.rel_l2(out[t], ref) < TOL, (t, orc.rel_l2(out[t], ref))
    finally:
        layer.drop(gpu)


@pytest.mark.parametrize("n_exp", [64, 128, 200])
def test_moe_ffn_dev_single_token_ties(gpu, orc, n_exp):
    """One token whose router gives two groups of equal logits, the second
    straddling the top-k cut: the expert kernels rank the token themselves
    (8, 4 and 2 counting threads per expert at these widths) and must keep
    the stable order of topk_softmax, lower index first, and the oracle's
    weights and output."""
    h, ffn, top_k = 512, 256, 6
    layer = Layer(orc, n_exp, h, ffn, top_k, 77 + n_exp)
    x = orc.normal(h, 1.0, 5, n_exp)
    r = layer.router.reshape(n_exp, h)
    first, second = [5, 33, n_exp - 1], [2, 9, 20, 47, n_exp - 2]
    for e in first:
        r[e] = np.float32(0.012) * x
    for e in second:
        r[e] = np.float32(0.008) * x
    layer.upload(gpu)
    try:
        out, idx, wgt = moe_dev(gpu, layer, x)
        ref, ri, rw = layer.cpu(orc, x)
        assert list(ri) == first + second[:3]
        assert np.array_equal(idx[0], ri), (idx[0], ri)
        assert orc.rel_l2(wgt[0], rw) < TOL
        assert orc.rel_l2(out[0], ref) < TOL
    finally:
        layer.drop(gpu)


def test_experts_block_host_path(gpu, orc):
    """expertos_bloque: the caller groups tokens by expert (here from the CPU
    routing); suma = weighted sum over the resolved experts in ranking order."""
    n_exp, h, ffn, top_k, n = 10, 512, 256, 3, 6
    layer = Layer(orc, n_exp, h, ffn, top_k, 91)
    xs = orc.normal(n * h, 1.0, 92, n)
    refs, idxs, ws = zip(*[layer.cpu(orc, xs[t * h:(t + 1) * h]) for t in range(n)])
    pesos = np.concatenate(ws).astype(np.float32)
    exps = []
    for e in range(n_exp):
        tok = [t for t in range(n) for j in range(top_k) if idxs[t][j] == e]
        dst = [t * top_k + j for t in range(n) for j in range(top_k) if idxs[t][j] == e]
        if tok:
            exps.append({"claves": layer.keys(e), "w": [layer.gate[e], layer.up[e], layer.down[e]],
                         "dtype": [Q4K, Q4K, Q4K], "tokens": tok, "destinos": dst})
    suma = np.zeros(n * h, np.float32)
    hecho = [False] * len(exps)
    try:
        assert gpu.expertos_bloque(xs, n, h, ffn, top_k, pesos, exps, suma, hecho) == 1, gpu.last_error()
        assert all(hecho)
        for t in range(n):
            assert orc.rel_l2(suma[t * h:(t + 1) * h], refs[t]) < TOL
    finally:
        layer.drop(gpu)


def test_experts_block_declines_shared_and_sums_the_rest(gpu, orc):
    """A shared expert is left to the caller (hecho false); the sum holds the
    other experts only."""
    n_exp, h, ffn, top_k, n = 4, 256, 256, 2, 2
    layer = Layer(orc, n_exp, h, ffn, top_k, 93)
    xs = orc.normal(n * h, 1.0, 94, n)
    refs, idxs, ws = zip(*[layer.cpu(orc, xs[t * h:(t + 1) * h]) for t in range(n)])
    pesos = np.concatenate(ws).astype(np.float32)
    exps = []
    for e in range(n_exp):
        tok = [t for t in range(n) for j in range(top_k) if idxs[t][j] == e]
        dst = [t * top_k + j for t in range(n) for j in range(top_k) if idxs[t][j] == e]
        if tok:
            exps.append({"claves": layer.keys(e), "w": [layer.gate[e], layer.up[e], layer.down[e]],
                         "dtype": [Q4K, Q4K, Q4K], "tokens": tok, "destinos": dst, "compartido": False})
    exps[0]["compartido"] = True
    suma = np.zeros(n * h, np.float32)
    hecho = [False] * len(exps)
    try:
        assert gpu.expertos_bloque(xs, n, h, ffn, top_k, pesos, exps, suma, hecho) == 0
        assert hecho[0] is False and all(hecho[1:])
        # add the shared-flagged expert's part on the CPU and compare with the full sum
        e0 = [e for e in range(n_exp) if layer.keys(e) == exps[0]["claves"]][0]
        full = suma.copy()
        for t, s in zip(exps[0]["tokens"], exps[0]["destinos"]):
            g = orc.matvec(Q4K, layer.gate[e0], ffn, h, xs[t * h:(t + 1) * h])
            u = orc.matvec(Q4K, layer.up[e0], ffn, h, xs[t * h:(t + 1) * h])
            act = (g / (1.0 + np.exp(-g.astype(np.float64))) * u).astype(np.float32)
            full[t * h:(t + 1) * h] += pesos[s] * orc.matvec(Q4K, layer.down[e0], h, ffn, act)
        for t in range(n):
            assert orc.rel_l2(full[t * h:(t + 1) * h], refs[t]) < 1e-5
    finally:
        layer.drop(gpu)


@pytest.mark.parametrize("n", [5, 20])
def test_moe_shared_joins_the_experts_block_sum(gpu, orc, n):
    """moe_compartido (gpu.rs:518-534): the shared expert of the block, c_t =
    down(silu(gate x_t) * up x_t) * sigmoid(x_t . pg_w), stays on the device
    and the next expertos_bloque for the same block adds it to its sum: per
    token the ranked experts (oracle or_moe_ffn) plus the oracle's shared
    expert (or_moe_shared), within 1e-5.  The shared expert is consumed: a
    second expertos_bloque sums the ranked experts alone.  One computed for a
    block of another size makes expertos_bloque fail.  (20 tokens take the
    shared matrices through the matrix-core matmul.)"""
    n_exp, h, ffn, top_k = 8, 512, 256, 2
    layer = Layer(orc, n_exp, h, ffn, top_k, 95 + n)
    sg = [orc.synth(Q4K, ffn, h, 96 + n, 1), orc.synth(Q4K, ffn, h, 96 + n, 2), orc.synth(Q4K, h, ffn, 96 + n, 3)]
    skeys = [f"shared{n}.gate", f"shared{n}.up", f"shared{n}.down"]
    pg = orc.normal(h, 0.05, 97 + n, 1)
    xs = orc.normal(n * h, 1.0, 98 + n, 1)
    refs, idxs, ws = zip(*[layer.cpu(orc, xs[t * h:(t + 1) * h]) for t in range(n)])
    shared = orc.moe_shared(pg, h, ffn, sg[0], sg[1], sg[2], Q4K, Q4K, xs, n)
    pesos = np.concatenate(ws).astype(np.float32)
    exps = []
    for e in range(n_exp):
        tok = [t for t in range(n) for j in range(top_k) if idxs[t][j] == e]
        dst = [t * top_k + j for t in range(n) for j in range(top_k) if idxs[t][j] == e]
        if tok:
            exps.append({"claves": layer.keys(e), "w": [layer.gate[e], layer.up[e], layer.down[e]],
                         "dtype": [Q4K, Q4K, Q4K], "tokens": tok, "destinos": dst})
    print(f"shared expert n={n}", flush=True)
    try:
        assert gpu.moe_compartido(skeys, sg, [Q4K] * 3, pg, xs, n, h, ffn), gpu.last_error()
        suma = np.zeros(n * h, np.float32)
        hecho = [False] * len(exps)
        assert gpu.expertos_bloque(xs, n, h, ffn, top_k, pesos, exps, suma, hecho) == 1, gpu.last_error()
        for t in range(n):
            want = refs[t] + shared[t * h:(t + 1) * h]
            assert orc.rel_l2(suma[t * h:(t + 1) * h], want) < TOL, (t, orc.rel_l2(suma[t * h:(t + 1) * h], want))
        # consumed: the next block sums the ranked experts alone
        suma2 = np.zeros(n * h, np.float32)
        assert gpu.expertos_bloque(xs, n, h, ffn, top_k, pesos, exps, suma2, [False] * len(exps)) == 1
        for t in range(n):
            assert orc.rel_l2(suma2[t * h:(t + 1) * h], refs[t]) < TOL
        # computed for a block of another size: the sum cannot hold it
        assert gpu.moe_compartido(skeys, None, [Q4K] * 3, pg, xs[:h], 1, h, ffn)
        with pytest.raises(RuntimeError, match="another block"):
            gpu.expertos_bloque(xs, n, h, ffn, top_k, pesos, exps, suma2, [False] * len(exps))
    finally:
        layer.drop(gpu)
        for k in skeys:
            gpu.weight_drop(k)


def test_moe_graph_survives_scratch_growth(gpu, orc):
    """A graph holding a single-token moe_ffn_dev keeps the scratch it was
    captured with: a later call that outgrows the MoE scratch slots (a
    256-token router call) must leave that memory alive, so replaying the
    graph gives the eager call's bits.  A call whose scratch would have to
    grow inside the capture is declined instead of allocating there."""
    n_exp, h, ffn, top_k = 128, 2048, 768, 8
    layer = Layer(orc, n_exp, h, ffn, top_k, 61)
    layer.upload(gpu)
    x = orc.normal(h, 1.0, 62, 1)
    xd = gpu.dev_alloc(x.nbytes)
    od = gpu.dev_alloc(h * 4)
    gid = None
    try:
        gpu.h2d(xd, x)
        assert gpu.moe_ffn_dev(layer.name, xd, 1, od), gpu.last_error()
        gpu.sync()
        eager = gpu.d2h(od, (h,), np.float32)
        gpu.graph_begin()
        try:
            ok = gpu.moe_ffn_dev(layer.name, xd, 1, od)
        finally:
            gid = gpu.graph_end()
        assert ok, gpu.last_error()
        # outgrow the MoE scratch slots while the graph exists
        n = 256
        w = orc.normal(n_exp * h, 0.02, 63, 1)
        xs = orc.normal(n * h, 1.0, 64, 1)
        idx = np.zeros(n * top_k, np.int32)
        wgt = np.zeros(n * top_k, np.float32)
        assert gpu.router_topk("router.growth", w, xs, n, h, n_exp, top_k, idx, wgt), gpu.last_error()
        for rep in range(3):
            gpu.h2d(od, np.zeros(h, np.float32))
            gpu.graph_launch(gid)
            gpu.sync()
            got = gpu.d2h(od, (h,), np.float32)
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), rep
        gpu.graph_destroy(gid)
        gid = None
        # a capture whose call would need more scratch than the slots hold is declined
        big = 500
        xb = gpu.dev_alloc(big * h * 4)
        ob = gpu.dev_alloc(big * h * 4)
        try:
            gpu.graph_begin()
            try:
                ok = gpu.moe_ffn_dev(layer.name, xb, big, ob)
            finally:
                g2 = gpu.graph_end()
                gpu.graph_destroy(g2)
            assert ok is False
            assert "inside graph capture" in gpu.last_error()
        finally:
            gpu.dev_free(xb)
            gpu.dev_free(ob)
    finally:
        if gid is not None:
            gpu.graph_destroy(gid)
        gpu.dev_free(xd)
        gpu.dev_free(od)
        layer.drop(gpu)


def test_moe_nan_token_at_batch_32(gpu, orc):
    """A token whose x holds a NaN has NaN logits: it ranks no expert, its
    eight slots name expert 0 with weight 0 (the matrix-core kernels then find
    all of them in expert 0's scan) and its output is NaN, as soso's NaN
    weights make it.  The other tokens keep the oracle's routing and outputs."""
    layer = Layer(orc, 16, 512, 256, 8, 91, Q4K)
    layer.upload(gpu)
    try:
        n, h = 32, layer.h
        xs = orc.normal(n * h, 1.0, 92, n).copy()
        xs[5 * h + 17] = np.nan
        out, idx, wgt = moe_dev(gpu, layer, xs)
        assert np.all(np.isnan(out[5]))
        assert np.array_equal(idx[5], np.zeros(8, np.int32)) and np.all(wgt[5] == 0.0), (idx[5], wgt[5])
        for t in range(n):
            if t == 5:
                continue
            ref, ri, rw = layer.cpu(orc, xs[t * h:(t + 1) * h])
            assert np.array_equal(idx[t], ri), (t, idx[t], ri)
            assert orc.rel_l2(wgt[t], rw) < TOL
            assert orc.rel_l2(out[t], ref) < TOL, (t, orc.rel_l2(out[t], ref))
    finally:
        layer.drop(gpu)
