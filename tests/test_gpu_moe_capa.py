"""GpuDispatch::moe_capa through the C ABI: one Qwen3-MoE-style layer at a
time (GQA attention with QK norm, NeoX RoPE and the f16 KV cache the device
keeps, then the router, top-k and the chosen experts), chained across layers
with continuar / encadenar, as capa_moe_en_gpu drives it
(crates/soso-llm-core/src/moe_gpu.rs:37-269; MoeCapa and its bookkeeping
methods, crates/soso-llm-core/src/gpu.rs:294-335, 380-426).

The CPU side is the oracle's composition of the same layers (the decode
tests' Model.cpu_step with MoE FFNs).  Bar: each layer's routing of each
token identical (the same experts in the same order, weights within relative
L2 1e-5), each token's hidden state within relative L2 1e-5, and the KV rows the device appended as close to the CPU's
f32 rows as soso's f32_to_f16 of those rows is, to 1e-5 relative L2, with
more than 95 % of the f16 values equal to it (where the two f32 rows, equal
to ~1e-6, straddle an f16 rounding point, or where a small element of a
row carries that absolute error, they differ).  Such differences move a
short context's attention by ~1e-5 on their own (one f16 step is 2^-11 of
the value), so the CPU attends to the device's f16 rows (the history both
sides then share) and its own rows are compared separately, as the decode
tests compare them.
"""
import numpy as np
import pytest

from test_gpu_decode import HD, Model, MoeFfn, Q4K, head_major

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture
def gpu():
    """A handle of its own per test: a discarded layer stays discarded for
    the handle's lifetime (moe_descartar), and the per-layer steps and KV
    caches go with the handle."""
    from soso_amd.dispatch import HipGpu
    g = HipGpu(0)
    yield g
    g.close()


class Stack:
    """A 2-layer model whose layers are both MoE layers, its weights made
    resident under soso's tensor names (gemma_subir)."""

    def __init__(self, orc, gpu, seed, L=2, H=1024, nh=8, nkv=2, n_exp=16, ffn=512, top_k=4, V=64):
        self.m = Model(orc, L, H, nh, nkv, 256, V, seed, qk_norm=True, neox=True)
        self.moe = {l: MoeFfn(orc, n_exp, H, ffn, top_k, seed + 1 + l) for l in range(L)}
        self.L, self.H, self.nh, self.nkv, self.n_exp, self.ffn, self.top_k = L, H, nh, nkv, n_exp, ffn, top_k
        self.uploaded = []
        for l in range(L):
            lw, p = self.m.layers[l], f"L{l:02}"
            for nm, key in (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output")):
                dt, r, c = self.m.shapes(nm)
                self.put(gpu, f"{p}.{key}", lw[nm], dt, r, c)
            f = self.moe[l]
            for e in range(n_exp):
                for nm, w, r, c in (("ffn_gate", f.gate[e], ffn, H), ("ffn_up", f.up[e], ffn, H),
                                    ("ffn_down", f.down[e], H, ffn)):
                    self.put(gpu, f"{p}.E{e:02}.{nm}", w, Q4K, r, c)

    def put(self, gpu, key, w, dtype, rows, cols):
        assert not gpu.gemma_residente(key)
        assert gpu.gemma_subir(key, np.ascontiguousarray(w).view(np.uint8), dtype, rows, cols), gpu.last_error()
        assert gpu.gemma_residente(key)
        self.uploaded.append(key)

    def capa(self, l, pos0, n, ctx, theta, eps, continuar, encadenar, normas):
        lw, p = self.m.layers[l], f"L{l:02}"
        c = dict(layer=l, pos0=pos0, n=n, hidden_dim=self.H, heads=self.nh, kv_heads=self.nkv, head_dim=HD,
                 ffn=self.ffn, n_exp=self.n_exp, top_k=self.top_k, ventana=0, ctx_max=ctx, eps=eps, theta=theta,
                 escala=np.float32(1.0) / np.sqrt(np.float32(HD)), rope_mscale=1.0, qk_norm=1,
                 continuar=int(continuar), encadenar=int(encadenar), key_q=f"{p}.attn_q", key_k=f"{p}.attn_k",
                 key_v=f"{p}.attn_v", key_o=f"{p}.attn_output", prefix=p)
        if normas:
            c.update(attn_norm=lw["attn_norm"], q_norm=lw["q_norm"], k_norm=lw["k_norm"], ffn_norm=lw["ffn_norm"],
                     router=self.moe[l].router)
        return c

    def drop(self, gpu):
        for k in self.uploaded:
            gpu.weight_drop(k)


def kv_rows_f16(gpu, layer, nkv, ctx, n):
    """The layer's device K and V rows 0..n-1, position-major f16 bits."""
    kd, vd = gpu.moe_capa_kv_dev(layer)
    out = []
    for d in (kd, vd):
        hm = gpu.d2h(d, (nkv, ctx, HD), np.uint16)
        out.append(np.ascontiguousarray(hm[:, :n, :].transpose(1, 0, 2)).reshape(n, nkv * HD))
    return out


def test_moe_capa_chained_layers_match_cpu(gpu, orc):
    """Five tokens, each through layer 0 (output left pending: encadenar) and
    layer 1 (input the pending output: continuar), the norms and router sent
    on each layer's first call only: routing identical (weights within
    1e-5), hidden within 1e-5 (the CPU attending
    to the device's f16 rows), the KV rows as close to the CPU's as soso's
    f16 rounding of them.  Then the same tokens with
    every layer's output brought down (no chaining) give the same bits, and a
    pending output comes down through moe_volcar."""
    theta, eps, ctx, T = 1000000.0, 1e-6, 16, 5
    st = Stack(orc, gpu, 170)
    m = st.m
    kc = np.zeros((st.L, ctx, m.kvd), np.float32)
    vc = np.zeros((st.L, ctx, m.kvd), np.float32)
    xs = [orc.normal(st.H, 1.0, 171, t) for t in range(T)]
    outs = []
    cpu_k = {l: [] for l in range(st.L)}
    cpu_v = {l: [] for l in range(st.L)}
    try:
        assert gpu.moe_puede(0) and not gpu.moe_lista(0)
        for t in range(T):
            hid = xs[t].copy()
            assert gpu.moe_capa(st.capa(0, t, 1, ctx, theta, eps, False, True, t == 0), hid), gpu.last_error()
            assert gpu.moe_pendiente(0, t, 1) and not gpu.moe_pendiente(1, t, 1)
            assert np.array_equal(hid, xs[t])  # encadenar: hidden untouched
            assert gpu.moe_capa(st.capa(1, t, 1, ctx, theta, eps, True, False, t == 0), hid), gpu.last_error()
            assert not gpu.moe_pendiente(0, t, 1) and not gpu.moe_pendiente(1, t, 1)
            routing = [gpu.moe_capa_routing(l, st.top_k) for l in range(st.L)]
            rows = {}
            for l in range(st.L):
                kg, vg = kv_rows_f16(gpu, l, st.nkv, ctx, t + 1)
                rows[l] = (orc.f16_to_f32(kg[t]), orc.f16_to_f32(vg[t]))
            m.cpu_step(orc, xs[t], kc, vc, t, theta, eps, kv_f16=True, moe=st.moe, kv_rows=rows)
            for l in range(st.L):
                cpu_k[l].append(m.last_kv[0][l])
                cpu_v[l].append(m.last_kv[1][l])
            for l in range(st.L):
                (gi, gw), (ri, rw) = routing[l], m.routing[l]
                assert np.array_equal(gi, ri), (t, l, gi, ri)
                assert orc.rel_l2(gw, rw) < TOL, (t, l, gw, rw)
            err = orc.rel_l2(hid, m.last_hidden)
            print(f"moe_capa token {t}: hidden rel_l2 {err:.3e}", flush=True)
            assert err < TOL, (t, err)
            outs.append(hid)
            assert gpu.moe_lista(0) and gpu.moe_lista(1)
        # the device's KV rows against soso's f16 rounding of the CPU's f32 rows
        for l in range(st.L):
            kg, vg = kv_rows_f16(gpu, l, st.nkv, ctx, T)
            for g, ref in ((kg, np.stack(cpu_k[l])), (vg, np.stack(cpu_v[l]))):
                want = orc.f32_to_f16(ref.ravel()).reshape(ref.shape)
                e_gpu = orc.rel_l2(orc.f16_to_f32(g), ref)
                e_orc = orc.rel_l2(orc.f16_to_f32(want), ref)
                assert e_gpu <= e_orc + 1e-5, (l, e_gpu, e_orc)
                assert (g == want).mean() > 0.95, (l, float((g == want).mean()))
        # the same tokens again from position 0, every output brought down
        for t in range(T):
            hid = xs[t].copy()
            assert gpu.moe_capa(st.capa(0, t, 1, ctx, theta, eps, False, False, False), hid)
            assert gpu.moe_capa(st.capa(1, t, 1, ctx, theta, eps, False, False, False), hid)
            assert np.array_equal(hid.view(np.uint32), outs[t].view(np.uint32)), t
        # a pending output comes down through moe_volcar
        hid = xs[0].copy()
        assert gpu.moe_capa(st.capa(0, 0, 1, ctx, theta, eps, False, True, False), hid)
        down = np.zeros(st.H, np.float32)
        gpu.moe_volcar(down)
        assert not gpu.moe_pendiente(0, 0, 1)
        ref = xs[0].copy()
        assert gpu.moe_capa(st.capa(0, 0, 1, ctx, theta, eps, False, False, False), ref)
        assert np.array_equal(down.view(np.uint32), ref.view(np.uint32))
    finally:
        st.drop(gpu)


def test_moe_capa_block_of_tokens_equals_one_at_a_time(gpu, orc):
    """A block of n = 4 tokens (pos0 = 0) chained through both layers gives
    the bits of the same tokens one call at a time (the layer takes them in
    order, each attending to the ones before it)."""
    theta, eps, ctx, T = 500000.0, 1e-5, 16, 4
    st = Stack(orc, gpu, 180, n_exp=8, top_k=2)
    xs = np.stack([orc.normal(st.H, 1.0, 181, t) for t in range(T)])
    try:
        one = []
        for t in range(T):
            hid = xs[t].copy()
            assert gpu.moe_capa(st.capa(0, t, 1, ctx, theta, eps, False, True, t == 0), hid), gpu.last_error()
            assert gpu.moe_capa(st.capa(1, t, 1, ctx, theta, eps, True, False, t == 0), hid), gpu.last_error()
            one.append(hid)
        blk = xs.copy()
        assert gpu.moe_capa(st.capa(0, 0, T, ctx, theta, eps, False, True, False), blk), gpu.last_error()
        assert gpu.moe_pendiente(0, 0, T)
        assert gpu.moe_capa(st.capa(1, 0, T, ctx, theta, eps, True, False, False), blk), gpu.last_error()
        assert np.array_equal(blk.view(np.uint32), np.stack(one).view(np.uint32))
    finally:
        st.drop(gpu)


def test_moe_capa_declines_what_it_does_not_run(gpu, orc):
    """Declined (the CPU keeps the layer): a sliding window, YaRN, another
    attention scale, positions beyond ctx_max, and a position whose earlier
    ones this layer's device KV does not hold; moe_descartar makes moe_puede
    false for good."""
    theta, eps, ctx = 500000.0, 1e-5, 16
    st = Stack(orc, gpu, 190, L=1, n_exp=8, top_k=2)
    x = orc.normal(st.H, 1.0, 191, 1)
    try:
        for change in (dict(ventana=8), dict(rope_mscale=1.1), dict(escala=0.1), dict(pos0=15, n=2)):
            c = st.capa(0, 0, 1, ctx, theta, eps, False, False, True)
            c.update(change)
            hid = x.copy()
            assert not gpu.moe_capa(c, hid), change
            assert np.array_equal(hid, x)
        # position 3 before 0..2 were computed here
        assert not gpu.moe_capa(st.capa(0, 3, 1, ctx, theta, eps, False, False, True), x.copy())
        assert gpu.moe_capa(st.capa(0, 0, 1, ctx, theta, eps, False, False, True), x.copy()), gpu.last_error()
        assert gpu.moe_capa(st.capa(0, 1, 1, ctx, theta, eps, False, False, False), x.copy())
        assert gpu.moe_puede(0)
        gpu.moe_descartar(0)
        assert not gpu.moe_puede(0) and not gpu.moe_lista(0)
        assert not gpu.moe_capa(st.capa(0, 2, 1, ctx, theta, eps, False, False, True), x.copy())
    finally:
        st.drop(gpu)
