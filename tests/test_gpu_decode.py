"""GPU parity of the device-resident dense decode step (configs[4]'s path).

Reference: LayerExecutor::forward_layer, dense GQA branch
(crates/soso-llm-core/src/layer.rs:1092-1389) -- rmsnorm (gemm.rs:93-100),
q/k/v matvecs, rope_cabezas non-NeoX (gemm.rs:1452-1490), KV append, decode
attention, o-proj + residual, ffn_norm, gate/up, swiglu (gemm.rs:210-226),
down + residual -- then Runtime::logits_gpu + argmax (runtime.rs:1976-2028,
last maximum wins).  The CPU side composes the oracle's restatements of those
functions; the KV cache is f32 on both sides.

Weights: f32 ~ N(0, 0.05) quantized with the reference quantizers
(quant.rs restated in the oracle): Q4_K projections, Q8_0 head (the path soso
runs after converting Q6_K heads to Q8_0, gguf2som/src/lib.rs:1592-1609).

Bar: logits within relative L2 1e-5, the greedy token identical; K/V rows
written at `pos` within relative L2 1e-5 (f32).  In f16 the GPU's row, widened,
must be as close to the CPU's f32 row as the oracle's rounding of that row is,
within the same 1e-5 (the f32 values feeding the rounding differ slightly
between CPU and GPU, so an element next to a rounding midpoint, or a small one
whose f16 step is finer than that difference, may land on a neighbour); most
elements must match bit for bit.  The rounding itself is checked bit for bit
on crafted inputs by test_kv_upload_rounds_like_soso.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4K, Q8, F32, Q6K = 3, 2, 1, 13
HD = 128


def head_major(kv, nkv):
    """[ctx][nkv*HD] (position-major, as the CPU side keeps it) -> [nkv][ctx][HD]."""
    ctx = kv.shape[0]
    return np.ascontiguousarray(kv.reshape(ctx, nkv, HD).transpose(1, 0, 2))


def quant(orc, dtype, w):
    w = np.ascontiguousarray(w, np.float32).ravel()
    rb = orc.row_bytes(dtype, 256 if dtype == Q4K else 32)
    out = np.zeros(w.size // (256 if dtype == Q4K else 32) * rb, np.uint8)
    fn = orc.lib().or_quantize_q4_k if dtype == Q4K else orc.lib().or_quantize_q8_0
    fn(w.ctypes.data, w.size, out.ctypes.data)
    return out


def q6k_small(orc, rows, cols, seed, stream):
    """Seeded Q6_K blocks (the oracle's generator) with the f16 block scale d
    set to 2^-12, so the weights stay within about +-1 (the generator's own d
    is |N(0, 0.01)|, sized for a lone matvec, not a stack of layers)."""
    w = orc.synth(Q6K, rows, cols, seed, stream).reshape(-1, 210).copy()
    w[:, 208:210] = np.frombuffer(np.float16(2.0 ** -12).tobytes(), np.uint8)
    return w.ravel()


class Model:
    """A seeded dense decoder.  `dt` gives a format per role (q, k, v, o,
    gate, up, down, head; Q4_K and the Q8_0 head by default): Q4_K and Q8_0
    weights are N(0, 0.05) through the reference quantizers, Q6_K ones the
    generator's blocks at a small scale."""

    ROLES = ("q", "k", "v", "o", "gate", "up", "down")
    qk_norm = neox = False  # also for instances built without __init__

    def __init__(self, orc, L, H, nh, nkv, F, V, seed, dt=None, qk_norm=False, neox=False):
        self.L, self.H, self.nh, self.nkv, self.F, self.V = L, H, nh, nkv, F, V
        self.qd, self.kvd = nh * HD, nkv * HD
        self.qk_norm, self.neox = qk_norm, neox
        self.dt = {r: Q4K for r in self.ROLES}
        self.dt["head"] = Q8
        self.dt.update(dt or {})
        tag = "" if dt is None else "." + ".".join(f"{k}{v}" for k, v in sorted(dt.items()))
        tag += (".qkn" if qk_norm else "") + (".neox" if neox else "")
        self.name = f"dec{seed}.{L}.{H}.{nh}.{nkv}.{F}.{V}{tag}"
        self.layers = []
        s = 0

        def mat(dtype, rows, cols):
            nonlocal s
            s += 1
            if dtype == Q6K:
                return q6k_small(orc, rows, cols, seed, s)
            return quant(orc, dtype, orc.normal(rows * cols, 0.05, seed, s))
        for l in range(L):
            s += 2
            lw = {"attn_norm": (1.0 + orc.normal(H, 0.1, seed, s - 1)).astype(np.float32),
                  "ffn_norm": (1.0 + orc.normal(H, 0.1, seed, s)).astype(np.float32)}
            for r in self.ROLES:
                _, rows, cols = self.shapes(r)
                lw[r] = mat(self.dt[r], rows, cols)
            if qk_norm:
                # attn_q_norm / attn_k_norm: F32 [head_dim]
                lw["q_norm"] = (1.0 + orc.normal(HD, 0.1, seed, 5000 + 2 * l)).astype(np.float32)
                lw["k_norm"] = (1.0 + orc.normal(HD, 0.1, seed, 5001 + 2 * l)).astype(np.float32)
            self.layers.append(lw)
        self.out_norm = (1.0 + orc.normal(H, 0.1, seed, 9000)).astype(np.float32)
        self.head_dtype = self.dt["head"]
        self.head = mat(self.head_dtype, V, H)

    def shapes(self, name):
        H, F, qd, kvd = self.H, self.F, self.qd, self.kvd
        dt = getattr(self, "dt", None) or {}
        rc = {"q": (qd, H), "k": (kvd, H), "v": (kvd, H), "o": (H, qd), "gate": (F, H), "up": (F, H), "down": (H, F),
              "attn_norm": (1, H), "ffn_norm": (1, H), "q_norm": (1, HD), "k_norm": (1, HD)}[name]
        return (F32 if name.endswith("norm") else dt.get(name, Q4K),) + rc

    def upload(self, gpu):
        def put(key, arr, dtype, rows, cols):
            b = np.ascontiguousarray(arr).view(np.uint8)
            d = gpu.dev_alloc(b.size)
            try:
                gpu.h2d(d, b)
                gpu.weight_from_dev(key, d, b.size, dtype, rows, cols)
            finally:
                gpu.dev_free(d)
        keys = []
        for l, lw in enumerate(self.layers):
            for nm in ("attn_norm", "q", "k", "v", "o", "ffn_norm", "gate", "up", "down") + (
                    ("q_norm", "k_norm") if self.qk_norm else ()):
                k = f"{self.name}.L{l}.{nm}"
                put(k, lw[nm], *self.shapes(nm))
                keys.append(k)
        put(self.name + ".out_norm", self.out_norm, F32, 1, self.H)
        put(self.name + ".head", self.head, self.head_dtype, self.V, self.H)
        keys += [self.name + ".out_norm", self.name + ".head"]
        self.keys = keys
        return keys

    def cpu_step(self, orc, x, kcache, vcache, pos, theta, eps, kv_f16=False, moe=None, kv_rows=None):
        """The layer stack on the CPU; kcache/vcache [L][ctx][kvd] get row pos
        (rounded through soso's f16 when kv_f16, as KvCache::append stores it).
        moe: {layer: MoeFfn} -- those layers' FFN is the MoE FFN (forward_moe_ffn,
        layer.rs:1938-1975: rmsnorm, or_moe_ffn, residual); their routing is
        kept in self.routing[layer].  kv_rows: {layer: (k, v)} rows to store at
        pos instead of the CPU's own (the f32 rows it computed are still kept
        in self.last_kv)."""
        L_ = orc.lib()
        h = x.astype(np.float32).copy()
        new_k, new_v = [], []
        self.last_kv = (new_k, new_v)  # the f32 rows appended at pos, per layer
        self.routing = {}
        for l, lw in enumerate(self.layers):
            xn = h.copy()
            L_.or_rmsnorm(xn.ctypes.data, lw["attn_norm"].ctypes.data, self.H, np.float32(eps))
            dt = getattr(self, "dt", None) or {}
            d = lambda r: dt.get(r, Q4K)
            q = orc.matvec(d("q"), lw["q"], self.qd, self.H, xn)
            k = orc.matvec(d("k"), lw["k"], self.kvd, self.H, xn)
            v = orc.matvec(d("v"), lw["v"], self.kvd, self.H, xn)
            if self.qk_norm:
                # per head, before RoPE (layer.rs:1164-1180)
                for vec, n, w in ((q, self.nh, lw["q_norm"]), (k, self.nkv, lw["k_norm"])):
                    for hh in range(n):
                        L_.or_rmsnorm(vec[hh * HD:].ctypes.data, w.ctypes.data, HD, np.float32(eps))
            neox = 1 if self.neox else 0
            L_.or_rope_heads(q.ctypes.data, self.nh, HD, pos, np.float32(theta), neox)
            L_.or_rope_heads(k.ctypes.data, self.nkv, HD, pos, np.float32(theta), neox)
            if kv_rows and l in kv_rows:
                kcache[l, pos], vcache[l, pos] = kv_rows[l]
            else:
                kcache[l, pos] = orc.f16_to_f32(orc.f32_to_f16(k)) if kv_f16 else k
                vcache[l, pos] = orc.f16_to_f32(orc.f32_to_f16(v)) if kv_f16 else v
            new_k.append(k)
            new_v.append(v)
            att = np.zeros(self.qd, np.float32)
            Kc = np.ascontiguousarray(kcache[l, :pos + 1])
            Vc = np.ascontiguousarray(vcache[l, :pos + 1])
            g = self.nh // self.nkv
            for hh in range(self.nh):
                qh = np.ascontiguousarray(q[hh * HD:(hh + 1) * HD])
                out = np.zeros(HD, np.float32)
                L_.or_attention_f32(qh.ctypes.data, Kc.ctypes.data, Vc.ctypes.data, HD, self.kvd, hh // g, pos + 1,
                                    out.ctypes.data)
                att[hh * HD:(hh + 1) * HD] = out
            h = h + orc.matvec(d("o"), lw["o"], self.H, self.qd, att)
            xn = h.copy()
            L_.or_rmsnorm(xn.ctypes.data, lw["ffn_norm"].ctypes.data, self.H, np.float32(eps))
            if moe and l in moe:
                out, idx, w = moe[l].cpu(orc, xn)
                self.routing[l] = (idx, w)
                h = h + out
                continue
            gt = orc.matvec(d("gate"), lw["gate"], self.F, self.H, xn)
            up = orc.matvec(d("up"), lw["up"], self.F, self.H, xn)
            L_.or_swiglu(up.ctypes.data, gt.ctypes.data, self.F)
            h = orc.matvec(d("down"), lw["down"], self.H, self.F, up) + h
        self.last_hidden = h  # the stack's output, before the output norm
        xn = h.copy()
        L_.or_rmsnorm(xn.ctypes.data, self.out_norm.ctypes.data, self.H, np.float32(eps))
        logits = orc.matvec(self.head_dtype, self.head, self.V, self.H, xn)
        return logits, int(L_.or_argmax(logits.ctypes.data, logits.size))


def check_greedy(orc, token, logits, ref_token, ref_logits):
    """The greedy token: always the last maximum of the GPU's own logits
    (Runtime::argmax), and one of the reference logits within the parity
    tolerance of the reference maximum; equal to the reference token when the
    reference's top two are further apart than that tolerance (the gap is
    printed either way, so a run shows which case it checked)."""
    assert token == int(orc.lib().or_argmax(logits.ctypes.data, logits.size)), token
    top2 = np.sort(ref_logits)[-2:]
    gap = float(top2[1] - top2[0])
    tol = 1e-3 * max(1.0, abs(float(top2[1])))
    near = np.flatnonzero(ref_logits >= top2[1] - tol)
    print(f"greedy token: gpu {token} cpu {ref_token}, cpu top-2 gap {gap:.4g} (tolerance {tol:.3g}, "
          f"{near.size} candidate(s))", flush=True)
    assert token in near, (token, ref_token, gap)
    if gap > tol:
        assert token == ref_token, (token, ref_token)


@pytest.mark.parametrize("kv_f16", [0, 1])
@pytest.mark.parametrize("L,H,nh,nkv,F,V,prefill", [
    (2, 512, 4, 2, 1024, 1000, 100),   # GQA group 2, two attention chunks
    (1, 1024, 8, 2, 2048, 512, 200),   # GQA group 4 (the 8B's ratio)
])
def test_decode_step_matches_cpu(gpu, orc, L, H, nh, nkv, F, V, prefill, kv_f16):
    theta, eps, ctx = 500000.0, 1e-5, 256
    m = Model(orc, L, H, nh, nkv, F, V, 50 + L)
    m.upload(gpu)
    name = m.name + ".model"
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=theta, rms_eps=eps, kv_f16=kv_f16)
    print(f"decode step L={L} H={H} heads={nh}/{nkv} prefill={prefill} kv_f16={kv_f16}", flush=True)
    assert gpu.decode_create(name, cfg, m.keys), gpu.last_error()
    kc = np.zeros((L, ctx, m.kvd), np.float32)
    vc = np.zeros((L, ctx, m.kvd), np.float32)
    kvt, esz = (np.uint16, 2) if kv_f16 else (np.float32, 4)
    for l in range(L):
        kr = orc.normal(prefill * m.kvd, 1.0, 60 + l, 1).reshape(prefill, m.kvd)
        vr = orc.normal(prefill * m.kvd, 1.0, 60 + l, 2).reshape(prefill, m.kvd)
        # decode_subir_estado: position-major f32 rows, rounded by the library
        gpu.decode_kv_upload(name, l, 0, kr, vr, rows_f32=True)
        if kv_f16:
            kb, vb = orc.f32_to_f16(kr).reshape(kr.shape), orc.f32_to_f16(vr).reshape(vr.shape)
            kd, vd = gpu.decode_kv_dev(name, l)
            gk = gpu.d2h(kd, (nkv, ctx, HD), np.uint16)[:, :prefill].transpose(1, 0, 2).reshape(prefill, m.kvd)
            gv = gpu.d2h(vd, (nkv, ctx, HD), np.uint16)[:, :prefill].transpose(1, 0, 2).reshape(prefill, m.kvd)
            assert np.array_equal(gk, kb) and np.array_equal(gv, vb), "uploaded f16 rows differ from soso's rounding"
            kr, vr = orc.f16_to_f32(kb), orc.f16_to_f32(vb)
        else:
            kd, vd = gpu.decode_kv_dev(name, l)
            assert np.array_equal(gpu.d2h(kd, (nkv, ctx, HD), np.float32)[:, :prefill], head_major(kr, nkv)[:, :prefill])
        kc[l, :prefill] = kr
        vc[l, :prefill] = vr
    x = orc.normal(H, 1.0, 70, 1)
    xd = gpu.dev_alloc(H * 4)
    ld = gpu.dev_alloc(V * 4)
    td = gpu.dev_alloc(4)
    rd = gpu.dev_alloc(L * 2 * m.kvd * esz)
    try:
        gpu.h2d(xd, x)
        gpu.decode_step_dev(name, xd, prefill, ld, td, rd)
        gpu.sync()
        logits = gpu.d2h(ld, (V,), np.float32)
        token = int(gpu.d2h(td, (1,), np.uint32)[0])
        rows = gpu.d2h(rd, (L, 2, m.kvd), kvt)
        kgpu = [gpu.d2h(gpu.decode_kv_dev(name, l)[0], (nkv, ctx, HD), kvt)[:, prefill].ravel() for l in range(L)]
        vgpu = [gpu.d2h(gpu.decode_kv_dev(name, l)[1], (nkv, ctx, HD), kvt)[:, prefill].ravel() for l in range(L)]
        # the kv_rows copy (decode_token's layout) equals what went into the cache
        for l in range(L):
            assert np.array_equal(rows[l, 0], kgpu[l]) and np.array_equal(rows[l, 1], vgpu[l]), l
        ref_logits, ref_token = m.cpu_step(orc, x, kc, vc, prefill, theta, eps, kv_f16=bool(kv_f16))
        k32, v32 = m.last_kv
        for l in range(L):
            if kv_f16:
                # ref32: the CPU's f32 row before rounding (kc holds it rounded)
                for got, ref32 in ((kgpu[l], k32[l]), (vgpu[l], v32[l])):
                    want = orc.f32_to_f16(ref32)
                    e_gpu = orc.rel_l2(orc.f16_to_f32(got), ref32)
                    e_orc = orc.rel_l2(orc.f16_to_f32(want), ref32)
                    assert e_gpu <= e_orc + 1e-5, (l, e_gpu, e_orc)
                    assert (got == want).mean() > 0.95, (l, float((got == want).mean()))
            else:
                assert orc.rel_l2(kgpu[l], kc[l, prefill]) < 1e-5, l
                assert orc.rel_l2(vgpu[l], vc[l, prefill]) < 1e-5, l
        assert orc.rel_l2(logits, ref_logits) < 1e-5, orc.rel_l2(logits, ref_logits)
        check_greedy(orc, token, logits, ref_token, ref_logits)
        # a second step at pos + 1 sees the row written by the first
        gpu.decode_step_dev(name, xd, prefill + 1, ld, td)
        gpu.sync()
        logits2 = gpu.d2h(ld, (V,), np.float32)
        ref2, _ = m.cpu_step(orc, x, kc, vc, prefill + 1, theta, eps, kv_f16=bool(kv_f16))
        assert orc.rel_l2(logits2, ref2) < 1e-5
    finally:
        for p in (xd, ld, td, rd):
            gpu.dev_free(p)
        gpu.decode_destroy(name)
        for k in m.keys:
            gpu.weight_drop(k)


@pytest.mark.parametrize("dt,F", [
    # soso's converted models carry Q8_0 wherever the GGUF had Q6_K
    ({"q": Q8, "k": Q8, "v": Q8, "o": Q8, "gate": Q6K, "up": Q6K, "down": Q8, "head": Q4K}, 1024),
    # Q6_K down rows split over two wavefronts, Q6_K head
    ({"q": Q6K, "k": Q6K, "v": Q6K, "o": Q4K, "gate": Q8, "up": Q8, "down": Q6K, "head": Q6K}, 8192),
    # Q8_0 down rows split over four wavefronts
    ({"down": Q8}, 16384),
])
def test_decode_step_mixed_formats(gpu, orc, dt, F):
    """Every role of the step in every quantized format the library keeps:
    Q4_K, Q8_0 and Q6_K q/k/v, o, gate/up, down and head, including the
    down projection's split rows.  Same bar: logits within relative L2 1e-5
    of the oracle's composition, the greedy token checked."""
    L, H, nh, nkv, V, prefill, ctx, theta, eps = 2, 512, 4, 2, 777, 37, 64, 500000.0, 1e-5
    m = Model(orc, L, H, nh, nkv, F, V, 300 + F // 1024, dt=dt)
    m.upload(gpu)
    name = m.name + ".model"
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=theta, rms_eps=eps)
    print(f"decode step mixed formats {dt} F={F}", flush=True)
    assert gpu.decode_create(name, cfg, m.keys), gpu.last_error()
    kc = np.zeros((L, ctx, m.kvd), np.float32)
    vc = np.zeros((L, ctx, m.kvd), np.float32)
    xd, ld, td = gpu.dev_alloc(H * 4), gpu.dev_alloc(V * 4), gpu.dev_alloc(4)
    try:
        for l in range(L):
            kr = orc.normal(prefill * m.kvd, 1.0, 310 + l, 1).reshape(prefill, m.kvd)
            vr = orc.normal(prefill * m.kvd, 1.0, 310 + l, 2).reshape(prefill, m.kvd)
            gpu.decode_kv_upload(name, l, 0, kr, vr, rows_f32=True)
            kc[l, :prefill], vc[l, :prefill] = kr, vr
        x = orc.normal(H, 1.0, 320, 1)
        gpu.h2d(xd, x)
        assert gpu.decode_step_dev(name, xd, prefill, ld, td), gpu.last_error()
        gpu.sync()
        logits = gpu.d2h(ld, (V,), np.float32)
        token = int(gpu.d2h(td, (1,), np.uint32)[0])
        ref, ref_token = m.cpu_step(orc, x, kc, vc, prefill, theta, eps)
        assert orc.rel_l2(logits, ref) < 1e-5, orc.rel_l2(logits, ref)
        check_greedy(orc, token, logits, ref_token, ref)
    finally:
        for p in (xd, ld, td):
            gpu.dev_free(p)
        gpu.decode_destroy(name)
        for k in m.keys:
            gpu.weight_drop(k)


@pytest.mark.parametrize("case", ["qkv_dtypes_differ", "group_of_3", "narrow_hidden"])
def test_decode_create_declines_what_the_step_cannot_run(gpu, orc, case):
    """decode_create refuses, with the reason, every model its step could not
    run to the end: q/k/v in different formats (the fused copy holds one),
    three query heads per KV head (attention is built for 1, 2, 4 and 8),
    a hidden width under 512 columns.  No model is registered then."""
    H, nh, nkv, F, V = (256, 4, 2, 512, 64) if case == "narrow_hidden" else (512, 6 if case == "group_of_3" else 4,
                                                                             2, 512, 64)
    dt = {"k": Q8} if case == "qkv_dtypes_differ" else None
    m = Model(orc, 1, H, nh, nkv, F, V, 330, dt=dt)
    m.upload(gpu)
    name = m.name + ".declined"
    cfg = dict(n_layers=1, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=16,
               rope_theta=1e4, rms_eps=1e-5)
    try:
        assert gpu.decode_create(name, cfg, m.keys) is False
        why = gpu.last_error()
        print(f"declined: {why}", flush=True)
        assert {"qkv_dtypes_differ": "dtypes differ", "group_of_3": "per KV head",
                "narrow_hidden": "narrower than 512"}[case] in why, why
        xd = gpu.dev_alloc(H * 4)
        try:
            assert gpu.decode_step_dev(name, xd, 0) is False  # nothing was registered
        finally:
            gpu.dev_free(xd)
    finally:
        for k in m.keys:
            gpu.weight_drop(k)


@pytest.mark.parametrize("dt", [
    {"q": Q8, "k": Q8, "v": Q8, "down": Q8, "head": Q8},
    {"q": Q6K, "k": Q6K, "v": Q6K, "down": Q6K, "head": Q6K},
    {"head": Q4K},
])
def test_decode_step_segmented_down(gpu, orc, dt):
    """Hidden 3072, FFN 9216: the width at which the step runs each down
    projection as four column segments whose partials the next layer's q/k/v
    staging (and, after the last layer, the head's) sums with the residual.
    Every format takes both sides of that hand-over here (the 8B tests cover
    Q4_K at 4096 x 14336).  Same bar: logits within relative L2 1e-5 of the
    oracle's composition, the greedy token checked."""
    L, H, nh, nkv, F, V, prefill, ctx, theta, eps = 2, 3072, 24, 6, 9216, 777, 70, 128, 500000.0, 1e-5
    m = Model(orc, L, H, nh, nkv, F, V, 700, dt=dt)
    m.upload(gpu)
    name = m.name + ".model"
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=theta, rms_eps=eps)
    print(f"decode step segmented down {dt}", flush=True)
    assert gpu.decode_create(name, cfg, m.keys), gpu.last_error()
    kc = np.zeros((L, ctx, m.kvd), np.float32)
    vc = np.zeros((L, ctx, m.kvd), np.float32)
    xd, ld, td = gpu.dev_alloc(H * 4), gpu.dev_alloc(V * 4), gpu.dev_alloc(4)
    try:
        for l in range(L):
            kr = orc.normal(prefill * m.kvd, 1.0, 710 + l, 1).reshape(prefill, m.kvd)
            vr = orc.normal(prefill * m.kvd, 1.0, 710 + l, 2).reshape(prefill, m.kvd)
            gpu.decode_kv_upload(name, l, 0, kr, vr, rows_f32=True)
            kc[l, :prefill], vc[l, :prefill] = kr, vr
        x = orc.normal(H, 1.0, 720, 1)
        gpu.h2d(xd, x)
        assert gpu.decode_step_dev(name, xd, prefill, ld, td), gpu.last_error()
        gpu.sync()
        logits = gpu.d2h(ld, (V,), np.float32)
        token = int(gpu.d2h(td, (1,), np.uint32)[0])
        ref, ref_token = m.cpu_step(orc, x, kc, vc, prefill, theta, eps)
        err = orc.rel_l2(logits, ref)
        print(f"  logits rel_l2 {err:.3e}", flush=True)
        assert err < 1e-5, err
        check_greedy(orc, token, logits, ref_token, ref)
    finally:
        for p in (xd, ld, td):
            gpu.dev_free(p)
        gpu.decode_destroy(name)
        for k in m.keys:
            gpu.weight_drop(k)


@pytest.mark.parametrize("kv_f16", [0, 1])
def test_decode_8b_layer_shape_matches_cpu(gpu, orc, kv_f16):
    """configs[4] at its real layer shape and context: one layer of hidden 4096,
    32 / 8 heads of 128 and FFN 14336 (synthetic Q4_K blocks like the bench's),
    at position 4096 of an f32 KV cache, then a 512-row Q8_0 head.  Same bar as
    above: logits within relative L2 1e-5 of the oracle's composition, the
    K / V rows of the step within 1e-5."""
    H, nh, nkv, F, V, ctx, theta, eps = 4096, 32, 8, 14336, 512, 4097, 500000.0, 1e-5
    m = Model.__new__(Model)
    m.L, m.H, m.nh, m.nkv, m.F, m.V = 1, H, nh, nkv, F, V
    m.qd, m.kvd = nh * HD, nkv * HD
    m.name = "dec8b.layer"
    sy = lambda r, c, st: orc.synth(Q4K, r, c, 61, st)
    m.layers = [{"attn_norm": (1.0 + orc.normal(H, 0.1, 61, 1)).astype(np.float32),
                 "ffn_norm": (1.0 + orc.normal(H, 0.1, 61, 2)).astype(np.float32),
                 "q": sy(m.qd, H, 3), "k": sy(m.kvd, H, 4), "v": sy(m.kvd, H, 5), "o": sy(H, m.qd, 6),
                 "gate": sy(F, H, 7), "up": sy(F, H, 8), "down": sy(H, F, 9)}]
    m.out_norm = (1.0 + orc.normal(H, 0.1, 61, 10)).astype(np.float32)
    m.head, m.head_dtype = quant(orc, Q8, orc.normal(V * H, 0.05, 61, 11)), Q8
    m.upload(gpu)
    name = m.name + ".model"
    cfg = dict(n_layers=1, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=theta, rms_eps=eps, kv_f16=kv_f16)
    print(f"decode 8B layer shape at position 4096, kv_f16={kv_f16}", flush=True)
    assert gpu.decode_create(name, cfg, m.keys), gpu.last_error()
    pos = ctx - 1
    kc = np.zeros((1, ctx, m.kvd), np.float32)
    vc = np.zeros((1, ctx, m.kvd), np.float32)
    kr = orc.normal(pos * m.kvd, 1.0, 62, 1).reshape(pos, m.kvd)
    vr = orc.normal(pos * m.kvd, 1.0, 62, 2).reshape(pos, m.kvd)
    gpu.decode_kv_upload(name, 0, 0, kr, vr, rows_f32=True)  # the library rounds to f16 when kv_f16
    if kv_f16:
        kr = orc.f16_to_f32(orc.f32_to_f16(kr)).reshape(kr.shape)
        vr = orc.f16_to_f32(orc.f32_to_f16(vr)).reshape(vr.shape)
    kc[0, :pos], vc[0, :pos] = kr, vr
    x = orc.normal(H, 1.0, 63, 1)
    xd, ld, rd = gpu.dev_alloc(H * 4), gpu.dev_alloc(V * 4), gpu.dev_alloc(2 * m.kvd * 4)
    try:
        gpu.h2d(xd, x)
        gpu.decode_step_dev(name, xd, pos, ld, None, rd)
        gpu.sync()
        logits = gpu.d2h(ld, (V,), np.float32)
        ref, _ = m.cpu_step(orc, x, kc, vc, pos, theta, eps, kv_f16=bool(kv_f16))
        k32, v32 = m.last_kv
        if kv_f16:
            rows = gpu.d2h(rd, (2, m.kvd), np.uint16)
            for got, ref32 in ((rows[0], k32[0]), (rows[1], v32[0])):
                e_gpu = orc.rel_l2(orc.f16_to_f32(got), ref32)
                e_orc = orc.rel_l2(orc.f16_to_f32(orc.f32_to_f16(ref32)), ref32)
                assert e_gpu <= e_orc + 1e-5, (e_gpu, e_orc)
        else:
            rows = gpu.d2h(rd, (2, m.kvd), np.float32)
            assert orc.rel_l2(rows[0], k32[0]) < 1e-5 and orc.rel_l2(rows[1], v32[0]) < 1e-5
        assert orc.rel_l2(logits, ref) < 1e-5, orc.rel_l2(logits, ref)
    finally:
        for p in (xd, ld, rd):
            gpu.dev_free(p)
        gpu.decode_destroy(name)
        for k in m.keys:
            gpu.weight_drop(k)


def test_decode_8b_full_step_matches_cpu(gpu, orc):
    """configs[4] end to end: the bench's 8B step (32 layers at the 8B shape,
    Q6_K head over 128256, f32 KV prefilled with N(0, 1) to position 4096) on
    the same seeded bytes as the CPU's composition.  The weights are made by
    the device generator and read back, so both sides hold the same bytes (the
    generators agree byte for byte: test_synth_device_equals_host).  Bar:
    logits within relative L2 1e-5, the greedy token equal."""
    L, H, nh, nkv, F, V, ctx, theta, eps = 32, 4096, 32, 8, 14336, 128256, 4097, 500000.0, 1e-5
    m = Model.__new__(Model)
    m.L, m.H, m.nh, m.nkv, m.F, m.V = L, H, nh, nkv, F, V
    m.qd, m.kvd = nh * HD, nkv * HD
    m.name = "dec8b.full"

    def raw(dtype, rows, cols, stream):
        nb = rows * (cols // 256) * (144 if dtype == Q4K else 210)
        d = gpu.dev_alloc(nb)
        try:
            gpu.synth_raw(d, dtype, rows, cols, 71, stream)
            return gpu.d2h(d, (nb,), np.uint8)
        finally:
            gpu.dev_free(d)

    print("decode 8B full step: generating weights", flush=True)
    m.layers = []
    st = 0
    for l in range(L):
        lw = {"attn_norm": (1.0 + orc.normal(H, 0.1, 72, 2 * l)).astype(np.float32),
              "ffn_norm": (1.0 + orc.normal(H, 0.1, 72, 2 * l + 1)).astype(np.float32)}
        for nm in ("q", "k", "v", "o", "gate", "up", "down"):
            _, r, c = m.shapes(nm)
            st += 1
            lw[nm] = raw(Q4K, r, c, st)
        m.layers.append(lw)
    m.out_norm = (1.0 + orc.normal(H, 0.1, 72, 999)).astype(np.float32)
    m.head, m.head_dtype = raw(Q6K, V, H, 10001), Q6K
    m.upload(gpu)
    name = m.name + ".model"
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=theta, rms_eps=eps)
    assert gpu.decode_create(name, cfg, m.keys, drop_sources=True), gpu.last_error()
    pos = ctx - 1
    kc = np.zeros((L, ctx, m.kvd), np.float32)
    vc = np.zeros((L, ctx, m.kvd), np.float32)
    xd, ld, td = gpu.dev_alloc(H * 4), gpu.dev_alloc(V * 4), gpu.dev_alloc(4)
    try:
        for l in range(L):
            kd, vd = gpu.decode_kv_dev(name, l)
            gpu.synth_normal(kd, ctx * m.kvd, 1.0, 73, 2 * l)
            gpu.synth_normal(vd, ctx * m.kvd, 1.0, 73, 2 * l + 1)
            # head-major on the device, position-major on the CPU side
            kc[l] = gpu.d2h(kd, (nkv, ctx, HD), np.float32).transpose(1, 0, 2).reshape(ctx, m.kvd)
            vc[l] = gpu.d2h(vd, (nkv, ctx, HD), np.float32).transpose(1, 0, 2).reshape(ctx, m.kvd)
        x = orc.normal(H, 1.0, 74, 1)
        gpu.h2d(xd, x)
        print("decode 8B full step: GPU step", flush=True)
        gpu.decode_step_dev(name, xd, pos, ld, td)
        gpu.sync()
        logits = gpu.d2h(ld, (V,), np.float32)
        token = int(gpu.d2h(td, (1,), np.uint32)[0])
        print("decode 8B full step: CPU step", flush=True)
        ref, ref_token = m.cpu_step(orc, x, kc, vc, pos, theta, eps)
        assert orc.rel_l2(logits, ref) < 1e-5, orc.rel_l2(logits, ref)
        check_greedy(orc, token, logits, ref_token, ref)
    finally:
        for p in (xd, ld, td):
            gpu.dev_free(p)
        gpu.decode_destroy(name)
        for k in m.keys:
            try:
                gpu.weight_drop(k)
            except Exception:  # noqa: BLE001 -- the q/k/v/gate/up sources were dropped with drop_sources
                pass


def test_decode_step_input_alignment(gpu, orc):
    """The step reads an aligned x in place and copies an unaligned one first:
    the same bits either way."""
    L, H, nh, nkv, F, V, ctx = 1, 512, 4, 2, 1024, 256, 16
    m = Model(orc, L, H, nh, nkv, F, V, 93)
    m.upload(gpu)
    name = m.name + ".align"
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=1e4, rms_eps=1e-5)
    assert gpu.decode_create(name, cfg, m.keys), gpu.last_error()
    x = orc.normal(H, 1.0, 94, 1)
    xd = gpu.dev_alloc((H + 4) * 4)
    ld = gpu.dev_alloc(V * 4)
    try:
        out = []
        for off in (0, 4):  # bytes
            gpu.h2d(xd + off, x)
            gpu.decode_step_dev(name, xd + off, 3, ld, None)
            gpu.sync()
            out.append(gpu.d2h(ld, (V,), np.float32))
        assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
    finally:
        gpu.dev_free(xd)
        gpu.dev_free(ld)
        gpu.decode_destroy(name)
        for k in m.keys:
            gpu.weight_drop(k)


def test_kv_upload_rounds_like_soso(gpu, orc):
    """f32 rows entering an f16 cache take soso's f32_to_f16 bit for bit:
    ties away from zero, subnormal rounding and flushing, overflow, NaN."""
    L, H, nh, nkv, F, V, ctx = 1, 512, 4, 2, 512, 64, 64
    m = Model(orc, L, H, nh, nkv, F, V, 91)
    m.upload(gpu)
    name = m.name + ".round"
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=1e4, rms_eps=1e-5, kv_f16=1)
    assert gpu.decode_create(name, cfg, m.keys), gpu.last_error()
    try:
        rng = np.random.default_rng(9)
        special = []
        for e in range(-26, 17):  # ties and near-ties at every f16 binade, subnormals included
            step = 2.0 ** max(e - 10, -24)
            base = 2.0 ** e
            for k in (0, 1, 3, 511):
                special += [base + (k + 0.5) * step, base + (k + 0.5) * step * (1 + 2 ** -20),
                            base + (k + 0.5) * step * (1 - 2 ** -20)]
        special += [2.0 ** -25, 2.0 ** -26, 3 * 2.0 ** -26, 65504.0, 65519.0, 65520.0, 1e6, np.inf, np.nan, 0.0]
        vals = np.array(special, np.float64)
        vals = np.concatenate([vals, -vals]).astype(np.float32)
        n_rows = -(-vals.size // m.kvd)
        rows = np.concatenate([vals, rng.standard_normal(n_rows * m.kvd - vals.size).astype(np.float32) * 100])
        rows = rows.reshape(n_rows, m.kvd)
        gpu.decode_kv_upload(name, 0, 3, rows, rows[::-1].copy(), rows_f32=True)
        kd, vd = gpu.decode_kv_dev(name, 0)
        gk = gpu.d2h(kd, (nkv, ctx, HD), np.uint16)[:, 3:3 + n_rows].transpose(1, 0, 2).reshape(n_rows, m.kvd)
        gv = gpu.d2h(vd, (nkv, ctx, HD), np.uint16)[:, 3:3 + n_rows].transpose(1, 0, 2).reshape(n_rows, m.kvd)
        want_k = orc.f32_to_f16(rows).reshape(rows.shape)
        want_v = orc.f32_to_f16(rows[::-1].copy()).reshape(rows.shape)
        bad = np.flatnonzero(gk.ravel() != want_k.ravel())
        assert bad.size == 0, [(float(rows.ravel()[i]), hex(int(gk.ravel()[i])), hex(int(want_k.ravel()[i])))
                               for i in bad[:6]]
        assert np.array_equal(gv, want_v)
        # rows already in f16 go in untouched
        bits = rng.integers(0, 0x7C00, size=(2, m.kvd), dtype=np.uint16)
        gpu.decode_kv_upload(name, 0, ctx - 2, bits, bits, rows_f32=False)
        gk = gpu.d2h(kd, (nkv, ctx, HD), np.uint16)[:, ctx - 2:].transpose(1, 0, 2).reshape(2, m.kvd)
        assert np.array_equal(gk, bits)
    finally:
        gpu.decode_destroy(name)
        for k in m.keys:
            gpu.weight_drop(k)


class MoeFfn:
    """A seeded MoE FFN for a decode layer: router f32 ~ N(0, 0.02), experts
    N(0, 0.05) through the reference quantizers (Q4_K), like the dense model's
    weights, so a stack of layers keeps its scale."""

    def __init__(self, orc, n_exp, h, ffn, top_k, seed):
        self.n_exp, self.h, self.ffn, self.top_k = n_exp, h, ffn, top_k
        self.router = orc.normal(n_exp * h, 0.02, seed, 1)
        self.gate = [quant(orc, Q4K, orc.normal(ffn * h, 0.05, seed, 100 + e)) for e in range(n_exp)]
        self.up = [quant(orc, Q4K, orc.normal(ffn * h, 0.05, seed, 1000 + e)) for e in range(n_exp)]
        self.down = [quant(orc, Q4K, orc.normal(h * ffn, 0.05, seed, 2000 + e)) for e in range(n_exp)]
        self.name = f"decmoe{seed}.{n_exp}.{h}.{ffn}.{top_k}"

    def cpu(self, orc, x):
        return orc.moe_ffn(self.router, self.n_exp, self.h, self.ffn, self.top_k, self.gate, self.up, self.down,
                           Q4K, Q4K, x)

    def upload(self, gpu):
        def put(key, arr, dtype, rows, cols):
            b = np.ascontiguousarray(arr).view(np.uint8)
            d = gpu.dev_alloc(b.size)
            try:
                gpu.h2d(d, b)
                gpu.weight_from_dev(key, d, b.size, dtype, rows, cols)
            finally:
                gpu.dev_free(d)
        keys = []
        for e in range(self.n_exp):
            for nm, w, r, c in (("gate", self.gate[e], self.ffn, self.h), ("up", self.up[e], self.ffn, self.h),
                                ("down", self.down[e], self.h, self.ffn)):
                k = f"{self.name}.E{e}.{nm}"
                put(k, w, Q4K, r, c)
                keys.append(k)
        put(self.name + ".router", self.router, F32, self.n_exp, self.h)
        self.keys = keys
        self.register(gpu)

    def register(self, gpu):
        gpu.moe_register(self.name, self.name + ".router", self.keys, self.n_exp, self.h, self.ffn, self.top_k)


@pytest.mark.parametrize("kv_f16", [0, 1])
def test_decode_step_with_moe_layers_matches_cpu(gpu, orc, kv_f16):
    """A GQA model whose layers 1 and 2 take registered MoE layers as their FFN
    (soso_hip_decode_create_moe; GpuDispatch::moe_capa for one token): one
    step at position 150 against the oracle's composition (the dense layer,
    then rmsnorm + or_moe_ffn + residual for the MoE layers): logits within
    1e-5, the greedy token, and each MoE layer's routing -- indices identical
    in ranking order, weights within 1e-5.  Layer 1's unused gate/up/down keys
    are passed as null.  Re-registering an MoE layer the model reads destroys
    the model."""
    L, H, nh, nkv, F, V, prefill = 3, 1024, 8, 2, 2048, 1000, 150
    theta, eps, ctx = 500000.0, 1e-5, 256
    m = Model(orc, L, H, nh, nkv, F, V, 80 + 10 * kv_f16)
    m.upload(gpu)
    moe = {1: MoeFfn(orc, 16, H, 512, 4, 81 + 10 * kv_f16), 2: MoeFfn(orc, 24, H, 256, 8, 82 + 10 * kv_f16)}
    for f in moe.values():
        f.upload(gpu)
    keys = list(m.keys)
    for j in (6, 7, 8):
        keys[9 * 1 + j] = None
    name = m.name + f".moe{kv_f16}"
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=theta, rms_eps=eps, kv_f16=kv_f16)
    assert gpu.decode_create(name, cfg, keys, moe_layers=[None, moe[1].name, moe[2].name]), gpu.last_error()
    kc = np.zeros((L, ctx, m.kvd), np.float32)
    vc = np.zeros((L, ctx, m.kvd), np.float32)
    for l in range(L):
        kr = orc.normal(prefill * m.kvd, 1.0, 90 + l, 1).reshape(prefill, m.kvd)
        vr = orc.normal(prefill * m.kvd, 1.0, 90 + l, 2).reshape(prefill, m.kvd)
        gpu.decode_kv_upload(name, l, 0, kr, vr, rows_f32=True)
        if kv_f16:
            kr, vr = orc.f16_to_f32(orc.f32_to_f16(kr)).reshape(kr.shape), orc.f16_to_f32(orc.f32_to_f16(vr)).reshape(
                vr.shape)
        kc[l, :prefill] = kr
        vc[l, :prefill] = vr
    x = orc.normal(H, 1.0, 95, 1)
    xd, ld, td = gpu.dev_alloc(H * 4), gpu.dev_alloc(V * 4), gpu.dev_alloc(4)
    try:
        gpu.h2d(xd, x)
        gpu.decode_step_dev(name, xd, prefill, ld, td)
        gpu.sync()
        logits = gpu.d2h(ld, (V,), np.float32)
        token = int(gpu.d2h(td, (1,), np.uint32)[0])
        ref, ref_tok = m.cpu_step(orc, x, kc, vc, prefill, theta, eps, kv_f16=bool(kv_f16), moe=moe)
        err = orc.rel_l2(logits, ref)
        print(f"decode with MoE layers kv_f16={kv_f16}: logits rel_l2 {err:.3e}", flush=True)
        assert err < 1e-5, err
        check_greedy(orc, token, logits, ref_tok, ref)
        for l, f in moe.items():
            idx, w = gpu.decode_moe_routing(name, l, f.top_k)
            ri, rw = m.routing[l]
            assert np.array_equal(idx, ri), (l, idx, ri)
            assert orc.rel_l2(w, rw) < 1e-5, (l, w, rw)
        # the same step replayed from a graph (after restoring the KV rows it
        # wrote) gives the same bits
        gpu.graph_begin()
        gpu.decode_step_dev(name, xd, prefill, ld, td)
        gid = gpu.graph_end()
        try:
            for _ in range(2):
                gpu.graph_launch(gid)
                gpu.sync()
                again = gpu.d2h(ld, (V,), np.float32)
                assert np.array_equal(again.view(np.uint32), logits.view(np.uint32))
        finally:
            gpu.graph_destroy(gid)
        # re-registering an MoE layer the model reads unregisters the model
        moe[2].register(gpu)
        assert not gpu.decode_step_dev(name, xd, prefill, ld, td)
    finally:
        for p in (xd, ld, td):
            gpu.dev_free(p)


@pytest.mark.parametrize("qk_norm,neox,kv_f16,with_moe,prefill,nh,nkv", [
    (True, True, 0, False, 90, 8, 2),    # Qwen3's attention: QK norm and NeoX RoPE
    (True, True, 0, False, 63, 8, 2),    # steps at 63 (one chunk) and 64 (a chunk of one new position)
    (True, True, 1, True, 90, 8, 2),     # the same over soso's f16 cache, layer 1 an MoE layer
    (True, False, 1, False, 127, 8, 2),  # QK norm alone; steps at 127 and 128
    (False, True, 0, False, 0, 8, 2),    # NeoX RoPE alone; steps at 0 and 1
    (True, True, 1, False, 70, 16, 2),   # groups of 8 query heads (Qwen3-30B-A3B's 32 / 4)
    (True, True, 0, False, 70, 4, 4),    # one query head per KV head
])
def test_decode_step_qk_norm_and_neox_rope(gpu, orc, qk_norm, neox, kv_f16, with_moe, prefill, nh, nkv):
    """soso_hip_decode_create_ex with SOSO_HIP_DECODE_QK_NORM (each q and k
    head RMS-normalised with the layer's attn_q_norm / attn_k_norm before RoPE,
    layer.rs:1164-1180) and SOSO_HIP_DECODE_ROPE_NEOX (rope_cabezas' NeoX
    pairs (i, i + head_dim/2), gemm.rs:1474-1479).  Two steps (positions
    `prefill` and `prefill` + 1, the second reading the row the first wrote;
    the attention's last chunk appends the row, so the positions straddle
    chunk ends) against the oracle's composition: logits within relative L2
    1e-5, the greedy token, and the K/V rows written at `prefill` under the
    bar of test_decode_step_matches_cpu."""
    L, H, F, V = 2, 1024, 2048, 1000
    theta, eps, ctx = 1000000.0, 1e-6, 192
    flags = (1 if qk_norm else 0) | (2 if neox else 0)  # SOSO_HIP_DECODE_QK_NORM | _ROPE_NEOX
    m = Model(orc, L, H, nh, nkv, F, V, 400 + flags + 4 * kv_f16 + nh, qk_norm=qk_norm, neox=neox)
    m.upload(gpu)
    kpl = 11 if qk_norm else 9
    keys, moe, moe_layers = list(m.keys), None, None
    if with_moe:
        moe = {1: MoeFfn(orc, 16, H, 512, 4, 410)}
        moe[1].upload(gpu)
        for j in (6, 7, 8):
            keys[kpl * 1 + j] = None
        moe_layers = [None, moe[1].name]
    name = m.name + ".model"
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=theta, rms_eps=eps, kv_f16=kv_f16)
    print(f"decode step qk_norm={qk_norm} neox={neox} kv_f16={kv_f16} moe={with_moe} heads={nh}/{nkv}", flush=True)
    assert gpu.decode_create(name, cfg, keys, moe_layers=moe_layers, flags=flags), gpu.last_error()
    kvt, esz = (np.uint16, 2) if kv_f16 else (np.float32, 4)
    kc = np.zeros((L, ctx, m.kvd), np.float32)
    vc = np.zeros((L, ctx, m.kvd), np.float32)
    xd, ld, td, rd = gpu.dev_alloc(H * 4), gpu.dev_alloc(V * 4), gpu.dev_alloc(4), gpu.dev_alloc(L * 2 * m.kvd * esz)
    try:
        for l in range(L if prefill else 0):
            kr = orc.normal(prefill * m.kvd, 1.0, 420 + l, 1).reshape(prefill, m.kvd)
            vr = orc.normal(prefill * m.kvd, 1.0, 420 + l, 2).reshape(prefill, m.kvd)
            gpu.decode_kv_upload(name, l, 0, kr, vr, rows_f32=True)
            if kv_f16:
                kr = orc.f16_to_f32(orc.f32_to_f16(kr)).reshape(kr.shape)
                vr = orc.f16_to_f32(orc.f32_to_f16(vr)).reshape(vr.shape)
            kc[l, :prefill], vc[l, :prefill] = kr, vr
        x = orc.normal(H, 1.0, 430, 1)
        gpu.h2d(xd, x)
        assert gpu.decode_step_dev(name, xd, prefill, ld, td, rd), gpu.last_error()
        gpu.sync()
        logits = gpu.d2h(ld, (V,), np.float32)
        token = int(gpu.d2h(td, (1,), np.uint32)[0])
        rows = gpu.d2h(rd, (L, 2, m.kvd), kvt)
        ref, ref_token = m.cpu_step(orc, x, kc, vc, prefill, theta, eps, kv_f16=bool(kv_f16), moe=moe)
        k32, v32 = m.last_kv
        for l in range(L):
            for got, ref32 in ((rows[l, 0], k32[l]), (rows[l, 1], v32[l])):
                if kv_f16:
                    want = orc.f32_to_f16(ref32)
                    e_gpu = orc.rel_l2(orc.f16_to_f32(got), ref32)
                    e_orc = orc.rel_l2(orc.f16_to_f32(want), ref32)
                    assert e_gpu <= e_orc + 1e-5, (l, e_gpu, e_orc)
                    assert (got == want).mean() > 0.95, (l, float((got == want).mean()))
                else:
                    assert orc.rel_l2(got, ref32) < 1e-5, l
        err = orc.rel_l2(logits, ref)
        print(f"  logits rel_l2 {err:.3e}", flush=True)
        assert err < 1e-5, err
        check_greedy(orc, token, logits, ref_token, ref)
        assert gpu.decode_step_dev(name, xd, prefill + 1, ld, td), gpu.last_error()
        gpu.sync()
        logits2 = gpu.d2h(ld, (V,), np.float32)
        ref2, _ = m.cpu_step(orc, x, kc, vc, prefill + 1, theta, eps, kv_f16=bool(kv_f16), moe=moe)
        assert orc.rel_l2(logits2, ref2) < 1e-5, orc.rel_l2(logits2, ref2)
    finally:
        for p in (xd, ld, td, rd):
            gpu.dev_free(p)
        gpu.decode_destroy(name)
        for k in m.keys:
            gpu.weight_drop(k)


def test_decode_create_ex_declines_bad_flags_and_norms(gpu, orc):
    """decode_create_ex rejects an unknown flag bit (an argument error) and
    declines QK norm whose q_norm key is not F32 [head_dim]; neither
    registers a model."""
    L, H, nh, nkv, F, V = 1, 512, 4, 2, 512, 64
    m = Model(orc, L, H, nh, nkv, F, V, 440, qk_norm=True)
    m.upload(gpu)
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=64,
               rope_theta=10000.0, rms_eps=1e-6)
    xd, ld = gpu.dev_alloc(H * 4), gpu.dev_alloc(V * 4)
    try:
        with pytest.raises(RuntimeError, match="unknown flags"):
            gpu.decode_create("bad.flags", cfg, m.keys, flags=4)
        bad = list(m.keys)
        bad[9] = m.keys[0]  # attn_norm: F32 [1 x hidden], not [1 x head_dim]
        assert not gpu.decode_create("bad.norm", cfg, bad, flags=1)
        assert "q_norm" in gpu.last_error(), gpu.last_error()
        for nm in ("bad.flags", "bad.norm"):
            assert not gpu.decode_step_dev(nm, xd, 0, ld, None)
        assert gpu.decode_create("good", cfg, m.keys, flags=3), gpu.last_error()
        gpu.decode_destroy("good")
    finally:
        for p in (xd, ld):
            gpu.dev_free(p)
        for k in m.keys:
            gpu.weight_drop(k)


def test_decode_token_host_buffers_and_host_experts(gpu, orc):
    """soso_hip_decode_token (GpuDispatch::decode_token, gpu.rs:670-685) on host
    buffers.  A dense model: logits, token and KV rows bit-identical to
    decode_step_dev at the same position, and the decode_* stats count the
    embedding row up, the logits and the KV rows down and one step.  A model
    whose layer 1 FFN is registered as its router alone (the experts stay on
    the host): the device routes, cpu_moe computes the chosen experts on the
    CPU (oracle matvecs and SwiGLU, summed in ranking order), the step goes
    on; the routing handed to cpu_moe equals the device-resident MoE model's,
    and the logits are within 1e-5 of that model's and of the oracle's
    composition.  decode_step_dev declines the host-expert model, and a
    failing cpu_moe fails decode_token with the callback's error."""
    L, H, nh, nkv, F, V, pos = 3, 1024, 8, 2, 2048, 1000, 150
    theta, eps, ctx = 500000.0, 1e-5, 256
    m = Model(orc, L, H, nh, nkv, F, V, 160)
    m.upload(gpu)
    moe = MoeFfn(orc, 16, H, 512, 4, 161)
    moe.upload(gpu)
    host_key = moe.name + ".host"
    assert gpu.moe_register(host_key, moe.name + ".router", None, moe.n_exp, H, moe.ffn, moe.top_k)
    keys = list(m.keys)
    for j in (6, 7, 8):
        keys[9 * 1 + j] = None
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=HD, ffn=F, vocab=V, ctx_max=ctx,
               rope_theta=theta, rms_eps=eps, kv_f16=0)
    names = {"dense": m.name + ".tok.dense", "dev": m.name + ".tok.devmoe", "host": m.name + ".tok.hostmoe"}
    assert gpu.decode_create(names["dense"], cfg, m.keys), gpu.last_error()
    assert gpu.decode_create(names["dev"], cfg, keys, moe_layers=[None, moe.name, None]), gpu.last_error()
    assert gpu.decode_create(names["host"], cfg, keys, moe_layers=[None, host_key, None]), gpu.last_error()
    kc = np.zeros((L, ctx, m.kvd), np.float32)
    vc = np.zeros((L, ctx, m.kvd), np.float32)
    for l in range(L):
        kr = orc.normal(pos * m.kvd, 1.0, 170 + l, 1).reshape(pos, m.kvd)
        vr = orc.normal(pos * m.kvd, 1.0, 170 + l, 2).reshape(pos, m.kvd)
        for name in names.values():
            gpu.decode_kv_upload(name, l, 0, kr, vr, rows_f32=True)
        kc[l, :pos], vc[l, :pos] = kr, vr
    x = orc.normal(H, 1.0, 175, 1)
    xd, ld, td, rd = gpu.dev_alloc(H * 4), gpu.dev_alloc(V * 4), gpu.dev_alloc(4), gpu.dev_alloc(L * 2 * m.kvd * 4)
    try:
        gpu.h2d(xd, x)
        # dense: the host entry against the device entry
        gpu.decode_step_dev(names["dense"], xd, pos, ld, td, rd)
        gpu.sync()
        l_dev, t_dev = gpu.d2h(ld, (V,), np.float32), int(gpu.d2h(td, (1,), np.uint32)[0])
        r_dev = gpu.d2h(rd, (L * 2 * m.kvd,), np.float32)
        s0 = gpu.stats()
        lg, tok, kv = gpu.decode_token(names["dense"], x, pos, logits=True, kv_rows=True)
        s1 = gpu.stats()
        assert np.array_equal(lg.view(np.uint32), l_dev.view(np.uint32)) and tok == t_dev
        assert np.array_equal(kv.view(np.uint32), r_dev.view(np.uint32))
        assert s1["decode_steps"] - s0["decode_steps"] == 1
        assert s1["decode_embed_up"] - s0["decode_embed_up"] == H * 4
        assert s1["decode_logits_down"] - s0["decode_logits_down"] == V * 4
        assert s1["decode_kv_down"] - s0["decode_kv_down"] == L * 2 * m.kvd * 4
        assert s1["decode_control_up"] == s0["decode_control_up"]
        # MoE layer 1 with resident experts (the device path) ...
        gpu.decode_step_dev(names["dev"], xd, pos, ld, td)
        gpu.sync()
        l_moe = gpu.d2h(ld, (V,), np.float32)
        dev_idx, dev_w = gpu.decode_moe_routing(names["dev"], 1, moe.top_k)
        # ... and with its experts on the host
        calls = []

        def cpu_moe(layer, xn, idx, wgt):
            calls.append((layer, idx, wgt))
            out = np.zeros(H, np.float32)
            for j in range(moe.top_k):
                e = int(idx[j])
                g = orc.matvec(Q4K, moe.gate[e], moe.ffn, H, xn)
                u = orc.matvec(Q4K, moe.up[e], moe.ffn, H, xn)
                orc.lib().or_swiglu(u.ctypes.data, g.ctypes.data, moe.ffn)
                out = out + np.float32(wgt[j]) * orc.matvec(Q4K, moe.down[e], H, moe.ffn, u)
            return out
        lh, th, _ = gpu.decode_token(names["host"], x, pos, cpu_moe=cpu_moe)
        assert len(calls) == 1 and calls[0][0] == 1
        assert np.array_equal(calls[0][1], dev_idx), (calls[0][1], dev_idx)
        assert orc.rel_l2(calls[0][2], dev_w) < 1e-5
        err = orc.rel_l2(lh, l_moe)
        ref, ref_tok = m.cpu_step(orc, x, kc, vc, pos, theta, eps, moe={1: moe})
        print(f"decode_token host experts: vs device experts {err:.3e}, vs oracle {orc.rel_l2(lh, ref):.3e}",
              flush=True)
        assert err < 1e-5 and orc.rel_l2(lh, ref) < 1e-5
        check_greedy(orc, th, lh, ref_tok, ref)
        # the device-only entries decline it; a failing callback fails the call
        assert not gpu.decode_step_dev(names["host"], xd, pos, ld, td)
        assert not gpu.moe_ffn_dev(host_key, xd, 1, rd)

        def broken(layer, xn, idx, wgt):
            raise RuntimeError("host experts unavailable")
        with pytest.raises(RuntimeError, match="host experts unavailable"):
            gpu.decode_token(names["host"], x, pos, cpu_moe=broken)
        # ... and so does a host-expert model called without one
        assert gpu.decode_token(names["host"], x, pos) is None
    finally:
        for p in (xd, ld, td, rd):
            gpu.dev_free(p)
        for name in names.values():
            gpu.decode_destroy(name)
        for k in m.keys + moe.keys + [moe.name + ".router"]:
            gpu.weight_drop(k)
