"""Benchmark of the decode hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): single-token Q4_K matvec at the
Llama FFN-up shape 14336 x 4096 in GB/s and as a fraction of the 8 TB/s HBM
peak.  A "step" is one matvec over one resident weight; 16 weight copies
(528 MB, above the 256 MB Infinity Cache) are rotated so HBM, not MALL,
serves them.  Inputs are synthetic (seeded counter-based generator) and
already resident in HBM when the timed region starts.

Prints ONE JSON line.  `value` and `roofline.achieved` are algorithmic bytes
over the average launch duration, measured with HIP events on the library's
stream around a graph of back-to-back launches; `cpu_baseline` times the
AVX2 restatement of soso's CPU kernels (oracle/) on the host cores for a
bounded sample.  Other configs of
BASELINE.json are reported under "configs" (they are parity cases, not the
headline).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBS = 8000.0
Q4K, Q8, Q6K, F32 = 3, 2, 13, 1
ROW_BYTES = {Q4K: lambda c: c // 256 * 144, Q8: lambda c: c // 32 * 36, Q6K: lambda c: c // 256 * 210}


def algo_bytes(dtype, rows, cols):
    """Algorithmic bytes of one matvec: weights + x + y, each moved once."""
    return rows * ROW_BYTES[dtype](cols) + 4 * cols + 4 * rows


def _capture(g, body):
    """Captures body() into a graph; the capture is always closed."""
    g.graph_begin()
    err = None
    try:
        body()
    except Exception as e:  # noqa: BLE001
        err = e
    gid = g.graph_end()
    if err is not None:
        g.graph_destroy(gid)
        raise err
    return gid


# The GPU's clocks climb over the first milliseconds of load: a timed region
# that starts on a rested GPU reads slower the shorter it is (measured 5-12 %
# at 20 steps against 100-1000, headline matvec to 64-token matmul).  Every
# timed region therefore starts behind at least SPIN_MS of untimed replays of
# the same launches, still running when the timed ones are enqueued, so the
# per-step figure is the steady state whatever `steps` is.
SPIN_MS = 30.0


def _spin(g, gid, replay_ms):
    """Enqueues untimed replays of graph gid (one takes replay_ms) covering
    SPIN_MS, without waiting for them.  Returns how many."""
    reps = max(2, int(SPIN_MS / max(replay_ms, 1e-3)) + 1)
    for _ in range(reps):
        g.graph_launch(gid)
    return reps


def _timed_graph(g, calls, steps):
    """Captures `calls` (which issues `steps` steps) into one graph, replays it
    once to warm it and once on an idle stream (the host wall figure), then
    enqueues untimed replays covering SPIN_MS (_spin) and, behind them, the
    timed replay between two HIP events on the library's stream: the events
    bracket exactly that replay's `steps` steps, started while the GPU is
    busy and its clocks up.  Returns (ms per step between the events, host
    wall ms per step of one replay on an idle stream)."""
    gid = _capture(g, calls)
    try:
        g.graph_launch(gid)
        g.sync()
        t0 = time.perf_counter()
        g.graph_launch(gid)
        g.sync()
        t1 = time.perf_counter()
        _spin(g, gid, (t1 - t0) * 1e3)
        g.event_record(0)
        g.graph_launch(gid)
        g.event_record(1)
        g.sync()
    finally:
        g.graph_destroy(gid)
    return g.event_elapsed(0, 1) / steps, (t1 - t0) * 1e3 / steps


# A timed window carries a fixed cost of its own besides its steps: the two
# event records and the restart of the stream behind them, measured 2-6 us
# per window with direct launches and 6-13 us from a graph (Q4_K/Q8_0
# matvecs, 20 and 50 steps against 1000, behind the spin-up).  At 20 steps of
# 7 us that is 2-9 % of the per-step figure.  The single-launch matvecs are
# therefore timed over at least MIN_TIMED launches (`timed_launches` in the
# JSON line; `steps` stays the count asked for), where it is below 0.2 %.
MIN_TIMED = 1000
SPIN_LAUNCHES = 256  # at least this many direct spin-up launches (eager windows)


def _timed_steps(g, launch, steps, eager=False):
    """Times exactly `steps` steps (launch(i) issues step i), behind SPIN_MS
    of untimed work: as one graph replay behind replays of it (_timed_graph),
    or with eager (for tracers and counter collectors) as direct launches
    behind direct spin-up launches of the same steps.  Returns (ms per step between the
    events, host wall ms per step of one replay or of the direct launches,
    on an idle stream)."""
    if not eager:
        return _timed_graph(g, lambda: [launch(i) for i in range(steps)], steps)
    g.sync()
    t0 = time.perf_counter()
    for i in range(steps):
        launch(i)
    g.sync()
    t1 = time.perf_counter()
    # the spin-up as direct launches too (no graph: counter collectors take
    # graph replays badly), issued for SPIN_MS of host time and at least
    # SPIN_LAUNCHES launches; the timed launches queue behind them
    i, t2 = 0, time.perf_counter()
    while i < SPIN_LAUNCHES or (time.perf_counter() - t2) * 1e3 < SPIN_MS:
        launch(i)
        i += 1
    g.event_record(0)
    for i in range(steps):
        launch(i)
    g.event_record(1)
    g.sync()
    return g.event_elapsed(0, 1) / steps, (t1 - t0) * 1e3 / steps


def time_matvec(g, dtype, rows, cols, copies, steps, warmup, seed=1, eager=False):
    """Average duration of one matvec launch, in ms.

    `copies` resident weights are rotated so HBM, not the MALL, serves them.
    The timed region is `steps` back-to-back launches on the library's stream
    (one HIP graph), behind untimed spin-up replays and bracketed by HIP
    events recorded on that stream (_timed_steps): the average is (event
    interval) / steps, the same per-dispatch figure rocprofv3 --kernel-trace
    reports (profiles/ holds that cross-check).  eager=True launches the
    steps directly (for counter and tracer runs).  Returns (ms_per_launch_events,
    ms_per_launch_host_wall on an idle stream)."""
    keys = [f"bench.{dtype}.{rows}x{cols}.{i}" for i in range(copies)]
    for i, k in enumerate(keys):
        g.weight_synth(k, dtype, rows, cols, seed, 1000 + i)
    x = g.dev_alloc(cols * 4)
    y = g.dev_alloc(rows * 4)
    g.synth_normal(x, cols, 1.0, seed, 7)
    try:
        for i in range(warmup):
            g.matvec_dev(keys[i % copies], x, y)
        g.sync()
        return _timed_steps(g, lambda i: g.matvec_dev(keys[i % copies], x, y), steps, eager)
    finally:
        g.sync()
        g.dev_free(x)
        g.dev_free(y)
        for k in keys:
            g.weight_drop(k)


def time_host_matvec(g, dtype, rows, cols, calls=300, seed=5):
    """What one op costs soso through the drop-in boundary: soso_hip_matvec on
    host buffers (matvec_step calls GpuDispatch::matvec synchronously per op,
    crates/soso-llm-core/src/layer.rs:644-672): x up, the kernel, y down and
    the wait, on a resident weight.  Returns (median, 10th, 90th percentile)
    microseconds per call, host wall clock."""
    import numpy as np
    key = f"bench.host.{dtype}.{rows}x{cols}"
    g.weight_synth(key, dtype, rows, cols, seed, 1)
    x = np.random.default_rng(seed).standard_normal(cols).astype(np.float32)
    y = np.empty(rows, np.float32)
    try:
        for _ in range(20):
            g.matvec(key, None, dtype, rows, cols, x, y)
        ts = []
        for _ in range(calls):
            t0 = time.perf_counter()
            g.matvec(key, None, dtype, rows, cols, x, y)
            ts.append((time.perf_counter() - t0) * 1e6)
        ts.sort()
        return ts[len(ts) // 2], ts[len(ts) // 10], ts[(9 * len(ts)) // 10]
    finally:
        g.weight_drop(key)


def time_matmul(g, rows, cols, n, copies, steps, warmup, seed=3, eager=False, dtype=Q4K):
    """matmul Y[n x rows] = X[n x cols] . W^T (GpuDispatch::matmul) with n
    tokens (Q4_K or Q8_0: on the matrix cores from 16 tokens); `copies`
    rotating weights.  Returns ms per call (HIP events around a graph of
    back-to-back calls; eager=True launches them directly, for tracers)."""
    keys = [f"bench.mm.{dtype}.{rows}x{cols}.{i}" for i in range(copies)]
    for i, k in enumerate(keys):
        g.weight_synth(k, dtype, rows, cols, seed, 3000 + i)
    x = g.dev_alloc(n * cols * 4)
    y = g.dev_alloc(n * rows * 4)
    try:
        g.synth_normal(x, n * cols, 1.0, seed, 9)
        for i in range(warmup):
            g.matmul_dev(keys[i % copies], n, x, y)
        g.sync()
        calls = lambda: [g.matmul_dev(keys[i % copies], n, x, y) for i in range(steps)]
        if eager:
            g.event_record(0)
            calls()
            g.event_record(1)
            g.sync()
        else:
            # (always a graph: issued directly, the matmul's host-side launch
            # selection showed through, 75 against 67 us per call at 100 calls)
            return _timed_graph(g, calls, steps)[0]
        return g.event_elapsed(0, 1) / steps
    finally:
        g.sync()
        g.dev_free(x)
        g.dev_free(y)
        for k in keys:
            g.weight_drop(k)


READ_SHAPES = ((1, 256), (2, 256), (4, 256), (8, 256), (1, 512), (2, 512), (4, 512), (1, 1024), (2, 1024))
# read-probe variants: grid-stride with K independent 16-byte loads per thread,
# or per-wavefront contiguous stretches with K 1-KiB buffer loads in flight
READ_VARIANTS = (("gs", 1), ("gs", 2), ("gs", 4), ("gs", 8), ("chunk", 2), ("chunk", 4), ("chunk", 8), ("chunk", 16),
                 ("gs_nt", 2), ("gs_nt", 4), ("chunk_nt", 4), ("chunk_nt", 8))  # _nt: nontemporal loads


def time_read_probe(g, nbytes, copies, steps, warmup, shapes=READ_SHAPES, variants=READ_VARIANTS):
    """Plain streaming reads (soso_hip_read_probe) of `nbytes` over `copies`
    rotating buffers, per variant (grid-stride with K independent loads per
    thread, or per-wavefront KiB stretches with K loads in flight) and launch
    shape (workgroups per CU, threads): the bandwidth ceiling the matvec is
    held against, timed like time_matvec (back-to-back graph replays between
    two HIP events).  Returns {(variant, K, wg_per_cu, threads): ms per launch}."""
    bufs = [g.dev_alloc(nbytes) for _ in range(copies)]
    out_len = 32 * 1024 * 1024
    out = g.dev_alloc(out_len * 4)
    res = {}
    try:
        for i, b in enumerate(bufs):
            g.synth_normal(b, nbytes // 4, 1.0, 5, 900 + i)
        for var, k in variants:
            for wpc, thr in shapes:
                def call(i):
                    g.read_probe(bufs[i % copies], nbytes, wpc, thr, out, out_len, loads=k,
                                 chunked=var.startswith("chunk"), stream=var.endswith("_nt"))
                for i in range(warmup):
                    call(i)
                g.sync()
                res[(var, k, wpc, thr)] = _timed_graph(g, lambda: [call(i) for i in range(steps)], steps)[0]
    finally:
        g.sync()
        for b in bufs:
            g.dev_free(b)
        g.dev_free(out)
    return res


def read_probe_bytes(var, nbytes):
    """Bytes a read-probe variant reads: whole 16-byte words, or whole KiB."""
    return nbytes // 1024 * 1024 if var.startswith("chunk") else nbytes // 16 * 16


def time_gdn(g, n, steps, layers=8, n_k=16, n_v=32, d=128, kernel=4, seed=41, eager=False):
    """A Qwen3-Next-80B-A3B-like Gated DeltaNet layer's recurrence
    (soso_hip_gdn_block_dev, GpuDispatch::gdn_bloque) for a block of `n`
    tokens: 16 q/k heads, 32 value heads of 128, conv kernel 4; seeded inputs
    and states (N(0, 1) projections, state ~ N(0, 0.05), decay in (0, 1],
    beta in (0, 1)).  `layers` independent states (32 x 128 x 128 f32 = 2 MiB
    each) are rotated so each call reads its state from HBM.  Returns (ms per
    call, algorithmic bytes per call: the state read and written, the conv
    history and weights, z, the gates and norm, the output, and the conv
    result u the two launches hand over)."""
    C, vd = (2 * n_k + n_v) * d, n_v * d
    sizes = [(kernel - 1 + n) * C, C * kernel, n * vd, n * n_v, n * n_v, d, n_v * d * d, n * vd]
    bufs = []
    try:
        for layer in range(layers):
            ptrs = []
            for i, sz in enumerate(sizes):
                p = g.dev_alloc(sz * 4)
                ptrs.append(p)
                sigma = (1.0, 0.5, 1.0, 0.3, 1.0, 0.1, 0.05, 1.0)[i]
                g.synth_normal(p, sz, sigma, seed + layer, i)
            # decay = exp(-|N|) in (0, 1] and beta = sigmoid(N) in (0, 1), as the model's gates give them
            for i, f in ((3, lambda a: np.exp(-np.abs(a))), (4, lambda a: 1.0 / (1.0 + np.exp(-a)))):
                a = g.d2h(ptrs[i], (sizes[i],), np.float32)
                g.h2d(ptrs[i], f(a).astype(np.float32))
            bufs.append(ptrs)
        call = [0]

        def one():
            b = bufs[call[0] % layers]
            call[0] += 1
            assert g.gdn_block_dev(*b, n, n_k, n_v, d, kernel, 1e-6), g.last_error()
        for _ in range(3):
            one()
        g.sync()
        if eager:
            g.event_record(0)
            for _ in range(steps):
                one()
            g.event_record(1)
            g.sync()
            ms = g.event_elapsed(0, 1) / steps
        else:
            ms = _timed_graph(g, lambda: [one() for _ in range(steps)], steps)[0]
    finally:
        for ptrs in bufs:
            for p in ptrs:
                g.dev_free(p)
    nbytes = 4 * (sizes[0] + sizes[1] + sizes[2] + sizes[3] + sizes[4] + sizes[5] + 2 * sizes[6] + sizes[7] + 2 * n * C)
    return ms, nbytes


def time_moe(g, n, steps, layers=4, n_x=8, seed=11, eager=False):
    """Qwen3-30B-A3B-like MoE FFN (hidden 2048, 128 experts of
    intermediate 768, top-8, Q4_K experts, f32 router ~ N(0, 0.02)), `n`
    tokens ~ N(0, 1) per call, routing from the seeded inputs.  `layers`
    independent layers and `n_x` input batches are rotated so that successive
    calls touch different experts (HBM, not the MALL).  The timed calls replay
    one HIP graph; eager=True launches them directly (for kernel tracers).
    Returns (ms per call, algorithmic bytes per call averaged over the
    rotation, distinct experts per call)."""
    E, H, F, K = 128, 2048, 768, 8
    names = []
    try:
        for L in range(layers):
            name = f"bm{n}.{L}"
            keys = []
            for e in range(E):
                for j, (r, c) in enumerate(((F, H), (F, H), (H, F))):
                    k = f"{name}.E{e}.{('gate', 'up', 'down')[j]}"
                    g.weight_synth(k, Q4K, r, c, seed, L * 1000 + 3 * e + j)
                    keys.append(k)
            d = g.dev_alloc(E * H * 4)
            try:
                g.synth_normal(d, E * H, 0.02, seed + 1, L)
                g.weight_from_dev(name + ".router", d, E * H * 4, F32, E, H)
            finally:
                g.dev_free(d)
            g.moe_register(name, name + ".router", keys, E, H, F, K)
            names.append((name, keys))
        xs = g.dev_alloc(n_x * n * H * 4)
        out = g.dev_alloc(n * H * 4)
        idx = g.dev_alloc(n * K * 4)
        try:
            g.synth_normal(xs, n_x * n * H, 1.0, seed + 2, n)
            per_expert = 3 * F * (H // 256) * 144
            nbytes = []
            for L in range(layers):
                for i in range(n_x):
                    g.moe_ffn_dev(names[L][0], xs + i * n * H * 4, n, out, idx, None)
                    ids = g.d2h(idx, (n * K,), np.int32)
                    u = len(set(ids.tolist()))
                    nbytes.append((E * H * 4 + u * per_expert + 2 * n * H * 4, u))
            g.sync()
            combos = layers * n_x
            calls = lambda: [g.moe_ffn_dev(names[i % layers][0], xs + ((i // layers) % n_x) * n * H * 4,
                                           n, out, None, None) for i in range(steps)]
            if eager:
                calls()
                g.sync()
                g.event_record(0)
                calls()
                g.event_record(1)
                g.sync()
                ms = g.event_elapsed(0, 1) / steps
            else:
                ms = _timed_graph(g, calls, steps)[0]
            order = [(i % layers) * n_x + (i // layers) % n_x for i in range(steps)]
            b = sum(nbytes[o][0] for o in order) / steps
            u = sum(nbytes[o][1] for o in order) / steps
            return ms, b, u, combos
        finally:
            g.dev_free(xs)
            g.dev_free(out)
            g.dev_free(idx)
    finally:
        for name, keys in names:
            for k in keys:
                g.weight_drop(k)
            g.weight_drop(name + ".router")


def time_decode_8b(g, steps, ctx=4096, seed=21, kv_f16=False, eager=False):
    """one greedy decode step of a random-init Llama-style 8B
    (32 layers, hidden 4096, 32 q / 8 KV heads of 128, RoPE theta 5e5,
    SwiGLU 14336, RMSNorm eps 1e-5, Q4_K projections, Q6_K head over 128256)
    with an f32 KV cache prefilled with N(0, 1) to `ctx` positions (kv_f16:
    soso's f16 KV instead, the same values rounded on upload); the step runs
    at position `ctx`.  The timed steps replay one HIP graph; eager=True launches
    them directly instead (for kernel tracers).  Returns (ms per token, bytes per
    token, token, ms per token of a host loop that launches a one-step graph and
    reads the token back each step -- None when eager)."""
    L, H, NH, NKV, HDIM, F, V = 32, 4096, 32, 8, 128, 14336, 128256
    qd, kvd = NH * HDIM, NKV * HDIM
    name = "llama8b"
    keys = []

    def norm(key, s):
        d = g.dev_alloc(H * 4)
        try:
            g.synth_normal(d, H, 1.0, seed, s)
            g.weight_from_dev(key, d, H * 4, F32, 1, H)
        finally:
            g.dev_free(d)

    s = 0
    for l in range(L):
        for nm, rows, cols in (("attn_norm", 1, H), ("q", qd, H), ("k", kvd, H), ("v", kvd, H), ("o", H, qd),
                               ("ffn_norm", 1, H), ("gate", F, H), ("up", F, H), ("down", H, F)):
            k = f"{name}.L{l}.{nm}"
            s += 1
            if rows == 1:
                norm(k, s)
            else:
                g.weight_synth(k, Q4K, rows, cols, seed, s)
            keys.append(k)
    norm(name + ".out_norm", 10000)
    g.weight_synth(name + ".head", Q6K, V, H, seed, 10001)
    keys += [name + ".out_norm", name + ".head"]
    cfg = dict(n_layers=L, hidden=H, n_heads=NH, n_kv_heads=NKV, head_dim=HDIM, ffn=F, vocab=V, ctx_max=ctx + 1,
               rope_theta=500000.0, rms_eps=1e-5, kv_f16=1 if kv_f16 else 0)
    g.decode_create(name, cfg, keys, drop_sources=True)
    x = g.dev_alloc(H * 4)
    tok = g.dev_alloc(4)
    try:
        if kv_f16:
            st = [g.dev_alloc((ctx + 1) * kvd * 4) for _ in range(2)]
            try:
                for l in range(L):
                    g.synth_normal(st[0], (ctx + 1) * kvd, 1.0, seed + 1, 2 * l)
                    g.synth_normal(st[1], (ctx + 1) * kvd, 1.0, seed + 1, 2 * l + 1)
                    g.decode_kv_upload(name, l, 0, (st[0], ctx + 1), (st[1], ctx + 1), rows_f32=True)
            finally:
                for p in st:
                    g.dev_free(p)
        else:
            for l in range(L):
                kd, vd = g.decode_kv_dev(name, l)
                g.synth_normal(kd, (ctx + 1) * kvd, 1.0, seed + 1, 2 * l)
                g.synth_normal(vd, (ctx + 1) * kvd, 1.0, seed + 1, 2 * l + 1)
        g.synth_normal(x, H, 1.0, seed + 2, 0)
        for _ in range(3):
            g.decode_step_dev(name, x, ctx, None, tok)
        g.sync()
        if eager:
            g.event_record(0)
            for _ in range(steps):
                g.decode_step_dev(name, x, ctx, None, tok)
            g.event_record(1)
            g.sync()
            ms = g.event_elapsed(0, 1) / steps
        else:
            ms = _timed_graph(g, lambda: [g.decode_step_dev(name, x, ctx, None, tok) for _ in range(steps)], steps)[0]
        token = int(g.d2h(tok, (1,), np.uint32)[0])
        # a serving loop's view: one step per graph launch, the host waiting
        # for each token (launch, sync and the 4-byte token read per step)
        host_ms = None
        if not eager:
            gid1 = _capture(g, lambda: g.decode_step_dev(name, x, ctx, None, tok))
            try:
                g.graph_launch(gid1)
                g.sync()
                n1 = max(10, steps // 2)
                t0 = time.perf_counter()
                for _ in range(n1):
                    g.graph_launch(gid1)
                    g.d2h(tok, (1,), np.uint32)
                host_ms = (time.perf_counter() - t0) * 1e3 / n1
            finally:
                g.graph_destroy(gid1)
        per_layer = (qd + 2 * kvd) * (H // 256) * 144 + H * (qd // 256) * 144 + 2 * F * (H // 256) * 144 \
            + H * (F // 256) * 144
        nbytes = L * per_layer + V * (H // 256) * 210 + L * 2 * (ctx + 1) * kvd * (2 if kv_f16 else 4) \
            + (2 * L + 1) * H * 4
        return ms, nbytes, token, host_ms
    finally:
        g.dev_free(x)
        g.dev_free(tok)
        g.decode_destroy(name)
        for k in keys:
            try:
                g.weight_drop(k)
            except Exception:  # noqa: BLE001 -- dropped with the sources
                pass


def time_decode_moe(g, steps, ctx=4096, seed=31, eager=False, qwen3_attn=True):
    """A Qwen3-30B-A3B-like decode step on the device (soso_hip_decode_create_ex
    with MoE layers; GpuDispatch::moe_capa): 48 layers of GQA attention (hidden
    2048, 32 query / 4 KV heads of 128, Q4_K q/k/v/o; with qwen3_attn, Qwen3's
    per-head QK RMSNorm (F32 attn_q_norm / attn_k_norm ~ N(0, 1)) and NeoX RoPE,
    otherwise the dense step's non-NeoX RoPE without QK norm) and an MoE FFN
    (f32 router ~ N(0, 0.02), 128 Q4_K experts of width 768, top-8), a Q6_K
    head over 151936, soso's f16 KV cache (the only KV type soso's device MoE
    layer takes) prefilled with N(0, 1) to `ctx` positions; the step runs at
    position `ctx`.  Timed like time_decode_8b.
    Returns (ms per token, bytes per token, token)."""
    L, H, NH, NKV, HDIM, E, F, K, V = 48, 2048, 32, 4, 128, 128, 768, 8, 151936
    qd, kvd = NH * HDIM, NKV * HDIM
    name = "qwen3moe"
    keys, moe_names, exp_keys = [], [], []
    s_ = 0

    def norm(key, st, n=H):
        d = g.dev_alloc(n * 4)
        try:
            g.synth_normal(d, n, 1.0, seed, st)
            g.weight_from_dev(key, d, n * 4, F32, 1, n)
        finally:
            g.dev_free(d)
    try:
        for l in range(L):
            for nm, rows, cols in (("attn_norm", 1, H), ("q", qd, H), ("k", kvd, H), ("v", kvd, H), ("o", H, qd),
                                   ("ffn_norm", 1, H)):
                k = f"{name}.L{l}.{nm}"
                s_ += 1
                if rows == 1:
                    norm(k, s_)
                else:
                    g.weight_synth(k, Q4K, rows, cols, seed, s_)
                keys.append(k)
            keys += [None, None, None]
            if qwen3_attn:
                for nm in ("q_norm", "k_norm"):
                    s_ += 1
                    norm(f"{name}.L{l}.{nm}", s_, HDIM)
                    keys.append(f"{name}.L{l}.{nm}")
            mk = f"{name}.L{l}.moe"
            ek = []
            for e in range(E):
                for j, (nm, r, c) in enumerate((("gate", F, H), ("up", F, H), ("down", H, F))):
                    k = f"{mk}.E{e}.{nm}"
                    g.weight_synth(k, Q4K, r, c, seed, 100000 + l * 1000 + 3 * e + j)
                    ek.append(k)
            d = g.dev_alloc(E * H * 4)
            try:
                g.synth_normal(d, E * H, 0.02, seed + 1, l)
                g.weight_from_dev(mk + ".router", d, E * H * 4, F32, E, H)
            finally:
                g.dev_free(d)
            g.moe_register(mk, mk + ".router", ek, E, H, F, K)
            moe_names.append(mk)
            exp_keys += ek + [mk + ".router"]
        norm(name + ".out_norm", 10000)
        g.weight_synth(name + ".head", Q6K, V, H, seed, 10001)
        keys += [name + ".out_norm", name + ".head"]
        cfg = dict(n_layers=L, hidden=H, n_heads=NH, n_kv_heads=NKV, head_dim=HDIM, ffn=F, vocab=V, ctx_max=ctx + 1,
                   rope_theta=1000000.0, rms_eps=1e-6, kv_f16=1)
        flags = 3 if qwen3_attn else 0  # SOSO_HIP_DECODE_QK_NORM | SOSO_HIP_DECODE_ROPE_NEOX
        assert g.decode_create(name, cfg, keys, drop_sources=True, moe_layers=moe_names, flags=flags), \
            g.last_error()
        x = g.dev_alloc(H * 4)
        tok = g.dev_alloc(4)
        st = [g.dev_alloc((ctx + 1) * kvd * 4) for _ in range(2)]
        try:
            for l in range(L):
                g.synth_normal(st[0], (ctx + 1) * kvd, 1.0, seed + 2, 2 * l)
                g.synth_normal(st[1], (ctx + 1) * kvd, 1.0, seed + 2, 2 * l + 1)
                g.decode_kv_upload(name, l, 0, (st[0], ctx + 1), (st[1], ctx + 1), rows_f32=True)
            g.synth_normal(x, H, 1.0, seed + 3, 0)
            for _ in range(3):
                g.decode_step_dev(name, x, ctx, None, tok)
            g.sync()
            if eager:
                g.event_record(0)
                for _ in range(steps):
                    g.decode_step_dev(name, x, ctx, None, tok)
                g.event_record(1)
                g.sync()
                ms = g.event_elapsed(0, 1) / steps
            else:
                ms = _timed_graph(g, lambda: [g.decode_step_dev(name, x, ctx, None, tok) for _ in range(steps)],
                                  steps)[0]
            token = int(g.d2h(tok, (1,), np.uint32)[0])
        finally:
            for p in st + [x, tok]:
                g.dev_free(p)
        attn = (qd + 2 * kvd) * (H // 256) * 144 + H * (qd // 256) * 144
        expert = 3 * F * (H // 256) * 144  # gate + up + down of one expert (F % 256 == 0 for down's rows)
        per_layer = attn + K * expert + E * H * 4 + 2 * H * 4 + (2 * HDIM * 4 if qwen3_attn else 0)
        nbytes = L * per_layer + V * (H // 256) * 210 + L * 2 * (ctx + 1) * kvd * 2 + H * 4
        return ms, nbytes, token
    finally:
        try:
            g.decode_destroy(name)
        except Exception:  # noqa: BLE001
            pass
        for k in [k for k in keys if k] + exp_keys:
            try:
                g.weight_drop(k)
            except Exception:  # noqa: BLE001 -- dropped with the sources
                pass


def copy_calibration(g, nbytes=512 << 20, reps=20):
    """A plain device-to-device copy of known size, for scaling rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters (run under --pmc)."""
    a, b = g.dev_alloc(nbytes), g.dev_alloc(nbytes)
    try:
        for _ in range(reps):
            g.d2d(b, a, nbytes)
        g.sync()
    finally:
        g.dev_free(a)
        g.dev_free(b)
    print(json.dumps({"copy_calibration_bytes": nbytes, "reps": reps}), flush=True)


CPU_ROTATE_BYTES = 512 << 20  # every CPU sample rotates this much: above any host last-level cache


def _cpu_copies(nbytes):
    return max(2, -(-CPU_ROTATE_BYTES // nbytes))


def _cpu_rate(fn, nbytes, budget):
    """Calls fn(i) for i = 0, 1, ... for `budget` seconds after one warm call;
    returns (GB/s of nbytes per call, calls)."""
    fn(0)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget:
        fn(n)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return round(nbytes / dt / 1e9, 2), n


def cpu_baseline(dtype, rows, cols, seconds, threads):
    """The AVX2+FMA restatement of soso's CPU matvec, contiguous row strips
    over `threads` host threads (HostPool), on a bounded sample over rotating
    copies (>= 512 MB).  Returns (GB/s, calls, ms per call, copies, the
    1-thread GB/s over the same copies)."""
    from oracle import oracle as orc
    nb = algo_bytes(dtype, rows, cols)
    copies = _cpu_copies(nb)
    ws = [orc.synth(dtype, rows, cols, 1, 1000 + i) for i in range(copies)]
    x = orc.normal(cols, 1.0, 1, 7)
    gbs, n = _cpu_rate(lambda i: orc.matvec(dtype, ws[i % copies], rows, cols, x, threads=threads, avx2=True), nb,
                       seconds)
    one, _ = _cpu_rate(lambda i: orc.matvec(dtype, ws[i % copies], rows, cols, x, threads=1, avx2=True), nb,
                       seconds / 4)
    return gbs, n, nb / gbs / 1e6, copies, one


def time_single_launch(g, dtype, rows, cols, reps=50, seed=1):
    """A graph holding ONE matvec launch, replayed `reps` times with a host
    synchronisation between replays; median event interval per replay in ms
    (the latency of an isolated call, launch included)."""
    key = f"bench.single.{dtype}.{rows}x{cols}"
    g.weight_synth(key, dtype, rows, cols, seed, 1000)
    x = g.dev_alloc(cols * 4)
    y = g.dev_alloc(rows * 4)
    try:
        g.synth_normal(x, cols, 1.0, seed, 7)
        gid = _capture(g, lambda: g.matvec_dev(key, x, y))
        try:
            ts = []
            for i in range(reps + 3):
                g.event_record(0)
                g.graph_launch(gid)
                g.event_record(1)
                g.sync()
                if i >= 3:
                    ts.append(g.event_elapsed(0, 1))
        finally:
            g.graph_destroy(gid)
        return float(np.median(ts))
    finally:
        g.sync()
        g.dev_free(x)
        g.dev_free(y)
        g.weight_drop(key)


def head_parity(g, threads, seed=1):
    """configs[2] checked in the bench run: the Q6_K head 128256 x 4096 on the
    GPU (matvec + argmax on the device) against the CPU restatement on the
    same seeded bytes (oracle/, `threads` host threads).  Returns the GPU and
    CPU argmax, the CPU logits' top-2 gap and the relative L2 of the logits."""
    from oracle import oracle as orc
    rows, cols = 128256, 4096
    key = "bench.head.parity"
    g.weight_synth(key, Q6K, rows, cols, seed, 1000)
    x = g.dev_alloc(cols * 4)
    y = g.dev_alloc(rows * 4)
    t = g.dev_alloc(4)
    try:
        g.synth_normal(x, cols, 1.0, seed, 7)
        g.matvec_dev(key, x, y)
        g.argmax_dev(y, rows, t)
        g.sync()
        logits = g.d2h(y, (rows,), np.float32)
        tok = int(g.d2h(t, (1,), np.uint32)[0])
    finally:
        g.dev_free(x)
        g.dev_free(y)
        g.dev_free(t)
        g.weight_drop(key)
    w = orc.synth(Q6K, rows, cols, seed, 1000)
    xc = orc.normal(cols, 1.0, seed, 7)
    ref = orc.matvec(Q6K, w, rows, cols, xc, threads=threads)
    ref_tok = int(orc.lib().or_argmax(ref.ctypes.data, rows))
    top2 = np.sort(ref)[-2:]
    return {"argmax_gpu": tok, "argmax_cpu": ref_tok, "argmax_equal": tok == ref_tok,
            "cpu_top2_gap": float(top2[1] - top2[0]), "logits_rel_l2": float(orc.rel_l2(logits, ref))}


def cpu_extra(seconds, threads):
    """The rest of the CPU baseline (oracle/ restatements, bounded samples,
    every one rotating >= 512 MB): host DRAM read bandwidth (STREAM-like sum,
    the CPU roofline), configs[0] Q8_0, and configs[2]'s head both ways soso
    could run it -- the restated Q6_K dequant+dot, and Q6_K requantized to
    Q8_0 (gguf2som/src/lib.rs:1592-1609) then AVX2 matvec_q8_0 -- on row
    samples.  GB/s are algorithmic bytes of the format the kernel reads."""
    from oracle import oracle as orc
    out = {}
    a = np.ones(1 << 28, np.float32)  # 1 GiB
    out["host_read_GB_s"], _ = _cpu_rate(lambda i: orc.lib().or_stream_read(a.ctypes.data, a.size, threads),
                                         a.nbytes, seconds / 4)
    del a
    nb8 = algo_bytes(Q8, 4096, 4096)
    c8 = _cpu_copies(nb8)
    ws = [orc.synth(Q8, 4096, 4096, 1, 1000 + i) for i in range(c8)]
    x = orc.normal(4096, 1.0, 1, 7)
    out["q8_0_4096x4096_GB_s"], _ = _cpu_rate(
        lambda i: orc.matvec(Q8, ws[i % c8], 4096, 4096, x, threads=threads, avx2=True), nb8, seconds / 4)
    del ws
    hr, cols = 16384, 4096  # head row samples: 55 MB of Q6_K, 75 MB of Q8_0 each
    ch = _cpu_copies(algo_bytes(Q6K, hr, cols))
    q6 = [orc.synth(Q6K, hr, cols, 1, 2000 + i) for i in range(ch)]
    out["q6_k_head_restated_GB_s"], _ = _cpu_rate(
        lambda i: orc.matvec(Q6K, q6[i % ch], hr, cols, x, threads=threads), algo_bytes(Q6K, hr, cols), seconds / 4)
    deq = np.empty(hr * cols, np.float32)
    q8 = []
    for w6 in q6:
        orc.lib().or_dequant_q6_k(w6.ctypes.data, w6.nbytes, deq.ctypes.data, deq.size)
        w8 = np.empty(hr * (cols // 32) * 36, np.uint8)
        orc.lib().or_quantize_q8_0(deq.ctypes.data, deq.size, w8.ctypes.data)
        q8.append(w8)
    del deq, q6
    out["q6_k_head_as_q8_0_GB_s"], _ = _cpu_rate(
        lambda i: orc.matvec(Q8, q8[i % ch], hr, cols, x, threads=threads, avx2=True), algo_bytes(Q8, hr, cols),
        seconds / 4)
    head_q8_ms = algo_bytes(Q8, 128256, 4096) / (out["q6_k_head_as_q8_0_GB_s"] * 1e9) * 1e3
    del q8
    out.update(cpu_more_configs(seconds, threads, head_q8_ms))
    out["sample"] = (f"~{1.75 * seconds:.0f} s in all, each sample rotating >= 512 MB: 1 GiB host read; {c8} Q8_0 "
                     f"4096x4096 copies; {ch} head row samples {hr}x{cols} (Q6_K restated, and requantized to Q8_0); "
                     f"MoE, decode layer and matmul samples as stated in their entries")
    return out


def cpu_more_configs(seconds, threads, head_q8_ms):
    """CPU baselines of configs[3] and configs[4] and of the 64-token matmul,
    the oracle's restatements on the same host threads: the MoE FFN of one
    token (forward_moe_ffn's CPU branch, layer.rs:1938-2105) over 2 rotated
    layers of 128 Q4_K experts; one dense 8B decode layer at position 4096 of
    an f32 KV cache (forward_layer, layer.rs:1092-1389) over 4 rotated layers,
    scaled to a token as 32 layers + the head as soso runs it (Q8_0, timed
    above); Q4_K 14336x4096 against 64 vectors (matvec_view_batch_par) over 4
    rotated copies."""
    import ctypes as C
    from oracle import oracle as orc
    out = {}
    E, H, F, K = 128, 2048, 768, 8
    layers = []
    for L in range(2):
        mats = [[orc.synth(Q4K, r, c, 11, L * 1000 + 3 * e + j) for j, (r, c) in enumerate(((F, H), (F, H), (H, F)))]
                for e in range(E)]
        tabs = [(C.c_void_p * E)(*[mats[e][j].ctypes.data for e in range(E)]) for j in range(3)]
        layers.append((orc.normal(E * H, 0.02, 12, L), mats, tabs))
    xs = orc.normal(8 * H, 1.0, 13, 1).reshape(8, H)
    y = np.empty(H, np.float32)
    idx = np.empty(K, np.int32)
    wgt = np.empty(K, np.float32)

    def moe(i):
        router, _, tabs = layers[i % 2]
        x = xs[(i // 2) % 8]
        orc.lib().or_moe_ffn(router.ctypes.data, E, H, F, K, C.cast(tabs[0], C.c_void_p), C.cast(tabs[1], C.c_void_p),
                             C.cast(tabs[2], C.c_void_p), Q4K, Q4K, x.ctypes.data, y.ctypes.data, idx.ctypes.data,
                             wgt.ctypes.data, threads, 1)
    moe_bytes = E * H * 4 + K * 3 * F * (H // 256) * 144
    gbs, n = _cpu_rate(moe, moe_bytes, seconds / 4)
    out["moe_qwen3_30b_a3b_batch1"] = {"us_per_layer": round(moe_bytes / (gbs * 1e9) * 1e6, 1), "GB_s": gbs,
                                       "sample": f"{n} tokens over 2 rotated layers of 128 Q4_K experts"}
    del layers
    Hd, NH, NKV, HDIM, Fd, ctx = 4096, 32, 8, 128, 14336, 4096
    qd, kvd = NH * HDIM, NKV * HDIM
    dec = []
    for L in range(4):
        w = [(1.0 + orc.normal(Hd, 0.1, 21, 100 * L)).astype(np.float32)]
        for j, (r, c) in enumerate(((qd, Hd), (kvd, Hd), (kvd, Hd), (Hd, qd))):
            w.append(orc.synth(Q4K, r, c, 21, 100 * L + 1 + j))
        w.append((1.0 + orc.normal(Hd, 0.1, 21, 100 * L + 5)).astype(np.float32))
        for j, (r, c) in enumerate(((Fd, Hd), (Fd, Hd), (Hd, Fd))):
            w.append(orc.synth(Q4K, r, c, 21, 100 * L + 6 + j))
        kc = orc.normal((ctx + 1) * kvd, 1.0, 22, 2 * L).reshape(ctx + 1, kvd)
        vc = orc.normal((ctx + 1) * kvd, 1.0, 22, 2 * L + 1).reshape(ctx + 1, kvd)
        dec.append((w, (C.c_void_p * 9)(*[a.ctypes.data for a in w]), kc, vc))
    hid = orc.normal(Hd, 1.0, 23, 0)

    def layer(i):
        _, ptrs, kc, vc = dec[i % 4]
        h = hid.copy()
        orc.lib().or_decode_layer(h.ctypes.data, C.cast(ptrs, C.c_void_p), Q4K, Hd, NH, NKV, HDIM, Fd, kc.ctypes.data,
                                  vc.ctypes.data, ctx, np.float32(500000.0), np.float32(1e-5), threads, 1)
    layer_bytes = ((qd + 2 * kvd) * Hd + Hd * qd + 3 * Fd * Hd) // 256 * 144 + 2 * (ctx + 1) * kvd * 4
    gbs, n = _cpu_rate(layer, layer_bytes, seconds / 4)
    layer_ms = layer_bytes / (gbs * 1e9) * 1e3
    tok_ms = 32 * layer_ms + head_q8_ms
    out["llama8b_decode_ctx4096"] = {
        "ms_per_layer": round(layer_ms, 3), "tokens_per_s_est": round(1e3 / tok_ms, 2), "GB_s": gbs,
        "sample": f"{n} layers over 4 rotated 8B layers (f32 KV at 4096 positions, attention as the oracle's "
                  f"scalar restatement over the head tasks); a token = 32 layers + the Q8_0 head ({head_q8_ms:.1f} ms)"}
    del dec
    rows, cols, nt = 14336, 4096, 64
    ws = [orc.synth(Q4K, rows, cols, 3, 3000 + i) for i in range(4)]
    xm = orc.normal(nt * cols, 1.0, 3, 9).reshape(nt, cols)
    ym = np.empty(nt * rows, np.float32)

    def mm(i):
        orc.lib().or_matmul_par(Q4K, ws[i % 4].ctypes.data, rows, cols, nt, xm.ctypes.data, ym.ctypes.data, threads, 1)
    mm_bytes = algo_bytes(Q4K, rows, cols)
    gbs, n = _cpu_rate(mm, mm_bytes, seconds / 4)
    mm_s = mm_bytes / (gbs * 1e9)
    out["q4_k_matmul_14336x4096_n64"] = {"us": round(mm_s * 1e6, 1),
                                         "gemm_TFLOP_s": round(2 * nt * rows * cols / mm_s / 1e12, 3),
                                         "sample": f"{n} calls over 4 rotated copies, as 64 per-vector AVX2 "
                                                   f"matvecs (soso's batched q4_k_nb kernel is not restated)"}
    return out


def load_traffic(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/), if recorded."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        return json.load(open(p)).get(name)
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="only the headline config")
    ap.add_argument("--copy-calibration", action="store_true", help="only run a 512 MiB D2D copy (PMC scaling)")
    ap.add_argument("--eager", action="store_true",
                    help="with --only: launch the timed steps directly instead of replaying a graph")
    ap.add_argument("--only", choices=["matvec", "q8_0", "down", "decode", "moe1", "moe32", "head", "matmul",
                                       "matmul_q8", "batch8", "decode_moe", "gdn", "readprobe"],
                    help="run one workload and print its own JSON line (for profiling runs)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the multi-GPU sharding is described in DESIGN.md, not run.", file=sys.stderr)
        sys.exit(2)

    from soso_amd.dispatch import HipGpu
    g = HipGpu(0)
    if args.copy_calibration:
        copy_calibration(g)
        g.close()
        return
    if args.only:
        if args.only == "matvec":
            ms, _ = time_matvec(g, Q4K, 14336, 4096, 16, max(args.steps, MIN_TIMED), args.warmup, eager=args.eager)
            res = {"q4_k_14336x4096_us": round(ms * 1e3, 3)}
        elif args.only == "q8_0":
            ms, _ = time_matvec(g, Q8, 4096, 4096, 28, max(args.steps, MIN_TIMED), args.warmup, eager=args.eager)
            res = {"q8_0_4096x4096_us": round(ms * 1e3, 3)}
        elif args.only == "down":
            ms, _ = time_matvec(g, Q4K, 4096, 14336, 16, max(args.steps, MIN_TIMED), args.warmup, eager=args.eager)
            res = {"q4_k_down_4096x14336_us": round(ms * 1e3, 3)}
        elif args.only == "head":
            ms, _ = time_matvec(g, Q6K, 128256, 4096, 2, max(20, args.steps // 10), min(args.warmup, 10),
                                eager=args.eager)
            res = {"q6_k_head_128256x4096_us": round(ms * 1e3, 3)}
        elif args.only == "decode_moe":
            ms, nb, tok = time_decode_moe(g, max(10, args.steps // 50), eager=args.eager)
            res = {"qwen3_30b_a3b_like_decode_ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
                   "bytes_per_token": int(nb), "greedy_token": tok}
        elif args.only == "batch8":
            ms = time_matmul(g, 14336, 4096, 8, 16, max(20, args.steps // 10), min(args.warmup, 10), eager=args.eager)
            res = {"q4_k_matmul_14336x4096_n8_us": round(ms * 1e3, 3)}
        elif args.only == "matmul_q8":
            ms = time_matmul(g, 4096, 4096, 64, 28, max(20, args.steps // 10), min(args.warmup, 10), eager=args.eager,
                             dtype=Q8)
            res = {"q8_0_matmul_4096x4096_n64_us": round(ms * 1e3, 3)}
        elif args.only == "matmul":
            ms = time_matmul(g, 14336, 4096, 64, 16, max(20, args.steps // 10), min(args.warmup, 10), eager=args.eager)
            res = {"q4_k_matmul_14336x4096_n64_us": round(ms * 1e3, 3)}
        elif args.only == "decode":
            print("decode: f32 KV", file=sys.stderr, flush=True)
            ms, _, tok, _ = time_decode_8b(g, max(10, args.steps // 50), eager=args.eager)
            print("decode: f16 KV", file=sys.stderr, flush=True)
            ms_h, _, tok_h, _ = time_decode_8b(g, max(10, args.steps // 50), kv_f16=True, eager=args.eager)
            res = {"llama8b_decode_ms_per_token": round(ms, 4), "greedy_token": tok,
                   "llama8b_decode_kv_f16_ms_per_token": round(ms_h, 4), "greedy_token_kv_f16": tok_h}
        elif args.only == "gdn":
            res = {}
            for n in (1, 64):
                ms, nb = time_gdn(g, n, max(40, args.steps // 10), eager=args.eager)
                res[f"gdn_block_n{n}_us"] = round(ms * 1e3, 3)
                res[f"gdn_block_n{n}_GB_s"] = round(nb / (ms * 1e-3) / 1e9, 1)
        elif args.only == "readprobe":
            nb = 14336 * ROW_BYTES[Q4K](4096)  # the headline's weight bytes
            nq = 4096 * ROW_BYTES[Q8](4096)  # configs[0]'s Q8_0 weight bytes
            small = time_read_probe(g, nb, 16, MIN_TIMED // 2, 20)
            q8 = time_read_probe(g, nq, 28, MIN_TIMED // 2, 20)
            big = time_read_probe(g, 512 << 20, 2, 20, 4)
            res = {"read_33MB_us": {f"{v}{k} {w}x{t}": round(ms * 1e3, 3) for (v, k, w, t), ms in small.items()},
                   "read_19MB_us": {f"{v}{k} {w}x{t}": round(ms * 1e3, 3) for (v, k, w, t), ms in q8.items()},
                   "read_512MB_us": {f"{v}{k} {w}x{t}": round(ms * 1e3, 3) for (v, k, w, t), ms in big.items()},
                   "bytes": [nb, nq, 512 << 20],
                   "key": "variant (gs: grid-stride, chunk: per-wavefront KiB stretches) and loads in flight, "
                          "workgroups per CU x threads"}
        else:
            n = 1 if args.only == "moe1" else 32
            ms, _, _, _ = time_moe(g, n, max(40, args.steps // 10), eager=args.eager)
            res = {f"moe_batch{n}_us_per_layer": round(ms * 1e3, 3)}
        g.close()
        print(json.dumps(res), flush=True)
        return
    rows, cols = 14336, 4096
    nbytes = algo_bytes(Q4K, rows, cols)
    timed = max(args.steps, MIN_TIMED)
    ms, ms_wall = time_matvec(g, Q4K, rows, cols, 16, timed, args.warmup)
    achieved = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "Q4_K matvec GB/s (% HBM peak) at 14336x4096; decode tok/s on 1 GPU",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "timed_launches": timed,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k",
        "data": "synthetic (seeded counter-based generator, BASELINE configs[1] distributions)",
        "config": {"workload": "Q4_K matvec 14336x4096, batch 1, 16 rotating resident copies (528 MB)",
                   "rows": rows, "cols": cols, "bytes_per_step": nbytes, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": load_traffic("q4k_14336x4096"),
                     "kernel_us": round(ms * 1e3, 3), "host_wall_us_per_step": round(ms_wall * 1e3, 3),
                     "graph_single_launch_us": round(time_single_launch(g, Q4K, rows, cols) * 1e3, 3),
                     "timed_as": (f"{timed} launches ({args.steps} asked for, at least {MIN_TIMED}) replayed "
                                  f"from one graph, behind {SPIN_MS:g} ms of untimed replays of the same launches")},
    }
    if not args.no_extra:
        extra = {}
        for name, dt, r, c, copies in (("q8_0_4096x4096", Q8, 4096, 4096, 28),
                                       ("q6_k_head_128256x4096", Q6K, 128256, 4096, 2),
                                       ("q4_k_down_4096x14336", Q4K, 4096, 14336, 16)):
            steps = max(20, args.steps // 10) if dt == Q6K else max(args.steps, MIN_TIMED)
            k_, _ = time_matvec(g, dt, r, c, copies, steps, min(args.warmup, 10))
            b = algo_bytes(dt, r, c)
            extra[name] = {"us_kernel": round(k_ * 1e3, 3), "GB_s": round(b / (k_ * 1e-3) / 1e9, 1),
                           "frac_hbm": round(b / (k_ * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes": b}
        # the same weight bytes read by a plain streaming kernel, best of its launch shapes:
        # the ceiling a dependent 33 MB launch can reach on this GPU
        nb = 14336 * ROW_BYTES[Q4K](4096)
        rd = time_read_probe(g, nb, 16, MIN_TIMED // 2, 20)
        (bv, bk, bw, bt), best = min(rd.items(), key=lambda kv: kv[1])
        rb = read_probe_bytes(bv, nb)
        extra["plain_read_33MB"] = {"us_kernel": round(best * 1e3, 3), "GB_s": round(rb / (best * 1e-3) / 1e9, 1),
                                    "frac_hbm": round(rb / (best * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes": rb,
                                    "shape": f"{'grid-stride' if bv.startswith('gs') else 'per-wavefront KiB stretches'}"
                                             f"{' (nontemporal loads)' if bv.endswith('_nt') else ''}, "
                                             f"{bk} loads in flight, {bw} workgroups per CU x {bt} threads "
                                             f"(best of {len(rd)} variants and shapes)",
                                    "headline_vs_read": round(best / ms, 4)}
        if not args.no_cpu:
            extra["q6_k_head_128256x4096"]["parity_vs_cpu"] = head_parity(g, args.cpu_threads)
        # the drop-in boundary's own cost per op (host buffers, synchronous)
        for name, dt, r, c in (("q8_0_4096x4096", Q8, 4096, 4096), ("q4_k_14336x4096", Q4K, 14336, 4096)):
            med, p10, p90 = time_host_matvec(g, dt, r, c)
            extra[f"host_call_{name}"] = {
                "us_per_call_median": round(med, 2), "us_p10": round(p10, 2), "us_p90": round(p90, 2),
                "what": "soso_hip_matvec on host x / y (upload, kernel, download, wait) on a resident weight; "
                        "the kernel alone is the entry of the same shape above"}
        mm_n = 64
        ms_mm = time_matmul(g, 14336, 4096, mm_n, 16, max(20, args.steps // 10), min(args.warmup, 10))
        b_mm = 14336 * (4096 // 256) * 144 + mm_n * 4096 * 4 + mm_n * 14336 * 4
        extra["q4_k_matmul_14336x4096_n64"] = {
            "us_kernel": round(ms_mm * 1e3, 3), "GB_s": round(b_mm / (ms_mm * 1e-3) / 1e9, 1),
            "frac_hbm": round(b_mm / (ms_mm * 1e-3) / 1e9 / PEAK_GBS, 4),
            "gemm_TFLOP_s": round(2 * mm_n * 14336 * 4096 / (ms_mm * 1e-3) / 1e12, 2), "tokens": mm_n,
            "path": "int8 MFMA 16x16x64 (exact codes x 3 digit planes of x)"}
        ms_q8 = time_matmul(g, 4096, 4096, mm_n, 28, max(20, args.steps // 10), min(args.warmup, 10), dtype=Q8)
        b_q8 = algo_bytes(Q8, 4096, 4096) + (mm_n - 1) * 4096 * 8
        extra["q8_0_matmul_4096x4096_n64"] = {
            "us_kernel": round(ms_q8 * 1e3, 3), "GB_s": round(b_q8 / (ms_q8 * 1e-3) / 1e9, 1),
            "frac_hbm": round(b_q8 / (ms_q8 * 1e-3) / 1e9 / PEAK_GBS, 4),
            "gemm_TFLOP_s": round(2 * mm_n * 4096 * 4096 / (ms_q8 * 1e-3) / 1e12, 2), "tokens": mm_n,
            "path": "int8 MFMA 16x16x32, one per 32-element block and 4-token tile"}
        for n in (1, 32):
            ms_m, b_m, u_m, _ = time_moe(g, n, max(40, args.steps // 10))
            extra[f"moe_qwen3_30b_a3b_batch{n}"] = {
                "us_per_layer": round(ms_m * 1e3, 3), "tokens_per_s_layer": round(n / (ms_m * 1e-3), 1),
                "GB_s": round(b_m / (ms_m * 1e-3) / 1e9, 1), "frac_hbm": round(b_m / (ms_m * 1e-3) / 1e9 / PEAK_GBS, 4),
                "bytes": int(b_m), "distinct_experts": round(u_m, 2)}
        for n in (1, 64):
            ms_g, b_g = time_gdn(g, n, max(40, args.steps // 10))
            extra[f"gdn_block_qwen3_next_like_n{n}"] = {
                "us": round(ms_g * 1e3, 3), "GB_s": round(b_g / (ms_g * 1e-3) / 1e9, 1),
                "frac_hbm": round(b_g / (ms_g * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes": int(b_g), "tokens": n,
                "shape": "16 q/k heads, 32 value heads of 128, conv kernel 4 (state 2 MiB, 8 rotated layers)"}
        ms_d, b_d, tok_d, host_d = time_decode_8b(g, max(10, args.steps // 10))
        extra["llama8b_decode_ctx4096"] = {
            "ms_per_token": round(ms_d, 4), "tokens_per_s": round(1e3 / ms_d, 1),
            "GB_s": round(b_d / (ms_d * 1e-3) / 1e9, 1), "frac_hbm": round(b_d / (ms_d * 1e-3) / 1e9 / PEAK_GBS, 4),
            "bytes_per_token": int(b_d), "greedy_token": tok_d,
            "host_loop_ms_per_token": round(host_d, 4)}
        ms_h, b_h, tok_h, _ = time_decode_8b(g, max(10, args.steps // 10), kv_f16=True)
        extra["llama8b_decode_ctx4096_kv_f16"] = {
            "ms_per_token": round(ms_h, 4), "tokens_per_s": round(1e3 / ms_h, 1),
            "GB_s": round(b_h / (ms_h * 1e-3) / 1e9, 1), "frac_hbm": round(b_h / (ms_h * 1e-3) / 1e9 / PEAK_GBS, 4),
            "bytes_per_token": int(b_h), "greedy_token": tok_h,
            "kv": "f16 (soso's KvDtype::F16), same N(0,1) prefill rounded on upload"}
        ms_q, b_q, tok_q = time_decode_moe(g, max(10, args.steps // 10))
        extra["qwen3_30b_a3b_like_decode_ctx4096_kv_f16"] = {
            "ms_per_token": round(ms_q, 4), "tokens_per_s": round(1e3 / ms_q, 1),
            "GB_s": round(b_q / (ms_q * 1e-3) / 1e9, 1), "frac_hbm": round(b_q / (ms_q * 1e-3) / 1e9 / PEAK_GBS, 4),
            "bytes_per_token": int(b_q), "greedy_token": tok_q,
            "model": "48 layers: GQA attention (32/4 heads of 128, hidden 2048, Q4_K, QK RMSNorm, NeoX RoPE) + MoE "
                     "FFN (128 Q4_K experts of 768, top-8, f32 router), Q6_K head over 151936, f16 KV"}
        # measured HBM traffic over algorithmic bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE, profiles/)
        for name, entry in extra.items():
            detail = load_traffic(name + "_detail")
            if isinstance(detail, dict) and "ratio" in detail:
                entry["traffic_ratio"] = detail["ratio"]
        line["configs"] = extra
    if not args.no_cpu:
        gbs, n, ms, copies, one = cpu_baseline(Q4K, rows, cols, args.cpu_seconds, args.cpu_threads)
        line["cpu_baseline"] = {"value": gbs, "unit": "GB/s", "cores": args.cpu_threads, "kind": "port",
                                "sample": f"{n} AVX2 Q4_K matvecs 14336x4096 over {copies} rotating copies "
                                          f"({ms:.2f} ms each) in ~{args.cpu_seconds:.0f} s",
                                "host_nproc": os.cpu_count(), "one_thread_GB_s": one}
        line["cpu_baseline"]["more"] = cpu_extra(args.cpu_seconds, args.cpu_threads)
    g.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
