"""The oracle's Gated DeltaNet restatement (or_gdn_step, or_gdn_gates,
or_gdn_block: GpuDispatch::gdn_bloque, gpu.rs:577-599, computed as
bloque35.rs:372-465 / arch.rs:358-415) pinned by what the mathematics fixes:

- gdn_step from a zero state is the rank-one update S = beta k v^T with
  out = beta (k . q) v; with g = 1 and beta = 0 the state stays and
  out = S^T q; in general it equals the matrix form delta = beta (v - g S^T k),
  S' = g S + k delta^T, out = S'^T q evaluated in float64;
- sigmoid / softplus / l2_normalize at known values;
- the whole block against an independent float64 formulation (conv as a
  matrix product over the history window, heads normalised by numpy norms,
  the recurrence in matrix form), and a block of n tokens equal, bit for
  bit, to n one-token blocks with the conv history carried between them.
"""
import numpy as np
import pytest


def f64_block(hist, conv, z, decay, beta, norm, state, n, n_k, n_v, d, kernel, eps):
    C = 2 * n_k * d + n_v * d
    qk, vd = n_k * d, n_v * d
    H = hist.astype(np.float64).reshape(kernel - 1 + n, C)
    W = conv.astype(np.float64).reshape(C, kernel)
    S = state.astype(np.float64).reshape(n_v, d, d).copy()
    out = np.zeros((n, vd))
    for t in range(n):
        u = np.einsum("ck,kc->c", W, H[t:t + kernel])
        u = u / (1.0 + np.exp(-u))
        for h in range(n_k):
            for off in (0, qk):
                seg = u[off + h * d:off + (h + 1) * d]
                u[off + h * d:off + (h + 1) * d] = seg / np.sqrt(np.dot(seg, seg) + eps)
        u[:qk] /= np.sqrt(d)
        for vh in range(n_v):
            kh = vh % n_k
            q, k, v = u[kh * d:(kh + 1) * d], u[qk + kh * d:qk + (kh + 1) * d], u[2 * qk + vh * d:2 * qk + (vh + 1) * d]
            g, b = float(decay[t * n_v + vh]), float(beta[t * n_v + vh])
            delta = b * (v - g * (S[vh].T @ k))
            S[vh] = g * S[vh] + np.outer(k, delta)
            o = S[vh].T @ q
            o = o / np.sqrt(np.mean(o * o) + eps) * norm.astype(np.float64)
            zz = z[t * vd + vh * d:t * vd + (vh + 1) * d].astype(np.float64)
            out[t, vh * d:(vh + 1) * d] = o * zz / (1.0 + np.exp(-zz))
    return out.ravel(), S.ravel()


def rnd(orc, n, sigma, seed, stream):
    return orc.normal(n, sigma, seed, stream)


def test_gdn_step_closed_forms(orc):
    L = orc.lib()
    d = 64
    q, k, v = (rnd(orc, d, 1.0, 500, s) for s in (1, 2, 3))
    out = np.zeros(d, np.float32)
    S = np.zeros(d * d, np.float32)
    beta = 0.75
    L.or_gdn_step(S.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, d, np.float32(0.3), np.float32(beta),
                  out.ctypes.data)
    want_S = beta * np.outer(k.astype(np.float64), v.astype(np.float64))
    assert np.allclose(S.reshape(d, d), want_S, rtol=1e-6, atol=1e-7)
    assert orc.rel_l2(out, beta * float(np.dot(k.astype(np.float64), q)) * v.astype(np.float64)) < 1e-6
    # g = 1, beta = 0: the state stays, out = S^T q
    S0 = rnd(orc, d * d, 0.1, 500, 4)
    S1 = S0.copy()
    L.or_gdn_step(S1.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, d, np.float32(1.0), np.float32(0.0),
                  out.ctypes.data)
    assert np.array_equal(S1, S0)
    assert orc.rel_l2(out, S0.reshape(d, d).astype(np.float64).T @ q.astype(np.float64)) < 1e-6


def test_gdn_step_matches_matrix_form(orc):
    L = orc.lib()
    d = 128
    q, k, v = (rnd(orc, d, 1.0, 501, s) for s in (1, 2, 3))
    S = rnd(orc, d * d, 0.05, 501, 4)
    g, b = 0.9, 0.4
    S64 = S.reshape(d, d).astype(np.float64)
    delta = b * (v - g * (S64.T @ k))
    S2 = g * S64 + np.outer(k, delta)
    out = np.zeros(d, np.float32)
    L.or_gdn_step(S.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, d, np.float32(g), np.float32(b),
                  out.ctypes.data)
    assert orc.rel_l2(S, S2) < 1e-6
    assert orc.rel_l2(out, S2.T @ q) < 1e-6


def test_gdn_scalar_functions(orc):
    L = orc.lib()
    assert L.or_sigmoid(np.float32(0.0)) == np.float32(0.5)
    assert abs(L.or_softplus(np.float32(0.0)) - np.log(2.0)) < 1e-7
    assert L.or_softplus(np.float32(25.0)) == np.float32(25.0)  # above 20 passes through
    assert abs(L.or_softplus(np.float32(-30.0)) - np.exp(-30.0)) < 1e-18
    x = np.array([3.0, 4.0], np.float32)
    L.or_l2_normalize(x.ctypes.data, 2, np.float32(0.0))
    assert np.allclose(x, [0.6, 0.8], rtol=1e-7)
    alpha, braw = rnd(orc, 6, 2.0, 502, 1), rnd(orc, 6, 2.0, 502, 2)
    dt, a = rnd(orc, 3, 1.0, 502, 3), -np.abs(rnd(orc, 3, 1.0, 502, 4))
    dec, bet = np.zeros(6, np.float32), np.zeros(6, np.float32)
    L.or_gdn_gates(alpha.ctypes.data, braw.ctypes.data, dt.ctypes.data, a.ctypes.data, 2, 3, dec.ctypes.data,
                   bet.ctypes.data)
    sp = np.log1p(np.exp(alpha.astype(np.float64).reshape(2, 3) + dt))
    assert orc.rel_l2(dec, np.exp(sp * a).ravel()) < 1e-6
    assert orc.rel_l2(bet, 1.0 / (1.0 + np.exp(-braw.astype(np.float64)))) < 1e-6


def make_block(orc, n, n_k, n_v, d, kernel, seed):
    C = 2 * n_k * d + n_v * d
    hist = rnd(orc, (kernel - 1 + n) * C, 1.0, seed, 1)
    conv = rnd(orc, C * kernel, 0.5, seed, 2)
    z = rnd(orc, n * n_v * d, 1.0, seed, 3)
    decay = np.exp(-np.abs(rnd(orc, n * n_v, 0.3, seed, 4))).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-rnd(orc, n * n_v, 1.0, seed, 5)))).astype(np.float32)
    norm = (1.0 + rnd(orc, d, 0.1, seed, 6)).astype(np.float32)
    state = rnd(orc, n_v * d * d, 0.05, seed, 7)
    return hist, conv, z, decay, beta, norm, state


@pytest.mark.parametrize("n,n_k,n_v,d,kernel", [(1, 2, 4, 32, 4), (3, 2, 4, 128, 4), (2, 1, 3, 16, 1)])
def test_gdn_block_matches_float64_form(orc, n, n_k, n_v, d, kernel):
    eps = 1e-6
    hist, conv, z, decay, beta, norm, state = make_block(orc, n, n_k, n_v, d, kernel, 510 + n)
    out, st = orc.gdn_block(hist, conv, z, decay, beta, norm, state, n, n_k, n_v, d, kernel, eps)
    ro, rs = f64_block(hist, conv, z, decay, beta, norm, state, n, n_k, n_v, d, kernel, eps)
    assert orc.rel_l2(out, ro) < 1e-5, orc.rel_l2(out, ro)
    assert orc.rel_l2(st, rs) < 1e-5, orc.rel_l2(st, rs)


def test_gdn_block_equals_token_by_token(orc):
    """n tokens at once = n one-token calls with the conv history carried
    (the last kernel - 1 rows) and the state carried: bit for bit."""
    n, n_k, n_v, d, kernel, eps = 4, 2, 4, 64, 4, 1e-6
    C = 2 * n_k * d + n_v * d
    hist, conv, z, decay, beta, norm, state = make_block(orc, n, n_k, n_v, d, kernel, 520)
    out, st = orc.gdn_block(hist, conv, z, decay, beta, norm, state, n, n_k, n_v, d, kernel, eps)
    H = hist.reshape(kernel - 1 + n, C)
    s1 = state.copy()
    for t in range(n):
        o1, s1 = orc.gdn_block(H[t:t + kernel].ravel(), conv, z[t * n_v * d:(t + 1) * n_v * d],
                               decay[t * n_v:(t + 1) * n_v], beta[t * n_v:(t + 1) * n_v], norm, s1, 1, n_k, n_v, d,
                               kernel, eps)
        assert np.array_equal(o1, out[t * n_v * d:(t + 1) * n_v * d]), t
    assert np.array_equal(s1, st)
