"""The oracle's shared expert (or_moe_shared: GpuDispatch::moe_compartido,
gpu.rs:518-534, computed as bloque35.rs:952-985) pinned against the MoE FFN
restatement (or_moe_ffn, pinned by the MoE tests): a one-expert MoE FFN is
the shared expert with gate weight 1, so

- with pg_w = 0 the gate is sigmoid(0) = 1/2 exactly and the shared expert
  equals half the one-expert FFN bit for bit;
- with x . pg_w = 100 the gate rounds to 1.0f and the two are equal;
- in general the gate is sigmoid(x . pg_w) of the float64 dot.
"""
import numpy as np

Q4K = 3


def quant(orc, w):
    w = np.ascontiguousarray(w, np.float32).ravel()
    out = np.zeros(w.size // 256 * 144, np.uint8)
    orc.lib().or_quantize_q4_k(w.ctypes.data, w.size, out.ctypes.data)
    return out


def test_shared_expert_against_one_expert_ffn(orc):
    h, ffn, n = 512, 256, 3
    g = quant(orc, orc.normal(ffn * h, 0.05, 700, 1))
    u = quant(orc, orc.normal(ffn * h, 0.05, 700, 2))
    d = quant(orc, orc.normal(h * ffn, 0.05, 700, 3))
    xs = orc.normal(n * h, 1.0, 700, 4)
    router = np.zeros(h, np.float32)  # one expert: softmax weight 1 whatever the logit
    one = np.concatenate([orc.moe_ffn(router, 1, h, ffn, 1, [g], [u], [d], Q4K, Q4K, xs[t * h:(t + 1) * h])[0]
                          for t in range(n)])
    half = orc.moe_shared(np.zeros(h, np.float32), h, ffn, g, u, d, Q4K, Q4K, xs, n)
    assert np.array_equal(half, (one * np.float32(0.5)).astype(np.float32))
    # x_t . pg_w = 100 for every token (pg_w along the first token, scaled so
    # the others' dots differ): sigmoid rounds to 1 where the dot is large
    x0 = xs[:h].astype(np.float64)
    pg = (100.0 * x0 / np.dot(x0, x0)).astype(np.float32)
    full = orc.moe_shared(pg, h, ffn, g, u, d, Q4K, Q4K, xs[:h], 1)
    assert np.array_equal(full, one[:h])
    # general gate: sigmoid of the float64 dot
    pg = orc.normal(h, 0.05, 700, 5)
    got = orc.moe_shared(pg, h, ffn, g, u, d, Q4K, Q4K, xs, n)
    for t in range(n):
        s = 1.0 / (1.0 + np.exp(-np.dot(xs[t * h:(t + 1) * h].astype(np.float64), pg.astype(np.float64))))
        assert orc.rel_l2(got[t * h:(t + 1) * h], one[t * h:(t + 1) * h].astype(np.float64) * s) < 1e-6
