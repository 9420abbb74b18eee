"""A converted model directory (.som) through the GPU path: the device decode
step built from the mapped tensors, and an MoE layer registered from them.

Reference: MmapTensorSource::tensor_view / load_f32_range
(crates/soso-llm-core/src/source.rs:308-352) feeding GpuDispatch under the
tensors' own names, the tensor names and shapes Runtime checks
(runtime.rs:330-475), the dense decode step (layer.rs:1092-1389,
runtime.rs:1976-2028) and the MoE FFN (layer.rs:1732-2105).  The CPU side is
the oracle's composition used by the direct decode and MoE tests; the head is
stored as Q6_K, this build's dtype 13.

Bar: logits within relative L2 1e-5 and the greedy token identical at every
step; MoE indices identical, outputs within relative L2 1e-5.
"""
import numpy as np
import pytest

from soso_amd import som
from test_gpu_decode import Model
from test_gpu_moe import Layer, moe_dev

pytestmark = pytest.mark.gpu

NAMES = {"attn_norm": "attn_norm", "q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output",
         "ffn_norm": "ffn_norm", "gate": "ffn_gate", "up": "ffn_up", "down": "ffn_down"}


def test_decode_from_som_matches_cpu(gpu, orc, tmp_path):
    L, H, nh, nkv, F, V, ctx, theta, eps = 2, 512, 4, 2, 1024, 1000, 16, 500000.0, 1e-5
    m = Model(orc, L, H, nh, nkv, F, V, 77)
    m.head, m.head_dtype = orc.synth(som.DTYPE_Q6_K, V, H, 77, 9001), som.DTYPE_Q6_K
    embed = orc.normal(V * H, 1.0, 77, 9002).reshape(V, H)
    man = som.Manifest(name="gpu-dense", vocab_size=V, hidden_dim=H, num_layers=L, num_heads=nh, num_kv_heads=nkv,
                       ffn_dim=F, max_seq=ctx, rope_theta=theta, rms_eps=eps)
    man.fill_layers_from_globals()
    ts = []
    for l, lw in enumerate(m.layers):
        for k, nm in NAMES.items():
            dt, r, c = m.shapes(k)
            ts.append((f"L{l:02}.{nm}", dt, (c,) if r == 1 else (r, c), lw[k]))
    ts += [("output_norm", som.DTYPE_F32, (H,), m.out_norm), ("embed", som.DTYPE_F32, (V, H), embed),
           ("lm_head", som.DTYPE_Q6_K, (V, H), m.head)]
    som.write_model(str(tmp_path), man, ts)
    print(f"som decode L={L} H={H} heads={nh}/{nkv} V={V}", flush=True)
    with som.SomModel.open(str(tmp_path)) as s:
        dec = som.prepare_decode(gpu, s, "som.dense", ctx_max=ctx)
        try:
            kc = np.zeros((L, ctx, m.kvd), np.float32)
            vc = np.zeros((L, ctx, m.kvd), np.float32)
            tok = 5
            for pos in range(5):
                got, logits = dec.step(tok, pos, logits=True)
                ref, ref_tok = m.cpu_step(orc, embed[tok], kc, vc, pos, theta, eps)
                assert orc.rel_l2(logits, ref) < 1e-5, (pos, orc.rel_l2(logits, ref))
                top2 = np.sort(ref)[-2:]
                if top2[1] - top2[0] > 1e-3 * max(1.0, abs(float(top2[1]))):
                    assert got == ref_tok, pos
                tok = ref_tok
        finally:
            dec.close()


def test_qwen3_style_decode_from_som_matches_cpu(gpu, orc, tmp_path):
    """A converted model with Qwen3's attention (FLAG_QK_NORM | FLAG_ROPE_NEOX
    on every layer, attn_q_norm / attn_k_norm tensors) whose layer 1 is an MoE
    layer (router L01.ffn_gate_inp, experts L01.Eee.ffn_*): decode_plan maps it
    onto soso_hip_decode_create_ex with the MoE layer registered from the
    mapped tensors; five greedy steps against the oracle's composition."""
    from test_gpu_decode import MoeFfn
    L, H, nh, nkv, F, V, ctx, theta, eps = 2, 1024, 8, 2, 2048, 800, 16, 1000000.0, 1e-6
    m = Model(orc, L, H, nh, nkv, F, V, 78, qk_norm=True, neox=True)
    moe = MoeFfn(orc, 8, H, 512, 2, 79)
    embed = orc.normal(V * H, 1.0, 78, 9002).reshape(V, H)
    man = som.Manifest(name="gpu-qwen3ish", vocab_size=V, hidden_dim=H, num_layers=L, num_heads=nh,
                       num_kv_heads=nkv, ffn_dim=F, max_seq=ctx, rope_theta=theta, rms_eps=eps)
    man.fill_layers_from_globals()
    for ls in man.layers:
        ls.flags = som.FLAG_QK_NORM | som.FLAG_ROPE_NEOX
    ls = man.layers[1]
    ls.ffn_kind, ls.num_experts, ls.num_experts_per_tok, ls.moe_ffn_dim = som.FFN_MOE, moe.n_exp, moe.top_k, moe.ffn
    ts = []
    for l, lw in enumerate(m.layers):
        for k, nm in NAMES.items():
            if l == 1 and k in ("gate", "up", "down"):
                continue
            dt, r, c = m.shapes(k)
            ts.append((f"L{l:02}.{nm}", dt, (c,) if r == 1 else (r, c), lw[k]))
        ts += [(f"L{l:02}.attn_q_norm", som.DTYPE_F32, (128,), lw["q_norm"]),
               (f"L{l:02}.attn_k_norm", som.DTYPE_F32, (128,), lw["k_norm"])]
    ts.append(("L01.ffn_gate_inp", som.DTYPE_F32, (moe.n_exp, H), moe.router))
    for e in range(moe.n_exp):
        ts += [(f"L01.E{e:02}.ffn_gate", som.DTYPE_Q4_K, (moe.ffn, H), moe.gate[e]),
               (f"L01.E{e:02}.ffn_up", som.DTYPE_Q4_K, (moe.ffn, H), moe.up[e]),
               (f"L01.E{e:02}.ffn_down", som.DTYPE_Q4_K, (H, moe.ffn), moe.down[e])]
    ts += [("output_norm", som.DTYPE_F32, (H,), m.out_norm), ("embed", som.DTYPE_F32, (V, H), embed),
           ("lm_head", m.head_dtype, (V, H), m.head)]
    som.write_model(str(tmp_path), man, ts)
    print(f"som qwen3-style decode L={L} H={H} heads={nh}/{nkv} moe layer 1 E={moe.n_exp}", flush=True)
    with som.SomModel.open(str(tmp_path)) as s:
        # f32 KV: at position 0 the new row is the whole context, and an f16
        # rounding that lands on the other neighbour (the GPU's f32 row differs
        # from the CPU's in the last bits) would move the logits by ~5e-5
        dec = som.prepare_decode(gpu, s, "som.qwen3ish", ctx_max=ctx)
        try:
            kc = np.zeros((L, ctx, m.kvd), np.float32)
            vc = np.zeros((L, ctx, m.kvd), np.float32)
            tok = 7
            for pos in range(5):
                got, logits = dec.step(tok, pos, logits=True)
                ref, ref_tok = m.cpu_step(orc, embed[tok], kc, vc, pos, theta, eps, moe={1: moe})
                assert orc.rel_l2(logits, ref) < 1e-5, (pos, orc.rel_l2(logits, ref))
                top2 = np.sort(ref)[-2:]
                if top2[1] - top2[0] > 1e-3 * max(1.0, abs(float(top2[1]))):
                    assert got == ref_tok, pos
                tok = ref_tok
        finally:
            dec.close()
            for name, *_ in ts:
                gpu.weight_drop(name)


def test_moe_layer_from_som_matches_cpu(gpu, orc, tmp_path):
    E, H, FF, K, n = 8, 256, 512, 2, 3
    layer = Layer(orc, E, H, FF, K, 81)
    man = som.Manifest(name="gpu-moe", vocab_size=64, hidden_dim=H, num_layers=1, num_heads=2, num_kv_heads=1,
                       ffn_dim=FF, max_seq=16, num_experts=E, num_experts_per_tok=K, moe_ffn_dim=FF)
    man.fill_layers_from_globals()
    ts = [("L00.ffn_gate_inp", som.DTYPE_F32, (E, H), layer.router)]
    for e in range(E):
        ts += [(f"L00.E{e:02}.ffn_gate", som.DTYPE_Q4_K, (FF, H), layer.gate[e]),
               (f"L00.E{e:02}.ffn_up", som.DTYPE_Q4_K, (FF, H), layer.up[e]),
               (f"L00.E{e:02}.ffn_down", som.DTYPE_Q4_K, (H, FF), layer.down[e])]
    som.write_model(str(tmp_path), man, ts)
    print(f"som moe E={E} H={H} ffn={FF} top{K} n={n}", flush=True)
    with som.SomModel.open(str(tmp_path)) as s:
        key = som.prepare_moe_layer(gpu, s, 0)
        try:
            layer.name = key
            xs = orc.normal(n * H, 1.0, 82, 1)
            out, idx, wgt = moe_dev(gpu, layer, xs)
            for t in range(n):
                ref, ri, rw = layer.cpu(orc, xs[t * H:(t + 1) * H])
                assert np.array_equal(idx[t], ri), (t, idx[t], ri)
                assert orc.rel_l2(wgt[t], rw) < 1e-5
                assert orc.rel_l2(out[t], ref) < 1e-5, (t, orc.rel_l2(out[t], ref))
        finally:
            for name, *_ in ts:
                gpu.weight_drop(name)


def test_prepare_decode_declined_leaves_nothing_resident(gpu, orc, tmp_path):
    """A model that passes decode_plan but that the device step declines
    (layer 1's MoE experts have Q8_0 down projections, which the step's
    single-token MoE path does not run): prepare_decode raises, and every
    weight it uploaded and the MoE layer it registered are gone again, so a
    caller that falls back to the CPU keeps no device memory for it."""
    L, H, nh, nkv, F, V, ctx = 2, 512, 4, 2, 1024, 300, 16
    m = Model(orc, L, H, nh, nkv, F, V, 83)
    E, FF, K = 4, 256, 2
    moe = Layer(orc, E, H, FF, K, 84, dt_down=som.DTYPE_Q8_0)
    embed = orc.normal(V * H, 1.0, 83, 9002).reshape(V, H)
    man = som.Manifest(name="gpu-declined", vocab_size=V, hidden_dim=H, num_layers=L, num_heads=nh,
                       num_kv_heads=nkv, ffn_dim=F, max_seq=ctx, rope_theta=5e5, rms_eps=1e-5)
    man.fill_layers_from_globals()
    ls = man.layers[1]
    ls.ffn_kind, ls.num_experts, ls.num_experts_per_tok, ls.moe_ffn_dim = som.FFN_MOE, E, K, FF
    ts = []
    for l, lw in enumerate(m.layers):
        for k, nm in NAMES.items():
            if l == 1 and k in ("gate", "up", "down"):
                continue
            dt, r, c = m.shapes(k)
            ts.append((f"L{l:02}.{nm}", dt, (c,) if r == 1 else (r, c), lw[k]))
    ts.append(("L01.ffn_gate_inp", som.DTYPE_F32, (E, H), moe.router))
    for e in range(E):
        ts += [(f"L01.E{e:02}.ffn_gate", som.DTYPE_Q4_K, (FF, H), moe.gate[e]),
               (f"L01.E{e:02}.ffn_up", som.DTYPE_Q4_K, (FF, H), moe.up[e]),
               (f"L01.E{e:02}.ffn_down", som.DTYPE_Q8_0, (H, FF), moe.down[e])]
    ts += [("output_norm", som.DTYPE_F32, (H,), m.out_norm), ("embed", som.DTYPE_F32, (V, H), embed),
           ("lm_head", m.head_dtype, (V, H), m.head)]
    som.write_model(str(tmp_path), man, ts)
    before = gpu.stats()
    with som.SomModel.open(str(tmp_path)) as s:
        som.decode_plan(s)  # the plan itself accepts the model
        with pytest.raises(som.SomError, match="declined"):
            som.prepare_decode(gpu, s, "som.declined", ctx_max=ctx)
    after = gpu.stats()
    assert after["weights_resident"] == before["weights_resident"], (before, after)
    assert after["weight_bytes_resident"] == before["weight_bytes_resident"]
    # no key of the model is resident any more: dropping one finds nothing
    for name, *_ in ts:
        assert not gpu.weight_drop(name), name
