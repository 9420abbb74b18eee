"""HipGpu -- soso's GpuDispatch (crates/soso-llm-core/src/gpu.rs:338-737) over
the C ABI of libsoso_hip.so, with numpy arrays in place of Rust slices.

Method names and return values follow the trait:
  matvec / matmul / router_topk -> True (computed), False (declined: the
  caller computes on the CPU); errors raise HipError.
  matvec_lote / expertos_bloque fill `hecho` like the trait does.
The decline-forever residency cache, the key-based uploads and the
synchronous semantics live in the native library.
"""
import ctypes as C

import numpy as np

from . import abi


def _key(k):
    b = k.encode() if isinstance(k, str) else bytes(k)
    return b, len(b)


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def _raw(w):
    """The tensor's bytes as soso holds them (TensorView.bytes): F32 weights are
    viewed, not converted."""
    return None if w is None else np.ascontiguousarray(w).reshape(-1).view(np.uint8)


class HipGpu:
    def __init__(self, device=0, vram_budget=0):
        self.lib = abi.load()
        h = C.c_void_p()
        rc = self.lib.soso_hip_create(device, vram_budget, C.byref(h))
        if rc != 0:
            raise abi.HipError(f"soso_hip_create({device}) failed: {rc}")
        self.h = h
        self._decode_cfg = {}  # model key -> the cfg it was created with (decode_token's buffer sizes)

    # -- lifetime ------------------------------------------------------------
    def close(self):
        if self.h:
            self.lib.soso_hip_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # -- helpers ---------------------------------------------------------------
    def last_error(self):
        return self.lib.soso_hip_last_error(self.h).decode(errors="replace")

    def _rc(self, rc, what):
        if rc < 0:
            raise abi.HipError(f"{what}: rc={rc}: {self.last_error()}")
        return rc == abi.OK

    # -- GpuDispatch -----------------------------------------------------------
    def available(self):
        return bool(self.lib.soso_hip_available(self.h))

    def dtype_soportado(self, dtype):
        return bool(self.lib.soso_hip_dtype_supported(self.h, dtype))

    def stats(self):
        s = abi.Stats()
        self.lib.soso_hip_stats(self.h, C.byref(s))
        return {f: getattr(s, f) for f, _ in abi.Stats._fields_}

    def matvec(self, key, w, dtype, rows, cols, x, out):
        """gpu.rs:432-440; overwrites `out` (float32, rows) on success."""
        k, kl = _key(key)
        wb = _raw(w)
        x = _f32(x)
        assert out.dtype == np.float32 and out.flags.c_contiguous and out.size == rows
        rc = self.lib.soso_hip_matvec(self.h, k, kl, None if wb is None else wb.ctypes.data,
                                      0 if wb is None else wb.size, dtype, rows, cols,
                                      x.ctypes.data, out.ctypes.data)
        return self._rc(rc, f"matvec {key}")

    def matmul(self, key, w, dtype, rows, cols, n, x, out):
        """gpu.rs:443-455: out[n x rows] = x[n x cols] . W^T."""
        k, kl = _key(key)
        wb = _raw(w)
        x = _f32(x)
        assert out.dtype == np.float32 and out.flags.c_contiguous and out.size == n * rows
        rc = self.lib.soso_hip_matmul(self.h, k, kl, None if wb is None else wb.ctypes.data,
                                      0 if wb is None else wb.size, dtype, rows, cols, n,
                                      x.ctypes.data, out.ctypes.data)
        return self._rc(rc, f"matmul {key}")

    def matvec_lote(self, ops, hecho):
        """gpu.rs:694-701.  ops: list of dicts key/w/dtype/rows/cols/x/out."""
        keep = []
        arr = (abi.Op * len(ops))()
        for i, op in enumerate(ops):
            k, kl = _key(op["key"])
            wb = _raw(op.get("w"))
            x = _f32(op["x"])
            keep += [k, wb, x]
            arr[i] = abi.Op(k, kl, None if wb is None else wb.ctypes.data, 0 if wb is None else wb.size,
                            op["dtype"], op["rows"], op["cols"], x.ctypes.data, op["out"].ctypes.data)
        done = np.zeros(len(ops), dtype=np.uint8)
        rc = self.lib.soso_hip_matvec_batch(self.h, arr, len(ops), done.ctypes.data)
        for i in range(len(ops)):
            hecho[i] = hecho[i] or bool(done[i])
        return self._rc(rc, "matvec_lote") if rc < 0 else rc

    def router_topk(self, key, w, xs, n, h, n_exp, top_k, idx, pesos):
        """gpu.rs:480-494; idx int32 (n*top_k), pesos float32 (n*top_k)."""
        k, kl = _key(key)
        w = None if w is None else _f32(w)
        xs = _f32(xs)
        rc = self.lib.soso_hip_router_topk(self.h, k, kl, None if w is None else w.ctypes.data, xs.ctypes.data,
                                           n, h, n_exp, top_k, idx.ctypes.data, pesos.ctypes.data)
        return self._rc(rc, "router_topk")

    def expertos_bloque(self, xs, n, h, ffn, top_k, pesos, exps, suma, hecho):
        """gpu.rs:461-475.  exps: list of dicts with keys (3 names), w (3 byte
        arrays or None), dtype (3 codes), tokens, destinos."""
        xs = _f32(xs)
        pesos = _f32(pesos)
        keep = []
        arr = (abi.Expert * len(exps))()
        for i, e in enumerate(exps):
            ex = abi.Expert()
            for j in range(3):
                k, kl = _key(e["claves"][j])
                wb = None
                if e.get("w") is not None and e["w"][j] is not None:
                    wb = _raw(e["w"][j])
                keep += [k, wb]
                ex.keys[j] = k
                ex.key_lens[j] = kl
                ex.w[j] = None if wb is None else wb.ctypes.data
                ex.w_len[j] = 0 if wb is None else wb.size
                ex.dtype[j] = 0 if wb is None else e["dtype"][j]
            tok = np.ascontiguousarray(e["tokens"], dtype=np.uint32)
            dst = np.ascontiguousarray(e["destinos"], dtype=np.uint32)
            keep += [tok, dst]
            ex.tokens = tok.ctypes.data
            ex.targets = dst.ctypes.data
            ex.n_tokens = tok.size
            ex.shared = int(e.get("compartido", False))
            arr[i] = ex
        done = np.zeros(len(exps), dtype=np.uint8)
        assert suma.dtype == np.float32 and suma.size == n * h
        rc = self.lib.soso_hip_experts_block(self.h, xs.ctypes.data, n, h, ffn, top_k, pesos.ctypes.data, arr,
                                             len(exps), suma.ctypes.data, done.ctypes.data)
        for i in range(len(exps)):
            hecho[i] = hecho[i] or bool(done[i])
        return self._rc(rc, "expertos_bloque") if rc < 0 else rc

    def moe_compartido(self, claves, vistas, dtypes, pg_w, xs, n, h, ffn):
        """gpu.rs:518-534: the shared expert of the block (3 keys, 3 byte arrays
        or None when resident, 3 dtype codes; pg_w: h f32), kept on the device
        and added by the next expertos_bloque call for the same block."""
        keep = []
        keys = (C.c_char_p * 3)()
        lens = (C.c_size_t * 3)()
        ws = (C.c_void_p * 3)()
        wl = (C.c_size_t * 3)()
        dt = (C.c_uint8 * 3)()
        for j in range(3):
            k, kl = _key(claves[j])
            keys[j], lens[j] = k, kl
            wb = None if vistas is None or vistas[j] is None else _raw(vistas[j])
            keep += [k, wb]
            ws[j] = None if wb is None else wb.ctypes.data
            wl[j] = 0 if wb is None else wb.size
            dt[j] = 0 if wb is None else dtypes[j]
        pg = _f32(pg_w)
        xs = _f32(xs)
        rc = self.lib.soso_hip_moe_shared(self.h, C.cast(keys, C.c_void_p), C.cast(lens, C.c_void_p),
                                          C.cast(ws, C.c_void_p), C.cast(wl, C.c_void_p), C.cast(dt, C.c_void_p),
                                          pg.ctypes.data, xs.ctypes.data, n, h, ffn)
        return self._rc(rc, "moe_compartido")

    # -- device-resident helpers (benchmarks, decode step, tests) ----------------
    def dev_alloc(self, nbytes):
        p = C.c_void_p()
        self._rc(self.lib.soso_hip_dev_alloc(self.h, nbytes, C.byref(p)), "dev_alloc")
        return p.value

    def dev_free(self, p):
        self._rc(self.lib.soso_hip_dev_free(self.h, p), "dev_free")

    def h2d(self, dst, arr):
        arr = np.ascontiguousarray(arr)
        self._rc(self.lib.soso_hip_h2d(self.h, dst, arr.ctypes.data, arr.nbytes), "h2d")

    def d2h(self, src, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        self._rc(self.lib.soso_hip_d2h(self.h, out.ctypes.data, src, out.nbytes), "d2h")
        return out

    def sync(self):
        self._rc(self.lib.soso_hip_sync(self.h), "sync")

    def weight_from_dev(self, key, raw_dev, w_len, dtype, rows, cols):
        k, kl = _key(key)
        return self._rc(self.lib.soso_hip_weight_from_dev(self.h, k, kl, raw_dev, w_len, dtype, rows, cols),
                        f"weight_from_dev {key}")

    def weight_synth(self, key, dtype, rows, cols, seed, stream):
        k, kl = _key(key)
        return self._rc(self.lib.soso_hip_weight_synth(self.h, k, kl, dtype, rows, cols, seed, stream),
                        f"weight_synth {key}")

    def synth_raw(self, dst, dtype, rows, cols, seed, stream):
        return self._rc(self.lib.soso_hip_synth_raw(self.h, dst, dtype, rows, cols, seed, stream), "synth_raw")

    def synth_normal(self, dst, n, sigma, seed, stream):
        return self._rc(self.lib.soso_hip_synth_normal(self.h, dst, n, sigma, seed, stream), "synth_normal")

    def read_probe(self, src_dev, nbytes, wg_per_cu, threads, out_dev, out_len, loads=1, chunked=False, stream=False):
        return self._rc(self.lib.soso_hip_read_probe(self.h, src_dev, nbytes, wg_per_cu, threads, loads,
                                                     (1 if chunked else 0) | (2 if stream else 0), out_dev, out_len),
                        "read_probe")

    def weight_drop(self, key):
        k, kl = _key(key)
        return self._rc(self.lib.soso_hip_weight_drop(self.h, k, kl), "weight_drop")

    def matvec_dev(self, key, x_dev, y_dev):
        k, kl = _key(key)
        return self._rc(self.lib.soso_hip_matvec_dev(self.h, k, kl, x_dev, y_dev), f"matvec_dev {key}")

    def matmul_dev(self, key, n, x_dev, y_dev):
        k, kl = _key(key)
        return self._rc(self.lib.soso_hip_matmul_dev(self.h, k, kl, n, x_dev, y_dev), f"matmul_dev {key}")

    def dequant_dev(self, key, out_dev):
        k, kl = _key(key)
        return self._rc(self.lib.soso_hip_dequant_dev(self.h, k, kl, out_dev), f"dequant_dev {key}")

    def argmax_dev(self, x_dev, n, idx_dev):
        return self._rc(self.lib.soso_hip_argmax_dev(self.h, x_dev, n, idx_dev), "argmax_dev")

    def timer_start(self):
        self._rc(self.lib.soso_hip_timer_start(self.h), "timer_start")

    def timer_stop(self):
        ms = C.c_float()
        self._rc(self.lib.soso_hip_timer_stop(self.h, C.byref(ms)), "timer_stop")
        return ms.value

    def event_record(self, slot):
        self._rc(self.lib.soso_hip_event_record(self.h, slot), "event_record")

    def event_elapsed(self, a, b):
        ms = C.c_float()
        self._rc(self.lib.soso_hip_event_elapsed(self.h, a, b, C.byref(ms)), "event_elapsed")
        return ms.value

    def graph_begin(self):
        self._rc(self.lib.soso_hip_graph_begin(self.h), "graph_begin")

    def graph_end(self):
        gid = C.c_int()
        self._rc(self.lib.soso_hip_graph_end(self.h, C.byref(gid)), "graph_end")
        return gid.value

    def graph_launch(self, gid):
        self._rc(self.lib.soso_hip_graph_launch(self.h, gid), "graph_launch")

    def graph_destroy(self, gid):
        self._rc(self.lib.soso_hip_graph_destroy(self.h, gid), "graph_destroy")

    def d2d(self, dst, src, nbytes):
        self._rc(self.lib.soso_hip_d2d(self.h, dst, src, nbytes), "d2d")

    # -- MoE FFN resident on the device (the FFN half of GpuDispatch::moe_capa) --
    def moe_register(self, layer_key, router_key, expert_keys, n_exp, hdim, ffn, top_k):
        """expert_keys: 3*n_exp names (gate_e, up_e, down_e for e = 0..n_exp-1),
        or None: the router alone, the experts staying on the host (a decode
        model's cpu_moe layer)."""
        lk, ll = _key(layer_key)
        rk, rl = _key(router_key)
        if expert_keys is None:
            arr = lens = None
        else:
            enc = [k.encode() for k in expert_keys]
            arr = C.cast((C.c_char_p * len(enc))(*enc), C.c_void_p)
            lens = C.cast((C.c_size_t * len(enc))(*[len(k) for k in enc]), C.c_void_p)
        return self._rc(self.lib.soso_hip_moe_register(self.h, lk, ll, rk, rl, arr, lens, n_exp, hdim, ffn, top_k),
                        f"moe_register {layer_key}")

    def moe_ffn_dev(self, layer_key, x_dev, n, out_dev, idx_dev=None, wgt_dev=None):
        k, kl = _key(layer_key)
        return self._rc(self.lib.soso_hip_moe_ffn_dev(self.h, k, kl, x_dev, n, out_dev, idx_dev, wgt_dev),
                        f"moe_ffn_dev {layer_key}")

    def moe_ffn_dev_noalloc(self, layer_key, x_dev, n, out_dev, idx_dev=None, wgt_dev=None):
        """moe_ffn_dev with the library's fixed scratch array: allocates nothing."""
        k, kl = _key(layer_key)
        return self._rc(self.lib.soso_hip_moe_ffn_dev_noalloc(self.h, k, kl, x_dev, n, out_dev, idx_dev, wgt_dev),
                        f"moe_ffn_dev_noalloc {layer_key}")

    # -- Gated DeltaNet (GpuDispatch::gdn_bloque) ---------------------------------
    def gdn_block(self, hist, conv, z, decay, beta, norm, state, n, n_k, n_v, d, kernel, eps):
        """gdn_bloque on host arrays: returns out [n * n_v * d]; `state` (f32,
        contiguous) is updated in place.  False when the shape is declined."""
        f = [np.ascontiguousarray(a, dtype=np.float32) for a in (hist, conv, z, decay, beta, norm)]
        if not (isinstance(state, np.ndarray) and state.dtype == np.float32 and state.flags.c_contiguous):
            raise ValueError("gdn_block: state must be a contiguous float32 array (updated in place)")
        out = np.zeros(n * n_v * d, np.float32)
        ok = self._rc(self.lib.soso_hip_gdn_block(self.h, *[a.ctypes.data for a in f], state.ctypes.data,
                                                  out.ctypes.data, n, n_k, n_v, d, kernel, C.c_float(eps)),
                      "gdn_block")
        return out if ok else False

    def gdn_block_dev(self, hist, conv, z, decay, beta, norm, state, out, n, n_k, n_v, d, kernel, eps):
        """gdn_bloque on device pointers, queued on the library's stream."""
        return self._rc(self.lib.soso_hip_gdn_block_dev(self.h, hist, conv, z, decay, beta, norm, state, out, n, n_k,
                                                        n_v, d, kernel, C.c_float(eps)), "gdn_block_dev")

    # -- dense decode step resident on the device (decode_preparar / decode_token) --
    def decode_create(self, model_key, cfg, keys, drop_sources=False, moe_layers=None, flags=0):
        """cfg: dict of soso_hip_decode_cfg fields; keys: 9 per layer (attn_norm,
        q, k, v, o, ffn_norm, gate, up, down), then output_norm and head.
        moe_layers: per layer, the key of a registered MoE layer that is its
        FFN, or None (soso_hip_decode_create_moe); an MoE layer's gate, up and
        down keys may be None.  flags: DECODE_QK_NORM (then 11 keys per layer,
        q_norm and k_norm last) and DECODE_ROPE_NEOX (soso_hip_decode_create_ex)."""
        mk, ml = _key(model_key)
        c = abi.DecodeCfg(**cfg)
        enc = [k.encode() if k is not None else None for k in keys]
        arr = (C.c_char_p * len(enc))(*enc)
        lens = (C.c_size_t * len(enc))(*[len(k) if k is not None else 0 for k in enc])
        drop = 1 if drop_sources else 0
        if flags:
            marr = mlens = None  # the arrays stay referenced until the call returns
            if moe_layers is not None:
                menc = [k.encode() if k is not None else None for k in moe_layers]
                marr = (C.c_char_p * len(menc))(*menc)
                mlens = (C.c_size_t * len(menc))(*[len(k) if k is not None else 0 for k in menc])
            ok = self._rc(self.lib.soso_hip_decode_create_ex(self.h, mk, ml, C.byref(c), flags,
                                                             C.cast(arr, C.c_void_p), C.cast(lens, C.c_void_p),
                                                             C.cast(marr, C.c_void_p) if marr is not None else None,
                                                             C.cast(mlens, C.c_void_p) if mlens is not None else None,
                                                             drop),
                          f"decode_create_ex {model_key}")
        elif moe_layers is None:
            ok = self._rc(self.lib.soso_hip_decode_create(self.h, mk, ml, C.byref(c), C.cast(arr, C.c_void_p),
                                                          C.cast(lens, C.c_void_p), drop),
                          f"decode_create {model_key}")
        else:
            menc = [k.encode() if k is not None else None for k in moe_layers]
            marr = (C.c_char_p * len(menc))(*menc)
            mlens = (C.c_size_t * len(menc))(*[len(k) if k is not None else 0 for k in menc])
            ok = self._rc(self.lib.soso_hip_decode_create_moe(self.h, mk, ml, C.byref(c), C.cast(arr, C.c_void_p),
                                                              C.cast(lens, C.c_void_p), C.cast(marr, C.c_void_p),
                                                              C.cast(mlens, C.c_void_p), drop),
                          f"decode_create_moe {model_key}")
        if ok:
            self._decode_cfg[model_key] = dict(cfg)
        return ok

    def decode_moe_routing(self, model_key, layer, top_k):
        """The routing of MoE layer `layer` in the model's last step: (indices, weights)."""
        mk, ml = _key(model_key)
        i, w = C.c_void_p(), C.c_void_p()
        self._rc(self.lib.soso_hip_decode_moe_routing_dev(self.h, mk, ml, layer, C.byref(i), C.byref(w)),
                 "decode_moe_routing")
        return self.d2h(i.value, (top_k,), np.int32), self.d2h(w.value, (top_k,), np.float32)

    # -- moe_capa: one GQA-MoE layer at a time (gpu.rs:380-426) ----------------
    def gemma_subir(self, key, w, dtype, rows, cols):
        """gpu.rs:368: makes `key` resident from its raw bytes."""
        k, kl = _key(key)
        wb = _raw(w)
        return self._rc(self.lib.soso_hip_weight_upload(self.h, k, kl, wb.ctypes.data, wb.size, dtype, rows, cols),
                        f"weight_upload {key}")

    def gemma_residente(self, key):
        k, kl = _key(key)
        return bool(self.lib.soso_hip_weight_resident(self.h, k, kl))

    def moe_capa(self, capa, hidden):
        """gpu.rs:426.  capa: a dict of MoeCapa's fields (soso_hip_moe_capa;
        norms/router numpy f32 or None; keys str); hidden: float32 n x h,
        read unless continuar, written unless encadenar."""
        c = abi.MoeCapa()
        keep = []
        for name, _ in abi.MoeCapa._fields_:
            if name not in capa or capa[name] is None:
                continue
            v = capa[name]
            if name.startswith("key_") or name == "prefix":
                v = v.encode()
            elif name in ("attn_norm", "q_norm", "k_norm", "ffn_norm", "router", "rope_factors"):
                v = _f32(v)
                keep.append(v)
                v = v.ctypes.data
            elif isinstance(v, np.generic):
                v = v.item()
            setattr(c, name, v)
        assert hidden is None or (hidden.dtype == np.float32 and hidden.flags.c_contiguous)
        rc = self.lib.soso_hip_moe_capa_run(self.h, C.byref(c), None if hidden is None else hidden.ctypes.data)
        return self._rc(rc, f"moe_capa layer {capa.get('layer')}")

    def moe_puede(self, layer):
        return bool(self.lib.soso_hip_moe_capa_can(self.h, layer))

    def moe_lista(self, layer):
        return bool(self.lib.soso_hip_moe_capa_ready(self.h, layer))

    def moe_pendiente(self, layer, pos0, n):
        return bool(self.lib.soso_hip_moe_capa_pending(self.h, layer, pos0, n))

    def moe_volcar(self, hidden):
        assert hidden.dtype == np.float32 and hidden.flags.c_contiguous
        self._rc(self.lib.soso_hip_moe_capa_flush(self.h, hidden.ctypes.data), "moe_volcar")

    def moe_descartar(self, layer):
        self.lib.soso_hip_moe_capa_discard(self.h, layer)

    def moe_capa_kv_dev(self, layer):
        k, v = C.c_void_p(), C.c_void_p()
        self._rc(self.lib.soso_hip_moe_capa_kv_dev(self.h, layer, C.byref(k), C.byref(v)), "moe_capa_kv_dev")
        return k.value, v.value

    def moe_capa_routing(self, layer, top_k):
        """The routing of the layer's last token: (indices, weights)."""
        i, w = C.c_void_p(), C.c_void_p()
        self._rc(self.lib.soso_hip_moe_capa_routing_dev(self.h, layer, C.byref(i), C.byref(w)), "moe_capa_routing")
        return self.d2h(i.value, (top_k,), np.int32), self.d2h(w.value, (top_k,), np.float32)

    def decode_kv_dev(self, model_key, layer):
        mk, ml = _key(model_key)
        k, v = C.c_void_p(), C.c_void_p()
        self._rc(self.lib.soso_hip_decode_kv_dev(self.h, mk, ml, layer, C.byref(k), C.byref(v)), "decode_kv_dev")
        return k.value, v.value

    def decode_kv_upload(self, model_key, layer, row0, k_rows, v_rows, rows_f32=True):
        """decode_subir_estado: position-major rows [n][kv_dim] of K and V (numpy
        arrays, f32 or uint16 f16 bits; or device pointers with n given as
        k_rows = (ptr, n)) into the cache at positions row0 .."""
        mk, ml = _key(model_key)
        if isinstance(k_rows, tuple):
            (kp, n), (vp, _) = k_rows, v_rows
        else:
            want = np.float32 if rows_f32 else np.uint16
            k_rows = np.ascontiguousarray(k_rows, dtype=want)
            v_rows = np.ascontiguousarray(v_rows, dtype=want)
            if k_rows.shape != v_rows.shape:
                raise ValueError("decode_kv_upload: K and V rows differ in shape")
            kp, vp, n = k_rows.ctypes.data, v_rows.ctypes.data, k_rows.shape[0]
        return self._rc(self.lib.soso_hip_decode_kv_upload(self.h, mk, ml, layer, row0, n, kp, vp,
                                                           1 if rows_f32 else 0), "decode_kv_upload")

    def decode_step_dev(self, model_key, x_dev, pos, logits_dev=None, token_dev=None, kv_rows_dev=None):
        mk, ml = _key(model_key)
        return self._rc(self.lib.soso_hip_decode_step_dev(self.h, mk, ml, x_dev, pos, logits_dev, token_dev,
                                                          kv_rows_dev), f"decode_step_dev {model_key}")

    def decode_token(self, model_key, embed, pos, cpu_moe=None, logits=True, kv_rows=False):
        """GpuDispatch::decode_token on host buffers (soso_hip_decode_token):
        embed (hidden f32) -> (logits or None, greedy token, kv rows or None).
        cpu_moe(layer, xn, idx, wgt) -> out (numpy f32, hidden) computes the
        FFN of layers whose experts stay on the host."""
        mk, ml = _key(model_key)
        embed = np.ascontiguousarray(embed, np.float32)
        cfg = self._decode_cfg[model_key]
        lg = np.zeros(cfg["vocab"], np.float32) if logits else None
        kv = None
        if kv_rows:
            n = cfg["n_layers"] * 2 * cfg["n_kv_heads"] * cfg["head_dim"]
            kv = np.zeros(n, np.uint16 if cfg.get("kv_f16") else np.float32)
        tok = np.zeros(1, np.uint32)
        err = []

        def trampoline(_ctx, layer, xn, idx, wgt, top_k, out):
            try:
                h = embed.size
                res = cpu_moe(int(layer), np.ctypeslib.as_array(xn, (h,)).copy(),
                              np.ctypeslib.as_array(idx, (top_k,)).copy(), np.ctypeslib.as_array(wgt, (top_k,)).copy())
                np.ctypeslib.as_array(out, (h,))[:] = np.asarray(res, np.float32)
                return 0
            except Exception as e:  # noqa: BLE001 -- reported to the caller after the call
                err.append(e)
                return 1
        cb = abi.CpuMoeFn(trampoline) if cpu_moe else abi.CpuMoeFn()
        rc = self.lib.soso_hip_decode_token(self.h, mk, ml, embed.ctypes.data, pos, cb, None,
                                            lg.ctypes.data if lg is not None else None,
                                            kv.ctypes.data if kv is not None else None, tok.ctypes.data)
        if err:
            raise err[0]
        if not self._rc(rc, f"decode_token {model_key}"):
            return None
        return lg, int(tok[0]), kv

    def decode_destroy(self, model_key):
        mk, ml = _key(model_key)
        return self._rc(self.lib.soso_hip_decode_destroy(self.h, mk, ml), "decode_destroy")
