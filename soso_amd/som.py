"""soso's on-disk model format (.som) on the GPU path.

Reading is native: libsoso_som.so (include/soso_som.h) parses manifest.som and
index.som, checks every CRC32C and maps the shards read-only, like sosomodel
(crates/sosomodel/src/{lib,index,manifest}.rs) and MmapTensorSource
(crates/soso-llm-core/src/source.rs).  This module binds it, restates the
Manifest accessors (manifest.rs:371-516), and holds:

* the writer side (pack_som lib.rs:63-76, pack_shard index.rs:103-112,
  TensorIndex::serialize index.rs:38-59, Manifest::serialize
  manifest.rs:916-1019, make_*_entry index.rs:131-259), which soso's
  converter uses, for building model directories from arrays;
* the mapping of a converted model onto the device: `prepare_decode` checks a
  dense GQA decoder the way Runtime does (runtime.rs:330-475), makes every
  tensor it needs resident under its soso name (the key GpuDispatch caches
  by) and builds the device decode step; `prepare_moe_layer` registers one
  MoE layer's router and experts for moe_ffn_dev.

Format extension owned by this build: dtype 13 = Q6_K (210 B per 256
elements), so a Q6_K output head can be stored as such instead of being
converted to Q8_0 at import (gguf2som/src/lib.rs:1592-1609).
"""
import ctypes as C
import os
import struct
from dataclasses import dataclass, field, fields, replace

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsoso_som.so")

MAGIC = b"SOMODL01"
HEADER = 24
CACHE_ALIGN = 64
BLOCK_ALIGN = 4096
SHARD_PAYLOAD_OFF = 64
MANIFEST_FILE, INDEX_FILE, SHARDS_DIR = "manifest.som", "index.som", "shards"

DTYPE_F32, DTYPE_Q8_0, DTYPE_Q4_K, DTYPE_MXFP4, DTYPE_Q4_0 = 1, 2, 3, 4, 5
DTYPE_Q6_K = 13
QUANT_NONE, QUANT_Q8_0, QUANT_Q4_K, QUANT_MXFP4, QUANT_Q4_0 = 0, 1, 2, 3, 4
# (elements, bytes) per block: layout.rs:57-83, Q6_K = GGML's block_q6_K
BLOCKS = {DTYPE_F32: (1, 4), DTYPE_Q8_0: (32, 36), DTYPE_Q4_K: (256, 144), DTYPE_MXFP4: (32, 20),
          DTYPE_Q4_0: (32, 18), DTYPE_Q6_K: (256, 210)}
QUANT_OF = {DTYPE_F32: QUANT_NONE, DTYPE_Q8_0: QUANT_Q8_0, DTYPE_Q4_K: QUANT_Q4_K, DTYPE_MXFP4: QUANT_MXFP4,
            DTYPE_Q4_0: QUANT_Q4_0, DTYPE_Q6_K: DTYPE_Q6_K}

ATTN_GQA, ATTN_MLA, ATTN_KDA, ATTN_GATED, ATTN_GDN, ATTN_BIDIRECTIONAL, ATTN_CROSS = range(7)
FFN_DENSE, FFN_MOE, FFN_LATENT_MOE, FFN_GELU_MLP = range(4)
MODEL_DECODER, MODEL_ASR, MODEL_DECISION = range(3)
NORM_RMS, NORM_LAYER = range(2)
FLAG_ROPE_NEOX, FLAG_QK_NORM, FLAG_SANDWICH_NORM = 1 << 3, 1 << 4, 1 << 5
FLAG_V_FROM_K, FLAG_V_NORM, FLAG_GEGLU, FLAG_LAYER_SCALE, FLAG_ROPE_FACTORS = 1 << 6, 1 << 7, 1 << 8, 1 << 9, 1 << 10

OK, ERR_IO, ERR_FORMAT, ERR_NOTFOUND, ERR_ARG, ERR_DTYPE = 0, -1, -2, -3, -4, -5


class SomError(Exception):
    def __init__(self, msg, rc=ERR_FORMAT):
        super().__init__(msg)
        self.rc = rc


# ---------------------------------------------------------------------------
# native library
# ---------------------------------------------------------------------------
class _Layer(C.Structure):
    _fields_ = [("attn_kind", C.c_uint8), ("ffn_kind", C.c_uint8), ("pad", C.c_uint16)] + [
        (n, C.c_uint32) for n in ("num_heads", "num_kv_heads", "ffn_dim", "kv_lora_rank", "q_lora_rank",
                                  "qk_rope_head_dim", "qk_nope_head_dim", "v_head_dim", "num_experts",
                                  "num_experts_per_tok", "moe_ffn_dim", "num_shared_experts", "flags")]


_U, _F = C.c_uint32, C.c_float


class _Manifest(C.Structure):
    _fields_ = [("version", _U), ("vocab_size", _U), ("hidden_dim", _U), ("num_layers", _U), ("num_heads", _U),
                ("num_kv_heads", _U), ("ffn_dim", _U), ("max_seq", _U), ("rope_theta", _F), ("rms_eps", _F),
                ("num_experts", _U), ("num_experts_per_tok", _U), ("moe_ffn_dim", _U), ("model_kind", C.c_uint8),
                ("norm_kind", C.c_uint8), ("pad", C.c_uint16)] + [
        (n, _U) for n in ("n_mels", "n_audio_ctx", "n_audio_state", "n_audio_layer", "n_audio_head", "n_text_ctx",
                          "n_text_state", "n_text_layer", "n_text_head")] + [
        ("embed_scale", _F), ("logit_softcap", _F), ("attn_scale", _F), ("tied_lm_head", _U), ("yarn_factor", _F),
        ("yarn_orig_ctx", _U), ("yarn_beta_fast", _F), ("yarn_beta_slow", _F), ("has_kev", _U),
        ("kev_temperature", _F), ("kev_pointer_dim", _U), ("n_layer_specs", _U), ("n_window", _U),
        ("n_rope_theta", _U), ("n_prefetch", _U)]


class _Tensor(C.Structure):
    _fields_ = [("id", _U), ("name", C.c_void_p), ("name_len", C.c_size_t), ("shard", C.c_void_p),
                ("shard_len", C.c_size_t), ("offset", C.c_uint64), ("byte_len", C.c_uint64), ("ndim", _U),
                ("shape", C.POINTER(_U)), ("dtype", C.c_uint8), ("quant", C.c_uint8)]


class _View(C.Structure):
    _fields_ = [("bytes", C.c_void_p), ("len", C.c_size_t), ("dtype", C.c_uint8), ("elems", C.c_uint64)]


_lib = None


def lib(path=LIB_PATH):
    """Loads libsoso_som.so (built in-tree by soso_amd.build)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise SomError(f"{path} is not built (run soso_amd.build)", ERR_IO)
    L = C.CDLL(path)
    P, S, I = C.c_void_p, C.c_size_t, C.c_int
    sig = {
        "soso_som_crc32c": (_U, [P, S]),
        "soso_som_crc32c_portable": (_U, [P, S]),
        "soso_som_error": (C.c_char_p, []),
        "soso_som_open": (I, [C.c_char_p, S, C.POINTER(P)]),
        "soso_som_open_bytes": (I, [P, S, P, S, C.c_char_p, S, C.POINTER(P)]),
        "soso_som_close": (None, [P]),
        "soso_som_verify_shard": (I, [P, S, C.POINTER(S), C.POINTER(S)]),
        "soso_som_manifest_get": (I, [P, C.POINTER(_Manifest)]),
        "soso_som_manifest_str": (I, [P, I, C.POINTER(P), C.POINTER(S)]),
        "soso_som_layer_spec": (I, [P, _U, C.POINTER(_Layer)]),
        "soso_som_ext_window": (I, [P, _U, C.POINTER(_U)]),
        "soso_som_ext_rope_theta": (I, [P, _U, C.POINTER(_F)]),
        "soso_som_prefetch": (I, [P, _U, C.POINTER(_U), C.POINTER(_U)]),
        "soso_som_prefetch_shard": (I, [P, _U, _U, C.POINTER(P), C.POINTER(S)]),
        "soso_som_tensor_count": (S, [P]),
        "soso_som_tensor_at": (I, [P, S, C.POINTER(_Tensor)]),
        "soso_som_find": (I, [P, C.c_char_p, S, C.POINTER(S)]),
        "soso_som_tensor_view": (I, [P, C.c_char_p, S, C.POINTER(_View)]),
        "soso_som_load_f32": (I, [P, C.c_char_p, S, P, S]),
        "soso_som_load_f32_range": (I, [P, C.c_char_p, S, S, P, S]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    _lib = L
    return L


def _err():
    return lib().soso_som_error().decode(errors="replace")


def _check(rc, what):
    if rc != OK:
        raise SomError(f"{what}: {_err()}", rc)


def crc32c(data):
    """CRC-32C of bytes or a numpy array's bytes (lib.rs:26-30)."""
    arr = np.ascontiguousarray(data).reshape(-1).view(np.uint8) if isinstance(data, np.ndarray) \
        else np.frombuffer(bytes(data), np.uint8)
    return int(lib().soso_som_crc32c(arr.ctypes.data if arr.size else None, arr.size))


def _str(ptr, n):
    return C.string_at(ptr, n).decode() if n else ""


# ---------------------------------------------------------------------------
# Manifest (manifest.rs:104-370) and its accessors
# ---------------------------------------------------------------------------
@dataclass
class LayerSpec:
    attn_kind: int = ATTN_GQA
    ffn_kind: int = FFN_DENSE
    num_heads: int = 0
    num_kv_heads: int = 0
    ffn_dim: int = 0
    kv_lora_rank: int = 0
    q_lora_rank: int = 0
    qk_rope_head_dim: int = 0
    qk_nope_head_dim: int = 0
    v_head_dim: int = 0
    num_experts: int = 0
    num_experts_per_tok: int = 0
    moe_ffn_dim: int = 0
    num_shared_experts: int = 0
    flags: int = 0


AUDIO_FIELDS = ("n_mels", "n_audio_ctx", "n_audio_state", "n_audio_layer", "n_audio_head", "n_text_ctx",
                "n_text_state", "n_text_layer", "n_text_head")
AUDIO_DEFAULT = (80, 1500, 384, 4, 6, 448, 384, 4, 6)  # AudioSpec::default, manifest.rs:178-192


@dataclass
class YarnSpec:
    factor: float = 0.0
    orig_ctx: int = 0
    beta_fast: float = 0.0
    beta_slow: float = 0.0

    def activa(self):
        return self.factor > 1.0 and self.orig_ctx > 0


@dataclass
class ManifestExt:
    embed_scale: float = 0.0
    logit_softcap: float = 0.0
    attn_scale: float = 0.0
    tied_lm_head: bool = False
    window: list = field(default_factory=list)
    rope_theta: list = field(default_factory=list)
    yarn: YarnSpec = field(default_factory=YarnSpec)

    def es_vacia(self):
        return self == ManifestExt()


@dataclass
class KevSpec:
    temperature: float = 0.0
    pointer_dim: int = 0


@dataclass
class Manifest:
    name: str = ""
    vocab_size: int = 0
    hidden_dim: int = 0
    num_layers: int = 0
    num_heads: int = 0
    num_kv_heads: int = 0
    ffn_dim: int = 0
    max_seq: int = 0
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    num_experts: int = 0
    num_experts_per_tok: int = 0
    moe_ffn_dim: int = 0
    layers: list = field(default_factory=list)
    prefetch: list = field(default_factory=list)  # [(layer, [shard names])]
    chat_template: str = ""
    model_kind: int = MODEL_DECODER
    audio: tuple = AUDIO_DEFAULT
    norm_kind: int = NORM_RMS
    ext: ManifestExt = field(default_factory=ManifestExt)
    kev: KevSpec = None
    version: int = 0  # of the record this was parsed from (0 = built in memory)

    # -- constructors of the reference's test models (manifest.rs:654-748) --
    @classmethod
    def tiny(cls, name):
        pf = [(l, [f"L{l:02}.{t}.tensor" for t in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                                    "ffn_norm", "ffn_up", "ffn_down")]) for l in range(4)]
        m = cls(name=name, vocab_size=256, hidden_dim=128, num_layers=4, num_heads=4, num_kv_heads=4, ffn_dim=256,
                max_seq=128, rope_theta=10000.0, rms_eps=1e-5, prefetch=pf)
        m.fill_layers_from_globals()
        return m

    @classmethod
    def tiny_moe(cls, name):
        pf = [(l, [f"L{l:02}.{t}.tensor" for t in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                                    "ffn_norm", "ffn_gate_inp")]) for l in range(2)]
        m = cls(name=name, vocab_size=64, hidden_dim=64, num_layers=2, num_heads=4, num_kv_heads=4, ffn_dim=128,
                max_seq=64, rope_theta=10000.0, rms_eps=1e-5, num_experts=4, num_experts_per_tok=2, moe_ffn_dim=32,
                prefetch=pf)
        m.fill_layers_from_globals()
        return m

    def fill_layers_from_globals(self):
        kind = FFN_MOE if self.num_experts > 0 else FFN_DENSE
        self.layers = [LayerSpec(attn_kind=ATTN_GQA, ffn_kind=kind) for _ in range(self.num_layers)]

    # -- accessors (manifest.rs:371-516) --
    @staticmethod
    def _spec_is_moe(s):
        return s.ffn_kind in (FFN_MOE, FFN_LATENT_MOE) or s.num_experts > 0

    def is_moe(self):
        return self.num_experts > 0 or any(self._spec_is_moe(s) for s in self.layers)

    def expert_ffn_dim(self):
        return self.moe_ffn_dim if self.num_experts > 0 and self.moe_ffn_dim > 0 else self.ffn_dim

    def layer_window(self, layer):
        return self.ext.window[layer] if layer < len(self.ext.window) else 0

    def layer_rope_theta(self, layer):
        t = self.ext.rope_theta[layer] if layer < len(self.ext.rope_theta) else 0.0
        return t if t > 0.0 else self.rope_theta

    def embed_scale(self):
        return self.ext.embed_scale if self.ext.embed_scale > 0.0 else 1.0

    def layer(self, i):
        return self.layers[i] if 0 <= i < len(self.layers) else None

    def attn_kind(self, layer):
        s = self.layer(layer)
        return s.attn_kind if s else ATTN_GQA

    def ffn_kind(self, layer):
        s = self.layer(layer)
        return s.ffn_kind if s else FFN_DENSE

    def layer_is_moe(self, layer):
        s = self.layer(layer)
        return self._spec_is_moe(s) if s else self.num_experts > 0

    def _eff(self, layer, attr, glob):
        s = self.layer(layer)
        v = getattr(s, attr) if s else 0
        return v if v > 0 else glob

    def effective_num_heads(self, layer):
        return self._eff(layer, "num_heads", self.num_heads)

    def effective_num_kv_heads(self, layer):
        return self._eff(layer, "num_kv_heads", self.num_kv_heads)

    def effective_ffn_dim(self, layer):
        return self._eff(layer, "ffn_dim", self.ffn_dim)

    def effective_head_dim(self, layer):
        s = self.layer(layer)
        if s and s.v_head_dim > 0:
            return s.v_head_dim
        h = self.effective_num_heads(layer)
        return self.hidden_dim // h if h else 0

    def effective_num_experts(self, layer):
        return self._eff(layer, "num_experts", self.num_experts)

    def effective_num_experts_per_tok(self, layer):
        return self._eff(layer, "num_experts_per_tok", self.num_experts_per_tok)

    def effective_moe_ffn_dim(self, layer):
        return self._eff(layer, "moe_ffn_dim", self.expert_ffn_dim())

    def layer_expert_ffn_dim(self, layer):
        return self.effective_moe_ffn_dim(layer) if self.layer_is_moe(layer) else self.effective_ffn_dim(layer)

    def max_router_experts(self):
        return max([self.num_experts] + [self.effective_num_experts(i)
                                         for i in range(min(len(self.layers), self.num_layers))])

    def max_ffn_dim(self):
        return max((self.layer_expert_ffn_dim(i) for i in range(self.num_layers)), default=self.ffn_dim)


# ---------------------------------------------------------------------------
# TensorIndex entries, views
# ---------------------------------------------------------------------------
@dataclass
class TensorEntry:
    id: int
    name: str
    shard: str
    offset: int
    byte_len: int
    shape: tuple
    dtype: int
    quant: int

    def elems(self):
        n = 1
        for d in self.shape:
            n *= d
        return n


@dataclass
class TensorView:
    """TensorView: the tensor's bytes inside the mapped shard (read-only, valid
    while the SomModel is open), its dtype and logical element count."""
    bytes: np.ndarray
    dtype: int
    elems: int


def make_entry(dtype, id, name, shard, offset, shape):
    """make_{f32,q8_0,q4_k,q4_0,mxfp4}_entry (index.rs:131-244), plus Q6_K:
    byte_len = ceil(elems / block) * block bytes."""
    if dtype not in BLOCKS:
        raise SomError(f"make_entry: dtype {dtype} has no block size here", ERR_DTYPE)
    be, bb = BLOCKS[dtype]
    n = 1
    for d in shape:
        n *= d
    return TensorEntry(id, name, shard, offset, -(-n // be) * bb, tuple(shape), dtype, QUANT_OF[dtype])


class SomModel:
    """A converted soso model: MmapTensorSource over index.som with the
    manifest (source.rs:60-352)."""

    def __init__(self, handle, keep=()):
        self._h = C.c_void_p(handle)
        self._keep = keep
        self.manifest = self._read_manifest()
        self.entries = self._read_entries()

    @classmethod
    def open(cls, path):
        L = lib()
        h = C.c_void_p()
        p = os.fsencode(path)
        _check(L.soso_som_open(p, len(p), C.byref(h)), f"open {path}")
        return cls(h.value)

    @classmethod
    def from_bytes(cls, manifest=None, index=None, shards_dir=""):
        L = lib()
        m = np.frombuffer(bytes(manifest), np.uint8) if manifest else None
        i = np.frombuffer(bytes(index), np.uint8) if index else None
        sd = os.fsencode(shards_dir)
        h = C.c_void_p()
        _check(L.soso_som_open_bytes(None if m is None or m.size == 0 else m.ctypes.data, 0 if m is None else m.size,
                                     None if i is None or i.size == 0 else i.ctypes.data, 0 if i is None else i.size,
                                     sd, len(sd), C.byref(h)), "open_bytes")
        return cls(h.value)

    def close(self):
        if self._h:
            lib().soso_som_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _read_manifest(self):
        L = lib()
        g = _Manifest()
        if L.soso_som_manifest_get(self._h, C.byref(g)) != OK:
            return None
        strs = []
        for which in (0, 1):
            p, n = C.c_void_p(), C.c_size_t()
            _check(L.soso_som_manifest_str(self._h, which, C.byref(p), C.byref(n)), "manifest_str")
            strs.append(_str(p.value, n.value))
        layers = []
        for l in range(g.n_layer_specs):
            s = _Layer()
            _check(L.soso_som_layer_spec(self._h, l, C.byref(s)), "layer_spec")
            layers.append(LayerSpec(**{f.name: getattr(s, f.name) for f in fields(LayerSpec)}))
        win, th = [], []
        for i in range(g.n_window):
            v = _U()
            _check(L.soso_som_ext_window(self._h, i, C.byref(v)), "ext_window")
            win.append(v.value)
        for i in range(g.n_rope_theta):
            v = _F()
            _check(L.soso_som_ext_rope_theta(self._h, i, C.byref(v)), "ext_rope_theta")
            th.append(v.value)
        pf = []
        for i in range(g.n_prefetch):
            lay, ns = _U(), _U()
            _check(L.soso_som_prefetch(self._h, i, C.byref(lay), C.byref(ns)), "prefetch")
            names = []
            for j in range(ns.value):
                p, n = C.c_void_p(), C.c_size_t()
                _check(L.soso_som_prefetch_shard(self._h, i, j, C.byref(p), C.byref(n)), "prefetch_shard")
                names.append(_str(p.value, n.value))
            pf.append((lay.value, names))
        ext = ManifestExt(g.embed_scale, g.logit_softcap, g.attn_scale, bool(g.tied_lm_head), win, th,
                          YarnSpec(g.yarn_factor, g.yarn_orig_ctx, g.yarn_beta_fast, g.yarn_beta_slow))
        return Manifest(name=strs[0], vocab_size=g.vocab_size, hidden_dim=g.hidden_dim, num_layers=g.num_layers,
                        num_heads=g.num_heads, num_kv_heads=g.num_kv_heads, ffn_dim=g.ffn_dim, max_seq=g.max_seq,
                        rope_theta=g.rope_theta, rms_eps=g.rms_eps, num_experts=g.num_experts,
                        num_experts_per_tok=g.num_experts_per_tok, moe_ffn_dim=g.moe_ffn_dim, layers=layers,
                        prefetch=pf, chat_template=strs[1], model_kind=g.model_kind,
                        audio=tuple(getattr(g, a) for a in AUDIO_FIELDS), norm_kind=g.norm_kind, ext=ext,
                        kev=KevSpec(g.kev_temperature, g.kev_pointer_dim) if g.has_kev else None,
                        version=g.version)

    def _read_entries(self):
        L = lib()
        out = []
        for i in range(L.soso_som_tensor_count(self._h)):
            t = _Tensor()
            _check(L.soso_som_tensor_at(self._h, i, C.byref(t)), "tensor_at")
            out.append(TensorEntry(t.id, _str(t.name, t.name_len), _str(t.shard, t.shard_len), t.offset, t.byte_len,
                                   tuple(t.shape[k] for k in range(t.ndim)), t.dtype, t.quant))
        return out

    def find(self, name):
        """TensorIndex::find (index.rs:93-95): the first entry of that name, or None."""
        b = name.encode()
        i = C.c_size_t()
        if lib().soso_som_find(self._h, b, len(b), C.byref(i)) != OK:
            return None
        return self.entries[i.value]

    def tensor_view(self, name):
        b = name.encode()
        v = _View()
        _check(lib().soso_som_tensor_view(self._h, b, len(b), C.byref(v)), f"tensor_view {name}")
        buf = (C.c_uint8 * v.len).from_address(v.bytes) if v.len else (C.c_uint8 * 0)()
        arr = np.frombuffer(buf, np.uint8)
        arr.flags.writeable = False
        return TensorView(arr, v.dtype, v.elems)

    def load_f32(self, name, n=None):
        e = self.find(name)
        n = e.elems() if (n is None and e is not None) else (n or 0)
        out = np.empty(n, np.float32)
        b = name.encode()
        _check(lib().soso_som_load_f32(self._h, b, len(b), out.ctypes.data if n else None, n), f"load_f32 {name}")
        return out

    def load_f32_range(self, name, elem_off, n):
        out = np.empty(n, np.float32)
        b = name.encode()
        _check(lib().soso_som_load_f32_range(self._h, b, len(b), elem_off, out.ctypes.data if n else None, n),
               f"load_f32_range {name}")
        return out


def verify_shard(data):
    """verify_shard (index.rs:114-130) -> the payload bytes."""
    a = np.frombuffer(bytes(data), np.uint8)
    off, n = C.c_size_t(), C.c_size_t()
    _check(lib().soso_som_verify_shard(a.ctypes.data if a.size else None, a.size, C.byref(off), C.byref(n)),
           "verify_shard")
    return a[off.value:off.value + n.value].tobytes()


# ---------------------------------------------------------------------------
# writer (the converter's side)
# ---------------------------------------------------------------------------
def _align(n, a):
    return (n + a - 1) & ~(a - 1)


def pack_som(body, version, align=CACHE_ALIGN):
    body = bytes(body)
    out = MAGIC + struct.pack("<IIQ", crc32c(body), version, len(body)) + body
    return out + b"\0" * (_align(len(out), align) - len(out))


def pack_shard(data):
    data = bytes(data)
    out = MAGIC + struct.pack("<IIQ", crc32c(data), 2, len(data))
    out += b"\0" * (SHARD_PAYLOAD_OFF - len(out)) + data
    return out + b"\0" * (_align(len(out), BLOCK_ALIGN) - len(out))


def _cstr(s):
    return s.encode() + b"\0"


def serialize_index(entries):
    body = [struct.pack("<I", len(entries))]
    for e in entries:
        body += [struct.pack("<I", e.id), _cstr(e.name), _cstr(e.shard), struct.pack("<QQI", e.offset, e.byte_len,
                                                                                      len(e.shape))]
        body += [struct.pack(f"<{len(e.shape)}I", *e.shape), bytes([e.dtype, e.quant, 0, 0])]
    return pack_som(b"".join(body), 1)


def serialize_manifest(m):
    b = [_cstr(m.name), struct.pack("<6I", m.vocab_size, m.hidden_dim, m.num_layers, m.num_heads, m.ffn_dim,
                                    m.max_seq),
         struct.pack("<Iff3I", m.num_kv_heads, m.rope_theta, m.rms_eps, m.num_experts, m.num_experts_per_tok,
                     m.moe_ffn_dim), struct.pack("<I", len(m.layers))]
    for s in m.layers:
        b.append(struct.pack("<BBH13I", s.attn_kind, s.ffn_kind, 0, s.num_heads, s.num_kv_heads, s.ffn_dim,
                             s.kv_lora_rank, s.q_lora_rank, s.qk_rope_head_dim, s.qk_nope_head_dim, s.v_head_dim,
                             s.num_experts, s.num_experts_per_tok, s.moe_ffn_dim, s.num_shared_experts, s.flags))
    b.append(struct.pack("<I", len(m.prefetch)))
    for layer, shards in m.prefetch:
        b.append(struct.pack("<II", layer, len(shards)) + b"".join(_cstr(s) for s in shards))
    b.append(_cstr(m.chat_template))
    b.append(struct.pack("<BBH9I", m.model_kind, m.norm_kind, 0, *m.audio))
    e = m.ext
    if e.yarn.activa() or not e.es_vacia():
        b.append(struct.pack("<fffII", e.embed_scale, e.logit_softcap, e.attn_scale, int(e.tied_lm_head),
                             len(e.window)) + struct.pack(f"<{len(e.window)}I", *e.window))
        b.append(struct.pack("<I", len(e.rope_theta)) + struct.pack(f"<{len(e.rope_theta)}f", *e.rope_theta))
        if e.yarn.activa():
            b.append(struct.pack("<fIff", e.yarn.factor, e.yarn.orig_ctx, e.yarn.beta_fast, e.yarn.beta_slow))
            version = 8
        else:
            version = 7
    elif m.model_kind == MODEL_ASR:
        version = 6
    else:
        version = 5
    if m.kev is not None:
        if version < 7:
            b.append(struct.pack("<fffIII", 0.0, 0.0, 0.0, 0, 0, 0))
            version = 7
        if version < 8:
            b.append(struct.pack("<fIff", 0.0, 0, 0.0, 0.0))
            version = 8
        b.append(struct.pack("<fI", m.kev.temperature, m.kev.pointer_dim))
        version = max(version, 9)
    return pack_som(b"".join(b), version)


def write_model(path, manifest, tensors):
    """Writes a model directory.  tensors: (name, dtype, shape, raw bytes) in
    soso's layout, shape [rows, cols] row-major; each goes to its own shard
    "<name>.tensor" at offset 0."""
    os.makedirs(os.path.join(path, SHARDS_DIR), exist_ok=True)
    entries = []
    for i, (name, dtype, shape, raw) in enumerate(tensors):
        raw = np.ascontiguousarray(raw).reshape(-1).view(np.uint8).tobytes()
        e = make_entry(dtype, i, name, f"{name}.tensor", 0, shape)
        if e.byte_len != len(raw):
            raise SomError(f"write_model: {name}: {len(raw)} bytes for a {e.byte_len}-byte entry", ERR_ARG)
        with open(os.path.join(path, SHARDS_DIR, e.shard), "wb") as f:
            f.write(pack_shard(raw))
        entries.append(e)
    with open(os.path.join(path, INDEX_FILE), "wb") as f:
        f.write(serialize_index(entries))
    with open(os.path.join(path, MANIFEST_FILE), "wb") as f:
        f.write(serialize_manifest(manifest))
    return entries


# ---------------------------------------------------------------------------
# onto the device
# ---------------------------------------------------------------------------
def _upload(gpu, key, view, rows, cols):
    """Makes a tensor resident under its soso name (the GpuDispatch residency
    key), from the mapped bytes, without computing anything."""
    d = gpu.dev_alloc(view.bytes.size)
    try:
        gpu.h2d(d, view.bytes)
        gpu.weight_from_dev(key, d, view.bytes.size, view.dtype, rows, cols)
    finally:
        gpu.dev_free(d)


DEVICE_LAYER_FLAGS = FLAG_ROPE_NEOX | FLAG_QK_NORM  # what soso_hip_decode_create_ex takes


def decode_plan(som):
    """The tensors a GQA decoder needs, in the device decode step's key order,
    after the checks Runtime makes (runtime.rs:330-475): per layer attn_norm,
    q, k, v, o, ffn_norm, gate, up, down (None for an MoE layer's FFN, which
    runs from its registered router and experts), then attn_q_norm /
    attn_k_norm with FLAG_QK_NORM (layer.rs:1164-1180); then output_norm and
    the head.  Returns (cfg, want, extra): extra = {"flags": the
    SOSO_HIP_DECODE_* flags, "moe_layers": the MoE layer indices}.  Raises
    SomError(ERR_ARG) for a model the device step does not run."""
    m = som.manifest
    if m is None:
        raise SomError("decode_plan: no manifest", ERR_NOTFOUND)
    why = None
    if m.model_kind != MODEL_DECODER or m.norm_kind != NORM_RMS:
        why = "only RMS-norm decoders"
    elif m.kev is not None or not replace(m.ext, tied_lm_head=False).es_vacia():
        why = "manifest extensions (softcap, scales, windows, per-layer RoPE, YaRN, Kev) are not on the device step"
    elif m.ext.tied_lm_head and som.find("lm_head") is not None:
        why = "lm_head present although the manifest ties it to embed (runtime.rs:349-353)"
    H, L = m.hidden_dim, m.num_layers
    nh, nkv, hd = m.effective_num_heads(0), m.effective_num_kv_heads(0), m.effective_head_dim(0)
    dense = [l for l in range(L) if not m.layer_is_moe(l)]
    F = m.effective_ffn_dim(dense[0]) if dense else 0
    flags0 = (m.layer(0) or LayerSpec()).flags
    moe_layers = []
    for l in range(L):
        s = m.layer(l) or LayerSpec()
        if why:
            break
        if s.attn_kind != ATTN_GQA:
            why = f"layer {l}: only GQA attention"
        elif m.layer_is_moe(l) and (s.ffn_kind != FFN_MOE or s.num_shared_experts):
            why = f"layer {l}: only plain MoE FFNs (no latent or shared experts)"
        elif not m.layer_is_moe(l) and s.ffn_kind != FFN_DENSE:
            why = f"layer {l}: FFN kind {s.ffn_kind} is not on the device step"
        elif s.flags & ~DEVICE_LAYER_FLAGS:
            why = f"layer {l}: flags {s.flags:#x} (Gemma norms, ...) are not on the device step"
        elif s.flags != flags0:
            why = f"layer {l}: layers differ in flags"
        elif (m.effective_num_heads(l), m.effective_num_kv_heads(l), m.effective_head_dim(l)) != (nh, nkv, hd) or \
                (not m.layer_is_moe(l) and m.effective_ffn_dim(l) != F):
            why = f"layer {l}: layers differ in shape"
        elif any(som.find(f"L{l:02}.attn_{p}.bias") is not None for p in ("q", "k", "v")):
            # Qwen2 conversions carry q/k/v biases (gguf2som/src/lib.rs:673-680);
            # the CPU adds them (layer.rs:1146-1163, add_optional_bias), the
            # device step has no bias term, and soso's own device MoE layer
            # declines such layers too (moe_gpu.rs:85-90)
            why = f"layer {l}: attention q/k/v biases are not on the device step"
        if m.layer_is_moe(l):
            moe_layers.append(l)
    if why:
        raise SomError(f"decode_plan: {why}", ERR_ARG)
    flags = (1 if flags0 & FLAG_QK_NORM else 0) | (2 if flags0 & FLAG_ROPE_NEOX else 0)  # SOSO_HIP_DECODE_*
    qd, kvd, V = nh * hd, nkv * hd, m.vocab_size
    # with tied embeddings (or no lm_head) the logits come from embed (runtime.rs:1165)
    head = "lm_head" if som.find("lm_head") is not None else "embed"
    want = []
    for l in range(L):
        p = f"L{l:02}"
        want += [(f"{p}.attn_norm", (H,)), (f"{p}.attn_q", (qd, H)), (f"{p}.attn_k", (kvd, H)),
                 (f"{p}.attn_v", (kvd, H)), (f"{p}.attn_output", (H, qd)), (f"{p}.ffn_norm", (H,))]
        if l in moe_layers:
            want += [(None, None)] * 3
        else:
            want += [(f"{p}.ffn_gate", (F, H)), (f"{p}.ffn_up", (F, H)), (f"{p}.ffn_down", (H, F))]
        if flags & 1:
            want += [(f"{p}.attn_q_norm", (hd,)), (f"{p}.attn_k_norm", (hd,))]
    want += [("output_norm", (H,)), (head, (V, H))]
    for name, shape in want + [("embed", (V, H))]:
        if name is None:
            continue
        e = som.find(name)
        if e is None:
            raise SomError(f"decode_plan: {name}: missing", ERR_ARG)
        if e.shape != shape:
            raise SomError(f"decode_plan: {name}: shape {list(e.shape)} vs {list(shape)}", ERR_ARG)
    cfg = dict(n_layers=L, hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=F or 1, vocab=V,
               rope_theta=m.rope_theta, rms_eps=m.rms_eps)
    return cfg, want, {"flags": flags, "moe_layers": moe_layers}


class SomDecoder:
    """One converted model's decode step on the device (decode_preparar /
    decode_token for a dense GQA decoder).  step(token, pos) embeds the token
    (an F32 `embed` row, source.rs:308-340), runs every layer, the output norm,
    the head and the greedy argmax, and returns the next token."""

    def __init__(self, gpu, som, model_key, cfg, keys, embed_scale):
        self.gpu, self.som, self.key, self.cfg, self.keys = gpu, som, model_key, cfg, keys
        self.embed_scale = embed_scale
        H, V = cfg["hidden"], cfg["vocab"]
        self._x = gpu.dev_alloc(H * 4)
        self._logits = gpu.dev_alloc(V * 4)
        self._tok = gpu.dev_alloc(4)

    def embed(self, token):
        H = self.cfg["hidden"]
        row = self.som.load_f32_range("embed", token * H, H)
        return row if self.embed_scale == 1.0 else (row * np.float32(self.embed_scale)).astype(np.float32)

    def step(self, token, pos, logits=False):
        g = self.gpu
        g.h2d(self._x, self.embed(token))
        g.decode_step_dev(self.key, self._x, pos, self._logits, self._tok)
        g.sync()
        t = int(g.d2h(self._tok, (1,), np.uint32)[0])
        if logits:
            return t, g.d2h(self._logits, (self.cfg["vocab"],), np.float32)
        return t

    def close(self):
        g = self.gpu
        if self._x is None:
            return
        for p in (self._x, self._logits, self._tok):
            g.dev_free(p)
        self._x = None
        g.decode_destroy(self.key)
        for k in dict.fromkeys(self.keys):
            if k is not None:
                g.weight_drop(k)


def prepare_decode(gpu, som, model_key, ctx_max=None, kv_f16=False):
    """Makes a converted model resident and builds its device decode step (KV
    cache of ctx_max positions, manifest max_seq by default): dense layers
    from their tensors, MoE layers registered first (prepare_moe_layer)."""
    cfg, want, extra = decode_plan(som)
    m = som.manifest
    cfg = dict(cfg, ctx_max=ctx_max or m.max_seq, kv_f16=1 if kv_f16 else 0)
    keys, moe_keys = [], [None] * cfg["n_layers"]
    uploaded = []

    def undo():
        # a declined or failed model leaves nothing resident, so a caller
        # that falls back to the CPU gets the device memory back (dropping a
        # weight also unregisters the MoE layers that read it)
        for k in dict.fromkeys(uploaded):
            gpu.weight_drop(k)

    try:
        for l in extra["moe_layers"]:
            moe_keys[l] = prepare_moe_layer(gpu, som, l, f"{model_key}.L{l:02}.moe", uploaded=uploaded)
        for name, shape in want:
            if name is not None and name not in keys:
                v = som.tensor_view(name)
                rows, cols = (1, shape[0]) if len(shape) == 1 else shape
                _upload(gpu, name, v, rows, cols)
                uploaded.append(name)
            keys.append(name)
        ok = gpu.decode_create(model_key, cfg, keys, moe_layers=moe_keys if extra["moe_layers"] else None,
                               flags=extra["flags"])
    except BaseException:
        undo()
        raise
    if not ok:
        err = gpu.last_error()
        undo()
        raise SomError(f"prepare_decode: the device step declined the model: {err}", ERR_ARG)
    return SomDecoder(gpu, som, model_key, cfg, keys, m.embed_scale())


def prepare_moe_layer(gpu, som, layer, layer_key=None, uploaded=None):
    """Registers layer `layer`'s MoE FFN (router L{ll}.ffn_gate_inp, experts
    L{ll}.E{e}.ffn_gate/up/down; runtime.rs:448-469) for moe_ffn_dev; returns
    the layer key.  The keys it makes resident are appended to `uploaded`
    (when given) as they go up, so that a caller can drop them on failure."""
    m = som.manifest
    if m is None or not m.layer_is_moe(layer):
        raise SomError(f"prepare_moe_layer: layer {layer} is not MoE", ERR_ARG)
    s = m.layer(layer) or LayerSpec()
    if s.ffn_kind == FFN_LATENT_MOE or s.num_shared_experts:
        raise SomError(f"prepare_moe_layer: layer {layer}: latent or shared experts are not on the device FFN",
                       ERR_ARG)
    H, E, k, F = m.hidden_dim, m.effective_num_experts(layer), m.effective_num_experts_per_tok(layer), \
        m.effective_moe_ffn_dim(layer)
    p = f"L{layer:02}"
    router = f"{p}.ffn_gate_inp"
    need = [(router, (E, H))]
    experts = []
    for e in range(E):
        ep = f"{p}.E{e:02}"
        experts += [f"{ep}.ffn_gate", f"{ep}.ffn_up", f"{ep}.ffn_down"]
        need += [(f"{ep}.ffn_gate", (F, H)), (f"{ep}.ffn_up", (F, H)), (f"{ep}.ffn_down", (H, F))]
    for name, shape in need:
        ent = som.find(name)
        if ent is None or ent.shape != shape:
            raise SomError(f"prepare_moe_layer: {name}: missing or shape "
                           f"{None if ent is None else list(ent.shape)} vs {list(shape)}", ERR_ARG)
        _upload(gpu, name, som.tensor_view(name), *shape)
        if uploaded is not None:
            uploaded.append(name)
    key = layer_key or f"{p}.moe"
    gpu.moe_register(key, router, experts, E, H, F, k)
    return key
