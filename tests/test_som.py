"""The .som reader (libsoso_som.so, soso_amd/som.py) on the CPU.

Pinned by:
* CRC-32C: the published check value and the iSCSI test vectors of RFC 3720
  (B.4), and the SSE4.2 path against the table path on every length and
  alignment up to 80 bytes;
* the reference's own converted records (tests/golden/som_tiny: rootfs/models/
  tiny's manifest.som and index.som, CRCs written by soso): they verify, and
  the manifest's globals equal Manifest::tiny's (crates/sosomodel/src/
  manifest.rs:654-700);
* the reference's tests of the format, restated case by case
  (crates/sosomodel/tests/roundtrip.rs, crates/soso-llm-core/src/source.rs:
  600-695), with our writer producing the records;
* malformed input: every truncation, a corrupted length, bad CRC, magic,
  enum values and UTF-8, refused without a crash (lib.rs:82-84).
"""
import os
import struct

import numpy as np
import pytest

from soso_amd import som

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "som_tiny")


def crc_portable(b):
    a = np.frombuffer(bytes(b), np.uint8)
    return int(som.lib().soso_som_crc32c_portable(a.ctypes.data if a.size else None, a.size))


# ---------------------------------------------------------------------------
# CRC-32C
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("data,want", [
    (b"123456789", 0xE3069283),            # the CRC-32C check value
    (bytes(32), 0x8A9136AA),               # RFC 3720 B.4: 32 bytes of zeros
    (b"\xff" * 32, 0x62A8AB43),            # 32 bytes of ones
    (bytes(range(32)), 0x46DD794E),        # incrementing
    (bytes(range(31, -1, -1)), 0x113FDB5C),  # decrementing
    (b"", 0x00000000),
])
def test_crc32c_published_vectors(data, want):
    assert som.crc32c(data) == want
    assert crc_portable(data) == want


def test_crc32c_paths_agree():
    rng = np.random.default_rng(5)
    buf = rng.integers(0, 256, 200, dtype=np.uint8).tobytes()
    for start in range(8):
        for n in range(80):
            b = buf[start:start + n]
            assert som.crc32c(b) == crc_portable(b), (start, n)
    big = rng.integers(0, 256, 1 << 20, dtype=np.uint8)
    assert som.crc32c(big) == crc_portable(big.tobytes())


# ---------------------------------------------------------------------------
# the reference's tiny model records
# ---------------------------------------------------------------------------
def test_reference_tiny_model_records():
    with som.SomModel.open(GOLD) as m:
        man = m.manifest
        assert man.version == 1
        # Manifest::tiny (manifest.rs:654-700); v1 records take the v1 defaults
        # for kv heads, RoPE base and eps (manifest.rs:1031-1035)
        assert (man.name, man.vocab_size, man.hidden_dim, man.num_layers, man.num_heads, man.num_kv_heads,
                man.ffn_dim, man.max_seq) == ("tiny", 256, 128, 4, 4, 4, 256, 128)
        assert man.rope_theta == 10000.0 and man.rms_eps == np.float32(1e-5)
        assert man.num_experts == 0 and not man.is_moe()
        # synthesized layer table: GQA + dense (manifest.rs:533-546)
        assert len(man.layers) == 4 and all(s == som.LayerSpec() for s in man.layers)
        assert man.effective_head_dim(3) == 32 and man.max_ffn_dim() == 256
        assert man.model_kind == som.MODEL_DECODER and man.audio == som.AUDIO_DEFAULT
        assert man.ext.es_vacia() and man.kev is None and man.chat_template == ""
        # the index: 22 F32 tensors, one shard each except the tied lm_head
        assert len(m.entries) == 22
        for e in m.entries:
            assert e.dtype == som.DTYPE_F32 and e.quant == som.QUANT_NONE and e.offset == 0
            assert e.byte_len == 4 * e.elems()
        assert m.find("L02.attn_k").shape == (128, 128)
        assert m.find("lm_head").shard == m.find("embed").shard == "embed.tensor"
        assert [e.id for e in m.entries] == list(range(22))
        # the prefetch graph names shards the index uses
        shards = {e.shard for e in m.entries}
        assert [l for l, _ in man.prefetch] == [0, 1, 2, 3]
        assert all(s in shards for _, names in man.prefetch for s in names)
        # the shards are not in the tree: a view fails cleanly
        with pytest.raises(som.SomError) as ei:
            m.tensor_view("L00.attn_q")
        assert ei.value.rc == som.ERR_IO


def test_legacy_headerless_shard_refused(tmp_path):
    """Shards of the tiny model predate the header: current soso refuses them
    (verify_shard), and so does the source."""
    raw = np.arange(16, dtype=np.float32).tobytes()
    os.makedirs(tmp_path / "shards")
    (tmp_path / "shards" / "w.tensor").write_bytes(raw + bytes(4096 - len(raw)))
    idx = som.serialize_index([som.make_entry(som.DTYPE_F32, 0, "w", "w.tensor", 0, (16,))])
    with som.SomModel.from_bytes(index=idx, shards_dir=str(tmp_path / "shards")) as m:
        with pytest.raises(som.SomError) as ei:
            m.load_f32("w")
        assert ei.value.rc == som.ERR_FORMAT


# ---------------------------------------------------------------------------
# crates/sosomodel/tests/roundtrip.rs, case by case
# ---------------------------------------------------------------------------
def parse_manifest(b):
    with som.SomModel.from_bytes(manifest=b) as m:
        return m.manifest


def test_manifest_roundtrip():
    p = parse_manifest(som.serialize_manifest(som.Manifest.tiny("test")))
    assert p.name == "test" and p.num_layers == 4 and p.version == 5


def test_manifest_v2_fields_gqa_rope():
    m = som.Manifest.tiny("test")
    m.num_kv_heads, m.rope_theta, m.rms_eps = 2, 500000.0, 1e-6
    p = parse_manifest(som.serialize_manifest(m))
    assert p.num_kv_heads == 2 and abs(p.rope_theta - 500000.0) < 1.0 and abs(p.rms_eps - 1e-6) < 1e-9


def test_manifest_v4_roundtrip_layer_specs():
    m = som.Manifest.tiny("v4")
    m.num_layers = 2
    m.prefetch = m.prefetch[:2]
    m.layers = [som.LayerSpec(attn_kind=som.ATTN_KDA, ffn_kind=som.FFN_LATENT_MOE, num_experts=896,
                              num_experts_per_tok=16, num_shared_experts=2, moe_ffn_dim=3072),
                som.LayerSpec(attn_kind=som.ATTN_MLA, ffn_kind=som.FFN_LATENT_MOE, kv_lora_rank=512, q_lora_rank=1536,
                              qk_rope_head_dim=64, qk_nope_head_dim=128, v_head_dim=128, num_experts=896,
                              num_experts_per_tok=16)]
    p = parse_manifest(som.serialize_manifest(m))
    assert len(p.layers) == 2 and p.layers == m.layers
    assert p.layers[0].num_shared_experts == 2 and p.layers[1].kv_lora_rank == 512
    assert p.prefetch == m.prefetch


def test_manifest_v4_qwen_gated_gdn_without_hidden_split():
    m = som.Manifest.tiny("qwen")
    m.hidden_dim, m.num_heads, m.num_kv_heads, m.num_layers = 20, 3, 1, 2
    m.prefetch = m.prefetch[:2]
    m.layers = [som.LayerSpec(attn_kind=som.ATTN_GDN, num_heads=2, num_kv_heads=4, v_head_dim=4, qk_rope_head_dim=2),
                som.LayerSpec(attn_kind=som.ATTN_GATED, num_heads=3, num_kv_heads=1, v_head_dim=8,
                              qk_rope_head_dim=2)]
    p = parse_manifest(som.serialize_manifest(m))
    assert p.layers[0].attn_kind == som.ATTN_GDN and p.layers[1].attn_kind == som.ATTN_GATED
    assert p.effective_head_dim(1) == 8


def v3_body(m):
    b = [m.name.encode() + b"\0", struct.pack("<6I", m.vocab_size, m.hidden_dim, m.num_layers, m.num_heads,
                                              m.ffn_dim, m.max_seq),
         struct.pack("<Iff3I", m.num_kv_heads, m.rope_theta, m.rms_eps, m.num_experts, m.num_experts_per_tok,
                     m.moe_ffn_dim), struct.pack("<I", len(m.prefetch))]
    for layer, shards in m.prefetch:
        b.append(struct.pack("<II", layer, len(shards)) + b"".join(s.encode() + b"\0" for s in shards))
    return b"".join(b)


def test_manifest_v3_synthesizes_layers():
    p = parse_manifest(som.pack_som(v3_body(som.Manifest.tiny("v3")), 3))
    assert len(p.layers) == 4 and p.layers[0].attn_kind == som.ATTN_GQA and p.layers[0].ffn_kind == som.FFN_DENSE
    moe = som.Manifest.tiny_moe("v3moe")
    p = parse_manifest(som.pack_som(v3_body(moe), 3))
    assert [s.ffn_kind for s in p.layers] == [som.FFN_MOE] * 2 and p.is_moe()


def test_manifest_max_ffn_dim_moe():
    m = som.Manifest.tiny_moe("moe")
    assert m.max_ffn_dim() == m.moe_ffn_dim
    p = parse_manifest(som.serialize_manifest(m))
    assert p.max_ffn_dim() == 32 and p.max_router_experts() == 4 and p.effective_num_experts_per_tok(1) == 2


def test_manifest_v8_yarn_roundtrip():
    m = som.Manifest.tiny("mellum")
    m.ext.window = [1024, 1024, 1024, 0]
    m.ext.yarn = som.YarnSpec(16.0, 8192, 32.0, 1.0)
    p = parse_manifest(som.serialize_manifest(m))
    assert p.version == 8 and p.ext.yarn == m.ext.yarn and p.ext.yarn.activa()
    assert p.layer_window(0) == 1024 and p.layer_window(3) == 0


def test_manifest_v7_ext_and_v6_audio():
    m = som.Manifest.tiny("gemma")
    m.ext = som.ManifestExt(embed_scale=11.3125, logit_softcap=30.0, attn_scale=1.0, tied_lm_head=True,
                            window=[512, 0], rope_theta=[10000.0, 1e6, 0.0])
    p = parse_manifest(som.serialize_manifest(m))
    assert p.version == 7 and p.ext == m.ext
    assert p.layer_rope_theta(1) == 1e6 and p.layer_rope_theta(2) == m.rope_theta and p.embed_scale() == 11.3125
    a = som.Manifest.tiny("asr")
    a.model_kind, a.norm_kind, a.audio = som.MODEL_ASR, som.NORM_LAYER, (128, 1500, 1280, 32, 20, 448, 1280, 32, 20)
    p = parse_manifest(som.serialize_manifest(a))
    assert p.version == 6 and p.model_kind == som.MODEL_ASR and p.norm_kind == som.NORM_LAYER and p.audio == a.audio
    # a plain decoder is written as version 5, whose readers stop before the
    # v6 block: its norm kind and audio read back as the defaults
    d = som.Manifest.tiny("ln")
    d.norm_kind = som.NORM_LAYER
    p = parse_manifest(som.serialize_manifest(d))
    assert p.version == 5 and p.norm_kind == som.NORM_RMS


def test_manifest_v9_kev_roundtrip():
    m = som.Manifest.tiny("kev")
    m.model_kind = som.MODEL_DECISION
    m.kev = som.KevSpec(2.41, 256)
    p = parse_manifest(som.serialize_manifest(m))
    assert p.version == 9 and p.model_kind == som.MODEL_DECISION
    assert abs(p.kev.temperature - 2.41) < 1e-6 and p.kev.pointer_dim == 256
    assert p.ext.es_vacia()


def test_index_roundtrip():
    es = [som.make_entry(som.DTYPE_F32, 0, "w", "s.tensor", 0, (4, 4)),
          som.make_entry(som.DTYPE_Q4_K, 7, "L00.ffn_up", "a.tensor", 4096, (768, 2048)),
          som.make_entry(som.DTYPE_Q8_0, 8, "x", "a.tensor", 0, (100,)),          # 4 blocks, the last partial
          som.make_entry(som.DTYPE_Q6_K, 9, "lm_head", "h.tensor", 64, (128256, 4096))]
    assert es[1].byte_len == 768 * 2048 // 256 * 144 and es[2].byte_len == 4 * 36
    assert es[3].byte_len == 128256 * 16 * 210 and es[3].quant == som.DTYPE_Q6_K
    with som.SomModel.from_bytes(index=som.serialize_index(es)) as m:
        assert m.entries == es and m.manifest is None
        assert m.find("lm_head") == es[3] and m.find("nope") is None


def test_shard_crc_ok_and_detects_corruption():
    packed = som.pack_shard(bytes([1, 2, 3, 4]))
    assert som.verify_shard(packed) == bytes([1, 2, 3, 4])
    bad = bytearray(packed)
    bad[0] ^= 0xFF
    with pytest.raises(som.SomError):
        som.verify_shard(bytes(bad))
    bad = bytearray(packed)
    bad[64] ^= 1  # a payload byte
    with pytest.raises(som.SomError):
        som.verify_shard(bytes(bad))


def test_shard_crc_ending_in_zero_is_not_trimmed():
    for seed in range(600):
        data = bytes((seed * 31 + i) % 251 for i in range(37))
        assert som.verify_shard(som.pack_shard(data)) == data, seed


def test_shard_v2_payload_aligned_to_64():
    data = bytes(range(100))
    packed = som.pack_shard(data)
    a = np.frombuffer(packed, np.uint8)
    import ctypes as C
    off, n = C.c_size_t(), C.c_size_t()
    assert som.lib().soso_som_verify_shard(a.ctypes.data, a.size, C.byref(off), C.byref(n)) == 0
    assert off.value == som.SHARD_PAYLOAD_OFF and off.value % 64 == 0 and n.value == 100
    assert len(packed) % 4096 == 0 and som.verify_shard(packed) == data
    # trailing zeros of the payload are kept
    assert som.verify_shard(som.pack_shard(bytes([1, 2, 3, 0, 0, 0]))) == bytes([1, 2, 3, 0, 0, 0])
    # a v1 shard keeps its payload right after the 24-byte header
    v1 = som.MAGIC + struct.pack("<IIQ", som.crc32c(data), 1, len(data)) + data
    assert som.verify_shard(v1) == data


def test_truncated_and_corrupt_records_never_crash():
    man = som.serialize_manifest(som.Manifest.tiny("t"))
    idx = som.serialize_index([som.make_entry(som.DTYPE_F32, 0, "w", "s.tensor", 0, (4,))])
    for data in (man, idx):
        for cut in range(len(data)):
            for kw in ("manifest", "index"):
                try:
                    som.SomModel.from_bytes(**{kw: data[:cut]}).close()
                except som.SomError:
                    pass
    evil = bytearray(man)
    evil[16:24] = struct.pack("<Q", 2 ** 64 - 1)
    with pytest.raises(som.SomError):
        parse_manifest(bytes(evil))


def resign(body, version):
    return som.pack_som(body, version)


@pytest.mark.parametrize("mutate,why", [
    (lambda b: b.replace(b"t\0", b"\xc3(\0", 1), "invalid UTF-8 in the name"),
    (lambda b: b[:2] + struct.pack("<I", 0) + b[6:], "zero heads"),
])
def test_bad_manifest_fields_refused(mutate, why):
    m = som.Manifest.tiny("t")
    body = som.serialize_manifest(m)
    plen = struct.unpack_from("<Q", body, 16)[0]
    raw = body[24:24 + plen]
    if "heads" in why:
        # num_heads sits after the name and three u32s
        off = raw.index(b"\0") + 1 + 12
        raw = raw[:off] + struct.pack("<I", 0) + raw[off + 4:]
    else:
        raw = mutate(raw)
    with pytest.raises(som.SomError):
        parse_manifest(resign(raw, 5))


def test_bad_enums_and_lists_refused():
    m = som.Manifest.tiny("t")
    m.num_layers, m.prefetch = 1, []
    m.fill_layers_from_globals()
    m.layers[0].attn_kind = 6
    parse_manifest(som.serialize_manifest(m))  # Cross: the last valid kind
    m.layers[0].attn_kind = 7
    with pytest.raises(som.SomError):
        parse_manifest(som.serialize_manifest(m))
    m.layers[0].attn_kind = som.ATTN_GQA
    m.ext.window = [0, 0]  # longer than num_layers
    with pytest.raises(som.SomError):
        parse_manifest(som.serialize_manifest(m))
    m.ext.window = []
    m.hidden_dim = 130  # GQA without v_head_dim must split hidden into heads
    with pytest.raises(som.SomError):
        parse_manifest(som.serialize_manifest(m))
    bad = bytearray(som.serialize_manifest(som.Manifest.tiny("t")))
    bad[0] = ord("X")
    with pytest.raises(som.SomError):
        parse_manifest(bytes(bad))
    bad = bytearray(som.serialize_manifest(som.Manifest.tiny("t")))
    bad[30] ^= 0x10  # a body byte: CRC
    with pytest.raises(som.SomError):
        parse_manifest(bytes(bad))


# ---------------------------------------------------------------------------
# MmapTensorSource (crates/soso-llm-core/src/source.rs:600-695)
# ---------------------------------------------------------------------------
def source_with(tmp_path, entries, shards):
    d = tmp_path / "shards"
    os.makedirs(d, exist_ok=True)
    for name, payload in shards.items():
        (d / name).write_bytes(som.pack_shard(payload))
    return som.SomModel.from_bytes(index=som.serialize_index(entries), shards_dir=str(d))


def f32b(*v):
    return np.array(v, np.float32).tobytes()


def test_load_f32_from_indexed_shard(tmp_path):
    with source_with(tmp_path, [som.make_entry(som.DTYPE_F32, 0, "L00.ffn_up", "L00.ffn_up.tensor", 0, (2, 2))],
                     {"L00.ffn_up.tensor": f32b(0, 1, 2, 3)}) as s:
        assert list(s.load_f32("L00.ffn_up")) == [0, 1, 2, 3]


def test_load_f32_range_reads_a_row(tmp_path):
    with source_with(tmp_path, [som.make_entry(som.DTYPE_F32, 0, "embed", "embed.tensor", 0, (4, 2))],
                     {"embed.tensor": f32b(0, 1, 10, 11, 20, 21, 30, 31)}) as s:
        assert list(s.load_f32_range("embed", 4, 2)) == [20, 21]
        with pytest.raises(som.SomError):
            s.load_f32_range("embed", 7, 2)


def test_load_f32_rejects_wrong_length(tmp_path):
    with source_with(tmp_path, [som.make_entry(som.DTYPE_F32, 0, "w", "w.tensor", 0, (2,))],
                     {"w.tensor": f32b(1, 2)}) as s:
        with pytest.raises(som.SomError):
            s.load_f32("w", 3)


def test_load_f32_from_packed_trunk(tmp_path):
    es = [som.make_entry(som.DTYPE_F32, 0, "L00.a", "L00.trunk.tensor", 0, (2,)),
          som.make_entry(som.DTYPE_F32, 1, "L00.b", "L00.trunk.tensor", 8, (2, 2))]
    with source_with(tmp_path, es, {"L00.trunk.tensor": f32b(1, 2, 3, 4, 5, 6)}) as s:
        assert list(s.load_f32("L00.a")) == [1, 2]
        b = s.load_f32("L00.b")
        assert b[0] == 3 and b[3] == 6
        # mapping the shard again changes nothing
        assert list(s.load_f32("L00.a")) == [1, 2]


def test_views_bounds_dtypes_and_duplicates(tmp_path):
    q = np.arange(2 * 144, dtype=np.uint8).tobytes()
    es = [som.make_entry(som.DTYPE_Q4_K, 0, "q", "q.tensor", 0, (2, 256)),
          som.make_entry(som.DTYPE_F32, 1, "past", "q.tensor", 200, (40,)),   # 160 B from 200: past 288
          som.make_entry(som.DTYPE_F32, 2, "dup", "d.tensor", 0, (1,)),
          som.make_entry(som.DTYPE_F32, 3, "dup", "d.tensor", 4, (1,))]
    with source_with(tmp_path, es, {"q.tensor": q, "d.tensor": f32b(7, 9)}) as s:
        v = s.tensor_view("q")
        assert v.dtype == som.DTYPE_Q4_K and v.elems == 512 and v.bytes.tobytes() == q
        assert not v.bytes.flags.writeable
        with pytest.raises(som.SomError) as ei:
            s.tensor_view("past")
        assert ei.value.rc == som.ERR_FORMAT
        with pytest.raises(som.SomError) as ei:
            s.load_f32("q")
        assert ei.value.rc == som.ERR_DTYPE
        # TensorIndex::find takes the first entry of a name, the source's
        # name map the last (source.rs:76-86, 94-103)
        assert s.find("dup").id == 2 and list(s.load_f32("dup")) == [9]
        with pytest.raises(som.SomError) as ei:
            s.tensor_view("missing")
        assert ei.value.rc == som.ERR_NOTFOUND


def test_write_model_and_decode_plan(tmp_path):
    """A dense GQA decoder passes the checks of Runtime (runtime.rs:330-475);
    NeoX RoPE and QK norm (with their attn_q_norm / attn_k_norm tensors) and
    plain MoE layers map onto the device step; what it does not run is
    refused with the reason."""
    H, nh, nkv, F, V, L = 256, 2, 1, 512, 64, 2
    man = som.Manifest(name="d", vocab_size=V, hidden_dim=H, num_layers=L, num_heads=nh, num_kv_heads=nkv,
                       ffn_dim=F, max_seq=64, rope_theta=5e5, rms_eps=1e-5)
    man.fill_layers_from_globals()
    qd, kvd = nh * 128, nkv * 128

    def t(name, dtype, shape):
        e = som.make_entry(dtype, 0, name, "", 0, shape)
        return (name, dtype, shape, np.zeros(e.byte_len, np.uint8))

    ts = []
    for l in range(L):
        p = f"L{l:02}"
        ts += [t(f"{p}.attn_norm", 1, (H,)), t(f"{p}.attn_q", 3, (qd, H)), t(f"{p}.attn_k", 3, (kvd, H)),
               t(f"{p}.attn_v", 3, (kvd, H)), t(f"{p}.attn_output", 3, (H, qd)), t(f"{p}.ffn_norm", 1, (H,)),
               t(f"{p}.ffn_gate", 3, (F, H)), t(f"{p}.ffn_up", 3, (F, H)), t(f"{p}.ffn_down", 3, (H, F))]
    ts += [t("output_norm", 1, (H,)), t("embed", 1, (V, H)), t("lm_head", 13, (V, H))]
    som.write_model(str(tmp_path / "ok"), man, ts)
    with som.SomModel.open(str(tmp_path / "ok")) as s:
        cfg, want, extra = som.decode_plan(s)
        assert extra == {"flags": 0, "moe_layers": []}
        assert cfg["n_layers"] == L and cfg["head_dim"] == 128 and cfg["rope_theta"] == np.float32(5e5)
        assert [n for n, _ in want][:9] == ["L00.attn_norm", "L00.attn_q", "L00.attn_k", "L00.attn_v",
                                            "L00.attn_output", "L00.ffn_norm", "L00.ffn_gate", "L00.ffn_up",
                                            "L00.ffn_down"]
        assert want[-1] == ("lm_head", (V, H)) and s.tensor_view("lm_head").dtype == som.DTYPE_Q6_K
    # tied: no lm_head, the logits come from embed
    som.write_model(str(tmp_path / "tied"), man, [x for x in ts if x[0] != "lm_head"])
    with som.SomModel.open(str(tmp_path / "tied")) as s:
        assert som.decode_plan(s)[1][-1] == ("embed", (V, H))
    import copy

    def flagged(fl):
        m2 = copy.deepcopy(man)
        for ls in m2.layers:
            ls.flags = fl
        return m2
    # NeoX RoPE on every layer: flags 2, the same tensors
    som.write_model(str(tmp_path / "neox"), flagged(som.FLAG_ROPE_NEOX), ts)
    with som.SomModel.open(str(tmp_path / "neox")) as s:
        _, want2, extra = som.decode_plan(s)
        assert extra["flags"] == 2 and want2 == want
    # QK norm: flags 1, attn_q_norm / attn_k_norm [head_dim] after each layer's nine
    qk = ts + [t(f"L{l:02}.attn_{w}_norm", 1, (128,)) for l in range(L) for w in "qk"]
    som.write_model(str(tmp_path / "qk"), flagged(som.FLAG_QK_NORM | som.FLAG_ROPE_NEOX), qk)
    with som.SomModel.open(str(tmp_path / "qk")) as s:
        _, want2, extra = som.decode_plan(s)
        assert extra["flags"] == 3
        assert [n for n, _ in want2][9:11] == ["L00.attn_q_norm", "L00.attn_k_norm"] and len(want2) == 11 * L + 2
    # an MoE layer: its gate/up/down slots are None, the layer listed
    m2 = copy.deepcopy(man)
    m2.layers[1].ffn_kind, m2.layers[1].num_experts, m2.layers[1].num_experts_per_tok = som.FFN_MOE, 4, 2
    som.write_model(str(tmp_path / "moe"), m2, ts)
    with som.SomModel.open(str(tmp_path / "moe")) as s:
        _, want2, extra = som.decode_plan(s)
        assert extra["moe_layers"] == [1] and want2[15:18] == [(None, None)] * 3
    refusals = {
        "qk_norm_missing": (lambda m: [setattr(x, "flags", som.FLAG_QK_NORM) for x in m.layers], "attn_q_norm"),
        "flags_differ": (lambda m: setattr(m.layers[1], "flags", som.FLAG_ROPE_NEOX), "differ in flags"),
        "sandwich": (lambda m: [setattr(x, "flags", som.FLAG_SANDWICH_NORM) for x in m.layers], "flags"),
        "latent_moe": (lambda m: setattr(m.layers[0], "ffn_kind", som.FFN_LATENT_MOE), "MoE"),
        "softcap": (lambda m: setattr(m.ext, "logit_softcap", 30.0), "extensions"),
        "asr": (lambda m: setattr(m, "model_kind", som.MODEL_ASR), "decoders"),
    }
    for why, (f, msg) in refusals.items():
        m2 = copy.deepcopy(man)
        f(m2)
        som.write_model(str(tmp_path / why), m2, ts)
        with som.SomModel.open(str(tmp_path / why)) as s:
            with pytest.raises(som.SomError, match=msg):
                som.decode_plan(s)
    som.write_model(str(tmp_path / "missing"), man, [x for x in ts if x[0] != "L01.ffn_gate"])
    with som.SomModel.open(str(tmp_path / "missing")) as s:
        with pytest.raises(som.SomError, match="L01.ffn_gate"):
            som.decode_plan(s)
    bad = [x if x[0] != "L00.attn_k" else t("L00.attn_k", 3, (2 * kvd, H)) for x in ts]
    som.write_model(str(tmp_path / "shape"), man, bad)
    with som.SomModel.open(str(tmp_path / "shape")) as s:
        with pytest.raises(som.SomError, match="L00.attn_k"):
            som.decode_plan(s)


@pytest.mark.parametrize("part", ["q", "k", "v"])
def test_decode_plan_refuses_attention_biases(tmp_path, part):
    """A Qwen2 conversion (NeoX RoPE) writes L{ll}.attn_{q,k,v}.bias
    (gguf2som/src/lib.rs:673-680), which soso's CPU layer adds
    (layer.rs:1146-1163).  The device step has no bias term, so decode_plan
    refuses such a model with the reason, as soso's device MoE layer declines
    it (moe_gpu.rs:85-90), instead of returning wrong logits."""
    import copy
    H, nh, nkv, F, V, L = 256, 2, 1, 512, 64, 2
    man = som.Manifest(name="b", vocab_size=V, hidden_dim=H, num_layers=L, num_heads=nh, num_kv_heads=nkv,
                       ffn_dim=F, max_seq=64, rope_theta=1e6, rms_eps=1e-6)
    man.fill_layers_from_globals()
    for ls in man.layers:
        ls.flags = som.FLAG_ROPE_NEOX
    qd, kvd = nh * 128, nkv * 128

    def t(name, dtype, shape):
        e = som.make_entry(dtype, 0, name, "", 0, shape)
        return (name, dtype, shape, np.zeros(e.byte_len, np.uint8))

    ts = []
    for l in range(L):
        p = f"L{l:02}"
        ts += [t(f"{p}.attn_norm", 1, (H,)), t(f"{p}.attn_q", 3, (qd, H)), t(f"{p}.attn_k", 3, (kvd, H)),
               t(f"{p}.attn_v", 3, (kvd, H)), t(f"{p}.attn_output", 3, (H, qd)), t(f"{p}.ffn_norm", 1, (H,)),
               t(f"{p}.ffn_gate", 3, (F, H)), t(f"{p}.ffn_up", 3, (F, H)), t(f"{p}.ffn_down", 3, (H, F))]
    ts += [t("output_norm", 1, (H,)), t("embed", 1, (V, H))]
    som.write_model(str(tmp_path / "nobias"), copy.deepcopy(man), ts)
    with som.SomModel.open(str(tmp_path / "nobias")) as s:
        assert som.decode_plan(s)[2]["flags"] == 2
    dim = qd if part == "q" else kvd
    som.write_model(str(tmp_path / "bias"), man, ts + [t(f"L01.attn_{part}.bias", 1, (dim,))])
    with som.SomModel.open(str(tmp_path / "bias")) as s:
        with pytest.raises(som.SomError, match="bias") as ei:
            som.decode_plan(s)
        assert ei.value.rc == som.ERR_ARG
