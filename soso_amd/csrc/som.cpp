// som.cpp -- reader of soso's on-disk model format (.som): manifest, tensor
// index, CRC-checked shards mapped read-only.  Host code (g++), no GPU calls.
//
// Reference: crates/sosomodel/src/lib.rs (header, CRC32C, bounds-checked
// reader), index.rs (TensorIndex, shards), manifest.rs (Manifest v1..v9,
// LayerSpec), and crates/soso-llm-core/src/source.rs (MmapTensorSource).
// Byte layouts follow the reference because they are the file format; the
// code is this build's.
#include "../../include/soso_som.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// CRC-32C.  Slicing-by-8 tables for the portable path; the SSE4.2 crc32
// instruction computes the same reflected Castagnoli CRC without the pre/post
// inversion, which soso_som_crc32c applies around either path.
// ---------------------------------------------------------------------------
struct CrcTables {
    uint32_t t[8][256];
    CrcTables()
    {
        for (uint32_t i = 0; i < 256; i++) {
            uint32_t c = i;
            for (int k = 0; k < 8; k++) c = (c & 1) ? (c >> 1) ^ 0x82F63B78u : c >> 1;
            t[0][i] = c;
        }
        for (int j = 1; j < 8; j++)
            for (uint32_t i = 0; i < 256; i++) t[j][i] = (t[j - 1][i] >> 8) ^ t[0][t[j - 1][i] & 0xff];
    }
};
const CrcTables &crc_tables()
{
    static const CrcTables tabs;
    return tabs;
}

uint32_t crc_portable(uint32_t c, const uint8_t *p, size_t n)
{
    const CrcTables &T = crc_tables();
    while (n >= 8) {
        uint32_t lo, hi;
        memcpy(&lo, p, 4);
        memcpy(&hi, p + 4, 4);
        lo ^= c;
        c = T.t[7][lo & 0xff] ^ T.t[6][(lo >> 8) & 0xff] ^ T.t[5][(lo >> 16) & 0xff] ^ T.t[4][lo >> 24] ^
            T.t[3][hi & 0xff] ^ T.t[2][(hi >> 8) & 0xff] ^ T.t[1][(hi >> 16) & 0xff] ^ T.t[0][hi >> 24];
        p += 8;
        n -= 8;
    }
    while (n--) c = (c >> 8) ^ T.t[0][(c ^ *p++) & 0xff];
    return c;
}

__attribute__((target("sse4.2"))) uint32_t crc_sse42(uint32_t c, const uint8_t *p, size_t n)
{
    uint64_t c64 = c;
    while (n >= 8) {
        uint64_t v;
        memcpy(&v, p, 8);
        c64 = __builtin_ia32_crc32di(c64, v);
        p += 8;
        n -= 8;
    }
    uint32_t c32 = (uint32_t)c64;
    while (n--) c32 = __builtin_ia32_crc32qi(c32, *p++);
    return c32;
}

bool have_sse42()
{
    static const bool yes = [] {
        __builtin_cpu_init();
        return __builtin_cpu_supports("sse4.2") != 0;
    }();
    return yes;
}

thread_local std::string g_err;

int fail(int rc, const std::string &msg)
{
    g_err = msg;
    return rc;
}

// ---------------------------------------------------------------------------
// Bounds-checked little-endian reader over a byte range (lib.rs:100-147).
// ---------------------------------------------------------------------------
// Rust's str::from_utf8: no overlong forms, no surrogates, nothing above
// U+10FFFF.
bool utf8_ok(const uint8_t *s, size_t n)
{
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int len;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) {
            len = 2;
            cp = c & 0x1F;
        } else if ((c & 0xF0) == 0xE0) {
            len = 3;
            cp = c & 0x0F;
        } else if ((c & 0xF8) == 0xF0) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + len > n) return false;
        for (int k = 1; k < len; k++) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000)) return false;
        if (cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += len;
    }
    return true;
}

struct Reader {
    const uint8_t *d;
    size_t n, off = 0;
    bool ok = true;
    Reader(const uint8_t *data, size_t len) : d(data), n(len) {}
    const uint8_t *take(size_t k)
    {
        if (!ok || k > n - off) {
            ok = false;
            return nullptr;
        }
        const uint8_t *p = d + off;
        off += k;
        return p;
    }
    uint8_t u8()
    {
        const uint8_t *p = take(1);
        return p ? p[0] : 0;
    }
    uint32_t u32()
    {
        uint32_t v = 0;
        if (const uint8_t *p = take(4)) memcpy(&v, p, 4);
        return v;
    }
    uint64_t u64()
    {
        uint64_t v = 0;
        if (const uint8_t *p = take(8)) memcpy(&v, p, 8);
        return v;
    }
    float f32()
    {
        float v = 0.0f;
        if (const uint8_t *p = take(4)) memcpy(&v, p, 4);
        return v;
    }
    // NUL-terminated UTF-8
    std::string cstr()
    {
        if (!ok) return std::string();
        const void *z = memchr(d + off, 0, n - off);
        if (!z) {
            ok = false;
            return std::string();
        }
        const size_t len = (const uint8_t *)z - (d + off);
        if (!utf8_ok(d + off, len)) {
            ok = false;
            return std::string();
        }
        std::string s((const char *)d + off, len);
        off += len + 1;
        return s;
    }
};

constexpr size_t HEADER = 24;      // magic 8 | crc u32 | version u32 | payload_len u64
constexpr size_t PAYLOAD_V2 = 64;  // shard payload offset from version 2 (index.rs:98-101)
const uint8_t MAGIC[8] = {'S', 'O', 'M', 'O', 'D', 'L', '0', '1'};

// parse_som (lib.rs:80-98): header, explicit length, CRC of the body.
bool parse_som(const uint8_t *d, size_t n, uint32_t *version, const uint8_t **body, size_t *body_len)
{
    if (!d || n < HEADER || memcmp(d, MAGIC, 8) != 0) return false;
    uint32_t crc;
    uint64_t len;
    memcpy(&crc, d + 8, 4);
    memcpy(version, d + 12, 4);
    memcpy(&len, d + 16, 8);
    if (len > n - HEADER) return false;
    *body = d + HEADER;
    *body_len = (size_t)len;
    return soso_som_crc32c(*body, *body_len) == crc;
}

// ---------------------------------------------------------------------------
// Manifest (manifest.rs:1021-1190)
// ---------------------------------------------------------------------------
struct Prefetch {
    uint32_t layer;
    std::vector<std::string> shards;
};

struct Manifest {
    soso_som_manifest g{};
    std::string name, chat_template;
    std::vector<soso_som_layer> layers; // v4+; empty with `synth` for v1-v3
    bool synth = false;
    soso_som_layer synth_spec{};
    std::vector<uint32_t> window;
    std::vector<float> rope_theta;
    std::vector<Prefetch> prefetch;

    bool layer(uint32_t i, soso_som_layer *out) const
    {
        if (synth) {
            if (i >= g.num_layers) return false;
            *out = synth_spec;
            return true;
        }
        if (i >= layers.size()) return false;
        *out = layers[i];
        return true;
    }
    // effective_* (manifest.rs:428-465)
    uint32_t heads(uint32_t l) const
    {
        soso_som_layer s;
        return layer(l, &s) && s.num_heads ? s.num_heads : g.num_heads;
    }
    uint32_t kv_heads(uint32_t l) const
    {
        soso_som_layer s;
        return layer(l, &s) && s.num_kv_heads ? s.num_kv_heads : g.num_kv_heads;
    }
    uint32_t head_dim(uint32_t l) const
    {
        soso_som_layer s;
        if (layer(l, &s) && s.v_head_dim) return s.v_head_dim;
        const uint32_t h = heads(l);
        return h ? g.hidden_dim / h : 0;
    }
    // validate_layer_divisibility (manifest.rs:548-593)
    bool layer_ok(uint32_t l) const
    {
        const uint32_t h = heads(l), kv = kv_heads(l);
        if (!h || !kv) return false;
        soso_som_layer s;
        const bool has = layer(l, &s);
        const uint8_t kind = has ? s.attn_kind : 0;
        switch (kind) {
        case 4: return kv % h == 0 && head_dim(l) != 0;             // Gdn
        case 3: return h % kv == 0 && head_dim(l) != 0;             // Gated
        case 1: return h % kv == 0;                                 // Mla
        case 0:
        case 2:                                                     // Gqa, Kda
            if (h % kv || head_dim(l) == 0) return false;
            return !((has ? s.v_head_dim : 0) == 0 && g.hidden_dim % h);
        default: return g.hidden_dim % h == 0 && h % kv == 0;       // Bidirectional, Cross
        }
    }
};

bool parse_layer_spec(Reader &r, soso_som_layer *s)
{
    s->attn_kind = r.u8();
    s->ffn_kind = r.u8();
    s->pad = 0;
    r.take(2);
    if (!r.ok || s->attn_kind > 6 || s->ffn_kind > 3) return false;
    uint32_t *f = &s->num_heads;
    for (int i = 0; i < 13; i++) f[i] = r.u32();
    return r.ok;
}

int parse_manifest(const uint8_t *d, size_t n, Manifest *m)
{
    uint32_t ver;
    const uint8_t *body;
    size_t blen;
    if (!parse_som(d, n, &ver, &body, &blen)) return fail(SOSO_SOM_ERR_FORMAT, "manifest: bad header or CRC");
    Reader r(body, blen);
    soso_som_manifest &g = m->g;
    g.version = ver;
    m->name = r.cstr();
    g.vocab_size = r.u32();
    g.hidden_dim = r.u32();
    g.num_layers = r.u32();
    g.num_heads = r.u32();
    g.ffn_dim = r.u32();
    g.max_seq = r.u32();
    if (ver >= 2) {
        g.num_kv_heads = r.u32();
        g.rope_theta = r.f32();
        g.rms_eps = r.f32();
    } else {
        g.num_kv_heads = g.num_heads;
        g.rope_theta = 10000.0f;
        g.rms_eps = 1e-5f;
    }
    if (ver >= 3) {
        g.num_experts = r.u32();
        g.num_experts_per_tok = r.u32();
        g.moe_ffn_dim = r.u32();
    }
    if (!r.ok) return fail(SOSO_SOM_ERR_FORMAT, "manifest: truncated globals");
    if (g.num_heads == 0 || g.num_kv_heads == 0) return fail(SOSO_SOM_ERR_FORMAT, "manifest: zero heads");
    if (ver < 4 && (g.hidden_dim % g.num_heads || g.num_heads % g.num_kv_heads))
        return fail(SOSO_SOM_ERR_FORMAT, "manifest: heads do not divide hidden / kv heads");
    if (ver >= 4) {
        const uint32_t ns = r.u32();
        if (!r.ok || ns != g.num_layers) return fail(SOSO_SOM_ERR_FORMAT, "manifest: layer table length");
        for (uint32_t i = 0; i < ns; i++) {
            soso_som_layer s;
            if (!parse_layer_spec(r, &s)) return fail(SOSO_SOM_ERR_FORMAT, "manifest: layer spec");
            m->layers.push_back(s);
        }
    } else {
        // synthesize_layers_from_globals (manifest.rs:533-546): Gqa, Moe if experts
        m->synth = true;
        m->synth_spec = soso_som_layer{};
        m->synth_spec.ffn_kind = g.num_experts > 0 ? 1 : 0;
    }
    const uint32_t npf = r.u32();
    for (uint32_t i = 0; r.ok && i < npf; i++) {
        Prefetch pf;
        pf.layer = r.u32();
        const uint32_t ns = r.u32();
        for (uint32_t j = 0; r.ok && j < ns; j++) pf.shards.push_back(r.cstr());
        if (r.ok) m->prefetch.push_back(std::move(pf));
    }
    if (!r.ok) return fail(SOSO_SOM_ERR_FORMAT, "manifest: prefetch graph");
    if (ver >= 5) m->chat_template = r.cstr();
    if (ver >= 6) {
        g.model_kind = r.u8();
        g.norm_kind = r.u8();
        r.take(2);
        if (r.ok && (g.model_kind > 2 || g.norm_kind > 1)) return fail(SOSO_SOM_ERR_FORMAT, "manifest: model/norm kind");
        uint32_t *a = &g.n_mels;
        for (int i = 0; i < 9; i++) a[i] = r.u32();
    } else {
        // AudioSpec::default (manifest.rs:178-192)
        const uint32_t dflt[9] = {80, 1500, 384, 4, 6, 448, 384, 4, 6};
        memcpy(&g.n_mels, dflt, sizeof(dflt));
    }
    if (ver >= 7 && r.ok) {
        g.embed_scale = r.f32();
        g.logit_softcap = r.f32();
        g.attn_scale = r.f32();
        g.tied_lm_head = r.u32() != 0;
        const uint32_t nw = r.u32();
        if (r.ok && nw > g.num_layers) return fail(SOSO_SOM_ERR_FORMAT, "manifest: window list");
        for (uint32_t i = 0; r.ok && i < nw; i++) m->window.push_back(r.u32());
        const uint32_t nt = r.u32();
        if (r.ok && nt > g.num_layers) return fail(SOSO_SOM_ERR_FORMAT, "manifest: rope theta list");
        for (uint32_t i = 0; r.ok && i < nt; i++) m->rope_theta.push_back(r.f32());
        if (ver >= 8) {
            g.yarn_factor = r.f32();
            g.yarn_orig_ctx = r.u32();
            g.yarn_beta_fast = r.f32();
            g.yarn_beta_slow = r.f32();
        }
    }
    if (ver >= 9 && r.ok) {
        g.has_kev = 1;
        g.kev_temperature = r.f32();
        g.kev_pointer_dim = r.u32();
    }
    if (!r.ok) return fail(SOSO_SOM_ERR_FORMAT, "manifest: truncated body");
    // v1-v3 layers are all the synthesized spec: one check covers them
    const uint32_t check = m->synth ? (g.num_layers ? 1 : 0) : g.num_layers;
    for (uint32_t l = 0; l < check; l++)
        if (!m->layer_ok(l)) return fail(SOSO_SOM_ERR_FORMAT, "manifest: layer " + std::to_string(l) + " head split");
    g.n_layer_specs = g.num_layers;
    g.n_window = (uint32_t)m->window.size();
    g.n_rope_theta = (uint32_t)m->rope_theta.size();
    g.n_prefetch = (uint32_t)m->prefetch.size();
    return SOSO_SOM_OK;
}

// ---------------------------------------------------------------------------
// TensorIndex (index.rs:61-91)
// ---------------------------------------------------------------------------
struct Entry {
    uint32_t id;
    std::string name, shard;
    uint64_t offset, byte_len;
    std::vector<uint32_t> shape;
    uint8_t dtype, quant;
};

int parse_index(const uint8_t *d, size_t n, std::vector<Entry> *out)
{
    uint32_t ver;
    const uint8_t *body;
    size_t blen;
    if (!parse_som(d, n, &ver, &body, &blen)) return fail(SOSO_SOM_ERR_FORMAT, "index: bad header or CRC");
    Reader r(body, blen);
    const uint32_t cnt = r.u32();
    for (uint32_t i = 0; r.ok && i < cnt; i++) {
        Entry e;
        e.id = r.u32();
        e.name = r.cstr();
        e.shard = r.cstr();
        e.offset = r.u64();
        e.byte_len = r.u64();
        const uint32_t nd = r.u32();
        for (uint32_t k = 0; r.ok && k < nd; k++) e.shape.push_back(r.u32());
        e.dtype = r.u8();
        e.quant = r.u8();
        r.take(2);
        if (r.ok) out->push_back(std::move(e));
    }
    if (!r.ok) return fail(SOSO_SOM_ERR_FORMAT, "index: truncated entry");
    return SOSO_SOM_OK;
}

struct Shard {
    void *map = nullptr;
    size_t map_len = 0;
    size_t payload_off = 0, payload_len = 0;
};

bool read_file(const std::string &path, std::vector<uint8_t> *out)
{
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return false;
    uint8_t buf[1 << 16];
    size_t k;
    while ((k = fread(buf, 1, sizeof(buf), f)) > 0) out->insert(out->end(), buf, buf + k);
    const bool ok = !ferror(f);
    fclose(f);
    return ok;
}

} // namespace

struct soso_som {
    bool has_manifest = false;
    Manifest m;
    std::vector<Entry> entries;
    std::unordered_map<std::string, size_t> first_by_name, last_by_name;
    std::string shards_dir;
    std::map<std::string, Shard> shards;
};

namespace {

// MmapTensorSource::ensure_mapped (source.rs:108-156): map once, verify once
int map_shard(soso_som *s, const std::string &name, Shard **out)
{
    auto it = s->shards.find(name);
    if (it != s->shards.end()) {
        *out = &it->second;
        return SOSO_SOM_OK;
    }
    const std::string path = s->shards_dir + "/" + name;
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(SOSO_SOM_ERR_IO, "shard " + path + ": cannot open");
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(SOSO_SOM_ERR_IO, "shard " + path + ": cannot stat");
    }
    Shard sh;
    sh.map_len = (size_t)st.st_size;
    if (sh.map_len) {
        sh.map = mmap(nullptr, sh.map_len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (sh.map == MAP_FAILED) {
            close(fd);
            return fail(SOSO_SOM_ERR_IO, "shard " + path + ": mmap failed");
        }
    }
    close(fd);
    if (soso_som_verify_shard((const uint8_t *)sh.map, sh.map_len, &sh.payload_off, &sh.payload_len) != SOSO_SOM_OK) {
        if (sh.map) munmap(sh.map, sh.map_len);
        return fail(SOSO_SOM_ERR_FORMAT, "shard " + path + ": bad header or CRC");
    }
    *out = &s->shards.emplace(name, sh).first->second;
    return SOSO_SOM_OK;
}

const Entry *lookup(const soso_som *s, const char *name, size_t len, bool last)
{
    if (!name) return nullptr;
    const auto &mp = last ? s->last_by_name : s->first_by_name;
    auto it = mp.find(std::string(name, len));
    return it == mp.end() ? nullptr : &s->entries[it->second];
}

bool elems_of(const Entry &e, uint64_t *out)
{
    uint64_t n = 1;
    for (uint32_t d : e.shape) {
        if (d && n > UINT64_MAX / d) return false;
        n *= d;
    }
    *out = n;
    return true;
}

// MmapTensorSource::tensor_bytes (source.rs:166-185)
int tensor_bytes(soso_som *s, const Entry &e, uint64_t off, uint64_t len, const uint8_t **out)
{
    if (len > UINT64_MAX - off || off + len > e.byte_len)
        return fail(SOSO_SOM_ERR_ARG, e.name + ": range past the tensor's bytes");
    Shard *sh;
    const int rc = map_shard(s, e.shard, &sh);
    if (rc != SOSO_SOM_OK) return rc;
    if (off > UINT64_MAX - e.offset || e.offset + off > sh->payload_len || len > sh->payload_len - (e.offset + off))
        return fail(SOSO_SOM_ERR_FORMAT, e.name + ": tensor past the end of shard " + e.shard);
    *out = (const uint8_t *)sh->map + sh->payload_off + e.offset + off;
    return SOSO_SOM_OK;
}

int finish_open(soso_som *s, soso_som **out)
{
    for (size_t i = 0; i < s->entries.size(); i++) {
        s->first_by_name.emplace(s->entries[i].name, i);
        s->last_by_name[s->entries[i].name] = i;
    }
    *out = s;
    return SOSO_SOM_OK;
}

} // namespace

extern "C" {

uint32_t soso_som_crc32c(const void *data, size_t len)
{
    const uint8_t *p = (const uint8_t *)data;
    if (!p) len = 0;
    const uint32_t c = have_sse42() ? crc_sse42(0xFFFFFFFFu, p, len) : crc_portable(0xFFFFFFFFu, p, len);
    return c ^ 0xFFFFFFFFu;
}

uint32_t soso_som_crc32c_portable(const void *data, size_t len)
{
    return crc_portable(0xFFFFFFFFu, (const uint8_t *)data, data ? len : 0) ^ 0xFFFFFFFFu;
}

const char *soso_som_error(void) { return g_err.c_str(); }

int soso_som_verify_shard(const uint8_t *data, size_t len, size_t *payload_off, size_t *payload_len)
{
    if (!data || len < HEADER || memcmp(data, MAGIC, 8) != 0) return fail(SOSO_SOM_ERR_FORMAT, "shard: no .som header");
    uint32_t crc, ver;
    uint64_t plen;
    memcpy(&crc, data + 8, 4);
    memcpy(&ver, data + 12, 4);
    memcpy(&plen, data + 16, 8);
    const size_t off = ver >= 2 ? PAYLOAD_V2 : HEADER;
    if (off > len || plen > len - off) return fail(SOSO_SOM_ERR_FORMAT, "shard: payload past the end");
    if (soso_som_crc32c(data + off, (size_t)plen) != crc) return fail(SOSO_SOM_ERR_FORMAT, "shard: CRC mismatch");
    if (payload_off) *payload_off = off;
    if (payload_len) *payload_len = (size_t)plen;
    return SOSO_SOM_OK;
}

int soso_som_open_bytes(const uint8_t *manifest, size_t manifest_len, const uint8_t *index, size_t index_len,
                        const char *shards_dir, size_t shards_dir_len, soso_som **out)
{
    if (!out) return fail(SOSO_SOM_ERR_ARG, "open: null handle pointer");
    *out = nullptr;
    soso_som *s = new soso_som;
    if (shards_dir) s->shards_dir.assign(shards_dir, shards_dir_len);
    int rc = SOSO_SOM_OK;
    if (manifest && manifest_len) {
        rc = parse_manifest(manifest, manifest_len, &s->m);
        s->has_manifest = rc == SOSO_SOM_OK;
    }
    if (rc == SOSO_SOM_OK && index && index_len) rc = parse_index(index, index_len, &s->entries);
    if (rc != SOSO_SOM_OK) {
        delete s;
        return rc;
    }
    return finish_open(s, out);
}

int soso_som_open(const char *dir, size_t dir_len, soso_som **out)
{
    if (!dir || !out) return fail(SOSO_SOM_ERR_ARG, "open: null argument");
    *out = nullptr;
    const std::string base(dir, dir_len);
    std::vector<uint8_t> man, idx;
    // layout.rs:4-6: manifest.som, index.som, shards/
    if (!read_file(base + "/manifest.som", &man)) return fail(SOSO_SOM_ERR_IO, base + "/manifest.som: cannot read");
    if (!read_file(base + "/index.som", &idx)) return fail(SOSO_SOM_ERR_IO, base + "/index.som: cannot read");
    const std::string sd = base + "/shards";
    if (man.empty()) return fail(SOSO_SOM_ERR_FORMAT, "manifest.som: empty");
    if (idx.empty()) return fail(SOSO_SOM_ERR_FORMAT, "index.som: empty");
    return soso_som_open_bytes(man.data(), man.size(), idx.data(), idx.size(), sd.data(), sd.size(), out);
}

void soso_som_close(soso_som *s)
{
    if (!s) return;
    for (auto &kv : s->shards)
        if (kv.second.map) munmap(kv.second.map, kv.second.map_len);
    delete s;
}

int soso_som_manifest_get(const soso_som *s, soso_som_manifest *out)
{
    if (!s || !out) return fail(SOSO_SOM_ERR_ARG, "manifest_get: null argument");
    if (!s->has_manifest) return fail(SOSO_SOM_ERR_NOTFOUND, "no manifest");
    *out = s->m.g;
    return SOSO_SOM_OK;
}

int soso_som_manifest_str(const soso_som *s, int which, const char **str, size_t *len)
{
    if (!s || !str || !len) return fail(SOSO_SOM_ERR_ARG, "manifest_str: null argument");
    if (!s->has_manifest) return fail(SOSO_SOM_ERR_NOTFOUND, "no manifest");
    const std::string *v = which == 0 ? &s->m.name : which == 1 ? &s->m.chat_template : nullptr;
    if (!v) return fail(SOSO_SOM_ERR_NOTFOUND, "manifest_str: no such string");
    *str = v->data();
    *len = v->size();
    return SOSO_SOM_OK;
}

int soso_som_layer_spec(const soso_som *s, uint32_t layer, soso_som_layer *out)
{
    if (!s || !out) return fail(SOSO_SOM_ERR_ARG, "layer_spec: null argument");
    if (!s->has_manifest || !s->m.layer(layer, out)) return fail(SOSO_SOM_ERR_NOTFOUND, "layer_spec: no such layer");
    return SOSO_SOM_OK;
}

int soso_som_ext_window(const soso_som *s, uint32_t i, uint32_t *out)
{
    if (!s || !out) return fail(SOSO_SOM_ERR_ARG, "ext_window: null argument");
    if (!s->has_manifest || i >= s->m.window.size()) return fail(SOSO_SOM_ERR_NOTFOUND, "ext_window: index");
    *out = s->m.window[i];
    return SOSO_SOM_OK;
}

int soso_som_ext_rope_theta(const soso_som *s, uint32_t i, float *out)
{
    if (!s || !out) return fail(SOSO_SOM_ERR_ARG, "ext_rope_theta: null argument");
    if (!s->has_manifest || i >= s->m.rope_theta.size()) return fail(SOSO_SOM_ERR_NOTFOUND, "ext_rope_theta: index");
    *out = s->m.rope_theta[i];
    return SOSO_SOM_OK;
}

int soso_som_prefetch(const soso_som *s, uint32_t i, uint32_t *layer, uint32_t *n_shards)
{
    if (!s || !layer || !n_shards) return fail(SOSO_SOM_ERR_ARG, "prefetch: null argument");
    if (!s->has_manifest || i >= s->m.prefetch.size()) return fail(SOSO_SOM_ERR_NOTFOUND, "prefetch: index");
    *layer = s->m.prefetch[i].layer;
    *n_shards = (uint32_t)s->m.prefetch[i].shards.size();
    return SOSO_SOM_OK;
}

int soso_som_prefetch_shard(const soso_som *s, uint32_t i, uint32_t j, const char **name, size_t *len)
{
    if (!s || !name || !len) return fail(SOSO_SOM_ERR_ARG, "prefetch_shard: null argument");
    if (!s->has_manifest || i >= s->m.prefetch.size() || j >= s->m.prefetch[i].shards.size())
        return fail(SOSO_SOM_ERR_NOTFOUND, "prefetch_shard: index");
    *name = s->m.prefetch[i].shards[j].data();
    *len = s->m.prefetch[i].shards[j].size();
    return SOSO_SOM_OK;
}

size_t soso_som_tensor_count(const soso_som *s) { return s ? s->entries.size() : 0; }

int soso_som_tensor_at(const soso_som *s, size_t i, soso_som_tensor *out)
{
    if (!s || !out) return fail(SOSO_SOM_ERR_ARG, "tensor_at: null argument");
    if (i >= s->entries.size()) return fail(SOSO_SOM_ERR_NOTFOUND, "tensor_at: index");
    const Entry &e = s->entries[i];
    out->id = e.id;
    out->name = e.name.data();
    out->name_len = e.name.size();
    out->shard = e.shard.data();
    out->shard_len = e.shard.size();
    out->offset = e.offset;
    out->byte_len = e.byte_len;
    out->ndim = (uint32_t)e.shape.size();
    out->shape = e.shape.data();
    out->dtype = e.dtype;
    out->quant = e.quant;
    return SOSO_SOM_OK;
}

int soso_som_find(const soso_som *s, const char *name, size_t name_len, size_t *i)
{
    if (!s || !name || !i) return fail(SOSO_SOM_ERR_ARG, "find: null argument");
    const Entry *e = lookup(s, name, name_len, false);
    if (!e) return fail(SOSO_SOM_ERR_NOTFOUND, std::string(name, name_len) + ": not in the index");
    *i = (size_t)(e - s->entries.data());
    return SOSO_SOM_OK;
}

int soso_som_tensor_view(soso_som *s, const char *name, size_t name_len, soso_som_view *out)
{
    if (!s || !name || !out) return fail(SOSO_SOM_ERR_ARG, "tensor_view: null argument");
    const Entry *e = lookup(s, name, name_len, true);
    if (!e) return fail(SOSO_SOM_ERR_NOTFOUND, std::string(name, name_len) + ": not in the index");
    uint64_t elems;
    if (!elems_of(*e, &elems)) return fail(SOSO_SOM_ERR_FORMAT, e->name + ": shape overflows");
    const uint8_t *p;
    const int rc = tensor_bytes(s, *e, 0, e->byte_len, &p);
    if (rc != SOSO_SOM_OK) return rc;
    out->bytes = p;
    out->len = (size_t)e->byte_len;
    out->dtype = e->dtype;
    out->elems = elems;
    return SOSO_SOM_OK;
}

int soso_som_load_f32_range(soso_som *s, const char *name, size_t name_len, size_t elem_off, float *out, size_t n)
{
    if (!s || !name || (!out && n)) return fail(SOSO_SOM_ERR_ARG, "load_f32_range: null argument");
    const Entry *e = lookup(s, name, name_len, true);
    if (!e) return fail(SOSO_SOM_ERR_NOTFOUND, std::string(name, name_len) + ": not in the index");
    uint64_t elems;
    if (!elems_of(*e, &elems)) return fail(SOSO_SOM_ERR_FORMAT, e->name + ": shape overflows");
    if (n > SIZE_MAX - elem_off || elem_off + n > elems) return fail(SOSO_SOM_ERR_ARG, e->name + ": range past the tensor");
    if (e->dtype != SOSO_SOM_DTYPE_F32) return fail(SOSO_SOM_ERR_DTYPE, e->name + ": not an F32 tensor");
    const uint8_t *p;
    const int rc = tensor_bytes(s, *e, (uint64_t)elem_off * 4, (uint64_t)n * 4, &p);
    if (rc != SOSO_SOM_OK) return rc;
    memcpy(out, p, n * 4); // little-endian host, as the file
    return SOSO_SOM_OK;
}

int soso_som_load_f32(soso_som *s, const char *name, size_t name_len, float *out, size_t n)
{
    if (!s || !name) return fail(SOSO_SOM_ERR_ARG, "load_f32: null argument");
    const Entry *e = lookup(s, name, name_len, true);
    if (!e) return fail(SOSO_SOM_ERR_NOTFOUND, std::string(name, name_len) + ": not in the index");
    uint64_t elems;
    if (!elems_of(*e, &elems) || elems != n) return fail(SOSO_SOM_ERR_ARG, e->name + ": element count differs");
    return soso_som_load_f32_range(s, name, name_len, 0, out, n);
}

} // extern "C"
