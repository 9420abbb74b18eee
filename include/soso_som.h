/* soso_som.h -- reader of soso's on-disk model format (.som), host code.
 *
 * Restates crates/sosomodel (lib.rs, layout.rs, index.rs, manifest.rs) and
 * soso-llm-core's MmapTensorSource (crates/soso-llm-core/src/source.rs) so
 * that a converted soso model directory
 *
 *     <dir>/manifest.som   architecture (Manifest, versions 1..9)
 *     <dir>/index.som      tensor name -> shard, offset, bytes, shape, dtype
 *     <dir>/shards/<name>  payload files with a CRC32C header
 *
 * feeds the GPU path of soso_hip.h: tensor_view returns the mmapped bytes of
 * one tensor, the same TensorView soso hands to GpuDispatch.  In soso the
 * Rust loader stays on its own side of the boundary; this library is for
 * callers that are not soso (tests, benchmarks, C/C++/Python hosts).
 *
 * Every parser is bounds-checked and returns an error on malformed or
 * truncated input, never crashes (lib.rs:82-84).  Not thread-safe: one caller
 * per handle at a time.
 *
 * Format extension owned by this build: dtype 13 = Q6_K (GGML's 210-byte
 * super-block of 256 elements), which sosomodel does not define
 * (layout.rs:8-21); soso converts Q6_K to Q8_0 at import instead
 * (crates/gguf2som/src/lib.rs:1592-1609).
 */
#ifndef SOSO_SOM_H
#define SOSO_SOM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SOSO_SOM_OK 0
#define SOSO_SOM_ERR_IO (-1)       /* file missing or unreadable, mmap failed */
#define SOSO_SOM_ERR_FORMAT (-2)   /* bad magic, CRC mismatch, truncated or malformed body */
#define SOSO_SOM_ERR_NOTFOUND (-3) /* no such tensor / layer / part */
#define SOSO_SOM_ERR_ARG (-4)      /* null pointer, range outside the tensor, wrong length */
#define SOSO_SOM_ERR_DTYPE (-5)    /* the call does not read this dtype */

/* layout.rs:8-21, plus the build-owned Q6_K */
#define SOSO_SOM_DTYPE_F32 1
#define SOSO_SOM_DTYPE_Q8_0 2
#define SOSO_SOM_DTYPE_Q4_K 3
#define SOSO_SOM_DTYPE_MXFP4 4
#define SOSO_SOM_DTYPE_Q4_0 5
#define SOSO_SOM_DTYPE_Q6_K 13

typedef struct soso_som soso_som;

/* LayerSpec (manifest.rs:196-219), its 60-byte on-disk record (:327-344) */
typedef struct {
    uint8_t attn_kind; /* 0 Gqa, 1 Mla, 2 Kda, 3 Gated, 4 Gdn, 5 Bidirectional, 6 Cross */
    uint8_t ffn_kind;  /* 0 Dense, 1 Moe, 2 LatentMoe, 3 GeluMlp */
    uint16_t pad;
    uint32_t num_heads, num_kv_heads, ffn_dim; /* 0 = inherit the global value */
    uint32_t kv_lora_rank, q_lora_rank, qk_rope_head_dim, qk_nope_head_dim, v_head_dim;
    uint32_t num_experts, num_experts_per_tok, moe_ffn_dim, num_shared_experts;
    uint32_t flags; /* FLAG_ROPE_NEOX = 1 << 3, FLAG_QK_NORM = 1 << 4, ... (manifest.rs:221-250) */
} soso_som_layer;

/* Manifest (manifest.rs:282-322): the scalar fields.  Strings, the layer
 * table, the prefetch graph and the per-layer v7 lists have accessors below. */
typedef struct {
    uint32_t version; /* of the manifest.som record */
    uint32_t vocab_size, hidden_dim, num_layers, num_heads, num_kv_heads, ffn_dim, max_seq;
    float rope_theta, rms_eps;
    uint32_t num_experts, num_experts_per_tok, moe_ffn_dim;
    uint8_t model_kind; /* 0 Decoder, 1 AsrEncoderDecoder, 2 Decision */
    uint8_t norm_kind;  /* 0 Rms, 1 Layer */
    uint16_t pad;
    /* AudioSpec (manifest.rs:166-194), in declaration order */
    uint32_t n_mels, n_audio_ctx, n_audio_state, n_audio_layer, n_audio_head;
    uint32_t n_text_ctx, n_text_state, n_text_layer, n_text_head;
    /* ManifestExt (manifest.rs:141-157) */
    float embed_scale, logit_softcap, attn_scale;
    uint32_t tied_lm_head;
    float yarn_factor;
    uint32_t yarn_orig_ctx;
    float yarn_beta_fast, yarn_beta_slow;
    /* KevSpec (manifest.rs:104-109); has_kev = 0 for classic decoders */
    uint32_t has_kev;
    float kev_temperature;
    uint32_t kev_pointer_dim;
    /* list lengths */
    uint32_t n_layer_specs, n_window, n_rope_theta, n_prefetch;
} soso_som_manifest;

/* TensorEntry (index.rs:13-23); the pointers live as long as the handle */
typedef struct {
    uint32_t id;
    const char *name;
    size_t name_len;
    const char *shard;
    size_t shard_len;
    uint64_t offset, byte_len;
    uint32_t ndim;
    const uint32_t *shape;
    uint8_t dtype, quant;
} soso_som_tensor;

/* TensorView (crates/soso-llm-core/src/layer.rs): bytes mapped from the shard */
typedef struct {
    const uint8_t *bytes;
    size_t len;
    uint8_t dtype;
    uint64_t elems;
} soso_som_view;

/* CRC-32C (Castagnoli, reflected 0x82F63B78, init and final xor 0xFFFFFFFF),
 * the checksum of every .som header (lib.rs:26-30, crc crate CRC_32_ISCSI). */
uint32_t soso_som_crc32c(const void *data, size_t len);
/* The same through the byte table alone (what runs where SSE4.2 is absent). */
uint32_t soso_som_crc32c_portable(const void *data, size_t len);

/* The message of the last failed call on this thread. */
const char *soso_som_error(void);

/* Opens <dir>/manifest.som and <dir>/index.som (both CRC-checked and fully
 * parsed); shards are mapped lazily from <dir>/shards. */
int soso_som_open(const char *dir, size_t dir_len, soso_som **out);

/* The same from bytes in memory; either record may be NULL (len 0) to parse
 * only the other.  Tensor views read shards from `shards_dir`. */
int soso_som_open_bytes(const uint8_t *manifest, size_t manifest_len, const uint8_t *index, size_t index_len,
                        const char *shards_dir, size_t shards_dir_len, soso_som **out);

void soso_som_close(soso_som *s);

/* verify_shard (index.rs:114-130): header, explicit payload length (v1 after
 * the 24-byte header, v2+ at offset 64) and CRC of the payload. */
int soso_som_verify_shard(const uint8_t *data, size_t len, size_t *payload_off, size_t *payload_len);

/* Manifest::parse (manifest.rs:1021-1190): ERR_NOTFOUND if the handle has no manifest */
int soso_som_manifest_get(const soso_som *s, soso_som_manifest *out);
/* which: 0 = name, 1 = chat_template */
int soso_som_manifest_str(const soso_som *s, int which, const char **str, size_t *len);
/* the v4 table, or the v1-v3 synthesized one (manifest.rs:533-546) */
int soso_som_layer_spec(const soso_som *s, uint32_t layer, soso_som_layer *out);
/* ManifestExt::window / rope_theta entry i (i < n_window / n_rope_theta) */
int soso_som_ext_window(const soso_som *s, uint32_t i, uint32_t *out);
int soso_som_ext_rope_theta(const soso_som *s, uint32_t i, float *out);
/* LayerPrefetch i: its layer and shard count; then shard j's name */
int soso_som_prefetch(const soso_som *s, uint32_t i, uint32_t *layer, uint32_t *n_shards);
int soso_som_prefetch_shard(const soso_som *s, uint32_t i, uint32_t j, const char **name, size_t *len);

/* TensorIndex (index.rs:33-96) */
size_t soso_som_tensor_count(const soso_som *s);
int soso_som_tensor_at(const soso_som *s, size_t i, soso_som_tensor *out);
int soso_som_find(const soso_som *s, const char *name, size_t name_len, size_t *i);

/* MmapTensorSource::tensor_view (source.rs:342-352): maps the tensor's shard
 * (CRC checked once per shard, source.rs:123-128) and returns its bytes; the
 * range [offset, offset + byte_len) must lie inside the shard's payload
 * (source.rs:166-185).  Names resolve like MmapTensorSource::buscar: on a
 * duplicated name the later entry wins (soso_som_find returns the first, as
 * TensorIndex::find does). */
int soso_som_tensor_view(soso_som *s, const char *name, size_t name_len, soso_som_view *out);

/* MmapTensorSource::load_f32 / load_f32_range (source.rs:275-340) for F32
 * tensors: copies elements [elem_off, elem_off + n).  load_f32 requires n to
 * be the tensor's element count (source.rs:277-279).  Quantized tensors are
 * ERR_DTYPE here: their bytes go to the GPU through tensor_view. */
int soso_som_load_f32(soso_som *s, const char *name, size_t name_len, float *out, size_t n);
int soso_som_load_f32_range(soso_som *s, const char *name, size_t name_len, size_t elem_off, float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
