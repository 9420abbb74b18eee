/*
 * soso_hip.h -- C ABI of the MI355X (gfx950) decode hot path for soso.
 *
 * Drop-in boundary for soso-llm-core's `GpuDispatch` trait
 * (crates/soso-llm-core/src/gpu.rs:338-737).  A thin Rust `impl GpuDispatch`
 * wraps these calls 1:1 (the binding is shown in INTEGRATION.md).  No torch or
 * HIP types cross this boundary: plain pointers, sizes and integer codes.
 *
 * Conventions, all taken from the trait and its CUDA implementor:
 *  - Return codes of the compute entry points mirror Result<bool, ()>:
 *      1  = computed (outputs valid on return)        -> Ok(true)
 *      0  = declined, the caller computes on the CPU  -> Ok(false)
 *     <0  = error; callers treat it like 0            -> Err(())
 *    (gpu.rs:432-440; try_gpu_matvec turns Err into CPU, gpu.rs:784-787).
 *  - Weights are resident and keyed by a stable tensor name: the first call
 *    for a key uploads `w` (and repacks it for the device); later calls read
 *    only the key.  A key that was declined once (dtype, shape, memory) stays
 *    declined (crates/soso-llm-api/src/cuda.rs:289-290, 2365-2380).
 *  - Host-pointer entry points are synchronous: outputs are valid on return
 *    (cuda.rs:2395-2408).  One caller at a time (the trait takes &mut self);
 *    a handle may be used from a thread other than its creator: the device is
 *    made current on every call (cuda.rs:2362-2364).
 *  - Nothing here aborts or throws.
 *
 * dtype codes are soso's (crates/sosomodel/src/layout.rs:8-12):
 *   1 = F32, 2 = Q8_0 (f32 scale + 32 x i8 = 36 B), 3 = Q4_K (GGML, 144 B),
 * plus 13 = Q6_K (GGML, 210 B), an extension of this library: soso itself
 * re-quantizes Q6_K to Q8_0 at import (crates/gguf2som/src/lib.rs:1592-1609).
 */
#ifndef SOSO_HIP_H
#define SOSO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SOSO_HIP_DTYPE_F32 1
#define SOSO_HIP_DTYPE_Q8_0 2
#define SOSO_HIP_DTYPE_Q4_K 3
#define SOSO_HIP_DTYPE_Q6_K 13

#define SOSO_HIP_OK 1
#define SOSO_HIP_DECLINED 0
#define SOSO_HIP_ERR (-1)
#define SOSO_HIP_ERR_ARG (-2)
#define SOSO_HIP_ERR_DEVICE (-3)
#define SOSO_HIP_ERR_NOMEM (-4)

typedef struct soso_hip soso_hip; /* opaque; one per device */

/* GpuStats (gpu.rs:18-36): the counters this library maintains. */
typedef struct soso_hip_stats {
    uint64_t launches;   /* entry-point calls that ran on the device */
    uint64_t total_ns;   /* wall time spent inside those calls */
    uint64_t bytes_up;   /* host -> device (activations, not weights) */
    uint64_t bytes_down; /* device -> host */
    uint64_t weight_bytes_resident;
    uint64_t weights_resident;
    uint64_t weights_declined;
    /* the per-token transfers of soso_hip_decode_token (GpuStats::decode_*,
     * gpu.rs:23-29): embedding rows up, control words up (none: the position
     * travels as a kernel argument), logits and KV rows down, steps */
    uint64_t decode_embed_up;
    uint64_t decode_control_up;
    uint64_t decode_logits_down;
    uint64_t decode_kv_down;
    uint64_t decode_steps;
} soso_hip_stats_t;

/* MatvecOp (gpu.rs:189-196) for soso_hip_matvec_batch. */
typedef struct soso_hip_op {
    const char *key;
    size_t key_len;
    const uint8_t *w; /* raw tensor bytes (read only on the key's first use) */
    size_t w_len;
    uint8_t dtype;
    size_t rows, cols;
    const float *x; /* cols */
    float *y;       /* rows */
} soso_hip_op;

/* ExpertoBloque (gpu.rs:176-186) for soso_hip_experts_block. */
typedef struct soso_hip_expert {
    const char *keys[3]; /* ffn_gate, ffn_up, ffn_down */
    size_t key_lens[3];
    const uint8_t *w[3]; /* raw bytes, or NULL when the caller believes them resident */
    size_t w_len[3];
    uint8_t dtype[3]; /* 0 when w is NULL */
    const uint32_t *tokens;  /* block-local token indices choosing this expert */
    const uint32_t *targets; /* token * top_k + rank, one per token */
    size_t n_tokens;
    int shared; /* 1 = shared expert */
} soso_hip_expert;

/* ---- lifetime ------------------------------------------------------------ */
/* Creates a handle on HIP device `device`.  vram_budget = bytes of weights the
 * handle may keep resident (0 = 90% of the device's free memory).
 * Returns 0 or a negative error. */
int soso_hip_create(int device, uint64_t vram_budget, soso_hip **out);
void soso_hip_destroy(soso_hip *h);

/* GpuDispatch::available (gpu.rs:339). */
int soso_hip_available(const soso_hip *h);
/* GpuDispatch::dtype_soportado (gpu.rs:343-345): 1 for F32, Q8_0, Q4_K, Q6_K. */
int soso_hip_dtype_supported(const soso_hip *h, uint8_t dtype);
/* GpuDispatch::stats (gpu.rs:352-354). */
void soso_hip_stats(const soso_hip *h, soso_hip_stats_t *out);
/* Last error message of this handle ("" if none); valid until the next call. */
const char *soso_hip_last_error(const soso_hip *h);

/* ---- matvec family (host pointers, synchronous) ---------------------------- */
/* GpuDispatch::matvec (gpu.rs:432-440): y[rows] = W[rows x cols] . x[cols].
 * Overwrites y.  w/w_len are read only on the first call for `key`. */
int soso_hip_matvec(soso_hip *h, const char *key, size_t key_len, const uint8_t *w, size_t w_len,
                    uint8_t dtype, size_t rows, size_t cols, const float *x, float *y);
/* GpuDispatch::matmul (gpu.rs:443-455): Y[n x rows] = X[n x cols] . W^T. */
int soso_hip_matmul(soso_hip *h, const char *key, size_t key_len, const uint8_t *w, size_t w_len,
                    uint8_t dtype, size_t rows, size_t cols, size_t n, const float *x, float *y);
/* GpuDispatch::matvec_lote (gpu.rs:694-701): every op with one wait at the
 * end; done[i] = 1 for the ops computed here.  Returns 1 if all were done,
 * 0 if some were declined, <0 on error (done[] still tells which finished). */
int soso_hip_matvec_batch(soso_hip *h, const soso_hip_op *ops, size_t n_ops, uint8_t *done);

/* ---- MoE ---------------------------------------------------------------------- */
/* GpuDispatch::router_topk (gpu.rs:480-494): logits = W[n_exp x h] . x (f32),
 * softmax, top-k per token in ranking order (ties: lowest index), weights
 * renormalised.  idx/wgt: n x top_k. */
int soso_hip_router_topk(soso_hip *h, const char *key, size_t key_len, const float *w, const float *xs,
                         size_t n, size_t hdim, size_t n_exp, size_t top_k, int32_t *idx, float *wgt);
/* GpuDispatch::expertos_bloque (gpu.rs:461-475): per expert, gate/up, SwiGLU
 * and down for the tokens choosing it; sum[n x h] receives, per token, the
 * weighted sum (weights wgt[n x top_k]) of the experts resolved here in
 * ranking order.  done[i] = 1 for the experts resolved.  Returns 1 if all were
 * resolved, 0 if some were declined (their contribution is not in sum).  A
 * shared expert computed by soso_hip_moe_shared for the same n and hdim is
 * added to sum after the ranked experts (and consumed); one computed for
 * another block makes the call fail (< 0). */
int soso_hip_experts_block(soso_hip *h, const float *xs, size_t n, size_t hdim, size_t ffn, size_t top_k,
                           const float *wgt, const soso_hip_expert *exps, size_t n_exps, float *sum,
                           uint8_t *done);
/* GpuDispatch::moe_compartido (gpu.rs:518-534): the shared expert of an MoE
 * block of n tokens (xs [n x hdim]), c_t = down(silu(gate x_t) * up x_t) *
 * sigmoid(x_t . pg_w) (soso's CPU path, bloque35.rs:950-1005), computed and
 * kept on the device for the next soso_hip_experts_block call with the same n
 * and hdim, which adds it to its sum.  keys / key_lens / w / w_len / dtype:
 * gate [ffn x hdim], up [ffn x hdim], down [hdim x ffn] (quantized; uploaded
 * on first use under their keys, as soso_hip_expert's); pg_w: the
 * ffn_gate_inp_shexp row, hdim f32.  1 = computed, 0 = declined, < 0 error. */
int soso_hip_moe_shared(soso_hip *h, const char *const *keys, const size_t *key_lens, const uint8_t *const *w,
                        const size_t *w_len, const uint8_t *dtype, const float *pg_w, const float *xs, size_t n,
                        size_t hdim, size_t ffn);

/* ---- MoE FFN resident on the device --------------------------------------------
 * The FFN half of GpuDispatch::moe_capa (gpu.rs; CudaGpu::moe_ejecutar,
 * crates/soso-llm-api/src/cuda/capa/moe.rs:316): router logits, softmax and
 * top-k, the chosen experts' gate/up + SwiGLU and down, and the weighted sum
 * in ranking order, all on the device with no host round trip.
 * register: router_key names a resident F32 weight [n_exp x hdim];
 * expert_keys holds 3*n_exp resident keys (gate_e, up_e, down_e for e = 0..):
 * gate/up [ffn x hdim], down [hdim x ffn], one quantized dtype per role.
 * Limits: n_exp <= 256, top_k <= 64.  Registering a key again replaces it.
 * For Q4_K experts the layer also keeps a tile-major copy of every expert
 * matrix (the same bytes again, counted in the handle's budget) that the
 * matrix-core path reads when a call routes two or more tokens per active
 * expert; it is skipped, and that path reads the resident weights, when the
 * budget has no room.  Dropping any of the layer's weights unregisters it and
 * frees the copy.
 * expert_keys = NULL registers the router alone: a layer whose experts stay
 * on the host (soso's layers whose experts are not on the card, computed by
 * decode_token's cpu_moe callback).  Such a layer serves as an FFN of
 * soso_hip_decode_create_moe models run through soso_hip_decode_token; the
 * MoE FFN entry points decline it. */
int soso_hip_moe_register(soso_hip *h, const char *layer_key, size_t layer_key_len, const char *router_key,
                          size_t router_key_len, const char *const *expert_keys, const size_t *expert_key_lens,
                          size_t n_exp, size_t hdim, size_t ffn, size_t top_k);
/* out_dev[n x hdim] = sum_j wgt[t,j] * down_e(silu(gate_e . x_t) * (up_e . x_t)),
 * e = idx[t,j], j in ranking order (residual not added, layer.rs:1389 adds it).
 * idx_dev / wgt_dev (n x top_k) receive the routing when non-null.
 * Asynchronous on the handle's stream. */
int soso_hip_moe_ffn_dev(soso_hip *h, const char *layer_key, size_t layer_key_len, const float *x_dev, size_t n,
                         float *out_dev, int32_t *idx_dev, float *wgt_dev);

/* No counterpart in the reference: soso_hip_moe_ffn_dev for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as soso_hip_moe_ffn_dev (the
 * same kernels), but its scratch (router logits, routing, slot lists, work
 * items, activations) is a fixed array of SOSO_HIP_MOE_NOALLOC_SCRATCH_BYTES
 * that the library holds on every GPU it runs on until the process ends; the
 * call allocates and frees nothing.  A call whose scratch (about
 * n * top_k * (ffn + hdim) * 4 bytes plus the routing lists) exceeds the
 * array returns SOSO_HIP_ERR_ARG.  Every call on a GPU shares that GPU's
 * array, so calls that overlap on one GPU (two streams, two handles) race;
 * calls in order on one stream do not.  Nothing in the array needs to start
 * at zero: each call writes every region before it reads it.  Asynchronous
 * on the handle's stream. */
#define SOSO_HIP_MOE_NOALLOC_SCRATCH_BYTES (8u << 20)
int soso_hip_moe_ffn_dev_noalloc(soso_hip *h, const char *layer_key, size_t layer_key_len, const float *x_dev,
                                 size_t n, float *out_dev, int32_t *idx_dev, float *wgt_dev);

/* ---- Gated DeltaNet (Qwen3.5's linear-attention layers) -------------------------
 * GpuDispatch::gdn_bloque (gpu.rs:577-599): the recurrence of a GDN layer for
 * a block of n tokens, on host buffers, synchronous.  With C = (2 n_k + n_v) d:
 *   hist  [(kernel - 1 + n) x C]  the conv state (oldest row first), then the
 *                                 n tokens' qkv projections
 *   conv  [C x kernel]            ssm_conv1d weights
 *   z     [n x n_v d]             attn_gate projections
 *   decay [n x n_v]               exp(softplus(alpha + ssm_dt) * ssm_a)
 *   beta  [n x n_v]               sigmoid(ssm_beta projection)
 *   norm  [d]                     ssm_norm
 *   state [n_v x d x d]           in and out (value head vh: row i, column j)
 *   out   [n x n_v d]             the gated, normalised heads (ssm_out's input)
 * Per token: causal conv + SiLU, q and k heads l2-normalised (q also scaled
 * by 1 / sqrt(d)), per value head vh (q/k head vh mod n_k) delta = beta (v -
 * decay S^T k), S <- decay S + k delta^T, o = S^T q, rmsnorm(o) * norm * silu(z)
 * (bloque35.rs:372-465).  The conv state after the block is the last
 * kernel - 1 rows of hist (the caller's, as in soso).  d must be 128 and
 * kernel 1..16 (others decline); eps is the model's rms_eps. */
int soso_hip_gdn_block(soso_hip *h, const float *hist, const float *conv, const float *z, const float *decay,
                       const float *beta, const float *norm, float *state, float *out, size_t n, size_t n_k,
                       size_t n_v, size_t d, size_t kernel, float eps);
/* The same with every buffer in device memory, queued on the library's
 * stream (no synchronisation; capturable in a HIP graph once its scratch of
 * n * C floats has been grown by an earlier call). */
int soso_hip_gdn_block_dev(soso_hip *h, const float *hist, const float *conv, const float *z, const float *decay,
                           const float *beta, const float *norm, float *state, float *out, size_t n, size_t n_k,
                           size_t n_v, size_t d, size_t kernel, float eps);

/* ---- dense decode step resident on the device -----------------------------------
 * The device-resident decode of GpuDispatch::decode_preparar / decode_token
 * (gpu.rs:653-690) for a Llama-style dense model (LayerExecutor::forward_layer,
 * crates/soso-llm-core/src/layer.rs:1092-1389, then Runtime::logits_gpu and
 * argmax, runtime.rs:1976-2028).
 * keys: 9 per layer -- attn_norm, q, k, v, o, ffn_norm, gate, up, down -- then
 * output_norm and head (9 * n_layers + 2 resident weights).  Norms are F32
 * [1 x hidden]; q [n_heads*head_dim x hidden], k and v [n_kv_heads*head_dim x
 * hidden], o [hidden x n_heads*head_dim], gate and up [ffn x hidden], down
 * [hidden x ffn], head [vocab x hidden].  q/k/v share one quantized dtype, gate/up
 * another; head_dim must be 128 and n_heads a multiple (1, 2, 4 or 8) of
 * n_kv_heads.  The library keeps fused copies (q|k|v rows; gate/up rows
 * interleaved) and allocates the KV cache (2 x n_layers x ctx_max x kv_dim
 * elements, zeroed) and the step's buffers; drop_sources = 1 drops the q, k, v,
 * gate and up weights once fused.  RoPE is non-NeoX (pairs 2i, 2i+1) with
 * rope_theta.
 * kv_f16 = 0: the KV cache holds f32.  kv_f16 = 1: it holds
 * IEEE half bits, as soso's KvCache does (KvDtype::F16, kv.rs:258-266, the only
 * KV type soso's device decode accepts, runtime/decode_gpu.rs:63): new rows are
 * rounded with soso's f32_to_f16 (f16.rs:10-36: nearest, ties away from zero,
 * NaN -> 0x7e00 | sign) and attention widens them to f32 exactly. */
typedef struct soso_hip_decode_cfg {
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, ctx_max;
    float rope_theta, rms_eps;
    uint32_t kv_f16;
} soso_hip_decode_cfg;
int soso_hip_decode_create(soso_hip *h, const char *model_key, size_t model_key_len, const soso_hip_decode_cfg *cfg,
                           const char *const *keys, const size_t *key_lens, int drop_sources);
/* The same step with MoE layers (GpuDispatch::moe_capa for one token,
 * crates/soso-llm-core/src/gpu.rs; the GQA-MoE layer that capa_moe_en_gpu,
 * crates/soso-llm-core/src/moe_gpu.rs:37, runs on the device): layer l's FFN
 * is the registered MoE layer moe_layer_keys[l] (soso_hip_moe_register, width
 * hidden) when that entry is non-null -- forward_moe_ffn, layer.rs:1938-1975:
 * x = rmsnorm(h) * ffn_norm, router + top-k, the chosen experts' gate/up +
 * SwiGLU and down, h += their ranking-order sum -- and the dense FFN of
 * soso_hip_decode_create otherwise.  The keys array keeps its 9 entries per
 * layer; an MoE layer's gate, up and down entries are ignored (may be null
 * with length 0).  Attention is the dense step's (non-NeoX RoPE, no QK norm;
 * soso_hip_decode_create_ex takes those).
 * MoE layers take the single-token expert path: gate/up Q4_K, Q8_0 or Q6_K
 * with hidden a multiple of 128 up to 4096, down Q4_K with an expert width of
 * 256 to 2048 (a multiple of 256), top_k <= 8; others are declined here.
 * Re-registering or unregistering an MoE layer the model reads destroys the
 * model. */
int soso_hip_decode_create_moe(soso_hip *h, const char *model_key, size_t model_key_len,
                               const soso_hip_decode_cfg *cfg, const char *const *keys, const size_t *key_lens,
                               const char *const *moe_layer_keys, const size_t *moe_layer_key_lens, int drop_sources);
/* The step for the Qwen-style attention variants soso's forward_layer takes
 * (layer.rs:1164-1192, its FLAG_QK_NORM and FLAG_ROPE_NEOX): flags
 * SOSO_HIP_DECODE_QK_NORM -- q and k are RMS-normalised per head before RoPE
 * with the layer's attn_q_norm / attn_k_norm weights (F32 [head_dim]), given
 * as two more keys per layer (11 per layer: the 9 of soso_hip_decode_create,
 * then q_norm, k_norm; then output_norm and head); SOSO_HIP_DECODE_ROPE_NEOX
 * -- RoPE turns the pairs (i, i + head_dim/2) (rope_cabezas with neox,
 * gemm.rs:1474-1479) instead of (2i, 2i + 1).  moe_layer_keys as in
 * soso_hip_decode_create_moe (null for a dense model).  The attention kernel
 * finishes the q/k/v rows either way, so the flags add no launch.  flags 0
 * is soso_hip_decode_create(_moe). */
#define SOSO_HIP_DECODE_QK_NORM 1u
#define SOSO_HIP_DECODE_ROPE_NEOX 2u
int soso_hip_decode_create_ex(soso_hip *h, const char *model_key, size_t model_key_len,
                              const soso_hip_decode_cfg *cfg, uint32_t flags, const char *const *keys,
                              const size_t *key_lens, const char *const *moe_layer_keys,
                              const size_t *moe_layer_key_lens, int drop_sources);
/* Device pointers of MoE layer `layer`'s routing in the last step: top_k
 * expert indices (int32) and weights (f32), in ranking order. */
int soso_hip_decode_moe_routing_dev(soso_hip *h, const char *model_key, size_t model_key_len, uint32_t layer,
                                    int32_t **idx_dev, float **wgt_dev);
/* Device pointers of layer `layer`'s K and V caches, head-major:
 * [n_kv_heads][ctx_max][head_dim] (a head's positions are contiguous), each
 * element f32 or f16 bits as kv_f16 says, for prefilling and inspection. */
int soso_hip_decode_kv_dev(soso_hip *h, const char *model_key, size_t model_key_len, uint32_t layer, void **k_dev,
                           void **v_dev);
/* decode_subir_estado (gpu.rs:665, EstadoCapaDec.k / .v, gpu.rs:167-173): writes
 * n_rows position-major rows [n_rows][kv_dim] of K and V into layer `layer`'s
 * cache at positions row0 .. row0 + n_rows - 1 (scattered to the head-major
 * layout).  rows_f32 = 1: the rows are f32 and an f16 cache receives them rounded
 * as KvCache::append does (kv.rs:264-266); rows_f32 = 0: they already hold the
 * cache's element type (f16 bits for soso's host KV).  k_rows / v_rows may be host
 * or device pointers.  Synchronous. */
int soso_hip_decode_kv_upload(soso_hip *h, const char *model_key, size_t model_key_len, uint32_t layer, uint32_t row0,
                              uint32_t n_rows, const void *k_rows, const void *v_rows, int rows_f32);
/* One token at position `pos` (KV rows 0..pos-1 already filled): hidden = x_dev
 * (the token's f32 embedding row); writes K/V row `pos` of every layer, the
 * logits (logits_dev, vocab f32, when non-null) and the greedy token
 * (*token_dev, last maximum wins).  kv_rows_dev, when non-null, also receives
 * the new rows in decode_token's `kv_rows` layout (gpu.rs:670-672): per layer,
 * k (kv_dim) then v (kv_dim), in the cache's element type.  Asynchronous;
 * allocates nothing, so it may be captured in a graph. */
int soso_hip_decode_step_dev(soso_hip *h, const char *model_key, size_t model_key_len, const float *x_dev, uint32_t pos,
                             float *logits_dev, uint32_t *token_dev, void *kv_rows_dev);
/* cpu_moe of decode_token (gpu.rs:674-679): for MoE layer `layer` whose
 * experts stay on the host, out[hidden] = the ranking-order weighted sum of
 * the chosen experts' SwiGLU FFNs of xn[hidden] (= rmsnorm(h) * ffn_norm),
 * experts idx[top_k] with weights wgt[top_k] as the device routed them.
 * Returns 0, or nonzero on failure. */
typedef int (*soso_hip_cpu_moe_fn)(void *ctx, uint32_t layer, const float *xn, const int32_t *idx, const float *wgt,
                                   size_t top_k, float *out);
/* GpuDispatch::decode_token (gpu.rs:670-685) on host buffers: embed (hidden
 * f32) up, one step at `pos`, then logits (vocab f32, when non-null), the new
 * KV rows (soso_hip_decode_step_dev's kv_rows layout, when non-null) and the
 * greedy token (when non-null) down; synchronous.  A layer whose FFN was
 * registered without experts stops the step after its routing: xn and the
 * routing go down, cpu_moe(cpu_moe_ctx, ...) computes the FFN, its output
 * comes up and is added to the hidden state, and the step goes on.  Models
 * with such layers run only here (soso_hip_decode_step_dev declines them), and
 * need cpu_moe.  Counts the transfers in the decode_* stats. */
int soso_hip_decode_token(soso_hip *h, const char *model_key, size_t model_key_len, const float *embed, uint32_t pos,
                          soso_hip_cpu_moe_fn cpu_moe, void *cpu_moe_ctx, float *logits, void *kv_rows,
                          uint32_t *token);
int soso_hip_decode_destroy(soso_hip *h, const char *model_key, size_t model_key_len);

/* ---- one GQA-MoE layer at a time: GpuDispatch::moe_capa -----------------------
 * The layer that capa_moe_en_gpu (crates/soso-llm-core/src/moe_gpu.rs:37-269)
 * hands to GpuDispatch::moe_capa (gpu.rs:426; MoeCapa, gpu.rs:294-335):
 * forward_layer of one Qwen3-MoE-style layer (layer.rs:1092-1389, 1938-1975)
 * -- attention with attn_norm, q/k/v, QK norm (qk_norm), NeoX RoPE and the f16
 * KV cache the device keeps for the layer, o with the residual, then ffn_norm,
 * router + top-k and the chosen experts' SwiGLU FFNs summed in ranking order,
 * with the residual -- for n tokens at positions pos0 .. pos0 + n - 1, taken
 * one after another (each sees the positions before it).
 * Fields follow MoeCapa: hidden_dim is MoeCapa::h; the q/k/v/o keys and
 * prefix are NUL-terminated; the experts are the resident weights
 * "{prefix}.E{ee}.ffn_gate" / "_up" / "_down" (ee two or more digits, as
 * soso names them); attn_norm, q_norm, k_norm (with qk_norm), ffn_norm
 * (hidden_dim floats, head_dim for the QK norms) and router (n_exp x
 * hidden_dim f32) are MoeNormas, needed on a layer's first call and ignored
 * once the layer is ready (soso_hip_moe_capa_ready).  escala must be
 * 1 / sqrt(head_dim).  Declined (0, the CPU keeps the layer): sliding windows
 * (ventana > 0), YaRN (rope_factors or rope_mscale != 1), shapes the decode
 * step does not run (head_dim 128, GQA groups 1/2/4/8, the single-token MoE
 * path's limits), pos0 beyond the positions this layer's device KV holds
 * (the earlier ones were computed elsewhere), pos0 + n > ctx_max.
 * continuar: the input is the pending output of layer - 1 for the same
 * tokens (soso_hip_moe_capa_pending), not `hidden`.  encadenar: the output
 * stays pending on the device and `hidden` is left as it is (no download, no
 * wait); otherwise it is written to `hidden` (n x hidden_dim) on return.
 * Returns 1 done, 0 declined, < 0 error. */
typedef struct soso_hip_moe_capa {
    uint32_t layer;
    size_t pos0, n;
    size_t hidden_dim, heads, kv_heads, head_dim, ffn, n_exp, top_k, ventana, ctx_max;
    float eps, theta, escala, rope_mscale;
    int qk_norm, continuar, encadenar;
    const char *key_q, *key_k, *key_v, *key_o, *prefix;
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm, *router, *rope_factors;
} soso_hip_moe_capa;
int soso_hip_moe_capa_run(soso_hip *h, const soso_hip_moe_capa *capa, float *hidden);
/* moe_puede (gpu.rs:380): 0 once the layer was discarded, else 1. */
int soso_hip_moe_capa_can(const soso_hip *h, uint32_t layer);
/* moe_lista (gpu.rs:386): 1 when the layer's norms, router and device step exist. */
int soso_hip_moe_capa_ready(const soso_hip *h, uint32_t layer);
/* moe_pendiente (gpu.rs:392): 1 when the output of `layer` for n tokens from
 * pos0 is pending on the device. */
int soso_hip_moe_capa_pending(const soso_hip *h, uint32_t layer, size_t pos0, size_t n);
/* moe_volcar (gpu.rs:398): writes the pending output (n x hidden_dim) to
 * hidden and clears it; nothing when none is pending.  Synchronous. */
int soso_hip_moe_capa_flush(soso_hip *h, float *hidden);
/* moe_descartar (gpu.rs:421): the layer is not tried again; its device step
 * and KV cache are freed. */
void soso_hip_moe_capa_discard(soso_hip *h, uint32_t layer);
/* Device pointers of the layer's K and V caches (head-major
 * [kv_heads][ctx_max][head_dim] f16 bits), for inspection. */
int soso_hip_moe_capa_kv_dev(soso_hip *h, uint32_t layer, void **k_dev, void **v_dev);
/* The layer's routing of the last token it computed: top_k int32 expert
 * indices in ranking order and their f32 weights (device pointers), for
 * inspection. */
int soso_hip_moe_capa_routing_dev(soso_hip *h, uint32_t layer, int32_t **idx_dev, float **wgt_dev);
/* gemma_subir / gemma_residente (gpu.rs:362-370), which soso uses to make a
 * moe_capa layer's attention and expert weights resident: upload makes `key`
 * resident from its raw bytes (1, 0 declined, < 0 error; a resident key is
 * kept as it is), resident says whether it is. */
int soso_hip_weight_upload(soso_hip *h, const char *key, size_t key_len, const uint8_t *w, size_t w_len,
                           uint8_t dtype, size_t rows, size_t cols);
int soso_hip_weight_resident(const soso_hip *h, const char *key, size_t key_len);

/* ---- device-resident API (no host copies; for the decode step, benchmarks
 * and tests that keep inputs in HBM).  Launches are asynchronous on the
 * handle's stream; soso_hip_sync waits. -------------------------------------- */
int soso_hip_dev_alloc(soso_hip *h, size_t bytes, void **dptr);
int soso_hip_dev_free(soso_hip *h, void *dptr);
int soso_hip_h2d(soso_hip *h, void *dst, const void *src, size_t bytes);
int soso_hip_d2h(soso_hip *h, void *dst, const void *src, size_t bytes);
int soso_hip_sync(soso_hip *h);
/* Device-to-device copy on the handle's stream (asynchronous). */
int soso_hip_d2d(soso_hip *h, void *dst, const void *src, size_t bytes);
/* Registers a resident weight whose raw (soso/GGML layout) bytes are already
 * on the device at `raw_dev`; the library repacks them into its own copy. */
int soso_hip_weight_from_dev(soso_hip *h, const char *key, size_t key_len, const void *raw_dev,
                             size_t w_len, uint8_t dtype, size_t rows, size_t cols);
int soso_hip_weight_drop(soso_hip *h, const char *key, size_t key_len);
/* y_dev[rows] = W(key) . x_dev; asynchronous on the handle's stream. */
int soso_hip_matvec_dev(soso_hip *h, const char *key, size_t key_len, const float *x_dev, float *y_dev);
/* Y[n x rows] = X[n x cols] . W(key)^T, device pointers, asynchronous. */
int soso_hip_matmul_dev(soso_hip *h, const char *key, size_t key_len, size_t n, const float *x_dev,
                        float *y_dev);
/* Exact dequantization of a resident weight into out_dev (rows*cols f32),
 * with the reference's arithmetic (no FMA): the bit-exactness witness. */
int soso_hip_dequant_dev(soso_hip *h, const char *key, size_t key_len, float *out_dev);
/* argmax over n values (last maximum wins, as Runtime::argmax,
 * crates/soso-llm-core/src/runtime.rs:2021-2028); result in *idx_dev. */
int soso_hip_argmax_dev(soso_hip *h, const float *x_dev, size_t n, uint32_t *idx_dev);

/* ---- timing on the handle's stream ------------------------------------------- */
int soso_hip_timer_start(soso_hip *h);
/* Milliseconds since the matching start, measured with HIP events. */
int soso_hip_timer_stop(soso_hip *h, float *ms);
/* Per-launch timing: records HIP event `slot` (0..65535) on the handle's
 * stream; elapsed waits for slot_b and returns ms between the two events. */
int soso_hip_event_record(soso_hip *h, int slot);
int soso_hip_event_elapsed(soso_hip *h, int slot_a, int slot_b, float *ms);

/* ---- HIP graphs of device-resident work ------------------------------------------
 * begin/end capture every launch (and event record) the handle issues between
 * them into one graph; launch replays it on the handle's stream.  Only the
 * *_dev entry points, event records and the decode step may be captured
 * (they neither allocate nor synchronize). */
int soso_hip_graph_begin(soso_hip *h);
int soso_hip_graph_end(soso_hip *h, int *graph_id);
int soso_hip_graph_launch(soso_hip *h, int graph_id);
int soso_hip_graph_destroy(soso_hip *h, int graph_id);

#ifdef __cplusplus
}
#endif
#endif
