// internal.hpp -- shared host structures and device helpers of libsoso_hip.
//
// Device code targets gfx950 (CDNA4, wave64) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/soso_hip.h"
#include "../../include/soso_hip_bench.h"

// ---------------------------------------------------------------------------
// Formats (crates/sosomodel/src/layout.rs:57-64; Q6_K from GGML via
// crates/gguf2som/src/lib.rs:1639-1661)
// ---------------------------------------------------------------------------
constexpr int Q8_0_ELEMS = 32, Q8_0_BYTES = 36;
constexpr int Q4_K_ELEMS = 256, Q4_K_BYTES = 144;
constexpr int Q6_K_ELEMS = 256, Q6_K_BYTES = 210;

// Every quantized kernel works on "units" of 64 consecutive-in-layout
// elements owned by one lane; a row of `cols` elements has cols/64 units.
constexpr int UNIT = 64;

// Bytes per row in soso's layout, or 0 when the shape is not representable
// (crates/sosomodel/src/dequant.rs:53-68).
inline size_t fmt_row_bytes(uint8_t dtype, size_t cols)
{
    switch (dtype) {
    case SOSO_HIP_DTYPE_F32: return cols * 4;
    case SOSO_HIP_DTYPE_Q8_0: return cols % 32 ? 0 : cols / 32 * Q8_0_BYTES;
    case SOSO_HIP_DTYPE_Q4_K: return cols % 256 ? 0 : cols / 256 * Q4_K_BYTES;
    case SOSO_HIP_DTYPE_Q6_K: return cols % 256 ? 0 : cols / 256 * Q6_K_BYTES;
    default: return 0;
    }
}

// ---------------------------------------------------------------------------
// Host-side state
// ---------------------------------------------------------------------------
struct Weight {
    void *dev = nullptr; // device copy in this library's layout
    size_t bytes = 0;
    uint8_t dtype = 0;
    size_t rows = 0, cols = 0;
    // columns of the packed copy the kernels walk when they differ from cols:
    // Q8_0 rows of an odd number of 32-element blocks get a zero block (scale
    // 0, codes 0) so that 64-element units tile them; 0 = cols
    size_t kcols = 0;
    bool declined = false;
};
inline size_t weight_kcols(const Weight &w) { return w.kcols ? w.kcols : w.cols; }

// A MoE FFN registered for the device-resident path (soso_hip_moe_register).
struct MoeLayer {
    const Weight *router = nullptr; // f32 [n_exp x hdim]
    size_t n_exp = 0, hdim = 0, ffn = 0, top_k = 0;
    uint8_t dt_gu = 0, dt_down = 0;
    const uint8_t **tab = nullptr; // device: gate[n_exp], up[n_exp], down[n_exp]
    std::vector<const void *> host_tab; // the same pointers, for unregistering on weight_drop
    // tile-major copies of the Q4_K experts for the matrix-core path (k_mfma.hip),
    // laid out like `tab`; tiled_gu / tiled_down say which roles have them
    const uint8_t **tiled = nullptr;
    void *tiled_mem = nullptr;
    size_t tiled_bytes = 0;
    bool tiled_gu = false, tiled_down = false;
};

// A dense decode model registered for the device-resident step (k_decode.hip).
// (k_moe.hip) -- device scratch of one MoE FFN call
struct MoeScratch {
    float *logits = nullptr; // n x n_exp
    int32_t *idx = nullptr;  // n x top_k
    float *wgt = nullptr;    // n x top_k
    int *cnt = nullptr, *offs = nullptr, *list = nullptr; // n_groups, n_groups + 1, n x top_k
    int *items = nullptr, *n_items = nullptr; // work items {group, count, first slot, chunk | chunks << 16}, count
    int *recs = nullptr, *n_recs = nullptr;   // active groups {group, count, first slot, 0} (ascending), count
    float *act = nullptr;    // n x top_k x ffn
    float *ydown = nullptr;  // n x top_k x hdim
};

struct DecodeLayer {
    const Weight *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;
    const float *attn_norm = nullptr, *ffn_norm = nullptr;
    const float *q_norm = nullptr, *k_norm = nullptr; // QK norm weights (head_dim), or null
    // a registered MoE layer as the FFN (instead of gu / down), its scratch
    // (carved from the model's buffer; idx / wgt per layer: the last step's routing)
    const MoeLayer *moe = nullptr;
    MoeScratch moe_s;
    // the down projection runs as MV_SEG column segments (EPI_PARTS) into the
    // model's dpart, summed into h by the next launch that stages h (the next
    // layer's q/k/v or the head, XS_RMSNORM_P4)
    bool down_parts = false;
};
struct DecodeModel {
    size_t n_layers = 0, hidden = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, ffn = 0, vocab = 0, ctx_max = 0;
    float theta = 0.0f, eps = 0.0f;
    std::vector<DecodeLayer> layers;
    std::vector<Weight> owned; // the fused qkv / gate-up copies
    const float *out_norm = nullptr;
    const Weight *head = nullptr;
    std::vector<std::string> uses;     // keys of the resident weights the model reads
    std::vector<std::string> moe_uses; // keys of the registered MoE layers it reads
    bool kv_f16 = false;                        // KV elements: f16 bits (soso's KvDtype::F16) or f32
    void *kcache = nullptr, *vcache = nullptr;  // [n_layers][n_kv_heads][ctx_max][head_dim]
    void *mem = nullptr;                         // activations below, one allocation
    float *hid = nullptr, *att = nullptr, *act = nullptr, *part = nullptr, *logits = nullptr;
    float *hid2 = nullptr;  // h summed from a segmented down projection (hidden floats)
    float *dpart = nullptr; // the segmented down projection's partials (MV_SEG x hidden floats)
    float *rope_freq = nullptr; // head_dim / 2 floats
    float *xn = nullptr;        // the MoE layers' normalized x (hidden floats)
    void *moe_mem = nullptr;    // the MoE layers' scratch and routing
    size_t n_host_moe = 0;      // MoE layers whose experts stay on the host (router only)
    // the step's q/k/v rows as the qkv matvec leaves them; the attention
    // normalises them per head (SOSO_HIP_DECODE_QK_NORM), rotates them (NeoX
    // pairs with SOSO_HIP_DECODE_ROPE_NEOX) and appends k and v to the cache
    bool qk_norm = false, rope_neox = false;
    float *qkv_raw = nullptr; // q_dim + 2 kv_dim floats
};

// decode_token's cpu_moe: what the step calls for a layer whose experts stay
// on the host (soso_hip_decode_token)
struct HostMoe {
    soso_hip_cpu_moe_fn fn = nullptr;
    void *ctx = nullptr;
};

constexpr size_t SOSO_TICKET_BYTES = 16384;
// (token, rank) slots one route launch sorts in LDS; larger MoE calls run in
// blocks of at most MOE_ROUTE_MAX_SLOTS / top_k tokens (a token's routing and
// expert work do not depend on the other tokens of the call)
constexpr int MOE_ROUTE_MAX_SLOTS = 4096;
inline size_t moe_block_tokens(size_t top_k) { return top_k ? (size_t)MOE_ROUTE_MAX_SLOTS / top_k : 1; }

struct soso_hip {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    uint64_t budget = 0, used = 0;
    int num_cu = 256;
    size_t max_lds = 65536;
    std::unordered_map<std::string, Weight> weights;
    std::unordered_map<std::string, void *> f32_tensors; // router weights etc.
    soso_hip_stats_t stats{};
    std::string err;
    // reusable device scratch, grown on demand (scratch_get).  A graph keeps
    // the scratch pointers it was captured with, so a slot outgrown while any
    // graph exists is retired, not freed: retired buffers are freed once no
    // graph is left (graph_destroy) or with the handle.
    static constexpr int N_SCRATCH = 17;
    void *scratch[N_SCRATCH] = {};
    size_t scratch_cap[N_SCRATCH] = {};
    std::vector<void *> retired;
    // pinned host staging (pinned_get)
    void *pinned = nullptr;
    size_t pinned_cap = 0;
    // SOSO_TICKET_BYTES of "last workgroup" state, zero between launches (each
    // kernel resets what it used): uint 0 the final counter (argmax, MoE
    // route), uints 64 .. 831 argmax partials (winner, index, holds-NaN flag per segment), uints 2048 .. 3071 the MoE
    // route's per-token-block counters
    unsigned *ticket = nullptr;
    // device address of this GPU's fixed scratch array (runtime.hip), the
    // scratch of soso_hip_moe_ffn_dev_noalloc; looked up once, at create
    void *fixed_scratch = nullptr;
    std::unordered_map<std::string, MoeLayer> moe_layers;
    std::unordered_map<std::string, DecodeModel> decode_models;
    // soso_hip_moe_capa: per layer, its one-layer device step ("moe_capa.L<l>"
    // in decode_models), the MoE layer it registered and the library's own
    // keys (norms, router); the positions its KV cache holds; discarded layers;
    // the pending output of the last chained call (encadenar)
    struct MoeCapaLayer {
        std::string model, moe_key;
        std::vector<std::string> own_keys;
        size_t kv_pos = 0;
        float theta = 0.0f, eps = 0.0f;
        int qk_norm = 0;
    };
    std::unordered_map<uint32_t, MoeCapaLayer> moe_capas;
    std::vector<uint32_t> moe_capa_discarded;
    struct {
        bool valid = false;
        uint32_t layer = 0;
        size_t pos0 = 0, n = 0, width = 0;
        const float *dev = nullptr; // n x width floats
    } moe_pend;
    // soso_hip_moe_shared's output (n x hdim f32 in scratch slot 12), waiting
    // for the next soso_hip_experts_block call, which adds it to its sum
    bool shared_pending = false;
    size_t shared_n = 0, shared_hdim = 0;
    std::vector<hipEvent_t> events; // per-launch timing slots
    std::vector<hipGraphExec_t> graphs;
    bool capturing = false;
};

// error helpers (defined in runtime.hip)
int set_err(soso_hip *h, int code, const std::string &msg);
int hip_check(soso_hip *h, hipError_t e, const char *what);
// Release-path calls (frees, destroys and the waits before them): a failure
// leaves nothing to undo, so the release goes on; the failure is appended to
// the handle's last error (keeping the error that led to the release) and
// SOSO_HIP_ERR_DEVICE returned for the caller to pass on.
int hip_release(soso_hip *h, hipError_t e, const char *what);
void *scratch_get(soso_hip *h, int slot, size_t bytes);
void *pinned_get(soso_hip *h, size_t bytes);

// Input and output variants of the matvec kernel (decode-step fusions).
// XS_RMSNORM_P4: x = ((p0 + p1) + p2) + p3, the four column-segment partials
// of an EPI_PARTS matvec (parts, MV_SEG rows of cols floats; p0 holds the
// residual), then RMSNorm as XS_RMSNORM; the summed x also goes to hout (each
// workgroup writes a share; hout must not alias parts).  in.x is not read.
// EPI_PARTS: the columns split into MV_SEG segments run by different
// workgroups; y receives MV_SEG rows of partial sums (segment s at y + s*rows,
// segment 0's plus ep.res when given), which an XS_RMSNORM_P4 consumer adds in
// segment order.
enum { XS_PLAIN = 0, XS_RMSNORM = 1, XS_RMSNORM_P4 = 2 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 3, EPI_PARTS = 4 };
constexpr int MV_SEG = 4;
struct MvIn {
    const float *x = nullptr;
    const float *norm_w = nullptr; // XS_RMSNORM: the norm's weight (cols)
    float eps = 0.0f;
    const float *parts = nullptr; // XS_RMSNORM_P4: MV_SEG partial vectors of cols floats
    float *hout = nullptr;        // XS_RMSNORM_P4: where the summed x goes
};
struct MvEpi {
    const float *res = nullptr; // EPI_RESID: y = res + W.x (res may be y)
};

// packed layouts (k_matvec.hip)
size_t packed_row_stride(uint8_t dtype, size_t cols);
bool packed_shape_ok(uint8_t dtype, size_t rows, size_t cols);
// shapes a weight may be uploaded with (packed_shape_ok, or Q8_0 rows of an
// odd number of blocks, padded to kernel_cols)
bool upload_shape_ok(uint8_t dtype, size_t rows, size_t cols);
size_t kernel_cols(uint8_t dtype, size_t cols);

// launchers (k_matvec.hip)
int repack_weight(soso_hip *h, uint8_t dtype, const void *raw_dev, void *packed_dev, size_t rows, size_t cols);
int launch_matvec(soso_hip *h, const Weight &w, const float *x_dev, float *y_dev, size_t n);
// One matvec with an input variant (xs) and an output variant (epi).  EPI_SWIGLU
// expects rows interleaved (gate_i, up_i) and writes rows/2 values silu(g)*u.
int launch_matvec_ex(soso_hip *h, const Weight &w, const MvIn &in, float *y_dev, const MvEpi &ep, int xs, int epi);
// Null when launch_matvec_ex runs this (dtype, shape, xs, epi), else why not.
const char *matvec_ex_unsupported(const soso_hip *h, uint8_t dtype, size_t rows, size_t cols, int xs, int epi);
int launch_dequant(soso_hip *h, const Weight &w, float *out_dev);
int launch_argmax(soso_hip *h, const float *x_dev, size_t n, uint32_t *idx_dev);
// (k_decode.hip)
constexpr int ATT_CHUNK = 64; // positions per split of the decode attention (a multiple of 16)
// The step's q/k/v rows as the qkv matvec stored them (raw: q heads, k heads,
// v heads, f32), finished per head by the attention (layer.rs:1164-1192):
// QK norm with qn / kn when non-null, RoPE (NeoX pairs (i, i + head_dim / 2)
// when neox, else (2i, 2i + 1)) with the frequency table `freq` -- q by
// every workgroup for its query heads, the new K/V row (stored at position
// T - 1, and at rows_out when non-null) by the workgroup of the last chunk.
struct QkvRows {
    const float *raw = nullptr;
    const float *qn = nullptr, *kn = nullptr; // attn_q_norm / attn_k_norm [head_dim], or null
    const float *freq = nullptr;              // RoPE frequencies [head_dim / 2]
    void *rows_out = nullptr;                 // [k row; v row] of the step, or null
    float eps = 0.0f;
    int neox = 0, n_heads = 0, n_kv = 0;
};
int launch_attention(soso_hip *h, const QkvRows &rows, const void *K, const void *V, bool kv_f16, int n_heads,
                     int n_kv_heads, int head_dim, int ctx, int T, float *part, float *out);
// host: the callback for layers whose experts stay on the host (those layers
// decline without one)
int decode_step(soso_hip *h, DecodeModel &m, const float *x, uint32_t pos, float *logits, uint32_t *token,
                void *kv_rows, const HostMoe *host = nullptr);
// y[i] += v[i] (i < n)
int launch_vec_add(soso_hip *h, float *y, const float *v, size_t n);
// Scatter n_rows position-major rows [n_rows][kv_dim] (f32 when src_f32, else
// the cache's element type) into a head-major cache at positions row0...
int launch_kv_scatter(soso_hip *h, const void *src, bool src_f32, void *cache, bool cache_f16, int kv_dim,
                      int head_dim, int ctx, int row0, int n_rows);
// (k_moe.hip) shared expert: u[i] = silu(g[i]) * u[i] (i < n); then per
// token t (rows of hdim) y_t *= sigmoid(x_t . pg_w)
int launch_shared_swiglu(soso_hip *h, const float *g, float *u, size_t n);
int launch_shared_gate(soso_hip *h, const float *x, const float *pg_w, float *y, size_t n, size_t hdim);
// (k_gdn.hip) Gated DeltaNet block (GpuDispatch::gdn_bloque): null when the
// shape runs, else why not; the launch needs u, n x (2 n_k + n_v) d floats.
const char *gdn_unsupported(size_t n, size_t n_k, size_t n_v, size_t d, size_t kernel);
int launch_gdn_block(soso_hip *h, const float *hist, const float *conv, const float *z, const float *decay,
                     const float *beta, const float *norm, float *state, float *out, float *u, int n, int n_k,
                     int n_v, int kernel, float eps);
// (k_synth.hip)
int launch_synth_raw(soso_hip *h, void *dst, uint8_t dtype, size_t rows, size_t cols, uint64_t seed,
                     uint64_t stream);
int launch_synth_normal(soso_hip *h, float *dst, size_t n, float sigma, uint64_t seed, uint64_t stream);
int launch_read_probe(soso_hip *h, const void *src, size_t bytes, unsigned wg_per_cu, unsigned threads,
                      unsigned loads, bool chunked, bool stream, uint32_t *out, size_t out_len);
bool moe_scratch(soso_hip *h, size_t n, size_t n_groups, size_t top_k, size_t hdim, size_t ffn, MoeScratch &s);
// The same regions in one buffer of `cap` bytes at `base` (256-byte aligned
// pieces); returns the bytes needed, and sets s only when they fit.
size_t moe_scratch_fixed(const soso_hip *h, size_t n, size_t n_groups, size_t top_k, size_t hdim, size_t ffn,
                         void *base, size_t cap, MoeScratch &s);
int moe_item_target(const soso_hip *h);
// (k_mfma.hip) -- Q4_K on the matrix cores for several tokens per row
bool mfma_shape_ok(uint8_t dtype, size_t rows, size_t cols);
int launch_mfma_moe(soso_hip *h, int nmat, const uint8_t *const *A, const uint8_t *const *B, size_t rows, size_t cols,
                    size_t max_recs, const float *xs, int xdiv, const int *list, const int *recs, const int *n_recs,
                    float *out, bool tiled, const int32_t *sidx = nullptr, size_t nslots = 0);
bool mfma_moe_scan_ok(size_t n, size_t top_k, size_t n_groups, uint8_t dt_gu, uint8_t dt_down, size_t hdim,
                      size_t ffn);
// tile-major Q4_K copies (same size as the row-major packing) for launch_mfma_moe
bool tiled_q4k_ok(uint8_t dtype, size_t rows, size_t cols);
int launch_tile_q4k(soso_hip *h, const void *src_dev, void *dst_dev, size_t rows, size_t cols);
int launch_mfma_matmul(soso_hip *h, const Weight &w, const float *x, size_t n, float *y);
size_t moe_max_items(const soso_hip *h, size_t slots, size_t n_groups);
int launch_router_topk(soso_hip *h, const float *w_dev, const float *x_dev, size_t n, size_t hdim,
                       size_t n_exp, size_t top_k, int32_t *idx_dev, float *wgt_dev, float *logits_dev);
// sort false: the ranking only (idx / wgt), no slot sort, work items or
// records -- for calls whose experts scan the ranking themselves
// (mfma_moe_scan_ok)
int launch_moe_route(soso_hip *h, const float *w_dev, const float *x_dev, size_t n, size_t hdim, size_t n_exp,
                     size_t top_k, const MoeScratch &s, bool sort = true);
// One token through a registered layer (route, gate/up + SwiGLU, down +
// weighted sum), three launches, the ranking done by the expert kernel
// (DECLINED when the layer's shapes need the general path); res: added to the
// output (may be out_dev); norm_w: x_dev is h and the FFN's input is
// rmsnorm(h) * norm_w, folded into the route and gate/up staging (only where
// moe_ffn1_norm_ok).
int launch_moe_ffn1(soso_hip *h, const MoeLayer &m, const float *x_dev, const MoeScratch &s, float *out_dev,
                    const float *res = nullptr, const float *norm_w = nullptr, float eps = 0.0f);
bool moe_ffn1_norm_ok(const MoeLayer &m);
const char *moe_ffn1_unsupported(const soso_hip *h, const MoeLayer &m);
// (k_decode.hip) out[n] = rmsnorm(x) * w (one workgroup)
int launch_rmsnorm(soso_hip *h, const float *x, const float *w, size_t n, float eps, float *out);
int launch_moe_experts(soso_hip *h, const float *xs_dev, size_t n, size_t hdim, size_t ffn, size_t top_k,
                       uint8_t dt_gu, uint8_t dt_down, const uint8_t *const *tab_dev, size_t n_groups,
                       const float *wgt_dev, const uint8_t *use_dev, const int32_t *route_idx_dev,
                       const MoeScratch &s, float *out_dev, const MoeLayer *layer = nullptr, bool scan = false);

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float half_bits_to_f32(uint32_t b16)
{
    return (float)__builtin_bit_cast(_Float16, (unsigned short)b16);
}

// f16 -> f32 exactly as crates/sosomodel/src/dequant.rs:26-45: the hardware
// conversion is exact for every finite half and infinity; NaN is made the
// canonical f32::NAN (0x7fc00000), as Rust's f32::NAN.
__device__ __forceinline__ float f16_to_f32_ref(uint32_t b16)
{
    b16 &= 0xffffu;
    if ((b16 & 0x7c00u) == 0x7c00u && (b16 & 0x3ffu)) return __builtin_bit_cast(float, 0x7fc00000u);
    return half_bits_to_f32(b16);
}

// f32 -> f16 bits with the rounding of crates/soso-llm-core/src/f16.rs:10-36,
// which the KV rows must reproduce bit for bit: nearest, a tie goes away from
// zero (the first dropped bit is added to the magnitude, so a carry may step
// into the exponent or up to infinity), magnitudes below 2^-25 flush to a
// signed zero, and every NaN becomes 0x7e00 with its sign.  The hardware
// conversion rounds ties to even, hence the integer form.
__device__ __forceinline__ uint32_t f32_to_f16_soso(float v)
{
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t sign = (b >> 16) & 0x8000u, mag = b & 0x7fffffffu, frac = b & 0x7fffffu;
    const int e = (int)(mag >> 23) - 112; // biased f16 exponent
    if (mag >= 0x7f800000u) return sign | 0x7c00u | (mag > 0x7f800000u ? 0x200u : 0u);
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        const uint32_t m = frac | 0x800000u, sh = (uint32_t)(14 - e);
        return sign | ((m >> sh) + ((m >> (sh - 1)) & 1u));
    }
    return (sign | ((uint32_t)e << 10) | (frac >> 13)) + ((frac >> 12) & 1u);
}

template <int W>
__device__ __forceinline__ float seg_sum(float v)
{
    // butterfly sum inside aligned groups of W lanes (W power of two <= 64)
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}


// DPP lane moves (gfx9 encodings): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] =
// 0x4E, row_half_mirror 0x141, row_mirror 0x140, row_bcast:15 0x142,
// row_bcast:31 0x143.  Lanes of rows outside `ROWS` keep `old` (= 0 here).
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xf, false));
}

// Sum over aligned segments of W lanes (W power of two <= 64) with DPP adds.
// For W <= 16 every lane of the segment holds the sum; for W = 32 and 64 the
// LAST lane of the segment does (lane 31/63, resp. 63).
template <int W>
__device__ __forceinline__ float seg_sum_dpp(float v)
{
    if (W >= 2) v += dpp_f<0xB1>(v);
    if (W >= 4) v += dpp_f<0x4E>(v);
    if (W >= 8) v += dpp_f<0x141>(v);
    if (W >= 16) v += dpp_f<0x140>(v);
    if (W >= 32) v += dpp_f<0x142, 0xA>(v);
    if (W >= 64) v += dpp_f<0x143, 0xC>(v);
    return v;
}

// DPP move where lanes without a source (and rows outside `ROWS`) keep their
// own value -- the form max-reductions need.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ uint32_t dpp_keep(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROWS, 0xf, false);
}

// Wavefront-wide max / sum by DPP (row butterflies, then the row broadcasts
// 15 and 31); the result is read from lane 63, uniform over the wavefront.
__device__ __forceinline__ float wave_max_dpp(float v)
{
    auto st = [](float a, uint32_t b) { return fmaxf(a, __uint_as_float(b)); };
    v = st(v, dpp_keep<0xB1>(__float_as_uint(v)));
    v = st(v, dpp_keep<0x4E>(__float_as_uint(v)));
    v = st(v, dpp_keep<0x141>(__float_as_uint(v)));
    v = st(v, dpp_keep<0x140>(__float_as_uint(v)));
    v = st(v, dpp_keep<0x142, 0xA>(__float_as_uint(v)));
    v = st(v, dpp_keep<0x143, 0xC>(__float_as_uint(v)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max of a 64-bit key over the wavefront (uniform result).
__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t k)
{
#define SOSO_U64_STEP(CTRL, ROWS)                                                                                 \
    {                                                                                                             \
        const uint64_t o = ((uint64_t)dpp_keep<CTRL, ROWS>((uint32_t)(k >> 32)) << 32) |                          \
                           dpp_keep<CTRL, ROWS>((uint32_t)k);                                                     \
        k = o > k ? o : k;                                                                                        \
    }
    SOSO_U64_STEP(0xB1, 0xf)
    SOSO_U64_STEP(0x4E, 0xf)
    SOSO_U64_STEP(0x141, 0xf)
    SOSO_U64_STEP(0x140, 0xf)
    SOSO_U64_STEP(0x142, 0xA)
    SOSO_U64_STEP(0x143, 0xC)
#undef SOSO_U64_STEP
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
    return ((uint64_t)hi << 32) | lo;
}

// Max over aligned 16-lane rows (every lane gets it).
__device__ __forceinline__ float row16_max(float v)
{
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}
__device__ __forceinline__ float row16_min(float v)
{
    v = fminf(v, dpp_f<0xB1>(v));
    v = fminf(v, dpp_f<0x4E>(v));
    v = fminf(v, dpp_f<0x141>(v));
    v = fminf(v, dpp_f<0x140>(v));
    return v;
}
