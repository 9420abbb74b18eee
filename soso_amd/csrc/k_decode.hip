// k_decode.hip -- one decode step of a Llama-style model on the device (dense
// FFN layers, or registered MoE layers as the FFN).
//
// Reference: LayerExecutor::forward_layer, dense GQA branch
// (crates/soso-llm-core/src/layer.rs:1092-1389): attn_norm -> q/k/v ->
// rope_cabezas (gemm.rs:1452-1490) -> KV append -> attention -> o-proj +
// residual -> ffn_norm -> gate/up -> swiglu -> down + residual; then
// Runtime::logits_gpu + argmax (crates/soso-llm-core/src/runtime.rs:1976-2028).
// The KV cache holds f32 or, as soso's KvCache (kv.rs:258-266),
// f16 bits rounded with soso's f32_to_f16 (f16.rs:10-36).
//
// Launches per layer (every weight byte read once, activations stay in HBM):
//   1. qkv matvec   x = rmsnorm(h) staged in LDS; rows [q; k; v] concatenated,
//                   stored as computed
//   2. k_attn_split finishes the rows (QK norm when the model has it, RoPE,
//                   the new K/V row into the cache at `pos`), then split-K
//                   decode attention over 64-position chunks, the G query
//                   heads of a KV head sharing every K/V read
//   3. k_attn_merge softmax-weighted merge of the chunks
//   4. o matvec     h += W_o . attn (residual in the epilogue)
//   5. gate/up      x = rmsnorm(h); rows interleaved (gate_i, up_i); the
//                   epilogue writes silu(gate_i) * up_i
//   6. down matvec  h += W_down . act
// or, for a layer whose FFN is a registered MoE layer (4-6): x = rmsnorm(h),
// then the single-token MoE path (route; gate/up + SwiGLU; down, weighted sum
// and residual).
// Head: matvec with rmsnorm(h) staged (Q6_K or Q8_0 / Q4_K), then argmax.
#include "internal.hpp"

#include <algorithm>
#include <cmath>
#include <vector>

constexpr int ATT_HD = 128;                // head_dim handled

// Split-K decode attention: k_attn_split writes one (m, l, acc) per chunk of
// ATT_CHUNK positions and query head, k_attn_merge combines the chunks.  (The merge
// runs as its own launch: a merge by the last workgroup of each head in the
// same launch needs a device-scope fence per wavefront, which writes back the
// XCD's L2 each time and cost more than the launch it saves.)
//
// k_attn_split<G, F16, PW>: grid (n_kv_heads, chunks), block 64 * ATT_CHUNK /
// PW.  Query heads g*G .. g*G + G - 1 share KV head g (GQA), so every K/V
// byte is read once for all G heads.  K, V of one layer are head-major,
// [n_kv_heads][ctx][HD]: a chunk of one head is 32 KB of contiguous HBM.
// Wavefront w owns positions t0 + PW w .. t0 + PW w + PW - 1 (PW = 16 or 8:
// fewer positions per wavefront put more wavefronts on the G heads' scores,
// which each wavefront computes head after head).
//
// Load order per lane: its K rows, then q, then its V rows.  Loads complete in
// issue order, so the scores start once K and q are in while V is still on
// the way.  K: 8 lanes per position (128 B per lane group, whole cache lines),
// PW / 8 groups of 8 positions; V: lane holds dims 2l, 2l+1 of the PW positions.
// Positions past T are clamped onto the last valid row and get weight 0.
//
// Scores s = (q . k) / sqrt(HD).  Each wavefront keeps its own softmax
// statistics (m_w = max s, p = e^{s - m_w}, l_w = sum p, acc_w = sum p v);
// the wavefronts' are merged in LDS into the chunk's (m, l, acc), stored at
// part[(head * chunks + c) * (HD + 2)].
//
// The qkv launch stores its rows as computed and this launch finishes them
// (QkvRows).  Every workgroup normalises (QK norm) and rotates (RoPE) its G
// query heads in registers while its V rows are in flight.  The new position
// T - 1 has a workgroup row of its own (row 0, dispatched first): it
// normalises, rotates and stores the new K row, copies the new V row into the
// cache (and the step's row copy), and scores it against the G heads from
// registers and LDS, as a chunk of one position; the other rows stream the
// cached positions and never read the new row, so nothing waits for its
// stores.  Measured on MI355X, ms per token (8B step with f32 / f16 KV;
// Qwen3-30B-A3B-like step with QK norm and NeoX RoPE):
//   this arrangement                                  1.664 / 1.627; 2.081
//   RoPE and KV append in the qkv epilogue            1.711 / 1.654
//   the last chunk's workgroup appending, then
//   reading the row back (store, wait, barrier)       1.713 / 1.654; 2.166
//   a separate finishing launch (QK norm / NeoX)                     2.306
//
// Streaming loads of cached K/V bytes (the nontemporal bit): every cached
// row is read once per step and layer.
typedef uint32_t kv_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t kv_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 kv_ld16(const void *p)
{
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load((const kv_u32x4 *)p));
}
__device__ __forceinline__ uint2 kv_ld8(const void *p)
{
    return __builtin_bit_cast(uint2, __builtin_nontemporal_load((const kv_u32x2 *)p));
}
__device__ __forceinline__ uint32_t kv_ld4(const void *p) { return __builtin_nontemporal_load((const uint32_t *)p); }

// (a, b) -> (a cos - b sin, a sin + b cos), rope_cabezas' rotation
// (gemm.rs:1452-1490) with each product rounded on its own.
__device__ __forceinline__ void turn_pair(float &a, float &b, float cs, float sn)
{
    const float na = __fsub_rn(__fmul_rn(a, cs), __fmul_rn(b, sn));
    const float nb = __fadd_rn(__fmul_rn(a, sn), __fmul_rn(b, cs));
    a = na;
    b = nb;
}

// QK norm and RoPE (layer.rs:1164-1192, FLAG_QK_NORM / FLAG_ROPE_NEOX) of one
// head of 128 held as one rotation pair (a, b) per lane.  With `norm`
// (uniform over the wavefront) the head is first RMS-normalised and scaled by
// the layer's attn_q_norm / attn_k_norm weights w0, w1 at the pair's elements
// (rmsnorm, gemm.rs:93-100: x * scale * w, scale = 1 / sqrt(sum(x^2) / n +
// eps)); then (a, b) turns by the angle whose cosine and sine are cs, sn.
__device__ __forceinline__ void head_post(float &a, float &b, bool norm, float w0, float w1, float eps, float cs,
                                          float sn)
{
    if (norm) {
        float ss = fmaf(a, a, b * b);
        ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, seg_sum_dpp<64>(ss)), 63));
        const float scale = 1.0f / sqrtf(ss / (float)ATT_HD + eps);
        a = __fmul_rn(__fmul_rn(a, scale), w0);
        b = __fmul_rn(__fmul_rn(b, scale), w1);
    }
    turn_pair(a, b, cs, sn);
}

// One element of a new K or V row: into the cache at `at` and, when asked,
// into the step's row copy at `row_at` (f16 with soso's rounding, or f32).
// Returns the value as the cache holds it.
template <bool F16>
__device__ __forceinline__ float kv_row_put(void *cache, void *rows_out, size_t at, int row_at, float v)
{
    if constexpr (F16) {
        const uint16_t bits = (uint16_t)f32_to_f16_soso(v);
        ((uint16_t *)cache)[at] = bits;
        if (rows_out) ((uint16_t *)rows_out)[row_at] = bits;
        return half_bits_to_f32(bits);
    } else {
        ((float *)cache)[at] = v;
        if (rows_out) ((float *)rows_out)[row_at] = v;
        return v;
    }
}

// QK norm and RoPE of the group's q in registers (layer.rs:1164-1192):
// thread t holds float4 t of the G heads (head t / 32, one half of a
// wavefront) and qw, the norm weights of its 4 elements; lane l computes the
// angle of pair l, (T - 1) * fr, and passes it to the lanes holding that pair.
__device__ __forceinline__ float4 finish_q(float4 qv, float4 qw, float fr, const QkvRows &rows, int T)
{
    constexpr int HD = ATT_HD;
    const int lane = threadIdx.x & 63, tq = lane & 31;
    if (rows.qn) {
        // lanes 31 and 63 hold their half's sum (readlane takes a uniform lane)
        float ss = seg_sum_dpp<32>((qv.x * qv.x + qv.y * qv.y) + (qv.z * qv.z + qv.w * qv.w));
        const float s_lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 31));
        const float s_hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 63));
        ss = lane < 32 ? s_lo : s_hi;
        const float scale = 1.0f / sqrtf(ss / (float)HD + rows.eps);
        qv = make_float4(__fmul_rn(__fmul_rn(qv.x, scale), qw.x), __fmul_rn(__fmul_rn(qv.y, scale), qw.y),
                         __fmul_rn(__fmul_rn(qv.z, scale), qw.z), __fmul_rn(__fmul_rn(qv.w, scale), qw.w));
    }
    float cs, sn;
    sincosf((float)(T - 1) * fr, &sn, &cs);
    if (!rows.neox) {
        // pairs (4tq, 4tq + 1) and (4tq + 2, 4tq + 3): 2tq and 2tq + 1
        turn_pair(qv.x, qv.y, __shfl(cs, 2 * tq, 64), __shfl(sn, 2 * tq, 64));
        turn_pair(qv.z, qv.w, __shfl(cs, 2 * tq + 1, 64), __shfl(sn, 2 * tq + 1, 64));
        return qv;
    }
    // pairs (i, i + 64): thread tq < 16 holds the first elements of pairs
    // 4tq .. 4tq + 3, thread tq + 16 the second ones
    const float ot[4] = {__shfl_xor(qv.x, 16, 64), __shfl_xor(qv.y, 16, 64), __shfl_xor(qv.z, 16, 64),
                         __shfl_xor(qv.w, 16, 64)};
    float me[4] = {qv.x, qv.y, qv.z, qv.w};
    const bool lo = tq < 16;
    const int i0 = 4 * (tq & 15);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float a = lo ? me[k] : ot[k], b = lo ? ot[k] : me[k];
        turn_pair(a, b, __shfl(cs, i0 + k, 64), __shfl(sn, i0 + k, 64));
        me[k] = lo ? a : b;
    }
    return make_float4(me[0], me[1], me[2], me[3]);
}

// grid (n_kv_heads, 1 + ceil((T - 1) / ATT_CHUNK)): workgroup row 0 appends
// the new position T - 1 and takes it as a chunk of its own (partial index
// chunks - 1); rows 1 .. hold the cached positions 0 .. T - 2 in chunks of
// ATT_CHUNK (partial index blockIdx.y - 1).
template <int G, bool F16, int PW>
__global__ void __launch_bounds__(64 * ATT_CHUNK / PW) k_attn_split(QkvRows rows, const void *__restrict__ Kc,
                                                                     const void *__restrict__ Vc, int ctx, int T,
                                                                     int chunks, float *__restrict__ part)
{
    static_assert(PW == 8 || PW == 16, "8 or 16 positions per wavefront");
    constexpr int HD = ATT_HD, NW = ATT_CHUNK / PW, NT = 64 * NW, KA = PW / 8;
    static_assert(G * HD / 4 <= NT, "one float4 of q per thread");
    __shared__ float qs[G * HD];
    __shared__ float wm[NW][G], wl[NW][G];
    __shared__ float2 accs[NW][G][HD / 2];
    const int g = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const size_t head_off = (size_t)g * ctx * HD;
    const float inv = 1.0f / sqrtf((float)HD);
    const float *qsrc = rows.raw + (size_t)g * G * HD;
    if (blockIdx.y == 0) {
        // The new position: its K row (wavefront 0: QK norm, RoPE; lane l
        // holds the rotation pair l, elements (l, l + 64) with NeoX RoPE,
        // (2l, 2l + 1) otherwise) and V row (wavefront 1: elements 2l, 2l + 1)
        // go into the cache at T - 1 and the step's row copy, and into LDS as
        // the cache holds them; then each query head's score against that one
        // row: (m, l, acc) = (q.k / sqrt(HD), 1, v).  Nothing in this launch
        // reads the stores back.
        float4 qv = make_float4(0.f, 0.f, 0.f, 0.f), qw = make_float4(1.f, 1.f, 1.f, 1.f);
        if (tid < G * HD / 4) qv = ((const float4 *)qsrc)[tid];
        if (rows.qn) qw = ((const float4 *)rows.qn)[lane & 31];
        const float fr = rows.freq[lane];
        float *knew = (float *)accs, *vnew = knew + HD; // LDS reused
        if (wave < 2) {
            const int d0 = wave == 0 && rows.neox ? lane : 2 * lane;
            const int d1 = wave == 0 && rows.neox ? lane + 64 : 2 * lane + 1;
            const float *src = rows.raw + (size_t)(rows.n_heads + wave * rows.n_kv + g) * HD;
            float a = src[d0], b = src[d1];
            if (wave == 0) {
                float cs, sn;
                sincosf((float)(T - 1) * fr, &sn, &cs);
                head_post(a, b, rows.kn != nullptr, rows.kn ? rows.kn[d0] : 1.0f, rows.kn ? rows.kn[d1] : 1.0f,
                          rows.eps, cs, sn);
            }
            void *cache = const_cast<void *>(wave == 0 ? Kc : Vc);
            const size_t at = head_off + (size_t)(T - 1) * HD;
            const int row = wave * rows.n_kv * HD + g * HD;
            float *dst = wave == 0 ? knew : vnew;
            dst[d0] = kv_row_put<F16>(cache, rows.rows_out, at + d0, row + d0, a);
            dst[d1] = kv_row_put<F16>(cache, rows.rows_out, at + d1, row + d1, b);
        }
        qv = finish_q(qv, qw, fr, rows, T);
        if (tid < G * HD / 4) *(float4 *)&qs[4 * tid] = qv;
        __syncthreads();
        for (int hh = wave; hh < G; hh += NW) {
            float acc = fmaf(qs[hh * HD + 2 * lane], knew[2 * lane], qs[hh * HD + 2 * lane + 1] * knew[2 * lane + 1]);
            acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(seg_sum_dpp<64>(acc)), 63));
            float *o = part + ((size_t)(g * G + hh) * chunks + (chunks - 1)) * (HD + 2);
            if (lane == 0) {
                o[0] = acc * inv;
                o[1] = 1.0f;
            }
            *(float2 *)(o + 2 + 2 * lane) = make_float2(vnew[2 * lane], vnew[2 * lane + 1]);
        }
        return;
    }
    // cached positions 0 .. T - 2
    const int c = (int)blockIdx.y - 1, Tc = T - 1;
    const int t0 = c * ATT_CHUNK, t1 = min(Tc, t0 + ATT_CHUNK);
    const int tw = t0 + PW * wave;
    const int pp = lane >> 3, j = lane & 7;
    // K: f32 rows are 512 B, lane j of a position takes float4 units j, j+8,
    // j+16, j+24 (dims 32i + 4j ..); f16 rows are 256 B, lane j takes 16-byte
    // units j, j+8 (dims 64i + 8j .. 64i + 8j + 7)
    float4 kv[KA][4];
    uint4 kh[KA][2];
#pragma unroll
    for (int a = 0; a < KA; a++) {
        const size_t row = head_off + (size_t)min(tw + 8 * a + pp, t1 - 1) * HD;
        if constexpr (F16) {
            const uint4 *k4 = (const uint4 *)((const uint16_t *)Kc + row);
#pragma unroll
            for (int i = 0; i < 2; i++) kh[a][i] = kv_ld16(k4 + 8 * i + j);
        } else {
            const float4 *k4 = (const float4 *)((const float *)Kc + row);
#pragma unroll
            for (int i = 0; i < 4; i++) kv[a][i] = __builtin_bit_cast(float4, kv_ld16(k4 + 8 * i + j));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // only the wavefronts holding q (one float4 per thread) finish it
    constexpr int QW = (G * HD / 4 + 63) / 64;
    const bool qwave = wave < QW;
    float4 qv = make_float4(0.f, 0.f, 0.f, 0.f), qw = make_float4(1.f, 1.f, 1.f, 1.f);
    float fr = 0.0f;
    if (qwave) {
        if (tid < G * HD / 4) qv = ((const float4 *)qsrc)[tid];
        if (rows.qn) qw = ((const float4 *)rows.qn)[lane & 31];
        fr = rows.freq[lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    // V: lane l holds dims 2l, 2l + 1 of the wavefront's PW positions
    float2 vr[PW];
    uint32_t vh[PW];
#pragma unroll
    for (int k = 0; k < PW; k++) {
        const size_t row = head_off + (size_t)min(tw + k, t1 - 1) * HD + 2 * lane;
        if constexpr (F16)
            vh[k] = kv_ld4((const uint16_t *)Vc + row);
        else
            vr[k] = __builtin_bit_cast(float2, kv_ld8((const float *)Vc + row));
    }
    __builtin_amdgcn_sched_barrier(0);
    if (qwave) {
        qv = finish_q(qv, qw, fr, rows, T);
        if (tid < G * HD / 4) *(float4 *)&qs[4 * tid] = qv;
    }
    if constexpr (F16) {
        // f16 -> f32 is exact; from here on the math is the f32 kernel's
#pragma unroll
        for (int a = 0; a < KA; a++)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint32_t w[4] = {kh[a][i].x, kh[a][i].y, kh[a][i].z, kh[a][i].w};
                kv[a][2 * i] = make_float4(half_bits_to_f32(w[0] & 0xffffu), half_bits_to_f32(w[0] >> 16),
                                           half_bits_to_f32(w[1] & 0xffffu), half_bits_to_f32(w[1] >> 16));
                kv[a][2 * i + 1] = make_float4(half_bits_to_f32(w[2] & 0xffffu), half_bits_to_f32(w[2] >> 16),
                                               half_bits_to_f32(w[3] & 0xffffu), half_bits_to_f32(w[3] >> 16));
            }
    }
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < G; hh++) {
        float s[KA];
#pragma unroll
        for (int a = 0; a < KA; a++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // kv[a][i] holds dims 32i + 4j .. (f32) or 64(i/2) + 8j + 4(i%2) .. (f16)
                const int d0 = F16 ? 64 * (i >> 1) + 8 * j + 4 * (i & 1) : 32 * i + 4 * j;
                const float4 qq = *(const float4 *)&qs[hh * HD + d0];
                acc = fmaf(kv[a][i].x, qq.x, acc);
                acc = fmaf(kv[a][i].y, qq.y, acc);
                acc = fmaf(kv[a][i].z, qq.z, acc);
                acc = fmaf(kv[a][i].w, qq.w, acc);
            }
            acc = seg_sum_dpp<8>(acc); // all 8 lanes of the position hold the sum
            s[a] = tw + 8 * a + pp < t1 ? acc * inv : -INFINITY;
        }
        float smax = s[0];
#pragma unroll
        for (int a = 1; a < KA; a++) smax = fmaxf(smax, s[a]);
        const float m = wave_max_dpp(smax);
        float p[KA];
#pragma unroll
        for (int a = 0; a < KA; a++) p[a] = s[a] == -INFINITY ? 0.0f : expf(s[a] - m);
        float2 acc = make_float2(0.f, 0.f);
        float l = 0.0f;
#pragma unroll
        for (int k = 0; k < PW; k++) {
            const float pk = __builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p[k >> 3]), 8 * (k & 7)));
            l += pk;
            const float2 vk = F16 ? make_float2(half_bits_to_f32(vh[k] & 0xffffu), half_bits_to_f32(vh[k] >> 16))
                                  : vr[k];
            acc.x = fmaf(pk, vk.x, acc.x);
            acc.y = fmaf(pk, vk.y, acc.y);
        }
        accs[wave][hh][lane] = acc;
        if (lane == 0) {
            wm[wave][hh] = m;
            wl[wave][hh] = l;
        }
    }
    __syncthreads();
    for (int e = tid; e < G * HD / 2; e += NT) { // a whole wavefront per head hh
        const int hh = e / (HD / 2), dl = e % (HD / 2);
        float M = wm[0][hh];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, wm[w][hh]);
        // lane w < NW takes wavefront w's factor, read by every lane of the head
        const float mw = wm[lane < NW ? lane : 0][hh];
        const float fw = mw == -INFINITY ? 0.0f : expf(mw - M);
        float L = 0.0f;
        float2 a = make_float2(0.f, 0.f);
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, fw), w));
            L = fmaf(f, wl[w][hh], L);
            a.x = fmaf(f, accs[w][hh][dl].x, a.x);
            a.y = fmaf(f, accs[w][hh][dl].y, a.y);
        }
        float *o = part + ((size_t)(g * G + hh) * chunks + c) * (HD + 2);
        if (dl == 0) {
            o[0] = M;
            o[1] = L;
        }
        *(float2 *)(o + 2 + 2 * dl) = a;
    }
}

// k_attn_merge: grid n_heads, block 256.  Wavefront w takes chunks w, w + 4,
// ... in batches of MERGE_B, all loads of a batch in flight together, and
// folds them into running (m, l, acc) (lane: dims 2l, 2l + 1); the four
// wavefronts are then merged in LDS:
//   out[h*HD + d] = sum_c e^{m_c - M} acc_c[d] / sum_c e^{m_c - M} l_c.
constexpr int MERGE_B = 20;
// Wavefronts per merge workgroup.  Measured on MI355X (8B decode step at 4096
// positions, 65 chunks per head): 2 / 4 / 8 wavefronts 1.505 / 1.474 / 1.477 ms.
constexpr int MERGE_NW = 4;

__global__ void __launch_bounds__(64 * MERGE_NW) k_attn_merge(const float *__restrict__ part, int chunks,
                                                     float *__restrict__ out)
{
    constexpr int HD = ATT_HD, NW = MERGE_NW;
    __shared__ float wm[NW], wl[NW];
    __shared__ float2 accs[NW][HD / 2];
    const int h = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float *ph = part + (size_t)h * chunks * (HD + 2);
    float m = -INFINITY, l = 0.0f;
    float2 acc = make_float2(0.f, 0.f);
    for (int c0 = wave; c0 < chunks; c0 += NW * MERGE_B) {
        const int n = min(MERGE_B, (chunks - c0 + NW - 1) / NW); // chunks c0 + NW*k, k < n
        float2 ml[MERGE_B], v[MERGE_B];
#pragma unroll
        for (int k = 0; k < MERGE_B; k++) {
            // no loads past the wavefront's last chunk (with a fixed batch of
            // MERGE_B clamped loads per wavefront, 8 wavefronts per head took
            // 1.524 ms against 1.485 with 4)
            ml[k] = make_float2(-INFINITY, 0.0f);
            v[k] = make_float2(0.f, 0.f);
            if (k < n) { // uniform
                const float *pc = ph + (size_t)(c0 + NW * k) * (HD + 2);
                ml[k] = *(const float2 *)pc;
                v[k] = *(const float2 *)(pc + 2 + 2 * lane);
            }
        }
        float bm = m;
#pragma unroll
        for (int k = 0; k < MERGE_B; k++) bm = fmaxf(bm, ml[k].x);
        const float r = m == -INFINITY ? 0.0f : expf(m - bm);
        l *= r;
        acc.x *= r;
        acc.y *= r;
        // the batch's weights are uniform: lane k computes chunk k's, every
        // lane reads them (one expf per lane instead of MERGE_B)
        float mk = -INFINITY;
#pragma unroll
        for (int k = 0; k < MERGE_B; k++) mk = lane == k && k < n ? ml[k].x : mk;
        const float wk = mk == -INFINITY ? 0.0f : expf(mk - bm);
#pragma unroll
        for (int k = 0; k < MERGE_B; k++) {
            const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k));
            l = fmaf(w, ml[k].y, l);
            acc.x = fmaf(w, v[k].x, acc.x);
            acc.y = fmaf(w, v[k].y, acc.y);
        }
        m = bm;
    }
    accs[wave][lane] = acc;
    if (lane == 0) {
        wm[wave] = m;
        wl[wave] = l;
    }
    __syncthreads();
    if (wave == 0) {
        float M = wm[0];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, wm[w]);
        const float mw = wm[lane < NW ? lane : 0];
        const float fw = mw == -INFINITY ? 0.0f : expf(mw - M);
        float L = 0.0f;
        float2 a = make_float2(0.f, 0.f);
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, fw), w));
            L = fmaf(f, wl[w], L);
            a.x = fmaf(f, accs[w][lane].x, a.x);
            a.y = fmaf(f, accs[w][lane].y, a.y);
        }
        const float r = L > 0.0f ? 1.0f / L : 0.0f;
        *(float2 *)(out + (size_t)h * HD + 2 * lane) = make_float2(a.x * r, a.y * r);
    }
}

// Positions per wavefront of the split kernel.  Measured on MI355X (graph-
// replayed steps at position 4096): f32 rows 8 (8B model, groups of 4: 1.686
// against 1.721 ms per token with 16); f16 rows 16 (8B: 1.701 against 1.709 ms;
// Qwen3-30B-A3B-like, groups of 8: 2.197 against 2.224 ms).
template <bool F16> constexpr int att_pw() { return F16 ? 16 : 8; }

int launch_attention(soso_hip *h, const QkvRows &rows, const void *K, const void *V, bool kv_f16, int n_heads,
                     int n_kv_heads, int head_dim, int ctx, int T, float *part, float *out)
{
    if (head_dim != ATT_HD || n_kv_heads <= 0 || n_heads % n_kv_heads || T <= 0 || T > ctx)
        return set_err(h, SOSO_HIP_DECLINED, "attention: head shape not handled here");
    const int G = n_heads / n_kv_heads;
    const int chunks = 1 + (T - 1 + ATT_CHUNK - 1) / ATT_CHUNK; // the new position, then the cached ones
    const dim3 grid((unsigned)n_kv_heads, (unsigned)chunks);
    if (!rows.raw || !rows.freq || rows.n_heads != n_heads || rows.n_kv != n_kv_heads)
        return set_err(h, SOSO_HIP_ERR_ARG, "attention: q/k/v rows missing");
#define ATT_LAUNCH(GG, F)                                                                                           \
    k_attn_split<GG, F, att_pw<F>()><<<grid, 64 * ATT_CHUNK / att_pw<F>(), 0, h->stream>>>(rows, K, V, ctx, T,      \
                                                                                           chunks, part)
#define ATT_CASE(GG)                                                                                                \
    case GG:                                                                                                        \
        if (kv_f16) ATT_LAUNCH(GG, true);                                                                           \
        else ATT_LAUNCH(GG, false);                                                                                 \
        break;
    switch (G) {
        ATT_CASE(1) ATT_CASE(2) ATT_CASE(4) ATT_CASE(8)
    default: return set_err(h, SOSO_HIP_DECLINED, "attention: GQA group size not handled here");
    }
#undef ATT_CASE
#undef ATT_LAUNCH
    int rc = hip_check(h, hipGetLastError(), "attention split launch");
    if (rc != SOSO_HIP_OK) return rc;
    k_attn_merge<<<(unsigned)n_heads, 64 * MERGE_NW, 0, h->stream>>>(part, chunks, out);
    return hip_check(h, hipGetLastError(), "attention merge launch");
}

// rmsnorm (crates/soso-llm-core/src/gemm.rs:93-100) into a new vector: one
// workgroup of 1024 threads, x loaded once into registers (n <= 8192),
// out_i = (x_i * scale) * w_i with scale = 1 / sqrt(sum(x^2) / n + eps) --
// the arithmetic the matvec staging's RMSNorm uses.  The MoE FFN of a decode
// layer reads it (its experts stage x as given).
constexpr int RMS_T = 1024, RMS_PER = 8; // threads, elements per thread
__global__ void __launch_bounds__(RMS_T) k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, int n,
                                                   float eps, float *__restrict__ out)
{
    __shared__ float red[RMS_T / 64];
    float v[RMS_PER];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < RMS_PER; k++) {
        const int i = k * RMS_T + (int)threadIdx.x;
        v[k] = i < n ? x[i] : 0.0f;
        ss = fmaf(v[k], v[k], ss);
    }
    ss = seg_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < RMS_T / 64; i++) tot += red[i];
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
#pragma unroll
    for (int k = 0; k < RMS_PER; k++) {
        const int i = k * RMS_T + (int)threadIdx.x;
        if (i < n) out[i] = __fmul_rn(__fmul_rn(v[k], scale), w[i]);
    }
}

int launch_rmsnorm(soso_hip *h, const float *x, const float *w, size_t n, float eps, float *out)
{
    if (n == 0 || n > (size_t)RMS_T * RMS_PER) return set_err(h, SOSO_HIP_DECLINED, "rmsnorm: width");
    k_rmsnorm<<<1, RMS_T, 0, h->stream>>>(x, w, (int)n, eps, out);
    return hip_check(h, hipGetLastError(), "rmsnorm launch");
}

// KV upload (decode_subir_estado): element e of the position-major rows
// [n_rows][kv_dim] goes to head e / head_dim, position row0 + e / kv_dim of
// the head-major cache; f32 rows entering an f16 cache take soso's rounding.
template <bool SRC_F32, bool DST_F16>
__global__ void __launch_bounds__(256) k_kv_scatter(const void *__restrict__ src, void *__restrict__ cache,
                                                     int kv_dim, int head_dim, int ctx, int row0, size_t n)
{
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    const int r = (int)(e / kv_dim), c = (int)(e % kv_dim);
    const size_t at = ((size_t)(c / head_dim) * ctx + row0 + r) * head_dim + c % head_dim;
    if constexpr (!DST_F16)
        ((float *)cache)[at] = ((const float *)src)[e];
    else if constexpr (SRC_F32)
        ((uint16_t *)cache)[at] = (uint16_t)f32_to_f16_soso(((const float *)src)[e]);
    else
        ((uint16_t *)cache)[at] = ((const uint16_t *)src)[e];
}

int launch_kv_scatter(soso_hip *h, const void *src, bool src_f32, void *cache, bool cache_f16, int kv_dim,
                      int head_dim, int ctx, int row0, int n_rows)
{
    const size_t n = (size_t)n_rows * kv_dim;
    if (n == 0) return SOSO_HIP_OK;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (!cache_f16)
        k_kv_scatter<true, false><<<grid, 256, 0, h->stream>>>(src, cache, kv_dim, head_dim, ctx, row0, n);
    else if (src_f32)
        k_kv_scatter<true, true><<<grid, 256, 0, h->stream>>>(src, cache, kv_dim, head_dim, ctx, row0, n);
    else
        k_kv_scatter<false, true><<<grid, 256, 0, h->stream>>>(src, cache, kv_dim, head_dim, ctx, row0, n);
    return hip_check(h, hipGetLastError(), "kv scatter launch");
}

__global__ void __launch_bounds__(256) k_vec_add(float *__restrict__ y, const float *__restrict__ v, int n)
{
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    if (i < n) y[i] += v[i];
}

int launch_vec_add(soso_hip *h, float *y, const float *v, size_t n)
{
    if (n == 0) return SOSO_HIP_OK;
    k_vec_add<<<(unsigned)((n + 255) / 256), 256, 0, h->stream>>>(y, v, (int)n);
    return hip_check(h, hipGetLastError(), "vec add launch");
}

// A layer whose experts stay on the host (decode_token's cpu_moe, gpu.rs:674-679):
// xn and the routing the device computed go down, the callback's weighted sum
// of the chosen experts comes up into xn's buffer and joins the residual.
static int host_moe_ffn(soso_hip *h, DecodeModel &m, size_t layer, const MoeLayer &ml, const MoeScratch &s,
                        const HostMoe &host)
{
    const size_t H = m.hidden, k = ml.top_k;
    char *st = (char *)pinned_get(h, (2 * H + 2 * k) * 4);
    if (!st) return set_err(h, SOSO_HIP_ERR_NOMEM, "decode_token: pinned staging");
    float *xn = (float *)st, *out = xn + H;
    int32_t *idx = (int32_t *)(out + H);
    float *wgt = (float *)(idx + k);
    int rc = hip_check(h, hipMemcpyAsync(xn, m.xn, H * 4, hipMemcpyDeviceToHost, h->stream), "xn down");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipMemcpyAsync(idx, s.idx, k * 4, hipMemcpyDeviceToHost, h->stream), "idx");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipMemcpyAsync(wgt, s.wgt, k * 4, hipMemcpyDeviceToHost, h->stream), "wgt");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "host moe sync");
    if (rc != SOSO_HIP_OK) return rc;
    if (host.fn(host.ctx, (uint32_t)layer, xn, idx, wgt, k, out) != 0)
        return set_err(h, SOSO_HIP_ERR_ARG, "decode_token: cpu_moe failed at layer " + std::to_string(layer));
    h->stats.bytes_down += (H + 2 * k) * 4;
    h->stats.bytes_up += H * 4;
    rc = hip_check(h, hipMemcpyAsync(m.xn, out, H * 4, hipMemcpyHostToDevice, h->stream), "moe out up");
    if (rc == SOSO_HIP_OK) rc = launch_vec_add(h, m.hid, m.xn, H);
    return rc;
}

// ---------------------------------------------------------------------------
// The decode step
// ---------------------------------------------------------------------------
int decode_step(soso_hip *h, DecodeModel &m, const float *x, uint32_t pos, float *logits, uint32_t *token,
                void *kv_rows, const HostMoe *host)
{
    const int kv_dim = (int)(m.n_kv_heads * m.head_dim);
    if (pos >= m.ctx_max) return set_err(h, SOSO_HIP_ERR_ARG, "decode: position beyond the KV capacity");
    float *hid = m.hid, *att = m.att, *act = m.act, *lg = logits ? logits : m.logits;
    // layer 0 reads the caller's x in place (its o projection writes the first
    // hid) when x is 16-byte aligned for the staging's vector loads; else a copy
    const bool direct = ((uintptr_t)x & 15) == 0;
    int rc = direct ? SOSO_HIP_OK
                    : hip_check(h, hipMemcpyAsync(hid, x, m.hidden * 4, hipMemcpyDeviceToDevice, h->stream), "x copy");
    // pending: hid lacks the last down projection, whose MV_SEG column-segment
    // partials wait in m.dpart; the next launch that stages h adds them (into
    // m.hid2, which then holds the layer's input h)
    bool pending = false;
    for (size_t l = 0; l < m.n_layers && rc == SOSO_HIP_OK; l++) {
        const float *hin = l == 0 && direct ? x : hid;
        const DecodeLayer &L = m.layers[l];
        const size_t esz = m.kv_f16 ? 2 : 4, layer_bytes = m.ctx_max * kv_dim * esz;
        void *K = (char *)m.kcache + l * layer_bytes, *V = (char *)m.vcache + l * layer_bytes;
        MvIn in;
        in.x = hin;
        in.norm_w = L.attn_norm;
        in.eps = m.eps;
        // the q/k/v rows as computed; the attention finishes them per head
        // (QK norm, RoPE) and appends the new K/V row
        QkvRows rows;
        rows.raw = m.qkv_raw;
        rows.qn = L.q_norm;
        rows.kn = L.k_norm;
        rows.freq = m.rope_freq;
        rows.rows_out = kv_rows ? (char *)kv_rows + l * 2 * kv_dim * esz : nullptr;
        rows.eps = m.eps;
        rows.neox = m.rope_neox ? 1 : 0;
        rows.n_heads = (int)m.n_heads;
        rows.n_kv = (int)m.n_kv_heads;
        if (pending) {
            in.parts = m.dpart;
            in.hout = m.hid2;
            hin = m.hid2;
        }
        rc = launch_matvec_ex(h, *L.qkv, in, m.qkv_raw, MvEpi(), pending ? XS_RMSNORM_P4 : XS_RMSNORM, EPI_STORE);
        pending = false;
        if (rc == SOSO_HIP_OK)
            rc = launch_attention(h, rows, K, V, m.kv_f16, (int)m.n_heads, (int)m.n_kv_heads, (int)m.head_dim,
                                  (int)m.ctx_max, (int)pos + 1, m.part, att);
        if (rc == SOSO_HIP_OK) {
            MvIn a;
            a.x = att;
            MvEpi r;
            r.res = hin;
            rc = launch_matvec_ex(h, *L.o, a, hid, r, XS_PLAIN, EPI_RESID);
        }
        if (L.moe && !L.moe->tab) {
            // experts on the host: routing here, the FFN by the caller's cpu_moe
            if (!host || !host->fn)
                return set_err(h, SOSO_HIP_DECLINED, "decode: a layer's experts stay on the host (decode_token)");
            const MoeLayer &ml = *L.moe;
            if (rc == SOSO_HIP_OK) rc = launch_rmsnorm(h, hid, L.ffn_norm, m.hidden, m.eps, m.xn);
            if (rc == SOSO_HIP_OK)
                rc = launch_moe_route(h, (const float *)ml.router->dev, m.xn, 1, ml.hdim, ml.n_exp, ml.top_k, L.moe_s);
            if (rc == SOSO_HIP_OK) rc = host_moe_ffn(h, m, l, ml, L.moe_s, *host);
        } else if (L.moe) {
            // MoE FFN (forward_moe_ffn, layer.rs:1938-1975): x = rmsnorm(h) * ffn_norm,
            // router + top-k, the chosen experts, h += their ranking-order sum;
            // the norm folded into the route's and the experts' x staging where
            // the route holds the row in one step, else a launch of its own
            if (moe_ffn1_norm_ok(*L.moe)) {
                if (rc == SOSO_HIP_OK) rc = launch_moe_ffn1(h, *L.moe, hid, L.moe_s, hid, hid, L.ffn_norm, m.eps);
            } else {
                if (rc == SOSO_HIP_OK) rc = launch_rmsnorm(h, hid, L.ffn_norm, m.hidden, m.eps, m.xn);
                if (rc == SOSO_HIP_OK) rc = launch_moe_ffn1(h, *L.moe, m.xn, L.moe_s, hid, hid);
            }
        } else {
            if (rc == SOSO_HIP_OK) {
                MvIn f;
                f.x = hid;
                f.norm_w = L.ffn_norm;
                f.eps = m.eps;
                rc = launch_matvec_ex(h, *L.gu, f, act, MvEpi(), XS_RMSNORM, EPI_SWIGLU);
            }
            if (rc == SOSO_HIP_OK) {
                MvIn a;
                a.x = act;
                MvEpi r;
                r.res = hid;
                if (L.down_parts) {
                    rc = launch_matvec_ex(h, *L.down, a, m.dpart, r, XS_PLAIN, EPI_PARTS);
                    pending = true;
                } else {
                    rc = launch_matvec_ex(h, *L.down, a, hid, r, XS_PLAIN, EPI_RESID);
                }
            }
        }
    }
    if (!m.head) return rc; // a stack of layers without the head (soso_hip_moe_capa)
    if (rc == SOSO_HIP_OK) {
        MvIn in;
        in.x = hid;
        in.norm_w = m.out_norm;
        in.eps = m.eps;
        if (pending) {
            in.parts = m.dpart;
            in.hout = m.hid2;
        }
        rc = launch_matvec_ex(h, *m.head, in, lg, MvEpi(), pending ? XS_RMSNORM_P4 : XS_RMSNORM, EPI_STORE);
    }
    if (rc == SOSO_HIP_OK && token) rc = launch_argmax(h, lg, m.vocab, token);
    return rc;
}
