// k_decode.hip -- one decode step of a dense Llama-style model on the device.
//
// Reference: LayerExecutor::forward_layer, dense GQA branch
// (crates/soso-llm-core/src/layer.rs:1092-1389): attn_norm -> q/k/v ->
// rope_cabezas (gemm.rs:1452-1490) -> KV append -> attention -> o-proj +
// residual -> ffn_norm -> gate/up -> swiglu -> down + residual; then
// Runtime::logits_gpu + argmax (crates/soso-llm-core/src/runtime.rs:1976-2028).
// The KV cache is f32 here; soso keeps f16 (kv.rs:349).
//
// Launches per layer (every weight byte read once, activations stay in HBM):
//   1. qkv matvec   x = rmsnorm(h) staged in LDS; rows [q; k; v] concatenated;
//                   RoPE applied to q/k row pairs in the epilogue, k and v
//                   written straight into the KV cache at `pos`
//   2. k_attn_split split-K decode attention over 64-position chunks, the
//                   G query heads of a KV head share every K/V read
//   3. k_attn_combine  softmax-weighted merge of the chunks
//   4. o matvec     h += W_o . attn (residual in the epilogue)
//   5. gate/up      x = rmsnorm(h); rows interleaved (gate_i, up_i); the
//                   epilogue writes silu(gate_i) * up_i
//   6. down matvec  h += W_down . act
// Head: matvec with rmsnorm(h) staged (Q6_K or Q8_0 / Q4_K), then argmax.
#include "internal.hpp"

#include <algorithm>
#include <cmath>
#include <vector>

constexpr int ATT_HD = 128;   // head_dim handled
constexpr int ATT_CHUNK = 64; // positions per split

// grid (n_kv_heads, chunks), block 256: q heads g*G .. g*G + G - 1 share KV
// head g (GQA).  Scores s = (q . k) / sqrt(hd); per chunk: m = max s,
// p = exp(s - m), l = sum p, acc = sum p v.  part[(head * chunks + c) *
// (HD + 2)] = {m, l, acc[0..HD)}.  K, V of one layer are head-major:
// [n_kv_heads][ctx][HD], so a chunk of one head is 32 KB of contiguous HBM.
// Wavefront w owns positions t0 + 16w .. t0 + 16w + 15 of the chunk for all G
// heads: its V rows are requested first, then its K rows, so both streams are
// in flight together; every K and V byte is read once.
template <int G>
__global__ void __launch_bounds__(256) k_attn_split(const float *__restrict__ q, const float *__restrict__ K,
                                                     const float *__restrict__ V, int ctx, int T, int chunks,
                                                     float *__restrict__ part)
{
    constexpr int HD = ATT_HD, NW = 4;
    __shared__ float qs[G][HD];
    __shared__ float sc[G][ATT_CHUNK];
    __shared__ float2 accs[NW][G][HD / 2];
    const int g = blockIdx.x, c = blockIdx.y;
    const int t0 = c * ATT_CHUNK, t1 = min(T, t0 + ATT_CHUNK), n = t1 - t0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tw = t0 + 16 * wave; // this wavefront's 16 positions
    // V rows: lane holds dims 2l, 2l+1 of each of the 16 positions
    float2 vr[16];
    const float *vb = V + (size_t)g * ctx * HD + 2 * lane;
#pragma unroll
    for (int k = 0; k < 16; k++)
        vr[k] = tw + k < t1 ? *(const float2 *)(vb + (size_t)(tw + k) * HD) : make_float2(0.f, 0.f);
    // K rows: 4 lanes per position; lane j reads the float4s 4j + 16i (i < 8)
    const int pp = lane >> 2, j = lane & 3, t = tw + pp;
    float4 kv[8];
    {
        const float4 *k4 = (const float4 *)(K + ((size_t)g * ctx + (t < t1 ? t : t0)) * HD);
#pragma unroll
        for (int i = 0; i < 8; i++) kv[i] = k4[4 * i + j];
    }
    for (int i = threadIdx.x; i < G * HD; i += 256) qs[i / HD][i % HD] = q[(size_t)g * G * HD + i];
    __syncthreads();
    const float inv = 1.0f / sqrtf((float)HD);
    {
        float acc[G];
#pragma unroll
        for (int hh = 0; hh < G; hh++) acc[hh] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int d = 16 * i + 4 * j;
#pragma unroll
            for (int hh = 0; hh < G; hh++) {
                acc[hh] = fmaf(kv[i].x, qs[hh][d], acc[hh]);
                acc[hh] = fmaf(kv[i].y, qs[hh][d + 1], acc[hh]);
                acc[hh] = fmaf(kv[i].z, qs[hh][d + 2], acc[hh]);
                acc[hh] = fmaf(kv[i].w, qs[hh][d + 3], acc[hh]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
            float v = acc[hh];
            v += dpp_f<0xB1>(v);
            v += dpp_f<0x4E>(v);
            if (j == 0 && t < t1) sc[hh][t - t0] = v * inv;
        }
    }
    __syncthreads();
    // softmax statistics of the chunk, one wavefront per head
    for (int hh = wave; hh < G; hh += NW) {
        const float s = lane < n ? sc[hh][lane] : -INFINITY;
        const float m = wave_max(s);
        const float p = lane < n ? expf(s - m) : 0.0f;
        const float l = seg_sum<64>(p);
        sc[hh][lane] = p;
        if (lane == 0) {
            float *o = part + ((size_t)(g * G + hh) * chunks + c) * (HD + 2);
            o[0] = m;
            o[1] = l;
        }
    }
    __syncthreads();
    // acc[h] over this wavefront's positions, then across the wavefronts
#pragma unroll
    for (int hh = 0; hh < G; hh++) {
        float2 a = make_float2(0.f, 0.f);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const float pk = tw + k < t1 ? sc[hh][16 * wave + k] : 0.0f;
            a.x = fmaf(pk, vr[k].x, a.x);
            a.y = fmaf(pk, vr[k].y, a.y);
        }
        accs[wave][hh][lane] = a;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < G * HD / 2; e += 256) {
        const int hh = e / (HD / 2), dl = e % (HD / 2);
        float2 a = accs[0][hh][dl];
#pragma unroll
        for (int w = 1; w < NW; w++) {
            a.x += accs[w][hh][dl].x;
            a.y += accs[w][hh][dl].y;
        }
        float *o = part + ((size_t)(g * G + hh) * chunks + c) * (HD + 2) + 2;
        *(float2 *)(o + 2 * dl) = a;
    }
}

// grid n_heads, block 8 * HD: out[h*HD + d] = sum_c e^{m_c - M} acc_c[d] /
// sum_c e^{m_c - M} l_c.  The 8 thread groups split the chunks (c = g mod 8)
// so a head's partials are read with up to 16 loads in flight per thread.
constexpr int CMB_G = 8;

__global__ void __launch_bounds__(CMB_G * ATT_HD) k_attn_combine(const float *__restrict__ part, int chunks,
                                                                  float *__restrict__ out)
{
    constexpr int HD = ATT_HD, NT = CMB_G * HD;
    __shared__ float wsh[1024];
    __shared__ float red[NT / 64];
    __shared__ float accs[CMB_G][HD];
    const int h = blockIdx.x, tid = threadIdx.x, grp = tid / HD, d = tid % HD, lane = tid & 63, wave = tid >> 6;
    const float *ph = part + (size_t)h * chunks * (HD + 2);
    float m = -INFINITY;
    for (int c = tid; c < chunks; c += NT) m = fmaxf(m, ph[(size_t)c * (HD + 2)]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    float M = red[0];
    for (int w = 1; w < NT / 64; w++) M = fmaxf(M, red[w]);
    __syncthreads();
    float l = 0.0f;
    for (int c = tid; c < chunks; c += NT) {
        const float w = expf(ph[(size_t)c * (HD + 2)] - M);
        wsh[c] = w;
        l += w * ph[(size_t)c * (HD + 2) + 1];
    }
    l = seg_sum<64>(l);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    float L = 0.0f;
    for (int w = 0; w < NT / 64; w++) L += red[w];
    float a = 0.0f;
    for (int c0 = grp; c0 < chunks; c0 += CMB_G * 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int c = c0 + CMB_G * k;
            v[k] = c < chunks ? ph[(size_t)c * (HD + 2) + 2 + d] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int c = c0 + CMB_G * k;
            if (c < chunks) a = fmaf(wsh[c], v[k], a);
        }
    }
    accs[grp][d] = a;
    __syncthreads();
    if (grp == 0) {
        float t = 0.0f;
#pragma unroll
        for (int g = 0; g < CMB_G; g++) t += accs[g][d];
        out[(size_t)h * HD + d] = L > 0.0f ? t / L : 0.0f;
    }
}

int launch_attention(soso_hip *h, const float *q, const float *K, const float *V, int n_heads, int n_kv_heads,
                     int head_dim, int ctx, int T, float *part, float *out)
{
    if (head_dim != ATT_HD || n_kv_heads <= 0 || n_heads % n_kv_heads || T <= 0)
        return set_err(h, SOSO_HIP_DECLINED, "attention: head shape not handled here");
    const int G = n_heads / n_kv_heads;
    const int chunks = (T + ATT_CHUNK - 1) / ATT_CHUNK;
    if (chunks > 1024) return set_err(h, SOSO_HIP_DECLINED, "attention: context longer than 65536");
    const dim3 grid((unsigned)n_kv_heads, (unsigned)chunks);
    switch (G) {
    case 1: k_attn_split<1><<<grid, 256, 0, h->stream>>>(q, K, V, ctx, T, chunks, part); break;
    case 2: k_attn_split<2><<<grid, 256, 0, h->stream>>>(q, K, V, ctx, T, chunks, part); break;
    case 4: k_attn_split<4><<<grid, 256, 0, h->stream>>>(q, K, V, ctx, T, chunks, part); break;
    case 8: k_attn_split<8><<<grid, 256, 0, h->stream>>>(q, K, V, ctx, T, chunks, part); break;
    default: return set_err(h, SOSO_HIP_DECLINED, "attention: GQA group size not handled here");
    }
    int rc = hip_check(h, hipGetLastError(), "attention split launch");
    if (rc != SOSO_HIP_OK) return rc;
    k_attn_combine<<<(unsigned)n_heads, CMB_G * ATT_HD, 0, h->stream>>>(part, chunks, out);
    return hip_check(h, hipGetLastError(), "attention combine launch");
}

// ---------------------------------------------------------------------------
// The decode step
// ---------------------------------------------------------------------------
int decode_step(soso_hip *h, DecodeModel &m, const float *x, uint32_t pos, float *logits, uint32_t *token)
{
    const int q_dim = (int)(m.n_heads * m.head_dim), kv_dim = (int)(m.n_kv_heads * m.head_dim);
    if (pos >= m.ctx_max) return set_err(h, SOSO_HIP_ERR_ARG, "decode: position beyond the KV capacity");
    float *hid = m.hid, *qb = m.qbuf, *att = m.att, *act = m.act, *lg = logits ? logits : m.logits;
    int rc = hip_check(h, hipMemcpyAsync(hid, x, m.hidden * 4, hipMemcpyDeviceToDevice, h->stream), "embed copy");
    for (size_t l = 0; l < m.n_layers && rc == SOSO_HIP_OK; l++) {
        const DecodeLayer &L = m.layers[l];
        float *K = m.kcache + l * m.ctx_max * kv_dim, *V = m.vcache + l * m.ctx_max * kv_dim;
        MvIn in;
        in.x = hid;
        in.norm_w = L.attn_norm;
        in.eps = m.eps;
        MvEpi ep;
        ep.k_out = K;
        ep.v_out = V;
        ep.kv_stride = m.ctx_max * m.head_dim;
        ep.q_dim = q_dim;
        ep.kv_dim = kv_dim;
        ep.head_dim = (int)m.head_dim;
        ep.pos = (int)pos;
        ep.theta = m.theta;
        rc = launch_matvec_ex(h, *L.qkv, in, qb, ep, XS_RMSNORM, EPI_QKV);
        if (rc == SOSO_HIP_OK)
            rc = launch_attention(h, qb, K, V, (int)m.n_heads, (int)m.n_kv_heads, (int)m.head_dim, (int)m.ctx_max,
                                  (int)pos + 1, m.part, att);
        if (rc == SOSO_HIP_OK) {
            MvIn a;
            a.x = att;
            MvEpi r;
            r.res = hid;
            rc = launch_matvec_ex(h, *L.o, a, hid, r, XS_PLAIN, EPI_RESID);
        }
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
            rc = launch_matvec_ex(h, *L.down, a, hid, r, XS_PLAIN, EPI_RESID);
        }
    }
    if (rc == SOSO_HIP_OK) {
        MvIn in;
        in.x = hid;
        in.norm_w = m.out_norm;
        in.eps = m.eps;
        rc = launch_matvec_ex(h, *m.head, in, lg, MvEpi(), XS_RMSNORM, EPI_STORE);
    }
    if (rc == SOSO_HIP_OK && token) rc = launch_argmax(h, lg, m.vocab, token);
    return rc;
}
