// k_moe.hip -- MoE router + top-k and the expert FFNs of a token block.
//
// Reference: topk_softmax (crates/soso-llm-core/src/gemm.rs:62-91), the CPU
// expert path of moe_expertos_agrupados (crates/soso-llm-core/src/layer.rs:
// 1869-1934) and GpuDispatch::{router_topk, expertos_bloque}
// (crates/soso-llm-core/src/gpu.rs:461-494).
#include "internal.hpp"

#include <vector>

// ---------------------------------------------------------------------------
// Router: logits = W[n_exp x h] . x (f32), softmax, top-k with ties to the
// lowest index, renormalised.  One workgroup per token.  exp() runs per
// element in parallel; the softmax sum and the top-k weight sum are taken
// sequentially in index / rank order as gemm.rs:62-91 does.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_router(const float *__restrict__ W, const float *__restrict__ xs,
                                                 float *__restrict__ logits, int32_t *__restrict__ idx,
                                                 float *__restrict__ wgt, int hdim, int n_exp, int top_k)
{
    extern __shared__ float p[]; // n_exp
    __shared__ float red[4];
    __shared__ int redi[4];
    __shared__ float sum_s;
    const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const float4 *x4 = (const float4 *)(xs + (size_t)t * hdim);
    for (int e = wave; e < n_exp; e += nw) {
        const float4 *w4 = (const float4 *)(W + (size_t)e * hdim);
        float a0 = 0.f, a1 = 0.f;
        for (int i = lane; i < (hdim >> 2); i += 64) {
            const float4 w = w4[i], v = x4[i];
            a0 = fmaf(w.x, v.x, a0);
            a1 = fmaf(w.y, v.y, a1);
            a0 = fmaf(w.z, v.z, a0);
            a1 = fmaf(w.w, v.w, a1);
        }
        const float s = seg_sum<64>(a0 + a1);
        if (lane == 0) p[e] = s;
    }
    __syncthreads();
    if (logits)
        for (int e = threadIdx.x; e < n_exp; e += blockDim.x) logits[(size_t)t * n_exp + e] = p[e];
    // max (f32::max ignores NaN like fmaxf)
    float m = -INFINITY;
    for (int e = threadIdx.x; e < n_exp; e += blockDim.x) m = fmaxf(m, p[e]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < nw; w++) m = fmaxf(m, red[w]);
    __syncthreads();
    for (int e = threadIdx.x; e < n_exp; e += blockDim.x) p[e] = expf(p[e] - m);
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.f;
        for (int e = 0; e < n_exp; e++) s += p[e];
        sum_s = s;
    }
    __syncthreads();
    const float s = sum_s;
    if (s > 0.f)
        for (int e = threadIdx.x; e < n_exp; e += blockDim.x) p[e] = p[e] / s;
    __syncthreads();
    // top-k: stable descending order == repeatedly take the largest weight,
    // lowest index among equals (gemm.rs:80-82).
    float tot = 0.f;
    for (int j = 0; j < top_k; j++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int e = threadIdx.x; e < n_exp; e += blockDim.x) {
            const float v = p[e];
            if (v > bv || (v == bv && e < bi)) {
                bv = v;
                bi = e;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            red[wave] = bv;
            redi[wave] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float v = red[0];
            int i = redi[0];
            for (int w = 1; w < nw; w++)
                if (red[w] > v || (red[w] == v && redi[w] < i)) {
                    v = red[w];
                    i = redi[w];
                }
            idx[(size_t)t * top_k + j] = i;
            wgt[(size_t)t * top_k + j] = v;
            tot += v; // sequential, rank order
            p[i] = -INFINITY;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0 && tot > 0.f)
        for (int j = 0; j < top_k; j++) wgt[(size_t)t * top_k + j] /= tot;
}

int launch_router_topk(soso_hip *h, const float *w, const float *x, size_t n, size_t hdim, size_t n_exp, size_t top_k,
                       int32_t *idx, float *wgt, float *logits)
{
    k_router<<<(unsigned)n, 256, n_exp * sizeof(float), h->stream>>>(w, x, logits, idx, wgt, (int)hdim, (int)n_exp,
                                                                     (int)top_k);
    return hip_check(h, hipGetLastError(), "router launch");
}

// ---------------------------------------------------------------------------
// Experts of a token block (first version: per-token matvec launches).
// act = silu(gate) * up (gemm.rs:210-226), y_slot = down . act, and
// sum[t] = sum_j wgt[t,j] * y_slot[t*top_k + j] over resolved slots, ranking
// order from 0 (layer.rs:1914-1924).
// ---------------------------------------------------------------------------
__global__ void k_swiglu(const float *__restrict__ g, float *__restrict__ u, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = g[i];
        u[i] = v / (1.0f + expf(-v)) * u[i];
    }
}

__global__ void k_combine(const float *__restrict__ ys, const uint8_t *__restrict__ resolved,
                          const float *__restrict__ wgt, float *__restrict__ sum, int n, int hdim, int top_k)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (i >= hdim || t >= n) return;
    float acc = 0.f;
    for (int j = 0; j < top_k; j++) {
        const int slot = t * top_k + j;
        if (resolved[slot]) acc += ys[(size_t)slot * hdim + i] * wgt[slot];
    }
    sum[(size_t)t * hdim + i] = acc;
}

int launch_experts(soso_hip *h, const float *xs, size_t n, size_t hdim, size_t ffn, size_t top_k, const float *wgt,
                   const Weight *const *wts, const soso_hip_expert *exps, const uint8_t *ok, size_t n_exps, float *sum)
{
    const size_t slots = n * top_k;
    float *ys = (float *)scratch_get(h, 6, slots * hdim * 4);
    float *gu = (float *)scratch_get(h, 7, 2 * ffn * 4 + slots + 16);
    if (!ys || !gu) return set_err(h, SOSO_HIP_ERR_NOMEM, "experts: scratch");
    float *g = gu, *u = gu + ffn;
    uint8_t *res_d = (uint8_t *)(gu + 2 * ffn);
    std::vector<uint8_t> resolved(slots, 0);
    for (size_t e = 0; e < n_exps; e++) {
        if (!ok[e]) continue;
        for (size_t k = 0; k < exps[e].n_tokens; k++) {
            const size_t t = exps[e].tokens[k], slot = exps[e].targets[k];
            int rc = launch_matvec(h, *wts[3 * e], xs + t * hdim, g, 1);
            if (rc == SOSO_HIP_OK) rc = launch_matvec(h, *wts[3 * e + 1], xs + t * hdim, u, 1);
            if (rc != SOSO_HIP_OK) return rc;
            k_swiglu<<<(unsigned)((ffn + 255) / 256), 256, 0, h->stream>>>(g, u, (int)ffn);
            rc = launch_matvec(h, *wts[3 * e + 2], u, ys + slot * hdim, 1);
            if (rc != SOSO_HIP_OK) return rc;
            resolved[slot] = 1;
        }
    }
    int rc = hip_check(h, hipMemcpyAsync(res_d, resolved.data(), slots, hipMemcpyHostToDevice, h->stream), "slots");
    if (rc != SOSO_HIP_OK) return rc;
    hipStreamSynchronize(h->stream); // `resolved` is a host temporary
    dim3 grid((unsigned)((hdim + 255) / 256), (unsigned)n);
    k_combine<<<grid, 256, 0, h->stream>>>(ys, res_d, wgt, sum, (int)n, (int)hdim, (int)top_k);
    return hip_check(h, hipGetLastError(), "combine launch");
}
