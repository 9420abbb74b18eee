// k_gdn.hip -- Gated DeltaNet (Qwen3.5) on the device: the recurrence of
// GpuDispatch::gdn_bloque (crates/soso-llm-core/src/gpu.rs:577-599), as
// soso's CPU path computes it (bloque35.rs:372-465; one token of the decode
// layer, arch.rs:586-768, is the same with n = 1).
//
// Two launches per block of n tokens:
//   k_gdn_conv  grid (2 n_k + n_v heads, n tokens), one thread per channel of
//               a head (d = 128): the causal conv over the history window,
//               SiLU, and for q / k heads the l2 normalisation (q also scaled
//               by 1 / sqrt(d)) -> u [n][C], C = 2 n_k d + n_v d
//   k_gdn_rec   one workgroup of 1024 threads per value head: the head's
//               d x d state lives in registers (thread (r, j) holds column j,
//               rows 16 r .. 16 r + 15) for the whole block, read once and
//               written once; per token
//                 delta_j = (v_j - g sum_i S_ij k_i) beta
//                 S_ij   <- g S_ij + k_i delta_j
//                 o_j     = sum_i S_ij q_i
//               then rmsnorm(o) with the ssm_norm weights and o *= silu(z).
// The column sums run as 16-row partial sums per thread, combined over the 8
// row groups through LDS (the CPU sums i in order; the bar is relative L2).
// The next token's q, k, v and z are requested while the current token's
// recurrence runs.
// State traffic per block: 2 * n_v d^2 * 4 bytes (2 MiB each way for 32 heads
// of 128), independent of n.
#include "internal.hpp"

constexpr int GDN_D = 128;             // head dim handled (gdn_bloque: d == 128 only)
constexpr int GDN_RG = 8;              // row groups of the state per workgroup
constexpr int GDN_RPT = GDN_D / GDN_RG; // state rows per thread

__device__ __forceinline__ float gdn_silu(float x) { return x / (1.0f + expf(-x)); }

// Workgroup barrier for LDS only: LDS operations complete, then s_barrier,
// without waiting for outstanding global loads (__syncthreads' fence would
// wait for the next token's q/k/v/z, requested ahead on purpose).  The memory
// clobber keeps the compiler from moving memory operations across it.
__device__ __forceinline__ void gdn_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// sum over the 128 threads of a two-wavefront workgroup, returned to all
__device__ __forceinline__ float gdn_sum128(float v, float *red)
{
    v = seg_sum_dpp<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 63) red[wave] = v;
    __syncthreads();
    const float s = red[0] + red[1];
    __syncthreads();
    return s;
}

__global__ void __launch_bounds__(GDN_D) k_gdn_conv(const float *__restrict__ hist, const float *__restrict__ conv,
                                                    int C, int n_k, int kernel, float eps, float *__restrict__ u)
{
    __shared__ float red[2];
    const int hh = blockIdx.x, t = blockIdx.y, ch = hh * GDN_D + (int)threadIdx.x;
    const int prev = kernel - 1;
    float acc = 0.0f;
    for (int k = 0; k < prev; k++) acc = __fadd_rn(acc, __fmul_rn(conv[(size_t)ch * kernel + k], hist[(size_t)(t + k) * C + ch]));
    acc = __fadd_rn(acc, __fmul_rn(conv[(size_t)ch * kernel + prev], hist[(size_t)(t + prev) * C + ch]));
    float x = gdn_silu(acc);
    if (hh < 2 * n_k) { // block-uniform
        const float ss = gdn_sum128(x * x, red);
        x *= 1.0f / sqrtf(ss + eps);
        if (hh < n_k) x *= 1.0f / sqrtf((float)GDN_D);
    }
    u[(size_t)t * C + ch] = x;
}

__global__ void __launch_bounds__(GDN_D * GDN_RG) k_gdn_rec(const float *__restrict__ u, const float *__restrict__ z,
                                                           const float *__restrict__ decay,
                                                           const float *__restrict__ beta,
                                                           const float *__restrict__ norm, float *__restrict__ state,
                                                           float *__restrict__ out, int n, int n_k, int n_v, float eps)
{
    constexpr int D = GDN_D;
    __shared__ float qs[D], ks[D], vs[D], zs[D], dl[D];
    __shared__ float part[GDN_RG][D];
    __shared__ float red[2];
    const int vh = blockIdx.x, kh = vh % n_k, tid = threadIdx.x;
    const int j = tid & (D - 1), r = tid >> 7;
    const int qk = n_k * D, C = 2 * qk + n_v * D, vd = n_v * D;
    float *st = state + (size_t)vh * D * D;
    float S[GDN_RPT];
#pragma unroll
    for (int ii = 0; ii < GDN_RPT; ii++) S[ii] = st[(size_t)(r * GDN_RPT + ii) * D + j];
    // threads 0 .. 127 carry one token's q, k, v, z ahead of the recurrence
    float nq = 0.0f, nk = 0.0f, nv = 0.0f, nz = 0.0f;
    auto fetch = [&](int t) {
        if (tid < D) {
            const float *ut = u + (size_t)t * C;
            nq = ut[kh * D + tid];
            nk = ut[qk + kh * D + tid];
            nv = ut[2 * qk + vh * D + tid];
            nz = z[(size_t)t * vd + vh * D + tid];
        }
    };
    fetch(0);
    for (int t = 0; t < n; t++) {
        if (tid < D) {
            qs[tid] = nq;
            ks[tid] = nk;
            vs[tid] = nv;
            zs[tid] = nz;
        }
        const float g = decay[(size_t)t * n_v + vh], b = beta[(size_t)t * n_v + vh];
        gdn_lds_barrier();
        if (t + 1 < n) fetch(t + 1); // in flight during this token's recurrence
        // delta_j = (v_j - g sum_i S_ij k_i) beta
        float p = 0.0f;
#pragma unroll
        for (int ii = 0; ii < GDN_RPT; ii++) p = __fadd_rn(p, __fmul_rn(S[ii], ks[r * GDN_RPT + ii]));
        part[r][j] = p;
        gdn_lds_barrier();
        if (tid < D) {
            float s = part[0][j];
#pragma unroll
            for (int q = 1; q < GDN_RG; q++) s = __fadd_rn(s, part[q][j]);
            dl[j] = __fmul_rn(__fsub_rn(vs[j], __fmul_rn(g, s)), b);
        }
        gdn_lds_barrier();
        // S_ij <- g S_ij + k_i delta_j;  o_j = sum_i S_ij q_i (updated state)
        const float dj = dl[j];
        p = 0.0f;
#pragma unroll
        for (int ii = 0; ii < GDN_RPT; ii++) {
            const int i = r * GDN_RPT + ii;
            S[ii] = __fadd_rn(__fmul_rn(g, S[ii]), __fmul_rn(ks[i], dj));
            p = __fadd_rn(p, __fmul_rn(S[ii], qs[i]));
        }
        part[r][j] = p;
        gdn_lds_barrier();
        // o_j in threads 0 .. 127 (wavefronts 0 and 1); rmsnorm over the head
        // (gemm.rs:93-100), then the SiLU gate
        float o = 0.0f;
        if (tid < D) {
            o = part[0][j];
#pragma unroll
            for (int q = 1; q < GDN_RG; q++) o = __fadd_rn(o, part[q][j]);
        }
        const float ws = seg_sum_dpp<64>(tid < D ? o * o : 0.0f);
        if ((tid & 63) == 63 && tid < D) red[tid >> 6] = ws;
        gdn_lds_barrier();
        if (tid < D) {
            const float scale = 1.0f / sqrtf((red[0] + red[1]) / (float)D + eps);
            o = __fmul_rn(__fmul_rn(o, scale), norm[j]);
            out[(size_t)t * vd + vh * D + j] = __fmul_rn(o, gdn_silu(zs[j]));
        }
        gdn_lds_barrier(); // qs / ks / vs / zs / part / red reused by the next token
    }
#pragma unroll
    for (int ii = 0; ii < GDN_RPT; ii++) st[(size_t)(r * GDN_RPT + ii) * D + j] = S[ii];
}

const char *gdn_unsupported(size_t n, size_t n_k, size_t n_v, size_t d, size_t kernel)
{
    if (d != GDN_D) return "gdn: head dim must be 128";
    if (n == 0 || n_k == 0 || n_v == 0 || kernel == 0 || kernel > 16) return "gdn: empty block or kernel outside 1..16";
    if (n_v > 65535 || n_k > 65535 || n > 65535) return "gdn: too many heads or tokens (grid limits)";
    return nullptr;
}

int launch_gdn_block(soso_hip *h, const float *hist, const float *conv, const float *z, const float *decay,
                     const float *beta, const float *norm, float *state, float *out, float *u, int n, int n_k,
                     int n_v, int kernel, float eps)
{
    const int C = 2 * n_k * GDN_D + n_v * GDN_D;
    k_gdn_conv<<<dim3((unsigned)(2 * n_k + n_v), (unsigned)n), GDN_D, 0, h->stream>>>(hist, conv, C, n_k, kernel, eps,
                                                                                      u);
    int rc = hip_check(h, hipGetLastError(), "gdn conv launch");
    if (rc != SOSO_HIP_OK) return rc;
    k_gdn_rec<<<(unsigned)n_v, GDN_D * GDN_RG, 0, h->stream>>>(u, z, decay, beta, norm, state, out, n, n_k, n_v, eps);
    return hip_check(h, hipGetLastError(), "gdn recurrence launch");
}
