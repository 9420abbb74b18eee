// k_moe.hip -- MoE decode: router + top-k, grouped expert FFNs, combine.
//
// Reference: topk_softmax (crates/soso-llm-core/src/gemm.rs:62-91), the CPU
// expert path of moe_expertos_agrupados (crates/soso-llm-core/src/layer.rs:
// 1869-1934), bloque35::moe_bloque's per-expert token grouping
// (crates/soso-llm-core/src/bloque35.rs:684-1016) and GpuDispatch::
// {router_topk, expertos_bloque} (crates/soso-llm-core/src/gpu.rs:461-494).
//
// Layout of one MoE FFN on the device:
//   k_moe_route   logits = W_router . x (f32) for every (token, expert); the
//                 last workgroup to finish runs softmax + top-k per token and
//                 counting-sorts the n*top_k slots by expert (cnt, offs, list).
//   k_moe_mv      grid (expert, row chunk): every weight row of an expert is
//                 read once from HBM and applied to all the tokens routed to
//                 it (their x staged in LDS).  Gate and up rows are read side
//                 by side and leave as silu(gate.x) * up.x; down rows leave as
//                 y[slot].  Experts nobody chose exit at once.
//   k_moe_combine out[t] = sum_j wgt[t,j] * y[t*top_k + j], j in ranking order.
// Slot s = t * top_k + j is token t's j-th ranked expert ("destinos" in
// ExpertoBloque, gpu.rs:176-186).
#include "mv_core.hpp"

#include <vector>

// ---------------------------------------------------------------------------
// Router
// ---------------------------------------------------------------------------
// Softmax and ranking of one token's logits by one wavefront (gemm.rs:62-91):
// max-shifted expf, normalised, then the top_k largest probabilities with
// ties to the lowest index (a stable descending sort), renormalised by their
// sum taken in rank order.
__device__ void topk_wave(const float *__restrict__ lg, int n_exp, int top_k, int32_t *__restrict__ idx,
                          float *__restrict__ wgt, float *sel)
{
    const int lane = threadIdx.x & 63;
    float m = -INFINITY;
    for (int e = lane; e < n_exp; e += 64) m = fmaxf(m, lg[e]);
    m = wave_max(m);
    float s = 0.0f;
    for (int e = lane; e < n_exp; e += 64) s += expf(lg[e] - m);
    s = seg_sum<64>(s);
    // each lane keeps the probabilities of experts lane, lane+64, ... (n_exp <= 256)
    float p[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int e = lane + 64 * q;
        p[q] = e < n_exp ? expf(lg[e] - m) / s : -INFINITY;
    }
    for (int j = 0; j < top_k; j++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = lane + 64 * q;
            if (p[q] > bv || (p[q] == bv && e < bi)) {
                bv = p[q];
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
        // NaN probabilities are never chosen; should fewer than top_k experts
        // remain, the slot points at expert 0 with weight 0 (indices stay valid)
        if (bi >= n_exp) {
            bi = 0;
            bv = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (lane + 64 * q == bi) p[q] = -INFINITY;
        if (lane == 0) {
            idx[j] = bi;
            sel[j] = bv;
        }
    }
    if (lane == 0) {
        float tot = 0.0f;
        for (int j = 0; j < top_k; j++) tot += sel[j];
        for (int j = 0; j < top_k; j++) wgt[j] = tot > 0.0f ? sel[j] / tot : sel[j];
    }
}

// grid: ceil(n_exp / waves) workgroups; wave w of workgroup b owns expert
// b*waves + w.  `ticket` is zero between launches (the last workgroup resets it).
__global__ void __launch_bounds__(512) k_moe_route(const float *__restrict__ W, const float *__restrict__ xs, int n,
                                                    int hdim, int n_exp, int top_k, float *__restrict__ logits,
                                                    int32_t *__restrict__ idx, float *__restrict__ wgt,
                                                    int *__restrict__ cnt, int *__restrict__ offs,
                                                    int *__restrict__ list, unsigned *__restrict__ ticket)
{
    __shared__ int last;
    __shared__ float sel[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int e = blockIdx.x * nw + wave;
    if (e < n_exp) {
        const float4 *w4 = (const float4 *)(W + (size_t)e * hdim);
        for (int t = 0; t < n; t++) {
            const float4 *x4 = (const float4 *)(xs + (size_t)t * hdim);
            float a0 = 0.f, a1 = 0.f;
            for (int i = lane; i < (hdim >> 2); i += 64) {
                const float4 w = w4[i], v = x4[i];
                a0 = fmaf(w.x, v.x, a0);
                a1 = fmaf(w.y, v.y, a1);
                a0 = fmaf(w.z, v.z, a0);
                a1 = fmaf(w.w, v.w, a1);
            }
            const float s = seg_sum<64>(a0 + a1);
            if (lane == 0) logits[(size_t)t * n_exp + e] = s;
        }
    }
    // the last workgroup to finish ranks the experts of every token
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(ticket, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int t = wave; t < n; t += nw)
        topk_wave(logits + (size_t)t * n_exp, n_exp, top_k, idx + (size_t)t * top_k, wgt + (size_t)t * top_k,
                  sel[wave]);
    __syncthreads();
    if (threadIdx.x == 0) {
        // counting sort of the slots by expert, slot order kept inside an expert
        for (int x = 0; x < n_exp; x++) cnt[x] = 0;
        for (int s = 0; s < n * top_k; s++) cnt[min(max(idx[s], 0), n_exp - 1)]++;
        int o = 0;
        for (int x = 0; x < n_exp; x++) {
            offs[x] = o;
            o += cnt[x];
        }
        offs[n_exp] = o;
        for (int x = 0; x < n_exp; x++) cnt[x] = 0;
        for (int s = 0; s < n * top_k; s++) {
            const int x = min(max(idx[s], 0), n_exp - 1);
            list[offs[x] + cnt[x]++] = s;
        }
        *ticket = 0u;
    }
}

// ---------------------------------------------------------------------------
// Grouped expert matvecs
// ---------------------------------------------------------------------------
constexpr int MOE_TCH = 8; // tokens staged per round

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// grid (experts, row chunks), 512 threads.  Expert e's slots are
// list[offs[e] .. offs[e] + cnt[e]); slot s reads x = xs + (s / xdiv) * cols
// and writes out[s * rows + r].  NMAT == 2: tabA = gate, tabB = up, output
// silu(gate.x) * up.x (swiglu, gemm.rs:210-226); NMAT == 1: tabA = down.
template <int FMT, int LPR, int NMAT>
__global__ void __launch_bounds__(512) k_moe_mv(const uint8_t *const *__restrict__ tabA,
                                                const uint8_t *const *__restrict__ tabB, size_t stride, int rows,
                                                int cols, int rows_per_wg, const float *__restrict__ xs, int xdiv,
                                                const int *__restrict__ cnt, const int *__restrict__ offs,
                                                const int *__restrict__ list, float *__restrict__ out)
{
    constexpr int RW = 64 / LPR;
    const int e = blockIdx.x;
    const int ne = cnt[e];
    const int r0 = blockIdx.y * rows_per_wg, r1 = min(rows, r0 + rows_per_wg);
    if (ne == 0 || r0 >= r1) return; // uniform over the workgroup
    extern __shared__ uint4 smem[];
    __shared__ int slot_s[MOE_TCH];
    const size_t tok_bytes = (stage_lds_bytes((size_t)cols) + 15) & ~(size_t)15;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nw = blockDim.x >> 6;
    const int U = cols >> 6;
    const int ul = lane & (LPR - 1), slot = lane / LPR;
    const bool uact = ul < U;
    const int u = uact ? ul : 0;
    UConst c;
    unit_setup_w<FMT>(u, c);
    const LaneOff L = lane_offsets<FMT>(cols, u, c);
    const rsrc_t rA = make_rsrc(tabA[e], (uint32_t)((size_t)rows * stride));
    const rsrc_t rB = make_rsrc(NMAT == 2 ? tabB[e] : tabA[e], (uint32_t)((size_t)rows * stride));
    const int np = (r1 - r0 + RW - 1) / RW;
    const int base = offs[e];

    for (int t0 = 0; t0 < ne; t0 += MOE_TCH) {
        const int nt = min(MOE_TCH, ne - t0);
        if (threadIdx.x < nt) slot_s[threadIdx.x] = list[base + t0 + threadIdx.x];
        __syncthreads();
        for (int j = 0; j < nt; j++) {
            uint8_t *reg = (uint8_t *)smem + j * tok_bytes;
            uint32_t *xd = (uint32_t *)reg;
            float *s16 = (float *)(xd + (cols >> 2) * XDIG);
            int *kx = (int *)(s16 + (cols >> 4));
            stage_x<FMT>(xs + (size_t)(slot_s[j] / xdiv) * cols, cols, xd, s16, kx);
        }
        for (int p = wave; p < np; p += nw) {
            const int r = r0 + p * RW + slot;
            const uint32_t rb = (uact && r < r1) ? (uint32_t)((size_t)r * stride) : 0x80000000u;
            WRow<FMT> wa, wb;
            load_row<FMT>(rA, rb, cols, L, wa);
            if constexpr (NMAT == 2) load_row<FMT>(rB, rb, cols, L, wb);
            for (int j = 0; j < nt; j++) {
                const uint8_t *reg = (const uint8_t *)smem + j * tok_bytes;
                const uint32_t *xd = (const uint32_t *)reg;
                const float *s16 = (const float *)(xd + (cols >> 2) * XDIG);
                const int *kx = (const int *)(s16 + (cols >> 4));
                XReg xv;
                UConst cj = c;
                unit_setup_x<FMT>(xd, s16, kx, u, U, xv, cj);
                float pa = unit_dot<FMT>(wa, xv, cj);
                pa = seg_sum_dpp<LPR>(uact ? pa : 0.0f);
                float v = pa;
                if constexpr (NMAT == 2) {
                    float pb = unit_dot<FMT>(wb, xv, cj);
                    pb = seg_sum_dpp<LPR>(uact ? pb : 0.0f);
                    v = silu(pa) * pb;
                }
                if (ul == LPR - 1 && r < r1) out[(size_t)slot_s[j] * rows + r] = v;
            }
        }
        __syncthreads(); // the next round restages LDS
    }
}

// out[t * hdim + i] = sum_j wgt[t*k + j] * y[(t*k + j) * hdim + i] over the
// slots marked in `use` (all when null), j in ranking order (layer.rs:1914-1924).
__global__ void k_moe_combine(const float *__restrict__ y, const float *__restrict__ wgt,
                              const uint8_t *__restrict__ use, int n, int hdim, int top_k, float *__restrict__ out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (i >= hdim || t >= n) return;
    float acc = 0.0f;
    for (int j = 0; j < top_k; j++) {
        const int s = t * top_k + j;
        if (!use || use[s]) acc = fmaf(y[(size_t)s * hdim + i], wgt[s], acc);
    }
    out[(size_t)t * hdim + i] = acc;
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
// Scratch slots 8..11 belong to the MoE path.
bool moe_scratch(soso_hip *h, size_t n, size_t n_groups, size_t top_k, size_t hdim, size_t ffn, MoeScratch &s)
{
    const size_t slots = n * top_k;
    char *f = (char *)scratch_get(h, 8, (n * (n_groups > 0 ? n_groups : 1) + 2 * slots) * 4);
    int *ints = (int *)scratch_get(h, 9, (2 * n_groups + 1 + slots) * 4);
    float *big = (float *)scratch_get(h, 10, slots * (ffn + hdim) * 4);
    if (!f || !ints || !big) return false;
    s.logits = (float *)f;
    s.idx = (int32_t *)(s.logits + n * n_groups);
    s.wgt = (float *)(s.idx + slots);
    s.cnt = ints;
    s.offs = ints + n_groups;
    s.list = ints + 2 * n_groups + 1;
    s.act = big;
    s.ydown = big + slots * ffn;
    return true;
}

int launch_moe_route(soso_hip *h, const float *w, const float *x, size_t n, size_t hdim, size_t n_exp, size_t top_k,
                     const MoeScratch &s)
{
    const unsigned grid = (unsigned)((n_exp + 7) / 8);
    k_moe_route<<<grid, 512, 0, h->stream>>>(w, x, (int)n, (int)hdim, (int)n_exp, (int)top_k, s.logits, s.idx, s.wgt,
                                              s.cnt, s.offs, s.list, h->ticket);
    return hip_check(h, hipGetLastError(), "moe route launch");
}

int launch_router_topk(soso_hip *h, const float *w, const float *x, size_t n, size_t hdim, size_t n_exp, size_t top_k,
                       int32_t *idx, float *wgt, float *logits)
{
    MoeScratch s;
    if (!moe_scratch(h, n, n_exp, top_k, 0, 0, s)) return set_err(h, SOSO_HIP_ERR_NOMEM, "router: scratch");
    s.idx = idx;
    s.wgt = wgt;
    s.logits = logits;
    return launch_moe_route(h, w, x, n, hdim, n_exp, top_k, s);
}

template <int FMT, int NMAT>
static void moe_mv_fmt(soso_hip *h, dim3 grid, size_t lds, int lpr, const uint8_t *const *A, const uint8_t *const *B,
                       size_t stride, int rows, int cols, int rpw, const float *xs, int xdiv, const MoeScratch &s,
                       float *out)
{
#define MOE_CASE(LP)                                                                                                   \
    case LP:                                                                                                           \
        k_moe_mv<FMT, LP, NMAT><<<grid, 512, lds, h->stream>>>(A, B, stride, rows, cols, rpw, xs, xdiv, s.cnt, s.offs, \
                                                                s.list, out);                                          \
        break;
    switch (lpr) {
        MOE_CASE(1) MOE_CASE(2) MOE_CASE(4) MOE_CASE(8) MOE_CASE(16) MOE_CASE(32) MOE_CASE(64)
    }
#undef MOE_CASE
}

// One grouped matvec over `n_groups` experts (pointer tables on the device).
static int launch_moe_mv(soso_hip *h, uint8_t dtype, int nmat, const uint8_t *const *A, const uint8_t *const *B,
                         size_t rows, size_t cols, size_t n_groups, size_t active_hint, const float *xs, int xdiv,
                         const MoeScratch &s, float *out)
{
    const int U = (int)(cols / 64);
    if (U < 1 || U > 64 || !packed_shape_ok(dtype, rows, cols))
        return set_err(h, SOSO_HIP_DECLINED, "moe: expert shape not handled here");
    const int lpr = U <= 1 ? 1 : U <= 2 ? 2 : U <= 4 ? 4 : U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
    const int rw = 64 / lpr;
    const size_t tok_bytes = (stage_lds_bytes(cols) + 15) & ~(size_t)15;
    const size_t lds = tok_bytes * MOE_TCH;
    if (lds > h->max_lds) return set_err(h, SOSO_HIP_DECLINED, "moe: x does not fit in LDS");
    // about two workgroups per CU over the experts expected to be active
    const size_t act = std::max<size_t>(1, std::min(active_hint, n_groups));
    size_t chunks = (2 * (size_t)h->num_cu + act - 1) / act;
    int rpw = (int)((rows + chunks - 1) / chunks);
    rpw = std::max(rpw, rw * 8);
    rpw = (rpw + rw - 1) / rw * rw;
    chunks = (rows + rpw - 1) / rpw;
    const dim3 grid((unsigned)n_groups, (unsigned)chunks);
    const size_t stride = packed_row_stride(dtype, cols);
    switch (dtype) {
    case SOSO_HIP_DTYPE_Q4_K:
        if (nmat == 2) moe_mv_fmt<FMT_Q4K, 2>(h, grid, lds, lpr, A, B, stride, (int)rows, (int)cols, rpw, xs, xdiv, s, out);
        else moe_mv_fmt<FMT_Q4K, 1>(h, grid, lds, lpr, A, B, stride, (int)rows, (int)cols, rpw, xs, xdiv, s, out);
        break;
    case SOSO_HIP_DTYPE_Q8_0:
        if (nmat == 2) moe_mv_fmt<FMT_Q80, 2>(h, grid, lds, lpr, A, B, stride, (int)rows, (int)cols, rpw, xs, xdiv, s, out);
        else moe_mv_fmt<FMT_Q80, 1>(h, grid, lds, lpr, A, B, stride, (int)rows, (int)cols, rpw, xs, xdiv, s, out);
        break;
    case SOSO_HIP_DTYPE_Q6_K:
        if (nmat == 2) moe_mv_fmt<FMT_Q6K, 2>(h, grid, lds, lpr, A, B, stride, (int)rows, (int)cols, rpw, xs, xdiv, s, out);
        else moe_mv_fmt<FMT_Q6K, 1>(h, grid, lds, lpr, A, B, stride, (int)rows, (int)cols, rpw, xs, xdiv, s, out);
        break;
    default: return set_err(h, SOSO_HIP_DECLINED, "moe: expert dtype not handled here");
    }
    return hip_check(h, hipGetLastError(), "moe mv launch");
}

// gate/up + swiglu, down, combine for the slots grouped in s.cnt/offs/list.
// tab: 3 * n_groups device pointers (gate[], up[], down[]).
int launch_moe_experts(soso_hip *h, const float *xs, size_t n, size_t hdim, size_t ffn, size_t top_k,
                       uint8_t dt_gu, uint8_t dt_down, const uint8_t *const *tab, size_t n_groups, const float *wgt,
                       const uint8_t *use, const MoeScratch &s, float *out)
{
    const size_t active = std::min(n_groups, n * top_k);
    int rc = launch_moe_mv(h, dt_gu, 2, tab, tab + n_groups, ffn, hdim, n_groups, active, xs, (int)top_k, s, s.act);
    if (rc == SOSO_HIP_OK)
        rc = launch_moe_mv(h, dt_down, 1, tab + 2 * n_groups, nullptr, hdim, ffn, n_groups, active, s.act, 1, s, s.ydown);
    if (rc != SOSO_HIP_OK) return rc;
    const dim3 grid((unsigned)((hdim + 255) / 256), (unsigned)n);
    k_moe_combine<<<grid, 256, 0, h->stream>>>(s.ydown, wgt, use, (int)n, (int)hdim, (int)top_k, out);
    return hip_check(h, hipGetLastError(), "moe combine launch");
}
