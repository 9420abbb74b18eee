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
//   k_moe_mv      a persistent grid over (active expert, row chunk) items:
//                 every weight row of an expert is read once from HBM and
//                 applied to all the tokens routed to it (their x staged in
//                 LDS).  Gate and up rows are read side by side and leave as
//                 silu(gate.x) * up.x; down rows leave as y[slot].
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
// b*waves + w.  `ticket` is zero between launches (the last workgroup resets
// it).  The last workgroup also writes the active-expert list act[0..*act_n)
// (experts chosen by at least one slot, ascending) for the grouped kernels.
constexpr int ROUTE_MAX_SLOTS = 4096; // n * top_k handled by the LDS sort

__global__ void __launch_bounds__(512) k_moe_route(const float *__restrict__ W, const float *__restrict__ xs, int n,
                                                    int hdim, int n_exp, int top_k, float *__restrict__ logits,
                                                    int32_t *__restrict__ idx, float *__restrict__ wgt,
                                                    int *__restrict__ cnt, int *__restrict__ offs,
                                                    int *__restrict__ list, int *__restrict__ act,
                                                    int *__restrict__ act_n, unsigned *__restrict__ ticket)
{
    __shared__ int last;
    __shared__ float sel[8][64];
    __shared__ int c_s[256], o_s[257], f_s[256];
    __shared__ int16_t e_s[ROUTE_MAX_SLOTS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int e = blockIdx.x * nw + wave;
    if (e < n_exp) {
        const float4 *w4 = (const float4 *)(W + (size_t)e * hdim);
        const int nv = hdim >> 2;
        for (int t = 0; t < n; t++) {
            const float4 *x4 = (const float4 *)(xs + (size_t)t * hdim);
            float a0 = 0.f, a1 = 0.f;
            for (int i0 = 0; i0 < nv; i0 += 64 * 4) {
                float4 w[4], v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int i = i0 + 64 * q + lane;
                    w[q] = i < nv ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                    v[q] = i < nv ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    a0 = fmaf(w[q].x, v[q].x, a0);
                    a1 = fmaf(w[q].y, v[q].y, a1);
                    a0 = fmaf(w[q].z, v[q].z, a0);
                    a1 = fmaf(w[q].w, v[q].w, a1);
                }
            }
            const float sum = seg_sum<64>(a0 + a1);
            if (lane == 0) logits[(size_t)t * n_exp + e] = sum;
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
    // counting sort of the slots by expert in LDS (a slot's position inside
    // its expert's list does not change any result)
    const int slots = n * top_k;
    for (int x = threadIdx.x; x < n_exp; x += blockDim.x) c_s[x] = f_s[x] = 0;
    __syncthreads();
    for (int sl = threadIdx.x; sl < slots; sl += blockDim.x) {
        const int x = min(max((int)idx[sl], 0), n_exp - 1);
        e_s[sl] = (int16_t)x;
        atomicAdd(&c_s[x], 1);
    }
    __syncthreads();
    if (wave == 0) {
        // exclusive scan over n_exp <= 256 counts, 4 per lane
        int v[4], tot = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int x = 4 * lane + q;
            v[q] = x < n_exp ? c_s[x] : 0;
            tot += v[q];
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o, 64);
            if (lane >= o) incl += y;
        }
        int run = incl - tot;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int x = 4 * lane + q;
            if (x < n_exp) o_s[x] = run;
            run += v[q];
        }
        if (lane == 63) o_s[n_exp] = incl;
    }
    __syncthreads();
    for (int sl = threadIdx.x; sl < slots; sl += blockDim.x) {
        const int x = e_s[sl];
        list[o_s[x] + atomicAdd(&f_s[x], 1)] = sl;
    }
    for (int x = threadIdx.x; x < n_exp; x += blockDim.x) {
        cnt[x] = c_s[x];
        offs[x] = o_s[x];
    }
    if (threadIdx.x == 0) offs[n_exp] = o_s[n_exp];
    if (wave == 0) {
        // active experts in ascending order: compaction by ballot over 64 at a time
        int base = 0;
        for (int x0 = 0; x0 < n_exp; x0 += 64) {
            const int x = x0 + lane;
            const bool on = x < n_exp && c_s[x] > 0;
            const unsigned long long m = __ballot(on);
            if (on) act[base + __popcll(m & ((1ull << lane) - 1ull))] = x;
            base += __popcll(m);
        }
        if (lane == 0) {
            *act_n = base;
            *ticket = 0u;
        }
    }
}

// ---------------------------------------------------------------------------
// Grouped expert matvecs
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Persistent grid of workgroups (512 threads) over the work items (active
// expert a, row chunk c), item w = a * chunks + c, w = blockIdx.x, +gridDim.x.
// A chunk is 2 passes per wavefront (rpw = 2 * 8 * RW rows): both passes'
// weights are requested before the tokens' x is staged, so the HBM reads of
// an item overlap its staging.  Expert e's slots are list[offs[e] ..
// offs[e] + cnt[e]), `tch` at a time; slot s reads x = xs + (s / xdiv) * cols
// and writes out[s * rows + r].  NMAT == 2: tabA = gate, tabB = up, output
// silu(gate.x) * up.x (swiglu, gemm.rs:210-226); NMAT == 1: tabA = down.
template <int FMT, int LPR, int NMAT>
__global__ void __launch_bounds__(512) k_moe_mv(const uint8_t *const *__restrict__ tabA,
                                                const uint8_t *const *__restrict__ tabB, size_t stride, int rows,
                                                int cols, int chunks, const float *__restrict__ xs, int xdiv,
                                                const int *__restrict__ cnt, const int *__restrict__ offs,
                                                const int *__restrict__ list, const int *__restrict__ act,
                                                const int *__restrict__ act_n, int tch, float *__restrict__ out)
{
    constexpr int RW = 64 / LPR, NW = 8, RPW = 2 * NW * RW;
    extern __shared__ uint4 smem[];
    __shared__ int slot_s[64];
    const size_t tok_bytes = (stage_lds_bytes((size_t)cols) + 15) & ~(size_t)15;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int U = cols >> 6;
    const int ul = lane & (LPR - 1), slot = lane / LPR;
    const bool uact = ul < U;
    const int u = uact ? ul : 0;
    UConst c;
    unit_setup_w<FMT>(u, c);
    const LaneOff L = lane_offsets<FMT>(cols, u, c);
    const int items = *act_n * chunks;
    for (int w = blockIdx.x; w < items; w += gridDim.x) {
        const int e = act[w / chunks];
        const int r0 = (w % chunks) * RPW, r1 = min(rows, r0 + RPW);
        const int ne = cnt[e], base = offs[e];
        const rsrc_t rA = make_rsrc(tabA[e], (uint32_t)((size_t)rows * stride));
        const rsrc_t rB = make_rsrc(NMAT == 2 ? tabB[e] : tabA[e], (uint32_t)((size_t)rows * stride));
        // this wavefront's two passes: rows r0 + (wave + 8q) * RW + slot
        int rq[2];
        uint32_t bq[2];
#pragma unroll
        for (int q = 0; q < 2; q++) {
            rq[q] = r0 + (wave + NW * q) * RW + slot;
            bq[q] = (uact && rq[q] < r1) ? (uint32_t)((size_t)rq[q] * stride) : 0x80000000u;
        }
        for (int t0 = 0; t0 < ne; t0 += tch) {
            const int nt = min(tch, ne - t0);
            WRow<FMT> wa[2], wb[2];
#pragma unroll
            for (int q = 0; q < 2; q++) {
                load_row<FMT>(rA, bq[q], cols, L, wa[q]);
                if constexpr (NMAT == 2) load_row<FMT>(rB, bq[q], cols, L, wb[q]);
            }
            __syncthreads(); // the previous round's readers of LDS are done
            if (threadIdx.x < nt) slot_s[threadIdx.x] = list[base + t0 + threadIdx.x];
            __syncthreads();
            for (int j = 0; j < nt; j++) {
                uint32_t *xd = (uint32_t *)((uint8_t *)smem + j * tok_bytes);
                float *s16 = (float *)(xd + (cols >> 2) * XDIG);
                int *kx = (int *)(s16 + (cols >> 4));
                stage_x<FMT>(xs + (size_t)(slot_s[j] / xdiv) * cols, cols, xd, s16, kx);
            }
            for (int j = 0; j < nt; j++) {
                const uint32_t *xd = (const uint32_t *)((const uint8_t *)smem + j * tok_bytes);
                const float *s16 = (const float *)(xd + (cols >> 2) * XDIG);
                const int *kx = (const int *)(s16 + (cols >> 4));
                XReg xv;
                UConst cj = c;
                unit_setup_x<FMT>(xd, s16, kx, u, U, xv, cj);
                const size_t ob = (size_t)slot_s[j] * rows;
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    float pa = unit_dot<FMT>(wa[q], xv, cj);
                    pa = seg_sum_dpp<LPR>(uact ? pa : 0.0f);
                    float v = pa;
                    if constexpr (NMAT == 2) {
                        float pb = unit_dot<FMT>(wb[q], xv, cj);
                        pb = seg_sum_dpp<LPR>(uact ? pb : 0.0f);
                        v = silu(pa) * pb;
                    }
                    if (ul == LPR - 1 && rq[q] < r1) out[ob + rq[q]] = v;
                }
            }
        }
        __syncthreads(); // LDS is restaged by the next item
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
    int *ints = (int *)scratch_get(h, 9, (3 * n_groups + 2 + slots) * 4);
    float *big = (float *)scratch_get(h, 10, slots * (ffn + hdim) * 4);
    if (!f || !ints || !big) return false;
    s.logits = (float *)f;
    s.idx = (int32_t *)(s.logits + n * n_groups);
    s.wgt = (float *)(s.idx + slots);
    s.cnt = ints;
    s.offs = ints + n_groups;
    s.list = ints + 2 * n_groups + 1;
    s.act_list = s.list + slots;
    s.act_n = s.act_list + n_groups;
    s.act = big;
    s.ydown = big + slots * ffn;
    return true;
}

int launch_moe_route(soso_hip *h, const float *w, const float *x, size_t n, size_t hdim, size_t n_exp, size_t top_k,
                     const MoeScratch &s)
{
    const unsigned grid = (unsigned)((n_exp + 7) / 8);
    if (n * top_k > ROUTE_MAX_SLOTS || n_exp > 256) return set_err(h, SOSO_HIP_DECLINED, "moe route: too many slots");
    k_moe_route<<<grid, 512, 0, h->stream>>>(w, x, (int)n, (int)hdim, (int)n_exp, (int)top_k, s.logits, s.idx, s.wgt,
                                              s.cnt, s.offs, s.list, s.act_list, s.act_n, h->ticket);
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
static void moe_mv_fmt(soso_hip *h, unsigned grid, size_t lds, int lpr, const uint8_t *const *A,
                       const uint8_t *const *B, size_t stride, int rows, int cols, int chunks, const float *xs,
                       int xdiv, int tch, const MoeScratch &s, float *out)
{
#define MOE_CASE(LP)                                                                                                   \
    case LP:                                                                                                           \
        k_moe_mv<FMT, LP, NMAT><<<grid, 512, lds, h->stream>>>(A, B, stride, rows, cols, chunks, xs, xdiv, s.cnt,     \
                                                                s.offs, s.list, s.act_list, s.act_n, tch, out);        \
        break;
    switch (lpr) {
        MOE_CASE(1) MOE_CASE(2) MOE_CASE(4) MOE_CASE(8) MOE_CASE(16) MOE_CASE(32) MOE_CASE(64)
    }
#undef MOE_CASE
}

// One grouped matvec over the active experts (pointer tables on the device).
// active_max bounds the number of active experts, tch the tokens per expert
// staged at a time (at most the tokens of the call).
static int launch_moe_mv(soso_hip *h, uint8_t dtype, int nmat, const uint8_t *const *A, const uint8_t *const *B,
                         size_t rows, size_t cols, size_t active_max, size_t tch, const float *xs, int xdiv,
                         const MoeScratch &s, float *out)
{
    const int U = (int)(cols / 64);
    if (U < 1 || U > 64 || !packed_shape_ok(dtype, rows, cols))
        return set_err(h, SOSO_HIP_DECLINED, "moe: expert shape not handled here");
    const int lpr = U <= 1 ? 1 : U <= 2 ? 2 : U <= 4 ? 4 : U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
    const size_t rpw = 2 * 8 * (64 / lpr);
    const size_t chunks = (rows + rpw - 1) / rpw;
    tch = std::max<size_t>(1, std::min<size_t>(tch, 64));
    const size_t tok_bytes = (stage_lds_bytes(cols) + 15) & ~(size_t)15;
    while (tch > 1 && tok_bytes * tch > h->max_lds) tch--;
    const size_t lds = tok_bytes * tch;
    if (lds > h->max_lds) return set_err(h, SOSO_HIP_DECLINED, "moe: x does not fit in LDS");
    const size_t items = active_max * chunks;
    const unsigned grid = (unsigned)std::max<size_t>(1, std::min<size_t>(items, 2 * (size_t)h->num_cu));
    const size_t stride = packed_row_stride(dtype, cols);
    const int ri = (int)rows, ci = (int)cols, ch = (int)chunks, ti = (int)tch;
    switch (dtype) {
    case SOSO_HIP_DTYPE_Q4_K:
        if (nmat == 2) moe_mv_fmt<FMT_Q4K, 2>(h, grid, lds, lpr, A, B, stride, ri, ci, ch, xs, xdiv, ti, s, out);
        else moe_mv_fmt<FMT_Q4K, 1>(h, grid, lds, lpr, A, B, stride, ri, ci, ch, xs, xdiv, ti, s, out);
        break;
    case SOSO_HIP_DTYPE_Q8_0:
        if (nmat == 2) moe_mv_fmt<FMT_Q80, 2>(h, grid, lds, lpr, A, B, stride, ri, ci, ch, xs, xdiv, ti, s, out);
        else moe_mv_fmt<FMT_Q80, 1>(h, grid, lds, lpr, A, B, stride, ri, ci, ch, xs, xdiv, ti, s, out);
        break;
    case SOSO_HIP_DTYPE_Q6_K:
        if (nmat == 2) moe_mv_fmt<FMT_Q6K, 2>(h, grid, lds, lpr, A, B, stride, ri, ci, ch, xs, xdiv, ti, s, out);
        else moe_mv_fmt<FMT_Q6K, 1>(h, grid, lds, lpr, A, B, stride, ri, ci, ch, xs, xdiv, ti, s, out);
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
    int rc = launch_moe_mv(h, dt_gu, 2, tab, tab + n_groups, ffn, hdim, active, n, xs, (int)top_k, s, s.act);
    if (rc == SOSO_HIP_OK)
        rc = launch_moe_mv(h, dt_down, 1, tab + 2 * n_groups, nullptr, hdim, ffn, active, n, s.act, 1, s, s.ydown);
    if (rc != SOSO_HIP_OK) return rc;
    const dim3 grid((unsigned)((hdim + 255) / 256), (unsigned)n);
    k_moe_combine<<<grid, 256, 0, h->stream>>>(s.ydown, wgt, use, (int)n, (int)hdim, (int)top_k, out);
    return hip_check(h, hipGetLastError(), "moe combine launch");
}
