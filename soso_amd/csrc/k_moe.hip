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
//                 Calls whose experts scan the ranking themselves (at most 512
//                 slots on the matrix cores) take the logits alone, then
//                 k_moe_rank (softmax + top-k, one wavefront per token).
//   k_moe_rows    workgroups over (expert, row chunk) items of equal work:
//                 every weight row of an expert is read once from HBM and
//                 applied to all the tokens routed to it (their x staged in
//                 LDS).  Gate and up rows are read side by side and leave as
//                 silu(gate.x) * up.x; down rows leave as y[slot].  (Two or
//                 more tokens per active expert: the matrix-core kernel of
//                 k_mfma.hip instead.)
//   k_moe_down_comb  up to 4 tokens: down and the weighted sum in one launch,
//                 one wavefront per ranked expert.
//   k_moe_combine out[t] = sum_j wgt[t,j] * y[t*top_k + j], j in ranking order.
// Slot s = t * top_k + j is token t's j-th ranked expert ("destinos" in
// ExpertoBloque, gpu.rs:176-186).
#include "mv_core.hpp"

#include <algorithm>
#include <type_traits>
#include <vector>

// ---------------------------------------------------------------------------
// Router
// ---------------------------------------------------------------------------
// Softmax and ranking of one token's logits by one wavefront (gemm.rs:62-91):
// max-shifted expf, normalised, then the top_k largest probabilities with
// ties to the lowest index (a stable descending sort), renormalised by their
// sum taken in rank order.  lg[q] holds the logit of expert lane + 64 q
// (n_exp <= 256).  Each round takes the wavefront max of a 64-bit key
// (probability bits + 1, then 0xFFFF - expert: larger probability first,
// then lower index); NaN probabilities and removed experts carry key 0 and
// are never chosen -- should fewer than top_k experts remain, the slot points
// at expert 0 with weight 0 (indices stay valid).  `sel`: top_k floats of LDS.
// The softmax and the ranking keys of one token's logits, by one wavefront.
__device__ __forceinline__ void topk_keys(const float (&lg)[4], int n_exp, uint64_t (&key)[4])
{
    const int lane = threadIdx.x & 63;
    const float m = wave_max_dpp(fmaxf(fmaxf(lg[0], lg[1]), fmaxf(lg[2], lg[3])));
    float ex[4], s = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        ex[q] = lane + 64 * q < n_exp ? expf(lg[q] - m) : 0.0f;
        s += ex[q];
    }
    s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(seg_sum_dpp<64>(s)), 63));
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int e = lane + 64 * q;
        const float p = ex[q] / s;
        const uint32_t k32 = e < n_exp && p >= 0.0f ? __float_as_uint(p) + 1u : 0u;
        key[q] = ((uint64_t)k32 << 32) | (uint32_t)(0xFFFF - e);
    }
}

__device__ void topk_regs(const float (&lg)[4], int n_exp, int top_k, int32_t *__restrict__ idx,
                          float *__restrict__ wgt, float *sel, int16_t *rank_lds)
{
    const int lane = threadIdx.x & 63;
    uint64_t key[4];
    topk_keys(lg, n_exp, key);
    for (int j = 0; j < top_k; j++) {
        uint64_t best = key[0];
#pragma unroll
        for (int q = 1; q < 4; q++) best = key[q] > best ? key[q] : best;
        best = wave_max_u64_dpp(best);
        const uint32_t k32 = (uint32_t)(best >> 32);
        const int bi = k32 ? 0xFFFF - (int)(best & 0xFFFFu) : 0;
        const float bv = k32 ? __uint_as_float(k32 - 1u) : 0.0f;
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (k32 && lane + 64 * q == bi) key[q] = 0;
        if (lane == 0) {
            // read by the workgroup that sorts the slots: a coherent store
            __hip_atomic_store(idx + j, (int32_t)bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sel[j] = bv;
            rank_lds[j] = (int16_t)bi;
        }
    }
    if (lane == 0) {
        float tot = 0.0f;
        for (int j = 0; j < top_k; j++) tot += sel[j];
        for (int j = 0; j < top_k; j++) wgt[j] = tot > 0.0f ? sel[j] / tot : sel[j];
    }
}

// grid (ceil(n_exp / waves), ceil(n / TT)); wave w of workgroup (bx, by)
// owns expert bx*waves + w for tokens by*TT .. + TT - 1.  `ticket` is zero
// between launches (the last workgroup resets it).  The last workgroup also
// writes the work items of the grouped kernels (about `target` of them, each
// an equal share of tokens x rows): items[4i .. 4i+3] = {expert, its slot
// count, its first slot in `list`, chunk j | chunks << 16} for i < *n_items,
// experts ascending.
constexpr int ROUTE_MAX_SLOTS = MOE_ROUTE_MAX_SLOTS; // n * top_k handled by the LDS sort
constexpr int ROUTE_TT = 4;           // tokens per wavefront (and per ranking workgroup) from 2 tokens
constexpr int ROUTE_T1 = 2048;        // first per-token-block counter in the ticket buffer
constexpr int MOE_SELF_K = 8;         // top_k of the self-ranked single-token path

// TT tokens per wavefront; each lane requests Q float4 of the expert row (and
// of every token's x) per step: TT = 1 (one token, the decode case) takes a
// 2048-wide row in a single round trip.
// norm_w (TT = 1, hdim <= 256 Q, so the row is one step): xs is h and the
// row is rmsnorm(h) * norm_w (gemm.rs:93-100), each wavefront taking sum(h^2)
// over the row it holds.
template <int TT, int Q, bool LOGITS_ONLY = false>
__global__ void __launch_bounds__(512) k_moe_route(const float *__restrict__ W, const float *__restrict__ xs, int n,
                                                    int hdim, int n_exp, int top_k, float *__restrict__ logits,
                                                    int32_t *__restrict__ idx, float *__restrict__ wgt,
                                                    int *__restrict__ cnt, int *__restrict__ offs,
                                                    int *__restrict__ list, int *__restrict__ items,
                                                    int *__restrict__ n_items, int target, int *__restrict__ recs,
                                                    int *__restrict__ n_recs, unsigned *__restrict__ ticket,
                                                    const float *__restrict__ norm_w = nullptr, float eps = 0.0f)
{
    __shared__ int last;
    __shared__ int pre_s[257];
    __shared__ float sel[8][64];
    __shared__ int c_s[256], o_s[257], f_s[256];
    __shared__ int16_t e_s[ROUTE_MAX_SLOTS];
    __shared__ int16_t rank_s[ROUTE_TT * 64]; // the ranking of a single token block, for its sort
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int e = blockIdx.x * nw + wave;
    const int t0 = blockIdx.y * TT, tn = min(TT, n - t0);
    if (e < n_exp) {
        // this wavefront's expert row against TT tokens: every load of a
        // 64*Q-float4 step is issued before its products
        const float4 *w4 = (const float4 *)(W + (size_t)e * hdim);
        const float4 *x4 = (const float4 *)(xs + (size_t)t0 * hdim);
        const int nv = hdim >> 2;
        float acc[TT];
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[tt] = 0.0f;
        for (int i0 = 0; i0 < nv; i0 += 64 * Q) {
            float4 w[Q], v[TT][Q], nw[Q];
#pragma unroll
            for (int q = 0; q < Q; q++) {
                const int i = i0 + 64 * q + lane;
                w[q] = i < nv ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
                    v[tt][q] = i < nv && tt < tn ? x4[(size_t)tt * nv + i] : make_float4(0.f, 0.f, 0.f, 0.f);
                if (TT == 1 && norm_w)
                    nw[q] = i < nv ? ((const float4 *)norm_w)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            if constexpr (TT == 1) {
                if (norm_w) {
                    float ss = 0.0f;
#pragma unroll
                    for (int q = 0; q < Q; q++) ss += sq4(v[0][q]);
                    ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                       __builtin_bit_cast(int, seg_sum_dpp<64>(ss)), 63));
                    const float scale = 1.0f / sqrtf(ss / (float)hdim + eps);
#pragma unroll
                    for (int q = 0; q < Q; q++) v[0][q] = norm4(v[0][q], scale, nw[q]);
                }
            }
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int q = 0; q < Q; q++) {
                    acc[tt] = fmaf(w[q].x, v[tt][q].x, acc[tt]);
                    acc[tt] = fmaf(w[q].y, v[tt][q].y, acc[tt]);
                    acc[tt] = fmaf(w[q].z, v[tt][q].z, acc[tt]);
                    acc[tt] = fmaf(w[q].w, v[tt][q].w, acc[tt]);
                }
        }
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const float sum = seg_sum_dpp<64>(acc[tt]); // lane 63 holds it
            if (lane == 63 && tt < tn) {
                float *dst = logits + (size_t)(t0 + tt) * n_exp + e;
                // the ranking workgroup of this launch reads it: a coherent store
                if constexpr (LOGITS_ONLY) *dst = sum;
                else __hip_atomic_store(dst, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if constexpr (LOGITS_ONLY) return; // the expert kernels rank the token themselves
    // Two-level tickets.  The last workgroup of token block by (counter
    // ticket[ROUTE_T1 + by]) ranks that block's tokens, one per wavefront;
    // the last token block to be ranked (counter ticket[0]) sorts the slots.
    // With a single token block the ranking workgroup sorts straight away,
    // from the ranking it kept in LDS.
    // What the next level reads (the logits, then the ranked experts) leaves
    // through agent-scope atomic stores, which reach the device's coherence
    // point; once every wavefront has them acknowledged (s_waitcnt, then the
    // barrier), thread 0 takes the ticket, and the next level reads them with
    // coherent loads.  No fence, so no write-back of the XCD's L2 (a
    // device-scope fence per workgroup costs microseconds here).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(ticket + ROUTE_T1 + blockIdx.y, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    if (wave < tn) {
        const int t = t0 + wave;
        float lg[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int x = lane + 64 * q;
            lg[q] = x < n_exp ? __hip_atomic_load(logits + (size_t)t * n_exp + x, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                              : -INFINITY;
        }
        topk_regs(lg, n_exp, top_k, idx + (size_t)t * top_k, wgt + (size_t)t * top_k, sel[wave],
                  rank_s + wave * top_k);
    }
    const bool single = gridDim.y == 1;
    __builtin_amdgcn_s_waitcnt(0); // the ranked experts acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        ticket[ROUTE_T1 + blockIdx.y] = 0u;
        if (!single) last = atomicAdd(ticket, 1u) == gridDim.y - 1;
    }
    __syncthreads();
    if (!last) return;
    // counting sort of the slots by expert in LDS (a slot's position inside
    // its expert's list does not change any result)
    const int slots = n * top_k;
    for (int x = threadIdx.x; x < n_exp; x += blockDim.x) c_s[x] = f_s[x] = 0;
    __syncthreads();
    for (int sl = threadIdx.x; sl < slots; sl += blockDim.x) {
        const int x = min(max((int)(single ? rank_s[sl]
                                           : __hip_atomic_load(idx + sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
                              0),
                          n_exp - 1);
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
        // work items: expert x with c tokens gets max(1, round(c * target /
        // slots)) row chunks, so every item carries about the same tokens x
        // rows; exclusive scan of the chunk counts over the experts
        int v[4], tot = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int x = 4 * lane + q;
            const int cx = x < n_exp ? c_s[x] : 0;
            v[q] = cx > 0 ? min(0xFFFF, max(1, (cx * target + slots / 2) / slots)) : 0;
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
            if (x < n_exp) pre_s[x] = run;
            run += v[q];
        }
        if (lane == 63) {
            pre_s[n_exp] = incl;
            *n_items = incl;
            if (!single) *ticket = 0u;
        }
    }
    if (wave == 1) {
        // active-expert records, ascending: recs[4a ..] = {expert, slots, first slot, 0}
        int nact = 0;
        for (int x0 = 0; x0 < n_exp; x0 += 64) {
            const int x = x0 + lane;
            const bool on = x < n_exp && c_s[x] > 0;
            const unsigned long long m = __ballot(on);
            if (on) {
                int *r = recs + 4 * (nact + __popcll(m & ((1ull << lane) - 1ull)));
                r[0] = x;
                r[1] = c_s[x];
                r[2] = o_s[x];
                r[3] = 0;
            }
            nact += __popcll(m);
        }
        if (lane == 0) *n_recs = nact;
    }
    __syncthreads();
    // items[4i .. 4i+3] = {expert, its slot count, its first slot, chunk | chunks << 16};
    // item i belongs to the expert x with pre_s[x] <= i < pre_s[x + 1]
    const int total = pre_s[n_exp];
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
        int lo = 0, hi = n_exp - 1; // last x with pre_s[x] <= i
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pre_s[mid] <= i) lo = mid;
            else hi = mid - 1;
        }
        const int nx = pre_s[lo + 1] - pre_s[lo];
        int4 r;
        r.x = lo;
        r.y = c_s[lo];
        r.z = o_s[lo];
        r.w = (i - pre_s[lo]) | (nx << 16);
        int *d = items + 4 * i;
        d[0] = r.x;
        d[1] = r.y;
        d[2] = r.z;
        d[3] = r.w;
    }
}

// The ranking of calls whose expert kernels scan it (no slot sort): one
// wavefront per token ranks its logits with topk_regs, as the route kernel's
// last workgroup would, in a launch of its own after k_moe_route<TT, Q, true>.
// On MI355X (configs[3] at batch 32) the layer took 88.7 us with this pair
// against 89.4 with the route's own ticket and last-workgroup ranking.
__global__ void __launch_bounds__(256) k_moe_rank(const float *__restrict__ logits, int n, int n_exp, int top_k,
                                                  int32_t *__restrict__ idx, float *__restrict__ wgt)
{
    __shared__ float sel[4][64];
    __shared__ int16_t rank_s[4 * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= n) return; // whole wavefronts
    float lg[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int x = lane + 64 * q;
        lg[q] = x < n_exp ? logits[(size_t)t * n_exp + x] : -INFINITY;
    }
    topk_regs(lg, n_exp, top_k, idx + (size_t)t * top_k, wgt + (size_t)t * top_k, sel[wave], rank_s + wave * 64);
}

// ---------------------------------------------------------------------------
// Grouped expert matvecs
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Grouped expert matvecs: workgroups (512 threads, 8 wavefronts) over the
// work items written by k_moe_route, item it = blockIdx.x, + gridDim.x (the
// host launches about one workgroup per item and the dispatcher balances
// them).  Item (expert e, chunk j of nx) covers passes [j * passes / nx,
// (j + 1) * passes / nx) of every wavefront: rows r0 + (p * 8 + wave) * RW +
// slot, so one item streams a contiguous block of an expert's rows.  Per item:
//   1. the x of the expert's tokens (up to `tch` at a time) is requested in
//      one batch -- slot s reads x = xs + (s / xdiv) * cols --,
//   2. then the weight ring (DEPTH passes, every load unconditional: rows
//      past the chunk read zeros through the buffer range check),
//   3. x is converted into LDS (digit planes, one region per token) while
//      the ring is in flight,
//   4. the passes stream through the ring; each pass applies its rows to
//      every staged token (x from LDS) and writes out[s * rows + r].
// NMAT == 2: tabA = gate, tabB = up, output silu(gate.x) * up.x (swiglu,
// gemm.rs:210-226); NMAT == 1: tabA = down.
constexpr int MOE_XK = 4; // x chunks (8 floats) per thread per staging round

// Q4_K unit of one row decoded once per pass and shared by the tokens: the
// codes of sub-blocks 2p (low nibbles) and 2p+1 (high nibbles), and the
// factors d*sc and dmin*m of both (get_scale_min_k4, crates/sosomodel/src/
// dequant.rs:150-159, four at a time per byte lane as in unit_dot).
struct Q4Prep {
    uint32_t lo[8], hi[8];
    float ka, kb, kma, kmb;
};

__device__ __forceinline__ void q4k_prep(const WRow<FMT_Q4K> &w, const UConst &c, Q4Prep &p)
{
    const uint32_t q[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
#pragma unroll
    for (int t = 0; t < 8; t++) {
        p.lo[t] = q[t] & 0x0F0F0F0Fu;
        p.hi[t] = (q[t] >> 4) & 0x0F0F0F0Fu;
    }
    const uint32_t SC4 = ((w.h.w & c.k1) | ((w.h.y >> c.s) & c.k2)) >> c.bsh;
    const uint32_t M4 = (((w.h.w >> 4) & c.k1) | ((w.h.z >> c.s) & c.k2)) >> c.bsh;
    const float d = half_bits_to_f32(w.h.x & 0xffffu), dmin = half_bits_to_f32(w.h.x >> 16);
    p.ka = d * (float)(SC4 & 0xffu);
    p.kb = d * (float)((SC4 >> 8) & 0xffu);
    p.kma = dmin * (float)(M4 & 0xffu);
    p.kmb = dmin * (float)((M4 >> 8) & 0xffu);
}

// sum over one sub-block (register groups g0 .. g0+7) of codes x digits
__device__ __forceinline__ void q4k_half(const uint32_t (&codes)[8], const uint32_t (&xh)[24], int (&s)[XDIG])
{
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
        for (int k = 0; k < XDIG; k++) s[k] = sdot4(codes[t], xh[XDIG * t + k], s[k]);
}

// Code l (0..31) of one sub-block's packed nibbles (four per dword), picked
// by a select chain: a dynamically indexed register array would go to scratch.
__device__ __forceinline__ uint32_t q4k_code(const uint32_t (&c)[8], int l)
{
    const int k = l >> 2;
    // opaque: a select chain over the array's elements could be folded into
    // one load at a computed address, which would move the array to scratch
    uint32_t v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = opaque(c[i]);
    const uint32_t a = k == 0 ? v[0] : k == 1 ? v[1] : k == 2 ? v[2] : v[3];
    const uint32_t b = k == 4 ? v[4] : k == 5 ? v[5] : k == 6 ? v[6] : v[7];
    return ((k < 4 ? a : b) >> (8 * (l & 3))) & 15u;
}

// Sum of w * x over the outliers (OUTL staging: the list ol of unit u's
// 128-element block, ocnt entries, onum the longest list of the wavefront)
// that fall in the unit, w decoded from the prepared unit exactly as
// dequant_q4_k_range decodes it (crates/sosomodel/src/dequant.rs:204-241):
// fl(fl(d sc) q) - fl(dmin m), with pr.ka = fl(d sc) and pr.kma = fl(dmin m).
template <int NMAT>
__device__ __forceinline__ void q4k_outliers(const Q4Prep (&pr)[NMAT], const uint32_t *ol, int ocnt, int onum, int u,
                                             float (&corr)[NMAT])
{
    for (int k = 0; k < onum; k++) {
        if (k < ocnt) {
            const uint32_t p = (ol[1 + (k >> 2)] >> (8 * (k & 3))) & 0xffu;
            if ((p >> 6) == ((uint32_t)u & 1u)) {
                const int e = (int)(p & 63u), sub = e >> 5, l = e & 31;
                const float v = __uint_as_float(ol[8 + k]);
#pragma unroll
                for (int m = 0; m < NMAT; m++) {
                    const uint32_t q = sub ? q4k_code(pr[m].hi, l) : q4k_code(pr[m].lo, l);
                    // (opaque for the same reason as in q4k_code)
                    const float ka = __uint_as_float(opaque(__float_as_uint(pr[m].ka)));
                    const float kb = __uint_as_float(opaque(__float_as_uint(pr[m].kb)));
                    const float kma = __uint_as_float(opaque(__float_as_uint(pr[m].kma)));
                    const float kmb = __uint_as_float(opaque(__float_as_uint(pr[m].kmb)));
                    const float w = __fsub_rn(__fmul_rn(sub ? kb : ka, (float)q), sub ? kmb : kma);
                    corr[m] = fmaf(w, v, corr[m]);
                }
            }
        }
    }
}

// One decoded row unit (pr[m], m < NMAT) against the x staged in LDS at xd
// (digit planes, then the 16-element sums s16, then the 128-block exponents
// kx, then the outlier lists): returns the row's dot in the last lane of each
// LPR-lane group.  OUTL: the outliers of the unit's block are added as w * x
// (the kernels take that variant only for rounds that have outliers).
template <int LPR, int NMAT, bool OUTL = false>
__device__ __forceinline__ void q4k_token_dot(const Q4Prep (&pr)[NMAT], const uint32_t *xd, int cols, int U, int u,
                                              bool uact, float (&val)[NMAT])
{
    const float *s16 = (const float *)(xd + (cols >> 2) * XDIG);
    const int *kx = (const int *)(s16 + (cols >> 4));
    const uint4 *x4 = (const uint4 *)xd;
    int sa[NMAT][XDIG], sb[NMAT][XDIG];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int k = 0; k < XDIG; k++) sa[m][k] = sb[m][k] = 0;
    uint32_t xh[24];
#pragma unroll
    for (int r = 0; r < 6; r++) {
        const uint4 v = x4[r * U + u];
        xh[4 * r] = v.x;
        xh[4 * r + 1] = v.y;
        xh[4 * r + 2] = v.z;
        xh[4 * r + 3] = v.w;
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++) q4k_half(pr[m].lo, xh, sa[m]);
#pragma unroll
    for (int r = 0; r < 6; r++) {
        const uint4 v = x4[(r + 6) * U + u];
        xh[4 * r] = v.x;
        xh[4 * r + 1] = v.y;
        xh[4 * r + 2] = v.z;
        xh[4 * r + 3] = v.w;
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++) q4k_half(pr[m].hi, xh, sb[m]);
    const float P = block_unscale(kx[u >> 1]);
    const float c0 = s16[4 * u] + s16[4 * u + 1], c1 = s16[4 * u + 2] + s16[4 * u + 3];
    float part[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const float uu = fmaf(pr[m].ka, digits_value(sa[m]), pr[m].kb * digits_value(sb[m]));
        const float vv = fmaf(pr[m].kmb, c1, pr[m].kma * c0);
        part[m] = uact ? fmaf(P, uu, -vv) : 0.0f;
    }
    if constexpr (OUTL) {
        const uint32_t *ol = out_lists(kx, cols) + (u >> 1) * OUT_DW;
        const int ocnt = uact ? min((int)ol[0], OUT_MAX) : 0;
        if (__ballot(ocnt > 0) != 0) q4k_outliers<NMAT>(pr, ol, ocnt, (int)wave_max_dpp((float)ocnt), u, part);
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++) val[m] = seg_sum_dpp<LPR>(part[m]);
}

// One token ranked by the expert kernel itself (SELF): every workgroup takes
// the softmax top-k of the token's logits (topk_regs, the same ranking as the
// route kernel's) and runs `chunks` row chunks of each ranked expert j on
// slot j; workgroup 0 also writes the ranking to idx / wgt for the kernels
// that follow.  No work items or slot lists are read.
struct MoeSelf {
    const float *logits = nullptr;
    int n_exp = 0, top_k = 0, chunks = 0;
    int32_t *idx = nullptr;
    float *wgt = nullptr;
    // when set, xs is h and the staged row is rmsnorm(h) * norm_w (the decode
    // step's MoE layers; cols <= 4096, one staging round)
    const float *norm_w = nullptr;
    float eps = 0.0f;
};

template <int FMT, int LPR, int NMAT, int DEPTH, bool SELF = false>
__global__ void __launch_bounds__(512) k_moe_rows(const uint8_t *const *__restrict__ tabA,
                                                  const uint8_t *const *__restrict__ tabB, size_t stride, int rows,
                                                  int cols, const float *__restrict__ xs, int xdiv,
                                                  const int *__restrict__ list, const int *__restrict__ items,
                                                  const int *__restrict__ n_items, int tch, float *__restrict__ out,
                                                  MoeSelf sr = MoeSelf())
{
    constexpr int RW = 64 / LPR, NW = 8;
    extern __shared__ uint4 smem[];
    __shared__ int slot_s[64];
    const int tok_bytes = (int)((stage_lds_bytes_o((size_t)cols) + 15) & ~(size_t)15);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int U = cols >> 6, nch = cols >> 3;
    const int ul = lane & (LPR - 1), slot = lane / LPR;
    const bool uact = ul < U;
    const int u = uact ? ul : 0;
    UConst c;
    unit_setup_w<FMT>(u, c);
    const LaneOff L = lane_offsets<FMT>(cols, u, c);
    const uint32_t pass_bytes = (uint32_t)(NW * RW * stride);
    const uint32_t lane_base = uact ? (uint32_t)((wave * RW + slot) * stride) : 0x80000000u;
    const int passes = (rows + NW * RW - 1) / (NW * RW);
    __shared__ int32_t self_idx[MOE_SELF_K];
    __shared__ float self_wgt[MOE_SELF_K], self_sel[MOE_SELF_K];
    __shared__ __align__(16) uint32_t self_keys[256];
    __shared__ float nrm_s[NW];
    __shared__ int found_s[NW]; // SELF: the wavefronts' staging found outliers
    int nit;
    bool oany = false; // SELF: the staged token has outliers (its passes take the exact-weight loop)
    if constexpr (SELF) {
        // The ranking of topk_regs, by the whole workgroup: wavefront 0 makes
        // the keys (topk_keys; the upper word is the order, 0 for experts
        // that cannot be chosen, the lower word breaks ties to the lower
        // index).  Expert e's rank is then the number of experts i with
        // k[i] > k[e], or k[i] == k[e] and i < e, counted by tpe adjacent
        // threads over one share each of the 256 zero-padded upper words.
        // Ranks below top_k fill the slots; slots no valid expert reaches
        // keep expert 0 with weight 0, as in topk_regs.
        // The one token's x row (every slot's row is row 0: xdiv = top_k) is
        // staged into LDS here, once; its loads are in flight with the logits'.
        // wavefront 0 requests the logits first: the norm's barrier below
        // then waits on them only as long as on x
        float lg[4];
        if (wave == 0) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int x = lane + 64 * q;
                lg[q] = x < sr.n_exp ? sr.logits[x] : -INFINITY;
            }
        }
        float4 xv0[MOE_XK], xv1[MOE_XK], nw0[MOE_XK], nw1[MOE_XK];
#pragma unroll
        for (int k = 0; k < MOE_XK; k++) {
            const int f = k * 512 + (int)threadIdx.x;
            xv0[k] = xv1[k] = nw0[k] = nw1[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (f < nch) {
                const float4 *x4 = (const float4 *)xs + 2 * f;
                xv0[k] = x4[0];
                xv1[k] = x4[1];
                if (sr.norm_w) {
                    const float4 *w4 = (const float4 *)sr.norm_w + 2 * f;
                    nw0[k] = w4[0];
                    nw1[k] = w4[1];
                }
            }
        }
        if (sr.norm_w) {
            // RMSNorm of the row (zeros past its end add nothing): every
            // workgroup takes sum(h^2) itself, as the matvec staging does
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < MOE_XK; k++) ss += sq4(xv0[k]) + sq4(xv1[k]);
            ss = seg_sum<64>(ss);
            if (lane == 0) nrm_s[wave] = ss;
            __syncthreads();
            float tot = 0.0f;
#pragma unroll
            for (int i = 0; i < NW; i++) tot += nrm_s[i];
            const float scale = 1.0f / sqrtf(tot / (float)cols + sr.eps);
#pragma unroll
            for (int k = 0; k < MOE_XK; k++) {
                xv0[k] = norm4(xv0[k], scale, nw0[k]);
                xv1[k] = norm4(xv1[k], scale, nw1[k]);
            }
        }
        if (wave == 0) {
            uint64_t key[4];
            topk_keys(lg, sr.n_exp, key);
#pragma unroll
            for (int q = 0; q < 4; q++) self_keys[lane + 64 * q] = (uint32_t)(key[q] >> 32);
            if (lane < sr.top_k) {
                self_idx[lane] = 0;
                self_sel[lane] = 0.0f;
            }
        }
        {
            uint32_t *xd = (uint32_t *)smem;
            float *s16 = (float *)(xd + (cols >> 2) * XDIG);
            int *kx = (int *)(s16 + (cols >> 4));
            // the cheap outlier test first; rounds whose blocks may hold
            // outliers are staged again through the full search
            bool found = false;
            uint32_t redo = 0;
#pragma unroll
            for (int k = 0; k < MOE_XK; k++) {
                const int f = k * 512 + (int)threadIdx.x;
                if (k * 512 < nch && !stage_chunk<FMT, true, true>(xv0[k], xv1[k], f % nch, f < nch, U, xd, s16, kx))
                    redo |= 1u << k;
            }
            if (__builtin_expect(redo != 0, 0)) {
#pragma unroll
                for (int k = 0; k < MOE_XK; k++) {
                    const int f = k * 512 + (int)threadIdx.x;
                    if ((redo >> k) & 1u) stage_chunk<FMT, true>(xv0[k], xv1[k], f % nch, f < nch, U, xd, s16, kx, &found);
                }
            }
            for (int fb = MOE_XK * 512; fb < nch; fb += 512) { // rows longer than one round holds
                const int f = fb + (int)threadIdx.x;
                float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
                if (f < nch) {
                    const float4 *x4 = (const float4 *)xs + 2 * f;
                    v0 = x4[0];
                    v1 = x4[1];
                }
                stage_chunk<FMT, true>(v0, v1, f % nch, f < nch, U, xd, s16, kx, &found);
            }
            // every wavefront writes its own word: nothing to clear between calls
            if (lane == 0) found_s[wave] = found ? 1 : 0;
        }
        __syncthreads();
        {
            const int tpe = sr.n_exp <= 64 ? 8 : sr.n_exp <= 128 ? 4 : 2; // threads per expert
            const int ex = (int)threadIdx.x / tpe, part = (int)threadIdx.x % tpe;
            const uint32_t mine = self_keys[ex];
            // share: n4 groups of 4 keys; tpe * 4 * n4 <= 256 for n_exp <= 256
            const int n4 = (sr.n_exp + 4 * tpe - 1) / (4 * tpe);
            const uint4 *kv = (const uint4 *)self_keys + part * n4;
            int above = 0, i = 4 * part * n4;
#pragma unroll 8
            for (int g = 0; g < n4; g++, i += 4) {
                const uint4 k = kv[g];
                above += (k.x > mine || (k.x == mine && i < ex)) ? 1 : 0;
                above += (k.y > mine || (k.y == mine && i + 1 < ex)) ? 1 : 0;
                above += (k.z > mine || (k.z == mine && i + 2 < ex)) ? 1 : 0;
                above += (k.w > mine || (k.w == mine && i + 3 < ex)) ? 1 : 0;
            }
            // the tpe counts of an expert sit in adjacent lanes
            float fa = (float)above;
            if (tpe >= 2) fa += dpp_f<0xB1>(fa);
            if (tpe >= 4) fa += dpp_f<0x4E>(fa);
            if (tpe >= 8) fa += dpp_f<0x141>(fa);
            const int rank = (int)fa;
            if (part == 0 && ex < sr.n_exp && mine != 0u && rank < sr.top_k) {
                self_idx[rank] = ex;
                self_sel[rank] = __uint_as_float(mine - 1u);
            }
        }
        __syncthreads();
        if ((int)threadIdx.x < sr.top_k) {
            float tot = 0.0f;
#pragma unroll
            for (int j = 0; j < MOE_SELF_K; j++)
                if (j < sr.top_k) tot += self_sel[j];
            const float sj = self_sel[threadIdx.x];
            self_wgt[threadIdx.x] = tot > 0.0f ? sj / tot : sj;
        }
        __syncthreads();
        if (blockIdx.x == 0 && (int)threadIdx.x < sr.top_k) {
            sr.idx[threadIdx.x] = self_idx[threadIdx.x];
            sr.wgt[threadIdx.x] = self_wgt[threadIdx.x];
        }
        nit = sr.top_k * sr.chunks;
#pragma unroll
        for (int i = 0; i < NW; i++) oany = oany || found_s[i] != 0;
    } else {
        nit = *n_items;
    }
    for (int it = blockIdx.x; it < nit; it += gridDim.x) {
        int e, ne, base, j, nx, self_slot = 0;
        if constexpr (SELF) {
            self_slot = it / sr.chunks; // rank = slot of the single token
            e = min(max((int)self_idx[self_slot], 0), sr.n_exp - 1);
            ne = 1;
            base = 0;
            j = it % sr.chunks;
            nx = sr.chunks;
        } else {
            const int *rec = items + 4 * it;
            e = rec[0];
            ne = rec[1];
            base = rec[2];
            j = rec[3] & 0xFFFF;
            nx = rec[3] >> 16;
        }
        const int p0 = (int)((long)j * passes / nx), p1 = (int)((long)(j + 1) * passes / nx), P = p1 - p0;
        if (P <= 0) continue; // more chunks than passes: an empty share
        const int r0 = p0 * NW * RW, rend = min(rows, p1 * NW * RW);
        const uint32_t strip = (uint32_t)((size_t)(rend - r0) * stride);
        const rsrc_t rA = make_rsrc(tabA[e] + (size_t)r0 * stride, strip);
        const rsrc_t rB = make_rsrc((NMAT == 2 ? tabB[e] : tabA[e]) + (size_t)r0 * stride, strip);
        for (int t0 = 0; t0 < ne; t0 += tch) {
            const int nt = min(tch, ne - t0), tot = nt * nch;
            // 1. x of the tokens: chunk f = token (f / nch), piece (f % nch)
            // (the self-ranked path staged its one row before the ranking)
            float4 xv0[MOE_XK], xv1[MOE_XK];
            if constexpr (!SELF) {
#pragma unroll
                for (int k = 0; k < MOE_XK; k++) {
                    const int f = k * 512 + (int)threadIdx.x;
                    xv0[k] = xv1[k] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (f < tot) {
                        const int sl = list[base + t0 + f / nch];
                        const float4 *x4 = (const float4 *)(xs + (size_t)(sl / xdiv) * cols) + 2 * (f % nch);
                        xv0[k] = x4[0];
                        xv1[k] = x4[1];
                    }
                }
                if ((int)threadIdx.x < nt) slot_s[threadIdx.x] = list[base + t0 + threadIdx.x];
            }
            __builtin_amdgcn_sched_barrier(0);
            // The passes: Q4_K rows are decoded once per pass (q4k_prep) and
            // applied to every staged token; a token's x is read from LDS one
            // sub-block (24 dwords) at a time.  OUTL (a constant): the
            // tokens' outliers are added with their exactly decoded weights
            // (the grouped path always; the self-ranked path only when its
            // token has some, through the loop just below).
            auto pass_q4k = [&](int j, const Q4Prep (&pr)[NMAT], auto outl) {
                const int row = r0 + (j * NW + wave) * RW + slot;
                for (int tk = 0; tk < nt; tk++) {
                    const uint32_t *xd = (const uint32_t *)((const uint8_t *)smem + (size_t)tk * tok_bytes);
                    float val[NMAT];
                    q4k_token_dot<LPR, NMAT, decltype(outl)::value>(pr, xd, cols, U, u, uact, val);
                    float v = val[0];
                    if constexpr (NMAT == 2) v = silu(val[0]) * val[1];
                    if (ul == LPR - 1 && row < rend) out[(size_t)(SELF ? self_slot : slot_s[tk]) * rows + row] = v;
                }
            };
            auto pass = [&](int j, const WRow<FMT> &pa_w, const WRow<FMT> &pb_w, auto outl) {
                constexpr bool OL = decltype(outl)::value;
                const int row = r0 + (j * NW + wave) * RW + slot;
                for (int tk = 0; tk < nt; tk++) {
                    const uint32_t *xd = (const uint32_t *)((const uint8_t *)smem + (size_t)tk * tok_bytes);
                    const float *s16 = (const float *)(xd + (cols >> 2) * XDIG);
                    const int *kx = (const int *)(s16 + (cols >> 4));
                    XReg xv;
                    UConst cj = c;
                    unit_setup_x<FMT, OL>(xd, s16, kx, u, U, xv, cj);
                    float pa = uact ? unit_dot<FMT>(pa_w, xv, cj) : 0.0f, pb = 0.0f;
                    if constexpr (NMAT == 2) pb = uact ? unit_dot<FMT>(pb_w, xv, cj) : 0.0f;
                    if (OL && cj.onum != 0) {
                        // the outliers of the unit's block, exactly weighted
                        cj.ocnt = uact ? cj.ocnt : 0;
                        cj.onum = (int)wave_max_dpp((float)cj.ocnt);
                        pa += unit_outliers<FMT>(pa_w, cj, u);
                        if constexpr (NMAT == 2) pb += unit_outliers<FMT>(pb_w, cj, u);
                    }
                    float v = seg_sum_dpp<LPR>(pa);
                    if constexpr (NMAT == 2) v = silu(v) * seg_sum_dpp<LPR>(pb);
                    if (ul == LPR - 1 && row < rend) out[(size_t)(SELF ? self_slot : slot_s[tk]) * rows + row] = v;
                }
            };
            if (SELF && __builtin_expect(oany, 0)) {
                // the self-ranked token has outliers (known before the ring is
                // issued): every pass loaded on its own and the outliers added
                // with their exactly decoded weights, so that the streaming
                // loop below stays free of that code
                for (int j = 0; j < P; j++) {
                    WRow<FMT> ra, rb;
                    load_row<FMT>(rA, lane_base + (uint32_t)j * pass_bytes, cols, L, ra);
                    if constexpr (NMAT == 2) load_row<FMT>(rB, lane_base + (uint32_t)j * pass_bytes, cols, L, rb);
                    if constexpr (FMT == FMT_Q4K) {
                        Q4Prep pr[NMAT];
                        q4k_prep(ra, c, pr[0]);
                        if constexpr (NMAT == 2) q4k_prep(rb, c, pr[NMAT - 1]);
                        pass_q4k(j, pr, std::true_type{});
                    } else {
                        pass(j, ra, rb, std::true_type{});
                    }
                }
                continue;
            }
            // 2. the ring
            WRow<FMT> wa[DEPTH], wb[DEPTH];
#pragma unroll
            for (int i = 0; i < DEPTH; i++) {
                load_row<FMT>(rA, lane_base + (uint32_t)i * pass_bytes, cols, L, wa[i]);
                if constexpr (NMAT == 2) load_row<FMT>(rB, lane_base + (uint32_t)i * pass_bytes, cols, L, wb[i]);
            }
            __builtin_amdgcn_sched_barrier(0);
            // 3. x into LDS (16-chunk blocks never straddle tokens: nch % 16 == 0)
            if constexpr (!SELF) {
#pragma unroll
                for (int k = 0; k < MOE_XK; k++) {
                    const int fb = k * 512;
                    if (fb < tot) {
                        const int f = fb + (int)threadIdx.x, tk = f / nch;
                        uint32_t *xd = (uint32_t *)((uint8_t *)smem + (size_t)(f < tot ? tk : 0) * tok_bytes);
                        float *s16 = (float *)(xd + (cols >> 2) * XDIG);
                        int *kx = (int *)(s16 + (cols >> 4));
                        stage_chunk<FMT, true>(xv0[k], xv1[k], f % nch, f < tot, U, xd, s16, kx);
                    }
                }
                for (int fb = MOE_XK * 512; fb < tot; fb += 512) { // more tokens than one round holds
                    const int f = fb + (int)threadIdx.x, tk = f / nch;
                    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
                    if (f < tot) {
                        const int sl = list[base + t0 + tk];
                        const float4 *x4 = (const float4 *)(xs + (size_t)(sl / xdiv) * cols) + 2 * (f % nch);
                        v0 = x4[0];
                        v1 = x4[1];
                    }
                    uint32_t *xd = (uint32_t *)((uint8_t *)smem + (size_t)(f < tot ? tk : 0) * tok_bytes);
                    float *s16 = (float *)(xd + (cols >> 2) * XDIG);
                    int *kx = (int *)(s16 + (cols >> 4));
                    stage_chunk<FMT, true>(v0, v1, f % nch, f < tot, U, xd, s16, kx);
                }
                __syncthreads();
            }
            // 4. passes through the ring: counted whole turns, then the rest.
            // Q4_K: each pass's rows are decoded once (q4k_prep) and the ring
            // slot is refilled before the tokens are applied; a token's x is
            // read from LDS one sub-block (24 dwords) at a time.
            const int turns = P / DEPTH;
            int j0 = 0;
            for (int tr = 0; tr < turns; tr++, j0 += DEPTH) {
#pragma unroll
                for (int i = 0; i < DEPTH; i++) {
                    if constexpr (FMT == FMT_Q4K) {
                        Q4Prep pr[NMAT];
                        q4k_prep(wa[i], c, pr[0]);
                        if constexpr (NMAT == 2) q4k_prep(wb[i], c, pr[NMAT - 1]);
                        load_row<FMT>(rA, lane_base + (uint32_t)(j0 + i + DEPTH) * pass_bytes, cols, L, wa[i]);
                        if constexpr (NMAT == 2)
                            load_row<FMT>(rB, lane_base + (uint32_t)(j0 + i + DEPTH) * pass_bytes, cols, L, wb[i]);
                        __builtin_amdgcn_sched_barrier(0);
                        pass_q4k(j0 + i, pr, std::integral_constant<bool, !SELF>{});
                    } else {
                        pass(j0 + i, wa[i], wb[i], std::integral_constant<bool, !SELF>{});
                        load_row<FMT>(rA, lane_base + (uint32_t)(j0 + i + DEPTH) * pass_bytes, cols, L, wa[i]);
                        if constexpr (NMAT == 2)
                            load_row<FMT>(rB, lane_base + (uint32_t)(j0 + i + DEPTH) * pass_bytes, cols, L, wb[i]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int i = 0; i < DEPTH - 1; i++)
                if (i < P - j0) {
                    if constexpr (FMT == FMT_Q4K) {
                        Q4Prep pr[NMAT];
                        q4k_prep(wa[i], c, pr[0]);
                        if constexpr (NMAT == 2) q4k_prep(wb[i], c, pr[NMAT - 1]);
                        pass_q4k(j0 + i, pr, std::integral_constant<bool, !SELF>{});
                    } else {
                        pass(j0 + i, wa[i], wb[i], std::integral_constant<bool, !SELF>{});
                    }
                }
            if constexpr (!SELF) __syncthreads(); // LDS and slot_s are restaged next
        }
    }
}

// Down projection and weighted sum in one launch, for calls with a few
// tokens (about one token per routed expert, where grouping tokens by expert
// saves no weight reads).  Work item = (token t, block of RW*P rows);
// wavefront j of the workgroup takes the token's j-th ranked expert: it stages
// its own act row (slot t*top_k + j) in LDS, streams the block's rows of that
// expert (all P passes requested at once) and leaves its dots in LDS; then one
// lane per row forms
//   out[t*rows + r] = sum_j wgt[t,j] * (down_{e_j} . act[t*top_k + j])[r]
// with the fmaf of k_moe_combine, j = 0, 1, ... in ranking order (the
// ranking-order sum of layer.rs:1914-1924).  Q4_K, top_k <= MDC_K.
constexpr int MDC_K = 8;  // ranked experts per token (one wavefront each)
constexpr int MDC_XR = 4; // act chunks (8 floats) per lane: cols <= 64 * 8 * MDC_XR

template <int LPR, int P>
__global__ void __launch_bounds__(512) k_moe_down_comb(const uint8_t *const *__restrict__ tab, size_t stride, int rows,
                                                       int cols, int n_exp, const float *__restrict__ act,
                                                       const int32_t *__restrict__ idx, const float *__restrict__ wgt,
                                                       int n, int top_k, const float *__restrict__ res,
                                                       float *__restrict__ out)
{
    constexpr int RW = 64 / LPR, RB = RW * P; // rows per item
    extern __shared__ uint4 smem[];
    __shared__ float dots[MDC_K][RB];
    const int tok_bytes = (int)((stage_lds_bytes_o((size_t)cols) + 15) & ~(size_t)15);
    const int lane = threadIdx.x & 63;
    const int j = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); // ranked slot of this wavefront
    const int U = cols >> 6, nch = cols >> 3;
    const int ul = lane & (LPR - 1), slot = lane / LPR;
    const bool uact = ul < U;
    const int u = uact ? ul : 0;
    UConst c;
    unit_setup_w<FMT_Q4K>(u, c);
    const LaneOff L = lane_offsets<FMT_Q4K>(cols, u, c);
    uint32_t *xd = (uint32_t *)((uint8_t *)smem + (size_t)j * tok_bytes);
    float *s16 = (float *)(xd + (cols >> 2) * XDIG);
    int *kx = (int *)(s16 + (cols >> 4));
    const bool on = j < top_k;
    const int blocks = (rows + RB - 1) / RB, items = n * blocks;
    for (int it = blockIdx.x; it < items; it += gridDim.x) {
        const int t = it / blocks, r0 = (it % blocks) * RB;
        const int sl = t * top_k + j;
        // 1. this wavefront's act row
        float4 xv0[MDC_XR], xv1[MDC_XR];
#pragma unroll
        for (int k = 0; k < MDC_XR; k++) {
            const int f = 64 * k + lane;
            xv0[k] = xv1[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (on && f < nch) {
                const float4 *x4 = (const float4 *)(act + (size_t)sl * cols) + 2 * f;
                xv0[k] = x4[0];
                xv1[k] = x4[1];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // 2. the block's rows of expert e_j, all passes in flight (rows past
        // the matrix and idle wavefronts read zeros through the range check)
        const int e = on ? min(max((int)idx[sl], 0), n_exp - 1) : 0;
        const rsrc_t rs = make_rsrc(tab[e] + (size_t)r0 * stride, (uint32_t)((size_t)(min(rows, r0 + RB) - r0) * stride));
        const uint32_t base = on && uact ? (uint32_t)(slot * stride) : 0x80000000u;
        WRow<FMT_Q4K> w[P];
#pragma unroll
        for (int p = 0; p < P; p++) load_row<FMT_Q4K>(rs, base + (uint32_t)(p * RW) * (uint32_t)stride, cols, L, w[p]);
        __builtin_amdgcn_sched_barrier(0);
        // 3. act into this wavefront's LDS region (16-chunk blocks: nch % 16 == 0)
        // (the cheap outlier test first; a wavefront whose act row may hold
        // outliers stages it again through the full search)
        bool oany = false;
        uint32_t redo = 0;
#pragma unroll
        for (int k = 0; k < MDC_XR; k++)
            if (64 * k < nch &&
                !stage_chunk<FMT_Q4K, true, true>(xv0[k], xv1[k], 64 * k + lane, 64 * k + lane < nch, U, xd, s16, kx))
                redo |= 1u << k;
        if (__builtin_expect(redo != 0, 0)) {
#pragma unroll
            for (int k = 0; k < MDC_XR; k++)
                if (64 * k < nch)
                    stage_chunk<FMT_Q4K, true>(xv0[k], xv1[k], 64 * k + lane, 64 * k + lane < nch, U, xd, s16, kx,
                                               &oany);
        }
        __syncthreads();
        // 4. the dots of this wavefront's rows
#pragma unroll
        for (int p = 0; p < P; p++) {
            Q4Prep pr[1];
            q4k_prep(w[p], c, pr[0]);
            float val[1];
            q4k_token_dot<LPR, 1>(pr, xd, cols, U, u, uact, val);
            if (ul == LPR - 1) dots[j][p * RW + slot] = val[0];
        }
        // ... and, when its act row has outliers (a uniform branch per
        // wavefront), their w * x, with the rows loaded again (the ring is
        // gone by now, so this adds no registers to the loop above) and w
        // decoded exactly as the reference decodes it
        if (__builtin_expect(oany, 0)) {
            UConst co = c;
            co.ol = out_lists(kx, cols) + (u >> 1) * OUT_DW;
            co.ocnt = uact ? min((int)co.ol[0], OUT_MAX) : 0;
            co.onum = (int)wave_max_dpp((float)co.ocnt);
            for (int p = 0; p < P; p++) {
                WRow<FMT_Q4K> wr;
                load_row<FMT_Q4K>(rs, base + (uint32_t)(p * RW) * (uint32_t)stride, cols, L, wr);
                const float corr = seg_sum_dpp<LPR>(unit_outliers<FMT_Q4K>(wr, co, u));
                if (ul == LPR - 1) dots[j][p * RW + slot] += corr;
            }
        }
        __syncthreads();
        // 5. the weighted sum in ranking order, one lane per row
        if ((int)threadIdx.x < RB) {
            const int r = r0 + (int)threadIdx.x;
            float acc = 0.0f;
            for (int q = 0; q < top_k; q++) acc = fmaf(dots[q][threadIdx.x], wgt[(size_t)t * top_k + q], acc);
            // res (may be out itself): the residual added after the sum, as layer.rs:1389 adds it
            if (r < rows) out[(size_t)t * rows + r] = res ? res[(size_t)t * rows + r] + acc : acc;
        }
        __syncthreads(); // dots and the act regions are rewritten by the next item
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
// Work items of the grouped kernels: about one per CU (the grouped kernel
// holds one workgroup per CU), plus at most one per group from rounding.
int moe_item_target(const soso_hip *h) { return h->num_cu; }
size_t moe_max_items(const soso_hip *h, size_t slots, size_t n_groups)
{
    return (size_t)moe_item_target(h) + std::min(slots, n_groups) + 1;
}

// Bytes of the three scratch regions of one MoE FFN call: f32 logits and the
// routing, the integer lists (counts, offsets, slots, work items, records),
// and the activations (gate/up results and down outputs per slot).
static void moe_scratch_sizes(const soso_hip *h, size_t n, size_t n_groups, size_t top_k, size_t hdim, size_t ffn,
                              size_t (&sz)[3])
{
    const size_t slots = n * top_k, n_g = n_groups > 0 ? n_groups : 1;
    sz[0] = (n * n_g + 2 * slots) * 4;
    sz[1] = (2 * n_g + 2 + slots + 4 * moe_max_items(h, slots, n_g) + 4 * n_g + 1) * 4;
    sz[2] = slots * (ffn + hdim) * 4;
}

static void moe_scratch_carve(const soso_hip *h, size_t n, size_t n_groups, size_t top_k, size_t ffn, char *f,
                              int *ints, float *big, MoeScratch &s)
{
    const size_t slots = n * top_k, n_g = n_groups > 0 ? n_groups : 1;
    s.logits = (float *)f;
    s.idx = (int32_t *)(s.logits + n * n_groups);
    s.wgt = (float *)(s.idx + slots);
    s.cnt = ints;
    s.offs = ints + n_groups;
    s.list = ints + 2 * n_groups + 1;
    s.items = s.list + slots;
    s.n_items = s.items + 4 * moe_max_items(h, slots, n_g);
    s.recs = s.n_items + 1;
    s.n_recs = s.recs + 4 * n_g;
    s.act = big;
    s.ydown = big + slots * ffn;
}

// Scratch slots 8..11 belong to the MoE path.
bool moe_scratch(soso_hip *h, size_t n, size_t n_groups, size_t top_k, size_t hdim, size_t ffn, MoeScratch &s)
{
    size_t sz[3];
    moe_scratch_sizes(h, n, n_groups, top_k, hdim, ffn, sz);
    char *f = (char *)scratch_get(h, 8, sz[0]);
    int *ints = (int *)scratch_get(h, 9, sz[1]);
    float *big = (float *)scratch_get(h, 10, sz[2]);
    if (!f || !ints || !big) return false;
    moe_scratch_carve(h, n, n_groups, top_k, ffn, f, ints, big, s);
    return true;
}

// The same regions carved out of one buffer of `cap` bytes at `base`, each on
// a 256-byte boundary.  Returns the bytes the call needs; s is set only when
// they fit.
size_t moe_scratch_fixed(const soso_hip *h, size_t n, size_t n_groups, size_t top_k, size_t hdim, size_t ffn,
                         void *base, size_t cap, MoeScratch &s)
{
    size_t sz[3];
    moe_scratch_sizes(h, n, n_groups, top_k, hdim, ffn, sz);
    auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t o1 = up(sz[0]), o2 = o1 + up(sz[1]), need = o2 + up(sz[2]);
    if (need > cap || !base) return need;
    char *b = (char *)base;
    moe_scratch_carve(h, n, n_groups, top_k, ffn, b, (int *)(b + o1), (float *)(b + o2), s);
    return need;
}

int launch_moe_route(soso_hip *h, const float *w, const float *x, size_t n, size_t hdim, size_t n_exp, size_t top_k,
                     const MoeScratch &s, bool sort)
{
    if (n * top_k > ROUTE_MAX_SLOTS || n_exp > 256 || (n + ROUTE_TT - 1) / ROUTE_TT > 1024)
        return set_err(h, SOSO_HIP_DECLINED, "moe route: too many slots");
    if (n == 1) {
        const dim3 grid((unsigned)((n_exp + 7) / 8), 1u);
        k_moe_route<1, 8><<<grid, 512, 0, h->stream>>>(w, x, (int)n, (int)hdim, (int)n_exp, (int)top_k, s.logits,
                                                        s.idx, s.wgt, s.cnt, s.offs, s.list, s.items, s.n_items,
                                                        moe_item_target(h), s.recs, s.n_recs, h->ticket);
    } else if (!sort) {
        // logits by two-wavefront workgroups, two tokens per wavefront (batch
        // 32: 87.3 us per layer against 87.6 with four tokens and with one),
        // then the ranking in a launch of its own
        const dim3 grid((unsigned)((n_exp + 1) / 2), (unsigned)((n + 1) / 2));
        k_moe_route<2, 4, true><<<grid, 128, 0, h->stream>>>(
            w, x, (int)n, (int)hdim, (int)n_exp, (int)top_k, s.logits, s.idx, s.wgt, s.cnt, s.offs, s.list, s.items,
            s.n_items, moe_item_target(h), s.recs, s.n_recs, h->ticket);
        int rc = hip_check(h, hipGetLastError(), "moe route launch");
        if (rc != SOSO_HIP_OK) return rc;
        k_moe_rank<<<(unsigned)((n + 3) / 4), 256, 0, h->stream>>>(s.logits, (int)n, (int)n_exp, (int)top_k, s.idx,
                                                                  s.wgt);
    } else {
        const dim3 grid((unsigned)((n_exp + 7) / 8), (unsigned)((n + ROUTE_TT - 1) / ROUTE_TT));
        k_moe_route<ROUTE_TT, 4><<<grid, 512, 0, h->stream>>>(w, x, (int)n, (int)hdim, (int)n_exp, (int)top_k,
                                                               s.logits, s.idx, s.wgt, s.cnt, s.offs, s.list, s.items,
                                                               s.n_items, moe_item_target(h), s.recs, s.n_recs,
                                                               h->ticket);
    }
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

// Weight ring depth of the grouped kernel: the deepest ring that fits the
// register file without spills at one workgroup (8 wavefronts) per CU
// (gate/up Q4_K: 239 VGPRs at depth 3; down Q4_K: 192 at depth 4; Q6_K gate/up
// spills beyond depth 2).
template <int FMT, int NMAT> constexpr int moe_depth() { return NMAT == 2 ? (FMT == FMT_Q6K ? 2 : 3) : 4; }

template <int FMT, int NMAT>
static void moe_rows_fmt(soso_hip *h, unsigned grid, size_t lds, int lpr, const uint8_t *const *A,
                         const uint8_t *const *B, size_t stride, int rows, int cols, const float *xs, int xdiv,
                         int tch, const MoeScratch &s, float *out)
{
#define MOE_CASE(LP)                                                                                                   \
    case LP:                                                                                                           \
        k_moe_rows<FMT, LP, NMAT, moe_depth<FMT, NMAT>()><<<grid, 512, lds, h->stream>>>(A, B, stride, rows, cols, xs, xdiv, s.list,        \
                                                                     s.items, s.n_items, tch, out);                   \
        break;
    switch (lpr) {
        MOE_CASE(1) MOE_CASE(2) MOE_CASE(4) MOE_CASE(8) MOE_CASE(16) MOE_CASE(32) MOE_CASE(64)
    }
#undef MOE_CASE
}

// One grouped matvec over the work items (pointer tables on the device).
// max_items bounds the items k_moe_route wrote; tch is the tokens per expert
// staged at a time (at most the tokens of the call).
static int launch_moe_mv(soso_hip *h, uint8_t dtype, int nmat, const uint8_t *const *A, const uint8_t *const *B,
                         size_t rows, size_t cols, size_t max_items, size_t tch, const float *xs, int xdiv,
                         const MoeScratch &s, float *out)
{
    const int U = (int)(cols / 64);
    if (U < 1 || U > 64 || cols % 128 || !packed_shape_ok(dtype, rows, cols))
        return set_err(h, SOSO_HIP_DECLINED, "moe: expert shape not handled here");
    const int lpr = U <= 1 ? 1 : U <= 2 ? 2 : U <= 4 ? 4 : U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
    const size_t rows_per_pass = 8 * (64 / lpr);
    const size_t passes = (rows + rows_per_pass - 1) / rows_per_pass;
    tch = std::max<size_t>(1, std::min<size_t>(tch, 64));
    const size_t tok_bytes = (stage_lds_bytes_o(cols) + 15) & ~(size_t)15;
    while (tch > 1 && tok_bytes * tch > h->max_lds) tch--;
    const size_t lds = tok_bytes * tch;
    if (lds > h->max_lds) return set_err(h, SOSO_HIP_DECLINED, "moe: x does not fit in LDS");
    const unsigned grid = (unsigned)std::max<size_t>(1, max_items);
    const size_t stride = packed_row_stride(dtype, cols);
    if ((passes + 2) * rows_per_pass * stride >= ((size_t)1 << 31))
        return set_err(h, SOSO_HIP_DECLINED, "moe: expert matrix exceeds 2 GiB");
    const int ri = (int)rows, ci = (int)cols, ti = (int)tch;
    switch (dtype) {
    case SOSO_HIP_DTYPE_Q4_K:
        if (nmat == 2) moe_rows_fmt<FMT_Q4K, 2>(h, grid, lds, lpr, A, B, stride, ri, ci, xs, xdiv, ti, s, out);
        else moe_rows_fmt<FMT_Q4K, 1>(h, grid, lds, lpr, A, B, stride, ri, ci, xs, xdiv, ti, s, out);
        break;
    case SOSO_HIP_DTYPE_Q8_0:
        if (nmat == 2) moe_rows_fmt<FMT_Q80, 2>(h, grid, lds, lpr, A, B, stride, ri, ci, xs, xdiv, ti, s, out);
        else moe_rows_fmt<FMT_Q80, 1>(h, grid, lds, lpr, A, B, stride, ri, ci, xs, xdiv, ti, s, out);
        break;
    case SOSO_HIP_DTYPE_Q6_K:
        if (nmat == 2) moe_rows_fmt<FMT_Q6K, 2>(h, grid, lds, lpr, A, B, stride, ri, ci, xs, xdiv, ti, s, out);
        else moe_rows_fmt<FMT_Q6K, 1>(h, grid, lds, lpr, A, B, stride, ri, ci, xs, xdiv, ti, s, out);
        break;
    default: return set_err(h, SOSO_HIP_DECLINED, "moe: expert dtype not handled here");
    }
    return hip_check(h, hipGetLastError(), "moe mv launch");
}

// ---------------------------------------------------------------------------
// One token through a registered layer, ranked by the expert kernel itself:
// logits (k_moe_route<1, 8, true>: no ticket, no sort), gate/up + swiglu of
// the ranked experts (k_moe_rows<..., SELF>), down and the ranking-order sum
// (k_moe_down_comb).  The route kernel's last-workgroup ranking and sort are
// chains of dependent round trips; here every expert workgroup ranks the
// token's logits itself, which costs less than those chains.
// ---------------------------------------------------------------------------
template <int FMT>
static void moe_rows_self(soso_hip *h, unsigned grid, size_t lds, int lpr, const uint8_t *const *A,
                          const uint8_t *const *B, size_t stride, int rows, int cols, const float *x, int top_k,
                          const MoeSelf &sr, float *out)
{
#define MOE_SELF_CASE(LP)                                                                                          \
    case LP:                                                                                                       \
        k_moe_rows<FMT, LP, 2, moe_depth<FMT, 2>(), true><<<grid, 512, lds, h->stream>>>(                          \
            A, B, stride, rows, cols, x, top_k, nullptr, nullptr, nullptr, 1, out, sr);                            \
        break;
    switch (lpr) {
        MOE_SELF_CASE(1) MOE_SELF_CASE(2) MOE_SELF_CASE(4) MOE_SELF_CASE(8) MOE_SELF_CASE(16) MOE_SELF_CASE(32)
        MOE_SELF_CASE(64)
    }
#undef MOE_SELF_CASE
}

static int launch_down_comb(soso_hip *h, const uint8_t *const *tab, size_t n_exp, size_t rows, size_t cols,
                            const float *act, const int32_t *idx, const float *wgt, size_t n, size_t top_k,
                            const float *res, float *out);

// The single-token path's limits (launch_moe_ffn1): why a layer cannot take
// it, or null.
const char *moe_ffn1_unsupported(const soso_hip *h, const MoeLayer &m)
{
    const size_t hdim = m.hdim, ffn = m.ffn, top_k = m.top_k, n_exp = m.n_exp;
    const int U = (int)(hdim / 64);
    const size_t Uf = ffn / 64;
    const bool gu_ok = (m.dt_gu == SOSO_HIP_DTYPE_Q4_K || m.dt_gu == SOSO_HIP_DTYPE_Q8_0 ||
                        m.dt_gu == SOSO_HIP_DTYPE_Q6_K) &&
                       U >= 1 && U <= 64 && hdim % 128 == 0 && packed_shape_ok(m.dt_gu, ffn, hdim);
    if (!gu_ok) return "gate/up: Q4_K, Q8_0 or Q6_K rows of 128 to 4096 columns (a multiple of 128)";
    const bool down_ok = m.dt_down == SOSO_HIP_DTYPE_Q4_K && ffn % 256 == 0 && Uf >= 4 && Uf <= 8 * (size_t)MDC_XR &&
                         ((stage_lds_bytes_o(ffn) + 15) & ~(size_t)15) * MDC_K <= h->max_lds &&
                         packed_shape_ok(m.dt_down, hdim, ffn);
    if (!down_ok) return "down: Q4_K, expert width 256 to 2048 (a multiple of 256)";
    if (top_k == 0 || top_k > (size_t)MOE_SELF_K || n_exp > 256) return "top_k above 8 or more than 256 experts";
    const int lpr = U <= 1 ? 1 : U <= 2 ? 2 : U <= 4 ? 4 : U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
    const size_t rows_per_pass = 8 * (64 / lpr), passes = (ffn + rows_per_pass - 1) / rows_per_pass;
    const size_t stride = packed_row_stride(m.dt_gu, hdim);
    const size_t lds = (stage_lds_bytes_o(hdim) + 15) & ~(size_t)15;
    if (lds > h->max_lds || (passes + 2) * rows_per_pass * stride >= ((size_t)1 << 31)) return "expert too large";
    return nullptr;
}

// res: added to the output after the ranking-order sum (may be out itself), or null.
// norm_w: x is h and the FFN's input is rmsnorm(h) * norm_w (moe_ffn1_norm_ok).
bool moe_ffn1_norm_ok(const MoeLayer &m) { return m.hdim <= 2048; } // the route's one-step rows (Q = 8)

int launch_moe_ffn1(soso_hip *h, const MoeLayer &m, const float *x, const MoeScratch &s, float *out, const float *res,
                    const float *norm_w, float eps)
{
    if (moe_ffn1_unsupported(h, m)) return set_err(h, SOSO_HIP_DECLINED, "moe ffn1: shape for the general path");
    if (norm_w && !moe_ffn1_norm_ok(m)) return set_err(h, SOSO_HIP_DECLINED, "moe ffn1: folded norm width");
    const size_t hdim = m.hdim, ffn = m.ffn, top_k = m.top_k, n_exp = m.n_exp;
    const int U = (int)(hdim / 64);
    const int lpr = U <= 1 ? 1 : U <= 2 ? 2 : U <= 4 ? 4 : U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
    const size_t stride = packed_row_stride(m.dt_gu, hdim);
    const size_t lds = (stage_lds_bytes_o(hdim) + 15) & ~(size_t)15;
    // the route kernel's item count for one token: about moe_item_target
    // chunks in all, the same share for every ranked expert
    const int chunks = std::max(1, (moe_item_target(h) + (int)top_k / 2) / (int)top_k);
    // one expert row per wavefront, two per workgroup: every wavefront reads the
    // token's x (and the norm's weights) besides its row, so the launch spreads
    // over 64 CUs instead of 16 (MI355X, Qwen3-30B-A3B-like layer: 18.6 ->
    // 18.0 us per batch-1 layer, 2.29 -> 2.19 ms per 48-layer decode step; one
    // wavefront per workgroup measured the same)
    k_moe_route<1, 8, true><<<dim3((unsigned)((n_exp + 1) / 2), 1u), 128, 0, h->stream>>>(
        (const float *)m.router->dev, x, 1, (int)hdim, (int)n_exp, (int)top_k, s.logits, s.idx, s.wgt, s.cnt, s.offs,
        s.list, s.items, s.n_items, moe_item_target(h), s.recs, s.n_recs, h->ticket, norm_w, eps);
    int rc = hip_check(h, hipGetLastError(), "moe ffn1 route launch");
    if (rc != SOSO_HIP_OK) return rc;
    MoeSelf sr;
    sr.logits = s.logits;
    sr.n_exp = (int)n_exp;
    sr.top_k = (int)top_k;
    sr.chunks = chunks;
    sr.idx = s.idx;
    sr.wgt = s.wgt;
    sr.norm_w = norm_w;
    sr.eps = eps;
    const unsigned grid = (unsigned)(top_k * chunks);
    const uint8_t *const *A = m.tab, *const *B = m.tab + n_exp;
    switch (m.dt_gu) {
    case SOSO_HIP_DTYPE_Q4_K: moe_rows_self<FMT_Q4K>(h, grid, lds, lpr, A, B, stride, (int)ffn, (int)hdim, x, (int)top_k, sr, s.act); break;
    case SOSO_HIP_DTYPE_Q8_0: moe_rows_self<FMT_Q80>(h, grid, lds, lpr, A, B, stride, (int)ffn, (int)hdim, x, (int)top_k, sr, s.act); break;
    default: moe_rows_self<FMT_Q6K>(h, grid, lds, lpr, A, B, stride, (int)ffn, (int)hdim, x, (int)top_k, sr, s.act); break;
    }
    rc = hip_check(h, hipGetLastError(), "moe ffn1 gate/up launch");
    if (rc != SOSO_HIP_OK) return rc;
    return launch_down_comb(h, m.tab + 2 * n_exp, n_exp, hdim, ffn, s.act, s.idx, s.wgt, 1, top_k, res, out);
}

// gate/up + swiglu, down, combine for the slots grouped in s.cnt/offs/list.
// tab: 3 * n_groups device pointers (gate[], up[], down[]).
// Down + combine in one launch for few tokens (k_moe_down_comb): at most
// this many tokens, where the ranked experts of different tokens rarely
// coincide and reading an expert once per token costs about what grouping saves.
constexpr size_t MDC_MAX_TOKENS = 4;

static int launch_down_comb(soso_hip *h, const uint8_t *const *tab, size_t n_exp, size_t rows, size_t cols,
                            const float *act, const int32_t *idx, const float *wgt, size_t n, size_t top_k,
                            const float *res, float *out)
{
    const int U = (int)(cols / 64);
    const int lpr = U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
    const size_t rw = 64 / lpr;
    // rows per item: the most passes that still give every CU a workgroup
    int P = 4;
    while (P > 1 && n * ((rows + rw * P - 1) / (rw * P)) < (size_t)h->num_cu) P >>= 1;
    const size_t items = n * ((rows + rw * P - 1) / (rw * P));
    const size_t lds = ((stage_lds_bytes_o(cols) + 15) & ~(size_t)15) * MDC_K;
    const size_t stride = packed_row_stride(SOSO_HIP_DTYPE_Q4_K, cols);
    const unsigned grid = (unsigned)std::min<size_t>(items, 4 * (size_t)h->num_cu);
    const int ri = (int)rows, ci = (int)cols, ne = (int)n_exp, ni = (int)n, ki = (int)top_k;
#define MDC_CASE(LP)                                                                                                   \
    case LP:                                                                                                           \
        if (P == 4)                                                                                                    \
            k_moe_down_comb<LP, 4><<<grid, 512, lds, h->stream>>>(tab, stride, ri, ci, ne, act, idx, wgt, ni, ki, res, out); \
        else if (P == 2)                                                                                               \
            k_moe_down_comb<LP, 2><<<grid, 512, lds, h->stream>>>(tab, stride, ri, ci, ne, act, idx, wgt, ni, ki, res, out); \
        else                                                                                                           \
            k_moe_down_comb<LP, 1><<<grid, 512, lds, h->stream>>>(tab, stride, ri, ci, ne, act, idx, wgt, ni, ki, res, out); \
        break;
    switch (lpr) {
        MDC_CASE(8) MDC_CASE(16) MDC_CASE(32) MDC_CASE(64)
    }
#undef MDC_CASE
    return hip_check(h, hipGetLastError(), "moe down+combine launch");
}

int launch_moe_experts(soso_hip *h, const float *xs, size_t n, size_t hdim, size_t ffn, size_t top_k,
                       uint8_t dt_gu, uint8_t dt_down, const uint8_t *const *tab, size_t n_groups, const float *wgt,
                       const uint8_t *use, const int32_t *route_idx, const MoeScratch &s, float *out,
                       const MoeLayer *layer, bool scan)
{
    const size_t max_items = moe_max_items(h, n * top_k, n_groups);
    // scan: the route wrote only the ranking (route_idx); each expert
    // workgroup of the matrix-core kernels finds its slots there
    if (scan && (!route_idx || use || !mfma_moe_scan_ok(n, top_k, n_groups, dt_gu, dt_down, hdim, ffn)))
        return set_err(h, SOSO_HIP_ERR_ARG, "moe experts: scanning the ranking needs the matrix-core path");
    const int32_t *sidx = scan ? route_idx : nullptr;
    // two or more slots per active expert on average: the matrix-core path
    // (its cost per weight row is flat up to 8 tokens); fewer: the dot4 path
    const size_t slots = n * top_k, max_recs = std::min(n_groups, slots);
    const bool many = slots >= 2 * max_recs;
    int rc;
    // a registered layer's tile-major copies, where it has them
    const bool tgu = layer && layer->tiled && layer->tiled_gu, tdn = layer && layer->tiled && layer->tiled_down;
    const uint8_t *const *ttab = layer ? layer->tiled : nullptr;
    if (many && dt_gu == SOSO_HIP_DTYPE_Q4_K && mfma_shape_ok(dt_gu, ffn, hdim))
        rc = launch_mfma_moe(h, 2, tgu ? ttab : tab, (tgu ? ttab : tab) + n_groups, ffn, hdim, max_recs, xs, (int)top_k,
                             s.list, s.recs, s.n_recs, s.act, tgu, sidx, n * top_k);
    else
        rc = launch_moe_mv(h, dt_gu, 2, tab, tab + n_groups, ffn, hdim, max_items, n, xs, (int)top_k, s, s.act);
    // few tokens with the device's own routing: down and the weighted sum in one launch
    const size_t Uf = ffn / 64;
    if (rc == SOSO_HIP_OK && route_idx && !use && n <= MDC_MAX_TOKENS && top_k <= (size_t)MDC_K &&
        dt_down == SOSO_HIP_DTYPE_Q4_K && ffn % 256 == 0 && Uf >= 4 && Uf <= 8 * MDC_XR &&
        ((stage_lds_bytes_o(ffn) + 15) & ~(size_t)15) * MDC_K <= h->max_lds && packed_shape_ok(dt_down, hdim, ffn))
        return launch_down_comb(h, tab + 2 * n_groups, n_groups, hdim, ffn, s.act, route_idx, wgt, n, top_k, nullptr,
                                out);
    if (rc == SOSO_HIP_OK) {
        if (many && dt_down == SOSO_HIP_DTYPE_Q4_K && mfma_shape_ok(dt_down, hdim, ffn))
            rc = launch_mfma_moe(h, 1, (tdn ? ttab : tab) + 2 * n_groups, nullptr, hdim, ffn, max_recs, s.act, 1, s.list,
                                 s.recs, s.n_recs, s.ydown, tdn, sidx, n * top_k);
        else
            rc = launch_moe_mv(h, dt_down, 1, tab + 2 * n_groups, nullptr, hdim, ffn, max_items, n, s.act, 1, s,
                               s.ydown);
    }
    if (rc != SOSO_HIP_OK) return rc;
    const dim3 grid((unsigned)((hdim + 255) / 256), (unsigned)n);
    k_moe_combine<<<grid, 256, 0, h->stream>>>(s.ydown, wgt, use, (int)n, (int)hdim, (int)top_k, out);
    return hip_check(h, hipGetLastError(), "moe combine launch");
}

// ---------------------------------------------------------------------------
// Shared expert of an MoE block (GpuDispatch::moe_compartido, gpu.rs:518-534;
// soso's CPU path bloque35.rs:950-985): gate / up / down run as matmuls, then
// these two finish it -- SwiGLU (gemm.rs:210-226) and the per-token sigmoid
// gate sigmoid(x_t . ffn_gate_inp_shexp) (bloque35.rs:955-960).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_shared_swiglu(const float *__restrict__ g, float *__restrict__ u, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        u[i] = silu(g[i]) * u[i];
}

// one workgroup per token: the dot in one 256-thread reduction, then the scale
__global__ void __launch_bounds__(256) k_shared_gate(const float *__restrict__ x, const float *__restrict__ pg_w,
                                                      float *__restrict__ y, int hdim)
{
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *xt = x + (size_t)t * hdim;
    float acc = 0.0f;
    for (int i = tid; i < hdim; i += 256) acc = fmaf(xt[i], pg_w[i], acc);
    acc = seg_sum_dpp<64>(acc);
    if ((tid & 63) == 63) red[tid >> 6] = acc;
    __syncthreads();
    const float pg = (red[0] + red[1]) + (red[2] + red[3]);
    const float s = 1.0f / (1.0f + expf(-pg));
    float *yt = y + (size_t)t * hdim;
    for (int i = tid; i < hdim; i += 256) yt[i] *= s;
}

int launch_shared_swiglu(soso_hip *h, const float *g, float *u, size_t n)
{
    const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    k_shared_swiglu<<<grid, 256, 0, h->stream>>>(g, u, n);
    return hip_check(h, hipGetLastError(), "shared swiglu launch");
}

int launch_shared_gate(soso_hip *h, const float *x, const float *pg_w, float *y, size_t n, size_t hdim)
{
    k_shared_gate<<<(unsigned)n, 256, 0, h->stream>>>(x, pg_w, y, (int)hdim);
    return hip_check(h, hipGetLastError(), "shared gate launch");
}
