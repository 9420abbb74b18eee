// mv_core.hpp -- device building blocks of the block-quantized matvecs:
// x staging into integer digits, per-format lane units (loads and the
// fused dequant-dot), and the cross-lane row gather.  Shared by the matvec
// kernels (k_matvec.hip) and the MoE expert kernels (k_moe.hip).
//
// Formats and arithmetic follow crates/sosomodel/src/dequant.rs (Q8_0, Q4_K)
// and crates/gguf2som/src/lib.rs:1639-1661 (Q6_K).
#pragma once

#include "internal.hpp"

// ---------------------------------------------------------------------------
// x staging (one barrier)
// Each thread converts chunks of 8 elements; the 16 chunks of a 128-element
// block sit in one 16-lane DPP row, which agrees on the block's exponent e
// (max|x| * 2^e <= 2^22).  Every element becomes the integer X = rint(x*2^e)
// (|X| <= 2^22, 22 significant bits), written as three balanced signed
// digits X = d2*2^16 + d1*2^8 + d0 (d0, d1 in [-128, 127], |d2| <= 64).  LDS
// receives, per 4-element group, one dword of bytes per digit, plus
//   s16[i] = f32 sum of x[16i .. 16i+16) (unscaled), kx[b] = e of block b.
// The weights' integer codes then meet x in v_dot4_i32_i8 (exact int32 sums
// per digit), and only the three digit sums of a sub-block are rounded.
// ---------------------------------------------------------------------------
enum { FMT_Q4K = 0, FMT_Q80 = 1, FMT_Q6K = 2 };

constexpr int XDIG = 3;        // digits per element
constexpr int XD = 16 * XDIG;  // dwords of x per lane unit (16 groups)

// Unit u and register group gi (0..15) of 4-element group g.  Q4_K and Q8_0
// units are 16 consecutive groups; a Q6_K unit (u = 4 sb + 2 h + kk) takes,
// for i, t < 4, group sb*64 + h*32 + 8i + 4kk + t as register group 4i + t.
template <int FMT>
__device__ __forceinline__ void xunit(int g, int &u, int &gi)
{
    if constexpr (FMT == FMT_Q6K) {
        const int sb = g >> 6, h = (g >> 5) & 1, i = (g >> 3) & 3, kk = (g >> 2) & 1, t = g & 3;
        u = 4 * sb + 2 * h + kk;
        gi = 4 * i + t;
    } else {
        u = g >> 4;
        gi = g & 15;
    }
}

// LDS dword of register dword w (= 3 gi + digit) of unit u: dwords 4r..4r+3
// of every unit sit in one 16-byte slot r*U + u, so the 64 lanes of a
// wavefront read 64 consecutive slots (no bank conflicts).
__device__ __forceinline__ int xdw(int u, int w, int U) { return ((w >> 2) * U + u) * 4 + (w & 3); }

// Three balanced base-256 digits of the four elements of v (scaled by 2^e),
// packed one byte per element per digit: X = rint(v 2^e) = d0 + 256 d1 +
// 65536 d2 with every d in [-128, 127].
//
// |X| <= 2^22 (the block exponent guarantees it), so adding 1.5 * 2^23 rounds
// v 2^e to an integer with ties to even (as rintf) and leaves X + 2^22 in the
// low mantissa bits.  Y = X + 0x808080 is then in [0, 2^24) and byte k of Y
// is digit k plus 128, so d_k = byte_k(Y) ^ 0x80: the same digits as the
// repeated "d = int8(X); X = (X - d) / 256" (checked for every |X| <= 2^22).
// Seven byte permutes gather the bytes of the four elements digit by digit.
__device__ __forceinline__ void digits4(float4 v, int e, uint32_t (&d)[XDIG])
{
    constexpr float MAGIC = 12582912.0f; // 1.5 * 2^23
    constexpr uint32_t OFF = 0x4B400000u - 0x808080u;
    const uint32_t y0 = __float_as_uint(__fadd_rn(ldexpf(v.x, e), MAGIC)) - OFF;
    const uint32_t y1 = __float_as_uint(__fadd_rn(ldexpf(v.y, e), MAGIC)) - OFF;
    const uint32_t y2 = __float_as_uint(__fadd_rn(ldexpf(v.z, e), MAGIC)) - OFF;
    const uint32_t y3 = __float_as_uint(__fadd_rn(ldexpf(v.w, e), MAGIC)) - OFF;
    // v_perm_b32 (s0, s1, sel): selector byte 0-3 picks byte of s1, 4-7 of s0
    const uint32_t A = __builtin_amdgcn_perm(y1, y0, 0x05010400u); // y0b0 y1b0 y0b1 y1b1
    const uint32_t B = __builtin_amdgcn_perm(y3, y2, 0x05010400u); // y2b0 y3b0 y2b1 y3b1
    const uint32_t C = __builtin_amdgcn_perm(y1, y0, 0x0c0c0602u); // y0b2 y1b2
    const uint32_t D = __builtin_amdgcn_perm(y3, y2, 0x0c0c0602u); // y2b2 y3b2
    d[0] = __builtin_amdgcn_perm(B, A, 0x05040100u) ^ 0x80808080u;
    d[1] = __builtin_amdgcn_perm(B, A, 0x07060302u) ^ 0x80808080u;
    d[2] = __builtin_amdgcn_perm(D, C, 0x05040100u) ^ 0x80808080u;
}

// A block of x holding an Inf or a NaN gets this exponent.  Its unscale
// factor is NaN, so every dot product that meets the block is NaN, as the
// CPU's f32 dot of such a row is Inf or NaN; the block's digits (of a
// non-finite value) are never used for a finite result.
constexpr int KX_NONFINITE = 0x40000000;
__device__ __forceinline__ float block_unscale(int k)
{
    return k == KX_NONFINITE ? __builtin_nanf("") : ldexpf(1.0f, -k);
}

// ---------------------------------------------------------------------------
// Outliers.  An element of x far above the rest of its 128-element block
// would set the block's exponent alone and leave the other elements few
// significant bits: where those elements carry the product (a large element
// meeting a small or zero weight), the error would be relative to the large
// element, not to the result.  Kernels that stage with OUTL therefore take
// such elements out of the digits.  An element is an outlier when it exceeds
// 16 times the third largest of the block's sixteen 8-element chunk maxima
// (ties counted): at most two chunks can hold outliers (so at most 16 per
// block), and a block without a few dominant elements (an N(0,1) block, for
// one) has none.  Outliers get zero digits and stay out of the block's
// exponent and f32 sums; their (position, value) pairs go to the block's
// list in LDS, in a fixed order, and the matvec adds w * x for each, with w
// dequantized exactly as the reference dequantizes (unit_outliers).
// List of block b: dword 0 the count, dwords 1-4 the positions (bytes, 0..127
// inside the block), dwords 8-23 the values.
// ---------------------------------------------------------------------------
constexpr int OUT_MAX = 16;
constexpr int OUT_DW = 24;
__host__ __device__ inline size_t out_lds_bytes(size_t cols) { return (cols + 127) / 128 * OUT_DW * 4; }
// the lists follow the exponents kx (one int per 128-element block)
__device__ __forceinline__ uint32_t *out_lists(int *kx, int cols) { return (uint32_t *)(kx + ((cols + 127) >> 7)); }
__device__ __forceinline__ const uint32_t *out_lists(const int *kx, int cols)
{
    return (const uint32_t *)(kx + ((cols + 127) >> 7));
}

// lanes of this lane's 16-lane row for which pred holds
__device__ __forceinline__ int row16_count(bool pred)
{
    const uint64_t b = __ballot(pred);
    return __popcll((b >> (threadIdx.x & 48u)) & 0xFFFFull);
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

// The outlier threshold of a 128-element block from its sixteen 8-element
// chunk maxima (m: this lane's chunk, one chunk per lane of the 16-lane row;
// m1: the block maximum): 16 times the third largest chunk maximum, ties
// counted; infinite for a non-finite block (its result is NaN anyway).
__device__ __forceinline__ float outlier_thr16(float m, float m1)
{
    const int n1 = row16_count(m == m1);
    const float m2 = row16_max(m < m1 ? m : -1.0f);
    const int n2 = row16_count(m == m2);
    const float m3b = row16_max(m < m2 ? m : -1.0f);
    return m1 < INFINITY ? 16.0f * (n1 >= 3 ? m1 : n1 + n2 >= 3 ? m2 : m3b) : INFINITY;
}

// One 8-element chunk c (thread lane == c % 64).  Every lane of the 16-lane
// DPP row takes part (invalid chunks carry zeros); only valid ones store.
// FAST (with OUTL): a wavefront that would have to search for outliers
// stages nothing and returns false (uniform), for the caller to stage the
// chunk again through the full path; otherwise returns true.  found (OUTL,
// when given) is set when some block of the wavefront has outliers.
template <int FMT, bool OUTL = false, bool FAST = false>
__device__ __forceinline__ bool stage_chunk(float4 v0, float4 v1, int c, bool valid, int U, uint32_t *xd, float *s16,
                                            int *kx, bool *found = nullptr)
{
    float m = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                    fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
    float sm = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w));
    // fmaxf passes over a NaN, which the sum keeps: a NaN element marks the
    // block as an infinite maximum would
    if (sm != sm) m = INFINITY;
    uint32_t om = 0; // OUTL: bit i = element i of the chunk is an outlier
    const float vo[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    bool none = !OUTL; // OUTL: no block of the wavefront has an outlier, m is the block maximum
    if constexpr (OUTL) {
        // maxima of the four 4-chunk quads, then of the block; the third
        // largest chunk maximum is at least the smallest quad maximum (the
        // two largest chunks sit in at most two quads), so blocks whose
        // maximum is within 16x of their smallest quad maximum have no
        // outlier, and a wavefront of such blocks (N(0,1), Laplace or
        // silu(g) * u blocks, all but a few percent of Student-t(3) ones)
        // skips the search
        float q = fmaxf(m, dpp_f<0xB1>(m));
        q = fmaxf(q, dpp_f<0x4E>(q));
        const float h = fmaxf(q, dpp_f<0x141>(q));
        const float m1 = fmaxf(h, dpp_f<0x140>(h));
        float qn = fminf(q, dpp_f<0x141>(q));
        qn = fminf(qn, dpp_f<0x140>(qn));
        none = __ballot(m1 > 16.0f * qn) == 0;
        if (FAST && !none) return false;
        if (__builtin_expect(!none, 0)) {
            const float thr = outlier_thr16(m, m1);
            none = __ballot(m1 > thr) == 0;
            if (found && !none) *found = true; // (uniform) some block of the wavefront has outliers
            if (__builtin_expect(!none, 0)) {
                float km = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (fabsf(vv[i]) > thr) {
                        om |= 1u << i;
                        vv[i] = 0.0f;
                    }
                    km = fmaxf(km, fabsf(vv[i]));
                }
                m = km;
                sm = ((vv[0] + vv[1]) + (vv[2] + vv[3])) + ((vv[4] + vv[5]) + (vv[6] + vv[7]));
            }
        }
        if (none) m = m1;
    }
    if (!none || !OUTL) m = row16_max(m);
    const bool finite = m < INFINITY;
    const int e = (m > 0.0f && finite) ? 22 - __builtin_amdgcn_frexp_expf(m) : 0;
    sm += dpp_f<0xB1>(sm);
    if constexpr (OUTL) {
        uint32_t *ol = out_lists(kx, 64 * U) + (c >> 4) * OUT_DW;
        if (__builtin_expect(none, 1)) {
            if (valid && (c & 15) == 0) ol[0] = 0u;
        } else {
            // the block's list, in chunk order then element order: an
            // inclusive scan of the chunks' counts over the 16-lane row gives
            // each chunk its first slot
            const int cnt = __popc(om);
            int incl = cnt;
            incl += dpp_i<0x111>(incl); // row_shr:1 (lanes with no source add 0)
            incl += dpp_i<0x112>(incl);
            incl += dpp_i<0x114>(incl);
            incl += dpp_i<0x118>(incl);
            const int tot = (int)row16_max((float)incl);
            if (valid) {
                if ((c & 15) == 0) ol[0] = (uint32_t)tot;
                int slot = incl - cnt;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (((om >> i) & 1u) && slot < OUT_MAX) {
                        ((uint8_t *)(ol + 1))[slot] = (uint8_t)(8 * (c & 15) + i);
                        ol[8 + slot] = __float_as_uint(vo[i]);
                        slot++;
                    }
                }
            }
        }
    }
    if (valid) {
        uint32_t d0[XDIG], d1[XDIG];
        digits4(make_float4(vv[0], vv[1], vv[2], vv[3]), e, d0);
        digits4(make_float4(vv[4], vv[5], vv[6], vv[7]), e, d1);
        if constexpr (FMT == FMT_Q6K) {
            int u, gi;
            xunit<FMT>(2 * c, u, gi);
#pragma unroll
            for (int k = 0; k < XDIG; k++) xd[xdw(u, XDIG * gi + k, U)] = d0[k];
            xunit<FMT>(2 * c + 1, u, gi);
#pragma unroll
            for (int k = 0; k < XDIG; k++) xd[xdw(u, XDIG * gi + k, U)] = d1[k];
        } else {
            // groups 2m, 2m + 1 (m = c mod 8) of unit c / 8 are register dwords
            // 6m .. 6m + 5 (xdw): one aligned 16-byte and one 8-byte store
            // instead of six 4-byte ones (on MI355X a 4096 x 4096 Q4_K matvec
            // went from 5.07 to 4.30 us with this alone)
            const int u = c >> 3, mm = c & 7, s0 = (3 * mm) >> 1;
            uint4 *slot = (uint4 *)xd + s0 * U + u;
            if ((mm & 1) == 0) {
                *slot = make_uint4(d0[0], d0[1], d0[2], d1[0]);
                *(uint2 *)(slot + U) = make_uint2(d1[1], d1[2]);
            } else {
                *((uint2 *)slot + 1) = make_uint2(d0[0], d0[1]);
                slot[U] = make_uint4(d0[2], d1[0], d1[1], d1[2]);
            }
        }
        if ((c & 1) == 0) s16[c >> 1] = sm;
        if ((c & 15) == 0) kx[c >> 4] = finite ? e : KX_NONFINITE;
    }
    return true;
}

// x is read in two steps so that its loads can be issued ahead of the weight
// loads: vector-memory results return in issue order, so x loads issued after
// a ring of weight loads would wait for all of those weights.
// The staging functions take the workgroup's thread count as an argument:
// kernels launched at one fixed size pass it as a constant, so that it is
// not re-read from the dispatch arguments (a vector load, whose wait would
// also wait for every weight load issued before it).
// XP chunks per thread are loaded ahead (the rest, past 8 * XP * nthr
// columns, are loaded as they are staged); kernels pick the smallest XP that
// covers their rows, as every unrolled round is code the wavefronts fetch.
template <int XP>
struct XPre {
    float4 v[2 * XP];
};

template <int XP>
__device__ __forceinline__ void stage_x_issue(const float *__restrict__ x, int cols, XPre<XP> &p, int nthr)
{
    const int nch = cols >> 3;
    const float4 *x4 = (const float4 *)x;
#pragma unroll
    for (int j = 0; j < XP; j++) {
        const int c = j * nthr + threadIdx.x;
        p.v[2 * j] = p.v[2 * j + 1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < nch) {
            p.v[2 * j] = x4[2 * c];
            p.v[2 * j + 1] = x4[2 * c + 1];
        }
    }
}

// nthr % 64 == 0: chunk c sits in lane c % 64, so the 16 chunks of a
// block form one DPP row.  Loop bounds are uniform over the workgroup (cols
// is a multiple of 64, so a trailing block may be half full).
template <int FMT, bool OUTL, int XP>
__device__ void stage_x_finish(const XPre<XP> &p, const float *__restrict__ x, int cols, uint32_t *xp, float *s16,
                               int *kx, int nthr)
{
    const int nch = cols >> 3, U = cols >> 6;
    // with several rounds, the rounds held in registers take the fast path
    // only, and the (rare) rounds that need the outlier search are staged
    // again below from x, through one copy of the full path
    constexpr bool FAST = OUTL && XP > 1;
    uint32_t redo = 0; // rounds to stage again (uniform)
#pragma unroll
    for (int j = 0; j < XP; j++) {
        const int base = j * nthr;
        if (base < nch) {
            const int c = base + threadIdx.x;
            if (!stage_chunk<FMT, OUTL, FAST>(p.v[2 * j], p.v[2 * j + 1], c, c < nch, U, xp, s16, kx)) redo |= 1u << j;
        }
    }
    const float4 *x4 = (const float4 *)x;
    auto full = [&](int base) {
        const int c = base + threadIdx.x;
        const bool valid = c < nch;
        float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
        if (valid) {
            v0 = x4[2 * c];
            v1 = x4[2 * c + 1];
        }
        stage_chunk<FMT, OUTL>(v0, v1, c, valid, U, xp, s16, kx);
    };
    // the rounds past the registers, and the rounds to stage again
    const int j0 = redo ? __builtin_ctz(redo) : XP;
#pragma unroll 1
    for (int j = j0, base = j0 * nthr; base < nch; j++, base += nthr)
        if (j >= XP || ((redo >> j) & 1u)) full(base);
    __syncthreads();
}

// RMSNorm folded into the staging (crates/soso-llm-core/src/gemm.rs:93-100):
// every workgroup takes sum(x^2) over the whole vector itself, then stages
// (x_i * scale) * w_i with scale = 1 / sqrt(sum / n + eps).
// XP chunks per thread, all loaded ahead (cols <= 8 * XP * nthr)
template <int XP>
struct XPreN {
    float4 v[2 * XP], w[2 * XP];
};

template <int XP>
__device__ __forceinline__ void stage_xn_issue(const float *__restrict__ x, const float *__restrict__ w, int cols,
                                               XPreN<XP> &p, int nthr)
{
    const int nch = cols >> 3;
    const float4 *x4 = (const float4 *)x, *w4 = (const float4 *)w;
#pragma unroll
    for (int j = 0; j < XP; j++) {
        const int c = j * nthr + threadIdx.x;
        p.v[2 * j] = p.v[2 * j + 1] = p.w[2 * j] = p.w[2 * j + 1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < nch) {
            p.v[2 * j] = x4[2 * c];
            p.v[2 * j + 1] = x4[2 * c + 1];
            p.w[2 * j] = w4[2 * c];
            p.w[2 * j + 1] = w4[2 * c + 1];
        }
    }
}

__device__ __forceinline__ float sq4(float4 v) { return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w); }
__device__ __forceinline__ float4 norm4(float4 v, float s, float4 w)
{
    return make_float4(__fmul_rn(__fmul_rn(v.x, s), w.x), __fmul_rn(__fmul_rn(v.y, s), w.y),
                       __fmul_rn(__fmul_rn(v.z, s), w.z), __fmul_rn(__fmul_rn(v.w, s), w.w));
}

// red: 16 floats of LDS.
template <int FMT, bool OUTL, int XP>
__device__ void stage_xn_finish(const XPreN<XP> &p, int cols, float eps, uint32_t *xp, float *s16, int *kx, float *red,
                                int nthr)
{
    const int nch = cols >> 3, U = cols >> 6;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < XP; j++) ss += sq4(p.v[2 * j]) + sq4(p.v[2 * j + 1]);
    ss = seg_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < (nthr >> 6); i++) tot += red[i];
    const float scale = 1.0f / sqrtf(tot / (float)cols + eps);
#pragma unroll
    for (int j = 0; j < XP; j++) {
        const int base = j * nthr;
        if (base < nch) {
            const int c = base + threadIdx.x;
            stage_chunk<FMT, OUTL>(norm4(p.v[2 * j], scale, p.w[2 * j]), norm4(p.v[2 * j + 1], scale, p.w[2 * j + 1]),
                                   c, c < nch, U, xp, s16, kx);
        }
    }
    __syncthreads();
}

// XS_RMSNORM_P4: x is the sum of the MV_SEG column-segment partials of the
// matvec that produced them (segment 0's with the residual in it), added in
// segment order: ((p0 + p1) + p2) + p3.  One round (cols <= 8 * nthr).
// Workgroup b writes the sums of the chunks c with c % gridDim.x == b to hout,
// so every chunk is written once.
struct XPreNP {
    float4 w[2], p[MV_SEG][2];
};

__device__ __forceinline__ void stage_xnp_issue(const MvIn &in, int cols, XPreNP &p, int nthr)
{
    const int nch = cols >> 3, c = threadIdx.x;
    const float4 *w4 = (const float4 *)in.norm_w;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    p.w[0] = p.w[1] = z;
#pragma unroll
    for (int s = 0; s < MV_SEG; s++) p.p[s][0] = p.p[s][1] = z;
    if (c < nch) {
#pragma unroll
        for (int s = 0; s < MV_SEG; s++) {
            const float4 *p4 = (const float4 *)(in.parts + (size_t)s * cols);
            p.p[s][0] = p4[2 * c];
            p.p[s][1] = p4[2 * c + 1];
        }
        p.w[0] = w4[2 * c];
        p.w[1] = w4[2 * c + 1];
    }
}

__device__ __forceinline__ float4 add4(float4 a, float4 b)
{
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

template <int FMT, bool OUTL>
__device__ void stage_xnp_finish(const XPreNP &p, const MvIn &in, int cols, uint32_t *xp, float *s16, int *kx,
                                 float *red, int nthr)
{
    XPreN<1> q;
#pragma unroll
    for (int k = 0; k < 2; k++) {
        float4 acc = p.p[0][k];
#pragma unroll
        for (int s = 1; s < MV_SEG; s++) acc = add4(acc, p.p[s][k]);
        q.v[k] = acc;
        q.w[k] = p.w[k];
    }
    const int c = threadIdx.x;
    if (c < (cols >> 3) && c % (int)gridDim.x == (int)blockIdx.x) {
        float4 *h4 = (float4 *)in.hout;
        h4[2 * c] = q.v[0];
        h4[2 * c + 1] = q.v[1];
    }
    stage_xn_finish<FMT, OUTL, 1>(q, cols, in.eps, xp, s16, kx, red, nthr);
}

template <int FMT, bool OUTL, int XP>
__device__ __forceinline__ void stage_x(const float *__restrict__ x, int cols, uint32_t *xp, float *s16, int *kx,
                                        int nthr)
{
    XPre<XP> p;
    stage_x_issue(x, cols, p, nthr);
    stage_x_finish<FMT, OUTL>(p, x, cols, xp, s16, kx, nthr);
}

__host__ __device__ inline size_t stage_lds_bytes(size_t cols) { return cols * XDIG + cols / 16 * 4 + (cols + 127) / 128 * 4; }
// ... with the outlier lists of OUTL staging
__host__ __device__ inline size_t stage_lds_bytes_o(size_t cols) { return stage_lds_bytes(cols) + out_lds_bytes(cols); }

// ---------------------------------------------------------------------------
// Per-format unit math
// ---------------------------------------------------------------------------

template <int FMT> struct WRow;
template <> struct WRow<FMT_Q4K> {
    uint4 h, a, b;
};
template <> struct WRow<FMT_Q80> {
    uint2 s;
    uint4 q[4];
};
template <> struct WRow<FMT_Q6K> {
    uint4 qh, la, lb;
    uint2 sc;
    uint32_t d;
};

// lane constants for one unit
struct UConst {
    float c[4];
    float P;                 // 2^-e of the unit's 128-element block: undoes the x scale
    uint32_t k1, k2, s, bsh; // Q4_K scale-decode selectors; Q6_K: s = half, bsh = 8*kk
    int sb;
    // OUTL staging: the list of the unit's block, its length, and whether any
    // lane of the wavefront has outliers (uniform; 0 = nothing to add; in
    // outlier_rows, the longest list over the wavefront)
    const uint32_t *ol = nullptr;
    int ocnt = 0, onum = 0;
};

// weight-side constants (needed before x is staged)
template <int FMT>
__device__ __forceinline__ void unit_setup_w(int u, UConst &c)
{
    if (FMT == FMT_Q4K) {
        const int p = u & 3;
        const bool hi = p >= 2;
        c.k1 = hi ? 0x0F0F0F0Fu : 0u;
        c.k2 = hi ? 0x30303030u : 0x3F3F3F3Fu;
        c.s = hi ? 2u : 0u;
        c.bsh = (uint32_t)(p & 1) * 16u;
        c.sb = u >> 2;
    } else if (FMT == FMT_Q6K) {
        c.sb = u >> 2;
        c.s = (uint32_t)((u >> 1) & 1);
        c.bsh = 8u * (uint32_t)(u & 1);
    }
}

// The unit's x digits in registers: XD dwords, dword 3 gi + k = digit k of
// register group gi.
struct XReg {
    uint32_t d[XD];
};

// x-side constants and the unit's x in registers (after stage_x)
template <int FMT, bool OUTL = false>
__device__ __forceinline__ void unit_setup_x(const uint32_t *xd, const float *s16, const int *kx, int u, int U, XReg &xv,
                                             UConst &c)
{
    if constexpr (OUTL) {
        c.ol = out_lists(kx, 64 * U) + (u >> 1) * OUT_DW;
        c.ocnt = min((int)c.ol[0], OUT_MAX);
        c.onum = __ballot(c.ocnt > 0) != 0;
    }
    c.P = block_unscale(kx[u >> 1]);
    const uint4 *x4 = (const uint4 *)xd;
#pragma unroll
    for (int r = 0; r < XD / 4; r++) {
        const uint4 v = x4[r * U + u];
        xv.d[4 * r] = v.x;
        xv.d[4 * r + 1] = v.y;
        xv.d[4 * r + 2] = v.z;
        xv.d[4 * r + 3] = v.w;
    }
    if (FMT == FMT_Q4K) {
        c.c[0] = s16[4 * u] + s16[4 * u + 1];
        c.c[1] = s16[4 * u + 2] + s16[4 * u + 3];
    } else if (FMT == FMT_Q6K) {
        const int sb = u >> 2, h = (u >> 1) & 1, kk = u & 1;
#pragma unroll
        for (int i = 0; i < 4; i++) c.c[i] = 32.0f * s16[sb * 16 + h * 8 + 2 * i + kk];
    }
}

// v_dot4_i32_i8: four signed byte products added to an int32 (exact).
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c)
{
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// v_dot4_i32_i8 onto an inline zero: starts a chain without first moving 0
// into the accumulator (the compiler otherwise picks the two-operand form,
// which adds one v_mov per digit and chain)
__device__ __forceinline__ int sdot4_first(uint32_t a, uint32_t b)
{
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// One code dword (four signed byte codes) against register group gi; FIRST
// starts the digit sums (their previous values are ignored).
template <bool FIRST = false>
__device__ __forceinline__ void dot_group(uint32_t q, const XReg &xv, int gi, int (&s)[XDIG])
{
#pragma unroll
    for (int k = 0; k < XDIG; k++) s[k] = FIRST ? sdot4_first(q, xv.d[XDIG * gi + k]) : sdot4(q, xv.d[XDIG * gi + k], s[k]);
}

// Sum over the digits: (s2 * 2^16 + s1 * 2^8 + s0), rounded once or twice.
__device__ __forceinline__ float digits_value(const int (&s)[XDIG])
{
    return fmaf((float)s[2], 65536.0f, (float)(s[1] * 256 + s[0]));
}

// Raw buffer loads over one wavefront's strip of rows.  A pass whose offset
// lies past the strip's byte count reads zeros without touching memory, so
// every load of the ring is issued unconditionally and the compiler can wait
// on exact vmcnt values.  (Raw-buffer range checks use the VGPR offset, so
// pass offsets are kept there, not in the scalar offset.)
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int RSRC_WORD3 = 0x00020000; // gfx9 raw buffer: 32-bit dwords, no swizzle

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, RSRC_WORD3);
}
// Cache policy of a buffer load (the instruction's cache-policy bits): 0 the
// default; LD_STREAM sets the nontemporal bit, for weight bytes a launch
// reads once.  Measured on MI355X (rotating weights): the Q4_K 14336 x 4096
// matvec 7.47 -> 7.02 us, Q8_0 4096 x 4096 5.58 -> 5.09 us, the 8B decode
// step 1.646 -> 1.622 ms per token.
constexpr int LD_STREAM = 2;
template <int POL = 0>
__device__ __forceinline__ uint4 bld16(rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, POL));
}
template <int POL = 0>
__device__ __forceinline__ uint2 bld8(rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, POL));
}
template <int POL = 0>
__device__ __forceinline__ uint32_t bld2(rsrc_t r, uint32_t off)
{
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, POL);
}

// Byte offsets, inside one packed row, of what lane unit u loads.
struct LaneOff {
    uint32_t o[3];
};

template <int FMT>
__device__ __forceinline__ LaneOff lane_offsets(int cols, int u, const UConst &c)
{
    LaneOff L;
    if constexpr (FMT == FMT_Q4K) {
        const int nb = cols >> 8, U = cols >> 6;
        L.o[0] = 16 * c.sb;          // H[sb]
        L.o[1] = 16 * nb + 16 * u;   // QA[u]
        L.o[2] = L.o[1] + 16 * U;    // QB[u]
    } else if constexpr (FMT == FMT_Q80) {
        const int nb = cols >> 5, sreg = (4 * nb + 15) & ~15;
        L.o[0] = 8 * u;              // S[2u], S[2u+1]
        L.o[1] = sreg + 16 * u;      // plane 0 (planes i at + 16*U*i)
        L.o[2] = 0;
    } else {
        const int nb = cols >> 8, U = cols >> 6;
        L.o[0] = 16 * nb + 16 * u;                 // QH[u] (QLa at +16U, QLb at +32U)
        L.o[1] = 16 * c.sb + 8 * c.s;              // SC[sb] half s
        L.o[2] = 16 * nb + 48 * U + 2 * c.sb;      // D[sb]
    }
    return L;
}

// Loads unit u of the row at byte offset `base` of the strip (streaming:
// each weight byte is read once per launch).
template <int FMT>
__device__ __forceinline__ void load_row(rsrc_t r, uint32_t base, int cols, const LaneOff &L, WRow<FMT> &w)
{
    if constexpr (FMT == FMT_Q4K) {
        w.h = bld16<LD_STREAM>(r, base + L.o[0]);
        w.a = bld16<LD_STREAM>(r, base + L.o[1]);
        w.b = bld16<LD_STREAM>(r, base + L.o[2]);
    } else if constexpr (FMT == FMT_Q80) {
        const uint32_t U16 = (uint32_t)(cols >> 6) * 16u;
        w.s = bld8<LD_STREAM>(r, base + L.o[0]);
#pragma unroll
        for (int i = 0; i < 4; i++) w.q[i] = bld16<LD_STREAM>(r, base + L.o[1] + U16 * i);
    } else {
        const uint32_t U16 = (uint32_t)(cols >> 6) * 16u;
        w.qh = bld16<LD_STREAM>(r, base + L.o[0]);
        w.la = bld16<LD_STREAM>(r, base + L.o[0] + U16);
        w.lb = bld16<LD_STREAM>(r, base + L.o[0] + 2 * U16);
        w.sc = bld8<LD_STREAM>(r, base + L.o[1]);
        w.d = bld2<LD_STREAM>(r, base + L.o[2]);
    }
}

// Partial dot of one unit of one row (in units of x).
template <int FMT>
__device__ __forceinline__ float unit_dot(const WRow<FMT> &w, const XReg &xv, const UConst &c)
{
    const float P = c.P;
    if constexpr (FMT == FMT_Q4K) {
        // qs byte l of the pair: low nibble = element l of sub-block 2p (unit
        // elements 0..31, register groups 0..7), high nibble = element l of
        // sub-block 2p+1 (register groups 8..15).
        const uint32_t q[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
        int sa[XDIG], sb[XDIG];
        dot_group<true>(q[0] & 0x0F0F0F0Fu, xv, 0, sa);
        dot_group<true>((q[0] >> 4) & 0x0F0F0F0Fu, xv, 8, sb);
#pragma unroll
        for (int t = 1; t < 8; t++) {
            dot_group(q[t] & 0x0F0F0F0Fu, xv, t, sa);
            dot_group((q[t] >> 4) & 0x0F0F0F0Fu, xv, 8 + t, sb);
        }
        // 6-bit scale/min of sub-blocks 2p, 2p+1 (get_scale_min_k4,
        // crates/sosomodel/src/dequant.rs:150-159), four at a time per byte lane.
        const uint32_t SC4 = ((w.h.w & c.k1) | ((w.h.y >> c.s) & c.k2)) >> c.bsh;
        const uint32_t M4 = (((w.h.w >> 4) & c.k1) | ((w.h.z >> c.s) & c.k2)) >> c.bsh;
        const float sca = (float)(SC4 & 0xffu), scb = (float)((SC4 >> 8) & 0xffu);
        const float ma = (float)(M4 & 0xffu), mb = (float)((M4 >> 8) & 0xffu);
        const float d = half_bits_to_f32(w.h.x & 0xffffu), dmin = half_bits_to_f32(w.h.x >> 16);
        const float uu = fmaf(sca, digits_value(sa), scb * digits_value(sb));
        const float vv = fmaf(mb, c.c[1], ma * c.c[0]);
        return fmaf(d * P, uu, -(dmin * vv));
    } else if constexpr (FMT == FMT_Q80) {
        // plane p holds bytes 16(p&1) .. +15 of block p>>1: register groups 4p .. 4p+3
        int s0[XDIG], s1[XDIG];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t q[4] = {w.q[p].x, w.q[p].y, w.q[p].z, w.q[p].w};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (p == 0 && t == 0) dot_group<true>(q[t], xv, 0, s0);
                else if (p == 2 && t == 0) dot_group<true>(q[t], xv, 8, s1);
                else if (p < 2) dot_group(q[t], xv, 4 * p + t, s0);
                else dot_group(q[t], xv, 4 * p + t, s1);
            }
        }
        return P * fmaf(__builtin_bit_cast(float, w.s.x), digits_value(s0),
                        __builtin_bit_cast(float, w.s.y) * digits_value(s1));
    } else {
        int s[4][XDIG];
        const uint32_t la[4] = {w.la.x, w.la.y, w.la.z, w.la.w}, lb[4] = {w.lb.x, w.lb.y, w.lb.z, w.lb.w};
        const uint32_t qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            // q = ql nibble | 2 bits of qh << 4 (dequantize_row_q6_K,
            // crates/gguf2som/src/lib.rs:1650-1658), four codes per dword.
            uint32_t q[4];
            q[0] = (la[t] & 0x0F0F0F0Fu) | ((qh[t] & 0x03030303u) << 4);
            q[1] = (lb[t] & 0x0F0F0F0Fu) | ((qh[t] & 0x0C0C0C0Cu) << 2);
            q[2] = ((la[t] >> 4) & 0x0F0F0F0Fu) | (qh[t] & 0x30303030u);
            q[3] = ((lb[t] >> 4) & 0x0F0F0F0Fu) | ((qh[t] >> 2) & 0x30303030u);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (t == 0) dot_group<true>(q[i], xv, 4 * i, s[i]);
                else dot_group(q[i], xv, 4 * i + t, s[i]);
            }
        }
        // sub-scales sc[h*8 + kk + 2i] (int8), the -32 offset through c[i] = 32*sum(x)
        const float sc0 = (float)(int8_t)(w.sc.x >> c.bsh), sc1 = (float)(int8_t)(w.sc.x >> (c.bsh + 16));
        const float sc2 = (float)(int8_t)(w.sc.y >> c.bsh), sc3 = (float)(int8_t)(w.sc.y >> (c.bsh + 16));
        float acc = sc0 * fmaf(digits_value(s[0]), P, -c.c[0]);
        acc = fmaf(sc1, fmaf(digits_value(s[1]), P, -c.c[1]), acc);
        acc = fmaf(sc2, fmaf(digits_value(s[2]), P, -c.c[2]), acc);
        acc = fmaf(sc3, fmaf(digits_value(s[3]), P, -c.c[3]), acc);
        return half_bits_to_f32(w.d) * acc;
    }
}

// The exactly dequantized weight of element e (0..63) of the unit, as the
// reference dequantizes it (crates/sosomodel/src/dequant.rs:74-97, 204-241;
// crates/gguf2som/src/lib.rs:1639-1661), with no FMA.
// A value the compiler cannot trace back to memory: a chain of selects over
// fields of a struct could otherwise be folded into one load at a computed
// address, which would move the whole struct (the row ring) into scratch.
__device__ __forceinline__ uint32_t opaque(uint32_t v)
{
    asm volatile("" : "+v"(v));
    return v;
}

template <int FMT>
__device__ __forceinline__ float unit_weight(const WRow<FMT> &wr, const UConst &c, int e)
{
    WRow<FMT> w = wr;
    if constexpr (FMT == FMT_Q4K) {
        w.a = make_uint4(opaque(w.a.x), opaque(w.a.y), opaque(w.a.z), opaque(w.a.w));
        w.b = make_uint4(opaque(w.b.x), opaque(w.b.y), opaque(w.b.z), opaque(w.b.w));
    } else if constexpr (FMT == FMT_Q80) {
        for (int i = 0; i < 4; i++)
            w.q[i] = make_uint4(opaque(w.q[i].x), opaque(w.q[i].y), opaque(w.q[i].z), opaque(w.q[i].w));
        w.s = make_uint2(opaque(w.s.x), opaque(w.s.y));
    } else {
        w.la = make_uint4(opaque(w.la.x), opaque(w.la.y), opaque(w.la.z), opaque(w.la.w));
        w.lb = make_uint4(opaque(w.lb.x), opaque(w.lb.y), opaque(w.lb.z), opaque(w.lb.w));
        w.qh = make_uint4(opaque(w.qh.x), opaque(w.qh.y), opaque(w.qh.z), opaque(w.qh.w));
        w.sc = make_uint2(opaque(w.sc.x), opaque(w.sc.y));
    }
    if constexpr (FMT == FMT_Q4K) {
        // element e: sub-block 2p + (e >> 5), qs byte e & 31 of the pair, low
        // nibble for the first sub-block, high for the second
        const int sub = e >> 5, l = e & 31, k = l >> 2;
        const uint32_t A = k == 0 ? w.a.x : k == 1 ? w.a.y : k == 2 ? w.a.z : w.a.w;
        const uint32_t B = k == 4 ? w.b.x : k == 5 ? w.b.y : k == 6 ? w.b.z : w.b.w;
        const uint32_t q = ((k < 4 ? A : B) >> (8 * (l & 3) + 4 * sub)) & 15u;
        const uint32_t SC4 = ((w.h.w & c.k1) | ((w.h.y >> c.s) & c.k2)) >> c.bsh;
        const uint32_t M4 = (((w.h.w >> 4) & c.k1) | ((w.h.z >> c.s) & c.k2)) >> c.bsh;
        const float sc = (float)((SC4 >> (8 * sub)) & 0xffu), m = (float)((M4 >> (8 * sub)) & 0xffu);
        const float d = half_bits_to_f32(w.h.x & 0xffffu), dmin = half_bits_to_f32(w.h.x >> 16);
        return __fsub_rn(__fmul_rn(__fmul_rn(d, sc), (float)q), __fmul_rn(dmin, m));
    } else if constexpr (FMT == FMT_Q80) {
        // plane e >> 4 holds bytes 16 (e >> 4 & 1) .. of block e >> 5
        const int pl = e >> 4, k = (e >> 2) & 3;
        const uint4 P = pl == 0 ? w.q[0] : pl == 1 ? w.q[1] : pl == 2 ? w.q[2] : w.q[3];
        const uint32_t dw = k == 0 ? P.x : k == 1 ? P.y : k == 2 ? P.z : P.w;
        const int q = (int)(int8_t)(dw >> (8 * (e & 3)));
        return __fmul_rn((float)q, __builtin_bit_cast(float, (e >> 5) ? w.s.y : w.s.x));
    } else {
        // element e = 16 i + j: quarter-run i, position 16 kk + j of the half
        const int i = e >> 4, j = e & 15, t = j >> 2, sh = 8 * (j & 3);
        const uint32_t la = t == 0 ? w.la.x : t == 1 ? w.la.y : t == 2 ? w.la.z : w.la.w;
        const uint32_t lb = t == 0 ? w.lb.x : t == 1 ? w.lb.y : t == 2 ? w.lb.z : w.lb.w;
        const uint32_t qh = t == 0 ? w.qh.x : t == 1 ? w.qh.y : t == 2 ? w.qh.z : w.qh.w;
        const uint32_t lo = (((i & 1) ? lb : la) >> (sh + ((i & 2) ? 4 : 0))) & 15u;
        const uint32_t hi = (qh >> (sh + 2 * i)) & 3u;
        const int q = (int)(lo | (hi << 4)) - 32;
        const uint32_t sw = (i & 2) ? w.sc.y : w.sc.x;
        const float sc = (float)(int8_t)(sw >> (c.bsh + ((i & 1) ? 16u : 0u)));
        return __fmul_rn(__fmul_rn(half_bits_to_f32(w.d), sc), (float)q);
    }
}

// Sum of w * x over the outliers of unit u's block that fall in the unit (OUTL
// staging), in list order; c.onum > 0.
template <int FMT>
__device__ __forceinline__ float unit_outliers(const WRow<FMT> &w, const UConst &c, int u)
{
    float corr = 0.0f;
    for (int k = 0; k < c.onum; k++) {
        if (k < c.ocnt) {
            const uint32_t p = (c.ol[1 + (k >> 2)] >> (8 * (k & 3))) & 0xffu;
            const uint32_t half = FMT == FMT_Q6K ? (p >> 4) & 1u : p >> 6;
            if (half == ((uint32_t)u & 1u)) {
                const int e = FMT == FMT_Q6K ? (int)((p >> 5) * 16 + (p & 15)) : (int)(p & 63);
                corr = fmaf(unit_weight<FMT>(w, c, e), __uint_as_float(c.ol[8 + k]), corr);
            }
        }
    }
    return corr;
}

// Moves the row sums of pass jw (last lane of each LPR-lane segment) into
// lanes jw*RW .. jw*RW+RW-1 of yacc.
template <int LPR>
__device__ __forceinline__ float gather_rows(float part, int jw, float yacc, int lane)
{
    constexpr int RW = 64 / LPR;
    if constexpr (LPR == 64) {
        const float s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 63));
        return lane == jw ? s : yacc;
    } else {
        const int d = lane - jw * RW;
        const bool in = d >= 0 && d < RW;
        const int src = in ? d * LPR + LPR - 1 : lane;
        const float v = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src * 4, __builtin_bit_cast(int, part)));
        return in ? v : yacc;
    }
}

// The outliers' share of a group's n passes, gathered as the row sums are
// (lane i: pass i / RW): a second walk over the passes, after the main one,
// in which only lanes whose unit's block has outliers load their unit again
// (the others address past the buffer and read zeros for free).  Taken only
// when some lane of the wavefront has outliers (c.onum > 0); the main loop
// stays free of the branch.  Every kernel that stages with OUTL adds this
// to the same row sums, so their results stay bit-identical.
template <int FMT, int LPR, class PassOff>
__device__ float outlier_rows(rsrc_t rs, uint32_t lane_base, PassOff pass_off, int j0, int j1, int cols,
                              const LaneOff &L, const UConst &c, int u, bool uact, int lane)
{
    float corr = 0.0f;
    UConst co = c;
    co.onum = (int)wave_max_dpp((float)c.ocnt);
    const uint32_t base = (uact && c.ocnt > 0) ? lane_base : 0x80000000u;
    for (int j = j0; j < j1; j++) {
        WRow<FMT> w;
        load_row<FMT>(rs, base + pass_off(j), cols, L, w);
        const float part = seg_sum_dpp<LPR>(uact ? unit_outliers<FMT>(w, co, u) : 0.0f);
        corr = gather_rows<LPR>(part, j - j0, corr, lane);
    }
    return corr;
}

