// k_mfma.hip -- products of several tokens per weight row on the matrix
// cores: the Q4_K MoE experts when a call routes two or more tokens to each
// active expert on average, and Q4_K or Q8_0 `matmul` (GpuDispatch::matmul,
// crates/soso-llm-core/src/gpu.rs:443-455) from 16 tokens up.
//
// Exact integer arithmetic, as in the single-token kernels: x is staged as
// three balanced signed base-256 digits of X = rint(x 2^e), one exponent e per
// 256-element super-block (|X| <= 2^22), and the Q4_K codes q (0..15) are
// int8 already, so v_mfma_i32_16x16x64_i8 returns exact int32 sums
//   S[digit][row] = sum_{k in unit} digit_k * q_k * s_k
// over one 64-element unit (two 32-element sub-blocks).  The 6-bit scale
// s_k of each sub-block enters the B operand (sc = 8 hi + lo, codes times hi
// and times lo are still int8), so two MFMA chains sum a whole super-block
// exactly (|S| < 2^25); per super-block in f32: y += d * 2^-e * (S0 + 256 S1 +
// 65536 S2) - dmin * sum_sb m_sb * sum(x over sb) -- the factorised Q4_K dot
// of crates/sosomodel/src/dequant.rs:172-201.
//
// MFMA operands (16 x 16 x 64, int8; lane l, g = l / 16):
//   A (16 x 64): row m = l % 16 = (token m / 4 of the tile, digit m % 4; digit
//                3 is a zero pad); bytes 0..7 elements 8g .. 8g + 7 of the
//                unit's first sub-block, bytes 8..15 the same of its second
//                <- LDS
//   B (64 x 16): column n = l % 16 = weight row, the same bytes of row n's
//                codes (low nibbles, then high nibbles), times a scale part
//   D (16 x 16): column n = l % 16, rows 4g .. 4g + 3 = token g of the tile,
//                digits 0..3
// A and B share the map from (lane group, byte) to k, so which k a byte is
// does not matter, only that both operands put the same element there.
// Every lane ends up with one (weight row, token) pair per tile: the row's
// scales apply lane by lane, and the min term is one FMA.
//
// Work: a workgroup of NW wavefronts (4 for the MoE experts; 4, 8 or 16 for
// a dense matmul, chosen by launch_mfma_matmul) owns 16 rows per wavefront of one
// expert (or of the dense weight) and loops over its tokens in rounds of
// 4 * MT, and over the columns in chunks of `kcmax` (as many as LDS holds for
// the round's tokens: one chunk for the MoE expert shapes).  Registered MoE
// layers are read from tile-major copies (below).
#include "mv_core.hpp"

typedef int mf_v4i __attribute__((ext_vector_type(4)));
typedef unsigned short mf_u16x2 __attribute__((ext_vector_type(2)));

constexpr int MF_NW = 4;            // wavefronts per workgroup
// Super-blocks of weights in flight per wavefront while one is applied
// (gate+up, single matrix).  Measured on MI355X at batch 32: one
// is fastest -- 136 us per layer; 2 / 3 ahead gave 144 us.
constexpr int MF_LA2 = 1, MF_LA1 = 1;
constexpr int MF_NW_GU = 4, MF_NW_DN = 4; // wavefronts per MoE workgroup: gate/up, down
constexpr int MF_SCAN_MAX = 512;    // ranked slots an expert workgroup scans itself (n * top_k)
// Dense matmul workgroups have 4, 8 or 16 wavefronts (launch_mfma_matmul).
constexpr int MF_NW_MAX = 16;

// LDS per token for kc staged columns: digits [sub-block][3][32 B], then the
// f32 sums of x per sub-block, then 2^-e per super-block, then (16-byte
// aligned) the outlier mask, one bit per element (byte c: chunk c's eight);
// the token stride is rounded up to 16 bytes (804 bytes per super-block would
// leave the 8-byte digit accesses of every other token misaligned when kc / 256
// is odd, e.g. the 768 columns of the MoE down projection: measured twice as
// slow).
__host__ __device__ constexpr inline int mf_mask_off(int kc) { return (kc / 32 * 100 + kc / 256 * 4 + 15) & ~15; }
__host__ __device__ constexpr inline int mf_tok_bytes(int kc)
{
    return (mf_mask_off(kc) + kc / 8 + 15) & ~15;
}
// The dense matmul's layout (k_mm_q4k) per token for kc staged columns: the
// digits of each pair of sub-blocks as [4 planes: digits 0..2 and a zero
// plane][4 lane groups][2 sub-blocks][8 bytes] (256 bytes per pair), so that a
// lane's A operand -- 8 bytes of each sub-block of a unit -- is one aligned
// 16-byte load and the zero-pad digit lanes load zeros; then the f32 sums per
// sub-block, 2^-e per super-block and (16-byte aligned) the outlier mask.
__host__ __device__ constexpr inline int mm_sum_off(int kc) { return 4 * kc; }
__host__ __device__ constexpr inline int mm_p_off(int kc) { return 4 * kc + kc / 8; }
__host__ __device__ constexpr inline int mm_mask_off(int kc) { return (4 * kc + kc / 8 + kc / 64 + 15) & ~15; }
__host__ __device__ constexpr inline int mm_tok_bytes(int kc) { return (mm_mask_off(kc) + kc / 8 + 15) & ~15; }
// The MoE experts that scan the ranking keep their slot list (16-bit entries)
// ahead of the tokens' staging in dynamic LDS.
__host__ __device__ inline int mf_scan_bytes(int nslots) { return (2 * nslots + 15) & ~15; }

// One super-block of one weight row as a lane loads it: the 16-byte header
// (d, dmin, 12 scale bytes) and, for each of the 4 units, the 8 code bytes of
// elements 8g .. 8g + 7 (low nibbles: sub-block 2p, high: 2p + 1).
struct MfSb {
    uint4 h;
    uint2 q[4];
};

// `in` false: the super-block lies past the chunk -- the offset is moved past
// the strip so the loads read zeros without touching memory.
__device__ __forceinline__ void mf_load_sb(rsrc_t r, uint32_t rowoff, uint32_t qoff, int sb, bool in, MfSb &s)
{
    rowoff = in ? rowoff : 0x80000000u;
    s.h = bld16(r, rowoff + 16u * (uint32_t)sb);
#pragma unroll
    for (int p = 0; p < 4; p++) s.q[p] = bld8(r, rowoff + qoff + 16u * (uint32_t)(4 * sb + p));
}

// Tile-major Q4_K (the registered MoE experts' copy for this kernel).  In the
// row-major packing a wavefront's 16 rows x one super-block are 48 pieces of
// 16-64 bytes spread over 16 rows (measured on MI355X: ~2.7 TB/s for that
// pattern, 5.7 TB/s for the same bytes read contiguously).  Here the rows of a
// 16-row tile are stored super-block by super-block, each block of 2304 bytes
// already in the order the lanes consume it:
//   [0, 256)     the 16 rows' 16-byte headers, row n at 16 n
//   [256, 1280)  lane l = 16 g + n: its pieces of units 0 and 1
//   [1280, 2304) lane l: its pieces of units 2 and 3
// where lane (n, g)'s piece of unit p is bytes 8g .. 8g + 7 of the unit's 32
// code bytes in row n (what mf_load_sb reads into q[p]).  A tile takes as many
// bytes as its 16 rows (nb * 2304 = 16 * row stride), so tile t starts where
// row 16 t would.  Every load below is contiguous across the wavefront.
constexpr int MF_TBLK = 2304; // bytes per (tile, super-block)
__device__ __forceinline__ void mf_load_sb_tiled(rsrc_t r, uint32_t tileoff, int nl, int lane, int sb, bool in,
                                                 MfSb &s)
{
    const uint32_t b = (in ? tileoff : 0x80000000u) + (uint32_t)MF_TBLK * (uint32_t)sb;
    s.h = bld16(r, b + 16u * (uint32_t)nl);
    const uint4 a = bld16(r, b + 256u + 16u * (uint32_t)lane);
    const uint4 c = bld16(r, b + 1280u + 16u * (uint32_t)lane);
    s.q[0] = make_uint2(a.x, a.y);
    s.q[1] = make_uint2(a.z, a.w);
    s.q[2] = make_uint2(c.x, c.y);
    s.q[3] = make_uint2(c.z, c.w);
}

// Row-major packed Q4_K -> tile-major (rows % 16 == 0): thread (tile,
// super-block, lane).
__global__ void tile_q4k(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int tiles, int nb)
{
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)tiles * nb * 64) return;
    const int lane = (int)(t & 63), sb = (int)((t >> 6) % nb), tile = (int)((t >> 6) / nb);
    const int n = lane & 15, g = lane >> 4, U = 4 * nb;
    const size_t stride = (size_t)nb * 144;
    const uint8_t *row = src + ((size_t)tile * 16 + n) * stride;
    uint8_t *blk = dst + ((size_t)tile * nb + sb) * MF_TBLK;
    if (g == 0) *(uint4 *)(blk + 16 * n) = *(const uint4 *)(row + 16 * sb);
    // piece of unit p: bytes 8g .. 8g+7 of its 32 code bytes (QA: 0..15, QB: 16..31)
    uint2 pc[4];
#pragma unroll
    for (int p = 0; p < 4; p++)
        pc[p] = *(const uint2 *)(row + 16 * nb + (g < 2 ? 0 : 16 * U) + 16 * (4 * sb + p) + 8 * (g & 1));
    *(uint4 *)(blk + 256 + 16 * lane) = make_uint4(pc[0].x, pc[0].y, pc[1].x, pc[1].y);
    *(uint4 *)(blk + 1280 + 16 * lane) = make_uint4(pc[2].x, pc[2].y, pc[3].x, pc[3].y);
}

bool tiled_q4k_ok(uint8_t dtype, size_t rows, size_t cols)
{
    return dtype == SOSO_HIP_DTYPE_Q4_K && rows % 16 == 0 && cols % 256 == 0 && cols >= 256;
}

int launch_tile_q4k(soso_hip *h, const void *src, void *dst, size_t rows, size_t cols)
{
    const size_t tiles = rows / 16, nb = cols / 256, n = tiles * nb * 64;
    tile_q4k<<<(unsigned)((n + 255) / 256), 256, 0, h->stream>>>((const uint8_t *)src, (uint8_t *)dst, (int)tiles,
                                                                   (int)nb);
    return hip_check(h, hipGetLastError(), "tile q4k launch");
}

// The scales of a super-block's 8 sub-blocks (get_scale_min_k4,
// dequant.rs:150-159), four per dword: sc[j] = byte j of sc4[j / 4], same for m.
struct MfScale {
    float d, dmin;
    uint32_t sc4[2], m4[2];
};

__device__ __forceinline__ void mf_scales(const uint4 &h, MfScale &s)
{
    s.d = half_bits_to_f32(h.x & 0xffffu);
    s.dmin = half_bits_to_f32(h.x >> 16);
    s.sc4[0] = h.y & 0x3F3F3F3Fu;
    s.m4[0] = h.z & 0x3F3F3F3Fu;
    s.sc4[1] = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    s.m4[1] = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
}

__device__ __forceinline__ int mf_byte(uint32_t w, int j) { return (int)((w >> (8 * j)) & 0xffu); }

// One 8-element chunk c of a token's row (tp: the token's staging) into LDS:
// the three digit planes, the sub-block's f32 sum, the super-block's 2^-e
// (NaN for a non-finite one) and the chunk's outlier bits.  The 32 lanes of a
// super-block and the 16 of a 128-element block run it together (invalid
// chunks carry zeros and write nothing).  Outliers follow the single-token
// staging's rule (stage_chunk<OUTL>) per 128-element block: above 16 times
// the third largest of the block's chunk maxima.  They get zero digits, stay
// out of the exponent and the sums, and are marked in the mask; the products
// then add w * x for them with w dequantized exactly (mf_outliers).  FAST:
// the cheap test only -- a block whose maximum is within 16x of its smallest
// 4-chunk maximum has none (the two largest chunks sit in at most two
// quads); when some block of the wavefront fails it, nothing is written and
// false is returned (uniform), for the caller to stage the chunk again
// through the full search.  The full search returns whether some block of
// the wavefront has outliers (uniform).
// Where chunk c's pieces go in a token's staging (mf_stage's layout, or with
// MM the dense matmul's: mm_*_off).
template <bool MM>
__device__ __forceinline__ void mf_write(uint8_t *tp, int c, int kc, const uint32_t (&d0)[XDIG],
                                         const uint32_t (&d1)[XDIG], float sm, bool finite, int ex, uint32_t om)
{
    const int sbl = c >> 2, qq = c & 3;
    if constexpr (MM) {
        uint8_t *dp = tp + (sbl >> 1) * 256 + 16 * qq + 8 * (sbl & 1);
#pragma unroll
        for (int kk = 0; kk < XDIG; kk++) *(uint2 *)(dp + 64 * kk) = make_uint2(d0[kk], d1[kk]);
        // (bytes 192 .. 255 of each 256, the A operand's zero pad, are left
        // unwritten: the matmul kernels clear them in LDS once, mm_zero_pad)
        if (qq == 0) *(float *)(tp + mm_sum_off(kc) + 4 * sbl) = sm;
        if ((c & 31) == 0)
            *(float *)(tp + mm_p_off(kc) + 4 * (c >> 5)) = finite ? ldexpf(1.0f, -ex) : __builtin_nanf("");
        tp[mm_mask_off(kc) + c] = (uint8_t)om;
    } else {
#pragma unroll
        for (int kk = 0; kk < XDIG; kk++)
            *(uint2 *)(tp + (sbl * 3 + kk) * 32 + 8 * qq) = make_uint2(d0[kk], d1[kk]);
        if (qq == 0) *(float *)(tp + (kc >> 5) * 96 + 4 * sbl) = sm;
        // a non-finite super-block: NaN products, as the CPU's dot gives Inf or NaN
        if ((c & 31) == 0)
            *(float *)(tp + (kc >> 5) * 100 + 4 * (c >> 5)) = finite ? ldexpf(1.0f, -ex) : __builtin_nanf("");
        tp[mf_mask_off(kc) + c] = (uint8_t)om;
    }
}

template <bool FAST, bool MM = false>
__device__ __forceinline__ bool mf_chunk(float4 v0, float4 v1, uint8_t *tp, int c, int kc, bool valid)
{
    float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float mx = fmaxf(fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3]))),
                     fmaxf(fmaxf(fabsf(vv[4]), fabsf(vv[5])), fmaxf(fabsf(vv[6]), fabsf(vv[7]))));
    // f32 sum of x over the 32-element sub-block: 4 aligned lanes
    float sm = ((vv[0] + vv[1]) + (vv[2] + vv[3])) + ((vv[4] + vv[5]) + (vv[6] + vv[7]));
    if (sm != sm) mx = INFINITY; // a NaN element: the super-block is non-finite
    float q = fmaxf(mx, dpp_f<0xB1>(mx));
    q = fmaxf(q, dpp_f<0x4E>(q));
    const float hq = fmaxf(q, dpp_f<0x141>(q));
    const float m1 = fmaxf(hq, dpp_f<0x140>(hq)); // the 128-element block's maximum
    float qn = fminf(q, dpp_f<0x141>(q));
    qn = fminf(qn, dpp_f<0x140>(qn));
    uint32_t om = 0;
    bool none = __ballot(m1 > 16.0f * qn) == 0;
    if constexpr (FAST) {
        if (!none) return false;
    } else if (!none) {
        const float thr = outlier_thr16(mx, m1);
        none = __ballot(m1 > thr) == 0;
        if (!none) {
            float km = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (fabsf(vv[i]) > thr) {
                    om |= 1u << i;
                    vv[i] = 0.0f;
                }
                km = fmaxf(km, fabsf(vv[i]));
            }
            mx = row16_max(km);
            sm = ((vv[0] + vv[1]) + (vv[2] + vv[3])) + ((vv[4] + vv[5]) + (vv[6] + vv[7]));
        }
    }
    const bool found = !none;
    if (none) mx = m1;
    // exponent of the 256-element super-block: 32 chunks = 32 aligned lanes
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    const bool finite = mx < INFINITY;
    const int ex = (mx > 0.0f && finite) ? 22 - __builtin_amdgcn_frexp_expf(mx) : 0;
    sm += dpp_f<0xB1>(sm);
    sm += dpp_f<0x4E>(sm);
    if (valid) {
        uint32_t d0[XDIG], d1[XDIG];
        digits4(make_float4(vv[0], vv[1], vv[2], vv[3]), ex, d0);
        digits4(make_float4(vv[4], vv[5], vv[6], vv[7]), ex, d1);
        mf_write<MM>(tp, c, kc, d0, d1, sm, finite, ex, om);
    }
    return !FAST || found;
}

// Writes one chunk staged without outliers: m is its 128-element block's
// maximum (the exponent takes the super-block's, over 32 lanes), sm the
// chunk's f32 sum (the sub-block's over 4 lanes).
template <bool MM = false>
__device__ __forceinline__ void mf_put(float4 v0, float4 v1, float m, float sm, uint8_t *tp, int c, int kc, bool valid)
{
    const float mx = fmaxf(m, __shfl_xor(m, 16, 64));
    const bool finite = mx < INFINITY;
    const int ex = (mx > 0.0f && finite) ? 22 - __builtin_amdgcn_frexp_expf(mx) : 0;
    sm += dpp_f<0xB1>(sm);
    sm += dpp_f<0x4E>(sm);
    if (valid) {
        uint32_t d0[XDIG], d1[XDIG];
        digits4(v0, ex, d0);
        digits4(v1, ex, d1);
        mf_write<MM>(tp, c, kc, d0, d1, sm, finite, ex, 0u);
    }
}

// Stages columns k0 .. k0 + kc of the round's nt tokens (x rows slot_s[t] / xdiv)
// into LDS, token t at t * mf_tok_bytes(kc).  Four chunks per thread are
// requested together (one L2 round trip per 4 * 64 * NW chunks); all four
// take the cheap outlier test first (mf_chunk<true>'s), and when no block of
// the wavefront fails it -- the common case -- they are staged straight away
// (mf_put), the four chunks' code interleaved.  Otherwise the round is staged
// again from x through the full search (mf_chunk<false>), one chunk at a
// time: that rare code stays out of the unrolled loop.
// A wavefront that finds outliers writes seq into *oflag (LDS): after the
// staging's barrier, *oflag == seq tells every wavefront that the chunk has
// some (no flag to clear: each chunk staged has its own seq).
template <int NW>
__device__ __forceinline__ void mf_stage(uint8_t *lds, const float *__restrict__ xs, const int *slot_s, int xdiv, int cols,
                                         int k0, int kc, int nt, int *oflag, int seq)
{
    const int tb = mf_tok_bytes(kc);
    const int cpt = kc >> 3, tot = nt * cpt; // 8-element chunks
    constexpr int NT = 64 * NW, XB = 4;
    auto xchunk = [&](int f) {
        return (const float4 *)(xs + (size_t)(slot_s[f / cpt] / xdiv) * cols + k0) + 2 * (f % cpt);
    };
    for (int fb = 0; fb < tot; fb += XB * NT) {
        float4 v0[XB], v1[XB];
#pragma unroll
        for (int k = 0; k < XB; k++) {
            const int f = fb + k * NT + (int)threadIdx.x;
            v0[k] = v1[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (f < tot) {
                const float4 *x4 = xchunk(f);
                v0[k] = x4[0];
                v1[k] = x4[1];
            }
        }
        float m1[XB], sm[XB];
        bool suspect = false;
#pragma unroll
        for (int k = 0; k < XB; k++) {
            m1[k] = sm[k] = 0.0f;
            if (fb + k * NT < tot) { // uniform
                const float4 a = v0[k], b = v1[k];
                float mx = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                                 fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
                sm[k] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
                if (sm[k] != sm[k]) mx = INFINITY; // a NaN element: the super-block is non-finite
                float q = fmaxf(mx, dpp_f<0xB1>(mx));
                q = fmaxf(q, dpp_f<0x4E>(q));
                const float hq = fmaxf(q, dpp_f<0x141>(q));
                m1[k] = fmaxf(hq, dpp_f<0x140>(hq));
                float qn = fminf(q, dpp_f<0x141>(q));
                qn = fminf(qn, dpp_f<0x140>(qn));
                suspect = suspect || m1[k] > 16.0f * qn;
            }
        }
        if (__builtin_expect(__ballot(suspect) == 0, 1)) {
#pragma unroll
            for (int k = 0; k < XB; k++) {
                if (fb + k * NT >= tot) break; // uniform
                const int f = fb + k * NT + (int)threadIdx.x;
                const bool valid = f < tot;
                mf_put(v0[k], v1[k], m1[k], sm[k], lds + (size_t)(valid ? f / cpt : 0) * tb, f % cpt, kc, valid);
            }
        } else {
#pragma unroll 1
            for (int k = 0; k < XB; k++) {
                if (fb + k * NT >= tot) break; // uniform
                const int f = fb + k * NT + (int)threadIdx.x;
                const bool valid = f < tot;
                float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
                if (valid) {
                    const float4 *x4 = xchunk(f);
                    a = x4[0];
                    b = x4[1];
                }
                if (mf_chunk<false>(a, b, lds + (size_t)(valid ? f / cpt : 0) * tb, f % cpt, kc, valid) &&
                    (threadIdx.x & 63) == 0)
                    *oflag = seq;
            }
        }
    }
}

// Dword di (0 .. 2N - 1) of lane src's pieces q[0 .. N - 1] (two dwords each),
// through ds_bpermute (every lane must run it).
template <int N>
__device__ __forceinline__ uint32_t mf_fetch(const uint2 (&q)[N], int src, int di)
{
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < N; i++) {
        const uint32_t x = (uint32_t)__builtin_amdgcn_ds_bpermute(src * 4, (int)q[i].x);
        const uint32_t y = (uint32_t)__builtin_amdgcn_ds_bpermute(src * 4, (int)q[i].y);
        r = di == 2 * i ? x : di == 2 * i + 1 ? y : r;
    }
    return r;
}

// Whether any of the round's nt tokens has outliers in super-block sbl of the
// staged chunk; uniform.
__device__ __forceinline__ bool mf_sb_has_outliers(const uint8_t *lds, int tb, int moff, int nt, int sbl)
{
    const int lane = (int)(threadIdx.x & 63), t = lane >> 1;
    bool any = false;
    for (int t0 = 0; t0 < nt; t0 += 32) {
        if (t0 + t < nt) {
            const uint4 m =
                *(const uint4 *)(lds + (size_t)(t0 + t) * tb + moff + 32 * sbl + 16 * (lane & 1));
            any = any || (m.x | m.y | m.z | m.w) != 0u;
        }
    }
    return __ballot(any) != 0;
}

// The outliers' share of super-block sbl for this lane's weight row and the
// token staged at tp, whose x row (from the chunk's first column) is xr
// (valid: a token of the round): sum of w * x over the elements marked in the
// super-block's mask, in column order, x read again from the row and w
// dequantized exactly as the reference dequantizes (get_code(e): element e's
// code of this lane's row, e in 0..255; wt(code, e): its weight).  Every lane
// runs the loop (the codes come from other lanes by ds_bpermute); the count is
// the wavefront's largest.
template <class Code, class Wt>
__device__ __forceinline__ float mf_outliers(const uint8_t *tp, const float *xr, int moff, int sbl, bool valid,
                                             Code get_code, Wt wt)
{
    uint4 ma = make_uint4(0u, 0u, 0u, 0u), mb = ma;
    if (valid) {
        ma = *(const uint4 *)(tp + moff + 32 * sbl);
        mb = *(const uint4 *)(tp + moff + 32 * sbl + 16);
    }
    uint32_t m[8] = {ma.x, ma.y, ma.z, ma.w, mb.x, mb.y, mb.z, mb.w};
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) cnt += __popc(m[i]);
    const int nmax = (int)wave_max_dpp((float)cnt);
    float corr = 0.0f;
    for (int k = 0; k < nmax; k++) {
        // this lane's next marked element: the lowest set bit left
        int e = 0;
        bool found = false;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (!found && m[i] != 0u) {
                e = 32 * i + __builtin_ctz(m[i]);
                m[i] &= m[i] - 1u;
                found = true;
            }
        }
        const float v = found ? xr[256 * sbl + e] : 0.0f;
        corr = fmaf(wt(get_code(e), e), v, corr);
    }
    return corr;
}

// The slots s < nslots with sidx[s] == e (the token t = s / top_k ranked expert
// e j = s % top_k-th), ascending, into scan_s; returns their count.  The MoE
// route then needs no slot sort: each expert's workgroups find their tokens
// in the n * top_k ranked indices (at most MF_SCAN_MAX of them).
template <int NW>
__device__ int mf_scan_slots(const int32_t *__restrict__ sidx, int nslots, int e, int16_t *scan_s, int *wtot_s)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int total = 0;
    for (int s0 = 0; s0 < nslots; s0 += 64 * NW) {
        const int sl = s0 + (int)threadIdx.x;
        const bool hit = sl < nslots && sidx[sl] == e;
        const uint64_t m = __ballot(hit);
        if (lane == 0) wtot_s[wave] = __popcll(m);
        __syncthreads();
        int before = total, all = total;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const int c = wtot_s[w];
            before += w < wave ? c : 0;
            all += c;
        }
        if (hit) scan_s[before + __popcll(m & ((1ull << lane) - 1ull))] = (int16_t)sl;
        total = all;
        __syncthreads(); // wtot_s is rewritten by the next stretch
    }
    return total;
}

// tabA/tabB: per-expert weight pointer tables (MoE), or null with W0 the dense
// weight.  recs[4a ..] = {expert, tokens, first slot, 0} for a < *n_recs
// (MoE), or dense_n > 0 tokens of one dense product (slot = token).  Item:
// blockIdx.x = a * nblk + row block (MoE), or row block + nblk * token round
// (dense).  Slot s reads x = xs + (s / xdiv) * cols and writes out[s * rows + r].
// FULL (dense products whose token count is a multiple of 4 MT): every round
// holds 4 MT tokens, so the per-tile checks compile away and the A operand is
// loaded by every lane (the zero-pad digit lanes read digit 2 and select 0).
template <int NMAT, int MT, int LA, bool TILED = false, int NW = MF_NW, bool SCAN = false, bool FULL = false,
          bool SPLIT = false>
__global__ void __launch_bounds__(64 * NW, NW == 4 && MT <= 2 ? (NMAT == 2 ? 3 : 4) : 1) k_mfma_q4k(const uint8_t *const *__restrict__ tabA,
                                                  const uint8_t *const *__restrict__ tabB,
                                                  const uint8_t *__restrict__ W0, size_t stride, int rows, int cols,
                                                  const float *__restrict__ xs, int xdiv, const int *__restrict__ list,
                                                  const int *__restrict__ recs, const int *__restrict__ n_recs,
                                                  int dense_n, int kcmax, float *__restrict__ out,
                                                  const int32_t *__restrict__ sidx, int nslots)
{
    constexpr int TR = 4 * MT; // tokens per round
    extern __shared__ uint4 mf_smem[];
    // SCAN: the expert's slots (16-bit, as many as the call ranked) ahead of
    // the staging: with 8 tokens' x staged (53.5 KB for 2048 columns), three
    // gate/up workgroups still fit a CU's 160 KB of LDS
    int16_t *scan_s = (int16_t *)mf_smem;
    uint8_t *lds = (uint8_t *)mf_smem + (SCAN ? mf_scan_bytes(nslots) : 0);
    __shared__ int slot_s[TR];
    __shared__ int oflag_s; // the seq of the last staged chunk with outliers
    if (threadIdx.x == 0) oflag_s = -1;
    int seq = 0;
    __shared__ int wtot_s[NW];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    constexpr int ROWS = 16 * NW; // rows per workgroup
    const int nblk = (rows + ROWS - 1) / ROWS;
    int e = 0, ne, base = 0, b, t_first, t_step;
    const uint8_t *WA, *WB;
    if (dense_n > 0) {
        b = blockIdx.x % nblk;
        ne = dense_n;
        t_first = (blockIdx.x / nblk) * TR; // one round per workgroup
        t_step = (int)(gridDim.x / nblk) * TR;
    } else if constexpr (SCAN) {
        // expert a's slots, ascending, read off the ranking itself
        e = blockIdx.x / nblk;
        b = blockIdx.x % nblk;
        // the expert's tables are requested before the scan, which does not need them
        WA = tabA[e];
        WB = NMAT == 2 ? tabB[e] : WA;
        ne = mf_scan_slots<NW>(sidx, nslots, e, scan_s, wtot_s);
        if (ne == 0) return; // uniform: nobody chose this expert
        t_first = 0;
        t_step = TR;
    } else {
        const int a = blockIdx.x / nblk;
        b = blockIdx.x % nblk;
        // the record and the count are requested together (the grid holds at
        // most as many records as `recs` has room for, so the read is in
        // bounds; `recs` is only int-aligned)
        const int *rec = recs + 4 * a;
        e = rec[0];
        ne = rec[1];
        base = rec[2];
        if (a >= *n_recs) return; // fewer active experts than the grid allows
        t_first = 0;
        t_step = TR;
    }
    if (!SCAN) {
        WA = dense_n > 0 ? W0 : tabA[e];
        WB = NMAT == 2 ? tabB[e] : WA;
    }
    const int nl = lane & 15, g = lane >> 4;
    // row-major: this lane's row; tiled: the wavefront's tile (past the strip: zeros)
    const uint32_t rowoff = (uint32_t)((16 * wave + (TILED ? 0 : nl)) * stride);
    const int nb = cols >> 8, U = cols >> 6;
    const uint32_t qoff = (uint32_t)(16 * nb + (g < 2 ? 0 : 16 * U) + 8 * (g & 1));
    // A operand of this lane: token (nl / 4) of a tile, digit nl % 4, bytes 8g .. 8g + 7
    const int a_tok = nl >> 2, a_dig = nl & 3;

    const int a_dg = a_dig < 3 ? a_dig : 2; // FULL: the pad lanes' (discarded) digit
    for (int t0 = t_first; t0 < ne; t0 += t_step) {
        const int nt = FULL ? TR : min(TR, ne - t0);
        __syncthreads(); // the previous round's readers of slot_s and LDS are done
        if ((int)threadIdx.x < nt)
            slot_s[threadIdx.x] = SCAN ? scan_s[t0 + threadIdx.x]
                                       : list ? list[base + t0 + threadIdx.x] : base + t0 + threadIdx.x;
        __syncthreads();
        const int r0 = b * ROWS, rend = min(rows, r0 + ROWS);
        const uint32_t strip = (uint32_t)((size_t)(rend - r0) * stride);
        const rsrc_t rA = make_rsrc(WA + (size_t)r0 * stride, strip);
        const rsrc_t rB = make_rsrc(WB + (size_t)r0 * stride, strip);
        const int row = r0 + 16 * wave + nl; // this lane's weight row
        float accf[NMAT][MT];
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) accf[m][mt] = 0.0f;
        for (int k0 = 0; k0 < cols; k0 += kcmax) {
            const int kc = min(kcmax, cols - k0), tb = mf_tok_bytes(kc), nsb = kc >> 8;
            const int sb0 = k0 >> 8;
            // the chunk's first weights are requested before x is staged, so
            // their latency overlaps the staging (loads return in issue order)
            auto load_sb = [&](rsrc_t r, int sb, bool in, MfSb &out) {
                if constexpr (TILED) mf_load_sb_tiled(r, rowoff, nl, lane, sb, in, out);
                else mf_load_sb(r, rowoff, qoff, sb, in, out);
            };
            MfSb ca, cb;
            load_sb(rA, sb0, true, ca);
            if constexpr (NMAT == 2) load_sb(rB, sb0, true, cb);
            __builtin_amdgcn_sched_barrier(0);
            // ---- stage x (columns k0 .. k0 + kc of the round's tokens) ----
            mf_stage<NW>(lds, xs, slot_s, xdiv, cols, k0, kc, nt, &oflag_s, ++seq);
            __syncthreads();
            const bool oany = __builtin_amdgcn_readfirstlane(oflag_s) == seq;
            // ---- stream this chunk's super-blocks of the wavefront's 16 rows ----
            // The 6-bit scale of each sub-block goes into the B operand: sc =
            // 8 hi + lo with hi, lo < 8, so q*lo and q*hi (<= 105) are int8 and
            // one packed 16-bit multiply scales four packed codes (each 16-bit
            // half holds two codes; the low one's product never carries into
            // the high byte).  Two MFMA chains (lo, hi) then sum a whole
            // super-block in the accumulators: S = Clo + 8 Chi = sum_sb sc_sb *
            // sum_k digit * q.
            // k: the factor in both 16-bit halves
            auto scaled = [](uint32_t codes, uint32_t k) {
                return __builtin_bit_cast(uint32_t, __builtin_bit_cast(mf_u16x2, codes) *
                                                        __builtin_bit_cast(mf_u16x2, k));
            };
            // {f, f} for the low / high 3 bits f of each sub-block's scale,
            // eight sub-blocks from two masked dwords: byte j % 4 of the
            // dword moved into bytes 0 and 2 by one permute, zeros elsewhere
            auto scale_parts = [](const MfScale &sc, uint32_t (&klo)[8], uint32_t (&khi)[8]) {
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t lo4 = sc.sc4[t] & 0x07070707u, hi4 = (sc.sc4[t] >> 3) & 0x07070707u;
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        const uint32_t sel = 0x0c000c00u | (uint32_t)b | ((uint32_t)b << 16);
                        klo[4 * t + b] = __builtin_amdgcn_perm(0u, lo4, sel);
                        khi[4 * t + b] = __builtin_amdgcn_perm(0u, hi4, sel);
                    }
                }
            };
            // SPLIT: one v_mfma_i32_16x16x32_i8 per sub-block on the raw codes
            // (0..15), the scale applied to its exact int32 sums by a 24-bit
            // multiply-add: S = sum_sb sc_sb * D_sb, the same integer as
            // Clo + 8 Chi, without the B operands' scale multiplies (for one
            // token tile per super-block, the MoE experts' usual case).
            auto superblock_split = [&](int sbl8, const MfSb &A_, const MfSb &B_) {
                MfScale sc_[NMAT];
                mf_scales(A_.h, sc_[0]);
                if constexpr (NMAT == 2) mf_scales(B_.h, sc_[NMAT - 1]);
                typedef long mf_i64;
                int S[NMAT][MT][3];
                float mins[NMAT][MT];
#pragma unroll
                for (int m = 0; m < NMAT; m++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        S[m][mt][0] = S[m][mt][1] = S[m][mt][2] = 0;
                        mins[m][mt] = 0.0f;
                    }
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const int j0 = 2 * p, j1 = 2 * p + 1;
                    mf_i64 bl[NMAT], bh[NMAT];
                    int s0[NMAT], s1[NMAT];
                    float m0[NMAT], m1[NMAT];
#pragma unroll
                    for (int m = 0; m < NMAT; m++) {
                        const uint2 q = m == 0 ? A_.q[p] : B_.q[p];
                        const uint32_t lx = q.x & 0x0F0F0F0Fu, ly = q.y & 0x0F0F0F0Fu;
                        const uint32_t hx = (q.x >> 4) & 0x0F0F0F0Fu, hy = (q.y >> 4) & 0x0F0F0F0Fu;
                        bl[m] = (mf_i64)(((uint64_t)ly << 32) | lx);
                        bh[m] = (mf_i64)(((uint64_t)hy << 32) | hx);
                        s0[m] = mf_byte(sc_[m].sc4[j0 >> 2], j0 & 3);
                        s1[m] = mf_byte(sc_[m].sc4[j1 >> 2], j1 & 3);
                        m0[m] = (float)mf_byte(sc_[m].m4[j0 >> 2], j0 & 3);
                        m1[m] = (float)mf_byte(sc_[m].m4[j1 >> 2], j1 & 3);
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        if (mt * 4 >= nt) break; // uniform
                        const int ta = mt * 4 + a_tok;
                        uint2 u0 = make_uint2(0u, 0u), u1 = u0;
                        if constexpr (FULL) {
                            const uint8_t *tp = lds + (size_t)ta * tb;
                            u0 = *(const uint2 *)(tp + ((sbl8 + j0) * 3 + a_dg) * 32 + 8 * g);
                            u1 = *(const uint2 *)(tp + ((sbl8 + j1) * 3 + a_dg) * 32 + 8 * g);
                            if (a_dig == 3) u0 = u1 = make_uint2(0u, 0u);
                        } else if (a_dig < 3 && ta < nt) {
                            const uint8_t *tp = lds + (size_t)ta * tb;
                            u0 = *(const uint2 *)(tp + ((sbl8 + j0) * 3 + a_dig) * 32 + 8 * g);
                            u1 = *(const uint2 *)(tp + ((sbl8 + j1) * 3 + a_dig) * 32 + 8 * g);
                        }
                        const mf_i64 a0 = (mf_i64)(((uint64_t)u0.y << 32) | u0.x);
                        const mf_i64 a1 = (mf_i64)(((uint64_t)u1.y << 32) | u1.x);
                        const int to = mt * 4 + g;
                        const float *xsum = (const float *)(lds + (size_t)(to < nt ? to : 0) * tb + (kc >> 5) * 96);
                        const float xs0 = xsum[sbl8 + j0], xs1 = xsum[sbl8 + j1];
#pragma unroll
                        for (int m = 0; m < NMAT; m++) {
                            const mf_v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bl[m], mf_v4i{0, 0, 0, 0}, 0, 0, 0);
                            const mf_v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bh[m], mf_v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                            for (int d = 0; d < 3; d++)
                                S[m][mt][d] = __mul24(s1[m], d1[d]) + (__mul24(s0[m], d0[d]) + S[m][mt][d]);
                            mins[m][mt] = fmaf(m0[m], xs0, fmaf(m1[m], xs1, mins[m][mt]));
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    if (mt * 4 >= nt) break;
                    const int to = mt * 4 + g;
                    const float P = *(const float *)(lds + (size_t)(to < nt ? to : 0) * tb + (kc >> 5) * 100 +
                                                     4 * (sbl8 >> 3));
#pragma unroll
                    for (int m = 0; m < NMAT; m++) {
                        const float t = fmaf((float)S[m][mt][2], 65536.0f,
                                             fmaf((float)S[m][mt][1], 256.0f, (float)S[m][mt][0]));
                        accf[m][mt] = fmaf(-sc_[m].dmin, mins[m][mt], fmaf(sc_[m].d * P, t, accf[m][mt]));
                    }
                }
            };
            auto superblock = [&](int sbl8, const MfSb &A_, const MfSb &B_) {
                // sbl8: first local sub-block of this super-block
                MfScale sc_[NMAT];
                mf_scales(A_.h, sc_[0]);
                if constexpr (NMAT == 2) mf_scales(B_.h, sc_[NMAT - 1]);
                uint32_t klo[NMAT][8], khi[NMAT][8];
#pragma unroll
                for (int m = 0; m < NMAT; m++) scale_parts(sc_[m], klo[m], khi[m]);
                mf_v4i clo[NMAT][MT], chi[NMAT][MT];
                float mins[NMAT][MT];
#pragma unroll
                for (int m = 0; m < NMAT; m++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        clo[m][mt] = chi[m][mt] = mf_v4i{0, 0, 0, 0};
                        mins[m][mt] = 0.0f;
                    }
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const int j0 = 2 * p, j1 = 2 * p + 1; // sub-blocks of the unit
                    // B operands of the unit's 64 elements: bytes 0..7 the
                    // codes of sub-block j0 (low nibbles), bytes 8..15 those
                    // of j1 (high nibbles), times sc lo (bl) or sc hi (bh); A
                    // holds the x digits in the same byte order, so one K=64
                    // product sums both sub-blocks (A and B share the lane /
                    // byte -> k map).  The min factors.
                    mf_v4i bl[NMAT], bh[NMAT];
                    float m0[NMAT], m1[NMAT];
#pragma unroll
                    for (int m = 0; m < NMAT; m++) {
                        const uint2 q = m == 0 ? A_.q[p] : B_.q[p];
                        const uint32_t lx = q.x & 0x0F0F0F0Fu, ly = q.y & 0x0F0F0F0Fu;
                        const uint32_t hx = (q.x >> 4) & 0x0F0F0F0Fu, hy = (q.y >> 4) & 0x0F0F0F0Fu;
                        bl[m] = mf_v4i{(int)scaled(lx, klo[m][j0]), (int)scaled(ly, klo[m][j0]),
                                       (int)scaled(hx, klo[m][j1]), (int)scaled(hy, klo[m][j1])};
                        bh[m] = mf_v4i{(int)scaled(lx, khi[m][j0]), (int)scaled(ly, khi[m][j0]),
                                       (int)scaled(hx, khi[m][j1]), (int)scaled(hy, khi[m][j1])};
                        m0[m] = (float)mf_byte(sc_[m].m4[j0 >> 2], j0 & 3);
                        m1[m] = (float)mf_byte(sc_[m].m4[j1 >> 2], j1 & 3);
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        if (mt * 4 >= nt) break; // uniform
                        // A: token mt*4 + a_tok, digit a_dig (3: zero), elements 8g..8g+7
                        const int ta = mt * 4 + a_tok;
                        mf_v4i xa = mf_v4i{0, 0, 0, 0};
                        if constexpr (FULL) {
                            const uint8_t *tp = lds + (size_t)ta * tb;
                            const uint2 u0 = *(const uint2 *)(tp + ((sbl8 + j0) * 3 + a_dg) * 32 + 8 * g);
                            const uint2 u1 = *(const uint2 *)(tp + ((sbl8 + j1) * 3 + a_dg) * 32 + 8 * g);
                            const bool z = a_dig == 3;
                            xa = mf_v4i{z ? 0 : (int)u0.x, z ? 0 : (int)u0.y, z ? 0 : (int)u1.x, z ? 0 : (int)u1.y};
                        } else if (a_dig < 3 && ta < nt) {
                            const uint8_t *tp = lds + (size_t)ta * tb;
                            const uint2 u0 = *(const uint2 *)(tp + ((sbl8 + j0) * 3 + a_dig) * 32 + 8 * g);
                            const uint2 u1 = *(const uint2 *)(tp + ((sbl8 + j1) * 3 + a_dig) * 32 + 8 * g);
                            xa = mf_v4i{(int)u0.x, (int)u0.y, (int)u1.x, (int)u1.y};
                        }
                        // the x sums of this lane's output token (mt*4 + g)
                        const int to = mt * 4 + g;
                        const float *xsum = (const float *)(lds + (size_t)(to < nt ? to : 0) * tb + (kc >> 5) * 96);
                        const float xs0 = xsum[sbl8 + j0], xs1 = xsum[sbl8 + j1];
#pragma unroll
                        for (int m = 0; m < NMAT; m++) {
                            clo[m][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, bl[m], clo[m][mt], 0, 0, 0);
                            chi[m][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, bh[m], chi[m][mt], 0, 0, 0);
                            mins[m][mt] = fmaf(m0[m], xs0, fmaf(m1[m], xs1, mins[m][mt]));
                        }
                    }
                    // one unit at a time: keeps each unit's LDS reads from being
                    // hoisted into the next (register pressure)
                    __builtin_amdgcn_sched_barrier(0);
                }
                // f32 per super-block: y += d 2^-e (S0 + 256 S1 + 65536 S2) - dmin * mins,
                // S_i = clo_i + 8 chi_i (|S_i| < 2^25)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    if (mt * 4 >= nt) break;
                    const int to = mt * 4 + g;
                    const float P = *(const float *)(lds + (size_t)(to < nt ? to : 0) * tb + (kc >> 5) * 100 +
                                                     4 * (sbl8 >> 3));
#pragma unroll
                    for (int m = 0; m < NMAT; m++) {
                        const int S0 = clo[m][mt][0] + 8 * chi[m][mt][0], S1 = clo[m][mt][1] + 8 * chi[m][mt][1];
                        const int S2 = clo[m][mt][2] + 8 * chi[m][mt][2];
                        const float t = fmaf((float)S2, 65536.0f, fmaf((float)S1, 256.0f, (float)S0));
                        accf[m][mt] = fmaf(-sc_[m].dmin, mins[m][mt], fmaf(sc_[m].d * P, t, accf[m][mt]));
                    }
                }
            };
            // super-blocks i + 1 .. i + LA are in flight while i is applied
            MfSb pa[LA], pb[LA];
#pragma unroll
            for (int k = 0; k < LA - 1; k++) {
                load_sb(rA, sb0 + 1 + k, 1 + k < nsb, pa[k]);
                if constexpr (NMAT == 2) load_sb(rB, sb0 + 1 + k, 1 + k < nsb, pb[k]);
            }
            for (int i = 0; i < nsb; i++) {
                load_sb(rA, sb0 + i + LA, i + LA < nsb, pa[LA - 1]);
                if constexpr (NMAT == 2) load_sb(rB, sb0 + i + LA, i + LA < nsb, pb[LA - 1]);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (SPLIT)
                    superblock_split(8 * i, ca, cb);
                else
                    superblock(8 * i, ca, cb);
                ca = pa[0];
                if constexpr (NMAT == 2) cb = pb[0];
#pragma unroll
                for (int k = 0; k < LA - 1; k++) {
                    pa[k] = pa[k + 1];
                    if constexpr (NMAT == 2) pb[k] = pb[k + 1];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            // ---- the outliers of the round's tokens: a second walk over the
            // super-blocks that hold some (rare; outside the streaming loop,
            // so that its registers do not add to the loop's), reloading the
            // codes: w * x with w = fl(fl(d sc) q) - fl(dmin m)
            // (dequant.rs:204-241).  Element e of a super-block: unit e / 64,
            // code byte l = e % 32 of the unit (lane group l / 8 of this row
            // holds it), the high nibble from 32 on.
            if (__builtin_expect(oany, 0)) {
                for (int i = 0; i < nsb; i++) {
                    if (!mf_sb_has_outliers(lds, tb, mf_mask_off(kc), nt, i)) continue; // uniform
                    MfSb S_[NMAT];
                    load_sb(rA, sb0 + i, true, S_[0]);
                    if constexpr (NMAT == 2) load_sb(rB, sb0 + i, true, S_[NMAT - 1]);
#pragma unroll
                    for (int m = 0; m < NMAT; m++) {
                        MfScale K_;
                        mf_scales(S_[m].h, K_);
                        auto code = [&](int e) {
                            const int eu = e & 63, l = eu & 31;
                            const uint32_t dw = mf_fetch<4>(S_[m].q, 16 * (l >> 3) + nl, 2 * (e >> 6) + ((l & 7) >> 2));
                            return (dw >> (8 * (l & 3) + (eu >= 32 ? 4 : 0))) & 15u;
                        };
                        auto wt = [&](uint32_t q, int e) {
                            const int j = 2 * (e >> 6) + ((e & 63) >= 32 ? 1 : 0), sh = 8 * (j & 3);
                            const float sc = (float)(((j < 4 ? K_.sc4[0] : K_.sc4[1]) >> sh) & 0xffu);
                            const float mn = (float)(((j < 4 ? K_.m4[0] : K_.m4[1]) >> sh) & 0xffu);
                            return __fsub_rn(__fmul_rn(__fmul_rn(K_.d, sc), (float)q), __fmul_rn(K_.dmin, mn));
                        };
#pragma unroll
                        for (int mt = 0; mt < MT; mt++) {
                            if (mt * 4 >= nt) break; // uniform
                            const int to = mt * 4 + g, tv = to < nt ? to : 0;
                            const float *xr = xs + (size_t)(slot_s[tv] / xdiv) * cols + k0;
                            accf[m][mt] +=
                                mf_outliers(lds + (size_t)tv * tb, xr, mf_mask_off(kc), i, to < nt, code, wt);
                        }
                    }
                }
            }
            __syncthreads(); // LDS is restaged for the next chunk or round
        }
        // ---- outputs: lane (row, token mt*4 + g) ----
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int to = mt * 4 + g;
            if (mt * 4 < nt && to < nt && row < rows) {
                float v = accf[0][mt];
                if constexpr (NMAT == 2) v = v / (1.0f + expf(-v)) * accf[NMAT - 1][mt];
                out[(size_t)slot_s[to] * rows + row] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Dense Q4_K products of many tokens (matmul with a token count that is a
// multiple of 16): x staged once per call, the workgroups' rounds always full.
//
// k_mfma_q4k stages its round's tokens itself, so every row block converts
// the same x again (14336 x 4096 at 64 tokens: 56 row blocks x 4 rounds, about
// 1,000 of its 7,100 VALU instructions per wavefront), and its code carries the
// checks of partial rounds and MoE token lists.  Here k_mm_stage converts the
// n rows of x once (the whole row as one chunk, token t at t *
// mm_tok_bytes(cols)), in the paired layout of mm_*_off: a lane's A operand is
// one 16-byte LDS load and the zero-pad digit lanes read a zero plane (against
// mf_stage's layout: two 8-byte loads and four selects per unit and token
// tile; 56.3 -> 51.9 us at 14336 x 4096 x 64).  Each workgroup of k_mm_q4k
// copies the stretch of its chunk from there into LDS (four contiguous regions
// per token: digits, sub-block sums, 2^-e per super-block, outlier mask).
// Arithmetic, operands and the order of every sum are k_mfma_q4k's (the
// outliers' corrections, where a token has some, join after each staged
// chunk, whose width may differ from k_mfma_q4k's).
// ---------------------------------------------------------------------------

// One wavefront per 512 columns (64 chunks: two super-blocks, the lanes of each
// 128-element block together) of one token; the outlier search as mf_stage's,
// the output in the paired layout (mf_write<true>).
__global__ void __launch_bounds__(256) k_mm_stage(const float *__restrict__ x, int n, int cols,
                                                  uint8_t *__restrict__ xg)
{
    const int lane = threadIdx.x & 63;
    const int gw = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    const int wpt = (cols + 511) / 512, nch = cols >> 3;
    const int t = gw / wpt, c = (gw % wpt) * 64 + lane;
    if (t >= n) return; // uniform per wavefront; no barriers here
    const bool valid = c < nch;
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    if (valid) {
        const float4 *x4 = (const float4 *)(x + (size_t)t * cols) + 2 * c;
        v0 = x4[0];
        v1 = x4[1];
    }
    uint8_t *tp = xg + (size_t)t * mm_tok_bytes(cols);
    float mx = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                     fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
    const float sm = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w));
    if (sm != sm) mx = INFINITY; // a NaN element: the super-block is non-finite
    float q = fmaxf(mx, dpp_f<0xB1>(mx));
    q = fmaxf(q, dpp_f<0x4E>(q));
    const float hq = fmaxf(q, dpp_f<0x141>(q));
    const float m1 = fmaxf(hq, dpp_f<0x140>(hq));
    float qn = fminf(q, dpp_f<0x141>(q));
    qn = fminf(qn, dpp_f<0x140>(qn));
    if (__builtin_expect(__ballot(m1 > 16.0f * qn) == 0, 1)) mf_put<true>(v0, v1, m1, sm, tp, c, cols, valid);
    else (void)mf_chunk<false, true>(v0, v1, tp, c, cols, valid);
}

// The zero pad of the A operand (digit plane 3: 64 bytes of every 256 of a
// token's digits) for tokens 0 .. TR - 1 of a chunk buffer in LDS: cleared
// once per workgroup, mm_copy never writes it.
template <int KC, int TR, int NT>
__device__ __forceinline__ void mm_zero_pad(uint8_t *lds)
{
    constexpr int tb = mm_tok_bytes(KC), PADW = KC / 16; // 16-byte pad words per token
    for (int i = (int)threadIdx.x; i < TR * PADW; i += NT) {
        const int t = i / PADW, u = i % PADW;
        *(uint4 *)(lds + (size_t)t * tb + 256 * (u >> 2) + 192 + 16 * (u & 3)) = make_uint4(0u, 0u, 0u, 0u);
    }
}

// Copies columns k0 .. k0 + KC of tokens t0 .. t0 + TR - 1 from the staged rows
// (xg, mm_tok_bytes(cols) bytes per token) into LDS (mm_tok_bytes(KC) per
// token, the same layout for the chunk); a thread that copies a nonzero
// outlier mask word writes seq into *oflag.  cols, k0 and KC are multiples of
// 256, so every region but the 2^-e one moves in 16-byte words: MB of them per
// thread are requested before any is stored, so a batch costs one round trip.
// The digits' zero pad (mm_zero_pad) is not copied: per 256 bytes, words 0 ..
// 11 (planes 0 .. 2) move and 12 .. 15 stay.  On MI355X, 64 tokens, per call:
// Q8_0 4096 x 4096 34.7 -> 32.8 us, Q4_K 14336 x 4096 47.8 -> 47.2 us (the
// Q8_0 kernel is bound by the bytes each CU pulls through its L1, about 8 per
// cycle: 64 rows of weights and 16 tokens of staged x per workgroup).
template <int KC, int TR, int NT, bool SUMS = true>
__device__ __forceinline__ void mm_copy(uint8_t *lds, const uint8_t *__restrict__ xg, int t0, int cols, int k0,
                                        int *oflag, int seq)
{
    // (SUMS false: the sub-block sums, which only Q4_K's min term reads, stay behind)
    constexpr int tb = mm_tok_bytes(KC), DW = KC * 3 / 16, SW = SUMS ? KC / 128 : 0, MW = KC / 128, PW = KC / 256;
    // MB words per thread in flight: all of a thread's words (one round trip
    // per chunk) up to 32, else batches of 8.  On MI355X, 64 tokens: Q8_0
    // 4096 x 4096 (256 threads, 13 words each per 1024 columns) 29.8-29.9 us
    // with batches of 8 -> 28.6-28.7 with one batch; Q4_K 14336 x 4096 (896
    // threads, 4 words) 47.2-47.9 -> 47.0-47.5.  (With the pad plane still
    // copied, 17 words per Q8_0 thread: batches of 4 / 8 / 16 37.0 / 34.7 /
    // 43.1 us.)
    constexpr int PT = DW + SW + MW, TOT = TR * PT, PER = (TOT + NT - 1) / NT, MB = PER <= 32 ? PER : 8;
    const int tbf = mm_tok_bytes(cols);
    const int dsrc = 4 * k0, ssrc = mm_sum_off(cols) + (k0 >> 3), psrc = mm_p_off(cols) + (k0 >> 6),
              msrc = mm_mask_off(cols) + (k0 >> 3);
    // word w of a token: its source and LDS offsets
    auto offs = [&](int w, int &src, int &dst) {
        if (w < DW) {
            const int wd = (w / 12) * 16 + w % 12; // the digit word, pad words skipped
            src = dsrc + 16 * wd;
            dst = 16 * wd;
        } else if (w < DW + SW) {
            src = ssrc + 16 * (w - DW);
            dst = mm_sum_off(KC) + 16 * (w - DW);
        } else {
            src = msrc + 16 * (w - DW - SW);
            dst = mm_mask_off(KC) + 16 * (w - DW - SW);
        }
    };
    // the 2^-e floats (one per thread) are requested with the first batch and
    // stored after the last: no round trip of their own (Q8_0 4096 x 4096 at
    // 64 tokens 29.97-30.03 -> 29.74-29.77 us per call; Q4_K unchanged)
    static_assert(TR * PW <= NT, "one 2^-e float per thread");
    const int pi = (int)threadIdx.x < TR * PW ? (int)threadIdx.x : 0;
    const float pv = *(const float *)(xg + (size_t)(t0 + pi / PW) * tbf + psrc + 4 * (pi % PW));
    bool any = false;
    for (int i0 = 0; i0 < TOT; i0 += MB * NT) {
        uint4 v[MB];
#pragma unroll
        for (int k = 0; k < MB; k++) {
            const int i = i0 + k * NT + (int)threadIdx.x;
            v[k] = make_uint4(0u, 0u, 0u, 0u);
            if (i < TOT) {
                int src, dst;
                offs(i % PT, src, dst);
                v[k] = *(const uint4 *)(xg + (size_t)(t0 + i / PT) * tbf + src);
            }
        }
#pragma unroll
        for (int k = 0; k < MB; k++) {
            const int i = i0 + k * NT + (int)threadIdx.x;
            if (i < TOT) {
                const int t = i / PT, w = i % PT;
                int src, dst;
                offs(w, src, dst);
                *(uint4 *)(lds + (size_t)t * tb + dst) = v[k];
                if (w >= DW + SW) any = any || (v[k].x | v[k].y | v[k].z | v[k].w) != 0u;
            }
        }
    }
    if ((int)threadIdx.x < TR * PW) *(float *)(lds + (size_t)(pi / PW) * tb + mm_p_off(KC) + 4 * (pi % PW)) = pv;
    if (any) *oflag = seq;
}

// gfx950 lane swaps: V32 exchanges a of lanes 32 .. 63 with b of lanes 0 ..
// 31, V16 a of the odd 16-lane rows with b of the even rows.  In the MFMA
// layouts here (lane = 16 g + n) they pair lanes (n, g) with (n, g ^ 2) and
// (n, g ^ 1): a row's four lanes can load its bytes contiguously and then
// regroup them.  (The Q4_K matmul keeps mf_load_sb's loads: with its codes
// and header loaded this way, 14336 x 4096 at 64 tokens measured 47.0-48.1 ->
// 48.5-49.3 us, the codes alone 47.3-47.8, the header alone 47.5-48.2.)
__device__ __forceinline__ void lane_swap32(uint32_t &a, uint32_t &b)
{
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void lane_swap16(uint32_t &a, uint32_t &b)
{
    const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}

// Two 16-byte pieces per lane of a row's four lanes (n, g), piece P of lane
// j = piece (plane P, unit j) -> lane (n, g) gets, for each j, the 8 bytes
// at half g & 1 of lane j's piece of plane g >> 1: q[j].  V32 then V16.
__device__ __forceinline__ void lane_regroup(uint4 A, uint4 B, uint2 (&q)[4])
{
    // lanes with g < 2 keep plane 0 and receive it from g + 2, the others
    // keep plane 1 and receive it from g - 2: A then holds the pieces of
    // source lane g & 1, B of (g & 1) + 2
    lane_swap32(A.x, B.x);
    lane_swap32(A.y, B.y);
    lane_swap32(A.z, B.z);
    lane_swap32(A.w, B.w);
    // the same across g ^ 1 with the halves: .xy then holds source lane
    // 2 s + 0, .zw source lane 2 s + 1 (s = 0 for A, 1 for B)
    lane_swap16(A.x, A.z);
    lane_swap16(A.y, A.w);
    lane_swap16(B.x, B.z);
    lane_swap16(B.y, B.w);
    q[0] = make_uint2(A.x, A.y);
    q[1] = make_uint2(A.z, A.w);
    q[2] = make_uint2(B.x, B.y);
    q[3] = make_uint2(B.z, B.w);
}

// NW wavefronts of 16 rows, rounds of 4 MT tokens, KC columns per staged
// chunk, LAH super-blocks of weights in flight per wavefront across chunk edges.
template <int NW, int MT, int KC, int LAH>
__global__ void __launch_bounds__(64 * NW) k_mm_q4k(const uint8_t *__restrict__ W, size_t stride, int rows, int cols,
                                                    const uint8_t *__restrict__ xg, const float *__restrict__ xs,
                                                    float *__restrict__ out)
{
    constexpr int TR = 4 * MT, ROWS = 16 * NW, NSB = KC / 256, MM_LAH = LAH;
    constexpr int tb = mm_tok_bytes(KC);
    extern __shared__ uint4 mm_smem[];
    uint8_t *lds = (uint8_t *)mm_smem;
    __shared__ int oflag_s;
    if (threadIdx.x == 0) oflag_s = -1;
    int seq = 0;
    mm_zero_pad<KC, TR, 64 * NW>(lds); // (the first chunk's copy follows a barrier)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nblk = (rows + ROWS - 1) / ROWS;
    const int b = (int)blockIdx.x % nblk, t0 = ((int)blockIdx.x / nblk) * TR;
    const int r0 = b * ROWS, rend = min(rows, r0 + ROWS);
    const rsrc_t rA = make_rsrc(W + (size_t)r0 * stride, (uint32_t)((size_t)(rend - r0) * stride));
    const int nl = lane & 15, g = lane >> 4;
    const uint32_t rowoff = (uint32_t)((16 * wave + nl) * stride);
    const int nb = cols >> 8, U = cols >> 6;
    const uint32_t qoff = (uint32_t)(16 * nb + (g < 2 ? 0 : 16 * U) + 8 * (g & 1));
    const int a_tok = nl >> 2, a_dig = nl & 3; // digit 3: the zero plane
    const int row = r0 + 16 * wave + nl;
    float accf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) accf[mt] = 0.0f;
    auto scaled = [](uint32_t codes, uint32_t k) {
        return __builtin_bit_cast(uint32_t, __builtin_bit_cast(mf_u16x2, codes) * __builtin_bit_cast(mf_u16x2, k));
    };
    // super-block i of the staged chunk with this lane's weights c
    auto superblock = [&](int i, const MfSb &c) {
        MfScale sc;
        mf_scales(c.h, sc);
        uint32_t klo[8], khi[8];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint32_t lo4 = sc.sc4[t] & 0x07070707u, hi4 = (sc.sc4[t] >> 3) & 0x07070707u;
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                const uint32_t sel = 0x0c000c00u | (uint32_t)bb | ((uint32_t)bb << 16);
                klo[4 * t + bb] = __builtin_amdgcn_perm(0u, lo4, sel);
                khi[4 * t + bb] = __builtin_amdgcn_perm(0u, hi4, sel);
            }
        }
        // the super-block's B operands (the four units' codes times the scale
        // parts) and min factors once, then token tile after token tile: its
        // four units' A operands, the two MFMA chains, the min term and the f32
        // step (the sums are k_mfma_q4k's, in its order)
        mf_v4i bl[4], bh[4];
        float mf[8];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int j0 = 2 * p, j1 = 2 * p + 1;
            const uint2 qv = c.q[p];
            const uint32_t lx = qv.x & 0x0F0F0F0Fu, ly = qv.y & 0x0F0F0F0Fu;
            const uint32_t hx = (qv.x >> 4) & 0x0F0F0F0Fu, hy = (qv.y >> 4) & 0x0F0F0F0Fu;
            bl[p] = mf_v4i{(int)scaled(lx, klo[j0]), (int)scaled(ly, klo[j0]), (int)scaled(hx, klo[j1]),
                           (int)scaled(hy, klo[j1])};
            bh[p] = mf_v4i{(int)scaled(lx, khi[j0]), (int)scaled(ly, khi[j0]), (int)scaled(hx, khi[j1]),
                           (int)scaled(hy, khi[j1])};
            mf[j0] = (float)mf_byte(sc.m4[j0 >> 2], j0 & 3);
            mf[j1] = (float)mf_byte(sc.m4[j1 >> 2], j1 & 3);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint8_t *tp = lds + (size_t)(mt * 4 + a_tok) * tb + (4 * i * 4 + a_dig) * 64 + 16 * g;
            mf_v4i xa[4];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint4 u = *(const uint4 *)(tp + 256 * p);
                xa[p] = mf_v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w};
            }
            const uint8_t *to = lds + (size_t)(mt * 4 + g) * tb;
            const float4 xs0 = *(const float4 *)(to + mm_sum_off(KC) + 32 * i);
            const float4 xs1 = *(const float4 *)(to + mm_sum_off(KC) + 32 * i + 16);
            const float xsm[8] = {xs0.x, xs0.y, xs0.z, xs0.w, xs1.x, xs1.y, xs1.z, xs1.w};
            const float P = *(const float *)(to + mm_p_off(KC) + 4 * i);
            mf_v4i clo = mf_v4i{0, 0, 0, 0}, chi = clo;
            float mins = 0.0f;
#pragma unroll
            for (int p = 0; p < 4; p++) {
                clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[p], bl[p], clo, 0, 0, 0);
                chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[p], bh[p], chi, 0, 0, 0);
                mins = fmaf(mf[2 * p], xsm[2 * p], fmaf(mf[2 * p + 1], xsm[2 * p + 1], mins));
            }
            const int S0 = clo[0] + 8 * chi[0], S1 = clo[1] + 8 * chi[1], S2 = clo[2] + 8 * chi[2];
            const float t = fmaf((float)S2, 65536.0f, fmaf((float)S1, 256.0f, (float)S0));
            accf[mt] = fmaf(-sc.dmin, mins, fmaf(sc.d * P, t, accf[mt]));
        }
    };
    // the outliers of the staged chunk (first column k0), as k_mfma_q4k adds them
    auto correct = [&](int k0) {
        for (int i = 0; i < NSB; i++) {
            if (!mf_sb_has_outliers(lds, tb, mm_mask_off(KC), TR, i)) continue; // uniform
            MfSb S_;
            mf_load_sb(rA, rowoff, qoff, (k0 >> 8) + i, true, S_);
            MfScale K_;
            mf_scales(S_.h, K_);
            auto code = [&](int e) {
                const int eu = e & 63, l = eu & 31;
                const uint32_t dw = mf_fetch<4>(S_.q, 16 * (l >> 3) + nl, 2 * (e >> 6) + ((l & 7) >> 2));
                return (dw >> (8 * (l & 3) + (eu >= 32 ? 4 : 0))) & 15u;
            };
            auto wt = [&](uint32_t q, int e) {
                const int j = 2 * (e >> 6) + ((e & 63) >= 32 ? 1 : 0), sh = 8 * (j & 3);
                const float scv = (float)(((j < 4 ? K_.sc4[0] : K_.sc4[1]) >> sh) & 0xffu);
                const float mn = (float)(((j < 4 ? K_.m4[0] : K_.m4[1]) >> sh) & 0xffu);
                return __fsub_rn(__fmul_rn(__fmul_rn(K_.d, scv), (float)q), __fmul_rn(K_.dmin, mn));
            };
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int to = mt * 4 + g;
                const float *xr = xs + (size_t)(t0 + to) * cols + k0;
                accf[mt] += mf_outliers(lds + (size_t)to * tb, xr, mm_mask_off(KC), i, true, code, wt);
            }
        }
    };
    MfSb w[MM_LAH];
#pragma unroll
    for (int k = 0; k < MM_LAH; k++) mf_load_sb(rA, rowoff, qoff, k, k < nb, w[k]);
    bool oany = false;
    for (int s0 = 0; s0 < nb; s0 += MM_LAH) {
#pragma unroll
        for (int j = 0; j < MM_LAH; j++) {
            const int s = s0 + j;
            if (s < nb) { // uniform
                if (s % NSB == 0) {
                    // a new chunk: the last one's outliers, then its staging
                    if (__builtin_expect(oany, 0)) correct((s - NSB) * 256); // (oany is false at s = 0)
                    __syncthreads(); // the previous chunk's readers of LDS are done
                    mm_copy<KC, TR, 64 * NW>(lds, xg, t0, cols, s * 256, &oflag_s, ++seq);
                    __syncthreads();
                    oany = __builtin_amdgcn_readfirstlane(oflag_s) == seq;
                }
                superblock(s % NSB, w[j]);
            }
            __builtin_amdgcn_sched_barrier(0);
            mf_load_sb(rA, rowoff, qoff, s + MM_LAH, s + MM_LAH < nb, w[j]);
        }
    }
    if (__builtin_expect(oany, 0)) correct((nb - NSB) * 256);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
        if (row < rows) out[(size_t)(t0 + mt * 4 + g) * rows + row] = accf[mt];
}

// ---------------------------------------------------------------------------
// Q8_0 products of several tokens per weight row (dense matmul from 16
// tokens).  The codes are int8 already and every 32-element block has its
// own f32 scale, so each block is one v_mfma_i32_16x16x32_i8 per 4-token
// tile: exact int32 sums S[digit] = sum_k digit_k * q_k (|S| < 2^20), then in
// f32 y += scale * 2^-e * (S0 + 256 S1 + 65536 S2), block by block in column
// order (the Q8_0 dot of crates/sosomodel/src/dequant.rs:292-315 with x in
// exact digits).  x is staged as for Q4_K (mf_stage: one exponent per 256
// columns).  Operands (16 x 16 x 32, int8; lane l, n = l % 16, g = l / 16):
//   A: row m = n = (token n / 4 of the tile, digit n % 4; 3 a zero pad),
//      bytes 0..7 = elements 8g .. 8g + 7 of the block      <- LDS
//   B: column n = weight row n, the same 8 code bytes of the block
//      (bytes 16 (g / 2) .. of the block are plane 2b + g / 2 of the packed
//      row, so the lane's 8 bytes are one aligned load)
//   D: column n, rows 4g .. 4g + 3 = token g of the tile, digits 0..3.
// A workgroup of NW wavefronts owns 16 rows per wavefront and one round of
// 4 MT tokens; it walks the columns 256 at a time (8 blocks), the next 256
// columns' loads in flight while one stretch is applied.  Measured on MI355X,
// 4096 x 4096 at 64 tokens: 45 us (one 64-column unit at a time: 54 us;
// three 256-column stretches in flight: 48 us).
// ---------------------------------------------------------------------------
struct MfQ80 {
    uint4 s[2]; // f32 scales of the 8 blocks of 256 columns (this lane's row)
    uint2 q[8]; // bytes 8g .. 8g + 7 of each block's codes
};

template <int MT, int NW>
__global__ void __launch_bounds__(64 * NW) k_mfma_q80(const uint8_t *__restrict__ W0, size_t stride, int rows, int cols,
                                                      const float *__restrict__ xs, int dense_n, int kcmax,
                                                      float *__restrict__ out)
{
    typedef long mf_i64;
    constexpr int TR = 4 * MT;
    extern __shared__ uint4 mf_smem[];
    uint8_t *lds = (uint8_t *)mf_smem;
    __shared__ int slot_s[TR];
    __shared__ int oflag_s; // the seq of the last staged chunk with outliers
    if (threadIdx.x == 0) oflag_s = -1;
    int seq = 0;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    constexpr int ROWS = 16 * NW;
    const int nblk = (rows + ROWS - 1) / ROWS;
    const int b = blockIdx.x % nblk;
    const int t_step = (int)(gridDim.x / nblk) * TR;
    const int nl = lane & 15, g = lane >> 4;
    const int U = cols >> 6, nbk = cols >> 5;
    // packed row: the f32 scales (8 bytes per unit, padded to 16), then 4
    // planes of 16 bytes per unit (plane i at + 16 U i)
    const uint32_t sreg = (uint32_t)((4 * nbk + 15) & ~15);
    const uint32_t rowoff = (uint32_t)((16 * wave + nl) * stride);
    const uint32_t qoff = sreg + (uint32_t)(16 * U * (g >> 1) + 8 * (g & 1));
    const int a_tok = nl >> 2, a_dig = nl & 3;
    for (int t0 = (blockIdx.x / nblk) * TR; t0 < dense_n; t0 += t_step) {
        const int nt = min(TR, dense_n - t0);
        __syncthreads();
        if ((int)threadIdx.x < nt) slot_s[threadIdx.x] = t0 + threadIdx.x;
        __syncthreads();
        const int r0 = b * ROWS, rend = min(rows, r0 + ROWS);
        const rsrc_t rA = make_rsrc(W0 + (size_t)r0 * stride, (uint32_t)((size_t)(rend - r0) * stride));
        const int row = r0 + 16 * wave + nl;
        float accf[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) accf[mt] = 0.0f;
        for (int k0 = 0; k0 < cols; k0 += kcmax) {
            const int kc = min(kcmax, cols - k0), tb = mf_tok_bytes(kc), nsb = kc >> 8, sb0 = k0 >> 8;
            auto load_sb = [&](int sb, bool in, MfQ80 &o) {
                const uint32_t off = in ? rowoff : 0x80000000u;
                o.s[0] = bld16(rA, off + 32u * (uint32_t)sb);
                o.s[1] = bld16(rA, off + 32u * (uint32_t)sb + 16u);
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const uint32_t u = 4u * (uint32_t)sb + (uint32_t)p;
                    o.q[2 * p] = bld8(rA, off + qoff + 16u * u);
                    o.q[2 * p + 1] = bld8(rA, off + qoff + 32u * (uint32_t)U + 16u * u);
                }
            };
            MfQ80 cur, nxt;
            load_sb(sb0, true, cur); // requested before x is staged: its latency overlaps the staging
            __builtin_amdgcn_sched_barrier(0);
            mf_stage<NW>(lds, xs, slot_s, 1, cols, k0, kc, nt, &oflag_s, ++seq);
            __syncthreads();
            const bool oany = __builtin_amdgcn_readfirstlane(oflag_s) == seq;
            for (int i = 0; i < nsb; i++) {
                load_sb(sb0 + i + 1, i + 1 < nsb, nxt);
                __builtin_amdgcn_sched_barrier(0);
                const uint32_t scs[8] = {cur.s[0].x, cur.s[0].y, cur.s[0].z, cur.s[0].w,
                                         cur.s[1].x, cur.s[1].y, cur.s[1].z, cur.s[1].w};
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int sbl = 8 * i + k; // the block's 32-element sub-block in the chunk
                    const float scale = __builtin_bit_cast(float, scs[k]);
                    // block k: unit k / 2, half k % 2 (q[2 p + half])
                    const uint2 qq = cur.q[2 * (k >> 1) + (k & 1)];
                    const mf_i64 bq = (mf_i64)(((uint64_t)qq.y << 32) | qq.x);
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        if (mt * 4 >= nt) break; // uniform
                        const int ta = mt * 4 + a_tok;
                        mf_i64 xa = 0;
                        if (a_dig < 3 && ta < nt) {
                            const uint2 u = *(const uint2 *)(lds + (size_t)ta * tb + (sbl * 3 + a_dig) * 32 + 8 * g);
                            xa = (mf_i64)(((uint64_t)u.y << 32) | u.x);
                        }
                        const mf_v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, bq, mf_v4i{0, 0, 0, 0}, 0, 0, 0);
                        const int to = mt * 4 + g;
                        const float P = *(const float *)(lds + (size_t)(to < nt ? to : 0) * tb + (kc >> 5) * 100 +
                                                         4 * i);
                        const float t = fmaf((float)d[2], 65536.0f, fmaf((float)d[1], 256.0f, (float)d[0]));
                        accf[mt] = fmaf(scale * P, t, accf[mt]);
                    }
                }
                cur = nxt;
                __builtin_amdgcn_sched_barrier(0);
            }
            // ---- the outliers of the round's tokens: a second walk over the
            // 256-column stretches that hold some (rare), reloading the codes:
            // w * x with w = fl(q * scale) (dequant.rs:74-97).  Element e of a
            // stretch: block e / 32, code byte l = e % 32 (lane group l / 8 of
            // this row holds it).
            if (__builtin_expect(oany, 0)) {
                for (int i = 0; i < nsb; i++) {
                    if (!mf_sb_has_outliers(lds, tb, mf_mask_off(kc), nt, i)) continue; // uniform
                    MfQ80 o;
                    load_sb(sb0 + i, true, o);
                    auto code = [&](int e) {
                        const int l = e & 31;
                        const uint32_t dw = mf_fetch<8>(o.q, 16 * (l >> 3) + nl, 2 * (e >> 5) + ((l & 7) >> 2));
                        return (dw >> (8 * (l & 3))) & 0xffu;
                    };
                    auto wt = [&](uint32_t q, int e) {
                        const int kb = e >> 5, kq = kb & 3;
                        const uint4 sv = kb < 4 ? o.s[0] : o.s[1];
                        const uint32_t sbits = kq == 0 ? sv.x : kq == 1 ? sv.y : kq == 2 ? sv.z : sv.w;
                        return __fmul_rn((float)(int8_t)(uint8_t)q, __builtin_bit_cast(float, opaque(sbits)));
                    };
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        if (mt * 4 >= nt) break; // uniform
                        const int to = mt * 4 + g, tv = to < nt ? to : 0;
                        const float *xr = xs + (size_t)slot_s[tv] * cols + k0;
                        accf[mt] += mf_outliers(lds + (size_t)tv * tb, xr, mf_mask_off(kc), i, to < nt, code, wt);
                    }
                }
            }
            __syncthreads(); // LDS is restaged for the next chunk or round
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int to = mt * 4 + g;
            if (mt * 4 < nt && to < nt && row < rows) out[(size_t)slot_s[to] * rows + row] = accf[mt];
        }
    }
}

// ---------------------------------------------------------------------------
// Dense Q8_0 products with x staged once (k_mm_stage, the paired layout), as
// k_mm_q4k is to k_mfma_q4k: k_mfma_q80's arithmetic and order of sums (one
// v_mfma_i32_16x16x32_i8 per 32-element block and 4-token tile, the block's
// f32 step at once), the A operand one 8-byte load (the zero plane for the
// pad lanes), full rounds only, token tile after token tile per 256 columns.
// ---------------------------------------------------------------------------
template <int NW, int MT, int KC>
__global__ void __launch_bounds__(64 * NW) k_mm_q80(const uint8_t *__restrict__ W, size_t stride, int rows, int cols,
                                                    const uint8_t *__restrict__ xg, const float *__restrict__ xs,
                                                    float *__restrict__ out)
{
    typedef long mf_i64;
    constexpr int TR = 4 * MT, ROWS = 16 * NW, NSB = KC / 256;
    constexpr int tb = mm_tok_bytes(KC);
    extern __shared__ uint4 mm_smem[];
    uint8_t *lds = (uint8_t *)mm_smem;
    __shared__ int oflag_s;
    if (threadIdx.x == 0) oflag_s = -1;
    int seq = 0;
    mm_zero_pad<KC, TR, 64 * NW>(lds); // (the first chunk's copy follows a barrier)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nblk = (rows + ROWS - 1) / ROWS;
    const int b = (int)blockIdx.x % nblk, t0 = ((int)blockIdx.x / nblk) * TR;
    const int r0 = b * ROWS, rend = min(rows, r0 + ROWS);
    const rsrc_t rA = make_rsrc(W + (size_t)r0 * stride, (uint32_t)((size_t)(rend - r0) * stride));
    const int nl = lane & 15, g = lane >> 4;
    const int U = cols >> 6, nbk = cols >> 5, nb = cols >> 8;
    // packed row: the f32 scales (padded to 16 bytes), then 4 planes of 16
    // bytes per unit (plane i at + 16 U i)
    const uint32_t sreg = (uint32_t)((4 * nbk + 15) & ~15);
    const uint32_t rowoff = (uint32_t)((16 * wave + nl) * stride);
    const uint32_t qoff = sreg + (uint32_t)(16 * U * (g >> 1) + 8 * (g & 1));
    const int a_tok = nl >> 2, a_dig = nl & 3; // digit 3: the zero plane
    const int row = r0 + 16 * wave + nl;
    auto load_sb = [&](int sb, bool in, MfQ80 &o) {
        const uint32_t off = in ? rowoff : 0x80000000u;
        o.s[0] = bld16(rA, off + 32u * (uint32_t)sb);
        o.s[1] = bld16(rA, off + 32u * (uint32_t)sb + 16u);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t u = 4u * (uint32_t)sb + (uint32_t)p;
            o.q[2 * p] = bld8(rA, off + qoff + 16u * u);
            o.q[2 * p + 1] = bld8(rA, off + qoff + 32u * (uint32_t)U + 16u * u);
        }
    };
    // The main loop's weights, one 256-column stretch: lane (n, g) loads 16
    // bytes of each plane p at unit 4 sb + g, so a row's four lanes read the
    // plane's 64 contiguous bytes (one 16-byte load per plane: 16 rows x 64
    // bytes per instruction, against 16 rows x 2 x 16 bytes for 8 bytes per
    // lane in the MFMA's order).  Two butterfly stages of lane swaps then give
    // lane (n, g) the 8 bytes of every block the MFMA wants from it (those
    // that load_sb reads): V32 swaps lanes g <-> g ^ 2 (the planes' odd/even
    // parts), V16 lanes g <-> g ^ 1 (the two 8-byte halves).  The row's 8
    // scales likewise: lane g loads scales 2g, 2g + 1, and two stages of
    // swaps of copies gather all 8.  Measured on MI355X, 4096 x 4096 at 64
    // tokens, per call: 32.6 us with 8-byte loads in the MFMA's order, 30.6
    // with the coalesced codes, 30.1 with the scales gathered too.  (The
    // kernel is bound by what each CU pulls through its L1, not by latency:
    // two or three stretches in flight measured 38.6 / 40.7 us, a second
    // wavefront per SIMD taking half the tokens 50.9 us.)
    struct MmQ80 {
        uint2 sc;   // scales 2g, 2g + 1 of the stretch
        uint4 v[4]; // plane p, unit 4 sb + g
    };
    auto load_mm = [&](int sb, bool in, MmQ80 &o) {
        const uint32_t off = in ? rowoff : 0x80000000u;
        o.sc = bld8(rA, off + 32u * (uint32_t)sb + 8u * (uint32_t)g);
#pragma unroll
        for (int p = 0; p < 4; p++)
            o.v[p] = bld16(rA, off + sreg + 16u * (uint32_t)U * (uint32_t)p + 16u * (4u * (uint32_t)sb + (uint32_t)g));
    };
    auto swap32 = lane_swap32;
    auto swap16 = lane_swap16;
    // MmQ80 -> MfQ80: q[2 j + q'] = bytes 8 g .. 8 g + 7 of block 2 (4 sb + j) + q'
    auto unpack = [&](const MmQ80 &c, MfQ80 &o) {
        {
            // after the V32 stage a* / b* hold scales 2c (+1) and 2c + 4 (+1),
            // c = g & 1; after the V16 stage *0 the c = 0 ones, *1 the c = 1 ones
            uint32_t a0 = c.sc.x, a1 = c.sc.x, b0 = c.sc.y, b1 = c.sc.y;
            swap32(a0, a1);
            swap32(b0, b1);
            uint32_t a0c = a0, a1c = a1, b0c = b0, b1c = b1;
            swap16(a0, a0c);
            swap16(b0, b0c);
            swap16(a1, a1c);
            swap16(b1, b1c);
            o.s[0] = make_uint4(a0, b0, a0c, b0c);
            o.s[1] = make_uint4(a1, b1, a1c, b1c);
        }
#pragma unroll
        for (int q = 0; q < 2; q++) { // planes 2q, 2q + 1: block parity q
            uint2 r[4];
            lane_regroup(c.v[2 * q], c.v[2 * q + 1], r);
#pragma unroll
            for (int j = 0; j < 4; j++) o.q[2 * j + q] = r[j];
        }
    };
    float accf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) accf[mt] = 0.0f;
    auto superblock = [&](int i, const MmQ80 &cm) {
        MfQ80 c;
        unpack(cm, c);
        const uint32_t scs[8] = {c.s[0].x, c.s[0].y, c.s[0].z, c.s[0].w, c.s[1].x, c.s[1].y, c.s[1].z, c.s[1].w};
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint8_t *tp = lds + (size_t)(mt * 4 + a_tok) * tb + (16 * i + a_dig) * 64 + 16 * g;
            const float P = *(const float *)(lds + (size_t)(mt * 4 + g) * tb + mm_p_off(KC) + 4 * i);
            uint2 u[8];
#pragma unroll
            for (int k = 0; k < 8; k++) u[k] = *(const uint2 *)(tp + (k >> 1) * 256 + 8 * (k & 1));
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint2 qq = c.q[2 * (k >> 1) + (k & 1)];
                const mf_i64 bq = (mf_i64)(((uint64_t)qq.y << 32) | qq.x);
                const mf_i64 xa = (mf_i64)(((uint64_t)u[k].y << 32) | u[k].x);
                const mf_v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, bq, mf_v4i{0, 0, 0, 0}, 0, 0, 0);
                const float t = fmaf((float)d[2], 65536.0f, fmaf((float)d[1], 256.0f, (float)d[0]));
                accf[mt] = fmaf(__builtin_bit_cast(float, scs[k]) * P, t, accf[mt]);
            }
        }
    };
    // the outliers of the staged chunk (first column k0): w * x with w =
    // fl(q * scale) (dequant.rs:74-97), as k_mfma_q80 adds them
    auto correct = [&](int k0) {
        for (int i = 0; i < NSB; i++) {
            if (!mf_sb_has_outliers(lds, tb, mm_mask_off(KC), TR, i)) continue; // uniform
            MfQ80 o;
            load_sb((k0 >> 8) + i, true, o);
            auto code = [&](int e) {
                const int l = e & 31;
                const uint32_t dw = mf_fetch<8>(o.q, 16 * (l >> 3) + nl, 2 * (e >> 5) + ((l & 7) >> 2));
                return (dw >> (8 * (l & 3))) & 0xffu;
            };
            auto wt = [&](uint32_t q, int e) {
                const int kb = e >> 5, kq = kb & 3;
                const uint4 sv = kb < 4 ? o.s[0] : o.s[1];
                const uint32_t sbits = kq == 0 ? sv.x : kq == 1 ? sv.y : kq == 2 ? sv.z : sv.w;
                return __fmul_rn((float)(int8_t)(uint8_t)q, __builtin_bit_cast(float, opaque(sbits)));
            };
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int to = mt * 4 + g;
                const float *xr = xs + (size_t)(t0 + to) * cols + k0;
                accf[mt] += mf_outliers(lds + (size_t)to * tb, xr, mm_mask_off(KC), i, true, code, wt);
            }
        }
    };
    MmQ80 cur;
    load_mm(0, true, cur);
    bool oany = false;
    for (int s = 0; s < nb; s++) {
        if (s % NSB == 0) {
            if (__builtin_expect(oany, 0)) correct((s - NSB) * 256); // (oany is false at s = 0)
            __syncthreads(); // the previous chunk's readers of LDS are done
            mm_copy<KC, TR, 64 * NW, false>(lds, xg, t0, cols, s * 256, &oflag_s, ++seq);
            __syncthreads();
            oany = __builtin_amdgcn_readfirstlane(oflag_s) == seq;
        }
        MmQ80 nxt;
        load_mm(s + 1, s + 1 < nb, nxt);
        __builtin_amdgcn_sched_barrier(0);
        superblock(s % NSB, cur);
        cur = nxt;
        __builtin_amdgcn_sched_barrier(0);
    }
    if (__builtin_expect(oany, 0)) correct((nb - NSB) * 256);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
        if (row < rows) out[(size_t)(t0 + mt * 4 + g) * rows + row] = accf[mt];
}

// Columns staged per chunk: the largest multiple of 256 whose x for `tokens`
// tokens fits `budget` bytes of LDS (the workgroup's whole LDS by default).
static int mf_kc(const soso_hip *h, size_t cols, int tokens, size_t budget = 0)
{
    if (budget == 0) budget = h->max_lds;
    int kc = (int)cols;
    while (kc > 256 && (size_t)tokens * mf_tok_bytes(kc) > budget) kc = ((kc / 2) + 255) / 256 * 256;
    return kc;
}

// Shapes the matrix-core path handles: Q4_K or Q8_0 rows of whole 256-column
// super-blocks (x's exponents), strips addressable with 32-bit offsets.
bool mfma_shape_ok(uint8_t dtype, size_t rows, size_t cols)
{
    return (dtype == SOSO_HIP_DTYPE_Q4_K || dtype == SOSO_HIP_DTYPE_Q8_0) && cols % 256 == 0 && cols >= 256 &&
           rows > 0 && (size_t)16 * MF_NW_MAX * packed_row_stride(dtype, cols) < ((size_t)1 << 31);
}

// MoE: one grouped product over the active-expert records (device), or, with
// sidx set, over every expert, each workgroup finding its expert's slots in
// the nslots ranked indices (the route then skips its slot sort).
template <int NMAT, bool TILED>
static void mfma_moe_one(soso_hip *h, unsigned grid, size_t lds, const uint8_t *const *A, const uint8_t *const *B,
                         size_t stride, int rows, int cols, const float *xs, int xdiv, const int *list, const int *recs,
                         const int *n_recs, int kc, float *out, const int32_t *sidx, int nslots)
{
    constexpr int MT = 2, LA = NMAT == 2 ? MF_LA2 : MF_LA1, NW = NMAT == 2 ? MF_NW_GU : MF_NW_DN;
    // The scanning launch (about two tokens per active expert): rounds of one
    // 4-token tile, one MFMA per sub-block with the scales applied to the
    // int32 sums (SPLIT).  Measured on MI355X, MoE batch 32 per layer: 92.3 us
    // with rounds of 8 tokens and the scales folded into the B operands; 91.3-
    // 91.7 with SPLIT for down; 90.4-90.7 with gate/up at 4 tokens and SPLIT
    // too; 88.9-89.1 with down at 4 tokens as well.  Rejected: SPLIT for
    // gate/up at 8 tokens (28 bytes per lane spilled, 97.9), gate/up at 4
    // tokens without SPLIT (92.3-93.0), gate/up held to 128 VGPRs for four
    // wavefronts per SIMD (91.4-91.9).
    if (sidx)
        k_mfma_q4k<NMAT, 1, LA, TILED, NW, true, false, true><<<grid, 64 * NW, lds, h->stream>>>(
            A, B, nullptr, stride, rows, cols, xs, xdiv, list, recs, n_recs, 0, kc, out, sidx, nslots);
    else
        k_mfma_q4k<NMAT, MT, LA, TILED, NW><<<grid, 64 * NW, lds, h->stream>>>(
            A, B, nullptr, stride, rows, cols, xs, xdiv, list, recs, n_recs, 0, kc, out, nullptr, 0);
}

int launch_mfma_moe(soso_hip *h, int nmat, const uint8_t *const *A, const uint8_t *const *B, size_t rows, size_t cols,
                    size_t max_recs, const float *xs, int xdiv, const int *list, const int *recs, const int *n_recs,
                    float *out, bool tiled, const int32_t *sidx, size_t nslots)
{
    if (!mfma_shape_ok(SOSO_HIP_DTYPE_Q4_K, rows, cols) || (tiled && !tiled_q4k_ok(SOSO_HIP_DTYPE_Q4_K, rows, cols)))
        return set_err(h, SOSO_HIP_DECLINED, "mfma: shape");
    if (sidx && nslots > (size_t)MF_SCAN_MAX) return set_err(h, SOSO_HIP_ERR_ARG, "mfma: too many slots to scan");
    const int MT = sidx ? 1 : 2; // tiles per round (mfma_moe_one)
    const size_t scan_b = sidx ? (size_t)mf_scan_bytes((int)nslots) : 0;
    const int kc = mf_kc(h, cols, 4 * MT, h->max_lds - scan_b);
    const size_t mrows = (size_t)16 * (nmat == 2 ? MF_NW_GU : MF_NW_DN); // rows per workgroup
    const size_t nblk = (rows + mrows - 1) / mrows;
    const size_t lds = scan_b + (size_t)4 * MT * mf_tok_bytes(kc);
    const unsigned grid = (unsigned)(max_recs * nblk);
    const size_t stride = packed_row_stride(SOSO_HIP_DTYPE_Q4_K, cols);
    const int ri = (int)rows, ci = (int)cols, ns = (int)nslots;
    if (nmat == 2 && tiled)
        mfma_moe_one<2, true>(h, grid, lds, A, B, stride, ri, ci, xs, xdiv, list, recs, n_recs, kc, out, sidx, ns);
    else if (nmat == 2)
        mfma_moe_one<2, false>(h, grid, lds, A, B, stride, ri, ci, xs, xdiv, list, recs, n_recs, kc, out, sidx, ns);
    else if (tiled)
        mfma_moe_one<1, true>(h, grid, lds, A, nullptr, stride, ri, ci, xs, xdiv, list, recs, n_recs, kc, out, sidx,
                              ns);
    else
        mfma_moe_one<1, false>(h, grid, lds, A, nullptr, stride, ri, ci, xs, xdiv, list, recs, n_recs, kc, out, sidx,
                               ns);
    return hip_check(h, hipGetLastError(), "mfma moe launch");
}

// The MoE calls whose experts both run on the matrix cores with each expert
// workgroup scanning the ranked slots itself (launch_moe_experts' choice, at
// most MF_SCAN_MAX slots): their route can skip the slot sort.
bool mfma_moe_scan_ok(size_t n, size_t top_k, size_t n_groups, uint8_t dt_gu, uint8_t dt_down, size_t hdim,
                      size_t ffn)
{
    const size_t slots = n * top_k, max_recs = std::min(n_groups, slots);
    return slots >= 2 * max_recs && slots <= (size_t)MF_SCAN_MAX && dt_gu == SOSO_HIP_DTYPE_Q4_K &&
           dt_down == SOSO_HIP_DTYPE_Q4_K && mfma_shape_ok(dt_gu, ffn, hdim) && mfma_shape_ok(dt_down, hdim, ffn);
}

template <int NW, int MT>
static void mfma_dense(soso_hip *h, const Weight &w, const float *x, size_t n, float *y, int kc, unsigned grid)
{
    const bool full = n % (4 * MT) == 0;
    const size_t kcols = weight_kcols(w);
    const size_t lds = (size_t)4 * MT * mf_tok_bytes(kc), stride = packed_row_stride(w.dtype, kcols);
    if (w.dtype == SOSO_HIP_DTYPE_Q8_0)
        k_mfma_q80<MT, NW><<<grid, 64 * NW, lds, h->stream>>>((const uint8_t *)w.dev, stride, (int)w.rows,
                                                              (int)kcols, x, (int)n, kc, y);
    else if (full)
        k_mfma_q4k<1, MT, MF_LA1, false, NW, false, true><<<grid, 64 * NW, lds, h->stream>>>(
            nullptr, nullptr, (const uint8_t *)w.dev, stride, (int)w.rows, (int)kcols, x, 1, nullptr, nullptr,
            nullptr, (int)n, kc, y, nullptr, 0);
    else
        k_mfma_q4k<1, MT, MF_LA1, false, NW><<<grid, 64 * NW, lds, h->stream>>>(
            nullptr, nullptr, (const uint8_t *)w.dev, stride, (int)w.rows, (int)kcols, x, 1, nullptr, nullptr,
            nullptr, (int)n, kc, y, nullptr, 0);
}

// Dense: Y[n x rows] = X[n x cols] . W^T.  The grid is (row block of 16 NW
// rows) x (round of 4 MT tokens), one round per workgroup.  A workgroup's own
// chain (staging x, then its rows' super-blocks with one wavefront per SIMD
// or two) sets the time, so the launch takes the (NW, MT) that gives the most
// workgroups still fitting one per CU -- ties to the cheaper workgroup, in
// the order below -- and, when even the largest tiles need more workgroups
// than CUs, the fewest workgroups with half the LDS each (two per CU).  Every
// choice computes the same bits: the integer sums are exact and each lane adds
// its super-blocks in column order whatever the chunking.
// Measured on MI355X, us for one round of workgroups at 4096 columns (any
// row count): (4,1) 17, (8,1) 24, (4,2) 28, (8,2) 28, (16,1) 41, (4,4) 45,
// (16,2) 46, (8,4) 47, (16,4) 66.  Chosen against the best of all 27 (NW, MT,
// LDS share) settings, us: 4096x4096 at 16/32/64/128 tokens 17/24/28/47 (best
// 17/24/28/47); 14336x4096 28/46/70/129 (28/46/66/129); 4096x14336 49/75/88/150
// (49/75/88/150); the rule it replaces gave 14336x4096 46/49/72/136 and
// 4096x14336 51/87/171/362.
static const int MF_DENSE[9][2] = {{4, 1}, {8, 1}, {4, 2}, {8, 2}, {16, 1}, {4, 4}, {16, 2}, {8, 4}, {16, 4}};

// Dense Q4_K with a token count that is a multiple of 16, whose grid fills the
// GPU: x staged once (k_mm_stage into scratch slot 16), then k_mm_q4k with 16
// wavefronts (256 rows), rounds of 16 tokens, 1024-column chunks and one
// super-block ahead.  Measured on MI355X, 14336 x 4096 at 64 tokens (us):
// this shape 56.3-56.7; 2048-column chunks 59.3; 512: 58.9; 256: 76.7;
// 8 wavefronts x 32 tokens 60.8, x 16 tokens 64.6-69.0; 4 wavefronts x 16
// tokens 72.1; 4 x 64 (1 wavefront per SIMD) 120.8; 16 x 8 tokens 88.3;
// k_mfma_q4k staging its own rounds 68.1-68.3.  The wavefront count is then
// chosen per shape among MM_NWS so that the workgroups fill the CUs best (one
// per CU; each CU's work is one workgroup's): 14336 rows at 64 tokens take 14
// wavefronts (224 rows, 64 row blocks x 4 rounds = 256 workgroups): 48.1 us
// against 51.1 with 16 (224 workgroups); 12 (300 workgroups, two per CU on
// some) 76.8 us.
constexpr int MM_MT = 4, MM_KC = 1024, MM_LA = 1;
constexpr int MM_NWS[3] = {16, 14, 12};

template <int NW, int MT, int KC, int LAH>
static void mm_launch(soso_hip *h, const Weight &w, size_t stride, const uint8_t *xg, const float *x, float *y,
                      unsigned grid)
{
    const size_t lds = (size_t)4 * MT * mm_tok_bytes(KC);
    k_mm_q4k<NW, MT, KC, LAH><<<grid, 64 * NW, lds, h->stream>>>((const uint8_t *)w.dev, stride, (int)w.rows,
                                                                 (int)weight_kcols(w), xg, x, y);
}

static int launch_mm_q4k(soso_hip *h, const Weight &w, const float *x, size_t n, float *y)
{
    constexpr int MT = MM_MT, KC = MM_KC, LAH = MM_LA;
    const size_t cols = weight_kcols(w), rounds = n / (4 * MT), cu = (size_t)h->num_cu;
    // the wavefront count whose workgroups keep the CUs busiest: rows over
    // (passes of one workgroup per CU x CUs x rows per workgroup), the larger
    // count on ties
    int NW = MM_NWS[0];
    double best = -1.0;
    for (int nw : MM_NWS) {
        const size_t g = (w.rows + 16 * nw - 1) / (16 * nw) * rounds, passes = (g + cu - 1) / cu;
        const double eff = (double)w.rows * (double)rounds / ((double)passes * (double)cu * 16.0 * nw);
        if (eff > best + 1e-9) {
            best = eff;
            NW = nw;
        }
    }
    const size_t nblk = (w.rows + 16 * NW - 1) / (16 * NW);
    if (n % (size_t)(4 * MT) || cols % KC || (size_t)4 * MT * mm_tok_bytes(KC) > h->max_lds ||
        nblk * rounds * 5 < cu * 4)
        return SOSO_HIP_DECLINED; // k_mfma_q4k's launch, which picks its shape from the grid, takes it
    uint8_t *xg = (uint8_t *)scratch_get(h, 16, n * (size_t)mm_tok_bytes((int)cols));
    if (!xg) return set_err(h, SOSO_HIP_ERR_NOMEM, "mfma: staged x");
    const size_t waves = n * ((cols + 511) / 512);
    k_mm_stage<<<(unsigned)((waves + 3) / 4), 256, 0, h->stream>>>(x, (int)n, (int)cols, xg);
    int rc = hip_check(h, hipGetLastError(), "mm stage launch");
    if (rc != SOSO_HIP_OK) return rc;
    const size_t stride = packed_row_stride(w.dtype, cols);
    const unsigned grid = (unsigned)(nblk * rounds);
    switch (NW) {
    case 16: mm_launch<16, MT, KC, LAH>(h, w, stride, xg, x, y, grid); break;
    case 14: mm_launch<14, MT, KC, LAH>(h, w, stride, xg, x, y, grid); break;
    default: mm_launch<12, MT, KC, LAH>(h, w, stride, xg, x, y, grid); break;
    }
    return hip_check(h, hipGetLastError(), "mm launch");
}

// Dense Q8_0 with x staged once: 4 wavefronts (64 rows), rounds of 16 tokens,
// 2048-column chunks where the width allows (else 1024), where that grid fills
// the GPU.  Measured on MI355X, 4096 x 4096 at 64 tokens (us): 1024-column
// chunks 28.71-28.74, 2048 28.08-28.15 (each chunk copied in one round trip;
// with the chunk copies in batches of 8 words: 1024 37.0, 512 / 2048 41.3 /
// 42.2); rounds of 8 tokens with 4 or 8 wavefronts 48.9 / 49.8; k_mfma_q80
// staging its own rounds 46.6.
constexpr int MQ_NW = 4, MQ_MT = 4, MQ_KC = 2048;

template <int KC>
static void mm_q80_launch(soso_hip *h, const Weight &w, size_t stride, const uint8_t *xg, const float *x, float *y,
                          unsigned grid)
{
    const size_t lds = (size_t)4 * MQ_MT * mm_tok_bytes(KC);
    k_mm_q80<MQ_NW, MQ_MT, KC><<<grid, 64 * MQ_NW, lds, h->stream>>>((const uint8_t *)w.dev, stride, (int)w.rows,
                                                                    (int)weight_kcols(w), xg, x, y);
}

static int launch_mm_q80(soso_hip *h, const Weight &w, const float *x, size_t n, float *y)
{
    constexpr int NW = MQ_NW, MT = MQ_MT;
    const size_t cols = weight_kcols(w), nblk = (w.rows + 16 * NW - 1) / (16 * NW);
    const int KC = cols % MQ_KC == 0 && (size_t)4 * MT * mm_tok_bytes(MQ_KC) <= h->max_lds ? MQ_KC : 1024;
    if (n % (size_t)(4 * MT) || cols % KC || (size_t)4 * MT * mm_tok_bytes(KC) > h->max_lds ||
        nblk * (n / (4 * MT)) * 5 < (size_t)h->num_cu * 4)
        return SOSO_HIP_DECLINED; // k_mfma_q80's launch takes it
    uint8_t *xg = (uint8_t *)scratch_get(h, 16, n * (size_t)mm_tok_bytes((int)cols));
    if (!xg) return set_err(h, SOSO_HIP_ERR_NOMEM, "mfma: staged x");
    const size_t waves = n * ((cols + 511) / 512);
    k_mm_stage<<<(unsigned)((waves + 3) / 4), 256, 0, h->stream>>>(x, (int)n, (int)cols, xg);
    int rc = hip_check(h, hipGetLastError(), "mm stage launch");
    if (rc != SOSO_HIP_OK) return rc;
    const size_t stride = packed_row_stride(w.dtype, cols);
    const unsigned grid = (unsigned)(nblk * (n / (4 * (size_t)MT)));
    if (KC == MQ_KC)
        mm_q80_launch<MQ_KC>(h, w, stride, xg, x, y, grid);
    else
        mm_q80_launch<1024>(h, w, stride, xg, x, y, grid);
    return hip_check(h, hipGetLastError(), "mm q80 launch");
}

int launch_mfma_matmul(soso_hip *h, const Weight &w, const float *x, size_t n, float *y)
{
    const size_t kcols = weight_kcols(w);
    if (!mfma_shape_ok(w.dtype, w.rows, kcols) || n == 0 || n > (1u << 20))
        return set_err(h, SOSO_HIP_DECLINED, "mfma: shape");
    {
        const int rc = w.dtype == SOSO_HIP_DTYPE_Q4_K ? launch_mm_q4k(h, w, x, n, y) : launch_mm_q80(h, w, x, n, y);
        if (rc != SOSO_HIP_DECLINED) return rc;
    }
    const size_t cu = (size_t)h->num_cu;
    auto groups = [&](int nw, int mt) { return (w.rows + 16 * nw - 1) / (16 * nw) * ((n + 4 * mt - 1) / (4 * mt)); };
    int pick = -1;
    for (int i = 0; i < 9; i++) { // the most workgroups within one per CU
        const size_t gi = groups(MF_DENSE[i][0], MF_DENSE[i][1]);
        if (gi <= cu && (pick < 0 || gi > groups(MF_DENSE[pick][0], MF_DENSE[pick][1]))) pick = i;
    }
    if (pick < 0) // else the fewest
        for (int i = 0; i < 9; i++)
            if (pick < 0 || groups(MF_DENSE[i][0], MF_DENSE[i][1]) < groups(MF_DENSE[pick][0], MF_DENSE[pick][1]))
                pick = i;
    const int nw = MF_DENSE[pick][0], mt = MF_DENSE[pick][1];
    const size_t grid = groups(nw, mt);
    const int kc = mf_kc(h, kcols, 4 * mt, grid > cu ? h->max_lds / 2 : h->max_lds);
    const unsigned gu = (unsigned)grid;
    switch (nw * 8 + mt) {
    case 4 * 8 + 1: mfma_dense<4, 1>(h, w, x, n, y, kc, gu); break;
    case 4 * 8 + 2: mfma_dense<4, 2>(h, w, x, n, y, kc, gu); break;
    case 4 * 8 + 4: mfma_dense<4, 4>(h, w, x, n, y, kc, gu); break;
    case 8 * 8 + 1: mfma_dense<8, 1>(h, w, x, n, y, kc, gu); break;
    case 8 * 8 + 2: mfma_dense<8, 2>(h, w, x, n, y, kc, gu); break;
    case 8 * 8 + 4: mfma_dense<8, 4>(h, w, x, n, y, kc, gu); break;
    case 16 * 8 + 1: mfma_dense<16, 1>(h, w, x, n, y, kc, gu); break;
    case 16 * 8 + 2: mfma_dense<16, 2>(h, w, x, n, y, kc, gu); break;
    default: mfma_dense<16, 4>(h, w, x, n, y, kc, gu); break;
    }
    return hip_check(h, hipGetLastError(), "mfma matmul launch");
}
