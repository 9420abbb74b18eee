// k_matvec.hip -- block-quantized matrix-vector products for gfx950.
//
// Reference path: soso-llm-core's fused dequant+dot matvecs
//   Q8_0  crates/soso-llm-core/src/gemm.rs:295-332, 806-836
//   Q4_K  crates/soso-llm-core/src/gemm.rs:402-461, 842-894
//   Q6_K  dequant of crates/gguf2som/src/lib.rs:1639-1661 + f32 dot
//   F32   crates/soso-llm-core/src/gemm.rs:34-56 (MoE router)
// and the exact dequantizers of crates/sosomodel/src/dequant.rs.
//
// Design (one GPU, HBM-bound):
//  * Weights are repacked once at upload into a per-row "planar" layout: every
//    lane of a wavefront owns one 64-element unit of a row, and the 16-byte
//    pieces of all units are stored plane by plane, so each 128-bit load
//    instruction of a wavefront reads 1 KiB of contiguous HBM.  Same bytes as
//    soso's layout (no inflation; Q8_0/Q6_K rows are padded to 16 B only when
//    their byte count is not a multiple of 16).
//  * x is staged once per workgroup in LDS as integers X = rint(x * 2^e), one
//    exponent e per 128-element block (|X| <= 2^22), written as three balanced
//    signed base-256 digit planes (one byte per element per digit), plus f32
//    sums of every 16 elements for the min / offset terms; each lane then keeps
//    its unit's digits in VGPRs for the whole launch.
//  * Quant codes are unpacked in registers (an AND or a shift per four codes)
//    and meet the digits in v_dot4_i32_i8: exact int32 sums per digit and
//    sub-block, rounded to f32 once per sub-block before the block scales are
//    applied.  The reduction across the lanes of a row uses DPP adds, and a
//    strip's row sums leave in one store.
#include "internal.hpp"

#include <algorithm>

// ---------------------------------------------------------------------------
// Packed layouts (per row; see the repack kernels for the exact byte moves)
//   Q4_K : H[sb] 16 B (d, dmin, scales) | QA[u] 16 B | QB[u] 16 B
//          unit u = pair p of superblock sb = 4*sb + p (64 elements);
//          QA/QB = first/second 16 qs bytes of the pair.
//   Q8_0 : S[b] f32 (region padded to 16 B) | 4 planes of 16 B per unit
//          unit u = blocks 2u, 2u+1 (64 elements, 64 qs bytes)
//   Q6_K : SC[sb] 16 B | QH[u] | QLa[u] | QLb[u] (16 B each) | D[sb] 2 B,
//          unit u = 4*sb + 2*h + kk covers, in half h, l in [16kk, 16kk+16)
//          for the four quarter-runs l, l+32, l+64, l+96.
// ---------------------------------------------------------------------------
static inline size_t rup16(size_t v) { return (v + 15) & ~(size_t)15; }

size_t packed_row_stride(uint8_t dtype, size_t cols)
{
    size_t nb;
    switch (dtype) {
    case SOSO_HIP_DTYPE_F32: return cols * 4;
    case SOSO_HIP_DTYPE_Q4_K: return cols / 256 * Q4_K_BYTES;
    case SOSO_HIP_DTYPE_Q8_0: nb = cols / 32; return rup16(4 * nb) + 32 * nb;
    case SOSO_HIP_DTYPE_Q6_K: nb = cols / 256; return rup16(210 * nb);
    default: return 0;
    }
}

// Q8_0 rows of an odd number of blocks (soso accepts any multiple of 32,
// dequant.rs:53-68) are stored with one zero block appended: its scale and
// codes are 0, so it adds exactly 0 to every sum, and the 64-element units of
// the layout tile the row.  The x a kernel reads over such a row is padded
// with zeros to match (launch_matvec).
size_t kernel_cols(uint8_t dtype, size_t cols)
{
    return dtype == SOSO_HIP_DTYPE_Q8_0 && cols % 64 == 32 ? cols + 32 : cols;
}

bool upload_shape_ok(uint8_t dtype, size_t rows, size_t cols)
{
    return packed_shape_ok(dtype, rows, kernel_cols(dtype, cols)) && (dtype != SOSO_HIP_DTYPE_Q8_0 || cols % 32 == 0);
}

// Shapes the quantized kernels accept: the 64-element unit must tile a row.
bool packed_shape_ok(uint8_t dtype, size_t rows, size_t cols)
{
    if (rows == 0 || cols == 0) return false;
    switch (dtype) {
    case SOSO_HIP_DTYPE_F32: return cols % 4 == 0;
    case SOSO_HIP_DTYPE_Q4_K:
    case SOSO_HIP_DTYPE_Q6_K: return cols % 256 == 0;
    case SOSO_HIP_DTYPE_Q8_0: return cols % 64 == 0;
    default: return false;
    }
}

__global__ void repack_q4k(const uint8_t *__restrict__ raw, uint8_t *__restrict__ out, int rows, int nb)
{
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)rows * nb) return;
    int r = (int)(t / nb), sb = (int)(t % nb);
    const uint4 *src = (const uint4 *)(raw + (size_t)r * nb * 144 + (size_t)sb * 144);
    uint8_t *row = out + (size_t)r * nb * 144;
    uint4 *H = (uint4 *)row, *QA = (uint4 *)(row + 16 * nb), *QB = QA + 4 * nb;
    H[sb] = src[0];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        QA[4 * sb + p] = src[1 + 2 * p];
        QB[4 * sb + p] = src[2 + 2 * p];
    }
}

// raw rows of nbs blocks -> packed rows of nb blocks (nb = nbs, or nbs + 1:
// the appended block is all zeros)
__global__ void repack_q80(const uint8_t *__restrict__ raw, uint8_t *__restrict__ out, int rows, int nbs, int nb,
                           int stride)
{
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)rows * nb) return;
    int r = (int)(t / nb), b = (int)(t % nb);
    uint32_t v[9] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if (b < nbs) {
        const uint32_t *src = (const uint32_t *)(raw + (size_t)r * nbs * 36 + (size_t)b * 36); // 4-byte aligned
#pragma unroll
        for (int i = 0; i < 9; i++) v[i] = src[i];
    }
    uint8_t *row = out + (size_t)r * stride;
    int sreg = (4 * nb + 15) & ~15, U = nb / 2;
    ((uint32_t *)row)[b] = v[0];
    int u = b >> 1, half = b & 1;
    uint32_t *pl0 = (uint32_t *)(row + sreg + (size_t)(2 * half) * 16 * U + 16 * u);
    uint32_t *pl1 = (uint32_t *)(row + sreg + (size_t)(2 * half + 1) * 16 * U + 16 * u);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        pl0[i] = v[1 + i];
        pl1[i] = v[5 + i];
    }
}

__global__ void repack_q6k(const uint8_t *__restrict__ raw, uint8_t *__restrict__ out, int rows, int nb,
                           int stride)
{
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)rows * nb) return;
    int r = (int)(t / nb), sb = (int)(t % nb);
    const uint8_t *blk = raw + (size_t)r * nb * 210 + (size_t)sb * 210;
    uint8_t *row = out + (size_t)r * stride;
    int U = 4 * nb;
    uint8_t *SC = row, *QH = row + 16 * nb, *QLa = QH + 16 * U, *QLb = QLa + 16 * U, *D = QLb + 16 * U;
    for (int i = 0; i < 16; i++) SC[16 * sb + i] = blk[192 + i];
    for (int h = 0; h < 2; h++)
        for (int kk = 0; kk < 2; kk++) {
            int u = 4 * sb + 2 * h + kk;
            for (int i = 0; i < 16; i++) {
                QH[16 * u + i] = blk[128 + h * 32 + kk * 16 + i];
                QLa[16 * u + i] = blk[h * 64 + kk * 16 + i];
                QLb[16 * u + i] = blk[h * 64 + 32 + kk * 16 + i];
            }
        }
    D[2 * sb] = blk[208];
    D[2 * sb + 1] = blk[209];
}

int repack_weight(soso_hip *h, uint8_t dtype, const void *raw, void *packed, size_t rows, size_t cols)
{
    const int T = 256;
    size_t nb;
    switch (dtype) {
    case SOSO_HIP_DTYPE_F32:
        return hip_check(h, hipMemcpyAsync(packed, raw, rows * cols * 4, hipMemcpyDeviceToDevice, h->stream),
                         "copy f32 weight");
    case SOSO_HIP_DTYPE_Q4_K:
        nb = cols / 256;
        repack_q4k<<<(unsigned)((rows * nb + T - 1) / T), T, 0, h->stream>>>((const uint8_t *)raw, (uint8_t *)packed,
                                                                              (int)rows, (int)nb);
        break;
    case SOSO_HIP_DTYPE_Q8_0: {
        const size_t kc = kernel_cols(dtype, cols);
        nb = kc / 32;
        repack_q80<<<(unsigned)((rows * nb + T - 1) / T), T, 0, h->stream>>>(
            (const uint8_t *)raw, (uint8_t *)packed, (int)rows, (int)(cols / 32), (int)nb,
            (int)packed_row_stride(dtype, kc));
        break;
    }
    case SOSO_HIP_DTYPE_Q6_K:
        nb = cols / 256;
        repack_q6k<<<(unsigned)((rows * nb + T - 1) / T), T, 0, h->stream>>>(
            (const uint8_t *)raw, (uint8_t *)packed, (int)rows, (int)nb, (int)packed_row_stride(dtype, cols));
        break;
    default: return set_err(h, SOSO_HIP_ERR_ARG, "repack: dtype");
    }
    return hip_check(h, hipGetLastError(), "repack launch");
}

#include "mv_core.hpp"

// ---------------------------------------------------------------------------
// The matvec kernel.  A "group" of S wavefronts shares a contiguous strip of
// row passes; wavefront s of the group owns units [64s, 64s+64) of every row
// (S = ceil(U/64), U = cols/64 units per row; for U <= 64, S = 1 and a pass
// covers 64/LPR rows, LPR = lanes per row).  Each lane keeps its x unit in
// VGPRs for the whole launch.  x is staged first, then the loads of the
// first DEPTH passes are issued and the ring rolls DEPTH passes ahead of the
// math.  Row sums are gathered into one
// VGPR (lane i = i-th row of the strip, at most 64 rows) and stored once.
// With S > 1 the per-wavefront sums meet in LDS and are added in wavefront
// order.
// ---------------------------------------------------------------------------
constexpr int COMBINE_CH = 64; // passes per LDS combine round (S > 1)

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// Output of the row sums gathered in yacc (lane i = row r0 + i, i < nrows).
// Lane `lane` holds row r (valid when ok); pair epilogues find the other row
// of a pair (2i, 2i + 1) in the neighbouring lane.
template <int EPI>
__device__ __forceinline__ void epilogue(float yacc, int lane, int r, bool ok, float *__restrict__ y, const MvEpi &ep)
{
    if constexpr (EPI == EPI_STORE) {
        if (ok) y[r] = yacc;
    } else if constexpr (EPI == EPI_RESID) {
        if (ok) y[r] = ep.res[r] + yacc;
    } else {
        static_assert(EPI == EPI_SWIGLU, "epilogue variant");
        // rows (2i, 2i+1) = (gate_i, up_i); strips start on even rows
        const float up = dpp_f<0xB1>(yacc);
        if (ok && (lane & 1) == 0) y[r >> 1] = silu_f(yacc) * up;
    }
}

// EPI_PARTS (column segments): workgroup b takes segment b % MV_SEG of every
// row (cols / MV_SEG columns, whose x alone it stages) and the row units of
// group b / MV_SEG as the plain kernel; the segment's sums go to row block
// b % MV_SEG of y, segment 0's plus the residual ep.res when given.  A row's
// segments are thus summed by the consumer, so no workgroup converts all of x
// nor meets the others in LDS.
template <int FMT, int LPR, int S, int DEPTH, bool XFIRST, int XS = XS_PLAIN, int EPI = EPI_STORE, bool IL = false>
__global__ void __launch_bounds__(512) mv_rows(const uint8_t *__restrict__ W, size_t stride, MvIn in,
                                               float *__restrict__ y, int rows, int cols, MvEpi ep)
{
    static_assert(S == 1 || !IL, "split rows walk contiguous strips");
    static_assert(EPI != EPI_PARTS || (S == 1 && LPR == 64 && XS == XS_PLAIN), "column segments: whole wavefronts");
    constexpr int SEG = EPI == EPI_PARTS ? MV_SEG : 1;
    static_assert(S == 1 || LPR == 64, "split rows use whole wavefronts");
    static_assert(S == 1 || COMBINE_CH % DEPTH == 0, "combine rounds keep the load ring aligned");
    static_assert(S == 1 || EPI == EPI_STORE || EPI == EPI_RESID, "pair epilogues need whole rows per wavefront");
    extern __shared__ uint4 smem[];
    const int seg = SEG > 1 ? (int)blockIdx.x % SEG : 0;
    const int bx = SEG > 1 ? (int)blockIdx.x / SEG : (int)blockIdx.x, nbx = (int)gridDim.x / SEG;
    const int xcols = cols / SEG; // columns of x this workgroup stages
    const float *__restrict__ x = in.x + (size_t)seg * xcols;
    uint32_t *xp = (uint32_t *)smem;                 // xcols/4 groups x XDIG digit dwords
    float *s16 = (float *)(xp + (xcols >> 2) * XDIG);
    int *kx = (int *)(s16 + (xcols >> 4));
    // after the outlier lists: [groups][COMBINE_CH][S] when S > 1; 16 floats for XS_RMSNORM
    float *red = (float *)(out_lists(kx, xcols) + ((xcols + 127) >> 7) * OUT_DW);

    constexpr int RW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    constexpr int gpw = 8 / S;          // groups of S wavefronts per workgroup
    constexpr int NTHR = 64 * S * gpw;  // the launch's thread count (launch_fmt, launch_ex_*)
    // x chunks per thread loaded ahead (rounds of NTHR chunks; rows of up to
    // 64 S units have at most 512 S chunks, so S = 1 needs one round).  The
    // rounds past the row end cost a skipped branch each, yet on MI355X the
    // 14336 x 4096 Q4_K matvec took 7.93 / 7.51 / 7.32 / 7.34 us with one to
    // four rounds built, and the 8B decode step 1.705 / - / 1.688 / 1.728 ms.
    constexpr int XP = S == 1 ? 3 : 4;
    const int grp = wave / S, sw = wave % S;
    const int U = xcols >> 6; // units of the staged x
    const int ul = lane & (LPR - 1), slot = lane / LPR;
    const int ug = sw * 64 + ul;
    const bool uact = ug < U;
    const int u = uact ? ug : 0;  // the lane's unit of the staged x
    const int uw = seg * U + u;   // ... and of the weight rows
    UConst c;
    unit_setup_w<FMT>(uw, c);
    const LaneOff L = lane_offsets<FMT>(cols, uw, c);

    const int passes = (rows + RW - 1) / RW;
    const int tg = nbx * gpw;
    // pair epilogues need whole pairs of rows (2i, 2i + 1) in neighbouring lanes
    constexpr int PU = (RW == 1 && EPI == EPI_SWIGLU) ? 2 : 1;
    static_assert(DEPTH % PU == 0, "a ring turn holds whole units");
    const int units = (passes + PU - 1) / PU;
    auto strip = [&](int g, int &q0, int &q1) {
        q0 = PU * (int)((long)units * g / tg);
        q1 = min(passes, PU * (int)((long)units * (g + 1) / tg));
    };
    const int g = bx * gpw + grp;
    // Rows reach the group in units of PU passes.  IL: group g takes units g,
    // g + tg, g + 2 tg, ..., so at every step of the ring the groups of the
    // whole grid read one contiguous stretch of the matrix (on MI355X the
    // 14336 x 4096 Q4_K matvec: 7.3 us against 7.7 us for contiguous strips,
    // whose concurrent reads sit a strip apart).  Otherwise group g takes the
    // contiguous strip of units [units g / tg, units (g + 1) / tg).
    int p0, n;
    if constexpr (IL) {
        p0 = PU * g;
        n = g < units ? PU * ((units - g + tg - 1) / tg) : 0; // the last unit may run past `passes`: zeros
    } else {
        int p1;
        strip(g, p0, p1);
        n = p1 - p0;
    }
    const int r0 = p0 * RW, rend = IL ? rows : min((p0 + n) * RW, rows);
    // From the group's first pass to the end of its rows is the buffer; the
    // host keeps it (plus DEPTH passes) under 2^31 bytes.
    const uint32_t pass_bytes = (uint32_t)(RW * stride);
    const rsrc_t rs = make_rsrc(W + (size_t)r0 * stride, (uint32_t)((size_t)(rend > r0 ? rend - r0 : 0) * stride));
    // byte offset of the group's pass k from its first pass
    auto pass_off = [&](int k) -> uint32_t {
        if constexpr (IL) return (uint32_t)((k / PU) * PU * tg + k % PU) * pass_bytes;
        else return (uint32_t)k * pass_bytes;
    };
    // row of the sum in lane i, once gathered (lane i holds pass i / RW)
    auto lane_row = [&](int i) -> int {
        const int k = i / RW;
        return RW * (IL ? PU * (g + (k / PU) * tg) + k % PU : p0 + k) + i % RW;
    };
    // inactive lanes (unit past the row end) read nothing
    const uint32_t lane_base = uact ? (uint32_t)(slot * stride) : 0x80000000u;

    WRow<FMT> buf[DEPTH];
    float resv = 0.0f; // EPI_PARTS: the residual added to segment 0's sums
    if constexpr (XS == XS_RMSNORM) {
        // one round: normalised rows are at most 8 * NTHR columns wide
        XPreN<1> xpre;
        stage_xn_issue<1>(x, in.norm_w, cols, xpre, NTHR);
#pragma unroll
        for (int i = 0; i < DEPTH; i++) load_row<FMT>(rs, lane_base + pass_off(i), cols, L, buf[i]);
        stage_xn_finish<FMT, true, 1>(xpre, cols, in.eps, xp, s16, kx, red, NTHR);
    } else if constexpr (XS == XS_RMSNORM_P4) {
        XPreNP xpre;
        stage_xnp_issue(in, cols, xpre, NTHR);
#pragma unroll
        for (int i = 0; i < DEPTH; i++) load_row<FMT>(rs, lane_base + pass_off(i), cols, L, buf[i]);
        stage_xnp_finish<FMT, true>(xpre, in, cols, xp, s16, kx, red, NTHR);
    } else if constexpr (XFIRST) {
        // x first: once the weight stream is requested, x's reads would queue
        // behind it in the shared L2 channels.
        stage_x<FMT, true, XP>(x, xcols, xp, s16, kx, NTHR);
#pragma unroll
        for (int i = 0; i < DEPTH; i++) load_row<FMT>(rs, lane_base + pass_off(i), cols, L, buf[i]);
    } else {
        // x's loads, then the ring's, then x's conversion while the ring is
        // in flight (loads return in issue order)
        constexpr int XPP = SEG > 1 ? 1 : XP; // a segment is at most 64 units: one round
        XPre<XPP> xpre;
        stage_x_issue<XPP>(x, xcols, xpre, NTHR);
        if constexpr (SEG > 1) {
            // segment 0 carries the residual of its rows (ep.res), loaded
            // behind x and ahead of the ring.  Measured on MI355X (8B decode
            // step): 1.522 ms per token, 1.529 with the load at the end.  The
            // EPI_RESID epilogue keeps its load at the end: loaded here or
            // behind the ring the step took 1.548 / 1.557 ms.
            const int rr = lane_row(lane);
            if (seg == 0 && ep.res && lane < n * RW && rr < rows) resv = ep.res[rr];
        }
#pragma unroll
        for (int i = 0; i < DEPTH; i++) load_row<FMT>(rs, lane_base + pass_off(i), cols, L, buf[i]);
        stage_x_finish<FMT, true, XPP>(xpre, x, xcols, xp, s16, kx, NTHR);
    }
    XReg xv;
    unit_setup_x<FMT, true>(xp, s16, kx, u, U, xv, c);
    auto dot = [&](const WRow<FMT> &w) -> float { return unit_dot<FMT>(w, xv, c); };

    if constexpr (S == 1) {
        // The host sizes the grid so that a strip holds at most 64 rows: the
        // loop then stores nothing and the strip's rows leave in one store at
        // the end.  The main loop is a counted loop of whole ring turns with
        // no branches inside (refills past the strip read zeros for free) and
        // its steps fenced from the scheduler, so the compiler waits on exact
        // vmcnt values; the last n % DEPTH passes are already in the ring.
        float yacc = 0.0f;
        const int turns = n / DEPTH;
        int j0 = 0;
        for (int it = 0; it < turns; it++, j0 += DEPTH) {
#pragma unroll
            for (int i = 0; i < DEPTH; i++) {
                const int j = j0 + i;
                float part = dot(buf[i]);
                load_row<FMT>(rs, lane_base + pass_off(j + DEPTH), cols, L, buf[i]);
                part = seg_sum_dpp<LPR>(uact ? part : 0.0f);
                yacc = gather_rows<LPR>(part, j, yacc, lane);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        const int rem = n - j0;
#pragma unroll
        for (int i = 0; i < DEPTH - 1; i++) {
            if (i < rem) {
                float part = dot(buf[i]);
                part = seg_sum_dpp<LPR>(uact ? part : 0.0f);
                yacc = gather_rows<LPR>(part, j0 + i, yacc, lane);
            }
        }
        if (__builtin_expect(c.onum != 0, 0))
            yacc += outlier_rows<FMT, LPR>(rs, lane_base, pass_off, 0, n, cols, L, c, uw, uact, lane);
        const int r = lane_row(lane);
        if constexpr (SEG > 1) yacc = resv + yacc;
        epilogue<(SEG > 1 ? EPI_STORE : EPI)>(yacc, lane, r, lane < n * RW && r < rows, y + (size_t)seg * rows, ep);
    } else {
        // the same number of combine rounds for every wavefront of the workgroup
        int nmax = 0;
        for (int q = 0; q < gpw; q++) {
            int a0, a1;
            strip(blockIdx.x * gpw + q, a0, a1);
            nmax = a1 - a0 > nmax ? a1 - a0 : nmax;
        }
        for (int c0 = 0; c0 < nmax; c0 += COMBINE_CH) {
            // passes c0 .. e1-1 of this group; only a group's last round can
            // end off a ring turn (COMBINE_CH is a multiple of DEPTH)
            const int e1 = c0 + COMBINE_CH < n ? c0 + COMBINE_CH : n;
            const int turns = e1 > c0 ? (e1 - c0) / DEPTH : 0;
            int j0 = c0;
            for (int it = 0; it < turns; it++, j0 += DEPTH) {
#pragma unroll
                for (int i = 0; i < DEPTH; i++) {
                    const int j = j0 + i;
                    float part = dot(buf[i]);
                    load_row<FMT>(rs, lane_base + pass_off(j + DEPTH), cols, L, buf[i]);
                    part = seg_sum_dpp<64>(uact ? part : 0.0f);
                    if (lane == 63) red[(grp * COMBINE_CH + (j - c0)) * S + sw] = part;
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            const int rem = e1 > j0 ? e1 - j0 : 0;
#pragma unroll
            for (int i = 0; i < DEPTH - 1; i++) {
                if (i < rem) {
                    float part = dot(buf[i]);
                    part = seg_sum_dpp<64>(uact ? part : 0.0f);
                    if (lane == 63) red[(grp * COMBINE_CH + (j0 + i - c0)) * S + sw] = part;
                }
            }
            if (__builtin_expect(c.onum != 0, 0)) {
                // the outliers' share of this round's passes, added to the
                // wavefront's own partial sums
                const float corr = outlier_rows<FMT, 64>(rs, lane_base, pass_off, c0, e1 > c0 ? e1 : c0, cols, L, c,
                                                         u, uact, lane);
                for (int i = 0; i < e1 - c0; i++) {
                    const float ci =
                        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), i));
                    if (lane == 63) red[(grp * COMBINE_CH + i) * S + sw] += ci;
                }
            }
            __syncthreads();
            for (int e = threadIdx.x; e < gpw * COMBINE_CH; e += NTHR) {
                const int q = e / COMBINE_CH, i = e % COMBINE_CH;
                int a0, a1;
                strip(blockIdx.x * gpw + q, a0, a1);
                const int pp = a0 + c0 + i;
                if (pp < a1) {
                    float acc = 0.0f;
#pragma unroll
                    for (int k = 0; k < S; k++) acc += red[(q * COMBINE_CH + i) * S + k];
                    y[pp] = EPI == EPI_RESID ? ep.res[pp] + acc : acc;
                }
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// Several tokens per launch: GpuDispatch::matmul (gpu.rs:443-455) with n > 1
// vectors, as soso's batched q4_k_nb / q8_0_nb kernels do on the CPU
// (crates/soso-llm-core/src/gemm.rs:902-1076): every weight row is read once
// for a group of tokens.  Rows of up to 64 units (4096 columns).
//
// A workgroup's 8 wavefronts form 8 / G "row groups" of G wavefronts; the G
// wavefronts of a row group walk the same rows (interleaved over the grid as
// in mv_rows), each for NT tokens of its own (tokens NT*q .. NT*q + NT - 1 for
// wavefront q of the group).  Each loaded unit meets the NT tokens' digit
// registers, and the G wavefronts of a row group request a row at about the
// same time, so it leaves HBM once and the other requests hit the cache.
// Every token of the launch is staged in LDS (one staging region each).  Per
// token the integer sums, the f32 steps and the lane reduction are exactly
// mv_rows', so each output is bit-identical to the token's own matvec.
// ---------------------------------------------------------------------------
constexpr int TOK_THREADS = 512; // mv_tok's launch size
template <int FMT, int LPR, int NT, int DEPTH>
__global__ void __launch_bounds__(512) mv_tok(const uint8_t *__restrict__ W, size_t stride, const float *__restrict__ x,
                                              float *__restrict__ y, int rows, int cols, int ntok, int G)
{
    constexpr int RW = 64 / LPR;
    extern __shared__ uint4 smem[];
    const size_t sl = (stage_lds_bytes_o((size_t)cols) + 15) & ~(size_t)15; // bytes of one token's staging
    auto region = [&](int t, uint32_t *&xp, float *&s16, int *&kx) {
        xp = (uint32_t *)((char *)smem + (size_t)t * sl);
        s16 = (float *)(xp + (cols >> 2) * XDIG);
        kx = (int *)(s16 + (cols >> 4));
    };
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int rgw = (TOK_THREADS >> 6) / G; // row groups per workgroup
    const int tq = wave % G, rgi = wave / G;
    const int t0 = tq * NT; // this wavefront's first token
    const int U = cols >> 6;
    const int ul = lane & (LPR - 1), slot = lane / LPR;
    const bool uact = ul < U;
    const int u = uact ? ul : 0;
    UConst c;
    unit_setup_w<FMT>(u, c);
    const LaneOff L = lane_offsets<FMT>(cols, u, c);
    const int passes = (rows + RW - 1) / RW;
    const int tg = gridDim.x * rgw;
    const int g = blockIdx.x * rgw + rgi;
    const int n = g < passes ? (passes - g + tg - 1) / tg : 0;
    const int r0 = g * RW;
    const uint32_t pass_bytes = (uint32_t)(RW * stride);
    const rsrc_t rs = make_rsrc(W + (size_t)r0 * stride, (uint32_t)((size_t)(rows > r0 ? rows - r0 : 0) * stride));
    auto pass_off = [&](int k) -> uint32_t { return (uint32_t)(k * tg) * pass_bytes; };
    const uint32_t lane_base = uact ? (uint32_t)(slot * stride) : 0x80000000u;

    WRow<FMT> buf[DEPTH];
#pragma unroll
    for (int i = 0; i < DEPTH; i++) load_row<FMT>(rs, lane_base + pass_off(i), cols, L, buf[i]);
    for (int t = 0; t < ntok; t++) {
        uint32_t *xp;
        float *s16;
        int *kx;
        region(t, xp, s16, kx);
        stage_x<FMT, true, 1>(x + (size_t)t * cols, cols, xp, s16, kx, TOK_THREADS); // cols <= 4096
    }
    XReg xv[NT];
    UConst ct[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        ct[t] = c;
        uint32_t *xp;
        float *s16;
        int *kx;
        region(t0 + t < ntok ? t0 + t : 0, xp, s16, kx);
        unit_setup_x<FMT, true>(xp, s16, kx, u, U, xv[t], ct[t]);
    }
    const int nt = max(0, min(NT, ntok - t0)); // tokens this wavefront computes (uniform)
    float yacc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) yacc[t] = 0.0f;
    auto row = [&](int i, int j) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t < nt) {
                const float part = seg_sum_dpp<LPR>(uact ? unit_dot<FMT>(buf[i], xv[t], ct[t]) : 0.0f);
                yacc[t] = gather_rows<LPR>(part, j, yacc[t], lane);
            }
        }
    };
    const int turns = n / DEPTH;
    int j0 = 0;
    for (int it = 0; it < turns; it++, j0 += DEPTH) {
#pragma unroll
        for (int i = 0; i < DEPTH; i++) {
            row(i, j0 + i);
            load_row<FMT>(rs, lane_base + pass_off(j0 + i + DEPTH), cols, L, buf[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const int rem = n - j0;
#pragma unroll
    for (int i = 0; i < DEPTH - 1; i++)
        if (i < rem) row(i, j0 + i);
#pragma unroll
    for (int t = 0; t < NT; t++)
        if (__builtin_expect(t < nt && ct[t].onum != 0, 0))
            yacc[t] += outlier_rows<FMT, LPR>(rs, lane_base, pass_off, 0, n, cols, L, ct[t], u, uact, lane);
    const int k = lane / RW;
    const int r = RW * (g + k * tg) + lane % RW;
    if (lane < n * RW && r < rows) {
#pragma unroll
        for (int t = 0; t < NT; t++)
            if (t < nt) y[(size_t)(t0 + t) * rows + r] = yacc[t];
    }
}

// ---------------------------------------------------------------------------
// F32 matvec (MoE router and other small f32 tensors): one wavefront per row,
// float4 loads, butterfly reduction.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) mv_f32(const float *__restrict__ W, const float *__restrict__ x,
                                              float *__restrict__ y, int rows, int cols)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (r >= rows) return; // wave-uniform
    const float4 *w4 = (const float4 *)(W + (size_t)r * cols);
    const float4 *x4 = (const float4 *)x;
    float a0 = 0.f, a1 = 0.f;
    for (int i = lane; i < (cols >> 2); i += 64) {
        float4 w = w4[i], v = x4[i];
        a0 = fmaf(w.x, v.x, a0);
        a1 = fmaf(w.y, v.y, a1);
        a0 = fmaf(w.z, v.z, a0);
        a1 = fmaf(w.w, v.w, a1);
    }
    float s = seg_sum<64>(a0 + a1);
    if (lane == 0) y[r] = s;
}

// ---------------------------------------------------------------------------
// Launch selection
// ---------------------------------------------------------------------------
// A group's strip (plus the DEPTH passes the ring reads past it, which come
// back as zeros) is addressed with 32-bit buffer offsets.
static bool strip_fits(int passes, int groups, size_t pass_bytes)
{
    const size_t per = ((size_t)passes + groups - 1) / groups + 16;
    return per * pass_bytes < ((size_t)1 << 31);
}

// The interleaved mapping addresses every pass of a group from its first one:
// the last ring offset (a whole grid of passes per unit step) must stay below
// 2^31 bytes.
static bool interleave_fits(int passes, int pu, int groups, size_t pass_bytes)
{
    const size_t units = ((size_t)passes + pu - 1) / pu;
    const size_t steps = (units + groups - 1) / groups + 16;
    return steps * (size_t)pu * groups * pass_bytes < ((size_t)1 << 31);
}

// Ring depth (passes in flight per wavefront) and issue order, measured on
// MI355X (back-to-back launches over rotating weights above the MALL size):
//   Q4_K 14336 x 4096: depth 2, ring loads before x's conversion (7.7 us;
//     depth 8 x-first 11.0 us -- with all of a wavefront's rows in flight at
//     once every wavefront's first row arrives late and the math cannot
//     overlap the stream);  Q8_0 4096 x 4096: depth 2 (5.6 us; 5.9 at depth 3,
//     6.3 at 4: a wavefront has two rows, so deeper rings only read past them);
//   Q6_K 128256 x 4096: depth 4 (79 us; 3 and 6 the same);  split rows 4096 x 14336: depth 4
//     (10.53 us against 10.80 at depth 2 and 12.8 at 8; the 8B step 1.644 against 1.667 ms);
//   narrow rows (LPR < 64, e.g. 768 x 2048): depth 2 with x staged first.
// Split rows (S > 1) need a depth that divides the combine round.
template <int FMT, int S> constexpr int ring_depth()
{
    return S > 1 || FMT == FMT_Q6K ? 4 : 2;
}
template <int LPR> constexpr bool x_first() { return LPR < 64; }

template <int FMT, int S>
static void launch_split(soso_hip *h, int grid, int threads, size_t lds, const uint8_t *W, size_t stride,
                         const float *x, float *y, int rows, int cols)
{
    MvIn in;
    in.x = x;
    mv_rows<FMT, 64, S, ring_depth<FMT, S>(), false><<<grid, threads, lds, h->stream>>>(W, stride, in, y, rows, cols,
                                                                                          MvEpi());
}

template <int FMT>
static int launch_fmt(soso_hip *h, const Weight &w, const float *x, float *y)
{
    const size_t kc = weight_kcols(w);
    const int rows = (int)w.rows, cols = (int)kc, U = cols / 64;
    const size_t stride = packed_row_stride(w.dtype, kc);
    const int S = (U + 63) / 64;
    if (S > 8) return set_err(h, SOSO_HIP_DECLINED, "matvec: rows wider than 512 units");
    const int gpw = 8 / S;                 // groups of S wavefronts per workgroup (<= 512 threads)
    const int threads = 64 * S * gpw;
    const size_t lds = stage_lds_bytes_o(kc) + (S > 1 ? (size_t)gpw * COMBINE_CH * S * 4 : 0);
    if (lds > h->max_lds) return set_err(h, SOSO_HIP_DECLINED, "matvec: x does not fit in LDS");
    const int per_cu = 1; // one 512-thread workgroup per CU (two measured slower for these shapes)
    const uint8_t *W = (const uint8_t *)w.dev;
    MvIn xin;
    xin.x = x;
    if (S == 1) {
        const int LPR = U <= 1 ? 1 : U <= 2 ? 2 : U <= 4 ? 4 : U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
        const int passes = (rows + 64 / LPR - 1) / (64 / LPR);
        int grid = std::min(h->num_cu * per_cu, (passes + gpw - 1) / gpw);
        // every group's strip holds at most 64 rows (the kernel's output register)
        const int ppw = LPR; // passes per 64 rows = 64 / (64 / LPR)
        grid = std::max(grid, ((passes + ppw - 1) / ppw + gpw - 1) / gpw);
        grid = std::max(grid, 1);
        if (!strip_fits(passes, grid * gpw, (size_t)(64 / LPR) * stride))
            return set_err(h, SOSO_HIP_DECLINED, "matvec: row strip exceeds 2 GiB");
        const bool il = interleave_fits(passes, 1, grid * gpw, (size_t)(64 / LPR) * stride);
#define MV_CASE(L)                                                                                                  \
    case L:                                                                                                         \
        if (il)                                                                                                     \
            mv_rows<FMT, L, 1, ring_depth<FMT, 1>(), x_first<L>(), XS_PLAIN, EPI_STORE, true>                        \
                <<<grid, threads, lds, h->stream>>>(W, stride, xin, y, rows, cols, MvEpi());                        \
        else                                                                                                        \
            mv_rows<FMT, L, 1, ring_depth<FMT, 1>(), x_first<L>()><<<grid, threads, lds, h->stream>>>(               \
                W, stride, xin, y, rows, cols, MvEpi());                                                            \
        break;
        switch (LPR) {
            MV_CASE(1) MV_CASE(2) MV_CASE(4) MV_CASE(8) MV_CASE(16) MV_CASE(32) MV_CASE(64)
        }
#undef MV_CASE
    } else {
        int grid = std::min(h->num_cu * per_cu, (rows + gpw - 1) / gpw);
        grid = std::max(grid, 1);
        if (!strip_fits(rows, grid * gpw, stride)) return set_err(h, SOSO_HIP_DECLINED, "matvec: row strip exceeds 2 GiB");
        switch (S) {
        case 2: launch_split<FMT, 2>(h, grid, threads, lds, W, stride, x, y, rows, cols); break;
        case 3: launch_split<FMT, 3>(h, grid, threads, lds, W, stride, x, y, rows, cols); break;
        case 4: launch_split<FMT, 4>(h, grid, threads, lds, W, stride, x, y, rows, cols); break;
        case 5: launch_split<FMT, 5>(h, grid, threads, lds, W, stride, x, y, rows, cols); break;
        case 6: launch_split<FMT, 6>(h, grid, threads, lds, W, stride, x, y, rows, cols); break;
        case 7: launch_split<FMT, 7>(h, grid, threads, lds, W, stride, x, y, rows, cols); break;
        case 8: launch_split<FMT, 8>(h, grid, threads, lds, W, stride, x, y, rows, cols); break;
        }
    }
    return hip_check(h, hipGetLastError(), "matvec launch");
}

// ---------------------------------------------------------------------------
// Matvec with an input / output variant (the decode step's fusions)
// ---------------------------------------------------------------------------
template <int FMT, int LPR, int XS, int EPI>
static void launch_ex1(soso_hip *h, bool il, unsigned grid, size_t lds, const uint8_t *W, size_t stride, const MvIn &in,
                       float *y, int rows, int cols, const MvEpi &ep)
{
    if (il)
        mv_rows<FMT, LPR, 1, ring_depth<FMT, 1>(), x_first<LPR>(), XS, EPI, true><<<grid, 512, lds, h->stream>>>(
            W, stride, in, y, rows, cols, ep);
    else if constexpr (EPI == EPI_STORE) // the head: contiguous strips past 2^31 bytes of interleaved offsets
        mv_rows<FMT, LPR, 1, ring_depth<FMT, 1>(), x_first<LPR>(), XS, EPI><<<grid, 512, lds, h->stream>>>(
            W, stride, in, y, rows, cols, ep);
}

template <int FMT, int XS, int EPI>
static void launch_ex_lpr(soso_hip *h, int lpr, bool il, unsigned grid, size_t lds, const uint8_t *W, size_t stride,
                          const MvIn &in, float *y, int rows, int cols, const MvEpi &ep)
{
    if constexpr (XS == XS_RMSNORM_P4 || EPI == EPI_PARTS) { // built for whole-wavefront rows only
        launch_ex1<FMT, 64, XS, EPI>(h, il, grid, lds, W, stride, in, y, rows, cols, ep);
    } else {
        switch (lpr) {
        case 8: launch_ex1<FMT, 8, XS, EPI>(h, il, grid, lds, W, stride, in, y, rows, cols, ep); break;
        case 16: launch_ex1<FMT, 16, XS, EPI>(h, il, grid, lds, W, stride, in, y, rows, cols, ep); break;
        case 32: launch_ex1<FMT, 32, XS, EPI>(h, il, grid, lds, W, stride, in, y, rows, cols, ep); break;
        default: launch_ex1<FMT, 64, XS, EPI>(h, il, grid, lds, W, stride, in, y, rows, cols, ep); break;
        }
    }
}

template <int FMT>
static void launch_ex_fmt(soso_hip *h, int xs, int epi, int lpr, bool il, unsigned grid, size_t lds, const uint8_t *W,
                          size_t stride, const MvIn &in, float *y, int rows, int cols, const MvEpi &ep)
{
    if (xs == XS_RMSNORM && epi == EPI_SWIGLU)
        launch_ex_lpr<FMT, XS_RMSNORM, EPI_SWIGLU>(h, lpr, il, grid, lds, W, stride, in, y, rows, cols, ep);
    else if (xs == XS_PLAIN && epi == EPI_RESID)
        launch_ex_lpr<FMT, XS_PLAIN, EPI_RESID>(h, lpr, il, grid, lds, W, stride, in, y, rows, cols, ep);
    else if (xs == XS_PLAIN && epi == EPI_PARTS)
        launch_ex_lpr<FMT, XS_PLAIN, EPI_PARTS>(h, lpr, il, grid, lds, W, stride, in, y, rows, cols, ep);
    else if (xs == XS_RMSNORM_P4)
        launch_ex_lpr<FMT, XS_RMSNORM_P4, EPI_STORE>(h, lpr, il, grid, lds, W, stride, in, y, rows, cols, ep);
    else
        launch_ex_lpr<FMT, XS_RMSNORM, EPI_STORE>(h, lpr, il, grid, lds, W, stride, in, y, rows, cols, ep);
}

template <int FMT, int S>
static void launch_ex_split(soso_hip *h, unsigned grid, size_t lds, const uint8_t *W, size_t stride, const MvIn &in,
                            float *y, int rows, int cols, const MvEpi &ep)
{
    mv_rows<FMT, 64, S, ring_depth<FMT, S>(), false, XS_PLAIN, EPI_RESID><<<grid, 512, lds, h->stream>>>(
        W, stride, in, y, rows, cols, ep);
}

// The launch of one decode-step matvec (input variant xs, output variant
// epi), or the reason it cannot run here.  The variants built: every
// quantized format (Q4_K, Q8_0, Q6_K) with (RMSNORM, QKV), (RMSNORM, SWIGLU),
// (PLAIN, RESID) and (RMSNORM, STORE); rows of up to 64 units (4096 columns)
// per wavefront, and the residual variant also with rows split over 2 or 4
// wavefronts (up to 16384 columns).
struct ExPlan {
    int S = 1, lpr = 64, grid = 1;
    size_t lds = 0, stride = 0;
    bool il = false;
};

static const char *plan_matvec_ex(const soso_hip *h, uint8_t dtype, size_t rows_, size_t cols_, int xs, int epi,
                                  ExPlan &p)
{
    if (dtype != SOSO_HIP_DTYPE_Q4_K && dtype != SOSO_HIP_DTYPE_Q8_0 && dtype != SOSO_HIP_DTYPE_Q6_K)
        return "matvec_ex: the decode matvecs take Q4_K, Q8_0 or Q6_K weights";
    if (!packed_shape_ok(dtype, rows_, cols_) || rows_ > (1u << 30) || cols_ > (1u << 20))
        return "matvec_ex: shape not handled here";
    if (!(xs == XS_RMSNORM && (epi == EPI_SWIGLU || epi == EPI_STORE)) &&
        !(xs == XS_PLAIN && (epi == EPI_RESID || epi == EPI_PARTS)) && !(xs == XS_RMSNORM_P4 && epi == EPI_STORE))
        return "matvec_ex: input/output variant not built";
    const int rows = (int)rows_, cols = (int)cols_, U = cols / 64;
    p.stride = packed_row_stride(dtype, cols_);
    p.S = (U + 63) / 64;
    if ((xs == XS_RMSNORM || xs == XS_RMSNORM_P4) && cols > 8 * 512)
        return "matvec_ex: normalised x wider than the staging registers";
    if (xs == XS_RMSNORM_P4 && U <= 32) return "matvec_ex: summed partials built for rows of 33-64 units";
    if (epi == EPI_PARTS) {
        // MV_SEG column segments of 33-64 units each, whole 256-column groups
        // (Q6_K's x layout spans super-blocks; the others' exponents span 128)
        const int us = U / MV_SEG;
        if (U % (4 * MV_SEG) || us <= 32 || us > 64) return "matvec_ex: column segments not built for this width";
        const int gpw = 8, per = std::max(1, h->num_cu / MV_SEG);
        p.lpr = 64;
        p.lds = stage_lds_bytes_o(cols_ / MV_SEG) + 64;
        if (p.lds > h->max_lds) return "matvec_ex: x does not fit in LDS";
        int grid = std::min(per, (rows + gpw - 1) / gpw);
        grid = std::max(grid, ((rows + 63) / 64 + gpw - 1) / gpw); // at most 64 rows per group
        p.grid = MV_SEG * std::max(grid, 1);
        p.S = 1;
        if (!strip_fits(rows, grid * gpw, p.stride)) return "matvec_ex: row strip exceeds 2 GiB";
        p.il = interleave_fits(rows, 1, grid * gpw, p.stride);
        if (!p.il) return "matvec_ex: matrix too large for the interleaved rows of this variant";
        return nullptr;
    }
    if (epi == EPI_SWIGLU && (p.S != 1 || rows % 2))
        return "matvec_ex: pair epilogue needs whole rows per wavefront";
    if (p.S > 1) {
        if (xs != XS_PLAIN || epi != EPI_RESID || (p.S != 2 && p.S != 4))
            return "matvec_ex: variant not built for split rows";
        const int gpw = 8 / p.S;
        p.lds = stage_lds_bytes_o(cols_) + (size_t)gpw * COMBINE_CH * p.S * 4;
        if (p.lds > h->max_lds) return "matvec_ex: x does not fit in LDS";
        p.grid = std::max(1, std::min(h->num_cu, (rows + gpw - 1) / gpw));
        if (!strip_fits(rows, p.grid * gpw, p.stride)) return "matvec_ex: row strip exceeds 2 GiB";
        return nullptr;
    }
    if (U < 8) return "matvec_ex: rows narrower than 512 columns";
    p.lpr = U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
    const int RW = 64 / p.lpr, gpw = 8;
    const int PU = (RW == 1 && epi == EPI_SWIGLU) ? 2 : 1;
    const int passes = (rows + RW - 1) / RW, units = (passes + PU - 1) / PU;
    p.lds = stage_lds_bytes_o(cols_) + 64;
    if (p.lds > h->max_lds) return "matvec_ex: x does not fit in LDS";
    // two workgroups per CU for the gate/up pair (2 x 14336 x 4096 on MI355X:
    // 15.2 us, 15.9 us at one per CU; in the 8B step three or four per CU took
    // 5 / 8 % longer, and one workgroup of 1024 threads per CU 4 %); one for
    // the others (qkv, o and the head were slower at two)
    const int wg_per_cu = epi == EPI_SWIGLU ? 2 : 1;
    int grid = std::min(h->num_cu * wg_per_cu, (units + gpw - 1) / gpw);
    const int upw = 64 / (PU * RW); // units per 64-row strip
    grid = std::max(grid, ((units + upw - 1) / upw + gpw - 1) / gpw);
    p.grid = std::max(grid, 1);
    if (!strip_fits(passes, p.grid * gpw, (size_t)RW * p.stride)) return "matvec_ex: row strip exceeds 2 GiB";
    p.il = interleave_fits(passes, PU, p.grid * gpw, (size_t)RW * p.stride);
    if (!p.il && epi != EPI_STORE) return "matvec_ex: matrix too large for the interleaved rows of this variant";
    return nullptr;
}

const char *matvec_ex_unsupported(const soso_hip *h, uint8_t dtype, size_t rows, size_t cols, int xs, int epi)
{
    ExPlan p;
    return plan_matvec_ex(h, dtype, rows, cols, xs, epi, p);
}

int launch_matvec_ex(soso_hip *h, const Weight &w, const MvIn &in, float *y, const MvEpi &ep, int xs, int epi)
{
    if (weight_kcols(w) != w.cols) return set_err(h, SOSO_HIP_DECLINED, "matvec_ex: padded Q8_0 rows not built here");
    ExPlan p;
    if (const char *why = plan_matvec_ex(h, w.dtype, w.rows, w.cols, xs, epi, p)) return set_err(h, SOSO_HIP_DECLINED, why);
    const int rows = (int)w.rows, cols = (int)w.cols;
    const uint8_t *W = (const uint8_t *)w.dev;
    const unsigned g = (unsigned)p.grid;
    if (p.S > 1) {
#define EX_SPLIT(F)                                                                                                    \
    if (p.S == 2) launch_ex_split<F, 2>(h, g, p.lds, W, p.stride, in, y, rows, cols, ep);                              \
    else launch_ex_split<F, 4>(h, g, p.lds, W, p.stride, in, y, rows, cols, ep);
        switch (w.dtype) {
        case SOSO_HIP_DTYPE_Q4_K: EX_SPLIT(FMT_Q4K) break;
        case SOSO_HIP_DTYPE_Q8_0: EX_SPLIT(FMT_Q80) break;
        default: EX_SPLIT(FMT_Q6K) break;
        }
#undef EX_SPLIT
        return hip_check(h, hipGetLastError(), "matvec_ex launch");
    }
    switch (w.dtype) {
    case SOSO_HIP_DTYPE_Q4_K:
        launch_ex_fmt<FMT_Q4K>(h, xs, epi, p.lpr, p.il, g, p.lds, W, p.stride, in, y, rows, cols, ep);
        break;
    case SOSO_HIP_DTYPE_Q8_0:
        launch_ex_fmt<FMT_Q80>(h, xs, epi, p.lpr, p.il, g, p.lds, W, p.stride, in, y, rows, cols, ep);
        break;
    default: launch_ex_fmt<FMT_Q6K>(h, xs, epi, p.lpr, p.il, g, p.lds, W, p.stride, in, y, rows, cols, ep); break;
    }
    return hip_check(h, hipGetLastError(), "matvec_ex launch");
}

// n vectors: from MATMUL_MFMA_MIN tokens up, Q4_K and Q8_0 rows of whole
// 256-column super-blocks go to the matrix cores (k_mfma.hip: within the same
// 1e-5 of the exact product, not bit-identical to the single-vector kernel);
// fewer vectors, Q6_K at any count and other Q8_0 widths run mv_tok (each row
// read once per launch of up to 16 tokens, every output bit-identical to its
// own matvec); rows wider than 4096 columns run the single-vector kernel once
// per vector.
constexpr size_t MATMUL_MFMA_MIN = 16;

// Tokens per wavefront of mv_tok: each loaded unit meets two tokens' digits
// (two tokens' digit registers, 96 VGPRs, leave two wavefronts per SIMD).
constexpr int TOK_NT = 2;

template <int FMT>
static int launch_tok_fmt(soso_hip *h, const Weight &w, const float *x, float *y, size_t n)
{
    const size_t kc = weight_kcols(w);
    const int rows = (int)w.rows, cols = (int)kc, U = cols / 64;
    const size_t stride = packed_row_stride(w.dtype, kc);
    const int LPR = U <= 1 ? 1 : U <= 2 ? 2 : U <= 4 ? 4 : U <= 8 ? 8 : U <= 16 ? 16 : U <= 32 ? 32 : 64;
    const int RW = 64 / LPR, passes = (rows + RW - 1) / RW;
    const size_t sl = (stage_lds_bytes_o(kc) + 15) & ~(size_t)15;
    // tokens per launch: as many as LDS stages, at most 8 row-group wavefronts x TOK_NT
    const size_t per = std::min<size_t>(std::min<size_t>(h->max_lds / sl, 8 * TOK_NT), n);
    for (size_t t0 = 0; t0 < n; t0 += per) {
        const int m = (int)std::min(per, n - t0);
        int G = (m + TOK_NT - 1) / TOK_NT;
        G = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
        const int rgw = 8 / G;
        // every row group holds at most 64 rows (one output register); one
        // workgroup per CU at least
        int grid = std::max(h->num_cu, ((passes + LPR - 1) / LPR + rgw - 1) / rgw);
        grid = std::min(grid, std::max(1, (passes + rgw - 1) / rgw));
        grid = std::max(grid, ((passes + LPR - 1) / LPR + rgw - 1) / rgw);
        if (!interleave_fits(passes, 1, grid * rgw, (size_t)RW * stride))
            return set_err(h, SOSO_HIP_DECLINED, "matmul: matrix too large for the batched kernel");
        const size_t lds = sl * (size_t)m;
        const float *xt = x + t0 * kc;
        float *yt = y + t0 * w.rows;
#define TOK_CASE(LP)                                                                                                   \
    case LP:                                                                                                          \
        mv_tok<FMT, LP, TOK_NT, ring_depth<FMT, 1>()><<<grid, TOK_THREADS, lds, h->stream>>>(                        \
            (const uint8_t *)w.dev, stride, xt, yt, rows, cols, m, G);                                                \
        break;
        switch (LPR) {
            TOK_CASE(1) TOK_CASE(2) TOK_CASE(4) TOK_CASE(8) TOK_CASE(16) TOK_CASE(32) TOK_CASE(64)
        }
#undef TOK_CASE
        const int rc = hip_check(h, hipGetLastError(), "matmul launch");
        if (rc != SOSO_HIP_OK) return rc;
    }
    return SOSO_HIP_OK;
}

// x rows of `cols` floats -> rows of `kcols` with zeros after each (the
// columns of a weight's appended zero block)
__global__ void k_pad_rows(const float *__restrict__ x, float *__restrict__ out, int cols, int kcols, long total)
{
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
        const long t = i / kcols;
        const int c = (int)(i % kcols);
        out[i] = c < cols ? x[t * cols + c] : 0.0f;
    }
}

int launch_matvec(soso_hip *h, const Weight &w, const float *x, float *y, size_t n)
{
    const size_t kc = weight_kcols(w);
    if (kc != w.cols) {
        // a padded weight reads padded x (scratch slot 13; under graph capture
        // only once an earlier call has grown it)
        float *xp = (float *)scratch_get(h, 13, n * kc * 4);
        if (!xp) return set_err(h, SOSO_HIP_ERR_NOMEM, "matvec: padded x");
        const long total = (long)(n * kc);
        k_pad_rows<<<(unsigned)std::min<long>((total + 255) / 256, 4096), 256, 0, h->stream>>>(x, xp, (int)w.cols,
                                                                                              (int)kc, total);
        const int rc = hip_check(h, hipGetLastError(), "pad x launch");
        if (rc != SOSO_HIP_OK) return rc;
        x = xp;
    }
    if (n >= MATMUL_MFMA_MIN && mfma_shape_ok(w.dtype, w.rows, kc)) return launch_mfma_matmul(h, w, x, n, y);
    // several tokens, rows of at most 64 units: each row read once per launch
    if (n > 1 && kc <= 4096 && w.dtype != SOSO_HIP_DTYPE_F32 &&
        (stage_lds_bytes_o(kc) + 15) / 16 * 16 * 2 <= h->max_lds) {
        switch (w.dtype) {
        case SOSO_HIP_DTYPE_Q4_K: return launch_tok_fmt<FMT_Q4K>(h, w, x, y, n);
        case SOSO_HIP_DTYPE_Q8_0: return launch_tok_fmt<FMT_Q80>(h, w, x, y, n);
        case SOSO_HIP_DTYPE_Q6_K: return launch_tok_fmt<FMT_Q6K>(h, w, x, y, n);
        default: break;
        }
    }
    for (size_t t = 0; t < n; t++) {
        const float *xt = x + t * kc;
        float *yt = y + t * w.rows;
        int rc;
        switch (w.dtype) {
        case SOSO_HIP_DTYPE_Q4_K: rc = launch_fmt<FMT_Q4K>(h, w, xt, yt); break;
        case SOSO_HIP_DTYPE_Q8_0: rc = launch_fmt<FMT_Q80>(h, w, xt, yt); break;
        case SOSO_HIP_DTYPE_Q6_K: rc = launch_fmt<FMT_Q6K>(h, w, xt, yt); break;
        case SOSO_HIP_DTYPE_F32: {
            const int rows = (int)w.rows;
            mv_f32<<<(rows + 3) / 4, 256, 0, h->stream>>>((const float *)w.dev, xt, yt, rows, (int)w.cols);
            rc = hip_check(h, hipGetLastError(), "matvec f32 launch");
            break;
        }
        default: rc = set_err(h, SOSO_HIP_ERR_ARG, "matvec: dtype");
        }
        if (rc < 0 || rc == 0) return rc;
    }
    return SOSO_HIP_OK;
}

// ---------------------------------------------------------------------------
// Exact dequantization from the packed layout (bit-exactness witness).
// Arithmetic as crates/sosomodel/src/dequant.rs (Q8_0 :74-97, Q4_K :204-241)
// and crates/gguf2som/src/lib.rs:1639-1661 (Q6_K), never contracted to FMA.
// ---------------------------------------------------------------------------
__global__ void dq_q4k(const uint8_t *__restrict__ W, float *__restrict__ out, int rows, int cols)
{
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int U = cols >> 6, nb = cols >> 8;
    if (t >= (long)rows * U) return;
    const int r = (int)(t / U), u = (int)(t % U), sb = u >> 2, p = u & 3;
    const uint8_t *Wr = W + (size_t)r * nb * 144;
    const uint8_t *H = Wr + 16 * sb;
    const uint8_t *qa = Wr + 16 * nb + 16 * u, *qb = Wr + 16 * nb + 16 * U + 16 * u;
    const float d = f16_to_f32_ref(H[0] | (H[1] << 8)), dmin = f16_to_f32_ref(H[2] | (H[3] << 8));
    const uint8_t *s = H + 4;
    uint8_t sc[2], m[2];
    for (int k = 0; k < 2; k++) {
        int j = 2 * p + k;
        if (j < 4) {
            sc[k] = s[j] & 63;
            m[k] = s[j + 4] & 63;
        } else {
            sc[k] = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
            m[k] = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
        }
    }
    const float d1 = __fmul_rn(d, (float)sc[0]), min1 = __fmul_rn(dmin, (float)m[0]);
    const float d2 = __fmul_rn(d, (float)sc[1]), min2 = __fmul_rn(dmin, (float)m[1]);
    float *o = out + (size_t)r * cols + 64 * u;
    for (int l = 0; l < 32; l++) {
        const uint8_t q = l < 16 ? qa[l] : qb[l - 16];
        o[l] = __fsub_rn(__fmul_rn(d1, (float)(q & 0x0F)), min1);
        o[32 + l] = __fsub_rn(__fmul_rn(d2, (float)(q >> 4)), min2);
    }
}

// cols: the caller's columns (the output's row length); kcols: the packed
// layout's (cols, or cols + 32 with an appended zero block)
__global__ void dq_q80(const uint8_t *__restrict__ W, float *__restrict__ out, int rows, int cols, int kcols,
                       int stride)
{
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int nb = cols >> 5, U = kcols >> 6, sreg = (4 * (kcols >> 5) + 15) & ~15;
    if (t >= (long)rows * nb) return;
    const int r = (int)(t / nb), b = (int)(t % nb), u = b >> 1, half = b & 1;
    const uint8_t *Wr = W + (size_t)r * stride;
    const float scale = ((const float *)Wr)[b];
    float *o = out + (size_t)r * cols + 32 * b;
    for (int i = 0; i < 32; i++) {
        const int plane = 2 * half + (i >> 4);
        const int8_t q = (int8_t)Wr[sreg + 16 * U * plane + 16 * u + (i & 15)];
        o[i] = __fmul_rn((float)q, scale);
    }
}

__global__ void dq_q6k(const uint8_t *__restrict__ W, float *__restrict__ out, int rows, int cols, int stride)
{
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int U = cols >> 6, nb = cols >> 8;
    if (t >= (long)rows * U) return;
    const int r = (int)(t / U), u = (int)(t % U), sb = u >> 2, h = (u >> 1) & 1, kk = u & 1;
    const uint8_t *Wr = W + (size_t)r * stride;
    const uint8_t *QH = Wr + 16 * nb + 16 * u, *QLa = Wr + 16 * nb + 16 * U + 16 * u;
    const uint8_t *QLb = Wr + 16 * nb + 32 * U + 16 * u, *Dp = Wr + 16 * nb + 48 * U + 2 * sb;
    const int8_t *sc = (const int8_t *)(Wr + 16 * sb + 8 * h);
    const float d = f16_to_f32_ref(Dp[0] | (Dp[1] << 8));
    float *o = out + (size_t)r * cols + 256 * sb + 128 * h;
    for (int i = 0; i < 16; i++) {
        const int l = 16 * kk + i;
        const int q1 = (int)((QLa[i] & 0x0F) | ((QH[i] & 3) << 4)) - 32;
        const int q2 = (int)((QLb[i] & 0x0F) | (((QH[i] >> 2) & 3) << 4)) - 32;
        const int q3 = (int)((QLa[i] >> 4) | (((QH[i] >> 4) & 3) << 4)) - 32;
        const int q4 = (int)((QLb[i] >> 4) | (((QH[i] >> 6) & 3) << 4)) - 32;
        o[l] = __fmul_rn(__fmul_rn(d, (float)sc[kk]), (float)q1);
        o[l + 32] = __fmul_rn(__fmul_rn(d, (float)sc[kk + 2]), (float)q2);
        o[l + 64] = __fmul_rn(__fmul_rn(d, (float)sc[kk + 4]), (float)q3);
        o[l + 96] = __fmul_rn(__fmul_rn(d, (float)sc[kk + 6]), (float)q4);
    }
}

int launch_dequant(soso_hip *h, const Weight &w, float *out)
{
    const int T = 256, rows = (int)w.rows, cols = (int)w.cols, kcols = (int)weight_kcols(w);
    const int stride = (int)packed_row_stride(w.dtype, kcols);
    long n;
    switch (w.dtype) {
    case SOSO_HIP_DTYPE_Q4_K:
        n = (long)rows * (cols / 64);
        dq_q4k<<<(unsigned)((n + T - 1) / T), T, 0, h->stream>>>((const uint8_t *)w.dev, out, rows, cols);
        break;
    case SOSO_HIP_DTYPE_Q8_0:
        n = (long)rows * (cols / 32);
        dq_q80<<<(unsigned)((n + T - 1) / T), T, 0, h->stream>>>((const uint8_t *)w.dev, out, rows, cols, kcols,
                                                                 stride);
        break;
    case SOSO_HIP_DTYPE_Q6_K:
        n = (long)rows * (cols / 64);
        dq_q6k<<<(unsigned)((n + T - 1) / T), T, 0, h->stream>>>((const uint8_t *)w.dev, out, rows, cols, stride);
        break;
    case SOSO_HIP_DTYPE_F32:
        return hip_check(h, hipMemcpyAsync(out, w.dev, w.rows * w.cols * 4, hipMemcpyDeviceToDevice, h->stream),
                         "dequant f32");
    default: return set_err(h, SOSO_HIP_ERR_ARG, "dequant: dtype");
    }
    return hip_check(h, hipGetLastError(), "dequant launch");
}

// ---------------------------------------------------------------------------
// argmax (crates/soso-llm-core/src/runtime.rs:2021-2028): Iterator::max_by
// with partial_cmp(..).unwrap_or(Equal), i.e. the fold "keep the running
// maximum only if it is strictly greater than the next element, else take the
// next": the LAST maximum wins, and a NaN compares Equal both ways, so it
// takes over the running maximum and hands it to the next element.  Every
// thread folds a contiguous stretch exactly so; stretches combine in order:
// the later stretch's winner replaces the earlier one unless the earlier is
// strictly greater -- or always, when the later stretch holds a NaN (the
// sequential fold restarts at that NaN whatever came before).  Every
// workgroup reduces one contiguous segment; the last one to finish (ticket)
// combines the segments' winners in order.
// ---------------------------------------------------------------------------
constexpr int ARGMAX_WG = 256; // workgroups (<= the block size; partials: 3 KiB after the ticket)

__device__ __forceinline__ void keep_later(float &bv, int &bi, int &bn, float ov, int oi, int on)
{
    // (bv, bi, bn) is the earlier stretch's (winner, index, holds a NaN)
    if (oi >= 0 && (bi < 0 || on || !(bv > ov))) {
        bv = ov;
        bi = oi;
    }
    bn |= on;
}

__global__ void __launch_bounds__(256) k_argmax(const float *__restrict__ x, int n, uint32_t *__restrict__ out,
                                                unsigned *__restrict__ ticket)
{
    __shared__ float sv[4];
    __shared__ int si[4], sn[4];
    __shared__ int last;
    float *pv = (float *)(ticket + 64);
    int *pi = (int *)(ticket + 64 + ARGMAX_WG);
    int *pn = (int *)(ticket + 64 + 2 * ARGMAX_WG);
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63;
    const int s0 = (int)((long)n * blockIdx.x / gridDim.x), s1 = (int)((long)n * (blockIdx.x + 1) / gridDim.x);
    const int c0 = s0 + (int)((long)(s1 - s0) * tid / nt), c1 = s0 + (int)((long)(s1 - s0) * (tid + 1) / nt);
    float bv = -INFINITY;
    int bi = -1, bn = 0;
    for (int i = c0; i < c1; i++) {
        const float v = x[i];
        keep_later(bv, bi, bn, v, i, v != v);
    }
    // lanes hold ordered stretches: fold pairs (lower lane = earlier)
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_down(bv, o, 64);
        const int oi = __shfl_down(bi, o, 64), on = __shfl_down(bn, o, 64);
        if (lane + o < 64 && (lane & (2 * o - 1)) == 0) keep_later(bv, bi, bn, ov, oi, on);
    }
    if (lane == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
        sn[tid >> 6] = bn;
    }
    __syncthreads();
    if (tid == 0) {
        float v = sv[0];
        int i = si[0], q = sn[0];
        for (int w = 1; w < (nt >> 6); w++) keep_later(v, i, q, sv[w], si[w], sn[w]);
        // the segment's winner leaves through agent-scope atomic stores (they
        // reach the coherence point; no fence, so no write-back of the XCD's
        // L2), acknowledged before the ticket; the last workgroup reads the
        // winners with coherent loads
        __hip_atomic_store(pv + blockIdx.x, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pi + blockIdx.x, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pn + blockIdx.x, q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        last = atomicAdd(ticket, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    // the segments' winners, in segment order, reduced by the same ordered tree
    bv = -INFINITY;
    bi = -1;
    bn = 0;
    for (int b = tid; b < (int)gridDim.x; b += nt)
        keep_later(bv, bi, bn, __hip_atomic_load(pv + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                   __hip_atomic_load(pi + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                   __hip_atomic_load(pn + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    // thread t now holds segments t, t + nt, ...: with gridDim <= blockDim
    // that is one segment per thread, in order
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_down(bv, o, 64);
        const int oi = __shfl_down(bi, o, 64), on = __shfl_down(bn, o, 64);
        if (lane + o < 64 && (lane & (2 * o - 1)) == 0) keep_later(bv, bi, bn, ov, oi, on);
    }
    __syncthreads();
    if (lane == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
        sn[tid >> 6] = bn;
    }
    __syncthreads();
    if (tid == 0) {
        float v = sv[0];
        int i = si[0], q = sn[0];
        for (int w = 1; w < (nt >> 6); w++) keep_later(v, i, q, sv[w], si[w], sn[w]);
        *out = (uint32_t)(i < 0 ? 0 : i);
        *ticket = 0u;
    }
}

int launch_argmax(soso_hip *h, const float *x, size_t n, uint32_t *idx)
{
    const unsigned grid = (unsigned)std::max<size_t>(1, std::min<size_t>(ARGMAX_WG, (n + 1023) / 1024));
    k_argmax<<<grid, 256, 0, h->stream>>>(x, (int)n, idx, h->ticket);
    return hip_check(h, hipGetLastError(), "argmax launch");
}
