/*
 * oracle.c -- scalar CPU restatement of soso-llm-core's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP library,
 * and, with oracle_avx2.c, the CPU baseline timed by bench.py.  Built with
 * -ffp-contract=off: the Rust sources never fuse a*b+c unless they call an
 * FMA intrinsic, and neither does this file.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static inline float bits_f32(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f32_bits(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float rd_f32(const uint8_t *p)
{
    uint32_t u = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    return bits_f32(u);
}

/* ---------------------------------------------------------------------------
 * f16 <-> f32
 * ------------------------------------------------------------------------- */

/* crates/sosomodel/src/dequant.rs:26-45 (`f16_to_f32`).  Subnormals are
 * (frac/1024)*2^-14 in two roundings (both exact); every NaN becomes Rust's
 * canonical f32::NAN (0x7fc00000), unlike the C twin, which keeps the sign. */
float or_f16_to_f32(uint16_t bits)
{
    const float pow2_neg14 = 6.1035156e-5f; /* dequant.rs:24, exactly 2^-14 */
    uint32_t sign = (bits >> 15) & 1u;
    uint32_t exp = (bits >> 10) & 0x1fu;
    uint32_t frac = bits & 0x3ffu;
    if (exp == 0) {
        if (frac == 0) return bits_f32(sign << 31);
        float v = ((float)frac / 1024.0f) * pow2_neg14;
        return sign ? -v : v;
    }
    if (exp == 31) return frac == 0 ? bits_f32((sign << 31) | 0x7f800000u) : bits_f32(0x7fc00000u);
    return bits_f32((sign << 31) | ((exp + 112u) << 23) | (frac << 13));
}

/* crates/soso-llm-core/src/f16.rs:10-37 (`f32_to_f16`): round to nearest with
 * ties UP (adds the first dropped bit), not IEEE ties-to-even. */
uint16_t or_f32_to_f16(float v)
{
    uint32_t bits = f32_bits(v);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exp = (int32_t)((bits >> 23) & 0xffu);
    uint32_t frac = bits & 0x7fffffu;
    if (exp == 255) return (uint16_t)(sign | 0x7c00u | (frac != 0 ? 0x200u : 0u));
    int32_t e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t f = frac | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint16_t sub = (uint16_t)(f >> shift);
        uint16_t round = (uint16_t)((f >> (shift - 1)) & 1u);
        return (uint16_t)(sign | (uint16_t)(sub + round));
    }
    uint32_t half = ((uint32_t)e << 10) | (frac >> 13);
    uint16_t round = (uint16_t)((frac >> 12) & 1u);
    return (uint16_t)((uint16_t)(sign | (uint16_t)half) + round); /* wrapping_add */
}

/* or_f32_to_f16 over n values (KvCache::append's conversion of a row,
 * kv.rs:264-266). */
void or_f32_to_f16_n(const float *v, size_t n, uint16_t *out)
{
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_f16(v[i]);
}

/* ---------------------------------------------------------------------------
 * layout
 * ------------------------------------------------------------------------- */

/* crates/sosomodel/src/dequant.rs:53-68 (`row_bytes`), restricted to the
 * block formats of this path plus Q4_0/MXFP4 (layout.rs:57-75); Q6_K (13) is
 * this build's extension with GGML's 210-byte block.  -1 = None. */
int64_t or_row_bytes(uint8_t dtype, size_t cols)
{
    size_t elems, bytes;
    switch (dtype) {
    case OR_DTYPE_Q8_0: elems = 32; bytes = 36; break;
    case OR_DTYPE_Q4_0: elems = 32; bytes = 18; break;
    case OR_DTYPE_Q4_K: elems = 256; bytes = 144; break;
    case OR_DTYPE_MXFP4: elems = 32; bytes = 20; break;
    case OR_DTYPE_Q6_K: elems = 256; bytes = 210; break;
    default: return -1;
    }
    if (cols == 0 || cols % elems != 0) return -1;
    return (int64_t)((cols / elems) * bytes);
}

/* ---------------------------------------------------------------------------
 * dequant
 * ------------------------------------------------------------------------- */

/* dequant.rs:74-97 (`dequant_q8_0_range`): v = (q as i8) as f32 * scale. */
int or_dequant_q8_0_range(const uint8_t *bytes, size_t nbytes, size_t elem_off, float *out, size_t n)
{
    if (nbytes % OR_Q8_0_BYTES != 0 || n == 0) return -1;
    size_t total = (nbytes / OR_Q8_0_BYTES) * OR_Q8_0_ELEMS;
    size_t end = elem_off + n;
    if (end < elem_off || end > total) return -1;
    for (size_t b = elem_off / OR_Q8_0_ELEMS; b <= (end - 1) / OR_Q8_0_ELEMS; b++) {
        const uint8_t *c = bytes + b * OR_Q8_0_BYTES;
        float scale = rd_f32(c);
        size_t base = b * OR_Q8_0_ELEMS;
        for (size_t j = 0; j < 32; j++) {
            size_t e = base + j;
            if (e >= elem_off && e < end) out[e - elem_off] = (float)(int8_t)c[4 + j] * scale;
        }
    }
    return 0;
}

/* dequant.rs:150-159 (`q4k_scale_min`, GGML get_scale_min_k4). */
void or_q4k_scale_min(const uint8_t *s, int j, uint8_t *sc, uint8_t *m)
{
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* crates/soso-llm-core/src/quant.rs:46-54 (`q4k_pack_scales`). */
void or_q4k_pack_scales(const uint8_t *sc, const uint8_t *m, uint8_t *s)
{
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0x0F) | ((m[j + 4] & 0x0F) << 4));
    }
}

/* dequant.rs:204-241 (`dequant_q4_k_range`):
 * v = fl(fl(d*sc)*q - fl(dmin*m)); byte qs[pair*32+l] holds element
 * pair*64+l in its low nibble and pair*64+32+l in its high nibble. */
int or_dequant_q4_k_range(const uint8_t *bytes, size_t nbytes, size_t elem_off, float *out, size_t n)
{
    if (nbytes % OR_Q4_K_BYTES != 0 || n == 0) return -1;
    size_t total = (nbytes / OR_Q4_K_BYTES) * OR_Q4_K_ELEMS;
    size_t end = elem_off + n;
    if (end < elem_off || end > total) return -1;
    for (size_t b = elem_off / OR_Q4_K_ELEMS; b <= (end - 1) / OR_Q4_K_ELEMS; b++) {
        const uint8_t *blk = bytes + b * OR_Q4_K_BYTES;
        float d = or_f16_to_f32(rd_u16(blk));
        float dmin = or_f16_to_f32(rd_u16(blk + 2));
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        for (int pair = 0; pair < 4; pair++) {
            uint8_t sc1, m1, sc2, m2;
            or_q4k_scale_min(scales, 2 * pair, &sc1, &m1);
            or_q4k_scale_min(scales, 2 * pair + 1, &sc2, &m2);
            float d1 = d * (float)sc1, min1 = dmin * (float)m1;
            float d2 = d * (float)sc2, min2 = dmin * (float)m2;
            size_t base = b * OR_Q4_K_ELEMS + (size_t)pair * 64;
            for (int l = 0; l < 32; l++) {
                uint8_t q = qs[pair * 32 + l];
                size_t e1 = base + l, e2 = base + 32 + l;
                if (e1 >= elem_off && e1 < end) out[e1 - elem_off] = d1 * (float)(q & 0x0F) - min1;
                if (e2 >= elem_off && e2 < end) out[e2 - elem_off] = d2 * (float)(q >> 4) - min2;
            }
        }
    }
    return 0;
}

/* crates/gguf2som/src/lib.rs:1639-1661 (`dequant_q6_k_block`, GGML
 * dequantize_row_q6_K): ql[128] | qh[64] | sc i8[16] | d f16; two halves of
 * 128 elements; v = fl(fl(d*sc)*q) with q in -32..31.  Whole blocks only. */
int or_dequant_q6_k(const uint8_t *bytes, size_t nbytes, float *out, size_t n)
{
    if (nbytes % OR_Q6_K_BYTES != 0 || n != (nbytes / OR_Q6_K_BYTES) * OR_Q6_K_ELEMS) return -1;
    for (size_t b = 0; b < nbytes / OR_Q6_K_BYTES; b++) {
        const uint8_t *blk = bytes + b * OR_Q6_K_BYTES;
        float d = or_f16_to_f32(rd_u16(blk + 208));
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
            const int8_t *sc = (const int8_t *)(blk + 192 + h * 8);
            float *y = out + b * 256 + h * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l] = d * (float)sc[is] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
    return 0;
}

/* dequant.rs:172-196 (`q4k_dot_sub`): accumulates sum(q*x) and sum(x) and
 * applies d*sc and dmin*m once.  Returns 0 for a short block or j >= 8. */
float or_q4k_dot_sub(const uint8_t *blk, size_t blk_len, int j, const float *x, size_t x_len)
{
    if (blk_len < OR_Q4_K_BYTES || j < 0 || j >= 8 || x_len < 32) return 0.0f;
    float d = or_f16_to_f32(rd_u16(blk));
    float dmin = or_f16_to_f32(rd_u16(blk + 2));
    uint8_t sc, m;
    or_q4k_scale_min(blk + 4, j, &sc, &m);
    const uint8_t *qs = blk + 16;
    int pair = j >> 1, alto = j & 1;
    float qx = 0.0f, sx = 0.0f;
    for (int l = 0; l < 32; l++) {
        uint8_t q = qs[pair * 32 + l];
        float v = (float)(alto ? (q >> 4) : (q & 0x0F));
        qx += v * x[l];
        sx += x[l];
    }
    return (d * (float)sc) * qx - (dmin * (float)m) * sx;
}

/* dequant.rs:198-201 (`q4k_dot_ref`). */
float or_q4k_dot_ref(const uint8_t *blk, const float *x)
{
    float acc = 0.0f;
    for (int j = 0; j < 8; j++) acc += or_q4k_dot_sub(blk, OR_Q4_K_BYTES, j, x + j * 32, 32);
    return acc;
}

/* dequant.rs:292-315 (`matvec_row`): dequantize the row, then a sequential
 * f32 dot.  Q6_K (this build's extension) follows the same recipe. */
int or_matvec_row(uint8_t dtype, const uint8_t *row, size_t row_len, size_t cols, const float *x, float *out)
{
    int64_t rb = or_row_bytes(dtype, cols);
    if (rb < 0 || (size_t)rb != row_len) return -1;
    float *s = (float *)malloc(cols * sizeof(float));
    if (!s) return -1;
    int rc;
    switch (dtype) {
    case OR_DTYPE_Q8_0: rc = or_dequant_q8_0_range(row, row_len, 0, s, cols); break;
    case OR_DTYPE_Q4_K: rc = or_dequant_q4_k_range(row, row_len, 0, s, cols); break;
    case OR_DTYPE_Q6_K: rc = or_dequant_q6_k(row, row_len, s, cols); break;
    default: rc = -1;
    }
    if (rc == 0) {
        float sum = 0.0f;
        for (size_t c = 0; c < cols; c++) sum += s[c] * x[c];
        *out = sum;
    }
    free(s);
    return rc;
}

/* ---------------------------------------------------------------------------
 * quantizers (used only to build round-trip tests)
 * ------------------------------------------------------------------------- */

/* crates/soso-llm-core/src/quant.rs:8-24 (`quantize_q8_0`). */
size_t or_quantize_q8_0(const float *src, size_t n, uint8_t *out)
{
    size_t blocks = (n + 31) / 32, o = 0;
    for (size_t b = 0; b < blocks; b++) {
        size_t len = n - b * 32 < 32 ? n - b * 32 : 32;
        float max = 0.0f;
        for (size_t i = 0; i < len; i++) max = fmaxf(max, fabsf(src[b * 32 + i]));
        float scale = max > 0.0f ? max / 127.0f : 1.0f;
        memcpy(out + o, &scale, 4);
        o += 4;
        for (size_t i = 0; i < 32; i++) {
            float v = i < len ? src[b * 32 + i] : 0.0f;
            float r = roundf(v / scale);
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            out[o++] = (uint8_t)(int8_t)r;
        }
    }
    return o;
}

static uint8_t q4k_nibble(float v, float s, float o)
{
    /* quant.rs:139-145 (`quantize_nibble`) */
    if (s <= 0.0f) return 0;
    float r = roundf((v + o) / s);
    if (r < 0.0f) r = 0.0f;
    if (r > 15.0f) r = 15.0f;
    return (uint8_t)r;
}

static uint8_t clamp63(float r)
{
    if (r < 0.0f) r = 0.0f;
    if (r > 63.0f) r = 63.0f;
    return (uint8_t)r;
}

/* quant.rs:75-136 (`quantize_q4_k`). */
size_t or_quantize_q4_k(const float *src, size_t n, uint8_t *out)
{
    size_t blocks = (n + 255) / 256, o = 0;
    for (size_t b = 0; b < blocks; b++) {
        size_t base = b * 256;
#define VAL(i) ((base + (i)) < n ? src[base + (i)] : 0.0f)
        float s_ideal[8], o_ideal[8];
        for (int j = 0; j < 8; j++) {
            float lo = 0.0f, hi = 0.0f;
            for (int l = 0; l < 32; l++) {
                float v = VAL(j * 32 + l);
                if (v < lo) lo = v;
                if (v > hi) hi = v;
            }
            s_ideal[j] = (hi - lo) / 15.0f;
            o_ideal[j] = -lo;
        }
        float max_s = 0.0f, max_o = 0.0f;
        for (int j = 0; j < 8; j++) {
            if (s_ideal[j] > max_s) max_s = s_ideal[j];
            if (o_ideal[j] > max_o) max_o = o_ideal[j];
        }
        uint16_t d_bits = or_f32_to_f16(max_s / 63.0f), dmin_bits = or_f32_to_f16(max_o / 63.0f);
        float d = or_f16_to_f32(d_bits), dmin = or_f16_to_f32(dmin_bits);
        uint8_t sc[8], m[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = d > 0.0f ? clamp63(roundf(s_ideal[j] / d)) : 0;
            m[j] = dmin > 0.0f ? clamp63(roundf(o_ideal[j] / dmin)) : 0;
        }
        out[o++] = (uint8_t)(d_bits & 0xff);
        out[o++] = (uint8_t)(d_bits >> 8);
        out[o++] = (uint8_t)(dmin_bits & 0xff);
        out[o++] = (uint8_t)(dmin_bits >> 8);
        or_q4k_pack_scales(sc, m, out + o);
        o += 12;
        for (int pair = 0; pair < 4; pair++) {
            float s1 = d * (float)sc[2 * pair], o1 = dmin * (float)m[2 * pair];
            float s2 = d * (float)sc[2 * pair + 1], o2 = dmin * (float)m[2 * pair + 1];
            for (int l = 0; l < 32; l++) {
                uint8_t q1 = q4k_nibble(VAL(pair * 64 + l), s1, o1);
                uint8_t q2 = q4k_nibble(VAL(pair * 64 + 32 + l), s2, o2);
                out[o++] = (uint8_t)(q1 | (q2 << 4));
            }
        }
#undef VAL
    }
    return o;
}

/* ---------------------------------------------------------------------------
 * scalar matvecs
 * ------------------------------------------------------------------------- */

/* crates/soso-llm-core/src/gemm.rs:47-56 (`matvec_f32_scalar`). */
void or_matvec_f32_scalar(const float *w, size_t rows, size_t cols, const float *x, float *out)
{
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        const float *row = w + r * cols;
        for (size_t c = 0; c < cols; c++) acc += row[c] * x[c];
        out[r] = acc;
    }
}

/* gemm.rs:315-332 (`matvec_q8_0_scalar`): s = sum(q*x) per block, acc += scale*s. */
void or_matvec_q8_0_scalar(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out)
{
    size_t nb = cols / 32, rb = nb * OR_Q8_0_BYTES;
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = w + r * rb;
        float acc = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *c = row + b * OR_Q8_0_BYTES;
            float scale = rd_f32(c);
            const float *xb = x + b * 32;
            float s = 0.0f;
            for (int l = 0; l < 32; l++) s += (float)(int8_t)c[4 + l] * xb[l];
            acc += scale * s;
        }
        out[r] = acc;
    }
}

/* gemm.rs:428-461 (`matvec_q4_k_scalar`): factorised per sub-block,
 * acc += d*sc*sum(q*x) - dmin*m*sum(x), lower nibble then upper nibble. */
void or_matvec_q4_k_scalar(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out)
{
    size_t nb = cols / 256, rb = nb * OR_Q4_K_BYTES;
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = w + r * rb;
        float acc = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * OR_Q4_K_BYTES;
            float d = or_f16_to_f32(rd_u16(blk));
            float dmin = or_f16_to_f32(rd_u16(blk + 2));
            const uint8_t *scales = blk + 4, *qs = blk + 16;
            const float *xb = x + b * 256;
            for (int pair = 0; pair < 4; pair++) {
                uint8_t sc1, m1, sc2, m2;
                or_q4k_scale_min(scales, 2 * pair, &sc1, &m1);
                or_q4k_scale_min(scales, 2 * pair + 1, &sc2, &m2);
                const float *x1 = xb + pair * 64, *x2 = xb + pair * 64 + 32;
                const uint8_t *q = qs + pair * 32;
                float s1 = 0.0f, sx1 = 0.0f, s2 = 0.0f, sx2 = 0.0f;
                for (int l = 0; l < 32; l++) {
                    s1 += (float)(q[l] & 0x0F) * x1[l];
                    sx1 += x1[l];
                    s2 += (float)(q[l] >> 4) * x2[l];
                    sx2 += x2[l];
                }
                acc += d * (float)sc1 * s1 - dmin * (float)m1 * sx1;
                acc += d * (float)sc2 * s2 - dmin * (float)m2 * sx2;
            }
        }
        out[r] = acc;
    }
}

/* Q6_K has no runtime matvec in the reference (gguf2som re-quantizes it to
 * Q8_0).  The oracle is `matvec_row`'s recipe (dequant.rs:292-315) applied to
 * `dequant_q6_k_block`: exact dequant, then a sequential f32 dot. */
void or_matvec_q6_k_scalar(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out)
{
    size_t rb = (cols / 256) * OR_Q6_K_BYTES;
    float *s = (float *)malloc(cols * sizeof(float));
    if (!s) return;
    for (size_t r = 0; r < rows; r++) {
        or_dequant_q6_k(w + r * rb, rb, s, cols);
        float sum = 0.0f;
        for (size_t c = 0; c < cols; c++) sum += s[c] * x[c];
        out[r] = sum;
    }
    free(s);
}

/* Brute-force reference: exact dequant, f64 accumulation (the pattern of
 * crates/soso-llm-api/tests/cuda_matvec.rs:35-81). */
int or_matvec_f64(uint8_t dtype, const uint8_t *w, size_t rows, size_t cols, const float *x, double *out)
{
    float *s = (float *)malloc(cols * sizeof(float));
    if (!s) return -1;
    int rc = 0;
    size_t rb = dtype == OR_DTYPE_F32 ? cols * 4 : (size_t)or_row_bytes(dtype, cols);
    for (size_t r = 0; r < rows && rc == 0; r++) {
        const uint8_t *row = w + r * rb;
        switch (dtype) {
        case OR_DTYPE_F32: memcpy(s, row, cols * 4); break;
        case OR_DTYPE_Q8_0: rc = or_dequant_q8_0_range(row, rb, 0, s, cols); break;
        case OR_DTYPE_Q4_K: rc = or_dequant_q4_k_range(row, rb, 0, s, cols); break;
        case OR_DTYPE_Q6_K: rc = or_dequant_q6_k(row, rb, s, cols); break;
        default: rc = -1;
        }
        double acc = 0.0;
        for (size_t c = 0; c < cols; c++) acc += (double)s[c] * (double)x[c];
        out[r] = acc;
    }
    free(s);
    return rc;
}

/* ---------------------------------------------------------------------------
 * Host thread pool: HostPool (crates/soso-llm-api/src/host_pool.rs:37-137).
 * n threads in all, the caller being thread 0; workers spin on an epoch
 * counter for OR_SPINS rounds and then sleep on a condition variable; a call
 * cuts `rows` into strips [rows*i/n, rows*(i+1)/n) (`franja`, :31-33), runs
 * strip 0 itself and spins until the n - 1 workers have counted themselves
 * done.  One caller at a time (the oracle is driven from one thread).
 * ------------------------------------------------------------------------- */
#include <stdatomic.h>

#define OR_SPINS 20000 /* GIROS_ANTES_DE_DORMIR, host_pool.rs:13 */

typedef void (*or_rows_fn)(void *ctx, size_t r0, size_t r1);

static struct {
    int n;
    pthread_t *tid;
    atomic_uint epoch;
    atomic_size_t done;
    atomic_int stop;
    size_t rows;
    or_rows_fn fn;
    void *ctx;
    pthread_mutex_t mu;
    pthread_cond_t cv;
} or_pool = {1, NULL, 0, 0, 0, 0, NULL, NULL, PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER};

static void pool_strip(size_t rows, int i, int n, size_t *r0, size_t *r1)
{
    *r0 = rows * (size_t)i / (size_t)n;
    *r1 = rows * (size_t)(i + 1) / (size_t)n;
}

static unsigned or_pool_start; /* the epoch when the workers were made */

static void *pool_worker(void *arg)
{
    const int i = (int)(intptr_t)arg;
    /* the epoch as it was before any call could bump it (a worker that read
     * the live value after the first call's bump would wait for the next) */
    unsigned last = or_pool_start;
    for (;;) {
        unsigned spins = 0;
        while (atomic_load_explicit(&or_pool.epoch, memory_order_acquire) == last) {
            if (atomic_load_explicit(&or_pool.stop, memory_order_acquire)) return NULL;
            if (++spins < OR_SPINS) continue;
            pthread_mutex_lock(&or_pool.mu);
            if (atomic_load_explicit(&or_pool.epoch, memory_order_acquire) == last &&
                !atomic_load_explicit(&or_pool.stop, memory_order_acquire))
                pthread_cond_wait(&or_pool.cv, &or_pool.mu);
            pthread_mutex_unlock(&or_pool.mu);
            spins = 0;
        }
        last = atomic_load_explicit(&or_pool.epoch, memory_order_acquire);
        size_t r0, r1;
        pool_strip(or_pool.rows, i, or_pool.n, &r0, &r1);
        if (r0 < r1) or_pool.fn(or_pool.ctx, r0, r1);
        atomic_fetch_add_explicit(&or_pool.done, 1, memory_order_acq_rel);
    }
}

static void pool_stop(void)
{
    if (!or_pool.tid) return;
    atomic_store_explicit(&or_pool.stop, 1, memory_order_release);
    pthread_mutex_lock(&or_pool.mu);
    pthread_cond_broadcast(&or_pool.cv);
    pthread_mutex_unlock(&or_pool.mu);
    for (int i = 1; i < or_pool.n; i++) pthread_join(or_pool.tid[i], NULL);
    free(or_pool.tid);
    or_pool.tid = NULL;
    or_pool.n = 1;
    atomic_store_explicit(&or_pool.stop, 0, memory_order_release);
}

/* A pool of `threads` threads (made once, remade when the count changes). */
static int pool_size(int threads)
{
    if (threads < 1) threads = 1;
    if (threads == or_pool.n) return 0;
    pool_stop();
    if (threads == 1) return 0;
    or_pool.tid = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
    if (!or_pool.tid) return -1;
    or_pool.n = threads;
    or_pool_start = atomic_load_explicit(&or_pool.epoch, memory_order_acquire);
    for (int i = 1; i < threads; i++)
        if (pthread_create(&or_pool.tid[i], NULL, pool_worker, (void *)(intptr_t)i)) {
            or_pool.n = i;
            pool_stop();
            return -1;
        }
    return 0;
}

/* for_rows (host_pool.rs:102-124). */
static int pool_for_rows(int threads, size_t rows, or_rows_fn fn, void *ctx)
{
    if (pool_size(threads)) return -1;
    if (or_pool.n <= 1 || rows == 0) {
        fn(ctx, 0, rows);
        return 0;
    }
    or_pool.rows = rows;
    or_pool.fn = fn;
    or_pool.ctx = ctx;
    atomic_store_explicit(&or_pool.done, 0, memory_order_release);
    atomic_fetch_add_explicit(&or_pool.epoch, 1, memory_order_acq_rel);
    pthread_mutex_lock(&or_pool.mu);
    pthread_cond_broadcast(&or_pool.cv);
    pthread_mutex_unlock(&or_pool.mu);
    size_t r0, r1;
    pool_strip(rows, 0, or_pool.n, &r0, &r1);
    if (r0 < r1) fn(ctx, r0, r1);
    while (atomic_load_explicit(&or_pool.done, memory_order_acquire) < (size_t)(or_pool.n - 1)) {
    }
    return 0;
}

/* ---------------------------------------------------------------------------
 * matvec_view_par: dtype dispatch + contiguous row strips
 * crates/soso-llm-core/src/layer.rs:124-240, run on the host pool above
 * (its strips, host_pool.rs:31-33).
 * ------------------------------------------------------------------------- */

typedef struct {
    uint8_t dtype;
    const uint8_t *w;
    size_t rows, cols, n;
    const float *xs;
    float *outs;
    size_t r0, r1;
    int avx2;
} strip_job;

static void run_strip(const strip_job *j)
{
    size_t rb = j->dtype == OR_DTYPE_F32 ? j->cols * 4 : (size_t)or_row_bytes(j->dtype, j->cols);
    size_t sub = j->r1 - j->r0;
    if (sub == 0) return;
    const uint8_t *w = j->w + j->r0 * rb;
    for (size_t v = 0; v < j->n; v++) {
        const float *x = j->xs + v * j->cols;
        float *o = j->outs + v * j->rows + j->r0;
        switch (j->dtype) {
        case OR_DTYPE_F32:
            if (j->avx2) or_matvec_f32_avx2((const float *)w, sub, j->cols, x, o);
            else or_matvec_f32_scalar((const float *)w, sub, j->cols, x, o);
            break;
        case OR_DTYPE_Q8_0:
            if (j->avx2) or_matvec_q8_0_avx2(w, sub, j->cols, x, o);
            else or_matvec_q8_0_scalar(w, sub, j->cols, x, o);
            break;
        case OR_DTYPE_Q4_K:
            if (j->avx2) or_matvec_q4_k_avx2(w, sub, j->cols, x, o);
            else or_matvec_q4_k_scalar(w, sub, j->cols, x, o);
            break;
        case OR_DTYPE_Q6_K: or_matvec_q6_k_scalar(w, sub, j->cols, x, o); break;
        default: break;
        }
    }
}

/* parallel.rs:22-31 (`row_strip`): the even split with the remainder spread
 * over the first strips (the read-bandwidth probe below uses it). */
static void row_strip(size_t rows, size_t i, size_t n, size_t *s, size_t *e)
{
    size_t base = rows / n, rem = rows % n;
    *s = i * base + (i < rem ? i : rem);
    *e = *s + base + (i < rem ? 1 : 0);
}

static void strip_rows(void *ctx, size_t r0, size_t r1)
{
    strip_job j = *(const strip_job *)ctx;
    j.r0 = r0;
    j.r1 = r1;
    run_strip(&j);
}

int or_matmul_par(uint8_t dtype, const uint8_t *w, size_t rows, size_t cols, size_t n, const float *xs,
                  float *outs, int threads, int avx2)
{
    if (dtype != OR_DTYPE_F32 && or_row_bytes(dtype, cols) < 0) return -1;
    if (rows == 0 || n == 0) return 0;
    if (avx2 && !or_have_avx2()) avx2 = 0;
    strip_job j = {dtype, w, rows, cols, n, xs, outs, 0, 0, avx2};
    return pool_for_rows(threads, rows, strip_rows, &j);
}

int or_matvec_par(uint8_t dtype, const uint8_t *w, size_t rows, size_t cols, const float *x, float *out,
                  int threads, int avx2)
{
    return or_matmul_par(dtype, w, rows, cols, 1, x, out, threads, avx2);
}

/* ---------------------------------------------------------------------------
 * small ops
 * ------------------------------------------------------------------------- */

/* gemm.rs:62-74 (`softmax_inplace`): max-shift, libm expf, sequential sum,
 * divide when the sum is positive.  f32::max ignores NaN, as fmaxf does. */
void or_softmax(float *x, size_t n)
{
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    if (sum > 0.0f)
        for (size_t i = 0; i < n; i++) x[i] /= sum;
}

/* gemm.rs:77-91 (`topk_softmax`): softmax, stable sort by weight descending
 * (equal weights keep index order, so the LOWEST index wins a tie; NaN
 * compares Equal), truncate to k, renormalise by the sequential sum. */
size_t or_topk_softmax(float *logits, size_t n, size_t k, int32_t *idx, float *w)
{
    or_softmax(logits, n);
    int32_t *ord = (int32_t *)malloc(n * sizeof(int32_t));
    if (!ord) return 0;
    for (size_t i = 0; i < n; i++) ord[i] = (int32_t)i;
    /* stable insertion sort with comparator b.partial_cmp(a) */
    for (size_t i = 1; i < n; i++) {
        int32_t v = ord[i];
        size_t j = i;
        while (j > 0 && logits[v] > logits[ord[j - 1]]) { /* Less => move before */
            ord[j] = ord[j - 1];
            j--;
        }
        ord[j] = v;
    }
    size_t kk = k < n ? k : n;
    float sum = 0.0f;
    for (size_t j = 0; j < kk; j++) {
        idx[j] = ord[j];
        w[j] = logits[ord[j]];
        sum += w[j];
    }
    if (sum > 0.0f)
        for (size_t j = 0; j < kk; j++) w[j] /= sum;
    free(ord);
    return kk;
}

/* gemm.rs:210-212 (`silu`). */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* gemm.rs:215-226 (`swiglu_inplace`, scalar branch). */
void or_swiglu(float *up, const float *gate, size_t n)
{
    for (size_t i = 0; i < n; i++) up[i] = or_silu(gate[i]) * up[i];
}

/* gemm.rs:93-100 (`rmsnorm`): var = sum(v*v)/n; x = x*scale*w. */
void or_rmsnorm(float *x, const float *w, size_t n, float eps)
{
    float var = 0.0f;
    for (size_t i = 0; i < n; i++) var += x[i] * x[i];
    var = var / (float)n;
    float scale = 1.0f / sqrtf(var + eps);
    for (size_t i = 0; i < n; i++) x[i] = x[i] * scale * w[i];
}

/* gemm.rs:1452-1490 (`rope_cabezas`): per pair i, freq = theta^(-2i/d),
 * angle = pos*freq; interleaved pairs (2i, 2i+1) unless neox. */
void or_rope_heads(float *x, size_t n_heads, size_t head_dim, size_t pos, float theta, int neox)
{
    if (head_dim < 2 || n_heads == 0) return;
    size_t half = head_dim / 2;
    float n_f = (float)head_dim;
    float *cs = (float *)malloc(half * 2 * sizeof(float));
    if (!cs) return;
    float *sn = cs + half;
    for (size_t i = 0; i < half; i++) {
        float freq = powf(theta, -2.0f * (float)i / n_f);
        float angle = (float)pos * freq;
        sn[i] = sinf(angle);
        cs[i] = cosf(angle);
    }
    for (size_t h = 0; h < n_heads; h++) {
        float *v = x + h * head_dim;
        for (size_t i = 0; i < half; i++) {
            if (neox) {
                float a = v[i], b = v[i + half];
                v[i] = a * cs[i] - b * sn[i];
                v[i + half] = a * sn[i] + b * cs[i];
            } else {
                float a = v[2 * i], b = v[2 * i + 1];
                v[2 * i] = a * cs[i] - b * sn[i];
                v[2 * i + 1] = a * sn[i] + b * cs[i];
            }
        }
    }
    free(cs);
}

/* crates/soso-llm-core/src/runtime.rs:2021-2028 (`Runtime::argmax`):
 * Iterator::max_by keeps the LATER element unless the earlier one compares
 * Greater; NaN compares Equal.  So the last maximum wins. */
uint32_t or_argmax(const float *x, size_t n)
{
    if (n == 0) return 0;
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (!(x[best] > x[i])) best = i;
    return (uint32_t)best;
}

/* crates/soso-llm-core/src/attn.rs:73-140
 * (`attention_decode_f16_tiled_scalar`) with f32 K/V instead of f16: tiles
 * of 64 tokens (attn.rs:15), online softmax, scale 1/sqrt(head_dim).  KV
 * layout [token][kv_dim], head at kv_head*head_dim. */
void or_attention_f32(const float *q, const float *k, const float *v, size_t hd, size_t kv_dim, size_t kv_head,
                      size_t n_tokens, float *out)
{
    for (size_t d = 0; d < hd; d++) out[d] = 0.0f;
    if (n_tokens == 0 || hd == 0) return;
    float inv = 1.0f / sqrtf((float)hd);
    float m = -INFINITY, l = 0.0f, ts[64];
    for (size_t t0 = 0; t0 < n_tokens; t0 += 64) {
        size_t t1 = t0 + 64 < n_tokens ? t0 + 64 : n_tokens;
        float tmax = -INFINITY;
        for (size_t t = t0; t < t1; t++) {
            const float *kr = k + t * kv_dim + kv_head * hd;
            float dot = 0.0f;
            for (size_t d = 0; d < hd; d++) dot += q[d] * kr[d];
            float s = dot * inv;
            ts[t - t0] = s;
            if (s > tmax) tmax = s;
        }
        float m_new = m > tmax ? m : tmax;
        float alpha = m == -INFINITY ? 0.0f : expf(m - m_new);
        for (size_t d = 0; d < hd; d++) out[d] *= alpha;
        l *= alpha;
        float tsum = 0.0f;
        for (size_t t = t0; t < t1; t++) {
            float p = expf(ts[t - t0] - m_new);
            tsum += p;
            const float *vr = v + t * kv_dim + kv_head * hd;
            for (size_t d = 0; d < hd; d++) out[d] += p * vr[d];
        }
        l += tsum;
        m = m_new;
    }
    if (l > 0.0f) {
        float il = 1.0f / l;
        for (size_t d = 0; d < hd; d++) out[d] *= il;
    }
}

/* Decode attention of every query head, heads spread over `threads` threads
 * (atencion_f16_grupos splits (KV head, chunk) tasks over the host pool,
 * layer.rs:804-896; here one task per query head).  q [n_heads * hd], caches
 * position-major [T][n_kv_heads * hd], out [n_heads * hd]. */
typedef struct {
    const float *q, *k, *v;
    size_t hd, kv_dim, group, T;
    float *out;
} attn_job;

static void attn_rows(void *ctx, size_t h0, size_t h1)
{
    const attn_job *j = (const attn_job *)ctx;
    for (size_t h = h0; h < h1; h++)
        or_attention_f32(j->q + h * j->hd, j->k, j->v, j->hd, j->kv_dim, h / j->group, j->T, j->out + h * j->hd);
}

int or_attention_heads_par(const float *q, const float *k, const float *v, size_t hd, size_t n_heads,
                           size_t n_kv_heads, size_t T, float *out, int threads)
{
    if (n_kv_heads == 0 || n_heads % n_kv_heads) return -1;
    attn_job j = {q, k, v, hd, n_kv_heads * hd, n_heads / n_kv_heads, T, out};
    return pool_for_rows(threads, n_heads, attn_rows, &j);
}

/* One dense decode layer on the CPU (the CPU baseline of the device decode
 * step): LayerExecutor::forward_layer's GQA branch (layer.rs:1092-1389) with
 * the pieces restated above -- rmsnorm, q/k/v, rope_cabezas (non-NeoX), K/V
 * rows appended at `pos` of position-major f32 caches [ctx][n_kv*hd],
 * attention over pos + 1 positions, o + residual, rmsnorm, gate/up, swiglu,
 * down + residual.  h is updated in place.  w[0..8] = attn_norm (f32), q, k,
 * v, o, ffn_norm (f32), gate, up, down (dtype). */
int or_decode_layer(float *h, const void *const *w, uint8_t dtype, size_t hidden, size_t n_heads, size_t n_kv_heads,
                    size_t hd, size_t ffn, float *kcache, float *vcache, size_t pos, float theta, float eps,
                    int threads, int avx2)
{
    const size_t qd = n_heads * hd, kvd = n_kv_heads * hd;
    float *xn = (float *)malloc(hidden * 4), *q = (float *)malloc(qd * 4), *att = (float *)malloc(qd * 4);
    float *o = (float *)malloc(hidden * 4), *g = (float *)malloc(ffn * 4), *u = (float *)malloc(ffn * 4);
    int rc = -1;
    if (!xn || !q || !att || !o || !g || !u) goto done;
    memcpy(xn, h, hidden * 4);
    or_rmsnorm(xn, (const float *)w[0], hidden, eps);
    if (or_matvec_par(dtype, (const uint8_t *)w[1], qd, hidden, xn, q, threads, avx2) ||
        or_matvec_par(dtype, (const uint8_t *)w[2], kvd, hidden, xn, kcache + pos * kvd, threads, avx2) ||
        or_matvec_par(dtype, (const uint8_t *)w[3], kvd, hidden, xn, vcache + pos * kvd, threads, avx2))
        goto done;
    or_rope_heads(q, n_heads, hd, pos, theta, 0);
    or_rope_heads(kcache + pos * kvd, n_kv_heads, hd, pos, theta, 0);
    if (or_attention_heads_par(q, kcache, vcache, hd, n_heads, n_kv_heads, pos + 1, att, threads)) goto done;
    if (or_matvec_par(dtype, (const uint8_t *)w[4], hidden, qd, att, o, threads, avx2)) goto done;
    for (size_t i = 0; i < hidden; i++) h[i] += o[i];
    memcpy(xn, h, hidden * 4);
    or_rmsnorm(xn, (const float *)w[5], hidden, eps);
    if (or_matvec_par(dtype, (const uint8_t *)w[6], ffn, hidden, xn, g, threads, avx2) ||
        or_matvec_par(dtype, (const uint8_t *)w[7], ffn, hidden, xn, u, threads, avx2))
        goto done;
    if (avx2 && or_have_avx2()) or_swiglu_avx2(u, g, ffn);
    else or_swiglu(u, g, ffn);
    if (or_matvec_par(dtype, (const uint8_t *)w[8], hidden, ffn, u, o, threads, avx2)) goto done;
    for (size_t i = 0; i < hidden; i++) h[i] += o[i];
    rc = 0;
done:
    free(xn);
    free(q);
    free(att);
    free(o);
    free(g);
    free(u);
    return rc;
}

/* ---------------------------------------------------------------------------
 * MoE FFN, one token
 * forward_moe_ffn (layer.rs:1938-1975) -> moe_expertos_agrupados CPU branch
 * (layer.rs:1869-1934): router matvec_f32, topk_softmax, gate+up for every
 * chosen expert, swiglu, down, acc = sum_j down_j * w_j in ranking order
 * starting from zero.  The residual is added by the caller (layer.rs:1389).
 * ------------------------------------------------------------------------- */
int or_moe_ffn(const float *router, size_t n_exp, size_t h, size_t ffn, size_t top_k,
               const uint8_t *const *gate, const uint8_t *const *up, const uint8_t *const *down,
               uint8_t dtype_gu, uint8_t dtype_down, const float *x, float *out, int32_t *idx_out,
               float *w_out, int threads, int avx2)
{
    float *logits = (float *)malloc(n_exp * sizeof(float));
    float *g = (float *)malloc(ffn * sizeof(float));
    float *u = (float *)malloc(ffn * sizeof(float));
    float *dn = (float *)malloc(h * sizeof(float));
    int32_t *idx = (int32_t *)malloc(top_k * sizeof(int32_t));
    float *w = (float *)malloc(top_k * sizeof(float));
    int rc = -1;
    if (!logits || !g || !u || !dn || !idx || !w) goto done;
    if (or_matvec_par(OR_DTYPE_F32, (const uint8_t *)router, n_exp, h, x, logits, threads, avx2)) goto done;
    size_t kk = or_topk_softmax(logits, n_exp, top_k, idx, w);
    for (size_t i = 0; i < h; i++) out[i] = 0.0f;
    for (size_t j = 0; j < kk; j++) {
        int32_t e = idx[j];
        if (or_matvec_par(dtype_gu, gate[e], ffn, h, x, g, threads, avx2)) goto done;
        if (or_matvec_par(dtype_gu, up[e], ffn, h, x, u, threads, avx2)) goto done;
        if (avx2 && or_have_avx2()) or_swiglu_avx2(u, g, ffn);
        else or_swiglu(u, g, ffn);
        if (or_matvec_par(dtype_down, down[e], h, ffn, u, dn, threads, avx2)) goto done;
        for (size_t i = 0; i < h; i++) out[i] += dn[i] * w[j];
    }
    for (size_t j = 0; j < kk; j++) {
        if (idx_out) idx_out[j] = idx[j];
        if (w_out) w_out[j] = w[j];
    }
    rc = 0;
done:
    free(logits);
    free(g);
    free(u);
    free(dn);
    free(idx);
    free(w);
    return rc;
}

/* ---------------------------------------------------------------------------
 * Shared expert of an MoE block (GpuDispatch::moe_compartido, gpu.rs:518-534)
 * as soso's CPU path computes it (bloque35.rs:952-985): per token t, puerta =
 * sigmoid(x_t . pg_w) (the f32 row ffn_gate_inp_shexp), gate and up matvecs,
 * swiglu_inplace, down; out_t = c_t * puerta (the block sum adds it last,
 * bloque35.rs:1000-1005).
 * ------------------------------------------------------------------------- */
int or_moe_shared(const float *pg_w, size_t h, size_t ffn, const uint8_t *gate, const uint8_t *up,
                  const uint8_t *down, uint8_t dtype_gu, uint8_t dtype_down, const float *xs, size_t n, float *out)
{
    float *g = (float *)malloc(ffn * sizeof(float));
    float *u = (float *)malloc(ffn * sizeof(float));
    int rc = -1;
    if (!g || !u) goto done;
    for (size_t t = 0; t < n; t++) {
        const float *x = xs + t * h;
        float pg;
        if (or_matvec_par(OR_DTYPE_F32, (const uint8_t *)pg_w, 1, h, x, &pg, 1, 0)) goto done;
        const float puerta = 1.0f / (1.0f + expf(-pg));
        if (or_matvec_par(dtype_gu, gate, ffn, h, x, g, 1, 0) || or_matvec_par(dtype_gu, up, ffn, h, x, u, 1, 0))
            goto done;
        or_swiglu(u, g, ffn);
        float *o = out + t * h;
        if (or_matvec_par(dtype_down, down, h, ffn, u, o, 1, 0)) goto done;
        for (size_t i = 0; i < h; i++) o[i] = o[i] * puerta;
    }
    rc = 0;
done:
    free(g);
    free(u);
    return rc;
}

/* ---------------------------------------------------------------------------
 * Gated DeltaNet (Qwen3.5): the recurrence of GpuDispatch::gdn_bloque
 * (gpu.rs:577-599) as soso's CPU path computes it (bloque35.rs:372-465 from
 * `hist` on; the decode layer forward_gdn_attn, arch.rs:586-768, is the same
 * for one token).
 * ------------------------------------------------------------------------- */

/* arch.rs:358-360 (`sigmoid`). */
float or_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* arch.rs:362-368 (`softplus`): x above 20 passes through. */
float or_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* arch.rs:370-380 (`l2_normalize`): x *= 1 / sqrt(sum(x^2) + eps). */
void or_l2_normalize(float *x, size_t n, float eps)
{
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss + eps);
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* arch.rs:382-415 (`gdn_step`): with S the d x d state (row i, column j),
 * delta_j = (v_j - g sum_i S_ij k_i) beta; S_ij <- g S_ij + k_i delta_j;
 * out_j = sum_i S_ij q_i over the updated state; sums in i order. */
void or_gdn_step(float *state, const float *q, const float *k, const float *v, size_t d, float g, float beta,
                 float *out)
{
    float delta[256];
    if (d > 256) return;
    for (size_t j = 0; j < d; j++) {
        delta[j] = 0.0f;
        out[j] = 0.0f;
    }
    for (size_t i = 0; i < d; i++)
        for (size_t j = 0; j < d; j++) delta[j] += state[i * d + j] * k[i];
    for (size_t j = 0; j < d; j++) delta[j] = (v[j] - g * delta[j]) * beta;
    for (size_t i = 0; i < d; i++)
        for (size_t j = 0; j < d; j++) {
            float ns = g * state[i * d + j] + k[i] * delta[j];
            state[i * d + j] = ns;
            out[j] += ns * q[i];
        }
}

/* bloque35.rs:391-395 / arch.rs:640-647: per token and value head, decay =
 * exp(softplus(alpha + dt) * a) and beta = sigmoid(beta_raw), from the
 * ssm_alpha / ssm_beta projections ([n][n_v]). */
void or_gdn_gates(const float *alpha, const float *beta_raw, const float *dt, const float *a, size_t n, size_t n_v,
                  float *decay, float *beta)
{
    for (size_t t = 0; t < n; t++)
        for (size_t i = 0; i < n_v; i++) {
            decay[t * n_v + i] = expf(or_softplus(alpha[t * n_v + i] + dt[i]) * a[i]);
            beta[t * n_v + i] = or_sigmoid(beta_raw[t * n_v + i]);
        }
}

/* GpuDispatch::gdn_bloque's contract, computed as bloque35.rs:412-465:
 *   hist  [(kernel - 1 + n) x C]  the conv state (oldest first), then the
 *                                 block's qkv projections (C = 2 n_k d + n_v d)
 *   conv  [C x kernel]            causal conv weights
 *   z [n x n_v d], decay / beta [n x n_v], norm [d]
 *   state [n_v x d x d]           in and out
 *   out   [n x n_v d]
 * Per token: u = silu(conv over hist rows t .. t + kernel - 1); q and k heads
 * l2-normalised, q scaled by 1 / sqrt(d); per value head vh (q/k head
 * vh mod n_k): gdn_step, rmsnorm(o, norm, eps), o *= silu(z).  The conv
 * state after the block (the last kernel - 1 rows of hist) is the caller's. */
int or_gdn_block(const float *hist, const float *conv, const float *z, const float *decay, const float *beta,
                 const float *norm, float *state, float *out, size_t n, size_t n_k, size_t n_v, size_t d,
                 size_t kernel, float eps)
{
    if (d == 0 || d > 256 || kernel == 0 || n_k == 0 || n_v == 0) return -1;
    const size_t qk_dim = n_k * d, v_dim = n_v * d, C = 2 * qk_dim + v_dim, prev = kernel - 1;
    float *ups = (float *)malloc(n * C * sizeof(float));
    if (!ups) return -1;
    const float scale = 1.0f / sqrtf((float)d);
    for (size_t t = 0; t < n; t++) {
        float *up = ups + t * C;
        for (size_t ch = 0; ch < C; ch++) {
            float acc = 0.0f;
            for (size_t k = 0; k < prev; k++) acc += conv[ch * kernel + k] * hist[(t + k) * C + ch];
            acc += conv[ch * kernel + prev] * hist[(t + prev) * C + ch];
            up[ch] = or_silu(acc);
        }
        for (size_t hh = 0; hh < n_k; hh++) {
            or_l2_normalize(up + hh * d, d, eps);
            or_l2_normalize(up + qk_dim + hh * d, d, eps);
        }
        for (size_t i = 0; i < qk_dim; i++) up[i] *= scale;
    }
    for (size_t vh = 0; vh < n_v; vh++) {
        const size_t kh = vh % n_k;
        float *st = state + vh * d * d;
        for (size_t t = 0; t < n; t++) {
            const float *base = ups + t * C;
            float *o = out + t * v_dim + vh * d;
            const float *g = z + t * v_dim + vh * d;
            or_gdn_step(st, base + kh * d, base + qk_dim + kh * d, base + 2 * qk_dim + vh * d, d,
                        decay[t * n_v + vh], beta[t * n_v + vh], o);
            or_rmsnorm(o, norm, d, eps);
            for (size_t i = 0; i < d; i++) o[i] *= or_silu(g[i]);
        }
    }
    free(ups);
    return 0;
}

/* ---------------------------------------------------------------------------
 * Synthetic inputs: counter-based SplitMix64 keyed by (seed, stream, index),
 * integer-only so that the device generator of the HIP library produces the
 * same bytes.  Normals are Irwin-Hall(12) over 16-bit uniforms, computed
 * exactly: N = (S - 393210) / 65536, variance 1.
 * ------------------------------------------------------------------------- */
static inline uint64_t fin64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t or_rng(uint64_t seed, uint64_t stream, uint64_t i)
{
    uint64_t key = fin64(seed ^ fin64(stream + 0x9E3779B97F4A7C15ull));
    return fin64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

float or_normal(uint64_t seed, uint64_t stream, uint64_t i)
{
    int32_t s = 0;
    for (int h = 0; h < 3; h++) {
        uint64_t r = or_rng(seed, stream, 3 * i + (uint64_t)h);
        s += (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) +
             (int32_t)(r >> 48);
    }
    return (float)(s - 393210) * (1.0f / 65536.0f);
}

/* stream layout: (stream << 4) | field */
#define SUB(s, f) (((s) << 4) | (f))

void or_synth_q4_k(uint8_t *out, size_t rows, size_t cols, uint64_t seed, uint64_t stream)
{
    size_t nblk = rows * (cols / 256);
    for (size_t b = 0; b < nblk; b++) {
        uint8_t *blk = out + b * OR_Q4_K_BYTES;
        uint16_t d = or_f32_to_f16(fabsf(or_normal(seed, SUB(stream, 0), b)) * 0.01f);
        uint16_t dm = or_f32_to_f16(fabsf(or_normal(seed, SUB(stream, 1), b)) * 0.01f);
        blk[0] = (uint8_t)d;
        blk[1] = (uint8_t)(d >> 8);
        blk[2] = (uint8_t)dm;
        blk[3] = (uint8_t)(dm >> 8);
        uint64_t a = or_rng(seed, SUB(stream, 2), 2 * b), c = or_rng(seed, SUB(stream, 2), 2 * b + 1);
        uint8_t sc[8], m[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = (uint8_t)((a >> (8 * j)) & 63);
            m[j] = (uint8_t)((c >> (8 * j)) & 63);
        }
        or_q4k_pack_scales(sc, m, blk + 4);
        for (int k = 0; k < 16; k++) {
            uint64_t r = or_rng(seed, SUB(stream, 3), 16 * b + (uint64_t)k);
            for (int j = 0; j < 8; j++) blk[16 + 8 * k + j] = (uint8_t)(r >> (8 * j));
        }
    }
}

void or_synth_q8_0(uint8_t *out, size_t rows, size_t cols, uint64_t seed, uint64_t stream)
{
    size_t nblk = rows * (cols / 32);
    for (size_t b = 0; b < nblk; b++) {
        uint8_t *blk = out + b * OR_Q8_0_BYTES;
        float s = or_f16_to_f32(or_f32_to_f16(fabsf(or_normal(seed, SUB(stream, 0), b)) * 0.02f));
        memcpy(blk, &s, 4);
        for (int k = 0; k < 8; k++) {
            uint64_t r = or_rng(seed, SUB(stream, 1), 8 * b + (uint64_t)k);
            for (int j = 0; j < 4; j++) {
                uint32_t u = (uint32_t)((r >> (16 * j)) & 0xffff);
                blk[4 + 4 * k + j] = (uint8_t)(int8_t)((int)(u % 255u) - 127);
            }
        }
    }
}

void or_synth_q6_k(uint8_t *out, size_t rows, size_t cols, uint64_t seed, uint64_t stream)
{
    size_t nblk = rows * (cols / 256);
    for (size_t b = 0; b < nblk; b++) {
        uint8_t *blk = out + b * OR_Q6_K_BYTES;
        for (int k = 0; k < 16; k++) {
            uint64_t r = or_rng(seed, SUB(stream, 0), 16 * b + (uint64_t)k);
            for (int j = 0; j < 8; j++) blk[8 * k + j] = (uint8_t)(r >> (8 * j));
        }
        for (int k = 0; k < 8; k++) {
            uint64_t r = or_rng(seed, SUB(stream, 1), 8 * b + (uint64_t)k);
            for (int j = 0; j < 8; j++) blk[128 + 8 * k + j] = (uint8_t)(r >> (8 * j));
        }
        for (int k = 0; k < 2; k++) {
            uint64_t r = or_rng(seed, SUB(stream, 2), 2 * b + (uint64_t)k);
            for (int j = 0; j < 8; j++) blk[192 + 8 * k + j] = (uint8_t)(r >> (8 * j));
        }
        uint16_t d = or_f32_to_f16(fabsf(or_normal(seed, SUB(stream, 3), b)) * 0.01f);
        blk[208] = (uint8_t)d;
        blk[209] = (uint8_t)(d >> 8);
    }
}

void or_synth_normal(float *out, size_t n, float sigma, uint64_t seed, uint64_t stream)
{
    for (size_t i = 0; i < n; i++) out[i] = or_normal(seed, stream, i) * sigma;
}

double or_now_seconds(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* ---------------------------------------------------------------------------
 * Host DRAM read bandwidth (STREAM-like "sum" kernel), the CPU roofline the
 * baseline is read against: `threads` contiguous strips of `a`, each summed
 * with four independent accumulators.  Returns the sum so nothing is elided.
 * ------------------------------------------------------------------------- */
typedef struct {
    const float *a;
    size_t s, e;
    double sum;
} read_job;

static void *read_thread(void *p)
{
    read_job *j = (read_job *)p;
    j->sum = or_sum_f32_avx2(j->a + j->s, j->e - j->s);
    return NULL;
}

double or_stream_read(const float *a, size_t n, int threads)
{
    if (threads < 1) threads = 1;
    read_job *jobs = (read_job *)calloc((size_t)threads, sizeof(read_job));
    pthread_t *tid = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
    double sum = 0.0;
    if (!jobs || !tid) {
        free(jobs);
        free(tid);
        return 0.0;
    }
    for (int i = 0; i < threads; i++) {
        jobs[i].a = a;
        row_strip(n, (size_t)i, (size_t)threads, &jobs[i].s, &jobs[i].e);
    }
    for (int i = 1; i < threads; i++) pthread_create(&tid[i], NULL, read_thread, &jobs[i]);
    read_thread(&jobs[0]);
    for (int i = 1; i < threads; i++) pthread_join(tid[i], NULL);
    for (int i = 0; i < threads; i++) sum += jobs[i].sum;
    free(jobs);
    free(tid);
    return sum;
}
