/*
 * oracle_avx2.c -- AVX2+FMA restatement of soso-llm-core's production CPU
 * kernels (the guest target enables +avx2,+fma, user/x86_64-soso-user.json:7).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the CPU baseline that bench.py
 * times beside the GPU, and a second oracle checked against the scalar one.
 * Same intrinsics, same order of operations as the Rust `avx2` module.
 */
#include "oracle.h"

#include <immintrin.h>
#include <string.h>

int or_have_avx2(void) { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }

/* crates/soso-llm-core/src/gemm.rs:693-702 (`hsum`). */
static inline float hsum(__m256 v)
{
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

/* gemm.rs:766-802 (`avx2::matvec_f32`): two 8-lane FMA accumulators over 16
 * columns, an 8-column tail, then a scalar tail after the horizontal sum. */
void or_matvec_f32_avx2(const float *w, size_t rows, size_t cols, const float *x, float *out)
{
    for (size_t r = 0; r < rows; r++) {
        const float *row = w + r * cols;
        __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
        size_t c = 0;
        for (; c + 16 <= cols; c += 16) {
            acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(row + c), _mm256_loadu_ps(x + c), acc0);
            acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(row + c + 8), _mm256_loadu_ps(x + c + 8), acc1);
        }
        for (; c + 8 <= cols; c += 8) acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(row + c), _mm256_loadu_ps(x + c), acc0);
        float s = hsum(_mm256_add_ps(acc0, acc1));
        for (; c < cols; c++) s += row[c] * x[c];
        out[r] = s;
    }
}

/* gemm.rs:806-836 (`avx2::matvec_q8_0`): per block, 4 FMAs of 8 lanes into a
 * block accumulator, then acc = fma(scale, blk, acc); one hsum per row. */
void or_matvec_q8_0_avx2(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out)
{
    size_t nb = cols / 32, rb = nb * OR_Q8_0_BYTES;
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = w + r * rb;
        __m256 acc = _mm256_setzero_ps();
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *c = row + b * OR_Q8_0_BYTES;
            float sf;
            memcpy(&sf, c, 4);
            __m256 scale = _mm256_set1_ps(sf);
            const uint8_t *q = c + 4;
            const float *xb = x + b * 32;
            __m256 blk = _mm256_setzero_ps();
            for (int g = 0; g < 4; g++) {
                __m128i qi = _mm_loadl_epi64((const __m128i *)(q + g * 8));
                __m256 qf = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(qi));
                blk = _mm256_fmadd_ps(qf, _mm256_loadu_ps(xb + g * 8), blk);
            }
            acc = _mm256_fmadd_ps(scale, blk, acc);
        }
        out[r] = hsum(acc);
    }
}

/* gemm.rs:842-894 (`avx2::matvec_q4_k`): per element
 * coef = fma(q, d*sc, -(dmin*m)), acc = fma(coef, x, acc), lower nibbles
 * (first 32 elements of the pair) then upper nibbles, 8 lanes at a time. */
void or_matvec_q4_k_avx2(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out)
{
    size_t nb = cols / 256, rb = nb * OR_Q4_K_BYTES;
    const __m256i mask = _mm256_set1_epi8(0x0F);
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = w + r * rb;
        __m256 acc = _mm256_setzero_ps();
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * OR_Q4_K_BYTES;
            float d = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            float dmin = or_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
            const uint8_t *scales = blk + 4;
            for (int pair = 0; pair < 4; pair++) {
                uint8_t sc1, m1, sc2, m2;
                or_q4k_scale_min(scales, 2 * pair, &sc1, &m1);
                or_q4k_scale_min(scales, 2 * pair + 1, &sc2, &m2);
                __m256 dsc[2] = {_mm256_set1_ps(d * (float)sc1), _mm256_set1_ps(d * (float)sc2)};
                __m256 dm[2] = {_mm256_set1_ps(-(dmin * (float)m1)), _mm256_set1_ps(-(dmin * (float)m2))};
                __m256i qv = _mm256_loadu_si256((const __m256i *)(blk + 16 + pair * 32));
                __m256i nib[2] = {_mm256_and_si256(qv, mask), _mm256_and_si256(_mm256_srli_epi16(qv, 4), mask)};
                const float *xb = x + b * 256 + pair * 64;
                for (int hsel = 0; hsel < 2; hsel++) {
                    __m128i l0 = _mm256_castsi256_si128(nib[hsel]);
                    __m128i l1 = _mm256_extracti128_si256(nib[hsel], 1);
                    __m128i quads[4] = {l0, _mm_srli_si128(l0, 8), l1, _mm_srli_si128(l1, 8)};
                    for (int g = 0; g < 4; g++) {
                        __m256 qf = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(quads[g]));
                        __m256 coef = _mm256_fmadd_ps(qf, dsc[hsel], dm[hsel]);
                        __m256 xv = _mm256_loadu_ps(xb + hsel * 32 + g * 8);
                        acc = _mm256_fmadd_ps(coef, xv, acc);
                    }
                }
            }
        }
        out[r] = hsum(acc);
    }
}

/* crates/soso-llm-core/src/simd_math.rs:13-35 (`exp256`): clamp to
 * [-87, 88], round(x*log2e), two-step ln2 reduction, degree-7 Taylor Horner,
 * scale by 2^n through the exponent field. */
static inline __m256 exp256(__m256 x)
{
    x = _mm256_min_ps(_mm256_max_ps(x, _mm256_set1_ps(-87.0f)), _mm256_set1_ps(88.0f));
    __m256 fx = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896340736f)),
                                _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 r = _mm256_fmadd_ps(fx, _mm256_set1_ps(-0.69314575f), x);
    r = _mm256_fmadd_ps(fx, _mm256_set1_ps(-1.4286068e-6f), r);
    __m256 p = _mm256_set1_ps(1.0f / 5040.0f);
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 720.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 120.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 24.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 6.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
    __m256i n = _mm256_cvtps_epi32(fx);
    __m256 pot = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_add_epi32(n, _mm256_set1_epi32(127)), 23));
    return _mm256_mul_ps(p, pot);
}

/* simd_math.rs:38-45 (`silu256`). */
static inline __m256 silu256(__m256 x)
{
    __m256 e = exp256(_mm256_sub_ps(_mm256_setzero_ps(), x));
    return _mm256_div_ps(x, _mm256_add_ps(_mm256_set1_ps(1.0f), e));
}

/* simd_math.rs:48-70 (`swiglu`): the tail (< 8) goes through the same vector
 * arithmetic on a zero-padded copy. */
void or_swiglu_avx2(float *up, const float *gate, size_t n)
{
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 g = _mm256_loadu_ps(gate + i);
        __m256 u = _mm256_loadu_ps(up + i);
        _mm256_storeu_ps(up + i, _mm256_mul_ps(silu256(g), u));
    }
    if (i < n) {
        float g8[8] = {0}, u8[8] = {0}, t[8];
        size_t r = n - i;
        memcpy(g8, gate + i, r * 4);
        memcpy(u8, up + i, r * 4);
        _mm256_storeu_ps(t, _mm256_mul_ps(silu256(_mm256_loadu_ps(g8)), _mm256_loadu_ps(u8)));
        memcpy(up + i, t, r * 4);
    }
}

/* The read kernel of the host-bandwidth measurement (not part of soso's path):
 * four independent 8-wide accumulators so the loop is bound by memory, not by
 * the add latency. */
double or_sum_f32_avx2(const float *a, size_t n)
{
    __m256 s0 = _mm256_setzero_ps(), s1 = s0, s2 = s0, s3 = s0;
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        s0 = _mm256_add_ps(s0, _mm256_loadu_ps(a + i));
        s1 = _mm256_add_ps(s1, _mm256_loadu_ps(a + i + 8));
        s2 = _mm256_add_ps(s2, _mm256_loadu_ps(a + i + 16));
        s3 = _mm256_add_ps(s3, _mm256_loadu_ps(a + i + 24));
    }
    float t[8];
    _mm256_storeu_ps(t, _mm256_add_ps(_mm256_add_ps(s0, s1), _mm256_add_ps(s2, s3)));
    double sum = 0.0;
    for (int k = 0; k < 8; k++) sum += t[k];
    for (; i < n; i++) sum += a[i];
    return sum;
}
