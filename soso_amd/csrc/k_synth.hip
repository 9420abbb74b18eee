// k_synth.hip -- seeded synthetic tensors on the device (bench / test inputs).
//
// Counter-based SplitMix64 keyed by (seed, stream, index) and integer-only
// derived values, so the host generator used by the tests produces the very
// same bytes.  Normals are Irwin-Hall(12) sums of 16-bit uniforms, computed
// exactly: N = (S - 393210) / 65536 (mean 0, variance 1).  Half-precision
// scales use soso's f32->f16 rounding (ties up,
// crates/soso-llm-core/src/f16.rs:10-37).
#include "internal.hpp"

#include <type_traits>

__device__ __forceinline__ uint64_t fin64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t rng(uint64_t seed, uint64_t stream, uint64_t i)
{
    const uint64_t key = fin64(seed ^ fin64(stream + 0x9E3779B97F4A7C15ull));
    return fin64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

__device__ __forceinline__ float normal(uint64_t seed, uint64_t stream, uint64_t i)
{
    int32_t s = 0;
    for (int h = 0; h < 3; h++) {
        const uint64_t r = rng(seed, stream, 3 * i + (uint64_t)h);
        s += (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) + (int32_t)(r >> 48);
    }
    return __fmul_rn((float)(s - 393210), 1.0f / 65536.0f);
}

// f32_to_f16_soso (internal.hpp) rounds the f16 scales as soso's quantizers do.

#define SUB(s, f) (((s) << 4) | (uint64_t)(f))

__global__ void synth_q4k(uint8_t *out, long nblk, uint64_t seed, uint64_t st)
{
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    uint8_t *blk = out + b * Q4_K_BYTES;
    const uint16_t d = f32_to_f16_soso(__fmul_rn(fabsf(normal(seed, SUB(st, 0), b)), 0.01f));
    const uint16_t dm = f32_to_f16_soso(__fmul_rn(fabsf(normal(seed, SUB(st, 1), b)), 0.01f));
    uint32_t *w = (uint32_t *)blk; // 144-byte blocks: 4-byte aligned
    w[0] = (uint32_t)d | ((uint32_t)dm << 16);
    const uint64_t a = rng(seed, SUB(st, 2), 2 * b), c = rng(seed, SUB(st, 2), 2 * b + 1);
    uint8_t sc[8], m[8], s[12];
    for (int j = 0; j < 8; j++) {
        sc[j] = (uint8_t)((a >> (8 * j)) & 63);
        m[j] = (uint8_t)((c >> (8 * j)) & 63);
    }
    // crates/soso-llm-core/src/quant.rs:46-54 (q4k_pack_scales)
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0x0F) | ((m[j + 4] & 0x0F) << 4));
    }
    for (int j = 0; j < 3; j++) w[1 + j] = s[4 * j] | (s[4 * j + 1] << 8) | (s[4 * j + 2] << 16) | ((uint32_t)s[4 * j + 3] << 24);
    for (int k = 0; k < 16; k++) {
        const uint64_t r = rng(seed, SUB(st, 3), 16 * b + k);
        w[4 + 2 * k] = (uint32_t)r;
        w[5 + 2 * k] = (uint32_t)(r >> 32);
    }
}

__global__ void synth_q80(uint8_t *out, long nblk, uint64_t seed, uint64_t st)
{
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    uint32_t *w = (uint32_t *)(out + b * Q8_0_BYTES);
    const uint16_t hb = f32_to_f16_soso(__fmul_rn(fabsf(normal(seed, SUB(st, 0), b)), 0.02f));
    w[0] = __builtin_bit_cast(uint32_t, half_bits_to_f32(hb)); // finite by construction
    for (int k = 0; k < 8; k++) {
        const uint64_t r = rng(seed, SUB(st, 1), 8 * b + k);
        uint32_t v = 0;
        for (int j = 0; j < 4; j++) {
            const uint32_t u = (uint32_t)((r >> (16 * j)) & 0xffff);
            v |= (uint32_t)(uint8_t)(int8_t)((int)(u % 255u) - 127) << (8 * j);
        }
        w[1 + k] = v;
    }
}

__global__ void synth_q6k(uint8_t *out, long nblk, uint64_t seed, uint64_t st)
{
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    uint16_t *w = (uint16_t *)(out + b * Q6_K_BYTES); // 210-byte blocks: 2-byte aligned
    for (int k = 0; k < 16; k++) {
        const uint64_t r = rng(seed, SUB(st, 0), 16 * b + k);
        for (int j = 0; j < 4; j++) w[4 * k + j] = (uint16_t)(r >> (16 * j));
    }
    for (int k = 0; k < 8; k++) {
        const uint64_t r = rng(seed, SUB(st, 1), 8 * b + k);
        for (int j = 0; j < 4; j++) w[64 + 4 * k + j] = (uint16_t)(r >> (16 * j));
    }
    for (int k = 0; k < 2; k++) {
        const uint64_t r = rng(seed, SUB(st, 2), 2 * b + k);
        for (int j = 0; j < 4; j++) w[96 + 4 * k + j] = (uint16_t)(r >> (16 * j));
    }
    w[104] = f32_to_f16_soso(__fmul_rn(fabsf(normal(seed, SUB(st, 3), b)), 0.01f));
}

__global__ void synth_normal_k(float *out, long n, float sigma, uint64_t seed, uint64_t st)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __fmul_rn(normal(seed, st, i), sigma);
}

int launch_synth_raw(soso_hip *h, void *dst, uint8_t dtype, size_t rows, size_t cols, uint64_t seed, uint64_t stream)
{
    const int T = 256;
    long nblk;
    switch (dtype) {
    case SOSO_HIP_DTYPE_Q4_K:
        if (cols % 256) return set_err(h, SOSO_HIP_ERR_ARG, "synth: cols");
        nblk = (long)(rows * (cols / 256));
        synth_q4k<<<(unsigned)((nblk + T - 1) / T), T, 0, h->stream>>>((uint8_t *)dst, nblk, seed, stream);
        break;
    case SOSO_HIP_DTYPE_Q8_0:
        if (cols % 32) return set_err(h, SOSO_HIP_ERR_ARG, "synth: cols");
        nblk = (long)(rows * (cols / 32));
        synth_q80<<<(unsigned)((nblk + T - 1) / T), T, 0, h->stream>>>((uint8_t *)dst, nblk, seed, stream);
        break;
    case SOSO_HIP_DTYPE_Q6_K:
        if (cols % 256) return set_err(h, SOSO_HIP_ERR_ARG, "synth: cols");
        nblk = (long)(rows * (cols / 256));
        synth_q6k<<<(unsigned)((nblk + T - 1) / T), T, 0, h->stream>>>((uint8_t *)dst, nblk, seed, stream);
        break;
    case SOSO_HIP_DTYPE_F32:
        return launch_synth_normal(h, (float *)dst, rows * cols, 1.0f, seed, stream);
    default: return set_err(h, SOSO_HIP_ERR_ARG, "synth: dtype");
    }
    return hip_check(h, hipGetLastError(), "synth launch");
}

int launch_synth_normal(soso_hip *h, float *dst, size_t n, float sigma, uint64_t seed, uint64_t stream)
{
    const int T = 256;
    synth_normal_k<<<(unsigned)((n + T - 1) / T), T, 0, h->stream>>>(dst, (long)n, sigma, seed, stream);
    return hip_check(h, hipGetLastError(), "synth normal launch");
}

// ---------------------------------------------------------------------------
// Plain streaming reads: the bandwidth reference the matvec kernels are held
// against (bench.py --only readprobe sweeps every variant and launch shape).
// Each thread xors what it read into out[thread] (threads past out_len keep
// theirs: the store is conditional at run time, so no load is dead).
//  - read_probe_gs<K>: grid-stride over 16-byte words, K independent loads
//    issued per thread before any is used;
//  - read_probe_chunk<K>: each wavefront streams its own contiguous stretch
//    of whole KiB, K 1-KiB wavefront loads in flight (raw buffer loads, as
//    the matvec kernels use; a load past the stretch returns zeros without
//    touching memory).
// ---------------------------------------------------------------------------
template <int K, bool NT>
__global__ void read_probe_gs(const uint4 *__restrict__ p, size_t n16, uint32_t *__restrict__ out, size_t out_len)
{
    const size_t T = (size_t)gridDim.x * blockDim.x, t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    size_t i = t;
    for (; i + (size_t)(K - 1) * T < n16; i += (size_t)K * T) {
        uint4 v[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            if constexpr (NT) {
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const u32x4 t4 = __builtin_nontemporal_load((const u32x4 *)(p + i + (size_t)k * T));
                v[k] = make_uint4(t4.x, t4.y, t4.z, t4.w);
            } else {
                v[k] = p[i + (size_t)k * T];
            }
        }
#pragma unroll
        for (int k = 0; k < K; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < n16; i += T) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (t < out_len) out[t] = acc;
}

template <int K, bool NT>
__global__ void read_probe_chunk(const uint8_t *__restrict__ p, uint32_t kib, uint32_t *__restrict__ out,
                                 size_t out_len)
{
    const int lane = threadIdx.x & 63;
    const uint32_t nw = gridDim.x * (blockDim.x >> 6);
    const uint32_t w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t c0 = (uint32_t)((uint64_t)kib * w / nw), c1 = (uint32_t)((uint64_t)kib * (w + 1) / nw);
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p) + (size_t)c0 * 1024,
                                                                       (short)0, (int)((c1 - c0) * 1024), 0x00020000);
    uint32_t acc = 0;
    for (uint32_t j = 0; j < c1 - c0; j += K) {
        uint4 v[K];
#pragma unroll
        for (int k = 0; k < K; k++)
            v[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)((j + k) * 1024u + 16u * lane),
                                                                                   0, NT ? 2 : 0));
#pragma unroll
        for (int k = 0; k < K; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < out_len) out[t] = acc;
}

int launch_read_probe(soso_hip *h, const void *src, size_t bytes, unsigned wg_per_cu, unsigned threads,
                      unsigned loads, bool chunked, bool stream, uint32_t *out, size_t out_len)
{
    const unsigned grid = wg_per_cu * (unsigned)h->num_cu;
    if (loads != 1 && loads != 2 && loads != 4 && loads != 8 && loads != 16)
        return set_err(h, SOSO_HIP_ERR_ARG, "read_probe: loads");
    auto go = [&](auto nt) {
        constexpr bool NT = decltype(nt)::value;
        if (chunked) {
            const uint32_t kib = (uint32_t)(bytes >> 10);
            const uint8_t *b = (const uint8_t *)src;
            switch (loads) {
            case 1: read_probe_chunk<1, NT><<<grid, threads, 0, h->stream>>>(b, kib, out, out_len); break;
            case 2: read_probe_chunk<2, NT><<<grid, threads, 0, h->stream>>>(b, kib, out, out_len); break;
            case 4: read_probe_chunk<4, NT><<<grid, threads, 0, h->stream>>>(b, kib, out, out_len); break;
            case 8: read_probe_chunk<8, NT><<<grid, threads, 0, h->stream>>>(b, kib, out, out_len); break;
            default: read_probe_chunk<16, NT><<<grid, threads, 0, h->stream>>>(b, kib, out, out_len); break;
            }
        } else {
            const uint4 *q = (const uint4 *)src;
            const size_t n16 = bytes / 16;
            switch (loads) {
            case 1: read_probe_gs<1, NT><<<grid, threads, 0, h->stream>>>(q, n16, out, out_len); break;
            case 2: read_probe_gs<2, NT><<<grid, threads, 0, h->stream>>>(q, n16, out, out_len); break;
            case 4: read_probe_gs<4, NT><<<grid, threads, 0, h->stream>>>(q, n16, out, out_len); break;
            case 8: read_probe_gs<8, NT><<<grid, threads, 0, h->stream>>>(q, n16, out, out_len); break;
            default: read_probe_gs<16, NT><<<grid, threads, 0, h->stream>>>(q, n16, out, out_len); break;
            }
        }
    };
    if (stream) go(std::true_type{});
    else go(std::false_type{});
    return hip_check(h, hipGetLastError(), "read probe launch");
}
