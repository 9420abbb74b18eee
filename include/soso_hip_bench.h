/*
 * soso_hip_bench.h -- bench and test support of libsoso_hip.so.
 *
 * None of these has a counterpart in soso's GpuDispatch trait: they generate
 * seeded synthetic inputs directly in device memory (so benchmarks and GPU
 * tests need no host copies of multi-GB tensors) and measure the plain
 * streaming-read bandwidth the matvec kernels are held against.  A Rust
 * `impl GpuDispatch` binds only include/soso_hip.h.
 */
#ifndef SOSO_HIP_BENCH_H
#define SOSO_HIP_BENCH_H

#include "soso_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Fills a new resident weight with seeded synthetic blocks (same bytes as the
 * documented counter-based generator that the CPU oracle also implements). */
int soso_hip_weight_synth(soso_hip *h, const char *key, size_t key_len, uint8_t dtype, size_t rows,
                          size_t cols, uint64_t seed, uint64_t stream);
/* Writes the synthetic raw (soso/GGML layout) bytes of a tensor to device memory. */
int soso_hip_synth_raw(soso_hip *h, void *dst_dev, uint8_t dtype, size_t rows, size_t cols, uint64_t seed,
                       uint64_t stream);
/* n f32 values ~ N(0,1)*sigma (Irwin-Hall(12) normals of the same generator). */
int soso_hip_synth_normal(soso_hip *h, float *dst_dev, size_t n, float sigma, uint64_t seed,
                          uint64_t stream);
/* A plain streaming read of `bytes` from src_dev: wg_per_cu (1..32)
 * workgroups per CU of `threads` (a multiple of 64, <= 1024).  chunked = 0:
 * grid-stride over 16-byte words (bytes rounded down to 16), `loads`
 * (1, 2, 4, 8 or 16) independent loads in flight per thread.  chunked = 1:
 * every wavefront streams its own contiguous stretch of whole KiB (bytes
 * rounded down to 1 KiB, < 2 GiB) with `loads` 1-KiB wavefront loads in
 * flight, through raw buffer loads as the matvec kernels issue them.
 * chunked | 2: the same with the loads' nontemporal (streaming) cache policy,
 * as the matvec's weight loads use.  Thread t < out_len writes the xor of
 * what it read to out_dev[t].  Asynchronous on the handle's stream. */
int soso_hip_read_probe(soso_hip *h, const void *src_dev, size_t bytes, uint32_t wg_per_cu, uint32_t threads,
                        uint32_t loads, uint32_t chunked, uint32_t *out_dev, size_t out_len);

#ifdef __cplusplus
}
#endif
#endif
