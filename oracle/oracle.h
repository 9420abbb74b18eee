/*
 * oracle.h -- CPU restatement of soso-llm-core's quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product (soso_amd/libsoso_hip.so) neither links nor calls it.
 *
 * Every function restates one reference function and cites it as
 * path:line inside demonodojo/soso.  Scalar code is compiled with
 * -ffp-contract=off so that a*b-c stays two roundings, as in Rust (which never
 * contracts).  The AVX2 restatements (oracle_avx2.c) use the same intrinsics
 * the Rust kernels use, so their summation order and FMA use match.
 *
 * Pinning (what checks each function, beyond retyping its formula):
 *   f16 decode / encode    -- reference unit cases (f16.rs:39-73), all 65536
 *                             bit patterns against the reference's own C twin
 *                             (lxdde/ports/nouveau/q4k_decode.h, built into
 *                             oracle/_ref by oracle/Makefile), and the
 *                             IEEE closed form of every half value.
 *   row_bytes              -- reference cases (quant.rs:409-420).
 *   Q4_K scale/min, dot    -- golden table and dot -15.875
 *                             (sosomodel/tests/dequant_golden.rs:18-93), the
 *                             reference C twin on random blocks, known
 *                             positions (quant.rs:433-449), pack round trip.
 *   Q8_0 dequant / dot     -- golden dot 172.59375 (dequant_golden.rs:95-114).
 *   Q6_K dequant           -- known answer all -1.0 (gguf2som/src/lib.rs:
 *                             1868-1889) plus an independent bit-field
 *                             decode written from GGML's published layout in
 *                             tests/test_oracle_golden.py.
 *   matvecs                -- f64 brute force, dequant-then-dot, AVX2 vs
 *                             scalar tolerance (gemm.rs:1204-1209).
 *   topk / softmax         -- sum-to-one and tie invariants (tests/moe.rs:146-153).
 *   argmax                 -- last-maximum-wins rule (runtime.rs:2021-2028).
 *   libm-dependent pieces  -- expf/powf/sinf/cosf are glibc here and Rust's
 *                             libm 0.2.16 in the reference: parity unpinned at
 *                             the ulp level (tolerance only).
 */
#ifndef SOSO_ORACLE_H
#define SOSO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: crates/sosomodel/src/layout.rs:8-12; 13 = Q6_K is an
 * extension of this build (soso re-quantizes Q6_K to Q8_0 at import). */
#define OR_DTYPE_F32 1
#define OR_DTYPE_Q8_0 2
#define OR_DTYPE_Q4_K 3
#define OR_DTYPE_MXFP4 4
#define OR_DTYPE_Q4_0 5
#define OR_DTYPE_Q6_K 13

#define OR_Q8_0_ELEMS 32
#define OR_Q8_0_BYTES 36
#define OR_Q4_K_ELEMS 256
#define OR_Q4_K_BYTES 144
#define OR_Q6_K_ELEMS 256
#define OR_Q6_K_BYTES 210

/* ---- f16 ---------------------------------------------------------------- */
float or_f16_to_f32(uint16_t bits);
uint16_t or_f32_to_f16(float v);
void or_f32_to_f16_n(const float *v, size_t n, uint16_t *out);

/* ---- layout ------------------------------------------------------------- */
int64_t or_row_bytes(uint8_t dtype, size_t cols); /* -1 = None */

/* ---- dequant (0 = Ok, -1 = Err) ----------------------------------------- */
int or_dequant_q8_0_range(const uint8_t *bytes, size_t nbytes, size_t elem_off, float *out, size_t n);
int or_dequant_q4_k_range(const uint8_t *bytes, size_t nbytes, size_t elem_off, float *out, size_t n);
int or_dequant_q6_k(const uint8_t *bytes, size_t nbytes, float *out, size_t n);
void or_q4k_scale_min(const uint8_t *scales, int j, uint8_t *sc, uint8_t *m);
void or_q4k_pack_scales(const uint8_t *sc8, const uint8_t *m8, uint8_t *out12);
float or_q4k_dot_sub(const uint8_t *blk, size_t blk_len, int j, const float *x, size_t x_len);
float or_q4k_dot_ref(const uint8_t *blk, const float *x);
int or_matvec_row(uint8_t dtype, const uint8_t *row, size_t row_len, size_t cols, const float *x, float *out);

/* ---- quantizers (quant.rs) ---------------------------------------------- */
size_t or_quantize_q8_0(const float *src, size_t n, uint8_t *out);
size_t or_quantize_q4_k(const float *src, size_t n, uint8_t *out);

/* ---- scalar matvecs ----------------------------------------------------- */
void or_matvec_f32_scalar(const float *w, size_t rows, size_t cols, const float *x, float *out);
void or_matvec_q8_0_scalar(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out);
void or_matvec_q4_k_scalar(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out);
void or_matvec_q6_k_scalar(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out);
/* dequantize each row exactly, accumulate the dot in f64 */
int or_matvec_f64(uint8_t dtype, const uint8_t *w, size_t rows, size_t cols, const float *x, double *out);

/* ---- AVX2+FMA matvecs (oracle_avx2.c) ----------------------------------- */
int or_have_avx2(void);
void or_matvec_f32_avx2(const float *w, size_t rows, size_t cols, const float *x, float *out);
void or_matvec_q8_0_avx2(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out);
void or_matvec_q4_k_avx2(const uint8_t *w, size_t rows, size_t cols, const float *x, float *out);
void or_swiglu_avx2(float *up, const float *gate, size_t n);

/* matvec_view_par: dtype dispatch + contiguous row strips over `threads`
 * threads.  avx2 != 0 selects the AVX2 kernels (the production CPU path).
 * Returns 0, or -1 on a shape/dtype error. */
int or_matvec_par(uint8_t dtype, const uint8_t *w, size_t rows, size_t cols, const float *x, float *out,
                  int threads, int avx2);
/* n vectors (xs: n*cols) against one matrix, outs: n*rows (bit-identical to n single calls) */
int or_matmul_par(uint8_t dtype, const uint8_t *w, size_t rows, size_t cols, size_t n, const float *xs,
                  float *outs, int threads, int avx2);

/* ---- elementwise / small ops -------------------------------------------- */
void or_softmax(float *x, size_t n);
size_t or_topk_softmax(float *logits, size_t n, size_t k, int32_t *idx, float *w);
float or_silu(float x);
void or_swiglu(float *up, const float *gate, size_t n);
void or_rmsnorm(float *x, const float *w, size_t n, float eps);
void or_rope_heads(float *x, size_t n_heads, size_t head_dim, size_t pos, float theta, int neox);
uint32_t or_argmax(const float *x, size_t n);
void or_attention_f32(const float *q, const float *k_cache, const float *v_cache, size_t head_dim,
                      size_t kv_dim, size_t kv_head, size_t n_tokens, float *out);

/* ---- MoE FFN for one token ------------------------------------------------
 * router (n_exp x h f32) -> topk_softmax -> per expert gate/up (ffn x h),
 * swiglu, down (h x ffn) -> out = sum_j w_j * down_j in ranking order.
 * Expert weights are given as arrays of pointers (dtype Q4_K or Q8_0). */
int or_attention_heads_par(const float *q, const float *k, const float *v, size_t hd, size_t n_heads,
                           size_t n_kv_heads, size_t T, float *out, int threads);
int or_decode_layer(float *h, const void *const *w, uint8_t dtype, size_t hidden, size_t n_heads, size_t n_kv_heads,
                    size_t hd, size_t ffn, float *kcache, float *vcache, size_t pos, float theta, float eps,
                    int threads, int avx2);
int or_moe_ffn(const float *router, size_t n_exp, size_t h, size_t ffn, size_t top_k,
               const uint8_t *const *gate, const uint8_t *const *up, const uint8_t *const *down,
               uint8_t dtype_gu, uint8_t dtype_down, const float *x, float *out, int32_t *idx_out,
               float *w_out, int threads, int avx2);

/* ---- shared expert of an MoE block (GpuDispatch::moe_compartido) ---------- */
int or_moe_shared(const float *pg_w, size_t h, size_t ffn, const uint8_t *gate, const uint8_t *up,
                  const uint8_t *down, uint8_t dtype_gu, uint8_t dtype_down, const float *xs, size_t n, float *out);

/* ---- Gated DeltaNet (GpuDispatch::gdn_bloque) ------------------------------ */
float or_sigmoid(float x);
float or_softplus(float x);
void or_l2_normalize(float *x, size_t n, float eps);
void or_gdn_step(float *state, const float *q, const float *k, const float *v, size_t d, float g, float beta,
                 float *out);
void or_gdn_gates(const float *alpha, const float *beta_raw, const float *dt, const float *a, size_t n, size_t n_v,
                  float *decay, float *beta);
int or_gdn_block(const float *hist, const float *conv, const float *z, const float *decay, const float *beta,
                 const float *norm, float *state, float *out, size_t n, size_t n_k, size_t n_v, size_t d,
                 size_t kernel, float eps);

/* ---- synthetic, counter-based generators ---------------------------------- */
uint64_t or_rng(uint64_t seed, uint64_t stream, uint64_t i);
float or_normal(uint64_t seed, uint64_t stream, uint64_t i);
void or_synth_q4_k(uint8_t *out, size_t rows, size_t cols, uint64_t seed, uint64_t stream);
void or_synth_q8_0(uint8_t *out, size_t rows, size_t cols, uint64_t seed, uint64_t stream);
void or_synth_q6_k(uint8_t *out, size_t rows, size_t cols, uint64_t seed, uint64_t stream);
void or_synth_normal(float *out, size_t n, float sigma, uint64_t seed, uint64_t stream);

/* ---- timing helper for the CPU baseline ---------------------------------- */
double or_now_seconds(void);
/* Sum of n floats with four 8-wide AVX2 accumulators (scalar without AVX2). */
double or_sum_f32_avx2(const float *a, size_t n);
/* STREAM-like threaded read of n floats (host DRAM roofline); returns the sum. */
double or_stream_read(const float *a, size_t n, int threads);

#ifdef __cplusplus
}
#endif
#endif
