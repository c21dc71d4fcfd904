/* CPU oracle for the quantized-weight path: a plain C restatement of the reference's codec,
 * matmul, GEMV, fake-quant snap and tolerance functions.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links or calls this code; only the
 * tests, the smoke check and the bench's cpu_baseline leg load it, and only as the checker (or,
 * for the bench, as the timed CPU baseline). Build: oracle/Makefile (gcc -O3 -ffp-contract=off).
 *
 * Every function names the reference file:line it follows (paths relative to the reference
 * repository root). Floating-point semantics follow Rust's: no FMA contraction (hence
 * -ffp-contract=off), round-half-away for f32::round, saturating float->int casts (NaN -> 0).
 */
#ifndef FERRUM_ORACLE_H
#define FERRUM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (ferrum_gguf/src/lib.rs:23,25,43,55). */
#define FO_F32 0u
#define FO_F16 1u
#define FO_Q4_0 2u
#define FO_Q8_0 8u
#define FO_QK 32u

/* ferrum_gguf/src/codec/f16.rs:4-22 */
float fo_f16_to_f32(uint16_t h);
/* ferrum_gguf/src/codec/f16.rs:25-53 */
uint16_t fo_f32_to_f16(float x);

/* ferrum_gguf/src/codec/quant.rs:17-47. Bytes for n elements of type ty, or -1 when ty is not
 * one of F32/F16/Q8_0/Q4_0 or n is not whole blocks. */
int64_t fo_nbytes(uint32_t ty, size_t n);

/* ferrum_gguf/src/codec/quant.rs:50-88. Decode n elements; 0 on success, -1 on a length or
 * type error. */
int fo_decode(uint32_t ty, const uint8_t *bytes, size_t len, size_t n, float *out);

/* ferrum_gguf/src/codec/quant.rs:91-136. Encode n elements into fo_nbytes(ty, n) bytes. */
int fo_encode(uint32_t ty, const float *data, size_t n, uint8_t *out);

/* ferrum_ref/src/models/llama/params.rs:24-32: out[c*rows + r] = data[r*cols + c]. */
void fo_transpose(const float *data, size_t rows, size_t cols, float *out);

/* ferrum_wgpu/src/ops/quant.rs:238-252: [k, n] (in, out) row-major f32 -> transpose -> encode,
 * giving GGUF rows [n][k/32 blocks]. 0 on success, -1 when k is not whole blocks. */
int fo_quantise_matrix(uint32_t ty, const float *w, size_t k, size_t n, uint8_t *out);

/* ferrum_ref/src/training/qat.rs:20-24: decode(encode(block)) for one block of 32. */
void fo_snap_block(const float *in, float *out);
/* ferrum_ref/src/training/qat.rs:27-35: in place, blocks of 32 consecutive values; a no-op
 * when ne0 is not a positive multiple of 32. The trailing partial block (len % 32) is left
 * as is (chunks_exact). */
void fo_snap_rows(float *data, size_t len, size_t ne0);
/* ferrum_ref/src/training/qat.rs:38-54: blocks run down the columns of [rows_in, cols_out]. */
void fo_snap_cols(float *data, size_t rows_in, size_t cols_out);

/* ferrum_ref/src/kernels/matmul.rs:49-69 (i-k-j, ascending k, separate mul and add). */
int fo_matmul(const float *a, const float *b, size_t m, size_t k, size_t n, float *out);
/* ferrum_ref/src/kernels/matmul.rs:73-94: the same rows split over threads (bit-identical). */
int fo_matmul_threaded(const float *a, const float *b, size_t m, size_t k, size_t n,
                       int threads, float *out);
/* ferrum_ref/src/kernels/tuned.rs:10-134: KC = NC = 256 panels, 4x8 register tile, rows split
 * over threads; ascending k per element, so bit-identical to fo_matmul. */
int fo_matmul_tuned(const float *a, const float *b, size_t m, size_t k, size_t n, int threads,
                    float *out);

/* ferrum_ref/src/models/gpt2/decode.rs:42-53: y = x * w (+ bias) for one row, w [k, n]. */
void fo_gemv(const float *x, const float *w, const float *bias, size_t k, size_t n, float *y);

/* ferrum_ref/src/kernels/matmul.rs:97-107: xorshift64 values in [-1, 1). */
void fo_rand_vec(size_t len, uint64_t seed, float *out);

/* ferrum_ref/src/kernels/rng.rs:5-41: xorshift64* generator. */
typedef struct { uint64_t s; } fo_rng;
void fo_rng_init(fo_rng *r, uint64_t seed);
uint64_t fo_rng_next_u64(fo_rng *r);
float fo_rng_next_f32(fo_rng *r);
size_t fo_rng_below(fo_rng *r, size_t n);

/* ferrum_wgpu/src/tolerance.rs:14-26: max |g - w| / max(|w|, 1); +inf on NaN. */
float fo_max_rel_err(const float *got, const float *want, size_t n);

#ifdef __cplusplus
}
#endif
#endif
