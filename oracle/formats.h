/* Block formats beyond Q8_0 / Q4_0 (test infrastructure only; see oracle.h): FP8 E4M3 / E5M2,
 * MXFP4 and Q2_K (encode and decode) and the read-only GGUF block types (decode). */
#ifndef FERRUM_ORACLE_FORMATS_H
#define FERRUM_ORACLE_FORMATS_H

#include "oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (ferrum_gguf/src/lib.rs:33-53) */
#define FO_Q4_1 3u
#define FO_Q5_0 6u
#define FO_Q5_1 7u
#define FO_Q8_1 9u
#define FO_Q2_K 10u
#define FO_Q3_K 11u
#define FO_Q4_K 12u
#define FO_Q5_K 13u
#define FO_Q6_K 14u
#define FO_MXFP4 39u
#define FO_QK_K 256u
/* The FP8 weight formats have no ggml type (ferrum_wgpu/src/ops/quant.rs:38-41); these ids are
 * this build's own, outside the ggml range. */
#define FO_FP8_E4M3 1024u
#define FO_FP8_E5M2 1025u

/* ferrum_gguf/src/codec/blocks.rs:34-48 (plus the FP8 formats, laid out like Q8_0): bytes and
 * elements per block, 0 when the type is not one of these. */
int fo_layout(uint32_t ty, size_t *block_bytes, size_t *block_elems);
/* ferrum_gguf/src/codec/blocks.rs:55-73 and fp8.rs:116-124: decode whole blocks. */
int fo_dequant(uint32_t ty, const uint8_t *raw, size_t nblocks, float *out);

/* ferrum_gguf/src/codec/fp8.rs:34-96 (e5m2 = 0 for E4M3) */
float fo_fp8_decode(int e5m2, uint8_t code);
uint8_t fo_fp8_encode(int e5m2, float x);
/* ferrum_gguf/src/codec/fp8.rs:99-113 */
void fo_fp8_encode_blocks(int e5m2, const float *data, size_t nblocks, uint8_t *out);

/* ferrum_gguf/src/codec/mxfp4.rs:26-33 */
float fo_mxfp4_half_scale(uint8_t e);
/* ferrum_gguf/src/codec/mxfp4.rs:73-83 */
void fo_mxfp4_encode_blocks(const float *data, size_t nblocks, uint8_t *out);

/* ferrum_gguf/src/codec/q2k.rs:16-19 */
int32_t fo_q2k_nearest_int(float x);
/* ferrum_gguf/src/codec/q2k.rs:24-93: one 16-value sub-block's (scale, negated min) and levels */
void fo_q2k_fit(const float *x16, uint8_t *levels16, float *scale, float *neg_min);
/* ferrum_gguf/src/codec/q2k.rs:96-150 */
void fo_q2k_encode_blocks(const float *data, size_t nblocks, uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
