/* Llama / Qwen2 forward and scoring oracle (test infrastructure only; see oracle.h). */
#ifndef FERRUM_ORACLE_LLAMA_H
#define FERRUM_ORACLE_LLAMA_H

#include "oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Tensors per block in the reference's Block order (ferrum_ref/src/models/llama/mod.rs:99-128):
 * attn_norm wq bq wk bk wv bv wo ffn_norm gate up down. Matrices are [in, out]; a bias pointer
 * is NULL when the model has none. */
#define FO_LLAMA_BLOCK_TENSORS 12

typedef struct {
    size_t vocab, ctx, dim, heads, kv_heads, head_dim, layers, hidden, rope_dim;
    float rope_base, eps;
    int neox;                    /* RopeType::Neox (qwen2) when nonzero, else Norm (llama) */
    const float *freq_factors;   /* rope_dim / 2 divisors, or NULL (RopeScaling::freq_factors) */
    float linear_factor;         /* RopeScaling::linear_factor */
    const float *tok;            /* [vocab, dim] */
    const float *const *blocks;  /* layers * FO_LLAMA_BLOCK_TENSORS pointers */
    const float *out_norm;       /* [dim] */
    const float *head;           /* [dim, vocab] */
} fo_llama;

void fo_rope_tables(size_t start, size_t n, size_t rope_dim, float base, const float *freq_factors,
                    float linear_factor, float *cos_out, float *sin_out);
void fo_rmsnorm(const float *x, const float *g, size_t rows, size_t cols, float eps, float *y);
void fo_apply_rope(float *x, size_t rows, size_t heads, size_t hd, size_t rope_dim, const float *cos_t,
                   const float *sin_t, int neox);
void fo_attend_row(const float *q, const float *k, const float *v, size_t len, size_t heads, size_t kv_heads,
                   size_t hd, float *scratch, float *out);
float fo_silu(float x);
void fo_swiglu(const float *gate, const float *up, size_t n, float *out);
void fo_score(const float *logits, const size_t *targets, size_t rows, size_t vocab, float *logprob,
              uint8_t *is_first_max);
int fo_llama_forward(const fo_llama *m, const size_t *ids, size_t n, int threads, float *logits);

#ifdef __cplusplus
}
#endif
#endif
