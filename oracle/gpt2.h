/* GPT-2 decode oracle (test infrastructure only; see oracle.h). */
#ifndef FERRUM_ORACLE_GPT2_H
#define FERRUM_ORACLE_GPT2_H

#include "oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Tensors per block in the reference's canonical order (ferrum_ref/src/models/gpt2/mod.rs:57-90):
 * ln1_g ln1_b wq bq wk bk wv bv wo bo ln2_g ln2_b w1 b1 w2 b2. Matrices are [in, out]. */
#define FO_GPT2_BLOCK_TENSORS 16

typedef struct {
    size_t vocab, ctx, dim, heads, layers, hidden;
    const float *tok;            /* [vocab, dim] */
    const float *pos;            /* [ctx, dim] */
    const float *const *blocks;  /* layers * FO_GPT2_BLOCK_TENSORS pointers */
    const float *lnf_g, *lnf_b;  /* [dim] */
    const float *head;           /* [dim, vocab] */
} fo_gpt2;

typedef struct fo_gpt2_cache fo_gpt2_cache;

float fo_gelu(float x);
void fo_layernorm(const float *x, const float *g, const float *b, size_t cols, float *y);
size_t fo_argmax(const float *v, size_t n);
fo_gpt2_cache *fo_gpt2_cache_new(const fo_gpt2 *m);
void fo_gpt2_cache_free(const fo_gpt2 *m, fo_gpt2_cache *c);
int fo_gpt2_feed(const fo_gpt2 *m, fo_gpt2_cache *cache, size_t token, float *logits);
int fo_gpt2_generate(const fo_gpt2 *m, const size_t *prompt, size_t n_prompt, size_t n_new,
                     size_t *out);

#ifdef __cplusplus
}
#endif
#endif
