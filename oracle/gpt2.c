/* GPT-2 cached decode on the CPU (test infrastructure only; see oracle.h): the oracle the
 * device decode's token IDs are compared against. Restates ferrum_ref's Gpt2::feed
 * (ferrum_ref/src/models/gpt2/decode.rs:57-117) over the ops of ferrum_ref/src/kernels/nn.rs and
 * the greedy pick of ferrum_model/src/sampling.rs:32-40. Weights are f32 [in, out] row-major;
 * a Q8_0 model is its fake-quantised (snapped) f32 weights, which is what the reference's CPU
 * path computes on. */
#include "gpt2.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ferrum_ref/src/kernels/nn.rs:6 */
#define LN_EPS 1e-5f

/* ferrum_ref/src/kernels/nn.rs:12-15 */
float fo_gelu(float x) {
    const float K = 0.7978846f;
    return 0.5f * x * (1.0f + tanhf(K * (x + 0.044715f * x * x * x)));
}

/* ferrum_ref/src/kernels/nn.rs:31-44 (one row). */
void fo_layernorm(const float *x, const float *g, const float *b, size_t cols, float *y) {
    float sum = 0.0f;
    for (size_t c = 0; c < cols; c++) sum += x[c];
    float mean = sum / (float)cols;
    float var = 0.0f;
    for (size_t c = 0; c < cols; c++) {
        float t = x[c] - mean;
        var += t * t;
    }
    var = var / (float)cols;
    float is = 1.0f / sqrtf(var + LN_EPS);
    for (size_t c = 0; c < cols; c++) y[c] = (x[c] - mean) * is * g[c] + b[c];
}

/* ferrum_model/src/sampling.rs:32-40: first maximum wins; a NaN never stays best. */
size_t fo_argmax(const float *v, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (v[i] > v[best] || (v[best] != v[best] && v[i] == v[i])) best = i;
    return best;
}

struct fo_gpt2_cache {
    size_t len;
    float **k, **v; /* per layer [ctx * dim] */
};

fo_gpt2_cache *fo_gpt2_cache_new(const fo_gpt2 *m) {
    fo_gpt2_cache *c = (fo_gpt2_cache *)calloc(1, sizeof *c);
    c->k = (float **)calloc(m->layers, sizeof(float *));
    c->v = (float **)calloc(m->layers, sizeof(float *));
    for (size_t l = 0; l < m->layers; l++) {
        c->k[l] = (float *)calloc(m->ctx * m->dim, sizeof(float));
        c->v[l] = (float *)calloc(m->ctx * m->dim, sizeof(float));
    }
    return c;
}

void fo_gpt2_cache_free(const fo_gpt2 *m, fo_gpt2_cache *c) {
    if (!c) return;
    for (size_t l = 0; l < m->layers; l++) { free(c->k[l]); free(c->v[l]); }
    free(c->k);
    free(c->v);
    free(c);
}

/* ferrum_ref/src/models/gpt2/decode.rs:57-117 */
int fo_gpt2_feed(const fo_gpt2 *m, fo_gpt2_cache *cache, size_t token, float *logits) {
    size_t d = m->dim, pos = cache->len, hd = m->dim / m->heads;
    if (pos >= m->ctx || token >= m->vocab) return -1;
    float *x = (float *)malloc(d * sizeof(float));
    float *h = (float *)malloc(d * sizeof(float));
    float *q = (float *)malloc(d * sizeof(float));
    float *a = (float *)malloc(d * sizeof(float));
    float *t = (float *)malloc(d * sizeof(float));
    float *f = (float *)malloc(m->hidden * sizeof(float));
    float *s = (float *)malloc((m->ctx + 1) * sizeof(float));
    for (size_t i = 0; i < d; i++) x[i] = m->tok[token * d + i] + m->pos[pos * d + i];
    for (size_t l = 0; l < m->layers; l++) {
        const float *const *b = m->blocks + l * FO_GPT2_BLOCK_TENSORS;
        fo_layernorm(x, b[0], b[1], d, h);
        fo_gemv(h, b[2], b[3], d, d, q);
        float *kc = cache->k[l], *vc = cache->v[l];
        fo_gemv(h, b[4], b[5], d, d, kc + pos * d);
        fo_gemv(h, b[6], b[7], d, d, vc + pos * d);
        float scale = 1.0f / sqrtf((float)hd);
        for (size_t hh = 0; hh < m->heads; hh++) {
            for (size_t j = 0; j <= pos; j++) {
                float dot = 0.0f;
                for (size_t i = 0; i < hd; i++) dot += q[hh * hd + i] * kc[j * d + hh * hd + i];
                s[j] = dot * scale;
            }
            float max = -INFINITY;
            for (size_t j = 0; j <= pos; j++) max = fmaxf(max, s[j]);
            float sum = 0.0f;
            for (size_t j = 0; j <= pos; j++) {
                s[j] = expf(s[j] - max);
                sum += s[j];
            }
            for (size_t i = 0; i < hd; i++) {
                float acc = 0.0f;
                for (size_t j = 0; j <= pos; j++) acc += s[j] / sum * vc[j * d + hh * hd + i];
                a[hh * hd + i] = acc;
            }
        }
        fo_gemv(a, b[8], b[9], d, d, t);
        for (size_t i = 0; i < d; i++) x[i] = x[i] + t[i];
        fo_layernorm(x, b[10], b[11], d, h);
        fo_gemv(h, b[12], b[13], d, m->hidden, f);
        for (size_t i = 0; i < m->hidden; i++) f[i] = fo_gelu(f[i]);
        fo_gemv(f, b[14], b[15], m->hidden, d, t);
        for (size_t i = 0; i < d; i++) x[i] = x[i] + t[i];
    }
    fo_layernorm(x, m->lnf_g, m->lnf_b, d, h);
    fo_gemv(h, m->head, NULL, d, m->vocab, logits);
    cache->len = pos + 1;
    free(x); free(h); free(q); free(a); free(t); free(f); free(s);
    return 0;
}

/* Greedy decode: feed the prompt, then n_new argmax tokens (the reference's generate loop with
 * greedy sampling, ferrum_gpu_core/src/engine/mod.rs:204-242, sampling.rs:56-57). */
int fo_gpt2_generate(const fo_gpt2 *m, const size_t *prompt, size_t n_prompt, size_t n_new,
                     size_t *out) {
    if (n_prompt == 0 || n_prompt + n_new > m->ctx + 1) return -1;
    fo_gpt2_cache *c = fo_gpt2_cache_new(m);
    float *logits = (float *)malloc(m->vocab * sizeof(float));
    int rc = 0;
    for (size_t i = 0; i < n_prompt && rc == 0; i++) rc = fo_gpt2_feed(m, c, prompt[i], logits);
    for (size_t i = 0; i < n_new && rc == 0; i++) {
        out[i] = fo_argmax(logits, m->vocab);
        if (i + 1 < n_new) rc = fo_gpt2_feed(m, c, out[i], logits);
    }
    free(logits);
    fo_gpt2_cache_free(m, c);
    return rc;
}
