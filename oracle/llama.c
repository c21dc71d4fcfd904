/* Llama / Qwen2 CPU oracle: a C restatement of ferrum_ref's Llama::forward_logits and the ops it
 * calls, plus nn::score. TEST INFRASTRUCTURE ONLY (see oracle.h). Operation order and rounding
 * follow the Rust code step by step (no FMA contraction, sequential f32 sums, glibc's expf,
 * sinf/cosf, sqrtf and pow, which are what Rust's f32/f64 methods call on Linux). The products
 * run on fo_matmul_tuned and the attention rows on worker threads: both are bit-identical to
 * the single-threaded reference for any thread count (rows are independent, and every output
 * element still accumulates in ascending k). */
#include "llama.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ferrum_ref/src/models/llama/ops.rs:78-101 (rope_tables) */
void fo_rope_tables(size_t start, size_t n, size_t rope_dim, float base, const float *freq_factors,
                    float linear_factor, float *cos_out, float *sin_out) {
    const size_t half = rope_dim / 2;
    for (size_t p = start; p < start + n; p++)
        for (size_t i = 0; i < half; i++) {
            const float freq = (float)pow((double)base, -2.0 * (double)i / (double)rope_dim);
            const float ff = freq_factors ? freq_factors[i] : 1.0f;
            const float theta = (float)p * freq / ff * (1.0f / linear_factor);
            const size_t o = (p - start) * half + i;
            sin_out[o] = sinf(theta);
            cos_out[o] = cosf(theta);
        }
}

/* ferrum_ref/src/models/llama/ops.rs:55-66 (rmsnorm) */
void fo_rmsnorm(const float *x, const float *g, size_t rows, size_t cols, float eps, float *y) {
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * cols;
        float ss = -0.0f;
        for (size_t c = 0; c < cols; c++) ss += row[c] * row[c];
        const float ms = ss / (float)cols;
        const float inv = 1.0f / sqrtf(ms + eps);
        for (size_t c = 0; c < cols; c++) y[r * cols + c] = row[c] * inv * g[c];
    }
}

/* ferrum_ref/src/models/llama/ops.rs:105-127 (apply_rope): NORM pairs (2i, 2i+1), NEOX pairs
 * (i, i + rope_dim/2); channels past rope_dim are left alone. */
void fo_apply_rope(float *x, size_t rows, size_t heads, size_t hd, size_t rope_dim, const float *cos_t,
                   const float *sin_t, int neox) {
    const size_t half = rope_dim / 2;
    for (size_t r = 0; r < rows; r++)
        for (size_t h = 0; h < heads; h++) {
            const size_t off = (r * heads + h) * hd;
            for (size_t i = 0; i < half; i++) {
                const size_t ia = neox ? off + i : off + 2 * i;
                const size_t ib = neox ? off + i + half : off + 2 * i + 1;
                const float c = cos_t[r * half + i], s = sin_t[r * half + i];
                const float a = x[ia], b = x[ib];
                x[ia] = a * c - b * s;
                x[ib] = a * s + b * c;
            }
        }
}

/* ferrum_ref/src/models/llama/ops.rs:131-162 (attend_row): query head h reads KV head
 * h / (heads / kv_heads); `scratch` holds `len` floats. */
void fo_attend_row(const float *q, const float *k, const float *v, size_t len, size_t heads, size_t kv_heads,
                   size_t hd, float *scratch, float *out) {
    const size_t kv_dim = kv_heads * hd, group = heads / kv_heads;
    const float scale = 1.0f / sqrtf((float)hd);
    float *s = scratch;
    for (size_t h = 0; h < heads; h++) {
        const size_t off = (h / group) * hd;
        for (size_t j = 0; j < len; j++) {
            float dot = -0.0f;
            for (size_t d = 0; d < hd; d++) dot += q[h * hd + d] * k[j * kv_dim + off + d];
            s[j] = dot * scale;
        }
        float max = -INFINITY;
        for (size_t j = 0; j < len; j++) max = fmaxf(max, s[j]);
        float sum = 0.0f;
        for (size_t j = 0; j < len; j++) {
            s[j] = expf(s[j] - max);
            sum += s[j];
        }
        for (size_t d = 0; d < hd; d++) {
            float acc = -0.0f;
            for (size_t j = 0; j < len; j++) acc += s[j] / sum * v[j * kv_dim + off + d];
            out[h * hd + d] = acc;
        }
    }
}

/* ferrum_ref/src/models/llama/ops.rs:69-76 */
float fo_silu(float x) { return x / (1.0f + expf(-x)); }

void fo_swiglu(const float *gate, const float *up, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = fo_silu(gate[i]) * up[i];
}

/* ferrum_ref/src/kernels/nn.rs:117-129 (score): the target's log-probability row[t] - max - lse
 * and whether it is the first maximum. */
void fo_score(const float *logits, const size_t *targets, size_t rows, size_t vocab, float *logprob,
              uint8_t *is_first_max) {
    for (size_t i = 0; i < rows; i++) {
        const float *row = logits + i * vocab;
        float max = -INFINITY;
        for (size_t j = 0; j < vocab; j++) max = fmaxf(max, row[j]);
        float sum = -0.0f;
        for (size_t j = 0; j < vocab; j++) sum += expf(row[j] - max);
        const float lse = logf(sum);
        size_t first = 0;
        for (size_t j = 0; j < vocab; j++)
            if (row[j] == max) {
                first = j;
                break;
            }
        logprob[i] = row[targets[i]] - max - lse;
        is_first_max[i] = first == targets[i];
    }
}

/* linear (mod.rs:190-197): matmul, then nn::add_bias when the bias is present */
static int linear(const float *x, const float *w, const float *bias, size_t rows, size_t k, size_t n, int threads,
                  float *y) {
    if (fo_matmul_tuned(x, w, rows, k, n, threads, y)) return -1;
    if (bias)
        for (size_t i = 0; i < rows * n; i++) y[i] = y[i] + bias[i % n];
    return 0;
}

typedef struct {
    const fo_llama *m;
    const float *q, *k, *v;
    float *a;
    size_t r0, r1;
} attn_job;

static void *attn_worker(void *p) {
    attn_job *j = (attn_job *)p;
    const fo_llama *m = j->m;
    const size_t qd = m->heads * m->head_dim;
    float *s = (float *)malloc((j->r1 + 1) * sizeof(float));
    if (!s) return (void *)1;
    for (size_t r = j->r0; r < j->r1; r++)
        fo_attend_row(j->q + r * qd, j->k, j->v, r + 1, m->heads, m->kv_heads, m->head_dim, s, j->a + r * qd);
    free(s);
    return NULL;
}

/* Every row's attention, rows interleaved over the threads so the long (late) rows spread. */
static int attend_rows(const fo_llama *m, const float *q, const float *k, const float *v, size_t n, int threads,
                       float *a) {
    size_t t = threads < 1 ? 1 : (size_t)threads;
    if (t > n) t = n;
    /* contiguous chunks of equal work: row r costs ~ r + 1 */
    pthread_t th[64];
    attn_job jobs[64];
    if (t > 64) t = 64;
    const double total = (double)n * (double)(n + 1) / 2.0;
    size_t r0 = 0;
    int bad = 0;
    for (size_t c = 0; c < t; c++) {
        size_t r1 = n;
        if (c + 1 < t) {
            const double want = total * (double)(c + 1) / (double)t;
            r1 = (size_t)ceil((sqrt(1.0 + 8.0 * want) - 1.0) / 2.0);
            if (r1 < r0) r1 = r0;
            if (r1 > n) r1 = n;
        }
        jobs[c] = (attn_job){m, q, k, v, a, r0, r1};
        r0 = r1;
    }
    for (size_t c = 0; c < t; c++) pthread_create(&th[c], NULL, attn_worker, &jobs[c]);
    for (size_t c = 0; c < t; c++) {
        void *ret = NULL;
        pthread_join(th[c], &ret);
        bad |= ret != NULL;
    }
    return bad ? -1 : 0;
}

/* ferrum_ref/src/models/llama/mod.rs:202-259: Llama::forward_logits, i.e. run() on an empty
 * cache (start = 0): every position's logits, [n, vocab]. Returns -1 for a bad length or token,
 * -2 when out of memory. */
int fo_llama_forward(const fo_llama *m, const size_t *ids, size_t n, int threads, float *logits) {
    if (n == 0 || n > m->ctx) return -1;
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= m->vocab) return -1;
    const size_t d = m->dim, qd = m->heads * m->head_dim, kvd = m->kv_heads * m->head_dim, hid = m->hidden;
    const size_t half = m->rope_dim / 2;
    float *cos_t = malloc((n * half + 1) * sizeof(float)), *sin_t = malloc((n * half + 1) * sizeof(float));
    float *x = malloc(n * d * sizeof(float)), *h = malloc(n * d * sizeof(float)), *o = malloc(n * d * sizeof(float));
    float *q = malloc(n * qd * sizeof(float)), *a = malloc(n * qd * sizeof(float));
    float *k = malloc(n * kvd * sizeof(float)), *v = malloc(n * kvd * sizeof(float));
    float *g = malloc(n * hid * sizeof(float)), *u = malloc(n * hid * sizeof(float));
    int rc = 0;
    if (!cos_t || !sin_t || !x || !h || !o || !q || !a || !k || !v || !g || !u) {
        rc = -2;
        goto done;
    }
    fo_rope_tables(0, n, m->rope_dim, m->rope_base, m->freq_factors, m->linear_factor, cos_t, sin_t);
    for (size_t r = 0; r < n; r++) memcpy(x + r * d, m->tok + ids[r] * d, d * sizeof(float));
    for (size_t l = 0; l < m->layers; l++) {
        const float *const *b = m->blocks + l * FO_LLAMA_BLOCK_TENSORS;
        fo_rmsnorm(x, b[0], n, d, m->eps, h);
        if (linear(h, b[1], b[2], n, d, qd, threads, q) || linear(h, b[3], b[4], n, d, kvd, threads, k) ||
            linear(h, b[5], b[6], n, d, kvd, threads, v)) {
            rc = -2;
            goto done;
        }
        fo_apply_rope(q, n, m->heads, m->head_dim, m->rope_dim, cos_t, sin_t, m->neox);
        fo_apply_rope(k, n, m->kv_heads, m->head_dim, m->rope_dim, cos_t, sin_t, m->neox);
        if (attend_rows(m, q, k, v, n, threads, a) || linear(a, b[7], NULL, n, qd, d, threads, o)) {
            rc = -2;
            goto done;
        }
        for (size_t i = 0; i < n * d; i++) x[i] = x[i] + o[i];
        fo_rmsnorm(x, b[8], n, d, m->eps, h);
        if (linear(h, b[9], NULL, n, d, hid, threads, g) || linear(h, b[10], NULL, n, d, hid, threads, u)) {
            rc = -2;
            goto done;
        }
        fo_swiglu(g, u, n * hid, g);
        if (linear(g, b[11], NULL, n, hid, d, threads, o)) {
            rc = -2;
            goto done;
        }
        for (size_t i = 0; i < n * d; i++) x[i] = x[i] + o[i];
    }
    fo_rmsnorm(x, m->out_norm, n, d, m->eps, h);
    if (linear(h, m->head, NULL, n, d, m->vocab, threads, logits)) rc = -2;
done:
    free(cos_t);
    free(sin_t);
    free(x);
    free(h);
    free(o);
    free(q);
    free(a);
    free(k);
    free(v);
    free(g);
    free(u);
    return rc;
}
