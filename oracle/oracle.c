/* CPU oracle (test infrastructure only; see oracle.h). Restates the reference's algorithms in
 * plain C so the HIP path can be checked against them bit for bit (codecs, snap) or within the
 * reference's frozen tolerance (products). Compiled with -ffp-contract=off: Rust never fuses
 * a*b+c, so neither may this file. */
#include "oracle.h"
#include "formats.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ferrum_gguf/src/codec/f16.rs:4-22 */
float fo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)(h >> 15)) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0 && man == 0) {
        bits = sign;
    } else if (exp == 0) {
        /* subnormal: normalise; man has at most 10 significant bits */
        uint32_t shift = (uint32_t)__builtin_clz(man) - 21;
        uint32_t m = (man << shift) & 0x3ff;
        uint32_t e = 127 - 15 + 1 - shift;
        bits = sign | (e << 23) | (m << 13);
    } else if (exp == 0x1f && man == 0) {
        bits = sign | 0x7f800000u;
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    return u2f(bits);
}

/* ferrum_gguf/src/codec/f16.rs:25-53: round to nearest even, overflow to inf, NaN quiet. */
uint16_t fo_f32_to_f16(float x) {
    uint32_t b = f2u(x);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    int32_t exp = (int32_t)((b >> 23) & 0xff);
    uint32_t man = b & 0x007fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (man != 0 ? 0x200 : 0));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = man | 0x00800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t mid = 1u << (shift - 1);
        uint32_t round = (rem > mid || (rem == mid && (half & 1) == 1)) ? 1u : 0u;
        return (uint16_t)(sign | (half + round));
    }
    uint32_t half = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fff;
    uint32_t round = (rem > 0x1000 || (rem == 0x1000 && (half & 1) == 1)) ? 1u : 0u;
    return (uint16_t)(sign | (half + round)); /* a carry into the exponent rounds up a binade */
}

/* ferrum_gguf/src/codec/quant.rs:17-47, with the block types of blocks.rs:34-48 and FP8. */
int64_t fo_nbytes(uint32_t ty, size_t n) {
    size_t bb, be;
    if (fo_layout(ty, &bb, &be)) return n % be ? -1 : (int64_t)(n / be * bb);
    switch (ty) {
    case FO_F32: return (int64_t)n * 4;
    case FO_F16: return (int64_t)n * 2;
    case FO_Q8_0:
        if (n % FO_QK) return -1;
        return (int64_t)(n / FO_QK) * (2 + FO_QK);
    case FO_Q4_0:
        if (n % FO_QK) return -1;
        return (int64_t)(n / FO_QK) * (2 + FO_QK / 2);
    default: return -1;
    }
}

static float half_at(const uint8_t *b) { return fo_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

/* ferrum_gguf/src/codec/quant.rs:50-88 */
int fo_decode(uint32_t ty, const uint8_t *bytes, size_t len, size_t n, float *out) {
    int64_t need = fo_nbytes(ty, n);
    if (need < 0 || (size_t)need != len) return -1;
    size_t bb, be;
    if (fo_layout(ty, &bb, &be)) return fo_dequant(ty, bytes, n / be, out);
    switch (ty) {
    case FO_F32:
        memcpy(out, bytes, n * 4);
        return 0;
    case FO_F16:
        for (size_t i = 0; i < n; i++) out[i] = half_at(bytes + 2 * i);
        return 0;
    case FO_Q8_0:
        for (size_t b = 0; b < n / FO_QK; b++) {
            const uint8_t *blk = bytes + b * 34;
            float d = half_at(blk);
            for (int e = 0; e < 32; e++) out[b * 32 + e] = d * (float)(int8_t)blk[2 + e];
        }
        return 0;
    case FO_Q4_0:
        /* low nibbles are elements 0..16, high nibbles 16..32 */
        for (size_t b = 0; b < n / FO_QK; b++) {
            const uint8_t *blk = bytes + b * 18;
            float d = half_at(blk);
            for (int j = 0; j < 16; j++) {
                uint8_t q = blk[2 + j];
                out[b * 32 + j] = d * ((float)(q & 0x0f) - 8.0f);
                out[b * 32 + 16 + j] = d * ((float)(q >> 4) - 8.0f);
            }
        }
        return 0;
    default: return -1;
    }
}

/* Rust `f as i8` / `f as i32`: truncate toward zero, saturate, NaN -> 0. */
static int32_t sat_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}
static int8_t sat_i8(float f) {
    if (f != f) return 0;
    if (f >= 127.0f) return 127;
    if (f <= -128.0f) return -128;
    return (int8_t)f;
}

/* ferrum_gguf/src/codec/quant.rs:111-119 (one Q8_0 block). */
static void encode_q8_0_block(const float *v, uint8_t *out) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t h = fo_f32_to_f16(d);
    out[0] = (uint8_t)(h & 0xff);
    out[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; i++) out[2 + i] = (uint8_t)sat_i8(roundf(v[i] * id));
}

/* ferrum_gguf/src/codec/quant.rs:120-133 (one Q4_0 block). */
static void encode_q4_0_block(const float *v, uint8_t *out) {
    /* the element with the largest magnitude (first one wins, keeping its sign) maps to -8 */
    float max = 0.0f;
    for (int i = 0; i < 32; i++)
        if (fabsf(v[i]) > fabsf(max)) max = v[i];
    float d = max / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t h = fo_f32_to_f16(d);
    out[0] = (uint8_t)(h & 0xff);
    out[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 16; j++) {
        int32_t lo = sat_i32(v[j] * id + 8.5f);
        int32_t hi = sat_i32(v[j + 16] * id + 8.5f);
        lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
        hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
        out[2 + j] = (uint8_t)(lo | (hi << 4));
    }
}

/* ferrum_gguf/src/codec/quant.rs:91-136 (Q2_K and MXFP4 by q2k.rs / mxfp4.rs, FP8 by fp8.rs; the
 * other block types are read-only: -2). */
int fo_encode(uint32_t ty, const float *data, size_t n, uint8_t *out) {
    if (fo_nbytes(ty, n) < 0) return -1;
    switch (ty) {
    case FO_Q2_K: fo_q2k_encode_blocks(data, n / 256, out); return 0;
    case FO_MXFP4: fo_mxfp4_encode_blocks(data, n / 32, out); return 0;
    case FO_FP8_E4M3: fo_fp8_encode_blocks(0, data, n / 32, out); return 0;
    case FO_FP8_E5M2: fo_fp8_encode_blocks(1, data, n / 32, out); return 0;
    default:
        if (fo_layout(ty, NULL, NULL)) return -2;
    }
    switch (ty) {
    case FO_F32:
        memcpy(out, data, n * 4);
        return 0;
    case FO_F16:
        for (size_t i = 0; i < n; i++) {
            uint16_t h = fo_f32_to_f16(data[i]);
            out[2 * i] = (uint8_t)(h & 0xff);
            out[2 * i + 1] = (uint8_t)(h >> 8);
        }
        return 0;
    case FO_Q8_0:
        for (size_t b = 0; b < n / FO_QK; b++) encode_q8_0_block(data + b * 32, out + b * 34);
        return 0;
    case FO_Q4_0:
        for (size_t b = 0; b < n / FO_QK; b++) encode_q4_0_block(data + b * 32, out + b * 18);
        return 0;
    default: return -1;
    }
}

/* ferrum_ref/src/models/llama/params.rs:24-32 */
void fo_transpose(const float *data, size_t rows, size_t cols, float *out) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) out[c * rows + r] = data[r * cols + c];
}

/* ferrum_wgpu/src/ops/quant.rs:238-252 */
int fo_quantise_matrix(uint32_t ty, const float *w, size_t k, size_t n, uint8_t *out) {
    size_t be = FO_QK;
    if (ty != FO_Q8_0 && ty != FO_Q4_0 && ty != FO_F16 && ty != FO_Q2_K && ty != FO_MXFP4 && ty != FO_FP8_E4M3 &&
        ty != FO_FP8_E5M2)
        return -1;
    fo_layout(ty, NULL, &be);
    if (k == 0 || k % be) return -1;
    float *rows = (float *)malloc(k * n * sizeof(float) + 1);
    if (!rows) return -1;
    fo_transpose(w, k, n, rows);
    int rc = fo_encode(ty, rows, k * n, out);
    free(rows);
    return rc;
}

/* ferrum_ref/src/training/qat.rs:20-24 */
void fo_snap_block(const float *in, float *out) {
    uint8_t b[34];
    encode_q8_0_block(in, b);
    fo_decode(FO_Q8_0, b, 34, 32, out);
}

/* ferrum_ref/src/training/qat.rs:15-17 */
static int eligible(size_t ne0) { return ne0 > 0 && ne0 % FO_QK == 0; }

/* ferrum_ref/src/training/qat.rs:27-35 */
void fo_snap_rows(float *data, size_t len, size_t ne0) {
    if (!eligible(ne0)) return;
    for (size_t b = 0; b + FO_QK <= len; b += FO_QK) {
        float tmp[32];
        fo_snap_block(data + b, tmp);
        memcpy(data + b, tmp, sizeof tmp);
    }
}

/* ferrum_ref/src/training/qat.rs:38-54 */
void fo_snap_cols(float *data, size_t rows_in, size_t cols_out) {
    if (!eligible(rows_in)) return;
    float buf[32], snapped[32];
    for (size_t j = 0; j < cols_out; j++)
        for (size_t i0 = 0; i0 < rows_in; i0 += FO_QK) {
            for (size_t e = 0; e < FO_QK; e++) buf[e] = data[(i0 + e) * cols_out + j];
            fo_snap_block(buf, snapped);
            for (size_t e = 0; e < FO_QK; e++) data[(i0 + e) * cols_out + j] = snapped[e];
        }
}

/* ferrum_ref/src/kernels/matmul.rs:49-59: out rows accumulate a[i,p] * b[p,:], p ascending. */
static void mm_rows(const float *a, const float *b, size_t k, size_t n, size_t nrows, float *out) {
    for (size_t i = 0; i < nrows; i++) {
        float *row = out + i * n;
        for (size_t p = 0; p < k; p++) {
            float av = a[i * k + p];
            const float *brow = b + p * n;
            for (size_t j = 0; j < n; j++) row[j] += av * brow[j];
        }
    }
}

/* ferrum_ref/src/kernels/matmul.rs:62-69 */
int fo_matmul(const float *a, const float *b, size_t m, size_t k, size_t n, float *out) {
    memset(out, 0, m * n * sizeof(float));
    if (n > 0) mm_rows(a, b, k, n, m, out);
    return 0;
}

typedef struct {
    const float *a, *b;
    size_t k, n, r0, r1, m;
    float *out;
    int tuned;
} mm_job;

static void tuned_block(const float *a, const float *b, size_t k, size_t n, size_t r0, size_t r1,
                        float *out);

static void *mm_worker(void *p) {
    mm_job *j = (mm_job *)p;
    if (j->tuned)
        tuned_block(j->a, j->b, j->k, j->n, j->r0, j->r1, j->out + j->r0 * j->n);
    else
        mm_rows(j->a + j->r0 * j->k, j->b, j->k, j->n, j->r1 - j->r0, j->out + j->r0 * j->n);
    return NULL;
}

static int mm_split(const float *a, const float *b, size_t m, size_t k, size_t n, int threads,
                    float *out, int tuned) {
    memset(out, 0, m * n * sizeof(float));
    if (m == 0 || n == 0) return 0;
    size_t t = threads < 1 ? 1 : (size_t)threads;
    size_t per = (m + t - 1) / t;
    size_t chunks = (m + per - 1) / per;
    pthread_t *th = (pthread_t *)calloc(chunks, sizeof(pthread_t));
    mm_job *jobs = (mm_job *)calloc(chunks, sizeof(mm_job));
    if (!th || !jobs) { free(th); free(jobs); return -1; }
    for (size_t c = 0; c < chunks; c++) {
        size_t r0 = c * per, r1 = r0 + per < m ? r0 + per : m;
        jobs[c] = (mm_job){a, b, k, n, r0, r1, m, out, tuned};
        pthread_create(&th[c], NULL, mm_worker, &jobs[c]);
    }
    for (size_t c = 0; c < chunks; c++) pthread_join(th[c], NULL);
    free(th);
    free(jobs);
    return 0;
}

/* ferrum_ref/src/kernels/matmul.rs:73-94 */
int fo_matmul_threaded(const float *a, const float *b, size_t m, size_t k, size_t n, int threads,
                       float *out) {
    return mm_split(a, b, m, k, n, threads, out, 0);
}

/* ferrum_ref/src/kernels/tuned.rs:10-13 */
enum { KC = 256, NC = 256, MR = 4, NR = 8 };

/* ferrum_ref/src/kernels/tuned.rs:46-75: MR x NR register tile over p in [pp, p1), ascending. */
static void tuned_micro(const float *a, const float *b, size_t k, size_t n, size_t i, size_t r0,
                        size_t j, size_t pp, size_t p1, float *out) {
    float acc[MR][NR];
    for (size_t r = 0; r < MR; r++) memcpy(acc[r], out + (i + r - r0) * n + j, NR * sizeof(float));
    for (size_t p = pp; p < p1; p++) {
        const float *bs = b + p * n + j;
        for (size_t r = 0; r < MR; r++) {
            float av = a[(i + r) * k + p];
            for (size_t c = 0; c < NR; c++) acc[r][c] += av * bs[c];
        }
    }
    for (size_t r = 0; r < MR; r++) memcpy(out + (i + r - r0) * n + j, acc[r], NR * sizeof(float));
}

/* ferrum_ref/src/kernels/tuned.rs:77-97 */
static void tuned_edge(const float *a, const float *b, size_t k, size_t n, size_t ia, size_t ib,
                       size_t r0, size_t ja, size_t jb, size_t pp, size_t p1, float *out) {
    for (size_t i = ia; i < ib; i++)
        for (size_t p = pp; p < p1; p++) {
            float aip = a[i * k + p];
            float *o = out + (i - r0) * n;
            for (size_t j = ja; j < jb; j++) o[j] += aip * b[p * n + j];
        }
}

/* ferrum_ref/src/kernels/tuned.rs:16-43 */
static void tuned_block(const float *a, const float *b, size_t k, size_t n, size_t r0, size_t r1,
                        float *out) {
    for (size_t jj = 0; jj < n;) {
        size_t j1 = jj + NC < n ? jj + NC : n;
        for (size_t pp = 0; pp < k;) {
            size_t p1 = pp + KC < k ? pp + KC : k;
            size_t i = r0;
            for (; i + MR <= r1; i += MR) {
                size_t j = jj;
                for (; j + NR <= j1; j += NR) tuned_micro(a, b, k, n, i, r0, j, pp, p1, out);
                if (j < j1) tuned_edge(a, b, k, n, i, i + MR, r0, j, j1, pp, p1, out);
            }
            if (i < r1) tuned_edge(a, b, k, n, i, r1, r0, jj, j1, pp, p1, out);
            pp = p1;
        }
        jj = j1;
    }
}

/* ferrum_ref/src/kernels/tuned.rs:99-134 */
int fo_matmul_tuned(const float *a, const float *b, size_t m, size_t k, size_t n, int threads,
                    float *out) {
    return mm_split(a, b, m, k, n, threads, out, 1);
}

/* ferrum_ref/src/models/gpt2/decode.rs:42-53 */
void fo_gemv(const float *x, const float *w, const float *bias, size_t k, size_t n, float *y) {
    memset(y, 0, n * sizeof(float));
    for (size_t p = 0; p < k; p++) {
        float xv = x[p];
        const float *wr = w + p * n;
        for (size_t j = 0; j < n; j++) y[j] += xv * wr[j];
    }
    if (bias)
        for (size_t j = 0; j < n; j++) y[j] += bias[j];
}

/* ferrum_ref/src/kernels/matmul.rs:97-107 */
void fo_rand_vec(size_t len, uint64_t seed, float *out) {
    uint64_t s = seed < 1 ? 1 : seed;
    for (size_t i = 0; i < len; i++) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        out[i] = ((float)(s >> 40) / (float)(1ull << 24)) * 2.0f - 1.0f;
    }
}

/* ferrum_ref/src/kernels/rng.rs:11-17 */
void fo_rng_init(fo_rng *r, uint64_t seed) { r->s = seed == 0 ? 0x9e3779b97f4a7c15ull : seed; }
/* ferrum_ref/src/kernels/rng.rs:20-25 */
uint64_t fo_rng_next_u64(fo_rng *r) {
    r->s ^= r->s >> 12;
    r->s ^= r->s << 25;
    r->s ^= r->s >> 27;
    return r->s * 0x2545f4914f6cdd1dull;
}
/* ferrum_ref/src/kernels/rng.rs:28-30 */
float fo_rng_next_f32(fo_rng *r) { return (float)(fo_rng_next_u64(r) >> 40) / (float)(1ull << 24); }
/* ferrum_ref/src/kernels/rng.rs:33-43 */
size_t fo_rng_below(fo_rng *r, size_t n) {
    uint64_t nn = (uint64_t)n;
    uint64_t zone = UINT64_MAX - (UINT64_MAX % nn);
    for (;;) {
        uint64_t v = fo_rng_next_u64(r);
        if (v < zone) return (size_t)(v % nn);
    }
}

/* ferrum_wgpu/src/tolerance.rs:14-26 */
float fo_max_rel_err(const float *got, const float *want, size_t n) {
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float d = fabsf(want[i]);
        float e = fabsf(got[i] - want[i]) / (d > 1.0f ? d : 1.0f);
        if (e != e) return INFINITY;
        m = fmaxf(m, e);
    }
    return m;
}
