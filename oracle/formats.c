/* Block formats beyond Q8_0 / Q4_0: a C restatement of ferrum_gguf's fp8.rs, mxfp4.rs, q2k.rs
 * and blocks.rs. TEST INFRASTRUCTURE ONLY (see oracle.h). Same operation order as the Rust code
 * (no FMA contraction; glibc log2f and floorf, which Rust's f32 methods call on Linux). */
#include "formats.h"

#include <math.h>
#include <string.h>

static float half_at(const uint8_t *b) { return fo_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

static float pow2i(int e) { /* 2^e for the small exponents used here, exact */
    return ldexpf(1.0f, e);
}

/* ---- FP8 (ferrum_gguf/src/codec/fp8.rs) ---- */

float fo_fp8_decode(int e5m2, uint8_t code) {
    const float sign = (code & 0x80) ? -1.0f : 1.0f;
    const unsigned ebits = e5m2 ? 5 : 4, mbits = e5m2 ? 2 : 3;
    const int bias = e5m2 ? 15 : 7;
    const unsigned e = ((unsigned)code >> mbits) & ((1u << ebits) - 1);
    const unsigned m = (unsigned)code & ((1u << mbits) - 1);
    const unsigned top = (1u << ebits) - 1;
    if (e == top) {
        if (!e5m2) {
            if (m == (1u << mbits) - 1) return NAN;
        } else {
            return m == 0 ? sign * INFINITY : NAN;
        }
    }
    const float frac = (float)m / (float)(1u << mbits);
    if (e == 0) return sign * frac * pow2i(1 - bias);
    return sign * (1.0f + frac) * pow2i((int)e - bias);
}

uint8_t fo_fp8_encode(int e5m2, float x) {
    if (x != x) return e5m2 ? 0x7e : 0x7f;
    const uint8_t sign = signbit(x) ? 0x80 : 0;
    const float max = e5m2 ? 57344.0f : 448.0f;
    const float a = fminf(fabsf(x), max);
    const uint8_t limit = e5m2 ? 0x7b : 0x7e;
    uint8_t lo = 0, hi = limit;
    while (lo < hi) {
        const uint8_t mid = (uint8_t)(lo + (hi - lo) / 2);
        if (fo_fp8_decode(e5m2, mid) < a)
            lo = (uint8_t)(mid + 1);
        else
            hi = mid;
    }
    const uint8_t up = lo, down = lo ? (uint8_t)(lo - 1) : 0;
    const float du = fabsf(fo_fp8_decode(e5m2, up) - a), dd = fabsf(a - fo_fp8_decode(e5m2, down));
    const uint8_t pick = (du < dd || (du == dd && up % 2 == 0)) ? up : down;
    return (uint8_t)(sign | pick);
}

void fo_fp8_encode_blocks(int e5m2, const float *data, size_t nblocks, uint8_t *out) {
    const float max = e5m2 ? 57344.0f : 448.0f;
    for (size_t b = 0; b < nblocks; b++) {
        const float *blk = data + b * 32;
        uint8_t *o = out + b * 34;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i]));
        const uint16_t d = fo_f32_to_f16(amax / max);
        const float df = fo_f16_to_f32(d);
        const float id = df != 0.0f ? 1.0f / df : 0.0f;
        o[0] = (uint8_t)(d & 0xff);
        o[1] = (uint8_t)(d >> 8);
        for (int i = 0; i < 32; i++) o[2 + i] = fo_fp8_encode(e5m2, blk[i] * id);
    }
}

/* ---- MXFP4 (ferrum_gguf/src/codec/mxfp4.rs) ---- */

static const int8_t MX_VALUES[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

float fo_mxfp4_half_scale(uint8_t e) {
    uint32_t bits = e < 2 ? 0x00200000u << e : ((uint32_t)e - 1) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint8_t mx_scale_byte(float amax) {
    if (amax <= 0.0f || !isfinite(amax)) return 0;
    int e = (int)floorf(log2f(amax)) - 2 + 127;
    return (uint8_t)(e < 0 ? 0 : (e > 254 ? 254 : e));
}

static uint8_t mx_nearest(float x, float d) {
    int best = 0;
    float best_err = fabsf((float)MX_VALUES[0] * d - x);
    for (int i = 1; i < 16; i++) {
        const float err = fabsf((float)MX_VALUES[i] * d - x);
        if (err < best_err) {
            best = i;
            best_err = err;
        }
    }
    return (uint8_t)best;
}

void fo_mxfp4_encode_blocks(const float *data, size_t nblocks, uint8_t *out) {
    for (size_t b = 0; b < nblocks; b++) {
        const float *blk = data + b * 32;
        uint8_t *o = out + b * 17;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i]));
        const uint8_t e = mx_scale_byte(amax);
        const float d = fo_mxfp4_half_scale(e);
        o[0] = e;
        for (int j = 0; j < 16; j++) o[1 + j] = (uint8_t)(mx_nearest(blk[j], d) | (mx_nearest(blk[j + 16], d) << 4));
    }
}

static void mxfp4_block(const uint8_t *b, float *out) {
    const float d = fo_mxfp4_half_scale(b[0]);
    for (int j = 0; j < 16; j++) {
        out[j] = (float)MX_VALUES[b[1 + j] & 15] * d;
        out[16 + j] = (float)MX_VALUES[b[1 + j] >> 4] * d;
    }
}

/* ---- Q2_K encoder (ferrum_gguf/src/codec/q2k.rs) ---- */

int32_t fo_q2k_nearest_int(float x) {
    const float t = x + 12582912.0f;
    int32_t bits;
    memcpy(&bits, &t, 4);
    return (bits & 0x007fffff) - 0x00400000;
}

static int32_t clamp3(int32_t q) { return q < 0 ? 0 : (q > 3 ? 3 : q); }

/* q2k.rs:24-93 (make_qkx2_quants with nmax 3, rmin -0.5, rdelta 0.1, nstep 15). Exported so the
 * tests can check the search's result against the weighted least-squares fit it claims to be. */
void fo_q2k_fit(const float *x, uint8_t *l, float *scale_out, float *min_out) {
    float weights[16];
    for (int i = 0; i < 16; i++) weights[i] = fabsf(x[i]);
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < 16; i++) {
        min = fminf(min, x[i]);
        max = fmaxf(max, x[i]);
        sum_w += weights[i];
        sum_x += weights[i] * x[i];
    }
    if (min > 0.0f) min = 0.0f;
    if (max == min) {
        memset(l, 0, 16);
        *scale_out = 0.0f;
        *min_out = -min;
        return;
    }
    float iscale = 3.0f / (max - min);
    float scale = 1.0f / iscale;
    float best_mad = 0.0f;
    for (int i = 0; i < 16; i++) {
        const int32_t q = clamp3(fo_q2k_nearest_int(iscale * (x[i] - min)));
        l[i] = (uint8_t)q;
        const float diff = scale * (float)q + min - x[i];
        best_mad += weights[i] * fabsf(diff);
    }
    for (int step = 0; step <= 15; step++) {
        iscale = (-0.5f + 0.1f * (float)step + 3.0f) / (max - min);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        uint8_t laux[16];
        for (int i = 0; i < 16; i++) {
            const int32_t q = clamp3(fo_q2k_nearest_int(iscale * (x[i] - min)));
            laux[i] = (uint8_t)q;
            const float w = weights[i], qf = (float)q;
            sum_l += w * qf;
            sum_l2 += w * qf * qf;
            sum_xl += w * qf * x[i];
        }
        const float d = sum_w * sum_l2 - sum_l * sum_l;
        if (d > 0.0f) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / d;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / d;
            if (this_min > 0.0f) {
                this_min = 0.0f;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0.0f;
            for (int i = 0; i < 16; i++) {
                const float diff = this_scale * (float)laux[i] + this_min - x[i];
                mad += weights[i] * fabsf(diff);
            }
            if (mad < best_mad) {
                memcpy(l, laux, 16);
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *scale_out = scale;
    *min_out = -min;
}

void fo_q2k_encode_blocks(const float *data, size_t nblocks, uint8_t *out) {
    for (size_t b = 0; b < nblocks; b++) {
        const float *blk = data + b * 256;
        uint8_t *o = out + b * 84;
        float scales[16], mins[16];
        uint8_t levels[256];
        for (int j = 0; j < 16; j++) fo_q2k_fit(blk + 16 * j, levels + 16 * j, &scales[j], &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 16; j++) {
            max_scale = fmaxf(max_scale, scales[j]);
            max_min = fmaxf(max_min, mins[j]);
        }
        uint8_t packed[16] = {0};
        uint16_t d = 0, dmin = 0;
        if (max_scale > 0.0f) {
            const float iscale = 15.0f / max_scale;
            for (int j = 0; j < 16; j++) packed[j] = (uint8_t)fo_q2k_nearest_int(iscale * scales[j]);
            d = fo_f32_to_f16(max_scale / 15.0f);
        }
        if (max_min > 0.0f) {
            const float iscale = 15.0f / max_min;
            for (int j = 0; j < 16; j++) packed[j] |= (uint8_t)((uint8_t)fo_q2k_nearest_int(iscale * mins[j]) << 4);
            dmin = fo_f32_to_f16(max_min / 15.0f);
        }
        const float d32 = fo_f16_to_f32(d), dmin32 = fo_f16_to_f32(dmin);
        for (int j = 0; j < 16; j++) {
            const float sc = d32 * (float)(packed[j] & 15);
            if (sc == 0.0f) continue;
            const float dm = dmin32 * (float)(packed[j] >> 4);
            for (int ii = 0; ii < 16; ii++)
                levels[16 * j + ii] = (uint8_t)clamp3(fo_q2k_nearest_int((blk[16 * j + ii] + dm) / sc));
        }
        memcpy(o, packed, 16);
        int at = 16;
        for (int half = 0; half < 256; half += 128)
            for (int l = 0; l < 32; l++)
                o[at++] = (uint8_t)(levels[half + l] | (levels[half + l + 32] << 2) | (levels[half + l + 64] << 4) |
                                    (levels[half + l + 96] << 6));
        o[80] = (uint8_t)(d & 0xff);
        o[81] = (uint8_t)(d >> 8);
        o[82] = (uint8_t)(dmin & 0xff);
        o[83] = (uint8_t)(dmin >> 8);
    }
}

/* ---- read-only block types (ferrum_gguf/src/codec/blocks.rs) ---- */

int fo_layout(uint32_t ty, size_t *bytes, size_t *elems) {
    size_t b = 0, e = 32;
    switch (ty) {
    case FO_Q4_1: b = 20; break;
    case FO_Q5_0: b = 22; break;
    case FO_Q5_1: b = 24; break;
    case FO_Q8_1: b = 36; break;
    case FO_Q2_K: b = 84, e = 256; break;
    case FO_Q3_K: b = 110, e = 256; break;
    case FO_Q4_K: b = 144, e = 256; break;
    case FO_Q5_K: b = 176, e = 256; break;
    case FO_Q6_K: b = 210, e = 256; break;
    case FO_MXFP4: b = 17; break;
    case FO_FP8_E4M3:
    case FO_FP8_E5M2: b = 34; break;
    default: return 0;
    }
    if (bytes) *bytes = b;
    if (elems) *elems = e;
    return 1;
}

static void q8_1_block(const uint8_t *b, float *out) {
    const float d = half_at(b);
    for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)b[4 + i];
}

static void q4_1_block(const uint8_t *b, float *out) {
    const float d = half_at(b), m = half_at(b + 2);
    for (int j = 0; j < 16; j++) {
        out[j] = d * (float)(b[4 + j] & 0x0f) + m;
        out[16 + j] = d * (float)(b[4 + j] >> 4) + m;
    }
}

static void q5_block(const uint8_t *b, int with_min, float *out) {
    const float d = half_at(b);
    const float m = with_min ? half_at(b + 2) : 0.0f;
    const int at = with_min ? 4 : 2;
    const uint32_t qh = (uint32_t)b[at] | ((uint32_t)b[at + 1] << 8) | ((uint32_t)b[at + 2] << 16) | ((uint32_t)b[at + 3] << 24);
    const uint8_t *qs = b + at + 4;
    for (int j = 0; j < 16; j++) {
        const uint32_t lo = (uint32_t)(qs[j] & 0x0f) | (((qh >> j) & 1) << 4);
        const uint32_t hi = (uint32_t)(qs[j] >> 4) | (((qh >> (j + 16)) & 1) << 4);
        out[j] = with_min ? d * (float)lo + m : d * (float)((int32_t)lo - 16);
        out[16 + j] = with_min ? d * (float)hi + m : d * (float)((int32_t)hi - 16);
    }
}

static void scale_min(int j, const uint8_t *q, uint8_t *s, uint8_t *m) {
    if (j < 4) {
        *s = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *s = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static void q45_k_block(const uint8_t *b, int five, float *out) {
    const float d = half_at(b), dmin = half_at(b + 2);
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = five ? b + 48 : b + 16;
    for (int pair = 0; pair < 4; pair++) {
        uint8_t s1, m1, s2, m2;
        scale_min(2 * pair, scales, &s1, &m1);
        scale_min(2 * pair + 1, scales, &s2, &m2);
        const float d1 = d * (float)s1, n1 = dmin * (float)m1, d2 = d * (float)s2, n2 = dmin * (float)m2;
        const uint8_t *q = qs + 32 * pair;
        const uint8_t u1 = (uint8_t)(1u << (2 * pair)), u2 = (uint8_t)(2u << (2 * pair));
        for (int l = 0; l < 32; l++) {
            const int h1 = five && (qh[l] & u1) ? 16 : 0, h2 = five && (qh[l] & u2) ? 16 : 0;
            out[64 * pair + l] = d1 * (float)((q[l] & 0x0f) + h1) - n1;
            out[64 * pair + 32 + l] = d2 * (float)((q[l] >> 4) + h2) - n2;
        }
    }
}

static void q6_k_block(const uint8_t *b, float *out) {
    const uint8_t *ql = b, *qh = b + 128, *scales = b + 192;
    const float d = half_at(b + 208);
    for (int half = 0; half < 2; half++) {
        const int qlo = half * 64, qho = half * 32, sco = half * 8, oo = half * 128;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
#define Q6(lo, hi) (((int32_t)(lo) | ((int32_t)((hi) & 3) << 4)) - 32)
            const int32_t q1 = Q6(ql[qlo + l] & 0x0f, qh[qho + l]);
            const int32_t q2 = Q6(ql[qlo + l + 32] & 0x0f, qh[qho + l] >> 2);
            const int32_t q3 = Q6(ql[qlo + l] >> 4, qh[qho + l] >> 4);
            const int32_t q4 = Q6(ql[qlo + l + 32] >> 4, qh[qho + l] >> 6);
#undef Q6
            out[oo + l] = d * (float)(int8_t)scales[sco + is] * (float)q1;
            out[oo + l + 32] = d * (float)(int8_t)scales[sco + is + 2] * (float)q2;
            out[oo + l + 64] = d * (float)(int8_t)scales[sco + is + 4] * (float)q3;
            out[oo + l + 96] = d * (float)(int8_t)scales[sco + is + 6] * (float)q4;
        }
    }
}

static void q2_k_block(const uint8_t *b, float *out) {
    const uint8_t *scales = b, *qs = b + 16;
    const float d = half_at(b + 80), dmin = half_at(b + 82);
    int is = 0, o = 0;
    for (int half = 0; half < 2; half++) {
        const uint8_t *q = qs + 32 * half;
        for (int shift = 0; shift < 8; shift += 2)
            for (int run = 0; run < 2; run++) {
                const uint8_t sc = scales[is++];
                const float dl = d * (float)(sc & 0x0f), ml = dmin * (float)(sc >> 4);
                for (int l = 16 * run; l < 16 * run + 16; l++) out[o++] = dl * (float)((q[l] >> shift) & 3) - ml;
            }
    }
}

static void q3_k_block(const uint8_t *b, float *out) {
    const uint8_t *hmask = b, *qs = b + 32, *sc = b + 96;
    const float d = half_at(b + 108);
    int8_t scales[16];
    for (int j = 0; j < 8; j++) {
        scales[j] = (int8_t)(sc[j] & 0x0f);
        scales[j + 8] = (int8_t)(sc[j] >> 4);
    }
    for (int j = 0; j < 16; j++) scales[j] = (int8_t)(scales[j] | (int8_t)(((sc[8 + j / 4] >> (2 * (j % 4))) & 3) << 4));
    int is = 0, o = 0;
    uint8_t m = 1;
    for (int half = 0; half < 2; half++) {
        const uint8_t *q = qs + 32 * half;
        for (int shift = 0; shift < 8; shift += 2) {
            for (int run = 0; run < 2; run++) {
                const float dl = d * (float)(scales[is] - 32);
                is++;
                for (int l = 16 * run; l < 16 * run + 16; l++) {
                    const int32_t low = (q[l] >> shift) & 3;
                    out[o++] = dl * (float)(low - ((hmask[l] & m) ? 0 : 4));
                }
            }
            m = (uint8_t)(m << 1);
        }
    }
}

int fo_dequant(uint32_t ty, const uint8_t *raw, size_t nblocks, float *out) {
    size_t bb, be;
    if (!fo_layout(ty, &bb, &be)) return -1;
    for (size_t i = 0; i < nblocks; i++) {
        const uint8_t *b = raw + i * bb;
        float *o = out + i * be;
        switch (ty) {
        case FO_Q4_1: q4_1_block(b, o); break;
        case FO_Q5_0: q5_block(b, 0, o); break;
        case FO_Q5_1: q5_block(b, 1, o); break;
        case FO_Q8_1: q8_1_block(b, o); break;
        case FO_Q2_K: q2_k_block(b, o); break;
        case FO_Q3_K: q3_k_block(b, o); break;
        case FO_Q4_K: q45_k_block(b, 0, o); break;
        case FO_Q5_K: q45_k_block(b, 1, o); break;
        case FO_Q6_K: q6_k_block(b, o); break;
        case FO_MXFP4: mxfp4_block(b, o); break;
        default: { /* FP8 (fp8.rs:116-124) */
            const int e5m2 = ty == FO_FP8_E5M2;
            const float d = half_at(b);
            for (int j = 0; j < 32; j++) o[j] = d * fo_fp8_decode(e5m2, b[2 + j]);
        }
        }
    }
    return 0;
}
