// Block formats beyond Q8_0 / Q4_0 (ferrum_gguf/src/codec/{fp8,mxfp4,q2k,blocks}.rs and the
// formats ferrum_wgpu adds to QKind, ferrum_wgpu/src/ops/quant.rs:27-121):
//   weight formats F16, MXFP4, FP8 E4M3, FP8 E5M2 and Q2_K: encode, decode, resident weights and
//   every linear path (one thread per output, batch-1 GEMV, tiled product);
//   read-only GGUF block types Q4_1, Q5_0, Q5_1, Q8_1, Q3_K, Q4_K, Q5_K, Q6_K: decode.
// A resident weight of these formats keeps its GGUF rows as they are (row-major, n rows of k/E
// blocks); every product decodes its operands on the fly and computes in f32. The decoders and
// encoders reproduce the reference's arithmetic bit for bit: no contraction into FMA anywhere in
// this file except the explicit fmaf of the tiled product.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.hpp"
#include "internal.hpp"

#pragma clang fp contract(off)

namespace fh {
namespace {

__device__ __forceinline__ float h16(const uint8_t *p) {
    return half_bits_to_float((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

// fp8.rs:34-63
__device__ float fp8_value(bool e5m2, uint32_t code) {
    const float sign = (code & 0x80u) ? -1.0f : 1.0f;
    const uint32_t ebits = e5m2 ? 5 : 4, mbits = e5m2 ? 2 : 3;
    const int bias = e5m2 ? 15 : 7;
    const uint32_t e = (code >> mbits) & ((1u << ebits) - 1), m = code & ((1u << mbits) - 1);
    if (e == (1u << ebits) - 1) {
        if (!e5m2) {
            if (m == (1u << mbits) - 1) return __uint_as_float(0x7fc00000u);
        } else {
            return m == 0 ? sign * __uint_as_float(0x7f800000u) : __uint_as_float(0x7fc00000u);
        }
    }
    const float frac = (float)m / (float)(1u << mbits);
    if (e == 0) return sign * frac * __uint_as_float((uint32_t)(127 + 1 - bias) << 23);
    return sign * (1.0f + frac) * __uint_as_float((uint32_t)(127 + (int)e - bias) << 23);
}

// mxfp4.rs:26-33, 13-14
__device__ __forceinline__ float mx_half_scale(uint32_t e) {
    return e < 2 ? __uint_as_float(0x00200000u << e) : __uint_as_float((e - 1) << 23);
}
__device__ __forceinline__ float mx_value(uint32_t nib) {
    const int v[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    return (float)v[nib & 15];
}

// ---- element i of one block (blocks.rs, fp8.rs, mxfp4.rs, quant.rs:64-70) ----
template <uint32_t T>
struct Fmt;

template <>
struct Fmt<FH_F16> {
    static constexpr uint32_t B = 64, E = 32;
    __device__ static float at(const uint8_t *b, uint32_t i) { return h16(b + 2 * i); }
};
template <>
struct Fmt<FH_FP8_E4M3> {
    static constexpr uint32_t B = 34, E = 32;
    __device__ static float at(const uint8_t *b, uint32_t i) { return h16(b) * fp8_value(false, b[2 + i]); }
};
template <>
struct Fmt<FH_FP8_E5M2> {
    static constexpr uint32_t B = 34, E = 32;
    __device__ static float at(const uint8_t *b, uint32_t i) { return h16(b) * fp8_value(true, b[2 + i]); }
};
template <>
struct Fmt<FH_MXFP4> {
    static constexpr uint32_t B = 17, E = 32;
    __device__ static float at(const uint8_t *b, uint32_t i) {
        const uint32_t q = i < 16 ? b[1 + i] & 15u : (uint32_t)b[1 + i - 16] >> 4;
        return mx_value(q) * mx_half_scale(b[0]);
    }
};
template <>
struct Fmt<FH_Q4_1> {
    static constexpr uint32_t B = 20, E = 32;
    __device__ static float at(const uint8_t *b, uint32_t i) {
        const uint32_t q = i < 16 ? b[4 + i] & 15u : (uint32_t)b[4 + i - 16] >> 4;
        return h16(b) * (float)q + h16(b + 2);
    }
};
template <bool MIN>
__device__ float q5_at(const uint8_t *b, uint32_t i) {
    const uint32_t at = MIN ? 4 : 2;
    const uint32_t qh = (uint32_t)b[at] | ((uint32_t)b[at + 1] << 8) | ((uint32_t)b[at + 2] << 16) |
                        ((uint32_t)b[at + 3] << 24);
    const uint32_t j = i % 16;
    const uint32_t nib = i < 16 ? b[at + 4 + j] & 15u : (uint32_t)b[at + 4 + j] >> 4;
    const uint32_t x = nib | (((qh >> i) & 1u) << 4);  // bit j (first half) or j + 16 (second)
    if (MIN) return h16(b) * (float)x + h16(b + 2);
    return h16(b) * (float)((int32_t)x - 16);
}
template <>
struct Fmt<FH_Q5_0> {
    static constexpr uint32_t B = 22, E = 32;
    __device__ static float at(const uint8_t *b, uint32_t i) { return q5_at<false>(b, i); }
};
template <>
struct Fmt<FH_Q5_1> {
    static constexpr uint32_t B = 24, E = 32;
    __device__ static float at(const uint8_t *b, uint32_t i) { return q5_at<true>(b, i); }
};
template <>
struct Fmt<FH_Q8_1> {
    static constexpr uint32_t B = 36, E = 32;
    __device__ static float at(const uint8_t *b, uint32_t i) { return h16(b) * (float)(int8_t)b[4 + i]; }
};
// Q2_K / Q3_K scan (blocks.rs:201-250): element i = 128 half + 32 s + l, shift 2 s, sub-block
// 8 half + 2 s + l / 16
template <>
struct Fmt<FH_Q2_K> {
    static constexpr uint32_t B = 84, E = 256;
    __device__ static float at(const uint8_t *b, uint32_t i) {
        const uint32_t half = i / 128, s = (i % 128) / 32, l = i % 32;
        const uint32_t sc = b[8 * half + 2 * s + l / 16];
        const float dl = h16(b + 80) * (float)(sc & 15u), ml = h16(b + 82) * (float)(sc >> 4);
        return dl * (float)(((uint32_t)b[16 + 32 * half + l] >> (2 * s)) & 3u) - ml;
    }
};
template <>
struct Fmt<FH_Q3_K> {
    static constexpr uint32_t B = 110, E = 256;
    __device__ static float at(const uint8_t *b, uint32_t i) {
        const uint32_t half = i / 128, s = (i % 128) / 32, l = i % 32;
        const uint32_t j = 8 * half + 2 * s + l / 16;
        const uint8_t *sc = b + 96;
        const int32_t lo4 = j < 8 ? sc[j] & 15 : sc[j - 8] >> 4;
        const int32_t hi2 = (sc[8 + j / 4] >> (2 * (j % 4))) & 3;
        const int32_t scale = (int32_t)(int8_t)(uint8_t)(lo4 | (hi2 << 4));
        const float dl = h16(b + 108) * (float)(scale - 32);
        const int32_t low = ((uint32_t)b[32 + 32 * half + l] >> (2 * s)) & 3u;
        const uint32_t m = 1u << (4 * half + s);
        return dl * (float)(low - ((b[l] & m) ? 0 : 4));
    }
};
__device__ __forceinline__ void k_scale_min(uint32_t j, const uint8_t *q, uint32_t *s, uint32_t *m) {
    if (j < 4) {
        *s = q[j] & 63u;
        *m = q[j + 4] & 63u;
    } else {
        *s = (q[j + 4] & 0x0fu) | (((uint32_t)q[j - 4] >> 6) << 4);
        *m = ((uint32_t)q[j + 4] >> 4) | (((uint32_t)q[j] >> 6) << 4);
    }
}
template <bool FIVE>
__device__ float q45k_at(const uint8_t *b, uint32_t i) {
    const uint32_t pair = i / 64, w = i % 64, l = w % 32, hi = w / 32;
    uint32_t sc, mn;
    k_scale_min(2 * pair + hi, b + 4, &sc, &mn);
    const float dd = h16(b) * (float)sc, nn = h16(b + 2) * (float)mn;
    const uint8_t q = b[(FIVE ? 48 : 16) + 32 * pair + l];
    uint32_t v = hi ? (uint32_t)q >> 4 : q & 15u;
    if (FIVE && (b[16 + l] & ((hi ? 2u : 1u) << (2 * pair)))) v += 16;
    return dd * (float)v - nn;
}
template <>
struct Fmt<FH_Q4_K> {
    static constexpr uint32_t B = 144, E = 256;
    __device__ static float at(const uint8_t *b, uint32_t i) { return q45k_at<false>(b, i); }
};
template <>
struct Fmt<FH_Q5_K> {
    static constexpr uint32_t B = 176, E = 256;
    __device__ static float at(const uint8_t *b, uint32_t i) { return q45k_at<true>(b, i); }
};
template <>
struct Fmt<FH_Q6_K> {
    static constexpr uint32_t B = 210, E = 256;
    __device__ static float at(const uint8_t *b, uint32_t i) {
        const uint32_t half = i / 128, quarter = (i % 128) / 32, l = i % 32;
        const uint8_t lq = b[64 * half + l + (quarter & 1) * 32];
        const uint32_t lo = quarter < 2 ? lq & 15u : (uint32_t)lq >> 4;
        const uint32_t hb = ((uint32_t)b[128 + 32 * half + l] >> (2 * quarter)) & 3u;
        const int32_t q = (int32_t)(lo | (hb << 4)) - 32;
        const float sc = (float)(int8_t)b[192 + 8 * half + l / 16 + 2 * quarter];
        return h16(b + 208) * sc * (float)q;
    }
};

// ---- decode: GGUF rows -> f32, one thread per element ----
template <uint32_t T>
__global__ __launch_bounds__(256) void decode_ext_kernel(const uint8_t *__restrict__ src, float *__restrict__ dst,
                                                         size_t n) {
    using F = Fmt<T>;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < n; idx += (size_t)gridDim.x * 256)
        dst[idx] = F::at(src + idx / F::E * F::B, (uint32_t)(idx % F::E));
}

// ---- encoders ----
__global__ __launch_bounds__(256) void encode_f16_kernel(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                                         size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const uint32_t h = float_to_half_bits(src[i]);
        dst[2 * i] = (uint8_t)(h & 0xff);
        dst[2 * i + 1] = (uint8_t)(h >> 8);
    }
}

// fp8.rs:65-113, one thread per block
__device__ uint32_t fp8_encode(bool e5m2, float x) {
    if (x != x) return e5m2 ? 0x7eu : 0x7fu;
    const uint32_t sign = (__float_as_uint(x) >> 31) ? 0x80u : 0u;
    const float a = fminf(fabsf(x), e5m2 ? 57344.0f : 448.0f);
    uint32_t lo = 0, hi = e5m2 ? 0x7bu : 0x7eu;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (fp8_value(e5m2, mid) < a)
            lo = mid + 1;
        else
            hi = mid;
    }
    const uint32_t up = lo, down = lo ? lo - 1 : 0;
    const float du = fabsf(fp8_value(e5m2, up) - a), dd = fabsf(a - fp8_value(e5m2, down));
    return sign | ((du < dd || (du == dd && up % 2 == 0)) ? up : down);
}

template <bool E5M2>
__global__ __launch_bounds__(256) void encode_fp8_kernel(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                                         size_t nblocks) {
    for (size_t b = (size_t)blockIdx.x * 256 + threadIdx.x; b < nblocks; b += (size_t)gridDim.x * 256) {
        const float *v = src + b * 32;
        uint8_t *o = dst + b * 34;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
        const uint32_t d = float_to_half_bits(amax / (E5M2 ? 57344.0f : 448.0f));
        const float df = half_bits_to_float(d);
        const float id = df != 0.0f ? 1.0f / df : 0.0f;
        o[0] = (uint8_t)(d & 0xff);
        o[1] = (uint8_t)(d >> 8);
        for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)fp8_encode(E5M2, v[i] * id);
    }
}

// mxfp4.rs:48-83, one thread per block. floor(log2(amax)) is the reference's f32 log2 rounded to
// nearest, computed here through a float64 log2 rounded to f32 (checked against glibc's log2f on
// the floats nearest every power of two, where the two could differ).
__global__ __launch_bounds__(256) void encode_mxfp4_kernel(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                                           size_t nblocks) {
    for (size_t b = (size_t)blockIdx.x * 256 + threadIdx.x; b < nblocks; b += (size_t)gridDim.x * 256) {
        const float *v = src + b * 32;
        uint8_t *o = dst + b * 17;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
        uint32_t e = 0;
        if (amax > 0.0f && amax <= 3.4028235e38f) {
            const int ex = (int)floorf((float)log2((double)amax)) - 2 + 127;
            e = (uint32_t)(ex < 0 ? 0 : (ex > 254 ? 254 : ex));
        }
        const float d = mx_half_scale(e);
        o[0] = (uint8_t)e;
        for (int j = 0; j < 16; j++) {
            uint32_t q[2];
            for (int h = 0; h < 2; h++) {
                const float x = v[j + 16 * h];
                uint32_t best = 0;
                float best_err = fabsf(mx_value(0) * d - x);
                for (uint32_t i = 1; i < 16; i++) {
                    const float err = fabsf(mx_value(i) * d - x);
                    if (err < best_err) {
                        best = i;
                        best_err = err;
                    }
                }
                q[h] = best;
            }
            o[1 + j] = (uint8_t)(q[0] | (q[1] << 4));
        }
    }
}

// q2k.rs:16-150, one thread per super-block
__device__ __forceinline__ int32_t nearest_int(float x) {
    const float t = x + 12582912.0f;
    return (int32_t)(__float_as_uint(t) & 0x007fffffu) - 0x00400000;
}
__device__ __forceinline__ int32_t clamp3(int32_t q) { return q < 0 ? 0 : (q > 3 ? 3 : q); }

__device__ void q2k_fit(const float *x, uint8_t *l, float *scale_out, float *min_out) {
    float weights[16];
    for (int i = 0; i < 16; i++) weights[i] = fabsf(x[i]);
    float mn = x[0], mx = x[0], sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < 16; i++) {
        mn = fminf(mn, x[i]);
        mx = fmaxf(mx, x[i]);
        sum_w += weights[i];
        sum_x += weights[i] * x[i];
    }
    if (mn > 0.0f) mn = 0.0f;
    if (mx == mn) {
        for (int i = 0; i < 16; i++) l[i] = 0;
        *scale_out = 0.0f;
        *min_out = -mn;
        return;
    }
    float iscale = 3.0f / (mx - mn);
    float scale = 1.0f / iscale;
    float best_mad = 0.0f;
    for (int i = 0; i < 16; i++) {
        const int32_t q = clamp3(nearest_int(iscale * (x[i] - mn)));
        l[i] = (uint8_t)q;
        const float diff = scale * (float)q + mn - x[i];
        best_mad += weights[i] * fabsf(diff);
    }
    for (int step = 0; step <= 15; step++) {
        iscale = (-0.5f + 0.1f * (float)step + 3.0f) / (mx - mn);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        uint8_t laux[16];
        for (int i = 0; i < 16; i++) {
            const int32_t q = clamp3(nearest_int(iscale * (x[i] - mn)));
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
                for (int i = 0; i < 16; i++) l[i] = laux[i];
                best_mad = mad;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *scale_out = scale;
    *min_out = -mn;
}

// Sixteen lanes per super-block, lane j fitting sub-block j (the same arithmetic as one thread
// doing all sixteen in turn): the super-block's largest scale and min meet by shuffles within
// the sixteen lanes, each lane requantises its own sub-block, and the 2-bit levels are packed
// through LDS (byte 16 + 32 half + l holds the levels of elements 128 half + l + 32 s, s = 0..3).
__global__ __launch_bounds__(256) void encode_q2k_kernel(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                                         size_t nblocks) {
    __shared__ uint8_t lv[16][256];  // the levels of the workgroup's sixteen super-blocks
    const uint32_t j = threadIdx.x % 16, slot = threadIdx.x / 16;
    for (size_t base = (size_t)blockIdx.x * 16; base < nblocks; base += (size_t)gridDim.x * 16) {
        const size_t b = base + slot;
        const bool live = b < nblocks;
        const float *blk = src + (live ? b : 0) * 256;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const f32x4 v = *(const f32x4 *)(blk + 16 * j + i);
            x[i] = v.x;
            x[i + 1] = v.y;
            x[i + 2] = v.z;
            x[i + 3] = v.w;
        }
        uint8_t lev[16];
        float scale, mn;
        q2k_fit(x, lev, &scale, &mn);
        float max_scale = scale, max_min = mn;
#pragma unroll
        for (int o = 8; o >= 1; o /= 2) {
            max_scale = fmaxf(max_scale, __shfl_xor(max_scale, o, 16));
            max_min = fmaxf(max_min, __shfl_xor(max_min, o, 16));
        }
        uint32_t packed = 0, d = 0, dmin = 0;
        if (max_scale > 0.0f) {
            packed = (uint8_t)nearest_int((15.0f / max_scale) * scale);
            d = float_to_half_bits(max_scale / 15.0f);
        }
        if (max_min > 0.0f) {
            packed |= (uint32_t)(uint8_t)((uint8_t)nearest_int((15.0f / max_min) * mn) << 4);
            dmin = float_to_half_bits(max_min / 15.0f);
        }
        packed &= 0xffu;
        const float sc = half_bits_to_float(d) * (float)(packed & 15u);
        if (sc != 0.0f) {
            const float dm = half_bits_to_float(dmin) * (float)(packed >> 4);
#pragma unroll
            for (int i = 0; i < 16; i++) lev[i] = (uint8_t)clamp3(nearest_int((x[i] + dm) / sc));
        }
#pragma unroll
        for (int i = 0; i < 16; i++) lv[slot][16 * j + i] = lev[i];
        __syncthreads();
        if (live) {
            uint8_t *o = dst + b * 84;
            o[j] = (uint8_t)packed;
            // lane j packs quant bytes 4 j .. 4 j + 3: half = j / 8, l = 4 (j % 8) .. + 3
            const uint32_t half = j / 8;
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t l = 4 * (j % 8) + e, at = 128 * half + l;
                const uint32_t byte = lv[slot][at] | (lv[slot][at + 32] << 2) | (lv[slot][at + 64] << 4) |
                                      (lv[slot][at + 96] << 6);
                word |= byte << (8 * e);
            }
            *(uint32_t *)(o + 16 + 4 * j) = word;
            if (j == 0) *(uint32_t *)(o + 80) = d | (dmin << 16);
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void transpose_kernel(const float *__restrict__ src, float *__restrict__ dst,
                                                        uint32_t rows, uint32_t cols) {
    __shared__ float t[32][33];
    const uint32_t c0 = blockIdx.x * 32, r0 = blockIdx.y * 32, tx = threadIdx.x % 32, ty = threadIdx.x / 32;
    for (uint32_t i = ty; i < 32; i += 8)
        if (r0 + i < rows && c0 + tx < cols) t[i][tx] = src[(size_t)(r0 + i) * cols + c0 + tx];
    __syncthreads();
    for (uint32_t i = ty; i < 32; i += 8)
        if (c0 + i < cols && r0 + tx < rows) dst[(size_t)(c0 + i) * rows + r0 + tx] = t[tx][i];
}

// ---- products on resident rows ----
// One thread per output, ascending k, the decoded weight formed first and then multiplied and
// added with separate roundings: the reference's qlinear_ext kernel and its CPU matmul
// (ferrum_ref/src/kernels/matmul.rs:49-69) on the decoded weights, operation for operation.
template <uint32_t T>
__global__ __launch_bounds__(256) void ext_naive_kernel(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                        float *__restrict__ y, uint32_t rows, uint32_t k, uint32_t n) {
    using F = Fmt<T>;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)rows * n) return;
    const uint32_t r = (uint32_t)(idx / n), c = (uint32_t)(idx % n);
    const uint8_t *row = w + (size_t)c * (k / F::E) * F::B;
    const float *xr = x + (size_t)r * k;
    float acc = 0.0f;
    for (uint32_t kk = 0; kk < k; kk++) acc = acc + xr[kk] * F::at(row + (kk / F::E) * F::B, kk % F::E);
    y[idx] = acc;
}

// Batch-1 with an x that is not 16-byte aligned: one workgroup per output; thread t takes elements
// t, t + 256, ...; a tree sum ends it.
template <uint32_t T>
__global__ __launch_bounds__(256) void ext_gemv_kernel(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                       float *__restrict__ y, uint32_t k) {
    using F = Fmt<T>;
    __shared__ float red[4];
    const uint32_t c = blockIdx.x;
    const uint8_t *row = w + (size_t)c * (k / F::E) * F::B;
    float acc = 0.0f;
    for (uint32_t kk = threadIdx.x; kk < k; kk += 256) acc = fmaf(x[kk], F::at(row + (kk / F::E) * F::B, kk % F::E), acc);
    for (int o = 32; o; o >>= 1) acc += __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) y[c] = (red[0] + red[1]) + (red[2] + red[3]);
}

// ---- batch-1 GEMV on resident rows, the one-row path ----
// A lane takes whole segments of a row (F16: 8 elements, FP8: 16, MXFP4: a block of 32, Q2_K: 32
// elements of one half super-block), loads the segment's x once and uses it for R rows (1, 2, 4 or
// 8), decodes the weights in registers and accumulates in f32: per segment the block's integer-valued
// codes are summed against x and the block scale is applied once (FP8 and Q2_K: the scale times
// the segment's sum, MXFP4: the power-of-two scale likewise). L lanes share a group of rows
// (segments l, l + L, ...), summed by shuffles and, for L > 64, through LDS. Rows are GGUF rows
// of B-byte blocks at any byte offset: a segment that is not 4-byte aligned is loaded as the
// dwords around it and realigned with v_alignbyte (allocations carry 256 zero bytes past their
// end, so the last block's over-read stays inside its buffer).

__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(const uint32_t *)p; }
// bytes [p, p + 16) for any p: five dwords from p rounded down, realigned
__device__ __forceinline__ u32x4 ld16_any(const uint8_t *p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint8_t *q = p - sh;  // derived from p, so the loads stay global ones
    const uint32_t d0 = ld32(q), d1 = ld32(q + 4), d2 = ld32(q + 8), d3 = ld32(q + 12), d4 = ld32(q + 16);
    return u32x4{__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh),
                 __builtin_amdgcn_alignbyte(d3, d2, sh), __builtin_amdgcn_alignbyte(d4, d3, sh)};
}
__device__ __forceinline__ float lo_half(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)v); }
__device__ __forceinline__ float hi_half(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}
__device__ __forceinline__ float ubyte(uint32_t v, int i) { return (float)((v >> (8 * i)) & 0xffu); }

template <uint32_t T>
struct ExtSeg;

template <>
struct ExtSeg<FH_F16> {  // segment s: halves 8 s .. 8 s + 7 of the row (16-byte aligned)
    static constexpr uint32_t SPB = 4, XN = 8;
    struct W {
        u32x4 q;
    };
    __device__ static void load(const uint8_t *row, uint32_t s, W &w) { w.q = *(const u32x4 *)(row + 16 * s); }
    __device__ static uint32_t xat(uint32_t s) { return 8 * s; }
    __device__ static float dot(const W &w, const float (&x)[XN]) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a = fmaf(x[2 * i], lo_half(w.q[i]), a);
            a = fmaf(x[2 * i + 1], hi_half(w.q[i]), a);
        }
        return a;
    }
};

// FP8 (fp8.rs:34-63): segment s = codes 16 p .. 16 p + 15 of block s / 2, p = s % 2, times the
// block's f16 scale. gfx950's conversions read OCP E4M3 / E5M2 (the reference's formats: E4M3
// NaN at 0x7f and 0xff only, E5M2 with infinities), two codes per instruction.
template <bool E5M2>
struct Fp8Seg {
    static constexpr uint32_t SPB = 2, XN = 16;
    struct W {
        uint32_t d;
        u32x4 c;
    };
    __device__ static void load(const uint8_t *row, uint32_t s, W &w) {
        const uint8_t *blk = row + 34 * (s / 2);
        w.d = *(const uint16_t *)blk;
        w.c = ld16_any(blk + 2 + 16 * (s % 2));
    }
    __device__ static uint32_t xat(uint32_t s) { return 16 * s; }
    __device__ static float dot(const W &w, const float (&x)[XN]) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int v = (int)w.c[i];
            const auto p0 = E5M2 ? __builtin_amdgcn_cvt_pk_f32_bf8(v, false) : __builtin_amdgcn_cvt_pk_f32_fp8(v, false);
            const auto p1 = E5M2 ? __builtin_amdgcn_cvt_pk_f32_bf8(v, true) : __builtin_amdgcn_cvt_pk_f32_fp8(v, true);
            a = fmaf(x[4 * i], p0[0], a);
            a = fmaf(x[4 * i + 1], p0[1], a);
            a = fmaf(x[4 * i + 2], p1[0], a);
            a = fmaf(x[4 * i + 3], p1[1], a);
        }
        return lo_half(w.d) * a;
    }
};
template <>
struct ExtSeg<FH_FP8_E4M3> : Fp8Seg<false> {};
template <>
struct ExtSeg<FH_FP8_E5M2> : Fp8Seg<true> {};

// MXFP4 (mxfp4.rs:13-33): segment = block s (E8M0 byte, then element i < 16 in the low nibble of
// byte 1 + i, element 16 + i in its high nibble). gfx950's scaled FP4 conversion turns one byte
// into its two E2M1 values (0, 0.5, 1, 1.5, 2, 3, 4, 6 and negatives: the reference's table halved),
// so sum(x v) = 2 sum(x e2m1) exactly, then times the half scale.
template <>
struct ExtSeg<FH_MXFP4> {
    static constexpr uint32_t SPB = 1, XN = 32;
    struct W {
        uint32_t e;
        u32x4 q;
    };
    __device__ static void load(const uint8_t *row, uint32_t s, W &w) {
        const uint8_t *blk = row + 17 * s;
        w.e = blk[0];
        w.q = ld16_any(blk + 1);
    }
    __device__ static uint32_t xat(uint32_t s) { return 32 * s; }
    __device__ static float dot(const W &w, const float (&x)[XN]) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // byte 4 i + b: elements 4 i + b (low nibble) and 16 + 4 i + b (high nibble)
            const auto v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w.q[i], 1.0f, 0);
            const auto v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w.q[i], 1.0f, 1);
            const auto v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w.q[i], 1.0f, 2);
            const auto v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w.q[i], 1.0f, 3);
            a = fmaf(x[4 * i], v0[0], a);
            a = fmaf(x[16 + 4 * i], v0[1], a);
            a = fmaf(x[4 * i + 1], v1[0], a);
            a = fmaf(x[16 + 4 * i + 1], v1[1], a);
            a = fmaf(x[4 * i + 2], v2[0], a);
            a = fmaf(x[16 + 4 * i + 2], v2[1], a);
            a = fmaf(x[4 * i + 3], v3[0], a);
            a = fmaf(x[16 + 4 * i + 3], v3[1], a);
        }
        return (a * 2.0f) * mx_half_scale(w.e);
    }
};

// Q2_K (blocks.rs:201-250): segment s of super-block s / 8: half h = (s % 8) / 4, quant bytes
// 16 + 32 h + 8 g .. + 7 (g = s % 4), i.e. elements 128 h + 32 j + 8 g + l for the four 2-bit
// planes j; plane j's sub-block scale byte is 8 h + 2 j + g / 2. Per plane: d (sc & 15) sum(x q)
// - dmin (sc >> 4) sum(x).
template <>
struct ExtSeg<FH_Q2_K> {
    static constexpr uint32_t SPB = 8, XN = 32;
    struct W {
        uint32_t q0, q1, s0, s1, dd;
    };
    __device__ static void load(const uint8_t *row, uint32_t s, W &w) {
        const uint8_t *blk = row + 84 * (s / 8);
        const uint32_t h = (s % 8) / 4, g = s % 4;
        w.q0 = ld32(blk + 16 + 32 * h + 8 * g);
        w.q1 = ld32(blk + 20 + 32 * h + 8 * g);
        w.s0 = ld32(blk + 8 * h);
        w.s1 = ld32(blk + 8 * h + 4);
        w.dd = ld32(blk + 80);
    }
    // x of the segment: plane j's 8 elements at x[xat(s) + 32 j ..]
    __device__ static uint32_t xat(uint32_t s) { return 256 * (s / 8) + 128 * ((s % 8) / 4) + 8 * (s % 4); }
    __device__ static float dot(const W &w, const float (&x)[XN], uint32_t s, const float (&xs)[4]) {
        const float d = lo_half(w.dd), dmin = hi_half(w.dd);
        const uint32_t g2 = (s % 4) / 2;
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t v0 = (w.q0 >> (2 * j)) & 0x03030303u, v1 = (w.q1 >> (2 * j)) & 0x03030303u;
            float t = 0.0f;
#pragma unroll
            for (int l = 0; l < 4; l++) t = fmaf(x[8 * j + l], ubyte(v0, l), t);
#pragma unroll
            for (int l = 0; l < 4; l++) t = fmaf(x[8 * j + 4 + l], ubyte(v1, l), t);
            const uint32_t sc = ((j < 2 ? w.s0 : w.s1) >> (8 * (2 * (j % 2) + g2))) & 0xffu;
            a = fmaf(d * (float)(sc & 15u), t, a);
            a = fmaf(-(dmin * (float)(sc >> 4)), xs[j], a);
        }
        return a;
    }
};

template <uint32_t T>
__device__ __forceinline__ void ext_load_x(const float *__restrict__ x, uint32_t s, float (&xv)[ExtSeg<T>::XN]) {
    using S = ExtSeg<T>;
    if constexpr (T == FH_Q2_K) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f32x4 a = *(const f32x4 *)(x + S::xat(s) + 32 * j), b = *(const f32x4 *)(x + S::xat(s) + 32 * j + 4);
#pragma unroll
            for (int l = 0; l < 4; l++) {
                xv[8 * j + l] = a[l];
                xv[8 * j + 4 + l] = b[l];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < (int)S::XN / 4; i++) {
            const f32x4 a = *(const f32x4 *)(x + S::xat(s) + 4 * i);
#pragma unroll
            for (int l = 0; l < 4; l++) xv[4 * i + l] = a[l];
        }
    }
}

template <uint32_t T, uint32_t R>
__global__ __launch_bounds__(256) void ext_gemv_rows_kernel(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                            float *__restrict__ y, uint32_t k, uint32_t n,
                                                            uint32_t lg) {
    using F = Fmt<T>;
    using S = ExtSeg<T>;
    constexpr uint32_t kExtRows = R;
    __shared__ float red[4][kExtRows];
    const uint32_t L = 1u << lg, tid = threadIdx.x, l = tid & (L - 1);
    const uint32_t grp = blockIdx.x * (256u >> lg) + (tid >> lg), r0 = grp * kExtRows;
    const size_t row_bytes = (size_t)(k / F::E) * F::B;
    const uint32_t segs = (k / F::E) * S::SPB;
    float acc[kExtRows] = {};
    if (r0 < n) {
        const uint8_t *rows[kExtRows];
#pragma unroll
        for (uint32_t r = 0; r < kExtRows; r++) rows[r] = w + (size_t)min(r0 + r, n - 1) * row_bytes;
#pragma unroll 2
        for (uint32_t s = l; s < segs; s += L) {
            float xv[S::XN];
            ext_load_x<T>(x, s, xv);
            typename S::W wv[kExtRows];
#pragma unroll
            for (uint32_t r = 0; r < kExtRows; r++) S::load(rows[r], s, wv[r]);
            if constexpr (T == FH_Q2_K) {
                float xs[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float t = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; e++) t += xv[8 * j + e];
                    xs[j] = t;
                }
#pragma unroll
                for (uint32_t r = 0; r < kExtRows; r++) acc[r] += S::dot(wv[r], xv, s, xs);
            } else {
#pragma unroll
                for (uint32_t r = 0; r < kExtRows; r++) acc[r] += S::dot(wv[r], xv);
            }
        }
    }
    // sum over the L lanes of the group: within the wavefront by shuffles, across wavefronts in LDS
#pragma unroll
    for (uint32_t o = 32; o; o >>= 1)
        if (o < L)
#pragma unroll
            for (uint32_t r = 0; r < kExtRows; r++) acc[r] += __shfl_xor(acc[r], (int)o);
    if (L > 64) {  // uniform over the launch
        if ((tid & 63) == 0)
#pragma unroll
            for (uint32_t r = 0; r < kExtRows; r++) red[tid / 64][r] = acc[r];
        __syncthreads();
        if (l == 0) {
            const uint32_t w0 = tid / 64, nw = L / 64;
#pragma unroll
            for (uint32_t r = 0; r < kExtRows; r++) {
                float t = red[w0][r];
                for (uint32_t i = 1; i < nw; i++) t += red[w0 + i][r];
                acc[r] = t;
            }
        }
    }
    if (l == 0)
#pragma unroll
        for (uint32_t r = 0; r < kExtRows; r++)
            if (r0 + r < n) y[r0 + r] = acc[r];
}

// Rows per lane group R (at most max_rows: 8, 4, 2 or 1) and lanes per group 2^lg (at most 256 and
// at most the row's segments): the largest R whose grid still holds about four wavefronts per
// SIMD, with about four segments per lane where the grid is that large already.
void ext_gemv_shape(uint32_t segs, uint64_t n, uint32_t max_rows, uint32_t *rows, uint32_t *lg) {
    constexpr uint64_t kTargetLanes = 256ull * 4 * 4 * 64;
    auto floor_log2 = [](uint64_t v) {
        uint32_t l = 0;
        while ((2ull << l) <= v) l++;
        return l;
    };
    const uint32_t cap = min(8u, floor_log2(max(segs, 1u)));
    const uint32_t work = min(cap, floor_log2(max(segs / 4, 1u)));
    for (uint32_t r = max_rows;; r /= 2) {
        const uint64_t groups = (n + r - 1) / r;
        uint32_t l = work;
        while (l < cap && (groups << l) < kTargetLanes) l++;
        if ((groups << l) >= kTargetLanes || r == 1) {
            *rows = r;
            *lg = l;
            return;
        }
    }
}

// Several rows: 32 x 64 output tiles; per 32-k step the x tile and the decoded weight tile
// (64 columns) are staged in LDS, each thread accumulating 2 x 4 outputs in f32.
template <uint32_t T>
__global__ __launch_bounds__(256) void ext_tiled_kernel(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                        float *__restrict__ y, uint32_t rows, uint32_t k, uint32_t n) {
    using F = Fmt<T>;
    __shared__ float xs[32][33];
    __shared__ float ws[64][33];
    const uint32_t tid = threadIdx.x, r0 = blockIdx.y * 32, c0 = blockIdx.x * 64;
    const uint32_t tx = tid % 16, ty = tid / 16;  // columns tx + 16 j, rows ty + 16 i
    const size_t row_bytes = (size_t)(k / F::E) * F::B;
    float acc[2][4] = {};
    for (uint32_t k0 = 0; k0 < k; k0 += 32) {
        for (uint32_t e = tid; e < 32 * 32; e += 256) {
            const uint32_t r = e / 32, kk = e % 32;
            xs[r][kk] = r0 + r < rows ? x[(size_t)(r0 + r) * k + k0 + kk] : 0.0f;
        }
        for (uint32_t e = tid; e < 64 * 32; e += 256) {
            const uint32_t c = e / 32, kk = e % 32, kg = k0 + kk;
            ws[c][kk] = c0 + c < n ? F::at(w + (size_t)(c0 + c) * row_bytes + (kg / F::E) * F::B, kg % F::E) : 0.0f;
        }
        __syncthreads();
        for (uint32_t kk = 0; kk < 32; kk++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(xs[ty + 16 * i][kk], ws[tx + 16 * j][kk], acc[i][j]);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t r = r0 + ty + 16 * i, c = c0 + tx + 16 * j;
            if (r < rows && c < n) y[(size_t)r * n + c] = acc[i][j];
        }
}

unsigned grid_of(size_t items, unsigned per) {
    const size_t g = (items + per - 1) / per;
    return (unsigned)(g < 65536 ? (g ? g : 1) : 65536);
}

template <uint32_t T>
hipError_t decode_as(hipStream_t s, const uint8_t *src, float *dst, size_t n) {
    decode_ext_kernel<T><<<grid_of(n, 256), 256, 0, s>>>(src, dst, n);
    return hipGetLastError();
}

template <uint32_t T>
hipError_t linear_as(hipStream_t s, fh_path path, const uint8_t *w, const float *x, float *y, size_t rows, size_t k,
                     size_t n) {
    if (path == FH_PATH_NAIVE) {
        ext_naive_kernel<T><<<(unsigned)((rows * n + 255) / 256), 256, 0, s>>>(w, x, y, (uint32_t)rows, (uint32_t)k,
                                                                               (uint32_t)n);
    } else if (path == FH_PATH_GEMV && ((uintptr_t)x & 15)) {  // x not 16-byte aligned: scalar loads
        ext_gemv_kernel<T><<<(unsigned)n, 256, 0, s>>>(w, x, y, (uint32_t)k);
    } else if (path == FH_PATH_GEMV) {
        uint32_t r, lg;
        // MXFP4 reads more x than weight bytes per segment: up to eight rows share it
        constexpr uint32_t kMaxRows = T == FH_MXFP4 ? 8 : 4;
        ext_gemv_shape((uint32_t)(k / Fmt<T>::E * ExtSeg<T>::SPB), n, kMaxRows, &r, &lg);
        const uint64_t per_cta = (256u >> lg) * r;
        const unsigned grid = (unsigned)((n + per_cta - 1) / per_cta);
        if (r == 8)
            ext_gemv_rows_kernel<T, kMaxRows><<<grid, 256, 0, s>>>(w, x, y, (uint32_t)k, (uint32_t)n, lg);
        else if (r == 4)
            ext_gemv_rows_kernel<T, 4><<<grid, 256, 0, s>>>(w, x, y, (uint32_t)k, (uint32_t)n, lg);
        else if (r == 2)
            ext_gemv_rows_kernel<T, 2><<<grid, 256, 0, s>>>(w, x, y, (uint32_t)k, (uint32_t)n, lg);
        else
            ext_gemv_rows_kernel<T, 1><<<grid, 256, 0, s>>>(w, x, y, (uint32_t)k, (uint32_t)n, lg);
    } else {
        const dim3 grid((unsigned)((n + 63) / 64), (unsigned)((rows + 31) / 32));
        ext_tiled_kernel<T><<<grid, 256, 0, s>>>(w, x, y, (uint32_t)rows, (uint32_t)k, (uint32_t)n);
    }
    return hipGetLastError();
}

}  // namespace

bool ext_kind(int kind) {
    return kind == FH_F16 || kind == FH_MXFP4 || kind == FH_Q2_K || kind == FH_FP8_E4M3 || kind == FH_FP8_E5M2;
}

bool ext_layout(uint32_t ty, size_t *block_bytes, size_t *block_elems) {
    size_t b = 0, e = 32;
    switch (ty) {
    case FH_F16: b = 64; break;
    case FH_FP8_E4M3:
    case FH_FP8_E5M2: b = 34; break;
    case FH_MXFP4: b = 17; break;
    case FH_Q4_1: b = 20; break;
    case FH_Q5_0: b = 22; break;
    case FH_Q5_1: b = 24; break;
    case FH_Q8_1: b = 36; break;
    case FH_Q2_K: b = 84, e = 256; break;
    case FH_Q3_K: b = 110, e = 256; break;
    case FH_Q4_K: b = 144, e = 256; break;
    case FH_Q5_K: b = 176, e = 256; break;
    case FH_Q6_K: b = 210, e = 256; break;
    default: return false;
    }
    if (block_bytes) *block_bytes = b;
    if (block_elems) *block_elems = e;
    return true;
}

const char *ext_label(int kind) {
    switch (kind) {
    case FH_F16: return "F16";
    case FH_MXFP4: return "MXFP4";
    case FH_Q2_K: return "Q2_K";
    case FH_FP8_E4M3: return "FP8 E4M3";
    case FH_FP8_E5M2: return "FP8 E5M2";
    default: return "block";
    }
}

hipError_t launch_decode_ext(hipStream_t s, uint32_t ty, const uint8_t *src, float *dst, size_t n) {
    if (!n) return hipSuccess;
    switch (ty) {
    case FH_F16: return decode_as<FH_F16>(s, src, dst, n);
    case FH_FP8_E4M3: return decode_as<FH_FP8_E4M3>(s, src, dst, n);
    case FH_FP8_E5M2: return decode_as<FH_FP8_E5M2>(s, src, dst, n);
    case FH_MXFP4: return decode_as<FH_MXFP4>(s, src, dst, n);
    case FH_Q4_1: return decode_as<FH_Q4_1>(s, src, dst, n);
    case FH_Q5_0: return decode_as<FH_Q5_0>(s, src, dst, n);
    case FH_Q5_1: return decode_as<FH_Q5_1>(s, src, dst, n);
    case FH_Q8_1: return decode_as<FH_Q8_1>(s, src, dst, n);
    case FH_Q2_K: return decode_as<FH_Q2_K>(s, src, dst, n);
    case FH_Q3_K: return decode_as<FH_Q3_K>(s, src, dst, n);
    case FH_Q4_K: return decode_as<FH_Q4_K>(s, src, dst, n);
    case FH_Q5_K: return decode_as<FH_Q5_K>(s, src, dst, n);
    case FH_Q6_K: return decode_as<FH_Q6_K>(s, src, dst, n);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_encode_ext(hipStream_t s, int kind, const float *src, uint8_t *dst, size_t n) {
    if (!n) return hipSuccess;
    switch (kind) {
    case FH_F16: encode_f16_kernel<<<grid_of(n, 256), 256, 0, s>>>(src, dst, n); break;
    case FH_FP8_E4M3: encode_fp8_kernel<false><<<grid_of(n / 32, 256), 256, 0, s>>>(src, dst, n / 32); break;
    case FH_FP8_E5M2: encode_fp8_kernel<true><<<grid_of(n / 32, 256), 256, 0, s>>>(src, dst, n / 32); break;
    case FH_MXFP4: encode_mxfp4_kernel<<<grid_of(n / 32, 256), 256, 0, s>>>(src, dst, n / 32); break;
    case FH_Q2_K: encode_q2k_kernel<<<grid_of(n / 256, 16), 256, 0, s>>>(src, dst, n / 256); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_transpose(hipStream_t s, const float *src, float *dst, size_t rows, size_t cols) {
    if (!rows || !cols) return hipSuccess;
    const dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
    transpose_kernel<<<grid, 256, 0, s>>>(src, dst, (uint32_t)rows, (uint32_t)cols);
    return hipGetLastError();
}

hipError_t launch_linear_ext(hipStream_t s, int kind, fh_path path, const uint8_t *w, const float *x, float *y,
                             size_t rows, size_t k, size_t n) {
    if (!rows || !n) return hipSuccess;
    switch (kind) {
    case FH_F16: return linear_as<FH_F16>(s, path, w, x, y, rows, k, n);
    case FH_FP8_E4M3: return linear_as<FH_FP8_E4M3>(s, path, w, x, y, rows, k, n);
    case FH_FP8_E5M2: return linear_as<FH_FP8_E5M2>(s, path, w, x, y, rows, k, n);
    case FH_MXFP4: return linear_as<FH_MXFP4>(s, path, w, x, y, rows, k, n);
    case FH_Q2_K: return linear_as<FH_Q2_K>(s, path, w, x, y, rows, k, n);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace fh
