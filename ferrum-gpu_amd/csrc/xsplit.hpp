// The fast GEMM's x operand (FH_PATH_TILED_FAST), one row per 256-thread workgroup: x = hi + lo
// with hi = f16(x) (saturated) in the MFMA operand order and lo = e4m3 of (x - hi) 2^s in natural
// order (s per row: 2^(E-10) > |lo| for the row's largest |x| in [2^E, 2^(E+1)), so s = 18 - E puts
// |lo| 2^s under 2^8; the row's tail up to a multiple of 64 is zero), and xsc[m] = the E8M0 byte
// of 2^-s, four copies. Used by split_x_kernel and by the scoring forward's producers, which
// write a row they hold in LDS straight into this form.
#ifndef FERRUM_XSPLIT_HPP
#define FERRUM_XSPLIT_HPP

#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.hpp"

namespace fh {

__device__ __forceinline__ _Float16 f16_sat(float e) { return (_Float16)fminf(fmaxf(e, -65504.0f), 65504.0f); }

__device__ __forceinline__ uint32_t fp8x4(float a, float b, float c, float d) {
    // e4m3 has no infinity: values beyond +-448 would become NaN, so they are clamped first
    const auto cl = [](float v) { return fminf(fmaxf(v, -448.0f), 448.0f); };
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(a), cl(b), 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(c), cl(d), w, true);
    return (uint32_t)w;
}

// Row m (K values, float4 q from get(q)) by the workgroup's 256 threads; red: 4 floats of LDS.
// The row is read once: thread t keeps float4 t + 256 i for i < kKeep in registers (rows up to
// 8192 wide; wider rows read the rest twice). Float4 q is elements 4 (q % 8) .. + 3 of block
// q / 8, so eight consecutive lanes hold one block.
template <int KIND, class Get>
__device__ __forceinline__ void split_row_fast(Get get, uint32_t m, uint32_t K, _Float16 *__restrict__ xh,
                                               uint8_t *__restrict__ xl, int32_t *__restrict__ xsc, float *red) {
    typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
    typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
    const uint32_t tid = threadIdx.x, nb = K / 32, K64 = (K + 63) / 64 * 64;
    if (K64 != K && tid < 8) *(uint32_t *)(xl + (size_t)m * K64 + K + 4 * tid) = 0u;  // the row's zero tail
    constexpr int kKeep = 8;
    const uint32_t nq = K / 4;
    f32x4 v[kKeep];
    float mx = 0.0f;
    auto amax = [](f32x4 a) { return fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))); };
#pragma unroll
    for (int i = 0; i < kKeep; i++) {
        const uint32_t q = tid + 256 * i;
        v[i] = q < nq ? get(q) : f32x4{0.f, 0.f, 0.f, 0.f};
        mx = fmaxf(mx, amax(v[i]));
    }
    for (uint32_t q = tid + 256 * kKeep; q < nq; q += 256) mx = fmaxf(mx, amax(get(q)));
    mx = wave_reduce(mx, MaxOp());
    if (tid % 64 == 0) red[tid / 64] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // 2^E <= mx < 2^(E+1); |lo| < 2^(E-10); s = 18 - E puts |lo| 2^s below 2^8
    int sc = 0;
    if (mx > 0.0f && mx <= 3.4028235e38f) sc = 18 - ((int)(__float_as_uint(mx) >> 23) - 127);
    sc = sc < -126 ? -126 : (sc > 126 ? 126 : sc);
    const float f = __uint_as_float((uint32_t)(127 + sc) << 23);
    if (tid == 0) xsc[m] = (127 - sc) * 0x01010101;
    const int j = tid % 8;
    // (q < nq is the same for the eight lanes of a block: nq is a multiple of 8)
    auto put = [&](uint32_t qi, f32x4 w) {
        const uint32_t t = qi / 8;
        _Float16 h[4];
#pragma unroll
        for (int q = 0; q < 4; q++) h[q] = f16_sat(w[q]);
        *(uint32_t *)(xl + (size_t)m * K64 + t * 32 + 4 * j) =
            fp8x4((w.x - (float)h[0]) * f, (w.y - (float)h[1]) * f, (w.z - (float)h[2]) * f, (w.w - (float)h[3]) * f);
        _Float16 *out = xh + ((size_t)m * nb + t) * 32;
        if constexpr (KIND == FH_Q8_0) {
            // positions 4j..4j+3 hold elements 4j + {0, 2, 1, 3}
            *(h16x4 *)(out + 4 * j) = h16x4{h[0], h[2], h[1], h[3]};
        } else {
            // positions 8i..8i+7 hold elements 4i + {0, 2, 1, 3} and 16 + 4i + {0, 2, 1, 3}: lane i < 4
            // takes lane i + 4's four values and writes the eight
            _Float16 o[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
                o[q] = __builtin_bit_cast(_Float16, (uint16_t)__shfl_xor((int)__builtin_bit_cast(uint16_t, h[q]), 4, 8));
            if (j < 4) *(h16x8 *)(out + 8 * j) = h16x8{h[0], h[2], h[1], h[3], o[0], o[2], o[1], o[3]};
        }
    };
#pragma unroll
    for (int i = 0; i < kKeep; i++) {
        const uint32_t q = tid + 256 * i;
        if (q < nq) put(q, v[i]);
    }
    for (uint32_t q = tid + 256 * kKeep; q < nq; q += 256) put(q, get(q));
}

}  // namespace fh

#endif
