// The fast GEMM's x operand (FH_PATH_TILED_FAST): x = hi + lo with hi = f16(x) (saturated) in the
// MFMA operand order, and lo = e4m3 of (x - hi) 2^s with s per row and 32-element block: for the
// block's largest |x| in [2^E, 2^(E+1)), 2^(E-10) > |lo|, so s = 18 - E puts |lo| 2^s under 2^8.
// Three planes:
// - xh: [M][K/32 blocks][32] f16, each block in the operand order of fast_elem_of_pos;
// - xl: [M][K64] e4m3 (K rounded up to 64), each 64 k (blocks 2p, 2p + 1) stored as block 2p's
//   elements 0-15, block 2p + 1's 0-15, block 2p's 16-31, block 2p + 1's 16-31 (lo_byte). The
//   scaled fp8 MFMA takes a lane's bytes 0-15 as its row's first scale block and bytes 16-31 as the
//   second, so each block then meets its own scale. An odd block count leaves the last pair's
//   second block zero;
// - xsb: [K64 / 64 pairs][MS rows][2] E8M0 bytes of 2^-s (block 2p, then 2p + 1), MS = M rounded
//   up to 8 (xsb_rows), so a tile's rows of one pair are contiguous and 16-byte aligned.
// A producer that holds a row's block writes that block's part of all three, so no pass over a
// whole row is needed: split_x_kernel, the scoring forward's producers (split_row_fast) and the
// SwiGLU GEMM epilogue (split_chunk4, eight lanes per block).
#ifndef FERRUM_XSPLIT_HPP
#define FERRUM_XSPLIT_HPP

#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.hpp"

namespace fh {

__host__ __device__ constexpr uint32_t xsb_rows(uint32_t M) { return (M + 7) / 8 * 8; }

// Byte of a row's x lo holding element e (0..31) of block b.
__device__ __forceinline__ uint32_t lo_byte(uint32_t b, uint32_t e) {
    return (b / 2) * 64 + (b % 2) * 16 + (e / 16) * 32 + e % 16;
}

// The scale byte of row m's block b.
__device__ __forceinline__ size_t xsb_at(uint32_t m, uint32_t b, uint32_t MS) {
    return ((size_t)(b / 2) * MS + m) * 2 + b % 2;
}

// The k order inside a block of the f16 operands: position p holds element fast_elem_of_pos(p).
// The unpack produces f16 pairs from a quant dword w: for Q8_0 the bytes (0, 2) and (1, 3), i.e.
// elements 4i + {0, 2, 1, 3}; for Q4_0 the low nibbles of bytes (0, 2), (1, 3), then the high
// nibbles, i.e. elements 4i + {0, 2, 1, 3} and 16 + 4i + {0, 2, 1, 3}.
template <int KIND>
__host__ __device__ constexpr int fast_elem_of_pos(int p) {
    const int sw = (p & 3) == 1 ? 2 : (p & 3) == 2 ? 1 : (p & 3);  // {0, 2, 1, 3}
    if (KIND == FH_Q8_0) return (p & ~3) + sw;
    return ((p % 8) < 4 ? 4 * (p / 8) : 16 + 4 * (p / 8)) + sw;
}

typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ _Float16 f16_sat(float e) { return (_Float16)fminf(fmaxf(e, -65504.0f), 65504.0f); }

__device__ __forceinline__ uint32_t fp8x4(float a, float b, float c, float d) {
    // e4m3 has no infinity: values beyond +-448 would become NaN, so they are clamped first
    const auto cl = [](float v) { return fminf(fmaxf(v, -448.0f), 448.0f); };
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(a), cl(b), 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(c), cl(d), w, true);
    return (uint32_t)w;
}

// s for a block whose largest |x| is mx (see above); zero and non-finite blocks keep s = 0.
__device__ __forceinline__ int lo_shift(float mx) {
    int sc = 0;
    if (mx > 0.0f && mx <= 3.4028235e38f) sc = 18 - ((int)(__float_as_uint(mx) >> 23) - 127);
    return sc < -126 ? -126 : (sc > 126 ? 126 : sc);
}

// The empty second block of the last pair of a row with an odd block count nb: zero lo, scale 2^0.
__device__ __forceinline__ void split_tail(uint32_t m, uint32_t nb, uint32_t K64, uint32_t MS, uint8_t *__restrict__ xl,
                                           uint8_t *__restrict__ xsb, uint32_t part) {
    *(u32x4 *)(xl + (size_t)m * K64 + lo_byte(nb, 16 * part)) = u32x4{0u, 0u, 0u, 0u};
    if (part == 0) xsb[xsb_at(m, nb, MS)] = 127;
}

// Elements 4 j .. 4 j + 3 of row m's block b, w, with the seven other lanes of an 8-lane group
// (lanes 8 g .. 8 g + 7, j = lane % 8) holding the block's other elements: the group finds the
// block's largest |x| among itself, then each lane writes its part of hi (for Q4_0 the lanes j < 4,
// with lane j + 4's values) and of lo, and lane 0 the scale byte. Every lane of the group must
// take part. MS = xsb_rows(M), nb = K / 32, K64 = K rounded up to 64.
// Cross-lane moves inside 8-lane groups on the DPP paths (no LDS): xor 1 and xor 2 inside a quad,
// and lane i <- lane 7 - i (row_half_mirror).
constexpr int kDppXor1 = 0xb1, kDppXor2 = 0x4e, kDppRev4 = 0x1b, kDppHalfMirror = 0x141;
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}

// The chunk's destinations: hb = the block's 32 hi halves, lw = its lo dword (lo_byte(b, 4 j) in
// the row), sb = the block's scale byte.
template <int KIND>
__device__ __forceinline__ void split_chunk4_at(f32x4 w, uint32_t j, _Float16 *__restrict__ hb, uint8_t *__restrict__ lw,
                                                uint8_t *__restrict__ sb) {
    typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
    typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
    float mx = fmaxf(fmaxf(fabsf(w.x), fabsf(w.y)), fmaxf(fabsf(w.z), fabsf(w.w)));
    mx = fmaxf(mx, dpp_f<kDppXor1>(mx));
    mx = fmaxf(mx, dpp_f<kDppXor2>(mx));
    mx = fmaxf(mx, dpp_f<kDppHalfMirror>(mx));  // the other quad's maximum
    const int sc = lo_shift(mx);
    const float f = __uint_as_float((uint32_t)(127 + sc) << 23);
    if (j == 0) *sb = (uint8_t)(127 - sc);
    _Float16 h[4];
#pragma unroll
    for (int q = 0; q < 4; q++) h[q] = f16_sat(w[q]);
    *(uint32_t *)lw =
        fp8x4((w.x - (float)h[0]) * f, (w.y - (float)h[1]) * f, (w.z - (float)h[2]) * f, (w.w - (float)h[3]) * f);
    _Float16 *out = hb;
    if constexpr (KIND == FH_Q8_0) {
        // positions 4j..4j+3 hold elements 4j + {0, 2, 1, 3}
        *(h16x4 *)(out + 4 * j) = h16x4{h[0], h[2], h[1], h[3]};
    } else {
        // positions 8i..8i+7 hold elements 4i + {0, 2, 1, 3} and 16 + 4i + {0, 2, 1, 3}: lane i < 4
        // takes lane i + 4's four values (reversed inside each quad, then mirrored inside the
        // eight: lane i reads lane 7 - i, which holds lane 4 + i's) and writes the eight
        const uint32_t p02 = __builtin_bit_cast(uint32_t, f16x2v{h[0], h[2]}),
                       p13 = __builtin_bit_cast(uint32_t, f16x2v{h[1], h[3]});
        const f16x2v o02 = __builtin_bit_cast(f16x2v, dpp_u<kDppHalfMirror>(dpp_u<kDppRev4>(p02))),
                     o13 = __builtin_bit_cast(f16x2v, dpp_u<kDppHalfMirror>(dpp_u<kDppRev4>(p13)));
        if (j < 4) *(h16x8 *)(out + 8 * j) = h16x8{h[0], h[2], h[1], h[3], o02[0], o02[1], o13[0], o13[1]};
    }
}
template <int KIND>
__device__ __forceinline__ void split_chunk4(f32x4 w, uint32_t m, uint32_t b, uint32_t j, uint32_t MS, uint32_t nb,
                                             uint32_t K64, _Float16 *__restrict__ xh, uint8_t *__restrict__ xl,
                                             uint8_t *__restrict__ xsb) {
    split_chunk4_at<KIND>(w, j, xh + ((size_t)m * nb + b) * 32, xl + (size_t)m * K64 + lo_byte(b, 4 * j),
                          xsb + xsb_at(m, b, MS));
    if (nb % 2 && b == nb - 1 && j < 2) split_tail(m, nb, K64, MS, xl, xsb, j);
}

// Row m (K values, float4 q from get(q)) by the workgroup's 256 threads (rows of M). Float4 q is
// elements 4 (q % 8) .. + 3 of block q / 8, so eight consecutive lanes hold one block
// (split_chunk4). A thread requests its first eight float4s before it writes any.
template <int KIND, class Get>
__device__ __forceinline__ void split_row_fast(Get get, uint32_t m, uint32_t M, uint32_t K, _Float16 *__restrict__ xh,
                                               uint8_t *__restrict__ xl, uint8_t *__restrict__ xsb) {
    const uint32_t tid = threadIdx.x, nb = K / 32, K64 = (K + 63) / 64 * 64, MS = xsb_rows(M);
    constexpr int kKeep = 8;
    const uint32_t nq = K / 4;
    f32x4 v[kKeep];
#pragma unroll
    for (int i = 0; i < kKeep; i++) {
        const uint32_t q = tid + 256 * i;
        v[i] = q < nq ? get(q) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // (q < nq is the same for the eight lanes of a block: nq is a multiple of 8)
#pragma unroll
    for (int i = 0; i < kKeep; i++) {
        const uint32_t q = tid + 256 * i;
        if (q < nq) split_chunk4<KIND>(v[i], m, q / 8, q % 8, MS, nb, K64, xh, xl, xsb);
    }
    for (uint32_t q = tid + 256 * kKeep; q < nq; q += 256)
        split_chunk4<KIND>(get(q), m, q / 8, q % 8, MS, nb, K64, xh, xl, xsb);
}

}  // namespace fh

#endif
