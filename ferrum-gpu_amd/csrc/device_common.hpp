// Device helpers shared by the kernels: exact f16 <-> f32 bit conversions, the saturating
// casts of the reference's Rust code, and dword-window loads of the 2-byte-aligned GGUF blocks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fh {

// Resident weights are stored as tiles: the rows of a weight are taken in groups of 32. In the
// quant plane the blocks of a group are stored block by block, the group's 32 rows side by side:
// the quants of block b of row n are slot tile_slot(n, b, nb) (QB bytes each), nb being the
// row's block count. In the scale plane a group's blocks are taken eight at a time, each row's
// eight f16 scales side by side (16 bytes), so the scale of block b of row n is element
// scale_slot(n, b, nb); the last run of eight is padded with zero scales.
__host__ __device__ __forceinline__ size_t tile_slot(size_t n, size_t b, size_t nb) {
    return ((n >> 5) * nb + b) * 32 + (n & 31);
}
__host__ __device__ __forceinline__ size_t scale_slot(size_t n, size_t b, size_t nb) {
    return (((n >> 5) * ((nb + 7) >> 3) + (b >> 3)) * 32 + (n & 31)) * 8 + (b & 7);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// IEEE binary16 bits -> f32, exact (subnormals normalised by count-leading-zeros). Restates
// ferrum_gguf/src/codec/f16.rs:4-22 with integer operations, so the result does not depend on
// the shader's denormal mode.
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    uint32_t sign = (h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            uint32_t shift = (uint32_t)__clz((int)man) - 21;
            uint32_t m = (man << shift) & 0x3ff;
            bits = sign | ((127u - 15u + 1u - shift) << 23) | (m << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    return __uint_as_float(bits);
}

// f32 -> binary16 bits, round to nearest even, overflow to infinity, NaN quiet
// (ferrum_gguf/src/codec/f16.rs:25-53), by integer operations.
__device__ __forceinline__ uint32_t float_to_half_bits(float x) {
    uint32_t b = __float_as_uint(x);
    uint32_t sign = (b >> 16) & 0x8000u;
    int32_t exp = (int32_t)((b >> 23) & 0xff);
    uint32_t man = b & 0x007fffffu;
    if (exp == 0xff) return sign | 0x7c00u | (man != 0 ? 0x200u : 0u);
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = man | 0x00800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t mid = 1u << (shift - 1u);
        uint32_t up = (rem > mid || (rem == mid && (half & 1u))) ? 1u : 0u;
        return sign | (half + up);
    }
    uint32_t half = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    uint32_t up = (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ? 1u : 0u;
    return sign | (half + up);
}

// Rust `f as i8` after f32::round: round half away from zero, saturate, NaN -> 0.
__device__ __forceinline__ int32_t round_sat_i8(float f) {
    if (f != f) return 0;
    float r = roundf(f);  // llvm.round: exact half-away-from-zero
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return (int32_t)r;
}

// Rust `(f as i32).clamp(0, 15)`: truncate toward zero, saturate, NaN -> 0, then clamp.
__device__ __forceinline__ int32_t trunc_clamp_0_15(float f) {
    if (f != f) return 0;
    float t = truncf(f);
    t = fminf(fmaxf(t, 0.0f), 15.0f);
    return (int32_t)t;
}

// A GGUF block starts at an even byte offset. Load the dword-aligned window that holds it
// (WORDS dwords starting at the block's offset rounded down to 4); the block's first byte is
// then at byte `(off & 3)` (0 or 2) of word 0. Reads at most 2 bytes past the block, which
// every allocation of this library pads for.
template <int WORDS>
__device__ __forceinline__ void load_window(const uint8_t *base, size_t off, uint32_t (&w)[WORDS]) {
    const uint32_t *p = (const uint32_t *)(base + (off & ~(size_t)3));
#pragma unroll
    for (int i = 0; i < WORDS; i++) w[i] = __builtin_nontemporal_load(p + i);
}

// Realign: the i-th dword of the block's quants (which start 2 bytes after the block start).
// sel = 0x05040302 when the block starts at byte 0 of the window, 0x07060504 when at byte 2.
__device__ __forceinline__ uint32_t quant_word(const uint32_t *w, int i, uint32_t sel) {
    return __builtin_amdgcn_perm(w[i + 1], w[i], sel);
}

__device__ __forceinline__ uint32_t quant_sel(size_t off) {
    return (off & 2) ? 0x07060504u : 0x05040302u;
}

__device__ __forceinline__ uint32_t scale_bits(uint32_t w0, size_t off) {
    return (off & 2) ? (w0 >> 16) : (w0 & 0xffffu);
}

// Reductions over lanes by DPP row operations (one VALU instruction a step, usually fused into
// the combining instruction) where the lanes share a 16-lane row, instead of LDS permutes:
// group_reduce<L> combines the lane's aligned group of L lanes (L = 2 .. 64: quad_perm lanes ^ 1,
// quad_perm lanes ^ 2, the half-row mirror, the row mirror, then permutes across rows) and leaves
// the result in every lane of the group; wave_reduce combines the four row results of a wavefront
// by readlane (a uniform value). A group's lanes must be active together.
template <int CTRL, class T>
__device__ __forceinline__ T dpp_mov(T v) {
    static_assert(sizeof(T) == 4, "32-bit values");
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <class T>
__device__ __forceinline__ T lane_value(T v, int l) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
struct AddOp {
    template <class T>
    __device__ T operator()(T a, T b) const { return a + b; }
};
struct MaxOp {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct AndOp {
    __device__ int operator()(int a, int b) const { return a & b; }
};
struct MaxUOp {
    __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
};
template <int L, class T, class Op>
__device__ __forceinline__ T group_reduce(T v, Op op) {
    static_assert(L == 2 || L == 4 || L == 8 || L == 16 || L == 32 || L == 64, "lane groups of 2 to 64");
    v = op(v, dpp_mov<0xB1>(v));                          // quad_perm [1, 0, 3, 2]
    if constexpr (L >= 4) v = op(v, dpp_mov<0x4E>(v));    // quad_perm [2, 3, 0, 1]
    if constexpr (L >= 8) v = op(v, dpp_mov<0x141>(v));   // row_half_mirror
    if constexpr (L >= 16) v = op(v, dpp_mov<0x140>(v));  // row_mirror
    if constexpr (L >= 32) v = op(v, __shfl_xor(v, 16, 64));
    if constexpr (L >= 64) v = op(v, __shfl_xor(v, 32, 64));
    return v;
}
// SwiGLU's activation of one unit (ferrum_ref/src/models/llama/ops.rs:69-76): silu(g) * u, with
// the reference's two roundings. Every kernel that applies it (the SwiGLU passes and the fast
// GEMM's fused epilogue) uses this one definition, so their results are bit-identical.
__device__ __forceinline__ float swiglu_act(float g, float u) { return __fmul_rn(g / (1.0f + expf(-g)), u); }

template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
    v = group_reduce<16>(v, op);
    return op(op(lane_value(v, 0), lane_value(v, 16)), op(lane_value(v, 32), lane_value(v, 48)));
}

}  // namespace fh
