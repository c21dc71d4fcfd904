// Device pieces shared by the batch-1 GEMV kernels (gemv.hip, decode.hip): the prepared-x
// record of a block (four signed-byte limb rows in the MFMA's k order, then the block's x scale
// and the Q4_0 biases) and the exact integer block products on the matrix cores. Included by .hip
// files only; everything is internal to the including file.
#pragma once

#include "device_common.hpp"
#include "internal.hpp"

namespace fh {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float half_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// A raw buffer resource over [base, base + bytes): loads at offsets at or past `bytes` return 0
// (gfx9 descriptor word 3 = 0x00020000, 32-bit data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
constexpr int kNonTemporal = 2;             // cache-policy bit of a streaming load
// Prepared-x record of a block (160 bytes): dwords 0..31 are the four limb rows (32 bytes each,
// most significant first), dword 32 the x scale, 33 and 34 the Q4_0 biases, 35..39 zero.
constexpr int kPrepBytes = 160;
constexpr int kBatch = 8;                   // blocks per pipeline batch

// k slot of the MFMA operands -> element of the block. Lane half h (lanes 32h..32h+31) holds
// 16 slots; B lane (row, h) loads quant bytes 8h..8h+7 (Q4_0: low nibbles are slots 0..7, high
// nibbles slots 8..15) or 16h..16h+15 (Q8_0: slot i is byte i).
template <int KIND>
__host__ __device__ constexpr int elem_of_slot(int h, int i) {
    if constexpr (KIND == FH_Q8_0)
        return 16 * h + i;
    else
        return i < 8 ? 8 * h + i : 16 + 8 * h + (i - 8);
}

// The prepared-x writer gives lane j (elements 4j .. 4j + 3 of a block) one dword of each
// 32-byte limb row: the slots of those four elements, in order.
template <int KIND>
__host__ __device__ constexpr int prep_dword(int j) {
    return KIND == FH_Q8_0 ? j : (j == 2 || j == 3) ? j + 2 : (j == 4 || j == 5) ? j - 2 : j;
}
template <int KIND>
constexpr bool prep_dwords_match_slots() {
    for (int j = 0; j < 8; j++)
        for (int k = 0; k < 4; k++) {
            const int byte = 4 * prep_dword<KIND>(j) + k;
            if (elem_of_slot<KIND>(byte / 16, byte % 16) != 4 * j + k) return false;
        }
    return true;
}
static_assert(prep_dwords_match_slots<FH_Q8_0>() && prep_dwords_match_slots<FH_Q4_0>(),
              "prepared-x dwords must hold the MFMA k slots");

// ---- x preparation: eight lanes per block, lane j taking elements 4j .. 4j + 3 ----
// Each block of x is put on the fixed-point grid of its largest magnitude: with
// 2^(E-1) <= amax < 2^E, xi = rint(x * 2^(30-E)) (|xi| <= 2^30, error <= 2^-30 amax per element,
// finer than the f32 rounding of any element above 2^-7 amax) and xi = a 2^24 + b 2^16 + c 2^8 + e
// with a, b, c, e signed bytes (|a| <= 64). The record's scale is 2^(E-30) (the grid is capped at
// 2^-149, where it holds every float exactly). For Q4_0 the stored nibbles (0..15) stand for
// q = nibble - 8, so the record carries the biases -8 sum(a 2^8 + b) and -8 sum(c 2^8 + e) that
// the two halves of the limb sums take (both exact in int32).
// Writes the record of the block whose elements 4j .. 4j + 3 are v at rec (a global or an LDS
// pointer). The eight lanes of a block must run this together (they reduce over one another
// by DPP).
template <int KIND, class U32Ptr>
__device__ __forceinline__ void prep_values(f32x4 v, int j, U32Ptr rec) {
    // the largest magnitude's bits, one integer reduction: the bit patterns of non-negative floats
    // order as the values do, and inf (0x7f800000) and NaN (above it) order above every finite one
    const uint32_t am = max(max(__float_as_uint(v.x) & 0x7fffffffu, __float_as_uint(v.y) & 0x7fffffffu),
                            max(__float_as_uint(v.z) & 0x7fffffffu, __float_as_uint(v.w) & 0x7fffffffu));
    const uint32_t abits = group_reduce<8>(am, MaxUOp());
    const int finite = abits < 0x7f800000u;  // 0: inf, NaN
    const float amax = __uint_as_float(abits);
    // grid 2^-sh with 2^29 <= amax * 2^sh < 2^30, at most 2^149 (subnormal amax: exponent field
    // 1); the scaling is split in two exact power-of-two products so that no factor overflows
    const int sh = min(156 - (int)max(__float_as_uint(amax) >> 23, 1u), 149);  // -98 .. 149
    const int sh1 = min(sh, 100);
    const float m1 = __uint_as_float((uint32_t)(127 + sh1) << 23);
    const float m2 = __uint_as_float((uint32_t)(127 + sh - sh1) << 23);
    const float xs = !finite ? __builtin_nanf("")
                     : sh <= 126 ? __uint_as_float((uint32_t)(127 - sh) << 23)  // 2^-sh, normal
                                 : __uint_as_float(1u << (149 - sh));            // 2^-sh, subnormal
    uint32_t la = 0, lb = 0, lc = 0, le = 0;
    int32_t shi = 0, slo = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        // |xi| <= 2^30; non-finite blocks take 0 here and NaN through xs
        const float sx = finite ? (v[k] * m1) * m2 : 0.0f;
        const int32_t xi = (int32_t)rintf(sx);
        const int32_t e = (xi << 24) >> 24;
        int32_t r = (xi - e) >> 8;
        const int32_t c = (r << 24) >> 24;
        r = (r - c) >> 8;
        const int32_t b = (r << 24) >> 24;
        const int32_t a = (r - b) >> 8;
        la |= (uint32_t)(a & 0xff) << (8 * k);
        lb |= (uint32_t)(b & 0xff) << (8 * k);
        lc |= (uint32_t)(c & 0xff) << (8 * k);
        le |= (uint32_t)(e & 0xff) << (8 * k);
        shi += a * 256 + b;
        slo += c * 256 + e;
    }
    if constexpr (KIND == FH_Q4_0) {
        shi = group_reduce<8>(shi, AddOp());
        slo = group_reduce<8>(slo, AddOp());
    }
    const int dw = prep_dword<KIND>(j);
    rec[dw] = la;
    rec[8 + dw] = lb;
    rec[16 + dw] = lc;
    rec[24 + dw] = le;
    if (j == 0) {
        rec[32] = __float_as_uint(xs);
        rec[33] = KIND == FH_Q4_0 ? (uint32_t)(-8 * shi) : 0u;
        rec[34] = KIND == FH_Q4_0 ? (uint32_t)(-8 * slo) : 0u;
    } else if (j < 6) {
        rec[34 + j] = 0u;  // dwords 35 .. 39 are zero
    }
}

// A zero record (a padding block: contributes 0), written by its eight lanes.
template <class U32Ptr>
__device__ __forceinline__ void zero_record(int j, U32Ptr rec) {
#pragma unroll
    for (int i = 0; i < kPrepBytes / 32; i++) rec[j * (kPrepBytes / 32) + i] = 0u;
}

// Per-lane byte offsets into the records of an 8-block batch: the MFMA's A operand (lane l
// holds A row l % 32, i.e. limb (l % 4) of block (l % 32) / 4, k half l / 32) and the record
// tails. Q8_0 needs only each block's scale: lanes 4j .. 4j + 3 and 32 + 4j .. 32 + 4j + 3 take
// dwords 32 .. 35 of block j (one dword load; the scales are read across lanes). Q4_0 needs the
// scale and both biases of the block a lane finishes: lane half h takes the 16-byte tail of block
// 2p + h for each block pair p (one 16-byte load per pair, at + 2 p kPrepBytes; every lane of a
// half reads the same bytes).
__device__ __forceinline__ uint32_t prep_a_offset(int lane) {
    const int r = lane % 32;
    return (uint32_t)((r / 4) * kPrepBytes + (r % 4) * 32 + 16 * (lane / 32));
}
template <int KIND>
__device__ __forceinline__ uint32_t prep_tail_offset(int lane) {
    const int r = lane % 32;
    return KIND == FH_Q8_0 ? (uint32_t)((r / 4) * kPrepBytes + 128 + 4 * (r % 4))
                           : (uint32_t)((lane / 32) * kPrepBytes + 128);
}
constexpr int kTailLoads = 4;  // Q4_0: 16-byte tail loads per batch (one per block pair)

// The same for block b of x in global memory.
template <int KIND, class U32Ptr>
__device__ __forceinline__ void prep_block(const float *__restrict__ x, bool aligned, uint32_t b, int j, U32Ptr rec) {
    // (global-address-space loads: flat ones would also count against the LDS counter)
    typedef __attribute__((address_space(1))) const float gfloat;
    typedef __attribute__((address_space(1))) const f32x4 gf32x4;
    gfloat *xb = (gfloat *)(x + (size_t)b * 32 + 4 * j);
    f32x4 v;
    if (aligned) {
        v = *(gf32x4 *)xb;
    } else {
        v = f32x4{xb[0], xb[1], xb[2], xb[3]};
    }
    prep_values<KIND>(v, j, rec);
}

template <int KIND>
struct Batch {  // what one lane loads for a batch of kBatch blocks of its task
    static constexpr int QL = KIND == FH_Q8_0 ? kBatch : kBatch / 2;  // 16-byte quant loads
    u32x4 q[QL];  // Q4_0: blocks 2i (lanes 0..31) and 2i + 1 (lanes 32..63) of row lane % 32
                  // Q8_0: bytes 16h .. 16h + 15 of block i of the row (h = lane / 32)
    u32x4 s;      // the row's eight scales
    i32x4 a;      // the prepared x of the eight blocks, as the MFMA's A operand
    static constexpr int TL = KIND == FH_Q8_0 ? 1 : kTailLoads;
    u32x4 t[TL];  // record tails (prep_tail_offset): Q8_0 t[0].x, Q4_0 t[p] = block 2p + h's tail
};

// The record tails of a batch whose records start at byte b_off: `load16(off)` reads 16 bytes,
// `load4(off)` 4 bytes, at byte offset off of the records' memory.
template <int KIND, class L16, class L4>
__device__ __forceinline__ void load_tails(Batch<KIND> &bt, uint32_t b_off, uint32_t lane_off, L16 load16, L4 load4) {
    if constexpr (KIND == FH_Q8_0) {
        bt.t[0].x = load4(b_off + lane_off);
    } else {
#pragma unroll
        for (int p = 0; p < kTailLoads; p++) bt.t[p] = load16(b_off + lane_off + 2 * p * kPrepBytes);
    }
}

__device__ __forceinline__ i32x4 nibbles(uint32_t q0, uint32_t q1) {
    return i32x4{(int32_t)(q0 & 0x0f0f0f0fu), (int32_t)(q1 & 0x0f0f0f0fu), (int32_t)((q0 >> 4) & 0x0f0f0f0fu),
                 (int32_t)((q1 >> 4) & 0x0f0f0f0fu)};
}

// The batch's contribution to the lane's accumulator: lanes 0..31 take the even blocks of the
// batch, lanes 32..63 the odd ones (row lane % 32 in both halves). Pipelined by block pair: the
// MFMAs of pair p + 1 are issued before pair p's sums are finished, and no more than two pairs'
// accumulators are live (scheduling barriers keep the compiler from issuing every MFMA first).
template <int KIND, int PAIRS = kBatch / 2>
__device__ __forceinline__ void compute_batch(const Batch<KIND> &bt, bool upper, float &acc) {
    i32x16 ce[2], co[2];
    auto issue = [&](int p) {  // blocks 2p and 2p + 1 of the batch
        i32x4 be, bo;
        if constexpr (KIND == FH_Q8_0) {
            be = __builtin_bit_cast(i32x4, bt.q[2 * p]);
            bo = __builtin_bit_cast(i32x4, bt.q[2 * p + 1]);
        } else {
            // lane r holds all 16 bytes of block 2p, lane 32 + r those of block 2p + 1; after
            // swapping the upper lanes' first 8 bytes with the lower lanes' last 8, each lane
            // holds half h of both blocks, as the MFMA's B operand takes them
            const auto s0 = __builtin_amdgcn_permlane32_swap(bt.q[p][0], bt.q[p][2], false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(bt.q[p][1], bt.q[p][3], false, false);
            be = nibbles(s0[0], s1[0]);
            bo = nibbles(s0[1], s1[1]);
        }
        // A rows 4j .. 4j + 3 hold block j's limb rows, so C rows 4j .. 4j + 3 are block j's
        // limb sums: for j = 2p in registers 4p .. 4p + 3 of lanes 0..31, for j = 2p + 1 in the
        // same registers of lanes 32..63. The other rows mix blocks and are not used.
        ce[p & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bt.a, be, i32x16{}, 0, 0, 0);
        co[p & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bt.a, bo, i32x16{}, 0, 0, 0);
    };
    auto finish = [&](int p) {
        const i32x16 &e = ce[p & 1], &o = co[p & 1];
        const int32_t c0 = upper ? o[4 * p] : e[4 * p];
        const int32_t c1 = upper ? o[4 * p + 1] : e[4 * p + 1];
        const int32_t c2 = upper ? o[4 * p + 2] : e[4 * p + 2];
        const int32_t c3 = upper ? o[4 * p + 3] : e[4 * p + 3];
        // the sum is hi 2^16 + lo; |hi|, |lo| < 2^27 (Q8_0), < 2^23 (Q4_0, biases included)
        int32_t hi = c0 * 256 + c1, lo = c2 * 256 + c3;
        float xs;
        if constexpr (KIND == FH_Q8_0) {
            // the block's x scale: block 2p in lanes 8p .., block 2p + 1 in lanes 8p + 4 ..
            const float xe = __int_as_float(__builtin_amdgcn_readlane(bt.t[0].x, 8 * p));
            const float xo = __int_as_float(__builtin_amdgcn_readlane(bt.t[0].x, 8 * p + 4));
            xs = upper ? xo : xe;
        } else {
            // this lane's block: its scale and biases
            xs = __uint_as_float(bt.t[p].x);
            hi += (int32_t)bt.t[p].y;
            lo += (int32_t)bt.t[p].z;
        }
        const float f = fmaf((float)hi, 65536.0f, (float)lo);  // Q4_0: one rounding
        const float d = half_to_float(bt.s[p] >> (upper ? 16 : 0));
        acc = fmaf(d * f, xs, acc);
    };
    issue(0);
#pragma unroll
    for (int p = 0; p < PAIRS; p++) {
        if (p + 1 < PAIRS) issue(p + 1);
        __builtin_amdgcn_sched_barrier(0);
        finish(p);
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace
}  // namespace fh
