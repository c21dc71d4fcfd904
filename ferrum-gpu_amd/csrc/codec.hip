// GGUF Q8_0 / Q4_0 codec kernels for gfx950: f32 -> blocks (encode), blocks -> f32 (decode) and
// the fused QAT snap (encode then decode), in "rows" form (blocks of 32 consecutive values, the
// GGUF tensor order) and "cols" form (blocks running down the columns of an [in, out] matrix).
// Bit-exact with ferrum_gguf/src/codec/quant.rs:50-136 and ferrum_ref/src/training/qat.rs:20-54.
//
// All of this is HBM-bound byte work. The rows kernels give each block to 8 lanes, each lane a
// 16-byte f32x4 of the block, so a wavefront reads or writes 1 KiB of f32 per instruction,
// perfectly coalesced; the odd-sized packed side (34 or 18 bytes per block) is staged through
// LDS so it, too, moves as aligned 16-byte chunks. The cols kernels map consecutive lanes to
// consecutive columns, which makes the column walks coalesced across the wavefront.
#include "device_common.hpp"
#include "internal.hpp"

// The codec must round exactly like the reference: v * id and (v * id) + 8.5 are separate
// roundings, never one fused multiply-add.
#pragma clang fp contract(off)

namespace fh {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;                            // 8-block groups per wavefront per task
constexpr int kTaskBlocks = (kThreads / 64) * kUnroll * 8;  // 128 blocks per workgroup task

template <int KIND>
struct Fmt;
template <>
struct Fmt<FH_Q8_0> {
    static constexpr int bytes = 34;
};
template <>
struct Fmt<FH_Q4_0> {
    static constexpr int bytes = 18;
};

// Reduce over the 8 lanes of a block (lanes 8b..8b+7 of the wavefront).
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, __shfl_xor(v, 1));
    v = fmaxf(v, __shfl_xor(v, 2));
    v = fmaxf(v, __shfl_xor(v, 4));
    return v;
}

// The signed value of largest magnitude, the lowest index winning ties (the reference's strict
// `>` fold from 0.0, quant.rs:123-126). `mine` is this lane's candidate for elements
// 4j..4j+3; lanes are ordered by element index.
__device__ __forceinline__ float argmax_abs8(float mine, int lane) {
#pragma unroll
    for (int s = 1; s < 8; s <<= 1) {
        float other = __shfl_xor(mine, s);
        bool lower = (lane & s) == 0;  // this lane's elements come first
        float lo = lower ? mine : other, hi = lower ? other : mine;
        mine = fabsf(hi) > fabsf(lo) ? hi : lo;
    }
    return mine;
}

// One quantisation step shared by encode and snap: from this lane's 4 values and the block's
// statistics, the 4 quant codes (Q8_0: signed q; Q4_0: nibble 0..15) and the f16 scale bits.
template <int KIND>
__device__ __forceinline__ void quantise4(const f32x4 v, int lane, int32_t (&q)[4], uint32_t &h) {
    if constexpr (KIND == FH_Q8_0) {
        float amax = fmaxf(fmaxf(fmaxf(0.0f, fabsf(v.x)), fmaxf(fabsf(v.y), fabsf(v.z))), fabsf(v.w));
        amax = max8(amax);
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        h = float_to_half_bits(d);
        q[0] = round_sat_i8(v.x * id);
        q[1] = round_sat_i8(v.y * id);
        q[2] = round_sat_i8(v.z * id);
        q[3] = round_sat_i8(v.w * id);
    } else {
        float m = 0.0f;
        if (fabsf(v.x) > fabsf(m)) m = v.x;
        if (fabsf(v.y) > fabsf(m)) m = v.y;
        if (fabsf(v.z) > fabsf(m)) m = v.z;
        if (fabsf(v.w) > fabsf(m)) m = v.w;
        m = argmax_abs8(m, lane);
        float d = m / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        h = float_to_half_bits(d);
        q[0] = trunc_clamp_0_15(v.x * id + 8.5f);
        q[1] = trunc_clamp_0_15(v.y * id + 8.5f);
        q[2] = trunc_clamp_0_15(v.z * id + 8.5f);
        q[3] = trunc_clamp_0_15(v.w * id + 8.5f);
    }
}

// ---- encode, rows: f32[nblocks * 32] -> GGUF blocks ----
template <int KIND>
__global__ __launch_bounds__(kThreads) void encode_rows_kernel(const float *__restrict__ src,
                                                               uint8_t *__restrict__ dst,
                                                               size_t nblocks) {
    constexpr int BB = Fmt<KIND>::bytes;
    constexpr int OUT = kTaskBlocks * BB;  // staged output bytes per task (16-byte multiple)
    __shared__ __attribute__((aligned(16))) uint8_t stage[OUT];
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const size_t ntasks = (nblocks + kTaskBlocks - 1) / kTaskBlocks;
    for (size_t task = blockIdx.x; task < ntasks; task += gridDim.x) {
        const size_t blk0 = task * kTaskBlocks;
        f32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            size_t blk = blk0 + (size_t)(wave * kUnroll + u) * 8 + lane / 8;
            v[u] = blk < nblocks ? __builtin_nontemporal_load((const f32x4 *)src + blk * 8 + lane % 8)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads();  // the previous task's stage has been written out
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int lb = (wave * kUnroll + u) * 8 + lane / 8;  // block within the task
            const int j = lane % 8;
            int32_t q[4];
            uint32_t h;
            quantise4<KIND>(v[u], lane, q, h);
            uint8_t *blk = stage + lb * BB;
            if (j == 0) *(uint16_t *)blk = (uint16_t)h;
            if constexpr (KIND == FH_Q8_0) {
                uint32_t w = (q[0] & 0xff) | (q[1] & 0xff) << 8 | (q[2] & 0xff) << 16 | (uint32_t)(q[3] & 0xff) << 24;
                *(uint16_t *)(blk + 2 + 4 * j) = (uint16_t)w;
                *(uint16_t *)(blk + 4 + 4 * j) = (uint16_t)(w >> 16);
            } else {
                // lanes j < 4 hold elements 4j.. (low nibbles), lane j + 4 the elements 16 + 4j..
                uint32_t lo = q[0] | q[1] << 8 | q[2] << 16 | (uint32_t)q[3] << 24;
                uint32_t hi = (uint32_t)__shfl_xor((int)lo, 4);
                if (j < 4) {
                    uint32_t w = lo | hi << 4;
                    *(uint16_t *)(blk + 2 + 4 * j) = (uint16_t)w;
                    *(uint16_t *)(blk + 4 + 4 * j) = (uint16_t)(w >> 16);
                }
            }
        }
        __syncthreads();
        const size_t nvalid = nblocks - blk0 < (size_t)kTaskBlocks ? nblocks - blk0 : kTaskBlocks;
        const size_t valid = nvalid * BB;
        uint8_t *out = dst + blk0 * BB;
        for (int c = tid; c < OUT / 16; c += kThreads) {
            size_t off = (size_t)c * 16;
            if (off + 16 <= valid) {
                *(u32x4 *)(out + off) = *(const u32x4 *)(stage + off);
            } else if (off < valid) {
                for (size_t b = off; b < valid; b += 2) *(uint16_t *)(out + b) = *(const uint16_t *)(stage + b);
            }
        }
    }
}

// ---- decode, rows: GGUF blocks -> f32[nblocks * 32] ----
template <int KIND>
__global__ __launch_bounds__(kThreads) void decode_rows_kernel(const uint8_t *__restrict__ src,
                                                               float *__restrict__ dst,
                                                               size_t nblocks) {
    constexpr int BB = Fmt<KIND>::bytes;
    constexpr int IN = kTaskBlocks * BB;
    __shared__ __attribute__((aligned(16))) uint8_t stage[IN];
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    constexpr int CH = (IN / 16 + kThreads - 1) / kThreads;  // 16-byte chunks per thread
    const size_t ntasks = (nblocks + kTaskBlocks - 1) / kTaskBlocks;
    // this thread's chunks of a task's packed bytes; the next task's are in flight while this
    // one is decoded
    auto fetch = [&](size_t task, u32x4 (&p)[CH]) {
        const size_t blk0 = task * kTaskBlocks;
        const size_t valid = (nblocks - blk0 < (size_t)kTaskBlocks ? nblocks - blk0 : kTaskBlocks) * BB;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const size_t off = (size_t)(tid + c * kThreads) * 16;
            if (off < IN && off < valid)  // a partial last chunk reads into the allocation's padding
                p[c] = __builtin_nontemporal_load((const u32x4 *)(src + blk0 * BB + off));
        }
    };
    u32x4 ahead[CH];
    if (blockIdx.x < ntasks) fetch(blockIdx.x, ahead);
    for (size_t task = blockIdx.x; task < ntasks; task += gridDim.x) {
        const size_t blk0 = task * kTaskBlocks;
        __syncthreads();  // the previous task's stage has been read
#pragma unroll
        for (int c = 0; c < CH; c++)
            if ((tid + c * kThreads) * 16 < IN) *(u32x4 *)(stage + (tid + c * kThreads) * 16) = ahead[c];
        __syncthreads();
        if (task + gridDim.x < ntasks) fetch(task + gridDim.x, ahead);
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int lb = (wave * kUnroll + u) * 8 + lane / 8;
            const int j = lane % 8;
            const size_t blk = blk0 + lb;
            if (blk >= nblocks) continue;
            const uint8_t *b = stage + lb * BB;
            float d = half_bits_to_float(*(const uint16_t *)b);
            f32x4 o;
            if constexpr (KIND == FH_Q8_0) {
                uint32_t w = *(const uint16_t *)(b + 2 + 4 * j) | (uint32_t) * (const uint16_t *)(b + 4 + 4 * j) << 16;
                o.x = d * (float)(int8_t)(w);
                o.y = d * (float)(int8_t)(w >> 8);
                o.z = d * (float)(int8_t)(w >> 16);
                o.w = d * (float)(int8_t)(w >> 24);
            } else {
                const int jj = j & 3, sh = (j >> 2) * 4;  // lanes 4..7 take the high nibbles
                uint32_t w = *(const uint16_t *)(b + 2 + 4 * jj) | (uint32_t) * (const uint16_t *)(b + 4 + 4 * jj) << 16;
                w >>= sh;
                o.x = d * ((float)(w & 15) - 8.0f);
                o.y = d * ((float)((w >> 8) & 15) - 8.0f);
                o.z = d * ((float)((w >> 16) & 15) - 8.0f);
                o.w = d * ((float)((w >> 24) & 15) - 8.0f);
            }
            __builtin_nontemporal_store(o, (f32x4 *)dst + blk * 8 + j);
        }
    }
}

// ---- snap, rows: f32 -> f32, decode(encode(block)) for blocks of 32 consecutive values ----
__global__ __launch_bounds__(kThreads) void snap_rows_kernel(const float *__restrict__ src,
                                                             float *__restrict__ dst,
                                                             size_t nblocks) {
    const int lane = threadIdx.x % 64;
    const size_t waves = (size_t)gridDim.x * (kThreads / 64);
    const size_t wave = (size_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
    const size_t groups = (nblocks + 7) / 8;
    for (size_t g0 = wave * kUnroll; g0 < groups; g0 += waves * kUnroll) {
        f32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            size_t blk = (g0 + u) * 8 + lane / 8;
            v[u] = blk < nblocks ? __builtin_nontemporal_load((const f32x4 *)src + blk * 8 + lane % 8)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            int32_t q[4];
            uint32_t h;
            quantise4<FH_Q8_0>(v[u], lane, q, h);
            float d = half_bits_to_float(h);
            f32x4 o = {d * (float)q[0], d * (float)q[1], d * (float)q[2], d * (float)q[3]};
            size_t blk = (g0 + u) * 8 + lane / 8;
            if (blk < nblocks) __builtin_nontemporal_store(o, (f32x4 *)dst + blk * 8 + lane % 8);
        }
    }
}

// ---- cols: one thread per (column c, block kb) of an [k, n] matrix ----
// Quantise down the columns into the planes of GGUF row c (quantise_matrix,
// ferrum_wgpu/src/ops/quant.rs:238-252): block (c, kb) goes to slot tile_slot(c, kb, nb) of the planes.
template <int KIND>
__global__ __launch_bounds__(kThreads) void encode_cols_kernel(const float *__restrict__ w,
                                                               uint8_t *__restrict__ qs,
                                                               uint16_t *__restrict__ ds, size_t k,
                                                               size_t n) {
    const size_t nb = k / 32;
    const size_t total = nb * n;
    for (size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (size_t)gridDim.x * kThreads) {
        const size_t kb = t / n, c = t % n;
        float v[32];
#pragma unroll
        for (int e = 0; e < 32; e++) v[e] = w[(kb * 32 + e) * n + c];
        const size_t blk = tile_slot(c, kb, nb), sc = scale_slot(c, kb, nb);
        if constexpr (KIND == FH_Q8_0) {
            float amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(v[e]));
            float d = amax / 127.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            ds[sc] = (uint16_t)float_to_half_bits(d);
            u32x4 o[2];
#pragma unroll
            for (int e = 0; e < 32; e += 4) {
                uint32_t word = (round_sat_i8(v[e] * id) & 0xff) | (round_sat_i8(v[e + 1] * id) & 0xff) << 8 |
                                (round_sat_i8(v[e + 2] * id) & 0xff) << 16 |
                                (uint32_t)(round_sat_i8(v[e + 3] * id) & 0xff) << 24;
                o[e / 16][(e / 4) % 4] = word;
            }
            *(u32x4 *)(qs + blk * 32) = o[0];
            *(u32x4 *)(qs + blk * 32 + 16) = o[1];
        } else {
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < 32; e++)
                if (fabsf(v[e]) > fabsf(m)) m = v[e];
            float d = m / -8.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            ds[sc] = (uint16_t)float_to_half_bits(d);
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 16; j += 4) {
                uint32_t word = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    uint32_t byte = trunc_clamp_0_15(v[j + b] * id + 8.5f) |
                                    trunc_clamp_0_15(v[j + b + 16] * id + 8.5f) << 4;
                    word |= byte << (8 * b);
                }
                o[j / 4] = word;
            }
            *(u32x4 *)(qs + blk * 16) = o;
        }
    }
}

// Dequantise the planes back to the [k, n] f32 weight (transpose(decode(bytes))).
template <int KIND>
__global__ __launch_bounds__(kThreads) void decode_cols_kernel(const uint8_t *__restrict__ qs,
                                                               const uint16_t *__restrict__ ds,
                                                               float *__restrict__ w, size_t k,
                                                               size_t n) {
    const size_t nb = k / 32;
    const size_t total = nb * n;
    for (size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (size_t)gridDim.x * kThreads) {
        const size_t kb = t / n, c = t % n;
        const size_t blk = tile_slot(c, kb, nb);
        const float d = half_bits_to_float(ds[scale_slot(c, kb, nb)]);
        float *col = w + kb * 32 * n + c;
        if constexpr (KIND == FH_Q8_0) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const u32x4 q = *(const u32x4 *)(qs + blk * 32 + 16 * h);
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int b = 0; b < 4; b++)
                        col[(16 * h + 4 * i + b) * n] = d * (float)(int8_t)(q[i] >> (8 * b));
            }
        } else {
            const u32x4 q = *(const u32x4 *)(qs + blk * 16);
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    col[(4 * i + b) * n] = d * ((float)((q[i] >> (8 * b)) & 15) - 8.0f);
                    col[(16 + 4 * i + b) * n] = d * ((float)((q[i] >> (8 * b + 4)) & 15) - 8.0f);
                }
            }
        }
    }
}

// ---- GGUF blocks <-> planes, one thread per block ----
template <int KIND>
__global__ __launch_bounds__(kThreads) void gguf_to_planes_kernel(const uint8_t *__restrict__ src,
                                                                  uint8_t *__restrict__ qs,
                                                                  uint16_t *__restrict__ ds, size_t n,
                                                                  size_t nb) {
    constexpr int BB = Fmt<KIND>::bytes;
    constexpr int WORDS = KIND == FH_Q8_0 ? 9 : 5;
    const size_t nblocks = n * nb;
    for (size_t blk = (size_t)blockIdx.x * kThreads + threadIdx.x; blk < nblocks;
         blk += (size_t)gridDim.x * kThreads) {
        const size_t off = blk * BB;  // block blk of the GGUF rows: row blk / nb, block blk % nb
        const size_t slot = tile_slot(blk / nb, blk % nb, nb);
        uint32_t win[WORDS];
        load_window<WORDS>(src, off, win);
        const uint32_t sel = quant_sel(off);
        ds[scale_slot(blk / nb, blk % nb, nb)] = (uint16_t)scale_bits(win[0], off);
#pragma unroll
        for (int h = 0; h < (KIND == FH_Q8_0 ? 2 : 1); h++) {
            u32x4 q;
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = quant_word(win, 4 * h + i, sel);
            __builtin_nontemporal_store(q, (u32x4 *)(qs + slot * (BB - 2) + 16 * h));
        }
    }
}

template <int KIND>
__global__ __launch_bounds__(kThreads) void planes_to_gguf_kernel(const uint8_t *__restrict__ qs,
                                                                  const uint16_t *__restrict__ ds,
                                                                  uint8_t *__restrict__ dst, size_t n,
                                                                  size_t nb) {
    constexpr int BB = Fmt<KIND>::bytes;
    const size_t nblocks = n * nb;
    for (size_t blk = (size_t)blockIdx.x * kThreads + threadIdx.x; blk < nblocks;
         blk += (size_t)gridDim.x * kThreads) {
        const size_t slot = tile_slot(blk / nb, blk % nb, nb);
        uint16_t *out = (uint16_t *)(dst + blk * BB);  // GGUF blocks are 2-byte aligned
        out[0] = ds[scale_slot(blk / nb, blk % nb, nb)];
#pragma unroll
        for (int h = 0; h < (KIND == FH_Q8_0 ? 2 : 1); h++) {
            const u32x4 q = *(const u32x4 *)(qs + slot * (BB - 2) + 16 * h);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                out[1 + 8 * h + 2 * i] = (uint16_t)q[i];
                out[2 + 8 * h + 2 * i] = (uint16_t)(q[i] >> 16);
            }
        }
    }
}

// Snap an [rows_in, cols_out] matrix down its columns (q8_snap_cols, ops/qat.rs:33-57).
// One wavefront per (block row kb, 64 columns): lane (cq = lane % 16, rg = lane / 16) holds four
// adjacent columns of rows 8rg..8rg+7 of the block row, so each load instruction moves four
// 256-byte row segments (16 bytes a lane) and a column's block spans lanes cq, cq+16, cq+32,
// cq+48, whose maxima meet by two lane exchanges. VEC: columns a multiple of 4 and 16-byte
// aligned buffers (f32x4 loads and stores); otherwise one guarded f32 per column. Task t of a
// matrix of cg = ceil(n / 64) column groups is block row t / cg, column group t % cg; the whole
// wavefront runs it (the lane exchanges need every lane).
template <bool VEC>
__device__ __forceinline__ void snap_cols_task(const float *__restrict__ src, float *__restrict__ dst, size_t n,
                                               size_t cg, size_t t, int lane) {
    const int cq = lane % 16, rg = lane / 16;
    const size_t c0 = (t % cg) * 64 + 4 * cq;
    const size_t at = (t / cg * 32 + (size_t)rg * 8) * n + c0;  // row 0 of this lane's rows
    f32x4 v[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        if constexpr (VEC) {
            v[r] = c0 < n ? __builtin_nontemporal_load((const f32x4 *)(src + at + r * n)) : f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) v[r][i] = c0 + i < n ? src[at + r * n + i] : 0.0f;
        }
    }
    f32x4 amax = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 8; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) amax[i] = fmaxf(amax[i], fabsf(v[r][i]));
    f32x4 id, dh;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float a = fmaxf(amax[i], __shfl_xor(amax[i], 16));
        a = fmaxf(a, __shfl_xor(a, 32));
        const float d = a / 127.0f;
        id[i] = d != 0.0f ? 1.0f / d : 0.0f;
        dh[i] = half_bits_to_float(float_to_half_bits(d));
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = dh[i] * (float)round_sat_i8(v[r][i] * id[i]);
        if constexpr (VEC) {
            if (c0 < n) __builtin_nontemporal_store(o, (f32x4 *)(dst + at + r * n));
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (c0 + i < n) dst[at + r * n + i] = o[i];
        }
    }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void snap_cols_kernel(const float *__restrict__ src,
                                                             float *__restrict__ dst, size_t k,
                                                             size_t n) {
    const size_t cg = (n + 63) / 64, tasks = k / 32 * cg;
    const size_t waves = (size_t)gridDim.x * (kThreads / 64);
    for (size_t t = (size_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64; t < tasks; t += waves)
        snap_cols_task<VEC>(src, dst, n, cg, t, (int)(threadIdx.x % 64));
}

// ---- a grouped snap pass (fh_snap_plan_*): every problem's wavefront tasks in one launch ----
constexpr uint32_t kSnapVec = 0x100;  // mode flag: a column snap that takes the f32x4 form
constexpr uint32_t kRowsTaskBlocks = 8 * kUnroll;  // rows snap: blocks per wavefront task
constexpr uint32_t kCopyTask = 1024;               // copy: floats per wavefront task

// The descriptor as wave-uniform values (every dword through readfirstlane).
__device__ __forceinline__ SnapDesc uniform_snap_desc(const SnapDesc *descs, uint32_t p) {
    constexpr int W = sizeof(SnapDesc) / 4;
    static_assert(sizeof(SnapDesc) % 4 == 0, "descriptor of whole dwords");
    struct Words {
        uint32_t w[W];
    };
    Words v = __builtin_bit_cast(Words, descs[p]);
#pragma unroll
    for (int i = 0; i < W; i++) v.w[i] = __builtin_amdgcn_readfirstlane(v.w[i]);
    return __builtin_bit_cast(SnapDesc, v);
}

__global__ __launch_bounds__(kThreads) void snap_group_kernel(const SnapDesc *__restrict__ descs, uint32_t count,
                                                              uint32_t tasks) {
    const int lane = threadIdx.x % 64;
    const uint32_t waves = gridDim.x * (kThreads / 64);
    for (uint32_t t = __builtin_amdgcn_readfirstlane(blockIdx.x * (kThreads / 64) + threadIdx.x / 64); t < tasks;
         t += waves) {
        // the problem holding task t: the last one whose first task is at most t
        uint32_t lo = 0, hi = count;
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) / 2;
            if (__builtin_amdgcn_readfirstlane(descs[mid].task0) <= t)
                lo = mid;
            else
                hi = mid;
        }
        const SnapDesc d = uniform_snap_desc(descs, lo);
        const uint32_t lt = t - d.task0;
        if ((d.mode & 0xff) == FH_SNAP_COLS) {
            const size_t cg = (d.n + 63) / 64;
            if (d.mode & kSnapVec)
                snap_cols_task<true>(d.src, d.dst, d.n, cg, lt, lane);
            else
                snap_cols_task<false>(d.src, d.dst, d.n, cg, lt, lane);
        } else if ((d.mode & 0xff) == FH_SNAP_ROWS) {
            // kUnroll groups of eight blocks, eight lanes a block (the rows snap's wavefront step)
            const size_t nblocks = d.len / 32, g0 = (size_t)lt * kUnroll;
            f32x4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                const size_t blk = (g0 + u) * 8 + lane / 8;
                v[u] = blk < nblocks ? __builtin_nontemporal_load((const f32x4 *)d.src + blk * 8 + lane % 8)
                                     : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                int32_t q[4];
                uint32_t h;
                quantise4<FH_Q8_0>(v[u], lane, q, h);
                const float dd = half_bits_to_float(h);
                const f32x4 o = {dd * (float)q[0], dd * (float)q[1], dd * (float)q[2], dd * (float)q[3]};
                const size_t blk = (g0 + u) * 8 + lane / 8;
                if (blk < nblocks) __builtin_nontemporal_store(o, (f32x4 *)d.dst + blk * 8 + lane % 8);
            }
        } else {
            const size_t base = (size_t)lt * kCopyTask;
#pragma unroll
            for (int i = 0; i < (int)(kCopyTask / 64); i++) {
                const size_t e = base + (size_t)i * 64 + lane;
                if (e < d.len) d.dst[e] = d.src[e];
            }
        }
    }
}

// ---- plain f32 copy (Gpu::copy_f32): 16-byte loads and stores when both ends allow them ----
__global__ __launch_bounds__(kThreads) void copy_f32x4_kernel(const f32x4 *__restrict__ src,
                                                              f32x4 *__restrict__ dst, size_t n4) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += (size_t)gridDim.x * kThreads)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

__global__ __launch_bounds__(kThreads) void copy_f32_kernel(const float *__restrict__ src,
                                                            float *__restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (size_t)gridDim.x * kThreads)
        dst[i] = src[i];
}

// ---- F16 tensor -> f32 (Gguf::tensor_f32 for GGML_F16), exact ----
__global__ __launch_bounds__(kThreads) void decode_f16_kernel(const uint16_t *__restrict__ src,
                                                              float *__restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (size_t)gridDim.x * kThreads)
        dst[i] = half_bits_to_float(src[i]);
}

unsigned grid_for(size_t work_items, size_t per_group, unsigned cap) {
    size_t g = (work_items + per_group - 1) / per_group;
    if (g < 1) g = 1;
    return g > cap ? cap : (unsigned)g;
}

// Workgroups for `tasks` equal tasks when at most `resident` fit the device at once: every
// workgroup takes the same number of tasks (the last fewer), so none waits on a second round
// of a few stragglers.
constexpr unsigned kResident = 2048;  // 8 workgroups of 256 on each of 256 CUs
unsigned balanced_grid(size_t tasks, unsigned resident) {
    if (tasks < 1) return 1;
    const size_t per = (tasks + resident - 1) / resident;
    return (unsigned)((tasks + per - 1) / per);
}

}  // namespace

hipError_t launch_encode_rows(hipStream_t s, fh_kind kind, const float *src, uint8_t *dst, size_t nblocks) {
    unsigned g = grid_for(nblocks, kTaskBlocks, 65535);
    if (kind == FH_Q8_0)
        encode_rows_kernel<FH_Q8_0><<<g, kThreads, 0, s>>>(src, dst, nblocks);
    else
        encode_rows_kernel<FH_Q4_0><<<g, kThreads, 0, s>>>(src, dst, nblocks);
    return hipGetLastError();
}

hipError_t launch_decode_rows(hipStream_t s, fh_kind kind, const uint8_t *src, float *dst, size_t nblocks) {
    unsigned g = balanced_grid((nblocks + kTaskBlocks - 1) / kTaskBlocks, kResident);
    if (kind == FH_Q8_0)
        decode_rows_kernel<FH_Q8_0><<<g, kThreads, 0, s>>>(src, dst, nblocks);
    else
        decode_rows_kernel<FH_Q4_0><<<g, kThreads, 0, s>>>(src, dst, nblocks);
    return hipGetLastError();
}

hipError_t launch_snap_rows(hipStream_t s, const float *src, float *dst, size_t nblocks) {
    unsigned g = grid_for(nblocks, kTaskBlocks, 65535);
    snap_rows_kernel<<<g, kThreads, 0, s>>>(src, dst, nblocks);
    return hipGetLastError();
}

hipError_t launch_encode_cols(hipStream_t s, fh_kind kind, const float *w, uint8_t *qs, uint16_t *ds, size_t k,
                              size_t n) {
    unsigned g = grid_for(k / 32 * n, kThreads, 65535);
    if (kind == FH_Q8_0)
        encode_cols_kernel<FH_Q8_0><<<g, kThreads, 0, s>>>(w, qs, ds, k, n);
    else
        encode_cols_kernel<FH_Q4_0><<<g, kThreads, 0, s>>>(w, qs, ds, k, n);
    return hipGetLastError();
}

hipError_t launch_decode_cols(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, float *w,
                              size_t k, size_t n) {
    unsigned g = grid_for(k / 32 * n, kThreads, 65535);
    if (kind == FH_Q8_0)
        decode_cols_kernel<FH_Q8_0><<<g, kThreads, 0, s>>>(qs, ds, w, k, n);
    else
        decode_cols_kernel<FH_Q4_0><<<g, kThreads, 0, s>>>(qs, ds, w, k, n);
    return hipGetLastError();
}

hipError_t launch_gguf_to_planes(hipStream_t s, fh_kind kind, const uint8_t *src, uint8_t *qs, uint16_t *ds,
                                 size_t n, size_t nb) {
    unsigned g = grid_for(n * nb, kThreads, 65535);
    if (kind == FH_Q8_0)
        gguf_to_planes_kernel<FH_Q8_0><<<g, kThreads, 0, s>>>(src, qs, ds, n, nb);
    else
        gguf_to_planes_kernel<FH_Q4_0><<<g, kThreads, 0, s>>>(src, qs, ds, n, nb);
    return hipGetLastError();
}

hipError_t launch_planes_to_gguf(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, uint8_t *dst,
                                 size_t n, size_t nb) {
    unsigned g = grid_for(n * nb, kThreads, 65535);
    if (kind == FH_Q8_0)
        planes_to_gguf_kernel<FH_Q8_0><<<g, kThreads, 0, s>>>(qs, ds, dst, n, nb);
    else
        planes_to_gguf_kernel<FH_Q4_0><<<g, kThreads, 0, s>>>(qs, ds, dst, n, nb);
    return hipGetLastError();
}

hipError_t launch_copy_f32(hipStream_t s, const float *src, float *dst, size_t n) {
    if (((uintptr_t)src | (uintptr_t)dst) % 16 == 0 && n % 4 == 0) {
        copy_f32x4_kernel<<<grid_for(n / 4, kThreads * 4, 16384), kThreads, 0, s>>>(
            (const f32x4 *)src, (f32x4 *)dst, n / 4);
    } else {
        copy_f32_kernel<<<grid_for(n, kThreads * 4, 16384), kThreads, 0, s>>>(src, dst, n);
    }
    return hipGetLastError();
}

hipError_t launch_decode_f16(hipStream_t s, const uint16_t *src, float *dst, size_t n) {
    decode_f16_kernel<<<grid_for(n, kThreads * 4, 16384), kThreads, 0, s>>>(src, dst, n);
    return hipGetLastError();
}

uint32_t snap_tasks(const SnapDesc &d) {
    switch (d.mode & 0xff) {
    case FH_SNAP_COLS: return (uint32_t)(d.k / 32 * ((d.n + 63) / 64));
    case FH_SNAP_ROWS: return (uint32_t)((d.len / 32 + kRowsTaskBlocks - 1) / kRowsTaskBlocks);
    default: return (uint32_t)((d.len + kCopyTask - 1) / kCopyTask);
    }
}

hipError_t launch_snap_group(hipStream_t s, const SnapDesc *descs, uint32_t count, uint32_t tasks, int cus) {
    if (!count || !tasks) return hipSuccess;
    // every wavefront the chip holds at once (eight workgroups of four per CU), each a strided share
    const unsigned g = grid_for(tasks, kThreads / 64, (unsigned)(cus > 0 ? cus : 256) * 8);
    snap_group_kernel<<<g, kThreads, 0, s>>>(descs, count, tasks);
    return hipGetLastError();
}

hipError_t launch_snap_cols(hipStream_t s, const float *src, float *dst, size_t rows_in, size_t cols_out) {
    unsigned g = grid_for(rows_in / 32 * ((cols_out + 63) / 64), kThreads / 64, 65535);
    if (cols_out % 4 == 0 && ((uintptr_t)src | (uintptr_t)dst) % 16 == 0)
        snap_cols_kernel<true><<<g, kThreads, 0, s>>>(src, dst, rows_in, cols_out);
    else
        snap_cols_kernel<false><<<g, kThreads, 0, s>>>(src, dst, rows_in, cols_out);
    return hipGetLastError();
}

}  // namespace fh
