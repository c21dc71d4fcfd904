// Multi-row products on resident Q8_0 / Q4_0 weights for gfx950: y[M, N] = x[M, K] * W^T, W held
// as the tiled quant and scale planes of its N GGUF rows of K/32 blocks (tile_slot, scale_slot).
//
// naive_kernel: one thread per output, ascending k, the dequantised value formed first and then
// multiplied (ferrum_wgpu/src/shaders/quant/qlinear.wgsl:18-59). Kept as the baseline path.
//
// Both MFMA dequant-GEMMs take the weights' quants as exact f16 integers (Q8_0 -128..127, Q4_0
// -8..7, a byte permute into an f16 exponent pattern and one packed f16 subtract) and scale each
// block's exact dot product by the block's f32 scale after the matrix cores (acc += d * P), so
// the weights carry no rounding; they differ in how finely x is carried:
//
// gemm_precise_kernel (FH_PATH_TILED, within the reference's 1e-5 product tolerance,
// ferrum_wgpu/src/tolerance.rs:7): x = hi + lo, two f16 parts (about 22 bits), split once per
// element by split_x_precise_kernel; per 32 x 32 tile and block four v_mfma_f32_32x32x16_f16.
//
// gemm_kernel (FH_PATH_TILED_FAST, the scoring GEMM, within |g - w| <= 1e-3 + 2e-3 |w|): x = hi
// + lo with hi in f16 and lo kept as e4m3 (about 15 bits in all). Per tile and block two f16
// MFMAs on hi; per two blocks one v_mfma_scale_f32_32x32x64_f8f6f4 on lo times the weights'
// e4m3 correction operand (d * q per element, made once per weight by make_b8_kernel), whose
// power-of-two scales (x lo: per row and 32-element block; the operand: per column) the
// instruction applies itself, so the correction accumulates over all of K with no per-block work.
// That is 1.5 f16-equivalent passes instead of 2. split_x_kernel prepares hi, lo and the scales
// (the layouts are in xsplit.hpp).
//
// k order inside a block (f16 operands): fast_elem_of_pos (xsplit.hpp), the order the quant
// unpack produces. The MFMA sums over k, so x is laid out in that same order and no shuffle is
// needed. The fp8 operands use the pair order of lo_byte (xsplit.hpp) on both sides (the
// instruction pairs lane (row, half h) byte j of A with lane (column, half h) byte j of B, and
// takes bytes 0-15 of every lane as the first scale block, bytes 16-31 as the second).
//
// Tile order (fast kernel): CTAs are dealt round-robin to the 8 XCDs, and each XCD works through
// whole 8 x 8 super-tiles, so the CTAs that run together share stripes of x and of the weights.
#include <type_traits>

#include "device_common.hpp"
#include "internal.hpp"
#include "xsplit.hpp"

namespace fh {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float half_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// A raw buffer resource over [base, base + bytes): loads at offsets at or past `bytes` return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// A CTA's tile: CTAs are dealt round-robin to the eight XCDs (blockIdx.x % 8), and XCD x takes
// the x-th equal contiguous run of the tiles in a grouped order (groups of four row tiles, column
// by column inside a group), so every XCD gets the same share and the CTAs running together on
// one XCD share x rows and weight columns in its L2. The grid is 8 * ceil(tiles / 8) CTAs.
__device__ __forceinline__ bool xcd_tile(uint32_t mt, uint32_t nt, uint32_t *mi, uint32_t *ni) {
    constexpr uint32_t GM = 4;
    const uint32_t tiles = mt * nt, per_xcd = (tiles + 7) / 8;
    const uint32_t local = blockIdx.x / 8, t = (blockIdx.x % 8) * per_xcd + local;
    if (local >= per_xcd || t >= tiles) return false;
    const uint32_t grp = t / (GM * nt), in = t % (GM * nt), gm = min(GM, mt - grp * GM);
    *mi = grp * GM + in % gm;
    *ni = in / gm;
    return true;
}

// ---- naive baseline ----
template <int KIND>
__global__ __launch_bounds__(256) void naive_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ ds,
                                                    const float *__restrict__ x, float *__restrict__ y,
                                                    uint32_t rows, uint32_t k, uint32_t n) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)rows * n) return;
    const uint32_t r = idx / n, c = idx % n, nb = k / 32;
    const float *xr = x + (size_t)r * k;
    float acc = 0.0f;
    for (uint32_t b = 0; b < nb; b++) {
        const size_t blk = tile_slot(c, b, nb);
        const float d = half_bits_to_float(ds[scale_slot(c, b, nb)]);
        if constexpr (KIND == FH_Q8_0) {
            for (int h = 0; h < 2; h++) {
                const u32x4 q = *(const u32x4 *)(qs + blk * 32 + 16 * h);
                for (int i = 0; i < 4; i++)
                    for (int e = 0; e < 4; e++)
                        acc += xr[b * 32 + 16 * h + 4 * i + e] * (d * (float)(int8_t)(q[i] >> (8 * e)));
            }
        } else {
            const u32x4 q = *(const u32x4 *)(qs + blk * 16);
            for (int i = 0; i < 4; i++) {
                for (int e = 0; e < 4; e++) {
                    acc += xr[b * 32 + 4 * i + e] * (d * ((float)((q[i] >> (8 * e)) & 15) - 8.0f));
                    acc += xr[b * 32 + 16 + 4 * i + e] * (d * ((float)((q[i] >> (8 * e + 4)) & 15) - 8.0f));
                }
            }
        }
    }
    y[idx] = acc;
}

// ---- x -> hi (f16, per block in operand order) and the fp8 correction (split_row_fast) ----
// One workgroup per row m (the grid: the M rows).
template <int KIND>
__global__ __launch_bounds__(256) void split_x_kernel(const float *__restrict__ x, _Float16 *__restrict__ xh,
                                                      uint8_t *__restrict__ xl, uint8_t *__restrict__ xsb, uint32_t K) {
    const f32x4 *xr = (const f32x4 *)(x + (size_t)blockIdx.x * K);
    split_row_fast<KIND>([&](uint32_t q) { return xr[q]; }, blockIdx.x, gridDim.x, K, xh, xl, xsb);
}

// ---- the weights' fp8 correction operand: e4m3 of d * q * 2^t per element in the pair order ----
// ---- of x lo (lo_byte), rows of K rounded up to 64 (an odd block count's last pair ends in zeros) ----
// One wavefront per weight row n (an output column of y): 2^t puts the row's largest |d q| just
// under 2^8; bsc[n] holds the E8M0 byte of 2^-t (four copies). Built once per weight.
template <int KIND>
__global__ __launch_bounds__(256) void make_b8_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ ds,
                                                      uint8_t *__restrict__ b8, int32_t *__restrict__ bsc, uint32_t K,
                                                      uint32_t N) {
    const uint32_t n = blockIdx.x * 4 + threadIdx.x / 64, lane = threadIdx.x % 64, nb = K / 32;
    const uint32_t K64 = (K + 63) / 64 * 64;
    if (n >= N) return;  // whole wavefront
    if (nb % 2 && lane < 2) *(u32x4 *)(b8 + (size_t)n * K64 + lo_byte(nb, 16 * lane)) = u32x4{0u, 0u, 0u, 0u};
    float dm = 0.0f;
    for (uint32_t b = lane; b < nb; b += 64) dm = fmaxf(dm, fabsf(half_bits_to_float(ds[scale_slot(n, b, nb)])));
#pragma unroll
    for (int o = 32; o >= 1; o /= 2) dm = fmaxf(dm, __shfl_xor(dm, o, 64));
    const float amax = dm * (KIND == FH_Q8_0 ? 127.0f : 8.0f);
    int t = 0;
    if (amax > 0.0f && amax <= 3.4028235e38f) t = 7 - ((int)(__float_as_uint(amax) >> 23) - 127);
    t = t < -126 ? -126 : (t > 126 ? 126 : t);
    const float f = __uint_as_float((uint32_t)(127 + t) << 23);
    if (lane == 0) bsc[n] = (127 - t) * 0x01010101;
    for (uint32_t c = lane; c < 2 * nb; c += 64) {  // half blocks of 16 elements
        const uint32_t b = c / 2, half = c % 2;
        const size_t slot = tile_slot(n, b, nb);
        const float d = half_bits_to_float(ds[scale_slot(n, b, nb)]) * f;  // exact: a power of two
        u32x4 q;
        if constexpr (KIND == FH_Q8_0)
            q = *(const u32x4 *)(qs + slot * 32 + 16 * half);
        else
            q = *(const u32x4 *)(qs + slot * 16);
        u32x4 o;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t byte = (q[w] >> (8 * i)) & 0xffu;
                e[i] = KIND == FH_Q8_0 ? (float)(int8_t)byte : (float)((int32_t)((byte >> (4 * half)) & 15u) - 8);
            }
            o[w] = fp8x4(d * e[0], d * e[1], d * e[2], d * e[3]);
        }
        *(u32x4 *)(b8 + (size_t)n * K64 + lo_byte(b, 16 * half)) = o;
    }
}

// ---- x -> (hi, lo) f16, per block in operand order: xs[m][b] = 32 hi halves then 32 lo ----
// Eight lanes per (row, block), lane j loading elements 4j..4j+3 (a wavefront reads 1 KiB of
// contiguous x per instruction). |x| beyond the f16 range saturates hi (|x| < 65504 is exact).
__device__ __forceinline__ void split1(float e, _Float16 &h, _Float16 &l) {
    h = (_Float16)fminf(fmaxf(e, -65504.0f), 65504.0f);
    l = (_Float16)(e - (float)h);
}

template <int KIND>
__global__ __launch_bounds__(256) void split_x_precise_kernel(const float *__restrict__ x, _Float16 *__restrict__ xs,
                                                      size_t items) {
    const int j = threadIdx.x % 8;
    for (size_t t = ((size_t)blockIdx.x * 256 + threadIdx.x) / 8; t < items; t += (size_t)gridDim.x * 32) {
        const f32x4 v = __builtin_nontemporal_load((const f32x4 *)(x + t * 32) + j);
        _Float16 *out = xs + t * 64;
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        if constexpr (KIND == 0) {  // natural k order (the other formats' MFMA GEMM)
            const float e[4] = {v.x, v.y, v.z, v.w};
            f16x4 hi, lo;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                _Float16 h, l;
                split1(e[q], h, l);
                hi[q] = h;
                lo[q] = l;
            }
            *(f16x4 *)(out + 4 * j) = hi;
            *(f16x4 *)(out + 32 + 4 * j) = lo;
        } else if constexpr (KIND == FH_Q8_0) {
            // positions 4j..4j+3 hold elements 4j + {0, 2, 1, 3}
            const float e[4] = {v.x, v.z, v.y, v.w};
            f16x4 hi, lo;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                _Float16 h, l;
                split1(e[q], h, l);
                hi[q] = h;
                lo[q] = l;
            }
            *(f16x4 *)(out + 4 * j) = hi;
            *(f16x4 *)(out + 32 + 4 * j) = lo;
        } else {
            // positions 8i..8i+7 hold elements 4i + {0, 2, 1, 3} (lane i) and 16 + 4i + {0, 2, 1, 3}
            // (lane i + 4): lane i < 4 writes the hi part of group i, lane i + 4 the lo part
            f32x4 o;
            o.x = __shfl_xor(v.x, 4, 8);
            o.y = __shfl_xor(v.y, 4, 8);
            o.z = __shfl_xor(v.z, 4, 8);
            o.w = __shfl_xor(v.w, 4, 8);
            const f32x4 a = j < 4 ? v : o, b = j < 4 ? o : v;  // elements 4i.. and 16 + 4i..
            const float e[8] = {a.x, a.z, a.y, a.w, b.x, b.z, b.y, b.w};
            f16x8 part;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                _Float16 h, l;
                split1(e[q], h, l);
                part[q] = j < 4 ? h : l;
            }
            *(f16x8 *)(out + (j < 4 ? 0 : 32) + 8 * (j % 4)) = part;
        }
    }
}

// ---- weight quants -> f16 pairs in operand order ----
__device__ __forceinline__ uint32_t f16x2_add(uint32_t w, _Float16 bias) {
    const f16x2 v = __builtin_bit_cast(f16x2, w) + f16x2{bias, bias};
    return __builtin_bit_cast(uint32_t, v);
}

// 16 quant bytes of a Q4_0 block -> its 32 elements as f16, positions 0..31 (8 per dword).
__device__ __forceinline__ void unpack_q4(const u32x4 q, u32x4 (&out)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t w = q[i];
        // (1024 + nibble) as f16 pairs, then - 1032: the exact value nibble - 8
        out[i][0] = f16x2_add((w & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f);
        out[i][1] = f16x2_add(((w >> 8) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f);
        out[i][2] = f16x2_add(((w >> 4) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f);
        out[i][3] = f16x2_add(((w >> 12) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f);
    }
}

// 16 quant bytes (half a Q8_0 block) -> 16 elements as f16, 4 per dword.
__device__ __forceinline__ void unpack_q8(const u32x4 q, u32x4 (&out)[2]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t t = q[i] ^ 0x80808080u;  // q + 128 as unsigned bytes
        // bytes 0,2 and 1,3 under an f16 exponent byte 0x64: 1024 + q + 128, then - 1152
        out[i / 2][2 * (i % 2)] = f16x2_add(__builtin_amdgcn_perm(0x64646464u, t, 0x04020400u), (_Float16)-1152.0f);
        out[i / 2][2 * (i % 2) + 1] = f16x2_add(__builtin_amdgcn_perm(0x64646464u, t, 0x04030401u), (_Float16)-1152.0f);
    }
}

struct GemmArgs {
    const _Float16 *xh;
    const uint8_t *xl;
    const uint8_t *xsb;
    const uint8_t *qs;
    const uint16_t *ds;
    const uint8_t *b8;
    const int32_t *bsc;
    float *y;
    float *partial;  // K-split partial products (up to 8 x M x N floats), or null: no split
    uint32_t M, K, N;
    SplitOut *defer = nullptr;  // set: the partial sums are left for the consumer
    GemmXSplit act{};           // SWIGLU: where the activation's split x goes
};

// ---- the MFMA GEMM ----
// Per pipeline stage (two blocks, 64 k) a CTA holds in LDS: x hi (f16, operand order), x lo (e4m3),
// the weights' quants unpacked to exact f16 integers, their e4m3 correction operand and the two
// blocks' scales. Per 32 x 32 output tile and block: P = hi * q (two v_mfma_f32_32x32x16_f16),
// acc += d * P; per stage: acc += (lo 2^s) * (d q 2^t) * 2^-s 2^-t (one scaled
// v_mfma_scale_f32_32x32x64_f8f6f4, which applies both powers of two and accumulates in f32).
constexpr int kAStr = 72;   // LDS halves per x row and stage: 64 hi + 8 pad
constexpr int kLStr = 80;   // LDS bytes per x row and stage: 64 e4m3 + 16 pad
constexpr int kBStr = 72;   // LDS halves per weight row and stage: 64 + 8 pad
constexpr int kB8Str = 80;  // LDS bytes per weight row and stage

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));

template <int KIND, int BM, int BN, int WAVES_M>
struct GemmCfg {
    static constexpr int WAVES_N = 4 / WAVES_M;
    static constexpr int TM = BM / WAVES_M / 32, TN = BN / WAVES_N / 32;  // 32x32 tiles per wave
    static constexpr int QB = KIND == FH_Q8_0 ? 32 : 16;                   // quant bytes per block
    static constexpr int XH = BM * 8 / 256;                                // 16-byte x-hi chunks per thread
    static constexpr int XL = (BM * 4 + 255) / 256;                        // 16-byte x-lo chunks per thread
    static constexpr int QC = BN * 2 * QB / 16;                            // 16-byte quant chunks per stage
    static constexpr int QL = (QC + 255) / 256;
    static constexpr int BL = (BN * 4 + 255) / 256;                        // 16-byte b8 chunks per thread
    static constexpr int DL = (BN * 2 + 255) / 256;                        // scales per thread
    static_assert(TM >= 1 && TN >= 1, "wave tile must be whole 32x32 tiles");
    static_assert(BM * 8 % 256 == 0, "x staging must divide over 256 threads");
};

// SWIGLU: the weight's rows are gate and up interleaved in runs of 32 (rows 64c .. 64c + 31 gate
// units 32c .., rows 64c + 32 .. up units 32c ..), so a wavefront's two 32-column fragments hold a
// unit's gate and up, 32 units: one block of the activation act = swiglu_act(gate, up). The
// epilogue passes the tile's activations through LDS and writes them into `act` as the next
// product's split x (split_chunk4) instead of the N outputs (one K split; N a multiple of 64; the
// activation's rows are M, its width N / 2).
template <int KIND, int BM, int BN, int WAVES_M, bool SWIGLU = false>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const _Float16 *__restrict__ xh, const uint8_t *__restrict__ xl,
                                                      const uint8_t *__restrict__ xsb, const uint8_t *__restrict__ qs,
                                                      const uint16_t *__restrict__ ds, const uint8_t *__restrict__ b8,
                                                      const int32_t *__restrict__ bsc, float *__restrict__ y,
                                                      uint32_t M, uint32_t K, uint32_t N, uint32_t mt, uint32_t nt,
                                                      uint32_t split_stages, GemmXSplit act) {
    using C = GemmCfg<KIND, BM, BN, WAVES_M>;
    constexpr uint32_t kA = BM * kAStr * 2, kL = BM * kLStr, kB = BN * kBStr * 2, kB8 = BN * kB8Str, kD = 2 * BN * 4;
    __shared__ __attribute__((aligned(16))) uint8_t arena[kA + kL + kB + kB8 + kD + 2 * BM];
    _Float16 *sA = (_Float16 *)arena;
    uint8_t *sL = arena + kA;
    _Float16 *sB = (_Float16 *)(arena + kA + kL);
    uint8_t *sB8 = arena + kA + kL + kB;
    float *sD = (float *)(arena + kA + kL + kB + kB8);
    uint8_t *sS = arena + kA + kL + kB + kB8 + kD;  // the stage's x lo scale bytes, two per row

    uint32_t mi, ni;
    if (!xcd_tile(mt, nt, &mi, &ni)) return;  // whole CTA: no barrier is left waiting
    const uint32_t m0 = mi * BM, n0 = ni * BN;

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    const uint32_t nb = K / 32, all_stages = (nb + 1) / 2;
    // K split blockIdx.y: stages [st0, st1) (one split: all of them); each split writes its own
    // partial product, y + split * M * N, added up by gemm_reduce_kernel in split order
    const uint32_t st0 = blockIdx.y * split_stages, st1 = min(all_stages, st0 + split_stages);
    y += (size_t)blockIdx.y * M * N;
    const int fr = lane % 32;        // fragment row (x) / column (weights)
    const int fk = 8 * (lane / 32);  // first of this lane's 8 positions in a K = 16 step
    const int f8 = 32 * (lane / 32); // first of this lane's 32 bytes in the K = 64 correction step

    // the correction's power-of-two scales per fragment column (the rows' come with each stage)
    int32_t bscv[C::TN];
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
        const uint32_t n = n0 + (wn * C::TN + j) * 32 + fr;
        bscv[j] = n < N ? bsc[n] : 0x7f7f7f7f;
    }
    // Drain these loads here (vmcnt 0, the other counters left alone): otherwise their possible
    // pendency at the loop head makes the compiler wait for every load in flight, the stage
    // prefetch included, at their first use inside the loop.
    __builtin_amdgcn_s_waitcnt(0x0f70);

    // Per-thread operand offsets at stage 0 (bytes), advanced by a fixed stride per stage. Buffer
    // loads return zeros past each array's end (rows past M and columns past the weight's padded
    // row count); the second block of an odd last stage reads whatever follows, which the f16 pass
    // skips, and the fp8 operands' zero row tails cover it for the correction.
    const uint32_t K64 = (K + 63) / 64 * 64;
    const uint32_t MS = xsb_rows(M);
    const uint32_t n_xh = M * nb * 64, n_xl = M * K64, n_q = (N + 31) / 32 * 32 * nb * C::QB, n_b8 = N * K64,
                   n_d = (N + 31) / 32 * 32 * ((nb + 7) / 8 * 8) * 2, n_sc = K64 / 64 * MS * 2;
    constexpr uint32_t kOut = 0x80000000u;  // an offset past every array: loads return zeros
    uint32_t o_xh[C::XH], o_xl[C::XL], o_q[C::QL], o_b8[C::BL], o_d;
    // threads t < BM / 2 stage 4 bytes of the tile's scale bytes (two per row) per stage
    const uint32_t o_sc = (uint32_t)tid < BM / 2 ? m0 * 2 + 4 * tid : kOut;
    uint32_t s_xh[C::XH], s_xl[C::XL], s_q[C::QL], s_b8[C::BL];  // LDS byte offsets
#pragma unroll
    for (int i = 0; i < C::XH; i++) {
        const int cc = tid + 256 * i, r = cc / 8, bb = (cc % 8) / 4, part = cc % 4;
        const uint32_t m = m0 + r;
        o_xh[i] = m < M ? ((m * nb + bb) * 32 + part * 8) * 2 : kOut;
        s_xh[i] = (r * kAStr + bb * 32 + part * 8) * 2;
    }
#pragma unroll
    for (int i = 0; i < C::XL; i++) {
        const int cc = tid + 256 * i, r = cc / 4, part = cc % 4;
        const uint32_t m = m0 + r;
        o_xl[i] = cc < BM * 4 && m < M ? m * K64 + part * 16 : kOut;
        s_xl[i] = cc < BM * 4 ? r * kLStr + part * 16 : 0u;
    }
#pragma unroll
    for (int i = 0; i < C::QL; i++) {
        const int cc = tid + 256 * i;
        constexpr int CPB = C::QB / 16;  // 16-byte chunks per block
        const int col = cc / (2 * CPB), bb = (cc % (2 * CPB)) / CPB, part = cc % CPB;
        const uint32_t n = n0 + col;
        o_q[i] = cc < C::QC ? (((n >> 5) * nb + bb) * 32 + (n & 31)) * C::QB + part * 16 : kOut;
        s_q[i] = cc < C::QC ? (col * kBStr + bb * 32 + (KIND == FH_Q8_0 ? 16 * part : 0)) * 2 : 0u;
    }
#pragma unroll
    for (int i = 0; i < C::BL; i++) {
        const int cc = tid + 256 * i, col = cc / 4, part = cc % 4;
        const uint32_t n = n0 + col;
        o_b8[i] = cc < BN * 4 && n < N ? n * K64 + part * 16 : kOut;
        s_b8[i] = cc < BN * 4 ? col * kB8Str + part * 16 : 0u;
    }
    {
        const uint32_t n = n0 + tid;  // thread t < BN loads column t's two scales of the stage
        o_d = tid < BN ? (((n >> 5) * ((nb + 7) / 8) * 32 + (n & 31)) * 8) * 2 : kOut;
    }
    // two register sets of staged operands: stage st + 2 is requested while stage st is computed
    u32x4 rxh[2][C::XH], rxl[2][C::XL], rq[2][C::QL], rb8[2][C::BL];
    uint32_t rd[2] = {0u, 0u}, rsc[2] = {0u, 0u};
    // Every stage issues its loads, also the two past the split's end (through empty resources,
    // which return zeros): the number of loads in flight is then the same on every path, so the
    // compiler's waits count exactly the older register set and never drain the prefetch.
    auto load_stage = [&](uint32_t st, int rs) {
        const bool live = st < st1;
        const auto r_xh = make_rsrc(xh, live ? n_xh : 0u);
        const auto r_xl = make_rsrc(xl, live ? n_xl : 0u);
        const auto r_q = make_rsrc(qs, live ? n_q : 0u);
        const auto r_b8 = make_rsrc(b8, live ? n_b8 : 0u);
        const auto r_d = make_rsrc(ds, live ? n_d : 0u);
        const auto r_sc = make_rsrc(xsb, live ? n_sc : 0u);
#pragma unroll
        for (int i = 0; i < C::XH; i++)
            rxh[rs][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_xh, (int)(o_xh[i] + st * 128), 0, 0));
#pragma unroll
        for (int i = 0; i < C::XL; i++)
            rxl[rs][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_xl, (int)(o_xl[i] + st * 64), 0, 0));
#pragma unroll
        for (int i = 0; i < C::QL; i++)
            rq[rs][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_q, (int)(o_q[i] + st * 64 * C::QB), 0, 0));
#pragma unroll
        for (int i = 0; i < C::BL; i++)
            rb8[rs][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_b8, (int)(o_b8[i] + st * 64), 0, 0));
        // blocks 2 st and 2 st + 1 are neighbours in one run of eight scales
        rd[rs] = __builtin_amdgcn_raw_buffer_load_b32(r_d, (int)(o_d + (st >> 2) * 512 + (st & 3) * 4), 0, 0);
        rsc[rs] = __builtin_amdgcn_raw_buffer_load_b32(r_sc, (int)(o_sc + st * MS * 2), 0, 0);
    };
    auto store_stage = [&](int rs) {
        uint8_t *sAb = (uint8_t *)sA, *sBb = (uint8_t *)sB;
#pragma unroll
        for (int i = 0; i < C::XH; i++) *(u32x4 *)(sAb + s_xh[i]) = rxh[rs][i];
#pragma unroll
        for (int i = 0; i < C::XL; i++)
            if (tid + 256 * i < BM * 4) *(u32x4 *)(sL + s_xl[i]) = rxl[rs][i];
#pragma unroll
        for (int i = 0; i < C::QL; i++) {
            if (tid + 256 * i < C::QC) {
                if constexpr (KIND == FH_Q8_0) {
                    u32x4 o[2];
                    unpack_q8(rq[rs][i], o);
                    *(u32x4 *)(sBb + s_q[i]) = o[0];
                    *(u32x4 *)(sBb + s_q[i] + 16) = o[1];
                } else {
                    u32x4 o[4];
                    unpack_q4(rq[rs][i], o);
#pragma unroll
                    for (int e = 0; e < 4; e++) *(u32x4 *)(sBb + s_q[i] + 16 * e) = o[e];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < C::BL; i++)
            if (tid + 256 * i < BN * 4) *(u32x4 *)(sB8 + s_b8[i]) = rb8[rs][i];
        if (tid < BN) {
            sD[tid] = half_to_float(rd[rs] & 0xffffu);
            sD[BN + tid] = half_to_float(rd[rs] >> 16);
        }
        if (tid < BM / 2) *(uint32_t *)(sS + 4 * tid) = rsc[rs];
    };

    f32x16 acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // one stage: store the staged registers of set RS, request stage st + 2 into that set, compute
    auto stage = [&](uint32_t st, auto rs_c) {
        constexpr int rs = decltype(rs_c)::value;
        __syncthreads();  // every wave is done reading the previous stage
        store_stage(rs);
        __syncthreads();
        load_stage(st + 2, rs);  // in flight during the next two stages' MFMAs
        const int nbb = nb - 2 * st < 2u ? 1 : 2;  // wave-uniform
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            if (bb >= nbb) break;
            f16x8 bf[C::TN][2];
            float dcol[C::TN];
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const int col = (wn * C::TN + j) * 32 + fr;
#pragma unroll
                for (int s2 = 0; s2 < 2; s2++) bf[j][s2] = *(const f16x8 *)(&sB[col * kBStr + bb * 32 + 16 * s2 + fk]);
                dcol[j] = sD[bb * BN + col];
            }
            f16x8 ah[C::TM][2];
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
                const int r = (wm * C::TM + i) * 32 + fr;
#pragma unroll
                for (int s2 = 0; s2 < 2; s2++) ah[i][s2] = *(const f16x8 *)(&sA[r * kAStr + bb * 32 + 16 * s2 + fk]);
            }
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++) {
                    f32x16 p = {};
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], bf[j][0], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], bf[j][1], p, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 16; q++) acc[i][j][q] = fmaf(dcol[j], p[q], acc[i][j][q]);
                }
        }
        // the correction over the stage's 64 k (blocks past nb hold zeros), with the scale of the
        // lane's half: block 2 st + lane / 32 of its fragment row (rows past M, lo zero, take 2^0)
        int32_t asc[C::TM];
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const uint32_t r = (wm * C::TM + i) * 32 + fr;
            asc[i] = m0 + r < M ? (int32_t)sS[2 * r + lane / 32] : 127;
        }
        i32x8 b8f[C::TN], a8[C::TM];
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int col = (wn * C::TN + j) * 32 + fr;
            b8f[j] = *(const i32x8 *)(&sB8[col * kB8Str + f8]);
        }
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int r = (wm * C::TM + i) * 32 + fr;
            a8[i] = *(const i32x8 *)(&sL[r * kLStr + f8]);
        }
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8[i], b8f[j], acc[i][j], 0, 0, 0, asc[i], 0,
                                                                            bscv[j]);
    };
    load_stage(st0, 0);
    load_stage(st0 + 1, 1);
    // unrolled by two (the register sets are named statically); an odd last stage runs after the
    // loop, so every trip round the loop issues the same loads
    uint32_t st = st0;
    for (; st + 1 < st1; st += 2) {
        stage(st, std::integral_constant<int, 0>{});
        stage(st + 1, std::integral_constant<int, 1>{});
    }
    if (st < st1) stage(st, std::integral_constant<int, 0>{});

    // D layout of a 32x32 tile: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32
    if constexpr (SWIGLU) {
        static_assert(C::TN % 2 == 0, "a wavefront's fragments pair gate and up");
        // the tile's BM x BN / 2 activations through LDS (rows kRow floats apart), then eight lanes
        // per row and block write the split x with whole 64-unit rows per group of 16 lanes
        constexpr uint32_t U = BN / 2, kRow = U + 4;
        static_assert(BM * kRow * 4 <= kA + kL + kB + kB8, "the epilogue's LDS fits the stage buffers");
        static_assert(BM * U / 4 % 256 == 0, "whole 8-lane groups");
        float *sT = (float *)arena;
        __syncthreads();  // every wave is done reading the last stage
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j += 2) {
                const uint32_t u = (wn * C::TN + j) * 16 + fr;  // the tile's unit (gate run / 2 + fr)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t rl = (wm * C::TM + i) * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                    sT[rl * kRow + u] = swiglu_act(acc[i][j][r], acc[i][j + 1][r]);
                }
            }
        __syncthreads();
        const uint32_t units = N / 2, MS = xsb_rows(M), onb = units / 32, oK64 = (units + 63) / 64 * 64;
        // thread t: float4 q = t % (U / 4) (the same block b and place j) of rows t / (U / 4) + i R
        constexpr uint32_t R = 256 / (U / 4);
        const uint32_t q = tid % (U / 4), unit = n0 / 2 + 4 * q, b = unit / 32, j = q % 8;
        if (unit < units) {  // (the same for the eight lanes of a block)
            const uint32_t r0 = tid / (U / 4);
            _Float16 *hb = act.xh + ((size_t)(m0 + r0) * onb + b) * 32;
            uint8_t *lw = act.xl + (size_t)(m0 + r0) * oK64 + lo_byte(b, 4 * j);
            uint8_t *sb = act.xsb + xsb_at(m0 + r0, b, MS);
            const bool tail = onb % 2 && b == onb - 1 && j < 2;
#pragma unroll
            for (uint32_t rl = r0; rl < BM; rl += R) {
                if (m0 + rl >= M) break;
                split_chunk4_at<KIND>(*(const f32x4 *)(sT + rl * kRow + 4 * q), j, hb, lw, sb);
                if (tail) split_tail(m0 + rl, onb, oK64, MS, act.xl, act.xsb, j);
                hb += (size_t)R * onb * 32;
                lw += (size_t)R * oK64;
                sb += 2 * R;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const uint32_t col = n0 + (wn * C::TN + j) * 32 + fr;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t row = m0 + (wm * C::TM + i) * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                    if (row < M && col < N) y[(size_t)row * N + col] = acc[i][j][r];
                }
            }
    }
}

// K splits for a grid of `tiles` CTAs over `stages` stages. Each split is at least four stages
// long (at most 8 splits; two-stage splits were 4% slower on the Qwen2 scoring forward); among
// those counts, the one with the least rounds x (stages per split + 2), a round being 512 CTAs
// (two per CU) and 2 stages a split's own cost (prologue, epilogue). Asking for two CTAs per CU
// regardless of rounds gave the 112-tile down product at M = 2048 five splits, 48 CTAs of them in
// a second round; four splits made the Qwen2 forward 4.5% faster there (7.77 -> 7.42 ms).
uint32_t gemm_splits(uint64_t tiles, uint32_t stages) {
    if (tiles >= 512) return 1;
    const uint32_t cap = min(8u, max(stages / 4, 1u));
    uint32_t best = 1;
    uint64_t cost = ~0ull;
    for (uint32_t sp = 1; sp <= cap; sp++) {
        const uint64_t rounds = (tiles * sp + 511) / 512, per = (stages + sp - 1) / sp;
        if (rounds * (per + 2) < cost) {
            cost = rounds * (per + 2);
            best = sp;
        }
    }
    return best;
}

__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float *__restrict__ part, float *__restrict__ y,
                                                          size_t n, uint32_t splits) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        float t = part[i];
        for (uint32_t s = 1; s < splits; s++) t += part[s * n + i];
        y[i] = t;
    }
}

template <int KIND, int BM, int BN, int WAVES_M, bool SWIGLU = false>
hipError_t run_gemm(hipStream_t s, const GemmArgs &g) {
    const uint32_t mt = (g.M + BM - 1) / BM, nt = (g.N + BN - 1) / BN;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7ffffff0ull) return hipErrorInvalidValue;
    const uint32_t grid = (uint32_t)((tiles + 7) / 8 * 8);  // an equal share for every XCD
    const uint32_t stages = (g.K / 32 + 1) / 2;
    const uint32_t sp = g.partial ? gemm_splits((uint64_t)mt * nt, stages) : 1;
    if (SWIGLU && sp != 1) return hipErrorInvalidValue;  // (gemm_swiglu_supported rules it out)
    const uint32_t per = (stages + sp - 1) / sp;
    float *out = sp > 1 ? g.partial : g.y;
    gemm_kernel<KIND, BM, BN, WAVES_M, SWIGLU><<<dim3(grid, sp), 256, 0, s>>>(g.xh, g.xl, g.xsb, g.qs, g.ds, g.b8, g.bsc,
                                                                               out, g.M, g.K, g.N, mt, nt, per, g.act);
    if (g.defer) *g.defer = sp > 1 ? SplitOut{g.partial, sp} : SplitOut{g.y, 1u};
    if (sp > 1 && !g.defer) {
        const size_t n = (size_t)g.M * g.N;
        const unsigned rg = (unsigned)min((n + 1023) / 1024, (size_t)16384);
        gemm_reduce_kernel<<<rg, 256, 0, s>>>(g.partial, g.y, n, sp);  // (a split past the last stage wrote zeros)
    }
    return hipGetLastError();
}

// The fast and the other formats' MFMA GEMMs take 64-row tiles up to 1024 rows (more row tiles,
// fewer K splits on the scoring shapes), 128 beyond (measured: the precise GEMM gains nothing).
constexpr uint32_t kMidRows = 1024;
void fast_tile(size_t rows, size_t *bm, size_t *bn) {
    *bm = rows <= 32 ? 32 : rows <= kMidRows ? 64 : 128;
    *bn = rows <= 32 ? 256 : 128;
}

template <int KIND, bool SWIGLU = false>
hipError_t gemm_dispatch(hipStream_t s, const GemmArgs &g) {
    if (g.M <= 32) return run_gemm<KIND, 32, 256, 1, SWIGLU>(s, g);
    if (g.M <= kMidRows) return run_gemm<KIND, 64, 128, 2, SWIGLU>(s, g);
    return run_gemm<KIND, 128, 128, 2, SWIGLU>(s, g);
}

// ---- the precise MFMA GEMM (FH_PATH_TILED): x as two f16 parts, about 22 bits ----
constexpr int kARow2 = 72;  // LDS halves per x row and block: 32 hi + 32 lo + 8 pad (144 B)
constexpr int kBRow2 = 40;  // LDS halves per weight row and block: 32 + 8 pad (80 B)
constexpr int kBKB = 1;    // blocks (of 32 k) per pipeline stage

template <int KIND, int BM, int BN, int WAVES_M>
struct GemmCfg2 {
    static constexpr int WAVES_N = 4 / WAVES_M;
    static constexpr int TM = BM / WAVES_M / 32, TN = BN / WAVES_N / 32;  // 32x32 tiles per wave
    static constexpr int QB = KIND == FH_Q8_0 ? 32 : 16;                   // quant bytes per block
    static constexpr int A_LD = kBKB * BM * 8 / 256;                       // 16-byte x chunks per thread
    static constexpr int B_LD = kBKB * BN * QB / 16;                       // 16-byte quant chunks per stage
    static constexpr int B_PER = (B_LD + 255) / 256;                       // of them per thread
    static constexpr int D_PER = (kBKB * BN + 255) / 256;                  // scales per thread
    static_assert(TM >= 1 && TN >= 1, "wave tile must be whole 32x32 tiles");
    static_assert(BM * 8 % 256 == 0, "x staging must divide over 256 threads");
    static_assert(B_LD % 256 == 0 || B_LD < 256, "weight chunks must divide over the threads");
};

template <int KIND, int BM, int BN, int WAVES_M>
__global__ __launch_bounds__(256, 2) void gemm_precise_kernel(const _Float16 *__restrict__ xs, const uint8_t *__restrict__ qs,
                                                      const uint16_t *__restrict__ ds, float *__restrict__ y,
                                                      uint32_t M, uint32_t K, uint32_t N, uint32_t mt, uint32_t nt,
                                                      uint32_t split_stages) {
    using C = GemmCfg2<KIND, BM, BN, WAVES_M>;
    // stage layout: x row r, block bb at r * kBKB * kARow2 + bb * kARow2; weight row likewise
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][BM * kBKB * kARow2];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][BN * kBKB * kBRow2];
    __shared__ float sD[2][kBKB * BN];

    // tile of this CTA: the XCD's contiguous share of the tiles, N fastest
    const uint32_t tiles = mt * nt, c = blockIdx.x;
    const uint32_t per_xcd = (tiles + 7) / 8;
    const uint32_t t = (c % 8) * per_xcd + c / 8;
    if (t >= tiles) return;  // whole CTA: no barrier is left waiting
    const uint32_t mi = t / nt, ni = t % nt;
    const uint32_t m0 = mi * BM, n0 = ni * BN;

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    const uint32_t nb = K / 32;
    // split blockIdx.y of the K range: stages st0 .. st1 - 1, its partial product at y + split * M * N
    // (added up by gemm_reduce_kernel in split order)
    const uint32_t all_stages = (nb + kBKB - 1) / kBKB;
    const uint32_t st0 = blockIdx.y * split_stages, st1 = min(all_stages, st0 + split_stages);
    y += (size_t)blockIdx.y * M * N;

    u32x4 ra[C::A_LD];
    u32x4 rb[C::B_PER];
    uint32_t rh[C::D_PER];

    // Stage st holds blocks st * kBKB .. + kBKB - 1; blocks past nb load zeros.
    auto load_stage = [&](uint32_t st) {
#pragma unroll
        for (int i = 0; i < C::A_LD; i++) {
            const int cc = tid + 256 * i, r = cc / (8 * kBKB), bb = (cc / 8) % kBKB, ch = cc % 8;
            const uint32_t m = m0 + r, kb = st * kBKB + bb;
            ra[i] = m < M && kb < nb ? *(const u32x4 *)(xs + ((size_t)m * nb + kb) * 64 + ch * 8)
                                     : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < C::B_PER; i++) {
            const int cc = tid + 256 * i;
            if (cc < C::B_LD) {
                constexpr int CPR = kBKB * C::QB / 16;  // chunks per weight row per stage
                const int col = cc / CPR, bb = (cc % CPR) / (C::QB / 16), part = cc % (C::QB / 16);
                const uint32_t n = n0 + col, kb = st * kBKB + bb;
                rb[i] = n < N && kb < nb ? __builtin_nontemporal_load(
                                               (const u32x4 *)(qs + tile_slot(n, kb, nb) * C::QB + part * 16))
                                         : u32x4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int i = 0; i < C::D_PER; i++) {
            const int cc = tid + 256 * i;
            if (cc < kBKB * BN) {
                const int col = cc / kBKB, bb = cc % kBKB;
                const uint32_t n = n0 + col, kb = st * kBKB + bb;
                rh[i] = n < N && kb < nb ? ds[scale_slot(n, kb, nb)] : 0u;
            }
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < C::A_LD; i++) {
            const int cc = tid + 256 * i, r = cc / (8 * kBKB), bb = (cc / 8) % kBKB, ch = cc % 8;
            *(u32x4 *)(&sA[buf][(r * kBKB + bb) * kARow2 + ch * 8]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < C::B_PER; i++) {
            const int cc = tid + 256 * i;
            if (cc < C::B_LD) {
                constexpr int CPR = kBKB * C::QB / 16;
                const int col = cc / CPR, bb = (cc % CPR) / (C::QB / 16), part = cc % (C::QB / 16);
                _Float16 *row = &sB[buf][(col * kBKB + bb) * kBRow2];
                if constexpr (KIND == FH_Q8_0) {
                    u32x4 o[2];
                    unpack_q8(rb[i], o);
                    *(u32x4 *)(row + 16 * part) = o[0];
                    *(u32x4 *)(row + 16 * part + 8) = o[1];
                } else {
                    u32x4 o[4];
                    unpack_q4(rb[i], o);
#pragma unroll
                    for (int e = 0; e < 4; e++) *(u32x4 *)(row + 8 * e) = o[e];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < C::D_PER; i++) {
            const int cc = tid + 256 * i;
            if (cc < kBKB * BN) sD[buf][(cc % kBKB) * BN + cc / kBKB] = half_to_float(rh[i]);
        }
    };

    f32x16 acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int fr = lane % 32;        // fragment row (x) / column (weights)
    const int fk = 8 * (lane / 32);  // first of this lane's 8 positions in a K = 16 step

    if (st0 < st1) {
        load_stage(st0);
        store_stage(0);
    }
    __syncthreads();
    for (uint32_t st = st0; st < st1; st++) {
        const int buf = (st - st0) & 1;
        const bool more = st + 1 < st1;
        if (more) load_stage(st + 1);  // in flight during the MFMAs below
        const int nbb = nb - st * kBKB < (uint32_t)kBKB ? (int)(nb - st * kBKB) : kBKB;  // wave-uniform
#pragma unroll
        for (int bb = 0; bb < kBKB; bb++) {
            if (bb >= nbb) break;
            f16x8 bf[C::TN][2];
            float dcol[C::TN];
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const int col = (wn * C::TN + j) * 32 + fr;
                const _Float16 *row = &sB[buf][(col * kBKB + bb) * kBRow2];
#pragma unroll
                for (int s = 0; s < 2; s++) bf[j][s] = *(const f16x8 *)(row + 16 * s + fk);
                dcol[j] = sD[buf][bb * BN + col];
            }
            f16x8 ah[C::TM][2], al[C::TM][2];
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
                const int r = (wm * C::TM + i) * 32 + fr;
                const _Float16 *row = &sA[buf][(r * kBKB + bb) * kARow2];
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    ah[i][s] = *(const f16x8 *)(row + 16 * s + fk);
                    al[i][s] = *(const f16x8 *)(row + 32 + 16 * s + fk);
                }
            }
            // Per tile: P = hi * q + lo * q over the block (four MFMAs), then acc += d * P.
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++) {
                    f32x16 p = {};
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], bf[j][0], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], bf[j][1], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], bf[j][0], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], bf[j][1], p, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 16; q++) acc[i][j][q] = fmaf(dcol[j], p[q], acc[i][j][q]);
                }
        }
        if (more) store_stage(buf ^ 1);  // nobody reads buf ^ 1 during this stage
        __syncthreads();
    }

    // D layout of a 32x32 tile: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const uint32_t col = n0 + (wn * C::TN + j) * 32 + fr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + (wm * C::TM + i) * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                if (row < M && col < N) y[(size_t)row * N + col] = acc[i][j][r];
            }
        }
}

// The precise kernel's tile shape by rows and its K split (the rule of gemm_splits).
void precise_tile(size_t rows, size_t *bm, size_t *bn) {
    *bm = rows <= 32 ? 32 : rows <= 64 ? 64 : 128;
    *bn = rows <= 32 ? 256 : 128;
}

uint32_t precise_splits(size_t rows, size_t k, size_t n) {
    size_t bm, bn;
    precise_tile(rows, &bm, &bn);
    const uint64_t tiles = (uint64_t)((rows + bm - 1) / bm) * ((n + bn - 1) / bn);
    return gemm_splits(tiles, (uint32_t)((k / 32 + kBKB - 1) / kBKB));
}

template <int KIND, int BM, int BN, int WAVES_M>
hipError_t run_gemm_precise(hipStream_t s, const _Float16 *xs, const uint8_t *qs, const uint16_t *ds, float *y,
                            float *partial, uint32_t M, uint32_t K, uint32_t N, SplitOut *defer) {
    const uint32_t mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7fffffffull) return hipErrorInvalidValue;
    const uint32_t grid = (uint32_t)((tiles + 7) / 8 * 8);  // a multiple of the XCD count
    const uint32_t stages = (K / 32 + kBKB - 1) / kBKB;
    const uint32_t sp = partial ? precise_splits(M, K, N) : 1;
    const uint32_t per = (stages + sp - 1) / sp;
    float *out = sp > 1 ? partial : y;
    gemm_precise_kernel<KIND, BM, BN, WAVES_M><<<dim3(grid, sp), 256, 0, s>>>(xs, qs, ds, out, M, K, N, mt, nt, per);
    if (defer) *defer = sp > 1 ? SplitOut{partial, sp} : SplitOut{y, 1u};
    if (sp > 1 && !defer) {
        const size_t n = (size_t)M * N;
        const unsigned rg = (unsigned)min((n + 1023) / 1024, (size_t)16384);
        gemm_reduce_kernel<<<rg, 256, 0, s>>>(partial, y, n, sp);  // (a split past the last stage wrote zeros)
    }
    return hipGetLastError();
}

// ---- the precise GEMM on a streaming 256 x 256 skeleton (products with at least 128 such tiles) ----
// Same numerics as gemm_precise_kernel (per 32 x 32 tile and block P = hi q + lo q on four
// v_mfma_f32_32x32x16_f16, then acc += d P), on gemm_f16_big_kernel's structure: eight wavefronts
// per CTA (two per SIMD), one CTA per CU working through its tiles as one stream of stages, so the
// next tile's first stages are loaded while the current one finishes and a tile's output stores
// drain during the next one. A stage is one block (32 k).
//
// Every operand goes from memory straight into LDS (buffer loads with the LDS destination, no
// registers), two stages ahead: x's hi and lo rows (128 bytes per row, 32 KB per stage) into a
// ring of three buffers; the block's packed quants (16 or 32 bytes per column) and the dwords
// holding its scales into a ring of two. At the top of stage p the quants of stage p + 1 are
// unpacked once, LDS to LDS, into exact f16 integers (and the scales to f32), double-buffered.
// One barrier per stage. A wavefront owns a 64 x 128 part (2 x 4 tiles): per stage eight 16-byte
// x reads and two weight reads per column tile feed 32 MFMAs.
//
// The loads are inline assembly with explicit s_waitcnt: the compiler's own wait insertion could
// not tell the LDS-destination loads apart and drained every load in flight at each barrier
// (one stage of lookahead instead of two), and a register destination written behind the
// compiler's back was copied before its data arrived. Per wave the loads go out as weights(p + 2)
// then x(p + 2) (four instructions) in stage p, so at the top of stage p + 1 waiting until at most
// four loads are outstanding (loads complete in order) leaves weights(p + 2) and x(p + 1) in LDS;
// the barrier then covers every wave's share.
//
// x rows in LDS are 128 bytes without padding; the 16-byte chunk c of row r sits at position
// c ^ ((r >> 1) & 7), so the sixteen rows that one cycle of a 16-byte fragment read serves (256
// bytes of the 64 banks) fall on sixteen different 16-byte bank groups (each wave's load
// instruction fills 1 KB of LDS, eight whole rows, choosing per lane which chunk it fetches).
// (With c ^ (r % 8), conflict-free for eight lanes per cycle, SQ_LDS_BANK_CONFLICT counted as
// many conflict cycles as LDS instruction cycles.)
constexpr int kSB = 40;  // LDS halves per weight column and stage: 32 + 8 pad (80 B)

// 2 quant dwords of a Q4_0 block (dwords 2h, 2h + 1) -> positions 16 h .. 16 h + 15 as exact f16
__device__ __forceinline__ void unpack_q4_half(uint32_t w0, uint32_t w1, u32x4 &o0, u32x4 &o1) {
    const uint32_t w[2] = {w0, w1};
    u32x4 o[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        o[i][0] = f16x2_add((w[i] & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f);
        o[i][1] = f16x2_add(((w[i] >> 8) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f);
        o[i][2] = f16x2_add(((w[i] >> 4) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f);
        o[i][3] = f16x2_add(((w[i] >> 12) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f);
    }
    o0 = o[0];
    o1 = o[1];
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// A raw buffer descriptor in scalar registers over [base, base + bytes) (the make_rsrc layout).
__device__ __forceinline__ i32x4 sgpr_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    return i32x4{__builtin_amdgcn_readfirstlane((int32_t)(uint32_t)a),
                 __builtin_amdgcn_readfirstlane((int32_t)((uint32_t)(a >> 32) & 0xffffu)),
                 __builtin_amdgcn_readfirstlane((int32_t)bytes), 0x00020000};
}
// 16 (4) bytes per lane from r at voff into LDS at lds + 16 (4) * lane; lds wave-uniform. An M0
// write needs one wait state before a load that reads it.
__device__ __forceinline__ void asm_load_lds16(i32x4 r, uint32_t lds, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(voff),
                 "s"(r)
                 : "m0");
}
__device__ __forceinline__ void asm_load_lds4(i32x4 r, uint32_t lds, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(lds), "v"(voff), "s"(r)
                 : "m0");
}

// ---- the scoring head's score epilogue (both streaming kernels) ----
// nn::score (ferrum_ref/src/kernels/nn.rs:117-129) per row is a maximum, a sum of exp(v - max) and
// the first column holding the maximum; they merge across stretches of the row as score_kernel's
// lane groups do (the sums rescaled to the larger maximum; the smaller column wins a tie). The
// head's epilogue reduces each row's 256 columns of a tile to these three (the logits themselves,
// 1.24 GB at 2048 x 151,936, are never written), a small pass merges the tiles in order.
constexpr uint32_t kNoCol = 0xffffffffu;
__device__ __forceinline__ void score_merge(float &m, float &s, uint32_t &f, float m2, float s2, uint32_t f2) {
    const float mx = fmaxf(m, m2);
    s = (m == -INFINITY ? 0.0f : s * __expf(m - mx)) + (m2 == -INFINITY ? 0.0f : s2 * __expf(m2 - mx));
    f = m2 > m || (m2 == m && f2 < f) ? f2 : f;
    m = mx;
}

// One halving step of score_tile's row exchange: lanes whose bit W is clear keep rows 0..W-1 of
// their set, the others rows W..2W-1 (renumbered from 0), each merged with its partner lane's copy.
template <int W>
__device__ __forceinline__ void score_halve(float (&vm)[32], float (&vs)[32], uint32_t (&vf)[32], int fr) {
    const bool hi = (fr & W) != 0;
#pragma unroll
    for (int k = 0; k < W; k++) {
        const float sm = hi ? vm[k] : vm[k + W], ss = hi ? vs[k] : vs[k + W];
        const uint32_t sf = hi ? vf[k] : vf[k + W];
        const float rm = __shfl_xor(sm, W), rs = __shfl_xor(ss, W);
        const uint32_t rf = (uint32_t)__shfl_xor((int)sf, W);
        float km = hi ? vm[k + W] : vm[k], ks = hi ? vs[k + W] : vs[k];
        uint32_t kf = hi ? vf[k + W] : vf[k];
        score_merge(km, ks, kf, rm, rs, rf);
        vm[k] = km;
        vs[k] = ks;
        vf[k] = kf;
    }
}

// The epilogue of the 256 x 256 tile at (m0, n0) (acc: the wavefront's 2 x 4 32x32 tiles, register
// r of lane l holding row 8 (r / 4) + 4 (l / 32) + r % 4 and column l % 32 of its tile). Per lane
// and row: the statistics of its four columns; then the 32 lanes of a half-wavefront, which share
// 16 x 2 rows, halve their rows five times (each lane keeps one half and merges the partner's copy
// of it), which leaves lane l with row l % 32 of its half over the wavefront's 128 columns; the
// wavefronts of the two column halves meet through xch (3 KB of LDS), and so.part[row][n0 / 256]
// gets the tile's statistics. The lane whose column is a row's target writes the logit. Every
// wavefront of the CTA calls it (one barrier).
__device__ __forceinline__ void score_tile(const f32x16 (&acc)[2][4], uint32_t m0, uint32_t n0, uint32_t M, uint32_t N,
                                           const ScoreOut &so, uint8_t *xch) {
    const int lane = threadIdx.x % 64, fr = lane % 32, hf = lane / 32;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), wm = wave % 4, wn = wave / 4;
    const uint32_t cb = n0 + wn * 128 + fr;  // the lane's column in tile j = 0 (+ 32 j)
    float vm[32], vs[32];
    uint32_t vf[32];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            // the targets of band rows i 32 + 8 q .. + 7 (scalar loads; so.tgt is padded)
            const int32_t *tb = so.tgt + m0 + wm * 64 + i * 32 + 8 * q;
            int32_t T[8];
#pragma unroll
            for (int e = 0; e < 8; e++) T[e] = tb[e];
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
                const int r = 4 * q + rr, k = 16 * i + r;
                float v[4], mx = -INFINITY;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    v[j] = cb + 32 * j < N ? acc[i][j][r] : -INFINITY;
                    mx = fmaxf(mx, v[j]);
                }
                uint32_t first = kNoCol;
#pragma unroll
                for (int j = 3; j >= 0; j--)
                    if (v[j] == mx) first = cb + 32 * j;
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (cb + 32 * j < N) sum += __expf(v[j] - mx);
                vm[k] = mx;
                vs[k] = sum;
                vf[k] = first;
                int32_t t0 = T[rr], t1 = T[4 + rr];  // (named values, as below)
                asm volatile("" : "+v"(t0), "+v"(t1));
                const int32_t t = hf ? t1 : t0;
                const int32_t dt = t - (int32_t)cb;
                const uint32_t row = m0 + wm * 64 + i * 32 + 8 * q + 4 * hf + rr;
                if (dt >= 0 && dt < 128 && (dt & 31) == 0 && row < M) {
                    // (four named values: a select among the array's elements would become an indexed
                    // access and put the accumulators in scratch memory)
                    float a0 = v[0], a1 = v[1], a2 = v[2], a3 = v[3];
                    asm volatile("" : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3));
                    so.tlogit[row] = dt == 0 ? a0 : dt == 32 ? a1 : dt == 64 ? a2 : a3;
                }
            }
        }
    score_halve<16>(vm, vs, vf, fr);
    score_halve<8>(vm, vs, vf, fr);
    score_halve<4>(vm, vs, vf, fr);
    score_halve<2>(vm, vs, vf, fr);
    score_halve<1>(vm, vs, vf, fr);
    // lane l now holds row k = l % 32 of its half: i = k / 16, r = k % 16
    float *xm = (float *)xch, *xs = xm + 256;
    uint32_t *xf = (uint32_t *)(xs + 256);
    const uint32_t slot = wm * 64 + lane;
    if (wn == 1) {
        xm[slot] = vm[0];
        xs[slot] = vs[0];
        xf[slot] = vf[0];
    }
    __syncthreads();
    if (wn == 0) {
        score_merge(vm[0], vs[0], vf[0], xm[slot], xs[slot], xf[slot]);
        const int k = fr, i = k / 16, r = k % 16;
        const uint32_t row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * hf + r % 4;
        if (row < M)
            *(f32x4 *)(so.part + ((size_t)row * so.ntn + n0 / 256) * 4) = f32x4{vm[0], vs[0], __uint_as_float(vf[0]), 0.0f};
    }
}

template <int KIND>
struct StreamLds {  // byte offsets of the rings inside the kernel's LDS arena
    static constexpr uint32_t QB = KIND == FH_Q8_0 ? 32 : 16;
    static constexpr uint32_t A = 0, A_SZ = 256 * 128;                      // x: three stages
    static constexpr uint32_t W = 3 * A_SZ, W_Q = 256 * QB, W_SZ = W_Q + 1024;  // raw weights: two
    static constexpr uint32_t B = W + 2 * W_SZ, B_SZ = 256 * kSB * 2;      // unpacked weights: two
    static constexpr uint32_t D = B + 2 * B_SZ, D_SZ = 1024;                // f32 scales: two
    static constexpr uint32_t TOTAL = D + 2 * D_SZ;
};

// SCORE: the scoring head's epilogue (score_tile into so) instead of the stores.
template <int KIND, bool SCORE = false>
__global__ __launch_bounds__(512, 1) void gemm_stream_precise_kernel(const _Float16 *__restrict__ xs,
                                                                     const uint8_t *__restrict__ qs,
                                                                     const uint16_t *__restrict__ ds,
                                                                     float *__restrict__ y, uint32_t M, uint32_t K,
                                                                     uint32_t N, uint32_t mt, uint32_t nt,
                                                                     uint32_t split_stages, ScoreOut so) {
    using S = StreamLds<KIND>;
    constexpr uint32_t QB = S::QB;
    __shared__ __attribute__((aligned(1024))) uint8_t arena[S::TOTAL + (SCORE ? 3072 : 0)];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t *)arena;

    // This CTA's tiles, as gemm_f16_big_kernel deals them: XCD x (blockIdx.x % 8) owns the x-th
    // equal run of a grouped tile order (groups of eight row tiles) and its CTAs take the run's
    // tiles round robin.
    constexpr uint32_t GM = 8;
    const uint32_t tiles = mt * nt, per_xcd = (tiles + 7) / 8, ctas = gridDim.x / 8;
    const uint32_t run0 = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8, run1 = min(tiles, (blockIdx.x % 8 + 1) * per_xcd);
    if (run0 >= run1) return;  // whole CTA: no barrier is left waiting
    const uint32_t my_tiles = (run1 - run0 + ctas - 1) / ctas;
    auto origin = [&](uint32_t k, uint32_t &m0, uint32_t &n0) {  // row and column of my k-th tile
        const uint32_t t = run0 + k * ctas;
        const uint32_t grp = t / (GM * nt), in = t % (GM * nt), gm = min(GM, mt - grp * GM);
        m0 = (grp * GM + in % gm) * 256;
        n0 = (in / gm) * 256;
    };

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, wm = wave % 4, wn = wave / 4;
    const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t nb = K / 32;
    const uint32_t st0 = blockIdx.y * split_stages, st1 = min(nb, st0 + split_stages);
    const uint32_t stream = my_tiles * split_stages;  // positions p: tile p / split_stages, block st0 + p % split_stages
    y += (size_t)blockIdx.y * M * N;
    const int fr = lane % 32, hf = lane / 32;

    // The stage whose loads go out next (block lb of tile lt at (lm0, ln0)), advanced once per
    // stage; the tile origin is recomputed only when the tile changes. A stage past the split or
    // the stream loads through empty buffer resources (zeros); rows past M and columns past the
    // padded weight rows fall past their resource's end by their offsets alone.
    uint32_t lb = st0, lt = 0, lm0, ln0;
    origin(0, lm0, ln0);
    auto advance = [&]() {
        if (++lb == st0 + split_stages) {
            lb = st0;
            ++lt;
            origin(min(lt, my_tiles - 1), lm0, ln0);
        }
    };
    // x: load instruction i of wave w fills rows 32 w + 8 i .. + 7 (1 KB); lane l fetches row
    // r = 32 w + 8 i + l / 8's chunk (l % 8) ^ ((r >> 1) & 7), landing at position l % 8 of the row
    const uint32_t xrow = 32 * wave + lane / 8;
    auto xchunk = [&](uint32_t row) { return ((lane % 8) ^ ((row >> 1) & 7)) * 16; };
    auto dma_x = [&](uint32_t ring) {
        const bool live = lt < my_tiles && lb < st1;
        const i32x4 r = sgpr_rsrc(xs, live ? M * nb * 128 : 0u);
        const uint32_t base = ((lm0 + xrow) * nb + lb) * 128;
        const uint32_t lds = lds0 + S::A + ring * S::A_SZ + wave_u * 32 * 128;
#pragma unroll
        for (int i = 0; i < 4; i++)
            asm_load_lds16(r, lds + 8 * i * 128, base + 8 * i * nb * 128 + xchunk(xrow + 8 * i));
    };
    // weights: the block's quants of 256 columns as they lie in the tile plane (QB bytes per
    // column, a group of 32 columns contiguous), one 1 KB load per wave (Q4_0: waves 0-3); the
    // scale dwords (the pair of blocks b & ~1, b | 1 of each column, scale_slot's runs of eight),
    // one 256-byte load per wave 4-7
    auto dma_w = [&](uint32_t ring) {
        const bool live = lt < my_tiles && lb < st1;
        const uint32_t lds = lds0 + S::W + ring * S::W_SZ;
        if (KIND == FH_Q8_0 || wave_u < 4) {
            const i32x4 rq = sgpr_rsrc(qs, live ? (N + 31) / 32 * 32 * nb * QB : 0u);
            // Q8_0: wave w, columns 32 w + lane / 2 (half lane % 2); Q4_0: columns 64 w + lane
            const uint32_t g = KIND == FH_Q8_0 ? ln0 / 32 + wave_u : ln0 / 32 + 2 * wave_u + lane / 32;
            const uint32_t r = KIND == FH_Q8_0 ? lane / 2 : lane % 32;
            const uint32_t off = ((g * nb + lb) * 32 + r) * QB + (KIND == FH_Q8_0 ? (lane % 2) * 16 : 0);
            asm_load_lds16(rq, lds + wave_u * 1024, off);
        }
        if (wave_u >= 4) {
            const i32x4 rd = sgpr_rsrc(ds, live ? (N + 31) / 32 * 32 * ((nb + 7) / 8 * 8) * 2 : 0u);
            const uint32_t n = ln0 + 64 * (wave_u - 4) + lane;
            const uint32_t so = ((n >> 5) * ((nb + 7) / 8) * 32 + (n & 31)) * 16 + (lb / 8) * 512 + (lb % 8) / 2 * 4;
            asm_load_lds4(rd, lds + S::W_Q + (wave_u - 4) * 256, so);
        }
    };
    // the raw weights of ring slot `ring` (block parity odd) -> exact f16 integers and f32 scales
    const int cq = tid % 256, hq = tid / 256;
    auto unpack_w = [&](uint32_t ring, uint32_t odd, uint32_t slot) {
        const uint8_t *raw = arena + S::W + ring * S::W_SZ;
        _Float16 *col = (_Float16 *)(arena + S::B + slot * S::B_SZ) + cq * kSB + 16 * hq;
        u32x4 o[2];
        if constexpr (KIND == FH_Q8_0) {
            unpack_q8(*(const u32x4 *)(raw + cq * 32 + hq * 16), o);
        } else {
            const u32x2 v = *(const u32x2 *)(raw + cq * 16 + hq * 8);
            unpack_q4_half(v[0], v[1], o[0], o[1]);
        }
        *(u32x4 *)col = o[0];
        *(u32x4 *)(col + 8) = o[1];
        if (hq == 0) {
            const uint32_t dd = *(const uint32_t *)(raw + S::W_Q + cq * 4);
            ((float *)(arena + S::D + slot * S::D_SZ))[cq] = half_to_float(odd ? dd >> 16 : dd & 0xffffu);
        }
    };

    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // x fragments of a stage: row tile i, k16 step s, hi and lo (logical chunks hf + 2 s and
    // 4 + hf + 2 s of the lane's row)
    f16x8 ah[2][2], al[2][2];
    auto read_a = [&](uint32_t ring) {
        const uint8_t *sa = arena + S::A + ring * S::A_SZ;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t r = wm * 64 + i * 32 + fr;
            const uint8_t *row = sa + r * 128;
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                ah[i][s2] = *(const f16x8 *)(row + (((hf + 2 * s2) ^ ((r >> 1) & 7)) * 16));
                al[i][s2] = *(const f16x8 *)(row + (((4 + hf + 2 * s2) ^ ((r >> 1) & 7)) * 16));
            }
        }
    };
    // Per stage the eight tiles (column tile j = t / 2, row tile i = t % 2) run as a software
    // pipeline over two block-product registers: tile t's four MFMAs (a dependent chain) are each
    // followed by four of tile t - 1's sixteen scale FMAs, which fill the chain's latency; the
    // next column tile's weight fragments and scale are read one tile ahead. Scheduling barriers
    // keep that order (left alone, the compiler started all eight products at once and spilled,
    // or put the FMAs of tile t - 1 right behind the last MFMA they wait for).
    auto compute = [&](uint32_t slot, auto &&hook) {
        const _Float16 *bp = (const _Float16 *)(arena + S::B + slot * S::B_SZ) + (wn * 128 + fr) * kSB + 8 * hf;
        const float *dp = (const float *)(arena + S::D + slot * S::D_SZ) + wn * 128 + fr;
        f32x16 p[2];
        f16x8 bq[2][2];
        float dq[2];
        bq[0][0] = *(const f16x8 *)bp;
        bq[0][1] = *(const f16x8 *)(bp + 16);
        dq[0] = dp[0];
#pragma unroll
        for (int t = 0; t <= 8; t++) {
            const int j = t / 2, i = t % 2, tp = t - 1, jp = tp / 2, ip = tp % 2;
            f32x16 q = {};
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++) {
                if (t < 8) {
                    const f16x8 a = s4 < 2 ? ah[i][s4] : al[i][s4 - 2];
                    q = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bq[j % 2][s4 % 2], q, 0, 0, 0);
                }
                if (t > 0) {
#pragma unroll
                    for (int r = 4 * s4; r < 4 * s4 + 4; r++)
                        acc[ip][jp][r] = fmaf(dq[jp % 2], p[tp % 2][r], acc[ip][jp][r]);
                }
            }
            if (t < 8) p[t % 2] = q;
            if (t < 6 && i == 0) {  // column tile j + 1's fragments (bq[(j + 1) % 2] was last used by tile t - 1)
                bq[(j + 1) % 2][0] = *(const f16x8 *)(bp + (j + 1) * 32 * kSB);
                bq[(j + 1) % 2][1] = *(const f16x8 *)(bp + (j + 1) * 32 * kSB + 16);
            }
            if (t < 6 && i == 1) dq[(j + 1) % 2] = dp[(j + 1) * 32];  // (dq[(j + 1) % 2]'s last FMA was at t - 1)
            if (t > 0) asm volatile("" : "+v"(acc[ip][jp]));  // the FMAs stay here (not sunk below later products)
            hook(t);  // the stage's other work, issued among the MFMAs
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++) {
                if (t < 8) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA of tile t
                if (t > 0) __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // four FMAs of tile t - 1
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    uint32_t ct = 0;  // the tile being computed
    auto epilogue = [&]() {
        uint32_t m0, n0;
        origin(ct++, m0, n0);
        if constexpr (SCORE) {
            score_tile(acc, m0, n0, M, N, so, arena + S::TOTAL);
        } else {
        // D layout of a 32x32 tile: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * hf + r % 4;
                if (row >= M) continue;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t col = n0 + wn * 128 + j * 32 + fr;
                    if (col < N) y[(size_t)row * N + col] = acc[i][j][r];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    };

    // prologue: stages 0 and 1 requested, stage 0's weights unpacked
    uint32_t par = lb & 1;  // block parity of the stage whose weights are unpacked next
    dma_w(0);
    dma_x(0);
    advance();
    dma_w(1);
    dma_x(1);
    advance();
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // weights(0): x(0), weights(1), x(1) came after
    __syncthreads();
    unpack_w(0, par, 0);
    par = st0 + 1 < st0 + split_stages ? (st0 + 1) & 1 : st0 & 1;
    uint32_t ra = 0, rw = 1;  // the x ring slot of stage p; the weights ring slot of stage p + 1
    for (uint32_t p = 0; p < stream; p++) {
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // x(p) and weights(p + 1) are in
        __syncthreads();
        read_a(ra);
        // The stage's MFMAs start as soon as its x fragments arrive; the rest of the stage's work
        // runs among them (issued after tiles 1 and 3): weights(p + 1) unpacked into slot
        // (p + 1) % 2 (last read in stage p - 1), then weights(p + 2) and x(p + 2) requested into
        // the raw slot unpacked in stage p - 1 and the x slot last read in stage p - 1. (Before, all
        // of it ran between the barrier and the first MFMA, while the MFMAs of both wavefronts of
        // a SIMD waited.)
        compute(p & 1, [&](int t) {
            if (t == 1) {
                unpack_w(rw, par, (p + 1) & 1);
                par = (st0 + (p + 2) % split_stages) & 1;  // the block parity of stage p + 2
            } else if (t == 3) {
                dma_w(rw ^ 1);
                dma_x(ra == 0 ? 2 : ra - 1);
                advance();
            }
        });
        if ((p + 1) % split_stages == 0) epilogue();  // the tile's last stage
        ra = ra == 2 ? 0 : ra + 1;
        rw ^= 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (the last loads, past the stream, read zeros)
}

// ---- the scoring GEMM (FH_PATH_TILED_FAST) on the streaming 256 x 256 skeleton ----
// gemm_kernel's numerics (x = hi + lo: hi in f16 times the exact f16 integer quants on
// v_mfma_f32_32x32x16_f16 with acc += d P per block; lo as e4m3 of lo 2^s times the weights' e4m3
// correction operand d q 2^t on v_mfma_scale_f32_32x32x64_f8f6f4, which applies 2^-s 2^-t and
// accumulates straight into acc, once per two blocks) on gemm_stream_precise_kernel's structure:
// 256 x 256 tiles streamed by one CTA per CU, every operand loaded straight into LDS by inline
// assembly with explicit waits, one barrier per stage of one block. Per stage: x hi (64 bytes per
// row) into a ring of three, two stages ahead; the weights' raw quants and scale dwords into a
// ring of two and unpacked one stage ahead, as in the precise kernel. Per pair of stages (the
// correction's 64 k): x lo and the correction operand (64 bytes per row and per column) and the
// power-of-two scales (x lo: the tile's rows' two block scales of the pair; the operand: per
// column), requested at the pair's first stage and used at its second. A wavefront owns 64 x 128 (2 x 4 tiles): per stage 16 f16 MFMAs and 128 scale FMAs, per
// pair 8 scaled fp8 MFMAs (1.5 f16-equivalent passes where the precise kernel makes 2).
//
// 64-byte rows (x hi, x lo, the correction operand) sit in LDS with the 16-byte chunk c of row r at
// position c ^ ((r >> 2) & 3), so the sixteen rows one cycle of a fragment read serves fall on
// sixteen different 16-byte bank groups; each 1 KB load instruction fills 16 whole rows.
template <int KIND>
struct FastLds {  // byte offsets inside the kernel's LDS arena
    static constexpr uint32_t QB = KIND == FH_Q8_0 ? 32 : 16;
    static constexpr uint32_t A = 0, A_SZ = 256 * 64;                          // x hi: three stages
    static constexpr uint32_t W = 3 * A_SZ, W_Q = 256 * QB, W_SZ = W_Q + 1024;  // raw weights: two
    static constexpr uint32_t B = W + 2 * W_SZ, B_SZ = 256 * kSB * 2;          // unpacked weights: two
    static constexpr uint32_t D = B + 2 * B_SZ, D_SZ = 1024;                    // f32 scales: two
    static constexpr uint32_t L8 = D + 2 * D_SZ, C8 = L8 + 256 * 64;            // x lo, correction (a pair)
    static constexpr uint32_t SC = C8 + 256 * 64;                               // row, column scales
    static constexpr uint32_t TOTAL = SC + 2048;
};

__device__ __forceinline__ uint32_t swz64(uint32_t r, uint32_t c) { return (r * 4 + (c ^ ((r >> 2) & 3))) * 16; }

// SCORE: the scoring head's epilogue (score_tile into so) instead of the stores.
template <int KIND, bool SCORE = false>
__global__ __launch_bounds__(512, 1) void gemm_stream_fast_kernel(const _Float16 *__restrict__ xh,
                                                                  const uint8_t *__restrict__ xl,
                                                                  const uint8_t *__restrict__ xsb,
                                                                  const uint8_t *__restrict__ qs,
                                                                  const uint16_t *__restrict__ ds,
                                                                  const uint8_t *__restrict__ b8,
                                                                  const int32_t *__restrict__ bsc,
                                                                  float *__restrict__ y, uint32_t M, uint32_t K,
                                                                  uint32_t N, uint32_t mt, uint32_t nt,
                                                                  uint32_t split_stages, ScoreOut so) {
    // split_stages is even, so every split and every tile starts on an even block (pairs never
    // straddle them)
    using S = FastLds<KIND>;
    constexpr uint32_t QB = S::QB;
    __shared__ __attribute__((aligned(1024))) uint8_t arena[S::TOTAL + (SCORE ? 3072 : 0)];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t *)arena;

    constexpr uint32_t GM = 8;
    const uint32_t tiles = mt * nt, per_xcd = (tiles + 7) / 8, ctas = gridDim.x / 8;
    const uint32_t run0 = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8, run1 = min(tiles, (blockIdx.x % 8 + 1) * per_xcd);
    if (run0 >= run1) return;  // whole CTA: no barrier is left waiting
    const uint32_t my_tiles = (run1 - run0 + ctas - 1) / ctas;
    auto origin = [&](uint32_t k, uint32_t &m0, uint32_t &n0) {  // row and column of my k-th tile
        const uint32_t t = run0 + k * ctas;
        const uint32_t grp = t / (GM * nt), in = t % (GM * nt), gm = min(GM, mt - grp * GM);
        m0 = (grp * GM + in % gm) * 256;
        n0 = (in / gm) * 256;
    };

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, wm = wave % 4, wn = wave / 4;
    const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t nb = K / 32, K64 = (K + 63) / 64 * 64, MS = xsb_rows(M);
    const uint32_t st0 = blockIdx.y * split_stages, st1 = min(nb, st0 + split_stages);
    const uint32_t stream = my_tiles * split_stages;
    y += (size_t)blockIdx.y * M * N;
    const int fr = lane % 32, hf = lane / 32;

    // the stage whose loads go out next (block lb of tile lt at (lm0, ln0))
    uint32_t lb = st0, lt = 0, lm0, ln0;
    origin(0, lm0, ln0);
    auto advance = [&]() {
        if (++lb == st0 + split_stages) {
            lb = st0;
            ++lt;
            origin(min(lt, my_tiles - 1), lm0, ln0);
        }
    };
    // 64-byte rows: load instruction i of wave w fills rows 16 (2 w + i) .. + 15; lane l fetches
    // row + l / 4's chunk (l % 4) ^ ((row >> 2) & 3), landing at position l % 4
    const uint32_t r64 = 32 * wave + lane / 4;  // (+ 16 i)
    auto chunk64 = [&](uint32_t row) { return ((lane % 4) ^ ((row >> 2) & 3)) * 16; };
    auto dma_x = [&](uint32_t ring) {
        const bool live = lt < my_tiles && lb < st1;
        const i32x4 r = sgpr_rsrc(xh, live ? M * nb * 64 : 0u);
        const uint32_t lds = lds0 + S::A + ring * S::A_SZ + wave_u * 2048;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t row = r64 + 16 * i;
            asm_load_lds16(r, lds + 1024 * i, ((lm0 + row) * nb + lb) * 64 + chunk64(row));
        }
    };
    auto dma_w = [&](uint32_t ring) {  // as gemm_stream_precise_kernel's
        const bool live = lt < my_tiles && lb < st1;
        const uint32_t lds = lds0 + S::W + ring * S::W_SZ;
        if (KIND == FH_Q8_0 || wave_u < 4) {
            const i32x4 rq = sgpr_rsrc(qs, live ? (N + 31) / 32 * 32 * nb * QB : 0u);
            const uint32_t g = KIND == FH_Q8_0 ? ln0 / 32 + wave_u : ln0 / 32 + 2 * wave_u + lane / 32;
            const uint32_t r = KIND == FH_Q8_0 ? lane / 2 : lane % 32;
            const uint32_t off = ((g * nb + lb) * 32 + r) * QB + (KIND == FH_Q8_0 ? (lane % 2) * 16 : 0);
            asm_load_lds16(rq, lds + wave_u * 1024, off);
        }
        if (wave_u >= 4) {
            const i32x4 rd = sgpr_rsrc(ds, live ? (N + 31) / 32 * 32 * ((nb + 7) / 8 * 8) * 2 : 0u);
            const uint32_t n = ln0 + 64 * (wave_u - 4) + lane;
            const uint32_t so = ((n >> 5) * ((nb + 7) / 8) * 32 + (n & 31)) * 16 + (lb / 8) * 512 + (lb % 8) / 2 * 4;
            asm_load_lds4(rd, lds + S::W_Q + (wave_u - 4) * 256, so);
        }
    };
    // the tile being computed (its origin), for the pair's correction operands and the epilogue
    uint32_t ct = 0, cm0, cn0;
    origin(0, cm0, cn0);
    // the pair starting at (even) block b of the computed tile: x lo and the correction operand
    // (rows of K64, 64 bytes per pair in the order of lo_byte), the pair's scale bytes of the tile's
    // rows (two per row) and the columns' scales (E8M0 bytes, four copies); rows past M and columns
    // past N read zeros, whose products are zero
    auto dma_corr = [&](uint32_t b) {
        const bool live = b < st1;
        const i32x4 rl = sgpr_rsrc(xl, live ? M * K64 : 0u);
        const i32x4 rc = sgpr_rsrc(b8, live ? N * K64 : 0u);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t row = r64 + 16 * i;
            asm_load_lds16(rl, lds0 + S::L8 + wave_u * 2048 + 1024 * i, (cm0 + row) * K64 + b * 32 + chunk64(row));
            asm_load_lds16(rc, lds0 + S::C8 + wave_u * 2048 + 1024 * i, (cn0 + row) * K64 + b * 32 + chunk64(row));
        }
        if (wave_u < 2) {  // the pair's scale bytes of the tile's 256 rows, two rows a lane
            const i32x4 rs = sgpr_rsrc(xsb, live ? K64 / 64 * MS * 2 : 0u);
            asm_load_lds4(rs, lds0 + S::SC + wave_u * 256, ((b / 2) * MS + cm0 + 128 * wave_u + 2 * lane) * 2);
        } else if (wave_u >= 4) {
            const i32x4 rs = sgpr_rsrc(bsc, N * 4);
            asm_load_lds4(rs, lds0 + S::SC + 1024 + (wave_u - 4) * 256, (cn0 + 64 * (wave_u - 4) + lane) * 4);
        }
    };
    const int cq = tid % 256, hq = tid / 256;
    auto unpack_w = [&](uint32_t ring, uint32_t odd, uint32_t slot) {
        const uint8_t *raw = arena + S::W + ring * S::W_SZ;
        _Float16 *col = (_Float16 *)(arena + S::B + slot * S::B_SZ) + cq * kSB + 16 * hq;
        u32x4 o[2];
        if constexpr (KIND == FH_Q8_0) {
            unpack_q8(*(const u32x4 *)(raw + cq * 32 + hq * 16), o);
        } else {
            const u32x2 v = *(const u32x2 *)(raw + cq * 16 + hq * 8);
            unpack_q4_half(v[0], v[1], o[0], o[1]);
        }
        *(u32x4 *)col = o[0];
        *(u32x4 *)(col + 8) = o[1];
        if (hq == 0) {
            const uint32_t dd = *(const uint32_t *)(raw + S::W_Q + cq * 4);
            ((float *)(arena + S::D + slot * S::D_SZ))[cq] = half_to_float(odd ? dd >> 16 : dd & 0xffffu);
        }
    };

    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    f16x8 ah[2][2];
    auto read_a = [&](uint32_t ring) {
        const uint8_t *sa = arena + S::A + ring * S::A_SZ;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t r = wm * 64 + i * 32 + fr;
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) ah[i][s2] = *(const f16x8 *)(sa + swz64(r, hf + 2 * s2));
        }
    };
    // the hi part, pipelined as in gemm_stream_precise_kernel: tile t's two MFMAs, each followed by
    // eight of tile t - 1's scale FMAs
    auto compute = [&](uint32_t slot, auto &&hook) {
        const _Float16 *bp = (const _Float16 *)(arena + S::B + slot * S::B_SZ) + (wn * 128 + fr) * kSB + 8 * hf;
        const float *dp = (const float *)(arena + S::D + slot * S::D_SZ) + wn * 128 + fr;
        f32x16 p[2];
        f16x8 bq[2][2];
        float dq[2];
        bq[0][0] = *(const f16x8 *)bp;
        bq[0][1] = *(const f16x8 *)(bp + 16);
        dq[0] = dp[0];
#pragma unroll
        for (int t = 0; t <= 8; t++) {
            const int j = t / 2, i = t % 2, tp = t - 1, jp = tp / 2, ip = tp % 2;
            f32x16 q = {};
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                if (t < 8) q = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][s2], bq[j % 2][s2], q, 0, 0, 0);
                if (t > 0) {
#pragma unroll
                    for (int r = 8 * s2; r < 8 * s2 + 8; r++)
                        acc[ip][jp][r] = fmaf(dq[jp % 2], p[tp % 2][r], acc[ip][jp][r]);
                }
            }
            if (t < 8) p[t % 2] = q;
            if (t < 6 && i == 0) {
                bq[(j + 1) % 2][0] = *(const f16x8 *)(bp + (j + 1) * 32 * kSB);
                bq[(j + 1) % 2][1] = *(const f16x8 *)(bp + (j + 1) * 32 * kSB + 16);
            }
            if (t < 6 && i == 1) dq[(j + 1) % 2] = dp[(j + 1) * 32];
            if (t > 0) asm volatile("" : "+v"(acc[ip][jp]));
            hook(t);
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                if (t < 8) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA of tile t
                if (t > 0) __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // eight FMAs of tile t - 1
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // the pair's correction: 32 bytes of x lo per row tile and of the operand per column tile
    // (the lane's half of the 64 k), the scaled fp8 MFMA applying 2^-s 2^-t
    typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
    auto correct = [&]() {
        const int32_t *scl = (const int32_t *)(arena + S::SC);
        int32_t asc[2], bscv[4];
        i32x8 a8[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t r = wm * 64 + i * 32 + fr;
            const u32x4 lo0 = *(const u32x4 *)(arena + S::L8 + swz64(r, 2 * hf));
            const u32x4 lo1 = *(const u32x4 *)(arena + S::L8 + swz64(r, 2 * hf + 1));
            a8[i] = i32x8{(int)lo0[0], (int)lo0[1], (int)lo0[2], (int)lo0[3], (int)lo1[0], (int)lo1[1], (int)lo1[2],
                          (int)lo1[3]};
            // the scale of the lane's block (2 p + hf) of its row; rows past M (lo zero) take 2^0
            asc[i] = cm0 + r < M ? (int32_t)(arena + S::SC)[2 * r + hf] : 127;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) bscv[j] = scl[256 + wn * 128 + j * 32 + fr];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t c = wn * 128 + j * 32 + fr;
            const u32x4 w0 = *(const u32x4 *)(arena + S::C8 + swz64(c, 2 * hf));
            const u32x4 w1 = *(const u32x4 *)(arena + S::C8 + swz64(c, 2 * hf + 1));
            const i32x8 b8f{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3], (int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
#pragma unroll
            for (int i = 0; i < 2; i++)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8[i], b8f, acc[i][j], 0, 0, 0, asc[i], 0,
                                                                            bscv[j]);
        }
    };
    auto epilogue = [&]() {
        if constexpr (SCORE) {
            score_tile(acc, cm0, cn0, M, N, so, arena + S::TOTAL);
        } else {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = cm0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * hf + r % 4;
                if (row >= M) continue;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t col = cn0 + wn * 128 + j * 32 + fr;
                    if (col < N) y[(size_t)row * N + col] = acc[i][j][r];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
        ++ct;
        origin(min(ct, my_tiles - 1), cm0, cn0);
    };

    // prologue: stages 0 and 1 requested, stage 0's weights unpacked
    uint32_t par = lb & 1;
    dma_w(0);
    dma_x(0);
    advance();
    dma_w(1);
    dma_x(1);
    advance();
    asm volatile("s_waitcnt vmcnt(5)" ::: "memory");  // weights(0): x(0), weights(1), x(1) came after
    __syncthreads();
    unpack_w(0, par, 0);
    par = (st0 + 1 % split_stages) & 1;
    uint32_t ra = 0, rw = 1;
    // Per wave the loads of stage p go out as [the pair's correction, at an even p] weights(p + 2),
    // x(p + 2) (two instructions): at the top of stage p, waiting until at most 2 are outstanding
    // leaves weights(p + 1), x(p) and the correction issued in stage p - 1 in LDS.
    for (uint32_t p = 0; p < stream; p++) {
        asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
        __syncthreads();
        read_a(ra);
        const uint32_t cb = st0 + p % split_stages;  // this stage's block
        compute(p & 1, [&](int t) {
            if (t == 0 && !(p & 1)) {
                dma_corr(cb);  // (the buffer's previous pair was used in stage p - 1)
            } else if (t == 1) {
                unpack_w(rw, par, (p + 1) & 1);
                par = (st0 + (p + 2) % split_stages) & 1;
            } else if (t == 5) {
                dma_w(rw ^ 1);
                dma_x(ra == 0 ? 2 : ra - 1);
                advance();
            }
        });
        if (p & 1) correct();  // the pair (p - 1, p)
        if ((p + 1) % split_stages == 0) epilogue();
        ra = ra == 2 ? 0 : ra + 1;
        rw ^= 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The streaming kernel's plan: taken when the product has at least 128 tiles of 256 x 256; the K
// split (at most 4, at least 16 blocks per split) that best fills whole rounds of one CTA per CU.
bool stream_plan(size_t rows, size_t k, size_t n, uint32_t *splits) {
    const uint64_t tiles = (uint64_t)((rows + 255) / 256) * ((n + 255) / 256);
    if (tiles < 128) return false;
    const uint32_t stages = (uint32_t)(k / 32), cus = 256;
    uint32_t best = 1;
    double best_eff = 0.0;
    for (uint32_t sp = 1; sp <= 4 && (sp == 1 || stages / sp >= 16); sp++) {
        const uint64_t ctas = tiles * sp, rounds = (ctas + cus - 1) / cus;
        const double eff = (double)ctas / (double)(rounds * cus) - 0.04 * (sp - 1);  // the reduce pass
        if (eff > best_eff + 1e-9) {
            best_eff = eff;
            best = sp;
        }
    }
    *splits = best;
    return true;
}

bool stream_supported(size_t rows, size_t k, size_t n) {
    // every byte offset a CTA forms (columns up to the last tile's end) fits the 32-bit offsets
    const size_t lim = (size_t)1 << 31;
    return (rows + 255) * k * 4 < lim && (n + 255) * (k / 32) * 32 < lim;
}

template <int KIND>
hipError_t run_gemm_stream_precise(hipStream_t s, const _Float16 *xs, const uint8_t *qs, const uint16_t *ds,
                                   float *y, float *partial, uint32_t M, uint32_t K, uint32_t N, uint32_t sp,
                                   SplitOut *defer) {
    const uint32_t mt = (M + 255) / 256, nt = (N + 255) / 256;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7ffffff0ull) return hipErrorInvalidValue;
    const uint32_t per_xcd = (uint32_t)((tiles + 7) / 8);
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8)
        cus = 256;
    const uint32_t ctas = min(per_xcd, (uint32_t)cus / 8);
    const uint32_t stages = K / 32;
    const uint32_t per = (stages + sp - 1) / sp;
    float *out = sp > 1 ? partial : y;
    gemm_stream_precise_kernel<KIND><<<dim3(8 * ctas, sp), 512, 0, s>>>(xs, qs, ds, out, M, K, N, mt, nt, per,
                                                                        ScoreOut{});
    if (defer) *defer = sp > 1 ? SplitOut{partial, sp} : SplitOut{y, 1u};
    if (sp > 1 && !defer) {
        const size_t n = (size_t)M * N;
        const unsigned rg = (unsigned)min((n + 1023) / 1024, (size_t)16384);
        gemm_reduce_kernel<<<rg, 256, 0, s>>>(partial, y, n, sp);
    }
    return hipGetLastError();
}

template <int KIND>
hipError_t gemm_precise_dispatch(hipStream_t s, const _Float16 *xs, const uint8_t *qs, const uint16_t *ds, float *y,
                                 float *partial, uint32_t M, uint32_t K, uint32_t N, SplitOut *defer) {
    uint32_t sp = 1;
    if (stream_plan(M, K, N, &sp) && stream_supported(M, K, N) && (sp == 1 || partial))
        return run_gemm_stream_precise<KIND>(s, xs, qs, ds, y, partial, M, K, N, sp, defer);
    if (M <= 32) return run_gemm_precise<KIND, 32, 256, 1>(s, xs, qs, ds, y, partial, M, K, N, defer);
    if (M <= 64) return run_gemm_precise<KIND, 64, 128, 2>(s, xs, qs, ds, y, partial, M, K, N, defer);
    return run_gemm_precise<KIND, 128, 128, 2>(s, xs, qs, ds, y, partial, M, K, N, defer);
}

bool stream_fast_supported(size_t rows, size_t k, size_t n) {
    // every byte offset a CTA forms (rows and columns up to the last tile's end) fits in 32 bits
    const size_t k64 = (k + 63) / 64 * 64, lim = (size_t)1 << 31;
    return (rows + 255) * k * 2 < lim && (rows + 255) * k64 < lim && (n + 255) * k64 < lim &&
           (n + 255) * (k / 32) * 32 < lim;
}

template <int KIND>
hipError_t run_gemm_stream_fast(hipStream_t s, const GemmArgs &g, uint32_t sp) {
    const uint32_t mt = (g.M + 255) / 256, nt = (g.N + 255) / 256;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7ffffff0ull) return hipErrorInvalidValue;
    const uint32_t per_xcd = (uint32_t)((tiles + 7) / 8);
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8)
        cus = 256;
    const uint32_t ctas = min(per_xcd, (uint32_t)cus / 8);
    const uint32_t stages = g.K / 32;
    const uint32_t per = ((stages + sp - 1) / sp + 1) & ~1u;  // even: pairs never straddle a split
    float *out = sp > 1 ? g.partial : g.y;
    gemm_stream_fast_kernel<KIND><<<dim3(8 * ctas, sp), 512, 0, s>>>(g.xh, g.xl, g.xsb, g.qs, g.ds, g.b8, g.bsc, out,
                                                                      g.M, g.K, g.N, mt, nt, per, ScoreOut{});
    if (g.defer) *g.defer = sp > 1 ? SplitOut{g.partial, sp} : SplitOut{g.y, 1u};
    if (sp > 1 && !g.defer) {
        const size_t n = (size_t)g.M * g.N;
        const unsigned rg = (unsigned)min((n + 1023) / 1024, (size_t)16384);
        gemm_reduce_kernel<<<rg, 256, 0, s>>>(g.partial, g.y, n, sp);
    }
    return hipGetLastError();
}

// The scoring GEMM takes the streaming kernel for products of at least 640 tiles of 256 x 256
// (two and a half rounds of one CTA per CU), gemm_kernel's 128-row tiles below that. Measured per
// product (Q4_0, x split included): the streaming kernel is faster on the Qwen2-0.5B head
// (151,936 columns; M = 2048: 1283 against 1426 us, M = 512: 349 against 440) and on the
// TinyLlama gate/up at M = 4096 (704 tiles: 429 against 473 us), slower where a product is one or
// two partly filled rounds (Qwen2 gate/up at M = 2048, 304 tiles: 121 against 98 us; TinyLlama
// products at M = 1024-4096 with 128-352 tiles: 1-23% slower).
bool stream_fast_plan(size_t rows, size_t k, size_t n, uint32_t *splits) {
    const uint64_t tiles = (uint64_t)((rows + 255) / 256) * ((n + 255) / 256);
    return tiles >= 640 && stream_plan(rows, k, n, splits);
}

template <int KIND>
hipError_t gemm_fast_dispatch(hipStream_t s, const GemmArgs &g) {
    uint32_t sp = 1;
    if (stream_fast_plan(g.M, g.K, g.N, &sp) && stream_fast_supported(g.M, g.K, g.N) && (sp == 1 || g.partial))
        return run_gemm_stream_fast<KIND>(s, g, sp);
    return gemm_dispatch<KIND>(s, g);
}

// The scoring head with the score epilogue: the streaming kernels with one K split (the head's K
// is the model width, a few dozen stages) over every tile.

template <int KIND>
hipError_t run_gemm_score(hipStream_t s, fh_path path, const void *xa, const uint8_t *xl, const uint8_t *xsb,
                          const uint8_t *qs, const uint16_t *ds, const uint8_t *b8, const int32_t *bsc, uint32_t M,
                          uint32_t K, uint32_t N, const ScoreOut &so) {
    const uint32_t mt = (M + 255) / 256, nt = (N + 255) / 256;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7ffffff0ull || nt != so.ntn) return hipErrorInvalidValue;
    const uint32_t per_xcd = (uint32_t)((tiles + 7) / 8);
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8)
        cus = 256;
    const uint32_t ctas = min(per_xcd, (uint32_t)cus / 8), stages = K / 32;
    if (path == FH_PATH_TILED_FAST)
        gemm_stream_fast_kernel<KIND, true><<<dim3(8 * ctas, 1), 512, 0, s>>>(
            (const _Float16 *)xa, xl, xsb, qs, ds, b8, bsc, nullptr, M, K, N, mt, nt, (stages + 1) & ~1u, so);
    else
        gemm_stream_precise_kernel<KIND, true><<<dim3(8 * ctas, 1), 512, 0, s>>>((const _Float16 *)xa, qs, ds, nullptr,
                                                                                 M, K, N, mt, nt, stages, so);
    return hipGetLastError();
}

// ---- the MFMA GEMM on the other weight formats' GGUF rows (F16, FP8 E4M3 / E5M2, MXFP4) ----
// Every element of these formats is an f16-exact value times a per-32-block f32 scale: F16 its
// own value (scale 1), E5M2 code c the f16 with bits c << 8 (fp8.rs:34-63), E4M3 code c the f16
// with bits (c & 0x7f) << 7 | (c & 0x80) << 8 times 2^8 (normal and subnormal alike), MXFP4
// nibble v the integer 0, 1, 2, 3, 4, 6, 8, 12 or its
// negative (mxfp4.rs:13-14) times the E8M0 half scale. A block holding a non-finite value (an
// F16 or E5M2 infinity or NaN, an E4M3 NaN) gets a NaN scale, so its outputs are NaN: the split
// x would otherwise meet an infinity with lo = 0 or of the other sign. The precise GEMM's
// arithmetic applies unchanged: x = hi + lo in f16 (natural k order here), per 32 x 32 tile and block
// P = hi * v + lo * v on four v_mfma_f32_32x32x16_f16, acc += scale * P. Per stage (one block)
// thread t < BN decodes column n0 + t's block from its row (unaligned for FP8 and MXFP4: the
// dwords around it, realigned with v_alignbyte; allocations carry 256 zero bytes past their end)
// into 32 f16 in LDS and the block's scale; the next stage's bytes are requested before the
// current stage's MFMAs.
__device__ __forceinline__ float e8m0_half_scale(uint32_t e) {  // mxfp4.rs:26-33
    return e < 2 ? __uint_as_float(0x00200000u << e) : __uint_as_float((e - 1) << 23);
}
__device__ __forceinline__ uint32_t mx_biased(uint32_t n) {  // 4 nibbles (one per byte) -> value + 16 per byte
    const uint32_t m = n & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x1c181614u, 0x13121110u, m);
    const uint32_t neg = __builtin_amdgcn_perm(0x04080a0cu, 0x0d0e0f10u, m);
    const uint32_t sgn = ((n >> 3) & 0x01010101u) * 0xffu;
    return (neg & sgn) | (pos & ~sgn);
}

template <uint32_t T>
struct ExtBlock;  // raw bytes of one block of a column, held in registers between stages
template <>
struct ExtBlock<FH_F16> {
    static constexpr uint32_t B = 64;
    u32x4 q[4];
    __device__ void load(const uint8_t *blk) {
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = *(const u32x4 *)(blk + 16 * i);
    }
    __device__ float unpack(u32x4 (&o)[4]) const {
        uint32_t bad = 0;  // an infinity or NaN half (exponent bits all ones)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[i] = q[i];
#pragma unroll
            for (int c = 0; c < 4; c++) bad |= ((q[i][c] & 0x7c007c00u) + 0x04000400u) & 0x80008000u;
        }
        return bad ? __uint_as_float(0x7fc00000u) : 1.0f;
    }
};
template <bool E5M2>
struct Fp8Block {
    static constexpr uint32_t B = 34;
    uint32_t d[9], sh;  // the dwords around the block, its byte offset in the first
    __device__ void load(const uint8_t *blk) {
        sh = (uint32_t)((uintptr_t)blk & 3);
        const uint8_t *q = blk - sh;
#pragma unroll
        for (int i = 0; i < 9; i++) d[i] = *(const uint32_t *)(q + 4 * i);
    }
    __device__ float unpack(u32x4 (&o)[4]) const {
        uint32_t a[9];  // block bytes 0 .. 35
#pragma unroll
        for (int i = 0; i < 8; i++) a[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
        a[8] = d[8] >> (8 * sh);
        uint32_t nan = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {  // codes 4i .. 4i + 3 = bytes 2 + 4i .. 5 + 4i
            const uint32_t v = __builtin_amdgcn_alignbyte(a[i + 1], a[i], 2);
            uint32_t p0, p1;
            if constexpr (E5M2) {
                p0 = __builtin_amdgcn_perm(v, 0u, 0x050c040cu);
                p1 = __builtin_amdgcn_perm(v, 0u, 0x070c060cu);
                nan |= ((v & 0x7c7c7c7cu) + 0x04040404u) & 0x80808080u;  // infinity and NaN codes
            } else {
                const uint32_t t0 = __builtin_amdgcn_perm(v, 0u, 0x0c050c04u), t1 = __builtin_amdgcn_perm(v, 0u, 0x0c070c06u);
                p0 = ((t0 & 0x007f007fu) << 7) | ((t0 & 0x00800080u) << 8);
                p1 = ((t1 & 0x007f007fu) << 7) | ((t1 & 0x00800080u) << 8);
                nan |= ((v & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;
            }
            o[i / 2][2 * (i % 2)] = p0;
            o[i / 2][2 * (i % 2) + 1] = p1;
        }
        const float sc = half_to_float(a[0] & 0xffffu) * (E5M2 ? 1.0f : 256.0f);
        return nan ? __uint_as_float(0x7fc00000u) : sc;
    }
};
template <>
struct ExtBlock<FH_FP8_E4M3> : Fp8Block<false> {};
template <>
struct ExtBlock<FH_FP8_E5M2> : Fp8Block<true> {};
template <>
struct ExtBlock<FH_MXFP4> {
    static constexpr uint32_t B = 17;
    uint32_t d[6], sh;
    __device__ void load(const uint8_t *blk) {
        sh = (uint32_t)((uintptr_t)blk & 3);
        const uint8_t *q = blk - sh;
#pragma unroll
        for (int i = 0; i < 6; i++) d[i] = *(const uint32_t *)(q + 4 * i);
    }
    __device__ float unpack(u32x4 (&o)[4]) const {
        uint32_t a[5];  // block bytes 0 .. 19
#pragma unroll
        for (int i = 0; i < 5; i++) a[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
#pragma unroll
        for (int i = 0; i < 4; i++) {  // nibble bytes 4i .. 4i + 3 (block bytes 1 + 4i ..)
            const uint32_t v = __builtin_amdgcn_alignbyte(a[i + 1], a[i], 1);
            const uint32_t lo = mx_biased(v & 0x0f0f0f0fu), hi = mx_biased((v >> 4) & 0x0f0f0f0fu);
            // elements 4i .. 4i + 3 (low nibbles) and 16 + 4i .. (high): 1024 + value + 16, - 1040
            const uint32_t l0 = f16x2_add(__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u), (_Float16)-1040.0f);
            const uint32_t l1 = f16x2_add(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u), (_Float16)-1040.0f);
            const uint32_t h0 = f16x2_add(__builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u), (_Float16)-1040.0f);
            const uint32_t h1 = f16x2_add(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u), (_Float16)-1040.0f);
            o[i / 2][2 * (i % 2)] = l0;
            o[i / 2][2 * (i % 2) + 1] = l1;
            o[2 + i / 2][2 * (i % 2)] = h0;
            o[2 + i / 2][2 * (i % 2) + 1] = h1;
        }
        return e8m0_half_scale(a[0] & 0xffu);
    }
};

// Q2_K (blocks.rs:201-250): stage kb = elements 32 kb .. 32 kb + 31 of the row, i.e. super-block
// kb / 8, half h = (kb % 8) / 4, 2-bit plane j = kb % 4: element 128 h + 32 j + l is bits 2j of
// quant byte 32 h + l, in sub-block 8 h + 2 j + l / 16 (value d (sc & 15) q - dmin (sc >> 4)). Two
// sub-blocks per stage, each one MFMA k-step: the stage carries both sub-blocks' d (sc & 15) and
// dmin (sc >> 4), and the kernel subtracts dmin (sc >> 4) times the row's sum of x over the
// sub-block.
template <>
struct ExtBlock<FH_Q2_K> {
    static constexpr uint32_t B = 84;
    uint32_t q[8], sc, dd;
    __device__ void load(const uint8_t *row, uint32_t kb) {
        const uint8_t *blk = row + 84 * (kb / 8);
        const uint32_t h = (kb % 8) / 4, j = kb % 4;
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = *(const uint32_t *)(blk + 16 + 32 * h + 4 * i);
        sc = *(const uint16_t *)(blk + 8 * h + 2 * j);
        dd = *(const uint32_t *)(blk + 80);
    }
    // 32 exact f16 quants and (dl0, dl1, ml0, ml1)
    __device__ void unpack(uint32_t kb, u32x4 (&o)[4], float (&s4)[4]) const {
        const uint32_t j = kb % 4;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t v = (q[i] >> (2 * j)) & 0x03030303u;  // elements 4i .. 4i + 3
            o[i / 2][2 * (i % 2)] = f16x2_add(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u), (_Float16)-1024.0f);
            o[i / 2][2 * (i % 2) + 1] = f16x2_add(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u), (_Float16)-1024.0f);
        }
        const float d = half_to_float(dd & 0xffffu), dmin = half_to_float(dd >> 16);
        s4[0] = d * (float)(sc & 15u);
        s4[1] = d * (float)((sc >> 8) & 15u);
        s4[2] = dmin * (float)((sc >> 4) & 15u);
        s4[3] = dmin * (float)((sc >> 12) & 15u);
    }
};

template <uint32_t T, int BM, int BN, int WAVES_M>
__global__ __launch_bounds__(256, 2) void gemm_ext_kernel(const _Float16 *__restrict__ xs, const uint8_t *__restrict__ w,
                                                          float *__restrict__ y, uint32_t M, uint32_t K, uint32_t N,
                                                          uint32_t mt, uint32_t nt, uint32_t split_stages) {
    constexpr int WAVES_N = 4 / WAVES_M, TM = BM / WAVES_M / 32, TN = BN / WAVES_N / 32;
    constexpr int A_LD = BM * 8 / 256;  // 16-byte x chunks per thread per block
    static_assert(TM >= 1 && TN >= 1 && BM * 8 % 256 == 0 && BN <= 256, "tile shape");
    using EB = ExtBlock<T>;
    constexpr bool Q2K = T == FH_Q2_K;
    constexpr int NS = Q2K ? 4 : 1;  // scales per column and stage
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][BM * kARow2];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][BN * kBRow2];
    __shared__ float sD[2][NS * BN];
    __shared__ __attribute__((aligned(16))) float sS[2][Q2K ? 2 * BM : 1];  // Q2_K: x sums per row and sub-block

    const uint32_t tiles = mt * nt, c = blockIdx.x, per_xcd = (tiles + 7) / 8;
    const uint32_t t = (c % 8) * per_xcd + c / 8;
    if (t >= tiles) return;  // whole CTA: no barrier is left waiting
    const uint32_t m0 = (t / nt) * BM, n0 = (t % nt) * BN;
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    const uint32_t nb = K / 32;
    const uint32_t st0 = blockIdx.y * split_stages, st1 = min(nb, st0 + split_stages);
    y += (size_t)blockIdx.y * M * N;
    const size_t row_bytes = (size_t)(Q2K ? nb / 8 : nb) * EB::B;
    const uint32_t wcol = n0 + tid;  // the column this thread decodes (tid < BN)
    const uint8_t *wrow = w + (size_t)min(wcol, N - 1) * row_bytes;

    u32x4 ra[A_LD];
    EB rb;
    auto load_stage = [&](uint32_t kb) {
#pragma unroll
        for (int i = 0; i < A_LD; i++) {
            const int cc = tid + 256 * i, r = cc / 8, ch = cc % 8;
            const uint32_t m = m0 + r;
            ra[i] = m < M ? *(const u32x4 *)(xs + ((size_t)m * nb + kb) * 64 + ch * 8) : u32x4{0u, 0u, 0u, 0u};
        }
        if (tid < BN) {
            if constexpr (Q2K)
                rb.load(wrow, kb);
            else
                rb.load(wrow + (size_t)kb * EB::B);
        }
    };
    auto store_stage = [&](int buf, uint32_t kb) {
#pragma unroll
        for (int i = 0; i < A_LD; i++) {
            const int cc = tid + 256 * i, r = cc / 8, ch = cc % 8;
            *(u32x4 *)(&sA[buf][r * kARow2 + ch * 8]) = ra[i];
            if constexpr (Q2K) {
                // chunk ch holds hi (ch < 4) or lo halves 8 (ch % 4) .. + 7: sub-block (ch >> 1) & 1;
                // the eight lanes of a row meet by shuffles
                typedef _Float16 h8 __attribute__((ext_vector_type(8)));
                const h8 v = __builtin_bit_cast(h8, ra[i]);
                float t = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) t += (float)v[e];
                t += __shfl_xor(t, 1);
                t += __shfl_xor(t, 4);
                if ((ch & 5) == 0) sS[buf][((ch >> 1) & 1) * BM + r] = t;
            }
        }
        if (tid < BN) {
            u32x4 o[4];
            float sc[NS];
            if constexpr (Q2K)
                rb.unpack(kb, o, sc);
            else
                sc[0] = rb.unpack(o);
            if (wcol >= N) {
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
                for (int i = 0; i < NS; i++) sc[i] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) *(u32x4 *)(&sB[buf][tid * kBRow2 + 8 * i]) = o[i];
#pragma unroll
            for (int i = 0; i < NS; i++) sD[buf][i * BN + tid] = sc[i];
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    const int fr = lane % 32, fk = 8 * (lane / 32);

    if (st0 < st1) {
        load_stage(st0);
        store_stage(0, st0);
    }
    __syncthreads();
    for (uint32_t kb = st0; kb < st1; kb++) {
        const int buf = (kb - st0) & 1;
        const bool more = kb + 1 < st1;
        if (more) load_stage(kb + 1);  // in flight during the MFMAs below
        f16x8 bf[TN][2];
        float dcol[TN][NS];
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int col = (wn * TN + j) * 32 + fr;
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) bf[j][s2] = *(const f16x8 *)(&sB[buf][col * kBRow2 + 16 * s2 + fk]);
#pragma unroll
            for (int i = 0; i < NS; i++) dcol[j][i] = sD[buf][i * BN + col];
        }
        f16x8 ah[TM][2], al[TM][2];
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int r = (wm * TM + i) * 32 + fr;
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                ah[i][s2] = *(const f16x8 *)(&sA[buf][r * kARow2 + 16 * s2 + fk]);
                al[i][s2] = *(const f16x8 *)(&sA[buf][r * kARow2 + 32 + 16 * s2 + fk]);
            }
        }
        if constexpr (Q2K) {
            // per sub-block s2: P = hi * q + lo * q over its 16 k, acc += dl P - ml sum(x)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int s2 = 0; s2 < 2; s2++) {
                    f32x4 sx[4];  // this lane's 16 rows: 8 g + 4 (lane / 32) + 0..3
#pragma unroll
                    for (int g = 0; g < 4; g++)
                        sx[g] = *(const f32x4 *)(&sS[buf][s2 * BM + (wm * TM + i) * 32 + 8 * g + 4 * (lane / 32)]);
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        f32x16 p = {};
                        p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][s2], bf[j][s2], p, 0, 0, 0);
                        p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][s2], bf[j][s2], p, 0, 0, 0);
#pragma unroll
                        for (int q = 0; q < 16; q++) {
                            acc[i][j][q] = fmaf(dcol[j][s2], p[q], acc[i][j][q]);
                            acc[i][j][q] = fmaf(-dcol[j][2 + s2], sx[q / 4][q % 4], acc[i][j][q]);
                        }
                    }
                }
        } else {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    f32x16 p = {};
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], bf[j][0], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], bf[j][1], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], bf[j][0], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], bf[j][1], p, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 16; q++) acc[i][j][q] = fmaf(dcol[j][0], p[q], acc[i][j][q]);
                }
        }
        if (more) store_stage(buf ^ 1, kb + 1);  // nobody reads buf ^ 1 during this stage
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const uint32_t col = n0 + (wn * TN + j) * 32 + fr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + (wm * TM + i) * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                if (row < M && col < N) y[(size_t)row * N + col] = acc[i][j][r];
            }
        }
}

// The other formats' GEMM tile (64-row tiles up to kMidRows rows, and always for Q2_K) and its K
// split (the rule of gemm_splits over those tiles).
void ext_tile(int kind, size_t rows, size_t *bm, size_t *bn) {
    *bm = rows <= 32 ? 32 : (rows <= kMidRows || kind == FH_Q2_K) ? 64 : 128;
    *bn = rows <= 32 ? 256 : 128;
}
uint32_t ext_splits(int kind, size_t rows, size_t k, size_t n) {
    size_t bm, bn;
    ext_tile(kind, rows, &bm, &bn);
    const uint64_t tiles = (uint64_t)((rows + bm - 1) / bm) * ((n + bn - 1) / bn);
    return gemm_splits(tiles, (uint32_t)(k / 32));
}

template <uint32_t T, int BM, int BN, int WAVES_M>
hipError_t run_gemm_ext(hipStream_t s, const _Float16 *xs, const uint8_t *w, float *y, float *partial, uint32_t M,
                        uint32_t K, uint32_t N) {
    const uint32_t mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7fffffffull) return hipErrorInvalidValue;
    const uint32_t grid = (uint32_t)((tiles + 7) / 8 * 8);
    const uint32_t stages = K / 32;
    const uint32_t sp = partial ? ext_splits((int)T, M, K, N) : 1;
    const uint32_t per = (stages + sp - 1) / sp;
    float *out = sp > 1 ? partial : y;
    gemm_ext_kernel<T, BM, BN, WAVES_M><<<dim3(grid, sp), 256, 0, s>>>(xs, w, out, M, K, N, mt, nt, per);
    if (sp > 1) {
        const size_t n = (size_t)M * N;
        const unsigned rg = (unsigned)min((n + 1023) / 1024, (size_t)16384);
        gemm_reduce_kernel<<<rg, 256, 0, s>>>(partial, y, n, sp);
    }
    return hipGetLastError();
}

template <uint32_t T>
hipError_t gemm_ext_dispatch(hipStream_t s, const _Float16 *xs, const uint8_t *w, float *y, float *partial,
                             uint32_t M, uint32_t K, uint32_t N) {
    size_t bm, bn;
    ext_tile((int)T, M, &bm, &bn);  // (Q2_K's per-sub-block terms would spill in a 128-row tile)
    if (bm == 32) return run_gemm_ext<T, 32, 256, 1>(s, xs, w, y, partial, M, K, N);
    if (bm == 64) return run_gemm_ext<T, 64, 128, 2>(s, xs, w, y, partial, M, K, N);
    return run_gemm_ext<T, 128, 128, 2>(s, xs, w, y, partial, M, K, N);
}

// ---- the dequant-f16 GEMM (FH_PATH_TILED_F16): weights dequantised into LDS, plain f16 MFMA ----
// x -> f16 of x 2^-s per row (2^s puts the row's largest |x| in [2^14, 2^15), so no element
// overflows and every one keeps f16's 11 bits), in operand order, and xs[m] = 2^s.
template <int KIND>
__global__ __launch_bounds__(256) void split_x_f16_kernel(const float *__restrict__ x, _Float16 *__restrict__ xh,
                                                          float *__restrict__ xs, uint32_t K) {
    // The row is read once: thread t keeps float4 t + 256 i for i < kKeep in registers (rows up to
    // 8192 wide; wider rows read the rest twice). Float4 q is elements 4 (q % 8) .. + 3 of block
    // q / 8, so eight consecutive lanes hold one block.
    constexpr int kKeep = 8;
    __shared__ float red[4];
    const uint32_t m = blockIdx.x, tid = threadIdx.x, nb = K / 32, nq = K / 4;
    const f32x4 *xr = (const f32x4 *)(x + (size_t)m * K);
    f32x4 v[kKeep];
    float mx = 0.0f;
    auto amax = [](f32x4 a) { return fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))); };
#pragma unroll
    for (int i = 0; i < kKeep; i++) {
        const uint32_t q = tid + 256 * i;
        v[i] = q < nq ? xr[q] : f32x4{0.f, 0.f, 0.f, 0.f};
        mx = fmaxf(mx, amax(v[i]));
    }
    for (uint32_t q = tid + 256 * kKeep; q < nq; q += 256) mx = fmaxf(mx, amax(xr[q]));
#pragma unroll
    for (int o = 32; o >= 1; o /= 2) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (tid % 64 == 0) red[tid / 64] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // 2^E <= mx < 2^(E+1); s = E - 14
    int sc = 0;
    if (mx > 0.0f && mx <= 3.4028235e38f) sc = ((int)(__float_as_uint(mx) >> 23) - 127) - 14;
    sc = sc < -126 ? -126 : (sc > 126 ? 126 : sc);  // both 2^s and 2^-s stay normal floats
    const float f = __uint_as_float((uint32_t)(127 - sc) << 23);
    if (tid == 0) xs[m] = __uint_as_float((uint32_t)(127 + sc) << 23);
    const int j = tid % 8;
    // (q < nq is the same for the eight lanes of a block: nq is a multiple of 8)
    auto put = [&](uint32_t q, f32x4 w) {
        const uint32_t t = q / 8;
        _Float16 h[4];
#pragma unroll
        for (int c = 0; c < 4; c++) h[c] = (_Float16)(w[c] * f);
        _Float16 *out = xh + ((size_t)m * nb + t) * 32;
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        if constexpr (KIND == FH_Q8_0) {
            *(f16x4 *)(out + 4 * j) = f16x4{h[0], h[2], h[1], h[3]};
        } else {
            _Float16 o[4];
#pragma unroll
            for (int c = 0; c < 4; c++)
                o[c] = __builtin_bit_cast(_Float16, (uint16_t)__shfl_xor((int)__builtin_bit_cast(uint16_t, h[c]), 4, 8));
            if (j < 4) *(f16x8 *)(out + 8 * j) = f16x8{h[0], h[2], h[1], h[3], o[0], o[2], o[1], o[3]};
        }
    };
#pragma unroll
    for (int i = 0; i < kKeep; i++) {
        const uint32_t q = tid + 256 * i;
        if (q < nq) put(q, v[i]);
    }
    for (uint32_t q = tid + 256 * kKeep; q < nq; q += 256) put(q, xr[q]);
}

// f16 pairs times one f16 scale (round to nearest: d q is exact before the rounding)
__device__ __forceinline__ uint32_t f16x2_mul(uint32_t w, _Float16 d) {
    const f16x2 v = __builtin_bit_cast(f16x2, w) * f16x2{d, d};
    return __builtin_bit_cast(uint32_t, v);
}

template <int KIND, int BM, int BN>
struct GemmCfgF16 {
    static constexpr int TM = BM / 32, TN = BN / 4 / 32;  // 32x32 tiles per wave (4 waves side by side along N)
    static constexpr int QB = KIND == FH_Q8_0 ? 32 : 16;  // quant bytes per block
    static constexpr int QD = QB / 4;                     // quant dwords per block
    static constexpr int BSTR = KIND == FH_Q8_0 ? 18 : 9; // LDS dwords per weight column and stage
    static constexpr int XH = BM * 8 / 256;               // 16-byte x chunks per thread
    static constexpr int QC = BN * 2 * QB / 16;           // 16-byte quant chunks per stage
    static constexpr int QL = (QC + 255) / 256;
    static_assert(BN % 128 == 0 && BM % 32 == 0 && BM * 8 % 256 == 0, "tile shape");
};

// 8 operand positions of a Q4_0 block from one quant dword (positions 8i..8i+7 come from dword
// i: the low nibbles of bytes (0, 2), (1, 3), then the high ones), times the block's scale
__device__ __forceinline__ f16x8 dequant_q4_frag(uint32_t w, _Float16 d) {
    u32x4 v;
    v[0] = f16x2_mul(f16x2_add((w & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f), d);
    v[1] = f16x2_mul(f16x2_add(((w >> 8) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f), d);
    v[2] = f16x2_mul(f16x2_add(((w >> 4) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f), d);
    v[3] = f16x2_mul(f16x2_add(((w >> 12) & 0x000f000fu) | 0x64006400u, (_Float16)-1032.0f), d);
    return __builtin_bit_cast(f16x8, v);
}

// 8 operand positions of a Q8_0 block from two quant dwords (positions 4j..4j+3 from dword j)
__device__ __forceinline__ f16x8 dequant_q8_frag(uint32_t w0, uint32_t w1, _Float16 d) {
    u32x4 v;
    const uint32_t t0 = w0 ^ 0x80808080u, t1 = w1 ^ 0x80808080u;
    v[0] = f16x2_mul(f16x2_add(__builtin_amdgcn_perm(0x64646464u, t0, 0x04020400u), (_Float16)-1152.0f), d);
    v[1] = f16x2_mul(f16x2_add(__builtin_amdgcn_perm(0x64646464u, t0, 0x04030401u), (_Float16)-1152.0f), d);
    v[2] = f16x2_mul(f16x2_add(__builtin_amdgcn_perm(0x64646464u, t1, 0x04020400u), (_Float16)-1152.0f), d);
    v[3] = f16x2_mul(f16x2_add(__builtin_amdgcn_perm(0x64646464u, t1, 0x04030401u), (_Float16)-1152.0f), d);
    return __builtin_bit_cast(f16x8, v);
}

// Per pipeline stage (two blocks, 64 k) a CTA holds x (f16, operand order) and the weights'
// packed quants with their scales in LDS, double-buffered: one barrier per stage, the next
// stage stored to the other buffer and the one after requested from memory while this one
// computes. Each wavefront owns a BM x BN/4 slab, so every weight fragment is dequantised by
// exactly one wavefront, in registers (the unpack, one packed f16 subtract and one packed f16
// multiply per pair: d q exact, then rounded once), right before its
// v_mfma_f32_32x32x16_f16; results accumulate straight into f32 and the epilogue scales each row
// by its 2^s. Tile order and the K split are those of gemm_kernel.
template <int KIND, int BM, int BN>
__global__ __launch_bounds__(256, 2) void gemm_f16_kernel(const _Float16 *__restrict__ xh, const float *__restrict__ xs,
                                                          const uint8_t *__restrict__ qs, const uint16_t *__restrict__ ds,
                                                          float *__restrict__ y, uint32_t M, uint32_t K, uint32_t N,
                                                          uint32_t mt, uint32_t nt, uint32_t split_stages) {
    using C = GemmCfgF16<KIND, BM, BN>;
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][BM * kAStr];
    __shared__ __attribute__((aligned(16))) uint32_t sB[2][BN * C::BSTR];

    uint32_t mi, ni;
    if (!xcd_tile(mt, nt, &mi, &ni)) return;  // whole CTA: no barrier is left waiting
    const uint32_t m0 = mi * BM, n0 = ni * BN;

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const uint32_t nb = K / 32, all_stages = (nb + 1) / 2;
    const uint32_t st0 = blockIdx.y * split_stages, st1 = min(all_stages, st0 + split_stages);
    y += (size_t)blockIdx.y * M * N;
    const int fr = lane % 32, hf = lane / 32, fk = 8 * hf;

    const auto r_xh = make_rsrc(xh, M * nb * 64);
    const auto r_q = make_rsrc(qs, (N + 31) / 32 * 32 * nb * C::QB);
    const auto r_d = make_rsrc(ds, (N + 31) / 32 * 32 * ((nb + 7) / 8 * 8) * 2);
    constexpr uint32_t kOut = 0x80000000u;
    uint32_t o_xh[C::XH], s_xh[C::XH], o_q[C::QL], s_q[C::QL], o_d, s_d;
#pragma unroll
    for (int i = 0; i < C::XH; i++) {
        const int cc = tid + 256 * i, r = cc / 8, bb = (cc % 8) / 4, part = cc % 4;
        const uint32_t m = m0 + r;
        o_xh[i] = m < M ? ((m * nb + bb) * 32 + part * 8) * 2 : kOut;
        s_xh[i] = (r * kAStr + bb * 32 + part * 8) * 2;
    }
#pragma unroll
    for (int i = 0; i < C::QL; i++) {
        const int cc = tid + 256 * i;
        constexpr int CPB = C::QB / 16;  // 16-byte chunks per block
        const int col = cc / (2 * CPB), bb = (cc % (2 * CPB)) / CPB, part = cc % CPB;
        const uint32_t n = n0 + col;
        o_q[i] = cc < C::QC ? (((n >> 5) * nb + bb) * 32 + (n & 31)) * C::QB + part * 16 : kOut;
        s_q[i] = cc < C::QC ? col * C::BSTR + bb * C::QD + part * 4 : 0u;
    }
    {
        const uint32_t n = n0 + tid;  // thread t < BN loads column t's scales of the stage's two blocks
        o_d = tid < BN ? (((n >> 5) * ((nb + 7) / 8) * 32 + (n & 31)) * 8) * 2 : kOut;
        s_d = tid * C::BSTR + 2 * C::QD;
    }
    u32x4 rxh[C::XH], rq[C::QL];
    uint32_t rd = 0;
    auto load_stage = [&](uint32_t st) {
#pragma unroll
        for (int i = 0; i < C::XH; i++)
            rxh[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_xh, (int)(o_xh[i] + st * 128), 0, 0));
#pragma unroll
        for (int i = 0; i < C::QL; i++)
            rq[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_q, (int)(o_q[i] + st * 64 * C::QB), 0, 0));
        rd = __builtin_amdgcn_raw_buffer_load_b32(r_d, (int)(o_d + (st >> 2) * 512 + (st & 3) * 4), 0, 0);
    };
    auto store_stage = [&](int buf) {
        uint8_t *sAb = (uint8_t *)sA[buf];
        uint32_t *sBb = sB[buf];
#pragma unroll
        for (int i = 0; i < C::XH; i++) *(u32x4 *)(sAb + s_xh[i]) = rxh[i];
#pragma unroll
        for (int i = 0; i < C::QL; i++)
            if (tid + 256 * i < C::QC)
#pragma unroll
                for (int w = 0; w < 4; w++) sBb[s_q[i] + w] = rq[i][w];
        if (tid < BN) sBb[s_d] = rd;
    };

    f32x16 acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    if (st0 < st1) {
        load_stage(st0);
        store_stage(0);
        if (st0 + 1 < st1) load_stage(st0 + 1);
    }
    for (uint32_t st = st0; st < st1; st++) {
        const int buf = (st - st0) & 1;
        __syncthreads();  // stage st is in buf; every wave is done with the other buffer
        if (st + 1 < st1) {
            store_stage(buf ^ 1);
            if (st + 2 < st1) load_stage(st + 2);  // in flight during this stage's MFMAs
        }
        const _Float16 *a = sA[buf];
        const uint32_t *bq = sB[buf];
        const int steps = nb - 2 * st < 2u ? 2 : 4;  // k16 steps: an odd last stage has one block
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            if (ks >= steps) break;
            const int bb = ks / 2, s2 = ks % 2;
            f16x8 bf[C::TN], ah[C::TM];
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const uint32_t *cp = bq + ((wave * C::TN + j) * 32 + fr) * C::BSTR;
                const uint32_t dd = cp[2 * C::QD];
                const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(bb ? dd >> 16 : dd & 0xffffu));
                if constexpr (KIND == FH_Q8_0) {
                    const uint32_t *w = cp + bb * C::QD + 2 * (2 * s2 + hf);
                    bf[j] = dequant_q8_frag(w[0], w[1], d);
                } else {
                    bf[j] = dequant_q4_frag(cp[bb * C::QD + 2 * s2 + hf], d);
                }
            }
#pragma unroll
            for (int i = 0; i < C::TM; i++) ah[i] = *(const f16x8 *)(&a[(i * 32 + fr) * kAStr + 16 * ks + fk]);
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }

#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const uint32_t row = m0 + i * 32 + 8 * (r / 4) + 4 * hf + r % 4;
            if (row >= M) continue;
            const float sx = xs[row];
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const uint32_t col = n0 + (wave * C::TN + j) * 32 + fr;
                if (col < N) y[(size_t)row * N + col] = acc[i][j][r] * sx;
            }
        }
}

// The large-tile variant: a CTA of eight wavefronts computes a 256 x 256 tile, each wavefront a
// 128 x 64 part (eight 32 x 32 accumulators), one CTA per CU, so every SIMD holds two wavefronts
// and one can issue MFMAs while the other waits. The weights are dequantised once per stage,
// when the staged quants are written to LDS (f16(d q), the values gemm_f16_kernel computes), so a
// stage's compute is LDS reads and MFMAs only: per k16 step four x and two weight fragments
// (16-byte reads) feed eight v_mfma_f32_32x32x16_f16. Tiles as xcd_tile deals them.
constexpr int kBigStr = 72;  // LDS halves per row (x) or column (weights) and stage: 64 + 8 pad

template <int KIND>
struct BigLoad {  // one thread's share of a stage in flight
    static constexpr int QB = KIND == FH_Q8_0 ? 32 : 16;  // quant bytes per block
    static constexpr int QL = QB / 16;                    // 16-byte quant loads: one block of its column
    u32x4 a[4], q[QL];
    uint32_t d, dmask, sx;
};

template <int KIND>
__global__ __launch_bounds__(512, 1) void gemm_f16_big_kernel(const _Float16 *__restrict__ xh,
                                                              const float *__restrict__ xs,
                                                              const uint8_t *__restrict__ qs,
                                                              const uint16_t *__restrict__ ds, float *__restrict__ y,
                                                              uint32_t M, uint32_t K, uint32_t N, uint32_t mt,
                                                              uint32_t nt, uint32_t split_stages) {
    // split_stages is even (the stage loop runs pairs)
    using L = BigLoad<KIND>;
    __shared__ __attribute__((aligned(16))) _Float16 sA0[256 * kBigStr], sA1[256 * kBigStr];
    __shared__ __attribute__((aligned(16))) _Float16 sB0[256 * kBigStr], sB1[256 * kBigStr];
    __shared__ float sxs[2][256];  // the row scales of the tiles in flight (by tile parity)

    // This CTA's tiles: XCD x (blockIdx.x % 8) owns the x-th equal run of a grouped tile order
    // (xcd_tile's, with groups of eight row tiles) and its CTAs take the run's tiles round robin.
    // A CTA works through its tiles' stages as one stream: the first stages of its next tile are
    // loaded and stored while it computes the last ones of the current tile, and a tile's output
    // stores drain during the next one.
    constexpr uint32_t GM = 8;  // (measured: 4% faster than groups of four on the widest product)
    const uint32_t tiles = mt * nt, per_xcd = (tiles + 7) / 8, ctas = gridDim.x / 8;
    const uint32_t run0 = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8, run1 = min(tiles, (blockIdx.x % 8 + 1) * per_xcd);
    if (run0 >= run1) return;  // whole CTA: no barrier is left waiting
    const uint32_t my_tiles = (run1 - run0 + ctas - 1) / ctas;
    auto origin = [&](uint32_t k, uint32_t &m0, uint32_t &n0) {  // row and column of my k-th tile
        const uint32_t t = run0 + k * ctas;
        const uint32_t grp = t / (GM * nt), in = t % (GM * nt), gm = min(GM, mt - grp * GM);
        m0 = (grp * GM + in % gm) * 256;
        n0 = (in / gm) * 256;
    };

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, wm = wave % 2, wn = wave / 2;
    const uint32_t nb = K / 32, all_stages = (nb + 1) / 2;
    const uint32_t st0 = blockIdx.y * split_stages, st1 = min(all_stages, st0 + split_stages);
    const uint32_t stream = my_tiles * split_stages;  // positions p: tile p / split_stages, stage st0 + p % split_stages
    y += (size_t)blockIdx.y * M * N;
    const int fr = lane % 32, hf = lane / 32;

    const auto r_xh = make_rsrc(xh, M * nb * 64);
    const auto r_q = make_rsrc(qs, (N + 31) / 32 * 32 * nb * L::QB);
    const auto r_d = make_rsrc(ds, (N + 31) / 32 * 32 * ((nb + 7) / 8 * 8) * 2);
    const auto r_s = make_rsrc(xs, M * 4);
    constexpr uint32_t kOut = 0x80000000u;
    // x: chunk c = tid + 512 i is row c / 8, 16 bytes (c % 8) of the row's 128-byte stage;
    // weights: thread t owns block bq = t / 256 of the stage in column n0 + t % 256 (its quants
    // and the column's scale dword, of which it uses half bq)
    const int cq = tid % 256, bq = tid / 256;

    L ld0, ld1;  // two stages in flight: each load has two stages of MFMAs to arrive
    auto load_stage = [&](L &ld, uint32_t p) {
        // past the tile's stages (the loop runs an even number) and past the stream everything
        // reads 0; an odd last stage of the product has one block, and its second block reads 0
        const uint32_t st = st0 + p % split_stages;
        const bool live = p < stream && st < st1, two = live && 2 * st + 1 < nb;
        uint32_t m0, n0;
        origin(min(p / split_stages, my_tiles - 1), m0, n0);  // (positions past the stream load nothing)
        uint32_t o_a[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t m = m0 + (tid + 512 * i) / 8;
            o_a[i] = m < M ? (m * nb * 32 + (tid % 8) * 8) * 2 : kOut;
        }
        const uint32_t n = n0 + cq;
        const uint32_t o_q = ((n >> 5) * nb * 32 + (n & 31)) * L::QB;
        const uint32_t o_d = ((n >> 5) * ((nb + 7) / 8) * 32 + (n & 31)) * 16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t off = (live && (tid % 8) < 4) || two ? o_a[i] + st * 128 : kOut;
            ld.a[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_xh, (int)off, 0, 0));
        }
        const bool mine = bq == 0 ? live : two;
#pragma unroll
        for (int i = 0; i < L::QL; i++) {
            const uint32_t off = mine ? o_q + ((2 * st + bq) * 32 * L::QB + i * 16) : kOut;
            ld.q[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_q, (int)off, 0, 0));
        }
        ld.d = __builtin_amdgcn_raw_buffer_load_b32(r_d, mine ? (int)(o_d + (st >> 2) * 512 + (st & 3) * 4) : (int)kOut,
                                                    0, 0);
        ld.dmask = mine ? 0xffffffffu : 0u;  // a missing block's scale is 0, so its values are 0
        // a tile's first stage also carries its row scales (thread t < 256: row m0 + t), for the
        // epilogue through LDS: a global load there would wait behind the next tile's loads
        ld.sx = __builtin_amdgcn_raw_buffer_load_b32(
            r_s, p % split_stages == 0 && p < stream && tid < 256 ? (int)((m0 + tid) * 4) : (int)kOut, 0, 0);
        // (applied when the stage is stored: using the loaded value here would wait for the load)
    };
    auto store_stage = [&](const L &ld, _Float16 *sa, _Float16 *sb, int first) {
        if (first >= 0 && tid < 256) sxs[first][tid] = __uint_as_float(ld.sx);
#pragma unroll
        for (int i = 0; i < 4; i++) *(u32x4 *)(sa + ((tid + 512 * i) / 8) * kBigStr + (tid % 8) * 8) = ld.a[i];
        _Float16 *col = sb + cq * kBigStr + bq * 32;
        const uint32_t dd = ld.d & ld.dmask;
        const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(bq ? dd >> 16 : dd & 0xffffu));
#pragma unroll
        for (int f = 0; f < 4; f++) {
            f16x8 v;
            if constexpr (KIND == FH_Q8_0) {
                const u32x4 &w = ld.q[f / 2];
                v = dequant_q8_frag(w[2 * (f % 2)], w[2 * (f % 2) + 1], d);
            } else {
                v = dequant_q4_frag(ld.q[0][f], d);
            }
            *(f16x8 *)(col + 8 * f) = v;
        }
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // The fragments of k16 step ks + 1 are read while step ks's eight MFMAs run (a read after
    // each of the first six, an order the scheduling-group barriers pin down); step 0's are read
    // before the stage's stores, so they arrive while the next stage is stored.
    f16x8 ah[2][4], bf[2][2];
    auto read = [&](const _Float16 *sa, const _Float16 *sb, int ks) {
        const _Float16 *a = sa + (wm * 128 + fr) * kBigStr + 8 * hf;
        const _Float16 *b = sb + (wn * 64 + fr) * kBigStr + 8 * hf;
#pragma unroll
        for (int i = 0; i < 4; i++) ah[ks % 2][i] = *(const f16x8 *)(a + i * 32 * kBigStr + 16 * ks);
#pragma unroll
        for (int j = 0; j < 2; j++) bf[ks % 2][j] = *(const f16x8 *)(b + j * 32 * kBigStr + 16 * ks);
    };
    auto compute = [&](const _Float16 *sa, const _Float16 *sb) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            if (ks < 3) read(sa, sb, ks + 1);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[ks % 2][i], bf[ks % 2][j], acc[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int ks = 0; ks < 3; ks++) {
#pragma unroll
            for (int r = 0; r < 6; r++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA of step ks
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a read of step ks + 1
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // step 3's MFMAs
    };

    auto epilogue = [&](uint32_t k) {
        uint32_t m0, n0;
        origin(k, m0, n0);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + wm * 128 + i * 32 + 8 * (r / 4) + 4 * hf + r % 4;
                if (row >= M) continue;
                const float sx = sxs[k % 2][row - m0];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t col = n0 + wn * 64 + j * 32 + fr;
                    if (col < N) y[(size_t)row * N + col] = acc[i][j][r] * sx;
                }
            }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    };

    load_stage(ld0, 0);
    load_stage(ld1, 1);
    store_stage(ld0, sA0, sB0, 0);
    load_stage(ld0, 2);
    // Two stages per trip (the buffers and staging registers are then known apart). Scheduling
    // barriers keep each phase in place: nothing that reads a staged load may be moved up into
    // the MFMAs issued while that load is in flight.
    for (uint32_t p = 0; p < stream; p += 2) {
        __syncthreads();  // stage p is in buffer 0; every wave is done with buffer 1
        __builtin_amdgcn_sched_barrier(0);
        read(sA0, sB0, 0);
        __builtin_amdgcn_sched_barrier(0);
        store_stage(ld1, sA1, sB1, -1);  // (odd stages never start a tile)
        load_stage(ld1, p + 3);
        __builtin_amdgcn_sched_barrier(0);
        compute(sA0, sB0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        read(sA1, sB1, 0);
        __builtin_amdgcn_sched_barrier(0);
        store_stage(ld0, sA0, sB0, (p + 2) % split_stages == 0 ? (int)(((p + 2) / split_stages) % 2) : -1);
        load_stage(ld0, p + 4);
        __builtin_amdgcn_sched_barrier(0);
        compute(sA1, sB1);
        if ((p + 2) % split_stages == 0) epilogue(p / split_stages);  // the tile's last stage pair
    }
}

struct GemmF16Args {
    const _Float16 *xh;
    const float *xs;
    const uint8_t *qs;
    const uint16_t *ds;
    float *y, *partial;
    uint32_t M, K, N;
    SplitOut *defer = nullptr;  // set: the partial sums are left for the consumer
};

template <int KIND, int BM, int BN>
hipError_t run_gemm_f16(hipStream_t s, const GemmF16Args &g) {
    const uint32_t mt = (g.M + BM - 1) / BM, nt = (g.N + BN - 1) / BN;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7ffffff0ull) return hipErrorInvalidValue;
    const uint32_t grid = (uint32_t)((tiles + 7) / 8 * 8);  // an equal share for every XCD
    const uint32_t stages = (g.K / 32 + 1) / 2;
    const uint32_t sp = g.partial ? gemm_splits((uint64_t)mt * nt, stages) : 1;
    const uint32_t per = (stages + sp - 1) / sp;
    float *out = sp > 1 ? g.partial : g.y;
    gemm_f16_kernel<KIND, BM, BN><<<dim3(grid, sp), 256, 0, s>>>(g.xh, g.xs, g.qs, g.ds, out, g.M, g.K, g.N, mt, nt,
                                                                  per);
    if (g.defer) *g.defer = sp > 1 ? SplitOut{g.partial, sp} : SplitOut{g.y, 1u};
    if (sp > 1 && !g.defer) {
        const size_t n = (size_t)g.M * g.N;
        const unsigned rg = (unsigned)min((n + 1023) / 1024, (size_t)16384);
        gemm_reduce_kernel<<<rg, 256, 0, s>>>(g.partial, g.y, n, sp);
    }
    return hipGetLastError();
}

// tile shape by rows
void f16_tile(size_t rows, size_t *bm, size_t *bn) {
    *bm = rows <= 32 ? 32 : rows <= 64 ? 64 : 128;
    *bn = 256;
}

// The 256 x 256 kernel's plan: taken when the product has at least 128 such tiles; the K split
// (at most 4, at least 8 stages per split) that best fills whole rounds of one CTA per CU.
bool f16_big_plan(size_t rows, size_t k, size_t n, uint32_t *splits) {
    const uint64_t tiles = (uint64_t)((rows + 255) / 256) * ((n + 255) / 256);
    if (tiles < 128) return false;
    const uint32_t stages = (uint32_t)((k / 32 + 1) / 2), cus = 256;
    uint32_t best = 1;
    double best_eff = 0.0;
    for (uint32_t sp = 1; sp <= 4 && (sp == 1 || stages / sp >= 8); sp++) {
        const uint64_t ctas = tiles * sp, rounds = (ctas + cus - 1) / cus;
        const double eff = (double)ctas / (double)(rounds * cus) - 0.04 * (sp - 1);  // the reduce pass
        if (eff > best_eff + 1e-9) {
            best_eff = eff;
            best = sp;
        }
    }
    *splits = best;
    return true;
}

template <int KIND>
hipError_t run_gemm_f16_big(hipStream_t s, const GemmF16Args &g, uint32_t sp) {
    const uint32_t mt = (g.M + 255) / 256, nt = (g.N + 255) / 256;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7ffffff0ull) return hipErrorInvalidValue;
    const uint32_t per_xcd = (uint32_t)((tiles + 7) / 8);
    // one CTA per CU, each XCD's CTAs working through its run of tiles
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8)
        cus = 256;
    const uint32_t ctas = min(per_xcd, (uint32_t)cus / 8);
    const uint32_t stages = (g.K / 32 + 1) / 2;
    const uint32_t per = ((stages + sp - 1) / sp + 1) & ~1u;  // even: the kernel runs stages in pairs
    float *out = sp > 1 ? g.partial : g.y;
    gemm_f16_big_kernel<KIND><<<dim3(8 * ctas, sp), 512, 0, s>>>(g.xh, g.xs, g.qs, g.ds, out, g.M, g.K, g.N, mt,
                                                                     nt, per);
    if (g.defer) *g.defer = sp > 1 ? SplitOut{g.partial, sp} : SplitOut{g.y, 1u};
    if (sp > 1 && !g.defer) {
        const size_t n = (size_t)g.M * g.N;
        const unsigned rg = (unsigned)min((n + 1023) / 1024, (size_t)16384);
        gemm_reduce_kernel<<<rg, 256, 0, s>>>(g.partial, g.y, n, sp);
    }
    return hipGetLastError();
}

template <int KIND>
hipError_t gemm_f16_dispatch(hipStream_t s, const GemmF16Args &g) {
    uint32_t sp = 1;
    if (f16_big_plan(g.M, g.K, g.N, &sp)) return run_gemm_f16_big<KIND>(s, g, sp);
    if (g.M <= 32) return run_gemm_f16<KIND, 32, 256>(s, g);
    if (g.M <= 64) return run_gemm_f16<KIND, 64, 256>(s, g);
    return run_gemm_f16<KIND, 128, 256>(s, g);
}

}  // namespace

GemmXSplit gemm_x_split(void *workspace, size_t rows, size_t k) {
    const auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    uint8_t *ws = (uint8_t *)workspace;
    return GemmXSplit{(_Float16 *)ws, ws + up(rows * k * 2), ws + up(rows * k * 2) + up(rows * ((k + 63) / 64 * 64))};
}

// x hi (2 bytes per element), x lo (1 byte, rows of k rounded up to 64), two scale bytes per row
// and 64 k (rows rounded up to 8), each piece 256-aligned (the planes of xsplit.hpp)
size_t gemm_xsplit_bytes(size_t rows, size_t k) {
    const auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    return up(rows * k * 2) + up(rows * ((k + 63) / 64 * 64)) + up((k + 63) / 64 * xsb_rows((uint32_t)rows) * 2);
}

size_t gemm_workspace_bytes(size_t rows, size_t k, size_t n) {
    return gemm_xsplit_bytes(rows, k) + gemm_partial_bytes(rows, k, n);
}

// Room for the K-split partial products when the product's tile grid is too small to fill the
// chip (the tile shapes of fast_tile and the split rule of run_gemm); none otherwise.
size_t gemm_partial_bytes(size_t rows, size_t k, size_t n) {
    size_t bm, bn;
    fast_tile(rows, &bm, &bn);
    const uint64_t tiles = (uint64_t)((rows + bm - 1) / bm) * ((n + bn - 1) / bn);
    uint32_t sp = gemm_splits(tiles, (uint32_t)((k / 32 + 1) / 2)), ssp = 1;
    if (stream_fast_plan(rows, k, n, &ssp) && stream_fast_supported(rows, k, n)) sp = max(sp, ssp);
    return sp > 1 ? (size_t)sp * rows * n * 4 : 0;
}

size_t gemm_b8_bytes(size_t k, size_t n) { return (n * ((k + 63) / 64 * 64) + 255) / 256 * 256 + n * 4; }

bool gemm_supported(size_t rows, size_t k, size_t n) {
    // every operand's byte offsets fit the kernel's 32-bit buffer offsets
    const size_t k64 = (k + 63) / 64 * 64, lim = (size_t)1 << 31;
    return rows * k * 2 < lim && rows * k64 < lim && n * k64 < lim && (n + 31) / 32 * 32 * (k / 32) * 32 < lim;
}

hipError_t launch_make_b8(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, uint8_t *b8, size_t k,
                          size_t n) {
    int32_t *bsc = (int32_t *)(b8 + (n * ((k + 63) / 64 * 64) + 255) / 256 * 256);
    const unsigned grid = (unsigned)((n + 3) / 4);
    if (kind == FH_Q8_0)
        make_b8_kernel<FH_Q8_0><<<grid, 256, 0, s>>>(qs, ds, b8, bsc, (uint32_t)k, (uint32_t)n);
    else
        make_b8_kernel<FH_Q4_0><<<grid, 256, 0, s>>>(qs, ds, b8, bsc, (uint32_t)k, (uint32_t)n);
    return hipGetLastError();
}

// x split into f16 pairs (4 bytes per element), then the K-split partial products (256-aligned)
size_t gemm_precise_workspace_bytes(size_t rows, size_t k, size_t n) {
    uint32_t sp = precise_splits(rows, k, n), ssp = 1;
    if (stream_plan(rows, k, n, &ssp) && stream_supported(rows, k, n)) sp = max(sp, ssp);
    return (rows * k * 4 + 255) / 256 * 256 + (sp > 1 ? (size_t)sp * rows * n * 4 : 0);
}

hipError_t launch_gemm_precise(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                               float *y, size_t rows, size_t k, size_t n, void *workspace, SplitOut *defer) {
    _Float16 *xs = (_Float16 *)workspace;
    const size_t xbytes = (rows * k * 4 + 255) / 256 * 256;
    float *partial = gemm_precise_workspace_bytes(rows, k, n) > xbytes ? (float *)((uint8_t *)workspace + xbytes)
                                                                       : nullptr;
    const size_t items = rows * (k / 32);
    const unsigned g = (unsigned)(items / 32 + 1 < 65535 ? items / 32 + 1 : 65535);
    if (kind == FH_Q8_0) {
        split_x_precise_kernel<FH_Q8_0><<<g, 256, 0, s>>>(x, xs, items);
        return gemm_precise_dispatch<FH_Q8_0>(s, xs, qs, ds, y, partial, (uint32_t)rows, (uint32_t)k, (uint32_t)n,
                                              defer);
    }
    split_x_precise_kernel<FH_Q4_0><<<g, 256, 0, s>>>(x, xs, items);
    return gemm_precise_dispatch<FH_Q4_0>(s, xs, qs, ds, y, partial, (uint32_t)rows, (uint32_t)k, (uint32_t)n,
                                          defer);
}

bool gemm_ext_kind(int kind) {
    return kind == FH_F16 || kind == FH_FP8_E4M3 || kind == FH_FP8_E5M2 || kind == FH_MXFP4 || kind == FH_Q2_K;
}

size_t gemm_ext_workspace_bytes(int kind, size_t rows, size_t k, size_t n) {
    const uint32_t sp = ext_splits(kind, rows, k, n);
    return (rows * k * 4 + 255) / 256 * 256 + (sp > 1 ? (size_t)sp * rows * n * 4 : 0);
}

hipError_t launch_gemm_ext(hipStream_t s, int kind, const uint8_t *w, const float *x, float *y, size_t rows, size_t k,
                           size_t n, void *workspace) {
    _Float16 *xs = (_Float16 *)workspace;
    float *partial = ext_splits(kind, rows, k, n) > 1
                         ? (float *)((uint8_t *)workspace + (rows * k * 4 + 255) / 256 * 256)
                         : nullptr;
    const size_t items = rows * (k / 32);
    const unsigned g = (unsigned)(items / 32 + 1 < 65535 ? items / 32 + 1 : 65535);
    split_x_precise_kernel<0><<<g, 256, 0, s>>>(x, xs, items);
    const uint32_t M = (uint32_t)rows, K = (uint32_t)k, N = (uint32_t)n;
    switch (kind) {
    case FH_F16: return gemm_ext_dispatch<FH_F16>(s, xs, w, y, partial, M, K, N);
    case FH_FP8_E4M3: return gemm_ext_dispatch<FH_FP8_E4M3>(s, xs, w, y, partial, M, K, N);
    case FH_FP8_E5M2: return gemm_ext_dispatch<FH_FP8_E5M2>(s, xs, w, y, partial, M, K, N);
    case FH_MXFP4: return gemm_ext_dispatch<FH_MXFP4>(s, xs, w, y, partial, M, K, N);
    case FH_Q2_K: return gemm_ext_dispatch<FH_Q2_K>(s, xs, w, y, partial, M, K, N);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_naive(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                        float *y, size_t rows, size_t k, size_t n) {
    const size_t total = rows * n;
    const unsigned grid = (unsigned)((total + 255) / 256);
    if (kind == FH_Q8_0)
        naive_kernel<FH_Q8_0><<<grid, 256, 0, s>>>(qs, ds, x, y, (uint32_t)rows, (uint32_t)k, (uint32_t)n);
    else
        naive_kernel<FH_Q4_0><<<grid, 256, 0, s>>>(qs, ds, x, y, (uint32_t)rows, (uint32_t)k, (uint32_t)n);
    return hipGetLastError();
}

hipError_t launch_gemm(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const uint8_t *b8,
                       const float *x, float *y, size_t rows, size_t k, size_t n, void *workspace, SplitOut *defer,
                       float *partial, const GemmXSplit *xs) {
    const auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    uint8_t *ws = (uint8_t *)workspace;
    const GemmXSplit sx = xs && !x ? *xs : gemm_x_split(ws, rows, k);
    GemmArgs g;
    g.xh = sx.xh;
    g.xl = sx.xl;
    g.xsb = sx.xsb;
    g.qs = qs;
    g.ds = ds;
    g.b8 = b8;
    g.bsc = (const int32_t *)(b8 + up(n * ((k + 63) / 64 * 64)));
    g.y = y;
    const size_t pb = gemm_partial_bytes(rows, k, n);
    g.partial = !pb ? nullptr : partial ? partial : (float *)(ws + gemm_xsplit_bytes(rows, k));
    g.M = (uint32_t)rows;
    g.K = (uint32_t)k;
    g.N = (uint32_t)n;
    g.defer = defer;
    if (kind == FH_Q8_0) {
        if (x) split_x_kernel<FH_Q8_0><<<(unsigned)rows, 256, 0, s>>>(x, sx.xh, sx.xl, sx.xsb, g.K);
        return gemm_fast_dispatch<FH_Q8_0>(s, g);
    }
    if (x) split_x_kernel<FH_Q4_0><<<(unsigned)rows, 256, 0, s>>>(x, sx.xh, sx.xl, sx.xsb, g.K);
    return gemm_fast_dispatch<FH_Q4_0>(s, g);
}

// The fast GEMM with SwiGLU in its epilogue (gemm_kernel<..., true>) takes the product when the
// plain fast product would run on gemm_kernel with one K split: not the streaming kernel, and a
// tile grid that fills the chip or a K too short to split; n (gate and up) a multiple of 64.
bool gemm_swiglu_supported(size_t rows, size_t k, size_t n) {
    if (!rows || n % 64 || !gemm_supported(rows, k, n)) return false;
    uint32_t ssp = 1;
    if (stream_fast_plan(rows, k, n, &ssp) && stream_fast_supported(rows, k, n)) return false;
    size_t bm, bn;
    fast_tile(rows, &bm, &bn);
    const uint64_t tiles = (uint64_t)((rows + bm - 1) / bm) * ((n + bn - 1) / bn);
    return gemm_splits(tiles, (uint32_t)((k / 32 + 1) / 2)) == 1;
}

hipError_t launch_gemm_swiglu(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const uint8_t *b8,
                              const float *x, const GemmXSplit &act, size_t rows, size_t k, size_t n,
                              void *workspace) {
    if (!gemm_swiglu_supported(rows, k, n)) return hipErrorInvalidValue;
    const auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    const GemmXSplit sx = gemm_x_split(workspace, rows, k);
    GemmArgs g;
    g.xh = sx.xh;
    g.xl = sx.xl;
    g.xsb = sx.xsb;
    g.qs = qs;
    g.ds = ds;
    g.b8 = b8;
    g.bsc = (const int32_t *)(b8 + up(n * ((k + 63) / 64 * 64)));
    g.y = nullptr;
    g.partial = nullptr;  // one K split
    g.M = (uint32_t)rows;
    g.K = (uint32_t)k;
    g.N = (uint32_t)n;
    g.act = act;
    if (kind == FH_Q8_0) {
        if (x) split_x_kernel<FH_Q8_0><<<(unsigned)rows, 256, 0, s>>>(x, sx.xh, sx.xl, sx.xsb, g.K);
        return gemm_dispatch<FH_Q8_0, true>(s, g);
    }
    if (x) split_x_kernel<FH_Q4_0><<<(unsigned)rows, 256, 0, s>>>(x, sx.xh, sx.xl, sx.xsb, g.K);
    return gemm_dispatch<FH_Q4_0, true>(s, g);
}

// x as f16 (2 bytes per element), the row scales, then the K-split partials, each 256-aligned
size_t gemm_f16_workspace_bytes(size_t rows, size_t k, size_t n) {
    const auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    uint32_t sp = 1;
    if (!f16_big_plan(rows, k, n, &sp)) {
        size_t bm, bn;
        f16_tile(rows, &bm, &bn);
        const uint64_t tiles = (uint64_t)((rows + bm - 1) / bm) * ((n + bn - 1) / bn);
        sp = gemm_splits(tiles, (uint32_t)((k / 32 + 1) / 2));
    }
    return up(rows * k * 2) + up(rows * 4) + (sp > 1 ? (size_t)sp * rows * n * 4 : 0);
}

bool gemm_f16_supported(size_t rows, size_t k, size_t n) {
    const size_t lim = (size_t)1 << 31;
    return rows * k * 2 < lim && (n + 31) / 32 * 32 * (k / 32) * 32 < lim;
}

hipError_t launch_gemm_f16(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x, float *y,
                           size_t rows, size_t k, size_t n, void *workspace, SplitOut *defer) {
    const auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    uint8_t *ws = (uint8_t *)workspace;
    GemmF16Args g;
    g.xh = (const _Float16 *)ws;
    g.xs = (const float *)(ws + up(rows * k * 2));
    g.qs = qs;
    g.ds = ds;
    g.y = y;
    g.partial = gemm_f16_workspace_bytes(rows, k, n) > up(rows * k * 2) + up(rows * 4)
                    ? (float *)(ws + up(rows * k * 2) + up(rows * 4))
                    : nullptr;
    g.M = (uint32_t)rows;
    g.K = (uint32_t)k;
    g.N = (uint32_t)n;
    g.defer = defer;
    if (kind == FH_Q8_0) {
        split_x_f16_kernel<FH_Q8_0><<<(unsigned)rows, 256, 0, s>>>(x, (_Float16 *)g.xh, (float *)g.xs, g.K);
        return gemm_f16_dispatch<FH_Q8_0>(s, g);
    }
    split_x_f16_kernel<FH_Q4_0><<<(unsigned)rows, 256, 0, s>>>(x, (_Float16 *)g.xh, (float *)g.xs, g.K);
    return gemm_f16_dispatch<FH_Q4_0>(s, g);
}

bool gemm_score_supported(fh_path path, size_t rows, size_t k, size_t n) {
    if (path == FH_PATH_TILED_FAST) return stream_fast_supported(rows, k, n) && gemm_supported(rows, k, n);
    if (path == FH_PATH_TILED) return stream_supported(rows, k, n);
    return false;
}

hipError_t launch_gemm_score(hipStream_t s, fh_path path, fh_kind kind, const uint8_t *qs, const uint16_t *ds,
                             const uint8_t *b8, const float *x, size_t rows, size_t k, size_t n, void *workspace,
                             const ScoreOut &so) {
    if (!gemm_score_supported(path, rows, k, n)) return hipErrorInvalidValue;
    const uint32_t M = (uint32_t)rows, K = (uint32_t)k, N = (uint32_t)n;
    if (path == FH_PATH_TILED_FAST) {
        const auto up = [](size_t v) { return (v + 255) / 256 * 256; };
        const GemmXSplit sx = gemm_x_split(workspace, rows, k);
        const int32_t *bsc = (const int32_t *)(b8 + up(n * ((k + 63) / 64 * 64)));
        if (kind == FH_Q8_0) {
            split_x_kernel<FH_Q8_0><<<M, 256, 0, s>>>(x, sx.xh, sx.xl, sx.xsb, K);
            return run_gemm_score<FH_Q8_0>(s, path, sx.xh, sx.xl, sx.xsb, qs, ds, b8, bsc, M, K, N, so);
        }
        split_x_kernel<FH_Q4_0><<<M, 256, 0, s>>>(x, sx.xh, sx.xl, sx.xsb, K);
        return run_gemm_score<FH_Q4_0>(s, path, sx.xh, sx.xl, sx.xsb, qs, ds, b8, bsc, M, K, N, so);
    }
    _Float16 *xs = (_Float16 *)workspace;
    const size_t items = rows * (k / 32);
    const unsigned g = (unsigned)(items / 32 + 1 < 65535 ? items / 32 + 1 : 65535);
    if (kind == FH_Q8_0) {
        split_x_precise_kernel<FH_Q8_0><<<g, 256, 0, s>>>(x, xs, items);
        return run_gemm_score<FH_Q8_0>(s, path, xs, nullptr, nullptr, qs, ds, nullptr, nullptr, M, K, N, so);
    }
    split_x_precise_kernel<FH_Q4_0><<<g, 256, 0, s>>>(x, xs, items);
    return run_gemm_score<FH_Q4_0>(s, path, xs, nullptr, nullptr, qs, ds, nullptr, nullptr, M, K, N, so);
}

}  // namespace fh
