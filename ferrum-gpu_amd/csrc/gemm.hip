// Multi-row products on resident Q8_0 / Q4_0 weights for gfx950: y[M, N] = x[M, K] * W^T, W held
// as the tiled quant and scale planes of its N GGUF rows of K/32 blocks (tile_slot, scale_slot).
//
// naive_kernel: one thread per output, ascending k, the dequantised value formed first and then
// multiplied (ferrum_wgpu/src/shaders/quant/qlinear.wgsl:18-59). Kept as the baseline path.
//
// The MFMA dequant-GEMM (the scoring / prefill path) runs in two launches:
//   1. split_x_kernel writes x as two f16 parts, x = hi + lo (about 22 significant bits), per
//      32-element block in the k order the MFMA operands use (below). Each x element is split
//      once, not once per weight tile.
//   2. gemm_kernel: a CTA computes a BM x BN tile of y with 4 wavefronts. A 32-element block of
//      x (hi and lo) and of the weights form a pipeline stage in LDS (double-buffered, one
//      barrier per stage; the next stage's global loads are in flight during the MFMAs); the
//      weight quants become exact f16 integers (Q8_0 -128..127, Q4_0 -8..7) with a byte permute
//      into an f16 exponent pattern and one packed f16 subtract; per 32 x 32 output tile,
//      P = hi * q + lo * q over the block with four v_mfma_f32_32x32x16_f16 (f32 accumulate),
//      then acc += d[col] * P with the block's f32 scale.
// The scale is applied in f32 after the exact integer dot, so the product meets the reference's
// 1e-5 relative bound for linear_q (ferrum_wgpu/src/tolerance.rs:7) as well as the
// 1e-3 + 2e-3 |y| GEMM bound; plain f16 or bf16 activations do not.
//
// k order inside a block. The unpack produces f16 pairs from a quant dword w: for Q8_0 the bytes
// (0, 2) and (1, 3), i.e. elements 4i + {0, 2, 1, 3}; for Q4_0 the low nibbles of bytes (0, 2),
// (1, 3), then the high nibbles, i.e. elements 4i + {0, 2, 1, 3} and 16 + 4i + {0, 2, 1, 3}. The
// MFMA sums over k, so x is laid out in that same order and no shuffle is needed.
//
// Tile order: CTAs are numbered so each XCD (CTAs go round-robin over the 8 XCDs) takes a
// contiguous range of tiles, walked along N for a fixed M stripe: the XCD's L2 keeps the x rows
// while the weights stream.
#include "device_common.hpp"
#include "internal.hpp"

namespace fh {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float half_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
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

// ---- the k order of a block (position p of the MFMA operands holds element elem(p)) ----
template <int KIND>
__device__ __forceinline__ int elem_of_pos(int p) {
    const int sw = (p & 3) == 1 ? 2 : (p & 3) == 2 ? 1 : (p & 3);  // {0, 2, 1, 3}
    if constexpr (KIND == FH_Q8_0) {
        return (p & ~3) + sw;
    } else {
        const int i = p / 8, j = p % 8;
        return (j < 4 ? 4 * i : 16 + 4 * i) + sw;
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
__global__ __launch_bounds__(256) void split_x_kernel(const float *__restrict__ x, _Float16 *__restrict__ xs,
                                                      size_t items) {
    const int j = threadIdx.x % 8;
    for (size_t t = ((size_t)blockIdx.x * 256 + threadIdx.x) / 8; t < items; t += (size_t)gridDim.x * 32) {
        const f32x4 v = __builtin_nontemporal_load((const f32x4 *)(x + t * 32) + j);
        _Float16 *out = xs + t * 64;
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        if constexpr (KIND == FH_Q8_0) {
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

// ---- the MFMA GEMM ----
constexpr int kARow = 72;  // LDS halves per x row and block: 32 hi + 32 lo + 8 pad (144 B)
constexpr int kBRow = 40;  // LDS halves per weight row and block: 32 + 8 pad (80 B)
constexpr int kBKB = 1;    // blocks (of 32 k) per pipeline stage

template <int KIND, int BM, int BN, int WAVES_M>
struct GemmCfg {
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
__global__ __launch_bounds__(256, 2) void gemm_kernel(const _Float16 *__restrict__ xs, const uint8_t *__restrict__ qs,
                                                      const uint16_t *__restrict__ ds, float *__restrict__ y,
                                                      uint32_t M, uint32_t K, uint32_t N, uint32_t mt, uint32_t nt) {
    using C = GemmCfg<KIND, BM, BN, WAVES_M>;
    // stage layout: x row r, block bb at r * kBKB * kARow + bb * kARow; weight row likewise
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][BM * kBKB * kARow];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][BN * kBKB * kBRow];
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
    const uint32_t stages = (nb + kBKB - 1) / kBKB;

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
            *(u32x4 *)(&sA[buf][(r * kBKB + bb) * kARow + ch * 8]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < C::B_PER; i++) {
            const int cc = tid + 256 * i;
            if (cc < C::B_LD) {
                constexpr int CPR = kBKB * C::QB / 16;
                const int col = cc / CPR, bb = (cc % CPR) / (C::QB / 16), part = cc % (C::QB / 16);
                _Float16 *row = &sB[buf][(col * kBKB + bb) * kBRow];
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

    if (stages > 0) {
        load_stage(0);
        store_stage(0);
    }
    __syncthreads();
    for (uint32_t st = 0; st < stages; st++) {
        const int buf = st & 1;
        const bool more = st + 1 < stages;
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
                const _Float16 *row = &sB[buf][(col * kBKB + bb) * kBRow];
#pragma unroll
                for (int s = 0; s < 2; s++) bf[j][s] = *(const f16x8 *)(row + 16 * s + fk);
                dcol[j] = sD[buf][bb * BN + col];
            }
            f16x8 ah[C::TM][2], al[C::TM][2];
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
                const int r = (wm * C::TM + i) * 32 + fr;
                const _Float16 *row = &sA[buf][(r * kBKB + bb) * kARow];
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

template <int KIND, int BM, int BN, int WAVES_M>
hipError_t run_gemm(hipStream_t s, const _Float16 *xs, const uint8_t *qs, const uint16_t *ds, float *y, uint32_t M,
                    uint32_t K, uint32_t N) {
    const uint32_t mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
    const uint64_t tiles = (uint64_t)mt * nt;
    if (tiles > 0x7fffffffull) return hipErrorInvalidValue;
    const uint32_t grid = (uint32_t)((tiles + 7) / 8 * 8);  // a multiple of the XCD count
    gemm_kernel<KIND, BM, BN, WAVES_M><<<grid, 256, 0, s>>>(xs, qs, ds, y, M, K, N, mt, nt);
    return hipGetLastError();
}

template <int KIND>
hipError_t gemm_dispatch(hipStream_t s, const _Float16 *xs, const uint8_t *qs, const uint16_t *ds, float *y,
                         uint32_t M, uint32_t K, uint32_t N) {
    if (M <= 32) return run_gemm<KIND, 32, 256, 1>(s, xs, qs, ds, y, M, K, N);
    if (M <= 64) return run_gemm<KIND, 64, 128, 2>(s, xs, qs, ds, y, M, K, N);
    return run_gemm<KIND, 128, 128, 2>(s, xs, qs, ds, y, M, K, N);
}

}  // namespace

size_t gemm_workspace_bytes(size_t rows, size_t k) { return rows * k * 4; }

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

hipError_t launch_gemm(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                       float *y, size_t rows, size_t k, size_t n, void *workspace) {
    _Float16 *xs = (_Float16 *)workspace;
    const size_t items = rows * (k / 32);
    const unsigned g = (unsigned)(items / 32 + 1 < 65535 ? items / 32 + 1 : 65535);
    if (kind == FH_Q8_0) {
        split_x_kernel<FH_Q8_0><<<g, 256, 0, s>>>(x, xs, items);
        return gemm_dispatch<FH_Q8_0>(s, xs, qs, ds, y, (uint32_t)rows, (uint32_t)k, (uint32_t)n);
    }
    split_x_kernel<FH_Q4_0><<<g, 256, 0, s>>>(x, xs, items);
    return gemm_dispatch<FH_Q4_0>(s, xs, qs, ds, y, (uint32_t)rows, (uint32_t)k, (uint32_t)n);
}

}  // namespace fh
