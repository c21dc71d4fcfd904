// Multi-row products on resident Q8_0 / Q4_0 weights for gfx950: y[M, N] = x[M, K] * W^T, W held
// as the quant and scale planes of its N GGUF rows of K/32 blocks (see gemv.hip).
//
// naive_kernel: one thread per output, ascending k, the dequantised value formed first and then
// multiplied (ferrum_wgpu/src/shaders/quant/qlinear.wgsl:18-59). Kept as the baseline path.
//
// gemm_kernel: the scoring/prefill GEMM on the matrix cores. Per K step of one 32-element block:
//   - stage x[BM rows, 32] from HBM, split each f32 into an f16 "hi" part and an f16 "lo" part
//     (x = hi + lo to ~22 significant bits) and write both to LDS;
//   - stage W[BN rows, one block]: the integer quants, exact in f16 (Q8_0 -128..127, Q4_0 -8..7),
//     and the block's f32 scale per output column;
//   - per 32x32 output tile: P = hi * q + lo * q over the block's 32 k with
//     v_mfma_f32_32x32x16_f16 (two K=16 steps each), f32 accumulate, then acc += d[col] * P.
// The per-block scale is applied in f32 after the exact integer dot, so the product meets the
// reference's 1e-5 relative bound for linear_q (ferrum_wgpu/src/tolerance.rs:7) as well as the
// 1e-3 + 2e-3|y| GEMM bound; plain f16 or bf16 activations do not.
//
// Global->register loads of the next block overlap the MFMAs of the current one; LDS rows are
// padded to 80 bytes so the 16-byte fragment reads of 32 lanes spread over the banks.
#include "device_common.hpp"
#include "internal.hpp"

namespace fh {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
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
        const size_t blk = (size_t)c * nb + b;
        const float d = half_bits_to_float(ds[blk]);
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

// ---- MFMA GEMM ----
constexpr int kRowHalfs = 40;  // LDS row: 32 f16 + 8 f16 padding = 80 bytes

template <int KIND, int BM, int BN, int WAVES_M>
struct GemmCfg {
    static constexpr int WAVES_N = 4 / WAVES_M;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // wave tile
    static constexpr int TM = WM / 32, TN = WN / 32;             // 32x32 MFMA tiles per wave
    static constexpr int A_CHUNKS = BM * 8 / 256;                // f32x4 of x per thread per step
    static constexpr int B_ITEMS = BN * 2 / 256;                 // (column, byte half) per thread
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be whole 32x32 tiles");
    static_assert(BM * 8 % 256 == 0 && BN * 2 % 256 == 0, "staging must divide over 256 threads");
};

// One (column, byte-half bh) item of a weight block: the 16 quants it owns (elements
// 8bh..8bh+7 and 16+8bh..16+8bh+7, in the order the MFMA B operand wants them) and the scale.
template <int KIND>
struct BItem {
    uint32_t w[4];
    uint32_t h;
};

template <int KIND>
__device__ __forceinline__ void load_b(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ ds,
                                       size_t blk, int bh, BItem<KIND> &it) {
    it.h = ds[blk];
    if constexpr (KIND == FH_Q8_0) {
        // bytes 8bh..8bh+7 and 16+8bh..16+8bh+7 of the block's 32 quants
        const uint2 a = *(const uint2 *)(qs + blk * 32 + 8 * bh);
        const uint2 b = *(const uint2 *)(qs + blk * 32 + 16 + 8 * bh);
        it.w[0] = a.x; it.w[1] = a.y; it.w[2] = b.x; it.w[3] = b.y;
    } else {
        // bytes 8bh..8bh+7: low nibbles are elements 8bh.., high nibbles 16+8bh..
        const uint2 a = *(const uint2 *)(qs + blk * 16 + 8 * bh);
        it.w[0] = a.x; it.w[1] = a.y; it.w[2] = 0; it.w[3] = 0;
    }
}

// Exact small integer -> f16 (|v| <= 128).
__device__ __forceinline__ _Float16 i2h(int v) { return (_Float16)(float)v; }

template <int KIND>
__device__ __forceinline__ void unpack_b(const BItem<KIND> &it, f16x8 &lo8, f16x8 &hi8, float &d) {
    d = half_to_float(it.h);
    if constexpr (KIND == FH_Q8_0) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            lo8[e] = i2h((int8_t)(it.w[0] >> (8 * e)));
            lo8[4 + e] = i2h((int8_t)(it.w[1] >> (8 * e)));
            hi8[e] = i2h((int8_t)(it.w[2] >> (8 * e)));
            hi8[4 + e] = i2h((int8_t)(it.w[3] >> (8 * e)));
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            lo8[e] = i2h((int)((it.w[0] >> (8 * e)) & 15) - 8);
            lo8[4 + e] = i2h((int)((it.w[1] >> (8 * e)) & 15) - 8);
            hi8[e] = i2h((int)((it.w[0] >> (8 * e + 4)) & 15) - 8);
            hi8[4 + e] = i2h((int)((it.w[1] >> (8 * e + 4)) & 15) - 8);
        }
    }
}

// x = hi + lo, both f16. |x| beyond the f16 range saturates hi (documented limit: |x| < 65504).
__device__ __forceinline__ void split_f16(float v, _Float16 &hi, _Float16 &lo) {
    float c = fminf(fmaxf(v, -65504.0f), 65504.0f);
    hi = (_Float16)c;
    lo = (_Float16)(v - (float)hi);
}

template <int KIND, int BM, int BN, int WAVES_M>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const uint8_t *__restrict__ qs,
                                                      const uint16_t *__restrict__ ds,
                                                      const float *__restrict__ x,
                                                      float *__restrict__ y, uint32_t M, uint32_t K,
                                                      uint32_t N) {
    using C = GemmCfg<KIND, BM, BN, WAVES_M>;
    __shared__ __attribute__((aligned(16))) _Float16 sAh[BM * kRowHalfs];
    __shared__ __attribute__((aligned(16))) _Float16 sAl[BM * kRowHalfs];
    __shared__ __attribute__((aligned(16))) _Float16 sB[BN * kRowHalfs];
    __shared__ float sD[BN];

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const uint32_t nb = K / 32;

    f32x4 ra[C::A_CHUNKS];
    BItem<KIND> rb[C::B_ITEMS];

    auto load_step = [&](uint32_t kb) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            const int c = tid + 256 * i, r = c / 8, kc = c % 8;
            const uint32_t m = m0 + r;
            ra[i] = m < M ? *((const f32x4 *)(x + (size_t)m * K + kb * 32) + kc) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < C::B_ITEMS; i++) {
            const int it = tid + 256 * i, col = it / 2, bh = it % 2;
            const uint32_t n = n0 + col;
            if (n < N) {
                load_b<KIND>(qs, ds, (size_t)n * nb + kb, bh, rb[i]);
            } else {
                rb[i].h = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) rb[i].w[t] = 0;
            }
        }
    };

    auto store_step = [&]() {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            const int c = tid + 256 * i, r = c / 8, kc = c % 8;
            f16x4 h, l;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                _Float16 hh, ll;
                split_f16(ra[i][e], hh, ll);
                h[e] = hh;
                l[e] = ll;
            }
            *(f16x4 *)(sAh + r * kRowHalfs + 4 * kc) = h;
            *(f16x4 *)(sAl + r * kRowHalfs + 4 * kc) = l;
        }
#pragma unroll
        for (int i = 0; i < C::B_ITEMS; i++) {
            const int it = tid + 256 * i, col = it / 2, bh = it % 2;
            f16x8 lo8, hi8;
            float d;
            unpack_b<KIND>(rb[i], lo8, hi8, d);
            // k layout in LDS: [0..7] = elements 0..7, [8..15] = 8..15, [16..23] = 16..23, ...
            *(f16x8 *)(sB + col * kRowHalfs + 8 * bh) = lo8;
            *(f16x8 *)(sB + col * kRowHalfs + 16 + 8 * bh) = hi8;
            if (bh == 0) sD[col] = d;
        }
    };

    f32x16 acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int fr = lane % 32;       // fragment row (A) / column (B)
    const int fk = 8 * (lane / 32);  // first k of this lane's 8 in a K=16 step

    if (nb > 0) load_step(0);
    for (uint32_t kb = 0; kb < nb; kb++) {
        __syncthreads();  // the previous step's fragments have been read
        store_step();
        __syncthreads();
        if (kb + 1 < nb) load_step(kb + 1);  // in flight during the MFMAs below

        f16x8 bf[C::TN][2];
        float dcol[C::TN];
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int col = wn * C::WN + j * 32 + fr;
#pragma unroll
            for (int s = 0; s < 2; s++) bf[j][s] = *(const f16x8 *)(sB + col * kRowHalfs + 16 * s + fk);
            dcol[j] = sD[col];
        }
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int row = wm * C::WM + i * 32 + fr;
            f16x8 ah[2], al[2];
#pragma unroll
            for (int s = 0; s < 2; s++) {
                ah[s] = *(const f16x8 *)(sAh + row * kRowHalfs + 16 * s + fk);
                al[s] = *(const f16x8 *)(sAl + row * kRowHalfs + 16 * s + fk);
            }
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                f32x16 p = {};
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0], bf[j][0], p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1], bf[j][1], p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[0], bf[j][0], p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[1], bf[j][1], p, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = fmaf(dcol[j], p[r], acc[i][j][r]);
            }
        }
    }

    // D layout of a 32x32 tile: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const uint32_t col = n0 + wn * C::WN + j * 32 + fr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + wm * C::WM + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                if (row < M && col < N) y[(size_t)row * N + col] = acc[i][j][r];
            }
        }
}

template <int KIND, int BM, int BN, int WAVES_M>
hipError_t run_gemm(hipStream_t s, const uint8_t *qs, const uint16_t *ds, const float *x, float *y, uint32_t M,
                    uint32_t K, uint32_t N) {
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    gemm_kernel<KIND, BM, BN, WAVES_M><<<grid, 256, 0, s>>>(qs, ds, x, y, M, K, N);
    return hipGetLastError();
}

template <int KIND>
hipError_t gemm_dispatch(hipStream_t s, const uint8_t *qs, const uint16_t *ds, const float *x, float *y,
                         uint32_t M, uint32_t K, uint32_t N) {
    if (M <= 32) return run_gemm<KIND, 32, 256, 1>(s, qs, ds, x, y, M, K, N);
    if (M <= 64) return run_gemm<KIND, 64, 128, 2>(s, qs, ds, x, y, M, K, N);
    return run_gemm<KIND, 128, 128, 2>(s, qs, ds, x, y, M, K, N);
}

}  // namespace

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
                       float *y, size_t rows, size_t k, size_t n) {
    if (kind == FH_Q8_0)
        return gemm_dispatch<FH_Q8_0>(s, qs, ds, x, y, (uint32_t)rows, (uint32_t)k, (uint32_t)n);
    return gemm_dispatch<FH_Q4_0>(s, qs, ds, x, y, (uint32_t)rows, (uint32_t)k, (uint32_t)n);
}

}  // namespace fh
