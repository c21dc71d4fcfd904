// Few-row products (2 <= M <= 64) on resident Q8_0 / Q4_0 weights for gfx950: y[M, N] = x[M, K] W^T.
// Replaces the multi-row use of the reference's qlinear.wgsl / qlinear_tiled.wgsl for small row
// counts (ferrum_wgpu/src/shaders/quant/qlinear.wgsl:18-59, qlinear_tiled.wgsl:93-128; the reference
// routes them by ferrum_wgpu/src/ops/quant.rs:306-323). Same dequantised values, f32 accumulation,
// within the reference's 1e-5 (ferrum_wgpu/src/tolerance.rs:7).
//
// This regime is bound by HBM, not by the matrix cores: at M = 8 a 2048 x 2048 Q4_0 product does
// 3.5 flops per weight byte. So the weights stream once from HBM straight into registers (the
// batch-1 GEMV's 16-byte loads of whole 32-row tiles), are unpacked there into exact f16 integers,
// and meet every row of x on the f16 matrix cores; nothing is split along K, so there is no
// partial-sum pass. Many products can share one launch (a task list, as the grouped GEMV).
//
// Numerics (those of the precise GEMM): x = hi + lo, two f16 parts (22 significant bits, per
// element), written once per product by rows_split_kernel in the operand order below; the quants
// are exact f16 integers; per block and tile four v_mfma_f32_32x32x16_f16 (hi and lo, two k steps
// of 16) give the block's dot products P in f32, and acc += d * P applies the block's f32 scale.
//
// Operand order of a block's 32 elements (positions p = 16 s + 8 h + j: k step s, lane half h,
// slot j, perm = {0, 2, 1, 3, 4, 6, 5, 7}): Q4_0 element 16 s + 8 h + perm[j] (lane half h holds
// bytes 8h .. 8h + 7 of the block: low nibbles are step 0, high nibbles step 1); Q8_0 element
// 16 h + 8 s + perm[j] (lane half h holds bytes 16h .. 16h + 15, step s the 8 bytes at 16h + 8s).
// perm is the order in which a dword unpacks into f16 pairs (bytes 0 and 2, then 1 and 3).
//
// Work: a task is 128 output rows (four wavefronts x one 32-row tile) of one product over all of K,
// or over one half of K for products of 64 blocks or more, in batches of four blocks. Small tasks
// keep a launch's workgroups evenly loaded (with tasks of 256 rows over all of K, the four
// TinyLlama products at M = 8 made 840 tasks for 768 resident workgroups, and the 72 that ran a
// second task set the launch's length). The two halves of K add their partial sums atomically
// into y, zeroed by the split pass: f32 addition is commutative and the first add onto +0 is
// exact, so the result does not depend on which half arrives first. Per batch the workgroup stages x's split rows for the batch in LDS
// (double buffered, one barrier per batch) and every wavefront reads its A fragments from there,
// while its own weights for the next batch are already in flight. Workgroups loop over the tasks.
#include "device_common.hpp"
#include "internal.hpp"

namespace fh {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// blocks per batch (one LDS stage of x): eight for up to 8 rows, else four (measured: eight
// blocks take more registers, and from 16 rows on the lost occupancy costs more than the fewer
// barriers save)
__host__ __device__ constexpr int rows_kb(int R) { return R > 8 ? 4 : 8; }
constexpr int kWaves = 4;  // wavefronts per workgroup
constexpr int kXRec = 72;  // LDS halves per (x row, block): 32 hi + 32 lo + 8 pad

// A launch's row capacity R (8, 16, 32 or 64: its largest product's rows, rounded up) sets the
// 32-row x tiles (MT), the weight tiles per wavefront (TW) and the accumulator groups of four
// rows a lane keeps per tile (RG: x rows 8 g + 4 h + 0..3 for g < RG).
__host__ __device__ constexpr int rows_cap(uint32_t max_m) { return max_m <= 8 ? 8 : max_m <= 16 ? 16 : max_m <= 32 ? 32 : 64; }
__host__ __device__ constexpr int rows_mt(int R) { return R > 32 ? 2 : 1; }
__host__ __device__ constexpr int rows_tw(int) { return 1; }
// K halves of a product of nb blocks (see above)
__host__ __device__ constexpr uint32_t rows_splits(uint32_t nb) { return nb >= 64 ? 2 : 1; }
__host__ __device__ constexpr int rows_rg(int R) { return R >= 32 ? 4 : R / 8; }
constexpr int kNonTemporal = 2;

__host__ __device__ constexpr int rows_perm(int j) { return j < 4 ? (j == 1 ? 2 : j == 2 ? 1 : j) : 4 + rows_perm(j - 4); }

template <int KIND>
__host__ __device__ constexpr int rows_elem_of_pos(int p) {
    const int s = p / 16, h = (p / 8) % 2, j = p % 8;
    return KIND == FH_Q4_0 ? 16 * s + 8 * h + rows_perm(j) : 16 * h + 8 * s + rows_perm(j);
}
template <int KIND>
constexpr bool rows_order_is_a_permutation() {
    int seen = 0;
    for (int p = 0; p < 32; p++) seen |= 1 << rows_elem_of_pos<KIND>(p);
    return seen == -1;
}
static_assert(rows_order_is_a_permutation<FH_Q8_0>() && rows_order_is_a_permutation<FH_Q4_0>(),
              "the operand order must use every element of a block once");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ float half_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// A product's descriptor as wave-uniform values (every dword through readfirstlane): read from the
// launch's array or the kernel argument, it would otherwise sit in vector registers and turn every
// buffer load built from it into a loop over lanes.
__device__ __forceinline__ RowsDesc uniform_desc(const RowsDesc *descs, uint32_t p, const RowsDesc &one) {
    constexpr int W = sizeof(RowsDesc) / 4;
    static_assert(sizeof(RowsDesc) % 4 == 0, "descriptor of whole dwords");
    struct Words {
        uint32_t w[W];
    };
    Words v = __builtin_bit_cast(Words, descs ? descs[p] : one);
#pragma unroll
    for (int i = 0; i < W; i++) v.w[i] = __builtin_amdgcn_readfirstlane(v.w[i]);
    return __builtin_bit_cast(RowsDesc, v);
}

// ---- x -> (hi, lo) f16 per block in operand order: xs[m][b] = 32 hi halves, then 32 lo ----
// Eight lanes per (row, block); lane j writes positions 4j .. 4j + 3 of hi and of lo. |x| beyond
// the f16 range saturates hi (below 65504 the split is exact to about 22 bits).
template <int KIND>
__global__ __launch_bounds__(256) void rows_split_kernel(const RowsDesc *__restrict__ descs, RowsDesc one) {
    const RowsDesc d = uniform_desc(descs, blockIdx.y, one);
    const size_t items = (size_t)d.m * d.nb;
    if (rows_splits(d.nb) > 1)  // the K halves add into y
        for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < (size_t)d.m * d.n; i += (size_t)gridDim.x * 256)
            d.y[i] = 0.0f;
    const int j = threadIdx.x % 8;
    for (size_t t = ((size_t)blockIdx.x * 256 + threadIdx.x) / 8; t < items; t += (size_t)gridDim.x * 32) {
        const float *src = d.x + t * 32;
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        f16x4 hi, lo;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float e = src[rows_elem_of_pos<KIND>(4 * j + q)];
            const _Float16 h = (_Float16)fminf(fmaxf(e, -65504.0f), 65504.0f);
            hi[q] = h;
            lo[q] = (_Float16)(e - (float)h);
        }
        _Float16 *out = d.xs + t * 64;
        *(f16x4 *)(out + 4 * j) = hi;
        *(f16x4 *)(out + 32 + 4 * j) = lo;
    }
}

// ---- weight quants -> exact f16 integers in operand order ----
__device__ __forceinline__ uint32_t f16x2_add(uint32_t w, _Float16 bias) {
    const f16x2 v = __builtin_bit_cast(f16x2, w) + f16x2{bias, bias};
    return __builtin_bit_cast(uint32_t, v);
}
// (v & m) | c in one instruction (the compiler splits it in two: this target's three-operand
// encoding takes no literal constants, so m comes in a scalar register and c in a vector one)
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(m), "v"(c));
    return r;
}
// Q4_0: nibbles under the f16 exponent of 1024, minus 1032 = nibble - 8 (exact); magic holds
// 0x64006400
__device__ __forceinline__ uint32_t q4_pair(uint32_t v, uint32_t magic) {
    return f16x2_add(and_or(v, 0x000f000fu, magic), (_Float16)-1032.0f);
}
// Q8_0: bytes (0, 2) or (1, 3) of w ^ 0x80808080 under the exponent of 1024, minus 1152 = q
__device__ __forceinline__ uint32_t q8_pair(uint32_t t, uint32_t sel) {
    return f16x2_add(__builtin_amdgcn_perm(0x64646464u, t, sel), (_Float16)-1152.0f);
}

template <int KIND, int TW, int KB>
struct RowsLoad {  // one lane's weights and scales for a batch
    static constexpr int QL = KIND == FH_Q8_0 ? KB : KB / 2;  // 16-byte quant loads per tile
    u32x4 q[TW][QL];
    u32x4 d[TW];  // the lane's row's scales of the batch's blocks (KB halves) per tile
};

template <int KIND, int R>
__global__ __launch_bounds__(256, 2) void rows_kernel(const RowsDesc *__restrict__ descs,
                                                      const uint32_t *__restrict__ map, RowsDesc one,
                                                      uint32_t tasks) {
    constexpr int MT = rows_mt(R), kTW = rows_tw(R), RG = rows_rg(R), kTaskRows = 32 * kTW * kWaves;
    constexpr int kKB = rows_kb(R);
    using L = RowsLoad<KIND, kTW, kKB>;
    constexpr int QB = KIND == FH_Q8_0 ? 32 : 16;  // quant bytes per block and row
    constexpr int XCH = R * kKB * 8 / 256;          // 16-byte x chunks each thread stages per batch
    // x rows of a batch in LDS, block by block (row stride 144 bytes: the eight lanes that read
    // together hit distinct banks)
    __shared__ __attribute__((aligned(16))) _Float16 sx[2][kKB * R * kXRec];
    // the A rows past the row capacity (lanes r >= R of a single x tile) read this zero row
    __shared__ __attribute__((aligned(16))) _Float16 zrow[kXRec];

    const int tid = threadIdx.x, lane = tid % 64, r = lane % 32, h = lane / 32;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    // lane offsets: Q4_0 quants of a block pair (lane l at 16 l), Q8_0 quants of a block (row r at
    // 32 r, half h at + 16 h), scales (row r's run of eight blocks at 16 r)
    const uint32_t oq = KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * h) : (uint32_t)(lane * 16);
    const uint32_t os = (uint32_t)(r * 16);
    if (R < 32) {
        for (int i = tid; i < kXRec / 8; i += 256) *(u32x4 *)&zrow[8 * i] = u32x4{0u, 0u, 0u, 0u};
        // (the first batch's barrier orders these stores before any read)
    }
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));  // kept in a vector register for and_or

    for (uint32_t task = blockIdx.x; task < tasks; task += gridDim.x) {
        const uint32_t p = map ? map[task] : 0;
        const RowsDesc d = uniform_desc(descs, p, one);
        const uint32_t nb = d.nb, nb8 = (nb + 7) / 8, groups = (d.n + 31) / 32, S = rows_splits(nb);
        const uint32_t tl = task - d.task0, split = tl % S;
        const uint32_t g0 = (tl / S) * (kTaskRows / 32) + wave * kTW;  // this wavefront's first tile
        __amdgpu_buffer_rsrc_t rq[kTW], rd[kTW];
#pragma unroll
        for (int j = 0; j < kTW; j++) {
            const uint32_t g = g0 + j;
            const bool live = g < groups;  // a tile past the product: every load reads 0
            rq[j] = make_rsrc(d.qs + (size_t)(live ? g : 0) * nb * 32 * QB, live ? nb * 32 * QB : 0);
            rd[j] = make_rsrc(d.ds + (size_t)(live ? g : 0) * nb8 * 256, live ? nb8 * 512 : 0);
        }
        const auto rx = make_rsrc(d.xs, d.m * nb * 128);
        // this task's batches: all of them, or one half of them
        const uint32_t all_bt = (nb + kKB - 1) / kKB, half = (all_bt + S - 1) / S;
        const uint32_t bt0 = split * half, nbt = min(all_bt, bt0 + half) - bt0;

        auto load_w = [&](L &ld, uint32_t bt) {
            const uint32_t b = (bt0 + bt) * kKB;
#pragma unroll
            for (int j = 0; j < kTW; j++) {
#pragma unroll
                for (int i = 0; i < L::QL; i++) {
                    const uint32_t off = KIND == FH_Q8_0 ? oq + (b + i) * 1024 : oq + (b + 2 * i) * 512;
                    ld.q[j][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq[j], (int)off, 0, kNonTemporal));
                }
                const uint32_t so = os + (b / 8) * 512 + (b % 8) * 2;
                if constexpr (kKB == 8) {
                    ld.d[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rd[j], (int)so, 0, 0));
                } else {
                    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rd[j], (int)so, 0, 0));
                    ld.d[j] = u32x4{v[0], v[1], 0u, 0u};
                }
            }
        };
        // x chunks of a batch: chunk c = tid + 256 i is block c / (8 R), row (c / 8) % R, part c % 8
        u32x4 xr[XCH];
        auto load_x = [&](uint32_t bt) {
#pragma unroll
            for (int i = 0; i < XCH; i++) {
                const uint32_t c = tid + 256 * i, m = (c / 8) % R, kb = (bt0 + bt) * kKB + c / (8 * R);
                const bool ok = m < d.m && kb < nb;
                xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rx, (int)(ok ? (m * nb + kb) * 128 + (c % 8) * 16 : 0x80000000u), 0, 0));
            }
        };
        auto store_x = [&](int buf) {
#pragma unroll
            for (int i = 0; i < XCH; i++) {
                const uint32_t c = tid + 256 * i;
                *(u32x4 *)&sx[buf][(c / 8) * kXRec + (c % 8) * 8] = xr[i];
            }
        };

        // accumulators: tile (i, j), group g of four x rows (8 g + 4 h + 0..3 of x tile i)
        f32x4 acc[MT][kTW][4];
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int j = 0; j < kTW; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) acc[i][j][q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        constexpr int G0 = RG;  // groups kept in x tile 0 (tile 1, when there is one, keeps all four)

        auto compute = [&](const L &ld, int buf) {
            decltype(__builtin_amdgcn_permlane32_swap(0u, 0u, false, false)) sw0[kTW], sw1[kTW];  // Q4_0 pair swaps
#pragma unroll
            for (int kb = 0; kb < kKB; kb++) {
                // B fragments: step 0 and step 1 of block kb for each tile
                f16x8 bf[kTW][2];
                float dv[kTW];
#pragma unroll
                for (int j = 0; j < kTW; j++) {
                    u32x4 b0, b1;
                    if constexpr (KIND == FH_Q8_0) {
                        const u32x4 q = ld.q[j][kb];
                        const uint32_t t0 = q[0] ^ 0x80808080u, t1 = q[1] ^ 0x80808080u, t2 = q[2] ^ 0x80808080u,
                                       t3 = q[3] ^ 0x80808080u;
                        b0 = u32x4{q8_pair(t0, 0x04020400u), q8_pair(t0, 0x04030401u), q8_pair(t1, 0x04020400u),
                                   q8_pair(t1, 0x04030401u)};
                        b1 = u32x4{q8_pair(t2, 0x04020400u), q8_pair(t2, 0x04030401u), q8_pair(t3, 0x04020400u),
                                   q8_pair(t3, 0x04030401u)};
                    } else {
                        // lane r holds block 2i of row r, lane 32 + r block 2i + 1; swapping the
                        // upper lanes' dwords 0, 1 with the lower lanes' 2, 3 gives each lane half h
                        // bytes 8h .. 8h + 7 of both blocks (one swap serves the pair)
                        if (kb % 2 == 0) {
                            const u32x4 q = ld.q[j][kb / 2];
                            sw0[j] = __builtin_amdgcn_permlane32_swap(q[0], q[2], false, false);
                            sw1[j] = __builtin_amdgcn_permlane32_swap(q[1], q[3], false, false);
                        }
                        const uint32_t w0 = kb % 2 ? sw0[j][1] : sw0[j][0], w1 = kb % 2 ? sw1[j][1] : sw1[j][0];
                        b0 = u32x4{q4_pair(w0, magic), q4_pair(w0 >> 8, magic), q4_pair(w1, magic), q4_pair(w1 >> 8, magic)};
                        b1 = u32x4{q4_pair(w0 >> 4, magic), q4_pair(w0 >> 12, magic), q4_pair(w1 >> 4, magic),
                                   q4_pair(w1 >> 12, magic)};
                    }
                    bf[j][0] = __builtin_bit_cast(f16x8, b0);
                    bf[j][1] = __builtin_bit_cast(f16x8, b1);
                    dv[j] = half_to_float(ld.d[j][kb / 2] >> (16 * (kb % 2)));
                }
                if constexpr (R <= 16) {
                    // Up to 16 rows: A rows 0..R-1 are x's hi parts and rows R..2R-1 its lo parts
                    // (rows past 2R zero), so one MFMA per k step covers both parts: C register
                    // 4g + q of lane (column, h) is hi of x row 8g + 4h + q and register
                    // 4g + q + R / 2 its lo, added before the block's scale. Two MFMAs per block
                    // instead of four.
                    const _Float16 *row = r < 2 * R ? &sx[buf][(kb * R + r % R) * kXRec] + (r < R ? 0 : 32) : zrow;
                    const f16x8 a0 = *(const f16x8 *)(row + 8 * h);
                    const f16x8 a1 = *(const f16x8 *)(row + 16 + 8 * h);
#pragma unroll
                    for (int j = 0; j < kTW; j++) {
                        f32x16 pp = {};
                        pp = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bf[j][0], pp, 0, 0, 0);
                        pp = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bf[j][1], pp, 0, 0, 0);
#pragma unroll
                        for (int g = 0; g < G0; g++)
#pragma unroll
                            for (int q = 0; q < 4; q++)
                                acc[0][j][g][q] = fmaf(dv[j], pp[4 * g + q] + pp[4 * g + q + R / 2], acc[0][j][g][q]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < MT; i++) {
                        // A fragments: x row i 32 + r (rows past the row capacity are zero)
                        const int xr_row = i * 32 + r;
                        const _Float16 *row = (R >= 32 || xr_row < R) ? &sx[buf][(kb * R + xr_row) * kXRec] : zrow;
                        const f16x8 a0 = *(const f16x8 *)(row + 8 * h);
                        const f16x8 a1 = *(const f16x8 *)(row + 16 + 8 * h);
                        const f16x8 l0 = *(const f16x8 *)(row + 32 + 8 * h);
                        const f16x8 l1 = *(const f16x8 *)(row + 48 + 8 * h);
#pragma unroll
                        for (int j = 0; j < kTW; j++) {
                            f32x16 pp = {};
                            pp = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bf[j][0], pp, 0, 0, 0);
                            pp = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bf[j][1], pp, 0, 0, 0);
                            pp = __builtin_amdgcn_mfma_f32_32x32x16_f16(l0, bf[j][0], pp, 0, 0, 0);
                            pp = __builtin_amdgcn_mfma_f32_32x32x16_f16(l1, bf[j][1], pp, 0, 0, 0);
#pragma unroll
                            for (int g = 0; g < (i == 0 ? G0 : 4); g++)
#pragma unroll
                                for (int q = 0; q < 4; q++)
                                    acc[i][j][g][q] = fmaf(dv[j], pp[4 * g + q], acc[i][j][g][q]);
                        }
                    }
                }
                // one block at a time: the scale FMAs are not sunk past the next block's MFMAs
                // (which would keep every block's products live)
#pragma unroll
                for (int i = 0; i < MT; i++)
#pragma unroll
                    for (int j = 0; j < kTW; j++)
#pragma unroll
                        for (int g = 0; g < (i == 0 ? G0 : 4); g++) asm volatile("" : "+v"(acc[i][j][g]));
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // x of the next batch is requested before its weights: loads complete in order, so the LDS
        // store of x waits only for x, and the weights stay in flight across the barrier until the
        // batch is computed
        L w0, w1;
        load_x(0);
        load_w(w0, 0);
        store_x(0);
        __syncthreads();
        for (uint32_t bt = 0; bt < nbt; bt += 2) {
            const bool m1 = bt + 1 < nbt;
            if (m1) {
                load_x(bt + 1);
                load_w(w1, bt + 1);
            }
            compute(w0, 0);
            if (m1) store_x(1);
            __syncthreads();
            if (!m1) break;
            const bool m2 = bt + 2 < nbt;
            if (m2) {
                load_x(bt + 2);
                load_w(w0, bt + 2);
            }
            compute(w1, 1);
            if (m2) store_x(0);
            __syncthreads();
        }

        // C layout of a 32 x 32 tile: register q of lane l is x row 8 (q / 4) + 4 (l / 32) + q % 4,
        // output row l % 32 of the tile
        typedef __attribute__((address_space(1))) float gfloat;
#pragma unroll
        for (int j = 0; j < kTW; j++) {
            const uint32_t n = (g0 + j) * 32 + r;
            if (n >= d.n) continue;
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int g = 0; g < (i == 0 ? G0 : 4); g++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const uint32_t m = i * 32 + 8 * g + 4 * h + q;
                        if (m >= d.m) continue;
                        if (S > 1)
                            unsafeAtomicAdd(d.y + (size_t)m * d.n + n, acc[i][j][g][q]);
                        else
                            ((gfloat *)d.y)[(size_t)m * d.n + n] = acc[i][j][g][q];
                    }
        }
    }
}

template <int KIND, int R>
int rows_resident_groups() {
    static int b = 0;
    if (b == 0 && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, rows_kernel<KIND, R>, 256, 0) != hipSuccess || b < 1))
        b = 1;
    return b;
}

template <int KIND, int R>
hipError_t launch_rows_kind(hipStream_t s, const RowsDesc *descs, const uint32_t *map, const RowsDesc &one,
                            uint32_t count, uint32_t tasks, uint32_t max_items, int cus) {
    const uint32_t gx = (max_items + 31) / 32;
    rows_split_kernel<KIND><<<dim3(gx < 8192 ? gx : 8192, count), 256, 0, s>>>(descs, one);
    const uint32_t slots = (uint32_t)(cus > 0 ? cus : 256) * (uint32_t)rows_resident_groups<KIND, R>();
    rows_kernel<KIND, R><<<tasks < slots ? tasks : slots, 256, 0, s>>>(descs, map, one, tasks);
    return hipGetLastError();
}

template <int KIND>
hipError_t launch_rows_mt(hipStream_t s, const RowsDesc *descs, const uint32_t *map, const RowsDesc &one,
                          uint32_t count, uint32_t tasks, uint32_t max_m, uint32_t max_items, int cus) {
    switch (rows_cap(max_m)) {
    case 8: return launch_rows_kind<KIND, 8>(s, descs, map, one, count, tasks, max_items, cus);
    case 16: return launch_rows_kind<KIND, 16>(s, descs, map, one, count, tasks, max_items, cus);
    case 32: return launch_rows_kind<KIND, 32>(s, descs, map, one, count, tasks, max_items, cus);
    default: return launch_rows_kind<KIND, 64>(s, descs, map, one, count, tasks, max_items, cus);
    }
}

}  // namespace

bool rows_supported(size_t rows, size_t k, size_t n) {
    // every buffer offset (x split, a tile's quants and scales) stays below 2^31
    const size_t nb = k / 32;
    return rows >= 1 && rows <= kRowsMax && nb > 0 && rows * nb * 128 < ((size_t)1 << 31) &&
           nb * 32 * 32 < ((size_t)1 << 31) && (n + 31) / 32 * 32 <= ((size_t)1 << 30);
}

size_t rows_xsplit_bytes(size_t rows, size_t k) { return rows * (k / 32) * 128; }

uint32_t rows_tasks(size_t n, size_t k, size_t max_m) {
    const size_t task_rows = 32 * rows_tw(rows_cap((uint32_t)max_m)) * kWaves;
    return (uint32_t)((n + task_rows - 1) / task_rows * rows_splits((uint32_t)(k / 32)));
}

hipError_t launch_rows(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x, float *y,
                       size_t rows, size_t k, size_t n, void *xsplit, int cus) {
    const RowsDesc one{qs, ds, x, (_Float16 *)xsplit, y, (uint32_t)(k / 32), (uint32_t)n, (uint32_t)rows, 0};
    const uint32_t items = (uint32_t)(rows * (k / 32));
    const uint32_t tasks = rows_tasks(n, k, rows);
    if (kind == FH_Q8_0) return launch_rows_mt<FH_Q8_0>(s, nullptr, nullptr, one, 1, tasks, (uint32_t)rows, items, cus);
    return launch_rows_mt<FH_Q4_0>(s, nullptr, nullptr, one, 1, tasks, (uint32_t)rows, items, cus);
}

hipError_t launch_rows_group(hipStream_t s, fh_kind kind, const RowsDesc *descs, const uint32_t *map, uint32_t count,
                             uint32_t tasks, uint32_t max_m, uint32_t max_items, int cus) {
    if (count == 0 || tasks == 0) return hipSuccess;
    const RowsDesc none{};
    if (kind == FH_Q8_0) return launch_rows_mt<FH_Q8_0>(s, descs, map, none, count, tasks, max_m, max_items, cus);
    return launch_rows_mt<FH_Q4_0>(s, descs, map, none, count, tasks, max_m, max_items, cus);
}

}  // namespace fh
