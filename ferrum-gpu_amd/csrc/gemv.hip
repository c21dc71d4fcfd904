// Batch-1 GEMV on GGUF-resident Q8_0 / Q4_0 weights for gfx950: y[r] = sum_k x[k] * W[r, k],
// W kept as GGUF rows (row r = the k/32 blocks of output r, contiguous). Replaces the reference's
// per-column qgemv.wgsl (ferrum_wgpu/src/shaders/quant/qgemv.wgsl:88-115) and the single-row use
// of qlinear.wgsl; same dequantised values, different summation order (tolerance 1e-5 relative,
// ferrum_wgpu/src/tolerance.rs:7).
//
// Mapping. A wavefront works on P = 64 / SEG rows at a time; inside a row, lane j of the
// row's segment owns blocks j, j + SEG, ... (ITERS of them), so consecutive lanes read
// consecutive 34- or 18-byte blocks and a segment's loads cover one contiguous span of the row.
// Each lane keeps the 32 x values of its blocks in registers for the whole launch (they do not
// change from row to row), reads each block as an aligned dword window (blocks are only 2-byte
// aligned) and realigns the quants with one v_perm_b32 per dword. The block sum runs in f32 FMA
// over the exact integer quants and is scaled once by the block's f32 scale; the segment's
// partial sums are added with DPP row shifts and row broadcasts (no LDS, no barriers).
//
// Q4_0 sums nibble * x and subtracts 8 * sum(x) once per block (sum(x) per block is computed
// with the registers), which turns 3 VALU operations per element into 2.
//
// Work split: a task is ROWS = P * U consecutive rows; each wavefront takes one contiguous range
// of tasks, so weight bytes stream in address order. The grouped kernel runs many independent
// products (descriptors in device memory) in one launch; a wavefront finds its first product by
// binary search and then walks forward.
#include "device_common.hpp"
#include "internal.hpp"

namespace fh {
namespace {

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over each segment of SEG (32 or 64) lanes; the total lands in the segment's last lane.
template <int SEG>
__device__ __forceinline__ float seg_sum(float v) {
    v += dpp<0x111>(v);        // row_shr:1
    v += dpp<0x112>(v);        // row_shr:2
    v += dpp<0x114>(v);        // row_shr:4
    v += dpp<0x118>(v);        // row_shr:8: lane 15 of each row of 16 holds the row's sum
    v += dpp<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    if constexpr (SEG == 64) v += dpp<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

__device__ __forceinline__ float half_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int KIND, int SEG, int ITERS, int U>
struct Gemv {
    static constexpr int P = 64 / SEG;
    static constexpr int ROWS = P * U;
    static constexpr int BB = KIND == FH_Q8_0 ? 34 : 18;
    static constexpr int WORDS = KIND == FH_Q8_0 ? 9 : 5;

    float xr[ITERS][32];
    float sx[ITERS];

    __device__ __forceinline__ void load_x(const float *__restrict__ x, uint32_t nb, int lane) {
        const int j0 = lane % SEG;
#pragma unroll
        for (int i = 0; i < ITERS; i++) {
            const uint32_t j = j0 + SEG * i;
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                f32x4 v = j < nb ? *((const f32x4 *)(x + (size_t)j * 32) + c) : f32x4{0.f, 0.f, 0.f, 0.f};
                xr[i][4 * c + 0] = v.x;
                xr[i][4 * c + 1] = v.y;
                xr[i][4 * c + 2] = v.z;
                xr[i][4 * c + 3] = v.w;
                s += (v.x + v.y) + (v.z + v.w);
            }
            sx[i] = s;
        }
    }

    __device__ __forceinline__ float block_dot(const uint32_t (&w)[WORDS], uint32_t odd, int i) const {
        const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
        const float d = half_to_float(odd ? (w[0] >> 16) : (w[0] & 0xffffu));
        float a = 0.0f;
        if constexpr (KIND == FH_Q8_0) {
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const uint32_t q = __builtin_amdgcn_perm(w[c + 1], w[c], sel);
#pragma unroll
                for (int b = 0; b < 4; b++) a = fmaf(xr[i][4 * c + b], (float)(int8_t)(q >> (8 * b)), a);
            }
            return d * a;
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t q = __builtin_amdgcn_perm(w[c + 1], w[c], sel);
                const uint32_t lo = q & 0x0f0f0f0fu, hi = (q >> 4) & 0x0f0f0f0fu;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    a = fmaf(xr[i][4 * c + b], (float)((lo >> (8 * b)) & 0xffu), a);
                    a = fmaf(xr[i][16 + 4 * c + b], (float)((hi >> (8 * b)) & 0xffu), a);
                }
            }
            return d * fmaf(-8.0f, sx[i], a);
        }
    }

    // Rows row0 .. row0 + ROWS - 1 (those < n) of one product.
    __device__ __forceinline__ void task(const uint8_t *__restrict__ w, float *__restrict__ y,
                                         uint32_t nb, uint32_t n, uint32_t row0, int lane) const {
        const int s = lane / SEG, j0 = lane % SEG;
        const size_t row_bytes = (size_t)nb * BB;
        uint32_t win[U][ITERS][WORDS];
        uint32_t odd[U][ITERS];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t row = row0 + u * P + s;
#pragma unroll
            for (int i = 0; i < ITERS; i++) {
                const uint32_t j = j0 + SEG * i;
                const size_t off = (size_t)row * row_bytes + (size_t)j * BB;
                odd[u][i] = (uint32_t)off & 2u;
                if (row < n && j < nb) {
                    load_window<WORDS>(w, off, win[u][i]);
                } else {
#pragma unroll
                    for (int t = 0; t < WORDS; t++) win[u][i][t] = 0u;  // scale 0: adds nothing
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < ITERS; i++) acc += block_dot(win[u][i], odd[u][i], i);
            acc = seg_sum<SEG>(acc);
            const uint32_t row = row0 + u * P + s;
            if (j0 == SEG - 1 && row < n) y[row] = acc;
        }
    }
};

// Class of a row width in blocks: 1 = up to 32 blocks (SEG 32), 2..5 = up to 64 * (class - 1).
constexpr int kMaxClass = 5;

template <int KIND, int SEG, int ITERS, int U>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t *__restrict__ w,
                                                   const float *__restrict__ x,
                                                   float *__restrict__ y, uint32_t nb, uint32_t n,
                                                   uint32_t tasks_per_wave) {
    using G = Gemv<KIND, SEG, ITERS, U>;
    const int lane = threadIdx.x % 64;
    const uint32_t wave = blockIdx.x * 4 + threadIdx.x / 64;
    const uint32_t tasks = (n + G::ROWS - 1) / G::ROWS;
    uint32_t t = wave * tasks_per_wave;
    if (t >= tasks) return;
    const uint32_t t1 = min(tasks, t + tasks_per_wave);
    G g;
    g.load_x(x, nb, lane);
    for (; t < t1; t++) g.task(w, y, nb, n, t * G::ROWS, lane);
}

template <int KIND, int SEG, int ITERS, int U>
__global__ __launch_bounds__(256) void gemv_group_kernel(const GemvDesc *__restrict__ descs,
                                                         uint32_t count, uint32_t tasks,
                                                         uint32_t tasks_per_wave) {
    using G = Gemv<KIND, SEG, ITERS, U>;
    const int lane = threadIdx.x % 64;
    const uint32_t wave = blockIdx.x * 4 + threadIdx.x / 64;
    uint32_t t = wave * tasks_per_wave;
    if (t >= tasks) return;
    const uint32_t t1 = min(tasks, t + tasks_per_wave);
    // the last product whose first task is <= t
    uint32_t lo = 0, hi = count;
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) / 2;
        if (descs[mid].task0 <= t) lo = mid; else hi = mid;
    }
    uint32_t p = lo;
    GemvDesc d = descs[p];
    uint32_t pend = p + 1 < count ? descs[p + 1].task0 : tasks;
    G g;
    g.load_x(d.x, d.nb, lane);
    for (; t < t1; t++) {
        while (t >= pend) {  // next product (wave-uniform)
            p++;
            d = descs[p];
            pend = p + 1 < count ? descs[p + 1].task0 : tasks;
            g.load_x(d.x, d.nb, lane);
        }
        g.task(d.w, d.y, d.nb, d.n, (t - d.task0) * G::ROWS, lane);
    }
}

// Launch shapes per class: <SEG, ITERS, U>.
template <int KIND, int CLS>
struct ClassCfg;
#define FH_CLASS(CLS, SEG_, ITERS_, U_)                                   \
    template <int KIND>                                                   \
    struct ClassCfg<KIND, CLS> {                                          \
        static constexpr int SEG = SEG_, ITERS = ITERS_, U = U_;          \
        using G = Gemv<KIND, SEG_, ITERS_, U_>;                           \
    };
FH_CLASS(1, 32, 1, 4)
FH_CLASS(2, 64, 1, 4)
FH_CLASS(3, 64, 2, 2)
FH_CLASS(4, 64, 3, 2)
FH_CLASS(5, 64, 4, 1)
#undef FH_CLASS

template <int KIND, int CLS>
hipError_t launch_one(hipStream_t s, const uint8_t *w, const float *x, float *y, uint32_t nb, uint32_t n, int cus) {
    using C = ClassCfg<KIND, CLS>;
    const uint32_t tasks = (n + C::G::ROWS - 1) / C::G::ROWS;
    // as many wavefronts as tasks up to 16 per CU, then several tasks per wavefront
    const uint32_t max_waves = (uint32_t)(cus > 0 ? cus : 256) * 16;
    const uint32_t per = (tasks + max_waves - 1) / max_waves;
    const uint32_t waves = (tasks + per - 1) / per;
    gemv_kernel<KIND, C::SEG, C::ITERS, C::U><<<(waves + 3) / 4, 256, 0, s>>>(w, x, y, nb, n, per);
    return hipGetLastError();
}

template <int KIND, int CLS>
hipError_t launch_grp(hipStream_t s, const GemvDesc *descs, uint32_t count, uint32_t tasks, int cus) {
    using C = ClassCfg<KIND, CLS>;
    const uint32_t max_waves = (uint32_t)(cus > 0 ? cus : 256) * 16;
    const uint32_t per = (tasks + max_waves - 1) / max_waves;
    const uint32_t waves = (tasks + per - 1) / per;
    gemv_group_kernel<KIND, C::SEG, C::ITERS, C::U><<<(waves + 3) / 4, 256, 0, s>>>(descs, count, tasks, per);
    return hipGetLastError();
}

template <int KIND>
hipError_t dispatch_one(hipStream_t s, int cls, const uint8_t *w, const float *x, float *y, uint32_t nb,
                        uint32_t n, int cus) {
    switch (cls) {
    case 1: return launch_one<KIND, 1>(s, w, x, y, nb, n, cus);
    case 2: return launch_one<KIND, 2>(s, w, x, y, nb, n, cus);
    case 3: return launch_one<KIND, 3>(s, w, x, y, nb, n, cus);
    case 4: return launch_one<KIND, 4>(s, w, x, y, nb, n, cus);
    case 5: return launch_one<KIND, 5>(s, w, x, y, nb, n, cus);
    default: return hipErrorInvalidValue;
    }
}

template <int KIND>
hipError_t dispatch_grp(hipStream_t s, int cls, const GemvDesc *d, uint32_t count, uint32_t tasks, int cus) {
    switch (cls) {
    case 1: return launch_grp<KIND, 1>(s, d, count, tasks, cus);
    case 2: return launch_grp<KIND, 2>(s, d, count, tasks, cus);
    case 3: return launch_grp<KIND, 3>(s, d, count, tasks, cus);
    case 4: return launch_grp<KIND, 4>(s, d, count, tasks, cus);
    case 5: return launch_grp<KIND, 5>(s, d, count, tasks, cus);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int gemv_class(size_t nb) {
    if (nb == 0) return 0;
    if (nb <= 32) return 1;
    size_t c = 1 + (nb + 63) / 64;
    return c <= (size_t)kMaxClass ? (int)c : 0;
}

uint32_t gemv_tasks(int cls, size_t n) {
    const int rows = cls == 1 ? ClassCfg<FH_Q8_0, 1>::G::ROWS
                   : cls == 2 ? ClassCfg<FH_Q8_0, 2>::G::ROWS
                   : cls == 3 ? ClassCfg<FH_Q8_0, 3>::G::ROWS
                   : cls == 4 ? ClassCfg<FH_Q8_0, 4>::G::ROWS
                              : ClassCfg<FH_Q8_0, 5>::G::ROWS;
    return (uint32_t)((n + rows - 1) / rows);
}

hipError_t launch_gemv(hipStream_t s, fh_kind kind, const uint8_t *w, const float *x, float *y, size_t k,
                       size_t n, int cus) {
    const uint32_t nb = (uint32_t)(k / 32);
    const int cls = gemv_class(nb);
    if (kind == FH_Q8_0) return dispatch_one<FH_Q8_0>(s, cls, w, x, y, nb, (uint32_t)n, cus);
    return dispatch_one<FH_Q4_0>(s, cls, w, x, y, nb, (uint32_t)n, cus);
}

hipError_t launch_gemv_group(hipStream_t s, fh_kind kind, int cls, const GemvDesc *descs, uint32_t count,
                             uint32_t tasks, int cus) {
    if (count == 0 || tasks == 0) return hipSuccess;
    if (kind == FH_Q8_0) return dispatch_grp<FH_Q8_0>(s, cls, descs, count, tasks, cus);
    return dispatch_grp<FH_Q4_0>(s, cls, descs, count, tasks, cus);
}

}  // namespace fh
