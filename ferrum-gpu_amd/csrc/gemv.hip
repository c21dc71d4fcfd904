// Batch-1 GEMV on resident Q8_0 / Q4_0 weights for gfx950: y[r] = sum_k x[k] * W[r, k].
// Replaces the reference's per-column qgemv.wgsl (ferrum_wgpu/src/shaders/quant/qgemv.wgsl:88-115)
// and the single-row use of qlinear.wgsl; same dequantised values, different summation order
// (tolerance 1e-5 relative, ferrum_wgpu/src/tolerance.rs:7).
//
// Resident layout (the "planes" a weight is repacked into at upload; same bytes as GGUF): row r
// of the weight is nb = k/32 blocks. Its quants are nb * QB contiguous bytes at
// qs + r * nb * QB (QB = 16 for Q4_0, 32 for Q8_0: the GGUF block without its scale) and its f16
// scales are nb contiguous halves at ds + r * nb. A "chunk" is 16 quant bytes: for Q4_0 one
// whole block (bytes j hold element j in the low nibble and j + 16 in the high one), for Q8_0
// half a block (elements 16h .. 16h + 15).
//
// Mapping. A wavefront works on P = 64 / SEG rows at a time; lane j of a row's segment owns
// chunks j, j + SEG, ... (ITERS of them), so each load instruction of a segment reads SEG * 16
// contiguous bytes (global_load_dwordx4, non-temporal: the weights stream through once). The
// lane keeps the x values of its chunks in registers for the whole launch (they are the same
// for every row), converts the quants in registers (v_cvt_f32_ubyteN on the masked nibbles;
// v_cvt_f32_i32 with a sign-extending byte select for Q8_0), sums x * q with f32 FMA, and scales
// the chunk sum once by the block's scale. Segment partial sums are added with DPP row shifts
// and row broadcasts (no LDS, no barriers). A task is U row groups; the next task's loads are
// issued before the current task is computed, so up to 2 * U * ITERS 16-byte loads per lane are
// in flight.
//
// Q4_0 sums nibble * x and subtracts 8 * sum(x) once per chunk (sum(x) per chunk is computed
// once with the registers), so an element costs one convert and one FMA.
//
// One kernel serves single products (descriptor passed by value) and grouped launches (many
// independent products, descriptors in device memory, each wavefront finds its first product by
// binary search). Each wavefront takes a contiguous range of row tasks, so it streams its
// weight bytes in address order.
#include <cstdlib>

#include "device_common.hpp"
#include "internal.hpp"

namespace fh {
namespace {

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over each segment of SEG (8, 16, 32 or 64) lanes; the total lands in the segment's last
// lane (lanes that receive no DPP source add the old value 0).
template <int SEG>
__device__ __forceinline__ float seg_sum(float v) {
    v += dpp<0x111>(v);  // row_shr:1
    v += dpp<0x112>(v);  // row_shr:2
    v += dpp<0x114>(v);  // row_shr:4: lane 8i + 7 holds the sum of its 8 lanes
    if constexpr (SEG >= 16) v += dpp<0x118>(v);       // row_shr:8: lane 15 of each row of 16
    if constexpr (SEG >= 32) v += dpp<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    if constexpr (SEG == 64) v += dpp<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

__device__ __forceinline__ float half_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Pointers read from descriptors are generic; in the global address space the loads are
// global_load (counted by vmcnt only) rather than flat_load (vmcnt and lgkmcnt), so waiting for
// one batch does not wait for the next.
template <class T>
using gptr = __attribute__((address_space(1))) T *;
template <class T>
__device__ __forceinline__ gptr<const T> glob(const T *p) {
    return (gptr<const T>)p;
}
template <class T>
__device__ __forceinline__ gptr<T> glob(T *p) {
    return (gptr<T>)p;
}

template <int KIND>
struct QF;
template <>
struct QF<FH_Q4_0> {
    static constexpr int CPB = 1;   // chunks per block
    static constexpr int XPC = 32;  // x values per chunk
};
template <>
struct QF<FH_Q8_0> {
    static constexpr int CPB = 2;
    static constexpr int XPC = 16;
};

// Row groups per task: with two tasks in flight, U * ITERS * 2 16-byte loads per lane.
constexpr int unroll_for(int iters) { return iters == 1 ? 4 : iters == 2 ? 2 : 1; }

// The x side of a lane: what it keeps in registers for its ITERS chunks, and the dot product of
// one 16-byte chunk of quants with it.
template <int KIND, int ITERS>
struct XState;

// Q8_0: the 16 f32 x values of each chunk; f32 FMA over exact integer quants (v_cvt_f32_i32 with
// a sign-extending byte select), one scale multiply per chunk.
template <int ITERS>
struct XState<FH_Q8_0, ITERS> {
    float xr[ITERS][16];

    __device__ __forceinline__ void load(const float *__restrict__ x, uint32_t nch, int j0, int seg) {
#pragma unroll
        for (int i = 0; i < ITERS; i++) {
            const uint32_t j = j0 + seg * i;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                f32x4 v = j < nch ? glob((const f32x4 *)(x + (size_t)j * 16))[c] : f32x4{0.f, 0.f, 0.f, 0.f};
                xr[i][4 * c + 0] = v.x;
                xr[i][4 * c + 1] = v.y;
                xr[i][4 * c + 2] = v.z;
                xr[i][4 * c + 3] = v.w;
            }
        }
    }

    __device__ __forceinline__ float dot(const u32x4 q, float d, int i) const {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const float qv = (float)(int32_t)(int8_t)(q[c] >> (8 * b));
                if (c & 1)
                    a1 = fmaf(xr[i][4 * c + b], qv, a1);
                else
                    a0 = fmaf(xr[i][4 * c + b], qv, a0);
            }
        }
        return d * (a0 + a1);
    }
};

// Q4_0: x on a per-chunk fixed-point grid, as three signed 8-bit limbs, and exact integer dot
// products with v_dot4_i32_i8. With amax the chunk's largest |x| and 2^(E-1) <= amax < 2^E,
// xi = rint(x * 2^(22-E)) (|xi| <= 2^22, error <= 2^-22 amax per element, the grid an f32 sum of
// the chunk would round to) and xi = a * 2^16 + b * 2^8 + c with a, b, c in [-128, 127]. Per
// chunk, S_l = sum(nibble * limb_l) - 8 * sum(limb_l) is exact in int32, and
// d * (S_a * 2^16 + S_b * 2^8 + S_c) * 2^(E-22) is the chunk's contribution, formed in f32. A
// chunk with a non-finite x contributes NaN; one whose amax is below 2^-103 contributes 0.
template <int ITERS>
struct XState<FH_Q4_0, ITERS> {
    uint32_t lo[ITERS][3][4];  // limbs of elements 4c..4c+3 (low nibbles), packed 4 per dword
    uint32_t hi[ITERS][3][4];  // limbs of elements 16+4c..16+4c+3 (high nibbles)
    int32_t bias[ITERS][3];    // -8 * sum of each limb over the chunk
    float xs[ITERS];           // 2^(E-22), 0 for a zero chunk, NaN for a non-finite one

    __device__ __forceinline__ static void limbs(float x, float m, int32_t &a, int32_t &b, int32_t &c) {
        const int32_t xi = (int32_t)rintf(x * m);
        c = (xi << 24) >> 24;
        const int32_t r = (xi - c) >> 8;
        b = (r << 24) >> 24;
        a = (r - b) >> 8;
    }

    __device__ __forceinline__ void load(const float *__restrict__ x, uint32_t nch, int j0, int seg) {
#pragma unroll
        for (int i = 0; i < ITERS; i++) {
            const uint32_t j = j0 + seg * i;
            float v[32];
#pragma unroll
            for (int c = 0; c < 8; c++) {
                f32x4 t = j < nch ? glob((const f32x4 *)(x + (size_t)j * 32))[c] : f32x4{0.f, 0.f, 0.f, 0.f};
                v[4 * c + 0] = t.x;
                v[4 * c + 1] = t.y;
                v[4 * c + 2] = t.z;
                v[4 * c + 3] = t.w;
            }
            float amax = 0.0f;
            bool finite = true;
#pragma unroll
            for (int e = 0; e < 32; e++) {
                amax = fmaxf(amax, fabsf(v[e]));
                finite = finite && (fabsf(v[e]) <= 3.4028235e38f);  // false for inf and NaN
            }
            const uint32_t eb = __float_as_uint(amax) >> 23;  // biased exponent of amax
            const bool zero = eb < 24;                         // amax < 2^-103 (or 0)
            const float m = zero ? 0.0f : __uint_as_float((275u - min(eb, 254u)) << 23);  // 2^(148-eb)
            xs[i] = !finite ? __builtin_nanf("") : zero ? 0.0f : __uint_as_float((eb - 21u) << 23);
            int32_t sa = 0, sb = 0, sc = 0;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                uint32_t la = 0, lb = 0, lc = 0, ha = 0, hb = 0, hc = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    int32_t a0, b0, c0, a1, b1, c1;
                    limbs(finite ? v[4 * c + b] : 0.0f, m, a0, b0, c0);
                    limbs(finite ? v[16 + 4 * c + b] : 0.0f, m, a1, b1, c1);
                    la |= (uint32_t)(a0 & 0xff) << (8 * b);
                    lb |= (uint32_t)(b0 & 0xff) << (8 * b);
                    lc |= (uint32_t)(c0 & 0xff) << (8 * b);
                    ha |= (uint32_t)(a1 & 0xff) << (8 * b);
                    hb |= (uint32_t)(b1 & 0xff) << (8 * b);
                    hc |= (uint32_t)(c1 & 0xff) << (8 * b);
                    sa += a0 + a1;
                    sb += b0 + b1;
                    sc += c0 + c1;
                }
                lo[i][0][c] = la; lo[i][1][c] = lb; lo[i][2][c] = lc;
                hi[i][0][c] = ha; hi[i][1][c] = hb; hi[i][2][c] = hc;
            }
            bias[i][0] = -8 * sa;
            bias[i][1] = -8 * sb;
            bias[i][2] = -8 * sc;
        }
    }

    __device__ __forceinline__ float dot(const u32x4 q, float d, int i) const {
        int32_t s0 = bias[i][0], s1 = bias[i][1], s2 = bias[i][2];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int32_t nl = (int32_t)(q[c] & 0x0f0f0f0fu);
            const int32_t nh = (int32_t)((q[c] >> 4) & 0x0f0f0f0fu);
            s0 = __builtin_amdgcn_sdot4(nl, (int32_t)lo[i][0][c], s0, false);
            s1 = __builtin_amdgcn_sdot4(nl, (int32_t)lo[i][1][c], s1, false);
            s2 = __builtin_amdgcn_sdot4(nl, (int32_t)lo[i][2][c], s2, false);
            s0 = __builtin_amdgcn_sdot4(nh, (int32_t)hi[i][0][c], s0, false);
            s1 = __builtin_amdgcn_sdot4(nh, (int32_t)hi[i][1][c], s1, false);
            s2 = __builtin_amdgcn_sdot4(nh, (int32_t)hi[i][2][c], s2, false);
        }
        const float f = fmaf((float)s0, 65536.0f, fmaf((float)s1, 256.0f, (float)s2));
        return (d * f) * xs[i];
    }
};

// A raw buffer resource over [base, base + bytes): loads at offsets at or past `bytes` return 0
// (gfx9 descriptor word 3 = 0x00020000, 32-bit data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
constexpr int kNonTemporal = 2;  // cache-policy bit of a streaming load

template <int KIND, int SEG, int ITERS>
struct Gemv {
    static constexpr int P = 64 / SEG;
    static constexpr int U = unroll_for(ITERS);
    static constexpr int ROWS = P * U;
    static constexpr int CPB = QF<KIND>::CPB;

    // Per-lane byte offsets, relative to a task's first row, of the quant chunks and scales the
    // lane loads (they depend only on the product's row width).
    struct Offsets {
        uint32_t voq[U][ITERS], vod[U][ITERS];

        __device__ __forceinline__ void set(const GemvDesc &d, int lane) {
            const uint32_t nch = d.nb * CPB;
            const int s = lane / SEG, j0 = lane % SEG;
#pragma unroll
            for (int i = 0; i < ITERS; i++) {
                const uint32_t j = j0 + SEG * i;
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const uint32_t r = s + u * P;
                    voq[u][i] = (r * nch + j) * 16u;
                    vod[u][i] = (r * d.nb + j / CPB) * 2u;
                }
            }
        }
    };

    XState<KIND, ITERS> xv;
    uint32_t keep[ITERS];  // 0xffff for a chunk inside the row, 0 for an idle lane (scale 0)

    // Set up the lane for the product it computes next: its x, and which of its chunks exist.
    __device__ __forceinline__ void begin(const GemvDesc &d, int lane) {
        const uint32_t nch = d.nb * CPB;
        xv.load(d.x, nch, lane % SEG, SEG);
#pragma unroll
        for (int i = 0; i < ITERS; i++) keep[i] = (uint32_t)(lane % SEG + SEG * i) < nch ? 0xffffu : 0u;
    }

    // The weight bytes of one task: rows row0 .. row0 + ROWS - 1 of the product. The buffer
    // ranges end at the product's last row, so rows past it load 0 (scale 0: they add nothing);
    // row0 == n gives empty ranges, loads that return 0 without touching memory.
    struct Batch {
        u32x4 q[U][ITERS];
        uint32_t h[U][ITERS];
    };

    __device__ __forceinline__ static void load(Batch &bt, const GemvDesc &d, uint32_t row0, const Offsets &o) {
        const uint32_t nch = d.nb * CPB;
        const uint32_t left = d.n - row0;
        const __amdgpu_buffer_rsrc_t rq = make_rsrc(d.qs + (size_t)row0 * nch * 16, left * nch * 16);
        const __amdgpu_buffer_rsrc_t rd = make_rsrc(d.ds + (size_t)row0 * d.nb, left * d.nb * 2);
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int i = 0; i < ITERS; i++) {
                bt.q[u][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)o.voq[u][i], 0, kNonTemporal));
                bt.h[u][i] = __builtin_amdgcn_raw_buffer_load_b16(rd, (int)o.vod[u][i], 0, 0);
            }
    }

    __device__ __forceinline__ void compute(const Batch &bt, float *__restrict__ y, uint32_t n, uint32_t row0,
                                            int lane) const {
        const int s = lane / SEG, j0 = lane % SEG;
#pragma unroll
        for (int u = 0; u < U; u++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < ITERS; i++) acc += xv.dot(bt.q[u][i], half_to_float(bt.h[u][i] & keep[i]), i);
            acc = seg_sum<SEG>(acc);
            const uint32_t row = row0 + u * P + s;
            if (j0 == SEG - 1 && row < n) glob(y)[row] = acc;
        }
    }
};

// Walks the products of a launch in task order (wave-uniform state).
struct Cursor {
    const GemvDesc *descs;
    uint32_t count, tasks;
    uint32_t p, pend;
    GemvDesc d;

    __device__ __forceinline__ void seek(uint32_t t, const GemvDesc &one) {
        p = 0;
        if (descs) {  // the last product whose first task is <= t
            uint32_t lo = 0, hi = count;
            while (hi - lo > 1) {
                const uint32_t mid = (lo + hi) / 2;
                if (descs[mid].task0 <= t) lo = mid; else hi = mid;
            }
            p = lo;
        }
        d = descs ? descs[p] : one;
        pend = p + 1 < count ? descs[p + 1].task0 : tasks;
    }
    // Advance to the product holding task t (t never decreases); true when it changed.
    __device__ __forceinline__ bool advance(uint32_t t) {
        bool moved = false;
        while (t >= pend) {
            p++;
            d = descs[p];
            pend = p + 1 < count ? descs[p + 1].task0 : tasks;
            moved = true;
        }
        return moved;
    }
};

// One launch: `count` products. count == 1 with descs == nullptr reads the product from `one`.
// Software-pipelined: the weight bytes of the wavefront's next task are in flight while the
// current task is computed (two register batches, used alternately).
template <int KIND, int SEG, int ITERS>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvDesc *__restrict__ descs, GemvDesc one,
                                                   uint32_t count, uint32_t tasks, uint32_t tasks_per_wave) {
    using G = Gemv<KIND, SEG, ITERS>;
    const int lane = threadIdx.x % 64;
    // wave-uniform (readfirstlane), so descriptor reads are scalar loads: a vector-memory wait
    // for them would also wait for the weight loads already in flight
    const uint32_t wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    uint32_t t = wave * tasks_per_wave;
    if (t >= tasks) return;
    const uint32_t t1 = min(tasks, t + tasks_per_wave);
    Cursor cl{descs, count, tasks, 0, 0, {}};  // product of the batch being loaded
    cl.seek(t, one);
    Cursor cc = cl;                            // product of the batch being computed
    G g;
    g.begin(cc.d, lane);
    typename G::Offsets lo;                    // load offsets, for cl's product
    lo.set(cl.d, lane);
    typename G::Batch b0, b1;
    G::load(b0, cl.d, (t - cl.d.task0) * G::ROWS, lo);
    // Each step: the lane set-up for the task about to be computed (only when its product
    // changed), then the next task's weights, then the current task's arithmetic. The prefetch is
    // issued on every step (past the wavefront's last task it reads an empty range), so the wait
    // before the arithmetic is the same on every path: it covers only the loads issued before the
    // prefetch.
    for (;;) {
        // b0 holds task t
        if (cc.advance(t)) g.begin(cc.d, lane);
        {
            const bool more = t + 1 < t1;
            if (more && cl.advance(t + 1)) lo.set(cl.d, lane);
            G::load(b1, cl.d, more ? (t + 1 - cl.d.task0) * G::ROWS : cl.d.n, lo);
        }
        g.compute(b0, cc.d.y, cc.d.n, (t - cc.d.task0) * G::ROWS, lane);
        if (++t >= t1) break;
        // b1 holds task t
        if (cc.advance(t)) g.begin(cc.d, lane);
        {
            const bool more = t + 1 < t1;
            if (more && cl.advance(t + 1)) lo.set(cl.d, lane);
            G::load(b0, cl.d, more ? (t + 1 - cl.d.task0) * G::ROWS : cl.d.n, lo);
        }
        g.compute(b1, cc.d.y, cc.d.n, (t - cc.d.task0) * G::ROWS, lane);
        if (++t >= t1) break;
    }
}

// The launch shapes, (SEG, ITERS): a row of nch chunks fits when SEG * ITERS >= nch.
#define FH_GEMV_SHAPES(X)                                                                      \
    X(0, 8, 1) X(1, 8, 2) X(2, 8, 3) X(3, 8, 4) X(4, 16, 1) X(5, 16, 2) X(6, 16, 3) X(7, 16, 4) \
    X(8, 32, 1) X(9, 32, 2) X(10, 32, 3) X(11, 32, 4) X(12, 64, 1) X(13, 64, 2) X(14, 64, 3)   \
    X(15, 64, 4) X(16, 64, 5) X(17, 64, 6) X(18, 64, 7) X(19, 64, 8)

struct Shape {
    int seg, iters;
};
constexpr Shape kShapes[] = {
#define FH_X(I, S, N) {S, N},
    FH_GEMV_SHAPES(FH_X)
#undef FH_X
};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);

constexpr int rows_per_task(int shape) { return (64 / kShapes[shape].seg) * unroll_for(kShapes[shape].iters); }

int xpc(fh_kind kind) { return kind == FH_Q8_0 ? 16 : 32; }

// Wavefronts per CU a launch aims for, at most what fits (FERRUM_HIP_GEMV_WAVES_PER_CU overrides,
// 1..32). Fewer, longer-running wavefronts each stream a longer contiguous span of weight bytes.
uint32_t waves_per_cu() {
    static const uint32_t w = [] {
        const char *e = getenv("FERRUM_HIP_GEMV_WAVES_PER_CU");
        const long v = e ? strtol(e, nullptr, 10) : 0;
        return (uint32_t)(v >= 1 && v <= 32 ? v : 32);
    }();
    return w;
}

template <int KIND, int SEG, int ITERS>
hipError_t launch_shape(hipStream_t s, const GemvDesc *descs, const GemvDesc &one, uint32_t count,
                        uint32_t tasks, int cus) {
    if constexpr (ITERS * QF<KIND>::XPC > 128) {
        return hipErrorInvalidValue;  // never chosen: more x registers than the kernel keeps
    } else {
        // As many wavefronts as fit on the chip at once (from the kernel's register use) or as
        // the requested per-CU count allows, whichever is fewer; each takes an equal share of
        // the tasks, so no wavefront waits for a second round.
        static const int resident = [] {
            int blocks = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, gemv_kernel<KIND, SEG, ITERS>, 256, 0) !=
                    hipSuccess ||
                blocks < 1)
                blocks = 1;
            return blocks * 4;  // wavefronts per CU
        }();
        const uint32_t per_cu = min((uint32_t)resident, waves_per_cu());
        const uint32_t max_waves = (uint32_t)(cus > 0 ? cus : 256) * per_cu;
        const uint32_t per = (tasks + max_waves - 1) / max_waves;
        const uint32_t waves = (tasks + per - 1) / per;
        gemv_kernel<KIND, SEG, ITERS><<<(waves + 3) / 4, 256, 0, s>>>(descs, one, count, tasks, per);
        return hipGetLastError();
    }
}

template <int KIND>
hipError_t dispatch(hipStream_t s, int shape, const GemvDesc *descs, const GemvDesc &one, uint32_t count,
                    uint32_t tasks, int cus) {
    switch (shape) {
#define FH_X(I, S, N) \
    case I: return launch_shape<KIND, S, N>(s, descs, one, count, tasks, cus);
        FH_GEMV_SHAPES(FH_X)
#undef FH_X
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int gemv_shape(fh_kind kind, size_t nb, size_t n) {
    const size_t nch = nb * (kind == FH_Q8_0 ? 2 : 1);
    if (n * nch * 16 >= (1ull << 31)) return -1;  // buffer offsets are 32-bit
    int best = -1;
    for (int i = 0; i < kNumShapes; i++) {
        const size_t cap = (size_t)kShapes[i].seg * kShapes[i].iters;
        if (cap < nch || kShapes[i].iters * xpc(kind) > 128) continue;
        // least idle lanes; then the wider segment (fewer x registers per lane)
        if (best < 0) { best = i; continue; }
        const size_t bcap = (size_t)kShapes[best].seg * kShapes[best].iters;
        if (cap < bcap || (cap == bcap && kShapes[i].seg > kShapes[best].seg)) best = i;
    }
    return best;
}

uint32_t gemv_tasks(int shape, size_t n) {
    const uint32_t rows = (uint32_t)rows_per_task(shape);
    return (uint32_t)((n + rows - 1) / rows);
}

hipError_t launch_gemv(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                       float *y, size_t k, size_t n, int cus) {
    const uint32_t nb = (uint32_t)(k / 32);
    const int shape = gemv_shape(kind, nb, n);
    if (shape < 0) return hipErrorInvalidValue;
    const GemvDesc one{qs, ds, x, y, nb, (uint32_t)n, 0, 0};
    const uint32_t tasks = gemv_tasks(shape, n);
    if (kind == FH_Q8_0) return dispatch<FH_Q8_0>(s, shape, nullptr, one, 1, tasks, cus);
    return dispatch<FH_Q4_0>(s, shape, nullptr, one, 1, tasks, cus);
}

hipError_t launch_gemv_group(hipStream_t s, fh_kind kind, int shape, const GemvDesc *descs, uint32_t count,
                             uint32_t tasks, int cus) {
    if (count == 0 || tasks == 0) return hipSuccess;
    const GemvDesc none{};
    if (kind == FH_Q8_0) return dispatch<FH_Q8_0>(s, shape, descs, none, count, tasks, cus);
    return dispatch<FH_Q4_0>(s, shape, descs, none, count, tasks, cus);
}

}  // namespace fh
