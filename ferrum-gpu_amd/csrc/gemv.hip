// Batch-1 GEMV on resident Q8_0 / Q4_0 weights for gfx950: y[r] = sum_k x[k] * W[r, k].
// Replaces the reference's per-column qgemv.wgsl (ferrum_wgpu/src/shaders/quant/qgemv.wgsl:88-115)
// and the single-row use of qlinear.wgsl; same dequantised values, different summation order
// (tolerance 1e-5 relative, ferrum_wgpu/src/tolerance.rs:7).
//
// The dot products run on the matrix cores as exact integer arithmetic.
//
// x side (gemv_prep_kernel, once per product): each 32-element block of x is put on the
// fixed-point grid of its largest magnitude: with 2^(E-1) <= amax < 2^E, xi = rint(x * 2^(30-E))
// (|xi| <= 2^30, error <= 2^-30 amax per element, so an element far below its block's largest
// still keeps more bits than its own f32 rounding when it is above 2^-7 amax) and
// xi = a 2^24 + b 2^16 + c 2^8 + e with a, b, c, e signed bytes. A 160-byte record per block holds
// the four limb rows in the MFMA's k order (32 bytes each), then the scale 2^(E-30) and, for
// Q4_0, the biases that turn the stored nibbles (0..15) into q = nibble - 8. A block holding a
// non-finite x contributes NaN.
//
// Weight side: the tiled planes (tile_slot, scale_slot). For 32 rows and one block the 32 quant
// slots are contiguous, so a wavefront reads one Q8_0 block or two Q4_0 blocks of 32 rows with one
// 16-byte load per lane (1 KiB, buffer loads, non-temporal), and the scales of eight blocks with
// one more.
//
// The dot products are exact integer arithmetic on the matrix cores: per block, one
// v_mfma_i32_32x32x32_i8 with B = the block's quants (Q8_0 bytes as they are; Q4_0 nibbles
// masked into bytes, after a lane-half swap that gives each lane half h of two blocks) and A =
// the prepared x of eight blocks at once, block j's limb rows in A rows 4j .. 4j + 3. C rows
// 4j .. 4j + 3 are then block j's four limb sums for each of the 32 rows, exact in int32, and
// they lie in lanes 0..31 for even j and lanes 32..63 for odd j, so each lane half finishes its
// own blocks: the sums combine in int32 into two halves (exact) and those into one f32, and the
// lane adds d * 2^(E-30) * S to its f32 accumulator. One cross-half add per row ends the task.
//
// Work: a task is one group of 32 rows of one product; each wavefront takes a contiguous range
// of tasks (one launch can hold many products: descriptors in device memory, and a map from
// task to product for each wavefront's first task) and streams them as one sequence of 8-block
// batches, the next batch's loads in flight while the current one is computed. A task's buffer
// descriptors end at its last block, and block offsets are added in the offset register the
// range check covers, so loads past it read 0. The prepared x comes from the preparation
// kernel's global buffer or, when a wavefront's share of tasks is long enough, from its own
// LDS region, filled when it starts each product (no separate launch).
#include <cstdlib>

#include "gemv_parts.hpp"
#include "internal.hpp"

namespace fh {
namespace {

// One workgroup row per product (blockIdx.x), 32 blocks per workgroup.
template <int KIND>
__global__ __launch_bounds__(256) void gemv_prep_kernel(const GemvDesc *__restrict__ descs, GemvDesc one) {
    const GemvDesc d = descs ? descs[blockIdx.x] : one;
    const bool aligned = ((uintptr_t)d.x & 15) == 0;
    // (the loop bound is the same for the eight lanes of a block)
    for (uint32_t b = (blockIdx.y * 256 + threadIdx.x) / 8; b < d.nb; b += gridDim.y * 32)
        prep_block<KIND>(d.x, aligned, b, threadIdx.x % 8,
                         (__attribute__((address_space(1))) uint32_t *)(d.prep + (size_t)b * kPrepBytes));
}

// ---- the GEMV ----
// Walks the products of a launch in task order (wave-uniform state).
struct Cursor {
    const GemvDesc *descs;
    uint32_t count, tasks;
    uint32_t p, pend;
    GemvDesc d;

    // Start at task t; map[t] is the product holding task t (no map: the one product).
    __device__ __forceinline__ void seek(uint32_t t, const uint32_t *__restrict__ map, const GemvDesc &one) {
        p = map ? map[t] : 0;
        d = descs ? descs[p] : one;
        pend = p + 1 < count ? descs[p + 1].task0 : tasks;
    }
    // Advance to the product holding task t (t never decreases).
    __device__ __forceinline__ void advance(uint32_t t) {
        while (t >= pend) {
            p++;
            d = descs[p];
            pend = p + 1 < count ? descs[p + 1].task0 : tasks;
        }
    }
};

template <int KIND>
struct Task {
    static constexpr int QB = KIND == FH_Q8_0 ? 32 : 16;
    __amdgpu_buffer_rsrc_t rq, rd, ra;  // quant slots, scales, prepared x of the task
    uint32_t nb;

    __device__ __forceinline__ void set(const GemvDesc &d, uint32_t g) {
        nb = d.nb;
        const uint32_t nb8 = (nb + 7) / 8;
        rq = make_rsrc(d.qs + (size_t)g * nb * 32 * QB, nb * 32 * QB);
        rd = make_rsrc(d.ds + (size_t)g * nb8 * 256, nb8 * 512);
        ra = make_rsrc(d.prep, nb * kPrepBytes);
    }
    // Empty ranges: every load returns 0 without touching memory.
    __device__ __forceinline__ void clear(const GemvDesc &d) {
        rq = make_rsrc(d.qs, 0);
        rd = make_rsrc(d.ds, 0);
        ra = make_rsrc(d.prep, 0);
    }
};

// A batch's place in the wavefront's stream: task t (row group g of its product, whose rows are
// n outputs of y and nb blocks wide), first block b.
struct Pos {
    uint32_t t, b, g, n, nb;
    float *y;
};

// Per-lane byte offsets inside a batch (the batch offset is added in the offset register, which
// the range check covers: batches past the task's last block read 0).
struct LaneOffsets {
    uint32_t q, s, a, t;
};

// Prepared x in LDS: one region per wavefront (kernel argument lds_blocks records, a multiple
// of eight), holding the records of the product the wavefront works on.
extern __shared__ __attribute__((aligned(16))) uint8_t gemv_lds[];

// Finished rows wait in LDS and are stored kStage tasks at a time (two tasks per store
// instruction): loads and stores share one in-order completion counter, so a store after every
// task would make the next batch's wait for its loads also wait for that store.
constexpr uint32_t kStage = 16;
struct StageMeta {
    float *y;
    uint32_t row0, n;
};

template <int KIND, bool LDSX>
__device__ __forceinline__ void load_batch(Batch<KIND> &bt, const Task<KIND> &tk, uint32_t b,
                                           const LaneOffsets &o, uint32_t lds_base) {
    if constexpr (KIND == FH_Q8_0) {
#pragma unroll
        for (int i = 0; i < kBatch; i++)
            bt.q[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(tk.rq, (int)(o.q + (b + i) * 1024), 0, kNonTemporal));
    } else {
#pragma unroll
        for (int i = 0; i < kBatch / 2; i++)
            bt.q[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(tk.rq, (int)(o.q + (b + 2 * i) * 512), 0, kNonTemporal));
    }
    bt.s = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(tk.rd, (int)(o.s + b * 64), 0, 0));
    if constexpr (LDSX) {
        const uint8_t *base = &gemv_lds[lds_base];
        bt.a = *(const i32x4 *)&base[b * kPrepBytes + o.a];
        load_tails<KIND>(bt, b * kPrepBytes, o.t, [&](uint32_t off) { return *(const u32x4 *)&base[off]; },
                         [&](uint32_t off) { return *(const uint32_t *)&base[off]; });
    } else {
        bt.a = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(tk.ra, (int)(o.a + b * kPrepBytes), 0, 0));
        load_tails<KIND>(
            bt, b * kPrepBytes, o.t,
            [&](uint32_t off) { return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(tk.ra, (int)off, 0, 0)); },
            [&](uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(tk.ra, (int)off, 0, 0); });
    }
}

// Workgroups are dealt to the eight XCDs round robin (workgroup b runs on XCD b % 8). This numbers
// them so that each XCD's workgroups hold one contiguous run of the task order: the tasks of a
// product, which all read its prepared x, then share one XCD's L2 instead of fetching the
// records into several.
__device__ __forceinline__ uint32_t xcd_order(uint32_t b, uint32_t groups) {
    const uint32_t per = groups / 8, rem = groups % 8, x = b % 8, i = b / 8;
    return x * per + min(x, rem) + i;
}

// Prepared-x jobs another launch of the same plan needs (run by this launch's workgroups before
// their own tasks: that launch starts only after this one ends, and this one reads none of them):
// job j prepares blocks 32 (j % py) .. + 31 of product j / py of descs.
struct PrepJobs {
    const GemvDesc *descs;
    uint32_t count, py;
};

template <int KIND, bool LDSX>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvDesc *__restrict__ descs,
                                                   const uint32_t *__restrict__ map, GemvDesc one, uint32_t count,
                                                   uint32_t tasks, uint32_t tasks_per_wave, uint32_t lds_blocks,
                                                   PrepJobs jobs) {
    const int lane = threadIdx.x % 64;
    // wave-uniform (readfirstlane): descriptor reads are scalar loads
    const uint32_t wave = xcd_order(blockIdx.x, gridDim.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t t0 = wave * tasks_per_wave;
    // the wavefront's tasks (waves past the last task have none), then its workgroup's share of
    // the preparation jobs: at the end, where they fill the launch's tail instead of delaying
    // every workgroup's first loads
    if (t0 < tasks) {
        const uint32_t t1 = min(tasks, t0 + tasks_per_wave);
        const int r = lane % 32;
        const bool upper = lane >= 32;
        // Q4_0: block pair chunk of 1 KiB, lane l at 16 l; Q8_0: block tile of 1 KiB, row r at 32 r;
        // scales: row r's eight at 16 r; prepared x: prep_a_offset, prep_tail_offset
        const LaneOffsets o{KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * upper) : (uint32_t)(lane * 16), (uint32_t)(r * 16),
                            prep_a_offset(lane), prep_tail_offset<KIND>(lane)};
        // The wavefront's tasks are one stream of batches: the loads of the next batch (of this task
        // or the next) are in flight while a batch is computed, so the pipeline never drains at a
        // task boundary. lp is the batch being loaded, cp the batch being computed.
        Cursor cur{descs, count, tasks, 0, 0, {}};
        cur.seek(t0, map, one);
        // With LDSX the wavefront prepares its product's x into its LDS region (all of it, padded
        // with zero records to a multiple of eight blocks), whenever it starts a product; the
        // batch in flight already holds its own x in registers, so the region can be rewritten.
        const uint32_t lds_base = (threadIdx.x / 64) * lds_blocks * kPrepBytes;
        auto prepare = [&](const GemvDesc &d) {
            if constexpr (LDSX) {
                const bool aligned = ((uintptr_t)d.x & 15) == 0;
                const uint32_t nb8 = (d.nb + 7) / 8 * 8;
                for (uint32_t b = lane / 8; b < nb8; b += 8) {
                    __attribute__((address_space(3))) uint32_t *rec =
                        (__attribute__((address_space(3))) uint32_t *)&gemv_lds[lds_base + b * kPrepBytes];
                    if (b < d.nb) {
                        prep_block<KIND>(d.x, aligned, b, lane % 8, rec);
                    } else {
                        zero_record(lane % 8, rec);  // padding records
                    }
                }
            }
        };
        prepare(cur.d);
        Task<KIND> ltk;
        Pos lp{t0, 0, t0 - cur.d.task0, cur.d.n, cur.d.nb, cur.d.y};
        ltk.set(cur.d, lp.g);
        auto advance = [&]() {
            lp.b += kBatch;
            if (lp.b >= lp.nb) {
                lp.t++;
                lp.b = 0;
                if (lp.t < t1) {
                    const uint32_t p0 = cur.p;
                    cur.advance(lp.t);
                    if (cur.p != p0) prepare(cur.d);
                    lp.g = lp.t - cur.d.task0;
                    lp.n = cur.d.n;
                    lp.nb = cur.d.nb;
                    lp.y = cur.d.y;
                    ltk.set(cur.d, lp.g);
                } else {
                    ltk.clear(cur.d);  // the stream's end: the last loads fetch nothing
                }
            }
        };
        float acc = 0.0f;
        __shared__ float stage_rows[4][kStage][32];
        __shared__ StageMeta stage_meta[4][kStage];
        const uint32_t wv = threadIdx.x / 64;
        uint32_t staged = 0;  // wave-uniform
        // Store the staged rows: lanes 0..31 take staged task 2i, lanes 32..63 task 2i + 1.
        auto flush = [&]() {
            for (uint32_t i = 0; i < staged; i += 2) {
                const uint32_t s = i + (upper ? 1 : 0);
                if (s < staged) {
                    const StageMeta m = stage_meta[wv][s];
                    const uint32_t row = m.row0 + r;
                    // (a global-address-space store: a flat store would also count against the
                    // scalar-load counter and make the next wait for loads a full drain)
                    if (row < m.n) ((__attribute__((address_space(1))) float *)m.y)[row] = stage_rows[wv][s][r];
                }
            }
            staged = 0;
        };
        // After computing batch cp: on a task's last batch, add the row's odd blocks (lane 32 + r) to
        // its even ones (lane r) and stage the row.
        auto finish = [&](const Pos &cp) {
            if (cp.b + kBatch >= cp.nb) {
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
                const float sum = acc + __uint_as_float(upper ? sw[0] : sw[1]);
                if (!upper) stage_rows[wv][staged][r] = sum;
                if (lane == 0) stage_meta[wv][staged] = StageMeta{cp.y, cp.g * 32, cp.n};
                acc = 0.0f;
                if (++staged == kStage) flush();
            }
        };
        Batch<KIND> b0, b1;
        load_batch<KIND, LDSX>(b0, ltk, lp.b, o, lds_base);
        Pos cp = lp;
        advance();
        // (scheduling barriers keep each batch's loads together, so a batch waits only for its own)
        for (;;) {
            load_batch<KIND, LDSX>(b1, ltk, lp.b, o, lds_base);
            __builtin_amdgcn_sched_barrier(0);
            if (cp.b + kBatch / 2 >= cp.nb)
                compute_batch<KIND, kBatch / 4>(b0, upper, acc);  // a task's last half batch
            else
                compute_batch<KIND>(b0, upper, acc);
            __builtin_amdgcn_sched_barrier(0);
            finish(cp);
            if (lp.t >= t1) break;
            cp = lp;
            advance();
            load_batch<KIND, LDSX>(b0, ltk, lp.b, o, lds_base);
            __builtin_amdgcn_sched_barrier(0);
            if (cp.b + kBatch / 2 >= cp.nb)
                compute_batch<KIND, kBatch / 4>(b1, upper, acc);
            else
                compute_batch<KIND>(b1, upper, acc);
            __builtin_amdgcn_sched_barrier(0);
            finish(cp);
            if (lp.t >= t1) break;
            cp = lp;
            advance();
        }
        flush();
    }
    for (uint32_t j = blockIdx.x; j < jobs.count * jobs.py; j += gridDim.x) {
        const GemvDesc d = jobs.descs[j / jobs.py];
        const uint32_t b = (j % jobs.py) * 32 + threadIdx.x / 8;  // (the eight lanes of a block agree)
        if (b < d.nb)
            prep_block<KIND>(d.x, ((uintptr_t)d.x & 15) == 0, b, threadIdx.x % 8,
                             (__attribute__((address_space(1))) uint32_t *)(d.prep + (size_t)b * kPrepBytes));
    }
}

// Wavefronts per CU a launch aims for (FERRUM_HIP_GEMV_WAVES_PER_CU overrides, 1..32), at most
// what fits.
uint32_t waves_per_cu() {
    static const uint32_t w = [] {
        const char *e = getenv("FERRUM_HIP_GEMV_WAVES_PER_CU");
        const long v = e ? strtol(e, nullptr, 10) : 0;
        return (uint32_t)(v >= 1 && v <= 32 ? v : 8);
    }();
    return w;
}

constexpr uint32_t kMaxLdsBlocks = kGemvLdsBlocks;  // per wavefront: 17.5 KiB of prepared x, 70 KiB per workgroup (two fit a CU)
constexpr uint32_t kMinLdsTasks = 8;     // tasks per wavefront below which x is prepared once, globally

// Resident workgroups per CU for a kernel and its dynamic LDS (cached per LDS size).
template <int KIND, bool LDSX>
int resident_groups(uint32_t lds_bytes) {
    static int cache[kMaxLdsBlocks / 8 + 1] = {};
    const uint32_t key = lds_bytes / (4 * 8 * kPrepBytes);
    if (key <= kMaxLdsBlocks / 8 && cache[key] > 0) return cache[key];
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, gemv_kernel<KIND, LDSX>, 256, lds_bytes) != hipSuccess ||
        b < 1)
        b = 1;
    if (key <= kMaxLdsBlocks / 8) cache[key] = b;
    return b;
}

// other: the products of another launch whose prepared x this launch may write (other->count 0:
// none). Returns through *other_done whether it did (then that launch skips its own preparation).
template <int KIND>
hipError_t launch_kind(hipStream_t s, const GemvDesc *descs, const uint32_t *map, const GemvDesc &one,
                       uint32_t count, uint32_t tasks, uint32_t max_nb, int cus, const GemvPrep &other,
                       bool skip_prep, bool *other_done) {
    // Prepared x in LDS when every product's fits in a wavefront's region and a wavefront's
    // share of tasks is long enough to pay for preparing it (each wavefront prepares every
    // product it touches); otherwise a separate preparation kernel (a row of workgroups per
    // product, 32 blocks per workgroup) writes it to global memory once.
    const uint32_t nb8 = (max_nb + 7) / 8 * 8;
    const uint32_t waves_est = (uint32_t)(cus > 0 ? cus : 256) * min(4u * resident_groups<KIND, false>(0), waves_per_cu());
    const bool ldsx = nb8 <= kMaxLdsBlocks && (tasks + waves_est - 1) / waves_est >= kMinLdsTasks;
    const uint32_t lds_bytes = ldsx ? 4 * nb8 * kPrepBytes : 0;
    PrepJobs jobs{other.descs, 0, (other.max_nb + 31) / 32};
    if (other_done) *other_done = false;
    if (!ldsx) {
        // one preparation launch for this launch's products and, when they follow them in the
        // descriptor array, the other launch's
        const bool both = other.count && other.descs == descs + count;
        const uint32_t py = (max(max_nb, both ? other.max_nb : 0u) + 31) / 32;
        if (!skip_prep || both)
            gemv_prep_kernel<KIND><<<dim3(count + (both ? other.count : 0), py < 4096 ? py : 4096), 256, 0, s>>>(
                descs, one);
        if (both && other_done) *other_done = true;
    } else {
        if (other.count && other_done) {
            jobs.count = other.count;
            *other_done = true;
        }
        static const hipError_t attr = hipFuncSetAttribute((const void *)gemv_kernel<KIND, true>,
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                                           (int)(4 * kMaxLdsBlocks * kPrepBytes));
        (void)attr;
    }
    // as many wavefronts as fit on the chip at once (or the requested per-CU count), each an
    // equal share of the tasks
    const int resident = 4 * (ldsx ? resident_groups<KIND, true>(lds_bytes) : resident_groups<KIND, false>(0));
    const uint32_t per_cu = min((uint32_t)resident, waves_per_cu());
    const uint32_t max_waves = (uint32_t)(cus > 0 ? cus : 256) * per_cu;
    const uint32_t per = (tasks + max_waves - 1) / max_waves;
    const uint32_t waves = (tasks + per - 1) / per;
    if (ldsx)
        gemv_kernel<KIND, true><<<(waves + 3) / 4, 256, lds_bytes, s>>>(descs, map, one, count, tasks, per, nb8, jobs);
    else
        gemv_kernel<KIND, false><<<(waves + 3) / 4, 256, 0, s>>>(descs, map, one, count, tasks, per, 0,
                                                                 PrepJobs{nullptr, 0, 1});
    return hipGetLastError();
}

}  // namespace

bool gemv_supported(fh_kind kind, size_t k, size_t n) {
    // a task's ranges (32 rows of quants, their scales, the prepared x) and every offset into
    // them, padding batches included, stay far below 2^31
    (void)kind;
    (void)n;
    const size_t nb = k / 32;
    return nb > 0 && nb <= (1u << 20);
}

size_t gemv_prep_bytes(size_t k) { return k / 32 * kPrepBytes; }

uint32_t gemv_tasks(size_t n) { return (uint32_t)((n + 31) / 32); }

hipError_t launch_gemv(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                       float *y, size_t k, size_t n, void *prep, int cus) {
    const GemvDesc one{qs, ds, x, y, (uint8_t *)prep, (uint32_t)(k / 32), (uint32_t)n, 0, 0};
    const GemvPrep none{nullptr, 0, 0};
    if (kind == FH_Q8_0)
        return launch_kind<FH_Q8_0>(s, nullptr, nullptr, one, 1, gemv_tasks(n), (uint32_t)(k / 32), cus, none, false,
                                    nullptr);
    return launch_kind<FH_Q4_0>(s, nullptr, nullptr, one, 1, gemv_tasks(n), (uint32_t)(k / 32), cus, none, false,
                                nullptr);
}

hipError_t launch_gemv_group(hipStream_t s, fh_kind kind, const GemvDesc *descs, const uint32_t *map,
                             uint32_t count, uint32_t tasks, uint32_t max_nb, int cus, const GemvPrep &other,
                             bool skip_prep, bool *other_done) {
    if (other_done) *other_done = false;
    if (count == 0 || tasks == 0) return hipSuccess;
    const GemvDesc none{};
    if (kind == FH_Q8_0)
        return launch_kind<FH_Q8_0>(s, descs, map, none, count, tasks, max_nb, cus, other, skip_prep, other_done);
    return launch_kind<FH_Q4_0>(s, descs, map, none, count, tasks, max_nb, cus, other, skip_prep, other_done);
}

}  // namespace fh
