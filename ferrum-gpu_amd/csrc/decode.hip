// GPT-2 KV-cached decode on resident Q8_0 / Q4_0 weights (replaces ferrum_wgpu's GpuGpt2,
// ferrum_wgpu/src/models/gpt2.rs:52-265, whose weights are f32; the CPU oracle is ferrum_ref's
// Gpt2::feed, ferrum_ref/src/models/gpt2/decode.rs:57-117, on the fake-quantised model).
//
// A decode step is latency-bound (GPT-2-small reads 131 MB of packed weights per token, 26 us
// at HBM speed), so it is built from few, fused launches and replayed as one HIP graph. Where
// the head width is 64, 128 or 256 (GPT-2-small's 64) a layer is four launches:
//   gemv LN|QKV         x = x_m + (sum_s down[s] + b_2) (layer 0: tok[token] + pos[p]);
//                       q | kcache[p] | vcache[p] = LN1(x) W_qkv + b   (one product, n = 3d)
//   attention + W_o     per head h: a_h = softmax(q k^T / sqrt(hd)) v, out[h] = a_h W_o[:, h]
//   gemv LN|GELU        x_m = x + (sum_h out[h] + b_o); f = gelu(LN2(x_m) W_1 + b_1)
//   gemv (K split)      down[s] = the split s share of f W_2
// (the partial rows are added by their consumer in a fixed order), then
//   final LN            LNf(x_m + (sum_s down[s] + b_2)) into prepared records
//   gemv STORE          logits = LNf(x) W_head
//   argmax              next token (sampling.rs:32-40), written to the device's input array;
//                       the position advances.
// Other head widths run five launches per layer (embed first; LN1|QKV, attention, W_o +
// residual, LN2|GELU, W_2 + residual; the final LN from x).
// The position lives in device memory, so the same graph serves every step, and greedy
// generation runs without a host round trip per token.
//
// The decode GEMV (decode_gemv_kernel) gives each group of 32 output rows one workgroup and
// splits the row's blocks over its wavefronts (one 8-block batch each where the row allows), so
// a small product still spreads over many CUs; the partial sums meet in LDS in a fixed order
// (results are reproducible). Each workgroup prepares the x blocks it needs itself, applying the
// LayerNorm prologue on the way, and the epilogue adds the bias and applies GELU, the residual or
// the QKV scatter into the caches. The block products are the exact integer MFMA products of the
// batch-1 GEMV (gemv_parts.hpp).
#include <algorithm>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "gemv_parts.hpp"
#include "internal.hpp"

namespace fh {
namespace {

enum { PRO_NONE = 0, PRO_LN = 1, PRO_GLOBAL = 2, PRO_LNR = 3 };  // PRO_LNR: LayerNorm of the residual row (residual_row)
enum { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_GELU = 2, EPI_QKV = 3, EPI_ARGMAX = 4, EPI_PARTIAL = 5 };

constexpr int kMaxWaves = 8;           // wavefronts per decode-GEMV workgroup (two per SIMD)
constexpr int kLnRed = 4 * kMaxWaves;  // reduction slots (floats) a LayerNorm prologue uses
constexpr uint32_t kMaxBlocks = 512;   // blocks per row (k <= 16384): 80 KiB of prepared x in LDS
constexpr uint32_t kLnSlots = 2;       // LayerNorm prologue: (block, lane) slots a thread keeps in registers
constexpr uint32_t kNone = 0xffffffffu;
constexpr int kAttnThreads = 512;
// Cache policy of the decode's weight loads: ordinary (cached) loads, so that a model whose
// weights fit in the last-level cache (GPT-2-small's 131 MB in 256 MB) finds them there on the
// next token (measured 3-11% faster per step than streaming loads).
#ifndef FH_DECODE_LOAD_POLICY
#define FH_DECODE_LOAD_POLICY 0
#endif
constexpr int kWeightPolicy = FH_DECODE_LOAD_POLICY;

struct DecodeGemv {
    const uint8_t *qs;
    const uint16_t *ds;
    const float *x;            // k inputs
    const float *ln_g, *ln_b;  // PRO_LN
    const uint8_t *prep;       // PRO_GLOBAL: the prepared records of x
    const float *bias;         // n, or null
    float *y;                  // n outputs; EPI_RESIDUAL adds into it; EPI_QKV: the q part
    float *kc, *vc;            // EPI_QKV: caches [ctx, split]
    int32_t *state;            // [0] position, [1] first position whose input a pick fills, [2] last pick
    int32_t *inputs;           // EPI_ARGMAX: the token of each position
    float *partial;            // split K: row sums [splits][groups * 32]; EPI_ARGMAX: best value per group
    uint32_t *pick;            // EPI_ARGMAX: best row per group
    uint32_t *ticket;          // split K: one counter per row group; EPI_ARGMAX: one counter
    uint32_t nb, n, split;     // split: EPI_QKV width of each of q, k, v
    uint32_t chunk;            // blocks per K split (a multiple of 8)
    float eps;
    // PRO_LNR: the residual row x_in + (sum of nparts rows of rpart + rbias), or the embedding
    // of inputs[state[0]] (x_in == null; emb_*, pos_tab); workgroup (0, 0) stores it at x_out
    const float *x_in, *rpart, *rbias;
    uint32_t nparts;
    const uint8_t *emb_qs;
    const uint16_t *emb_ds;
    const float *pos_tab;
    float *x_out;
};

// ferrum_ref/src/kernels/nn.rs:12-15
__device__ __forceinline__ float gelu(float x) {
    return 0.5f * x * (1.0f + tanhf(0.7978846f * (x + 0.044715f * x * x * x)));
}

typedef __attribute__((address_space(1))) const f32x4 gf32x4;

__device__ __forceinline__ f32x4 gload4(const float *p) { return *(gf32x4 *)p; }

// Agent-coherent stores (relaxed atomics at agent scope: written through to the point where every
// XCD sees them) for data one workgroup of a launch writes and another reads in the same launch,
// without cache-wide fences. The readers use ordinary loads: each such address is written once per
// launch before anything in the launch reads it (the one-launch step keeps a copy of every buffer
// per layer), so no XCD's L2 can hold an older copy of it.
typedef __attribute__((address_space(1))) uint64_t g_u64;
typedef __attribute__((address_space(1))) uint32_t g_u32;
__device__ __forceinline__ void cstore(float *p, float v) {
    __hip_atomic_store((g_u32 *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstore4(float *p, f32x4 v) {
    g_u64 *q = (g_u64 *)p;
    __hip_atomic_store(q, (uint64_t)__float_as_uint(v[0]) | (uint64_t)__float_as_uint(v[1]) << 32, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, (uint64_t)__float_as_uint(v[2]) | (uint64_t)__float_as_uint(v[3]) << 32, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}


// Loads from memory other workgroups wrote in this launch (past the per-CU caches).
__device__ __forceinline__ float coherent_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The first maximum wins; NaN never does (ferrum_model/src/sampling.rs:32-40). kNone: no candidate.
__device__ __forceinline__ bool better(float v2, uint32_t i2, float v1, uint32_t i1) {
    return i2 != kNone && (i1 == kNone || v2 > v1 || (v2 == v1 && i2 < i1));
}

struct LnParams {  // a LayerNorm's gain and bias in the thread's slots (see ln_records_p)
    f32x4 g[kLnSlots], b[kLnSlots];
};

__device__ __forceinline__ void load_ln(const float *lg, const float *lb, uint32_t nb, LnParams &p) {
#pragma unroll
    for (uint32_t u = 0; u < kLnSlots; u++) {
        const uint32_t sl = threadIdx.x + u * blockDim.x;
        if (sl / 8 < nb) {
            p.g[u] = gload4(lg + sl * 4);
            p.b[u] = gload4(lb + sl * 4);
        }
    }
}

// LayerNorm (ferrum_ref/src/kernels/nn.rs:31-44) of the k = 32 nb values that the workgroup
// holds in registers (thread slot u: block sl / 8, elements 4 sl .. 4 sl + 3 with
// sl = threadIdx.x + u blockDim.x; slots past nb hold nothing), with gain and bias pa (load_ln),
// written as the prepared records of `span` blocks (zero records past nb) at out (LDS, or global
// when GLOBAL). span * 8 <= kLnSlots * blockDim.x. red: kLnRed floats (16-byte aligned) that no
// wavefront may still be reading from an earlier use.
//
// The mean and variance take one barrier: each wavefront sums its values' offsets from a shift c_w
// (its lane 0's first value) and their squares, and the wavefronts' sums meet through LDS, where
// sum (x - mean)^2 = sum_w [S2_w - 2 (mean - c_w) S1_w + n_w (mean - c_w)^2] (S1_w, S2_w: the
// wavefront's sums of x - c_w and of its squares; n_w its count). A shift taken from the data keeps
// the squares' sums from cancelling; the result differs from the two-pass statistics of nn.rs only
// in rounding.
template <int KIND, bool GLOBAL>
__device__ __forceinline__ void ln_records_p(const f32x4 (&v)[kLnSlots], const LnParams &pa, float eps, uint32_t nb,
                                             uint32_t span, uint8_t *out, float *red) {
    const uint32_t k = nb * 32, nw = blockDim.x / 64, w = threadIdx.x / 64;
    // the wavefront's count: its slots below 8 nb, four values each
    uint32_t cnt = 0;
#pragma unroll
    for (uint32_t u = 0; u < kLnSlots; u++) {
        const int32_t r = (int32_t)(8 * nb) - (int32_t)(64 * w + u * blockDim.x);
        cnt += (uint32_t)min(max(r, 0), 64);
    }
    const float cw = 8 * w < nb ? lane_value(v[0].x, 0) : 0.0f;  // lane 0's slot 0 holds data iff any lane does
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < kLnSlots; u++) {
        const uint32_t sl = threadIdx.x + u * blockDim.x;
        if (sl / 8 < nb) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float t = v[u][c] - cw;
                s1 += t;
                s2 += t * t;
            }
        }
    }
    s1 = wave_reduce(s1, AddOp());
    s2 = wave_reduce(s2, AddOp());
    if (threadIdx.x % 64 == 0)
        *(f32x4 *)&red[4 * w] = f32x4{s1, s2, cw, (float)(4 * cnt)};
    __syncthreads();
    // (the reads issued together: a loop that waits for each read costs an LDS latency a step)
    f32x4 rw[kMaxWaves];
#pragma unroll
    for (uint32_t i = 0; i < kMaxWaves; i++) rw[i] = i < nw ? *(const f32x4 *)&red[4 * i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float tot = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < kMaxWaves; i++) tot += rw[i].x + rw[i].w * rw[i].z;
    const float mean = tot / (float)k;
    float m2 = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < kMaxWaves; i++) {
        const float dl = mean - rw[i].z;
        m2 += rw[i].y - 2.0f * dl * rw[i].x + rw[i].w * dl * dl;
    }
    const float rstd = 1.0f / sqrtf(fmaxf(m2, 0.0f) / (float)k + eps);
#pragma unroll
    for (uint32_t u = 0; u < kLnSlots; u++) {
        const uint32_t sl = threadIdx.x + u * blockDim.x, blk = sl / 8;
        const int j = (int)(sl % 8);
        if (blk >= span) continue;  // the eight lanes of a block agree
        uint8_t *rec = out + blk * kPrepBytes;
        if (blk < nb) {
            f32x4 h;
#pragma unroll
            for (int c = 0; c < 4; c++) h[c] = (v[u][c] - mean) * rstd * pa.g[u][c] + pa.b[u][c];
            if constexpr (GLOBAL)
                prep_values<KIND>(h, j, (__attribute__((address_space(1))) uint32_t *)rec);
            else
                prep_values<KIND>(h, j, (__attribute__((address_space(3))) uint32_t *)rec);
        } else {
            if constexpr (GLOBAL)
                zero_record(j, (__attribute__((address_space(1))) uint32_t *)rec);
            else
                zero_record(j, (__attribute__((address_space(3))) uint32_t *)rec);
        }
    }
}

// As ln_records_p, reading the gain lg and bias lb here.
template <int KIND, bool GLOBAL>
__device__ __forceinline__ void ln_records(const f32x4 (&v)[kLnSlots], const float *lg, const float *lb, float eps,
                                           uint32_t nb, uint32_t span, uint8_t *out, float *red) {
    LnParams pa;
    load_ln(lg, lb, nb, pa);
    ln_records_p<KIND, GLOBAL>(v, pa, eps, nb, span, out, red);
}

// The LayerNorm of x (k = 32 nb values in global memory) into prepared records (ln_records); x is
// read once.
template <int KIND, bool GLOBAL>
__device__ __forceinline__ void ln_prep(const float *x, const float *lg, const float *lb, float eps, uint32_t nb,
                                        uint32_t span, uint8_t *out, float *red) {
    f32x4 v[kLnSlots];
#pragma unroll
    for (uint32_t u = 0; u < kLnSlots; u++) {
        const uint32_t sl = threadIdx.x + u * blockDim.x;
        if (sl / 8 < nb) v[u] = gload4(x + sl * 4);
    }
    ln_records<KIND, GLOBAL>(v, lg, lb, eps, nb, span, out, red);
}

// One workgroup: LayerNorm of x into global prepared records (for a product whose many row groups
// would each repeat it).
template <int KIND>
__global__ __launch_bounds__(64 * kMaxWaves) void ln_prep_kernel(const float *__restrict__ x, const float *__restrict__ lg,
                                                                 const float *__restrict__ lb, float eps, uint32_t nb,
                                                                 uint8_t *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) float red[kLnRed];
    ln_prep<KIND, true>(x, lg, lb, eps, nb, (nb + 7) / 8 * 8, out, red);
}

struct StepArgs {
    // the residual row: x_in + (sum over nparts rows of part + pbias), or (x_in == null) the
    // embedding tok[inputs[p]] + pos_tab[p]
    const float *x_in, *part, *pbias;
    uint32_t nparts;
    const uint8_t *emb_qs;
    const uint16_t *emb_ds;
    const float *pos_tab;
    const int32_t *inputs;
    const int32_t *state;
    float *x_out;  // workgroup (0, 0) stores the residual row here
    const float *ln_g, *ln_b;
    float eps;
    // attn_out_kernel: the query row, the caches [ctx][d], and the output projection (d rows of
    // nb2 blocks; the workgroup takes blocks blockIdx.x * hd / 32 .. of each row)
    const float *q;
    float *kc, *vc;
    const uint8_t *qs2;
    const uint16_t *ds2;
    uint32_t nb2;
    float *out_part;  // [gridDim.x][d]
    uint32_t d, nb;
    float scale;
};

// The residual row into the thread's slots (see ln_records); workgroup (0, 0) stores it.
// rb: the bias's slots already loaded (or null: read here).
template <int KIND>
__device__ __forceinline__ void residual_row(const StepArgs &a, f32x4 (&v)[kLnSlots], const f32x4 *rb = nullptr) {
    const uint32_t nb = a.nb, d = a.d;
#pragma unroll
    for (uint32_t u = 0; u < kLnSlots; u++) {
        const uint32_t sl = threadIdx.x + u * blockDim.x;
        if (sl / 8 >= nb) continue;
        if (a.x_in == nullptr) {
            // x = tok[t] + pos[p] (decode.rs:72-74), as embed_kernel
            const uint32_t p = (uint32_t)a.state[0];
            const uint32_t t = (uint32_t)a.inputs[p];
            const f32x4 pv = gload4(a.pos_tab + (size_t)p * d + sl * 4);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t i = sl * 4 + c, b = i / 32, j = i % 32;
                const size_t slot = tile_slot(t, b, nb);
                float q;
                if constexpr (KIND == FH_Q8_0) {
                    q = (float)(int8_t)a.emb_qs[slot * 32 + j];
                } else {
                    const uint32_t byte = a.emb_qs[slot * 16 + (j % 16)];
                    q = (float)((int32_t)(j < 16 ? byte & 15u : byte >> 4) - 8);
                }
                v[u][c] = half_bits_to_float(a.emb_ds[scale_slot(t, b, nb)]) * q + pv[c];
            }
        } else {
            // nn::add(x, gemv(..) + b) (decode.rs:100,111): the partial sums in order, then the
            // bias; sixteen rows' loads are issued before any of them is added (rows past
            // nparts read as zero and add nothing)
            const f32x4 x = gload4(a.x_in + sl * 4);
            f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
            const float *pp = a.part + sl * 4;
            for (uint32_t j = 0; j < a.nparts; j += 16) {
                f32x4 r[16];
#pragma unroll
                for (int k = 0; k < 16; k++)
                    r[k] = j + k < a.nparts ? gload4(pp + (size_t)(j + k) * d) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int k = 0; k < 16; k++) t += r[k];
            }
            t += rb ? rb[u] : gload4(a.pbias + sl * 4);
            v[u] = x + t;
        }
        if (blockIdx.x == 0 && blockIdx.y == 0 && a.x_out) *(f32x4 *)(a.x_out + sl * 4) = v[u];
    }
}

template <int KIND>
__device__ __forceinline__ void load_weights(Batch<KIND> &bt, __amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rd,
                                             uint32_t oq, uint32_t os, uint32_t b) {
    if constexpr (KIND == FH_Q8_0) {
#pragma unroll
        for (int i = 0; i < kBatch; i++)
            bt.q[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(oq + (b + i) * 1024), 0, kWeightPolicy));
    } else {
#pragma unroll
        for (int i = 0; i < kBatch / 2; i++)
            bt.q[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(oq + (b + 2 * i) * 512), 0, kWeightPolicy));
    }
    bt.s = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rd, (int)(os + b * 64), 0, 0));
}

// Workgroup (g, s): the 32 output rows g (blockIdx.x) over the blocks [s chunk, (s + 1) chunk)
// of their rows (blockIdx.y, a K split); W = blockDim.x / 64 wavefronts, wavefront w taking the
// batches 8w, 8w + 8W, ... of the split. With more than one split the splits' row sums go to
// a.partial and the last split to arrive (a counter per row group) adds them in split order and
// runs the epilogue, so the result does not depend on timing.
template <int KIND, int PRO, int EPI>
__global__ __launch_bounds__(64 * kMaxWaves) void decode_gemv_kernel(DecodeGemv a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t dlds[];
    const uint32_t W = blockDim.x / 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64, r = lane % 32;
    const bool upper = lane >= 32;
    const uint32_t nb = a.nb, nb8 = (nb + 7) / 8, span = nb8 * 8;
    constexpr uint32_t QB = KIND == FH_Q8_0 ? 32 : 16;
    const uint32_t g = blockIdx.x, S = gridDim.y, sp = blockIdx.y;
    const uint32_t b0 = sp * a.chunk, b1 = min(span, b0 + a.chunk);
    const auto rq = make_rsrc(a.qs + (size_t)g * nb * 32 * QB, nb * 32 * QB);
    const auto rd = make_rsrc(a.ds + (size_t)g * nb8 * 256, nb8 * 512);
    const auto ra = make_rsrc(a.prep, PRO == PRO_GLOBAL ? span * kPrepBytes : 0);
    const uint32_t oq = KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * upper) : (uint32_t)(lane * 16);
    const uint32_t os = (uint32_t)(r * 16), oa = prep_a_offset(lane), ot = prep_tail_offset<KIND>(lane);
    const auto g16 = [&](uint32_t off) { return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)off, 0, 0)); };
    const auto g4 = [&](uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(ra, (int)off, 0, 0); };
    uint8_t *prep = dlds;  // records of blocks b0 .. b1 (PRO_LN: of every block)
    constexpr bool kLn = PRO == PRO_LN || PRO == PRO_LNR;  // every block's records in LDS
    float *part = (float *)(dlds + (PRO == PRO_GLOBAL ? 0 : (kLn ? span : a.chunk) * kPrepBytes));
    float *red = part + W * 32;

    // the epilogue's bias and residual inputs are requested first (the epilogue runs in lanes 0..31
    // of wavefront 0; nothing in this launch writes them before it)
    float pre_bias = 0.0f, pre_y = 0.0f;
    if (wave == 0 && !upper && g * 32 + r < a.n) {
        if (a.bias) pre_bias = a.bias[g * 32 + r];
        if constexpr (EPI == EPI_RESIDUAL) pre_y = a.y[g * 32 + r];
    }
    // the wavefront's first batch is requested before x is prepared
    Batch<KIND> cur, nx;
    uint32_t bb = b0 + wave * kBatch;
    if (bb < b1) {
        load_weights<KIND>(cur, rq, rd, oq, os, bb);
        if constexpr (PRO == PRO_GLOBAL) {
            cur.a = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(bb * kPrepBytes + oa), 0, 0));
            load_tails<KIND>(cur, bb * kPrepBytes, ot, g16, g4);
        }
    }
    if constexpr (PRO == PRO_LN) {
        ln_prep<KIND, false>(a.x, a.ln_g, a.ln_b, a.eps, nb, span, prep, red);
        __syncthreads();
    } else if constexpr (PRO == PRO_LNR) {
        StepArgs f{};
        f.x_in = a.x_in;
        f.part = a.rpart;
        f.pbias = a.rbias;
        f.nparts = a.nparts;
        f.emb_qs = a.emb_qs;
        f.emb_ds = a.emb_ds;
        f.pos_tab = a.pos_tab;
        f.inputs = a.inputs;
        f.state = a.state;
        f.x_out = a.x_out;
        f.d = nb * 32;
        f.nb = nb;
        f32x4 v[kLnSlots];
        residual_row<KIND>(f, v);
        ln_records<KIND, false>(v, a.ln_g, a.ln_b, a.eps, nb, span, prep, red);
        __syncthreads();
    } else if constexpr (PRO == PRO_NONE) {
        // the split's blocks of x, eight lanes per block (the eight lanes share the loop bound)
        for (uint32_t blk = b0 + threadIdx.x / 8; blk < b1; blk += blockDim.x / 8) {
            const int j = threadIdx.x % 8;
            __attribute__((address_space(3))) uint32_t *rec =
                (__attribute__((address_space(3))) uint32_t *)(prep + (blk - b0) * kPrepBytes);
            if (blk < nb)
                prep_values<KIND>(gload4(a.x + blk * 32 + 4 * j), j, rec);
            else
                zero_record(j, rec);
        }
        __syncthreads();
    }
    const uint32_t pbase = kLn ? 0 : b0;
    float acc = 0.0f;
    while (bb < b1) {
        const uint32_t nxt = bb + W * kBatch;
        if (nxt < b1) {
            load_weights<KIND>(nx, rq, rd, oq, os, nxt);
            if constexpr (PRO == PRO_GLOBAL) {
                nx.a = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(nxt * kPrepBytes + oa), 0, 0));
                load_tails<KIND>(nx, nxt * kPrepBytes, ot, g16, g4);
            }
        }
        if constexpr (PRO != PRO_GLOBAL) {
            typedef __attribute__((address_space(3))) const uint8_t lbyte;
            lbyte *lp = (lbyte *)prep;
            cur.a = *(const __attribute__((address_space(3))) i32x4 *)(lp + (bb - pbase) * kPrepBytes + oa);
            load_tails<KIND>(cur, (bb - pbase) * kPrepBytes, ot,
                             [&](uint32_t off) { return *(const __attribute__((address_space(3))) u32x4 *)(lp + off); },
                             [&](uint32_t off) { return *(const __attribute__((address_space(3))) uint32_t *)(lp + off); });
        }
        compute_batch<KIND>(cur, upper, acc);
        cur = nx;
        bb = nxt;
    }
    // row r's odd blocks (lane 32 + r) join its even ones (lane r); the wavefronts' partial sums
    // meet in LDS and are added in wavefront order
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
    const float sum = acc + __uint_as_float(upper ? sw[0] : sw[1]);
    if (!upper) part[wave * 32 + r] = sum;
    __syncthreads();
    if (wave != 0 || upper) return;
    float pw[kMaxWaves];  // (the reads issued together)
#pragma unroll
    for (uint32_t w = 0; w < kMaxWaves; w++) pw[w] = w < W ? part[w * 32 + r] : 0.0f;
    float t = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < kMaxWaves; w++)
        if (w < W) t += pw[w];
    const uint32_t row = g * 32 + r;
    if constexpr (EPI == EPI_PARTIAL) {
        // the split's row sums, added in split order by their consumer (residual_row)
        if (row < a.n) a.y[(size_t)sp * a.n + row] = t;
        return;
    }
    if (S > 1) {
        a.partial[(size_t)sp * gridDim.x * 32 + row] = t;
        __threadfence();
        uint32_t last = 0;
        if (r == 0) last = atomicAdd(&a.ticket[g], 1u) == S - 1 ? 1u : 0u;
        if (__shfl(last, 0, 32) == 0) return;
        __threadfence();
        t = 0.0f;
        for (uint32_t q = 0; q < S; q++) t += coherent_load(&a.partial[(size_t)q * gridDim.x * 32 + row]);
        if (r == 0) a.ticket[g] = 0;  // every split has arrived: ready for the next launch
    }
    if constexpr (EPI == EPI_ARGMAX) {
        // the logits row, and the row group's offer for the pick (pick_kernel reduces the offers)
        if (row < a.n) a.y[row] = t;
        float bv = t;
        uint32_t bi = (row < a.n && t == t) ? row : kNone;
#pragma unroll
        for (int o = 16; o >= 1; o /= 2) {
            const float ov = __shfl_xor(bv, o, 32);
            const uint32_t oi = __shfl_xor(bi, o, 32);
            if (better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (r == 0) {
            a.partial[g] = bv;
            a.pick[g] = bi;
        }
        return;
    }
    if (row >= a.n) return;
    if (a.bias) t = t + pre_bias;  // decode.rs:42-53: the bias joins after the products
    if constexpr (EPI == EPI_STORE) {
        a.y[row] = t;
    } else if constexpr (EPI == EPI_RESIDUAL) {
        a.y[row] = pre_y + t;  // nn::add(x, gemv(..)), decode.rs:100,111
    } else if constexpr (EPI == EPI_GELU) {
        a.y[row] = gelu(t);
    } else {
        const uint32_t p = (uint32_t)a.state[0];
        if (row < a.split)
            a.y[row] = t;
        else if (row < 2 * a.split)
            a.kc[(size_t)p * a.split + row - a.split] = t;
        else
            a.vc[(size_t)p * a.split + row - 2 * a.split] = t;
    }
}

// x = tok[t] + pos[p] (decode.rs:72-74) with t = inputs[p]: row t of a resident weight of
// k = d inputs, dequantised exactly as quant::decode.
template <int KIND>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ ds,
                                                    const float *__restrict__ pos_tab, const int32_t *__restrict__ state,
                                                    const int32_t *__restrict__ inputs, float *__restrict__ x,
                                                    uint32_t d) {
    const uint32_t p = (uint32_t)state[0];
    const uint32_t t = (uint32_t)inputs[p];
    const uint32_t nb = d / 32;
    for (uint32_t i = threadIdx.x; i < d; i += blockDim.x) {
        const uint32_t b = i / 32, j = i % 32;
        const size_t slot = tile_slot(t, b, nb);
        float q;
        if constexpr (KIND == FH_Q8_0) {
            q = (float)(int8_t)qs[slot * 32 + j];
        } else {
            const uint32_t byte = qs[slot * 16 + (j % 16)];
            q = (float)((int32_t)(j < 16 ? byte & 15u : byte >> 4) - 8);
        }
        const float v = half_bits_to_float(ds[scale_slot(t, b, nb)]) * q;
        x[i] = v + pos_tab[(size_t)p * d + i];
    }
}

// The greedy pick over the head's row-group offers (the first maximum; NaN never wins), then
// the step's bookkeeping: the pick becomes the next input when the position is past the prompt,
// and the position advances.
__global__ __launch_bounds__(1024) void pick_kernel(const float *__restrict__ offer_v, const uint32_t *__restrict__ offer_i,
                                                    uint32_t groups, int32_t *__restrict__ state,
                                                    int32_t *__restrict__ inputs) {
    __shared__ float sv[16];
    __shared__ uint32_t si[16];
    float bv = 0.0f;
    uint32_t bi = kNone;
    for (uint32_t q = threadIdx.x; q < groups; q += blockDim.x)
        if (better(offer_v[q], offer_i[q], bv, bi)) {
            bv = offer_v[q];
            bi = offer_i[q];
        }
#pragma unroll
    for (int o = 32; o >= 1; o /= 2) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (threadIdx.x % 64 == 0) {
        sv[threadIdx.x / 64] = bv;
        si[threadIdx.x / 64] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / 64; w++)
            if (better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        const int32_t pick = bi == kNone ? 0 : (int32_t)bi;
        const int32_t p = state[0];
        state[2] = pick;
        if (p + 1 >= state[1]) inputs[p + 1] = pick;
        state[0] = p + 1;
        state[3] = state[3] + 1;  // the step's epoch (one_step_kernel's counters)
    }
}

// One workgroup per head (decode.rs:81-105 over the cached positions 0..p). L = hd / 4 lanes
// share a cache row (a 16-byte load each), so a pass over the workgroup reads kAttnThreads / L
// rows at once; the lanes of a row add their parts with shuffles.
template <int L>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const float *__restrict__ q, const float *__restrict__ kc,
                                                                 const float *__restrict__ vc, const int32_t *__restrict__ state,
                                                                 float *__restrict__ out, uint32_t d, uint32_t ctx,
                                                                 float scale) {
    constexpr uint32_t hd = 4 * L, NR = kAttnThreads / L;
    extern __shared__ float alds[];
    float *s = alds;              // [ctx] scores, then probabilities
    float *accs = alds + ctx;     // [NR][hd] output partial sums
    float *red = accs + NR * hd;  // [2 * waves]
    const uint32_t h = blockIdx.x, T = (uint32_t)state[0] + 1, tid = threadIdx.x;
    const uint32_t li = tid % L, rg = tid / L;
    const f32x4 qv = gload4(q + h * hd + 4 * li);
    const float *kb = kc + h * hd + 4 * li;
    const float *vb = vc + h * hd + 4 * li;
    for (uint32_t j = rg; j < T; j += 2 * NR) {  // the L lanes of a row share the loop bound
        const bool two = j + NR < T;
        const f32x4 k0 = gload4(kb + (size_t)j * d);
        const f32x4 k1 = two ? gload4(kb + (size_t)(j + NR) * d) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float d0 = (qv.x * k0.x + qv.y * k0.y) + (qv.z * k0.z + qv.w * k0.w);
        float d1 = (qv.x * k1.x + qv.y * k1.y) + (qv.z * k1.z + qv.w * k1.w);
        d0 = group_reduce<L>(d0, AddOp());
        d1 = group_reduce<L>(d1, AddOp());
        if (li == 0) {
            s[j] = d0 * scale;
            if (two) s[j + NR] = d1 * scale;
        }
    }
    __syncthreads();
    constexpr uint32_t NW = kAttnThreads / 64;
    float m = -INFINITY;
    for (uint32_t j = tid; j < T; j += kAttnThreads) m = fmaxf(m, s[j]);
    m = wave_reduce(m, MaxOp());
    if (tid % 64 == 0) red[tid / 64] = m;
    __syncthreads();
    m = red[0];
    for (uint32_t w = 1; w < NW; w++) m = fmaxf(m, red[w]);
    float z = 0.0f;
    for (uint32_t j = tid; j < T; j += kAttnThreads) {
        const float e = expf(s[j] - m);
        s[j] = e;
        z += e;
    }
    z = wave_reduce(z, AddOp());
    if (tid % 64 == 0) red[NW + tid / 64] = z;
    __syncthreads();
    float sum = 0.0f;
    for (uint32_t w = 0; w < NW; w++) sum += red[NW + w];
    for (uint32_t j = tid; j < T; j += kAttnThreads) s[j] = s[j] / sum;
    __syncthreads();
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t j = rg; j < T; j += 2 * NR) {
        const bool two = j + NR < T;
        const f32x4 v0 = gload4(vb + (size_t)j * d);
        const f32x4 v1 = two ? gload4(vb + (size_t)(j + NR) * d) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const float p0 = s[j], p1 = two ? s[j + NR] : 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] += p0 * v0[c] + p1 * v1[c];
    }
    *(f32x4 *)&accs[rg * hd + 4 * li] = acc;
    __syncthreads();
    if (tid < hd) {
        float t = 0.0f;
        for (uint32_t g = 0; g < NR; g++) t += accs[g * hd + tid];
        out[h * hd + tid] = t;
    }
}

// ---- the four-launch step's own kernels ----
// attn_out_kernel (one workgroup per head h): a_h = softmax(q k^T / sqrt(hd)) v over the cached
// positions, then out_part[h] = a_h W_o[:, h] (the head's columns of the output projection). Its
// partial rows, and those of the FFN-down product split along K, are added in a fixed order by
// the next launch's prologue (residual_row), so a step's results do not depend on timing; no
// workgroup waits for another inside a launch.
constexpr int kStepThreads = 512;
constexpr int kStepWaves = kStepThreads / 64;
constexpr uint32_t kAttnSlots = 2 * kStepThreads / 16;  // attend_head: two floats per lane group (L >= 16)

// The second product's task for row group rg and head h: blocks b0 = h * 2 PAIRS .. b0 + 2 PAIRS - 1
// of its rows (b0 even, all in one run of eight scales).
template <int KIND, int PAIRS>
__device__ __forceinline__ void load_task2(Batch<KIND> &bt, const StepArgs &a, uint32_t h, uint32_t rg, uint32_t oq,
                                           uint32_t os) {
    constexpr uint32_t QB = KIND == FH_Q8_0 ? 32 : 16;
    const uint32_t nb2 = a.nb2, nb28 = (nb2 + 7) / 8, b0 = h * (2 * PAIRS);
    const auto rq = make_rsrc(a.qs2 + (size_t)rg * nb2 * 32 * QB, nb2 * 32 * QB);
    const auto rd = make_rsrc(a.ds2 + (size_t)rg * nb28 * 256, nb28 * 512);
    if constexpr (KIND == FH_Q8_0) {
#pragma unroll
        for (int i = 0; i < 2 * PAIRS; i++)
            bt.q[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(oq + (b0 + i) * 1024), 0, kWeightPolicy));
    } else {
#pragma unroll
        for (int i = 0; i < PAIRS; i++)
            bt.q[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(oq + (b0 + 2 * i) * 512), 0, kWeightPolicy));
    }
#pragma unroll
    for (int p = 0; p < PAIRS; p++)
        bt.s[p] = __builtin_amdgcn_raw_buffer_load_b32(rd, (int)(os + (b0 / 8) * 512 + ((b0 % 8) / 2 + p) * 4), 0, 0);
}

typedef __attribute__((address_space(3))) const uint8_t lds_byte;

// x operand and record tails of a batch whose records start at rec (LDS).
template <int KIND>
__device__ __forceinline__ void lds_operands(Batch<KIND> &bt, const uint8_t *rec, uint32_t oa, uint32_t ot) {
    lds_byte *lp = (lds_byte *)rec;
    bt.a = *(const __attribute__((address_space(3))) i32x4 *)(lp + oa);
    load_tails<KIND>(bt, 0, ot, [&](uint32_t off) { return *(const __attribute__((address_space(3))) u32x4 *)(lp + off); },
                     [&](uint32_t off) { return *(const __attribute__((address_space(3))) uint32_t *)(lp + off); });
}

// Row r's sum over both lane halves (lanes 0..31 hold it).
__device__ __forceinline__ float half_sum(float acc, bool upper) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
    return acc + __uint_as_float(upper ? sw[0] : sw[1]);
}

// The second product: row groups w, w + W, ... of the d rows, K in flight as above;
// out_part[h] gets head h's share of each row (COH: agent-coherent stores).
template <int KIND, int PAIRS, int K, bool COH = false>
__device__ __forceinline__ void run_tasks2(const StepArgs &a, uint32_t h, Batch<KIND> (&set)[K], const uint8_t *recs,
                                           uint32_t oq, uint32_t os, uint32_t oa, uint32_t ot) {
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64;
    const bool upper = lane >= 32;
    const uint32_t groups = a.d / 32;
    for (uint32_t base = wave; base < groups; base += K * kStepWaves) {
#pragma unroll
        for (int i = 0; i < K; i++) {
            const uint32_t rg = base + i * kStepWaves;
            if (rg < groups) {
                lds_operands<KIND>(set[i], recs, oa, ot);
                float acc = 0.0f;
                compute_batch<KIND, PAIRS>(set[i], upper, acc);
                const float sum = half_sum(acc, upper);
                if (!upper) {
                    if constexpr (COH)
                        cstore(a.out_part + (size_t)h * a.d + rg * 32 + lane, sum);
                    else
                        a.out_part[(size_t)h * a.d + rg * 32 + lane] = sum;
                }
                if (rg + K * kStepWaves < groups) load_task2<KIND, PAIRS>(set[i], a, h, rg + K * kStepWaves, oq, os);
            }
        }
    }
}

// Attention of one head over positions 0..T-1 (decode.rs:81-105) with q and the newest
// position's k and v rows (T - 1) given apart (they may not be in the caches yet); the result a
// (hd floats) goes to recs (LDS) as its prepared records. One pass over the caches: L = hd / 4 lanes share a cache row (a
// 16-byte load each of its k and v), a lane group takes U rows at a time with all their loads
// issued together and keeps a running maximum, sum and output (the softmax's max-subtracted
// exponentials, rescaled when the maximum grows); the groups of a wavefront then meet through
// lane exchanges and the wavefronts through LDS, each rescaled to the common maximum. Rows past T
// are read as row T - 1 and dropped. h: the head. pre: the first rows of the thread's lane group,
// requested ahead by attend_issue.
constexpr int kAttnU = 8;  // rows a lane group takes at a time
struct AttnRows {
    f32x4 k[kAttnU], v[kAttnU];
};

// attend_head's first rows of the thread's lane group (rows rg, rg + NR, ... below T - 1): the
// cached rows below the newest position do not change during a step, so they can be requested
// before the newest row and q exist.
template <int L>
__device__ __forceinline__ void attend_issue(uint32_t h, const float *kc, const float *vc, uint32_t T, uint32_t d,
                                             AttnRows &pre) {
    constexpr uint32_t hd = 4 * L, NR = kStepThreads / L;
    const uint32_t li = threadIdx.x % L, rg = threadIdx.x / L, last = T - 1;
    const float *kb = kc + h * hd + 4 * li;
    const float *vb = vc + h * hd + 4 * li;
#pragma unroll
    for (int u = 0; u < kAttnU; u++) {
        const uint32_t j = min(rg + u * NR, last);
        pre.k[u] = j < last ? gload4(kb + (size_t)j * d) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        pre.v[u] = j < last ? gload4(vb + (size_t)j * d) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

template <int KIND, int L>
__device__ __forceinline__ void attend_head(uint32_t h, const float *qh, const float *knew, const float *vnew,
                                             const float *kc, const float *vc, uint32_t T, uint32_t d, float scale,
                                             float *s, float *accs, float *red, uint8_t *recs, const AttnRows &pre) {
    constexpr uint32_t hd = 4 * L, NR = kStepThreads / L;
    constexpr int U = kAttnU;
    const uint32_t tid = threadIdx.x;
    const uint32_t li = tid % L, rg = tid / L, last = T - 1;
    (void)red;
    const f32x4 qv = *(const f32x4 *)(qh + 4 * li);
    const float *kb = kc + h * hd + 4 * li;
    const float *vb = vc + h * hd + 4 * li;
    const f32x4 kl = *(const f32x4 *)(knew + 4 * li), vl = *(const f32x4 *)(vnew + 4 * li);
    float m = -INFINITY, z = 0.0f;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // rows j0, j0 + NR, ... (row T - 1 and those past it: the newest row, dropped past T). Rows
    // past T are skipped (branches uniform over a lane group): their weight would be exp(-inf) = 0,
    // which adds nothing.
    auto chunk = [&](uint32_t j0, const f32x4 (&kr)[U], const f32x4 (&vr)[U]) {
        float sc[U];
        float mc = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; u++) {
            sc[u] = -INFINITY;
            if (j0 + u * NR < T) {
                float dt = (qv.x * kr[u].x + qv.y * kr[u].y) + (qv.z * kr[u].z + qv.w * kr[u].w);
                dt = group_reduce<L>(dt, AddOp());
                sc[u] = dt * scale;
            }
            mc = fmaxf(mc, sc[u]);
        }
        const float mn = fmaxf(m, mc);  // finite: row j0 < T is in the chunk
        const float corr = expf(m - mn);
        z *= corr;
        acc *= corr;
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (j0 + u * NR < T) {
                const float e = expf(sc[u] - mn);
                z += e;
#pragma unroll
                for (int c = 0; c < 4; c++) acc[c] += e * vr[u][c];
            }
        }
        m = mn;
    };
    if (rg < T) {  // the first rows: requested ahead (the L lanes of a row share the bounds)
        f32x4 kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool nw = min(rg + u * NR, last) == last;
            kr[u] = nw ? kl : pre.k[u];
            vr[u] = nw ? vl : pre.v[u];
        }
        chunk(rg, kr, vr);
    }
    for (uint32_t j0 = rg + U * NR; j0 < T; j0 += U * NR) {
        f32x4 kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t j = min(j0 + u * NR, last);
            kr[u] = j == last ? kl : gload4(kb + (size_t)j * d);
            vr[u] = j == last ? vl : gload4(vb + (size_t)j * d);
        }
        chunk(j0, kr, vr);
    }
    // the wavefront's groups pairwise (lanes li + L, li + 2L, ...), at the larger maximum; groups
    // with no rows (maximum -inf) add nothing
#pragma unroll
    for (uint32_t o = L; o < 64; o *= 2) {
        const float mo = __shfl_xor(m, o, 64), zo = __shfl_xor(z, o, 64);
        f32x4 ao;
#pragma unroll
        for (int c = 0; c < 4; c++) ao[c] = __shfl_xor(acc[c], o, 64);
        const float mn = fmaxf(m, mo);
        const float fa = m == -INFINITY ? 0.0f : expf(m - mn), fb = mo == -INFINITY ? 0.0f : expf(mo - mn);
        z = z * fa + zo * fb;
        acc = acc * fa + ao * fb;
        m = mn;
    }
    // then the wavefronts: their maxima, then each one's sum and output at the common maximum
    constexpr uint32_t NW = kStepThreads / 64;
    const uint32_t wv = tid / 64, lw = tid % 64;
    if (lw == 0) s[wv] = m;
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (uint32_t g = 0; g < NW; g++) M = fmaxf(M, s[g]);
    const float f = m == -INFINITY ? 0.0f : expf(m - M);
    if (lw < L) *(f32x4 *)&accs[wv * hd + 4 * li] = acc * f;
    if (lw == 0) s[NW + wv] = z * f;
    __syncthreads();
    // the output a = (sum of the wavefronts' outputs) / (sum of their sums), straight into the
    // prepared records of its hd / 32 blocks (eight records, zero past them; wavefront 0's lanes,
    // eight a block)
    if (tid < 64) {
        const uint32_t blk = tid / 8;
        const int j = (int)(tid % 8);
        auto *rec = (__attribute__((address_space(3))) uint32_t *)(recs + blk * kPrepBytes);
        if (blk < hd / 32) {
            float zs = 0.0f;
            f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t g = 0; g < NW; g++) {
                zs += s[NW + g];
                t += *(const f32x4 *)&accs[g * hd + blk * 32 + 4 * j];
            }
            f32x4 o;
#pragma unroll
            for (int c = 0; c < 4; c++) o[c] = t[c] / zs;
            prep_values<KIND>(o, j, rec);
        } else {
            zero_record(j, rec);
        }
    }
}

// LDS of attn_out_kernel: the lane groups' maxima and sums, output partials, reduction slots, the
// head's output, its prepared records.
__host__ __device__ inline uint32_t attn_out_lds(uint32_t hd) {
    return kAttnSlots * 4 + kStepThreads * 16 + 2 * kStepWaves * 4 + hd * 4 + 8 * kPrepBytes;
}

// Attention of head blockIdx.x over the cached positions 0..p (the query row and the caches
// written by the QKV launch), then the head's columns of the output projection:
// out_part[h] = a_h W_o[:, h] (hd = 4 L, PAIRS = hd / 64); the weights are requested first.
template <int KIND, int L, int K2>
__global__ __launch_bounds__(kStepThreads) void attn_out_kernel(StepArgs a) {
    constexpr int PAIRS = L / 16;
    constexpr uint32_t hd = 4 * L;
    extern __shared__ __attribute__((aligned(16))) uint8_t flds[];
    float *s = (float *)flds;
    float *accs = s + kAttnSlots;
    float *red = accs + kStepThreads * 4;
    float *att = red + 2 * kStepWaves;
    uint8_t *recs2 = (uint8_t *)(att + hd);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64, r = lane % 32;
    const uint32_t oq = KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * (lane >= 32)) : (uint32_t)(lane * 16);
    const uint32_t os = (uint32_t)(r * 16), oa = prep_a_offset(lane), ot = prep_tail_offset<KIND>(lane);
    Batch<KIND> s2[K2];
#pragma unroll
    for (int i = 0; i < K2; i++)
        if (wave + i * kStepWaves < a.d / 32) load_task2<KIND, PAIRS>(s2[i], a, blockIdx.x, wave + i * kStepWaves, oq, os);
    const uint32_t p = (uint32_t)a.state[0];
    const size_t off = (size_t)blockIdx.x * hd;
    AttnRows pre;
    attend_issue<L>(blockIdx.x, a.kc, a.vc, p + 1, a.d, pre);
    attend_head<KIND, L>(blockIdx.x, a.q + off, a.kc + (size_t)p * a.d + off, a.vc + (size_t)p * a.d + off, a.kc, a.vc,
                         p + 1, a.d, a.scale, s, accs, red, recs2, pre);
    __syncthreads();
    run_tasks2<KIND, PAIRS, K2>(a, blockIdx.x, s2, recs2, oq, os, oa, ot);
}

// After the last layer: x = x_in + (sum_j part[j] + b) and its final LayerNorm into global
// prepared records (the head's x); one workgroup.
template <int KIND>
__global__ __launch_bounds__(kStepThreads) void final_ln_kernel(StepArgs a, uint8_t *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) float red[kLnRed];
    f32x4 v[kLnSlots];
    residual_row<KIND>(a, v);
    ln_records<KIND, true>(v, a.ln_g, a.ln_b, a.eps, a.nb, (a.nb + 7) / 8 * 8, out, red);
}

// ---- the one-launch step: every layer in one launch ----
// In the four-launch step each launch costs about 2 us of dispatch gap (the last workgroup's end to
// the next launch's first workgroup, measured with wall-clock stamps inside the kernels) before
// its first dependent load even leaves; with 48 launches per token that is a third of the step.
// Here one launch runs all the layers. Each workgroup keeps one role through the layers: a QKV row
// group (nA of them), an attention head with its output-projection columns (nB), an FFN-up row
// group (nC) or an FFN-down task (nD: row group x K split), exactly the four-launch step's
// workgroups with the same lane-level arithmetic, so a step's results are the same bit for bit.
// Between phases a workgroup requests its next task's weights, then waits for the phase it
// depends on: a completion counter per layer and phase, which every task of the phase
// increments once its stores have landed, polled by one lane with agent-scope loads. What one
// phase writes and a later phase of the same launch reads is stored with agent-coherent stores,
// each address once per launch (every buffer has a copy per layer), and read with ordinary loads:
// no L2 can hold an older copy, so no cache-wide release or acquire is needed (with 240
// workgroups each fencing four times per layer, L2 write-backs and invalidations made the step
// 2.7x slower; reading the shared rows with coherent loads instead, 1.6x slower: every workgroup
// then fetched them past its L2). The counters only grow: the step
// with epoch e (state[3], advanced by the pick) waits for (e + 1) x the phase's tasks. Every wait
// is bounded: after kSpinLimit polls (about a second), or once another workgroup has given up,
// it sets the error flag and goes on, so every wavefront reaches its end; the host reports the
// flag. The launch needs all of its workgroups resident at once: the host takes this form only
// where the occupancy query says they fit.
struct OneLayer {  // one layer's operands and buffers (a device table, read with scalar loads)
    const uint8_t *qkv_qs, *o_qs, *w1_qs, *w2_qs;
    const uint16_t *qkv_ds, *o_ds, *w1_ds, *w2_ds;
    const float *ln1_g, *ln1_b, *bqkv, *bo, *ln2_g, *ln2_b, *b1, *b2;
    float *kc, *vc;
    // this layer's copies of the step's buffers: the query row, the residual rows before and after
    // the attention block, the attention's and FFN-down's partial rows, the FFN activation
    float *q, *xc, *xm, *po, *pf, *f;
};

struct OneArgs {
    const OneLayer *layers;
    uint32_t n_layers;
    const uint8_t *emb_qs;
    const uint16_t *emb_ds;
    const float *pos_tab;
    int32_t *inputs;
    int32_t *state;
    float *x_final;
    const float *lnf_g, *lnf_b;
    const uint8_t *head_qs;  // the head (tied: the token embedding), vocab rows of d
    const uint16_t *head_ds;
    uint32_t vocab;
    float *logits;
    uint64_t *offers;  // per head row group: its first maximum (value bits, row << 32)
    uint32_t *sync;  // completion counters, [n_layers][slots] (one_counter), then the error flag, the head ticket
    uint32_t d, hidden, heads, S, chunk_down;
    float eps, scale;
    uint32_t nA, nB, nC, nD;
    uint32_t slots;  // counters per layer: heads (QKV, one per head) + 1 (attention) + S (FFN-up, one per
                     // FFN-down K chunk) + 1 (FFN-down)
};
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kOneMaxLayers = 256;
// Every counter has kCopies copies, a cache line apart, each incremented by every task of its phase
// (one lane per copy); workgroup w polls copy w % kCopies. With one copy, about a hundred workgroups
// polling one address while the tasks' atomics queued behind them made the step 1.5x slower than
// with 8 copies. Measured on GPT-2-small (us per step): 16 copies 207.5, 32 copies 204.5, 64
// copies 202.1, 128 copies 204.1, 256 copies 217.7 (each task's 256 atomics then cost more than the
// pollers they spread). Four wavefronts polling each (staggered) cost 20 us: polls are not free.
constexpr uint32_t kCopies = 64, kCopyStride = 32;  // (in uint32_t)
constexpr uint32_t kCounter = kCopies * kCopyStride;  // uint32_t per counter
__host__ __device__ constexpr uint32_t one_counter(uint32_t l, uint32_t slot, uint32_t slots) {
    return (l * slots + slot) * kCounter;
}

// Waits until the counter at cnt reaches target (wrapping compare), bounded as above.
__device__ __forceinline__ void one_wait(uint32_t *cnt, uint32_t target, uint32_t *err) {
    cnt += (blockIdx.x % kCopies) * kCopyStride;
    if (threadIdx.x == 0) {
        uint32_t n = 0;
        while ((int32_t)(__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
            if ((++n & 63u) == 0 &&
                (n >= kSpinLimit || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// After the task's agent-coherent stores (each wavefront that stored waited for them): one increment
// of the counter.
__device__ __forceinline__ void one_signal(uint32_t *cnt) {
    __syncthreads();
    if (threadIdx.x < kCopies)
        __hip_atomic_fetch_add(cnt + threadIdx.x * kCopyStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KIND>
struct OneGemv {  // a decode-GEMV task's requested first batch and bias; PRO_LNR: its LayerNorm's
                  // gain and bias and the residual row's bias (one_issue_ln)
    Batch<KIND> cur;
    float pre_bias;
    LnParams ln;
    f32x4 rb[kLnSlots];
};

// Requests task (g, sp)'s first batch (wavefront w: blocks b0 + 8 w ..) and the lane's bias, as
// decode_gemv_kernel does at its start.
template <int KIND>
__device__ __forceinline__ void one_issue(const DecodeGemv &a, uint32_t g, uint32_t sp, OneGemv<KIND> &t) {
    constexpr uint32_t QB = KIND == FH_Q8_0 ? 32 : 16;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64, r = lane % 32;
    const bool upper = lane >= 32;
    const uint32_t nb = a.nb, nb8 = (nb + 7) / 8, span = nb8 * 8;
    const uint32_t b0 = sp * a.chunk, b1 = min(span, b0 + a.chunk);
    const auto rq = make_rsrc(a.qs + (size_t)g * nb * 32 * QB, nb * 32 * QB);
    const auto rd = make_rsrc(a.ds + (size_t)g * nb8 * 256, nb8 * 512);
    const uint32_t oq = KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * upper) : (uint32_t)(lane * 16);
    const uint32_t bb = b0 + wave * kBatch;
    if (bb < b1) load_weights<KIND>(t.cur, rq, rd, oq, (uint32_t)(r * 16), bb);
    t.pre_bias = 0.0f;
    if (wave == 0 && !upper && g * 32 + r < a.n && a.bias) t.pre_bias = a.bias[g * 32 + r];
}

// PRO_LNR: requests the LayerNorm's gain and bias and the residual row's bias (constants of the
// model, so they can be read before the wait for the row).
template <int KIND>
__device__ __forceinline__ void one_issue_ln(const DecodeGemv &a, OneGemv<KIND> &t) {
    load_ln(a.ln_g, a.ln_b, a.nb, t.ln);
    if (a.x_in) {
#pragma unroll
        for (uint32_t u = 0; u < kLnSlots; u++) {
            const uint32_t sl = threadIdx.x + u * blockDim.x;
            if (sl / 8 < a.nb) t.rb[u] = gload4(a.rbias + sl * 4);
        }
    }
}

// The rest of decode_gemv_kernel's task (g, sp) for PRO_LNR / PRO_NONE and EPI_QKV / EPI_GELU /
// EPI_PARTIAL, with the workgroup's eight wavefronts (those past the task's batches add zeros,
// after the others, so the sums are those of the narrower launch). store_x: this task stores the
// residual row at a.x_out. Outputs are written with agent-coherent stores; each wavefront that
// stored waits until its stores have landed.
template <int KIND, int PRO, int EPI>
__device__ __forceinline__ void one_run(const DecodeGemv &a, uint32_t g, uint32_t sp, OneGemv<KIND> &t, uint8_t *lds,
                                        bool store_x) {
    constexpr uint32_t QB = KIND == FH_Q8_0 ? 32 : 16;
    constexpr uint32_t W = kStepWaves;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64, r = lane % 32;
    const bool upper = lane >= 32;
    const uint32_t nb = a.nb, nb8 = (nb + 7) / 8, span = nb8 * 8;
    const uint32_t b0 = sp * a.chunk, b1 = min(span, b0 + a.chunk);
    const auto rq = make_rsrc(a.qs + (size_t)g * nb * 32 * QB, nb * 32 * QB);
    const auto rd = make_rsrc(a.ds + (size_t)g * nb8 * 256, nb8 * 512);
    const uint32_t oq = KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * upper) : (uint32_t)(lane * 16);
    const uint32_t os = (uint32_t)(r * 16), oa = prep_a_offset(lane), ot = prep_tail_offset<KIND>(lane);
    constexpr bool kLn = PRO == PRO_LNR;
    uint8_t *prep = lds;
    float *part = (float *)(lds + (kLn ? span : a.chunk) * kPrepBytes);
    float *red = part + W * 32;
    f32x4 v[kLnSlots];
    if constexpr (kLn) {
        StepArgs f{};
        f.x_in = a.x_in;
        f.part = a.rpart;
        f.pbias = a.rbias;
        f.nparts = a.nparts;
        f.emb_qs = a.emb_qs;
        f.emb_ds = a.emb_ds;
        f.pos_tab = a.pos_tab;
        f.inputs = a.inputs;
        f.state = a.state;
        f.x_out = nullptr;  // stored at the end (store_x)
        f.d = nb * 32;
        f.nb = nb;
        residual_row<KIND>(f, v, t.rb);
        ln_records_p<KIND, false>(v, t.ln, a.eps, nb, span, prep, red);
    } else {
        for (uint32_t blk = b0 + threadIdx.x / 8; blk < b1; blk += blockDim.x / 8) {
            const int j = threadIdx.x % 8;
            __attribute__((address_space(3))) uint32_t *rec =
                (__attribute__((address_space(3))) uint32_t *)(prep + (blk - b0) * kPrepBytes);
            if (blk < nb)
                prep_values<KIND>(gload4(a.x + blk * 32 + 4 * j), j, rec);
            else
                zero_record(j, rec);
        }
    }
    __syncthreads();
    const uint32_t pbase = kLn ? 0 : b0;
    float acc = 0.0f;
    uint32_t bb = b0 + wave * kBatch;
    Batch<KIND> nx;
    while (bb < b1) {
        const uint32_t nxt = bb + W * kBatch;
        if (nxt < b1) load_weights<KIND>(nx, rq, rd, oq, os, nxt);
        lds_byte *lp = (lds_byte *)prep;
        t.cur.a = *(const __attribute__((address_space(3))) i32x4 *)(lp + (bb - pbase) * kPrepBytes + oa);
        load_tails<KIND>(t.cur, (bb - pbase) * kPrepBytes, ot,
                         [&](uint32_t off) { return *(const __attribute__((address_space(3))) u32x4 *)(lp + off); },
                         [&](uint32_t off) { return *(const __attribute__((address_space(3))) uint32_t *)(lp + off); });
        compute_batch<KIND>(t.cur, upper, acc);
        t.cur = nx;
        bb = nxt;
    }
    const float sum = half_sum(acc, upper);
    if (!upper) part[wave * 32 + r] = sum;
    __syncthreads();
    if (wave == 0 && !upper) {
        float s = 0.0f;
        for (uint32_t w = 0; w < W; w++) s += part[w * 32 + r];
        const uint32_t row = g * 32 + r;
        if (row < a.n) {
            if constexpr (EPI == EPI_PARTIAL) {
                cstore(a.y + (size_t)sp * a.n + row, s);
            } else {
                if (a.bias) s = s + t.pre_bias;
                if constexpr (EPI == EPI_GELU) {
                    cstore(a.y + row, gelu(s));
                } else {
                    const uint32_t p = (uint32_t)a.state[0];
                    if (row < a.split)
                        cstore(a.y + row, s);
                    else if (row < 2 * a.split)
                        cstore(a.kc + (size_t)p * a.split + row - a.split, s);
                    else
                        cstore(a.vc + (size_t)p * a.split + row - 2 * a.split, s);
                }
            }
        }
    }
    if (store_x) {
#pragma unroll
        for (uint32_t u = 0; u < kLnSlots; u++) {
            const uint32_t sl = threadIdx.x + u * blockDim.x;
            if (sl / 8 < nb) cstore4(a.x_out + sl * 4, v[u]);
        }
    }
    if (wave == 0 || store_x) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the stores have landed
}

// One layer of a role (the arguments live in device memory and are read with scalar loads, which
// keeps the kernel's scalar registers free). e1: this step's counter multiple; lds: the
// workgroup's dynamic LDS.
template <int KIND>
__device__ __forceinline__ void one_qkv(const OneArgs *A, uint32_t l, uint32_t task, uint32_t e1, uint8_t *lds) {
    // LN1 + QKV (layer 0: the embedding), as dgemv<PRO_LNR, EPI_QKV>
    const OneLayer &Y = A->layers[l];
    const uint32_t d = A->d, nb = d / 32;
    DecodeGemv g{};
    g.qs = Y.qkv_qs;
    g.ds = Y.qkv_ds;
    g.nb = nb;
    g.n = 3 * d;
    g.chunk = (nb + 7) / 8 * 8;
    g.bias = Y.bqkv;
    g.y = Y.q;
    g.kc = Y.kc;
    g.vc = Y.vc;
    g.split = d;
    g.state = A->state;
    g.inputs = A->inputs;
    g.ln_g = Y.ln1_g;
    g.ln_b = Y.ln1_b;
    g.eps = A->eps;
    g.x_out = Y.xc;
    if (l == 0) {
        g.emb_qs = A->emb_qs;
        g.emb_ds = A->emb_ds;
        g.pos_tab = A->pos_tab;
    } else {
        g.x_in = A->layers[l - 1].xm;
        g.rpart = A->layers[l - 1].pf;
        g.rbias = A->layers[l - 1].b2;
        g.nparts = A->S;
    }
    OneGemv<KIND> t;
    one_issue<KIND>(g, task, 0, t);
    one_issue_ln<KIND>(g, t);
    const uint32_t H = A->heads, S = A->S, Z = A->slots;
    if (l > 0) one_wait(A->sync + one_counter(l - 1, H + 1 + S, Z), e1 * A->nD, A->sync + one_counter(A->n_layers, 0, Z));
    one_run<KIND, PRO_LNR, EPI_QKV>(g, task, 0, t, lds, task == 0);
    one_signal(A->sync + one_counter(l, (task * 32 % d) / (d / H), Z));  // this row group's head
}

template <int KIND, int L, int K2>
__device__ __forceinline__ void one_attn(const OneArgs *A, uint32_t l, uint32_t task, uint32_t e1, uint8_t *lds) {
    // attention of head `task` + its output-projection columns, as attn_out_kernel
    constexpr int PAIRS = L / 16;
    constexpr uint32_t hd = 4 * L;
    const OneLayer &Y = A->layers[l];
    const uint32_t d = A->d, nb = d / 32;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64, r = lane % 32;
    StepArgs sa{};
    sa.q = Y.q;
    sa.kc = Y.kc;
    sa.vc = Y.vc;
    sa.state = A->state;
    sa.d = d;
    sa.nb = nb;
    sa.scale = A->scale;
    sa.qs2 = Y.o_qs;
    sa.ds2 = Y.o_ds;
    sa.nb2 = nb;
    sa.out_part = Y.po;
    const uint32_t oq = KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * (lane >= 32)) : (uint32_t)(lane * 16);
    const uint32_t os = (uint32_t)(r * 16), oa = prep_a_offset(lane), ot = prep_tail_offset<KIND>(lane);
    Batch<KIND> s2[K2];
#pragma unroll
    for (int i = 0; i < K2; i++)
        if (wave + i * kStepWaves < nb) load_task2<KIND, PAIRS>(s2[i], sa, task, wave + i * kStepWaves, oq, os);
    const uint32_t p = (uint32_t)A->state[0];  // (the pick at the step's end advances it)
    AttnRows pre;
    // the first cache rows before the wait (with head width 256 after it: their registers on top of
    // the W_o sets' would spill)
    if constexpr (L < 64) attend_issue<L>(task, Y.kc, Y.vc, p + 1, d, pre);
    // the head's q, k and v row groups
    one_wait(A->sync + one_counter(l, task, A->slots), e1 * 3 * (hd / 32), A->sync + one_counter(A->n_layers, 0, A->slots));
    if constexpr (L >= 64) attend_issue<L>(task, Y.kc, Y.vc, p + 1, d, pre);
    float *s = (float *)lds;
    float *accs = s + kAttnSlots;
    float *red = accs + kStepThreads * 4;
    float *att = red + 2 * kStepWaves;
    uint8_t *recs2 = (uint8_t *)(att + hd);
    const size_t off = (size_t)task * hd;
    attend_head<KIND, L>(task, Y.q + off, Y.kc + (size_t)p * d + off, Y.vc + (size_t)p * d + off, Y.kc, Y.vc, p + 1, d,
                         A->scale, s, accs, red, recs2, pre);
    __syncthreads();
    run_tasks2<KIND, PAIRS, K2, true>(sa, task, s2, recs2, oq, os, oa, ot);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial rows have landed
    one_signal(A->sync + one_counter(l, A->heads, A->slots));
}

template <int KIND>
__device__ __forceinline__ void one_up(const OneArgs *A, uint32_t l, uint32_t task, uint32_t e1, uint8_t *lds) {
    // LN2 + FFN-up + GELU, as dgemv<PRO_LNR, EPI_GELU>
    const OneLayer &Y = A->layers[l];
    const uint32_t nb = A->d / 32;
    DecodeGemv g{};
    g.qs = Y.w1_qs;
    g.ds = Y.w1_ds;
    g.nb = nb;
    g.n = A->hidden;
    g.chunk = (nb + 7) / 8 * 8;
    g.bias = Y.b1;
    g.y = Y.f;
    g.state = A->state;
    g.ln_g = Y.ln2_g;
    g.ln_b = Y.ln2_b;
    g.eps = A->eps;
    g.x_in = Y.xc;
    g.rpart = Y.po;
    g.rbias = Y.bo;
    g.nparts = A->heads;
    g.x_out = Y.xm;
    OneGemv<KIND> t;
    one_issue<KIND>(g, task, 0, t);
    one_issue_ln<KIND>(g, t);
    one_wait(A->sync + one_counter(l, A->heads, A->slots), e1 * A->nB, A->sync + one_counter(A->n_layers, 0, A->slots));
    one_run<KIND, PRO_LNR, EPI_GELU>(g, task, 0, t, lds, task == 0);
    // the FFN-down K chunk this row group of f belongs to
    one_signal(A->sync + one_counter(l, A->heads + 1 + task * 32 / A->chunk_down / 32, A->slots));
}

template <int KIND>
__device__ __forceinline__ void one_down(const OneArgs *A, uint32_t l, uint32_t task, uint32_t e1, uint8_t *lds) {
    // FFN-down task (row group, K split), as dgemv<PRO_NONE, EPI_PARTIAL>
    const OneLayer &Y = A->layers[l];
    const uint32_t gd = A->d / 32;
    DecodeGemv g{};
    g.qs = Y.w2_qs;
    g.ds = Y.w2_ds;
    g.nb = A->hidden / 32;
    g.n = A->d;
    g.chunk = A->chunk_down;
    g.x = Y.f;
    g.y = Y.pf;
    g.state = A->state;
    const uint32_t rg = task % gd, sp = task / gd;
    OneGemv<KIND> t;
    one_issue<KIND>(g, rg, sp, t);
    // the FFN-up row groups of this task's K chunk
    const uint32_t cb = A->chunk_down, in_chunk = min(cb, A->hidden / 32 - sp * cb);
    one_wait(A->sync + one_counter(l, A->heads + 1 + sp, A->slots), e1 * in_chunk,
             A->sync + one_counter(A->n_layers, 0, A->slots));
    one_run<KIND, PRO_NONE, EPI_PARTIAL>(g, rg, sp, t, lds, false);
    one_signal(A->sync + one_counter(l, A->heads + 1 + A->S, A->slots));
}

constexpr uint32_t kHeadPre = 3;  // head batches each wavefront has requested ahead
// The most head items (row group, batch) a workgroup takes: groups row groups over G workgroups.
__host__ __device__ inline uint32_t one_head_items(uint32_t groups, uint32_t G, uint32_t nb8) {
    return (groups + G - 1) / G * nb8;
}

// The head, folded into the step (decode_gemv_kernel<PRO_GLOBAL, EPI_ARGMAX> and pick_kernel):
// every workgroup with head row groups forms x = x_m + (the down partial rows + b_2) and its final
// LayerNorm into its own LDS records (workgroup 0 also stores x), then takes row groups w, w + G,
// ... as items (row group, batch of eight blocks) spread over its eight wavefronts, each with
// kHeadPre items requested ahead (the first ones before the wait), so that every wavefront keeps
// loads in flight; a group's batch sums are added in batch order as the four-launch head adds its
// wavefronts' (d <= 2048: one batch per wavefront there). The logits go to A->logits and each
// group's offer (its first maximum; NaN never wins) to A->offers with agent-coherent stores. A
// ticket counts the finished workgroups; the last one picks the next token over the offers as
// pick_kernel does and advances the state (position, input, epoch).
template <int KIND>
__device__ __forceinline__ void one_head(const OneArgs *A, uint32_t e1, uint8_t *lds, uint32_t w, uint32_t G) {
    const uint32_t d = A->d, nb = d / 32, nb8 = (nb + 7) / 8, span = nb8 * 8, L = A->n_layers;
    const uint32_t groups = (A->vocab + 31) / 32;
    uint32_t *err = A->sync + one_counter(L, 0, A->slots);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64, r = lane % 32;
    const bool upper = lane >= 32;
    DecodeGemv g{};
    g.qs = A->head_qs;
    g.ds = A->head_ds;
    g.nb = nb;
    g.n = A->vocab;
    g.chunk = span;
    g.state = A->state;
    g.ln_g = A->lnf_g;
    g.ln_b = A->lnf_b;
    g.x_in = A->layers[L - 1].xm;
    g.rbias = A->layers[L - 1].b2;
    // the workgroup's row groups w, w + G, ... (K of them) as items (group k, batch b), i = k nb8 + b,
    // wavefront v taking items v, v + 8, ... with kHeadPre of them requested ahead
    constexpr uint32_t QB = KIND == FH_Q8_0 ? 32 : 16;
    const uint32_t K = w < groups ? (groups - w + G - 1) / G : 0, items = K * nb8;
    const uint32_t oq = KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * upper) : (uint32_t)(lane * 16);
    const uint32_t os = (uint32_t)(r * 16), oa = prep_a_offset(lane), ot = prep_tail_offset<KIND>(lane);
    auto issue = [&](Batch<KIND> &b, uint32_t i) {
        const uint32_t rg = w + (i / nb8) * G;
        load_weights<KIND>(b, make_rsrc(g.qs + (size_t)rg * nb * 32 * QB, nb * 32 * QB),
                           make_rsrc(g.ds + (size_t)rg * nb8 * 256, nb8 * 512), oq, os, (i % nb8) * kBatch);
    };
    Batch<KIND> hb[kHeadPre];
#pragma unroll
    for (uint32_t p = 0; p < kHeadPre; p++)
        if (wave + p * kStepWaves < items) issue(hb[p], wave + p * kStepWaves);
    OneGemv<KIND> t;
    if (w < groups) one_issue_ln<KIND>(g, t);
    one_wait(A->sync + one_counter(L - 1, A->heads + 1 + A->S, A->slots), e1 * A->nD, err);
    uint8_t *prep = lds;
    float *part = (float *)(lds + span * kPrepBytes);  // [items][32]
    float *red = part + one_head_items(groups, G, nb8) * 32;
    if (w < groups) {
        StepArgs z{};
        z.x_in = A->layers[L - 1].xm;
        z.part = A->layers[L - 1].pf;
        z.pbias = A->layers[L - 1].b2;
        z.nparts = A->S;
        z.state = A->state;
        z.x_out = A->x_final;  // (workgroup 0 stores it)
        z.d = d;
        z.nb = nb;
        f32x4 v[kLnSlots];
        residual_row<KIND>(z, v, t.rb);
        ln_records_p<KIND, false>(v, t.ln, A->eps, nb, span, prep, red);
        __syncthreads();
        lds_byte *lp = (lds_byte *)prep;
        for (uint32_t base = wave; base < items; base += kHeadPre * kStepWaves) {
#pragma unroll
            for (uint32_t p = 0; p < kHeadPre; p++) {
                const uint32_t i = base + p * kStepWaves;
                if (i < items) {
                    const uint32_t bb = (i % nb8) * kBatch;
                    hb[p].a = *(const __attribute__((address_space(3))) i32x4 *)(lp + bb * kPrepBytes + oa);
                    load_tails<KIND>(hb[p], bb * kPrepBytes, ot,
                                     [&](uint32_t off) { return *(const __attribute__((address_space(3))) u32x4 *)(lp + off); },
                                     [&](uint32_t off) { return *(const __attribute__((address_space(3))) uint32_t *)(lp + off); });
                    float acc = 0.0f;
                    compute_batch<KIND>(hb[p], upper, acc);
                    const float sum = half_sum(acc, upper);
                    if (!upper) part[i * 32 + r] = sum;
                    if (i + kHeadPre * kStepWaves < items) issue(hb[p], i + kHeadPre * kStepWaves);
                }
            }
        }
        __syncthreads();
        // row group k in wavefront k % 8: its batches' sums in batch order (the four-launch head's
        // idle wavefronts add zeros), the logits, and the group's offer
        for (uint32_t k = wave; k < K; k += kStepWaves) {
            if (upper) continue;
            float s = 0.0f;
            for (uint32_t b = 0; b < kStepWaves; b++) s += b < nb8 ? part[(k * nb8 + b) * 32 + r] : 0.0f;
            const uint32_t rg = w + k * G, row = rg * 32 + r;
            if (row < A->vocab) A->logits[row] = s;
            float bv = s;
            uint32_t bi = (row < A->vocab && s == s) ? row : kNone;
#pragma unroll
            for (int o = 16; o >= 1; o /= 2) {
                const float ov = __shfl_xor(bv, o, 32);
                const uint32_t oi = __shfl_xor(bi, o, 32);
                if (better(ov, oi, bv, bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (r == 0) {
                __hip_atomic_store((g_u64 *)(A->offers + rg), (uint64_t)bi << 32 | __float_as_uint(bv), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this workgroup's offers have landed
    __syncthreads();
    uint32_t *flag = (uint32_t *)red;
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(A->sync + one_counter(L, 1, A->slots), 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        flag[0] = old + 1 == e1 * G ? 1u : 0u;
    }
    __syncthreads();
    if (!flag[0]) return;
    // the last workgroup: pick_kernel over the offers (written in this launch: agent-coherent loads)
    float bv = 0.0f;
    uint32_t bi = kNone;
    for (uint32_t q = threadIdx.x; q < groups; q += blockDim.x) {
        const uint64_t o = __hip_atomic_load((g_u64 *)(A->offers + q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float ov = __uint_as_float((uint32_t)o);
        const uint32_t oi = (uint32_t)(o >> 32);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o /= 2) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    float *sv = part;
    uint32_t *si = (uint32_t *)(part + kStepWaves);
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (uint32_t k = 1; k < kStepWaves; k++)
        if (better(sv[k], si[k], bv, bi)) {
            bv = sv[k];
            bi = si[k];
        }
    const int32_t pick = bi == kNone ? 0 : (int32_t)bi;
    int32_t *state = A->state;
    const int32_t p = state[0];
    state[2] = pick;
    if (p + 1 >= state[1]) A->inputs[p + 1] = pick;
    state[0] = p + 1;
    state[3] = state[3] + 1;  // the step's epoch
}

// One decode step: the whole layer stack, then the head and the greedy pick (one_head). The first max(nA, nC) workgroups take QKV task w and FFN-up task w, the next
// max(nB, nD) attention head t and FFN-down task t: each pair of roles is one phase apart in both
// directions (QKV, then attention, FFN-up, FFN-down, the next layer's QKV), so a workgroup's next
// weights are requested a phase before they are needed. A workgroup runs its tasks in the phases'
// order, and a phase waits only for earlier phases, so with every workgroup resident each wait
// ends.
template <int KIND, int L, int K2>
__global__ __launch_bounds__(kStepThreads) void one_step_kernel(const OneArgs *__restrict__ A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t olds[];
    const uint32_t w = blockIdx.x;
    const uint32_t e1 = (uint32_t)A->state[3] + 1u;  // this step's counters reach e1 x tasks
    const uint32_t nA = A->nA, nB = A->nB, nC = A->nC, nD = A->nD, layers = A->n_layers;
    const uint32_t nAC = nA > nC ? nA : nC;
    for (uint32_t l = 0; l < layers; l++) {
        if (w < nAC) {
            if (w < nA) one_qkv<KIND>(A, l, w, e1, olds);
            if (w < nC) one_up<KIND>(A, l, w, e1, olds);
        } else {
            const uint32_t t = w - nAC;
            if (t < nB) one_attn<KIND, L, K2>(A, l, t, e1, olds);
            if (t < nD) one_down<KIND>(A, l, t, e1, olds);
        }
    }
    one_head<KIND>(A, e1, olds, w, gridDim.x);
}

// LDS of one_step_kernel: the largest of its roles'. G: the grid.
__host__ inline size_t one_lds(size_t d, size_t hd, uint32_t chunk_down, uint32_t vocab, uint32_t G) {
    const size_t nb = d / 32, nb8 = (nb + 7) / 8, span = nb8 * 8;
    const size_t tail = (size_t)kStepWaves * 32 * 4 + kLnRed * 4;
    const size_t b = std::max(span * kPrepBytes + tail, (size_t)chunk_down * kPrepBytes + tail);
    const size_t head = span * kPrepBytes + (size_t)one_head_items((vocab + 31) / 32, G, (uint32_t)nb8) * 32 * 4 + kLnRed * 4;
    return std::max(std::max(b, head), (size_t)attn_out_lds((uint32_t)hd));
}

// Sets the position and the first position whose input the argmax writes.
__global__ void set_state_kernel(int32_t *state, int32_t pos, int32_t fill_from) {
    state[0] = pos;
    state[1] = fill_from;
}

// Writes one input token (a host-provided token for feed).
__global__ void set_input_kernel(int32_t *inputs, int32_t at, int32_t token) { inputs[at] = token; }

}  // namespace
}  // namespace fh

using namespace fh;

struct fh_gpt2 {
    fh_device *dev = nullptr;
    size_t vocab = 0, ctx = 0, dim = 0, heads = 0, layers = 0, hidden = 0;
    float eps = 1e-5f;
    fh_kind kind = FH_Q8_0;
    fh_qweight *tok = nullptr, *head = nullptr;  // head == tok when tied
    struct Layer {
        fh_qweight *wqkv = nullptr, *wo = nullptr, *w1 = nullptr, *w2 = nullptr;
        fh_buffer *ln1_g = nullptr, *ln1_b = nullptr, *bqkv = nullptr, *bo = nullptr;
        fh_buffer *ln2_g = nullptr, *ln2_b = nullptr, *b1 = nullptr, *b2 = nullptr;
        float *kc = nullptr, *vc = nullptr;
    };
    std::vector<Layer> blocks;
    fh_buffer *pos_tab = nullptr, *lnf_g = nullptr, *lnf_b = nullptr;
    // device scratch, one allocation: caches, x, q, attention output, f, logits, state, inputs
    void *arena = nullptr;
    float *x = nullptr, *q = nullptr, *att = nullptr, *f = nullptr, *logits = nullptr;
    int32_t *state = nullptr, *inputs = nullptr;
    uint8_t *prep = nullptr;      // prepared records of the final LayerNorm's output (the head's x)
    float *partial = nullptr;     // split-K row sums, and the head's per-group best values
    uint32_t *pick = nullptr;     // the head's per-group best rows
    uint32_t *tickets = nullptr;  // split-K counters per row group; the last one is the head's
    size_t n_tickets = 0;
    size_t pos = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool use_graph = true;
    bool split_k = false;  // FERRUM_HIP_DECODE_SPLIT_K=1: K splits for the narrow products
    // the step's form: 4 launches per layer (the attention with the output projection's head
    // columns; FFN-down split along K) where the model allows, else 5; FERRUM_HIP_DECODE_STEP=5
    // at load keeps 5
    int form = 5;
    uint32_t down_splits = 0;
    float *xc = nullptr, *xm = nullptr;  // the residual row before / after the attention block
    float *po = nullptr, *pf = nullptr;  // partial rows: [heads][dim], [down_splits][dim]
    uint64_t step_bytes = 0;
    // the one-launch step (form 1): the layer table, the phase counters and error flag, the grid
    void *one_mem = nullptr;
    uint32_t *sync = nullptr;
    const void *one_args = nullptr;  // the kernel's arguments (OneArgs), in device memory
    uint32_t one_tasks[4] = {0, 0, 0, 0};
    size_t one_lds_bytes = 0;
};

namespace {

fh_status gpt2_fail_free(fh_gpt2 *m, fh_status st) {
    fh_gpt2_free(m);
    return st;
}

// K splits for a product of `groups` row groups and nb8 batches per row: enough workgroups to
// spread a narrow product (few row groups) over the chip, each split a whole number of batches.
void plan_splits(uint32_t groups, uint32_t nb8, uint32_t *splits, uint32_t *chunk8) {
    uint32_t s = (192 + groups - 1) / groups;
    if (s > nb8) s = nb8;
    if (s < 1) s = 1;
    const uint32_t c = (nb8 + s - 1) / s;
    *chunk8 = c;
    *splits = (nb8 + c - 1) / c;
}

// Launch shape of a decode GEMV: workgroups of 32 rows (x K splits), wavefronts sharing the
// split's batches.
template <int KIND, int PRO, int EPI>
hipError_t launch_dgemv(hipStream_t s, DecodeGemv a, bool allow_split) {
    const uint32_t nb8 = (a.nb + 7) / 8, groups = (a.n + 31) / 32;
    uint32_t splits = 1, chunk8 = nb8;
    if ((allow_split || EPI == EPI_PARTIAL) && PRO == PRO_NONE && EPI != EPI_ARGMAX)
        plan_splits(groups, nb8, &splits, &chunk8);
    a.chunk = chunk8 * 8;
    const uint32_t W = chunk8 < (uint32_t)kMaxWaves ? chunk8 : (uint32_t)kMaxWaves;
    const size_t recs = PRO == PRO_GLOBAL ? 0 : (PRO == PRO_LN || PRO == PRO_LNR ? nb8 * 8 : a.chunk);
    const size_t lds = recs * kPrepBytes + (size_t)W * 32 * 4 + (size_t)kLnRed * 4;
    decode_gemv_kernel<KIND, PRO, EPI><<<dim3(groups, splits), 64 * W, lds, s>>>(a);
    return hipGetLastError();
}

#define FH_DGEMV_KERNELS(K)                                                                             \
    (const void *)decode_gemv_kernel<K, PRO_LN, EPI_QKV>, (const void *)decode_gemv_kernel<K, PRO_NONE, EPI_RESIDUAL>, \
        (const void *)decode_gemv_kernel<K, PRO_LN, EPI_GELU>, (const void *)decode_gemv_kernel<K, PRO_GLOBAL, EPI_ARGMAX>, \
        (const void *)decode_gemv_kernel<K, PRO_NONE, EPI_STORE>, (const void *)decode_gemv_kernel<K, PRO_LNR, EPI_QKV>, \
        (const void *)decode_gemv_kernel<K, PRO_LNR, EPI_GELU>, (const void *)decode_gemv_kernel<K, PRO_NONE, EPI_PARTIAL>

// Register sets in flight per wavefront of attn_out_kernel's product.
template <int L> constexpr int attn_k2() { return L == 64 ? 2 : 3; }
#define FH_ATTN_OUT_KERNELS(K)                                                                                    \
    (const void *)attn_out_kernel<K, 16, attn_k2<16>()>, (const void *)attn_out_kernel<K, 32, attn_k2<32>()>,     \
        (const void *)attn_out_kernel<K, 64, attn_k2<64>()>
constexpr uint32_t kAttnOutLdsMax = 96 * 1024;
#define FH_ONE_KERNELS(K)                                                                                         \
    (const void *)one_step_kernel<K, 16, attn_k2<16>()>, (const void *)one_step_kernel<K, 32, attn_k2<32>()>,     \
        (const void *)one_step_kernel<K, 64, attn_k2<64>()>

// Dynamic LDS beyond the default 64 KiB: prepared x of up to kMaxBlocks blocks plus the row
// sums, and the attention scores of up to 16384 positions. Set once, before any capture.
hipError_t set_lds_limits() {
    static const hipError_t e = [] {
        const int gemv_lds = (int)(kMaxBlocks * kPrepBytes + kMaxWaves * 33 * 4);
        const void *fns[] = {FH_DGEMV_KERNELS(FH_Q8_0), FH_DGEMV_KERNELS(FH_Q4_0)};
        for (const void *f : fns) {
            hipError_t r = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, gemv_lds);
            if (r) return r;
        }
        const void *ao[] = {FH_ATTN_OUT_KERNELS(FH_Q8_0), FH_ATTN_OUT_KERNELS(FH_Q4_0), FH_ONE_KERNELS(FH_Q8_0),
                            FH_ONE_KERNELS(FH_Q4_0)};
        for (const void *f : ao) {
            hipError_t r = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAttnOutLdsMax);
            if (r) return r;
        }
        const void *att[] = {(const void *)attention_kernel<2>, (const void *)attention_kernel<4>,
                             (const void *)attention_kernel<8>, (const void *)attention_kernel<16>,
                             (const void *)attention_kernel<32>, (const void *)attention_kernel<64>};
        for (const void *f : att) {
            hipError_t r = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
            if (r) return r;
        }
        return hipSuccess;
    }();
    return e;
}
#undef FH_DGEMV_KERNELS
#undef FH_ATTN_OUT_KERNELS
#undef FH_ONE_KERNELS

template <int PRO, int EPI>
hipError_t dgemv(hipStream_t s, fh_kind kind, const DecodeGemv &a, bool allow_split = false) {
    return kind == FH_Q8_0 ? launch_dgemv<FH_Q8_0, PRO, EPI>(s, a, allow_split)
                           : launch_dgemv<FH_Q4_0, PRO, EPI>(s, a, allow_split);
}

DecodeGemv dg(const fh_gpt2 *m, const fh_qweight *w, const float *x, float *y) {
    DecodeGemv a{};
    a.qs = w->qs;
    a.ds = w->ds;
    a.x = x;
    a.y = y;
    a.nb = (uint32_t)(w->k / 32);
    a.n = (uint32_t)w->n;
    a.partial = m->partial;
    a.ticket = m->tickets;
    a.state = m->state;
    return a;
}

const float *fp(const fh_buffer *b) { return (const float *)b->ptr; }

hipError_t attention(hipStream_t s, const fh_gpt2 *m, const fh_gpt2::Layer &L) {
    const uint32_t d = (uint32_t)m->dim, hd = (uint32_t)(m->dim / m->heads);
    const float scale = 1.0f / sqrtf((float)hd);
    const uint32_t nr = kAttnThreads / (hd / 4);
    const size_t lds = (m->ctx + (size_t)nr * hd + 2 * kAttnThreads / 64) * sizeof(float);
    const dim3 grid((uint32_t)m->heads);
    switch (hd) {
    case 8: attention_kernel<2><<<grid, kAttnThreads, lds, s>>>(m->q, L.kc, L.vc, m->state, m->att, d, (uint32_t)m->ctx, scale); break;
    case 16: attention_kernel<4><<<grid, kAttnThreads, lds, s>>>(m->q, L.kc, L.vc, m->state, m->att, d, (uint32_t)m->ctx, scale); break;
    case 32: attention_kernel<8><<<grid, kAttnThreads, lds, s>>>(m->q, L.kc, L.vc, m->state, m->att, d, (uint32_t)m->ctx, scale); break;
    case 64: attention_kernel<16><<<grid, kAttnThreads, lds, s>>>(m->q, L.kc, L.vc, m->state, m->att, d, (uint32_t)m->ctx, scale); break;
    case 128: attention_kernel<32><<<grid, kAttnThreads, lds, s>>>(m->q, L.kc, L.vc, m->state, m->att, d, (uint32_t)m->ctx, scale); break;
    default: attention_kernel<64><<<grid, kAttnThreads, lds, s>>>(m->q, L.kc, L.vc, m->state, m->att, d, (uint32_t)m->ctx, scale); break;
    }
    return hipGetLastError();
}

// Enqueue one decode step (the graph's body).
hipError_t enqueue_step(fh_gpt2 *m, hipStream_t s) {
    const uint32_t d = (uint32_t)m->dim;
    if (m->kind == FH_Q8_0)
        embed_kernel<FH_Q8_0><<<1, 256, 0, s>>>(m->tok->qs, m->tok->ds, fp(m->pos_tab), m->state, m->inputs, m->x, d);
    else
        embed_kernel<FH_Q4_0><<<1, 256, 0, s>>>(m->tok->qs, m->tok->ds, fp(m->pos_tab), m->state, m->inputs, m->x, d);
    hipError_t e = hipGetLastError();
    for (auto &L : m->blocks) {
        if (e) return e;
        DecodeGemv a = dg(m, L.wqkv, m->x, m->q);
        a.ln_g = fp(L.ln1_g);
        a.ln_b = fp(L.ln1_b);
        a.eps = m->eps;
        a.bias = fp(L.bqkv);
        a.kc = L.kc;
        a.vc = L.vc;
        a.split = d;
        if ((e = dgemv<PRO_LN, EPI_QKV>(s, m->kind, a))) return e;
        if ((e = attention(s, m, L))) return e;
        a = dg(m, L.wo, m->att, m->x);
        a.bias = fp(L.bo);
        if ((e = dgemv<PRO_NONE, EPI_RESIDUAL>(s, m->kind, a, m->split_k))) return e;
        a = dg(m, L.w1, m->x, m->f);
        a.ln_g = fp(L.ln2_g);
        a.ln_b = fp(L.ln2_b);
        a.eps = m->eps;
        a.bias = fp(L.b1);
        if ((e = dgemv<PRO_LN, EPI_GELU>(s, m->kind, a))) return e;
        a = dg(m, L.w2, m->f, m->x);
        a.bias = fp(L.b2);
        if ((e = dgemv<PRO_NONE, EPI_RESIDUAL>(s, m->kind, a, m->split_k))) return e;
    }
    if (e) return e;
    const uint32_t nbd = d / 32;
    if (m->kind == FH_Q8_0)
        ln_prep_kernel<FH_Q8_0><<<1, 64 * kMaxWaves, 0, s>>>(m->x, fp(m->lnf_g), fp(m->lnf_b), m->eps, nbd, m->prep);
    else
        ln_prep_kernel<FH_Q4_0><<<1, 64 * kMaxWaves, 0, s>>>(m->x, fp(m->lnf_g), fp(m->lnf_b), m->eps, nbd, m->prep);
    if ((e = hipGetLastError())) return e;
    DecodeGemv a = dg(m, m->head, m->x, m->logits);
    a.prep = m->prep;
    a.pick = m->pick;
    if ((e = dgemv<PRO_GLOBAL, EPI_ARGMAX>(s, m->kind, a))) return e;
    pick_kernel<<<1, 1024, 0, s>>>(m->partial, m->pick, (uint32_t)((m->vocab + 31) / 32), m->state, m->inputs);
    return hipGetLastError();
}

// Splits along K of the four-launch step's FFN-down product (launch_dgemv's EPI_PARTIAL rule).
uint32_t down_splits(size_t d, size_t hidden) {
    uint32_t sp, c8;
    plan_splits((uint32_t)(d / 32), (uint32_t)((hidden / 32 + 7) / 8), &sp, &c8);
    return sp;
}

// Whether the four-launch step takes this model (head width 64, 128 or 256, LDS within bounds).
bool four_fits(size_t d, size_t heads) {
    const size_t hd = d / heads;
    if (hd != 64 && hd != 128 && hd != 256) return false;
    return heads <= 64 && attn_out_lds((uint32_t)hd) <= kAttnOutLdsMax;
}

template <int KIND>
hipError_t launch_attn_out(hipStream_t s, uint32_t hd, uint32_t heads, const StepArgs &a) {
    const size_t lds = attn_out_lds(hd);
    switch (hd) {
    case 64: attn_out_kernel<KIND, 16, attn_k2<16>()><<<heads, kStepThreads, lds, s>>>(a); break;
    case 128: attn_out_kernel<KIND, 32, attn_k2<32>()><<<heads, kStepThreads, lds, s>>>(a); break;
    default: attn_out_kernel<KIND, 64, attn_k2<64>()><<<heads, kStepThreads, lds, s>>>(a); break;
    }
    return hipGetLastError();
}

// The head: the final LayerNorm of x_in + (sum of the partial rows + b), the head product and the
// greedy pick.
hipError_t enqueue_head(fh_gpt2 *m, hipStream_t s, const float *x_in, const float *part, uint32_t nparts,
                        const float *b) {
    StepArgs z{};
    z.x_in = x_in;
    z.part = part;
    z.pbias = b;
    z.nparts = nparts;
    z.state = m->state;
    z.x_out = m->x;
    z.ln_g = fp(m->lnf_g);
    z.ln_b = fp(m->lnf_b);
    z.eps = m->eps;
    z.d = (uint32_t)m->dim;
    z.nb = (uint32_t)(m->dim / 32);
    if (m->kind == FH_Q8_0)
        final_ln_kernel<FH_Q8_0><<<1, kStepThreads, 0, s>>>(z, m->prep);
    else
        final_ln_kernel<FH_Q4_0><<<1, kStepThreads, 0, s>>>(z, m->prep);
    hipError_t e = hipGetLastError();
    if (e) return e;
    DecodeGemv a = dg(m, m->head, m->x, m->logits);
    a.prep = m->prep;
    a.pick = m->pick;
    if ((e = dgemv<PRO_GLOBAL, EPI_ARGMAX>(s, m->kind, a))) return e;
    pick_kernel<<<1, 1024, 0, s>>>(m->partial, m->pick, (uint32_t)((m->vocab + 31) / 32), m->state, m->inputs);
    return hipGetLastError();
}

// Enqueue one four-launch step: per layer LN1 + QKV (the residual row formed from the previous
// layer's partial rows), attention + the output projection's head columns (partial rows per
// head), LN2 + FFN-up + GELU (the residual row from those), FFN-down split along K (partial rows
// per split); then the head.
hipError_t enqueue_four(fh_gpt2 *m, hipStream_t s) {
    const uint32_t d = (uint32_t)m->dim, hd = (uint32_t)(m->dim / m->heads), nb = d / 32;
    const uint32_t heads = (uint32_t)m->heads, S = m->down_splits;
    hipError_t e = hipSuccess;
    for (size_t l = 0; l < m->blocks.size(); l++) {
        const auto &L = m->blocks[l];
        DecodeGemv a = dg(m, L.wqkv, nullptr, m->q);
        if (l == 0) {
            a.emb_qs = m->tok->qs;
            a.emb_ds = m->tok->ds;
            a.pos_tab = fp(m->pos_tab);
        } else {
            a.x_in = m->xm;
            a.rpart = m->pf;
            a.rbias = fp(m->blocks[l - 1].b2);
            a.nparts = S;
        }
        a.inputs = m->inputs;
        a.x_out = m->xc;
        a.ln_g = fp(L.ln1_g);
        a.ln_b = fp(L.ln1_b);
        a.eps = m->eps;
        a.bias = fp(L.bqkv);
        a.kc = L.kc;
        a.vc = L.vc;
        a.split = d;
        if ((e = dgemv<PRO_LNR, EPI_QKV>(s, m->kind, a))) return e;
        StepArgs t{};
        t.q = m->q;
        t.kc = L.kc;
        t.vc = L.vc;
        t.state = m->state;
        t.d = d;
        t.nb = nb;
        t.scale = 1.0f / sqrtf((float)hd);
        t.qs2 = L.wo->qs;
        t.ds2 = L.wo->ds;
        t.nb2 = nb;
        t.out_part = m->po;
        if ((e = m->kind == FH_Q8_0 ? launch_attn_out<FH_Q8_0>(s, hd, heads, t) : launch_attn_out<FH_Q4_0>(s, hd, heads, t)))
            return e;
        a = dg(m, L.w1, nullptr, m->f);
        a.x_in = m->xc;
        a.rpart = m->po;
        a.rbias = fp(L.bo);
        a.nparts = heads;
        a.x_out = m->xm;
        a.ln_g = fp(L.ln2_g);
        a.ln_b = fp(L.ln2_b);
        a.eps = m->eps;
        a.bias = fp(L.b1);
        if ((e = dgemv<PRO_LNR, EPI_GELU>(s, m->kind, a))) return e;
        a = dg(m, L.w2, m->f, m->pf);
        if ((e = dgemv<PRO_NONE, EPI_PARTIAL>(s, m->kind, a))) return e;
    }
    return enqueue_head(m, s, m->xm, m->pf, S, fp(m->blocks.back().b2));
}

template <int KIND>
const void *one_kernel(uint32_t hd) {
    return hd == 64 ? (const void *)one_step_kernel<KIND, 16, attn_k2<16>()>
                    : hd == 128 ? (const void *)one_step_kernel<KIND, 32, attn_k2<32>()>
                                : (const void *)one_step_kernel<KIND, 64, attn_k2<64>()>;
}

// Enqueue one one-launch step: every layer, the head and the pick in one_step_kernel.
hipError_t enqueue_one(fh_gpt2 *m, hipStream_t s) {
    const uint32_t hd = (uint32_t)(m->dim / m->heads);
    const uint32_t grid = std::max(m->one_tasks[0], m->one_tasks[2]) + std::max(m->one_tasks[1], m->one_tasks[3]);
    const OneArgs *args = (const OneArgs *)m->one_args;
    void *kargs[] = {&args};
    hipError_t e = hipLaunchKernel(m->kind == FH_Q8_0 ? one_kernel<FH_Q8_0>(hd) : one_kernel<FH_Q4_0>(hd), dim3(grid),
                                   dim3(kStepThreads), kargs, m->one_lds_bytes, s);
    return e;
}

// Sets up the one-launch step where it fits: head widths 64, 128, 256, and all of its workgroups
// resident at once (the occupancy query). Returns false (the four-launch step stays) otherwise.
bool one_setup(fh_gpt2 *m) {
    const size_t d = m->dim, hd = d / m->heads;
    // (d <= 2048: one_head takes one batch of eight blocks per item)
    if (m->form != 4 || m->layers > kOneMaxLayers || (d / 32 + 7) / 8 > kStepWaves) return false;
    uint32_t sp, c8;
    plan_splits((uint32_t)(d / 32), (uint32_t)((m->hidden / 32 + 7) / 8), &sp, &c8);
    const uint32_t tasks[4] = {(uint32_t)(3 * d / 32), (uint32_t)m->heads, (uint32_t)(m->hidden / 32),
                               (uint32_t)(d / 32) * sp};
    const uint32_t grid = std::max(tasks[0], tasks[2]) + std::max(tasks[1], tasks[3]);
    const size_t lds = one_lds(d, hd, c8 * 8, (uint32_t)m->vocab, grid);
    if (lds > kAttnOutLdsMax) return false;
    int dev = 0, cus = 0, per = 0;
    const void *k = m->kind == FH_Q8_0 ? one_kernel<FH_Q8_0>((uint32_t)hd) : one_kernel<FH_Q4_0>((uint32_t)hd);
    if (hipGetDevice(&dev) || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, kStepThreads, lds))
        return false;
    if ((uint64_t)per * (uint64_t)cus < grid) return false;
    auto up = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    const uint32_t slots = (uint32_t)m->heads + sp + 2;
    const size_t table = m->layers * sizeof(OneLayer), sync = (size_t)one_counter((uint32_t)m->layers, 2, slots) * 4;
    const size_t per_layer = 3 * up(d * 4) + up(m->heads * d * 4) + up((size_t)sp * d * 4) + up(m->hidden * 4);
    const size_t bufs0 = up(table) + up(sync) + up(sizeof(OneArgs));
    if (alloc_bytes(m->dev, bufs0 + m->layers * per_layer, &m->one_mem)) return false;
    std::vector<OneLayer> t(m->layers);
    for (size_t l = 0; l < m->layers; l++) {
        const auto &L = m->blocks[l];
        uint8_t *b = (uint8_t *)m->one_mem + bufs0 + l * per_layer;
        float *q = (float *)b, *xc = (float *)(b + up(d * 4)), *xm = (float *)(b + 2 * up(d * 4));
        float *po = (float *)(b + 3 * up(d * 4)), *pf = (float *)((uint8_t *)po + up(m->heads * d * 4));
        float *f = (float *)((uint8_t *)pf + up((size_t)sp * d * 4));
        t[l] = OneLayer{L.wqkv->qs, L.wo->qs, L.w1->qs, L.w2->qs, L.wqkv->ds, L.wo->ds, L.w1->ds, L.w2->ds,
                        fp(L.ln1_g), fp(L.ln1_b), fp(L.bqkv), fp(L.bo), fp(L.ln2_g), fp(L.ln2_b), fp(L.b1), fp(L.b2),
                        L.kc, L.vc, q, xc, xm, po, pf, f};
    }
    m->sync = (uint32_t *)((uint8_t *)m->one_mem + up(table));
    OneArgs a{};
    a.layers = (const OneLayer *)m->one_mem;
    a.n_layers = (uint32_t)m->layers;
    a.emb_qs = m->tok->qs;
    a.emb_ds = m->tok->ds;
    a.pos_tab = fp(m->pos_tab);
    a.inputs = m->inputs;
    a.state = m->state;
    a.x_final = m->x;
    a.lnf_g = fp(m->lnf_g);
    a.lnf_b = fp(m->lnf_b);
    a.head_qs = m->head->qs;
    a.head_ds = m->head->ds;
    a.vocab = (uint32_t)m->vocab;
    a.logits = m->logits;
    a.offers = (uint64_t *)m->partial;
    a.sync = m->sync;
    a.d = (uint32_t)d;
    a.hidden = (uint32_t)m->hidden;
    a.heads = (uint32_t)m->heads;
    a.S = sp;
    a.chunk_down = c8 * 8;
    a.eps = m->eps;
    a.scale = 1.0f / sqrtf((float)hd);
    a.nA = tasks[0];
    a.nB = tasks[1];
    a.nC = tasks[2];
    a.nD = tasks[3];
    a.slots = slots;
    m->one_args = (const void *)((uint8_t *)m->sync + up(sync));
    // on the device stream, after the allocation's own clearing; the host copies are pageable
    hipStream_t st = m->dev->stream;
    if (hipMemcpyAsync(m->one_mem, t.data(), table, hipMemcpyHostToDevice, st) ||
        hipMemsetAsync(m->sync, 0, sync, st) ||
        hipMemcpyAsync((void *)m->one_args, &a, sizeof(a), hipMemcpyHostToDevice, st) || hipStreamSynchronize(st)) {
        (void)hipFree(m->one_mem);
        m->one_mem = nullptr;
        m->sync = nullptr;
        return false;
    }
    for (int i = 0; i < 4; i++) m->one_tasks[i] = tasks[i];
    m->one_lds_bytes = lds;
    m->form = 1;
    return true;
}

// After a one-launch step's work has completed: a wait that gave up (a workgroup not resident)
// leaves its flag; the counters are then reset and the model keeps the four-launch step.
fh_status one_check(fh_gpt2 *m) {
    if (m->form != 1) return FH_OK;
    uint32_t flag = 0;
    hipStream_t st = m->dev->stream;
    const uint32_t slots = (uint32_t)m->heads + m->down_splits + 2;
    hipError_t e = hipMemcpyAsync(&flag, m->sync + one_counter((uint32_t)m->layers, 0, slots), 4, hipMemcpyDeviceToHost, st);
    if (!e) e = hipStreamSynchronize(st);
    if (e) return hip_fail(m->dev, e, "gpt2 step");
    if (!flag) return FH_OK;
    (void)hipMemsetAsync(m->sync, 0, (size_t)one_counter((uint32_t)m->layers, 2, slots) * 4, st);
    (void)hipMemsetAsync(m->state + 3, 0, 4, st);
    (void)hipStreamSynchronize(st);
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    m->form = 4;
    return fail(FH_ERR_DEVICE, "gpt2 step: the one-launch step's workgroups did not all run at once (a wait gave "
                               "up); the model now runs the four-launch step");
}

hipError_t enqueue_any(fh_gpt2 *m, hipStream_t s) {
    return m->form == 1 ? enqueue_one(m, s) : m->form == 4 ? enqueue_four(m, s) : enqueue_step(m, s);
}

// Run one step on the device stream: the captured graph (made on first use), or the launches. The
// one-launch step is launched directly: replaying a one-node graph measured 6 us slower per step
// (233 against 227 us at GPT-2-small).
fh_status run_step(fh_gpt2 *m) {
    fh_device *dev = m->dev;
    fh_status st = begin_command(dev, "gpt2 step");
    if (st) return st;
    const bool graph = m->use_graph && m->form != 1;
    if (graph && !m->exec) {
        hipError_t e = hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal);
        if (e) return hip_fail(dev, e, "gpt2 step capture");
        const hipError_t le = enqueue_any(m, dev->stream);
        e = hipStreamEndCapture(dev->stream, &m->graph);
        if (le) return hip_fail(dev, le, "gpt2 step capture");
        if (e) return hip_fail(dev, e, "gpt2 step capture");
        e = hipGraphInstantiate(&m->exec, m->graph, nullptr, nullptr, 0);
        if (e) {
            m->exec = nullptr;
            return hip_fail(dev, e, "gpt2 step graph");
        }
    }
    hipError_t e = graph ? hipGraphLaunch(m->exec, dev->stream) : enqueue_any(m, dev->stream);
    if (e) return hip_fail(dev, e, "gpt2 step");
    return end_command(dev, "gpt2 step");
}

}  // namespace

namespace fh {

hipError_t decode_lds_limits() { return set_lds_limits(); }

bool gemv_latency_fits(size_t k, size_t n, int cus) {
    // one workgroup per 32 rows holding all of x's prepared records in LDS; worth it while the
    // row groups are few enough that their workgroups run in about one round
    const size_t env = [] {
        const char *e = getenv("FERRUM_HIP_GEMV_LATENCY_GROUPS_PER_CU");
        const long v = e ? strtol(e, nullptr, 10) : 0;
        return (size_t)(v >= 0 && v <= 64 && e ? v : 2);  // (measured: 2 to 8 alike; 1 leaves 352 groups slow)
    }();
    return k / 32 <= kMaxBlocks && (n + 31) / 32 <= env * (size_t)(cus > 0 ? cus : 256);
}

hipError_t launch_gemv_latency(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                               float *y, size_t k, size_t n) {
    DecodeGemv a{};
    a.qs = qs;
    a.ds = ds;
    a.x = x;
    a.y = y;
    a.nb = (uint32_t)(k / 32);
    a.n = (uint32_t)n;
    return dgemv<PRO_NONE, EPI_STORE>(s, kind, a);
}

}  // namespace fh


extern "C" {

fh_status fh_gpt2_from_gguf(fh_device *dev, const fh_gguf *g, fh_gpt2 **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!g || !out) return fail(FH_ERR_INVALID, "gpt2: no file or output");
    *out = nullptr;
    const char *arch;
    size_t alen;
    if ((st = fh_gguf_get_string(g, "general.architecture", &arch, &alen))) return st;
    if (std::string(arch, alen) != "gpt2")
        return fail(FH_ERR_INVALID, "gpt2: general.architecture is '%.*s', not gpt2", (int)alen, arch);
    fh_gpt2 *m = new (std::nothrow) fh_gpt2;
    if (!m) return fail(FH_ERR_OOM, "host out of memory");
    dev_retain(dev);
    m->dev = dev;
    if ((st = cfg_uint(g, "gpt2.context_length", &m->ctx)) || (st = cfg_uint(g, "gpt2.embedding_length", &m->dim)) ||
        (st = cfg_uint(g, "gpt2.block_count", &m->layers)) ||
        (st = cfg_uint(g, "gpt2.feed_forward_length", &m->hidden)) ||
        (st = cfg_uint(g, "gpt2.attention.head_count", &m->heads)))
        return gpt2_fail_free(m, st);
    size_t kidx;
    if (fh_gguf_find_key(g, "gpt2.attention.layer_norm_epsilon", &kidx) == FH_OK &&
        (st = fh_gguf_get_float(g, "gpt2.attention.layer_norm_epsilon", &m->eps)))
        return gpt2_fail_free(m, st);
    size_t tidx;
    fh_gguf_tensor tt;
    if ((st = fh_gguf_find_tensor(g, "token_embd.weight", &tidx)) || (st = fh_gguf_tensor_info(g, tidx, &tt)))
        return gpt2_fail_free(m, st);
    m->vocab = tt.n_dims == 2 ? (size_t)tt.dims[1] : 0;
    const size_t d = m->dim, h = m->hidden;
    // Config::validate (ferrum_ref/src/models/gpt2/mod.rs:38-58) plus what the kernels need
    if (!m->vocab || !m->ctx || !d || !m->heads || !m->layers || !h)
        return gpt2_fail_free(m, fail(FH_ERR_INVALID, "gpt2: every dimension must be positive"));
    if (d % m->heads)
        return gpt2_fail_free(m, fail(FH_ERR_INVALID, "gpt2: dim %zu is not divisible by heads %zu", d, m->heads));
    const size_t hd = d / m->heads;
    if (d % 32 || h % 32 || d > 4096 || h / 32 > kMaxBlocks || (hd != 8 && hd != 16 && hd != 32 && hd != 64 && hd != 128 && hd != 256) ||
        m->ctx > 16384 ||
        m->vocab > (1u << 30))
        return gpt2_fail_free(m, fail(FH_ERR_UNSUPPORTED,
                                      "gpt2: dim %zu / hidden %zu / head %zu / ctx %zu outside what the decode kernels "
                                      "take (dim a multiple of 32 up to 4096, hidden up to 16384, heads 8, 16, 32, "
                                      "64, 128 or 256 wide, ctx up to 16384)",
                                      d, h, hd, m->ctx));
    fh_kind kind = (fh_kind)0;
    if ((st = load_mat(dev, g, "gpt2", "token_embd.weight", d, m->vocab, &kind, &m->tok))) return gpt2_fail_free(m, st);
    if (fh_gguf_find_tensor(g, "output.weight", &tidx) == FH_OK) {
        if ((st = load_mat(dev, g, "gpt2", "output.weight", d, m->vocab, &kind, &m->head))) return gpt2_fail_free(m, st);
    } else {
        m->head = m->tok;  // tied (ferrum_model/src/gguf/gpt2.rs:228-231 omits a tied head)
    }
    m->kind = kind;
    if ((st = load_vec(dev, g, "gpt2", "position_embd.weight", m->ctx * d, &m->pos_tab)) ||
        (st = load_vec(dev, g, "gpt2", "output_norm.weight", d, &m->lnf_g)) || (st = load_vec(dev, g, "gpt2", "output_norm.bias", d, &m->lnf_b)))
        return gpt2_fail_free(m, st);
    m->blocks.resize(m->layers);
    for (size_t l = 0; l < m->layers; l++) {
        auto &L = m->blocks[l];
        if ((st = load_vec(dev, g, "gpt2", tensor_name("blk.", l, "attn_norm.weight"), d, &L.ln1_g)) ||
            (st = load_vec(dev, g, "gpt2", tensor_name("blk.", l, "attn_norm.bias"), d, &L.ln1_b)) ||
            (st = load_mat(dev, g, "gpt2", tensor_name("blk.", l, "attn_qkv.weight"), d, 3 * d, &kind, &L.wqkv)) ||
            (st = load_vec(dev, g, "gpt2", tensor_name("blk.", l, "attn_qkv.bias"), 3 * d, &L.bqkv)) ||
            (st = load_mat(dev, g, "gpt2", tensor_name("blk.", l, "attn_output.weight"), d, d, &kind, &L.wo)) ||
            (st = load_vec(dev, g, "gpt2", tensor_name("blk.", l, "attn_output.bias"), d, &L.bo)) ||
            (st = load_vec(dev, g, "gpt2", tensor_name("blk.", l, "ffn_norm.weight"), d, &L.ln2_g)) ||
            (st = load_vec(dev, g, "gpt2", tensor_name("blk.", l, "ffn_norm.bias"), d, &L.ln2_b)) ||
            (st = load_mat(dev, g, "gpt2", tensor_name("blk.", l, "ffn_up.weight"), d, h, &kind, &L.w1)) ||
            (st = load_vec(dev, g, "gpt2", tensor_name("blk.", l, "ffn_up.bias"), h, &L.b1)) ||
            (st = load_mat(dev, g, "gpt2", tensor_name("blk.", l, "ffn_down.weight"), h, d, &kind, &L.w2)) ||
            (st = load_vec(dev, g, "gpt2", tensor_name("blk.", l, "ffn_down.bias"), d, &L.b2)))
            return gpt2_fail_free(m, st);
        m->step_bytes += L.wqkv->nbytes + L.wo->nbytes + L.w1->nbytes + L.w2->nbytes;
    }
    m->step_bytes += m->head->nbytes;
    // caches and scratch in one allocation (every piece 256-byte aligned)
    auto up = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    const size_t cache = up(m->ctx * d * 4);
    // split-K scratch: the split products (attention output, FFN down) have d outputs and d or h
    // inputs; the head needs one value per row group
    const size_t groups_v = (m->vocab + 31) / 32, groups_d = d / 32;
    size_t part_floats = 2 * groups_v;  // (the one-launch step keeps a 64-bit offer per row group here)
    for (size_t k : {d, h}) {
        uint32_t sp, c8;
        plan_splits((uint32_t)groups_d, (uint32_t)((k / 32 + 7) / 8), &sp, &c8);
        part_floats = std::max(part_floats, (size_t)sp * groups_d * 32);
    }
    const size_t max_groups = groups_d;
    m->n_tickets = max_groups + 1;
    const char *sf = getenv("FERRUM_HIP_DECODE_STEP");
    m->form = !(sf && atoi(sf) == 5) && four_fits(d, m->heads) ? 4 : 5;
    m->down_splits = down_splits(d, h);
    const size_t four_bytes =
        m->form == 4 ? 2 * up(d * 4) + up(m->heads * d * 4) + up((size_t)m->down_splits * d * 4) : 0;
    const size_t total = 2 * m->layers * cache + 3 * up(d * 4) + up(h * 4) + up(m->vocab * 4) + up(16) +
                         up((m->ctx + 1) * 4) + up((d / 32 + 7) / 8 * 8 * kPrepBytes) + up(part_floats * 4) +
                         up(groups_v * 4) + up(m->n_tickets * 4) + four_bytes;
    if ((st = alloc_bytes(dev, total, &m->arena))) return gpt2_fail_free(m, st);
    uint8_t *p = (uint8_t *)m->arena;
    for (auto &L : m->blocks) {
        L.kc = (float *)p;
        p += cache;
        L.vc = (float *)p;
        p += cache;
    }
    m->x = (float *)p;
    p += up(d * 4);
    m->q = (float *)p;
    p += up(d * 4);
    m->att = (float *)p;
    p += up(d * 4);
    m->f = (float *)p;
    p += up(h * 4);
    m->logits = (float *)p;
    p += up(m->vocab * 4);
    m->state = (int32_t *)p;
    p += up(16);
    m->inputs = (int32_t *)p;
    p += up((m->ctx + 1) * 4);
    m->prep = p;
    p += up((d / 32 + 7) / 8 * 8 * kPrepBytes);
    m->partial = (float *)p;
    p += up(part_floats * 4);
    m->pick = (uint32_t *)p;
    p += up(groups_v * 4);
    m->tickets = (uint32_t *)p;  // zero from the allocation; every launch leaves them zero
    p += up(m->n_tickets * 4);
    if (m->form == 4) {
        m->xc = (float *)p;
        p += up(d * 4);
        m->xm = (float *)p;
        p += up(d * 4);
        m->po = (float *)p;
        p += up(m->heads * d * 4);
        m->pf = (float *)p;
    }
    if (hipError_t e = set_lds_limits()) return gpt2_fail_free(m, hip_fail(dev, e, "gpt2 kernels"));
    if (!(sf && atoi(sf) == 4)) (void)one_setup(m);
    const char *ng = getenv("FERRUM_HIP_NO_GRAPH");
    m->use_graph = !(ng && ng[0] == '1');
    const char *sk = getenv("FERRUM_HIP_DECODE_SPLIT_K");
    m->split_k = sk && sk[0] == '1';
    // the caches need no clearing: position p reads only entries 0..p, all written by then
    if ((st = begin_command(dev, "gpt2 state"))) return gpt2_fail_free(m, st);
    set_state_kernel<<<1, 1, 0, dev->stream>>>(m->state, 0, 0);
    if ((st = end_command(dev, "gpt2 state"))) return gpt2_fail_free(m, st);
    *out = m;
    return FH_OK;
}

fh_status fh_gpt2_config(const fh_gpt2 *m, size_t *vocab, size_t *ctx, size_t *dim, size_t *heads, size_t *layers,
                         size_t *hidden) {
    if (!m) return fail(FH_ERR_INVALID, "gpt2: no model");
    if (vocab) *vocab = m->vocab;
    if (ctx) *ctx = m->ctx;
    if (dim) *dim = m->dim;
    if (heads) *heads = m->heads;
    if (layers) *layers = m->layers;
    if (hidden) *hidden = m->hidden;
    return FH_OK;
}

fh_kind fh_gpt2_kind(const fh_gpt2 *m) { return m ? m->kind : (fh_kind)0; }
size_t fh_gpt2_pos(const fh_gpt2 *m) { return m ? m->pos : 0; }
uint64_t fh_gpt2_step_bytes(const fh_gpt2 *m) { return m ? m->step_bytes : 0; }
size_t fh_gpt2_step_launches(const fh_gpt2 *m) {
    if (!m) return 0;
    return m->form == 1 ? 1 : m->form == 4 ? 4 * m->layers + 3 : 5 * m->layers + 4;
}
void fh_gpt2_reset(fh_gpt2 *m) {
    if (m) m->pos = 0;  // later positions overwrite the cache rows they read
}

fh_status fh_gpt2_feed(fh_device *dev, fh_gpt2 *m, size_t token, float *logits) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!m || m->dev != dev) return fail(FH_ERR_INVALID, "gpt2: no model on this device");
    if (m->pos >= m->ctx) return fail(FH_ERR_INVALID, "context of %zu tokens is full", m->ctx);
    if (token >= m->vocab) return fail(FH_ERR_INVALID, "token %zu is out of range for vocab %zu", token, m->vocab);
    if ((st = begin_command(dev, "gpt2 feed"))) return st;
    set_state_kernel<<<1, 1, 0, dev->stream>>>(m->state, (int32_t)m->pos, 0x7fffffff);
    set_input_kernel<<<1, 1, 0, dev->stream>>>(m->inputs, (int32_t)m->pos, (int32_t)token);
    if ((st = end_command(dev, "gpt2 feed"))) return st;
    if ((st = run_step(m))) return st;
    if (m->form == 1) {
        hipError_t e = hipStreamSynchronize(dev->stream);
        if (e) return hip_fail(dev, e, "gpt2 feed");
        if ((st = one_check(m))) return st;
    }
    if (logits) {
        if ((st = begin_command(dev, "gpt2 logits"))) return st;
        hipError_t e = hipMemcpyAsync(logits, m->logits, m->vocab * 4, hipMemcpyDeviceToHost, dev->stream);
        if (e) return hip_fail(dev, e, "gpt2 logits");
        e = hipStreamSynchronize(dev->stream);
        if (e) return hip_fail(dev, e, "gpt2 logits");
    }
    m->pos++;  // only a feed that completed advances the context (the device state is reset per call)
    return FH_OK;
}

fh_status fh_gpt2_generate(fh_device *dev, fh_gpt2 *m, const int32_t *prompt, size_t n_prompt, size_t n_new,
                           int32_t *out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!m || m->dev != dev) return fail(FH_ERR_INVALID, "gpt2: no model on this device");
    if (n_prompt == 0 || !prompt) return fail(FH_ERR_INVALID, "gpt2: generate needs a prompt");
    if (n_new && !out) return fail(FH_ERR_INVALID, "gpt2: no output for %zu tokens", n_new);
    // positions p0 .. p0 + n_prompt + n_new - 2 are fed; the last pick is not
    const size_t steps = n_prompt + (n_new ? n_new - 1 : 0);
    if (m->pos + steps > m->ctx)
        return fail(FH_ERR_INVALID, "context of %zu tokens is full (%zu used, %zu more needed)", m->ctx, m->pos, steps);
    for (size_t i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || (size_t)prompt[i] >= m->vocab)
            return fail(FH_ERR_INVALID, "token %d is out of range for vocab %zu", prompt[i], m->vocab);
    const size_t p0 = m->pos;
    if ((st = begin_command(dev, "gpt2 prompt"))) return st;
    hipError_t e = hipMemcpyAsync(m->inputs + p0, prompt, n_prompt * 4, hipMemcpyHostToDevice, dev->stream);
    if (e) return hip_fail(dev, e, "gpt2 prompt");
    set_state_kernel<<<1, 1, 0, dev->stream>>>(m->state, (int32_t)p0, (int32_t)(p0 + n_prompt));
    if ((st = end_command(dev, "gpt2 prompt"))) return st;
    if ((e = hipStreamSynchronize(dev->stream))) return hip_fail(dev, e, "gpt2 prompt");  // prompt is pageable
    for (size_t i = 0; i < steps; i++)
        if ((st = run_step(m))) return st;
    if (n_new) {
        if ((st = begin_command(dev, "gpt2 tokens"))) return st;
        e = hipMemcpyAsync(out, m->inputs + p0 + n_prompt, n_new * 4, hipMemcpyDeviceToHost, dev->stream);
        if (e) return hip_fail(dev, e, "gpt2 tokens");
    }
    if ((e = hipStreamSynchronize(dev->stream))) return hip_fail(dev, e, "gpt2 generate");
    if ((st = one_check(m))) return st;
    m->pos = p0 + steps;
    return FH_OK;
}

void fh_gpt2_free(fh_gpt2 *m) {
    if (!m) return;
    if (m->dev) (void)hipStreamSynchronize(m->dev->stream);
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    if (m->head && m->head != m->tok) fh_qweight_free(m->head);
    fh_qweight_free(m->tok);
    for (auto &L : m->blocks) {
        for (fh_qweight *w : {L.wqkv, L.wo, L.w1, L.w2}) fh_qweight_free(w);
        for (fh_buffer *b : {L.ln1_g, L.ln1_b, L.bqkv, L.bo, L.ln2_g, L.ln2_b, L.b1, L.b2}) fh_buffer_free(b);
    }
    for (fh_buffer *b : {m->pos_tab, m->lnf_g, m->lnf_b}) fh_buffer_free(b);
    if (m->arena) (void)hipFree(m->arena);
    if (m->one_mem) (void)hipFree(m->one_mem);
    if (m->dev) dev_release(m->dev);
    delete m;
}

}  // extern "C"
