// Llama / Qwen2 full-sequence forward and scoring on resident Q8_0 / Q4_0 weights.
//
// Replaces the batched passes of ferrum_wgpu's GpuLlama (ferrum_wgpu/src/models/llama/
// forward.rs:13-88: forward_all and score over the ops of ops/llama.rs), whose CPU oracle is
// ferrum_ref's Llama::forward_logits (ferrum_ref/src/models/llama/mod.rs:166-259) and
// nn::score (ferrum_ref/src/kernels/nn.rs:117-129). The model comes from a `llama` or `qwen2`
// GGUF as ferrum_model writes and reads it (ferrum_model/src/gguf/llama/mod.rs:107-323).
//
// One forward over t rows, all on the device stream, every activation row-major f32:
//   embed (rows of the packed token_embd)                       -> x [t, d]
//   per block: RMSNorm (fused with the previous residual add)   -> h
//              h . [Wq; Wk; Wv] (one stacked weight)             -> qkv [t, qd + 2 kvd]
//              bias + RoPE in place (host-built tables)
//              causal GQA attention (f32 MFMA, online softmax)   -> att [t, qd]
//              att . Wo                                         -> o
//              x += o, RMSNorm                                   -> h
//              h . [Wgate; Wup] (one stacked weight)             -> gu [t, 2 hidden]
//              SwiGLU                                           -> act [t, hidden]
//              act . Wdown                                      -> o
//   x += o, final RMSNorm, h . head (chunks of rows)            -> logits, or straight into score
// The products are the library's MFMA GEMMs on the packed weights, chosen at load: the precise
// one (x as two f16 parts, FH_PATH_TILED), the fast scoring one (FH_PATH_TILED_FAST) or the
// dequant-f16 one (FH_PATH_TILED_F16).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "device_common.hpp"
#include "internal.hpp"
#include "xsplit.hpp"

using namespace fh;

struct fh_llama {
    fh_device *dev = nullptr;
    size_t vocab = 0, ctx = 0, dim = 0, heads = 0, kv_heads = 0, head_dim = 0, layers = 0, hidden = 0, rope_dim = 0;
    float rope_base = 10000.0f, eps = 1e-5f, linear_factor = 1.0f;
    bool neox = false, tied = false;
    bool fuse_rope = true;  // qkv_rope_split_kernel where it fits (FERRUM_HIP_ROPE_UNFUSED=1 at load: never)
    // on the fast path with the split attention, the attention writes the output product's split x
    // itself (FERRUM_HIP_ATTN_SPLIT_UNFUSED=1 at load: f32 rows, then the product's split pass)
    bool att_split = true;
    // the score in the head GEMM's epilogue (launch_gemm_score) on the TILED and TILED_FAST paths
    // where it takes the shape (FERRUM_HIP_SCORE_UNFUSED=1 at load: the logits and score_kernel)
    bool fuse_score = true;
    fh_kind kind = (fh_kind)0;
    fh_path path = FH_PATH_TILED;
    // A weight matrix of k inputs and n outputs: packed (q), or the f32 rows (f: n rows of k
    // values, the GGUF row order) of a matrix the file does not store as Q8_0/Q4_0, e.g. one whose
    // width is not whole 32-blocks (Lin::upload keeps those f32, ferrum_wgpu/src/models/llama/
    // lin.rs:30-62).
    struct Mat {
        fh_qweight *q = nullptr;
        fh_buffer *f = nullptr;
        size_t k = 0, n = 0;
        uint64_t bytes() const { return q ? q->nbytes : (uint64_t)k * n * 4; }
        uint64_t device_bytes() const { return q ? fh_qweight_device_bytes(q) : f ? f->nbytes : 0; }
        void release() {
            fh_qweight_free(q);
            fh_buffer_free(f);
            q = nullptr;
            f = nullptr;
        }
    };
    struct Layer {
        fh_buffer *attn_norm = nullptr, *ffn_norm = nullptr, *bqkv = nullptr;
        Mat wqkv, wo, wgu, down;
    };
    std::vector<Layer> blocks;
    Mat tok, head;  // head is tok's copy when tied
    bool packed = true;  // every block matrix packed (the fast path's fused producers need it)
    // the gate/up weights interleaved in runs of 32 rows for gemm_kernel's SwiGLU epilogue (the fast
    // path with every block matrix packed, unless FERRUM_HIP_SWIGLU_UNFUSED=1 at load)
    bool gu_inter = false;
    fh_buffer *out_norm = nullptr, *rope_cos = nullptr, *rope_sin = nullptr;
    uint64_t weight_bytes = 0;
    // Activations for up to `rows` rows, grown on demand and kept.
    void *arena = nullptr;
    size_t arena_bytes = 0;
    size_t rows = 0, chunk = 0;  // chunk: rows of logits the arena holds
    float *x = nullptr, *h = nullptr, *qkv = nullptr, *att = nullptr, *o = nullptr, *gu = nullptr, *act = nullptr,
          *logits = nullptr, *scores = nullptr;
    int32_t *ids = nullptr;
    float *sfold = nullptr;  // the score epilogue's per-tile statistics, target logits and padded targets
    void *ws = nullptr;
    // fast path: the GEMMs' K-split partial products, after the widest split x in ws (the fused
    // RMSNorm reads one product's deferred partial sums while it writes the next product's split
    // x, which is sized for another width)
    float *part = nullptr;
    // split attention operands (head dims 32, 64, 128): f16 parts and exponents, rows padded to 32
    _Float16 *sqh = nullptr, *sql = nullptr, *skh = nullptr, *skl = nullptr, *svh = nullptr, *svl = nullptr;
    int8_t *seq = nullptr, *sek = nullptr, *sev = nullptr;

    size_t q_dim() const { return heads * head_dim; }
    size_t kv_dim() const { return kv_heads * head_dim; }
    size_t qkv_width() const { return q_dim() + 2 * kv_dim(); }
};

namespace {

constexpr uint32_t kMaxQkvWidth = 12288;  // floats of one qkv row the RoPE kernel stages in LDS (48 KiB)
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---- kernels ----

// Row r of x = the token embedding of ids[r], dequantised from the packed rows. An id outside
// the vocabulary reads row 0 and poisons the row with NaN (the host entry points refuse such ids
// before launching; the device-resident one documents it).
template <fh_kind KIND>
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ ds,
                                                         const int32_t *__restrict__ ids, float *__restrict__ x, uint32_t d,
                                                         uint32_t vocab) {
    const uint32_t r = blockIdx.x;
    const int32_t id = ids[r];
    const bool ok = id >= 0 && (uint32_t)id < vocab;
    const uint32_t t = ok ? (uint32_t)id : 0u;
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
        x[(size_t)r * d + i] = ok ? half_bits_to_float(ds[scale_slot(t, b, nb)]) * q : NAN;
    }
}

// Row r of x = row ids[r] of an f32 token embedding (vocab rows of d); an id outside the
// vocabulary poisons the row with NaN, as above.
__global__ __launch_bounds__(256) void embed_rows_f32_kernel(const float *__restrict__ tok, const int32_t *__restrict__ ids,
                                                             float *__restrict__ x, uint32_t d, uint32_t vocab) {
    const uint32_t r = blockIdx.x;
    const int32_t id = ids[r];
    const bool ok = id >= 0 && (uint32_t)id < vocab;
    const size_t row = (size_t)(ok ? (uint32_t)id : 0u) * d;
    for (uint32_t i = threadIdx.x; i < d; i += blockDim.x) x[(size_t)r * d + i] = ok ? tok[row + i] : NAN;
}

// y[M][N] = x[M][K] . W^T for an f32 matrix held as N rows of K (the product of an unpacked
// Mat; any K). 64 x 64 outputs a workgroup, K in steps of 16 staged in LDS (k-major, so a
// wavefront reads 16 consecutive columns and 4 broadcast rows), 4 x 4 outputs a thread (rows
// ty + 16 i, columns tx + 16 j), each an fma chain in ascending k.
__global__ __launch_bounds__(256) void linear_f32_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                         float *__restrict__ y, uint32_t M, uint32_t K, uint32_t N) {
    __shared__ float xs[16][65], ws[16][65];
    const uint32_t m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const uint32_t tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const uint32_t lr = threadIdx.x / 4, lk = threadIdx.x % 4 * 4;  // this thread's loads: row lr, k lk..lk+3
    float acc[4][4] = {};
    for (uint32_t k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t k = k0 + lk + e;
            xs[lk + e][lr] = m0 + lr < M && k < K ? x[(size_t)(m0 + lr) * K + k] : 0.0f;
            ws[lk + e][lr] = n0 + lr < N && k < K ? w[(size_t)(n0 + lr) * K + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = xs[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = ws[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (m0 + ty + 16 * i < M && n0 + tx + 16 * j < N)
                y[(size_t)(m0 + ty + 16 * i) * N + n0 + tx + 16 * j] = acc[i][j];
}

// Sum over a block of 256 threads (four wavefronts); every thread gets the total.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
    v = wave_reduce(v, AddOp());
    const uint32_t w = threadIdx.x >> 6;
    __syncthreads();  // red may still be read by a previous call
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}


// Element i of a product that a GEMM left as K-split partial sums (SplitOut: `splits` slices
// `stride` floats apart, summed in split order as the reduction kernel would; one slice: p[i]).
__device__ __forceinline__ float split_sum(const float *__restrict__ p, size_t i, uint32_t splits, size_t stride) {
    float t = p[i];
    for (uint32_t sl = 1; sl < splits; sl++) t += p[sl * stride + i];
    return t;
}

// One row of an RMSNorm's input (ferrum_ref/src/models/llama/ops.rs:55-66): v = x, or with ADD
// v = x + o (the residual add, nn::add; o possibly K-split partial sums, added in split order)
// stored back into x. A thread takes float4 chunks q = tid + 256 i: chunk i < kKeepRow stays in
// registers (rows up to 8192 floats; wider rows are read again), and a chunk's x and partial-sum
// loads are issued together before any is added (a loop of dependent loads cost one round trip
// per split). Returns the thread's sum of squares, chunk by chunk in order. Rows of whole float4s.
constexpr int kKeepRow = 8;
constexpr uint32_t kMaxSplits = 8;  // the MFMA GEMMs' K splits (gemm_splits)
// Four consecutive elements (at offset off) of a product left as `splits` partial sums `stride`
// floats apart, added in split order; the first kMaxSplits loads are issued together.
__device__ __forceinline__ f32x4 split_chunk(const float *__restrict__ o, size_t off, uint32_t splits, size_t stride) {
    f32x4 p[kMaxSplits];
#pragma unroll
    for (uint32_t sl = 0; sl < kMaxSplits; sl++) p[sl] = *(const f32x4 *)(o + (sl < splits ? sl : 0u) * stride + off);
    f32x4 t = p[0];
#pragma unroll
    for (uint32_t sl = 1; sl < kMaxSplits; sl++) t = sl < splits ? t + p[sl] : t;
    for (uint32_t sl = kMaxSplits; sl < splits; sl++) t += *(const f32x4 *)(o + sl * stride + off);
    return t;
}
template <bool ADD>
__device__ __forceinline__ f32x4 row_chunk(float *__restrict__ x, const float *__restrict__ o, size_t base, uint32_t q,
                                           uint32_t splits, size_t stride) {
    f32x4 v = *(const f32x4 *)(x + base + 4 * q);
    if constexpr (ADD) v = v + split_chunk(o, base + 4 * q, splits, stride);
    return v;
}
template <bool ADD>
__device__ __forceinline__ float row_load4(float *__restrict__ x, const float *__restrict__ o, size_t base, uint32_t nq,
                                           uint32_t splits, size_t stride, f32x4 (&v)[kKeepRow]) {
    float ss = 0.0f;
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kKeepRow; i++) {
        v[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (256u * i >= nq) continue;  // the workgroup agrees
        const uint32_t q = tid + 256 * i;
        const f32x4 w = row_chunk<ADD>(x, o, base, q < nq ? q : nq - 1, splits, stride);
        if (q < nq) {
            if constexpr (ADD) *(f32x4 *)(x + base + 4 * q) = w;
            v[i] = w;
#pragma unroll
            for (int c = 0; c < 4; c++) ss += w[c] * w[c];
        }
    }
    for (uint32_t q = tid + 256 * kKeepRow; q < nq; q += 256) {
        const f32x4 w = row_chunk<ADD>(x, o, base, q, splits, stride);
        if constexpr (ADD) *(f32x4 *)(x + base + 4 * q) = w;
#pragma unroll
        for (int c = 0; c < 4; c++) ss += w[c] * w[c];
    }
    return ss;
}
// Chunk q of the normalised row h = v / sqrt(mean(v^2) + eps) * g (two roundings, as ops.rs).
__device__ __forceinline__ f32x4 row_norm4(f32x4 v, const float *__restrict__ g, uint32_t q, float inv) {
    const f32x4 gg = *(const f32x4 *)(g + 4 * q);
    f32x4 h;
#pragma unroll
    for (int c = 0; c < 4; c++) h[c] = __fmul_rn(__fmul_rn(v[c], inv), gg[c]);
    return h;
}

// RMSNorm per row (ferrum_ref/src/models/llama/ops.rs:55-66): h = v / sqrt(mean(v^2) + eps) * g,
// v = x, or with ADD v = x + o stored back into x first (the residual add, nn::add). Rows of whole
// float4s take row_load4 (as rmsnorm_split_kernel, so the fast path's fused producers give the same
// bits); others one element per thread.
template <bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_kernel(float *__restrict__ x, const float *__restrict__ o,
                                                      const float *__restrict__ g, float *__restrict__ h, uint32_t d,
                                                      float eps, uint32_t o_splits, size_t o_stride) {
    __shared__ float red[4];
    const size_t base = (size_t)blockIdx.x * d;
    if (d % 4 == 0) {
        const uint32_t nq = d / 4;
        f32x4 v[kKeepRow];
        const float ms = block_sum_256(row_load4<ADD>(x, o, base, nq, o_splits, o_stride, v), red) / (float)d;
        const float inv = 1.0f / sqrtf(ms + eps);
#pragma unroll
        for (int i = 0; i < kKeepRow; i++) {
            const uint32_t q = threadIdx.x + 256 * i;
            if (q < nq) *(f32x4 *)(h + base + 4 * q) = row_norm4(v[i], g, q, inv);
        }
        for (uint32_t q = threadIdx.x + 256 * kKeepRow; q < nq; q += 256)
            *(f32x4 *)(h + base + 4 * q) = row_norm4(*(const f32x4 *)(x + base + 4 * q), g, q, inv);
        return;
    }
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < d; i += 256) {
        float v = x[base + i];
        if constexpr (ADD) {
            v = v + split_sum(o, base + i, o_splits, o_stride);
            x[base + i] = v;
        }
        ss += v * v;
    }
    const float ms = block_sum_256(ss, red) / (float)d;
    const float inv = 1.0f / sqrtf(ms + eps);
    for (uint32_t i = threadIdx.x; i < d; i += 256) h[base + i] = __fmul_rn(__fmul_rn(x[base + i], inv), g[i]);
}

// The fast path's fused producers: rmsnorm_kernel and swiglu_kernel with the same arithmetic,
// written straight into the fast GEMM's split x (split_chunk4: from the threads' registers where
// the row is whole 32-element blocks, else through a row in LDS and split_row_fast), so the f32
// activation is never written to memory and read back by a split pass. One workgroup per row.
template <bool ADD, int KIND>
__global__ __launch_bounds__(256) void rmsnorm_split_kernel(float *__restrict__ x, const float *__restrict__ o,
                                                            const float *__restrict__ g, uint32_t d, float eps,
                                                            uint32_t o_splits, size_t o_stride, GemmXSplit dst) {
    extern __shared__ __attribute__((aligned(16))) float hrow[];
    __shared__ float red[4];
    const size_t base = (size_t)blockIdx.x * d;
    if (d % 32 == 0) {
        // a thread's chunks go from registers straight into the split (float4 q = tid + 256 i is
        // the one split_row_fast gives it: eight consecutive lanes hold a block)
        const uint32_t nq = d / 4, nb = d / 32, K64 = (d + 63) / 64 * 64, MS = xsb_rows(gridDim.x), m = blockIdx.x;
        f32x4 v[kKeepRow];
        const float ms = block_sum_256(row_load4<ADD>(x, o, base, nq, o_splits, o_stride, v), red) / (float)d;
        const float inv = 1.0f / sqrtf(ms + eps);
#pragma unroll
        for (int i = 0; i < kKeepRow; i++) {
            const uint32_t q = threadIdx.x + 256 * i;
            if (q < nq)
                split_chunk4<KIND>(row_norm4(v[i], g, q, inv), m, q / 8, q % 8, MS, nb, K64, dst.xh, dst.xl, dst.xsb);
        }
        for (uint32_t q = threadIdx.x + 256 * kKeepRow; q < nq; q += 256)
            split_chunk4<KIND>(row_norm4(*(const f32x4 *)(x + base + 4 * q), g, q, inv), m, q / 8, q % 8, MS, nb, K64,
                               dst.xh, dst.xl, dst.xsb);
        return;
    }
    if (d % 4 == 0) {
        const uint32_t nq = d / 4;
        f32x4 v[kKeepRow];
        const float ms = block_sum_256(row_load4<ADD>(x, o, base, nq, o_splits, o_stride, v), red) / (float)d;
        const float inv = 1.0f / sqrtf(ms + eps);
#pragma unroll
        for (int i = 0; i < kKeepRow; i++) {
            const uint32_t q = threadIdx.x + 256 * i;
            if (q < nq) *(f32x4 *)&hrow[4 * q] = row_norm4(v[i], g, q, inv);
        }
        for (uint32_t q = threadIdx.x + 256 * kKeepRow; q < nq; q += 256)
            *(f32x4 *)&hrow[4 * q] = row_norm4(*(const f32x4 *)(x + base + 4 * q), g, q, inv);
    } else {
        float ss = 0.0f;
        for (uint32_t i = threadIdx.x; i < d; i += 256) {
            float v = x[base + i];
            if constexpr (ADD) {
                v = v + split_sum(o, base + i, o_splits, o_stride);
                x[base + i] = v;
            }
            ss += v * v;
        }
        const float ms = block_sum_256(ss, red) / (float)d;
        const float inv = 1.0f / sqrtf(ms + eps);
        for (uint32_t i = threadIdx.x; i < d; i += 256) hrow[i] = __fmul_rn(__fmul_rn(x[base + i], inv), g[i]);
    }
    __syncthreads();
    split_row_fast<KIND>([&](uint32_t q) { return *(const f32x4 *)&hrow[4 * q]; }, blockIdx.x, gridDim.x, d, dst.xh,
                         dst.xl, dst.xsb);
}

// INTER: gu's columns are gate and up interleaved in runs of 32 (the weight loaded for the
// SwiGLU epilogue, when a product's shape does not take that epilogue): unit j's gate at column
// 64 (j / 32) + j % 32, its up 32 columns later.
template <int KIND, bool INTER = false>
__global__ __launch_bounds__(256) void swiglu_split_kernel(const float *__restrict__ gu, uint32_t hid, GemmXSplit dst) {
    extern __shared__ __attribute__((aligned(16))) float hrow[];
    const size_t r = blockIdx.x;
    const uint32_t nq = hid / 4;
    auto act = [&](uint32_t j, f32x4 gg, f32x4 u) {
        f32x4 y;
#pragma unroll
        for (int c = 0; c < 4; c++) y[c] = swiglu_act(gg[c], u[c]);
        *(f32x4 *)&hrow[4 * j] = y;
    };
    // units 4j .. 4j + 3: their gate columns (up: + hid, or + 32 when interleaved)
    auto gcol = [&](uint32_t j) { return INTER ? 64 * (4 * j / 32) + (4 * j) % 32 : 4 * j; };
    const uint32_t uoff = INTER ? 32 : hid;
    // the row's first kKeepRow chunks are all requested before any is used (one round trip)
    f32x4 gk[kKeepRow], uk[kKeepRow];
#pragma unroll
    for (int i = 0; i < kKeepRow; i++) {
        if (256u * i >= nq) continue;  // the workgroup agrees
        const uint32_t j = min(threadIdx.x + 256 * i, nq - 1);
        gk[i] = *(const f32x4 *)(gu + r * 2 * hid + gcol(j));
        uk[i] = *(const f32x4 *)(gu + r * 2 * hid + uoff + gcol(j));
    }
#pragma unroll
    for (int i = 0; i < kKeepRow; i++) {
        const uint32_t j = threadIdx.x + 256 * i;
        if (256u * i < nq && j < nq) act(j, gk[i], uk[i]);
    }
    for (uint32_t j = threadIdx.x + 256 * kKeepRow; j < nq; j += 256)
        act(j, *(const f32x4 *)(gu + r * 2 * hid + gcol(j)), *(const f32x4 *)(gu + r * 2 * hid + uoff + gcol(j)));
    __syncthreads();
    split_row_fast<KIND>([&](uint32_t q) { return *(const f32x4 *)&hrow[4 * q]; }, (uint32_t)r, gridDim.x, hid, dst.xh,
                         dst.xl, dst.xsb);
}

// q/k/v bias and RoPE on one row of qkv (ferrum_ref/src/models/llama/ops.rs:105-127): the row's
// q and k heads rotate their first rope_dim channels by table row `row` (the position), NORM
// pairing (2i, 2i + 1) or NEOX (i, i + rope_dim / 2). The row is staged in LDS so every output
// reads the biased inputs. qkv_rope_row loads row `r` (its K-split partial sums and the bias)
// into LDS; rope_value is channel c of the rotated row.
__device__ __forceinline__ void qkv_rope_row(const float *__restrict__ src, uint32_t src_splits, size_t src_stride,
                                             const float *__restrict__ bias, uint32_t width, uint32_t r,
                                             float *row) {
    const size_t base = (size_t)r * width;
    if (width % 4 == 0) {  // four elements a thread, the splits' loads issued together
        for (uint32_t q = threadIdx.x; q < width / 4; q += 256) {
            const f32x4 v = split_chunk(src, base + 4 * q, src_splits, src_stride);
            *(f32x4 *)&row[4 * q] = bias ? v + *(const f32x4 *)(bias + 4 * q) : v;
        }
    } else {
        for (uint32_t c = threadIdx.x; c < width; c += 256) {
            const float v = split_sum(src, base + c, src_splits, src_stride);
            row[c] = bias ? v + bias[c] : v;
        }
    }
}

__device__ __forceinline__ float rope_value(const float *row, uint32_t c, const float *cr, const float *sr,
                                            uint32_t rotated, uint32_t hd, uint32_t rope_dim, int neox) {
    float v = row[c];
    if (c < rotated) {
        const uint32_t j = c % hd, off = c - j, half = rope_dim / 2;
        if (j < rope_dim) {
            const bool first = neox ? j < half : (j & 1u) == 0;
            const uint32_t i = neox ? (first ? j : j - half) : j / 2;
            const uint32_t ia = neox ? off + i : off + 2 * i, ib = neox ? ia + half : ia + 1;
            const float a = row[ia], b = row[ib], cs = cr[i], sn = sr[i];
            v = first ? __fsub_rn(__fmul_rn(a, cs), __fmul_rn(b, sn)) : __fadd_rn(__fmul_rn(a, sn), __fmul_rn(b, cs));
        }
    }
    return v;
}

__global__ __launch_bounds__(256) void qkv_rope_kernel(const float *__restrict__ src, uint32_t src_splits,
                                                       size_t src_stride, float *__restrict__ qkv,
                                                       const float *__restrict__ bias, const float *__restrict__ cos_t,
                                                       const float *__restrict__ sin_t, uint32_t width,
                                                       uint32_t rot_heads, uint32_t hd, uint32_t rope_dim, int neox) {
    extern __shared__ __attribute__((aligned(16))) float row[];
    qkv_rope_row(src, src_splits, src_stride, bias, width, blockIdx.x, row);
    __syncthreads();
    const uint32_t half = rope_dim / 2;
    const float *cr = cos_t + (size_t)blockIdx.x * half, *sr = sin_t + (size_t)blockIdx.x * half;
    for (uint32_t c = threadIdx.x; c < width; c += 256)
        qkv[(size_t)blockIdx.x * width + c] = rope_value(row, c, cr, sr, rot_heads * hd, hd, rope_dim, neox);
}

// Causal grouped-query attention (ferrum_ref/src/models/llama/ops.rs:131-162 for every row) from
// qkv [t, width] (the q heads, then the k heads, then the v heads, each HD wide) into att
// [t, heads * HD]. A workgroup takes 32 query rows of one head; its W wavefronts split the key
// tiles (32 keys each) round robin, each keeping an online softmax, and are merged through LDS
// at the end. Both products run on v_mfma_f32_32x32x2_f32 in f32:
//   S^T (32 keys x 32 queries) = K . Q^T: lane l (key or query l % 32, slot l / 32) feeds dims
//     8m + 4 slot + c at step 4m + c, so K and Q load as float4;
//   O^T (32 dims x 32 queries) += V^T . P^T: at step s the B operand is the S^T accumulator's
//     register s (key 8 (s / 4) + 4 slot + s % 4 of query l % 32) and the A operand that key's
//     value at dim l % 32, a coalesced row segment.
// Each lane owns one query (l % 32) throughout: lanes l and l ^ 32 share its running maximum and
// split its running sum. A wavefront loads the next tile's K and V while it computes the current
// one.
template <int HD>
struct AttnTile {
    static constexpr int M4 = HD / 8;                  // float4 pairs per row
    static constexpr int DB = HD >= 32 ? HD / 32 : 1;  // 32-dim blocks of the output
    f32x4 k[M4];
    float v[DB][16];
};

template <int HD>
__device__ __forceinline__ void attn_load(AttnTile<HD> &T, const float *__restrict__ qkv, uint32_t k0, uint32_t t,
                                          uint32_t width, uint32_t kofs, uint32_t vofs, uint32_t col, uint32_t slot) {
    const uint32_t key = k0 + col;
    const bool ok = key < t;
    const float *krow = qkv + (size_t)(ok ? key : 0u) * width + kofs + 4 * slot;
#pragma unroll
    for (int m = 0; m < AttnTile<HD>::M4; m++) T.k[m] = ok ? *(const f32x4 *)(krow + 8 * m) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < AttnTile<HD>::DB; b++) {
        const uint32_t dim = 32 * b + col;
        const bool dok = dim < (uint32_t)HD;
#pragma unroll
        for (int st = 0; st < 16; st++) {
            const uint32_t kk = k0 + 8 * (st / 4) + 4 * slot + (st % 4);
            T.v[b][st] = dok && kk < t ? qkv[(size_t)kk * width + vofs + dim] : 0.0f;
        }
    }
}

template <int HD, int W>
__global__ __launch_bounds__(64 * W) void attention_kernel(const float *__restrict__ qkv, float *__restrict__ att,
                                                           uint32_t t, uint32_t width, uint32_t heads, uint32_t group,
                                                           float scale) {
    using T = AttnTile<HD>;
    constexpr int DB = T::DB;
    __shared__ float red[W][2 + 16 * DB][64];
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6, col = lane & 31u, slot = lane >> 5;
    // grid (heads, query blocks): workgroups are dispatched x fastest, so every head's longest
    // query blocks start first and the short ones fill in at the end
    const uint32_t q0 = (gridDim.y - 1 - blockIdx.y) * 32;
    const uint32_t h = blockIdx.x, g = h / group, kv_heads = heads / group;
    const uint32_t qd = heads * HD;
    const uint32_t kofs = qd + g * HD, vofs = qd + kv_heads * HD + g * HD;
    const uint32_t query = q0 + col;
    f32x4 qf[T::M4];
    {
        const bool ok = query < t;
        const float *qrow = qkv + (size_t)(ok ? query : 0u) * width + h * HD + 4 * slot;
#pragma unroll
        for (int m = 0; m < T::M4; m++) qf[m] = ok ? *(const f32x4 *)(qrow + 8 * m) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    f32x16 o[DB];
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[b][i] = 0.0f;
    float mrun = -INFINITY, lrun = 0.0f;
    const uint32_t tiles = (min(q0 + 31u, t - 1u)) / 32 + 1;  // key tiles any valid query of the block sees
    T cur, nxt;
    if (w < tiles) attn_load<HD>(cur, qkv, 32 * w, t, width, kofs, vofs, col, slot);
    for (uint32_t kt = w; kt < tiles; kt += W) {
        const uint32_t k0 = 32 * kt;
        if (kt + W < tiles) attn_load<HD>(nxt, qkv, k0 + 32 * W, t, width, kofs, vofs, col, slot);
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; i++) s[i] = 0.0f;
#pragma unroll
        for (int m = 0; m < T::M4; m++)
#pragma unroll
            for (int c = 0; c < 4; c++) s = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.k[m][c], qf[m][c], s, 0, 0, 0);
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t key = k0 + 8 * (i / 4) + 4 * slot + (i % 4);
            const float v = key <= query ? s[i] * scale : -INFINITY;
            s[i] = v;
            mt = fmaxf(mt, v);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mnew = fmaxf(mrun, mt);  // finite: key k0 <= query in every tile
        const float alpha = __expf(mrun - mnew);
        float ls = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            s[i] = __expf(s[i] - mnew);
            ls += s[i];
        }
        lrun = lrun * alpha + ls;
        mrun = mnew;
#pragma unroll
        for (int b = 0; b < DB; b++) {
#pragma unroll
            for (int i = 0; i < 16; i++) o[b][i] *= alpha;
#pragma unroll
            for (int st = 0; st < 16; st++) o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.v[b][st], s[st], o[b], 0, 0, 0);
        }
        cur = nxt;
    }
    // merge the wavefronts' partial softmaxes: M = max m_w, O = sum O_w e^(m_w - M), l likewise
    red[w][0][lane] = mrun;
    red[w][1][lane] = lrun;
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) red[w][2 + 16 * b + i][lane] = o[b][i];
    __syncthreads();
    if (w) return;
    float M = red[0][0][lane];
#pragma unroll
    for (int j = 1; j < W; j++) M = fmaxf(M, red[j][0][lane]);
    float f[W], l = 0.0f;
#pragma unroll
    for (int j = 0; j < W; j++) {
        f[j] = __expf(red[j][0][lane] - M);  // a wavefront without tiles: e^(-inf) = 0
        l += red[j][1][lane] * f[j];
    }
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    if (query >= t) return;
    float *out = att + (size_t)query * qd + h * HD;
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t dim = 32 * b + 8 * (i / 4) + 4 * slot + (i % 4);
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < W; j++) acc += red[j][2 + 16 * b + i][lane] * f[j];
            if (dim < (uint32_t)HD) out[dim] = acc * inv;
        }
}

// ---- attention on the f16 matrix cores, f32-accurate (head dims 32, 64, 128) ----
// Every head row of q, k and v (after RoPE) is put on a power-of-two scale, x' = x 2^-e with
// max |x'| in [2^14, 2^15), and split into two f16 parts x' = hi + lo (hi = f16(x'), lo =
// f16(x' - hi): 22 significant bits, no f16 overflow or underflow to speak of). A product of
// two such values is hi hi + hi lo + lo hi up to 2^-22 of its size (the lo lo term dropped), so
// each f32-accurate 32 x 32 x 16 product costs three v_mfma_f32_32x32x16_f16 instead of eight
// v_mfma_f32_32x32x2_f32 of twice the length. Layouts (tp = t rounded up to 32, rows t .. tp - 1
// zero with exponent -127): q' [tp, heads HD] row-major; k' and v' in the attention kernel's
// fragment order, per kv head and 32-key tile one 32 HD block, in which every 64-lane load
// instruction of the kernel reads 1 KB contiguous (a row-major k' spread each such load over 32
// key rows): k' [s = dim / 16][lane][8], the lane being the A-matrix row that holds the key
// (key_row) plus 32 for dims 8..15 of the 16; v' [b = dim / 32][u = key / 16 % 2][lane][8], lane
// = dim % 32 + 32 (key / 8 % 2), the 8 being keys; exponents [slot, tp] as bytes.
constexpr int kSplitPad = -127;

// The A-matrix row of S^T that holds key r of a 32-key tile: row rho = 16 u + w holds key 16 u +
// 8 ((w % 8) / 4) + 4 (w / 8) + w % 4, so that accumulator register i of lane half h holds key
// 16 (i / 8) + 8 h + i % 8; the map swaps bits 2 and 3 of the key's index within its 16.
__device__ __forceinline__ uint32_t key_row(uint32_t r) { return (r & 19u) | ((r & 4u) << 1) | ((r & 8u) >> 1); }

// Offsets (in halves) of the fragment-order k' and v' element (key, dim) of kv head g.
template <int HD>
__device__ __forceinline__ size_t frag_k(uint32_t g, uint32_t key, uint32_t dim, uint32_t tp) {
    const uint32_t lane = key_row(key % 32) + 32 * ((dim % 16) / 8);
    return ((size_t)g * (tp / 32) + key / 32) * (32 * HD) + (dim / 16) * 512 + lane * 8 + dim % 8;
}
template <int HD>
__device__ __forceinline__ size_t frag_v(uint32_t g, uint32_t key, uint32_t dim, uint32_t tp) {
    const uint32_t lane = dim % 32 + 32 * ((key % 16) / 8);
    return ((size_t)g * (tp / 32) + key / 32) * (32 * HD) + ((dim / 32) * 2 + (key % 32) / 16) * 512 + lane * 8 +
           key % 8;
}

// Where the split operands go (layouts above).
struct SplitDst {
    _Float16 *qh, *ql, *kh, *kl, *vh, *vl;
    int8_t *eq, *ek, *ev;
};

// The exponent e of one (row, head) of the split operands, from the head's values v[i] (dim lane
// + 64 i) over the wavefront: 2^E <= max |v| < 2^(E+1), e = E - 14; zero rows, padding rows and
// non-finite rows keep e = 0 (non-finite values then stay non-finite).
__device__ __forceinline__ int head_exponent(const float (&v)[2]) {
    float mx = fmaxf(fabsf(v[0]), fabsf(v[1]));
    mx = wave_reduce(mx, MaxOp());
    int e = 0;
    if (mx > 0.0f && mx <= 3.4028235e38f) e = ((int)(__float_as_uint(mx) >> 23) - 127) - 14;
    return e < -100 ? -100 : (e > 100 ? 100 : e);
}

// Row `row` of every q, k and v head into its split form, one head per wavefront at a time;
// get(slot, d) is element d of head slot (q heads, then k heads, then v heads) of the row.
template <int HD, class Get>
__device__ __forceinline__ void split_heads(Get get, const SplitDst &o, uint32_t row, uint32_t t, uint32_t tp,
                                            uint32_t heads, uint32_t kv_heads) {
    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const uint32_t qd = heads * HD;
    for (uint32_t slot = wave; slot < heads + 2 * kv_heads; slot += 4) {
        float v[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t d = lane + 64 * i;
            v[i] = row < t && d < (uint32_t)HD ? get(slot, d) : 0.0f;
        }
        const int e = head_exponent(v);  // padding rows report kSplitPad
        const float f = ldexpf(1.0f, -e);
        const int8_t code = row < t ? (int8_t)e : (int8_t)kSplitPad;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t d = lane + 64 * i;
            if (d >= (uint32_t)HD) continue;
            const float x = v[i] * f;
            const _Float16 hi = (_Float16)x, lo = (_Float16)(x - (float)hi);
            if (slot < heads) {
                const size_t at = (size_t)row * qd + slot * HD + d;
                o.qh[at] = hi;
                o.ql[at] = lo;
            } else if (slot < heads + kv_heads) {
                const size_t at = frag_k<HD>(slot - heads, row, d, tp);
                o.kh[at] = hi;
                o.kl[at] = lo;
            } else {
                const size_t at = frag_v<HD>(slot - heads - kv_heads, row, d, tp);
                o.vh[at] = hi;
                o.vl[at] = lo;
            }
        }
        if (lane == 0) {
            if (slot < heads)
                o.eq[(size_t)slot * tp + row] = code;
            else if (slot < heads + kv_heads)
                o.ek[(size_t)(slot - heads) * tp + row] = code;
            else
                o.ev[(size_t)(slot - heads - kv_heads) * tp + row] = code;
        }
    }
}

// The split operands from qkv [t, width] (already biased and rotated); one workgroup per row of
// tp, rows t .. tp - 1 written as zeros.
template <int HD>
__global__ __launch_bounds__(256) void attn_split_kernel(const float *__restrict__ qkv, SplitDst o, uint32_t t,
                                                         uint32_t tp, uint32_t width, uint32_t heads,
                                                         uint32_t kv_heads) {
    const uint32_t row = blockIdx.x;
    split_heads<HD>([&](uint32_t slot, uint32_t d) { return qkv[(size_t)row * width + slot * HD + d]; }, o, row, t,
                    tp, heads, kv_heads);
}

// qkv_rope_kernel and attn_split_kernel in one pass, per R-row tile of tp (R = 16 or 32) and head
// slot (q heads, then k heads, then v heads): the tile's rows of the slot (the QKV product's
// K-split partial sums in split order, then the bias) into LDS; per row, RoPE (rope_value, the same
// roundings) and the split as split_heads, assembled in LDS in the destination's order (q' rows,
// or the tile's part of a 32-key fragment block of k' or v', whose keys 0-15 and 16-31 fill
// separate 128-byte lines); then 16-byte stores, so each destination line is written whole by one
// workgroup. The f32 q, k and v are not written. Grid (tp / R, heads + 2 kv_heads); rows t .. tp - 1
// are written as zeros.
template <int HD, int R>
__global__ __launch_bounds__(256) void qkv_rope_split_kernel(const float *__restrict__ src, uint32_t src_splits,
                                                             size_t src_stride, const float *__restrict__ bias,
                                                             const float *__restrict__ cos_t,
                                                             const float *__restrict__ sin_t, SplitDst o, uint32_t t,
                                                             uint32_t tp, uint32_t width, uint32_t heads,
                                                             uint32_t kv_heads, uint32_t rope_dim, int neox) {
    static_assert(R == 16 || R == 32, "tiles of half or whole 32-key fragment blocks");
    constexpr uint32_t C4 = HD / 4, C8 = HD / 8;  // float4 chunks and 8-half chunks per row of a head
    __shared__ __attribute__((aligned(16))) float tile[R][HD];
    __shared__ __attribute__((aligned(16))) _Float16 part[2][32 * HD];  // hi and lo, destination order
    const uint32_t r0 = blockIdx.x * R, slot = blockIdx.y, tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const uint32_t kind = slot < heads ? 0u : slot < heads + kv_heads ? 1u : 2u;  // q, k, v
    const uint32_t k0 = r0 % 32;  // the tile's first key in its fragment block
    for (uint32_t q = tid; q < R * C4; q += 256) {
        const uint32_t rr = q / C4, c = q % C4, r = r0 + rr;
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (r < t) {
            v = split_chunk(src, (size_t)r * width + slot * HD + 4 * c, src_splits, src_stride);
            if (bias) v = v + *(const f32x4 *)(bias + slot * HD + 4 * c);
        }
        *(f32x4 *)&tile[rr][4 * c] = v;
    }
    __syncthreads();
    const uint32_t half = rope_dim / 2;
    // LPR lanes per row, four dims each, RPI rows of the wavefront's R / 4 at a time; the row's
    // largest |value| (head_exponent's) by shuffles within its LPR lanes
    constexpr uint32_t LPR = HD / 4, RPI = 64 / LPR, ROWS = R / 4;
    for (uint32_t it = 0; it < (ROWS + RPI - 1) / RPI; it++) {
        const uint32_t rl = it * RPI + lane / LPR;
        if (rl >= ROWS) break;  // (a whole group of LPR lanes)
        const uint32_t rr = wave * ROWS + rl, r = r0 + rr, d0 = 4 * (lane % LPR);
        float v[4], mx = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            v[c] = r < t ? rope_value(tile[rr], d0 + c, cos_t + (size_t)r * half, sin_t + (size_t)r * half,
                                      kind < 2 ? HD : 0u, HD, rope_dim, neox)
                         : 0.0f;
            mx = fmaxf(mx, fabsf(v[c]));
        }
#pragma unroll
        for (uint32_t o = 1; o < LPR; o *= 2) mx = fmaxf(mx, __shfl_xor(mx, o, LPR));
        int e = 0;  // as head_exponent
        if (mx > 0.0f && mx <= 3.4028235e38f) e = ((int)(__float_as_uint(mx) >> 23) - 127) - 14;
        e = e < -100 ? -100 : (e > 100 ? 100 : e);
        const float f = ldexpf(1.0f, -e);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t d = d0 + c;
            const float x = v[c] * f;
            const _Float16 hi = (_Float16)x, lo = (_Float16)(x - (float)hi);
            const size_t at =
                kind == 0 ? rr * HD + d : kind == 1 ? frag_k<HD>(0, k0 + rr, d, 32) : frag_v<HD>(0, k0 + rr, d, 32);
            part[0][at] = hi;
            part[1][at] = lo;
        }
        if (lane % LPR == 0) {
            const int8_t code = r < t ? (int8_t)e : (int8_t)kSplitPad;
            if (kind == 0)
                o.eq[(size_t)slot * tp + r] = code;
            else if (kind == 1)
                o.ek[(size_t)(slot - heads) * tp + r] = code;
            else
                o.ev[(size_t)(slot - heads - kv_heads) * tp + r] = code;
        }
    }
    __syncthreads();
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    for (uint32_t c = tid; c < R * C8; c += 256) {
        // chunk c's place among the 8-half chunks of the q' tile or of the 32-key block: a 16-key
        // tile holds, of k', lanes k0 .. k0 + 15 and 32 + k0 .. of each 16-dim slab (key_row keeps
        // bit 4), and of v', the u = k0 / 16 halves of each 32-dim part
        uint32_t ch = c;
        if (R == 16 && kind == 1) ch = c / 32 * 64 + (c % 32 < 16 ? k0 + c % 32 : 32 + k0 + c % 32 - 16);
        if (R == 16 && kind == 2) ch = (c / 64 * 2 + k0 / 16) * 64 + c % 64;
        const h8 a = *(const h8 *)&part[0][8 * ch], b = *(const h8 *)&part[1][8 * ch];
        if (kind == 0) {
            const size_t at = (size_t)(r0 + c / C8) * (heads * HD) + slot * HD + 8 * (c % C8);
            *(h8 *)(o.qh + at) = a;
            *(h8 *)(o.ql + at) = b;
        } else {
            const uint32_t g = kind == 1 ? slot - heads : slot - heads - kv_heads;
            const size_t at = ((size_t)g * (tp / 32) + r0 / 32) * (32 * HD) + 8 * ch;
            *(h8 *)((kind == 1 ? o.kh : o.vh) + at) = a;
            *(h8 *)((kind == 1 ? o.kl : o.vl) + at) = b;
        }
    }
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// One key tile (32 keys) of one wavefront's lanes: k' fragments of A row l % 32 (key k0 + pi(l %
// 32)) and the exponents of the lane's sixteen accumulator keys 16 u + 8 (l / 32) + 0..7 (loaded
// a tile ahead); v' fragments (dims 32 b + l % 32, keys 16 u + 8 (l / 32) + 0..7), loaded when the
// tile starts.
template <int HD>
struct SplitTile {
    static constexpr int KS = HD / 16, DB = HD / 32;
    f16x8 kh[KS], kl[KS];
    uint64_t ek[2], ev[2];
};
template <int HD>
struct SplitV {
    f16x8 vh[HD / 32][2], vl[HD / 32][2];
};

template <int HD>
__device__ __forceinline__ void split_load_v(SplitV<HD> &T, const _Float16 *__restrict__ vh,
                                             const _Float16 *__restrict__ vl, uint32_t k0, uint32_t tp, uint32_t g,
                                             uint32_t col, uint32_t hf) {
    const size_t vo = frag_v<HD>(g, k0 + 8 * hf, col, tp);  // (b, u) = (0, 0); each further one 512 on
#pragma unroll
    for (int b = 0; b < HD / 32; b++)
#pragma unroll
        for (int u = 0; u < 2; u++) {
            T.vh[b][u] = *(const f16x8 *)(vh + vo + (2 * b + u) * 512);
            T.vl[b][u] = *(const f16x8 *)(vl + vo + (2 * b + u) * 512);
        }
}

template <int HD>
__device__ __forceinline__ void split_load(SplitTile<HD> &T, const _Float16 *__restrict__ kh,
                                           const _Float16 *__restrict__ kl, const int8_t *__restrict__ ek,
                                           const int8_t *__restrict__ ev, uint32_t k0, uint32_t tp, uint32_t g,
                                           uint32_t col, uint32_t hf) {
    // lane (col, hf) holds A row col of S^T, the tile's key key_row(col) (key_row is its own
    // inverse), dims 16 s + 8 hf + 0..7
    const size_t ko = frag_k<HD>(g, k0 + key_row(col), 8 * hf, tp);  // s = 0; each further one 512 on
#pragma unroll
    for (int s = 0; s < SplitTile<HD>::KS; s++) {
        T.kh[s] = *(const f16x8 *)(kh + ko + 512 * s);
        T.kl[s] = *(const f16x8 *)(kl + ko + 512 * s);
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        T.ek[u] = *(const uint64_t *)(ek + (size_t)g * tp + k0 + 16 * u + 8 * hf);
        T.ev[u] = *(const uint64_t *)(ev + (size_t)g * tp + k0 + 16 * u + 8 * hf);
    }
}

__device__ __forceinline__ int exp_byte(uint64_t w, int i) { return (int)(int8_t)(uint8_t)(w >> (8 * i)); }

// Causal grouped-query attention on the split operands; the work split, the online softmax and
// the merge are attention_kernel's. Per key tile: S'^T = k' q'^T (three f16 MFMAs per 16 dims),
// S = S' 2^(e_q + e_k) scale log2(e), masked, online softmax in base 2 -> p;
// p' = p 2^(14 + e_v - sigma) (sigma the
// tile's largest v exponent, so p' <= 2^14) split into two f16 parts; the tile's O'^T = v'^T p'^T
// (three f16 MFMAs per 16 keys per 32 dims) enters the f32 accumulator scaled by 2^(sigma - 14).
// XKIND 0: the output goes to att as f32 [t][heads HD]; FH_Q8_0 / FH_Q4_0: it goes to xo as the
// fast GEMM's split x for a weight of that kind (xsplit.hpp, t rows of heads HD), the same values
// split_x_kernel would make of the f32 rows.
template <int HD, int W, int XKIND = 0>
__global__ __launch_bounds__(64 * W) void attention_split_kernel(
    const _Float16 *__restrict__ qh, const _Float16 *__restrict__ ql, const _Float16 *__restrict__ kh,
    const _Float16 *__restrict__ kl, const _Float16 *__restrict__ vh, const _Float16 *__restrict__ vl,
    const int8_t *__restrict__ eq, const int8_t *__restrict__ ek, const int8_t *__restrict__ ev,
    float *__restrict__ att, uint32_t t, uint32_t tp, uint32_t heads, uint32_t group, float scale,
    GemmXSplit xo = GemmXSplit{}) {
    using T = SplitTile<HD>;
    constexpr int DB = T::DB, KS = T::KS;
    __shared__ float red[W][2 + 16 * DB][64];
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6, col = lane & 31u, hf = lane >> 5;
    // grid (heads, query blocks): workgroups are dispatched x fastest, so every head's longest
    // query blocks start first and the short ones fill in at the end
    const uint32_t q0 = (gridDim.y - 1 - blockIdx.y) * 32;
    const uint32_t h = blockIdx.x, g = h / group;
    const uint32_t qd = heads * HD;
    const uint32_t query = q0 + col;
    f16x8 qfh[KS], qfl[KS];
    {
        const size_t qo = (size_t)query * qd + h * HD + 8 * hf;  // query < tp: rows past t are zero
#pragma unroll
        for (int s = 0; s < KS; s++) {
            qfh[s] = *(const f16x8 *)(qh + qo + 16 * s);
            qfl[s] = *(const f16x8 *)(ql + qo + 16 * s);
        }
    }
    const int e_q = (int)eq[(size_t)h * tp + query];
    f32x16 o[DB];
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[b][i] = 0.0f;
    // scores in the base-2 domain (scale log2(e) folded in), so each exponential is one v_exp_f32
    const float sl2 = scale * 1.44269504088896341f;
    float mrun = -INFINITY, lrun = 0.0f;
    const uint32_t tiles = (min(q0 + 31u, t - 1u)) / 32 + 1;  // key tiles any valid query of the block sees
    T cur, nxt;
    if (w < tiles) split_load<HD>(cur, kh, kl, ek, ev, 32 * w, tp, g, col, hf);
    for (uint32_t kt = w; kt < tiles; kt += W) {
        const uint32_t k0 = 32 * kt;
        SplitV<HD> vt;  // the tile's values, needed after the softmax
        split_load_v<HD>(vt, vh, vl, k0, tp, g, col, hf);
        if (kt + W < tiles) split_load<HD>(nxt, kh, kl, ek, ev, k0 + 32 * W, tp, g, col, hf);
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; i++) s[i] = 0.0f;
#pragma unroll
        for (int st = 0; st < KS; st++) {
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.kh[st], qfh[st], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.kh[st], qfl[st], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.kl[st], qfh[st], s, 0, 0, 0);
        }
        float mt = -INFINITY;
        int sig = kSplitPad;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t key = k0 + 16 * (i / 8) + 8 * hf + i % 8;
            const float v = key <= query ? ldexpf(s[i], e_q + exp_byte(cur.ek[i / 8], i % 8)) * sl2 : -INFINITY;
            s[i] = v;
            mt = fmaxf(mt, v);
            sig = max(sig, exp_byte(cur.ev[i / 8], i % 8));
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        sig = max(sig, __shfl_xor(sig, 32));
        const float mnew = fmaxf(mrun, mt);  // finite: key k0 <= query in every tile
        const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
        float ls = 0.0f;
        f16x8 ph[2], pl[2];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float p = __builtin_amdgcn_exp2f(s[i] - mnew);
            ls += p;
            const float x = ldexpf(p, 14 + exp_byte(cur.ev[i / 8], i % 8) - sig);
            const _Float16 hi = (_Float16)x;
            ph[i / 8][i % 8] = hi;
            pl[i / 8][i % 8] = (_Float16)(x - (float)hi);
        }
        lrun = lrun * alpha + ls;
        mrun = mnew;
        const float back = ldexpf(1.0f, sig - 14);
#pragma unroll
        for (int b = 0; b < DB; b++) {
            f32x16 tb;
#pragma unroll
            for (int i = 0; i < 16; i++) tb[i] = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                tb = __builtin_amdgcn_mfma_f32_32x32x16_f16(vt.vh[b][u], ph[u], tb, 0, 0, 0);
                tb = __builtin_amdgcn_mfma_f32_32x32x16_f16(vt.vh[b][u], pl[u], tb, 0, 0, 0);
                tb = __builtin_amdgcn_mfma_f32_32x32x16_f16(vt.vl[b][u], ph[u], tb, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 16; i++) o[b][i] = fmaf(tb[i], back, o[b][i] * alpha);
        }
        cur = nxt;
    }
    // merge the wavefronts' partial softmaxes: M = max m_w, O = sum O_w e^(m_w - M), l likewise
    red[w][0][lane] = mrun;
    red[w][1][lane] = lrun;
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) red[w][2 + 16 * b + i][lane] = o[b][i];
    __syncthreads();
    if (w) return;
    float M = red[0][0][lane];
#pragma unroll
    for (int j = 1; j < W; j++) M = fmaxf(M, red[j][0][lane]);
    float f[W], l = 0.0f;
#pragma unroll
    for (int j = 0; j < W; j++) {
        f[j] = __builtin_amdgcn_exp2f(red[j][0][lane] - M);  // a wavefront without tiles: 2^(-inf) = 0
        l += red[j][1][lane] * f[j];
    }
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    if (query >= t) return;  // (the same for lanes l and l ^ 32)
    if constexpr (XKIND != 0) {
        // per 32-dim block b: lane (query, hf) holds its dims 8 k + 4 hf + 0..3, i.e. element groups
        // G = 2 k + hf of four; the block's largest |x| with the partner lane, then the split
        typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
        typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
        const uint32_t nb = qd / 32, K64 = (qd + 63) / 64 * 64, MS = xsb_rows(t);
#pragma unroll
        for (int b = 0; b < DB; b++) {
            float v[16], mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < W; j++) acc += red[j][2 + 16 * b + i][lane] * f[j];
                v[i] = acc * inv;
                mx = fmaxf(mx, fabsf(v[i]));
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const int sc = lo_shift(mx);
            const float sf = __uint_as_float((uint32_t)(127 + sc) << 23);
            const uint32_t blk = h * HD / 32 + b;
            if (hf == 0) xo.xsb[xsb_at(query, blk, MS)] = (uint8_t)(127 - sc);
            _Float16 hv[16];
#pragma unroll
            for (int i = 0; i < 16; i++) hv[i] = f16_sat(v[i]);
            uint8_t *lo = xo.xl + (size_t)query * K64;
#pragma unroll
            for (int k = 0; k < 4; k++)
                *(uint32_t *)(lo + lo_byte(blk, 4 * (2 * k + hf))) =
                    fp8x4((v[4 * k] - (float)hv[4 * k]) * sf, (v[4 * k + 1] - (float)hv[4 * k + 1]) * sf,
                          (v[4 * k + 2] - (float)hv[4 * k + 2]) * sf, (v[4 * k + 3] - (float)hv[4 * k + 3]) * sf);
            _Float16 *hb = xo.xh + ((size_t)query * nb + blk) * 32;
            if constexpr (XKIND == FH_Q8_0) {
                // positions 4 G .. 4 G + 3 hold group G's elements {0, 2, 1, 3}
#pragma unroll
                for (int k = 0; k < 4; k++)
                    *(h16x4 *)(hb + 4 * (2 * k + hf)) = h16x4{hv[4 * k], hv[4 * k + 2], hv[4 * k + 1], hv[4 * k + 3]};
            } else {
                // positions 8 I .. 8 I + 7 hold groups I and I + 4 (both this lane's for I = 2 k + hf)
#pragma unroll
                for (int k = 0; k < 2; k++)
                    *(h16x8 *)(hb + 8 * (2 * k + hf)) =
                        h16x8{hv[4 * k], hv[4 * k + 2], hv[4 * k + 1], hv[4 * k + 3], hv[4 * k + 8], hv[4 * k + 10],
                              hv[4 * k + 9], hv[4 * k + 11]};
            }
            if (nb % 2 && blk == nb - 1) split_tail(query, nb, K64, MS, xo.xl, xo.xsb, hf);
        }
        return;
    }
    float *out = att + (size_t)query * qd + h * HD;
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t dim = 32 * b + 8 * (i / 4) + 4 * hf + (i % 4);
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < W; j++) acc += red[j][2 + 16 * b + i][lane] * f[j];
            out[dim] = acc * inv;
        }
}

// SwiGLU (ferrum_ref/src/models/llama/ops.rs:69-76): act[r][j] = silu(gu[r][j]) * gu[r][hid + j].
// Widths that are not a multiple of 4 take swiglu_scalar_kernel.
__global__ __launch_bounds__(256) void swiglu_scalar_kernel(const float *__restrict__ gu, uint32_t gu_splits,
                                                            size_t gu_stride, float *__restrict__ act, uint32_t rows,
                                                            uint32_t hid) {
    const size_t n = (size_t)rows * hid;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t r = i / hid, j = i % hid;
        const float g = split_sum(gu, r * 2 * hid + j, gu_splits, gu_stride);
        const float u = split_sum(gu, r * 2 * hid + hid + j, gu_splits, gu_stride);
        act[i] = swiglu_act(g, u);
    }
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float *__restrict__ gu, uint32_t gu_splits, size_t gu_stride,
                                                     float *__restrict__ act, uint32_t rows, uint32_t hid) {
    const uint32_t q = hid / 4;
    const size_t n = (size_t)rows * q;
    auto load4 = [&](size_t o) {  // four consecutive elements of the (possibly K-split) product
        f32x4 v = *(const f32x4 *)(gu + o);
        for (uint32_t sl = 1; sl < gu_splits; sl++) v += *(const f32x4 *)(gu + sl * gu_stride + o);
        return v;
    };
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t r = i / q, j = i % q;
        const f32x4 g = load4(r * 2 * hid + 4 * j);
        const f32x4 u = load4(r * 2 * hid + hid + 4 * j);
        f32x4 y;
#pragma unroll
        for (int c = 0; c < 4; c++) y[c] = swiglu_act(g[c], u[c]);
        *(f32x4 *)(act + r * hid + 4 * j) = y;
    }
}

// Per row (nn::score, ferrum_ref/src/kernels/nn.rs:117-129): out[2r] = logits[r][t] - max -
// ln(sum exp(logits[r] - max)), out[2r + 1] = 1 when t is the first maximum, else 0; t =
// targets[r]. One pass with a running maximum per thread (rescaled when a larger value
// arrives), four logits per load when rows are 16-byte aligned; a target outside the vocabulary
// gives NaN.
__device__ __forceinline__ void score_take(float v, uint32_t j, float &m, float &s, uint32_t &first) {
    if (v > m) {
        s = m == -INFINITY ? 0.0f : s * __expf(m - v);
        m = v;
        first = j;
    }
    s += __expf(v - m);
}

__global__ __launch_bounds__(256) void score_kernel(const float *__restrict__ logits, const int32_t *__restrict__ targets,
                                                    float *__restrict__ out, uint32_t vocab) {
    __shared__ float sm[4], ss[4];
    __shared__ uint32_t sf[4];
    const float *x = logits + (size_t)blockIdx.x * vocab;
    float m = -INFINITY, s = 0.0f;
    uint32_t first = 0xffffffffu;
    if ((vocab & 3u) == 0) {
        const f32x4 *x4 = (const f32x4 *)x;
        const uint32_t n4 = vocab / 4;
        auto take4 = [&](f32x4 v, uint32_t j) {
            const float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
            if (mx > m) {
                s = m == -INFINITY ? 0.0f : s * __expf(m - mx);
                m = mx;
                first = 4 * j + (v[0] == mx ? 0u : v[1] == mx ? 1u : v[2] == mx ? 2u : 3u);
            }
            s += (__expf(v[0] - m) + __expf(v[1] - m)) + (__expf(v[2] - m) + __expf(v[3] - m));
        };
        // four float4 loads in flight per thread, taken in the same order as one at a time
        uint32_t j = threadIdx.x;
        for (; j + 3 * 256 < n4; j += 4 * 256) {
            f32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = x4[j + 256 * u];
#pragma unroll
            for (int u = 0; u < 4; u++) take4(v[u], j + 256 * u);
        }
        for (; j < n4; j += 256) take4(x4[j], j);
    } else {
        for (uint32_t j = threadIdx.x; j < vocab; j += 256) score_take(x[j], j, m, s, first);
    }
    for (int o = 32; o; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
        const uint32_t f2 = __shfl_xor(first, o);
        const float mx = fmaxf(m, m2);
        s = (m == -INFINITY ? 0.0f : s * __expf(m - mx)) + (m2 == -INFINITY ? 0.0f : s2 * __expf(m2 - mx));
        first = m2 > m || (m2 == m && f2 < first) ? f2 : first;
        m = mx;
    }
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sm[w] = m;
        ss[w] = s;
        sf[w] = first;
    }
    __syncthreads();
    if (threadIdx.x) return;
    float M = sm[0], S = ss[0];
    uint32_t F = sf[0];
    for (int i = 1; i < 4; i++) {
        const float mx = fmaxf(M, sm[i]);
        S = (M == -INFINITY ? 0.0f : S * __expf(M - mx)) + (sm[i] == -INFINITY ? 0.0f : ss[i] * __expf(sm[i] - mx));
        F = sm[i] > M || (sm[i] == M && sf[i] < F) ? sf[i] : F;
        M = mx;
    }
    const int32_t t = targets[blockIdx.x];
    const bool ok = t >= 0 && (uint32_t)t < vocab;
    out[2 * (size_t)blockIdx.x] = ok ? x[t] - M - logf(S) : NAN;
    out[2 * (size_t)blockIdx.x + 1] = ok && F == (uint32_t)t ? 1.0f : 0.0f;
}

// score_kernel's result from the head GEMM's per-tile statistics (ScoreOut: for every row and
// 256-column tile the maximum, the sum of exp(v - maximum) and the first column holding the
// maximum, and the target's logit): one wavefront per row merges the row's tiles (lane l tiles l,
// l + 64, ... in order, then the lanes pairwise; the smaller column wins a tie, as a left-to-right
// scan would have it), out[2r] = logit[t] - max - ln(sum), out[2r + 1] = (first == t); a target
// outside the vocabulary gives NaN.
__device__ __forceinline__ void score_combine(float &m, float &s, uint32_t &f, float m2, float s2, uint32_t f2) {
    const float mx = fmaxf(m, m2);
    s = (m == -INFINITY ? 0.0f : s * __expf(m - mx)) + (m2 == -INFINITY ? 0.0f : s2 * __expf(m2 - mx));
    f = m2 > m || (m2 == m && f2 < f) ? f2 : f;
    m = mx;
}

__global__ __launch_bounds__(256) void score_merge_kernel(const float *__restrict__ part, const float *__restrict__ tlogit,
                                                          const int32_t *__restrict__ targets, float *__restrict__ out,
                                                          uint32_t rows, uint32_t ntn, uint32_t vocab) {
    const uint32_t row = blockIdx.x * 4 + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= rows) return;  // (whole wavefronts)
    float m = -INFINITY, s = 0.0f;
    uint32_t f = 0xffffffffu;
    for (uint32_t c = lane; c < ntn; c += 64) {
        const f32x4 p = *(const f32x4 *)(part + ((size_t)row * ntn + c) * 4);
        score_combine(m, s, f, p.x, p.y, __float_as_uint(p.z));
    }
    for (int o = 32; o; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
        const uint32_t f2 = (uint32_t)__shfl_xor((int)f, o);
        score_combine(m, s, f, m2, s2, f2);
    }
    if (lane) return;
    const int32_t t = targets[row];
    const bool ok = t >= 0 && (uint32_t)t < vocab;
    out[2 * (size_t)row] = ok ? tlogit[row] - m - logf(s) : NAN;
    out[2 * (size_t)row + 1] = ok && f == (uint32_t)t ? 1.0f : 0.0f;
}

// The score epilogue's targets: rows 0..rows-1 from ids, then -1 up to `padded` (a multiple of 256).
__global__ __launch_bounds__(256) void pad_targets_kernel(const int32_t *__restrict__ ids, int32_t *__restrict__ tgt,
                                                          uint32_t rows, uint32_t padded) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < padded) tgt[i] = i < rows ? ids[i] : -1;
}

// ---- host side ----

fh_status llama_fail_free(fh_llama *m, fh_status st) {
    fh_llama_free(m);
    return st;
}

const float *fp(const fh_buffer *b) { return b ? (const float *)b->ptr : nullptr; }

// RoPE scaling as the reference reads it (ferrum_model/src/gguf/llama/mod.rs:56-100): linear
// (`rope.scaling.factor`, else `rope.scale_linear`), "none" only with factor 1, yarn and the rest
// refused, attn_factor must be 1, per-frequency divisors from `rope_freqs.weight`.
fh_status rope_scaling(const fh_gguf *g, const std::string &arch, size_t rope_dim, float *linear,
                       std::vector<float> *freq) {
    auto key = [&](const char *k) { return arch + ".rope." + k; };
    auto opt_float = [&](const std::string &k, float *v, bool *has) -> fh_status {
        size_t idx;
        *has = fh_gguf_find_key(g, k.c_str(), &idx) == FH_OK;
        return *has ? fh_gguf_get_float(g, k.c_str(), v) : FH_OK;
    };
    float factor = 0.0f;
    bool has = false;
    fh_status st = opt_float(key("scaling.factor"), &factor, &has);
    if (st) return st;
    if (!has && (st = opt_float(key("scale_linear"), &factor, &has))) return st;
    if (!has || factor == 0.0f) factor = 1.0f;
    std::string ty = "linear";
    size_t idx;
    if (fh_gguf_find_key(g, key("scaling.type").c_str(), &idx) == FH_OK) {
        const char *s;
        size_t n;
        if ((st = fh_gguf_get_string(g, key("scaling.type").c_str(), &s, &n))) return st;
        ty.assign(s, n);
    }
    if (ty == "none") {
        if (factor != 1.0f)
            return fail(FH_ERR_INVALID, "rope scaling type is \"none\" but the factor is %g", (double)factor);
    } else if (ty != "linear") {
        return fail(FH_ERR_INVALID, "rope scaling type '%s' is not supported (none, linear and rope_freqs.weight are)",
                    ty.c_str());
    }
    *linear = ty == "linear" ? factor : 1.0f;
    float attn = 1.0f;
    if ((st = opt_float(key("scaling.attn_factor"), &attn, &has))) return st;
    if (has && attn != 1.0f) return fail(FH_ERR_INVALID, "rope scaling attn_factor %g is not supported", (double)attn);
    freq->clear();
    if (fh_gguf_find_tensor(g, "rope_freqs.weight", &idx) == FH_OK) {
        fh_gguf_tensor t;
        if ((st = fh_gguf_tensor_info(g, idx, &t))) return st;
        if (t.n_dims != 1 || t.dims[0] != rope_dim / 2)
            return fail(FH_ERR_INVALID, "tensor 'rope_freqs.weight' has the wrong dims, expected [%zu] from the metadata",
                        rope_dim / 2);
        if ((st = host_vec(g, "llama", "rope_freqs.weight", rope_dim / 2, freq))) return st;
    }
    // RopeScaling::check (ferrum_ref/src/models/llama/ops.rs:38-52)
    auto ok = [](float v) { return std::isfinite(v) && v > 0.0f; };
    bool good = ok(*linear);
    for (float v : *freq) good = good && ok(v);
    if (!good) return fail(FH_ERR_INVALID, "RoPE scaling factors must be finite and > 0");
    return FH_OK;
}

// rope_tables (ferrum_ref/src/models/llama/ops.rs:78-101) for positions 0 .. ctx - 1, built on
// the host with the same f64 power and f32 sin/cos, so device and CPU share the exact angles.
void rope_tables(size_t ctx, size_t rope_dim, float base, const std::vector<float> &ff, float linear,
                 std::vector<float> *c, std::vector<float> *s) {
    const size_t half = rope_dim / 2;
    c->resize(ctx * half);
    s->resize(ctx * half);
    for (size_t p = 0; p < ctx; p++)
        for (size_t i = 0; i < half; i++) {
            const float freq = (float)std::pow((double)base, -2.0 * (double)i / (double)rope_dim);
            const float f = ff.empty() ? 1.0f : ff[i];
            const float theta = (float)p * freq / f * (1.0f / linear);
            (*s)[p * half + i] = ::sinf(theta);
            (*c)[p * half + i] = ::cosf(theta);
        }
}

size_t up256(size_t b) { return (b + 255) / 256 * 256; }

// Rows of logits per head product: as many as keep the logits under 2^31 bytes.
size_t logit_chunk(const fh_llama *m, size_t t) {
    const size_t lim = (((size_t)1 << 31) - 1) / (m->vocab * 4);
    return std::max<size_t>(1, std::min(t, lim));
}

// Workspace of the precise and dequant-f16 paths (split x, then their partial products).
size_t linear_ws(const fh_llama *m, size_t rows, size_t k, size_t n) {
    return m->path == FH_PATH_TILED_F16 ? gemm_f16_workspace_bytes(rows, k, n)
                                        : gemm_precise_workspace_bytes(rows, k, n);
}

// The score epilogue's buffers for `rows` rows (enqueue_score): the per-tile statistics (four floats
// per row and 256-column tile), the target logits, the targets padded to a multiple of 256 rows.
size_t score_fold_bytes(size_t rows, size_t vocab) {
    return up256(rows * ((vocab + 255) / 256) * 16) + up256(rows * 4) + up256((rows + 255) / 256 * 256 * 4);
}

// The activations for t rows (kept when already large enough).
// Head dims whose attention runs on the split f16 operands (the f32-MFMA kernel takes the rest).
bool split_attention(const fh_llama *m) { return m->head_dim == 32 || m->head_dim == 64 || m->head_dim == 128; }

fh_status ensure_rows(fh_llama *m, size_t t) {
    if (t <= m->rows) return FH_OK;
    const size_t d = m->dim, qd = m->q_dim(), w = m->qkv_width(), hid = m->hidden, chunk = logit_chunk(m, t);
    size_t ws = 0, part = 0;
    const bool fast = m->path == FH_PATH_TILED_FAST;
    const std::pair<size_t, size_t> prods[] = {{t, d}, {t, qd}, {t, hid}, {chunk, d}};
    const std::pair<size_t, size_t> kns[] = {{d, w}, {qd, d}, {d, 2 * hid}, {hid, d}};
    if (fast) {
        for (auto rk : prods) ws = std::max(ws, gemm_xsplit_bytes(rk.first, rk.second));
        for (auto kn : kns) part = std::max(part, gemm_partial_bytes(t, kn.first, kn.second));
        part = std::max(part, gemm_partial_bytes(chunk, d, m->vocab));
    } else {
        for (auto kn : kns) ws = std::max(ws, linear_ws(m, t, kn.first, kn.second));
        ws = std::max(ws, linear_ws(m, chunk, d, m->vocab));
    }
    const size_t tp = (t + 31) / 32 * 32, kvd = m->kv_dim();
    const size_t split = split_attention(m) ? 2 * up256(tp * qd * 2) + 4 * up256(tp * kvd * 2) + up256(tp * m->heads) +
                                                  2 * up256(tp * m->kv_heads)
                                            : 0;
    const size_t sfold = score_fold_bytes(chunk, m->vocab);
    // act: the f32 activation, or on the fast path the down product's split x (the SwiGLU epilogue)
    const size_t act = std::max(t * hid * 4, fast ? gemm_xsplit_bytes(t, hid) : (size_t)0);
    // att: the f32 attention output, or on the fast path the output product's split x
    const size_t att = std::max(t * qd * 4, fast ? gemm_xsplit_bytes(t, qd) : (size_t)0);
    const size_t total = 3 * up256(t * d * 4) + up256(t * w * 4) + up256(att) + up256(t * 2 * hid * 4) +
                         up256(act) + up256(chunk * m->vocab * 4) + up256(2 * t * 4) + up256((t + 1) * 4) +
                         up256(ws) + up256(part) + split + up256(sfold);
    void *p = nullptr;
    fh_status st = alloc_bytes(m->dev, total, &p);
    if (st) return st;
    if (m->arena) {
        (void)hipStreamSynchronize(m->dev->stream);
        (void)hipFree(m->arena);
    }
    m->arena = p;
    m->arena_bytes = total;
    m->rows = t;
    m->chunk = chunk;
    uint8_t *q = (uint8_t *)p;
    auto take = [&](size_t bytes) {
        void *r = q;
        q += up256(bytes);
        return r;
    };
    m->x = (float *)take(t * d * 4);
    m->h = (float *)take(t * d * 4);
    m->o = (float *)take(t * d * 4);
    m->qkv = (float *)take(t * w * 4);
    m->att = (float *)take(att);
    m->gu = (float *)take(t * 2 * hid * 4);
    m->act = (float *)take(act);
    m->logits = (float *)take(chunk * m->vocab * 4);
    m->scores = (float *)take(2 * t * 4);
    m->ids = (int32_t *)take((t + 1) * 4);
    m->ws = take(ws);
    m->part = part ? (float *)take(part) : nullptr;
    m->sfold = (float *)take(sfold);
    if (split) {
        m->sqh = (_Float16 *)take(tp * qd * 2);
        m->sql = (_Float16 *)take(tp * qd * 2);
        m->skh = (_Float16 *)take(tp * kvd * 2);
        m->skl = (_Float16 *)take(tp * kvd * 2);
        m->svh = (_Float16 *)take(tp * kvd * 2);
        m->svl = (_Float16 *)take(tp * kvd * 2);
        m->seq = (int8_t *)take(tp * m->heads);
        m->sek = (int8_t *)take(tp * m->kv_heads);
        m->sev = (int8_t *)take(tp * m->kv_heads);
    }
    return FH_OK;
}

bool linear_supported(const fh_llama *m, size_t rows, const fh_llama::Mat &w) {
    const size_t k = w.k, n = w.n;
    if (!w.q) return rows <= 65535 * 64;  // the f32 product's grid rows
    switch (m->path) {
    case FH_PATH_TILED_FAST: return gemm_supported(rows, k, n);
    case FH_PATH_TILED_F16: return gemm_f16_supported(rows, k, n);
    default: return true;
    }
}

fh_status check_shapes(const fh_llama *m, size_t t) {
    for (const auto &L : m->blocks)
        for (const fh_llama::Mat *w : {&L.wqkv, &L.wo, &L.wgu, &L.down})
            if (!linear_supported(m, t, *w))
                return fail(FH_ERR_UNSUPPORTED, "llama: %zu rows exceed the GEMM's 32-bit offsets for a %zu x %zu weight",
                            t, w->n, w->k);
    if (!linear_supported(m, logit_chunk(m, t), m->head))
        return fail(FH_ERR_UNSUPPORTED, "llama: the head exceeds the GEMM's 32-bit offsets");
    return FH_OK;
}

// With defer, a K-split product is left as partial sums in the workspace for the next kernel to
// add up (every consumer runs before the next product overwrites the workspace).
hipError_t linear(const fh_llama *m, hipStream_t s, const fh_llama::Mat &mat, const float *x, float *y, size_t rows,
                  SplitOut *defer = nullptr, const GemmXSplit *xs = nullptr) {
    if (!mat.q) {  // f32 rows: x is always given (the fused producers run only when every matrix is packed)
        const dim3 grid((unsigned)((mat.n + 63) / 64), (unsigned)((rows + 63) / 64));
        linear_f32_kernel<<<grid, 256, 0, s>>>(x, (const float *)mat.f->ptr, y, (uint32_t)rows, (uint32_t)mat.k,
                                               (uint32_t)mat.n);
        return hipGetLastError();
    }
    const fh_qweight *w = mat.q;
    switch (m->path) {
    case FH_PATH_TILED_FAST:
        return launch_gemm(s, w->kind, w->qs, w->ds, w->b8, x, y, rows, w->k, w->n, m->ws, defer, m->part, xs);
    case FH_PATH_TILED_F16: return launch_gemm_f16(s, w->kind, w->qs, w->ds, x, y, rows, w->k, w->n, m->ws, defer);
    default: return launch_gemm_precise(s, w->kind, w->qs, w->ds, x, y, rows, w->k, w->n, m->ws, defer);
    }
}

// RoPE (with the q/k/v bias and the QKV product's K-split partial sums) and the attention of t
// rows. The split attention's head dims take qkv_rope_split_kernel (the f32 q, k, v are then
// never written), or, when the model was loaded with FERRUM_HIP_ROPE_UNFUSED=1, qkv_rope_kernel
// and attn_split_kernel, with the same results; the other head dims qkv_rope_kernel and the f32
// attention_kernel.
// xo: where the split attention writes its output as the output product's split x (m->kind's
// operand order) instead of f32 rows in m->att; only when split_attention(m).
hipError_t launch_attention(const fh_llama *m, hipStream_t s, size_t t, const SplitOut &qkv, const float *bias,
                            const GemmXSplit *xo = nullptr) {
    const dim3 grid((unsigned)m->heads, (unsigned)((t + 31) / 32));
    const uint32_t w = (uint32_t)m->qkv_width(), group = (uint32_t)(m->heads / m->kv_heads);
    const float scale = 1.0f / sqrtf((float)m->head_dim);
    const uint32_t T = (uint32_t)t, H = (uint32_t)m->heads, KV = (uint32_t)m->kv_heads;
    const uint32_t hd = (uint32_t)m->head_dim, rd = (uint32_t)m->rope_dim;
    const int neox = m->neox ? 1 : 0;
    const float *cos_t = fp(m->rope_cos), *sin_t = fp(m->rope_sin);
    const bool fused = m->fuse_rope && split_attention(m);
    if (!fused)
        qkv_rope_kernel<<<T, 256, w * 4, s>>>(qkv.part, qkv.splits, t * w, m->qkv, bias, cos_t, sin_t, w,
                                              H + KV, hd, rd, neox);
    if (split_attention(m)) {
        const uint32_t tp = (T + 31) / 32 * 32;
        const SplitDst o{m->sqh, m->sql, m->skh, m->skl, m->svh, m->svl, m->seq, m->sek, m->sev};
        // 16-row tiles while 32-row ones would give fewer than two workgroups per CU
        const bool small = (size_t)(tp / 32) * (H + 2 * KV) < 512;
#define FH_SPLIT_ATTN(HD, W)                                                                                      \
    if (fused && small)                                                                                           \
        qkv_rope_split_kernel<HD, 16><<<dim3(tp / 16, H + 2 * KV), 256, 0, s>>>(qkv.part, qkv.splits, t * w,     \
                                                                                bias, cos_t, sin_t, o, T, tp, w,  \
                                                                                H, KV, rd, neox);                 \
    else if (fused)                                                                                               \
        qkv_rope_split_kernel<HD, 32><<<dim3(tp / 32, H + 2 * KV), 256, 0, s>>>(qkv.part, qkv.splits, t * w,     \
                                                                                bias, cos_t, sin_t, o, T, tp, w,  \
                                                                                H, KV, rd, neox);                 \
    else                                                                                                          \
        attn_split_kernel<HD><<<tp, 256, 0, s>>>(m->qkv, o, T, tp, w, H, KV);                                     \
    if (xo && m->kind == FH_Q8_0)                                                                                 \
        attention_split_kernel<HD, W, FH_Q8_0><<<grid, 64 * W, 0, s>>>(                                           \
            m->sqh, m->sql, m->skh, m->skl, m->svh, m->svl, m->seq, m->sek, m->sev, m->att, T, tp, H, group, scale, \
            *xo);                                                                                                 \
    else if (xo)                                                                                                  \
        attention_split_kernel<HD, W, FH_Q4_0><<<grid, 64 * W, 0, s>>>(                                           \
            m->sqh, m->sql, m->skh, m->skl, m->svh, m->svl, m->seq, m->sek, m->sev, m->att, T, tp, H, group, scale, \
            *xo);                                                                                                 \
    else                                                                                                          \
        attention_split_kernel<HD, W><<<grid, 64 * W, 0, s>>>(m->sqh, m->sql, m->skh, m->skl, m->svh, m->svl,     \
                                                              m->seq, m->sek, m->sev, m->att, T, tp, H, group,    \
                                                              scale)
        switch (m->head_dim) {
        case 32: FH_SPLIT_ATTN(32, 4); break;
        case 64: FH_SPLIT_ATTN(64, 4); break;
        default: FH_SPLIT_ATTN(128, 2); break;
        }
#undef FH_SPLIT_ATTN
        return hipGetLastError();
    }
    switch (m->head_dim) {
    case 8: attention_kernel<8, 4><<<grid, 256, 0, s>>>(m->qkv, m->att, T, w, H, group, scale); break;
    case 16: attention_kernel<16, 4><<<grid, 256, 0, s>>>(m->qkv, m->att, T, w, H, group, scale); break;
    case 32: attention_kernel<32, 4><<<grid, 256, 0, s>>>(m->qkv, m->att, T, w, H, group, scale); break;
    case 64: attention_kernel<64, 4><<<grid, 256, 0, s>>>(m->qkv, m->att, T, w, H, group, scale); break;
    default: attention_kernel<128, 2><<<grid, 128, 0, s>>>(m->qkv, m->att, T, w, H, group, scale); break;
    }
    return hipGetLastError();
}

// The forward over the t ids already in m->ids, up to the final norm's output in m->h.
hipError_t enqueue_body(fh_llama *m, hipStream_t s, size_t t) {
    const uint32_t d = (uint32_t)m->dim, T = (uint32_t)t;
    const fh_qweight *tq = m->tok.q;
    if (!tq)
        embed_rows_f32_kernel<<<T, 256, 0, s>>>((const float *)m->tok.f->ptr, m->ids, m->x, d, (uint32_t)m->vocab);
    else if (tq->kind == FH_Q8_0)
        embed_rows_kernel<FH_Q8_0><<<T, 256, 0, s>>>(tq->qs, tq->ds, m->ids, m->x, d, (uint32_t)m->vocab);
    else
        embed_rows_kernel<FH_Q4_0><<<T, 256, 0, s>>>(tq->qs, tq->ds, m->ids, m->x, d, (uint32_t)m->vocab);
    hipError_t e = hipGetLastError();
    const size_t td = t * m->dim;
    // The fast path's RMSNorms and SwiGLU write the next product's split x themselves (the
    // product then skips its split pass); rows up to 16384 wide, held in LDS.
    const bool fused = m->path == FH_PATH_TILED_FAST && m->packed && m->dim <= 16384 && m->hidden <= 16384;
    const GemmXSplit xd = gemm_x_split(m->ws, t, m->dim), xh = gemm_x_split(m->ws, t, m->hidden);
    // the attention's output as the output product's split x, in att
    const bool att_split = fused && m->att_split && split_attention(m);
    const GemmXSplit xatt = gemm_x_split(m->att, t, m->q_dim());
    auto norm = [&](bool add, const fh_buffer *g, const SplitOut &o) {
        if (fused && m->kind == FH_Q8_0) {
            if (add)
                rmsnorm_split_kernel<true, FH_Q8_0><<<T, 256, d * 4, s>>>(m->x, o.part, fp(g), d, m->eps, o.splits, td, xd);
            else
                rmsnorm_split_kernel<false, FH_Q8_0><<<T, 256, d * 4, s>>>(m->x, nullptr, fp(g), d, m->eps, 1, 0, xd);
        } else if (fused) {
            if (add)
                rmsnorm_split_kernel<true, FH_Q4_0><<<T, 256, d * 4, s>>>(m->x, o.part, fp(g), d, m->eps, o.splits, td, xd);
            else
                rmsnorm_split_kernel<false, FH_Q4_0><<<T, 256, d * 4, s>>>(m->x, nullptr, fp(g), d, m->eps, 1, 0, xd);
        } else if (add) {
            rmsnorm_kernel<true><<<T, 256, 0, s>>>(m->x, o.part, fp(g), m->h, d, m->eps, o.splits, td);
        } else {
            rmsnorm_kernel<false><<<T, 256, 0, s>>>(m->x, nullptr, fp(g), m->h, d, m->eps, 1, 0);
        }
    };
    const float *hx = fused ? nullptr : m->h;  // the input the next products read
    SplitOut down{m->o, 1};  // the previous block's FFN output, added to x by the next RMSNorm
    for (size_t l = 0; l < m->layers && !e; l++) {
        const auto &L = m->blocks[l];
        norm(l > 0, L.attn_norm, down);
        SplitOut qkv{m->qkv, 1}, att{m->o, 1}, gu{m->gu, 1};
        if ((e = linear(m, s, L.wqkv, hx, m->qkv, t, &qkv))) break;
        if ((e = launch_attention(m, s, t, qkv, fp(L.bqkv), att_split ? &xatt : nullptr))) break;
        if ((e = linear(m, s, L.wo, att_split ? nullptr : m->att, m->o, t, &att, att_split ? &xatt : nullptr))) break;
        norm(true, L.ffn_norm, att);
        if (fused && m->gu_inter && gemm_swiglu_supported(t, d, 2 * m->hidden)) {
            // SwiGLU in the gate/up product's epilogue (interleaved weight), which writes the
            // activation as the down product's split x, in act (the gate/up product still reads its
            // own split x from the workspace)
            const fh_qweight *w = L.wgu.q;
            const GemmXSplit xa = gemm_x_split(m->act, t, m->hidden);
            if ((e = launch_gemm_swiglu(s, w->kind, w->qs, w->ds, w->b8, nullptr, xa, t, w->k, w->n, m->ws))) break;
            if ((e = linear(m, s, L.down, nullptr, m->o, t, &down, &xa))) break;
        } else if (fused) {
            // (gate/up reduced in place: SwiGLU's split x would overwrite its partial sums)
            if ((e = linear(m, s, L.wgu, nullptr, m->gu, t))) break;
            if (m->gu_inter) {
                if (m->kind == FH_Q8_0)
                    swiglu_split_kernel<FH_Q8_0, true><<<T, 256, m->hidden * 4, s>>>(m->gu, (uint32_t)m->hidden, xh);
                else
                    swiglu_split_kernel<FH_Q4_0, true><<<T, 256, m->hidden * 4, s>>>(m->gu, (uint32_t)m->hidden, xh);
            } else if (m->kind == FH_Q8_0) {
                swiglu_split_kernel<FH_Q8_0><<<T, 256, m->hidden * 4, s>>>(m->gu, (uint32_t)m->hidden, xh);
            } else {
                swiglu_split_kernel<FH_Q4_0><<<T, 256, m->hidden * 4, s>>>(m->gu, (uint32_t)m->hidden, xh);
            }
            if ((e = linear(m, s, L.down, nullptr, m->o, t, &down))) break;
        } else {
            if ((e = linear(m, s, L.wgu, m->h, m->gu, t, &gu))) break;
            if (m->hidden % 4) {
                swiglu_scalar_kernel<<<(unsigned)std::min<size_t>((t * m->hidden + 255) / 256, 65536), 256, 0, s>>>(
                    gu.part, gu.splits, t * 2 * m->hidden, m->act, T, (uint32_t)m->hidden);
            } else {
                const size_t quads = t * m->hidden / 4;
                swiglu_kernel<<<(unsigned)std::min<size_t>((quads + 255) / 256, 65536), 256, 0, s>>>(
                    gu.part, gu.splits, t * 2 * m->hidden, m->act, T, (uint32_t)m->hidden);
            }
            if ((e = linear(m, s, L.down, m->act, m->o, t, &down))) break;
        }
        e = hipGetLastError();
    }
    if (e) return e;
    rmsnorm_kernel<true><<<T, 256, 0, s>>>(m->x, down.part, fp(m->out_norm), m->h, d, m->eps, down.splits, td);
    return hipGetLastError();
}

fh_status check_ids(const fh_llama *m, const int32_t *ids, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (ids[i] < 0 || (size_t)ids[i] >= m->vocab)
            return fail(FH_ERR_INVALID, "token %lld is out of range for vocab %zu", (long long)ids[i], m->vocab);
    return FH_OK;
}

fh_status check_len(const fh_llama *m, size_t t) {
    if (t == 0 || t > m->ctx) return fail(FH_ERR_INVALID, "sequence length %zu must be in 1..=%zu", t, m->ctx);
    return check_shapes(m, t);
}

// The score pass over t rows whose ids (t + 1 of them, the targets being ids[1..]) are in m->ids;
// out receives 2 t floats on the device.
// With the score in the head GEMM's epilogue (fuse_score), no logits are written: sfold holds the
// per-tile statistics, the target logits and the padded targets.
hipError_t enqueue_score(fh_llama *m, hipStream_t s, size_t t, float *out) {
    hipError_t e = enqueue_body(m, s, t);
    const fh_qweight *w = m->head.q;
    const size_t most = std::min(m->chunk, t), ntn = (m->vocab + 255) / 256;
    const bool fold = m->fuse_score && w && (m->path == FH_PATH_TILED_FAST || m->path == FH_PATH_TILED) &&
                      gemm_score_supported(m->path, most, w->k, w->n);
    for (size_t r0 = 0; r0 < t && !e; r0 += m->chunk) {
        const size_t rows = std::min(m->chunk, t - r0);
        if (fold) {
            const uint32_t padded = (uint32_t)((rows + 255) / 256 * 256);
            ScoreOut so;
            so.part = m->sfold;  // (laid out as score_fold_bytes)
            so.tlogit = (float *)((uint8_t *)so.part + up256(rows * ntn * 16));
            int32_t *tgt = (int32_t *)((uint8_t *)so.tlogit + up256(rows * 4));
            so.tgt = tgt;
            so.ntn = (uint32_t)ntn;
            pad_targets_kernel<<<padded / 256, 256, 0, s>>>(m->ids + 1 + r0, tgt, (uint32_t)rows, padded);
            if ((e = launch_gemm_score(s, m->path, w->kind, w->qs, w->ds, w->b8, m->h + r0 * m->dim, rows, w->k, w->n,
                                       m->ws, so)))
                break;
            score_merge_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(so.part, so.tlogit, tgt, out + 2 * r0,
                                                                         (uint32_t)rows, (uint32_t)ntn, (uint32_t)m->vocab);
        } else {
            if ((e = linear(m, s, m->head, m->h + r0 * m->dim, m->logits, rows))) break;
            score_kernel<<<(unsigned)rows, 256, 0, s>>>(m->logits, m->ids + 1 + r0, out + 2 * r0, (uint32_t)m->vocab);
        }
        e = hipGetLastError();
    }
    return e;
}

// A block matrix of k inputs, or the stacked rows of several (q/k/v, gate/up): packed when every
// part is stored Q8_0 or Q4_0 (in the model's one format), else f32 rows, each part decoded on the
// device from what the file stores and stacked in order (Lin::upload, ferrum_wgpu/src/models/
// llama/lin.rs:30-62: a width that is not whole 32-blocks stays f32; the GGUF writer stores such
// matrices as F32, ferrum_model/src/gguf/quant.rs:57-69).
fh_status load_lin(fh_device *dev, const fh_gguf *g, const std::string *names, const size_t *ns, size_t count,
                   size_t k, fh_kind *kind, fh_llama::Mat *out, bool interleave = false) {
    bool packed = true;
    size_t n = 0;
    for (size_t i = 0; i < count; i++) {
        size_t idx;
        fh_gguf_tensor t;
        fh_status st;
        if ((st = fh_gguf_find_tensor(g, names[i].c_str(), &idx)) || (st = fh_gguf_tensor_info(g, idx, &t))) return st;
        if (t.n_dims != 2 || t.dims[0] != k || t.dims[1] != ns[i])
            return fail(FH_ERR_INVALID, "llama: tensor '%s' must have dims [%zu, %zu]", names[i].c_str(), k, ns[i]);
        if (t.ggml_type != FH_Q8_0 && t.ggml_type != FH_Q4_0) packed = false;
        n += ns[i];
    }
    out->k = k;
    out->n = n;
    if (packed)
        return count == 1 ? load_mat(dev, g, "llama", names[0], k, n, kind, &out->q)
                          : load_mat_rows(dev, g, "llama", names, ns, count, k, kind, &out->q, interleave);
    fh_status st = fh_buffer_zeros(dev, k * n, &out->f);
    size_t at = 0;
    for (size_t i = 0; i < count && !st; i++) {
        fh_buffer *part = nullptr;
        if ((st = fh_gguf_upload_f32(dev, g, names[i].c_str(), &part))) break;
        st = fh_copy_f32(dev, part, 0, out->f, at, k * ns[i]);
        if (!st) st = fh_device_sync(dev);
        fh_buffer_free(part);
        at += k * ns[i];
    }
    return st;
}

fh_status load_lin(fh_device *dev, const fh_gguf *g, const std::string &name, size_t k, size_t n, fh_kind *kind,
                   fh_llama::Mat *out) {
    return load_lin(dev, g, &name, &n, 1, k, kind, out);
}

}  // namespace

extern "C" {

fh_status fh_llama_from_gguf(fh_device *dev, const fh_gguf *g, fh_path path, fh_llama **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!g || !out) return fail(FH_ERR_INVALID, "llama: no file or output");
    *out = nullptr;
    if (path == FH_PATH_AUTO) path = FH_PATH_TILED;
    if (path != FH_PATH_TILED && path != FH_PATH_TILED_FAST && path != FH_PATH_TILED_F16)
        return fail(FH_ERR_INVALID, "llama: the forward runs on FH_PATH_TILED, TILED_FAST or TILED_F16, not path %d",
                    (int)path);
    const char *a;
    size_t alen;
    if ((st = fh_gguf_get_string(g, "general.architecture", &a, &alen))) return st;
    const std::string arch(a, alen);
    if (arch != "llama" && arch != "qwen2")
        return fail(FH_ERR_INVALID, "architecture is '%s', only 'llama' and 'qwen2' are supported", arch.c_str());
    fh_llama *m = new (std::nothrow) fh_llama;
    if (!m) return fail(FH_ERR_OOM, "host out of memory");
    dev_retain(dev);
    m->dev = dev;
    m->path = path;
    m->neox = arch == "qwen2";  // ferrum_model/src/gguf/llama/mod.rs:108-117
    const char *unfused = getenv("FERRUM_HIP_ROPE_UNFUSED");
    m->fuse_rope = !(unfused && unfused[0] == '1');
    const char *su = getenv("FERRUM_HIP_SCORE_UNFUSED");
    m->fuse_score = !(su && su[0] == '1');
    const char *au = getenv("FERRUM_HIP_ATTN_SPLIT_UNFUSED");
    m->att_split = !(au && au[0] == '1');
    auto key = [&](const char *k) { return arch + "." + k; };
    auto has = [&](const std::string &k) {
        size_t i;
        return fh_gguf_find_key(g, k.c_str(), &i) == FH_OK;
    };
    auto opt_uint = [&](const char *k, size_t dflt, size_t *v) -> fh_status {
        if (!has(key(k))) {
            *v = dflt;
            return FH_OK;
        }
        return cfg_uint(g, key(k).c_str(), v);
    };
    auto opt_float = [&](const char *k, float dflt, float *v) -> fh_status {
        if (!has(key(k))) {
            *v = dflt;
            return FH_OK;
        }
        return fh_gguf_get_float(g, key(k).c_str(), v);
    };
    if ((st = cfg_uint(g, key("embedding_length").c_str(), &m->dim)) ||
        (st = cfg_uint(g, key("attention.head_count").c_str(), &m->heads)) ||
        (st = opt_uint("attention.head_count_kv", m->heads, &m->kv_heads)) ||
        (st = cfg_uint(g, key("block_count").c_str(), &m->layers)))
        return llama_fail_free(m, st);
    if (m->layers > fh_gguf_tensor_count(g))
        return llama_fail_free(m, fail(FH_ERR_INVALID, "block_count %zu exceeds the file's %zu tensors", m->layers,
                                       fh_gguf_tensor_count(g)));
    if ((st = opt_uint("attention.key_length", m->heads ? m->dim / m->heads : 0, &m->head_dim)) ||
        (st = opt_float("attention.layer_norm_rms_epsilon", 1e-5f, &m->eps)))
        return llama_fail_free(m, st);
    size_t tidx;
    fh_gguf_tensor tt;
    if ((st = fh_gguf_find_tensor(g, "token_embd.weight", &tidx)) || (st = fh_gguf_tensor_info(g, tidx, &tt)))
        return llama_fail_free(m, st);
    if (tt.n_dims != 2 || tt.dims[0] != m->dim)
        return llama_fail_free(m, fail(FH_ERR_INVALID, "token_embd.weight must be [embedding_length, vocab]"));
    m->vocab = (size_t)tt.dims[1];
    if ((st = opt_uint("context_length", 2048, &m->ctx)) || (st = cfg_uint(g, key("feed_forward_length").c_str(), &m->hidden)) ||
        (st = opt_uint("rope.dimension_count", m->head_dim, &m->rope_dim)) ||
        (st = opt_float("rope.freq_base", 10000.0f, &m->rope_base)))
        return llama_fail_free(m, st);
    // Config::validate (ferrum_ref/src/models/llama/mod.rs:63-95)
    if (!m->vocab || !m->ctx || !m->dim || !m->heads || !m->kv_heads || !m->head_dim || !m->layers || !m->hidden ||
        !m->rope_dim)
        return llama_fail_free(m, fail(FH_ERR_INVALID, "every dimension must be positive"));
    if (m->heads % m->kv_heads)
        return llama_fail_free(m, fail(FH_ERR_INVALID, "heads %zu is not a multiple of kv_heads %zu", m->heads, m->kv_heads));
    if (m->rope_dim > m->head_dim || m->rope_dim % 2)
        return llama_fail_free(m, fail(FH_ERR_INVALID, "rope_dim %zu must be even and at most head_dim %zu", m->rope_dim,
                                       m->head_dim));
    if (!std::isfinite(m->eps) || m->eps <= 0.0f || !std::isfinite(m->rope_base) || m->rope_base <= 0.0f)
        return llama_fail_free(m, fail(FH_ERR_INVALID, "eps and rope_base must be finite and positive"));
    const size_t d = m->dim, hid = m->hidden, qd = m->q_dim(), kvd = m->kv_dim(), hd = m->head_dim;
    // what the kernels take (matrices of any width: those not stored packed are multiplied as f32)
    if ((hd != 8 && hd != 16 && hd != 32 && hd != 64 && hd != 128) || m->qkv_width() > kMaxQkvWidth ||
        m->ctx > (1u << 20) || m->vocab > (1u << 30))
        return llama_fail_free(m, fail(FH_ERR_UNSUPPORTED,
                                       "llama: head %zu / q + k + v width %zu outside what the kernels take "
                                       "(heads 8, 16, 32, 64 or 128 wide; q + k + v at most %u wide)",
                                       hd, m->qkv_width(), kMaxQkvWidth));
    std::vector<float> ff, cos_t, sin_t;
    if ((st = rope_scaling(g, arch, m->rope_dim, &m->linear_factor, &ff))) return llama_fail_free(m, st);
    fh_kind kind = (fh_kind)0;
    if ((st = load_lin(dev, g, "token_embd.weight", d, m->vocab, &kind, &m->tok))) return llama_fail_free(m, st);
    m->tied = fh_gguf_find_tensor(g, "output.weight", &tidx) != FH_OK;
    if (m->tied) {
        m->head = m->tok;  // the file omits a head tied to the embedding (llama/mod.rs:191-197)
    } else if ((st = load_lin(dev, g, "output.weight", d, m->vocab, &kind, &m->head))) {
        return llama_fail_free(m, st);
    }
    if (fh_gguf_find_tensor(g, "output.bias", &tidx) == FH_OK)
        return llama_fail_free(m, fail(FH_ERR_INVALID, "tensor 'output.bias' is not supported"));
    if ((st = load_vec(dev, g, "llama", "output_norm.weight", d, &m->out_norm))) return llama_fail_free(m, st);
    m->blocks.resize(m->layers);
    {  // every block matrix stored Q8_0 / Q4_0 (what the fused producers need): then interleave gate / up
        bool all = true;
        for (size_t l = 0; l < m->layers && all; l++)
            for (const char *stem : {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                                     "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"}) {
                fh_gguf_tensor ti;
                const std::string nm = tensor_name("blk.", l, stem);
                if (fh_gguf_find_tensor(g, nm.c_str(), &tidx) != FH_OK || fh_gguf_tensor_info(g, tidx, &ti) != FH_OK ||
                    (ti.ggml_type != FH_Q8_0 && ti.ggml_type != FH_Q4_0)) {
                    all = false;
                    break;
                }
            }
        const char *sw = getenv("FERRUM_HIP_SWIGLU_UNFUSED");
        m->gu_inter = all && path == FH_PATH_TILED_FAST && hid % 32 == 0 && d <= 16384 && hid <= 16384 &&
                      !(sw && sw[0] == '1');
    }
    for (size_t l = 0; l < m->layers; l++) {
        auto &L = m->blocks[l];
        auto n = [&](const char *s) { return tensor_name("blk.", l, s); };
        for (const char *stem : {"attn_output.bias", "ffn_gate.bias", "ffn_up.bias", "ffn_down.bias"})
            if (fh_gguf_find_tensor(g, n(stem).c_str(), &tidx) == FH_OK)
                return llama_fail_free(m, fail(FH_ERR_INVALID,
                                               "tensor '%s' is not supported: biases are loaded only for attn_q/k/v",
                                               n(stem).c_str()));
        const std::string qkv[3] = {n("attn_q.weight"), n("attn_k.weight"), n("attn_v.weight")};
        const size_t qkv_n[3] = {qd, kvd, kvd};
        const std::string gu[2] = {n("ffn_gate.weight"), n("ffn_up.weight")};
        const size_t gu_n[2] = {hid, hid};
        if ((st = load_vec(dev, g, "llama", n("attn_norm.weight"), d, &L.attn_norm)) ||
            (st = load_lin(dev, g, qkv, qkv_n, 3, d, &kind, &L.wqkv)) ||
            (st = load_lin(dev, g, n("attn_output.weight"), qd, d, &kind, &L.wo)) ||
            (st = load_vec(dev, g, "llama", n("ffn_norm.weight"), d, &L.ffn_norm)) ||
            (st = load_lin(dev, g, gu, gu_n, 2, d, &kind, &L.wgu, m->gu_inter)) ||
            (st = load_lin(dev, g, n("ffn_down.weight"), hid, d, &kind, &L.down)))
            return llama_fail_free(m, st);
        m->packed = m->packed && L.wqkv.q && L.wo.q && L.wgu.q && L.down.q;
        // q/k/v biases, absent ones zero (one vector over the stacked rows)
        std::vector<float> bias(m->qkv_width(), 0.0f), part;
        bool any = false;
        const char *bnames[3] = {"attn_q.bias", "attn_k.bias", "attn_v.bias"};
        size_t at = 0;
        for (int i = 0; i < 3; i++) {
            if (fh_gguf_find_tensor(g, n(bnames[i]).c_str(), &tidx) == FH_OK) {
                if ((st = host_vec(g, "llama", n(bnames[i]), qkv_n[i], &part))) return llama_fail_free(m, st);
                std::copy(part.begin(), part.end(), bias.begin() + at);
                any = true;
            }
            at += qkv_n[i];
        }
        if (any && (st = fh_buffer_upload(dev, bias.data(), bias.size(), &L.bqkv))) return llama_fail_free(m, st);
        m->weight_bytes += L.wqkv.bytes() + L.wo.bytes() + L.wgu.bytes() + L.down.bytes();
    }
    m->weight_bytes += m->head.bytes();
    m->kind = kind;
    rope_tables(m->ctx, m->rope_dim, m->rope_base, ff, m->linear_factor, &cos_t, &sin_t);
    if ((st = fh_buffer_upload(dev, cos_t.data(), cos_t.size(), &m->rope_cos)) ||
        (st = fh_buffer_upload(dev, sin_t.data(), sin_t.size(), &m->rope_sin)))
        return llama_fail_free(m, st);
    if (path == FH_PATH_TILED_FAST) {  // the fast GEMM's fp8 correction operand of every weight
        std::vector<fh_qweight *> ws = {m->head.q};
        for (auto &L : m->blocks) ws.insert(ws.end(), {L.wqkv.q, L.wo.q, L.wgu.q, L.down.q});
        for (fh_qweight *w : ws) {
            if (!w) continue;  // f32 rows
            void *b8 = nullptr;
            if ((st = alloc_bytes(dev, gemm_b8_bytes(w->k, w->n), &b8))) return llama_fail_free(m, st);
            w->b8 = (uint8_t *)b8;
            if ((st = begin_command(dev, "llama load"))) return llama_fail_free(m, st);
            (void)launch_make_b8(dev->stream, w->kind, w->qs, w->ds, w->b8, w->k, w->n);
            if ((st = end_command(dev, "llama load"))) return llama_fail_free(m, st);
        }
    }
    if ((st = fh_device_sync(dev))) return llama_fail_free(m, st);
    *out = m;
    return FH_OK;
}

void fh_llama_free(fh_llama *m) {
    if (!m) return;
    if (m->dev) (void)hipStreamSynchronize(m->dev->stream);
    if (!m->tied) m->head.release();
    m->tok.release();
    for (auto &L : m->blocks) {
        for (fh_llama::Mat *w : {&L.wqkv, &L.wo, &L.wgu, &L.down}) w->release();
        for (fh_buffer *b : {L.attn_norm, L.ffn_norm, L.bqkv}) fh_buffer_free(b);
    }
    for (fh_buffer *b : {m->out_norm, m->rope_cos, m->rope_sin}) fh_buffer_free(b);
    if (m->arena) (void)hipFree(m->arena);
    if (m->dev) dev_release(m->dev);
    delete m;
}

fh_status fh_llama_config(const fh_llama *m, fh_llama_cfg *out) {
    if (!m || !out) return fail(FH_ERR_INVALID, "llama: no model or output");
    out->vocab = m->vocab;
    out->ctx = m->ctx;
    out->dim = m->dim;
    out->heads = m->heads;
    out->kv_heads = m->kv_heads;
    out->head_dim = m->head_dim;
    out->layers = m->layers;
    out->hidden = m->hidden;
    out->rope_dim = m->rope_dim;
    out->rope_base = m->rope_base;
    out->eps = m->eps;
    out->linear_factor = m->linear_factor;
    out->neox = m->neox ? 1 : 0;
    out->tied = m->tied ? 1 : 0;
    out->kind = m->kind;
    out->path = m->path;
    return FH_OK;
}

uint64_t fh_llama_weight_bytes(const fh_llama *m) { return m ? m->weight_bytes : 0; }

uint64_t fh_llama_device_bytes(const fh_llama *m) {
    if (!m) return 0;
    uint64_t b = m->tok.device_bytes() + m->arena_bytes;
    if (!m->tied) b += m->head.device_bytes();
    for (const fh_buffer *v : {m->out_norm, m->rope_cos, m->rope_sin})
        if (v) b += v->nbytes;
    for (const auto &L : m->blocks) {
        for (const fh_llama::Mat *w : {&L.wqkv, &L.wo, &L.wgu, &L.down}) b += w->device_bytes();
        for (const fh_buffer *v : {L.attn_norm, L.ffn_norm, L.bqkv})
            if (v) b += v->nbytes;
    }
    return b;
}

fh_status fh_llama_forward_all(fh_device *dev, fh_llama *m, const int32_t *ids, size_t n, float *logits) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!m || m->dev != dev) return fail(FH_ERR_INVALID, "llama: no model on this device");
    if ((st = check_len(m, n))) return st;
    if (!ids || !logits) return fail(FH_ERR_INVALID, "llama: no ids or output");
    if ((st = check_ids(m, ids, n)) || (st = ensure_rows(m, n))) return st;
    if ((st = begin_command(dev, "llama forward"))) return st;
    hipStream_t s = dev->stream;
    hipError_t e = hipMemcpyAsync(m->ids, ids, n * 4, hipMemcpyHostToDevice, s);
    if (!e) e = enqueue_body(m, s, n);
    for (size_t r0 = 0; r0 < n && !e; r0 += m->chunk) {
        const size_t rows = std::min(m->chunk, n - r0);
        if ((e = linear(m, s, m->head, m->h + r0 * m->dim, m->logits, rows))) break;
        e = hipMemcpyAsync(logits + r0 * m->vocab, m->logits, rows * m->vocab * 4, hipMemcpyDeviceToHost, s);
    }
    if (!e) e = hipStreamSynchronize(s);
    if (e) return hip_fail(dev, e, "llama forward");
    return end_command(dev, "llama forward");
}

fh_status fh_llama_score(fh_device *dev, fh_llama *m, const int32_t *ids, size_t n, float *logprob,
                         uint8_t *is_first_max) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!m || m->dev != dev) return fail(FH_ERR_INVALID, "llama: no model on this device");
    if (n < 2) return fail(FH_ERR_INVALID, "scoring needs at least 2 tokens");
    if (!ids || !logprob || !is_first_max) return fail(FH_ERR_INVALID, "llama: no ids or output");
    const size_t t = n - 1;
    if ((st = check_len(m, t)) || (st = check_ids(m, ids, n)) || (st = ensure_rows(m, t))) return st;
    if ((st = begin_command(dev, "llama score"))) return st;
    hipStream_t s = dev->stream;
    std::vector<float> pairs(2 * t);
    hipError_t e = hipMemcpyAsync(m->ids, ids, n * 4, hipMemcpyHostToDevice, s);
    if (!e) e = enqueue_score(m, s, t, m->scores);
    if (!e) e = hipMemcpyAsync(pairs.data(), m->scores, 2 * t * 4, hipMemcpyDeviceToHost, s);
    if (!e) e = hipStreamSynchronize(s);
    if (e) return hip_fail(dev, e, "llama score");
    for (size_t r = 0; r < t; r++) {
        logprob[r] = pairs[2 * r];
        is_first_max[r] = pairs[2 * r + 1] == 1.0f;
    }
    return end_command(dev, "llama score");
}

fh_status fh_llama_score_device(fh_device *dev, fh_llama *m, const fh_buffer *ids, size_t n, fh_buffer *out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!m || m->dev != dev) return fail(FH_ERR_INVALID, "llama: no model on this device");
    if (n < 2) return fail(FH_ERR_INVALID, "scoring needs at least 2 tokens");
    if (!ids || !out || ids->dev != dev || out->dev != dev) return fail(FH_ERR_INVALID, "llama: ids or output not on this device");
    if (ids->nbytes < n * 4) return fail(FH_ERR_INVALID, "llama: the ids buffer holds %zu bytes, needs %zu", ids->nbytes, n * 4);
    const size_t t = n - 1;
    if (out->nbytes < 2 * t * 4)
        return fail(FH_ERR_INVALID, "llama: the output holds %zu bytes, needs %zu", out->nbytes, 2 * t * 4);
    if ((st = check_len(m, t)) || (st = ensure_rows(m, t))) return st;
    if ((st = begin_command(dev, "llama score"))) return st;
    hipStream_t s = dev->stream;
    hipError_t e = hipMemcpyAsync(m->ids, ids->ptr, n * 4, hipMemcpyDeviceToDevice, s);
    if (!e) e = enqueue_score(m, s, t, (float *)out->ptr);
    if (e) return hip_fail(dev, e, "llama score");
    return end_command(dev, "llama score");
}

}  // extern "C"
