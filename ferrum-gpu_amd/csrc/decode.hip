// GPT-2 KV-cached decode on resident Q8_0 / Q4_0 weights (replaces ferrum_wgpu's GpuGpt2,
// ferrum_wgpu/src/models/gpt2.rs:52-265, whose weights are f32; the CPU oracle is ferrum_ref's
// Gpt2::feed, ferrum_ref/src/models/gpt2/decode.rs:57-117, on the fake-quantised model).
//
// A decode step is latency-bound (GPT-2-small reads 131 MB of packed weights per token, 26 us
// at HBM speed), so it is built from few, fused launches and replayed as one HIP graph:
//   embed                 x = tok[token] + pos[p]                     (token and p from device state)
//   per layer:
//     gemv LN|QKV         q | kcache[p] | vcache[p] = LN1(x) W_qkv + b  (one product, n = 3d)
//     attention           a = softmax(q k^T / sqrt(hd)) v, a workgroup per head
//     gemv RESIDUAL       x += a W_o + b_o
//     gemv LN|GELU        f = gelu(LN2(x) W_1 + b_1)
//     gemv RESIDUAL       x += f W_2 + b_2
//   gemv LN|STORE         logits = LNf(x) W_head
//   argmax                next token (sampling.rs:32-40), written to the device's input array;
//                         the position advances
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
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "gemv_parts.hpp"
#include "internal.hpp"

namespace fh {
namespace {

enum { PRO_NONE = 0, PRO_LN = 1 };
enum { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_GELU = 2, EPI_QKV = 3 };

constexpr int kMaxWaves = 8;          // wavefronts per decode-GEMV workgroup (two per SIMD)
constexpr uint32_t kMaxBlocks = 512;  // blocks per row (k <= 16384): 64 KiB of prepared x in LDS

struct DecodeGemv {
    const uint8_t *qs;
    const uint16_t *ds;
    const float *x;            // k inputs
    const float *ln_g, *ln_b;  // PRO_LN
    const float *bias;         // n, or null
    float *y;                  // n outputs; EPI_RESIDUAL adds into it; EPI_QKV: the q part
    float *kc, *vc;            // EPI_QKV: caches [ctx, split]
    const int32_t *state;      // state[0]: the position
    uint32_t nb, n, split;     // split: EPI_QKV width of each of q, k, v
    float eps;
};

// ferrum_ref/src/kernels/nn.rs:12-15
__device__ __forceinline__ float gelu(float x) {
    return 0.5f * x * (1.0f + tanhf(0.7978846f * (x + 0.044715f * x * x * x)));
}

// Sum over the workgroup (every thread gets the total); red holds one float per wavefront.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int m = 32; m >= 1; m /= 2) v += __shfl_xor(v, m, 64);
    const uint32_t w = threadIdx.x / 64, nw = blockDim.x / 64;
    __syncthreads();  // red may still be read by a previous call
    if (threadIdx.x % 64 == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (uint32_t i = 0; i < nw; i++) t += red[i];
    return t;
}

template <int KIND>
__device__ __forceinline__ void load_weights(Batch<KIND> &bt, __amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rd,
                                             uint32_t oq, uint32_t os, uint32_t b) {
    if constexpr (KIND == FH_Q8_0) {
#pragma unroll
        for (int i = 0; i < kBatch; i++)
            bt.q[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(oq + (b + i) * 1024), 0, kNonTemporal));
    } else {
#pragma unroll
        for (int i = 0; i < kBatch / 2; i++)
            bt.q[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(oq + (b + 2 * i) * 512), 0, kNonTemporal));
    }
    bt.s = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rd, (int)(os + b * 64), 0, 0));
}

// One workgroup per 32 output rows (blockIdx.x), W = blockDim.x / 64 wavefronts; wavefront w
// takes the batches 8w, 8w + 8W, ... of the row's blocks.
template <int KIND, int PRO, int EPI>
__global__ __launch_bounds__(64 * kMaxWaves) void decode_gemv_kernel(DecodeGemv a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t dlds[];
    const uint32_t W = blockDim.x / 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64, r = lane % 32;
    const bool upper = lane >= 32;
    const uint32_t nb = a.nb, nb8 = (nb + 7) / 8, span = nb8 * 8;
    constexpr uint32_t QB = KIND == FH_Q8_0 ? 32 : 16;
    const uint32_t g = blockIdx.x;
    const auto rq = make_rsrc(a.qs + (size_t)g * nb * 32 * QB, nb * 32 * QB);
    const auto rd = make_rsrc(a.ds + (size_t)g * nb8 * 256, nb8 * 512);
    const uint32_t oq = KIND == FH_Q8_0 ? (uint32_t)(r * 32 + 16 * upper) : (uint32_t)(lane * 16);
    const uint32_t os = (uint32_t)(r * 16), oa = (uint32_t)(r * 32 + 16 * upper);
    uint8_t *prep = dlds;                                   // span records
    float *part = (float *)(dlds + span * kPrepBytes);      // [W][32] row sums
    float *red = part + W * 32;                             // [W] reduction scratch

    // the weights of the wavefront's first batch are requested before x is prepared
    Batch<KIND> cur;
    uint32_t b = wave * kBatch;  // W <= nb8: every wavefront has a batch
    load_weights<KIND>(cur, rq, rd, oq, os, b);

    const uint32_t k = nb * 32;
    float mean = 0.0f, rstd = 1.0f;
    if constexpr (PRO == PRO_LN) {  // ferrum_ref/src/kernels/nn.rs:31-44
        float s = 0.0f;
        for (uint32_t i = threadIdx.x; i < k; i += blockDim.x) s += a.x[i];
        mean = block_sum(s, red) / (float)k;
        float v = 0.0f;
        for (uint32_t i = threadIdx.x; i < k; i += blockDim.x) {
            const float t = a.x[i] - mean;
            v += t * t;
        }
        rstd = 1.0f / sqrtf(block_sum(v, red) / (float)k + a.eps);
    }
    // every block's prepared x, eight lanes per block (the eight lanes share the loop bound)
    for (uint32_t blk = threadIdx.x / 8; blk < span; blk += blockDim.x / 8) {
        const int j = threadIdx.x % 8;
        __attribute__((address_space(3))) uint32_t *rec =
            (__attribute__((address_space(3))) uint32_t *)(prep + blk * kPrepBytes);
        if (blk < nb) {
            const uint32_t e = blk * 32 + 4 * j;
            f32x4 v = *(const __attribute__((address_space(1))) f32x4 *)(a.x + e);
            if constexpr (PRO == PRO_LN) {
                const f32x4 gg = *(const __attribute__((address_space(1))) f32x4 *)(a.ln_g + e);
                const f32x4 bb = *(const __attribute__((address_space(1))) f32x4 *)(a.ln_b + e);
#pragma unroll
                for (int c = 0; c < 4; c++) v[c] = (v[c] - mean) * rstd * gg[c] + bb[c];
            }
            prep_values<KIND>(v, j, rec);
        } else {
            *(__attribute__((address_space(3))) u32x4 *)(rec + 4 * j) = u32x4{0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();

    float acc = 0.0f;
    for (;;) {
        const uint32_t nxt = b + W * kBatch;
        Batch<KIND> nx;
        if (nxt < span) load_weights<KIND>(nx, rq, rd, oq, os, nxt);
        cur.a = *(const __attribute__((address_space(3))) i32x4 *)(prep + b * kPrepBytes + oa);
        compute_batch<KIND>(cur, upper, acc);
        if (nxt >= span) break;
        cur = nx;
        b = nxt;
    }
    // row r's odd blocks (lane 32 + r) join its even ones (lane r); the wavefronts' partial sums
    // meet in LDS and are added in wavefront order
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
    const float sum = acc + __uint_as_float(upper ? sw[0] : sw[1]);
    if (!upper) part[wave * 32 + r] = sum;
    __syncthreads();
    if (wave != 0 || upper) return;
    float t = 0.0f;
    for (uint32_t w = 0; w < W; w++) t += part[w * 32 + r];
    const uint32_t row = g * 32 + r;
    if (row >= a.n) return;
    if (a.bias) t = t + a.bias[row];  // decode.rs:42-53: the bias joins after the products
    if constexpr (EPI == EPI_STORE) {
        a.y[row] = t;
    } else if constexpr (EPI == EPI_RESIDUAL) {
        a.y[row] = a.y[row] + t;  // nn::add(x, gemv(..)), decode.rs:100,111
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

// One workgroup (256 threads) per head: decode.rs:81-105 over the cached positions 0..p.
__global__ __launch_bounds__(256) void attention_kernel(const float *__restrict__ q, const float *__restrict__ kc,
                                                        const float *__restrict__ vc, const int32_t *__restrict__ state,
                                                        float *__restrict__ out, uint32_t d, uint32_t hd, uint32_t ctx,
                                                        float scale) {
    extern __shared__ float alds[];
    float *s = alds;          // [ctx] scores, then probabilities
    float *red = alds + ctx;  // [256]
    const uint32_t h = blockIdx.x, T = (uint32_t)state[0] + 1, tid = threadIdx.x;
    const float *qh = q + h * hd;
    for (uint32_t j = tid; j < T; j += 256) {
        const float *kj = kc + (size_t)j * d + h * hd;
        float dot = 0.0f;
        for (uint32_t i = 0; i < hd; i++) dot += qh[i] * kj[i];
        s[j] = dot * scale;
    }
    __syncthreads();
    float m = -INFINITY;
    for (uint32_t j = tid; j < T; j += 256) m = fmaxf(m, s[j]);
#pragma unroll
    for (int o = 32; o >= 1; o /= 2) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (tid % 64 == 0) red[tid / 64] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float z = 0.0f;
    for (uint32_t j = tid; j < T; j += 256) {
        const float e = expf(s[j] - m);
        s[j] = e;
        z += e;
    }
    __syncthreads();  // red is rewritten below
#pragma unroll
    for (int o = 32; o >= 1; o /= 2) z += __shfl_xor(z, o, 64);
    if (tid % 64 == 0) red[4 + tid / 64] = z;
    __syncthreads();
    const float sum = red[4] + red[5] + red[6] + red[7];
    for (uint32_t j = tid; j < T; j += 256) s[j] = s[j] / sum;
    __syncthreads();
    // output element i of the head from positions j = part, part + P, ...; the P partial sums
    // are added in order
    const uint32_t P = 256 / hd, i = tid % hd, part = tid / hd;
    float acc = 0.0f;
    if (part < P)
        for (uint32_t j = part; j < T; j += P) acc += s[j] * vc[(size_t)j * d + h * hd + i];
    __syncthreads();
    red[tid] = acc;
    __syncthreads();
    if (tid < hd) {
        float t = 0.0f;
        for (uint32_t pp = 0; pp < P; pp++) t += red[pp * hd + tid];
        out[h * hd + tid] = t;
    }
}

// Greedy pick (ferrum_model/src/sampling.rs:32-40: the first maximum; NaN never wins), then the
// step's bookkeeping: the pick becomes the next input when the position is past the prompt, and
// the position advances.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ logits, uint32_t vocab,
                                                      int32_t *__restrict__ state, int32_t *__restrict__ inputs) {
    __shared__ float bv[1024];
    __shared__ uint32_t bi[1024];
    const uint32_t tid = threadIdx.x;
    float best = 0.0f;
    uint32_t idx = 0xffffffffu;  // none yet
    for (uint32_t i = tid; i < vocab; i += 1024) {
        const float v = logits[i];
        if (v == v && (idx == 0xffffffffu || v > best)) {
            best = v;
            idx = i;
        }
    }
    bv[tid] = best;
    bi[tid] = idx;
    __syncthreads();
    for (uint32_t o = 512; o >= 1; o /= 2) {
        if (tid < o) {
            const float v2 = bv[tid + o];
            const uint32_t i2 = bi[tid + o];
            const uint32_t i1 = bi[tid];
            if (i2 != 0xffffffffu &&
                (i1 == 0xffffffffu || v2 > bv[tid] || (v2 == bv[tid] && i2 < i1))) {
                bv[tid] = v2;
                bi[tid] = i2;
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        const int32_t pick = bi[0] == 0xffffffffu ? 0 : (int32_t)bi[0];
        const int32_t p = state[0];
        state[2] = pick;
        if (p + 1 >= state[1]) inputs[p + 1] = pick;
        state[0] = p + 1;
    }
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
    size_t pos = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool use_graph = true;
    uint64_t step_bytes = 0;
};

namespace {

fh_status gpt2_fail_free(fh_gpt2 *m, fh_status st) {
    fh_gpt2_free(m);
    return st;
}

// Launch shape of a decode GEMV: workgroups of 32 rows, wavefronts sharing the row's batches.
template <int KIND, int PRO, int EPI>
hipError_t launch_dgemv(hipStream_t s, const DecodeGemv &a) {
    const uint32_t nb8 = (a.nb + 7) / 8;
    const uint32_t W = nb8 < (uint32_t)kMaxWaves ? nb8 : (uint32_t)kMaxWaves;
    const size_t lds = (size_t)nb8 * 8 * kPrepBytes + (size_t)W * 32 * 4 + (size_t)W * 4;
    decode_gemv_kernel<KIND, PRO, EPI><<<(a.n + 31) / 32, 64 * W, lds, s>>>(a);
    return hipGetLastError();
}

// Dynamic LDS beyond the default 64 KiB: prepared x of up to kMaxBlocks blocks plus the row
// sums, and the attention scores of up to 16384 positions. Set once, before any capture.
hipError_t set_lds_limits() {
    static const hipError_t e = [] {
        const int gemv_lds = (int)(kMaxBlocks * kPrepBytes + kMaxWaves * 33 * 4);
        const void *fns[] = {
            (const void *)decode_gemv_kernel<FH_Q8_0, PRO_LN, EPI_QKV>, (const void *)decode_gemv_kernel<FH_Q8_0, PRO_NONE, EPI_RESIDUAL>,
            (const void *)decode_gemv_kernel<FH_Q8_0, PRO_LN, EPI_GELU>, (const void *)decode_gemv_kernel<FH_Q8_0, PRO_LN, EPI_STORE>,
            (const void *)decode_gemv_kernel<FH_Q4_0, PRO_LN, EPI_QKV>, (const void *)decode_gemv_kernel<FH_Q4_0, PRO_NONE, EPI_RESIDUAL>,
            (const void *)decode_gemv_kernel<FH_Q4_0, PRO_LN, EPI_GELU>, (const void *)decode_gemv_kernel<FH_Q4_0, PRO_LN, EPI_STORE>};
        for (const void *f : fns) {
            hipError_t r = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, gemv_lds);
            if (r) return r;
        }
        return hipFuncSetAttribute((const void *)attention_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (16384 + 256) * 4);
    }();
    return e;
}

template <int PRO, int EPI>
hipError_t dgemv(hipStream_t s, fh_kind kind, const DecodeGemv &a) {
    return kind == FH_Q8_0 ? launch_dgemv<FH_Q8_0, PRO, EPI>(s, a) : launch_dgemv<FH_Q4_0, PRO, EPI>(s, a);
}

DecodeGemv dg(const fh_qweight *w, const float *x, float *y) {
    DecodeGemv a{};
    a.qs = w->qs;
    a.ds = w->ds;
    a.x = x;
    a.y = y;
    a.nb = (uint32_t)(w->k / 32);
    a.n = (uint32_t)w->n;
    return a;
}

const float *fp(const fh_buffer *b) { return (const float *)b->ptr; }

// Enqueue one decode step (the graph's body).
hipError_t enqueue_step(fh_gpt2 *m, hipStream_t s) {
    const uint32_t d = (uint32_t)m->dim;
    if (m->kind == FH_Q8_0)
        embed_kernel<FH_Q8_0><<<1, 256, 0, s>>>(m->tok->qs, m->tok->ds, fp(m->pos_tab), m->state, m->inputs, m->x, d);
    else
        embed_kernel<FH_Q4_0><<<1, 256, 0, s>>>(m->tok->qs, m->tok->ds, fp(m->pos_tab), m->state, m->inputs, m->x, d);
    hipError_t e = hipGetLastError();
    const uint32_t hd = (uint32_t)(m->dim / m->heads);
    const float scale = 1.0f / sqrtf((float)hd);
    for (auto &L : m->blocks) {
        if (e) return e;
        DecodeGemv a = dg(L.wqkv, m->x, m->q);
        a.ln_g = fp(L.ln1_g);
        a.ln_b = fp(L.ln1_b);
        a.eps = m->eps;
        a.bias = fp(L.bqkv);
        a.kc = L.kc;
        a.vc = L.vc;
        a.state = m->state;
        a.split = d;
        if ((e = dgemv<PRO_LN, EPI_QKV>(s, m->kind, a))) return e;
        attention_kernel<<<(uint32_t)m->heads, 256, (m->ctx + 256) * sizeof(float), s>>>(
            m->q, L.kc, L.vc, m->state, m->att, d, hd, (uint32_t)m->ctx, scale);
        if ((e = hipGetLastError())) return e;
        a = dg(L.wo, m->att, m->x);
        a.bias = fp(L.bo);
        if ((e = dgemv<PRO_NONE, EPI_RESIDUAL>(s, m->kind, a))) return e;
        a = dg(L.w1, m->x, m->f);
        a.ln_g = fp(L.ln2_g);
        a.ln_b = fp(L.ln2_b);
        a.eps = m->eps;
        a.bias = fp(L.b1);
        if ((e = dgemv<PRO_LN, EPI_GELU>(s, m->kind, a))) return e;
        a = dg(L.w2, m->f, m->x);
        a.bias = fp(L.b2);
        if ((e = dgemv<PRO_NONE, EPI_RESIDUAL>(s, m->kind, a))) return e;
    }
    if (e) return e;
    DecodeGemv a = dg(m->head, m->x, m->logits);
    a.ln_g = fp(m->lnf_g);
    a.ln_b = fp(m->lnf_b);
    a.eps = m->eps;
    if ((e = dgemv<PRO_LN, EPI_STORE>(s, m->kind, a))) return e;
    argmax_kernel<<<1, 1024, 0, s>>>(m->logits, (uint32_t)m->vocab, m->state, m->inputs);
    return hipGetLastError();
}

// Run one step on the device stream: the captured graph (made on first use), or the launches.
fh_status run_step(fh_gpt2 *m) {
    fh_device *dev = m->dev;
    fh_status st = begin_command(dev, "gpt2 step");
    if (st) return st;
    if (m->use_graph && !m->exec) {
        hipError_t e = hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal);
        if (e) return hip_fail(dev, e, "gpt2 step capture");
        const hipError_t le = enqueue_step(m, dev->stream);
        e = hipStreamEndCapture(dev->stream, &m->graph);
        if (le) return hip_fail(dev, le, "gpt2 step capture");
        if (e) return hip_fail(dev, e, "gpt2 step capture");
        e = hipGraphInstantiate(&m->exec, m->graph, nullptr, nullptr, 0);
        if (e) {
            m->exec = nullptr;
            return hip_fail(dev, e, "gpt2 step graph");
        }
    }
    hipError_t e = m->use_graph ? hipGraphLaunch(m->exec, dev->stream) : enqueue_step(m, dev->stream);
    if (e) return hip_fail(dev, e, "gpt2 step");
    return end_command(dev, "gpt2 step");
}

std::string tname(const char *base, size_t layer, const char *suffix) {
    return std::string(base) + std::to_string(layer) + "." + suffix;
}

// A GGUF vector of `len` floats on the device.
fh_status vec(fh_device *dev, const fh_gguf *g, const std::string &name, size_t len, fh_buffer **out) {
    size_t idx;
    fh_status st = fh_gguf_find_tensor(g, name.c_str(), &idx);
    if (st) return st;
    fh_gguf_tensor t;
    if ((st = fh_gguf_tensor_info(g, idx, &t))) return st;
    if (t.elements != len || t.ggml_type != FH_GGML_F32)
        return fail(FH_ERR_INVALID, "gpt2: tensor '%s' must be %zu F32 values (has %llu of ggml type %u)", name.c_str(),
                    len, (unsigned long long)t.elements, t.ggml_type);
    return fh_gguf_upload_f32(dev, g, name.c_str(), out);
}

// A GGUF matrix of k inputs and n outputs (GGML dims [k, n]) as a resident weight.
fh_status mat(fh_device *dev, const fh_gguf *g, const std::string &name, size_t k, size_t n, fh_kind *kind,
              fh_qweight **out) {
    size_t idx;
    fh_status st = fh_gguf_find_tensor(g, name.c_str(), &idx);
    if (st) return st;
    fh_gguf_tensor t;
    if ((st = fh_gguf_tensor_info(g, idx, &t))) return st;
    if (t.n_dims != 2 || t.dims[0] != k || t.dims[1] != n)
        return fail(FH_ERR_INVALID, "gpt2: tensor '%s' must have dims [%zu, %zu]", name.c_str(), k, n);
    if (t.ggml_type != FH_GGML_Q8_0 && t.ggml_type != FH_GGML_Q4_0)
        return fail(FH_ERR_UNSUPPORTED, "gpt2: tensor '%s' has ggml type %u; the decoder multiplies Q8_0 or Q4_0 matrices",
                    name.c_str(), t.ggml_type);
    if (*kind == (fh_kind)0) *kind = (fh_kind)t.ggml_type;
    if ((fh_kind)t.ggml_type != *kind)
        return fail(FH_ERR_UNSUPPORTED, "gpt2: tensor '%s' mixes block formats (the model's matrices must share one)",
                    name.c_str());
    return fh_gguf_upload_qweight(dev, g, name.c_str(), out);
}

fh_status cfg_uint(const fh_gguf *g, const char *key, size_t *out) {
    uint64_t v;
    fh_status st = fh_gguf_get_uint(g, key, &v);
    if (st) return st;
    *out = (size_t)v;
    return FH_OK;
}

}  // namespace

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
    if (d % 32 || h % 32 || d / 32 > kMaxBlocks || h / 32 > kMaxBlocks || hd > 256 || m->ctx > 16384 ||
        m->vocab > (1u << 30))
        return gpt2_fail_free(m, fail(FH_ERR_UNSUPPORTED,
                                      "gpt2: dim %zu / hidden %zu / head %zu / ctx %zu outside what the decode kernels "
                                      "take (multiples of 32 up to 16384, heads up to 256 wide, ctx up to 16384)",
                                      d, h, hd, m->ctx));
    fh_kind kind = (fh_kind)0;
    if ((st = mat(dev, g, "token_embd.weight", d, m->vocab, &kind, &m->tok))) return gpt2_fail_free(m, st);
    if (fh_gguf_find_tensor(g, "output.weight", &tidx) == FH_OK) {
        if ((st = mat(dev, g, "output.weight", d, m->vocab, &kind, &m->head))) return gpt2_fail_free(m, st);
    } else {
        m->head = m->tok;  // tied (ferrum_model/src/gguf/gpt2.rs:228-231 omits a tied head)
    }
    m->kind = kind;
    if ((st = vec(dev, g, "position_embd.weight", m->ctx * d, &m->pos_tab)) ||
        (st = vec(dev, g, "output_norm.weight", d, &m->lnf_g)) || (st = vec(dev, g, "output_norm.bias", d, &m->lnf_b)))
        return gpt2_fail_free(m, st);
    m->blocks.resize(m->layers);
    for (size_t l = 0; l < m->layers; l++) {
        auto &L = m->blocks[l];
        if ((st = vec(dev, g, tname("blk.", l, "attn_norm.weight"), d, &L.ln1_g)) ||
            (st = vec(dev, g, tname("blk.", l, "attn_norm.bias"), d, &L.ln1_b)) ||
            (st = mat(dev, g, tname("blk.", l, "attn_qkv.weight"), d, 3 * d, &kind, &L.wqkv)) ||
            (st = vec(dev, g, tname("blk.", l, "attn_qkv.bias"), 3 * d, &L.bqkv)) ||
            (st = mat(dev, g, tname("blk.", l, "attn_output.weight"), d, d, &kind, &L.wo)) ||
            (st = vec(dev, g, tname("blk.", l, "attn_output.bias"), d, &L.bo)) ||
            (st = vec(dev, g, tname("blk.", l, "ffn_norm.weight"), d, &L.ln2_g)) ||
            (st = vec(dev, g, tname("blk.", l, "ffn_norm.bias"), d, &L.ln2_b)) ||
            (st = mat(dev, g, tname("blk.", l, "ffn_up.weight"), d, h, &kind, &L.w1)) ||
            (st = vec(dev, g, tname("blk.", l, "ffn_up.bias"), h, &L.b1)) ||
            (st = mat(dev, g, tname("blk.", l, "ffn_down.weight"), h, d, &kind, &L.w2)) ||
            (st = vec(dev, g, tname("blk.", l, "ffn_down.bias"), d, &L.b2)))
            return gpt2_fail_free(m, st);
        m->step_bytes += L.wqkv->nbytes + L.wo->nbytes + L.w1->nbytes + L.w2->nbytes;
    }
    m->step_bytes += m->head->nbytes;
    // caches and scratch in one allocation (every piece 256-byte aligned)
    auto up = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    const size_t cache = up(m->ctx * d * 4);
    const size_t total = 2 * m->layers * cache + 3 * up(d * 4) + up(h * 4) + up(m->vocab * 4) + up(16) +
                         up((m->ctx + 1) * 4);
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
    if (hipError_t e = set_lds_limits()) return gpt2_fail_free(m, hip_fail(dev, e, "gpt2 kernels"));
    const char *ng = getenv("FERRUM_HIP_NO_GRAPH");
    m->use_graph = !(ng && ng[0] == '1');
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
    if (m->dev) dev_release(m->dev);
    delete m;
}

}  // extern "C"
