/* ferrum_hip: MI355X-native (gfx950) quantized-weight path for ferrum-gpu.
 *
 * C ABI over hand-written HIP kernels. It is a drop-in for ferrum_wgpu's `ops_quant` and
 * `ops_qat` modules and the slice of the `Gpu`/`GpuBuf` device layer they use. Every entry point
 * names the reference interface it replaces (paths relative to the ferrum-gpu repository).
 * Plain pointers, sizes and opaque handles only; no C++ or HIP types cross the boundary.
 *
 * Formats: GGUF Q8_0 (34-byte blocks: f16 scale + 32 x i8) and Q4_0 (18-byte blocks: f16 scale
 * + 16 bytes, byte j holds element j in its low nibble and element j+16 in its high nibble),
 * blocks of 32 along the input dimension. A quantized weight W of k inputs and n outputs is
 * uploaded as GGUF rows (n rows of k/32 blocks, the tensor data of a GGUF file) and kept as the
 * same bytes repacked into tiles for the matrix cores: a plane of quants and a plane of f16 scales,
 * rows padded to a multiple of 32 and scales to a multiple of eight blocks. fh_qweight_read_gguf
 * gives the GGUF rows back bit for bit.
 *
 * Errors: every call returns an fh_status; on failure fh_last_error() (thread-local) holds a
 * message carrying the same substrings the reference's GpuError texts carry, so tests can match
 * them: "linear_q x", "linear_q y", "one row", "whole", "needs", "injected fault",
 * "GPU out of memory", "destination", "is not". A device fault makes the device "lost"
 * (sticky). Nothing aborts the process.
 *
 * Ordering: each device owns one HIP stream. Calls enqueue asynchronously and in order on it
 * (ferrum_wgpu/src/device/runtime.rs:152-192); results are observed by the reading calls, which
 * synchronize (device/tensor.rs:128-160).
 */
#ifndef FERRUM_HIP_H
#define FERRUM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FH_ABI_VERSION 1

#if defined(__GNUC__)
#define FH_API __attribute__((visibility("default")))
#else
#define FH_API
#endif

typedef enum fh_status {
    FH_OK = 0,
    FH_ERR_INVALID = 1,     /* bad argument or shape */
    FH_ERR_UNSUPPORTED = 2, /* a block format other than Q8_0 / Q4_0 */
    FH_ERR_DEVICE = 3,      /* HIP runtime error */
    FH_ERR_OOM = 4,         /* "GPU out of memory" */
    FH_ERR_INJECTED = 5,    /* "injected fault" from fh_debug_fail_after */
    FH_ERR_LOST = 6         /* the device faulted earlier; sticky */
} fh_status;

/* Block formats, by ggml tensor type id (ferrum_gguf/src/lib.rs:25-55). Replaces
 * ferrum_wgpu::ops_quant::QKind (ferrum_wgpu/src/ops/quant.rs:27-121): Q8_0, Q4_0 (the tiled
 * planes and the MFMA kernels), F16, MXFP4 (Fp4), FP8 E4M3 / E5M2 (no ggml type: the ids 1024 and
 * 1025 are this library's) and Q2_K (resident as GGUF rows, decoded on the fly: an f32-accumulating
 * GEMV for one row, an MFMA GEMM with x carried to about 22 bits for more; a block holding an
 * infinity or NaN makes that GEMM's outputs NaN).
 * The read-only GGUF block types (ferrum_gguf/src/codec/blocks.rs:34-48) are accepted by
 * fh_nbytes and fh_decode only. */
typedef enum fh_kind {
    FH_F16 = 1,
    FH_Q4_0 = 2,
    FH_Q4_1 = 3,
    FH_Q5_0 = 6,
    FH_Q5_1 = 7,
    FH_Q8_0 = 8,
    FH_Q8_1 = 9,
    FH_Q2_K = 10,
    FH_Q3_K = 11,
    FH_Q4_K = 12,
    FH_Q5_K = 13,
    FH_Q6_K = 14,
    FH_MXFP4 = 39,
    FH_FP8_E4M3 = 1024,
    FH_FP8_E5M2 = 1025
} fh_kind;

/* Which kernel runs a quantized linear layer. Replaces QPath (ferrum_wgpu/src/ops/quant.rs:292-305):
 * NAIVE = one thread per output (the baseline kernel), GEMV = batch-1 wavefront GEMV (exactly one
 * row), TILED = the LDS-staged MFMA dequant-GEMM (any rows; x carried to about 22 bits, within the
 * reference's 1e-5 product tolerance), AUTO = fh_choose. No counterpart in the reference:
 * TILED_FAST = the scoring GEMM (x as f16 plus an fp8 correction on the fp8 matrix cores; within
 * the MFMA-GEMM tolerance |g - w| <= 1e-3 + 2e-3 |w|, about 5e-5 absolute at the scoring shapes);
 * TILED_F16 = the dequant-f16 GEMM (weights dequantised to f16 d*q in LDS, x as f16 with a
 * power-of-two row scale, plain f16 MFMA with f32 accumulation; each product rounds both operands
 * to f16, so |g - w| <= 2^-10 sum_k |x_k w_k| roughly: it does NOT meet the MFMA-GEMM tolerance
 * per output; measured at the TinyLlama-1.1B shapes, M = 4096, 5.4e-5 (Q4_0) and 1.1e-4 (Q8_0)
 * of the outputs fall outside it, the worst at 1.8 to 2.0 times the bound);
 * ROWS = the few-row kernel for 2..64 rows (the weights streamed once from HBM into registers for
 * every row, x carried to about 22 bits as TILED does; within the reference's 1e-5). */
typedef enum fh_path {
    FH_PATH_AUTO = 0,
    FH_PATH_NAIVE = 1,
    FH_PATH_GEMV = 2,
    FH_PATH_TILED = 3,
    FH_PATH_TILED_FAST = 4,
    FH_PATH_TILED_F16 = 5,
    FH_PATH_ROWS = 6
} fh_path;

typedef struct fh_device fh_device;   /* replaces ferrum_wgpu::device::Gpu */
typedef struct fh_buffer fh_buffer;   /* replaces ferrum_wgpu::tensor::GpuBuf (plus byte buffers) */
typedef struct fh_qweight fh_qweight; /* replaces ferrum_wgpu::ops_quant::QWeight */
typedef struct fh_gemv_plan fh_gemv_plan;

/* ---- errors and version ---- */
FH_API const char *fh_last_error(void); /* thread-local message of this thread's last failure */
FH_API int fh_abi_version(void);

/* ---- device (ferrum_wgpu/src/device/mod.rs:127-165 Gpu::open; runtime.rs:67-93 check) ---- */
FH_API fh_status fh_device_open(int ordinal, fh_device **out);
FH_API void fh_device_close(fh_device *dev);
/* Wait for every command enqueued so far (the reference waits inside Gpu::read). */
FH_API fh_status fh_device_sync(fh_device *dev);
/* Adapter name and compute-unit count (device/mod.rs:88-95 AdapterInfo). */
FH_API fh_status fh_device_info(fh_device *dev, char *name, size_t cap, int *compute_units);
/* The device's HIP stream (a hipStream_t) for callers that interleave their own work. */
FH_API void *fh_device_stream(fh_device *dev);
/* Test hook: the n-th command from now fails with "injected fault"; n < 0 disarms
 * (device/runtime.rs:218-240 Gpu::fail_after). */
FH_API void fh_debug_fail_after(fh_device *dev, int64_t n);
/* Commands (kernel launches and copies) issued so far on this device (runtime.rs:127-135). */
FH_API uint64_t fh_debug_commands(fh_device *dev);

/* ---- buffers (ferrum_wgpu/src/device/tensor.rs:7-160) ---- */
/* f32 buffer of len zeros (Gpu::zeros, tensor.rs:36-66). */
FH_API fh_status fh_buffer_zeros(fh_device *dev, size_t len, fh_buffer **out);
/* f32 buffer holding host[0..len) (Gpu::upload, tensor.rs:69-101). */
FH_API fh_status fh_buffer_upload(fh_device *dev, const float *host, size_t len, fh_buffer **out);
/* Copy the whole buffer to host (len must equal its length); synchronizes (Gpu::read). */
FH_API fh_status fh_buffer_read(fh_device *dev, const fh_buffer *buf, float *host, size_t len);
/* Overwrite the whole buffer from host (queue.write_buffer). */
FH_API fh_status fh_buffer_write(fh_device *dev, fh_buffer *buf, const float *host, size_t len);
/* Byte buffers hold packed blocks for the device codec. */
FH_API fh_status fh_bytes_zeros(fh_device *dev, size_t nbytes, fh_buffer **out);
FH_API fh_status fh_bytes_upload(fh_device *dev, const uint8_t *host, size_t nbytes, fh_buffer **out);
FH_API fh_status fh_bytes_read(fh_device *dev, const fh_buffer *buf, uint8_t *host, size_t nbytes);
FH_API size_t fh_buffer_len(const fh_buffer *buf);    /* f32 elements (nbytes / 4) */
FH_API size_t fh_buffer_nbytes(const fh_buffer *buf);
FH_API void *fh_buffer_device_ptr(const fh_buffer *buf);
FH_API void fh_buffer_free(fh_buffer *buf);
/* dst[dst_off..+len) = src[src_off..+len) in f32 elements (Gpu::copy_f32, runtime.rs:294-336). */
FH_API fh_status fh_copy_f32(fh_device *dev, const fh_buffer *src, size_t src_off, fh_buffer *dst,
                      size_t dst_off, size_t len);

/* ---- block codec on the device (ferrum_gguf/src/codec/quant.rs) ---- */
/* Bytes n elements occupy, 0 with an error for an unsupported kind or n not whole blocks
 * (quant.rs:17-47). */
FH_API size_t fh_nbytes(fh_kind kind, size_t n);
/* Encode n f32 values (blocks of 32 consecutive values) into GGUF blocks (quant::encode,
 * quant.rs:91-136), bit-exact. src holds >= n floats, dst >= fh_nbytes bytes. */
FH_API fh_status fh_encode(fh_device *dev, fh_kind kind, const fh_buffer *src, size_t n, fh_buffer *dst);
/* Decode n elements of GGUF blocks to f32 (quant::decode, quant.rs:50-88), bit-exact. */
FH_API fh_status fh_decode(fh_device *dev, fh_kind kind, const fh_buffer *src, size_t n, fh_buffer *dst);

/* ---- resident quantized weights (ferrum_wgpu/src/ops/quant.rs:155-288) ---- */
/* upload_qweight (quant.rs:267-277): bytes are GGUF rows, n rows of k/32 blocks; kept bit-exact.
 * Errors: "whole" when k is not a positive multiple of 32, "needs" when len is wrong. */
FH_API fh_status fh_qweight_upload_gguf(fh_device *dev, fh_kind kind, const uint8_t *bytes, size_t len,
                                 size_t k, size_t n, fh_qweight **out);
/* upload_quantised (quant.rs:279-288): w is the [k, n] (in, out) row-major f32 weight on the
 * host; it is uploaded and quantised on the device (transpose + encode, quantise_matrix). */
FH_API fh_status fh_qweight_upload_f32(fh_device *dev, fh_kind kind, const float *w, size_t k, size_t n,
                                fh_qweight **out);
/* quantise_matrix on the device (quant.rs:238-252) from a resident [k, n] f32 buffer. */
FH_API fh_status fh_qweight_quantise(fh_device *dev, fh_kind kind, const fh_buffer *w, size_t k,
                              size_t n, fh_qweight **out);
FH_API void fh_qweight_free(fh_qweight *w);
/* QWeight::{kind, k, n, device_bytes} (quant.rs:163-182). device_bytes is the device memory the
 * weight holds: its padded tile planes (the GGUF rows for F16, MXFP4, FP8 and Q2_K) and, once a
 * multi-row FH_PATH_TILED_FAST product or a fast-path model has built it, the fast GEMM's e4m3
 * correction operand (about one byte per weight). */
FH_API fh_kind fh_qweight_kind(const fh_qweight *w);
FH_API size_t fh_qweight_k(const fh_qweight *w);
FH_API size_t fh_qweight_n(const fh_qweight *w);
FH_API uint64_t fh_qweight_device_bytes(const fh_qweight *w);
/* The resident GGUF bytes, read back bit-exactly (len must equal n * k/32 * block bytes). */
FH_API fh_status fh_qweight_read_gguf(fh_device *dev, const fh_qweight *w, uint8_t *host, size_t len);
/* dequantise_bytes + transpose on the device: out = the [k, n] f32 weight the CPU multiplies by
 * (quant.rs:256-264; models/llama/mod.rs:188-213). out holds k*n floats. */
FH_API fh_status fh_qweight_dequantise(fh_device *dev, const fh_qweight *w, fh_buffer *out);

/* ---- quantized linear layers (ferrum_wgpu/src/ops/quant.rs:306-381) ---- */
/* choose (quant.rs:306-323): the kernel AUTO picks for rows x (k, n), from MI355X measurements. */
FH_API fh_path fh_choose(size_t rows, fh_kind kind, size_t k, size_t n);
/* linear_q / linear_q_with: y[rows, n] = x[rows, k] * W, W dequantized in the kernel, no bias.
 * x must hold exactly rows*k floats ("linear_q x"), y exactly rows*n ("linear_q y"); y is
 * overwritten. GEMV takes exactly one row ("one row"). One command; does not wait. */
FH_API fh_status fh_linear_q(fh_device *dev, const fh_buffer *x, const fh_qweight *w, fh_buffer *y,
                      size_t rows, fh_path path);
/* The same product on raw device pointers (x: rows*k floats, y: rows*n floats), for callers that
 * own their memory (a torch tensor, a KV-cache arena). Same checks on rows and shapes. */
FH_API fh_status fh_linear_q_ptr(fh_device *dev, const float *x, const fh_qweight *w, float *y,
                          size_t rows, fh_path path);
/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): fh_linear_q_ptr with
 * the same kernels and results, but no device allocation or free of any kind. Its scratch (the
 * GEMV's prepared x, the GEMMs' split x and K-split partial sums) is one static device array of
 * FH_NOALLOC_SCRATCH_BYTES per GPU, made when the library loads on that GPU and held until the
 * process ends; a product that needs more fails with "scratch". Every call on one GPU shares that
 * array and it keeps the last call's contents: calls that overlap on one GPU (from two threads, or
 * through two fh_device handles of one ordinal, each with its own stream) race. FH_PATH_TILED_FAST
 * also needs the weight's correction operand, built by an ordinary multi-row FH_PATH_TILED_FAST
 * linear_q on that weight; without it the call fails. */
#define FH_NOALLOC_SCRATCH_BYTES (32u << 20)
FH_API fh_status fh_linear_q_noalloc(fh_device *dev, const float *x, const fh_qweight *w, float *y,
                                     size_t rows, fh_path path);

/* No counterpart in the reference: one launch for many independent batch-1 products
 * y_i = x_i * W_i (a decode step's projections, or several models' layers). The plan is built
 * once (the descriptors are uploaded then) and run any number of times; x_i and y_i are device
 * pointers of k_i and n_i floats. Per block format, the products up to 3,584 inputs wide share
 * one launch (x prepared in the product kernel, or by a preparation kernel first) and the wider
 * ones another, whose prepared x the first launch writes. */
typedef struct fh_gemv_problem {
    const fh_qweight *w;
    const float *x;
    float *y;
} fh_gemv_problem;
FH_API fh_status fh_gemv_plan_create(fh_device *dev, const fh_gemv_problem *problems, size_t count,
                              fh_gemv_plan **out);
FH_API fh_status fh_gemv_plan_run(fh_device *dev, const fh_gemv_plan *plan);
/* Launch i of a plan alone (fh_gemv_plan_run is launches 0 .. n-1 in order; a launch may write
 * the prepared x of the next one, so run them in order): for timing a launch on its own. */
FH_API fh_status fh_gemv_plan_run_launch(fh_device *dev, const fh_gemv_plan *plan, size_t i);
/* Grouped launches one run issues (one per block format), and the algorithmic bytes it moves (weights + x + y). */
FH_API size_t fh_gemv_plan_launches(const fh_gemv_plan *plan);
FH_API uint64_t fh_gemv_plan_bytes(const fh_gemv_plan *plan);
FH_API void fh_gemv_plan_free(fh_gemv_plan *plan);

/* No counterpart in the reference: one launch pair for many independent few-row products
 * y_i = x_i * W_i, x_i of rows_i x k_i and y_i of rows_i x n_i floats (device pointers), rows_i in
 * 1..64, on the FH_PATH_ROWS kernel (the reference issues one linear_q per matrix,
 * ferrum_wgpu/src/ops/quant.rs:326-381). Built once, run any number of times; products with the
 * same block format share a launch (two kernels: x split, then the products). Q8_0 and Q4_0 only. */
typedef struct fh_rows_plan fh_rows_plan;
typedef struct fh_rows_problem {
    const fh_qweight *w;
    const float *x;
    float *y;
    size_t rows;
} fh_rows_problem;
FH_API fh_status fh_rows_plan_create(fh_device *dev, const fh_rows_problem *problems, size_t count,
                                     fh_rows_plan **out);
FH_API fh_status fh_rows_plan_run(fh_device *dev, const fh_rows_plan *plan);
FH_API size_t fh_rows_plan_launches(const fh_rows_plan *plan);
/* Algorithmic bytes one run moves: the packed weights, x and y of every product. */
FH_API uint64_t fh_rows_plan_bytes(const fh_rows_plan *plan);
FH_API void fh_rows_plan_free(fh_rows_plan *plan);

/* ---- quantisation-aware training snap (ferrum_wgpu/src/ops/qat.rs:21-57) ---- */
/* q8_snap_rows: snap src into dst along rows (blocks of 32 consecutive values). ne0 not a
 * positive multiple of 32, or a length that is not whole blocks, copies unchanged.
 * "destination" when the lengths differ. Bit-exact with decode(encode(block)). */
FH_API fh_status fh_q8_snap_rows(fh_device *dev, const fh_buffer *src, fh_buffer *dst, size_t ne0);
/* q8_snap_cols: snap an [rows_in, cols_out] row-major weight down its columns. "is not" when
 * the length is not rows_in*cols_out; rows_in not a multiple of 32 copies unchanged. */
FH_API fh_status fh_q8_snap_cols(fh_device *dev, const fh_buffer *src, fh_buffer *dst, size_t rows_in,
                          size_t cols_out);

/* A whole QAT snap pass in one launch: replaces the loop of GpuTrainer::record_snap
 * (ferrum_wgpu/src/training/gpt2/qat.rs:58-72), which records one q8_snap_rows / q8_snap_cols /
 * copy per parameter. Each problem is one of those calls on device pointers of len floats:
 * FH_SNAP_ROWS (a = ne0), FH_SNAP_COLS (a = rows_in, b = cols_out, len = a * b) or FH_SNAP_COPY;
 * the same fallbacks apply (a rows snap whose ne0 or len is not whole 32-blocks, or a column snap
 * whose rows_in is not, copies). Built once, run any number of times; every problem shares one
 * launch, bit-identical to its single call. */
typedef enum fh_snap_mode { FH_SNAP_ROWS = 0, FH_SNAP_COLS = 1, FH_SNAP_COPY = 2 } fh_snap_mode;
typedef struct fh_snap_problem {
    const float *src;
    float *dst;
    size_t len;
    size_t a, b;
    int mode; /* fh_snap_mode */
} fh_snap_problem;
typedef struct fh_snap_plan fh_snap_plan;
FH_API fh_status fh_snap_plan_create(fh_device *dev, const fh_snap_problem *problems, size_t count,
                                     fh_snap_plan **out);
FH_API fh_status fh_snap_plan_run(fh_device *dev, const fh_snap_plan *plan);
/* Bytes one run reads and writes (8 per value). */
FH_API uint64_t fh_snap_plan_bytes(const fh_snap_plan *plan);
FH_API void fh_snap_plan_free(fh_snap_plan *plan);

/* ---- GGUF v3 container (ferrum_gguf/src/io/reader.rs:167-322) ----
 * Replaces ferrum_gguf::Gguf. The parser is hostile-input safe: every read is bounds-checked,
 * sizes use checked arithmetic, and nothing is allocated from a header count before the count is
 * proven to fit in the file. Failures return FH_ERR_INVALID (FH_ERR_UNSUPPORTED for an unknown
 * ggml tensor type) with fh_last_error() text "gguf: ..." carrying the reference's substrings:
 * "magic", "version", "unexpected end of file", "exceed", "array length", "nested arrays",
 * "unknown metadata value type", "dims", "alignment", "past the end", "duplicate",
 * "missing key", "non-negative integer", "is not an f32", "is not a string", "missing tensor",
 * "header-only", "not a multiple of the block size", "unsupported ggml tensor type".
 * A parsed file keeps its bytes (an owned copy, or a read-only mapping of the file); every
 * pointer handed out below stays valid until fh_gguf_close. */
typedef struct fh_gguf fh_gguf;

/* ggml tensor type ids (ferrum_gguf/src/lib.rs:24-55). */
enum {
    FH_GGML_F32 = 0, FH_GGML_F16 = 1, FH_GGML_Q4_0 = 2, FH_GGML_Q4_1 = 3, FH_GGML_Q5_0 = 6,
    FH_GGML_Q5_1 = 7, FH_GGML_Q8_0 = 8, FH_GGML_Q8_1 = 9, FH_GGML_Q2_K = 10, FH_GGML_Q3_K = 11,
    FH_GGML_Q4_K = 12, FH_GGML_Q5_K = 13, FH_GGML_Q6_K = 14, FH_GGML_I16 = 25, FH_GGML_I32 = 26,
    FH_GGML_MXFP4 = 39
};
/* Metadata value tags (GGUF v3; reader.rs:125-155): U8 0, I8 1, U16 2, I16 3, U32 4, I32 5,
 * F32 6, BOOL 7, STRING 8, ARRAY 9, U64 10, I64 11, F64 12. */

/* quant::nbytes (ferrum_gguf/src/codec/quant.rs:17-47): bytes n elements of a ggml type occupy. */
FH_API fh_status fh_ggml_nbytes(uint32_t ggml_type, uint64_t n, uint64_t *out);

/* Gguf::parse (reader.rs:165-170): parse a whole file held in memory (the bytes are copied). */
FH_API fh_status fh_gguf_parse(const uint8_t *bytes, size_t len, fh_gguf **out);
/* Gguf::parse_prefix (reader.rs:172-247): parse from the first `len` bytes of a file `total`
 * bytes long; tensor extents are checked against `total`, and reading data beyond `len` fails
 * ("header-only"). */
FH_API fh_status fh_gguf_parse_prefix(const uint8_t *bytes, size_t len, uint64_t total, fh_gguf **out);
/* Open a file by path through a read-only memory mapping: nothing is read until used, and
 * tensor bytes go from the mapping to the device without an intermediate host copy. */
FH_API fh_status fh_gguf_open(const char *path, fh_gguf **out);
FH_API void fh_gguf_close(fh_gguf *g);
/* Debug summary (reader.rs:91-101): "Gguf { K keys, T tensors, B bytes }" into buf. */
FH_API size_t fh_gguf_describe(const fh_gguf *g, char *buf, size_t cap);

/* Metadata, in file order (Gguf::kv, reader.rs:83-84). Strings are not NUL-terminated. */
FH_API size_t fh_gguf_kv_count(const fh_gguf *g);
FH_API fh_status fh_gguf_kv_key(const fh_gguf *g, size_t i, const char **key, size_t *len);
/* Entry i: its tag, and for scalars and strings the little-endian payload (a string's bytes).
 * For arrays: data and nbytes span the packed elements, and fh_gguf_kv_array gives the element
 * tag and count. */
FH_API fh_status fh_gguf_kv_value(const fh_gguf *g, size_t i, uint32_t *type, const uint8_t **data,
                                  size_t *nbytes);
FH_API fh_status fh_gguf_kv_array(const fh_gguf *g, size_t i, uint32_t *elem_type, uint64_t *count);
/* Element j of a string array. */
FH_API fh_status fh_gguf_kv_array_string(const fh_gguf *g, size_t i, uint64_t j, const char **s,
                                         size_t *len);
/* Gguf::get (reader.rs:249-252): index of the first entry with this key, or "missing key". */
FH_API fh_status fh_gguf_find_key(const fh_gguf *g, const char *key, size_t *index);
/* Typed getters (reader.rs:254-286). */
FH_API fh_status fh_gguf_get_uint(const fh_gguf *g, const char *key, uint64_t *out);
FH_API fh_status fh_gguf_get_float(const fh_gguf *g, const char *key, float *out);
FH_API fh_status fh_gguf_get_string(const fh_gguf *g, const char *key, const char **s, size_t *len);

/* Tensor directory, in file order (TensorInfo, reader.rs:58-80). */
typedef struct fh_gguf_tensor {
    const char *name; /* not NUL-terminated */
    size_t name_len;
    uint32_t n_dims;  /* 1 to 4 */
    uint64_t dims[4]; /* ggml order: dims[0] is contiguous */
    uint32_t ggml_type;
    uint64_t offset;   /* from the start of the data section */
    uint64_t elements;
    uint64_t nbytes;
} fh_gguf_tensor;
FH_API size_t fh_gguf_tensor_count(const fh_gguf *g);
FH_API fh_status fh_gguf_tensor_info(const fh_gguf *g, size_t i, fh_gguf_tensor *out);
/* Gguf::tensor (reader.rs:289-291): "missing tensor" when absent. */
FH_API fh_status fh_gguf_find_tensor(const fh_gguf *g, const char *name, size_t *index);
/* Gguf::tensor_bytes (reader.rs:294-305): the stored bytes, undecoded. */
FH_API fh_status fh_gguf_tensor_bytes(const fh_gguf *g, const char *name, const uint8_t **data,
                                      size_t *len);
/* Gguf::data_offset (reader.rs:308-310). */
FH_API uint64_t fh_gguf_data_offset(const fh_gguf *g);

/* No dequantise/requantise round trip: a Q8_0 or Q4_0 tensor of ggml dims [k, n...] becomes a
 * resident weight of k inputs and n = dims[1]*...*dims[nd-1] outputs straight from its stored
 * bytes (the rows are the weight's GGUF rows). Replaces the load-time re-encode the reference's
 * GGUF loaders perform (ferrum_model/src/gguf/quant.rs:57-69 into ops_quant::upload_quantised). */
FH_API fh_status fh_gguf_upload_qweight(fh_device *dev, const fh_gguf *g, const char *name,
                                        fh_qweight **out);
/* Gguf::tensor_f32 (reader.rs:313-318) onto the device: the tensor decoded to f32 in GGUF order
 * (dims[0] contiguous) in a new buffer. F32 is copied; F16, Q8_0 and Q4_0 are decoded by the
 * device codec. Other types: FH_ERR_UNSUPPORTED. */
FH_API fh_status fh_gguf_upload_f32(fh_device *dev, const fh_gguf *g, const char *name, fh_buffer **out);

/* ---- GPT-2 KV-cached decode on resident Q8_0 / Q4_0 weights ----
 * Replaces ferrum_wgpu::models::gpt2::GpuGpt2 (ferrum_wgpu/src/models/gpt2.rs:52-265: new, feed,
 * reset, pos), whose weights are f32; here every matrix stays packed. The model comes from a
 * `gpt2` GGUF laid out as ferrum_model writes it (ferrum_model/src/gguf/gpt2.rs:179-233): Q8_0 or
 * Q4_0 matrices (one format per model), F32 vectors, `output.weight` absent for a head tied to
 * `token_embd.weight`. Its CPU counterpart is ferrum_ref's Gpt2::feed on the fake-quantised
 * weights (ferrum_ref/src/models/gpt2/decode.rs:57-117). One step is one HIP graph launch
 * (FERRUM_HIP_NO_GRAPH=1: plain launches); the position lives on the device. */
typedef struct fh_gpt2 fh_gpt2;
FH_API fh_status fh_gpt2_from_gguf(fh_device *dev, const fh_gguf *g, fh_gpt2 **out);
FH_API void fh_gpt2_free(fh_gpt2 *m);
/* Config (ferrum_ref/src/models/gpt2/mod.rs:16-31); any pointer may be NULL. */
FH_API fh_status fh_gpt2_config(const fh_gpt2 *m, size_t *vocab, size_t *ctx, size_t *dim, size_t *heads,
                                size_t *layers, size_t *hidden);
FH_API fh_kind fh_gpt2_kind(const fh_gpt2 *m);
/* GpuGpt2::pos / reset (gpt2.rs:205-213). */
FH_API size_t fh_gpt2_pos(const fh_gpt2 *m);
FH_API void fh_gpt2_reset(fh_gpt2 *m);
/* Packed weight bytes one step reads (every matrix and the head). */
FH_API uint64_t fh_gpt2_step_bytes(const fh_gpt2 *m);
/* Kernel launches in one step (no counterpart in the reference): 4 per layer + 3 where the head
 * width is 64, 128 or 256 (FERRUM_HIP_DECODE_STEP=5 at load keeps the five-launch form), else 5 per
 * layer + 4. */
FH_API size_t fh_gpt2_step_launches(const fh_gpt2 *m);
/* GpuGpt2::feed (gpt2.rs:216-265): consume `token` at the next position; when logits is not NULL
 * it receives the vocab next-token logits (and the call waits for them). Errors: "context of N
 * tokens is full", "token T is out of range for vocab V". */
FH_API fh_status fh_gpt2_feed(fh_device *dev, fh_gpt2 *m, size_t token, float *logits);
/* Greedy generation from the current position: feed the prompt, then pick n_new tokens by argmax
 * (ferrum_model/src/sampling.rs:32-40), each fed back except the last (the reference's generate
 * loop, ferrum_gpu_core/src/engine/mod.rs:204-242). Picks stay on the device; out receives them
 * at the end, after the only wait. */
FH_API fh_status fh_gpt2_generate(fh_device *dev, fh_gpt2 *m, const int32_t *prompt, size_t n_prompt,
                                  size_t n_new, int32_t *out);

/* ---- Llama / Qwen2 full-sequence forward and scoring on resident Q8_0 / Q4_0 weights ----
 * Replaces the batched passes of ferrum_wgpu::models::llama::GpuLlama (ferrum_wgpu/src/models/
 * llama/forward.rs:13-88: forward_all, score). The model comes from a `llama` (NORM RoPE) or
 * `qwen2` (NEOX RoPE) GGUF as ferrum_model reads and writes it (ferrum_model/src/gguf/llama/
 * mod.rs:56-323): Q8_0 or Q4_0 matrices (one format per model) stay packed; a matrix stored in
 * another type, as the writer stores one whose width is not whole 32-blocks (F32), is decoded to
 * f32 rows and multiplied as f32 (Lin::upload, ferrum_wgpu/src/models/llama/lin.rs:30-62); F32
 * vectors, optional q/k/v biases, `output.weight` absent for a head tied to `token_embd.weight`,
 * linear / rope_freqs RoPE scaling.
 * Its CPU counterpart is ferrum_ref's Llama::forward_logits on the decoded weights
 * (ferrum_ref/src/models/llama/mod.rs:166-259) and nn::score (ferrum_ref/src/kernels/nn.rs:117-129).
 * `path` picks the products: FH_PATH_TILED (or AUTO) the precise MFMA GEMM, FH_PATH_TILED_FAST
 * the scoring GEMM (x as f16 + an fp8 correction) or FH_PATH_TILED_F16 the dequant-f16 GEMM; their
 * error bounds are those fh_path states. */
typedef struct fh_llama fh_llama;
typedef struct fh_llama_cfg {
    size_t vocab, ctx, dim, heads, kv_heads, head_dim, layers, hidden, rope_dim;
    float rope_base, eps, linear_factor;
    int neox, tied;
    fh_kind kind;
    fh_path path;
} fh_llama_cfg;
FH_API fh_status fh_llama_from_gguf(fh_device *dev, const fh_gguf *g, fh_path path, fh_llama **out);
FH_API void fh_llama_free(fh_llama *m);
/* Config (ferrum_ref/src/models/llama/mod.rs:24-51) and how the model is stored. */
FH_API fh_status fh_llama_config(const fh_llama *m, fh_llama_cfg *out);
/* Weight bytes one forward reads (every block matrix and the head: GGUF sizes when packed, 4 per
 * weight when f32). */
FH_API uint64_t fh_llama_weight_bytes(const fh_llama *m);
/* Device memory the model holds: every weight's device_bytes (the tied head once), the vectors,
 * the RoPE tables and the activation arena at its current size (no counterpart in the reference,
 * whose GpuLlama keeps f32 weights). */
FH_API uint64_t fh_llama_device_bytes(const fh_llama *m);
/* GpuLlama::forward_all (forward.rs:13-73): every position's logits of ids[0..n), [n, vocab]
 * row-major into host memory. Errors: "sequence length N must be in 1..=ctx", "token T is out of
 * range for vocab V". */
FH_API fh_status fh_llama_forward_all(fh_device *dev, fh_llama *m, const int32_t *ids, size_t n, float *logits);
/* GpuLlama::score (forward.rs:76-88): for each i < n - 1 the log-probability of ids[i + 1] after
 * ids[..=i] and whether it is the first argmax; only 2 (n - 1) floats leave the device. Errors:
 * "scoring needs at least 2 tokens" and those of forward_all. */
FH_API fh_status fh_llama_score(fh_device *dev, fh_llama *m, const int32_t *ids, size_t n, float *logprob,
                                uint8_t *is_first_max);
/* The same pass on device-resident ids (n int32 values) into out (2 (n - 1) floats: log-probability,
 * then 1.0 for a first argmax else 0.0, per row, as ops::score writes them, ferrum_wgpu/src/ops/
 * mod.rs:157-175). Asynchronous on the device's stream. The ids are not read on the host: one
 * outside the vocabulary is never read past, but it turns its row and the rows after it to NaN. */
FH_API fh_status fh_llama_score_device(fh_device *dev, fh_llama *m, const fh_buffer *ids, size_t n, fh_buffer *out);

#ifdef __cplusplus
}
#endif
#endif
