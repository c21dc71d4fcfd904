// Internal declarations shared by the runtime and the kernel files of libferrum_hip.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ferrum_hip.h"

// A device lives until fh_device_close AND the last buffer, weight and plan made on it are
// freed: each of those holds a reference (the reference shares Gpu through Arc, engine/gpu.rs:18-22),
// so freeing a buffer after its device was closed is safe.
struct fh_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    int cus = 0;
    std::string name;
    std::atomic<int64_t> fail_after{-1};
    std::atomic<uint64_t> commands{0};
    std::atomic<bool> lost{false};
    std::atomic<bool> closed{false};
    std::atomic<int64_t> refs{1};  // the opener's reference, dropped by fh_device_close
    // Scratch device memory some launches need (the GEMM's split x), grown on demand and kept
    // until the device goes away. Commands on the one stream use it in order.
    std::mutex ws_mu;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // This GPU's copy of the no-allocation entry point's static scratch array (its device
    // address, taken when the device is opened).
    void *scratch = nullptr;
};

struct fh_buffer {
    fh_device *dev = nullptr;
    void *ptr = nullptr;
    size_t nbytes = 0;
};

// A resident quantized weight of k inputs and n outputs (n GGUF rows of nb = k/32 blocks),
// repacked at upload into two planes holding the GGUF bytes as tiles (see tile_slot and
// scale_slot in device_common.hpp): the quants (QB = 16 Q4_0 / 32 Q8_0 bytes per block, the
// block without its scale) and the f16 scales. Rows are padded to a multiple of 32 with zero
// blocks.
struct fh_qweight {
    fh_device *dev = nullptr;
    fh_kind kind = FH_Q8_0;
    size_t k = 0, n = 0;
    uint8_t *ptr = nullptr;   // the allocation: quant plane, then scale plane
    uint8_t *qs = nullptr;    // quant plane (256-byte aligned)
    uint16_t *ds = nullptr;   // scale plane
    size_t nbytes = 0;        // exact GGUF byte count of the weight
    size_t alloc = 0;         // bytes of the allocation (the padded planes)
    // The MFMA GEMM's fp8 correction operand (e4m3 of d * q per element, per-row power-of-two
    // scales; gemm_b8_bytes), built on the weight's first multi-row product and freed with it.
    mutable uint8_t *b8 = nullptr;
};

namespace fh {

constexpr size_t QK = 32;
// Every device allocation is padded so kernels may read a dword window that runs up to a few
// bytes past the last block (the 34- and 18-byte blocks are only 2-byte aligned).
constexpr size_t kPad = 256;

inline size_t block_bytes(fh_kind k) { return k == FH_Q8_0 ? 34 : 18; }
inline size_t quant_bytes(fh_kind k) { return k == FH_Q8_0 ? 32 : 16; }
// Quant slots of a weight of n rows and nb blocks per row (rows padded to a multiple of 32).
inline size_t tile_slots(size_t n, size_t nb) { return (n + 31) / 32 * 32 * nb; }
// Scale-plane elements of the same weight (blocks padded to a multiple of 8).
inline size_t scale_slots(size_t n, size_t nb) { return (n + 31) / 32 * 32 * ((nb + 7) / 8 * 8); }
// Offset of the scale plane inside a weight allocation of `slots` quant slots.
inline size_t scale_plane_offset(fh_kind k, size_t slots) {
    return (slots * quant_bytes(k) + 255) / 256 * 256;
}
inline bool kind_ok(int k) { return k == FH_Q8_0 || k == FH_Q4_0; }

// Thread-local error text; returns the status for `return fail(...)`.
fh_status fail(fh_status st, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Account for one command about to be issued on dev: reports a lost device or an armed
// injected fault, and counts the command (device/runtime.rs:218-256 semantics).
fh_status begin_command(fh_device *dev, const char *what);
// Check the launch that was just issued; a launch error marks the device lost.
fh_status end_command(fh_device *dev, const char *what);
// Map a HIP error to a status and message; illegal-address style errors make dev lost.
fh_status hip_fail(fh_device *dev, hipError_t e, const char *what);

fh_status alloc_bytes(fh_device *dev, size_t nbytes, void **out);

// A usable device: open, not closed, not lost; makes it the current HIP device.
fh_status check_dev(fh_device *dev);

// The device's workspace, at least `bytes` long (grown after the stream drains).
fh_status workspace(fh_device *dev, size_t bytes, void **out);

// Reference counting of devices (see struct fh_device).
void dev_retain(fh_device *dev);
void dev_release(fh_device *dev);  // destroys the stream and the device on the last release

// ---- model loading from GGUF (gguf.cpp); `who` prefixes the error messages ----
std::string tensor_name(const char *base, size_t layer, const char *suffix);
fh_status cfg_uint(const fh_gguf *g, const char *key, size_t *out);
// An F32 vector of exactly `len` values, copied out of the file's bytes.
fh_status host_vec(const fh_gguf *g, const char *who, const std::string &name, size_t len, std::vector<float> *out);
fh_status load_vec(fh_device *dev, const fh_gguf *g, const char *who, const std::string &name, size_t len,
                   fh_buffer **out);
// A Q8_0/Q4_0 matrix of GGML dims [k, n] as a resident weight; *kind is the model's one block
// format (0: taken from this tensor).
fh_status load_mat(fh_device *dev, const fh_gguf *g, const char *who, const std::string &name, size_t k, size_t n,
                   fh_kind *kind, fh_qweight **out);
// Several matrices of k inputs stacked into one weight: the rows of names[0] (ns[0] of them),
// then those of names[1], ... (a fused projection). interleave (two parts of equal rows, a multiple
// of 32): runs of 32 rows alternate between the parts instead (gemm_kernel's SwiGLU epilogue).
fh_status load_mat_rows(fh_device *dev, const fh_gguf *g, const char *who, const std::string *names,
                        const size_t *ns, size_t count, size_t k, fh_kind *kind, fh_qweight **out,
                        bool interleave = false);

// ---- kernel launchers (on dev->stream; a command may issue several) ----
// codec.hip
hipError_t launch_encode_rows(hipStream_t s, fh_kind kind, const float *src, uint8_t *dst,
                              size_t nblocks);
hipError_t launch_decode_rows(hipStream_t s, fh_kind kind, const uint8_t *src, float *dst,
                              size_t nblocks);
// quantise_matrix into planes / dequantise planes back to the [k, n] f32 weight
hipError_t launch_encode_cols(hipStream_t s, fh_kind kind, const float *w, uint8_t *qs, uint16_t *ds,
                              size_t k, size_t n);
hipError_t launch_decode_cols(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, float *w,
                              size_t k, size_t n);
hipError_t launch_snap_rows(hipStream_t s, const float *src, float *dst, size_t nblocks);
// A grouped snap pass: one descriptor per problem (mode FH_SNAP_ROWS / COLS / COPY after the
// host's fallbacks), task0 = its first wavefront task; tasks = the launch's total.
struct SnapDesc {
    const float *src;
    float *dst;
    uint64_t len;  // floats
    uint32_t k, n;  // COLS: rows_in, cols_out
    uint32_t mode, task0;
};
uint32_t snap_tasks(const SnapDesc &d);
hipError_t launch_snap_group(hipStream_t s, const SnapDesc *descs, uint32_t count, uint32_t tasks, int cus);
hipError_t launch_snap_cols(hipStream_t s, const float *src, float *dst, size_t rows_in,
                            size_t cols_out);
hipError_t launch_copy_f32(hipStream_t s, const float *src, float *dst, size_t n);
hipError_t launch_decode_f16(hipStream_t s, const uint16_t *src, float *dst, size_t n);

// GGUF rows (n rows of nb blocks) <-> tiled planes (upload_qweight and read_gguf)
hipError_t launch_gguf_to_planes(hipStream_t s, fh_kind kind, const uint8_t *src, uint8_t *qs,
                                 uint16_t *ds, size_t n, size_t nb);
hipError_t launch_planes_to_gguf(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds,
                                 uint8_t *dst, size_t n, size_t nb);

// formats.hip: F16, MXFP4, FP8 E4M3 / E5M2, Q2_K weights (GGUF rows, decoded on the fly) and the
// read-only block types (decode)
bool ext_kind(int kind);                                               // a weight format of formats.hip
bool ext_layout(uint32_t ty, size_t *block_bytes, size_t *block_elems);  // any type formats.hip decodes
const char *ext_label(int kind);
hipError_t launch_decode_ext(hipStream_t s, uint32_t ty, const uint8_t *src, float *dst, size_t n);
hipError_t launch_encode_ext(hipStream_t s, int kind, const float *src, uint8_t *dst, size_t n);
hipError_t launch_transpose(hipStream_t s, const float *src, float *dst, size_t rows, size_t cols);
hipError_t launch_linear_ext(hipStream_t s, int kind, fh_path path, const uint8_t *w, const float *x, float *y,
                             size_t rows, size_t k, size_t n);

// gemv.hip
struct GemvDesc {          // one batch-1 product, as the kernels read it
    const uint8_t *qs;     // quant plane
    const uint16_t *ds;    // scale plane
    const float *x;
    float *y;
    uint8_t *prep;         // gemv_prep_bytes(k) bytes of prepared x
    uint32_t nb;           // blocks per row (k / 32)
    uint32_t n;            // rows (outputs)
    uint32_t task0;        // first task (group of 32 rows) of this product in its launch
    uint32_t pad;
};
// A single batch-1 product on the decode GEMV's kernel (decode.hip: one workgroup per 32 rows,
// its wavefronts splitting the row's blocks, x prepared in LDS by every workgroup): a lower
// latency than launch_gemv when the product's row groups alone leave the chip underfilled
// (gemv_latency_fits). decode_lds_limits raises the decode kernels' LDS limit (once per process,
// before any graph capture).
hipError_t decode_lds_limits();
bool gemv_latency_fits(size_t k, size_t n, int cus);
hipError_t launch_gemv_latency(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                               float *y, size_t k, size_t n);
// Widest product (in 32-blocks) whose prepared x the GEMV keeps in a wavefront's LDS region.
constexpr uint32_t kGemvLdsBlocks = 112;
// Whether the kernel's 32-bit offsets cover rows of k inputs (k a multiple of 32, up to 2^25).
bool gemv_supported(fh_kind kind, size_t k, size_t n);
size_t gemv_prep_bytes(size_t k);
uint32_t gemv_tasks(size_t n);
// Two launches: prepare x into `prep` (gemv_prep_bytes(k) bytes), then the product.
hipError_t launch_gemv(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                       float *y, size_t k, size_t n, void *prep, int cus);
// Many products of one format: `descs` (device memory) in task order with task0 prefix sums,
// `map` (device memory) the product of each of the `tasks` tasks, max_nb the widest product's
// block count.
// Products of another launch of the same plan (descs, count, their widest nb) whose prepared x a
// launch may write for it: fused into its product kernel when that one prepares its own x in
// LDS, else into its preparation kernel when their descriptors follow its own.
struct GemvPrep {
    const GemvDesc *descs;
    uint32_t count, max_nb;
};
hipError_t launch_gemv_group(hipStream_t s, fh_kind kind, const GemvDesc *descs, const uint32_t *map,
                             uint32_t count, uint32_t tasks, uint32_t max_nb, int cus, const GemvPrep &other,
                             bool skip_prep, bool *other_done);

// rows.hip: few-row products (2 <= rows <= kRowsMax)
constexpr size_t kRowsMax = 64;
struct RowsDesc {          // one few-row product, as the kernels read it
    const uint8_t *qs;     // quant plane
    const uint16_t *ds;    // scale plane
    const float *x;        // rows x k
    _Float16 *xs;          // rows_xsplit_bytes(rows, k) bytes: x split into f16 parts
    float *y;              // rows x n
    uint32_t nb;           // blocks per row (k / 32)
    uint32_t n;            // outputs per row
    uint32_t m;            // rows
    uint32_t task0;        // first task of this product in its launch (rows_tasks)
};
bool rows_supported(size_t rows, size_t k, size_t n);
size_t rows_xsplit_bytes(size_t rows, size_t k);
// Tasks of a product of k inputs and n outputs in a launch whose products have at most max_m rows.
uint32_t rows_tasks(size_t n, size_t k, size_t max_m);
// Two launches: split x into `xsplit`, then the product.
hipError_t launch_rows(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x, float *y,
                       size_t rows, size_t k, size_t n, void *xsplit, int cus);
// Many products of one format: descs and map (device memory) as for launch_gemv_group; max_m the
// most rows of any product, max_items the largest rows * k / 32.
hipError_t launch_rows_group(hipStream_t s, fh_kind kind, const RowsDesc *descs, const uint32_t *map, uint32_t count,
                             uint32_t tasks, uint32_t max_m, uint32_t max_items, int cus);

// A K-split product left unreduced for its consumer: y(r, c) = the sum over s < splits of
// part[s * rows * n + r * n + c], added in split order (the reduction kernel's order, so a
// consumer that sums them reproduces the reduced product bit for bit). splits == 1: part is y.
struct SplitOut {
    float *part;
    uint32_t splits;
};

// gemm.hip
hipError_t launch_naive(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                        float *y, size_t rows, size_t k, size_t n);
// The fast MFMA GEMM (two launches: split x into workspace, then the product); workspace holds
// gemm_workspace_bytes(rows, k) bytes, b8 the weight's correction operand (launch_make_b8).
// The workspace is the split x (gemm_xsplit_bytes) followed by the K-split partial products
// (gemm_partial_bytes).
size_t gemm_workspace_bytes(size_t rows, size_t k, size_t n);
size_t gemm_xsplit_bytes(size_t rows, size_t k);
size_t gemm_partial_bytes(size_t rows, size_t k, size_t n);
size_t gemm_b8_bytes(size_t k, size_t n);
// Whether the GEMM's 32-bit buffer offsets cover rows x (k, n) (every operand under 2^31 bytes).
bool gemm_supported(size_t rows, size_t k, size_t n);
hipError_t launch_make_b8(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, uint8_t *b8, size_t k,
                          size_t n);
// Where the fast GEMM's split x lives (gemm_x_split: at the start of its workspace): hi (rows x k
// f16), lo (rows x k rounded up to 64, e4m3), the scale bytes (two per row and 64 k); the layouts
// are in xsplit.hpp.
struct GemmXSplit {
    _Float16 *xh;
    uint8_t *xl;
    uint8_t *xsb;
};
GemmXSplit gemm_x_split(void *workspace, size_t rows, size_t k);
// x == nullptr: x is already in the split form (written by split_row_fast or split_chunk4 in
// xsplit.hpp), in the workspace or, when xs is given, at xs. partial != nullptr: the K-split
// partial products go there (gemm_partial_bytes) instead of after the split x, so that a consumer
// of deferred partial sums can write the next product's split x (of another width) while it reads
// them.
hipError_t launch_gemm(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const uint8_t *b8,
                       const float *x, float *y, size_t rows, size_t k, size_t n, void *workspace,
                       SplitOut *defer = nullptr, float *partial = nullptr, const GemmXSplit *xs = nullptr);
// The fast GEMM with SwiGLU fused into its epilogue: the weight's n rows are gate and up
// interleaved in runs of 32 (load_mat_rows with interleave); the rows x n / 2 activations
// (swiglu_act) are written as the down product's split x at act (gemm_xsplit_bytes(rows, n / 2)
// bytes, apart from the workspace). Only where gemm_swiglu_supported; x null: the split x is
// already in the workspace.
bool gemm_swiglu_supported(size_t rows, size_t k, size_t n);
hipError_t launch_gemm_swiglu(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const uint8_t *b8,
                              const float *x, const GemmXSplit &act, size_t rows, size_t k, size_t n,
                              void *workspace);
// The dequant-f16 MFMA GEMM (x as f16 with a power-of-two row scale, weights dequantised to f16
// in LDS; split into workspace, then the product).
size_t gemm_f16_workspace_bytes(size_t rows, size_t k, size_t n);
bool gemm_f16_supported(size_t rows, size_t k, size_t n);
hipError_t launch_gemm_f16(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x, float *y,
                           size_t rows, size_t k, size_t n, void *workspace, SplitOut *defer = nullptr);
// The precise MFMA GEMM (x as two f16 parts; split into workspace, then the product).
size_t gemm_precise_workspace_bytes(size_t rows, size_t k, size_t n);
// The MFMA GEMM on the GGUF rows of F16, FP8 E4M3 / E5M2, MXFP4 and Q2_K weights (rows >= 2) and
// its workspace (x split, then the K-split partial products).
bool gemm_ext_kind(int kind);
size_t gemm_ext_workspace_bytes(int kind, size_t rows, size_t k, size_t n);
hipError_t launch_gemm_ext(hipStream_t s, int kind, const uint8_t *w, const float *x, float *y, size_t rows, size_t k,
                           size_t n, void *workspace);
hipError_t launch_gemm_precise(hipStream_t s, fh_kind kind, const uint8_t *qs, const uint16_t *ds, const float *x,
                               float *y, size_t rows, size_t k, size_t n, void *workspace,
                               SplitOut *defer = nullptr);

// The scoring head's product with the score folded into its epilogue: no logits are written;
// per row and 256-column tile the tile's softmax statistics (maximum, sum of exp(v - maximum),
// first column holding the maximum), and the target column's logit from the tile holding it.
struct ScoreOut {
    const int32_t *tgt;  // the target column of every row, rows padded to a multiple of 256
    float *part;         // [rows][ntn][4]: maximum, sum, first column (as bits), 0
    float *tlogit;       // [rows]
    uint32_t ntn;        // column tiles: ceil(n / 256)
};
// Whether the score epilogue takes this product (the streaming 256 x 256 kernels' limits); path
// FH_PATH_TILED_FAST or FH_PATH_TILED. b8: the fast path's correction operand.
bool gemm_score_supported(fh_path path, size_t rows, size_t k, size_t n);
hipError_t launch_gemm_score(hipStream_t s, fh_path path, fh_kind kind, const uint8_t *qs, const uint16_t *ds,
                             const uint8_t *b8, const float *x, size_t rows, size_t k, size_t n, void *workspace,
                             const ScoreOut &so);

}  // namespace fh
