// Runtime of libferrum_hip: devices, buffers, resident quantized weights, argument checks,
// kernel choice and the C ABI declared in include/ferrum_hip.h. Kernels live in codec.hip,
// gemv.hip and gemm.hip; this file only validates, accounts and launches.
#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <new>
#include <utility>
#include <vector>

#include "internal.hpp"

// Scratch of the no-allocation entry point (fh_linear_q_noalloc): one array per GPU, made when
// the library's code object loads on that GPU and held until the process ends. Host code never
// uses this name as an address: fh_device_open takes this GPU's device address of it with
// hipGetSymbolAddress, and every launch gets that pointer.
static __device__ __align__(256) uint8_t scratch[FH_NOALLOC_SCRATCH_BYTES];

namespace fh {

static thread_local std::string g_err;

fh_status fail(fh_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return st;
}

// Byte ranges [a, a + an) and [b, b + bn) share a byte.
static bool overlaps(const void *a, size_t an, const void *b, size_t bn) {
    const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    return an && bn && a0 < b0 + bn && b0 < a0 + an;
}

// Grouped launches read every product's x while they write (and, for the few-row kernel, first
// zero) every product's y, so no x may overlap any y and no two y may overlap. `xs` and `ys` are
// (address, bytes) per product; returns the product whose range collides, or -1.
static long plan_overlap(const std::vector<std::pair<uintptr_t, size_t>> &xs,
                         std::vector<std::pair<uintptr_t, size_t>> ys) {
    std::vector<size_t> order(ys.size());
    for (size_t i = 0; i < order.size(); i++) order[i] = i;
    std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return ys[a].first < ys[b].first; });
    for (size_t i = 1; i < order.size(); i++) {
        const auto &p = ys[order[i - 1]], &q = ys[order[i]];
        if (p.second && q.second && q.first < p.first + p.second) return (long)order[i];
    }
    for (size_t j = 0; j < xs.size(); j++) {
        const uintptr_t x0 = xs[j].first, x1 = xs[j].first + xs[j].second;
        // the y range starting last before x's end is the only one that can reach into x
        size_t lo = 0, hi = order.size();
        while (lo < hi) {
            const size_t mid = (lo + hi) / 2;
            if (ys[order[mid]].first < x1) lo = mid + 1;
            else hi = mid;
        }
        if (lo > 0) {
            const auto &y = ys[order[lo - 1]];
            if (xs[j].second && y.second && y.first + y.second > x0) return (long)j;
        }
    }
    return -1;
}

// Calls of fh_linear_q_noalloc on one GPU share its one scratch array whichever handle (stream)
// they come through: each call waits for the previous call's work on that GPU (an event per GPU,
// made when a handle is opened, recorded after each call), so calls through different handles of
// one GPU do not race on it. Under stream capture no cross-stream wait is recorded (the caller
// orders the captured work); the event is left alone.
struct NoallocOrder {
    std::mutex mu;
    hipEvent_t ev = nullptr;
    bool recorded = false;
};
static constexpr int kMaxOrdinals = 64;
static NoallocOrder g_noalloc[kMaxOrdinals];

static bool is_fatal(hipError_t e) {
    switch (e) {
    case hipErrorIllegalAddress:
    case hipErrorLaunchFailure:
    case hipErrorLaunchTimeOut:
    case hipErrorAssert:
    case hipErrorUnknown:
        return true;
    default:
        return false;
    }
}

fh_status hip_fail(fh_device *dev, hipError_t e, const char *what) {
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return fail(FH_ERR_OOM, "%s: GPU out of memory", what);
    if (dev && is_fatal(e)) {
        dev->lost.store(true);
        return fail(FH_ERR_LOST, "%s: device lost: %s", what, hipGetErrorString(e));
    }
    return fail(FH_ERR_DEVICE, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

fh_status begin_command(fh_device *dev, const char *what) {
    if (dev->lost.load()) return fail(FH_ERR_LOST, "%s: the device was lost earlier", what);
    int64_t n = dev->fail_after.load();
    if (n == 0) return fail(FH_ERR_INJECTED, "%s: injected fault", what);
    if (n > 0) dev->fail_after.store(n - 1);
    dev->commands.fetch_add(1);
    return FH_OK;
}

fh_status end_command(fh_device *dev, const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(dev, e, what);
    return FH_OK;
}

void dev_retain(fh_device *dev) { dev->refs.fetch_add(1); }

void dev_release(fh_device *dev) {
    if (dev->refs.fetch_sub(1) != 1) return;
    (void)hipSetDevice(dev->ordinal);
    (void)hipStreamSynchronize(dev->stream);
    if (dev->ws) (void)hipFree(dev->ws);
    (void)hipStreamDestroy(dev->stream);
    delete dev;
}

// Free device memory made by alloc_bytes once no queued command can still use it.
static void free_bytes(fh_device *dev, void *p) {
    (void)hipSetDevice(dev->ordinal);
    (void)hipStreamSynchronize(dev->stream);
    (void)hipFree(p);
}

fh_status workspace(fh_device *dev, size_t bytes, void **out) {
    std::lock_guard<std::mutex> lock(dev->ws_mu);
    if (bytes > dev->ws_bytes) {
        if (dev->ws) {
            free_bytes(dev, dev->ws);  // waits for the commands still using it
            dev->ws = nullptr;
            dev->ws_bytes = 0;
        }
        void *p = nullptr;
        const size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
        hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return hip_fail(dev, e, "workspace");
        }
        dev->ws = p;
        dev->ws_bytes = want;
    }
    *out = dev->ws;
    return FH_OK;
}

fh_status alloc_bytes(fh_device *dev, size_t nbytes, void **out) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, nbytes + kPad);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(dev, e, "allocate");
    }
    e = hipMemsetAsync(p, 0, nbytes + kPad, dev->stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(dev, e, "allocate");
    }
    *out = p;
    return FH_OK;
}

}  // namespace fh

using namespace fh;

fh_status fh::check_dev(fh_device *dev) {
    if (!dev) return fail(FH_ERR_INVALID, "no device");
    if (dev->closed.load()) return fail(FH_ERR_INVALID, "the device was closed");
    if (dev->lost.load()) return fail(FH_ERR_LOST, "the device was lost earlier");
    hipError_t e = hipSetDevice(dev->ordinal);
    if (e != hipSuccess) return hip_fail(dev, e, "select device");
    return FH_OK;
}

namespace {

fh_status sync(fh_device *dev, const char *what) {
    hipError_t e = hipStreamSynchronize(dev->stream);
    if (e != hipSuccess) return hip_fail(dev, e, what);
    return FH_OK;
}

fh_status new_buffer(fh_device *dev, size_t nbytes, fh_buffer **out) {
    void *p = nullptr;
    fh_status st = alloc_bytes(dev, nbytes, &p);
    if (st) return st;
    fh_buffer *b = new (std::nothrow) fh_buffer;
    if (!b) {
        (void)hipFree(p);
        return fail(FH_ERR_OOM, "host out of memory");
    }
    dev_retain(dev);
    b->dev = dev;
    b->ptr = p;
    b->nbytes = nbytes;
    *out = b;
    return FH_OK;
}

fh_status upload_bytes(fh_device *dev, void *dst, const void *src, size_t nbytes, const char *w) {
    if (nbytes == 0) return FH_OK;
    fh_status st = begin_command(dev, w);
    if (st) return st;
    hipError_t e = hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, dev->stream);
    if (e != hipSuccess) return hip_fail(dev, e, w);
    return sync(dev, w);  // the host memory may be reused as soon as this returns
}

fh_status read_bytes(fh_device *dev, void *dst, const void *src, size_t nbytes, const char *w) {
    fh_status st = begin_command(dev, w);
    if (st) return st;
    if (nbytes) {
        hipError_t e = hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, dev->stream);
        if (e != hipSuccess) return hip_fail(dev, e, w);
    }
    return sync(dev, w);
}

fh_status need(const char *name, const fh_buffer *b, size_t want) {
    if (!b) return fail(FH_ERR_INVALID, "%s: no buffer", name);
    size_t have = b->nbytes / 4;
    if (have != want)
        return fail(FH_ERR_INVALID, "%s: buffer holds %zu elements, expected %zu", name, have, want);
    return FH_OK;
}

// A weight of a formats.hip kind: its GGUF rows as they are.
fh_status new_ext_qweight(fh_device *dev, fh_kind kind, size_t k, size_t n, fh_qweight **out) {
    size_t bb, be;
    ext_layout(kind, &bb, &be);
    if (k == 0 || k % be)
        return fail(FH_ERR_INVALID, "a %zu x %zu weight is not whole %zu-element blocks", k, n, be);
    if (n == 0 || n > (1u << 30) || k > (1u << 30) || (k / be) * n > (1ull << 32))
        return fail(FH_ERR_INVALID, "a %zu x %zu weight is out of range", k, n);
    const size_t nbytes = (k / be) * n * bb;
    void *p = nullptr;
    fh_status st = alloc_bytes(dev, nbytes, &p);
    if (st) return st;
    fh_qweight *w = new (std::nothrow) fh_qweight;
    if (!w) {
        (void)hipFree(p);
        return fail(FH_ERR_OOM, "host out of memory");
    }
    dev_retain(dev);
    w->dev = dev;
    w->kind = kind;
    w->k = k;
    w->n = n;
    w->ptr = (uint8_t *)p;
    w->qs = (uint8_t *)p;
    w->ds = nullptr;
    w->nbytes = nbytes;
    w->alloc = nbytes;
    *out = w;
    return FH_OK;
}

fh_status new_qweight(fh_device *dev, fh_kind kind, size_t k, size_t n, fh_qweight **out) {
    if (ext_kind(kind)) return new_ext_qweight(dev, kind, k, n, out);
    if (!kind_ok(kind)) return fail(FH_ERR_UNSUPPORTED, "unsupported block format %d", (int)kind);
    if (k == 0 || k % QK)
        return fail(FH_ERR_INVALID, "a %zu x %zu weight is not whole 32-element blocks", k, n);
    if (n == 0 || n > (1u << 30) || k > (1u << 30) || (k / QK) * n > (1ull << 32))
        return fail(FH_ERR_INVALID, "a %zu x %zu weight is out of range", k, n);
    const size_t slots = tile_slots(n, k / QK);
    size_t nbytes = (k / QK) * n * block_bytes(kind);
    const size_t alloc = scale_plane_offset(kind, slots) + scale_slots(n, k / QK) * 2;
    void *p = nullptr;
    fh_status st = alloc_bytes(dev, alloc, &p);
    if (st) return st;
    fh_qweight *w = new (std::nothrow) fh_qweight;
    if (!w) {
        (void)hipFree(p);
        return fail(FH_ERR_OOM, "host out of memory");
    }
    dev_retain(dev);
    w->dev = dev;
    w->kind = kind;
    w->k = k;
    w->n = n;
    w->ptr = (uint8_t *)p;
    w->qs = (uint8_t *)p;
    w->ds = (uint16_t *)((uint8_t *)p + scale_plane_offset(kind, slots));
    w->nbytes = nbytes;
    w->alloc = alloc;
    *out = w;
    return FH_OK;
}

}  // namespace

struct fh_gemv_plan {
    fh_device *dev = nullptr;
    struct Launch {
        fh_kind kind;
        size_t first, count;  // descriptors
        size_t map0;          // first entry of the launch's task -> product map
        uint32_t tasks, max_nb;
        bool narrow;          // every product's x fits the kernel's LDS region
        bool prepared;        // the previous (narrow) launch of its format writes its prepared x
    };
    std::vector<Launch> launches;
    GemvDesc *descs = nullptr;  // device array
    uint32_t *map = nullptr;    // device array: per launch, the product of each task
    uint8_t *prep = nullptr;    // prepared x of every product
    uint64_t bytes = 0;
};

extern "C" {

const char *fh_last_error(void) { return g_err.c_str(); }
int fh_abi_version(void) { return FH_ABI_VERSION; }

fh_status fh_device_open(int ordinal, fh_device **out) {
    if (!out) return fail(FH_ERR_INVALID, "fh_device_open: null out");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) {
        (void)hipGetLastError();
        return fail(FH_ERR_DEVICE, "no HIP device available");
    }
    if (ordinal < 0 || ordinal >= count)
        return fail(FH_ERR_INVALID, "device %d does not exist (%d present)", ordinal, count);
    if ((e = hipSetDevice(ordinal)) != hipSuccess) return hip_fail(nullptr, e, "select device");
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, ordinal)) != hipSuccess)
        return hip_fail(nullptr, e, "device properties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(FH_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950",
                    ordinal, prop.gcnArchName);
    fh_device *d = new (std::nothrow) fh_device;
    if (!d) return fail(FH_ERR_OOM, "host out of memory");
    d->ordinal = ordinal;
    d->cus = prop.multiProcessorCount;
    d->name = prop.name[0] ? prop.name : prop.gcnArchName;
    // this GPU's copy of the no-allocation scratch (the device is current), and the event that
    // orders the calls using it
    if ((e = hipGetSymbolAddress(&d->scratch, HIP_SYMBOL(scratch))) != hipSuccess) {
        delete d;
        return hip_fail(nullptr, e, "scratch address");
    }
    if (ordinal < kMaxOrdinals) {
        std::lock_guard<std::mutex> lock(g_noalloc[ordinal].mu);
        if (!g_noalloc[ordinal].ev &&
            (e = hipEventCreateWithFlags(&g_noalloc[ordinal].ev, hipEventDisableTiming)) != hipSuccess) {
            g_noalloc[ordinal].ev = nullptr;
            delete d;
            return hip_fail(nullptr, e, "scratch event");
        }
    }
    if ((e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking)) != hipSuccess) {
        delete d;
        return hip_fail(nullptr, e, "create stream");
    }
    if ((e = decode_lds_limits()) != hipSuccess) {  // (before any capture a caller may start)
        (void)hipStreamDestroy(d->stream);
        delete d;
        return hip_fail(nullptr, e, "kernel LDS limits");
    }
    *out = d;
    return FH_OK;
}

void fh_device_close(fh_device *dev) {
    if (!dev || dev->closed.exchange(true)) return;
    (void)hipSetDevice(dev->ordinal);
    (void)hipStreamSynchronize(dev->stream);
    dev_release(dev);
}

fh_status fh_device_sync(fh_device *dev) {
    fh_status st = check_dev(dev);
    if (st) return st;
    return sync(dev, "sync");
}

fh_status fh_device_info(fh_device *dev, char *name, size_t cap, int *compute_units) {
    if (!dev) return fail(FH_ERR_INVALID, "no device");
    if (name && cap) snprintf(name, cap, "%s", dev->name.c_str());
    if (compute_units) *compute_units = dev->cus;
    return FH_OK;
}

void *fh_device_stream(fh_device *dev) { return dev ? (void *)dev->stream : nullptr; }
void fh_debug_fail_after(fh_device *dev, int64_t n) {
    if (dev) dev->fail_after.store(n < 0 ? -1 : n);
}
uint64_t fh_debug_commands(fh_device *dev) { return dev ? dev->commands.load() : 0; }

// ---- buffers ----

fh_status fh_buffer_zeros(fh_device *dev, size_t len, fh_buffer **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (len > (SIZE_MAX / 8)) return fail(FH_ERR_INVALID, "buffer of %zu elements is too large", len);
    return new_buffer(dev, len * 4, out);
}

fh_status fh_buffer_upload(fh_device *dev, const float *host, size_t len, fh_buffer **out) {
    fh_status st = fh_buffer_zeros(dev, len, out);
    if (st) return st;
    st = upload_bytes(dev, (*out)->ptr, host, len * 4, "upload");
    if (st) {
        fh_buffer_free(*out);
        *out = nullptr;
    }
    return st;
}

fh_status fh_buffer_read(fh_device *dev, const fh_buffer *buf, float *host, size_t len) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if ((st = need("read", buf, len))) return st;
    return read_bytes(dev, host, buf->ptr, len * 4, "read");
}

fh_status fh_buffer_write(fh_device *dev, fh_buffer *buf, const float *host, size_t len) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if ((st = need("write", buf, len))) return st;
    return upload_bytes(dev, buf->ptr, host, len * 4, "write");
}

fh_status fh_bytes_zeros(fh_device *dev, size_t nbytes, fh_buffer **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    return new_buffer(dev, nbytes, out);
}

fh_status fh_bytes_upload(fh_device *dev, const uint8_t *host, size_t nbytes, fh_buffer **out) {
    fh_status st = fh_bytes_zeros(dev, nbytes, out);
    if (st) return st;
    st = upload_bytes(dev, (*out)->ptr, host, nbytes, "upload");
    if (st) {
        fh_buffer_free(*out);
        *out = nullptr;
    }
    return st;
}

fh_status fh_bytes_read(fh_device *dev, const fh_buffer *buf, uint8_t *host, size_t nbytes) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!buf || buf->nbytes != nbytes)
        return fail(FH_ERR_INVALID, "read: buffer holds %zu bytes, expected %zu",
                    buf ? buf->nbytes : 0, nbytes);
    return read_bytes(dev, host, buf->ptr, nbytes, "read");
}

size_t fh_buffer_len(const fh_buffer *buf) { return buf ? buf->nbytes / 4 : 0; }
size_t fh_buffer_nbytes(const fh_buffer *buf) { return buf ? buf->nbytes : 0; }
void *fh_buffer_device_ptr(const fh_buffer *buf) { return buf ? buf->ptr : nullptr; }

void fh_buffer_free(fh_buffer *buf) {
    if (!buf) return;
    fh_device *dev = buf->dev;
    free_bytes(dev, buf->ptr);  // no queued kernel may still use it
    delete buf;
    dev_release(dev);
}

fh_status fh_copy_f32(fh_device *dev, const fh_buffer *src, size_t src_off, fh_buffer *dst,
                      size_t dst_off, size_t len) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!src || !dst) return fail(FH_ERR_INVALID, "copy_f32: no buffer");
    if (src_off + len > src->nbytes / 4 || dst_off + len > dst->nbytes / 4)
        return fail(FH_ERR_INVALID, "copy_f32: range out of bounds");
    if ((st = begin_command(dev, "copy_f32"))) return st;
    if (len)
        (void)launch_copy_f32(dev->stream, (const float *)src->ptr + src_off, (float *)dst->ptr + dst_off, len);
    return end_command(dev, "copy_f32");
}

// ---- device codec ----

size_t fh_nbytes(fh_kind kind, size_t n) {
    size_t bb, be;
    if (!kind_ok(kind) && ext_layout(kind, &bb, &be)) {
        if (n % be) {
            fail(FH_ERR_INVALID, "%zu elements is not a multiple of the block size %zu", n, be);
            return 0;
        }
        return n / be * bb;
    }
    if (!kind_ok(kind)) {
        fail(FH_ERR_UNSUPPORTED, "unsupported block format %d", (int)kind);
        return 0;
    }
    if (n % QK) {
        fail(FH_ERR_INVALID, "%zu elements is not a multiple of the block size 32", n);
        return 0;
    }
    return n / QK * block_bytes(kind);
}

fh_status fh_encode(fh_device *dev, fh_kind kind, const fh_buffer *src, size_t n, fh_buffer *dst) {
    fh_status st = check_dev(dev);
    if (st) return st;
    size_t bb, be;
    if (!kind_ok(kind) && ext_layout(kind, &bb, &be)) {
        if (!ext_kind(kind))
            return fail(FH_ERR_UNSUPPORTED, "tensor type %d is read-only: it can be loaded but not written", (int)kind);
        if (n % be) return fail(FH_ERR_INVALID, "%zu elements is not a multiple of the block size %zu", n, be);
        if (!src || !dst || src->nbytes < n * 4 || dst->nbytes < n / be * bb)
            return fail(FH_ERR_INVALID, "encode: buffers too small for %zu elements", n);
        if ((st = begin_command(dev, "encode"))) return st;
        (void)launch_encode_ext(dev->stream, kind, (const float *)src->ptr, (uint8_t *)dst->ptr, n);
        return end_command(dev, "encode");
    }
    if (!kind_ok(kind)) return fail(FH_ERR_UNSUPPORTED, "unsupported block format %d", (int)kind);
    if (n % QK) return fail(FH_ERR_INVALID, "%zu elements is not a multiple of the block size 32", n);
    if (!src || !dst || src->nbytes < n * 4 || dst->nbytes < n / QK * block_bytes(kind))
        return fail(FH_ERR_INVALID, "encode: buffers too small for %zu elements", n);
    if ((st = begin_command(dev, "encode"))) return st;
    if (n) (void)launch_encode_rows(dev->stream, kind, (const float *)src->ptr, (uint8_t *)dst->ptr, n / QK);
    return end_command(dev, "encode");
}

fh_status fh_decode(fh_device *dev, fh_kind kind, const fh_buffer *src, size_t n, fh_buffer *dst) {
    fh_status st = check_dev(dev);
    if (st) return st;
    size_t bb, be;
    if (!kind_ok(kind) && ext_layout(kind, &bb, &be)) {
        if (n % be) return fail(FH_ERR_INVALID, "%zu elements is not a multiple of the block size %zu", n, be);
        if (!src || !dst || src->nbytes < n / be * bb || dst->nbytes < n * 4)
            return fail(FH_ERR_INVALID, "decode: buffers too small for %zu elements", n);
        if ((st = begin_command(dev, "decode"))) return st;
        (void)launch_decode_ext(dev->stream, kind, (const uint8_t *)src->ptr, (float *)dst->ptr, n);
        return end_command(dev, "decode");
    }
    if (!kind_ok(kind)) return fail(FH_ERR_UNSUPPORTED, "unsupported block format %d", (int)kind);
    if (n % QK) return fail(FH_ERR_INVALID, "%zu elements is not a multiple of the block size 32", n);
    if (!src || !dst || src->nbytes < n / QK * block_bytes(kind) || dst->nbytes < n * 4)
        return fail(FH_ERR_INVALID, "decode: buffers too small for %zu elements", n);
    if ((st = begin_command(dev, "decode"))) return st;
    if (n) (void)launch_decode_rows(dev->stream, kind, (const uint8_t *)src->ptr, (float *)dst->ptr, n / QK);
    return end_command(dev, "decode");
}

// ---- resident weights ----

fh_status fh_qweight_upload_gguf(fh_device *dev, fh_kind kind, const uint8_t *bytes, size_t len,
                                 size_t k, size_t n, fh_qweight **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (ext_kind(kind)) {  // kept as the GGUF rows
        size_t bb, be;
        ext_layout(kind, &bb, &be);
        if (k == 0 || k % be)
            return fail(FH_ERR_INVALID, "a %zu x %zu weight is not whole %zu-element blocks", k, n, be);
        const size_t want = k / be * n * bb;
        if (len != want)
            return fail(FH_ERR_INVALID, "%zu bytes is not the %zu a %zu x %zu %s weight needs", len, want, k, n,
                        ext_label(kind));
        if ((st = new_qweight(dev, kind, k, n, out))) return st;
        if ((st = upload_bytes(dev, (*out)->qs, bytes, len, "upload_qweight"))) {
            fh_qweight_free(*out);
            *out = nullptr;
        }
        return st;
    }
    if (!kind_ok(kind)) return fail(FH_ERR_UNSUPPORTED, "unsupported block format %d", (int)kind);
    if (k == 0 || k % QK)
        return fail(FH_ERR_INVALID, "a %zu x %zu weight is not whole 32-element blocks", k, n);
    size_t want = k / QK * n * block_bytes(kind);
    if (len != want)
        return fail(FH_ERR_INVALID, "%zu bytes is not the %zu a %zu x %zu %s weight needs", len,
                    want, k, n, kind == FH_Q8_0 ? "Q8_0" : "Q4_0");
    if ((st = new_qweight(dev, kind, k, n, out))) return st;
    // the GGUF bytes go to a staging buffer and are repacked into the weight's planes
    void *stage = nullptr;
    if ((st = alloc_bytes(dev, len, &stage)) == FH_OK) {
        st = upload_bytes(dev, stage, bytes, len, "upload_qweight");
        if (st == FH_OK && (st = begin_command(dev, "upload_qweight")) == FH_OK) {
            (void)launch_gguf_to_planes(dev->stream, kind, (const uint8_t *)stage, (*out)->qs, (*out)->ds, n,
                                        k / QK);
            st = end_command(dev, "upload_qweight");
        }
        free_bytes(dev, stage);  // waits for the repack
    }
    if (st) {
        fh_qweight_free(*out);
        *out = nullptr;
    }
    return st;
}

fh_status fh_qweight_quantise(fh_device *dev, fh_kind kind, const fh_buffer *w, size_t k, size_t n,
                              fh_qweight **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (ext_kind(kind)) {  // transpose to GGUF rows, then encode them
        size_t bb, be;
        ext_layout(kind, &bb, &be);
        if (k == 0 || k % be || !w || w->nbytes / 4 != k * n)
            return fail(FH_ERR_INVALID, "cannot quantise %zu elements as a %zu x %zu weight in whole %zu-blocks",
                        w ? w->nbytes / 4 : 0, k, n, be);
        if ((st = new_qweight(dev, kind, k, n, out))) return st;
        void *rows = nullptr;
        if ((st = alloc_bytes(dev, k * n * 4, &rows)) == FH_OK) {
            if ((st = begin_command(dev, "quantise_matrix")) == FH_OK) {
                (void)launch_transpose(dev->stream, (const float *)w->ptr, (float *)rows, k, n);
                (void)launch_encode_ext(dev->stream, kind, (const float *)rows, (*out)->qs, k * n);
                st = end_command(dev, "quantise_matrix");
            }
            free_bytes(dev, rows);  // waits for the encode
        }
        if (st) {
            fh_qweight_free(*out);
            *out = nullptr;
        }
        return st;
    }
    if (!kind_ok(kind)) return fail(FH_ERR_UNSUPPORTED, "unsupported block format %d", (int)kind);
    if (k == 0 || k % QK || !w || w->nbytes / 4 != k * n)
        return fail(FH_ERR_INVALID,
                    "cannot quantise %zu elements as a %zu x %zu weight in whole 32-blocks",
                    w ? w->nbytes / 4 : 0, k, n);
    if ((st = new_qweight(dev, kind, k, n, out))) return st;
    if ((st = begin_command(dev, "quantise_matrix")) == FH_OK) {
        (void)launch_encode_cols(dev->stream, kind, (const float *)w->ptr, (*out)->qs, (*out)->ds, k, n);
        st = end_command(dev, "quantise_matrix");
    }
    if (st) {
        fh_qweight_free(*out);
        *out = nullptr;
    }
    return st;
}

fh_status fh_qweight_upload_f32(fh_device *dev, fh_kind kind, const float *w, size_t k, size_t n,
                                fh_qweight **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!kind_ok(kind) && !ext_kind(kind))
        return fail(FH_ERR_UNSUPPORTED, "unsupported block format %d", (int)kind);
    size_t be = QK;
    if (ext_kind(kind)) ext_layout(kind, nullptr, &be);
    if (k == 0 || k % be)
        return fail(FH_ERR_INVALID,
                    "cannot quantise %zu elements as a %zu x %zu weight in whole %zu-blocks",
                    k * n, k, n, be);
    fh_buffer *tmp = nullptr;
    if ((st = fh_buffer_upload(dev, w, k * n, &tmp))) return st;
    st = fh_qweight_quantise(dev, kind, tmp, k, n, out);
    fh_buffer_free(tmp);  // synchronizes: the encode has finished reading it
    return st;
}

void fh_qweight_free(fh_qweight *w) {
    if (!w) return;
    fh_device *dev = w->dev;
    free_bytes(dev, w->ptr);
    if (w->b8) free_bytes(dev, w->b8);
    delete w;
    dev_release(dev);
}

fh_kind fh_qweight_kind(const fh_qweight *w) { return w->kind; }
size_t fh_qweight_k(const fh_qweight *w) { return w->k; }
size_t fh_qweight_n(const fh_qweight *w) { return w->n; }
uint64_t fh_qweight_device_bytes(const fh_qweight *w) {
    return w->alloc + (w->b8 ? gemm_b8_bytes(w->k, w->n) : 0);
}

fh_status fh_qweight_read_gguf(fh_device *dev, const fh_qweight *w, uint8_t *host, size_t len) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!w || len != w->nbytes)
        return fail(FH_ERR_INVALID, "read_gguf: %zu bytes requested, the weight holds %zu", len,
                    w ? w->nbytes : 0);
    if (ext_kind(w->kind)) return read_bytes(dev, host, w->qs, len, "read_gguf");
    void *stage = nullptr;
    if ((st = alloc_bytes(dev, len, &stage))) return st;
    if ((st = begin_command(dev, "read_gguf")) == FH_OK) {
        (void)launch_planes_to_gguf(dev->stream, w->kind, w->qs, w->ds, (uint8_t *)stage, w->n, w->k / QK);
        if ((st = end_command(dev, "read_gguf")) == FH_OK) st = read_bytes(dev, host, stage, len, "read_gguf");
    }
    free_bytes(dev, stage);
    return st;
}

fh_status fh_qweight_dequantise(fh_device *dev, const fh_qweight *w, fh_buffer *out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!w) return fail(FH_ERR_INVALID, "dequantise: no weight");
    if ((st = need("dequantise out", out, w->k * w->n))) return st;
    if (ext_kind(w->kind)) {  // decode the rows, then transpose to [k, n]
        void *rows = nullptr;
        if ((st = alloc_bytes(dev, w->k * w->n * 4, &rows))) return st;
        if ((st = begin_command(dev, "dequantise")) == FH_OK) {
            (void)launch_decode_ext(dev->stream, w->kind, w->qs, (float *)rows, w->k * w->n);
            (void)launch_transpose(dev->stream, (const float *)rows, (float *)out->ptr, w->n, w->k);
            st = end_command(dev, "dequantise");
        }
        free_bytes(dev, rows);
        return st;
    }
    if ((st = begin_command(dev, "dequantise"))) return st;
    (void)launch_decode_cols(dev->stream, w->kind, w->qs, w->ds, (float *)out->ptr, w->k, w->n);
    return end_command(dev, "dequantise");
}

// ---- linear layers ----

// The few-row / GEMM boundary, measured on one MI355X with one linear_q per product (each call
// reading its weight from HBM) at the Qwen2-0.5B and TinyLlama-1.1B shapes, Q4_0 and Q8_0, rows
// 2 to 128. Single calls at these sizes are latency-bound: the MFMA GEMM costs a nearly flat
// 17-33 us, while the few-row kernel's time steps up with its row capacity class (16, 32, 64)
// and grows with k. Up to 16 rows the few-row kernel wins everywhere (by 20-45%); from 17 to 32
// rows while k <= 4864 (at k = 5632 the GEMM is 4-5% faster); from 33 to 64 rows only on the wide,
// short products (n >= 2560, k <= 2048: 896 x 4864, 2048 x 2560, 2048 x 11264).
fh_path fh_choose(size_t rows, fh_kind kind, size_t k, size_t n) {
    if (ext_kind(kind)) return rows == 1 ? FH_PATH_GEMV : FH_PATH_TILED;
    if (rows == 1 && kind_ok(kind) && gemv_supported(kind, k, n)) return FH_PATH_GEMV;
    if (rows >= 2 && rows <= kRowsMax && kind_ok(kind) && rows_supported(rows, k, n)) {
        if (rows <= 16) return FH_PATH_ROWS;
        if (rows <= 32) return k <= 4864 ? FH_PATH_ROWS : FH_PATH_TILED;
        return n >= 2560 && k <= 2048 ? FH_PATH_ROWS : FH_PATH_TILED;
    }
    return FH_PATH_TILED;
}

// Scratch for one linear command: the device's workspace (grown on demand) or, for the
// no-allocation entry point (fixed = the device's static scratch), that array within its size.
static fh_status command_scratch(fh_device *dev, void *fixed, size_t bytes, void **out) {
    if (!fixed) return workspace(dev, bytes, out);
    if (bytes > FH_NOALLOC_SCRATCH_BYTES)
        return fail(FH_ERR_INVALID,
                    "linear_q_noalloc: the product needs %zu bytes of scratch, more than the %u the library holds",
                    bytes, (unsigned)FH_NOALLOC_SCRATCH_BYTES);
    *out = fixed;
    return FH_OK;
}

static fh_status linear(fh_device *dev, const float *x, const fh_qweight *w, float *y, size_t rows,
                        fh_path path, void *fixed = nullptr) {
    if (path == FH_PATH_AUTO) path = fh_choose(rows, w->kind, w->k, w->n);
    fh_status st;
    if (ext_kind(w->kind)) {  // decoded on the fly (formats.hip; the multi-row MFMA GEMM in gemm.hip)
        if (path != FH_PATH_NAIVE && path != FH_PATH_GEMV && path != FH_PATH_TILED)
            return fail(FH_ERR_UNSUPPORTED, "kernel path %d does not take %s weights", (int)path, ext_label(w->kind));
        if (path == FH_PATH_GEMV && rows != 1)
            return fail(FH_ERR_INVALID, "the GEMV kernel takes one row, not %zu", rows);
        if (path == FH_PATH_TILED && rows >= 2 && gemm_ext_kind(w->kind)) {  // the MFMA GEMM (gemm.hip)
            void *ws = nullptr;
            const size_t wsb = gemm_ext_workspace_bytes(w->kind, rows, w->k, w->n);
            if ((st = command_scratch(dev, fixed, wsb, &ws))) return st;
            if ((st = begin_command(dev, "linear_q"))) return st;
            (void)launch_gemm_ext(dev->stream, w->kind, w->qs, x, y, rows, w->k, w->n, ws);
            return end_command(dev, "linear_q");
        }
        if ((st = begin_command(dev, "linear_q"))) return st;
        (void)launch_linear_ext(dev->stream, w->kind, path, w->qs, x, y, rows, w->k, w->n);
        return end_command(dev, "linear_q");
    }
    switch (path) {
    case FH_PATH_GEMV: {
        if (rows != 1) return fail(FH_ERR_INVALID, "the GEMV kernel takes one row, not %zu", rows);
        if (!gemv_supported(w->kind, w->k, w->n))
            return fail(FH_ERR_INVALID, "the GEMV kernel's 32-bit offsets do not cover a %zu x %zu weight",
                        w->n, w->k);
        if (gemv_latency_fits(w->k, w->n, dev->cus) && ((uintptr_t)x & 15) == 0) {  // few row groups
            if ((st = begin_command(dev, "linear_q"))) return st;
            (void)launch_gemv_latency(dev->stream, w->kind, w->qs, w->ds, x, y, w->k, w->n);
            return end_command(dev, "linear_q");
        }
        void *prep = nullptr;
        if ((st = command_scratch(dev, fixed, gemv_prep_bytes(w->k), &prep))) return st;
        if ((st = begin_command(dev, "linear_q"))) return st;
        (void)launch_gemv(dev->stream, w->kind, w->qs, w->ds, x, y, w->k, w->n, prep, dev->cus);
        return end_command(dev, "linear_q");
    }
    case FH_PATH_ROWS: {
        if (rows > kRowsMax)
            return fail(FH_ERR_INVALID, "the few-row kernel takes 1 to %zu rows, not %zu", kRowsMax, rows);
        if (rows && !rows_supported(rows, w->k, w->n))
            return fail(FH_ERR_INVALID, "the few-row kernel's 32-bit offsets do not cover %zu rows of a %zu x %zu weight",
                        rows, w->n, w->k);
        void *xs = nullptr;
        if (rows && (st = command_scratch(dev, fixed, rows_xsplit_bytes(rows, w->k), &xs))) return st;
        if ((st = begin_command(dev, "linear_q"))) return st;
        if (rows) (void)launch_rows(dev->stream, w->kind, w->qs, w->ds, x, y, rows, w->k, w->n, xs, dev->cus);
        return end_command(dev, "linear_q");
    }
    case FH_PATH_NAIVE:
        if ((st = begin_command(dev, "linear_q"))) return st;
        if (rows) (void)launch_naive(dev->stream, w->kind, w->qs, w->ds, x, y, rows, w->k, w->n);
        return end_command(dev, "linear_q");
    case FH_PATH_TILED: {
        void *ws = nullptr;
        if (rows && (st = command_scratch(dev, fixed, gemm_precise_workspace_bytes(rows, w->k, w->n), &ws)))
            return st;
        if ((st = begin_command(dev, "linear_q"))) return st;
        if (rows) (void)launch_gemm_precise(dev->stream, w->kind, w->qs, w->ds, x, y, rows, w->k, w->n, ws);
        return end_command(dev, "linear_q");
    }
    case FH_PATH_TILED_FAST: {
        if (!gemm_supported(rows, w->k, w->n))
            return fail(FH_ERR_INVALID, "the MFMA GEMM's 32-bit offsets do not cover %zu rows of a %zu x %zu weight",
                        rows, w->n, w->k);
        if (fixed && rows && !w->b8)
            return fail(FH_ERR_INVALID, "linear_q_noalloc: the fast GEMM needs the weight's correction operand, "
                                        "which its first multi-row FH_PATH_TILED_FAST linear_q builds");
        void *ws = nullptr;
        if (rows && (st = command_scratch(dev, fixed, gemm_workspace_bytes(rows, w->k, w->n), &ws))) return st;
        void *fresh = nullptr;  // the correction operand, built within the weight's first multi-row command
        if (rows && !w->b8 && (st = alloc_bytes(dev, gemm_b8_bytes(w->k, w->n), &fresh))) return st;
        if ((st = begin_command(dev, "linear_q"))) {
            if (fresh) free_bytes(dev, fresh);
            return st;
        }
        if (fresh) {
            (void)launch_make_b8(dev->stream, w->kind, w->qs, w->ds, (uint8_t *)fresh, w->k, w->n);
            w->b8 = (uint8_t *)fresh;
        }
        if (rows) (void)launch_gemm(dev->stream, w->kind, w->qs, w->ds, w->b8, x, y, rows, w->k, w->n, ws);
        return end_command(dev, "linear_q");
    }
    case FH_PATH_TILED_F16: {
        if (!gemm_f16_supported(rows, w->k, w->n))
            return fail(FH_ERR_INVALID, "the MFMA GEMM's 32-bit offsets do not cover %zu rows of a %zu x %zu weight",
                        rows, w->n, w->k);
        void *ws = nullptr;
        if (rows && (st = command_scratch(dev, fixed, gemm_f16_workspace_bytes(rows, w->k, w->n), &ws))) return st;
        if ((st = begin_command(dev, "linear_q"))) return st;
        if (rows) (void)launch_gemm_f16(dev->stream, w->kind, w->qs, w->ds, x, y, rows, w->k, w->n, ws);
        return end_command(dev, "linear_q");
    }
    default:
        return fail(FH_ERR_INVALID, "unknown kernel path %d", (int)path);
    }
}

fh_status fh_linear_q(fh_device *dev, const fh_buffer *x, const fh_qweight *w, fh_buffer *y,
                      size_t rows, fh_path path) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!w) return fail(FH_ERR_INVALID, "linear_q: no weight");
    if (rows > (1u << 24)) return fail(FH_ERR_INVALID, "linear_q: %zu rows is too many", rows);
    if ((st = need("linear_q x", x, rows * w->k))) return st;
    if ((st = need("linear_q y", y, rows * w->n))) return st;
    if (overlaps(x->ptr, rows * w->k * 4, y->ptr, rows * w->n * 4))
        return fail(FH_ERR_INVALID, "linear_q: x and y overlap");
    return linear(dev, (const float *)x->ptr, w, (float *)y->ptr, rows, path);
}

fh_status fh_linear_q_ptr(fh_device *dev, const float *x, const fh_qweight *w, float *y,
                          size_t rows, fh_path path) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!w) return fail(FH_ERR_INVALID, "linear_q: no weight");
    if (rows > (1u << 24)) return fail(FH_ERR_INVALID, "linear_q: %zu rows is too many", rows);
    if (!x) return fail(FH_ERR_INVALID, "linear_q x: null pointer");
    if (!y) return fail(FH_ERR_INVALID, "linear_q y: null pointer");
    if (overlaps(x, rows * w->k * 4, y, rows * w->n * 4)) return fail(FH_ERR_INVALID, "linear_q: x and y overlap");
    return linear(dev, x, w, y, rows, path);
}

fh_status fh_linear_q_noalloc(fh_device *dev, const float *x, const fh_qweight *w, float *y, size_t rows,
                              fh_path path) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!w) return fail(FH_ERR_INVALID, "linear_q: no weight");
    if (rows > (1u << 24)) return fail(FH_ERR_INVALID, "linear_q: %zu rows is too many", rows);
    if (!x) return fail(FH_ERR_INVALID, "linear_q x: null pointer");
    if (!y) return fail(FH_ERR_INVALID, "linear_q y: null pointer");
    if (overlaps(x, rows * w->k * 4, y, rows * w->n * 4)) return fail(FH_ERR_INVALID, "linear_q: x and y overlap");
    if (!dev->scratch) return fail(FH_ERR_DEVICE, "linear_q_noalloc: the device has no scratch address");
    if (dev->ordinal >= kMaxOrdinals || !g_noalloc[dev->ordinal].ev)
        return fail(FH_ERR_DEVICE, "linear_q_noalloc: no scratch order for device %d", dev->ordinal);
    NoallocOrder &o = g_noalloc[dev->ordinal];
    std::lock_guard<std::mutex> lock(o.mu);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(dev->stream, &cs) != hipSuccess) cs = hipStreamCaptureStatusNone;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    hipError_t e;
    if (!capturing && o.recorded && (e = hipStreamWaitEvent(dev->stream, o.ev, 0)) != hipSuccess)
        return hip_fail(dev, e, "linear_q_noalloc: wait for the previous call");
    if ((st = linear(dev, x, w, y, rows, path, dev->scratch))) return st;
    if (!capturing) {
        if ((e = hipEventRecord(o.ev, dev->stream)) != hipSuccess) return hip_fail(dev, e, "linear_q_noalloc: order");
        o.recorded = true;
    }
    return FH_OK;
}

// ---- grouped batch-1 GEMV ----

fh_status fh_gemv_plan_create(fh_device *dev, const fh_gemv_problem *problems, size_t count,
                              fh_gemv_plan **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!out || (count && !problems)) return fail(FH_ERR_INVALID, "gemv plan: null argument");
    fh_gemv_plan *plan = new (std::nothrow) fh_gemv_plan;
    if (!plan) return fail(FH_ERR_OOM, "host out of memory");
    dev_retain(dev);
    plan->dev = dev;
    // Check every problem, then group by format and, within a format, by width (the products whose
    // x fits the kernel's LDS region, then the wider ones), keeping the caller's order inside a
    // group: each group is one launch. The narrow launch prepares x in LDS and also writes the wide
    // launch's prepared x, which then needs no preparation kernel of its own.
    for (size_t i = 0; i < count; i++) {
        const fh_gemv_problem &p = problems[i];
        if (!p.w || !p.x || !p.y) {
            fh_gemv_plan_free(plan);
            return fail(FH_ERR_INVALID, "gemv plan: problem %zu has a null pointer", i);
        }
        if (p.w->dev != dev) {
            fh_gemv_plan_free(plan);
            return fail(FH_ERR_INVALID, "gemv plan: problem %zu lives on another device", i);
        }
        if (!kind_ok(p.w->kind)) {
            fh_gemv_plan_free(plan);
            return fail(FH_ERR_UNSUPPORTED, "gemv plan: problem %zu is a %s weight; plans take Q8_0 and Q4_0", i,
                        ext_label(p.w->kind));
        }
        if (!gemv_supported(p.w->kind, p.w->k, p.w->n)) {
            fh_gemv_plan_free(plan);
            return fail(FH_ERR_INVALID, "gemv plan: problem %zu (%zu x %zu) is too large for one product", i,
                        p.w->n, p.w->k);
        }
    }
    {
        std::vector<std::pair<uintptr_t, size_t>> xr, yr;
        for (size_t i = 0; i < count; i++) {
            xr.emplace_back((uintptr_t)problems[i].x, problems[i].w->k * 4);
            yr.emplace_back((uintptr_t)problems[i].y, problems[i].w->n * 4);
        }
        const long bad = plan_overlap(xr, yr);
        if (bad >= 0) {
            fh_gemv_plan_free(plan);
            return fail(FH_ERR_INVALID, "gemv plan: problem %ld's x or y overlaps another product's y", bad);
        }
    }
    std::vector<GemvDesc> host;
    std::vector<uint32_t> map;      // per launch, the product (launch-local index) of each task
    std::vector<size_t> prep_off;  // byte offset of each product's prepared x in plan->prep
    host.reserve(count);
    size_t prep_bytes = 0;
    for (int kind : {FH_Q8_0, FH_Q4_0})
    for (bool narrow : {true, false}) {
        fh_gemv_plan::Launch L{(fh_kind)kind, host.size(), 0, map.size(), 0, 0, narrow, false};
        for (size_t i = 0; i < count; i++) {
            const fh_gemv_problem &p = problems[i];
            if ((int)p.w->kind != kind || (p.w->k / QK <= kGemvLdsBlocks) != narrow) continue;
            const uint32_t nb = (uint32_t)(p.w->k / QK);
            GemvDesc d{p.w->qs, p.w->ds, p.x, p.y, nullptr, nb, (uint32_t)p.w->n, L.tasks, 0};
            const uint64_t t = (uint64_t)L.tasks + gemv_tasks(p.w->n);
            if (t >= (1ull << 31)) {
                fh_gemv_plan_free(plan);
                return fail(FH_ERR_INVALID, "gemv plan: too many rows in one launch");
            }
            map.insert(map.end(), gemv_tasks(p.w->n), (uint32_t)L.count);
            L.tasks = (uint32_t)t;
            L.max_nb = nb > L.max_nb ? nb : L.max_nb;
            host.push_back(d);
            prep_off.push_back(prep_bytes);
            prep_bytes += gemv_prep_bytes(p.w->k);
            plan->bytes += p.w->nbytes + 4ull * (p.w->k + p.w->n);
            L.count++;
        }
        if (L.count) {
            L.prepared = !narrow && !plan->launches.empty() && plan->launches.back().kind == L.kind &&
                         plan->launches.back().narrow;
            plan->launches.push_back(L);
        }
    }
    if (!host.empty()) {
        void *p = nullptr;
        if ((st = alloc_bytes(dev, prep_bytes, &p))) {
            fh_gemv_plan_free(plan);
            return st;
        }
        plan->prep = (uint8_t *)p;
        for (size_t i = 0; i < host.size(); i++) host[i].prep = plan->prep + prep_off[i];
        if ((st = alloc_bytes(dev, host.size() * sizeof(GemvDesc), &p))) {
            fh_gemv_plan_free(plan);
            return st;
        }
        plan->descs = (GemvDesc *)p;
        if ((st = upload_bytes(dev, p, host.data(), host.size() * sizeof(GemvDesc), "gemv plan"))) {
            fh_gemv_plan_free(plan);
            return st;
        }
        if ((st = alloc_bytes(dev, map.size() * sizeof(uint32_t), &p))) {
            fh_gemv_plan_free(plan);
            return st;
        }
        plan->map = (uint32_t *)p;
        if ((st = upload_bytes(dev, p, map.data(), map.size() * sizeof(uint32_t), "gemv plan"))) {
            fh_gemv_plan_free(plan);
            return st;
        }
    }
    *out = plan;
    return FH_OK;
}

fh_status fh_gemv_plan_run_launch(fh_device *dev, const fh_gemv_plan *plan, size_t i) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!plan || plan->dev != dev) return fail(FH_ERR_INVALID, "gemv plan: wrong device");
    if (i >= plan->launches.size())
        return fail(FH_ERR_INVALID, "gemv plan: launch %zu of %zu", i, plan->launches.size());
    const auto &L = plan->launches[i];
    GemvPrep other{nullptr, 0, 0};
    if (i + 1 < plan->launches.size() && plan->launches[i + 1].prepared) {
        const auto &W = plan->launches[i + 1];
        other = GemvPrep{plan->descs + W.first, (uint32_t)W.count, W.max_nb};
    }
    bool done = false;
    if ((st = begin_command(dev, "gemv plan"))) return st;
    (void)launch_gemv_group(dev->stream, L.kind, plan->descs + L.first, plan->map + L.map0, (uint32_t)L.count,
                            L.tasks, L.max_nb, dev->cus, other, L.prepared, &done);
    if ((st = end_command(dev, "gemv plan"))) return st;
    if (other.count && !done)  // (not reached: the wide launch's descriptors follow the narrow one's)
        return fail(FH_ERR_DEVICE, "gemv plan: launch %zu did not prepare the next launch's x", i);
    return FH_OK;
}

fh_status fh_gemv_plan_run(fh_device *dev, const fh_gemv_plan *plan) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!plan || plan->dev != dev) return fail(FH_ERR_INVALID, "gemv plan: wrong device");
    for (size_t i = 0; i < plan->launches.size(); i++)
        if ((st = fh_gemv_plan_run_launch(dev, plan, i))) return st;
    return FH_OK;
}

size_t fh_gemv_plan_launches(const fh_gemv_plan *plan) { return plan ? plan->launches.size() : 0; }
uint64_t fh_gemv_plan_bytes(const fh_gemv_plan *plan) { return plan ? plan->bytes : 0; }

void fh_gemv_plan_free(fh_gemv_plan *plan) {
    if (!plan) return;
    fh_device *dev = plan->dev;
    if (plan->descs) free_bytes(dev, plan->descs);
    if (plan->prep) free_bytes(dev, plan->prep);
    if (plan->map) free_bytes(dev, plan->map);
    delete plan;
    dev_release(dev);
}

// ---- grouped few-row products ----

struct fh_rows_plan {
    fh_device *dev = nullptr;
    struct Launch {
        fh_kind kind;
        size_t first, count;  // descriptors
        size_t map0;          // first entry of the launch's task -> product map
        uint32_t tasks, max_m, max_items;
    };
    std::vector<Launch> launches;
    RowsDesc *descs = nullptr;  // device array
    uint32_t *map = nullptr;    // device array: per launch, the product of each task
    _Float16 *xs = nullptr;     // split x of every product
    uint64_t bytes = 0;
};

fh_status fh_rows_plan_create(fh_device *dev, const fh_rows_problem *problems, size_t count, fh_rows_plan **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!out || (count && !problems)) return fail(FH_ERR_INVALID, "rows plan: null argument");
    fh_rows_plan *plan = new (std::nothrow) fh_rows_plan;
    if (!plan) return fail(FH_ERR_OOM, "host out of memory");
    dev_retain(dev);
    plan->dev = dev;
    for (size_t i = 0; i < count; i++) {
        const fh_rows_problem &p = problems[i];
        const char *why = !p.w || !p.x || !p.y ? "has a null pointer"
                          : !kind_ok(p.w->kind) ? "is not a Q8_0 or Q4_0 weight"
                          : p.rows < 1 || p.rows > kRowsMax ? "needs 1 to 64 rows"
                          : !rows_supported(p.rows, p.w->k, p.w->n) ? "is too large for one product"
                                                                    : nullptr;
        if (why) {
            fh_rows_plan_free(plan);
            return fail(FH_ERR_INVALID, "rows plan: problem %zu %s", i, why);
        }
    }
    if (count > 65535) {
        fh_rows_plan_free(plan);
        return fail(FH_ERR_INVALID, "rows plan: %zu products, at most 65535 per plan", count);
    }
    {
        std::vector<std::pair<uintptr_t, size_t>> xr, yr;
        for (size_t i = 0; i < count; i++) {
            const fh_rows_problem &p = problems[i];
            xr.emplace_back((uintptr_t)p.x, p.rows * p.w->k * 4);
            yr.emplace_back((uintptr_t)p.y, p.rows * p.w->n * 4);
        }
        const long bad = plan_overlap(xr, yr);
        if (bad >= 0) {
            fh_rows_plan_free(plan);
            return fail(FH_ERR_INVALID, "rows plan: problem %ld's x or y overlaps another product's y", bad);
        }
    }
    std::vector<RowsDesc> host;
    std::vector<uint32_t> map;
    std::vector<size_t> xs_off;
    size_t xs_bytes = 0;
    for (int kind : {FH_Q8_0, FH_Q4_0}) {
        fh_rows_plan::Launch L{(fh_kind)kind, host.size(), 0, map.size(), 0, 0, 0};
        for (size_t i = 0; i < count; i++)  // the launch's tile shape follows its largest row count
            if ((int)problems[i].w->kind == kind) L.max_m = std::max<uint32_t>(L.max_m, (uint32_t)problems[i].rows);
        for (size_t i = 0; i < count; i++) {
            const fh_rows_problem &p = problems[i];
            if ((int)p.w->kind != kind) continue;
            const uint32_t nb = (uint32_t)(p.w->k / QK), tasks = rows_tasks(p.w->n, p.w->k, L.max_m);
            const uint64_t t = (uint64_t)L.tasks + tasks;
            if (t >= (1ull << 31)) {
                fh_rows_plan_free(plan);
                return fail(FH_ERR_INVALID, "rows plan: too many rows in one launch");
            }
            host.push_back(RowsDesc{p.w->qs, p.w->ds, p.x, nullptr, p.y, nb, (uint32_t)p.w->n, (uint32_t)p.rows, L.tasks});
            map.insert(map.end(), tasks, (uint32_t)L.count);
            L.tasks = (uint32_t)t;
            L.max_items = std::max<uint32_t>(L.max_items, (uint32_t)(p.rows * nb));
            xs_off.push_back(xs_bytes);
            xs_bytes += (rows_xsplit_bytes(p.rows, p.w->k) + 255) / 256 * 256;
            plan->bytes += p.w->nbytes + 4ull * p.rows * (p.w->k + p.w->n);
            L.count++;
        }
        if (L.count) plan->launches.push_back(L);
    }
    if (!host.empty()) {
        void *p = nullptr;
        if ((st = alloc_bytes(dev, xs_bytes, &p))) {
            fh_rows_plan_free(plan);
            return st;
        }
        plan->xs = (_Float16 *)p;
        for (size_t i = 0; i < host.size(); i++) host[i].xs = (_Float16 *)((uint8_t *)plan->xs + xs_off[i]);
        if ((st = alloc_bytes(dev, host.size() * sizeof(RowsDesc), &p)) == FH_OK) {
            plan->descs = (RowsDesc *)p;
            st = upload_bytes(dev, p, host.data(), host.size() * sizeof(RowsDesc), "rows plan");
        }
        if (st == FH_OK && (st = alloc_bytes(dev, map.size() * sizeof(uint32_t), &p)) == FH_OK) {
            plan->map = (uint32_t *)p;
            st = upload_bytes(dev, p, map.data(), map.size() * sizeof(uint32_t), "rows plan");
        }
        if (st) {
            fh_rows_plan_free(plan);
            return st;
        }
    }
    *out = plan;
    return FH_OK;
}

fh_status fh_rows_plan_run(fh_device *dev, const fh_rows_plan *plan) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!plan || plan->dev != dev) return fail(FH_ERR_INVALID, "rows plan: wrong device");
    for (const auto &L : plan->launches) {
        if ((st = begin_command(dev, "rows plan"))) return st;
        (void)launch_rows_group(dev->stream, L.kind, plan->descs + L.first, plan->map + L.map0, (uint32_t)L.count,
                                L.tasks, L.max_m, L.max_items, dev->cus);
        if ((st = end_command(dev, "rows plan"))) return st;
    }
    return FH_OK;
}

size_t fh_rows_plan_launches(const fh_rows_plan *plan) { return plan ? plan->launches.size() : 0; }
uint64_t fh_rows_plan_bytes(const fh_rows_plan *plan) { return plan ? plan->bytes : 0; }

void fh_rows_plan_free(fh_rows_plan *plan) {
    if (!plan) return;
    fh_device *dev = plan->dev;
    if (plan->descs) free_bytes(dev, plan->descs);
    if (plan->xs) free_bytes(dev, plan->xs);
    if (plan->map) free_bytes(dev, plan->map);
    delete plan;
    dev_release(dev);
}

// ---- QAT snap ----

fh_status fh_q8_snap_rows(fh_device *dev, const fh_buffer *src, fh_buffer *dst, size_t ne0) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!src || !dst) return fail(FH_ERR_INVALID, "q8_snap: no buffer");
    size_t len = src->nbytes / 4;
    if (len != dst->nbytes / 4)
        return fail(FH_ERR_INVALID, "q8_snap: source holds %zu elements but destination %zu", len,
                    dst->nbytes / 4);
    if (ne0 == 0 || ne0 % QK || len % QK) return fh_copy_f32(dev, src, 0, dst, 0, len);
    if ((st = begin_command(dev, "q8_snap"))) return st;
    if (len) (void)launch_snap_rows(dev->stream, (const float *)src->ptr, (float *)dst->ptr, len / QK);
    return end_command(dev, "q8_snap");
}

fh_status fh_q8_snap_cols(fh_device *dev, const fh_buffer *src, fh_buffer *dst, size_t rows_in,
                          size_t cols_out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!src || !dst) return fail(FH_ERR_INVALID, "q8_snap: no buffer");
    size_t len = src->nbytes / 4;
    if (len != dst->nbytes / 4)
        return fail(FH_ERR_INVALID, "q8_snap: source holds %zu elements but destination %zu", len,
                    dst->nbytes / 4);
    if (len != rows_in * cols_out)
        return fail(FH_ERR_INVALID, "q8_snap: %zu elements is not %zu x %zu", len, rows_in, cols_out);
    if (rows_in == 0 || rows_in % QK) return fh_copy_f32(dev, src, 0, dst, 0, len);
    if ((st = begin_command(dev, "q8_snap"))) return st;
    if (len)
        (void)launch_snap_cols(dev->stream, (const float *)src->ptr, (float *)dst->ptr, rows_in, cols_out);
    return end_command(dev, "q8_snap");
}

// ---- grouped snap pass ----

}  // extern "C"

struct fh_snap_plan {
    fh_device *dev = nullptr;
    SnapDesc *descs = nullptr;  // device array
    uint32_t count = 0, tasks = 0;
    uint64_t bytes = 0;
};

extern "C" {

fh_status fh_snap_plan_create(fh_device *dev, const fh_snap_problem *problems, size_t count, fh_snap_plan **out) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!out || (count && !problems)) return fail(FH_ERR_INVALID, "snap plan: null argument");
    *out = nullptr;
    std::vector<SnapDesc> host;
    host.reserve(count);
    uint64_t tasks = 0, bytes = 0;
    for (size_t i = 0; i < count; i++) {
        const fh_snap_problem &p = problems[i];
        if (p.len && (!p.src || !p.dst))
            return fail(FH_ERR_INVALID, "snap plan: problem %zu has a null pointer", i);
        if (p.len > ((size_t)1 << 36))
            return fail(FH_ERR_INVALID, "snap plan: problem %zu holds too many values (%zu)", i, p.len);
        SnapDesc d{p.src, p.dst, (uint64_t)p.len, 0, 0, FH_SNAP_COPY, 0};
        switch (p.mode) {
        case FH_SNAP_ROWS:  // q8_snap_rows' fallback: ne0 or the length not whole blocks copies
            if (p.a && p.a % QK == 0 && p.len % QK == 0) d.mode = FH_SNAP_ROWS;
            break;
        case FH_SNAP_COLS:
            if (p.len != p.a * p.b)
                return fail(FH_ERR_INVALID, "snap plan: problem %zu: %zu elements is not %zu x %zu", i, p.len, p.a, p.b);
            if (p.a && p.a % QK == 0) {  // q8_snap_cols' fallback: rows_in not whole blocks copies
                if (p.a >= (1ull << 32) || p.b >= (1ull << 32))
                    return fail(FH_ERR_INVALID, "snap plan: problem %zu is too large", i);
                d.mode = FH_SNAP_COLS;
                d.k = (uint32_t)p.a;
                d.n = (uint32_t)p.b;
                if (p.b % 4 == 0 && ((uintptr_t)p.src | (uintptr_t)p.dst) % 16 == 0) d.mode |= 0x100;  // f32x4 form
            }
            break;
        case FH_SNAP_COPY: break;
        default: return fail(FH_ERR_INVALID, "snap plan: problem %zu has mode %d", i, p.mode);
        }
        if (!p.len) continue;
        d.task0 = (uint32_t)tasks;
        tasks += snap_tasks(d);
        if (tasks >= (1ull << 31)) return fail(FH_ERR_INVALID, "snap plan: too many values for one launch");
        bytes += 8ull * p.len;
        host.push_back(d);
    }
    fh_snap_plan *plan = new (std::nothrow) fh_snap_plan;
    if (!plan) return fail(FH_ERR_OOM, "host out of memory");
    dev_retain(dev);
    plan->dev = dev;
    plan->count = (uint32_t)host.size();
    plan->tasks = (uint32_t)tasks;
    plan->bytes = bytes;
    if (!host.empty()) {
        void *p = nullptr;
        if ((st = alloc_bytes(dev, host.size() * sizeof(SnapDesc), &p)) ||
            (plan->descs = (SnapDesc *)p,
             (st = upload_bytes(dev, p, host.data(), host.size() * sizeof(SnapDesc), "snap plan")))) {
            fh_snap_plan_free(plan);
            return st;
        }
    }
    *out = plan;
    return FH_OK;
}

fh_status fh_snap_plan_run(fh_device *dev, const fh_snap_plan *plan) {
    fh_status st = check_dev(dev);
    if (st) return st;
    if (!plan || plan->dev != dev) return fail(FH_ERR_INVALID, "snap plan: wrong device");
    if (!plan->count) return FH_OK;
    if ((st = begin_command(dev, "snap plan"))) return st;
    (void)launch_snap_group(dev->stream, plan->descs, plan->count, plan->tasks, dev->cus);
    return end_command(dev, "snap plan");
}

uint64_t fh_snap_plan_bytes(const fh_snap_plan *plan) { return plan ? plan->bytes : 0; }

void fh_snap_plan_free(fh_snap_plan *plan) {
    if (!plan) return;
    fh_device *dev = plan->dev;
    if (plan->descs) free_bytes(dev, plan->descs);
    delete plan;
    dev_release(dev);
}

}  // extern "C"
