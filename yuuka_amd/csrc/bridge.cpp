// bridge.cpp — implementation of the yuuka_hip.h C ABI on HIP for gfx950.
//
// Mirrors the contract of the reference bridge (backend/hip/bridge/bridge.cpp):
// opaque handles, thread-local error text (:47-57), an exception guard on every
// entry (:1893-1906), per-op validation before a plan op is appended
// (reject-without-append, yuuka_hip.h:330-334), asynchronous submission with a
// completion event (:3837-3870). Kernels live in k_*.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <exception>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "internal.h"
#include "model_kernels.h"
#include "ops.h"
#include "plan.h"

namespace yk {

static thread_local std::string g_last_error;

yuuka_status fail(yuuka_status status, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

const char *hip_error(hipError_t err) { return hipGetErrorString(err); }

yuuka_status ensure_scratch(yuuka_stream *stream, yk_scratch *area, uint64_t bytes) {
    if (area->bytes >= bytes) return YUUKA_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(YUUKA_ERR_UNSUPPORTED, "workspace must be sized before graph capture");
    // Outstanding work may still use the old area.
    hipError_t err = hipStreamSynchronize(stream->stream);
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "stream synchronize: %s", hip_error(err));
    if (area->ptr) (void)hipFree(area->ptr);
    area->ptr = nullptr;
    area->bytes = 0;
    const uint64_t want = (bytes + 0xfffffull) & ~0xfffffull;
    err = hipMalloc(&area->ptr, want);
    if (err != hipSuccess) {
        area->ptr = nullptr;
        return fail(YUUKA_ERR_ALLOCATION, "workspace of %llu bytes: %s", (unsigned long long)want,
                    hip_error(err));
    }
    err = hipMemset(area->ptr, 0, want);
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "workspace clear: %s", hip_error(err));
    area->bytes = want;
    return YUUKA_OK;
}

template <typename F>
static yuuka_status guard(const char *what, F &&f) {
    try {
        return f();
    } catch (const std::bad_alloc &) {
        return fail(YUUKA_ERR_ALLOCATION, "%s: host allocation failed", what);
    } catch (const std::exception &e) {
        return fail(YUUKA_ERR_INTERNAL, "%s: %s", what, e.what());
    } catch (...) {
        return fail(YUUKA_ERR_INTERNAL, "%s: unknown exception", what);
    }
}

static bool range_ok(const yuuka_buffer *b, uint64_t off, uint64_t bytes) {
    return b != nullptr && off <= b->bytes && bytes <= b->bytes - off;
}

static yuuka_status record(yuuka_stream *stream, yuuka_event *completion) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "kernel launch: %s", hip_error(err));
    if (completion) {
        err = hipEventRecord(completion->event, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "event record: %s", hip_error(err));
    }
    return YUUKA_OK;
}

// Shared validation of the verify GEMM shape (reference bridge.cpp:303-349).
yuuka_status check_verify_gemm(uint64_t n_in, uint64_t n_out, uint64_t rows, uint32_t dtype,
                               uint64_t max_rows) {
    if (dtype != YUUKA_DTYPE_Q4_K && dtype != YUUKA_DTYPE_Q6_K)
        return fail(YUUKA_ERR_UNSUPPORTED, "verify GEMM dtype %u is not Q4_K or Q6_K", dtype);
    if (n_in == 0 || n_in % 256 != 0)
        return fail(YUUKA_ERR_UNSUPPORTED, "verify GEMM input width %llu is not a multiple of 256",
                    (unsigned long long)n_in);
    if (n_out == 0 || rows == 0 || rows > max_rows)
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid output width %llu or row block %llu",
                    (unsigned long long)n_out, (unsigned long long)rows);
    if (n_in > (1ull << 24) || n_out > (1ull << 26))
        return fail(YUUKA_ERR_UNSUPPORTED, "verify GEMM shape %llux%llu too large",
                    (unsigned long long)n_out, (unsigned long long)n_in);
    const uint64_t wb = row_bytes(dtype, n_in) * n_out;
    if (wb >= (1ull << 32) - 16)
        return fail(YUUKA_ERR_UNSUPPORTED, "weight matrix of %llu bytes exceeds 4 GiB",
                    (unsigned long long)wb);
    return YUUKA_OK;
}

// Runs quantize + GEMM using `ws` (>= xq + partials) and `tickets`.
yuuka_status run_verify_gemm(hipStream_t stream, const void *w, uint32_t dtype, const float *x,
                             float *out, uint64_t n_in, uint64_t n_out, uint64_t rows, void *ws,
                             uint32_t *tickets) {
    const GemmPlan plan = gemm_plan(n_in, n_out, rows, dtype);
    uint8_t *xq = static_cast<uint8_t *>(ws);
    void *partials = xq + ((plan.xq_bytes + 255) & ~255ull);
    hipError_t err = launch_quantize_x(x, n_in, rows, xq, stream);
    if (err == hipSuccess)
        err = launch_gemm_q(w, dtype, xq, out, n_in, n_out, rows, plan, partials, tickets, stream);
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "verify GEMM launch: %s", hip_error(err));
    return YUUKA_OK;
}

uint64_t verify_gemm_ws_bytes(uint64_t n_in, uint64_t n_out, uint64_t rows, uint32_t dtype) {
    const GemmPlan plan = gemm_plan(n_in, n_out, rows, dtype);
    return ((plan.xq_bytes + 255) & ~255ull) + plan.part_bytes + 256;
}

uint32_t verify_gemm_tickets(uint64_t n_in, uint64_t n_out, uint64_t rows, uint32_t dtype) {
    return gemm_plan(n_in, n_out, rows, dtype).tickets;
}

}  // namespace yk

using namespace yk;

#define UNSUPPORTED_ENTRY(name) \
    return fail(YUUKA_ERR_UNSUPPORTED, "%s is outside the verify path served by this library", name)

extern "C" {

uint32_t yuuka_abi_version(void) { return YUUKA_HIP_ABI_VERSION; }
uint32_t yuuka_ext_version(void) { return YUUKA_EXT_VERSION; }
const char *yuuka_last_error(void) { return g_last_error.c_str(); }

// Fixed scratch of yuuka_verify_accept_noalloc. Each GPU the library runs
// on holds its own copy until the process ends. In host code `scratch` only
// names the symbol: its device address (per GPU) comes from
// hipGetSymbolAddress, called once per device with that device current.
static __device__ __align__(256) uint8_t scratch[YUUKA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's scratch array; the device must be current.
yuuka_status noalloc_scratch_address(int index, void **out) {
    if (index < 0 || index >= kMaxDevices)
        return fail(YUUKA_ERR_UNSUPPORTED, "device index %d beyond the no-allocation table", index);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[index]) {
        void *p = nullptr;
        hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p)
            return fail(YUUKA_ERR_DEVICE, "scratch symbol address: %s", hip_error(err));
        g_scratch_ptr[index] = p;
    }
    *out = g_scratch_ptr[index];
    return YUUKA_OK;
}
}  // namespace

yuuka_status yuuka_device_open(int32_t index, yuuka_device **out) {
    return guard("device_open", [&]() -> yuuka_status {
        if (!out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null output handle");
        *out = nullptr;
        int count = 0;
        hipError_t err = hipGetDeviceCount(&count);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "device count: %s", hip_error(err));
        if (index < 0 || index >= count)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "device index %d outside 0..%d", index, count - 1);
        err = hipSetDevice(index);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "set device: %s", hip_error(err));
        auto *dev = new yuuka_device();
        dev->index = index;
        err = hipGetDeviceProperties(&dev->props, index);
        if (err != hipSuccess) {
            delete dev;
            return fail(YUUKA_ERR_DEVICE, "device properties: %s", hip_error(err));
        }
        yuuka_status st = noalloc_scratch_address(index, &dev->noalloc_scratch);
        if (st != YUUKA_OK) {
            delete dev;
            return st;
        }
        *out = dev;
        return YUUKA_OK;
    });
}

void yuuka_device_close(yuuka_device *dev) { delete dev; }

yuuka_status yuuka_device_info_get(const yuuka_device *dev, yuuka_device_info *info) {
    return guard("device_info", [&]() -> yuuka_status {
        if (!dev || !info) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null device or info");
        std::memset(info, 0, sizeof(*info));
        std::snprintf(info->name, sizeof(info->name), "%s", dev->props.name);
        std::snprintf(info->gcn_arch, sizeof(info->gcn_arch), "%s", dev->props.gcnArchName);
        int rt = 0;
        (void)hipRuntimeGetVersion(&rt);
        std::snprintf(info->hip_version, sizeof(info->hip_version), "%d", rt);
        info->total_memory = dev->props.totalGlobalMem;
        info->compute_units = (uint32_t)dev->props.multiProcessorCount;
        info->clock_mhz = (uint32_t)(dev->props.clockRate / 1000);
        info->pci_domain = dev->props.pciDomainID;
        info->pci_bus = dev->props.pciBusID;
        info->pci_device = dev->props.pciDeviceID;
        return YUUKA_OK;
    });
}

yuuka_status yuuka_buffer_alloc(yuuka_device *dev, uint64_t bytes, yuuka_buffer **out) {
    return guard("buffer_alloc", [&]() -> yuuka_status {
        if (!dev || !out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null device or output");
        *out = nullptr;
        if (bytes == 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "zero-byte allocation");
        hipError_t err = hipSetDevice(dev->index);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "set device: %s", hip_error(err));
        void *ptr = nullptr;
        err = hipMalloc(&ptr, bytes);
        if (err != hipSuccess)
            return fail(YUUKA_ERR_ALLOCATION, "hipMalloc(%llu): %s", (unsigned long long)bytes,
                        hip_error(err));
        auto *b = new yuuka_buffer();
        b->dev = dev;
        b->ptr = ptr;
        b->bytes = bytes;
        *out = b;
        return YUUKA_OK;
    });
}

void yuuka_buffer_free(yuuka_buffer *buf) {
    if (!buf) return;
    if (buf->ptr) (void)hipFree(buf->ptr);
    delete buf;
}

uint64_t yuuka_buffer_size(const yuuka_buffer *buf) { return buf ? buf->bytes : 0; }
void *yuuka_buffer_ptr(const yuuka_buffer *buf) { return buf ? buf->ptr : nullptr; }

yuuka_status yuuka_stream_create(yuuka_device *dev, yuuka_stream **out) {
    return guard("stream_create", [&]() -> yuuka_status {
        if (!dev || !out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null device or output");
        *out = nullptr;
        hipError_t err = hipSetDevice(dev->index);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "set device: %s", hip_error(err));
        auto *s = new yuuka_stream();
        s->dev = dev;
        err = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
        if (err != hipSuccess) {
            delete s;
            return fail(YUUKA_ERR_DEVICE, "stream create: %s", hip_error(err));
        }
        *out = s;
        return YUUKA_OK;
    });
}

void yuuka_stream_destroy(yuuka_stream *stream) {
    if (!stream) return;
    (void)hipStreamSynchronize(stream->stream);
    if (stream->scratch.ptr) (void)hipFree(stream->scratch.ptr);
    if (stream->tickets.ptr) (void)hipFree(stream->tickets.ptr);
    (void)hipStreamDestroy(stream->stream);
    delete stream;
}

yuuka_status yuuka_stream_synchronize(yuuka_stream *stream) {
    return guard("stream_synchronize", [&]() -> yuuka_status {
        if (!stream) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null stream");
        hipError_t err = hipStreamSynchronize(stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "stream synchronize: %s", hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_event_create(yuuka_device *dev, yuuka_event **out) {
    return guard("event_create", [&]() -> yuuka_status {
        if (!dev || !out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null device or output");
        *out = nullptr;
        auto *e = new yuuka_event();
        hipError_t err = hipEventCreateWithFlags(&e->event, hipEventDisableTiming);
        if (err != hipSuccess) {
            delete e;
            return fail(YUUKA_ERR_DEVICE, "event create: %s", hip_error(err));
        }
        *out = e;
        return YUUKA_OK;
    });
}

void yuuka_event_destroy(yuuka_event *event) {
    if (!event) return;
    (void)hipEventDestroy(event->event);
    delete event;
}

yuuka_status yuuka_event_wait(yuuka_event *event) {
    return guard("event_wait", [&]() -> yuuka_status {
        if (!event) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null event");
        hipError_t err = hipEventSynchronize(event->event);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "event wait: %s", hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_memcpy_h2d(yuuka_buffer *dst, const void *src, uint64_t bytes) {
    return guard("memcpy_h2d", [&]() -> yuuka_status {
        if (!dst || (!src && bytes)) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null buffer or source");
        if (bytes > dst->bytes) return fail(YUUKA_ERR_INVALID_ARGUMENT, "copy exceeds buffer");
        if (!bytes) return YUUKA_OK;
        hipError_t err = hipMemcpy(dst->ptr, src, bytes, hipMemcpyHostToDevice);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "memcpy h2d: %s", hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_memcpy_d2h(void *dst, const yuuka_buffer *src, uint64_t bytes) {
    return yuuka_memcpy_d2h_at(dst, src, 0, bytes);
}

yuuka_status yuuka_memcpy_d2h_at(void *dst, const yuuka_buffer *src, uint64_t offset, uint64_t bytes) {
    return guard("memcpy_d2h", [&]() -> yuuka_status {
        if (!src || (!dst && bytes)) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null buffer or destination");
        if (!range_ok(src, offset, bytes)) return fail(YUUKA_ERR_INVALID_ARGUMENT, "copy exceeds buffer");
        if (!bytes) return YUUKA_OK;
        hipError_t err = hipMemcpy(dst, static_cast<const uint8_t *>(src->ptr) + offset, bytes,
                                   hipMemcpyDeviceToHost);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "memcpy d2h: %s", hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_memset(yuuka_stream *stream, yuuka_buffer *dst, int value, uint64_t bytes) {
    return guard("memset", [&]() -> yuuka_status {
        if (!stream || !dst) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null stream or buffer");
        if (bytes > dst->bytes) return fail(YUUKA_ERR_INVALID_ARGUMENT, "memset exceeds buffer");
        hipError_t err = hipMemsetAsync(dst->ptr, value, bytes, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "memset: %s", hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_buffer_copy(yuuka_stream *stream, yuuka_buffer *dst, uint64_t dst_offset,
                               const yuuka_buffer *src, uint64_t src_offset, uint64_t bytes,
                               yuuka_event *completion) {
    return guard("buffer_copy", [&]() -> yuuka_status {
        if (!stream || !dst || !src) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (!range_ok(dst, dst_offset, bytes) || !range_ok(src, src_offset, bytes))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "copy range exceeds a buffer");
        if (bytes) {
            hipError_t err = hipMemcpyAsync(static_cast<uint8_t *>(dst->ptr) + dst_offset,
                                            static_cast<const uint8_t *>(src->ptr) + src_offset, bytes,
                                            hipMemcpyDeviceToDevice, stream->stream);
            if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "buffer copy: %s", hip_error(err));
        }
        return record(stream, completion);
    });
}

yuuka_status yuuka_dynamic_set(yuuka_stream *stream, yuuka_buffer *dynamic, int32_t token,
                               uint32_t position) {
    return guard("dynamic_set", [&]() -> yuuka_status {
        if (!stream || !dynamic) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (dynamic->bytes < 8) return fail(YUUKA_ERR_INVALID_ARGUMENT, "dynamic buffer under 8 bytes");
        const int32_t v[2] = {token, (int32_t)position};
        hipError_t err = hipMemcpyAsync(dynamic->ptr, v, 8, hipMemcpyHostToDevice, stream->stream);
        if (err == hipSuccess) err = hipStreamSynchronize(stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "dynamic set: %s", hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_add_f32(yuuka_stream *stream, yuuka_buffer *dst, const yuuka_buffer *a,
                           const yuuka_buffer *b, uint64_t n, yuuka_event *completion) {
    return guard("add_f32", [&]() -> yuuka_status {
        if (!stream || !dst || !a || !b) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (!range_ok(dst, 0, n * 4) || !range_ok(a, 0, n * 4) || !range_ok(b, 0, n * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "add exceeds a buffer");
        hipError_t err = launch_add_f32(static_cast<float *>(dst->ptr), static_cast<const float *>(a->ptr),
                                        static_cast<const float *>(b->ptr), n, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "add launch: %s", hip_error(err));
        return record(stream, completion);
    });
}

static yuuka_status direct_gemm(const char *what, yuuka_stream *stream, yuuka_buffer *out,
                                const yuuka_buffer *x, const yuuka_buffer *w, uint64_t n_in,
                                uint64_t n_out, uint64_t rows, uint32_t dtype,
                                yuuka_event *completion) {
    return guard(what, [&]() -> yuuka_status {
        if (!stream || !out || !x || !w) return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: null argument", what);
        yuuka_status st = check_verify_gemm(n_in, n_out, rows, dtype, 16);
        if (st != YUUKA_OK) return st;
        if (!range_ok(w, 0, row_bytes(dtype, n_in) * n_out))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s weight buffer is too small", what);
        if (!range_ok(x, 0, n_in * rows * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s input buffer is too small", what);
        if (!range_ok(out, 0, n_out * rows * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s output buffer is too small", what);
        yuuka_op op{};
        op.code = YUUKA_OP_LM_HEAD;
        op.buf[0] = const_cast<yuuka_buffer *>(w);
        op.buf[1] = const_cast<yuuka_buffer *>(x);
        op.buf[2] = out;
        op.n[0] = n_in;
        op.n[1] = n_out;
        op.n[2] = rows;
        op.u[0] = dtype;
        uint64_t ws = 0;
        uint32_t tickets = 0;
        st = verify_gemm_op_needs(op, &ws, &tickets);
        if (st != YUUKA_OK) return st;
        st = ensure_scratch(stream, &stream->scratch, ws + 256);
        if (st != YUUKA_OK) return st;
        st = ensure_scratch(stream, &stream->tickets, (uint64_t)tickets * 4 + 4);
        if (st != YUUKA_OK) return st;
        st = run_verify_gemm_op(op, stream->stream, stream->scratch.ptr, static_cast<uint32_t *>(stream->tickets.ptr));
        if (st != YUUKA_OK) return st;
        return record(stream, completion);
    });
}

yuuka_status yuuka_lm_head(yuuka_stream *stream, yuuka_buffer *out, const yuuka_buffer *x,
                           const yuuka_buffer *w, uint64_t n_in, uint64_t n_out, uint64_t rows,
                           uint32_t dtype, yuuka_event *completion) {
    return direct_gemm("lm_head", stream, out, x, w, n_in, n_out, rows, dtype, completion);
}

yuuka_status yuuka_gemv(yuuka_stream *stream, yuuka_buffer *out, const yuuka_buffer *x,
                        const yuuka_buffer *w, uint64_t n_in, uint64_t n_out, uint32_t dtype,
                        yuuka_event *completion) {
    return direct_gemm("gemv", stream, out, x, w, n_in, n_out, 1, dtype, completion);
}

yuuka_status yuuka_gemv_batch(yuuka_stream *stream, yuuka_buffer *out, const yuuka_buffer *x,
                              const yuuka_buffer *w, uint64_t n_in, uint64_t n_out, uint64_t batch,
                              uint32_t dtype, yuuka_event *completion) {
    return direct_gemm("gemv_batch", stream, out, x, w, n_in, n_out, batch, dtype, completion);
}

yuuka_status yuuka_gemm(yuuka_stream *, yuuka_buffer *, const yuuka_buffer *, const yuuka_buffer *,
                        uint64_t, uint64_t, uint64_t, uint32_t, yuuka_event *) {
    UNSUPPORTED_ENTRY("yuuka_gemm (prefill GEMM)");
}
yuuka_status yuuka_gemm_wmma(yuuka_stream *, yuuka_buffer *, const yuuka_buffer *, const yuuka_buffer *,
                             uint64_t, uint64_t, uint64_t, uint32_t, yuuka_event *) {
    UNSUPPORTED_ENTRY("yuuka_gemm_wmma (rocWMMA prefill GEMM)");
}
// Q8_1 activations of the int8 decode matvec (reference mmq_gemm.hip
// quantize_q8_1_kernel contract): qs[n * batch] int8 digits, ds[n * batch /
// 32] {d, d * sum} pairs; n a multiple of 128.
yuuka_status yuuka_quantize_q8_1(yuuka_stream *stream, yuuka_buffer *qs, yuuka_buffer *ds, const yuuka_buffer *x,
                                 uint64_t n, uint64_t batch, yuuka_event *completion) {
    return guard("quantize_q8_1", [&]() -> yuuka_status {
        if (!stream || !qs || !ds || !x) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (!n || n % 128 || !batch) return fail(YUUKA_ERR_INVALID_ARGUMENT, "Q8_1 width must be a multiple of 128");
        const uint64_t total = n * batch;
        if (!range_ok(x, 0, total * 4) || !range_ok(qs, 0, total) || !range_ok(ds, 0, total / 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "Q8_1 buffers too small");
        hipError_t err = launch_quant_q8_1(static_cast<const float *>(x->ptr), nullptr, qs->ptr, ds->ptr, total,
                                           stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "quantize launch: %s", hip_error(err));
        return record(stream, completion);
    });
}
yuuka_status yuuka_gemm_mmq(yuuka_stream *, yuuka_buffer *, const yuuka_buffer *, const yuuka_buffer *,
                            const yuuka_buffer *, uint64_t, uint64_t, uint64_t, uint32_t, yuuka_event *) {
    UNSUPPORTED_ENTRY("yuuka_gemm_mmq (MMQ prefill route)");
}
yuuka_status yuuka_gemm_blas(yuuka_stream *, yuuka_buffer *, yuuka_buffer *, const yuuka_buffer *,
                             const yuuka_buffer *, uint64_t, uint64_t, uint64_t, yuuka_event *) {
    UNSUPPORTED_ENTRY("yuuka_gemm_blas (rocBLAS prefill route)");
}

static yuuka_status dequant_entry(const char *what, yuuka_stream *stream, yuuka_buffer *dst,
                                  const yuuka_buffer *src, uint64_t n_in, uint64_t n_out,
                                  uint32_t dtype, uint64_t elem_bytes, yuuka_event *completion) {
    return guard(what, [&]() -> yuuka_status {
        if (!stream || !dst || !src) return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: null argument", what);
        const uint64_t rb = row_bytes(dtype, n_in);
        if (rb == 0 || dtype == YUUKA_DTYPE_Q4_0 || dtype == YUUKA_DTYPE_Q5_0)
            return fail(YUUKA_ERR_UNSUPPORTED, "%s: dtype %u / width %llu unsupported", what, dtype,
                        (unsigned long long)n_in);
        if (n_out == 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: zero rows", what);
        if (!range_ok(src, 0, rb * n_out)) return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: source too small", what);
        if (!range_ok(dst, 0, n_in * n_out * elem_bytes))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: destination too small", what);
        hipError_t err = elem_bytes == 4
                             ? launch_dequant_f32(src->ptr, dtype, static_cast<float *>(dst->ptr), n_in, n_out, stream->stream)
                             : launch_dequant_f16(src->ptr, dtype, static_cast<uint16_t *>(dst->ptr), n_in, n_out, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "%s launch: %s", what, hip_error(err));
        return record(stream, completion);
    });
}

yuuka_status yuuka_dequant_f32(yuuka_stream *stream, yuuka_buffer *dst, const yuuka_buffer *src,
                               uint64_t n_in, uint64_t n_out, uint32_t dtype, yuuka_event *completion) {
    return dequant_entry("dequant_f32", stream, dst, src, n_in, n_out, dtype, 4, completion);
}

yuuka_status yuuka_dequant_f16(yuuka_stream *stream, yuuka_buffer *dst, const yuuka_buffer *src,
                               uint64_t n_in, uint64_t n_out, uint32_t dtype, yuuka_event *completion) {
    return dequant_entry("dequant_f16", stream, dst, src, n_in, n_out, dtype, 2, completion);
}

yuuka_status yuuka_cast_f32_to_f16(yuuka_stream *stream, yuuka_buffer *dst, const yuuka_buffer *src,
                                   uint64_t n, yuuka_event *completion) {
    return guard("cast_f16", [&]() -> yuuka_status {
        if (!stream || !dst || !src) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (!range_ok(src, 0, n * 4) || !range_ok(dst, 0, n * 2))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "cast exceeds a buffer");
        hipError_t err = launch_cast_f16(static_cast<const float *>(src->ptr),
                                         static_cast<uint16_t *>(dst->ptr), n, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "cast launch: %s", hip_error(err));
        return record(stream, completion);
    });
}

yuuka_status yuuka_moe_pack_q4k(yuuka_stream *stream, yuuka_buffer *dst, const yuuka_buffer *src, uint64_t rows,
                                uint64_t n_in, yuuka_event *completion) {
    return guard("moe_pack_q4k", [&]() -> yuuka_status {
        if (!stream || !dst || !src) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (rows == 0 || rows % 16 || n_in == 0 || n_in % 256 || n_in > (1u << 30))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE pack: %llu rows of %llu columns (rows %% 16, columns %% 256)",
                        (unsigned long long)rows, (unsigned long long)n_in);
        const uint64_t bytes = rows * (n_in / 256) * 144;
        if (!range_ok(src, 0, bytes) || !range_ok(dst, 0, bytes))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE pack exceeds a buffer");
        const uintptr_t d = reinterpret_cast<uintptr_t>(dst->ptr), r = reinterpret_cast<uintptr_t>(src->ptr);
        if (d < r + bytes && r < d + bytes) return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE pack buffers overlap");
        hipError_t err = launch_moe_pack_q4k(src->ptr, dst->ptr, rows, (int)n_in, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "MoE pack launch: %s", hip_error(err));
        return record(stream, completion);
    });
}

// Shared argument checks of the acceptance entry points.
static yuuka_status check_accept(const yuuka_accept_params &p, const yuuka_buffer *logits, uint64_t logits_offset,
                                 const yuuka_buffer *drafts, uint64_t drafts_offset, const yuuka_buffer *result,
                                 uint64_t result_offset, const yuuka_buffer *debug) {
    if (p.mode != YUUKA_ACCEPT_GREEDY && p.mode != YUUKA_ACCEPT_STOCHASTIC)
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "unknown accept mode %u", p.mode);
    if (p.batch == 0 || p.vocab == 0 || p.vocab > (1u << 30) || p.drafts > 255)
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid batch %u, drafts %u or vocab %u", p.batch,
                    p.drafts, p.vocab);
    if (p.mode == YUUKA_ACCEPT_STOCHASTIC && !(p.top_p >= 0.0f && p.top_p <= 1.0f) && p.top_p != 0.0f)
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "top-p must be in (0,1]");
    const uint64_t stride = p.row_stride ? p.row_stride : p.vocab;
    if (stride < p.vocab) return fail(YUUKA_ERR_INVALID_ARGUMENT, "row stride below vocab");
    const uint64_t rows = (uint64_t)p.batch * (p.drafts + 1);
    if (logits_offset % 4 || !range_ok(logits, logits_offset, ((rows - 1) * stride + p.vocab) * 4))
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "logits buffer too small or misaligned");
    if (p.drafts > 0 && (!drafts || drafts_offset % 4 ||
                         !range_ok(drafts, drafts_offset, (uint64_t)p.batch * p.drafts * 4)))
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "drafts buffer too small or misaligned");
    if (result_offset % 4 || !range_ok(result, result_offset, (uint64_t)p.batch * 16))
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "result buffer too small or misaligned");
    if (debug && !range_ok(debug, 0, rows * 32))
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "debug buffer too small");
    return YUUKA_OK;
}

yuuka_status yuuka_verify_accept(yuuka_stream *stream, const yuuka_buffer *logits,
                                 uint64_t logits_offset, const yuuka_buffer *drafts,
                                 uint64_t drafts_offset, yuuka_buffer *result,
                                 uint64_t result_offset, yuuka_buffer *debug,
                                 const yuuka_accept_params *params, yuuka_event *completion) {
    return guard("verify_accept", [&]() -> yuuka_status {
        if (!stream || !logits || !result || !params)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        const yuuka_accept_params &p = *params;
        yuuka_status st = check_accept(p, logits, logits_offset, drafts, drafts_offset, result, result_offset,
                                       debug);
        if (st != YUUKA_OK) return st;
        st = ensure_scratch(stream, &stream->scratch, accept_scratch_bytes(p));
        if (st != YUUKA_OK) return st;
        const int32_t *dp = p.drafts > 0
                                ? reinterpret_cast<const int32_t *>(static_cast<const uint8_t *>(drafts->ptr) + drafts_offset)
                                : nullptr;
        hipError_t err = launch_verify_accept(
            reinterpret_cast<const float *>(static_cast<const uint8_t *>(logits->ptr) + logits_offset), dp,
            reinterpret_cast<int32_t *>(static_cast<uint8_t *>(result->ptr) + result_offset),
            debug ? static_cast<double *>(debug->ptr) : nullptr, p, stream->scratch.ptr, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "accept launch: %s", hip_error(err));
        return record(stream, completion);
    });
}


uint64_t yuuka_noalloc_accept_bytes(const yuuka_accept_params *params) {
    return params ? accept_scratch_bytes(*params) : 0;
}

yuuka_status yuuka_verify_accept_noalloc(yuuka_stream *stream, const yuuka_buffer *logits,
                                         uint64_t logits_offset, const yuuka_buffer *drafts,
                                         uint64_t drafts_offset, yuuka_buffer *result,
                                         uint64_t result_offset, const yuuka_accept_params *params,
                                         yuuka_event *completion) {
    return guard("verify_accept_noalloc", [&]() -> yuuka_status {
        if (!stream || !stream->dev || !logits || !result || !params)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        const yuuka_accept_params &p = *params;
        yuuka_status st = check_accept(p, logits, logits_offset, drafts, drafts_offset, result, result_offset,
                                       nullptr);
        if (st != YUUKA_OK) return st;
        const uint64_t need = accept_scratch_bytes(p);
        if (need > YUUKA_NOALLOC_SCRATCH_BYTES)
            return fail(YUUKA_ERR_INVALID_ARGUMENT,
                        "acceptance partials of %llu bytes exceed the fixed scratch of %u bytes",
                        (unsigned long long)need, (unsigned)YUUKA_NOALLOC_SCRATCH_BYTES);
        if (!stream->dev->noalloc_scratch) return fail(YUUKA_ERR_DEVICE, "no scratch address for this device");
        const int32_t *dp = p.drafts > 0
                                ? reinterpret_cast<const int32_t *>(static_cast<const uint8_t *>(drafts->ptr) + drafts_offset)
                                : nullptr;
        hipError_t err = launch_verify_accept(
            reinterpret_cast<const float *>(static_cast<const uint8_t *>(logits->ptr) + logits_offset), dp,
            reinterpret_cast<int32_t *>(static_cast<uint8_t *>(result->ptr) + result_offset), nullptr, p,
            stream->dev->noalloc_scratch, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "accept launch: %s", hip_error(err));
        return record(stream, completion);
    });
}

yuuka_status yuuka_event_create_timed(yuuka_device *dev, yuuka_event **out) {
    return guard("event_create_timed", [&]() -> yuuka_status {
        if (!dev || !out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null device or output");
        *out = nullptr;
        auto *e = new yuuka_event();
        hipError_t err = hipEventCreate(&e->event);
        if (err != hipSuccess) {
            delete e;
            return fail(YUUKA_ERR_DEVICE, "event create: %s", hip_error(err));
        }
        *out = e;
        return YUUKA_OK;
    });
}

yuuka_status yuuka_event_record(yuuka_event *event, yuuka_stream *stream) {
    return guard("event_record", [&]() -> yuuka_status {
        if (!event || !stream) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null event or stream");
        hipError_t err = hipEventRecord(event->event, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "event record: %s", hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_event_elapsed_ms(yuuka_event *start, yuuka_event *end, float *ms) {
    return guard("event_elapsed", [&]() -> yuuka_status {
        if (!start || !end || !ms) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        hipError_t err = hipEventElapsedTime(ms, start->event, end->event);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "event elapsed: %s", hip_error(err));
        return YUUKA_OK;
    });
}

uint64_t yuuka_quantized_bytes(uint64_t n_in, uint64_t rows) {
    if (n_in == 0 || n_in % 256 || rows == 0 || rows > 16) return 0;
    return gemm_plan(n_in, 1, rows, YUUKA_DTYPE_Q4_K).xq_bytes;
}

yuuka_status yuuka_quantize_activations(yuuka_stream *stream, yuuka_buffer *xq, const yuuka_buffer *x,
                                        uint64_t n_in, uint64_t rows, yuuka_event *completion) {
    return guard("quantize_activations", [&]() -> yuuka_status {
        if (!stream || !xq || !x) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        const uint64_t need = yuuka_quantized_bytes(n_in, rows);
        if (!need) return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid width %llu or rows %llu",
                               (unsigned long long)n_in, (unsigned long long)rows);
        if (!range_ok(xq, 0, need) || !range_ok(x, 0, n_in * rows * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "quantize buffers too small");
        hipError_t err = launch_quantize_x(static_cast<const float *>(x->ptr), n_in, rows, xq->ptr, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "quantize launch: %s", hip_error(err));
        return record(stream, completion);
    });
}

yuuka_status yuuka_gemm_quantized(yuuka_stream *stream, yuuka_buffer *out, const yuuka_buffer *xq,
                                  const yuuka_buffer *w, uint64_t n_in, uint64_t n_out, uint64_t rows,
                                  uint32_t dtype, yuuka_event *completion) {
    return guard("gemm_quantized", [&]() -> yuuka_status {
        if (!stream || !out || !xq || !w) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        yuuka_status st = check_verify_gemm(n_in, n_out, rows, dtype, 16);
        if (st != YUUKA_OK) return st;
        const GemmPlan plan = gemm_plan(n_in, n_out, rows, dtype);
        if (!range_ok(w, 0, row_bytes(dtype, n_in) * n_out) || !range_ok(xq, 0, plan.xq_bytes) ||
            !range_ok(out, 0, n_out * rows * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "gemm buffers too small");
        st = ensure_scratch(stream, &stream->scratch, plan.part_bytes + 256);
        if (st != YUUKA_OK) return st;
        st = ensure_scratch(stream, &stream->tickets, (uint64_t)plan.tickets * 4 + 4);
        if (st != YUUKA_OK) return st;
        hipError_t err = launch_gemm_q(w->ptr, dtype, xq->ptr, static_cast<float *>(out->ptr), n_in, n_out,
                                       rows, plan, stream->scratch.ptr,
                                       static_cast<uint32_t *>(stream->tickets.ptr), stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "gemm launch: %s", hip_error(err));
        return record(stream, completion);
    });
}

}  // extern "C"
