// The C-ABI's plumbing: error state, device queries, device memory, streams and events, the host half of numpy
// broadcasting, and the calibration copy kernel.
#include <algorithm>
#include <cstdio>
#include <mutex>
#include <vector>

#include "common.h"

namespace xs_hip {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return XS_HIP_OK;
    return fail(XS_HIP_ERUNTIME, std::string(what) + ": " + hipGetErrorString(e));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

const char* dtype_name(xs_dtype t) {
    switch (t) {
        case XS_F32: return "f32";
        case XS_F16: return "f16";
        case XS_BF16: return "bf16";
        case XS_I64: return "i64";
        case XS_I32: return "i32";
        case XS_I8: return "i8";
        case XS_U8: return "u8";
        case XS_BOOL: return "bool";
    }
    return "unknown";
}

int device_cus() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (static_cast<size_t>(dev) >= cache.size()) cache.resize(static_cast<size_t>(dev) + 1, 0);
    if (cache[static_cast<size_t>(dev)] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        cache[static_cast<size_t>(dev)] = cus;
    }
    return cache[static_cast<size_t>(dev)];
}

namespace {

// Threads of a copy workgroup.
constexpr int kCopyBlock = 64;

// y = x in 16-byte vectors, one per lane: a tile of kCopyBlock vectors per workgroup, as many workgroups as tiles.
__global__ __launch_bounds__(kCopyBlock) void copy_kernel(const u32x4* __restrict__ x, u32x4* __restrict__ y,
                                                          int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kCopyBlock + threadIdx.x;
    if (i < n) st128_nt(y + i, ld128_nt(x + i));
}

// y[r, :] = x[r, :] for rows of `cols` elements of type E, rows `xs` / `ys` bytes apart: grid (column tiles, row
// groups), each workgroup walking its rows gridDim.y apart.
// Non-temporal loads and stores: the gate half of config 1's fused [2048, 19456] bf16 buffer in 14.4 us against
// 17.1 us with plain ones, on MI355X (a 40 MiB copy: 14.0 us).
template <typename E>
__global__ __launch_bounds__(kBlock) void copy_rows_kernel(const char* __restrict__ x, int64_t xs, char* __restrict__ y,
                                                           int64_t ys, int64_t rows, int64_t cols) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= cols) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y)
        __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const E*>(x + r * xs) + c),
                                    reinterpret_cast<E*>(y + r * ys) + c);
}

}  // namespace

}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

const char* xs_hip_last_error(void) { return g_last_error.c_str(); }

int xs_hip_abi_version(void) { return 1; }

int xs_hip_broadcast_fill(xs_broadcast* bc, const int64_t* a_shape, int32_t a_rank, const int64_t* b_shape,
                          int32_t b_rank) {
    if (bc == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_broadcast_fill: null descriptor");
    if (a_rank < 0 || b_rank < 0 || a_rank > XS_MAX_RANK || b_rank > XS_MAX_RANK)
        return fail(XS_HIP_EINVAL, "xs_hip_broadcast_fill: ranks " + std::to_string(a_rank) + " and " +
                                       std::to_string(b_rank) + " exceed " + std::to_string(XS_MAX_RANK));
    if ((a_rank > 0 && a_shape == nullptr) || (b_rank > 0 && b_shape == nullptr))
        return fail(XS_HIP_EINVAL, "xs_hip_broadcast_fill: null shape");
    const int rank = std::max(a_rank, b_rank);
    *bc = xs_broadcast{};
    bc->rank = rank;
    // Shapes align on the right; a dim of 1 stretches (cpu_ref::broadcast_shape, ops.cpp:42-53).
    for (int i = 0; i < rank; ++i) {
        const int64_t da = i < rank - a_rank ? 1 : a_shape[i - (rank - a_rank)];
        const int64_t db = i < rank - b_rank ? 1 : b_shape[i - (rank - b_rank)];
        if (da < 0 || db < 0 || !(da == db || da == 1 || db == 1)) {
            std::string sa, sb;
            for (int k = 0; k < a_rank; ++k) sa += (k ? "," : "") + std::to_string(a_shape[k]);
            for (int k = 0; k < b_rank; ++k) sb += (k ? "," : "") + std::to_string(b_shape[k]);
            return fail(XS_HIP_EINVAL, "cannot broadcast [" + sa + "] with [" + sb + "]");
        }
        bc->out[i] = da == 1 ? db : da;
    }
    // Row-major strides aligned to out, 0 on broadcast dims (cpu_ref::broadcast_strides, ops.cpp:55-66).
    int64_t sa = 1, sb = 1, sy = 1;
    for (int i = rank - 1; i >= 0; --i) {
        const int ia = i - (rank - a_rank), ib = i - (rank - b_rank);
        if (ia >= 0) {
            bc->stride_a[i] = a_shape[ia] == 1 ? 0 : sa;
            sa *= a_shape[ia];
        }
        if (ib >= 0) {
            bc->stride_b[i] = b_shape[ib] == 1 ? 0 : sb;
            sb *= b_shape[ib];
        }
        bc->stride_y[i] = sy;
        sy *= bc->out[i];
    }
    return XS_HIP_OK;
}

int xs_hip_device_count(int* count) {
    if (count == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_device_count: null output");
    return check_hip(hipGetDeviceCount(count), "hipGetDeviceCount");
}

int xs_hip_device_info(int device, char* name, size_t name_len, uint64_t* memory_bytes, int* compute_units) {
    hipDeviceProp_t p;
    const int rc = check_hip(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
    if (rc != XS_HIP_OK) return rc;
    if (name != nullptr && name_len > 0) {
        // The marketing name can be empty (seen on MI355X boxes); the arch, CU count and memory always identify it.
        std::snprintf(name, name_len, "%s%s%s, %d CUs, %.0f GiB", p.name, p.name[0] != '\0' ? " " : "", p.gcnArchName,
                      p.multiProcessorCount, static_cast<double>(p.totalGlobalMem) / (1u << 30));
    }
    if (memory_bytes != nullptr) *memory_bytes = p.totalGlobalMem;
    if (compute_units != nullptr) *compute_units = p.multiProcessorCount;
    return XS_HIP_OK;
}

int xs_hip_set_device(int device) { return check_hip(hipSetDevice(device), "hipSetDevice"); }

int xs_hip_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_malloc: null output");
    *ptr = nullptr;
    if (bytes == 0) return XS_HIP_OK;
    const hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        size_t free_b = 0, total_b = 0;
        (void)hipGetLastError();
        (void)hipMemGetInfo(&free_b, &total_b);
        return fail(XS_HIP_ERUNTIME, "xs_hip_malloc of " + std::to_string(bytes) + " bytes failed (" +
                                         hipGetErrorString(e) + "); free " + std::to_string(free_b) + " of " +
                                         std::to_string(total_b));
    }
    return XS_HIP_OK;
}

int xs_hip_free(void* ptr) { return ptr == nullptr ? XS_HIP_OK : check_hip(hipFree(ptr), "hipFree"); }

int xs_hip_memset(void* ptr, int value, size_t bytes, void* stream) {
    return check_hip(hipMemsetAsync(ptr, value, bytes, as_stream(stream)), "hipMemsetAsync");
}

int xs_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    int rc = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)), "memcpy h2d");
    if (rc != XS_HIP_OK) return rc;
    return check_hip(hipStreamSynchronize(as_stream(stream)), "memcpy h2d sync");
}

int xs_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    int rc = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)), "memcpy d2h");
    if (rc != XS_HIP_OK) return rc;
    return check_hip(hipStreamSynchronize(as_stream(stream)), "memcpy d2h sync");
}

int xs_hip_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)), "memcpy h2d");
}

int xs_hip_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)), "memcpy d2h");
}

int xs_hip_host_alloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_host_alloc: null output");
    *ptr = nullptr;
    if (bytes == 0) return XS_HIP_OK;
    return check_hip(hipHostMalloc(ptr, bytes, hipHostMallocDefault), "hipHostMalloc");
}

int xs_hip_host_free(void* ptr) { return ptr == nullptr ? XS_HIP_OK : check_hip(hipHostFree(ptr), "hipHostFree"); }

int xs_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)), "memcpy d2d");
}

int xs_hip_stream_create(void** stream) {
    if (stream == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_stream_create: null output");
    hipStream_t s = nullptr;
    // Default priority, non-blocking with respect to the null stream.
    const int rc = check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
    return rc;
}

int xs_hip_stream_destroy(void* stream) {
    return stream == nullptr ? XS_HIP_OK : check_hip(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
}

int xs_hip_stream_synchronize(void* stream) {
    return check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}

int xs_hip_device_synchronize(void) { return check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

int xs_hip_event_create(void** event) {
    if (event == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_event_create: null output");
    hipEvent_t e = nullptr;
    const int rc = check_hip(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return rc;
}

int xs_hip_event_destroy(void* event) {
    return event == nullptr ? XS_HIP_OK : check_hip(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}

int xs_hip_event_record(void* event, void* stream) {
    return check_hip(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)), "hipEventRecord");
}

int xs_hip_event_elapsed_ms(float* ms, void* start, void* end) {
    if (ms == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_event_elapsed_ms: null output");
    int rc = check_hip(hipEventSynchronize(static_cast<hipEvent_t>(end)), "hipEventSynchronize");
    if (rc != XS_HIP_OK) return rc;
    return check_hip(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)),
                     "hipEventElapsedTime");
}

int xs_hip_stream_begin_capture(void* stream) {
    if (stream == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_stream_begin_capture: the null stream cannot be captured");
    return check_hip(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
}

int xs_hip_stream_end_capture(void* stream, void** graph_exec) {
    if (graph_exec == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_stream_end_capture: null output");
    *graph_exec = nullptr;
    hipGraph_t graph = nullptr;
    int rc = check_hip(hipStreamEndCapture(as_stream(stream), &graph), "hipStreamEndCapture");
    if (rc != XS_HIP_OK) return rc;
    hipGraphExec_t exec = nullptr;
    rc = check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(graph);
    if (rc != XS_HIP_OK) return rc;
    *graph_exec = exec;
    return XS_HIP_OK;
}

int xs_hip_graph_launch(void* graph_exec, void* stream) {
    if (graph_exec == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_graph_launch: null graph");
    return check_hip(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)), "hipGraphLaunch");
}

int xs_hip_graph_destroy(void* graph_exec) {
    return graph_exec == nullptr ? XS_HIP_OK
                                 : check_hip(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)),
                                             "hipGraphExecDestroy");
}

int xs_hip_copy_rows(void* stream, const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride, int64_t rows,
                     int64_t row_bytes) {
    if (rows < 0 || row_bytes < 0 || x_row_stride < row_bytes || y_row_stride < row_bytes)
        return fail(XS_HIP_EINVAL, "xs_hip_copy_rows: " + std::to_string(rows) + " rows of " +
                                       std::to_string(row_bytes) + " bytes with strides " +
                                       std::to_string(x_row_stride) + ", " + std::to_string(y_row_stride));
    if (rows == 0 || row_bytes == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_copy_rows: null buffer");
    // The widest element that divides the row, both strides and both addresses.
    const uint64_t bits = static_cast<uint64_t>(row_bytes) | static_cast<uint64_t>(x_row_stride) |
                          static_cast<uint64_t>(y_row_stride) | reinterpret_cast<uintptr_t>(x) |
                          reinterpret_cast<uintptr_t>(y);
    const int64_t e = bits % 16 == 0 ? 16 : bits % 8 == 0 ? 8 : bits % 4 == 0 ? 4 : bits % 2 == 0 ? 2 : 1;
    const int64_t cols = row_bytes / e;
    const int64_t col_blocks = (cols + kBlock - 1) / kBlock;
    if (col_blocks > 0x7fffffffLL) return fail(XS_HIP_EUNSUPPORTED, "xs_hip_copy_rows: rows too long");
    const dim3 grid(static_cast<unsigned>(col_blocks), static_cast<unsigned>(rows < 65535 ? rows : 65535));
    const hipStream_t s = as_stream(stream);
    const char* xc = static_cast<const char*>(x);
    char* yc = static_cast<char*>(y);
    switch (e) {
        case 16: copy_rows_kernel<u32x4><<<grid, kBlock, 0, s>>>(xc, x_row_stride, yc, y_row_stride, rows, cols); break;
        case 8: copy_rows_kernel<uint64_t><<<grid, kBlock, 0, s>>>(xc, x_row_stride, yc, y_row_stride, rows, cols); break;
        case 4: copy_rows_kernel<uint32_t><<<grid, kBlock, 0, s>>>(xc, x_row_stride, yc, y_row_stride, rows, cols); break;
        case 2: copy_rows_kernel<uint16_t><<<grid, kBlock, 0, s>>>(xc, x_row_stride, yc, y_row_stride, rows, cols); break;
        default: copy_rows_kernel<uint8_t><<<grid, kBlock, 0, s>>>(xc, x_row_stride, yc, y_row_stride, rows, cols); break;
    }
    return check_launch("xs_hip_copy_rows");
}

int xs_hip_copy(void* stream, const void* x, void* y, size_t bytes) {
    if (bytes == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr || bytes % 16 != 0 || !aligned16(x) || !aligned16(y))
        return fail(XS_HIP_EINVAL, "xs_hip_copy: needs non-null 16-byte aligned buffers and a multiple of 16 bytes, got " +
                                       std::to_string(bytes));
    const int64_t n = static_cast<int64_t>(bytes / 16);
    if (n > 0xffffffffLL - kCopyBlock) return fail(XS_HIP_EUNSUPPORTED, "xs_hip_copy: too many bytes");
    copy_kernel<<<static_cast<unsigned>((n + kCopyBlock - 1) / kCopyBlock), kCopyBlock, 0, as_stream(stream)>>>(
        static_cast<const u32x4*>(x), static_cast<u32x4*>(y), n);
    return check_launch("xs_hip_copy");
}

}  // extern "C"
