// Context, device discovery, buffers, flags and timing.
//
// Mirrors the reference's Provider construction and buffer model
// (src/provider.rs:119-179, src/device.rs:41-92, src/kernels.rs:1630-1665,
// :2118-2164) with the HIP runtime: the kernels are compiled ahead of time
// for gfx950 into this library, so there is no runtime compiler step.
#include "common.hpp"

#include <cstdio>
#include <cstring>
#include <string>

namespace {
thread_local std::string g_last_error;
}

namespace mhip {

mhip_status fail(mhip_status status, const std::string& detail) {
    g_last_error = detail;
    return status;
}

mhip_status from_hip(hipError_t err, const char* what) {
    if (err == hipSuccess) return MHIP_OK;
    mhip_status status = MHIP_DRIVER_FAILED;
    if (err == hipErrorOutOfMemory || err == hipErrorMemoryAllocation) {
        status = MHIP_OUT_OF_DEVICE_MEMORY;
    } else if (err == hipErrorNoDevice || err == hipErrorInvalidDevice ||
               err == hipErrorInsufficientDriver || err == hipErrorNotInitialized) {
        status = MHIP_DEVICE_UNAVAILABLE;
    }
    // The HIP error string only: never an address or handle.
    return fail(status, std::string(what) + ": " + hipGetErrorString(err));
}

mhip_status check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return from_hip(err, what);
    return MHIP_OK;
}

}  // namespace mhip

extern "C" {

const char* mhip_last_error_detail(void) { return g_last_error.c_str(); }

const char* mhip_status_name(mhip_status status) {
    switch (status) {
        case MHIP_OK: return "Ok";
        case MHIP_SHAPE_UNSUPPORTED: return "ShapeUnsupported";
        case MHIP_DTYPE_UNSUPPORTED: return "DTypeUnsupported";
        case MHIP_LAYOUT_UNSUPPORTED: return "LayoutUnsupported";
        case MHIP_EXECUTION_FAILED: return "ExecutionFailed";
        case MHIP_OUT_OF_DEVICE_MEMORY: return "OutOfDeviceMemory";
        case MHIP_COMPILATION_FAILED: return "CompilationFailed";
        case MHIP_DRIVER_FAILED: return "DriverFailed";
        case MHIP_DEVICE_UNAVAILABLE: return "DeviceUnavailable";
        case MHIP_CAPTURE_UNSUPPORTED: return "CaptureUnsupported";
    }
    return "Unknown";
}

const char* mhip_version(void) { return "0.1.0"; }

mhip_status mhip_device_count(int* count) {
    if (!count) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "count is null");
    int n = 0;
    hipError_t err = hipGetDeviceCount(&n);
    // No driver, no device node or no GPU: zero devices, not an error
    // (graceful unavailability, src/provider.rs:1-35).
    *count = (err == hipSuccess && n > 0) ? n : 0;
    return MHIP_OK;
}

mhip_status mhip_ctx_create(int ordinal, mhip_ctx** out) {
    if (!out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "out is null");
    *out = nullptr;
    int n = 0;
    mhip_device_count(&n);
    if (ordinal < 0 || ordinal >= n)
        return mhip::fail(MHIP_DEVICE_UNAVAILABLE,
                          "no HIP device at ordinal " + std::to_string(ordinal));
    hipError_t err = hipSetDevice(ordinal);
    if (err != hipSuccess) return mhip::from_hip(err, "selecting the device");
    mhip_ctx* ctx = new mhip_ctx();
    ctx->device = ordinal;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, ordinal) == hipSuccess)
        ctx->compute_units = static_cast<uint32_t>(prop.multiProcessorCount);
    // Default priority stream, non-blocking with respect to the null stream.
    if ((err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess ||
        (err = hipMalloc(reinterpret_cast<void**>(&ctx->flags), 256)) != hipSuccess ||
        (err = hipMemset(ctx->flags, 0, 256)) != hipSuccess ||

        (err = hipEventCreate(&ctx->timer_start)) != hipSuccess ||
        (err = hipEventCreate(&ctx->timer_stop)) != hipSuccess) {
        mhip_status st = mhip::from_hip(err, "creating the device context");
        mhip_ctx_destroy(ctx);
        return st;
    }
    *out = ctx;
    return MHIP_OK;
}

mhip_status mhip_ctx_destroy(mhip_ctx* ctx) {
    if (!ctx) return MHIP_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->flags) (void)hipFree(ctx->flags);
    for (auto& table : ctx->rope_tables) (void)hipFree(table.device);
    if (ctx->workspace) (void)hipFree(ctx->workspace);

    if (ctx->timer_start) (void)hipEventDestroy(ctx->timer_start);
    if (ctx->timer_stop) (void)hipEventDestroy(ctx->timer_stop);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return MHIP_OK;
}

mhip_status mhip_device_query(mhip_ctx* ctx, mhip_device_info* info) {
    MHIP_REQUIRE_CTX(ctx);
    if (!info) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "info is null");
    std::memset(info, 0, sizeof(*info));
    hipDeviceProp_t prop;
    hipError_t err = hipGetDeviceProperties(&prop, ctx->device);
    if (err != hipSuccess) return mhip::from_hip(err, "reading device properties");
    info->ordinal = ctx->device;
    std::snprintf(info->name, sizeof(info->name), "%s", prop.name);
    std::snprintf(info->architecture, sizeof(info->architecture), "%s", prop.gcnArchName);
    info->total_memory = prop.totalGlobalMem;
    info->compute_units = static_cast<uint32_t>(prop.multiProcessorCount);
    info->wavefront_size = static_cast<uint32_t>(prop.warpSize);
    info->lds_per_workgroup = prop.sharedMemPerBlock;
    size_t free_b = 0, total_b = 0;
    (void)hipSetDevice(ctx->device);
    if (hipMemGetInfo(&free_b, &total_b) == hipSuccess && total_b > 0) {
        info->free_memory = free_b;
        double ratio = static_cast<double>(free_b) / static_cast<double>(total_b);
        info->pressure = ratio > 0.5 ? 0 : ratio > 0.2 ? 1 : ratio > 0.05 ? 2 : 3;
    } else {
        info->pressure = -1;
    }
    return MHIP_OK;
}

mhip_status mhip_alloc(mhip_ctx* ctx, size_t bytes, void** device_ptr) {
    MHIP_REQUIRE_CTX(ctx);
    if (!device_ptr) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "device_ptr is null");
    *device_ptr = nullptr;
    (void)hipSetDevice(ctx->device);
    // A zero-byte tensor still gets a distinct, valid allocation.
    hipError_t err = hipMalloc(device_ptr, bytes ? bytes : 256);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        std::string what = "allocating " + std::to_string(bytes) + " device bytes";
        return mhip::from_hip(err, what.c_str());
    }
    return MHIP_OK;
}

mhip_status mhip_free(mhip_ctx* ctx, void* device_ptr) {
    MHIP_REQUIRE_CTX(ctx);
    if (!device_ptr) return MHIP_OK;
    (void)hipSetDevice(ctx->device);
    return mhip::from_hip(hipFree(device_ptr), "freeing a device buffer");
}

mhip_status mhip_upload(mhip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    MHIP_REQUIRE_CTX(ctx);
    if (bytes == 0) return MHIP_OK;
    // Ordered after earlier kernels on the stream; waits for the copy so the
    // host buffer may be reused on return.
    hipError_t err = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    return mhip::from_hip(err, "uploading to the device");
}

mhip_status mhip_download(mhip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    MHIP_REQUIRE_CTX(ctx);
    if (bytes == 0) return mhip::from_hip(hipStreamSynchronize(ctx->stream), "synchronizing");
    hipError_t err = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    return mhip::from_hip(err, "downloading from the device");
}

mhip_status mhip_copy(mhip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    MHIP_REQUIRE_CTX(ctx);
    if (bytes == 0) return MHIP_OK;
    return mhip::from_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream),
                          "copying on the device");
}

mhip_status mhip_zero(mhip_ctx* ctx, void* dst, size_t bytes) {
    MHIP_REQUIRE_CTX(ctx);
    if (bytes == 0) return MHIP_OK;
    return mhip::from_hip(hipMemsetAsync(dst, 0, bytes, ctx->stream), "zeroing a device buffer");
}

mhip_status mhip_sync(mhip_ctx* ctx) {
    MHIP_REQUIRE_CTX(ctx);
    return mhip::from_hip(hipStreamSynchronize(ctx->stream), "synchronizing the stream");
}

mhip_status mhip_check_flags(mhip_ctx* ctx, uint32_t* flags_out) {
    MHIP_REQUIRE_CTX(ctx);
    uint32_t flags = 0;
    hipError_t err = hipMemcpyAsync(&flags, ctx->flags, sizeof(flags), hipMemcpyDeviceToHost,
                                    ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    if (err != hipSuccess) return mhip::from_hip(err, "reading the failure flags");
    if (flags) {
        err = hipMemsetAsync(ctx->flags, 0, sizeof(uint32_t), ctx->stream);
        if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
        if (err != hipSuccess) return mhip::from_hip(err, "clearing the failure flags");
    }
    if (flags_out) *flags_out = flags;
    if (flags & MHIP_FLAG_EMBEDDING_INVALID_ID)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "embedding lookup id is not a valid in-range non-negative integer");
    if (flags & MHIP_FLAG_SOFTMAX_NON_FINITE)
        return mhip::fail(MHIP_EXECUTION_FAILED,
                          "softmax has a row with no finite entry to normalize");
    return MHIP_OK;
}

mhip_status mhip_timer_start(mhip_ctx* ctx) {
    MHIP_REQUIRE_CTX(ctx);
    return mhip::from_hip(hipEventRecord(ctx->timer_start, ctx->stream), "recording an event");
}

mhip_status mhip_timer_stop(mhip_ctx* ctx, float* elapsed_ms) {
    MHIP_REQUIRE_CTX(ctx);
    hipError_t err = hipEventRecord(ctx->timer_stop, ctx->stream);
    if (err == hipSuccess) err = hipEventSynchronize(ctx->timer_stop);
    float ms = 0.0f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, ctx->timer_start, ctx->timer_stop);
    if (elapsed_ms) *elapsed_ms = ms;
    return mhip::from_hip(err, "timing the stream");
}

}  // extern "C"
