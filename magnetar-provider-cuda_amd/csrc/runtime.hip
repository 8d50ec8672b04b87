// Context, device discovery, buffers, flags and timing.
//
// Mirrors the reference's Provider construction and buffer model
// (src/provider.rs:119-179, src/device.rs:41-92, src/kernels.rs:1630-1665,
// :2118-2164) with the HIP runtime: the kernels are compiled ahead of time
// for gfx950 into this library, so there is no runtime compiler step.
#include "common.hpp"
#include "internal.hpp"

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

mhip_status forbid_in_capture(mhip_ctx* ctx, const char* what) {
    if (!ctx || !ctx->capturing) return MHIP_OK;
    const std::string reason = std::string(what) + " cannot be captured";
    if (ctx->capture_failure.empty()) ctx->capture_failure = reason;
    return fail(MHIP_CAPTURE_UNSUPPORTED, reason);
}

uint32_t capture_advancing(const mhip_ctx* ctx) {
    return ctx && ctx->capturing ? ctx->advancing : 0u;
}

const uint64_t* advance_ptr(mhip_ctx* ctx, uint32_t bit, uint64_t max_offset) {
    if (!ctx->capturing || !(ctx->advancing & bit)) return nullptr;
    if (max_offset < ctx->max_offset) ctx->max_offset = max_offset;
    ctx->offset_read = true;
    return ctx->capture_offset;
}

// Frees `p` now, or keeps it until the last live graph is destroyed.
static void release_buffer(mhip_ctx* ctx, void* p) {
    if (!p) return;
    if (ctx->live_graphs > 0) ctx->retired.push_back(p);
    else (void)hipFree(p);
}

mhip_status workspace(mhip_ctx* ctx, size_t bytes, void** out) {
    if (ctx->workspace_bytes < bytes) {
        mhip_status st = forbid_in_capture(ctx, "growing the workspace");
        if (st != MHIP_OK) return st;
        if (ctx->workspace) {
            (void)hipStreamSynchronize(ctx->stream);
            release_buffer(ctx, ctx->workspace);
            ctx->workspace = nullptr;
            ctx->workspace_bytes = 0;
        }
        hipError_t err = hipMalloc(&ctx->workspace, bytes);
        if (err != hipSuccess) {
            ctx->workspace = nullptr;
            return from_hip(err, "allocating the workspace");
        }
        ctx->workspace_bytes = bytes;
    }
    *out = ctx->workspace;
    return MHIP_OK;
}

}  // namespace mhip

// A captured step: its recorded launches, re-issued in order on the
// context's stream by mhip_graph_launch. An advancing launch read the replay
// offset through a pointer that was the address of the word `offset` when
// recorded; a replay at offset t points it at entry t of `table`, a device
// array holding 0, 1, 2, ..., so nothing is written per replay. Offsets past
// the table's reach (kTableCap entries) are written into `offset` by one
// small kernel ahead of the launches instead.
struct mhip_graph {
    mhip_ctx* ctx = nullptr;
    std::vector<mhip_ctx::RecordedLaunch> launches;
    std::vector<std::vector<void*>> argv;  // argument pointers into launches[i].args
    uint64_t* offset = nullptr;
    uint64_t max_offset = 0;
    bool offset_read = false;  // some launch of the step reads the offset
    uint64_t* table = nullptr;
    uint64_t table_entries = 0;
    std::vector<uint64_t*> old_tables;  // outgrown; replays in flight may read them
};

namespace {

constexpr uint64_t kTableCap = uint64_t(1) << 22;  // 32 MiB of offsets at most

// A replay's offset beyond the table: written into the offset word on the
// stream, ahead of the step's launches. The failure flags are left alone:
// like eager calls, a replay only sets them, and mhip_check_flags clears
// them when it reports them.
__global__ void replay_offset_kernel(uint64_t* word, uint64_t value) { *word = value; }

// table[i] = first + i for i < n.
__global__ void iota_kernel(uint64_t* table, uint64_t first, uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) table[i] = first + i;
}

// Grows the graph's offset table to cover `offset` (doubling, up to
// kTableCap entries); the old table is kept until the graph goes.
mhip_status cover_offset(mhip_graph* g, uint64_t offset) {
    if (offset < g->table_entries) return MHIP_OK;
    uint64_t entries = std::max<uint64_t>(4096, g->table_entries * 2);
    while (entries <= offset) entries *= 2;
    entries = std::min(entries, kTableCap);
    uint64_t* table = nullptr;
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&table), entries * sizeof(uint64_t));
    if (err != hipSuccess) return mhip::from_hip(err, "allocating a replay offset table");
    mhip::launch(g->ctx, iota_kernel, dim3(static_cast<unsigned>((entries + 255) / 256)), dim3(256), 0,
                 table, uint64_t(0), entries);
    if (mhip_status st = mhip::check_launch("filling a replay offset table"); st != MHIP_OK) {
        (void)hipFree(table);
        return st;
    }
    if (g->table) g->old_tables.push_back(g->table);
    g->table = table;
    g->table_entries = entries;
    return MHIP_OK;
}

}  // namespace

namespace mhip {

void record_launch(mhip_ctx* ctx, mhip_ctx::RecordedLaunch&& launch) {
    // Pointers sit at 8-byte offsets within an argument aligned to 8; the
    // offset word's address in any of them is an advancing launch's offset
    // pointer (a padding byte pattern equal to a live device address would
    // only be rewritten harmlessly).
    const uint64_t word = reinterpret_cast<uintptr_t>(ctx->capture_offset);
    for (size_t i = 0; i < launch.offsets.size(); ++i) {
        const size_t begin = launch.offsets[i];
        const size_t end = i + 1 < launch.offsets.size() ? launch.offsets[i + 1] : launch.args.size();
        if (begin % 8 != 0) continue;
        for (size_t at = begin; at + 8 <= end; at += 8) {
            uint64_t v;
            std::memcpy(&v, launch.args.data() + at, 8);
            if (v == word) launch.patches.push_back(at);
        }
    }
    ctx->recorded.push_back(std::move(launch));
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
        (err = hipMalloc(reinterpret_cast<void**>(&ctx->select_state), 256)) != hipSuccess ||
        (err = hipMemset(ctx->select_state, 0, 256)) != hipSuccess ||
        (err = hipHostMalloc(reinterpret_cast<void**>(&ctx->select_host), 256,
                             hipHostMallocCoherent)) != hipSuccess ||
        // The context's stream does not wait for the null stream's memsets.
        (err = hipDeviceSynchronize()) != hipSuccess ||
        (err = hipEventCreate(&ctx->timer_start)) != hipSuccess ||
        (err = hipEventCreate(&ctx->timer_stop)) != hipSuccess) {
        mhip_status st = mhip::from_hip(err, "creating the device context");
        mhip_ctx_destroy(ctx);
        return st;
    }
    // The allocation-free matmul's scratch address on this device (a failure
    // here is reported by that entry point's own call).
    (void)mhip::noalloc_scratch(ctx, nullptr);
    *out = ctx;
    return MHIP_OK;
}

mhip_status mhip_ctx_destroy(mhip_ctx* ctx) {
    if (!ctx) return MHIP_OK;
    (void)hipSetDevice(ctx->device);
    mhip_capture_abort(ctx);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->flags) (void)hipFree(ctx->flags);
    if (ctx->select_state) (void)hipFree(ctx->select_state);
    if (ctx->select_host) (void)hipHostFree(ctx->select_host);
    for (auto& table : ctx->rope_tables) (void)hipFree(table.device);
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    // Graphs not destroyed by now can no longer run: their buffers go too.
    for (void* p : ctx->retired) (void)hipFree(p);

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
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a device allocation"); st != MHIP_OK)
        return st;
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
    if (ctx->capturing) {  // hipFree would wait on the capturing stream
        ctx->deferred_frees.push_back(device_ptr);
        return MHIP_OK;
    }
    (void)hipSetDevice(ctx->device);
    return mhip::from_hip(hipFree(device_ptr), "freeing a device buffer");
}

mhip_status mhip_upload(mhip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    MHIP_REQUIRE_CTX(ctx);
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a host-to-device upload"); st != MHIP_OK)
        return st;
    if (bytes == 0) return MHIP_OK;
    // Ordered after earlier kernels on the stream; waits for the copy so the
    // host buffer may be reused on return.
    hipError_t err = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    return mhip::from_hip(err, "uploading to the device");
}

mhip_status mhip_download(mhip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    MHIP_REQUIRE_CTX(ctx);
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a device-to-host download"); st != MHIP_OK)
        return st;
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
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a device memset"); st != MHIP_OK) return st;
    if (bytes == 0) return MHIP_OK;
    return mhip::from_hip(hipMemsetAsync(dst, 0, bytes, ctx->stream), "zeroing a device buffer");
}

mhip_status mhip_sync(mhip_ctx* ctx) {
    MHIP_REQUIRE_CTX(ctx);
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a stream synchronization"); st != MHIP_OK)
        return st;
    return mhip::from_hip(hipStreamSynchronize(ctx->stream), "synchronizing the stream");
}

mhip_status mhip_check_flags(mhip_ctx* ctx, uint32_t* flags_out) {
    MHIP_REQUIRE_CTX(ctx);
    if (mhip_status st = mhip::forbid_in_capture(ctx, "reading the failure flags"); st != MHIP_OK)
        return st;
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
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a timer"); st != MHIP_OK) return st;
    return mhip::from_hip(hipEventRecord(ctx->timer_start, ctx->stream), "recording an event");
}

mhip_status mhip_timer_stop(mhip_ctx* ctx, float* elapsed_ms) {
    MHIP_REQUIRE_CTX(ctx);
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a timer"); st != MHIP_OK) return st;
    hipError_t err = hipEventRecord(ctx->timer_stop, ctx->stream);
    if (err == hipSuccess) err = hipEventSynchronize(ctx->timer_stop);
    float ms = 0.0f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, ctx->timer_start, ctx->timer_stop);
    if (elapsed_ms) *elapsed_ms = ms;
    return mhip::from_hip(err, "timing the stream");
}

// ---- step capture (src/kernels.rs:1019-1349) ----
//
// A captured step is the list of its launches (kernel, grid, argument
// values), recorded by mhip::launch while capturing and re-issued in order on
// the stream by mhip_graph_launch. HIP graphs were used first: a
// hipGraphLaunch of the same launches ran 4.6-7 us slower than issuing them
// on the stream (the C1 block's seven launches 43.3 vs 38.6 us, the C5
// decode step 171.4 vs 164.5 us including a kernel writing the offset word),
// with or without the runtime's graph packet capture. Re-issued launches run
// exactly as eager ones, and each copies its argument values when issued,
// so a replay queued behind another never sees the next one's offset.

mhip_status mhip_capture_begin(mhip_ctx* ctx, uint32_t advancing) {
    MHIP_REQUIRE_CTX(ctx);
    if (ctx->capturing)
        return mhip::fail(MHIP_CAPTURE_UNSUPPORTED, "a step capture is already in progress");
    (void)hipSetDevice(ctx->device);
    // The word whose address advancing launches record (and that offsets past
    // a replay's table are written into); allocated before capturing, since
    // nothing allocates while capturing.
    uint64_t* offset = nullptr;
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&offset), 256);
    if (err == hipSuccess) err = hipMemset(offset, 0, 256);
    if (err == hipSuccess) err = hipDeviceSynchronize();
    if (err != hipSuccess) {
        if (offset) (void)hipFree(offset);
        return mhip::from_hip(err, "beginning a step capture");
    }
    ctx->capturing = true;
    ctx->advancing = advancing;
    ctx->capture_offset = offset;
    ctx->max_offset = UINT64_MAX;
    ctx->offset_read = false;
    ctx->capture_failure.clear();
    ctx->recorded.clear();
    return MHIP_OK;
}

// Ends capture mode; the recorded launches stay in ctx->recorded.
static void stop_capture(mhip_ctx* ctx) {
    ctx->capturing = false;
    for (void* p : ctx->deferred_frees) (void)hipFree(p);
    ctx->deferred_frees.clear();
}

mhip_status mhip_capture_end(mhip_ctx* ctx, mhip_graph** out, uint64_t* max_offset) {
    MHIP_REQUIRE_CTX(ctx);
    if (out) *out = nullptr;
    if (!ctx->capturing) return mhip::fail(MHIP_CAPTURE_UNSUPPORTED, "no step capture is in progress");
    stop_capture(ctx);
    std::string failure = ctx->capture_failure;
    if (failure.empty() && ctx->recorded.empty()) failure = "the step capture recorded no work";
    if (failure.empty() && !out) failure = "no graph handle";
    if (!failure.empty()) {
        ctx->recorded.clear();
        (void)hipFree(ctx->capture_offset);
        ctx->capture_offset = nullptr;
        return mhip::fail(MHIP_CAPTURE_UNSUPPORTED, failure);
    }
    mhip_graph* g = new mhip_graph();
    g->ctx = ctx;
    g->launches = std::move(ctx->recorded);
    ctx->recorded.clear();
    for (auto& l : g->launches) {
        std::vector<void*> argv;
        for (size_t at : l.offsets) argv.push_back(l.args.data() + at);
        g->argv.push_back(std::move(argv));
    }
    g->offset = ctx->capture_offset;
    g->max_offset = ctx->max_offset;
    g->offset_read = ctx->offset_read;
    ctx->capture_offset = nullptr;
    ctx->live_graphs += 1;
    *out = g;
    if (max_offset) *max_offset = g->max_offset;
    return MHIP_OK;
}

mhip_status mhip_capture_abort(mhip_ctx* ctx) {
    MHIP_REQUIRE_CTX(ctx);
    if (!ctx->capturing) return MHIP_OK;
    stop_capture(ctx);
    ctx->recorded.clear();
    if (ctx->capture_offset) (void)hipFree(ctx->capture_offset);
    ctx->capture_offset = nullptr;
    ctx->capture_failure.clear();
    return MHIP_OK;
}

int mhip_capture_active(const mhip_ctx* ctx) { return ctx && ctx->capturing ? 1 : 0; }

mhip_status mhip_graph_launch(mhip_graph* graph, uint64_t offset) {
    if (!graph) return mhip::fail(MHIP_DEVICE_UNAVAILABLE, "no captured step");
    mhip_ctx* ctx = graph->ctx;
    if (ctx->capturing)
        return mhip::fail(MHIP_CAPTURE_UNSUPPORTED, "a captured step cannot run while capturing");
    if (offset > graph->max_offset)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "offset " + std::to_string(offset) + " leaves the captured bounds (at most " +
                              std::to_string(graph->max_offset) + ")");
    // Where the advancing launches read the offset: entry `offset` of the
    // table, or (past the table's reach) the offset word, written first.
    uint64_t word = 0;
    if (graph->offset_read) {
        if (offset < kTableCap) {
            if (mhip_status st = cover_offset(graph, offset); st != MHIP_OK) return st;
            word = reinterpret_cast<uintptr_t>(graph->table + offset);
        } else {
            mhip::launch(ctx, replay_offset_kernel, dim3(1), dim3(1), 0, graph->offset, offset);
            if (mhip_status st = mhip::check_launch("writing the replay offset"); st != MHIP_OK)
                return st;
            word = reinterpret_cast<uintptr_t>(graph->offset);
        }
    }
    for (size_t i = 0; i < graph->launches.size(); ++i) {
        mhip_ctx::RecordedLaunch& l = graph->launches[i];
        for (size_t at : l.patches) std::memcpy(l.args.data() + at, &word, sizeof(word));
        hipError_t err = hipLaunchKernel(l.kernel, l.grid, l.block, graph->argv[i].data(), l.shmem,
                                         ctx->stream);
        if (err != hipSuccess) return mhip::from_hip(err, "launching a captured step");
    }
    return MHIP_OK;
}

uint64_t mhip_graph_max_offset(const mhip_graph* graph) { return graph ? graph->max_offset : 0; }

mhip_status mhip_graph_destroy(mhip_graph* graph) {
    if (!graph) return MHIP_OK;
    mhip_ctx* ctx = graph->ctx;
    if (ctx->capturing)
        return mhip::fail(MHIP_CAPTURE_UNSUPPORTED, "a captured step cannot be released while capturing");
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(graph->offset);
    if (graph->table) (void)hipFree(graph->table);
    for (uint64_t* t : graph->old_tables) (void)hipFree(t);
    ctx->live_graphs -= 1;
    if (ctx->live_graphs == 0) {
        for (void* p : ctx->retired) (void)hipFree(p);
        ctx->retired.clear();
    }
    delete graph;
    return MHIP_OK;
}

}  // extern "C"
