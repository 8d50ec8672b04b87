// Internal helpers shared by the HIP translation units of libmagnetar_hip.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <tuple>
#include <type_traits>
#include <utility>
#include <vector>

#include "magnetar_hip.h"

// One bound device: its stream (all work is ordered on it), the flag word for
// data-dependent failures and the timing events.
struct mhip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t* flags = nullptr;  // device word, bits MHIP_FLAG_*
    // Greedy selection: a device key word and workgroup counter, zero between
    // calls (each call's last workgroup resets them), and a pinned host word
    // the last workgroup writes the answer into.
    uint64_t* select_state = nullptr;
    uint64_t* select_host = nullptr;
    hipEvent_t timer_start = nullptr;
    hipEvent_t timer_stop = nullptr;
    uint32_t compute_units = 0;
    // RoPE per-pair (frequency, amplitude) tables already on the device,
    // keyed by their exact host contents; a decoder reuses one table.
    struct RopeTable {
        std::vector<float> host;
        float* device = nullptr;
    };
    std::vector<RopeTable> rope_tables;
    // Grow-only device workspace for split-k partial sums (matmul, attention).
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    // Set only for the duration of an mhip_matmul_f32_noalloc call: the
    // device's fixed scratch array, which the matmul then uses instead of the
    // workspace (never grown; a larger need is refused).
    void* fixed_scratch = nullptr;
    size_t fixed_scratch_bytes = 0;

    // Step capture: while `capturing`, launches are recorded (kernel, grid,
    // argument values; mhip::launch) instead of running. Launches whose
    // attribute is in `advancing` (MHIP_ADVANCE_* bits) add the replay offset
    // they read through a pointer that is the address of the word
    // `capture_offset` when recorded; each records how far it may advance in
    // `max_offset`. `failure` keeps the first reason the capture cannot be
    // replayed (an allocation, a transfer, a synchronisation).
    bool capturing = false;
    struct RecordedLaunch {
        const void* kernel = nullptr;
        dim3 grid, block;
        size_t shmem = 0;
        std::vector<unsigned char> args;  // argument values, each at its alignment
        std::vector<size_t> offsets;      // argument i at args[offsets[i]]
        std::vector<size_t> patches;      // where args holds the offset word's address
    };
    std::vector<RecordedLaunch> recorded;
    uint32_t advancing = 0;
    uint64_t* capture_offset = nullptr;
    uint64_t max_offset = 0;
    bool offset_read = false;  // a captured launch reads the offset word
    std::string capture_failure;
    std::vector<void*> deferred_frees;  // mhip_free calls made while capturing
    // Graphs alive on this context; while any is, buffers it may read (the
    // workspace, RoPE tables) are retired instead of freed.
    int live_graphs = 0;
    std::vector<void*> retired;
};

namespace mhip {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming outputs: a non-temporal dwordx4 store, which skips allocating the
// line in L2 (each output is written once and read, if at all, by a later
// launch).
__device__ __forceinline__ void store_nt(float4* p, float4 v) {
    f32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(p));
}
__device__ __forceinline__ void store_nt(uint4* p, uint4 v) {
    u32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4*>(p));
}

// Streaming inputs read exactly once: a non-temporal dwordx4 load.
__device__ __forceinline__ float4 load_nt(const float4* p) {
    const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint4 load_nt(const uint4* p) {
    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// Operand elements: f32, or bf16 bit patterns (compact weights) widened to
// f32 exactly -- a bf16 value is the f32 whose low 16 bits are zero.
__device__ __forceinline__ float elem(const float* p) { return *p; }
__device__ __forceinline__ float elem(const uint16_t* p) {
    return __uint_as_float(static_cast<uint32_t>(*p) << 16);
}
__device__ __forceinline__ float4 widen(uint2 u) {
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u),
                       __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xFFFF0000u));
}
// Four consecutive elements (16-byte aligned f32, 8-byte aligned bf16).
__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load4(const uint16_t* p) {
    return widen(*reinterpret_cast<const uint2*>(p));
}
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
// The same, read once (streamed): non-temporal.
__device__ __forceinline__ float4 load4_nt(const float* p) {
    return load_nt(reinterpret_cast<const float4*>(p));
}
__device__ __forceinline__ float4 load4_nt(const uint16_t* p) {
    const u32x2 t = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return widen(make_uint2(t.x, t.y));
}

// silu(v) = v * (1 / (1 + e^-v)) (src/kernels.cu:73-79).
__device__ __forceinline__ float silu1(float v) { return v * (1.0f / (1.0f + expf(-v))); }

// An embedding id is valid iff id >= 0, id == floor(id) and id < vocab
// (src/kernels.cu:127-176); NaN fails the first test.
__device__ __forceinline__ bool valid_embedding_id(float raw, uint64_t vocab, uint64_t* id) {
    if (raw < 0.0f || raw != floorf(raw)) return false;
    if (static_cast<double>(raw) >= static_cast<double>(vocab)) return false;
    *id = static_cast<uint64_t>(raw);
    return true;
}

// RoPE: the position of `row` (src/kernels.cu:1190-1196), the scaled
// (cos, sin) of pair p from a (frequency, amplitude) table of 2 * half
// floats, and the rotation of one pair.
__device__ __forceinline__ float rope_position(uint64_t offset, uint64_t row, float scale) {
    return static_cast<float>(offset + row) * scale;
}
// Cosine and sine of one pair at `position` from its frequency and amplitude.
__device__ __forceinline__ void rope_freq_cs(float position, float freq, float amp, float* cs,
                                             float* sn) {
    const float angle = position * freq;
    float s, c;
    sincosf(angle, &s, &c);
    *sn = s * amp;
    *cs = c * amp;
}
__device__ __forceinline__ void rope_pair_cs(float position, const float* table, uint64_t half,
                                             uint64_t p, float* cs, float* sn) {
    rope_freq_cs(position, table[p], table[half + p], cs, sn);
}
__device__ __forceinline__ void rope_rotate(float a, float b, float c, float s, float* o1,
                                            float* o2) {
#pragma clang fp contract(off)
    *o1 = a * c - b * s;
    *o2 = a * s + b * c;
}

// Records `detail` as this thread's last error and returns `status`.
mhip_status fail(mhip_status status, const std::string& detail);
// Maps a HIP runtime error onto the stable categories (src/error.rs:71-91).
mhip_status from_hip(hipError_t err, const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Checks the launch that was just enqueued.
mhip_status check_launch(const char* what);

// While capturing: records that `what` cannot be captured (the first such
// reason fails the capture) and returns MHIP_CAPTURE_UNSUPPORTED. MHIP_OK
// otherwise.
mhip_status forbid_in_capture(mhip_ctx* ctx, const char* what);

// While capturing a launch whose attribute `bit` (MHIP_ADVANCE_*) advances:
// the device address of the replay offset, after recording that this launch
// stays in bounds for offsets up to `max_offset`. nullptr otherwise (no
// offset is added).
const uint64_t* advance_ptr(mhip_ctx* ctx, uint32_t bit, uint64_t max_offset);

// Appends a recorded launch to the capture in progress, noting each 8-byte
// field of its arguments that holds the capture's offset-word address (an
// advancing launch's offset pointer) for the replay to redirect.
void record_launch(mhip_ctx* ctx, mhip_ctx::RecordedLaunch&& launch);

// Every kernel launch of the library goes through here: the arguments are
// converted to the kernel's parameter types and launched on the context's
// stream (hipLaunchKernel with the kernel's host handle), or, while a step
// capture is in progress, recorded with their values for mhip_graph_launch
// to re-issue. The launch's error is left for check_launch, as with a plain
// launch.
template <typename... P, typename... A>
void launch(mhip_ctx* ctx, void (*kernel)(P...), dim3 grid, dim3 block, size_t shmem, A&&... args) {
    static_assert(sizeof...(P) == sizeof...(A), "a kernel argument is missing or extra");
    std::tuple<std::decay_t<P>...> values(std::forward<A>(args)...);
    if (ctx->capturing) {
        mhip_ctx::RecordedLaunch r;
        r.kernel = reinterpret_cast<const void*>(kernel);
        r.grid = grid;
        r.block = block;
        r.shmem = shmem;
        std::apply(
            [&r](const auto&... v) {
                auto append = [&r](const void* src, size_t size, size_t align) {
                    const size_t at = (r.args.size() + align - 1) / align * align;
                    r.args.resize(at + size);
                    std::memcpy(r.args.data() + at, src, size);
                    r.offsets.push_back(at);
                };
                (append(&v, sizeof(v), alignof(std::decay_t<decltype(v)>)), ...);
            },
            values);
        record_launch(ctx, std::move(r));
        return;
    }
    void* argv[sizeof...(P) > 0 ? sizeof...(P) : 1] = {};
    std::apply(
        [&argv](auto&... v) {
            size_t i = 0;
            ((argv[i++] = static_cast<void*>(&v)), ...);
        },
        values);
    (void)hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, argv, shmem,
                          ctx->stream);
}

// The context's grow-only scratch of at least `bytes` (split-k partials,
// attention chunk records). Growing it waits for the stream; a buffer a live
// graph may read is retired, not freed. Refused while capturing.
mhip_status workspace(mhip_ctx* ctx, size_t bytes, void** out);

// Looks up (once per device, with the context's device current) the device
// address of the allocation-free matmul's fixed scratch array; called when a
// context is created. Returns it through `out` when not null.
mhip_status noalloc_scratch(mhip_ctx* ctx, float** out);

// The device (frequency, amplitude) table of a RoPE call's pairs, computed
// on the host with the f32 operations of src/kernels.cu:1197-1221 and cached
// per context.
mhip_status rope_device_table(mhip_ctx* ctx, const mhip_rope_params& p, const float** table);

}  // namespace mhip

#define MHIP_REQUIRE_CTX(ctx)                                                     \
    do {                                                                          \
        if ((ctx) == nullptr)                                                     \
            return mhip::fail(MHIP_DEVICE_UNAVAILABLE, "no device context");      \
    } while (0)
