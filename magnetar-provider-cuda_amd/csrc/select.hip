// On-device greedy next-token selection (`select_greedy_column`,
// src/kernels.rs:4437-4488; semantics of src/kernels.cu:1808-1866): the
// column of one logits row with the largest score / temperature (the score
// itself when temperature is 0) among columns whose raw score is finite and
// that lie outside every excluded [start, end) range; ties go to the lowest
// column, and -0 ranks equal to +0.
//
// Each eligible column becomes one 64-bit key: the score's bits mapped so
// that unsigned order is float order, above the complement of the column.
// The largest key names the answer whatever order workgroups finish in, so
// a grid-wide atomic max over per-workgroup maxima is deterministic.
//
// One launch does the whole call: each workgroup folds its maximum into the
// context's device key word and then counts itself in with a wrapping
// increment; the workgroup that counts last swaps the key back to zero (the
// counter has wrapped to zero by itself) and stores the key into a pinned
// host word with a system-scope store, so the host only synchronises and
// reads 8 bytes: no clearing launch and no copy.
#include "common.hpp"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ uint64_t column_key(float value, uint64_t column) {
    if (value == 0.0f) value = 0.0f;  // -0 ranks as +0
    const uint32_t bits = __float_as_uint(value);
    const uint32_t ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    return (static_cast<uint64_t>(ordered) << 32) | (0xFFFFFFFFull - (column & 0xFFFFFFFFull));
}

__global__ __launch_bounds__(kThreads) void greedy_select_kernel(
    const float* __restrict__ row, uint64_t cols, const uint64_t* __restrict__ ranges,
    uint32_t range_count, float temperature, unsigned long long* state, uint64_t* host) {
    __shared__ unsigned long long wave_best[kThreads / 64];
    __shared__ bool last;
    uint64_t key = 0;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < cols; i += stride) {
        float value = row[i];
        if (!isfinite(value)) continue;
        bool excluded = false;
        for (uint32_t r = 0; r < range_count && !excluded; ++r)
            excluded = i >= ranges[2 * r] && i < ranges[2 * r + 1];
        if (excluded) continue;
        if (temperature != 0.0f) value = value / temperature;
        const uint64_t k = column_key(value, i);
        key = k > key ? k : key;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t other = __shfl_xor(static_cast<unsigned long long>(key), off, 64);
        key = other > key ? other : key;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) wave_best[wave] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t k = wave_best[0];
        for (int w = 1; w < kThreads / 64; ++w) k = wave_best[w] > k ? wave_best[w] : k;
        if (k != 0) atomicMax(&state[0], static_cast<unsigned long long>(k));
        __threadfence();  // the maximum lands before this workgroup counts in
        auto* counter = reinterpret_cast<unsigned int*>(&state[1]);
        last = atomicInc(counter, gridDim.x - 1) == gridDim.x - 1;
        if (last) {
            __threadfence();  // every other workgroup's maximum is visible
            const unsigned long long best = atomicExch(&state[0], 0ull);
            __hip_atomic_store(host, static_cast<uint64_t>(best), __ATOMIC_RELEASE,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

}  // namespace

extern "C" mhip_status mhip_greedy_select_f32(mhip_ctx* ctx, const float* logits, uint64_t rows,
                                              uint64_t cols, uint64_t row,
                                              const uint64_t* excluded, uint32_t range_count,
                                              float temperature, int64_t* column) {
    MHIP_REQUIRE_CTX(ctx);
    if (!column) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "greedy selection: null result");
    *column = -1;
    if (cols == 0 || row >= rows || cols > 0xFFFFFFFFull)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "no logits row " + std::to_string(row) + " of " +
                                                      std::to_string(rows) + " rows of " +
                                                      std::to_string(cols) + " columns");
    if (!logits || (range_count && !excluded))
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "greedy selection: null buffer");
    // The answer is downloaded, so the call cannot be captured.
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a device-to-host download"); st != MHIP_OK)
        return st;
    // The excluded ranges go to the workspace; the key and counter live in
    // the context, zero between calls.
    uint64_t* ranges = nullptr;
    if (range_count) {
        void* scratch = nullptr;
        mhip_status st = mhip::workspace(ctx, static_cast<size_t>(range_count) * 2 * sizeof(uint64_t),
                                         &scratch);
        if (st != MHIP_OK) return st;
        ranges = static_cast<uint64_t*>(scratch);
        hipError_t err = hipMemcpyAsync(ranges, excluded,
                                        static_cast<size_t>(range_count) * 2 * sizeof(uint64_t),
                                        hipMemcpyHostToDevice, ctx->stream);
        if (err != hipSuccess) return mhip::from_hip(err, "uploading the excluded ranges");
    }
    volatile uint64_t* answer = ctx->select_host;
    *answer = ~0ull;
    const uint64_t blocks = std::min<uint64_t>(256, (cols + 4 * kThreads - 1) / (4 * kThreads));
    mhip::launch(ctx, greedy_select_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                 logits + row * cols, cols, ranges, range_count, temperature,
                 reinterpret_cast<unsigned long long*>(ctx->select_state), ctx->select_host);
    mhip_status st = mhip::check_launch("greedy selection");
    if (st != MHIP_OK) return st;
    const hipError_t err = hipStreamSynchronize(ctx->stream);
    if (err != hipSuccess) return mhip::from_hip(err, "reading the greedy selection");
    const uint64_t key = *answer;
    if (key == ~0ull)
        return mhip::fail(MHIP_EXECUTION_FAILED, "greedy selection: the kernel left no answer");
    if (key != 0) *column = static_cast<int64_t>(0xFFFFFFFFull - (key & 0xFFFFFFFFull));
    return MHIP_OK;
}
