// In-place KV cache append: store rows [row_offset, row_offset + count) =
// rows (`kv-write`, src/kernels.rs:2270-2325). A kernel rather than a copy
// engine transfer, so the write is an ordinary launch on the context's
// stream (capturable, and ordered with the attention that reads the rows).
#include "common.hpp"

namespace {

// dst row = row_offset (+ the replay offset of a captured step).
__device__ __forceinline__ uint64_t first_row(uint64_t row_offset, const uint64_t* advance) {
    return row_offset + (advance ? *advance : 0);
}

__global__ __launch_bounds__(256) void kv_write_vec_kernel(const float4* __restrict__ rows,
                                                           float* __restrict__ store,
                                                           uint64_t width, uint64_t row_offset,
                                                           const uint64_t* advance, uint64_t n4) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n4) return;
    float4* dst = reinterpret_cast<float4*>(store + first_row(row_offset, advance) * width);
    dst[i] = rows[i];
}

__global__ __launch_bounds__(256) void kv_write_scalar_kernel(const float* __restrict__ rows,
                                                              float* __restrict__ store,
                                                              uint64_t width, uint64_t row_offset,
                                                              const uint64_t* advance, uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    store[first_row(row_offset, advance) * width + i] = rows[i];
}

}  // namespace

extern "C" mhip_status mhip_kv_write_f32(mhip_ctx* ctx, float* store, uint64_t capacity,
                                         uint64_t width, const float* rows, uint64_t count,
                                         uint64_t row_offset) {
    MHIP_REQUIRE_CTX(ctx);
    if (row_offset > capacity || count > capacity - row_offset)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "kv-write of " + std::to_string(count) + " rows at " +
                              std::to_string(row_offset) + " exceeds the store's " +
                              std::to_string(capacity) + " rows");
    // A captured write may move down by up to the rows left after it.
    const uint64_t* advance =
        mhip::advance_ptr(ctx, MHIP_ADVANCE_ROW_OFFSET, capacity - (row_offset + count));
    const uint64_t n = count * width;
    if (n == 0) return MHIP_OK;
    if (!store || !rows) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "kv-write: null buffer");
    if (n % 4 == 0 && width % 4 == 0 && mhip::aligned16(store) && mhip::aligned16(rows)) {
        const uint64_t n4 = n / 4;
        mhip::launch(ctx, kv_write_vec_kernel, dim3(static_cast<unsigned>((n4 + 255) / 256)),
                     dim3(256), 0, reinterpret_cast<const float4*>(rows), store, width, row_offset,
                     advance, n4);
    } else {
        mhip::launch(ctx, kv_write_scalar_kernel, dim3(static_cast<unsigned>((n + 255) / 256)),
                     dim3(256), 0, rows, store, width, row_offset, advance, n);
    }
    return mhip::check_launch("kv-write");
}
