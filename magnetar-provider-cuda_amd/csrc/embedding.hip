// Embedding gather: out[r, :] = table[ids[r], :].
//
// The reference gives one thread per id, each copying its whole row serially
// (src/kernels.cu:127-176), so neighbouring threads touch addresses `dim`
// floats apart. Here a group of threads (one wave for rows up to 256
// vectors, four waves above) copies one row with coalesced dwordx4 loads,
// all loads issued before the stores. Ids are f32 values (src/kernels.rs:3833-3840);
// an id is valid iff id >= 0, id == floor(id) and id < vocab. An invalid id
// leaves its row unwritten and sets MHIP_FLAG_EMBEDDING_INVALID_ID, which
// mhip_check_flags reports as the reference's ShapeUnsupported failure
// (src/kernels.rs:3984-3997).
#include "common.hpp"

namespace {

constexpr int kThreads = 256;

using mhip::valid_embedding_id;

// TPR threads per row, 256 / TPR rows per workgroup, UNROLL vectors per
// thread in flight.
template <int TPR, int UNROLL, class T>
__global__ __launch_bounds__(kThreads) void embedding_vec_kernel(
    const T* __restrict__ table, uint64_t vocab, uint64_t dim4, const float* __restrict__ ids,
    uint64_t num_ids, float* __restrict__ out, uint32_t* flags) {
    constexpr int kRows = kThreads / TPR;
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * kRows + threadIdx.x / TPR;
    const int lane = threadIdx.x % TPR;
    if (row >= num_ids) return;
    uint64_t id = 0;
    if (!valid_embedding_id(ids[row], vocab, &id)) {
        if (lane == 0) atomicOr(flags, MHIP_FLAG_EMBEDDING_INVALID_ID);
        return;
    }
    const T* src = table + id * dim4 * 4;
    float4* dst = reinterpret_cast<float4*>(out) + row * dim4;
    for (uint64_t c0 = lane; c0 < dim4; c0 += static_cast<uint64_t>(TPR) * UNROLL) {
        float4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t c = c0 + static_cast<uint64_t>(u) * TPR;
            if (c < dim4) v[u] = mhip::load4_nt(src + 4 * c);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            uint64_t c = c0 + static_cast<uint64_t>(u) * TPR;
            if (c < dim4) mhip::store_nt(dst + c, v[u]);
        }
    }
}

// Rows of whole 1024-float blocks: one workgroup per block, one dwordx4 per
// thread (short-lived workgroups keep reads and writes interleaved).
template <class T>
__global__ __launch_bounds__(kThreads) void embedding_block_kernel(
    const T* __restrict__ table, uint64_t vocab, uint64_t dim4, const float* __restrict__ ids,
    uint64_t num_ids, float* __restrict__ out, uint32_t* flags) {
    const uint64_t blocks_per_row = dim4 / kThreads;
    const uint64_t row = blockIdx.x / blocks_per_row;
    const uint64_t c = (blockIdx.x % blocks_per_row) * kThreads + threadIdx.x;
    uint64_t id = 0;
    if (!valid_embedding_id(ids[row], vocab, &id)) {
        if (c == 0) atomicOr(flags, MHIP_FLAG_EMBEDDING_INVALID_ID);
        return;
    }
    mhip::store_nt(reinterpret_cast<float4*>(out) + row * dim4 + c, mhip::load4_nt(table + (id * dim4 + c) * 4));
}

// Any dim or alignment: one wave per row, scalar copies.
template <class T>
__global__ __launch_bounds__(kThreads) void embedding_scalar_kernel(
    const T* table, uint64_t vocab, uint64_t dim, const float* ids, uint64_t num_ids,
    float* out, uint32_t* flags) {
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (row >= num_ids) return;
    uint64_t id = 0;
    if (!valid_embedding_id(ids[row], vocab, &id)) {
        if (lane == 0) atomicOr(flags, MHIP_FLAG_EMBEDDING_INVALID_ID);
        return;
    }
    for (uint64_t c = lane; c < dim; c += 64) out[row * dim + c] = mhip::elem(table + id * dim + c);
}

// f32 table, or a compact table of bf16 bit patterns widened exactly.
template <class T>
mhip_status embedding_impl(mhip_ctx* ctx, const T* table, uint64_t vocab, uint64_t dim,
                           const float* ids, uint64_t num_ids, float* out) {
    MHIP_REQUIRE_CTX(ctx);
    if (num_ids == 0 || dim == 0) return MHIP_OK;
    if (!table || !ids || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "embedding: null buffer");
    if (num_ids >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "embedding: too many ids");
    const uintptr_t table_align = sizeof(T) == 4 ? 15u : 7u;
    const bool vec = dim % 4 == 0 && (reinterpret_cast<uintptr_t>(table) & table_align) == 0 &&
                     mhip::aligned16(out);
    const uint64_t dim4 = dim / 4;
    if (vec && dim4 >= 256 && dim4 % 256 == 0 && num_ids * (dim4 / 256) < (1ull << 31)) {
        mhip::launch(ctx, (embedding_block_kernel<T>),
                     dim3(static_cast<unsigned>(num_ids * (dim4 / 256))), dim3(kThreads), 0, table,
                     vocab, dim4, ids, num_ids, out, ctx->flags);
    } else if (vec && dim4 > 256) {
        mhip::launch(ctx, (embedding_vec_kernel<256, 4, T>), dim3(static_cast<unsigned>(num_ids)),
                     dim3(kThreads), 0, table, vocab, dim4, ids, num_ids, out, ctx->flags);
    } else if (vec) {
        mhip::launch(ctx, (embedding_vec_kernel<64, 4, T>),
                     dim3(static_cast<unsigned>(mhip::ceil_div(num_ids, 4))), dim3(kThreads), 0,
                     table, vocab, dim4, ids, num_ids, out, ctx->flags);
    } else {
        mhip::launch(ctx, (embedding_scalar_kernel<T>),
                     dim3(static_cast<unsigned>(mhip::ceil_div(num_ids, 4))), dim3(kThreads), 0,
                     table, vocab, dim, ids, num_ids, out, ctx->flags);
    }
    return mhip::check_launch("embedding lookup");
}

}  // namespace

extern "C" mhip_status mhip_embedding_f32(mhip_ctx* ctx, const float* table, uint64_t vocab,
                                          uint64_t dim, const float* ids, uint64_t num_ids,
                                          float* out) {
    return embedding_impl<float>(ctx, table, vocab, dim, ids, num_ids, out);
}

extern "C" mhip_status mhip_embedding_bf16w_f32(mhip_ctx* ctx, const uint16_t* table,
                                                uint64_t vocab, uint64_t dim, const float* ids,
                                                uint64_t num_ids, float* out) {
    return embedding_impl<uint16_t>(ctx, table, vocab, dim, ids, num_ids, out);
}
