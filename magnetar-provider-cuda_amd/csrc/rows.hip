// Row reductions: RMSNorm and row softmax.
//
// A row is read from HBM once into registers (VPT dwordx4 vectors per
// thread), reduced across a group of G threads -- one wave64 (G = 64, four
// rows per workgroup) for rows up to 1024 floats, one four-wave workgroup
// (G = 256) up to 16384 floats -- with butterfly shuffles inside each wave
// and one LDS exchange between waves, then written once. Many RMSNorm rows of
// 2052-4096 floats take a 1024-thread workgroup per two rows instead, the
// second row's loads ahead of the first row's reduction, with the same bits.
// Rows that are longer, not a multiple of 4 or not 16-byte aligned take a
// looped kernel that re-reads the row from cache.
//
// The reference uses one 256-thread block and a shared-memory tree for
// RMSNorm (src/kernels.cu:1098-1138) and one thread per row for softmax
// (src/kernels.cu:1232-1260). The results here differ from the CPU oracle's
// ascending sums only in summation order.
#include "common.hpp"
#include "internal.hpp"
#include "reduce.hpp"

#include <cmath>

namespace {

constexpr int kThreads = 256;

using mhip::group_reduce;
using mhip::MaxOp;
using mhip::SumOp;
using mhip::wave_reduce;

// With `ids` set, row r of the input is row ids[r] of `in` (an embedding
// table of `vocab` rows) and is also copied to `copy` row r: the embedding
// lookup and the RMSNorm of its output in one pass.
template <int G, int VPT, class TT = float>
__global__ __launch_bounds__(kThreads) void rmsnorm_vec_kernel(
    const TT* __restrict__ in, const float* __restrict__ weight, float* __restrict__ out,
    uint64_t rows, uint64_t cols, uint64_t weight_row_stride, float eps,
    const float* __restrict__ ids, uint64_t vocab, float* __restrict__ copy, uint32_t* flags) {
#pragma clang fp contract(off)
    __shared__ float chunk[4 * VPT];  // G == 256: the row's chunk sums
    constexpr int kRowsPerBlock = kThreads / G;
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / G;
    const int lane = threadIdx.x % G;
    const uint64_t cols4 = cols / 4;
    bool live = row < rows;  // G == 256 rows are always live; waves may not be
    uint64_t src = row;
    if (ids && live && !mhip::valid_embedding_id(ids[row], vocab, &src)) {
        if (lane == 0) atomicOr(flags, MHIP_FLAG_EMBEDDING_INVALID_ID);
        live = false;  // still takes part in the group reduction below
    }
    const TT* xr = in + src * cols;
    const float4* w4 = weight ? reinterpret_cast<const float4*>(weight + row * weight_row_stride)
                              : nullptr;
    float4 x[VPT], wv[VPT];
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
        uint64_t c = lane + static_cast<uint64_t>(v) * G;
        x[v] = (live && c < cols4) ? mhip::load4_nt(xr + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
        // The gain goes out with the row, not after the reduction.
        if (w4 && live && c < cols4) wv[v] = w4[c];
    }
    // The sum of squares chunk by chunk (mhip::chunk_sumsq): vector v of a
    // wave's lanes is chunk v (G = 64), or chunk wave + 4 v (G = 256).
    if constexpr (G == 64) {
#pragma unroll
        for (int v = 0; v < VPT; ++v) ss = ss + mhip::chunk_sumsq(x[v]);
    } else {
        const int wave = threadIdx.x / 64;
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
            const float cs = mhip::chunk_sumsq(x[v]);
            if ((threadIdx.x & 63) == 0) chunk[wave + 4 * v] = cs;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4 * VPT; ++j) ss = ss + chunk[j];
    }
    if (!live) return;
    const float inv = mhip::inv_rms(ss, cols, eps);
    float4* o4 = reinterpret_cast<float4*>(out) + row * cols4;
    float4* c4 = copy ? reinterpret_cast<float4*>(copy) + row * cols4 : nullptr;
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
        uint64_t c = lane + static_cast<uint64_t>(v) * G;
        if (c < cols4) {
            if (c4) mhip::store_nt(c4 + c, x[v]);
            float4 y;
            if (w4) {
                const float4 w = wv[v];
                y = make_float4(x[v].x * inv * w.x, x[v].y * inv * w.y, x[v].z * inv * w.z,
                                x[v].w * inv * w.w);
            } else {
                y = make_float4(x[v].x * inv, x[v].y * inv, x[v].z * inv, x[v].w * inv);
            }
            mhip::store_nt(o4 + c, y);
        }
    }
}

// Many rows of 513-1024 four-float vectors: a workgroup of 1024 threads (one
// vector each) takes R consecutive rows, the next row's loads in flight
// while the current one is reduced and written, so a row's wait at the
// reduction's barrier does not idle the workgroup's memory traffic. Wave w
// holds chunk w, and the row's sum adds the 16 chunk sums in order, as
// rmsnorm_vec_kernel<256, 4> does: the same bits. Nothing is conditional
// (a load or store under a branch makes the compiler wait for every load in
// flight, the next row's included): rows past the end and lanes past the
// row are clamped to the last row and column, which recomputes and rewrites
// exactly those values, and clamped lanes add zero to the sum. GAIN: one
// gain row for all rows.
template <bool GAIN, int R>
__global__ __launch_bounds__(1024) void rmsnorm_rows_kernel(const float* __restrict__ in,
                                                            const float* __restrict__ weight,
                                                            float* __restrict__ out, uint64_t rows,
                                                            uint64_t cols, float eps) {
#pragma clang fp contract(off)
    __shared__ float chunk[2][16];  // by row parity: one barrier per row
    const int t = threadIdx.x, wave = t >> 6;
    const uint64_t cols4 = cols / 4;
    const bool on = static_cast<uint64_t>(t) < cols4;
    const uint64_t tc = on ? static_cast<uint64_t>(t) : cols4 - 1;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 w = zero;
    if constexpr (GAIN) w = reinterpret_cast<const float4*>(weight)[tc];
    const uint64_t first = static_cast<uint64_t>(blockIdx.x) * R;
    auto row_of = [&](int i) { return min(first + i, rows - 1); };
    float4 x[R];
    x[0] = mhip::load4_nt(in + row_of(0) * cols + 4 * tc);
#pragma unroll
    for (int i = 0; i < R; ++i) {
        if (i + 1 < R) x[i + 1] = mhip::load4_nt(in + row_of(i + 1) * cols + 4 * tc);
        const float cs = mhip::chunk_sumsq(on ? x[i] : zero);
        if ((t & 63) == 0) chunk[i & 1][wave] = cs;
        __syncthreads();
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) ss = ss + chunk[i & 1][j];
        const float inv = mhip::inv_rms(ss, cols, eps);
        const float4 v = x[i];
        float4 y;
        if constexpr (GAIN)
            y = make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
        else
            y = make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv);
        mhip::store_nt(reinterpret_cast<float4*>(out) + row_of(i) * cols4 + tc, y);
    }
}

constexpr float kLog2e = 1.4426950408889634f;

// Softmax partial state over a set of entries: their maximum m (NaN-ignoring,
// as fmaxf) and s = the sum of exp(x - m) over them. Two states merge into
// the state of their union by rescaling each sum to the larger maximum; no
// finite maximum leaves s = 0 (the row then fails). A NaN entry makes s NaN,
// which every merge keeps, so the whole row comes out NaN as in the
// reference's sum.
__device__ __forceinline__ void merge_state(float& m, float& s, float m2, float s2) {
    const float mm = fmaxf(m, m2);
    if (mm == -INFINITY) {
        m = mm;
        s = 0.0f;
        return;
    }
    s = s * exp2f((m - mm) * kLog2e) + s2 * exp2f((m2 - mm) * kLog2e);
    m = mm;
}

// Merges the states of the G threads of this row's group; every thread gets
// the same (m, s). The butterfly merges both partners in the same order up
// to commutation, so all lanes agree bit for bit; for G == 256 the four waves'
// states meet in `scratch` and every thread merges them in wave order.
template <int G>
__device__ __forceinline__ void group_merge(float& m, float& s, float2* scratch) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float m2 = __shfl_xor(m, off, 64);
        const float s2 = __shfl_xor(s, off, 64);
        merge_state(m, s, m2, s2);
    }
    if constexpr (G == 256) {
        const int wave = threadIdx.x / 64;
        if ((threadIdx.x & 63) == 0) scratch[wave] = make_float2(m, s);
        __syncthreads();
        m = scratch[0].x;
        s = scratch[0].y;
#pragma unroll
        for (int w = 1; w < 4; ++w) merge_state(m, s, scratch[w].x, scratch[w].y);
    }
}

// One pass over the row in registers: each thread takes the maximum m_t of
// its own entries and e = exp(x - m_t) for each of them (exp2 of the
// difference scaled by log2 e), then the group merges the (max, sum) states
// once, and the output is e * exp(m_t - M) / S, the reciprocal of S taken
// once per thread. Within a few ulp of exp(x - M) / S.
template <int G, int VPT>
__global__ __launch_bounds__(kThreads) void softmax_vec_kernel(const float* __restrict__ in,
                                                               float* __restrict__ out,
                                                               uint64_t rows, uint64_t cols,
                                                               uint32_t* flags) {
    __shared__ float2 scratch[4];
    constexpr int kRowsPerBlock = kThreads / G;
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / G;
    const int lane = threadIdx.x % G;
    const uint64_t cols4 = cols / 4;
    const bool live = row < rows;
    const float4* x4 = reinterpret_cast<const float4*>(in) + row * cols4;
    float4 x[VPT];
    float mt = -INFINITY;
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
        uint64_t c = lane + static_cast<uint64_t>(v) * G;
        x[v] = (live && c < cols4) ? mhip::load_nt(x4 + c)
                                   : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        mt = fmaxf(mt, fmaxf(fmaxf(x[v].x, x[v].y), fmaxf(x[v].z, x[v].w)));
    }
    // Entries of a thread whose own maximum is -inf are all -inf (or NaN):
    // their exponentials are taken against 0 (giving 0, or NaN).
    const float base = mt == -INFINITY ? 0.0f : mt;
    float st = 0.0f;
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
        x[v] = make_float4(exp2f((x[v].x - base) * kLog2e), exp2f((x[v].y - base) * kLog2e),
                           exp2f((x[v].z - base) * kLog2e), exp2f((x[v].w - base) * kLog2e));
        st += (x[v].x + x[v].y) + (x[v].z + x[v].w);
    }
    float M = mt, S = st;
    group_merge<G>(M, S, scratch);
    // A row with no finite maximum fails the call (src/kernels.rs:4371-4378).
    if (!live) return;
    if (!isfinite(M)) {
        if (lane == 0) atomicOr(flags, MHIP_FLAG_SOFTMAX_NON_FINITE);
        return;
    }
    const float scale = exp2f((mt - M) * kLog2e) * (1.0f / S);
    float4* o4 = reinterpret_cast<float4*>(out) + row * cols4;
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
        uint64_t c = lane + static_cast<uint64_t>(v) * G;
        if (c < cols4)
            mhip::store_nt(o4 + c, make_float4(x[v].x * scale, x[v].y * scale, x[v].z * scale,
                                               x[v].w * scale));
    }
}

// Looped fallbacks: one workgroup per row, any cols and alignment.
__device__ __forceinline__ float block_reduce_sum(float v, float* scratch) {
    return group_reduce<256>(v, SumOp{}, scratch);
}

__global__ __launch_bounds__(kThreads) void rmsnorm_loop_kernel(
    const float* in, const float* weight, float* out, uint64_t cols, uint64_t weight_row_stride,
    float eps) {
#pragma clang fp contract(off)
    __shared__ float scratch[4];
    const uint64_t row = blockIdx.x;
    const float* x = in + row * cols;
    float ss = 0.0f;
    for (uint64_t c = threadIdx.x; c < cols; c += kThreads) ss += x[c] * x[c];
    ss = block_reduce_sum(ss, scratch);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
    const float* w = weight ? weight + row * weight_row_stride : nullptr;
    float* y = out + row * cols;
    for (uint64_t c = threadIdx.x; c < cols; c += kThreads)
        y[c] = w ? x[c] * inv * w[c] : x[c] * inv;
}

__global__ __launch_bounds__(kThreads) void softmax_loop_kernel(const float* in, float* out,
                                                                uint64_t cols, uint32_t* flags) {
    __shared__ float scratch[4];
    const uint64_t row = blockIdx.x;
    const float* x = in + row * cols;
    float m = -INFINITY;
    for (uint64_t c = threadIdx.x; c < cols; c += kThreads) m = fmaxf(m, x[c]);
    m = group_reduce<256>(m, MaxOp{}, scratch);
    if (!isfinite(m)) {
        if (threadIdx.x == 0) atomicOr(flags, MHIP_FLAG_SOFTMAX_NON_FINITE);
        return;
    }
    float s = 0.0f;
    for (uint64_t c = threadIdx.x; c < cols; c += kThreads) s += expf(x[c] - m);
    s = block_reduce_sum(s, scratch);
    float* y = out + row * cols;
    for (uint64_t c = threadIdx.x; c < cols; c += kThreads) y[c] = expf(x[c] - m) / s;
}

enum class RowKind { Rms, Softmax };

// Embedding gather for the RMSNorm kernel (unused by the other kinds); the
// table is f32, or bf16 bit patterns when `bf16`.
struct Gather {
    const float* ids = nullptr;
    uint64_t vocab = 0;
    float* copy = nullptr;
    bool bf16 = false;
};

template <RowKind KIND, int G, int VPT>
void launch_vec(mhip_ctx* ctx, uint64_t rows, const float* in, const float* weight, float* out,
                uint64_t cols, uint64_t wstride, float eps, const Gather& g) {
    const unsigned blocks = static_cast<unsigned>(mhip::ceil_div(rows, kThreads / G));
    if constexpr (KIND == RowKind::Rms) {
        if (g.bf16)
            mhip::launch(ctx, (rmsnorm_vec_kernel<G, VPT, uint16_t>), dim3(blocks), dim3(kThreads),
                         0, reinterpret_cast<const uint16_t*>(in), weight, out, rows, cols, wstride,
                         eps, g.ids, g.vocab, g.copy, ctx->flags);
        else
            mhip::launch(ctx, (rmsnorm_vec_kernel<G, VPT, float>), dim3(blocks), dim3(kThreads), 0,
                         in, weight, out, rows, cols, wstride, eps, g.ids, g.vocab, g.copy,
                         ctx->flags);
    }
    else
        mhip::launch(ctx, (softmax_vec_kernel<G, VPT>), dim3(blocks), dim3(kThreads), 0, in, out,
                     rows, cols, ctx->flags);
}

// Picks (G, VPT) for a row of cols4 vectors; returns false when the row
// does not fit the register-resident kernels.
template <RowKind KIND>
bool dispatch_vec(mhip_ctx* ctx, uint64_t rows, const float* in, const float* weight, float* out,
                  uint64_t cols, uint64_t wstride, float eps, const Gather& g = Gather{}) {
    int gs = 0, vpt = 0;
    if (!mhip::rms_layout(cols / 4, &gs, &vpt)) return false;
    // Rows of 513-1024 vectors, two per 1024-thread workgroup (see
    // rmsnorm_rows_kernel), for enough rows to fill the device. C3 [8192,
    // 4096]: 46.05 -> 45.4 us, the same bits; four rows per workgroup 45.8,
    // eight 48.7.
    constexpr int kRowsPerGroup = 2;
    if (KIND == RowKind::Rms && gs == 256 && vpt == 4 && !g.ids && !g.bf16 && wstride == 0 &&
        rows >= 1024) {
        const dim3 grid(static_cast<unsigned>(mhip::ceil_div(rows, kRowsPerGroup)));
        if (weight)
            mhip::launch(ctx, rmsnorm_rows_kernel<true, kRowsPerGroup>, grid, dim3(1024), 0, in,
                         weight, out, rows, cols, eps);
        else
            mhip::launch(ctx, rmsnorm_rows_kernel<false, kRowsPerGroup>, grid, dim3(1024), 0, in,
                         weight, out, rows, cols, eps);
        return true;
    }
    if (gs == 64 && vpt == 1) launch_vec<KIND, 64, 1>(ctx, rows, in, weight, out, cols, wstride, eps, g);
    else if (gs == 64 && vpt == 2) launch_vec<KIND, 64, 2>(ctx, rows, in, weight, out, cols, wstride, eps, g);
    else if (gs == 64) launch_vec<KIND, 64, 4>(ctx, rows, in, weight, out, cols, wstride, eps, g);
    else if (vpt == 2) launch_vec<KIND, 256, 2>(ctx, rows, in, weight, out, cols, wstride, eps, g);
    else if (vpt == 4) launch_vec<KIND, 256, 4>(ctx, rows, in, weight, out, cols, wstride, eps, g);
    else if (vpt == 8) launch_vec<KIND, 256, 8>(ctx, rows, in, weight, out, cols, wstride, eps, g);
    else launch_vec<KIND, 256, 16>(ctx, rows, in, weight, out, cols, wstride, eps, g);
    return true;
}

}  // namespace

extern "C" {

mhip_status mhip_rmsnorm_f32(mhip_ctx* ctx, const float* in, const float* weight, float* out,
                             uint64_t rows, uint64_t cols, uint64_t weight_row_stride,
                             float eps) {
    MHIP_REQUIRE_CTX(ctx);
    if (cols == 0) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "RMSNorm hidden dimension is 0");
    if (!(eps > 0.0f)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "RMSNorm epsilon must be positive");
    if (weight_row_stride != 0 && weight_row_stride != cols)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "RMSNorm weight stride must be 0 or cols");
    if (rows == 0) return MHIP_OK;
    if (!in || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "rmsnorm: null buffer");
    if (rows >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "rmsnorm: too many rows");
    const bool vec = cols % 4 == 0 && mhip::aligned16(in) && mhip::aligned16(out) &&
                     (!weight || mhip::aligned16(weight));
    if (!(vec && dispatch_vec<RowKind::Rms>(ctx, rows, in, weight, out, cols, weight_row_stride,
                                             eps)))
        mhip::launch(ctx, rmsnorm_loop_kernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0,
                     in, weight, out, cols, weight_row_stride, eps);
    return mhip::check_launch("rmsnorm");
}

mhip_status mhip_softmax_rows_f32(mhip_ctx* ctx, const float* in, float* out, uint64_t rows,
                                  uint64_t cols) {
    MHIP_REQUIRE_CTX(ctx);
    if (rows == 0 || cols == 0) {
        // Every row of zero columns has max -inf: the reference fails it.
        if (rows != 0) return mhip::fail(MHIP_EXECUTION_FAILED,
                                         "softmax has a row with no finite entry to normalize");
        return MHIP_OK;
    }
    if (!in || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "softmax: null buffer");
    if (rows >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "softmax: too many rows");
    const bool vec = cols % 4 == 0 && mhip::aligned16(in) && mhip::aligned16(out);
    if (!(vec && dispatch_vec<RowKind::Softmax>(ctx, rows, in, nullptr, out, cols, 0, 0.0f)))
        mhip::launch(ctx, softmax_loop_kernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0,
                     in, out, cols, ctx->flags);
    return mhip::check_launch("softmax");
}

}  // extern "C"

namespace mhip {

mhip_status embed_rmsnorm_f32(mhip_ctx* ctx, const void* table, uint64_t vocab, uint64_t dim,
                              const float* ids, uint64_t rows, const float* weight, float eps,
                              float* out, float* h, bool bf16_table) {
    MHIP_REQUIRE_CTX(ctx);
    if (rows == 0) return MHIP_OK;
    const uintptr_t table_align = bf16_table ? 7u : 15u;
    if (dim == 0 || dim % 4 != 0 || dim / 4 > 4096 || !(eps > 0.0f) || !table || !ids || !out ||
        !h || (reinterpret_cast<uintptr_t>(table) & table_align) != 0 || !aligned16(out) || !aligned16(h) ||
        (weight && !aligned16(weight)) || rows >= (1ULL << 31))
        return MHIP_LAYOUT_UNSUPPORTED;
    Gather g;
    g.ids = ids;
    g.vocab = vocab;
    g.copy = out;
    g.bf16 = bf16_table;
    dispatch_vec<RowKind::Rms>(ctx, rows, static_cast<const float*>(table), weight, h, dim, 0, eps, g);
    return check_launch("embedding + rmsnorm");
}

}  // namespace mhip
