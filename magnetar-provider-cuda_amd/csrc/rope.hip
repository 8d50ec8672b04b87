// Rotary position embedding.
//
// Semantics are `rope_kernel`'s (src/kernels.cu:1147-1229) with the checks
// of `rope_scaled` (src/kernels.rs:4224-4355): each row holds head_count
// heads of head_width = cols / head_count columns; in each head the first
// `dimension` columns rotate in pairs -- interleaved (2p, 2p+1) or half-split
// (p, p + dimension/2) -- by angle (offset + row) * scale * freq[p]; the
// other columns pass through.
//
// Two things differ from the reference's one-thread-per-pair launch:
//  - the per-pair frequency (powf, then the banded / YaRN adjustment) depends
//    on the pair only, so the host computes it once per call with the same
//    f32 operations and keeps the table on the device; a position of 8191
//    turns a one-ulp frequency difference into 1e-4 of angle, so this also
//    makes the angles bit-identical to the CPU oracle's;
//  - sin/cos depend on (row, pair) only, so one workgroup per row computes
//    them once into LDS and every head of the row reuses them; the row then
//    streams through with dwordx4 loads.
#include "common.hpp"

#include <cmath>
#include <cstring>

namespace {

// The host-side frequency table: the f32 operations of src/kernels.cu:1197-1221.
void rope_table(const mhip_rope_params& p, std::vector<float>& t) {
    const uint64_t half = p.dimension / 2;
    t.assign(2 * half, 0.0f);
    for (uint64_t pair = 0; pair < half; ++pair) {
        float frequency = powf(p.base, -2.0f * static_cast<float>(pair) / static_cast<float>(p.dimension));
        if (p.banded_factor > 0.0f) {
            float wavelength = 6.283185307179586f / frequency;
            if (wavelength < p.original_context_length / p.high_freq_factor) {
                // High frequencies are kept.
            } else if (wavelength > p.original_context_length / p.low_freq_factor) {
                frequency = frequency / p.banded_factor;
            } else {
                float smooth = (p.original_context_length / wavelength - p.low_freq_factor) /
                               (p.high_freq_factor - p.low_freq_factor);
                frequency = (1.0f - smooth) * frequency / p.banded_factor + smooth * frequency;
            }
        }
        if (p.yarn_factor > 0.0f) {
            float high = p.yarn_low == p.yarn_high ? p.yarn_high + 0.001f : p.yarn_high;
            float ramp = (static_cast<float>(pair) - p.yarn_low) / (high - p.yarn_low);
            ramp = fminf(fmaxf(ramp, 0.0f), 1.0f);
            float interpolated = frequency / p.yarn_factor;
            frequency = interpolated * ramp + frequency * (1.0f - ramp);
        }
        const bool rotated = pair < p.rotated_pairs;
        t[pair] = rotated ? frequency : 0.0f;
        t[half + pair] = rotated ? p.amplitude : 1.0f;
    }
}

// Returns the device copy of `table`, uploading it on first use.
mhip_status device_table(mhip_ctx* ctx, const std::vector<float>& table, const float** out) {
    for (auto& entry : ctx->rope_tables) {
        if (entry.host.size() == table.size() &&
            std::memcmp(entry.host.data(), table.data(), table.size() * sizeof(float)) == 0) {
            *out = entry.device;
            return MHIP_OK;
        }
    }
    if (mhip_status st = mhip::forbid_in_capture(ctx, "a host-to-device upload"); st != MHIP_OK)
        return st;
    if (ctx->rope_tables.size() >= 16 && ctx->live_graphs == 0) {
        // Wait for kernels that may still read the oldest table, then drop it
        // (never while a captured step may read it).
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(ctx->rope_tables.front().device);
        ctx->rope_tables.erase(ctx->rope_tables.begin());
    }
    mhip_ctx::RopeTable entry;
    entry.host = table;
    const size_t bytes = table.size() * sizeof(float);
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&entry.device), bytes ? bytes : 4);
    if (err == hipSuccess)
        err = hipMemcpyAsync(entry.device, table.data(), bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    if (err != hipSuccess) {
        if (entry.device) (void)hipFree(entry.device);
        return mhip::from_hip(err, "uploading the RoPE frequency table");
    }
    ctx->rope_tables.push_back(entry);
    *out = ctx->rope_tables.back().device;
    return MHIP_OK;
}

}  // namespace

namespace mhip {

mhip_status rope_device_table(mhip_ctx* ctx, const mhip_rope_params& p, const float** table) {
    std::vector<float> host;
    rope_table(p, host);
    return device_table(ctx, host, table);
}

}  // namespace mhip

namespace {

constexpr int kThreads = 256;
constexpr uint64_t kMaxHalf = 4096;  // LDS table: 2 x half floats, at most 32 KiB

struct RopeArgs {
    const float* in;
    float* out;
    const float* table;  // [half] frequencies then [half] amplitudes
    uint64_t rows, cols, head_width, dimension, half, position_offset;
    float scale;
    const uint64_t* advance;  // captured step: replay offset added to position_offset
};

// Fills LDS with (cos, sin) * amplitude for this row's pairs (a workgroup of
// THREADS threads).
template <int THREADS = kThreads>
__device__ __forceinline__ void row_sincos(const RopeArgs& a, uint64_t row, float* cs, float* sn) {
    const uint64_t offset = a.position_offset + (a.advance ? *a.advance : 0);
    const float position = mhip::rope_position(offset, row, a.scale);
    for (uint64_t p = threadIdx.x; p < a.half; p += THREADS)
        mhip::rope_pair_cs(position, a.table, a.half, p, &cs[p], &sn[p]);
}

using mhip::rope_rotate;

// Interleaved pairing, vector path: cols, head_width and dimension are
// multiples of 4, so a dwordx4 at head offset j holds pairs j/2 and j/2+1
// (both rotated or both passed through).
// The row's first kVecBatch vectors per thread are loaded before the sin/cos
// table is built, so the table's math overlaps the loads; longer rows
// continue in a loop.
constexpr int kVecBatch = 4;

__global__ __launch_bounds__(kThreads) void rope_interleaved_vec_kernel(RopeArgs a) {
    extern __shared__ float lds[];
    float* cs = lds;
    float* sn = lds + a.half;
    const uint64_t row = blockIdx.x;
    const uint64_t cols4 = a.cols / 4, hw4 = a.head_width / 4;
    const float4* x4 = reinterpret_cast<const float4*>(a.in) + row * cols4;
    float4* o4 = reinterpret_cast<float4*>(a.out) + row * cols4;
    float4 v[kVecBatch];
#pragma unroll
    for (int u = 0; u < kVecBatch; ++u) {
        const uint64_t c = threadIdx.x + static_cast<uint64_t>(u) * kThreads;
        if (c < cols4) v[u] = mhip::load_nt(x4 + c);
    }
    row_sincos(a, row, cs, sn);
    __syncthreads();
    auto rotate_store = [&](uint64_t c, float4 x) {
        const uint64_t j = (c % hw4) * 4;
        if (j < a.dimension) {
            const uint64_t p = j / 2;
            float4 r;
            rope_rotate(x.x, x.y, cs[p], sn[p], &r.x, &r.y);
            rope_rotate(x.z, x.w, cs[p + 1], sn[p + 1], &r.z, &r.w);
            x = r;
        }
        mhip::store_nt(o4 + c, x);
    };
#pragma unroll
    for (int u = 0; u < kVecBatch; ++u) {
        const uint64_t c = threadIdx.x + static_cast<uint64_t>(u) * kThreads;
        if (c < cols4) rotate_store(c, v[u]);
    }
    for (uint64_t c = threadIdx.x + static_cast<uint64_t>(kVecBatch) * kThreads; c < cols4; c += kThreads)
        rotate_store(c, mhip::load_nt(x4 + c));
}

// Interleaved pairing for rows of at most G dwordx4 vectors (4G floats): one
// row per workgroup of G threads, one vector per thread, loaded before the
// row's sin/cos table is built, with 32-bit index arithmetic (the host
// checks the row fits). At C3 ([8192, 32 x 128]) this shape streams about
// 3 points of HBM peak faster than four vectors per thread with 64-bit
// column arithmetic (a probe of both: 80.6 vs 78.1 %).
template <int G>
__global__ __launch_bounds__(G) void rope_interleaved_row_kernel(RopeArgs a) {
    extern __shared__ float lds[];
    float* cs = lds;
    float* sn = lds + a.half;
    const uint32_t t = threadIdx.x;
    const uint32_t cols4 = static_cast<uint32_t>(a.cols / 4);
    const uint32_t hw4 = static_cast<uint32_t>(a.head_width / 4);
    const uint32_t dimension = static_cast<uint32_t>(a.dimension);
    const uint64_t row = blockIdx.x;
    const float4* x4 = reinterpret_cast<const float4*>(a.in) + row * cols4;
    float4* o4 = reinterpret_cast<float4*>(a.out) + row * cols4;
    // This thread's first pair's table entries are read before the row, so
    // the sin/cos waits only for them: loads complete in issue order as far
    // as s_waitcnt can tell, and behind the row's HBM load the table's L2
    // hits would wait for the row too (that cost C3 2.7 us).
    // The loads are unconditional (indices clamped into the table and the
    // row, both non-empty), so the code up to the sin/cos is one block and
    // the wait before it counts only the table's two loads.
    const uint32_t half = static_cast<uint32_t>(a.half);
    const uint32_t tp = min(t, half - 1);
    const float freq = a.table[tp];
    const float amp = a.table[half + tp];
    const uint64_t offset = a.position_offset + (a.advance ? *a.advance : 0);
    float4 x = mhip::load_nt(x4 + min(t, cols4 - 1));
    const float position = mhip::rope_position(offset, row, a.scale);
    if (t < half) mhip::rope_freq_cs(position, freq, amp, &cs[t], &sn[t]);
    for (uint64_t p = t + G; p < half; p += G)
        mhip::rope_pair_cs(position, a.table, half, p, &cs[p], &sn[p]);
    __syncthreads();
    if (t >= cols4) return;
    const uint32_t j = (t % hw4) * 4;
    if (j < dimension) {
        const uint32_t p = j / 2;
        float4 r;
        rope_rotate(x.x, x.y, cs[p], sn[p], &r.x, &r.y);
        rope_rotate(x.z, x.w, cs[p + 1], sn[p + 1], &r.z, &r.w);
        x = r;
    }
    mhip::store_nt(o4 + t, x);
}

// Half-split pairing, vector path: half is a multiple of 4, so the dwordx4
// at head offset j < half pairs with the one at j + half.
__global__ __launch_bounds__(kThreads) void rope_half_split_vec_kernel(RopeArgs a) {
    extern __shared__ float lds[];
    float* cs = lds;
    float* sn = lds + a.half;
    const uint64_t row = blockIdx.x;
    row_sincos(a, row, cs, sn);
    __syncthreads();
    const uint64_t cols4 = a.cols / 4, hw4 = a.head_width / 4, half4 = a.half / 4;
    const uint64_t dim4 = a.dimension / 4;
    const float4* x4 = reinterpret_cast<const float4*>(a.in) + row * cols4;
    float4* o4 = reinterpret_cast<float4*>(a.out) + row * cols4;
    // Per head: half4 rotating slot pairs, then hw4 - dim4 pass-through slots.
    const uint64_t per_head = half4 + (hw4 - dim4);
    const uint64_t heads = a.cols / a.head_width;
    for (uint64_t t = threadIdx.x; t < heads * per_head; t += kThreads) {
        const uint64_t h = t / per_head, k = t % per_head;
        const uint64_t base = h * hw4;
        if (k < half4) {
            float4 u = mhip::load_nt(x4 + base + k), w = mhip::load_nt(x4 + base + k + half4);
            const uint64_t p = k * 4;
            float4 ru, rw;
            rope_rotate(u.x, w.x, cs[p], sn[p], &ru.x, &rw.x);
            rope_rotate(u.y, w.y, cs[p + 1], sn[p + 1], &ru.y, &rw.y);
            rope_rotate(u.z, w.z, cs[p + 2], sn[p + 2], &ru.z, &rw.z);
            rope_rotate(u.w, w.w, cs[p + 3], sn[p + 3], &ru.w, &rw.w);
            mhip::store_nt(o4 + base + k, ru);
            mhip::store_nt(o4 + base + k + half4, rw);
        } else {
            const uint64_t s = base + dim4 + (k - half4);
            mhip::store_nt(o4 + s, x4[s]);
        }
    }
}

// Any shape or alignment: one thread per (head, pair) plus one per
// pass-through column of the row.
__global__ __launch_bounds__(kThreads) void rope_scalar_kernel(RopeArgs a, uint32_t half_split) {
    extern __shared__ float lds[];
    float* cs = lds;
    float* sn = lds + a.half;
    const uint64_t row = blockIdx.x;
    row_sincos(a, row, cs, sn);
    __syncthreads();
    const uint64_t heads = a.cols / a.head_width;
    const float* x = a.in + row * a.cols;
    float* o = a.out + row * a.cols;
    const uint64_t rest = a.head_width - a.dimension;
    for (uint64_t t = threadIdx.x; t < heads * (a.half + rest); t += kThreads) {
        const uint64_t h = t / (a.half + rest), k = t % (a.half + rest);
        const uint64_t base = h * a.head_width;
        if (k < a.half) {
            const uint64_t first = half_split ? base + k : base + 2 * k;
            const uint64_t second = half_split ? base + k + a.half : base + 2 * k + 1;
            float r1, r2;
            rope_rotate(x[first], x[second], cs[k], sn[k], &r1, &r2);
            o[first] = r1;
            o[second] = r2;
        } else {
            const uint64_t col = base + a.dimension + (k - a.half);
            o[col] = x[col];
        }
    }
}

}  // namespace

extern "C" {

void mhip_rope_params_default(mhip_rope_params* p, uint64_t dimension, uint64_t head_count) {
    if (!p) return;
    std::memset(p, 0, sizeof(*p));
    p->base = 10000.0f;
    p->scale = 1.0f;
    p->dimension = dimension;
    p->head_count = head_count;
    p->rotated_pairs = dimension / 2;
    p->amplitude = 1.0f;
}

mhip_status mhip_rope_f32(mhip_ctx* ctx, const float* in, float* out, uint64_t rows,
                          uint64_t cols, const mhip_rope_params* params) {
    MHIP_REQUIRE_CTX(ctx);
    if (!params) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "rope: null params");
    mhip_rope_params p = *params;
    if (p.head_count == 0 || cols % p.head_count != 0)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "RoPE head_count " + std::to_string(p.head_count) +
                              " must be positive and evenly divide the row width " +
                              std::to_string(cols));
    const uint64_t head_width = cols / p.head_count;
    if (p.dimension == 0 || p.dimension % 2 != 0 || p.dimension > head_width)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "RoPE dimension " + std::to_string(p.dimension) +
                              " must be positive, even, and at most the head width " +
                              std::to_string(head_width));
    if (!std::isfinite(p.base) || p.base <= 0.0f)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "RoPE base must be finite and positive");
    if (!std::isfinite(p.scale) || p.scale <= 0.0f)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "RoPE scale must be finite and positive");
    if (p.banded_factor > 0.0f && p.yarn_factor > 0.0f)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "RoPE takes one frequency scaling, not banded and YaRN together");
    const uint64_t half = p.dimension / 2;
    if (half > kMaxHalf)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "RoPE dimension exceeds 8192");
    if (p.rotated_pairs > half) p.rotated_pairs = half;
    if (rows == 0) return MHIP_OK;
    if (!in || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "rope: null buffer");
    if (rows >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "rope: too many rows");
    const float* dtable = nullptr;
    mhip_status st = mhip::rope_device_table(ctx, p, &dtable);
    if (st != MHIP_OK) return st;
    RopeArgs a{in, out, dtable, rows, cols, head_width, p.dimension, half, p.position_offset,
               p.scale, mhip::advance_ptr(ctx, MHIP_ADVANCE_POSITION_OFFSET, UINT64_MAX)};
    const unsigned lds = static_cast<unsigned>(2 * half * sizeof(float));
    const bool aligned = mhip::aligned16(in) && mhip::aligned16(out) && cols % 4 == 0 &&
                         head_width % 4 == 0;
    const uint64_t cols4 = cols / 4;
    if (aligned && !p.half_split && p.dimension % 4 == 0 && cols4 <= 1024) {
        // One vector per thread: the smallest of 64, 256 or 1024 threads that covers the row.
        if (cols4 <= 64)
            mhip::launch(ctx, rope_interleaved_row_kernel<64>, dim3(static_cast<unsigned>(rows)),
                         dim3(64), lds, a);
        else if (cols4 <= 256)
            mhip::launch(ctx, rope_interleaved_row_kernel<256>, dim3(static_cast<unsigned>(rows)),
                         dim3(256), lds, a);
        else
            mhip::launch(ctx, rope_interleaved_row_kernel<1024>, dim3(static_cast<unsigned>(rows)),
                         dim3(1024), lds, a);
    } else if (aligned && !p.half_split && p.dimension % 4 == 0) {
        mhip::launch(ctx, rope_interleaved_vec_kernel, dim3(static_cast<unsigned>(rows)),
                     dim3(kThreads), lds, a);
    } else if (aligned && p.half_split && half % 4 == 0) {
        mhip::launch(ctx, rope_half_split_vec_kernel, dim3(static_cast<unsigned>(rows)),
                     dim3(kThreads), lds, a);
    } else {
        mhip::launch(ctx, rope_scalar_kernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), lds,
                     a, p.half_split);
    }
    return mhip::check_launch("rope");
}

}  // extern "C"
