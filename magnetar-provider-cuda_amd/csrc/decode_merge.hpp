// The ordered merge of split-KV decode attention's key-chunk records, shared
// by the attention's own merge kernel and the output projection that merges
// inside its partial launch (the decoder block), so both give the same bits.
//
// Records of one (batch, head): chunk c holds its output o_c (normalised by
// its own weight sum), its score max m_c (log2 domain) and weight sum l_c.
// The merge is out = sum_c w_c o_c with w_c = l_c 2^(m_c - M) / sum_c' l_c'
// 2^(m_c' - M) and M = max_c m_c; chunks with no admitted key (l_c = 0) weigh
// nothing, and a head with none at all gives zeros. The same online-softmax
// merge as src/kernels.cu:1868-1959 computes within one pass.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mhip {

// Every one of the workgroup's 256 threads calls it (it synchronises). The
// sums run in a fixed order: M and the weight total over the threads'
// chunk strides, then the wave butterfly, then the 4 waves in order; each
// output column quad t over the chunks c = g, g + G, g + 2G, ... of each of
// the G = 256 / D4 thread groups g, then the groups in order. Only the column
// quads [q0, q0 + nq) are computed; afterwards thread t (t < D4) holds quad t
// of the merged output (zeros outside the range). One call per workgroup.
template <int D4>
__device__ __forceinline__ float4 merge_decode_chunks(const float* __restrict__ ml,
                                                      const float* __restrict__ po,
                                                      uint64_t chunks, int q0, int nq) {
    constexpr int D = 4 * D4;
    constexpr int kGroups = 256 / D4;
    __shared__ float rm[4], rt[4];
    __shared__ float4 red[kGroups][D4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gi = threadIdx.x / D4, t = threadIdx.x % D4;
    const bool active = t >= q0 && t < q0 + nq;

    // The loads of each loop's first pass go out together, before any is
    // used (one memory round trip for up to 256 chunks and 4 per group): this
    // thread's first (max, sum) pair, and its group's first four chunk
    // outputs with their pairs.
    float2 mine = make_float2(-INFINITY, 0.0f);
    if (threadIdx.x < chunks) mine = *reinterpret_cast<const float2*>(ml + 2 * threadIdx.x);
    float4 o0[4];
    float2 e0[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint64_t c = gi + u * kGroups;
        o0[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        e0[u] = make_float2(0.f, 0.f);
        if (active && c < chunks) {
            o0[u] = *reinterpret_cast<const float4*>(po + c * D + 4 * t);
            e0[u] = *reinterpret_cast<const float2*>(ml + 2 * c);
        }
    }

    float mx = fmaxf(-INFINITY, mine.x);
    for (uint64_t c = threadIdx.x + 256; c < chunks; c += 256) mx = fmaxf(mx, ml[2 * c]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) rm[wave] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(rm[0], rm[1]), fmaxf(rm[2], rm[3]));
    float tot = 0.0f;
    if (M != -INFINITY && threadIdx.x < chunks) {
        if (mine.y > 0.0f) tot += mine.y * exp2f(mine.x - M);
        for (uint64_t c = threadIdx.x + 256; c < chunks; c += 256) {
            const float2 e = *reinterpret_cast<const float2*>(ml + 2 * c);
            if (e.y > 0.0f) tot += e.y * exp2f(e.x - M);
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) tot += __shfl_xor(tot, off, 64);
    if (lane == 0) rt[wave] = tot;
    __syncthreads();
    const float total = (rt[0] + rt[1]) + (rt[2] + rt[3]);

    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (active && total > 0.0f) {
        const float inv_total = 1.0f / total;
        auto add = [&](const float4& o, const float2& e) {
            const float w = e.y > 0.0f ? e.y * exp2f(e.x - M) * inv_total : 0.0f;
            acc.x += w * o.x; acc.y += w * o.y; acc.z += w * o.z; acc.w += w * o.w;
        };
        uint64_t c = gi;
        if (c + 3 * kGroups < chunks) {
#pragma unroll
            for (int u = 0; u < 4; ++u) add(o0[u], e0[u]);
            c += 4 * kGroups;
        } else {
            // At most three chunks for this group, all prefetched.
#pragma unroll
            for (int u = 0; u < 3; ++u)
                if (gi + u * kGroups < chunks) add(o0[u], e0[u]);
            c = chunks;
        }
        for (; c + 3 * kGroups < chunks; c += 4 * kGroups) {
            float4 o[4];
            float2 e[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                o[u] = *reinterpret_cast<const float4*>(po + (c + u * kGroups) * D + 4 * t);
                e[u] = *reinterpret_cast<const float2*>(ml + 2 * (c + u * kGroups));
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) add(o[u], e[u]);
        }
        for (; c < chunks; c += kGroups)
            add(*reinterpret_cast<const float4*>(po + c * D + 4 * t),
                *reinterpret_cast<const float2*>(ml + 2 * c));
    }
    red[gi][t] = acc;
    __syncthreads();
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (threadIdx.x < D4 && threadIdx.x >= q0 && threadIdx.x < q0 + nq) {
        v = red[0][threadIdx.x];
        for (int g = 1; g < kGroups; ++g) {
            const float4 r = red[g][threadIdx.x];
            v.x += r.x; v.y += r.y; v.z += r.z; v.w += r.w;
        }
    }
    return v;
}

}  // namespace mhip
