// Row reductions shared by the RMSNorm / softmax kernels and the decode
// projections that normalise their input row themselves: one summation
// order, so a fused RMSNorm gives the bits of the RMSNorm kernel.
#pragma once

#include "common.hpp"

namespace mhip {

struct SumOp {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = op(v, __shfl_xor(v, off, 64));
    return v;
}

// Reduces over the G threads of this row's group (G = 64: a wave; G = 256:
// the four waves of a workgroup, meeting in `scratch`, 4 floats); every
// thread gets the result. REUSE: the caller reduces through `scratch`
// again, so the reads of this call must finish before the next call's
// writes (a second barrier).
template <int G, class Op, bool REUSE = true>
__device__ __forceinline__ float group_reduce(float v, Op op, float* scratch) {
    v = wave_reduce(v, op);
    if constexpr (G == 256) {
        const int wave = threadIdx.x / 64;
        if ((threadIdx.x & 63) == 0) scratch[wave] = v;
        __syncthreads();
        v = op(op(scratch[0], scratch[1]), op(scratch[2], scratch[3]));
        if constexpr (REUSE) __syncthreads();
    }
    return v;
}

// RMSNorm's sum of squares: a thread adds its four-float vectors in order.
__device__ __forceinline__ float add_squares(float ss, float4 x) {
    return ss + (x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w);
}

// RMSNorm's sum of squares is taken chunk by chunk: a chunk is 64
// consecutive four-float vectors (256 floats) held one per lane of a wave,
// lane l holding vector l; its sum is the wave butterfly of the lanes'
// squares, and the row's sum adds the chunk sums in chunk order from 0. Any
// kernel that holds a chunk that way gets the same chunk sum bit for bit: the
// decode block's O-projection reduction writes them, and the gate/up
// projections normalise their input row from them without reading it whole.
__device__ __forceinline__ float chunk_sumsq(float4 x) {
    return wave_reduce(add_squares(0.0f, x), SumOp{});
}

// RMSNorm's scale of a row from the row's sum of squares.
__device__ __forceinline__ float inv_rms(float ss, uint64_t cols, float eps) {
    return 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
}

// How the RMSNorm kernel lays out a row of cols4 four-float vectors: G
// threads per row (a wave up to 256 vectors, else a workgroup of 256) and
// VPT vectors per thread (vectors lane, lane + G, ...). Returns false when
// the row is too long for the register-resident kernel.
__host__ __device__ inline bool rms_layout(uint64_t cols4, int* g, int* vpt) {
    if (cols4 <= 64) { *g = 64; *vpt = 1; }
    else if (cols4 <= 128) { *g = 64; *vpt = 2; }
    else if (cols4 <= 256) { *g = 64; *vpt = 4; }
    else if (cols4 <= 512) { *g = 256; *vpt = 2; }
    else if (cols4 <= 1024) { *g = 256; *vpt = 4; }
    else if (cols4 <= 2048) { *g = 256; *vpt = 8; }
    else if (cols4 <= 4096) { *g = 256; *vpt = 16; }
    else return false;
    return true;
}

}  // namespace mhip
