// Native f16 / bf16 add and mul on 2-byte device buffers, plus the device-side
// codec (f32 <-> half) that replaces the reference executor's four host
// crossings per call (src/executor.rs:1970-2013).
//
// Arithmetic: decode both operands exactly to f32, one f32 add or mul, RNE
// encode -- the reference's kernels (src/kernels.cu:2913-2939) and its exact
// model (src/tests_conformance.rs:2334-2347); a NaN result's payload follows
// the convention stated at nan_rule. The codec matches
// src/half_precision.rs:14-125 bit for bit:
//  - f16 decode uses v_cvt_f32_f16 (exact for every finite value, subnormals
//    included) and rebuilds NaNs from their bits so a signalling payload is
//    kept as the reference keeps it;
//  - f16 encode uses v_cvt_f16_f32 (round-to-nearest-even, overflow to inf,
//    subnormal results rounded) and applies the reference's NaN payload rule;
//  - bf16 is the reference's integer rounding itself (bits + 0x7FFF + lsb).
// Each thread moves 8 halves per 16-byte access, non-temporal in and out.
#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 1;
constexpr uint64_t kPerBlock = static_cast<uint64_t>(kThreads) * kUnroll;  // 8-half slots

__device__ __forceinline__ float f16_decode(uint32_t h) {
    _Float16 hv = __builtin_bit_cast(_Float16, static_cast<uint16_t>(h));
    float f = static_cast<float>(hv);
    if ((h & 0x7C00u) == 0x7C00u && (h & 0x3FFu) != 0u) {
        uint32_t bits = ((h & 0x8000u) << 16) | 0x7F800000u | ((h & 0x3FFu) << 13);
        f = __builtin_bit_cast(float, bits);
    }
    return f;
}

__device__ __forceinline__ uint32_t f16_encode(float v) {
    uint32_t bits = __builtin_bit_cast(uint32_t, v);
    uint32_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x007FFFFFu) != 0u) {
        uint32_t payload = (bits & 0x007FFFFFu) >> 13;
        h = ((bits >> 16) & 0x8000u) | 0x7C00u | (payload ? payload : 1u);
    }
    return h;
}

__device__ __forceinline__ float bf16_decode(uint32_t h) {
    return __builtin_bit_cast(float, h << 16);
}

__device__ __forceinline__ uint32_t bf16_encode(float v) {
    uint32_t bits = __builtin_bit_cast(uint32_t, v);
    if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x007FFFFFu) != 0u) {
        uint32_t mant7 = (bits >> 16) & 0x7Fu;
        return ((bits >> 16) & 0x8000u) | 0x7F80u | (mant7 ? mant7 : 0x40u);
    }
    return (bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16;
}

template <int DT>
__device__ __forceinline__ float dec(uint32_t h) {
    return DT == MHIP_BF16 ? bf16_decode(h) : f16_decode(h);
}
template <int DT>
__device__ __forceinline__ uint32_t enc(float v) {
    return DT == MHIP_BF16 ? bf16_encode(v) : f16_encode(v);
}

// The f32 result passes through an empty asm statement before it is encoded:
// without it the backend folds the multiply and the f16 conversion into
// v_fma_mix(x, y, +0), which turns -0 * 1 into +0. The barrier emits nothing.
__device__ __forceinline__ float materialize(float v) {
    __asm__ volatile("" : "+v"(v));
    return v;
}

// A NaN result carries a NaN operand's payload, quieted -- the first
// operand's when both are NaN; a NaN made from non-NaN operands (inf - inf,
// 0 * inf) is the negative default quiet NaN. This is the convention of the
// reference CPU Provider's scalar f32 arithmetic as LLVM compiles it for
// x86-64, stated explicitly (the GPU's ALU would pick a NaN of its own). Which
// operand survives NaN op NaN is not fixed by the ISA on the reference's side
// (it follows the compiler's operand order), so only the other rules are
// pinned bit for bit.
__device__ __forceinline__ float nan_rule(float x, float y, float r) {
    if (r == r) return r;
    const uint32_t bits = x != x ? __float_as_uint(x) | 0x00400000u
                                 : (y != y ? __float_as_uint(y) | 0x00400000u : 0xFFC00000u);
    return __uint_as_float(bits);
}

template <int DT, int OP>
__device__ __forceinline__ uint32_t op1(uint32_t a, uint32_t b) {
    float x = dec<DT>(a), y = dec<DT>(b);
    return enc<DT>(nan_rule(x, y, materialize(OP ? x * y : x + y)));
}

// One 32-bit word holds two halves (low half first in memory).
template <int DT, int OP>
__device__ __forceinline__ uint32_t op2(uint32_t a, uint32_t b) {
    return op1<DT, OP>(a & 0xFFFFu, b & 0xFFFFu) | (op1<DT, OP>(a >> 16, b >> 16) << 16);
}

// The same operation when neither operand is infinite or NaN: the sum or
// product of two finite halves is finite or overflows to infinity in f32, so
// no NaN arises and the codec's NaN handling drops out. The results are
// those of op1 bit for bit.
template <int DT, int OP>
__device__ __forceinline__ uint32_t op1_finite(uint32_t a, uint32_t b) {
    float x, y;
    if constexpr (DT == MHIP_BF16) {
        x = bf16_decode(a);
        y = bf16_decode(b);
    } else {
        x = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(a)));
        y = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
    }
    const float r = materialize(OP ? x * y : x + y);
    if constexpr (DT == MHIP_BF16) {
        const uint32_t bits = __builtin_bit_cast(uint32_t, r);
        return (bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16;
    } else {
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(r));
    }
}

template <int DT, int OP>
__device__ __forceinline__ uint32_t op2_finite(uint32_t a, uint32_t b) {
    return op1_finite<DT, OP>(a & 0xFFFFu, b & 0xFFFFu) |
           (op1_finite<DT, OP>(a >> 16, b >> 16) << 16);
}

// Whether any of the 16 halves of two 16-byte vectors has an all-ones
// exponent (infinity or NaN). Each half's exponent field, masked in place,
// is at most the all-ones pattern and equals it only for those values, so
// the lane-wise maximum of the masked fields over the eight words shows it.
template <int DT>
__device__ __forceinline__ bool any_special(const uint4& a, const uint4& b) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    constexpr uint32_t kExp = DT == MHIP_BF16 ? 0x7F807F80u : 0x7C007C00u;
    auto field = [](uint32_t w) { return __builtin_bit_cast(u16x2, w & kExp); };
    const u16x2 ma = __builtin_elementwise_max(__builtin_elementwise_max(field(a.x), field(a.y)),
                                               __builtin_elementwise_max(field(a.z), field(a.w)));
    const u16x2 mb = __builtin_elementwise_max(__builtin_elementwise_max(field(b.x), field(b.y)),
                                               __builtin_elementwise_max(field(b.z), field(b.w)));
    const u16x2 m = __builtin_elementwise_max(ma, mb);
    return m.x == (kExp & 0xFFFFu) || m.y == (kExp & 0xFFFFu);
}

template <int DT, int OP>
__global__ __launch_bounds__(kThreads) void half_binary_kernel(const uint16_t* __restrict__ a,
                                                               const uint16_t* __restrict__ b,
                                                               uint16_t* __restrict__ out,
                                                               uint64_t n) {
    const uint64_t full = n >> 3;
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kPerBlock + threadIdx.x;
    const uint4* a4 = reinterpret_cast<const uint4*>(a);
    const uint4* b4 = reinterpret_cast<const uint4*>(b);
    uint4* o4 = reinterpret_cast<uint4*>(out);
    uint4 va[kUnroll], vb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
        if (i < full) {
            va[u] = mhip::load_nt(a4 + i);
            vb[u] = mhip::load_nt(b4 + i);
        }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
        if (i < full) {
            uint4 r;
            if (!any_special<DT>(va[u], vb[u])) {
                r.x = op2_finite<DT, OP>(va[u].x, vb[u].x);
                r.y = op2_finite<DT, OP>(va[u].y, vb[u].y);
                r.z = op2_finite<DT, OP>(va[u].z, vb[u].z);
                r.w = op2_finite<DT, OP>(va[u].w, vb[u].w);
            } else {
                r.x = op2<DT, OP>(va[u].x, vb[u].x);
                r.y = op2<DT, OP>(va[u].y, vb[u].y);
                r.z = op2<DT, OP>(va[u].z, vb[u].z);
                r.w = op2<DT, OP>(va[u].w, vb[u].w);
            }
            mhip::store_nt(o4 + i, r);
        } else if (i == full) {
            for (uint64_t e = full * 8; e < n; ++e)
                out[e] = static_cast<uint16_t>(op1<DT, OP>(a[e], b[e]));
        }
    }
}

template <int DT, int OP>
__global__ __launch_bounds__(kThreads) void half_binary_scalar_kernel(const uint16_t* a,
                                                                      const uint16_t* b,
                                                                      uint16_t* out, uint64_t n) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        out[i] = static_cast<uint16_t>(op1<DT, OP>(a[i], b[i]));
}

template <int DT>
__global__ __launch_bounds__(kThreads) void encode_kernel(const float* __restrict__ in,
                                                          uint16_t* __restrict__ out, uint64_t n) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        out[i] = static_cast<uint16_t>(enc<DT>(in[i]));
}

template <int DT>
__global__ __launch_bounds__(kThreads) void decode_kernel(const uint16_t* __restrict__ in,
                                                          float* __restrict__ out, uint64_t n) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        out[i] = dec<DT>(in[i]);
}

inline unsigned grid_stride_blocks(uint64_t n) {
    uint64_t b = mhip::ceil_div(n, kThreads);
    return static_cast<unsigned>(b > 65536 ? 65536 : (b == 0 ? 1 : b));
}

template <int DT, int OP>
void launch_half(mhip_ctx* ctx, const uint16_t* a, const uint16_t* b, uint16_t* out, uint64_t n) {
    if (mhip::aligned16(a) && mhip::aligned16(b) && mhip::aligned16(out)) {
        uint64_t slots = (n + 7) / 8;
        mhip::launch(ctx, (half_binary_kernel<DT, OP>),
                     dim3(static_cast<unsigned>(mhip::ceil_div(slots, kPerBlock))), dim3(kThreads),
                     0, a, b, out, n);
    } else {
        mhip::launch(ctx, (half_binary_scalar_kernel<DT, OP>), dim3(grid_stride_blocks(n)),
                     dim3(kThreads), 0, a, b, out, n);
    }
}

mhip_status half_entry(mhip_ctx* ctx, const uint16_t* a, const uint16_t* b, uint16_t* out,
                       uint64_t n, mhip_half_dtype dtype, int op) {
    MHIP_REQUIRE_CTX(ctx);
    if (dtype != MHIP_F16 && dtype != MHIP_BF16)
        return mhip::fail(MHIP_DTYPE_UNSUPPORTED, "half kernels take F16 or BF16");
    if (n == 0) return MHIP_OK;
    if (!a || !b || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "half kernel: null buffer");
    if (n / 8 >= (1ULL << 31) * kPerBlock)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "half kernel: too many elements");
    if (dtype == MHIP_F16) {
        if (op) launch_half<MHIP_F16, 1>(ctx, a, b, out, n);
        else launch_half<MHIP_F16, 0>(ctx, a, b, out, n);
    } else {
        if (op) launch_half<MHIP_BF16, 1>(ctx, a, b, out, n);
        else launch_half<MHIP_BF16, 0>(ctx, a, b, out, n);
    }
    return mhip::check_launch(op ? "mul-half" : "add-half");
}

}  // namespace

extern "C" {

mhip_status mhip_add_half(mhip_ctx* ctx, const uint16_t* a, const uint16_t* b, uint16_t* out,
                          uint64_t n, mhip_half_dtype dtype) {
    return half_entry(ctx, a, b, out, n, dtype, 0);
}

mhip_status mhip_mul_half(mhip_ctx* ctx, const uint16_t* a, const uint16_t* b, uint16_t* out,
                          uint64_t n, mhip_half_dtype dtype) {
    return half_entry(ctx, a, b, out, n, dtype, 1);
}

mhip_status mhip_encode_half(mhip_ctx* ctx, const float* in, uint16_t* out, uint64_t n,
                             mhip_half_dtype dtype) {
    MHIP_REQUIRE_CTX(ctx);
    if (dtype != MHIP_F16 && dtype != MHIP_BF16)
        return mhip::fail(MHIP_DTYPE_UNSUPPORTED, "half codec takes F16 or BF16");
    if (n == 0) return MHIP_OK;
    if (dtype == MHIP_F16)
        mhip::launch(ctx, encode_kernel<MHIP_F16>, dim3(grid_stride_blocks(n)), dim3(kThreads), 0,
                     in, out, n);
    else
        mhip::launch(ctx, encode_kernel<MHIP_BF16>, dim3(grid_stride_blocks(n)), dim3(kThreads), 0,
                     in, out, n);
    return mhip::check_launch("half encode");
}

mhip_status mhip_decode_half(mhip_ctx* ctx, const uint16_t* in, float* out, uint64_t n,
                             mhip_half_dtype dtype) {
    MHIP_REQUIRE_CTX(ctx);
    if (dtype != MHIP_F16 && dtype != MHIP_BF16)
        return mhip::fail(MHIP_DTYPE_UNSUPPORTED, "half codec takes F16 or BF16");
    if (n == 0) return MHIP_OK;
    if (dtype == MHIP_F16)
        mhip::launch(ctx, decode_kernel<MHIP_F16>, dim3(grid_stride_blocks(n)), dim3(kThreads), 0,
                     in, out, n);
    else
        mhip::launch(ctx, decode_kernel<MHIP_BF16>, dim3(grid_stride_blocks(n)), dim3(kThreads), 0,
                     in, out, n);
    return mhip::check_launch("half decode");
}

}  // extern "C"
