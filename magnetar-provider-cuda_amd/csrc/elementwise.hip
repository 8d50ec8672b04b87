// f32 streaming kernels: add, bias-add, mul, mul-by-scalar, silu, silu-mul,
// scale. All are HBM-bound (8-12 bytes moved per flop). Each thread moves one
// dwordx4 per operand with non-temporal loads and stores (every byte is
// touched once, so nothing is worth keeping in L2); the launch has one
// workgroup per 4 KB of output, tens of thousands at the benchmark sizes.
// Measured on MI355X with inputs rotated past the Infinity Cache, this shape
// beat 2-8 vectors per thread and cached accesses by 10-15 %.
//
// Semantics follow the reference kernels one element at a time
// (src/kernels.cu:30-117, :1091-1096); the vector width changes nothing in
// the arithmetic, so add/mul/bias-add/scale are bit-identical to the CPU
// oracle and silu differs only by the last bit of expf.
#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 1;
constexpr uint64_t kPerBlock = static_cast<uint64_t>(kThreads) * kUnroll;  // float4 slots

using mhip::silu1;

struct AddOp {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct MulOp {
    __device__ float operator()(float a, float b) const { return a * b; }
};
struct SiluMulOp {
    __device__ float operator()(float g, float u) const { return silu1(g) * u; }
};
struct SiluOp {
    __device__ float operator()(float x) const { return silu1(x); }
};
struct ScaleOp {
    float factor;
    __device__ float operator()(float x) const { return x * factor; }
};

template <class Op>
__device__ __forceinline__ float4 apply2(const Op& op, float4 a, float4 b) {
    return make_float4(op(a.x, b.x), op(a.y, b.y), op(a.z, b.z), op(a.w, b.w));
}
template <class Op>
__device__ __forceinline__ float4 apply1(const Op& op, float4 a) {
    return make_float4(op(a.x), op(a.y), op(a.z), op(a.w));
}

// out = op(a, b) over n elements; slot i covers elements [4i, 4i+4). The
// last slot may be partial (n % 4 != 0) and is done with scalar accesses.
template <class Op>
__global__ __launch_bounds__(kThreads) void binary_kernel(const float* __restrict__ a,
                                                          const float* __restrict__ b,
                                                          float* __restrict__ out, uint64_t n,
                                                          Op op) {
    const uint64_t full = n >> 2;
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kPerBlock + threadIdx.x;
    const float4* a4 = reinterpret_cast<const float4*>(a);
    const float4* b4 = reinterpret_cast<const float4*>(b);
    float4* o4 = reinterpret_cast<float4*>(out);
    float4 va[kUnroll], vb[kUnroll];
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
            mhip::store_nt(o4 + i, apply2(op, va[u], vb[u]));
        } else if (i == full) {
            for (uint64_t e = full * 4; e < n; ++e) out[e] = op(a[e], b[e]);
        }
    }
}

template <class Op>
__global__ __launch_bounds__(kThreads) void unary_kernel(const float* __restrict__ x,
                                                         float* __restrict__ out, uint64_t n,
                                                         Op op) {
    const uint64_t full = n >> 2;
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kPerBlock + threadIdx.x;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4* o4 = reinterpret_cast<float4*>(out);
    float4 vx[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
        if (i < full) vx[u] = mhip::load_nt(x4 + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
        if (i < full) {
            mhip::store_nt(o4 + i, apply1(op, vx[u]));
        } else if (i == full) {
            for (uint64_t e = full * 4; e < n; ++e) out[e] = op(x[e]);
        }
    }
}

// out[i] = a[i] * b[0]: the scalar is read on the device (it may be the
// output of an earlier Kernel), once per thread.
__global__ __launch_bounds__(kThreads) void mul_scalar_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ b,
                                                              float* __restrict__ out,
                                                              uint64_t n) {
    const float s = b[0];
    const uint64_t full = n >> 2;
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kPerBlock + threadIdx.x;
    const float4* a4 = reinterpret_cast<const float4*>(a);
    float4* o4 = reinterpret_cast<float4*>(out);
    float4 va[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
        if (i < full) va[u] = mhip::load_nt(a4 + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
        if (i < full) {
            mhip::store_nt(o4 + i, make_float4(va[u].x * s, va[u].y * s, va[u].z * s, va[u].w * s));
        } else if (i == full) {
            for (uint64_t e = full * 4; e < n; ++e) out[e] = a[e] * s;
        }
    }
}

__global__ __launch_bounds__(kThreads) void mul_scalar_any_kernel(const float* a, const float* b,
                                                                  float* out, uint64_t n) {
    const float s = b[0];
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        out[i] = a[i] * s;
}

// out[i] = a[i] + bias[i % cols] with cols % 4 == 0: slot i reads bias
// slot (i % (cols / 4)); the bias row stays in cache.
__global__ __launch_bounds__(kThreads) void bias_add_vec_kernel(const float* __restrict__ a,
                                                                const float* __restrict__ bias,
                                                                float* __restrict__ out,
                                                                uint64_t cols4, uint64_t n4) {
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kPerBlock + threadIdx.x;
    const float4* a4 = reinterpret_cast<const float4*>(a);
    const float4* c4 = reinterpret_cast<const float4*>(bias);
    float4* o4 = reinterpret_cast<float4*>(out);
    float4 va[kUnroll], vb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
        if (i < n4) {
            va[u] = mhip::load_nt(a4 + i);
            vb[u] = c4[i % cols4];
        }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        uint64_t i = base + static_cast<uint64_t>(u) * kThreads;
        if (i < n4) mhip::store_nt(o4 + i, apply2(AddOp{}, va[u], vb[u]));
    }
}

// Any alignment, any cols: one element per thread, grid-stride.
__global__ __launch_bounds__(kThreads) void bias_add_scalar_kernel(const float* __restrict__ a,
                                                                   const float* __restrict__ bias,
                                                                   float* __restrict__ out,
                                                                   uint64_t cols, uint64_t n) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        out[i] = a[i] + bias[i % cols];
}

template <class Op>
__global__ __launch_bounds__(kThreads) void binary_scalar_kernel(const float* a, const float* b,
                                                                 float* out, uint64_t n, Op op) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        out[i] = op(a[i], b[i]);
}

template <class Op>
__global__ __launch_bounds__(kThreads) void unary_scalar_kernel(const float* x, float* out,
                                                                uint64_t n, Op op) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        out[i] = op(x[i]);
}

inline unsigned vec_blocks(uint64_t n) {
    uint64_t slots = (n + 3) / 4;
    return static_cast<unsigned>(mhip::ceil_div(slots, kPerBlock));
}

inline unsigned scalar_blocks(uint64_t n) {
    uint64_t b = mhip::ceil_div(n, kThreads);
    return static_cast<unsigned>(b > 65536 ? 65536 : (b == 0 ? 1 : b));
}

constexpr uint64_t kMaxElements = (1ULL << 31) * kPerBlock;  // grid.x limit x slots

template <class Op>
mhip_status launch_binary(mhip_ctx* ctx, const float* a, const float* b, float* out, uint64_t n,
                          Op op, const char* what) {
    MHIP_REQUIRE_CTX(ctx);
    if (n == 0) return MHIP_OK;
    if (!a || !b || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, std::string(what) + ": null buffer");
    if (n / 4 >= kMaxElements) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, std::string(what) + ": too many elements");
    if (mhip::aligned16(a) && mhip::aligned16(b) && mhip::aligned16(out)) {
        mhip::launch(ctx, binary_kernel<Op>, dim3(vec_blocks(n)), dim3(kThreads), 0, a, b, out, n,
                     op);
    } else {
        mhip::launch(ctx, binary_scalar_kernel<Op>, dim3(scalar_blocks(n)), dim3(kThreads), 0, a, b,
                     out, n, op);
    }
    return mhip::check_launch(what);
}

template <class Op>
mhip_status launch_unary(mhip_ctx* ctx, const float* x, float* out, uint64_t n, Op op,
                         const char* what) {
    MHIP_REQUIRE_CTX(ctx);
    if (n == 0) return MHIP_OK;
    if (!x || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, std::string(what) + ": null buffer");
    if (n / 4 >= kMaxElements) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, std::string(what) + ": too many elements");
    if (mhip::aligned16(x) && mhip::aligned16(out)) {
        mhip::launch(ctx, unary_kernel<Op>, dim3(vec_blocks(n)), dim3(kThreads), 0, x, out, n, op);
    } else {
        mhip::launch(ctx, unary_scalar_kernel<Op>, dim3(scalar_blocks(n)), dim3(kThreads), 0, x, out,
                     n, op);
    }
    return mhip::check_launch(what);
}

}  // namespace

extern "C" {

mhip_status mhip_add_f32(mhip_ctx* ctx, const float* a, const float* b, float* out, uint64_t n) {
    return launch_binary(ctx, a, b, out, n, AddOp{}, "add");
}

mhip_status mhip_mul_f32(mhip_ctx* ctx, const float* a, const float* b, float* out, uint64_t n) {
    return launch_binary(ctx, a, b, out, n, MulOp{}, "mul");
}

mhip_status mhip_silu_mul_f32(mhip_ctx* ctx, const float* gate, const float* up, float* out,
                              uint64_t n) {
    return launch_binary(ctx, gate, up, out, n, SiluMulOp{}, "silu-mul");
}

mhip_status mhip_silu_f32(mhip_ctx* ctx, const float* x, float* out, uint64_t n) {
    return launch_unary(ctx, x, out, n, SiluOp{}, "silu");
}

mhip_status mhip_scale_f32(mhip_ctx* ctx, const float* x, float* out, float factor, uint64_t n) {
    return launch_unary(ctx, x, out, n, ScaleOp{factor}, "scale");
}

mhip_status mhip_mul_scalar_f32(mhip_ctx* ctx, const float* a, const float* b, float* out,
                                uint64_t n) {
    MHIP_REQUIRE_CTX(ctx);
    if (n == 0) return MHIP_OK;
    if (!a || !b || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "mul: null buffer");
    if (mhip::aligned16(a) && mhip::aligned16(out)) {
        mhip::launch(ctx, mul_scalar_kernel, dim3(vec_blocks(n)), dim3(kThreads), 0, a, b, out, n);
    } else {
        mhip::launch(ctx, mul_scalar_any_kernel, dim3(scalar_blocks(n)), dim3(kThreads), 0, a, b,
                     out, n);
    }
    return mhip::check_launch("mul by a scalar");
}

mhip_status mhip_bias_add_f32(mhip_ctx* ctx, const float* a, const float* bias, float* out,
                              uint64_t cols, uint64_t n) {
    MHIP_REQUIRE_CTX(ctx);
    if (cols == 0 || n % cols != 0)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "add data length " + std::to_string(n) +
                              " is not divisible by broadcast dimension " + std::to_string(cols));
    if (n == 0) return MHIP_OK;
    if (!a || !bias || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "add: null buffer");
    if (cols % 4 == 0 && mhip::aligned16(a) && mhip::aligned16(bias) && mhip::aligned16(out)) {
        uint64_t n4 = n / 4;
        mhip::launch(ctx, bias_add_vec_kernel,
                     dim3(static_cast<unsigned>(mhip::ceil_div(n4, kPerBlock))), dim3(kThreads), 0,
                     a, bias, out, cols / 4, n4);
    } else {
        mhip::launch(ctx, bias_add_scalar_kernel, dim3(scalar_blocks(n)), dim3(kThreads), 0, a, bias,
                     out, cols, n);
    }
    return mhip::check_launch("bias add");
}

}  // extern "C"
