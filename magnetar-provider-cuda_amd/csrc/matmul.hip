// f32 matmul: C[m, n] = A[m, k] . B[k, n] (+ a row bias or a residual).
//
// Semantics are the reference's `matmul_with_addend` (src/kernels.rs:5518-5789,
// src/kernels.cu:1262-1306): optional transposes (A stored [k, m], B stored
// [n, k]), f32 accumulation, the addend added to the finished sum.
//
// Two kernels, chosen by shape:
//  - m > kGemvMaxRows: fp32 MFMA tiles. A workgroup owns a BM x BN tile of C
//    and walks k in BK slices. Both operand slices are staged k-major in LDS
//    (A as [BK][BM], B as [BK][BN]), double-buffered: the next slice is
//    loaded from global memory into registers while the MFMAs run on the
//    current one. Each wave owns WM x WN of the tile as (WM/32) x (WN/32)
//    v_mfma_f32_32x32x2_f32 accumulators; per k step of 2, lane l feeds
//    A[row l%32][k + l/32] and B[k + l/32][col l%32] straight from LDS, so
//    operand reads are 32 consecutive words per half-wave (no bank
//    conflicts). LDS rows are padded: +1 word where a slice is stored
//    transposed (scattered 4-byte writes land in distinct banks), +4 where
//    it is copied as dwordx4. Tiles are ordered so that consecutive tiles
//    share a block row of A and each of the 8 XCDs (own L2) gets a contiguous
//    band of tiles.
//  - m <= kGemvMaxRows (decode): the work is reading B once (HBM-bound), so
//    each wave streams 256 columns of B with dwordx4 loads over one k slice,
//    keeping m x 4 partial sums per lane; partial sums per k slice go to a
//    workspace and a second launch adds them in a fixed order
//    (deterministic), four waves per 256 columns.
#include "common.hpp"

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kGemvMaxRows = 8;

// ---------------------------------------------------------------------------
// MFMA tiles
// ---------------------------------------------------------------------------

template <int BM, int BN, int BK, int WM, int WN, bool A_T, bool B_T>
struct TileCfg {
    static constexpr int kWavesN = BN / WN;
    static constexpr int kWaves = (BM / WM) * kWavesN;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kMI = WM / 32;
    static constexpr int kNI = WN / 32;
    // A slice in LDS is [BK][sA]; stored transposed (from [m][k] rows) unless A_T.
    static constexpr int sA = A_T ? BM + 4 : BM + 1;
    // B slice in LDS is [BK][sB]; stored transposed (from [n][k] rows) if B_T.
    static constexpr int sB = B_T ? BN + 1 : BN + 4;
    static constexpr int kLdsA = BK * sA;
    static constexpr int kLdsB = BK * sB;
    static constexpr int kLdsFloats = 2 * (kLdsA + kLdsB);
    // Global slices as (rows x cols) with cols contiguous in memory.
    static constexpr int kARows = A_T ? BK : BM, kACols = A_T ? BM : BK;
    static constexpr int kBRows = B_T ? BN : BK, kBCols = B_T ? BK : BN;
    static constexpr int kAChunks = kARows * kACols / 4 / kThreads;
    static constexpr int kBChunks = kBRows * kBCols / 4 / kThreads;
    static_assert(kARows * kACols % (4 * kThreads) == 0, "A slice must split evenly");
    static_assert(kBRows * kBCols % (4 * kThreads) == 0, "B slice must split evenly");
};

// Loads this thread's chunks of a (ROWS x COLS) slice whose columns are
// contiguous in memory (leading dimension ld), rows from r0 and columns from
// c0, zero-filling outside (rows_total, cols_total).
template <int ROWS, int COLS, int CHUNKS, int THREADS, bool VEC>
__device__ __forceinline__ void load_slice(float4 (&regs)[CHUNKS], const float* __restrict__ g,
                                           uint64_t ld, uint64_t r0, uint64_t c0,
                                           uint64_t rows_total, uint64_t cols_total) {
    constexpr int kChunksPerRow = COLS / 4;
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        const int chunk = threadIdx.x + i * THREADS;
        const int r = chunk / kChunksPerRow;
        const int c = (chunk % kChunksPerRow) * 4;
        const uint64_t gr = r0 + r, gc = c0 + c;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (gr < rows_total) {
            const float* p = g + gr * ld + gc;
            if (VEC && gc + 3 < cols_total) {
                v = *reinterpret_cast<const float4*>(p);
            } else {
                if (gc + 0 < cols_total) v.x = p[0];
                if (gc + 1 < cols_total) v.y = p[1];
                if (gc + 2 < cols_total) v.z = p[2];
                if (gc + 3 < cols_total) v.w = p[3];
            }
        }
        regs[i] = v;
    }
}

// Stores the chunks into an LDS slice laid out [k][mn] with row stride S.
// TRANSPOSED: the global rows were mn and the columns k (write 4 words down
// a column); otherwise the global rows were k (write one dwordx4).
template <int ROWS, int COLS, int CHUNKS, int THREADS, int S, bool TRANSPOSED>
__device__ __forceinline__ void store_slice(const float4 (&regs)[CHUNKS], float* lds) {
    constexpr int kChunksPerRow = COLS / 4;
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        const int chunk = threadIdx.x + i * THREADS;
        const int r = chunk / kChunksPerRow;
        const int c = (chunk % kChunksPerRow) * 4;
        if constexpr (TRANSPOSED) {
            lds[(c + 0) * S + r] = regs[i].x;
            lds[(c + 1) * S + r] = regs[i].y;
            lds[(c + 2) * S + r] = regs[i].z;
            lds[(c + 3) * S + r] = regs[i].w;
        } else {
            *reinterpret_cast<float4*>(lds + r * S + c) = regs[i];
        }
    }
}

// Maps the linear workgroup id to a (tile_m, tile_n): each XCD (ids are
// dealt round-robin over 8) takes a contiguous band, and inside a band tiles
// go down groups of 8 tile rows so neighbours share A rows and B columns.
__device__ __forceinline__ void tile_coords(uint32_t tiles_m, uint32_t tiles_n, uint32_t* tm,
                                            uint32_t* tn) {
    const uint32_t total = tiles_m * tiles_n;
    uint32_t id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    constexpr uint32_t kGroup = 8;
    const uint32_t per_group = kGroup * tiles_n;
    const uint32_t group = id / per_group;
    const uint32_t first_m = group * kGroup;
    const uint32_t rows_in_group = min(tiles_m - first_m, kGroup);
    const uint32_t in_group = id % per_group;
    *tm = first_m + in_group % rows_in_group;
    *tn = in_group / rows_in_group;
}

template <int BM, int BN, int BK, int WM, int WN, bool A_T, bool B_T, bool VEC>
__global__ __launch_bounds__((TileCfg<BM, BN, BK, WM, WN, A_T, B_T>::kThreads), 2) void mfma_gemm_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, uint64_t M,
    uint64_t K, uint64_t N, const float* __restrict__ addend, int addend_mode) {
    using Cfg = TileCfg<BM, BN, BK, WM, WN, A_T, B_T>;
    constexpr int T = Cfg::kThreads;
    extern __shared__ float lds[];
    // Buffer b of the A slices at lds + b * kLdsA; the B slices follow both.
    float* const lds_b0 = lds + 2 * Cfg::kLdsA;

    uint32_t tm, tn;
    tile_coords(static_cast<uint32_t>((M + BM - 1) / BM), static_cast<uint32_t>((N + BN - 1) / BN),
                &tm, &tn);
    const uint64_t m0 = static_cast<uint64_t>(tm) * BM;
    const uint64_t n0 = static_cast<uint64_t>(tn) * BN;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave / Cfg::kWavesN, wn = wave % Cfg::kWavesN;
    const int lrow = lane & 31, lk = lane >> 5;

    v16f acc[Cfg::kMI][Cfg::kNI];
#pragma unroll
    for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::kNI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    float4 ra[Cfg::kAChunks], rb[Cfg::kBChunks];
    auto load = [&](uint64_t k0) {
        if constexpr (A_T)
            load_slice<Cfg::kARows, Cfg::kACols, Cfg::kAChunks, T, VEC>(ra, A, M, k0, m0, K, M);
        else
            load_slice<Cfg::kARows, Cfg::kACols, Cfg::kAChunks, T, VEC>(ra, A, K, m0, k0, M, K);
        if constexpr (B_T)
            load_slice<Cfg::kBRows, Cfg::kBCols, Cfg::kBChunks, T, VEC>(rb, B, K, n0, k0, N, K);
        else
            load_slice<Cfg::kBRows, Cfg::kBCols, Cfg::kBChunks, T, VEC>(rb, B, N, k0, n0, K, N);
    };
    auto store = [&](int buf) {
        store_slice<Cfg::kARows, Cfg::kACols, Cfg::kAChunks, T, Cfg::sA, !A_T>(ra, lds + buf * Cfg::kLdsA);
        store_slice<Cfg::kBRows, Cfg::kBCols, Cfg::kBChunks, T, Cfg::sB, B_T>(rb, lds_b0 + buf * Cfg::kLdsB);
    };

    const uint64_t slices = (K + BK - 1) / BK;
    load(0);
    store(0);
    __syncthreads();
    for (uint64_t s = 0; s < slices; ++s) {
        const int buf = static_cast<int>(s & 1);
        if (s + 1 < slices) load((s + 1) * BK);
        const float* sa = lds + buf * Cfg::kLdsA + lk * Cfg::sA + wm * WM + lrow;
        const float* sb = lds_b0 + buf * Cfg::kLdsB + lk * Cfg::sB + wn * WN + lrow;
#pragma unroll
        for (int k = 0; k < BK; k += 2) {
            float af[Cfg::kMI], bf[Cfg::kNI];
#pragma unroll
            for (int i = 0; i < Cfg::kMI; ++i) af[i] = sa[k * Cfg::sA + i * 32];
#pragma unroll
            for (int j = 0; j < Cfg::kNI; ++j) bf[j] = sb[k * Cfg::sB + j * 32];
#pragma unroll
            for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
                for (int j = 0; j < Cfg::kNI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < slices) store(buf ^ 1);
        __syncthreads();
    }

    // Accumulator r of lane l holds C[8*(r/4) + 4*(l/32) + r%4][l%32] of its 32x32 block.
#pragma unroll
    for (int i = 0; i < Cfg::kMI; ++i) {
#pragma unroll
        for (int j = 0; j < Cfg::kNI; ++j) {
            const uint64_t col = n0 + wn * WN + j * 32 + lrow;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint64_t row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * lk + (r % 4);
                if (row < M) {
                    float v = acc[i][j][r];
                    if (addend_mode == 1) v = v + addend[col];
                    else if (addend_mode == 2) v = v + addend[row * N + col];
                    C[row * N + col] = v;
                }
            }
        }
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool A_T, bool B_T>
mhip_status launch_mfma(mhip_ctx* ctx, const float* a, const float* b, float* c, uint64_t m,
                        uint64_t k, uint64_t n, const float* addend, int mode, bool vec) {
    using Cfg = TileCfg<BM, BN, BK, WM, WN, A_T, B_T>;
    const uint64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (tiles >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul: too many tiles");
    const size_t lds = Cfg::kLdsFloats * sizeof(float);
    static bool configured = false;  // raise the dynamic-LDS cap above 64 KiB once
    if (!configured) {
        (void)hipFuncSetAttribute(
            reinterpret_cast<const void*>(&mfma_gemm_kernel<BM, BN, BK, WM, WN, A_T, B_T, true>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        (void)hipFuncSetAttribute(
            reinterpret_cast<const void*>(&mfma_gemm_kernel<BM, BN, BK, WM, WN, A_T, B_T, false>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        configured = true;
    }
    if (vec)
        hipLaunchKernelGGL((mfma_gemm_kernel<BM, BN, BK, WM, WN, A_T, B_T, true>),
                           dim3(static_cast<unsigned>(tiles)), dim3(Cfg::kThreads), lds,
                           ctx->stream, a, b, c, m, k, n, addend, mode);
    else
        hipLaunchKernelGGL((mfma_gemm_kernel<BM, BN, BK, WM, WN, A_T, B_T, false>),
                           dim3(static_cast<unsigned>(tiles)), dim3(Cfg::kThreads), lds,
                           ctx->stream, a, b, c, m, k, n, addend, mode);
    return mhip::check_launch("matmul (MFMA tiles)");
}

// ---------------------------------------------------------------------------
// Decode GEMV: m <= kGemvMaxRows, B row-major [k][n] with n % 4 == 0.
// ---------------------------------------------------------------------------

constexpr int kGemvThreads = 256;
constexpr int kGemvCols = 256;  // columns per workgroup: 64 lanes x 4

// Workgroup (column group x, k slice y): its 4 waves split the slice's rows
// and meet in LDS. With one slice it writes C (+ addend) itself; otherwise it
// writes the slice's partial sums for gemv_reduce_kernel.
template <int ROWS>
__global__ __launch_bounds__(kGemvThreads) void gemv_partial_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ partial,
    float* __restrict__ C, uint64_t K, uint64_t N, uint64_t k_per_slice, uint32_t slices,
    const float* __restrict__ addend, int addend_mode) {
    __shared__ float4 red[4][ROWS][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t col = static_cast<uint64_t>(blockIdx.x) * kGemvCols + lane * 4;
    const bool live = col < N;
    const uint64_t k_begin = static_cast<uint64_t>(blockIdx.y) * k_per_slice;
    const uint64_t k_end = min(K, k_begin + k_per_slice);
    float4 acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
        constexpr int kU = 8;
        uint64_t kk = k_begin + wave;
        for (; kk + 4 * (kU - 1) < k_end; kk += 4 * kU) {
            float4 bv[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u)
                bv[u] = mhip::load_nt(reinterpret_cast<const float4*>(B + (kk + 4 * u) * N + col));
#pragma unroll
            for (int u = 0; u < kU; ++u) {
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const float a = A[r * K + kk + 4 * u];
                    acc[r].x = __builtin_fmaf(a, bv[u].x, acc[r].x);
                    acc[r].y = __builtin_fmaf(a, bv[u].y, acc[r].y);
                    acc[r].z = __builtin_fmaf(a, bv[u].z, acc[r].z);
                    acc[r].w = __builtin_fmaf(a, bv[u].w, acc[r].w);
                }
            }
        }
        for (; kk < k_end; kk += 4) {
            const float4 bv = mhip::load_nt(reinterpret_cast<const float4*>(B + kk * N + col));
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const float a = A[r * K + kk];
                acc[r].x = __builtin_fmaf(a, bv.x, acc[r].x);
                acc[r].y = __builtin_fmaf(a, bv.y, acc[r].y);
                acc[r].z = __builtin_fmaf(a, bv.z, acc[r].z);
                acc[r].w = __builtin_fmaf(a, bv.w, acc[r].w);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    if (wave != 0 || !live) return;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        float4 v = red[0][r][lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const float4 o = red[w][r][lane];
            v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
        }
        if (slices == 1) {
            if (addend_mode == 1) {
                const float4 b4 = *reinterpret_cast<const float4*>(addend + col);
                v.x = v.x + b4.x; v.y = v.y + b4.y; v.z = v.z + b4.z; v.w = v.w + b4.w;
            } else if (addend_mode == 2) {
                const float4 b4 = *reinterpret_cast<const float4*>(addend + r * N + col);
                v.x = v.x + b4.x; v.y = v.y + b4.y; v.z = v.z + b4.z; v.w = v.w + b4.w;
            }
            *reinterpret_cast<float4*>(C + r * N + col) = v;
        } else {
            *reinterpret_cast<float4*>(partial + (static_cast<uint64_t>(blockIdx.y) * ROWS + r) * N + col) = v;
        }
    }
}

// C = the slices' partial sums (+ addend). A workgroup covers 256 columns:
// wave w adds a fixed quarter of the slices (eight loads in flight), then
// the quarters are added in order -- the same order on every run.
template <int ROWS>
__global__ __launch_bounds__(kGemvThreads) void gemv_reduce_kernel(
    const float* __restrict__ partial, float* __restrict__ C, uint64_t N, uint32_t slices,
    const float* __restrict__ addend, int addend_mode) {
    __shared__ float4 red[4][ROWS][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t col = static_cast<uint64_t>(blockIdx.x) * kGemvCols + lane * 4;
    const bool live = col < N;
    const uint32_t quarter = (slices + 3) / 4;
    const uint32_t s_begin = min(slices, wave * quarter), s_end = min(slices, s_begin + quarter);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live) {
            uint32_t s = s_begin;
            for (; s + 7 < s_end; s += 8) {
                float4 p[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    p[u] = *reinterpret_cast<const float4*>(partial + ((s + u) * static_cast<uint64_t>(ROWS) + r) * N + col);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    v.x += p[u].x; v.y += p[u].y; v.z += p[u].z; v.w += p[u].w;
                }
            }
            for (; s < s_end; ++s) {
                const float4 p = *reinterpret_cast<const float4*>(partial + (s * static_cast<uint64_t>(ROWS) + r) * N + col);
                v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
            }
        }
        red[wave][r][lane] = v;
    }
    __syncthreads();
    if (wave != 0 || !live) return;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        float4 v = red[0][r][lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const float4 o = red[w][r][lane];
            v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
        }
        if (addend_mode == 1) {
            const float4 b4 = *reinterpret_cast<const float4*>(addend + col);
            v.x = v.x + b4.x; v.y = v.y + b4.y; v.z = v.z + b4.z; v.w = v.w + b4.w;
        } else if (addend_mode == 2) {
            const float4 b4 = *reinterpret_cast<const float4*>(addend + r * N + col);
            v.x = v.x + b4.x; v.y = v.y + b4.y; v.z = v.z + b4.z; v.w = v.w + b4.w;
        }
        *reinterpret_cast<float4*>(C + r * N + col) = v;
    }
}

mhip_status workspace(mhip_ctx* ctx, size_t bytes, float** out) {
    if (ctx->workspace_bytes < bytes) {
        if (ctx->workspace) {
            (void)hipStreamSynchronize(ctx->stream);
            (void)hipFree(ctx->workspace);
            ctx->workspace = nullptr;
            ctx->workspace_bytes = 0;
        }
        hipError_t err = hipMalloc(&ctx->workspace, bytes);
        if (err != hipSuccess) return mhip::from_hip(err, "allocating the matmul workspace");
        ctx->workspace_bytes = bytes;
    }
    *out = static_cast<float*>(ctx->workspace);
    return MHIP_OK;
}

template <int ROWS>
mhip_status launch_gemv(mhip_ctx* ctx, const float* a, const float* b, float* c, uint64_t k,
                        uint64_t n, const float* addend, int mode) {
    const uint64_t col_groups = (n + kGemvCols - 1) / kGemvCols;
    // About four workgroups per CU, each slice a multiple of 32 rows (four
    // waves x eight rows in flight); one slice when the column groups alone
    // fill the device.
    const uint64_t target_blocks = static_cast<uint64_t>(ctx->compute_units ? ctx->compute_units : 256) * 4;
    uint64_t slices = (target_blocks + col_groups - 1) / col_groups;
    uint64_t k_per_slice = ((k + slices - 1) / slices + 31) / 32 * 32;
    if (k_per_slice < 32) k_per_slice = 32;
    slices = (k + k_per_slice - 1) / k_per_slice;
    if (slices <= 1) {
        slices = 1;
        k_per_slice = k;
    }
    float* partial = nullptr;
    if (slices > 1) {
        mhip_status st = workspace(ctx, slices * ROWS * n * sizeof(float), &partial);
        if (st != MHIP_OK) return st;
    }
    hipLaunchKernelGGL(gemv_partial_kernel<ROWS>,
                       dim3(static_cast<unsigned>(col_groups), static_cast<unsigned>(slices)),
                       dim3(kGemvThreads), 0, ctx->stream, a, b, partial, c, k, n, k_per_slice,
                       static_cast<uint32_t>(slices), addend, mode);
    mhip_status st = mhip::check_launch("matmul (decode partial sums)");
    if (st != MHIP_OK || slices == 1) return st;
    hipLaunchKernelGGL(gemv_reduce_kernel<ROWS>, dim3(static_cast<unsigned>(col_groups)),
                       dim3(kGemvThreads), 0, ctx->stream, partial, c, n,
                       static_cast<uint32_t>(slices), addend, mode);
    return mhip::check_launch("matmul (decode reduction)");
}

mhip_status dispatch_gemv(mhip_ctx* ctx, const float* a, const float* b, float* c, uint64_t m,
                          uint64_t k, uint64_t n, const float* addend, int mode) {
    switch (m) {
        case 1: return launch_gemv<1>(ctx, a, b, c, k, n, addend, mode);
        case 2: return launch_gemv<2>(ctx, a, b, c, k, n, addend, mode);
        case 3: return launch_gemv<3>(ctx, a, b, c, k, n, addend, mode);
        case 4: return launch_gemv<4>(ctx, a, b, c, k, n, addend, mode);
        case 5: return launch_gemv<5>(ctx, a, b, c, k, n, addend, mode);
        case 6: return launch_gemv<6>(ctx, a, b, c, k, n, addend, mode);
        case 7: return launch_gemv<7>(ctx, a, b, c, k, n, addend, mode);
        default: return launch_gemv<8>(ctx, a, b, c, k, n, addend, mode);
    }
}

// Zero-inner-dimension product: C = 0 (+ addend).
__global__ void fill_addend_kernel(float* C, uint64_t M, uint64_t N, const float* addend,
                                   int mode) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= M * N) return;
    float v = 0.0f;
    if (mode == 1) v = v + addend[idx % N];
    else if (mode == 2) v = v + addend[idx];
    C[idx] = v;
}

}  // namespace

extern "C" mhip_status mhip_matmul_f32(mhip_ctx* ctx, const float* a, const float* b, float* out,
                                       uint64_t m, uint64_t k, uint64_t n, int transpose_a,
                                       int transpose_b, const float* addend, int addend_mode) {
    MHIP_REQUIRE_CTX(ctx);
    if (addend_mode < 0 || addend_mode > 2)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul addend mode must be 0, 1 or 2");
    if (addend_mode != 0 && !addend)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul addend is null");
    if (m == 0 || n == 0) return MHIP_OK;
    if (!a || !b || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul: null buffer");
    if (k == 0) {
        hipLaunchKernelGGL(fill_addend_kernel, dim3(static_cast<unsigned>((m * n + 255) / 256)),
                           dim3(256), 0, ctx->stream, out, m, n, addend, addend_mode);
        return mhip::check_launch("matmul (empty inner dimension)");
    }
    const bool ta = transpose_a != 0, tb = transpose_b != 0;
    if (m <= kGemvMaxRows && !ta && !tb && n % 4 == 0 && mhip::aligned16(b))
        return dispatch_gemv(ctx, a, b, out, m, k, n, addend, addend_mode);
    // Vector loads need 16-byte aligned rows on both operands.
    const uint64_t lda = ta ? m : k, ldb = tb ? k : n;
    const bool vec = lda % 4 == 0 && ldb % 4 == 0 && mhip::aligned16(a) && mhip::aligned16(b);
    if (!ta && !tb)
        return launch_mfma<128, 128, 32, 64, 64, false, false>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
    if (ta && !tb)
        return launch_mfma<128, 128, 32, 64, 64, true, false>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
    if (!ta && tb)
        return launch_mfma<128, 128, 32, 64, 64, false, true>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
    return launch_mfma<128, 128, 32, 64, 64, true, true>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
}
