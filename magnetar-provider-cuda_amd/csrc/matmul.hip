// f32 matmul: C[m, n] = A[m, k] . B[k, n] (+ a row bias or a residual).
//
// Semantics are the reference's `matmul_with_addend` (src/kernels.rs:5518-5789,
// src/kernels.cu:1262-1306): optional transposes (A stored [k, m], B stored
// [n, k]), f32 accumulation, the addend added to the finished sum.
//
// Two kernel families, chosen by shape:
//  - MFMA tiles. A workgroup owns a BM x BN tile of C and walks k in BK
//    slices, double-buffered in LDS. Each slice keeps its operand's global
//    orientation, unpadded: rows along k (B stored [k, n], A stored [k, m])
//    as they are, rows along m or n (A stored [m, k], B stored [n, k]) with
//    their 16-byte chunks XOR-swizzled. Interior slices of f32 operands go
//    straight from global memory to LDS (buffer_load_dwordx4 with the lds bit: no
//    registers, no LDS write instructions) while the MFMAs run on the other
//    buffer; edge and partial slices, and compact bf16 B, go through
//    registers (zero-filled, widened) and one 16-byte LDS write per chunk.
//    Each wave owns WM x WN of the tile as (WM/32) x (WN/32)
//    v_mfma_f32_32x32x2_f32 accumulators. A slice's k is summed in the order
//    8g + 4h + e (group g, lane half h, step e), so a swizzled row gives a
//    half's four k values of a group in one 16-byte read, and a k-major row
//    is read as 32 consecutive words per half-wave; every fill path and
//    transpose uses this order and gives the same bits. Four
//    configurations, picked by a time model: 256 x 256 tiles of 8 waves
//    (one per CU) for large products; 128 x 128 of 4 waves (two per CU) or
//    of 8 waves (one per CU, in steps of two slices when every workgroup
//    fits on the CUs at once); 64 x 64 of 8 waves in two k groups, in steps
//    of four slices, for products of about one such tile per CU. With one
//    slice per barrier every wave issues a part of the next slice's direct
//    loads at each of its k groups; the stepped kernels spread the older
//    waves' loads over the step (64 x 64) or issue them in one burst
//    (128 x 128). Tiles are ordered so that
//    consecutive tiles share a block row of A and each of the 8 XCDs (own
//    L2) gets a contiguous band of tiles. When the tiles cannot fill the
//    device, k is split: over up to 8 workgroups per tile (split-k), or in
//    equal runs of (tile, k slice) units per workgroup (stream-K) when the
//    tiles divide the device badly; partial tiles go to a workspace and a
//    second launch adds them in k order (deterministic) with the addend.
//  - m <= kGemvMaxRows (decode), or up to 32 rows of a small product with
//    k > 1024 in row blocks of 8: the work is reading B once (HBM-bound), so
//    each wave streams 256 columns of B (512 for compact bf16 weights on up
//    to 4 rows) with 16-byte loads over one k slice, keeping m x 4 partial
//    sums per lane; partial sums per k slice go to a workspace and a second
//    launch adds them in a fixed order (deterministic), four waves per 256
//    columns.
//  - 16-32 rows of a small product with k <= 1024: one launch of 32 x 32
//    MFMA tiles whose 16 waves split k and meet in LDS (small_mfma_kernel).
#include <type_traits>

#include <utility>

#include "common.hpp"

#include <mutex>
#include "internal.hpp"
#include "decode_merge.hpp"
#include "reduce.hpp"

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kGemvMaxRows = 8;

// The epilogue of a finished sum v with its addend element a. Modes 1 (a bias
// row, indexed by column) and 2 (a full matrix) add it; mode 3, internal to
// the library (the up product of a gated matmul, its addend the gate
// product), gates the sum as the silu-mul kernel does: silu(a) * v, so the
// gated product equals the two matmuls and silu-mul bit for bit. Modes 2 and
// 3 index the addend as the output.
__device__ __forceinline__ float apply_addend(float v, float a, int mode) {
    return mode == 3 ? mhip::silu1(a) * v : v + a;
}
__device__ __forceinline__ float4 apply_addend(float4 v, float4 a, int mode) {
    return make_float4(apply_addend(v.x, a.x, mode), apply_addend(v.y, a.y, mode),
                       apply_addend(v.z, a.z, mode), apply_addend(v.w, a.w, mode));
}
// Largest product (m x k x n multiply-adds) that 16-32 rows run on the small
// MFMA tiles or the GEMV's row blocks rather than on the large MFMA tiles.
constexpr uint64_t kGemvSmallProduct = 1ull << 26;

// Split-k partial sums live in the context's workspace; stream order makes
// reuse by the next call safe. During mhip_matmul_f32_noalloc they live in
// the device's fixed scratch array instead, and a product that needs more
// than it holds is refused.
mhip_status workspace(mhip_ctx* ctx, size_t bytes, float** out) {
    if (ctx->fixed_scratch) {
        if (bytes > ctx->fixed_scratch_bytes)
            return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                              "matmul: this product needs " + std::to_string(bytes) +
                                  " bytes of scratch; the allocation-free matmul has " +
                                  std::to_string(ctx->fixed_scratch_bytes));
        *out = static_cast<float*>(ctx->fixed_scratch);
        return MHIP_OK;
    }
    void* p = nullptr;
    mhip_status st = mhip::workspace(ctx, bytes, &p);
    *out = static_cast<float*>(p);
    return st;
}

// ---------------------------------------------------------------------------
// MFMA tiles
// ---------------------------------------------------------------------------

// KG: the waves form KG groups that each cover the whole tile over every
// KG-th part of each slice's k (summed in LDS at the end), so a small tile
// still gives each SIMD two waves.
template <int BM, int BN, int BK, int WM, int WN, bool A_T, bool B_T, int KG = 1, int STEP = 0>
struct TileCfg {
    static constexpr int kWavesN = BN / WN;
    static constexpr int kTileWaves = (BM / WM) * kWavesN;
    static constexpr int kWaves = kTileWaves * KG;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kMI = WM / 32;
    static constexpr int kNI = WN / 32;
    // LDS slices keep the operand's global orientation, unpadded: A as
    // [BK][BM] when stored [k, m] (A_T), else [BM][BK]; B as [BK][BN], or
    // [BN][BK] when stored [n, k] (B_T). Rows along m or n (BK floats each)
    // have their 16-byte chunks XOR-swizzled; rows along k are plain.
    static constexpr int kLdsA = BM * BK;
    static constexpr int kLdsB = BK * BN;
    // Tiles of at most 64 x 64 give a wave only 8 MFMAs per slice, too few
    // to cover a barrier and the first LDS reads of each slice: they move in
    // steps of kGroup slices (one barrier per step), double-buffered, so
    // kStages = 2 * kGroup slice buffers per operand. STEP > 0 sets kGroup
    // (launch_mfma picks 2 for 8-wave 128 x 128 tiles in a single wave of
    // workgroups).
    static constexpr int kGroup = STEP > 0 ? STEP : (BM * BN <= 64 * 64 ? 4 : 1);
    static constexpr int kStages = 2 * kGroup;
    static constexpr int kLdsFloats = kStages * (kLdsA + kLdsB);
    // Global slices as (rows x cols) with cols contiguous in memory.
    static constexpr int kARows = A_T ? BK : BM, kACols = A_T ? BM : BK;
    static constexpr int kBRows = B_T ? BN : BK, kBCols = B_T ? BK : BN;
    static constexpr int kAChunks = kARows * kACols / 4 / kThreads;
    static constexpr int kBChunks = kBRows * kBCols / 4 / kThreads;
    static_assert(kARows * kACols % (4 * kThreads) == 0, "A slice must split evenly");
    static_assert(kBRows * kBCols % (4 * kThreads) == 0, "B slice must split evenly");
    static_assert(BK == 32, "swizzled rows hold 8 chunks");
    static_assert(KG == 1 || KG == 2 || KG == 4, "k groups split a slice's 4 groups of 8");
    static_assert(KG == 1 || kTileWaves * kMI * kNI * 16 * 64 <= kLdsFloats,
                  "the k groups' sums are staged in the slice buffers");
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// XOR pattern of the 16-byte chunks of row r of an m- or n-major slice (8
// chunks per row). Distinct over any 8 consecutive rows, and (r & 1, pattern)
// distinct over 16, so 16-byte reads of one chunk position down 16 rows hit
// distinct banks.
__device__ __forceinline__ int chunk_swizzle(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Float offset in an LDS slice of the 16-byte chunk whose global position is
// (row r, column c) of a slice with COLS columns; SWZ for m- or n-major rows.
template <int COLS, bool SWZ>
__device__ __forceinline__ int chunk_offset(int r, int c) {
    if constexpr (SWZ)
        return r * COLS + (((c >> 2) ^ chunk_swizzle(r)) << 2);
    else
        return r * COLS + c;
}

using mhip::elem;
using mhip::load4;
using mhip::load4_nt;

// Loads this thread's chunks of a (ROWS x COLS) slice whose columns are
// contiguous in memory (leading dimension ld), rows from r0 and columns from
// c0, zero-filling outside (rows_total, cols_total).
template <int ROWS, int COLS, int CHUNKS, int THREADS, bool VEC, class T>
__device__ __forceinline__ void load_slice(float4 (&regs)[CHUNKS], const T* __restrict__ g,
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
            const T* p = g + gr * ld + gc;
            if (VEC && gc + 3 < cols_total) {
                v = load4(p);
            } else {
                if (gc + 0 < cols_total) v.x = elem(p + 0);
                if (gc + 1 < cols_total) v.y = elem(p + 1);
                if (gc + 2 < cols_total) v.z = elem(p + 2);
                if (gc + 3 < cols_total) v.w = elem(p + 3);
            }
        }
        regs[i] = v;
    }
}

// The same slice when it lies wholly inside the matrix (rows r0 .. r0 + ROWS
// and columns c0 .. c0 + COLS in range, 16-byte aligned rows): plain
// dwordx4 loads with no bounds checks, issued back to back.
template <int ROWS, int COLS, int CHUNKS, int THREADS, class T>
__device__ __forceinline__ void load_slice_interior(float4 (&regs)[CHUNKS], const T* __restrict__ g,
                                                    uint64_t ld, uint64_t r0, uint64_t c0) {
    constexpr int kChunksPerRow = COLS / 4;
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        const int chunk = threadIdx.x + i * THREADS;
        const int r = chunk / kChunksPerRow;
        const int c = (chunk % kChunksPerRow) * 4;
        regs[i] = load4(g + (r0 + r) * ld + c0 + c);
    }
}

// Stores the chunks into an LDS slice (one 16-byte write each, at the
// chunk's possibly swizzled position).
template <int ROWS, int COLS, int CHUNKS, int THREADS, bool SWZ>
__device__ __forceinline__ void store_slice(const float4 (&regs)[CHUNKS], float* lds) {
    constexpr int kChunksPerRow = COLS / 4;
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        const int chunk = threadIdx.x + i * THREADS;
        const int r = chunk / kChunksPerRow;
        const int c = (chunk % kChunksPerRow) * 4;
        *reinterpret_cast<float4*>(lds + chunk_offset<COLS, SWZ>(r, c)) = regs[i];
    }
}

// The same slice copied straight from global memory into LDS (interior
// slices of f32 operands, 16-byte aligned rows): one buffer_load_dwordx4 with
// the lds bit fills 64 consecutive 16-byte slots, lane i slot i, so each lane
// fetches the chunk that belongs in its slot. No registers, no LDS write
// instructions; completion is tracked by vmcnt (wait before the barrier).
// Buffer loads, not global_load_lds: the compiler counts a pending global
// (FLAT) load into LDS as a possible LDS access, and then waits for every
// LDS read at once (lgkmcnt(0)) before each MFMA group, so no operand read
// could run ahead of the MFMAs (4096^3 985 -> 961-968 us, 2048^3 141 ->
// 134 us). The buffer is the slice itself, from its first element, so the
// lane offsets are 32-bit: launch_mfma takes this path only for leading
// dimensions up to kDmaMaxLd.
// Word 3 of a raw (unformatted, unswizzled) buffer descriptor on gfx950.
constexpr int kRawBufferWord3 = 0x00020000;
// Longest leading dimension (floats) whose 256-row slice stays under 2^31
// bytes, the reach of a buffer's 32-bit lane offsets.
constexpr uint64_t kDmaMaxLd = 1ull << 21;

template <int ROWS, int COLS, int WAVES, bool SWZ>
__device__ __forceinline__ void dma_slice(const float* __restrict__ g, uint64_t ld, uint64_t r0,
                                          uint64_t c0, float* lds, int wave, int lane, int part = 0,
                                          int parts = 1) {
    constexpr unsigned kChunksPerRow = COLS / 4;
    static_assert(64 % kChunksPerRow == 0, "an instruction covers whole rows");
    constexpr unsigned kRowsPerInstr = 64 / kChunksPerRow;
    constexpr unsigned kPerWave = ROWS / kRowsPerInstr / WAVES;
    static_assert(kPerWave * kRowsPerInstr * WAVES == ROWS, "slice must split over the waves");
    // Lane l fills row l / kChunksPerRow of the instruction's rows, slot
    // l % kChunksPerRow. A swizzled row (8 chunks) r takes chunk
    // slot ^ (r & 7) ^ ((r >> 3) & 1): r & 7 is the lane's row, and bit 3
    // flips with the instruction's first row (a multiple of 8).
    const unsigned lr = static_cast<unsigned>(lane) / kChunksPerRow;
    const unsigned pos = static_cast<unsigned>(lane) % kChunksPerRow;
    const unsigned off0 = SWZ ? (pos ^ lr) * 4u : pos * 4u;
    const unsigned off1 = SWZ ? (pos ^ lr ^ 1u) * 4u : pos * 4u;
    const float* base = g + r0 * ld + c0;
    const uint32_t bytes = static_cast<uint32_t>(((ROWS - 1) * ld + COLS) * sizeof(float));
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, static_cast<int>(bytes), kRawBufferWord3);
    const unsigned j0 = kPerWave * part / parts, j1 = kPerWave * (part + 1) / parts;
#pragma unroll
    for (unsigned j = j0; j < j1; ++j) {
        const unsigned first = (static_cast<unsigned>(wave) * kPerWave + j) * kRowsPerInstr;
        const unsigned off = (SWZ && ((first >> 3) & 1u)) ? off1 : off0;
        const uint32_t voff = static_cast<uint32_t>(((lr + first) * ld + off) * sizeof(float));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(lds + first * COLS), 16, voff, 0, 0, 0);
    }
}

// Workgroup barrier of the stepped pipeline, where LDS is written only by
// direct loads that each issuing wave has already waited for: s_barrier
// without the release fence of __syncthreads (whose waits are done). Every
// LDS read of the previous step has returned (its MFMA was issued) before a
// wave arrives. The memory clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void step_barrier() { __asm__ volatile("s_barrier" ::: "memory"); }

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

// Scheduling of one slice's k steps (4 per group of 8 k): the LDS reads of
// step s + 2 are placed after the MFMAs of step s, so each step's operands
// are read a whole step ahead. Read counts per step for A swizzled (one
// 16-byte read per m block at a group's first step) and B k-major (the
// step's KNI floats, read in pairs).
template <int KMI, int KNI>
constexpr int step_reads(int s) { return (s % 4 == 0 ? KMI : 0) + (KNI + 1) / 2; }
template <int KMI, int KNI, int... S>
__device__ __forceinline__ void sched_reads_ahead(std::integer_sequence<int, S...>) {
    constexpr int kSteps = sizeof...(S);
    constexpr int kDsRead = 0x100, kMfma = 0x008;
    __builtin_amdgcn_sched_group_barrier(kDsRead, step_reads<KMI, KNI>(0), 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, step_reads<KMI, KNI>(1), 0);
    ((__builtin_amdgcn_sched_group_barrier(kMfma, KMI * KNI, 0),
      __builtin_amdgcn_sched_group_barrier(kDsRead, S + 2 < kSteps ? step_reads<KMI, KNI>(S + 2) : 0, 0)),
     ...);
}

// One tile's product, C[m0 .., n0 ..] summed over k in [k_begin, k_end),
// written to out[(row - out_r0) * ldo + (col - out_c0)] for the rows < M and
// columns < N, plus the addend when addend_mode is 1 or 2. LDS (`lds`) is
// free on entry and again on return. SPREAD lets the one-slice-per-barrier
// loop have every wave issue part of the next slice's direct loads (the
// stream-K kernel turns it off).
template <int BM, int BN, int BK, int WM, int WN, bool A_T, bool B_T, bool VEC, class BT, int KG = 1,
          int STEP = 0, bool SPREAD = true>
__device__ __forceinline__ void gemm_tile(const float* __restrict__ A, const BT* __restrict__ B,
                                          uint64_t M, uint64_t K, uint64_t N, uint64_t m0,
                                          uint64_t n0, uint64_t k_begin, uint64_t k_end,
                                          float* lds, float* __restrict__ out, uint64_t out_r0,
                                          uint64_t out_c0, uint64_t ldo,
                                          const float* __restrict__ addend, int addend_mode) {
    using Cfg = TileCfg<BM, BN, BK, WM, WN, A_T, B_T, KG, STEP>;
    constexpr int T = Cfg::kThreads;
    // A rows along m (not A_T) and B rows along n (B_T) are swizzled.
    constexpr bool kASwz = !A_T, kBSwz = B_T;
    constexpr bool kBDma = std::is_same<BT, float>::value;  // compact B is widened on the way
    // Buffer b of the A slices at lds + b * kLdsA; the B slices follow them all.
    float* const lds_b0 = lds + Cfg::kStages * Cfg::kLdsA;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int kg = wave / Cfg::kTileWaves;  // this wave's k group
    const int wt = wave % Cfg::kTileWaves;
    const int wm = wt / Cfg::kWavesN, wn = wt % Cfg::kWavesN;
    const int lrow = lane & 31, lk = lane >> 5;

    v16f acc[Cfg::kMI][Cfg::kNI];
#pragma unroll
    for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::kNI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Filling buffer `buf` with the slice at k0. A slice wholly inside the
    // matrices (every slice of an interior tile but the last partial one)
    // goes straight to LDS (f32 operands) or through unchecked loads
    // (compact B); any other slice through bounds-checked loads that
    // zero-fill past k_end and the matrix edges. `issue` starts the fill,
    // `finish` writes whatever went through registers.
    float4 ra[Cfg::kAChunks], rb[Cfg::kBChunks];
    const bool interior_tile = VEC && m0 + BM <= M && n0 + BN <= N;
    auto direct = [&](uint64_t k0) { return interior_tile && k0 + BK <= k_end; };
    // The direct loads of a slice are all issued by the first half of the
    // waves: the older wave on each SIMD, which wins MFMA arbitration and
    // otherwise finishes its share of the slice first and waits at the
    // barrier; the younger one starts its MFMAs at once. Measured: 4096^3
    // 87.4-88.3 -> 88.3-88.9 %, 8192^3 89.1 -> 89.8 %.
    constexpr int kDmaWaves = Cfg::kWaves / 2;
    auto issue = [&](uint64_t k0, int buf) {
        float* la = lds + buf * Cfg::kLdsA;
        float* lb = lds_b0 + buf * Cfg::kLdsB;
        if (direct(k0)) {
            if (wave < kDmaWaves) {
                if constexpr (A_T)
                    dma_slice<Cfg::kARows, Cfg::kACols, kDmaWaves, kASwz>(A, M, k0, m0, la, wave, lane);
                else
                    dma_slice<Cfg::kARows, Cfg::kACols, kDmaWaves, kASwz>(A, K, m0, k0, la, wave, lane);
                if constexpr (kBDma) {
                    if constexpr (B_T)
                        dma_slice<Cfg::kBRows, Cfg::kBCols, kDmaWaves, kBSwz>(
                            reinterpret_cast<const float*>(B), K, n0, k0, lb, wave, lane);
                    else
                        dma_slice<Cfg::kBRows, Cfg::kBCols, kDmaWaves, kBSwz>(
                            reinterpret_cast<const float*>(B), N, k0, n0, lb, wave, lane);
                }
            }
            if constexpr (!kBDma) {
                if constexpr (B_T)
                    load_slice_interior<Cfg::kBRows, Cfg::kBCols, Cfg::kBChunks, T>(rb, B, K, n0, k0);
                else
                    load_slice_interior<Cfg::kBRows, Cfg::kBCols, Cfg::kBChunks, T>(rb, B, N, k0, n0);
            }
            return;
        }
        if constexpr (A_T)
            load_slice<Cfg::kARows, Cfg::kACols, Cfg::kAChunks, T, VEC>(ra, A, M, k0, m0, k_end, M);
        else
            load_slice<Cfg::kARows, Cfg::kACols, Cfg::kAChunks, T, VEC>(ra, A, K, m0, k0, M, k_end);
        if constexpr (B_T)
            load_slice<Cfg::kBRows, Cfg::kBCols, Cfg::kBChunks, T, VEC>(rb, B, K, n0, k0, N, k_end);
        else
            load_slice<Cfg::kBRows, Cfg::kBCols, Cfg::kBChunks, T, VEC>(rb, B, N, k0, n0, k_end, N);
    };
    // Part `part` of `parts` of a direct slice's loads, issued by a DMA
    // wave (the caller's branch).
    auto issue_part_dma = [&](uint64_t k0, int buf, int part, int parts) {
        float* la = lds + buf * Cfg::kLdsA;
        float* lb = lds_b0 + buf * Cfg::kLdsB;
        if constexpr (kBDma) {
            if constexpr (A_T)
                dma_slice<Cfg::kARows, Cfg::kACols, kDmaWaves, kASwz>(A, M, k0, m0, la, wave, lane, part, parts);
            else
                dma_slice<Cfg::kARows, Cfg::kACols, kDmaWaves, kASwz>(A, K, m0, k0, la, wave, lane, part, parts);
            if constexpr (B_T)
                dma_slice<Cfg::kBRows, Cfg::kBCols, kDmaWaves, kBSwz>(
                    reinterpret_cast<const float*>(B), K, n0, k0, lb, wave, lane, part, parts);
            else
                dma_slice<Cfg::kBRows, Cfg::kBCols, kDmaWaves, kBSwz>(
                    reinterpret_cast<const float*>(B), N, k0, n0, lb, wave, lane, part, parts);
        }
    };
    auto finish = [&](uint64_t k0, int buf) {
        const bool dma = direct(k0);
        if (!dma)
            store_slice<Cfg::kARows, Cfg::kACols, Cfg::kAChunks, T, kASwz>(ra, lds + buf * Cfg::kLdsA);
        if (!dma || !kBDma)
            store_slice<Cfg::kBRows, Cfg::kBCols, Cfg::kBChunks, T, kBSwz>(rb, lds_b0 + buf * Cfg::kLdsB);
        __builtin_amdgcn_s_waitcnt(0);  // the direct loads have landed in LDS
    };

    // Operand reads. Every slice sums k in the order k = 8g + 4h + e over
    // groups g, halves h and steps e (0..3): at step (g, e) lanes of half h
    // (lane / 32) feed k = 8g + 4h + e. A swizzled row yields that half's 4
    // values of a group as one 16-byte read; a k-major slice is read one row
    // per step. Every fill path and operand orientation uses this order, so
    // they all give the same bits.
    const int hsw = lk ^ chunk_swizzle(lrow);  // rows wm*WM + i*32 + lrow share lrow & 15
    // Groups g0 + [0, count) of one slice (g0 < 0: this wave's k group's
    // share, kg * count + [0, count)); hook(gg, count) runs before group gg.
    auto compute_range = [&](int buf, auto hook, auto g0c, auto countc) {
        constexpr int g0 = decltype(g0c)::value, count = decltype(countc)::value;
        const float* la = lds + buf * Cfg::kLdsA;
        const float* lb = lds_b0 + buf * Cfg::kLdsB;
#pragma unroll
        for (int gg = 0; gg < count; ++gg) {
            hook(gg, count);
            const int g = (g0 < 0 ? kg * count : g0) + gg;
            mhip::f32x4 a4[Cfg::kMI], b4[Cfg::kNI];
            if constexpr (kASwz) {
#pragma unroll
                for (int i = 0; i < Cfg::kMI; ++i)
                    a4[i] = *reinterpret_cast<const mhip::f32x4*>(la + (wm * WM + i * 32 + lrow) * BK +
                                                             (((2 * g) ^ hsw) << 2));
            }
            if constexpr (kBSwz) {
#pragma unroll
                for (int j = 0; j < Cfg::kNI; ++j)
                    b4[j] = *reinterpret_cast<const mhip::f32x4*>(lb + (wn * WN + j * 32 + lrow) * BK +
                                                             (((2 * g) ^ hsw) << 2));
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = 8 * g + 4 * lk + e;
                float af[Cfg::kMI], bf[Cfg::kNI];
#pragma unroll
                for (int i = 0; i < Cfg::kMI; ++i) {
                    if constexpr (kASwz) af[i] = a4[i][e];
                    else af[i] = la[k * BM + wm * WM + i * 32 + lrow];
                }
#pragma unroll
                for (int j = 0; j < Cfg::kNI; ++j) {
                    if constexpr (kBSwz) bf[j] = b4[j][e];
                    else bf[j] = lb[k * BN + wn * WN + j * 32 + lrow];
                }
#pragma unroll
                for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::kNI; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
    };
    constexpr int kGroups = BK / 8 / KG;  // groups of 8 k per wave and slice
    auto compute_body = [&](int buf, auto hook) {
        compute_range(buf, hook, std::integral_constant<int, -1>{}, std::integral_constant<int, kGroups>{});
    };
    // The 64-tile kernel (k groups, one MFMA per k step) gets its LDS reads
    // ahead of the MFMAs (1024^3 25.4 -> 24.4 us); the larger tiles' own
    // schedule was as fast. N k steps in one scheduling region.
    constexpr bool kReadAhead = KG > 1 && kASwz && !kBSwz;
    auto schedule = [&](auto n) {
        if constexpr (kReadAhead)
            sched_reads_ahead<Cfg::kMI, Cfg::kNI>(std::make_integer_sequence<int, decltype(n)::value>{});
    };
    constexpr int kSliceSteps = BK / 8 / KG * 4;  // k steps per wave and slice
    auto no_hook = [](int, int) {};
    // Two k groups split a slice's four groups of 8 k unevenly on every
    // fourth slice from the start of the k range (first of each step):
    // group 0 (waves 0-3) takes groups 0-2, group 1 group 3; elsewhere 0-1
    // and 2-3. Group 0's waves are the older wave on each SIMD, which wins
    // MFMA arbitration and finished its even share ~1,700 cycles per step
    // before the younger one, which then ran alone (1024^3 21.8-21.9 ->
    // 21.1-21.3 us; 10 of 16 groups to group 0 was slower, 21.5-21.8; the
    // uneven slice's place in the step did not matter). Every path of the
    // kernel follows the same split, so its results stay independent of
    // operand layout and weight format.
    constexpr bool kUneven = KG == 2 && Cfg::kGroup % 4 == 0;  // steps start every fourth slice
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    // Slice `s` (from k_begin) by k group `grp` (0 or 1).
    auto compute_uneven = [&](int buf, auto hook, bool first, auto grp) {
        if constexpr (decltype(grp)::value == 0) {
            if (first) compute_range(buf, hook, I0{}, I3{});
            else compute_range(buf, hook, I0{}, I2{});
        } else {
            if (first) compute_range(buf, hook, I3{}, I1{});
            else compute_range(buf, hook, I2{}, I2{});
        }
    };
    auto compute = [&](int buf, uint64_t s) {
        if constexpr (kUneven) {
            // Outside whole steps (edge tiles, a last partial step, compact
            // B): the same groups in the same order, one group at a time.
            const bool first = s % 4 == 0;
            const int g_lo = kg == 0 ? 0 : (first ? 3 : 2);
            const int g_hi = kg == 0 ? (first ? 3 : 2) : 4;
            const float* la = lds + buf * Cfg::kLdsA;
            const float* lb = lds_b0 + buf * Cfg::kLdsB;
            for (int g = g_lo; g < g_hi; ++g) {
                mhip::f32x4 a4[Cfg::kMI], b4[Cfg::kNI];
                if constexpr (kASwz) {
#pragma unroll
                    for (int i = 0; i < Cfg::kMI; ++i)
                        a4[i] = *reinterpret_cast<const mhip::f32x4*>(la + (wm * WM + i * 32 + lrow) * BK +
                                                                 (((2 * g) ^ hsw) << 2));
                }
                if constexpr (kBSwz) {
#pragma unroll
                    for (int j = 0; j < Cfg::kNI; ++j)
                        b4[j] = *reinterpret_cast<const mhip::f32x4*>(lb + (wn * WN + j * 32 + lrow) * BK +
                                                                 (((2 * g) ^ hsw) << 2));
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = 8 * g + 4 * lk + e;
                    float af[Cfg::kMI], bf[Cfg::kNI];
#pragma unroll
                    for (int i = 0; i < Cfg::kMI; ++i) {
                        if constexpr (kASwz) af[i] = a4[i][e];
                        else af[i] = la[k * BM + wm * WM + i * 32 + lrow];
                    }
#pragma unroll
                    for (int j = 0; j < Cfg::kNI; ++j) {
                        if constexpr (kBSwz) bf[j] = b4[j][e];
                        else bf[j] = lb[k * BN + wn * WN + j * 32 + lrow];
                    }
#pragma unroll
                    for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
                        for (int j = 0; j < Cfg::kNI; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
            }
        } else {
            compute_body(buf, no_hook);
            schedule(std::integral_constant<int, kSliceSteps>{});
        }
    };

    const uint64_t slices = (k_end - k_begin + BK - 1) / BK;
    constexpr int G = Cfg::kGroup;
    // One slice per barrier (the 256 x 256 and 128 x 128 tiles): the next
    // slice's direct loads are issued by every wave, a part at the start of
    // each of its k groups, between the MFMAs (4096^3 968 -> 942-947 us,
    // 6144^3 3470 -> 3390 us, 3072^3 480 -> 461 us; the same bits). Issued in
    // one burst by the older wave of each SIMD, they held that wave ~1,400
    // cycles per slice before its first MFMA. The stream-K kernel spreads
    // the first part of each run only: a second spread copy spilled.
    constexpr bool kSpread = SPREAD && KG == 1 && G == 1 && kBDma;
    auto part_all = [&](uint64_t k0, int buf, int part, int parts) {
        if constexpr (kSpread) {
            float* la = lds + buf * Cfg::kLdsA;
            float* lb = lds_b0 + buf * Cfg::kLdsB;
            if constexpr (A_T)
                dma_slice<Cfg::kARows, Cfg::kACols, Cfg::kWaves, kASwz>(A, M, k0, m0, la, wave, lane, part, parts);
            else
                dma_slice<Cfg::kARows, Cfg::kACols, Cfg::kWaves, kASwz>(A, K, m0, k0, la, wave, lane, part, parts);
            if constexpr (B_T)
                dma_slice<Cfg::kBRows, Cfg::kBCols, Cfg::kWaves, kBSwz>(
                    reinterpret_cast<const float*>(B), K, n0, k0, lb, wave, lane, part, parts);
            else
                dma_slice<Cfg::kBRows, Cfg::kBCols, Cfg::kWaves, kBSwz>(
                    reinterpret_cast<const float*>(B), N, k0, n0, lb, wave, lane, part, parts);
        }
    };
    if (G > 1 && kBDma && interior_tile && (k_end - k_begin) % BK == 0) {
        // Every slice goes straight to LDS. Steps of G slices, double-
        // buffered: at step t the DMA waves wait for step t's loads, the
        // barrier publishes them and frees the other buffer set (read in
        // step t - 1), which then takes step t + 1 while step t computes.
        // (Three sets of three-slice steps, or four of two-slice steps, with
        // the loads two or three steps ahead, ran 1024^3 at 26.1 and 27.5 us
        // against 24.0: the barriers per step cost more than load latency.)
        const uint64_t steps = (slices + G - 1) / G;
        const uint64_t full_steps = slices / G;
        auto set_of = [&](uint64_t t) { return static_cast<int>(t & 1) * G; };
        auto issue_step = [&](uint64_t t) {
            const int set = set_of(t);
#pragma unroll
            for (int j = 0; j < G; ++j)
                if (t * G + j < slices) issue(k_begin + (t * G + j) * BK, set + j);
        };
        issue_step(0);
        for (uint64_t t = 0; t < steps; ++t) {
            __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of step t have landed
            step_barrier();
            const int set = set_of(t);
            const uint64_t tn = t + 1;  // the step whose loads go out now
            const bool next = tn < steps;
            const int nset = set_of(tn);
            if constexpr (kReadAhead) {
                // Several slices per step, each step in one scheduling region,
                // so the reads of each slice's first k steps go out during
                // the previous slice's MFMAs (1024^3 24.3-24.6 -> 23.9-24.1
                // us). When the next step is whole, its loads go out spread
                // over this step's k groups, slice j's during slice j (1024^3
                // 23.9 -> 22.2 us); DMA and other waves then run separate
                // copies of the step, so neither branches inside it.
                auto loads_of = [&](int j) {
                    return [&, j](int gg, int groups) {
                        issue_part_dma(k_begin + (tn * G + j) * BK, nset + j, gg, groups);
                    };
                };
                auto none = [&](int) { return no_hook; };
                // A whole step by k group grp (the DMA waves are group 0).
                auto run_step = [&](auto hook, auto grp) {
                    if constexpr (kUneven && G % 4 == 0) {
#pragma unroll
                        for (int j = 0; j < G; ++j) compute_uneven(set + j, hook(j), j % 4 == 0, grp);
                        constexpr int kFirst = decltype(grp)::value == 0 ? 12 : 4;
                        schedule(std::integral_constant<int, G / 4 * kFirst + (G - G / 4) * 8>{});
                    } else {
#pragma unroll
                        for (int j = 0; j < G; ++j) compute_body(set + j, hook(j));
                        schedule(std::integral_constant<int, G * kSliceSteps>{});
                    }
                };
                static_assert(!kUneven || kDmaWaves == Cfg::kTileWaves, "the DMA waves are k group 0");
                if (next && tn < full_steps) {
                    if (wave < kDmaWaves) run_step(loads_of, I0{});
                    else run_step(none, I1{});
                    continue;
                }
                if (next) issue_step(tn);
                if (t < full_steps) {
                    if (wave < kDmaWaves) run_step(none, I0{});
                    else run_step(none, I1{});
                    continue;
                }
#pragma unroll
                for (int j = 0; j < G; ++j)
                    if (t * G + j < slices) compute(set + j, t * G + j);
            } else {
                // The 8-wave 128 x 128 tiles: the loads in one burst, one
                // block per slice (their own schedule of whole steps was
                // slower, 2048^3 134.4 -> 138.5 us, and so was spreading
                // the loads, 134.5 -> 135.9-141 us in three arrangements, or
                // issuing each slice's loads just before the same slice of
                // this step, 134.2 -> 134.7-135.3 us; every wave issuing a
                // part of them at each k group, 134.3-134.5 -> 134.2-134.9).
                if (next) issue_step(tn);
#pragma unroll
                for (int j = 0; j < G; ++j)
                    if (t * G + j < slices) compute(set + j, t * G + j);
            }
        }
        __syncthreads();
    } else if (kSpread && interior_tile && k_end > k_begin && (k_end - k_begin) % BK == 0) {
        // Every slice goes straight to LDS, double-buffered, one barrier per
        // slice: each wave waits for its own loads of slice s + 1 (issued
        // during slice s), then the barrier publishes them and frees the
        // buffer slice s was read from.
        if constexpr (kSpread) {
            part_all(k_begin, 0, 0, 1);
            __builtin_amdgcn_s_waitcnt(0);
            step_barrier();
            for (uint64_t s = 0; s + 1 < slices; ++s) {
                const int buf = static_cast<int>(s & 1);
                const uint64_t k_next = k_begin + (s + 1) * BK;
                compute_body(buf, [&](int gg, int groups) { part_all(k_next, buf ^ 1, gg, groups); });
                // Each k step's LDS reads after the previous step's MFMAs
                // (A stored [m, k], B stored [k, n]): 3072^3 460 -> 455 us,
                // 4096^3 and 6144^3 within 0.3 %, the same bits.
                if constexpr (kASwz && !kBSwz)
                    sched_reads_ahead<Cfg::kMI, Cfg::kNI>(std::make_integer_sequence<int, kSliceSteps>{});
                __builtin_amdgcn_s_waitcnt(0);
                step_barrier();
            }
            compute(static_cast<int>((slices - 1) & 1), slices - 1);
            __syncthreads();
        }
    } else {
        issue(k_begin, 0);
        finish(k_begin, 0);
        __syncthreads();
        for (uint64_t s = 0; s < slices; ++s) {
            const int buf = static_cast<int>(s & 1);
            const uint64_t k_next = k_begin + (s + 1) * BK;
            if (s + 1 < slices) issue(k_next, buf ^ 1);
            compute(buf, s);
            if (s + 1 < slices) finish(k_next, buf ^ 1);
            __syncthreads();
        }
    }

    // Accumulator r of lane l holds C[8*(r/4) + 4*(l/32) + r%4][l%32] of its
    // 32x32 block; registers [R0, R1) are written.
    auto store = [&](auto r0, auto r1) {
#pragma unroll
        for (int i = 0; i < Cfg::kMI; ++i) {
#pragma unroll
            for (int j = 0; j < Cfg::kNI; ++j) {
                const uint64_t col = n0 + wn * WN + j * 32 + lrow;
                if (col >= N) continue;
#pragma unroll
                for (int r = decltype(r0)::value; r < decltype(r1)::value; ++r) {
                    const uint64_t row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * lk + (r % 4);
                    if (row < M) {
                        float v = acc[i][j][r];
                        if (addend_mode == 1) v = v + addend[col];
                        else if (addend_mode >= 2) v = apply_addend(v, addend[row * N + col], addend_mode);
                        // The 64-tile kernel writes C non-temporally: all
                        // its workgroups store at once, at the end (1024^3
                        // 21.0-21.3 -> 20.9 us, 768x1024x1024 28.7 -> 28.0
                        // us); for the larger tiles it was 0.5-0.9 % slower.
                        if constexpr (KG == 2)
                            __builtin_nontemporal_store(v, out + (row - out_r0) * ldo + (col - out_c0));
                        else
                            out[(row - out_r0) * ldo + (col - out_c0)] = v;
                    }
                }
            }
        }
    };
    using R0 = std::integral_constant<int, 0>;
    using R8 = std::integral_constant<int, 8>;
    using R16 = std::integral_constant<int, 16>;

    if constexpr (KG == 2) {
        // Two k groups: each finishes half of every block's rows, group 0
        // registers 0-7 (rows 0-15 of a 32x32 block), group 1 registers
        // 8-15, handing the other half to its partner through LDS (free
        // after the loop's last barrier), so both groups add and write. The
        // sum is group 0's plus group 1's either way.
        constexpr int kHalf = Cfg::kMI * Cfg::kNI * 8 * 64;  // floats per wave and half
        float* const given = lds + (kg * Cfg::kTileWaves + wt) * kHalf;
        const float* const taken = lds + ((1 - kg) * Cfg::kTileWaves + wt) * kHalf;
        auto give = [&](auto base) {
#pragma unroll
            for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
                for (int j = 0; j < Cfg::kNI; ++j)
#pragma unroll
                    for (int r = 0; r < 8; ++r)
                        given[((i * Cfg::kNI + j) * 8 + r) * 64 + lane] = acc[i][j][decltype(base)::value + r];
        };
        auto take = [&](auto base, auto first) {
#pragma unroll
            for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
                for (int j = 0; j < Cfg::kNI; ++j)
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const float a = acc[i][j][decltype(base)::value + r];
                        const float b = taken[((i * Cfg::kNI + j) * 8 + r) * 64 + lane];
                        acc[i][j][decltype(base)::value + r] = decltype(first)::value ? a + b : b + a;
                    }
        };
        if (kg == 0) give(R8{});
        else give(R0{});
        __syncthreads();
        if (kg == 0) take(R0{}, std::true_type{});
        else take(R8{}, std::false_type{});
        __syncthreads();  // LDS is free again
        if (kg == 0) store(R0{}, R8{});
        else store(R8{}, R16{});
        return;
    } else if constexpr (KG > 1) {
        // k groups: the others' sums meet group 0's in LDS (free after the
        // loop's last barrier), added in group order; group 0 writes the tile.
        constexpr int kPer = Cfg::kMI * Cfg::kNI * 16 * 64;  // floats per wave
        for (int q = 1; q < KG; ++q) {
            if (kg == q) {
#pragma unroll
                for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::kNI; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            lds[wt * kPer + ((i * Cfg::kNI + j) * 16 + r) * 64 + lane] = acc[i][j][r];
            }
            __syncthreads();
            if (kg == 0) {
#pragma unroll
                for (int i = 0; i < Cfg::kMI; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::kNI; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[i][j][r] += lds[wt * kPer + ((i * Cfg::kNI + j) * 16 + r) * 64 + lane];
            }
            __syncthreads();  // LDS is free again
        }
        if (kg != 0) return;
    }
    store(R0{}, R16{});
}

// One tile per workgroup. blockIdx.y is the k split: the workgroup sums k in
// [y * k_split, min(K, (y + 1) * k_split)) and, with more than one split,
// writes that partial product to C + y * M * N (no addend) for
// splitk_reduce_kernel.
template <int BM, int BN, int BK, int WM, int WN, bool A_T, bool B_T, bool VEC, class BT, int KG, int STEP>
__global__ __launch_bounds__((TileCfg<BM, BN, BK, WM, WN, A_T, B_T, KG, STEP>::kThreads), 2) void mfma_gemm_kernel(
    const float* __restrict__ A, const BT* __restrict__ B, float* __restrict__ C, uint64_t M,
    uint64_t K, uint64_t N, const float* __restrict__ addend, int addend_mode, uint64_t k_split) {
    extern __shared__ float lds[];
    uint32_t tm, tn;
    tile_coords(static_cast<uint32_t>((M + BM - 1) / BM), static_cast<uint32_t>((N + BN - 1) / BN),
                &tm, &tn);
    const uint64_t k_begin = static_cast<uint64_t>(blockIdx.y) * k_split;
    const uint64_t k_end = min(K, k_begin + k_split);
    const bool split = gridDim.y > 1;
    float* out = split ? C + static_cast<uint64_t>(blockIdx.y) * M * N : C;
    gemm_tile<BM, BN, BK, WM, WN, A_T, B_T, VEC, BT, KG, STEP>(
        A, B, M, K, N, static_cast<uint64_t>(tm) * BM, static_cast<uint64_t>(tn) * BN, k_begin,
        k_end, lds, out, 0, 0, N, addend, split ? 0 : addend_mode);
}

// Stream-K: the (tile, k slice) units, tile-major (tile t = tm * tiles_n +
// tn, its slices in k order), are dealt in equal runs of `per` to the
// workgroups, so every CU does the same MFMA work however the tiles divide.
// Workgroup w covers units [w * per, (w + 1) * per); per <= slices per tile,
// so that run touches at most two tiles, and the part of the j-th one goes to
// slot 2w + j as a BM x BN tile for stream_reduce_kernel.
template <int BM, int BN, int BK, int WM, int WN, bool A_T, bool B_T, bool VEC, class BT, int KG, int STEP>
__global__ __launch_bounds__((TileCfg<BM, BN, BK, WM, WN, A_T, B_T, KG, STEP>::kThreads), 2) void mfma_gemm_stream_kernel(
    const float* __restrict__ A, const BT* __restrict__ B, float* __restrict__ slots, uint64_t M,
    uint64_t K, uint64_t N, uint64_t per) {
    extern __shared__ float lds[];
    const uint64_t tiles_n = (N + BN - 1) / BN;
    const uint64_t kslices = (K + BK - 1) / BK;
    const uint64_t total = (M + BM - 1) / BM * tiles_n * kslices;
    const uint64_t u0 = static_cast<uint64_t>(blockIdx.x) * per;
    const uint64_t end = min(total, u0 + per);
    if (u0 >= end) return;
    // The run's first part and, when it crosses into the next tile, its
    // second (k from 0). Only the first spreads its direct loads over the
    // waves (SPREAD): with both, or with the parts in a loop, the kernel
    // spilled registers. 1280 x 512 x 3328 60.5 -> 59.5 us, 512 x 4096 x
    // 11008 356.5 -> 356.0 us, the same bits.
    const uint64_t t0 = u0 / kslices, a0 = u0 % kslices;
    const uint64_t b0 = min(kslices, a0 + (end - u0));
    {
        const uint64_t m0 = t0 / tiles_n * BM, n0 = t0 % tiles_n * BN;
        gemm_tile<BM, BN, BK, WM, WN, A_T, B_T, VEC, BT, KG, STEP, true>(
            A, B, M, K, N, m0, n0, a0 * BK, min(K, b0 * BK), lds,
            slots + (2 * static_cast<uint64_t>(blockIdx.x)) * (BM * BN), m0, n0, BN, nullptr, 0);
    }
    const uint64_t u1 = u0 + (b0 - a0);
    if (u1 < end) {
        const uint64_t t1 = u1 / kslices;
        const uint64_t b1 = min(kslices, end - u1);
        const uint64_t m0 = t1 / tiles_n * BM, n0 = t1 % tiles_n * BN;
        gemm_tile<BM, BN, BK, WM, WN, A_T, B_T, VEC, BT, KG, STEP, false>(
            A, B, M, K, N, m0, n0, 0, min(K, b1 * BK), lds,
            slots + (2 * static_cast<uint64_t>(blockIdx.x) + 1) * (BM * BN), m0, n0, BN, nullptr, 0);
    }
}

// C = the stream-K slots covering each output's tile, added in k order (the
// workgroups' order), + addend: deterministic. Four consecutive outputs per
// thread; `vec` (N % 4 == 0, aligned C and addend): one dwordx4 each.
template <int BM, int BN>
__global__ __launch_bounds__(256) void stream_reduce_kernel(const float* __restrict__ slots,
                                                            float* __restrict__ C, uint64_t M,
                                                            uint64_t N, uint64_t kslices,
                                                            uint64_t per,
                                                            const float* __restrict__ addend,
                                                            int addend_mode, int vec) {
    const uint64_t total = M * N;
    const uint64_t i = (static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= total) return;
    const uint64_t tiles_n = (N + BN - 1) / BN;
    auto slot_of = [&](uint64_t row, uint64_t col, uint64_t* w_first, uint64_t* w_last) {
        const uint64_t t = row / BM * tiles_n + col / BN;
        *w_first = t * kslices / per;
        *w_last = ((t + 1) * kslices - 1) / per;
        return t * kslices;  // the tile's first unit
    };
    auto at = [&](uint64_t w, uint64_t first_unit, uint64_t row, uint64_t col) {
        const uint64_t seg = w * per < first_unit ? 1 : 0;
        return slots + (2 * w + seg) * (BM * BN) + (row % BM) * BN + col % BN;
    };
    if (vec && i + 3 < total) {
        const uint64_t row = i / N, col = i % N;  // four columns of one tile (BN % 4 == 0)
        uint64_t w0, w1;
        const uint64_t first = slot_of(row, col, &w0, &w1);
        float4 v = mhip::load_nt(reinterpret_cast<const float4*>(at(w0, first, row, col)));
        for (uint64_t w = w0 + 1; w <= w1; ++w) {
            const float4 p = mhip::load_nt(reinterpret_cast<const float4*>(at(w, first, row, col)));
            v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
        }
        if (addend_mode == 1) {
            const float4 b = *reinterpret_cast<const float4*>(addend + col);
            v.x = v.x + b.x; v.y = v.y + b.y; v.z = v.z + b.z; v.w = v.w + b.w;
        } else if (addend_mode >= 2) {
            v = apply_addend(v, *reinterpret_cast<const float4*>(addend + i), addend_mode);
        }
        *reinterpret_cast<float4*>(C + i) = v;
        return;
    }
    for (uint64_t e = i; e < i + 4 && e < total; ++e) {
        const uint64_t row = e / N, col = e % N;
        uint64_t w0, w1;
        const uint64_t first = slot_of(row, col, &w0, &w1);
        float v = *at(w0, first, row, col);
        for (uint64_t w = w0 + 1; w <= w1; ++w) v += *at(w, first, row, col);
        if (addend_mode == 1) v = v + addend[col];
        else if (addend_mode >= 2) v = apply_addend(v, addend[e], addend_mode);
        C[e] = v;
    }
}

// C = sum over splits s = 0, 1, ... of partial[s] (+ addend), added in split
// order: deterministic. Four floats per thread; `vec`: as one dwordx4.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial,
                                                            float* __restrict__ C, uint64_t M,
                                                            uint64_t N, uint32_t splits,
                                                            const float* __restrict__ addend,
                                                            int addend_mode, int vec) {
    const uint64_t total = M * N;
    const uint64_t i = (static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= total) return;
    if (vec && i + 3 < total) {
        float4 v = mhip::load_nt(reinterpret_cast<const float4*>(partial + i));
        for (uint32_t s = 1; s < splits; ++s) {
            const float4 p = mhip::load_nt(reinterpret_cast<const float4*>(partial + s * total + i));
            v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
        }
        if (addend_mode == 1) {
            const float4 b = *reinterpret_cast<const float4*>(addend + i % N);
            v.x = v.x + b.x; v.y = v.y + b.y; v.z = v.z + b.z; v.w = v.w + b.w;
        } else if (addend_mode >= 2) {
            v = apply_addend(v, *reinterpret_cast<const float4*>(addend + i), addend_mode);
        }
        *reinterpret_cast<float4*>(C + i) = v;
        return;
    }
    for (uint64_t e = i; e < i + 4 && e < total; ++e) {
        float v = partial[e];
        for (uint32_t s = 1; s < splits; ++s) v += partial[s * total + e];
        if (addend_mode == 1) v = v + addend[e % N];
        else if (addend_mode >= 2) v = apply_addend(v, addend[e], addend_mode);
        C[e] = v;
    }
}

// How many k splits fill the device best: minimises the number of rounds of
// `slots` resident workgroups per unit of full-k work, ceil(tiles * s /
// slots) / s, keeping each split at least 256 deep (and a multiple of bk).
uint64_t choose_splits(uint64_t tiles, uint64_t k, uint64_t slots, uint64_t bk,
                       uint64_t* k_split) {
    uint64_t best = 1;
    double best_cost = static_cast<double>((tiles + slots - 1) / slots);
    for (uint64_t s = 2; s <= 8; ++s) {
        if (k / s < 256) break;
        const double cost = static_cast<double>((tiles * s + slots - 1) / slots) / static_cast<double>(s);
        if (cost < best_cost * (1.0 - 1e-9)) {
            best = s;
            best_cost = cost;
        }
    }
    uint64_t per = (k + best - 1) / best;
    per = (per + bk - 1) / bk * bk;
    *k_split = per;
    return (k + per - 1) / per;
}

// How one tile configuration covers an m x k x n product on `slots`
// resident workgroups: k splits of whole tiles (split-k, one launch per
// round of tiles), or stream-K runs of `per` (tile, k slice) units when that
// gives every workgroup less work (tiles that do not divide the device).
struct GemmPlan {
    uint64_t tiles, kslices;
    uint64_t splits, k_split;  // split-k
    bool stream;
    uint64_t per, groups;      // stream-K: units per workgroup, workgroups
    uint64_t steps;            // k slices per workgroup along the critical path
    double partial_tiles;      // partial-result traffic, in whole products (m x n)
};

GemmPlan plan_gemm(uint64_t m, uint64_t k, uint64_t n, uint64_t bm, uint64_t bn, uint64_t bk,
                   uint64_t slots) {
    GemmPlan p{};
    p.tiles = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    p.kslices = (k + bk - 1) / bk;
    p.splits = choose_splits(p.tiles, k, slots, bk, &p.k_split);
    const uint64_t rounds = (p.tiles * p.splits + slots - 1) / slots;
    p.steps = rounds * ((p.k_split + bk - 1) / bk);
    p.partial_tiles = p.splits > 1 ? static_cast<double>(p.splits) : 0.0;
    const uint64_t units = p.tiles * p.kslices;
    const uint64_t per = (units + slots - 1) / slots;
    // Stream-K when it cuts the critical path by over 10 %; its runs must
    // stay within two tiles (per <= kslices) and, as splits do, cover at
    // least 256 of k (8 slices of 32), or partial results outweigh them.
    if (p.tiles < slots && per <= p.kslices && per * bk >= 256 && per * 10 < p.steps * 9) {
        p.stream = true;
        p.per = per;
        p.groups = (units + per - 1) / per;
        p.steps = per;
        p.partial_tiles = static_cast<double>(p.groups + p.tiles) / static_cast<double>(p.tiles);
    }
    return p;
}

// Estimated seconds for an m x k x n product with one tile configuration:
// the critical path's k slices at the configuration's measured fraction of
// peak, plus the partial results' traffic, plus a fixed cost per launch (a
// k split or stream-K adds the reduction's). Splits are planned for
// `plan_per_cu` workgroups per CU. The workgroups resident on a CU share its
// MFMA pipes; below two waves per SIMD a wave's LDS reads are exposed, so
// the fraction scales with waves per SIMD / 2 (one 4-wave workgroup per CU
// measured about half the 2-workgroup rate). Picks among the tile kernels.
double gemm_seconds(const mhip_ctx* ctx, uint64_t m, uint64_t k, uint64_t n, uint64_t bm,
                    uint64_t bn, uint64_t bk, uint64_t plan_per_cu, int waves, double efficiency) {
    const uint64_t cus = ctx->compute_units ? ctx->compute_units : 256;
    const uint64_t slots = plan_per_cu * cus;
    const GemmPlan p = plan_gemm(m, k, n, bm, bn, bk, slots);
    const uint64_t wgs = p.stream ? p.groups : p.tiles * p.splits;
    const uint64_t resident =
        std::max<uint64_t>(1, std::min<uint64_t>(plan_per_cu, (std::min(wgs, slots) + cus - 1) / cus));
    const double per_simd = static_cast<double>(resident * waves) / 4.0;
    const double occupancy = std::min(1.0, per_simd / 2.0);
    const double cu_flops = 157.3e12 / 256.0;  // dense fp32 MFMA per CU per second
    const double slot_flops = cu_flops * efficiency * occupancy / static_cast<double>(resident);
    // A dependent launch costs about 4 us on this device even when it moves
    // little (start-up, the first memory latency, end-of-kernel cache work).
    constexpr double kLaunchSeconds = 4.0e-6;
    double t = static_cast<double>(p.steps) * 2.0 * bm * bn * bk / slot_flops + kLaunchSeconds;
    if (p.partial_tiles > 0.0) t += (p.partial_tiles + 1.0) * m * n * 4.0 / 5.0e12 + kLaunchSeconds;
    return t;
}

// Workgroups per CU a tile configuration is planned for: as many as fit the
// 160 KB of LDS, except that a configuration of 8 waves already gives each
// SIMD two waves with one workgroup, so it is planned one per CU.
template <class Cfg>
constexpr uint64_t plan_per_cu() {
    return Cfg::kWaves >= 8 ? 1 : std::max<uint64_t>(1, (160u * 1024u) / (Cfg::kLdsFloats * sizeof(float)));
}

template <int BM, int BN, int BK, int WM, int WN, bool A_T, bool B_T, class BT, int KG = 1,
          int STEP = 0>
mhip_status launch_mfma(mhip_ctx* ctx, const float* a, const BT* b, float* c, uint64_t m,
                        uint64_t k, uint64_t n, const float* addend, int mode, bool vec) {
    using Cfg = TileCfg<BM, BN, BK, WM, WN, A_T, B_T, KG, STEP>;
    const uint64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (tiles >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul: too many tiles");
    const uint64_t slots = plan_per_cu<Cfg>() * (ctx->compute_units ? ctx->compute_units : 256);
    const GemmPlan plan = plan_gemm(m, k, n, BM, BN, BK, slots);
    // 8-wave 128 x 128 tiles whose workgroups all fit in one wave on the CUs
    // take the stepped pipeline (two slices per barrier; 128 KB of LDS, which
    // leaves no room for a second workgroup, so only then): 2048^3 143 ->
    // 139 us, 512 x 4096 x 4096 148 -> 145 us; at 3072^3 (nine workgroups per
    // CU in turn) it was 488 -> 515 us. The same bits either way.
    if constexpr (STEP == 0 && BM * BN == 128 * 128 && Cfg::kWaves >= 8) {
        const uint64_t wgs = plan.stream ? plan.groups : tiles * plan.splits;
        if (wgs <= (ctx->compute_units ? ctx->compute_units : 256))
            return launch_mfma<BM, BN, BK, WM, WN, A_T, B_T, BT, KG, 2>(ctx, a, b, c, m, k, n, addend, mode, vec);
    }
    const size_t lds = Cfg::kLdsFloats * sizeof(float);
    static bool configured = false;  // raise the dynamic-LDS cap above 64 KiB once
    if (!configured) {
        for (const void* f : {reinterpret_cast<const void*>(&mfma_gemm_kernel<BM, BN, BK, WM, WN, A_T, B_T, true, BT, KG, STEP>),
                              reinterpret_cast<const void*>(&mfma_gemm_kernel<BM, BN, BK, WM, WN, A_T, B_T, false, BT, KG, STEP>),
                              reinterpret_cast<const void*>(&mfma_gemm_stream_kernel<BM, BN, BK, WM, WN, A_T, B_T, true, BT, KG, STEP>),
                              reinterpret_cast<const void*>(&mfma_gemm_stream_kernel<BM, BN, BK, WM, WN, A_T, B_T, false, BT, KG, STEP>)})
            (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        configured = true;
    }
    const uint64_t groups_out = (m * n + 1023) / 1024;
    if (groups_out >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul: output too large");
    // dwordx4 reduction: whole rows of 4 and 16-byte aligned output and addend.
    const int vec4 = n % 4 == 0 && mhip::aligned16(c) && (mode == 0 || mhip::aligned16(addend));

    if (plan.stream) {
        float* slot_mem = nullptr;
        mhip_status st = workspace(ctx, plan.groups * 2 * BM * BN * sizeof(float), &slot_mem);
        if (st != MHIP_OK) return st;
        const dim3 grid(static_cast<unsigned>(plan.groups));
        if (vec)
            mhip::launch(ctx,
                         (mfma_gemm_stream_kernel<BM, BN, BK, WM, WN, A_T, B_T, true, BT, KG, STEP>),
                         grid, dim3(Cfg::kThreads), lds, a, b, slot_mem, m, k, n, plan.per);
        else
            mhip::launch(ctx,
                         (mfma_gemm_stream_kernel<BM, BN, BK, WM, WN, A_T, B_T, false, BT, KG, STEP>),
                         grid, dim3(Cfg::kThreads), lds, a, b, slot_mem, m, k, n, plan.per);
        st = mhip::check_launch("matmul (MFMA stream-K)");
        if (st != MHIP_OK) return st;
        mhip::launch(ctx, (stream_reduce_kernel<BM, BN>), dim3(static_cast<unsigned>(groups_out)),
                     dim3(256), 0, slot_mem, c, m, n, plan.kslices, plan.per, addend, mode, vec4);
        return mhip::check_launch("matmul (stream-K reduction)");
    }

    float* target = c;
    if (plan.splits > 1) {
        mhip_status st = workspace(ctx, plan.splits * m * n * sizeof(float), &target);
        if (st != MHIP_OK) return st;
    }
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(plan.splits));
    if (vec)
        mhip::launch(ctx, (mfma_gemm_kernel<BM, BN, BK, WM, WN, A_T, B_T, true, BT, KG, STEP>), grid,
                     dim3(Cfg::kThreads), lds, a, b, target, m, k, n, addend, mode, plan.k_split);
    else
        mhip::launch(ctx, (mfma_gemm_kernel<BM, BN, BK, WM, WN, A_T, B_T, false, BT, KG, STEP>),
                     grid, dim3(Cfg::kThreads), lds, a, b, target, m, k, n, addend, mode,
                     plan.k_split);
    mhip_status st = mhip::check_launch("matmul (MFMA tiles)");
    if (st != MHIP_OK || plan.splits == 1) return st;
    mhip::launch(ctx, splitk_reduce_kernel, dim3(static_cast<unsigned>(groups_out)), dim3(256), 0,
                 target, c, m, n, static_cast<uint32_t>(plan.splits), addend, mode, vec4);
    return mhip::check_launch("matmul (split-k reduction)");
}

// ---------------------------------------------------------------------------
// Decode GEMV: m <= kGemvMaxRows, B row-major [k][n] with n % 4 == 0.
// ---------------------------------------------------------------------------

constexpr int kGemvThreads = 256;
constexpr int kGemvCols = 256;  // columns per workgroup: 64 lanes x 4

// How a GEMV lane reads CPL consecutive columns of one row of B: f32 as one
// dwordx4, compact bf16 as 8 bytes (CPL 4) or one dwordx4 of 8 values (CPL
// 8), kept raw in registers until widened (exactly) at use.
template <class BT, int CPL>
struct GemvLoad;
template <>
struct GemvLoad<float, 4> {
    using Raw = float4;
    template <bool NT>
    static __device__ __forceinline__ Raw load(const float* p) {
        if constexpr (NT) return load4_nt(p);
        else return load4(p);
    }
    static __device__ __forceinline__ float4 part(const Raw& v, int) { return v; }
};
template <>
struct GemvLoad<uint16_t, 4> {
    using Raw = uint2;
    template <bool NT>
    static __device__ __forceinline__ Raw load(const uint16_t* p) {
        if constexpr (NT) {
            const mhip::u32x2 t = __builtin_nontemporal_load(reinterpret_cast<const mhip::u32x2*>(p));
            return make_uint2(t.x, t.y);
        } else {
            return *reinterpret_cast<const uint2*>(p);
        }
    }
    static __device__ __forceinline__ float4 part(const Raw& v, int) { return mhip::widen(v); }
};
template <>
struct GemvLoad<uint16_t, 8> {
    using Raw = uint4;
    template <bool NT>
    static __device__ __forceinline__ Raw load(const uint16_t* p) {
        if constexpr (NT) return mhip::load_nt(reinterpret_cast<const uint4*>(p));
        else return *reinterpret_cast<const uint4*>(p);
    }
    static __device__ __forceinline__ float4 part(const Raw& v, int h) {
        return mhip::widen(h ? make_uint2(v.z, v.w) : make_uint2(v.x, v.y));
    }
};

// One workgroup's share of a decode GEMV: column group `cg` (64 * CPL
// columns, CPL per lane) and k slice `slice`. Its 4 waves split the slice's
// rows and meet in LDS. Each column's sum runs over the same k in the same
// order whatever CPL is, so CPL changes loads, not results.
// `direct`: write C (+ addend) itself (the only slice); otherwise write the
// slice's partial sums for the reduction. STREAM: read B non-temporally (a
// matrix larger than an XCD's L2, read once per call); a small B is read
// through the caches, where it stays between calls. (A template parameter:
// a run-time choice inside the load loop doubled the registers.)
// The GEMV's input as stored: row r of A [rows, K].
struct StoredRows {
    const float* __restrict__ a;
    uint64_t k;
    __device__ __forceinline__ float operator()(int r, uint64_t kk) const { return a[r * k + kk]; }
};

// `A(r, k)` gives the input's row r at k (StoredRows, or a row normalised in
// the launch). `prologue()` runs on every thread after the first batch of B
// rows is in flight (a normalised input's scale; its latency hides under
// theirs), before any A is read.
struct NoPrologue {
    __device__ __forceinline__ void operator()() const {}
};
template <int ROWS, class BT, bool STREAM, int CPL, class AF, class PRO = NoPrologue>
__device__ __forceinline__ void gemv_partial_body(
    const AF& A, const PRO& prologue, const BT* __restrict__ B, float* __restrict__ partial,
    float* __restrict__ C, uint64_t K, uint64_t N, uint64_t k_per_slice, uint32_t cg,
    uint32_t slice, bool direct, const float* __restrict__ addend, int addend_mode) {
    constexpr int H = CPL / 4;  // float4 groups per lane
    using L = GemvLoad<BT, CPL>;
    __shared__ float4 red[4][ROWS][H][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t col = static_cast<uint64_t>(cg) * (64 * CPL) + lane * CPL;
    const bool live = col < N;  // N % CPL == 0: a live lane's columns are all in range
    const uint64_t k_begin = static_cast<uint64_t>(slice) * k_per_slice;
    const uint64_t k_end = min(K, k_begin + k_per_slice);
    float4 acc[ROWS][H];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int h = 0; h < H; ++h) acc[r][h] = make_float4(0.f, 0.f, 0.f, 0.f);
    auto fma_row = [&](const typename L::Raw& raw, uint64_t k) {
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const float4 b = L::part(raw, h);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const float a = A(r, k);
                acc[r][h].x = __builtin_fmaf(a, b.x, acc[r][h].x);
                acc[r][h].y = __builtin_fmaf(a, b.y, acc[r][h].y);
                acc[r][h].z = __builtin_fmaf(a, b.z, acc[r][h].z);
                acc[r][h].w = __builtin_fmaf(a, b.w, acc[r][h].w);
            }
        }
    };
    // B rows in flight per lane: 256 bytes for compact weights read 8
    // columns at a time and for blocks of 8 rows (measured: bf16
    // 1x4096x11008 22.1 -> 18.3 us, the C1 block 80 -> 61 us), 128 bytes
    // otherwise (256 was no faster for the f32 decode GEMVs).
    constexpr int kU = (CPL == 8 || ROWS >= 8 ? 256 : 128) / sizeof(typename L::Raw);
    uint64_t kk = k_begin + wave;
    typename L::Raw first[kU];
    const bool first_batch = live && kk + 4 * (kU - 1) < k_end;
    if (first_batch) {
#pragma unroll
        for (int u = 0; u < kU; ++u) first[u] = L::template load<STREAM>(B + (kk + 4 * u) * N + col);
    }
    prologue();
    if (live) {
        if (first_batch) {
#pragma unroll
            for (int u = 0; u < kU; ++u) fma_row(first[u], kk + 4 * u);
            kk += 4 * kU;
        }
        for (; kk + 4 * (kU - 1) < k_end; kk += 4 * kU) {
            typename L::Raw bv[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) bv[u] = L::template load<STREAM>(B + (kk + 4 * u) * N + col);
#pragma unroll
            for (int u = 0; u < kU; ++u) fma_row(bv[u], kk + 4 * u);
        }
        for (; kk < k_end; kk += 4) fma_row(L::template load<STREAM>(B + kk * N + col), kk);
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int h = 0; h < H; ++h) red[wave][r][h][lane] = acc[r][h];
    __syncthreads();
    if (wave != 0 || !live) return;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const uint64_t c = col + 4 * h;
            float4 v = red[0][r][h][lane];
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                const float4 o = red[w][r][h][lane];
                v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
            }
            if (direct) {
                if (addend_mode == 1) {
                    const float4 b4 = *reinterpret_cast<const float4*>(addend + c);
                    v.x = v.x + b4.x; v.y = v.y + b4.y; v.z = v.z + b4.z; v.w = v.w + b4.w;
                } else if (addend_mode >= 2) {
                    v = apply_addend(v, *reinterpret_cast<const float4*>(addend + r * N + c), addend_mode);
                }
                *reinterpret_cast<float4*>(C + r * N + c) = v;
            } else {
                *reinterpret_cast<float4*>(partial + (static_cast<uint64_t>(slice) * ROWS + r) * N + c) = v;
            }
        }
    }
}

// blockIdx.z is a block of ROWS rows of A and C: each is an independent
// ROWS-row GEMV with its own partial sums (B is shared through L2).
template <int ROWS, class BT, bool STREAM, int CPL>
__global__ __launch_bounds__(kGemvThreads) void gemv_partial_kernel(
    const float* __restrict__ A, const BT* __restrict__ B, float* __restrict__ partial,
    float* __restrict__ C, uint64_t K, uint64_t N, uint64_t k_per_slice, uint32_t slices,
    const float* __restrict__ addend, int addend_mode) {
    const uint64_t rb = blockIdx.z;
    A += rb * ROWS * K;
    C += rb * ROWS * N;
    if (partial) partial += rb * slices * ROWS * N;
    if (addend_mode >= 2) addend += rb * ROWS * N;
    gemv_partial_body<ROWS, BT, STREAM, CPL>(StoredRows{A, K}, NoPrologue{}, B, partial, C, K, N, k_per_slice,
                                             blockIdx.x, blockIdx.y, slices == 1, addend, addend_mode);
}

// A one-row decode GEMV whose input row is attention's output, merged here
// from its key-chunk records (mhip::merge_decode_chunks, the merge kernel's
// order) instead of by a merge launch: each workgroup merges its k slice,
// which lies within one head of D = 4 * D4 columns, into LDS once its first
// weight rows are in flight.
template <class BT, bool STREAM, int CPL, int D4>
__global__ __launch_bounds__(kGemvThreads) void gemv_partial_merge_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml, uint64_t chunks,
    const BT* __restrict__ B, float* __restrict__ partial, uint64_t K, uint64_t N,
    uint64_t k_per_slice, uint32_t slices) {
    static_assert(kGemvThreads == 256, "the merge takes 256 threads");
    constexpr int D = 4 * D4;
    __shared__ float sa[D];
    const uint32_t slice = blockIdx.y;
    const uint64_t k0 = static_cast<uint64_t>(slice) * k_per_slice;
    const uint64_t head = k0 / D;
    const int q0 = static_cast<int>(k0 % D) / 4;
    const int nq = static_cast<int>(min(K, k0 + k_per_slice) - k0) / 4;
    auto merge = [&]() {
        const float4 v = mhip::merge_decode_chunks<D4>(part_ml + 2 * head * chunks,
                                                       part_o + head * chunks * D, chunks, q0, nq);
        if (static_cast<int>(threadIdx.x) >= q0 && static_cast<int>(threadIdx.x) < q0 + nq)
            *reinterpret_cast<float4*>(sa + 4 * (threadIdx.x - q0)) = v;
        __syncthreads();
    };
    auto merged = [&](int, uint64_t k) { return sa[k - k0]; };
    gemv_partial_body<1, BT, STREAM, CPL>(merged, merge, B, partial, nullptr, K, N, k_per_slice,
                                          blockIdx.x, slice, slices == 1, nullptr, 0);
}

// Sums of the slices' partial sums of 256 columns, for NSEG matrices of the
// same shape at once: wave w adds a fixed quarter of the slices, each row in
// slice order, then wave 0 adds the quarters in order -- the same order on
// every run. Loads go out in batches of 16 float4 (every segment's rows of
// 16 / (ROWS * NSEG) slices) before any is added, so a quarter costs
// ceil(slices / 4 / batch) memory round trips for all segments together,
// not one per slice, row or segment. The results are valid in wave 0 only;
// every thread of the workgroup must call it (it synchronises), and a second
// call must come after a __syncthreads().
template <int ROWS, int NSEG = 1>
__device__ __forceinline__ void gemv_reduce_sum(const float* const (&partial)[NSEG], uint64_t N,
                                                uint32_t slices, uint64_t col, bool live,
                                                float4 (&out)[NSEG][ROWS]) {
    __shared__ float4 red[4][ROWS][64];
    constexpr int kBatch = ROWS * NSEG >= 16 ? 1 : 16 / (ROWS * NSEG);  // slices per batch
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t quarter = (slices + 3) / 4;
    const uint32_t s_begin = min(slices, wave * quarter), s_end = min(slices, s_begin + quarter);
    float4 v[NSEG][ROWS];
#pragma unroll
    for (int q = 0; q < NSEG; ++q)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) v[q][r] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
        for (uint32_t s = s_begin; s < s_end; s += kBatch) {
            float4 p[NSEG][kBatch][ROWS];
#pragma unroll
            for (int q = 0; q < NSEG; ++q)
#pragma unroll
                for (int u = 0; u < kBatch; ++u)
#pragma unroll
                    for (int r = 0; r < ROWS; ++r)
                        if (s + u < s_end)
                            p[q][u][r] = *reinterpret_cast<const float4*>(
                                partial[q] + ((s + u) * static_cast<uint64_t>(ROWS) + r) * N + col);
#pragma unroll
            for (int q = 0; q < NSEG; ++q)
#pragma unroll
                for (int u = 0; u < kBatch; ++u)
#pragma unroll
                    for (int r = 0; r < ROWS; ++r)
                        if (s + u < s_end) {
                            v[q][r].x += p[q][u][r].x; v[q][r].y += p[q][u][r].y;
                            v[q][r].z += p[q][u][r].z; v[q][r].w += p[q][u][r].w;
                        }
        }
    }
#pragma unroll
    for (int q = 0; q < NSEG; ++q) {
        if (q > 0) __syncthreads();  // wave 0 has read the previous segment's quarters
#pragma unroll
        for (int r = 0; r < ROWS; ++r) red[wave][r][lane] = v[q][r];
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                float4 t = red[0][r][lane];
#pragma unroll
                for (int w = 1; w < 4; ++w) {
                    const float4 o = red[w][r][lane];
                    t.x += o.x; t.y += o.y; t.z += o.z; t.w += o.w;
                }
                out[q][r] = t;
            }
        }
    }
}

// C = the slices' partial sums (+ addend).
// chunk_ss (one row): also the RMSNorm chunk sum of squares of the 256
// columns written (mhip::chunk_sumsq), at chunk_ss[column group].
template <int ROWS>
__global__ __launch_bounds__(kGemvThreads) void gemv_reduce_kernel(
    const float* __restrict__ partial, float* __restrict__ C, uint64_t N, uint32_t slices,
    const float* __restrict__ addend, int addend_mode, float* __restrict__ chunk_ss) {
    const uint64_t rb = blockIdx.z;  // row block, as in gemv_partial_kernel
    partial += rb * slices * ROWS * N;
    C += rb * ROWS * N;
    if (addend_mode >= 2) addend += rb * ROWS * N;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t col = static_cast<uint64_t>(blockIdx.x) * kGemvCols + lane * 4;
    const bool live = col < N;
    // The addend goes out with the partial sums (one memory round trip).
    float4 add[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        add[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (wave == 0 && live && addend_mode != 0)
            add[r] = *reinterpret_cast<const float4*>(addend + (addend_mode >= 2 ? r * N : 0) + col);
    }
    float4 v[1][ROWS];
    gemv_reduce_sum<ROWS>({partial}, N, slices, col, live, v);
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        float4& o = v[0][r];
        if (!live) {
            o = make_float4(0.f, 0.f, 0.f, 0.f);
            continue;
        }
        if (addend_mode == 3) {
            o = apply_addend(o, add[r], 3);
        } else if (addend_mode != 0) {
            o.x = o.x + add[r].x; o.y = o.y + add[r].y; o.z = o.z + add[r].z; o.w = o.w + add[r].w;
        }
        *reinterpret_cast<float4*>(C + r * N + col) = o;
    }
    if constexpr (ROWS == 1) {
        if (chunk_ss) {
            const float cs = mhip::chunk_sumsq(v[0][0]);  // dead lanes hold zeros
            if (lane == 0) chunk_ss[blockIdx.x] = cs;
        }
    }
}

// ---------------------------------------------------------------------------
// Sets of decode GEMVs over one input, with fused epilogues
// ---------------------------------------------------------------------------

struct GemvSeg {
    const void* b;  // f32, or bf16 bits (the set's element type)
    float* partial;
    float* out;
    const uint64_t* out_advance;  // captured step: rows of `out` move by the replay offset
    uint64_t n;
    uint64_t k_per_slice;
    uint32_t col_groups, slices;
    uint32_t first_block;  // this segment's first workgroup in the partial launch
    uint32_t first_group;  // ... and in the reduction launch
};

struct GemvSet {
    GemvSeg seg[3];
    int count;
};

// Rotation of one projection's rows: interleaved pairs, head_width and
// dimension multiples of 4 (the vector RoPE kernel's case).
struct RopeEpi {
    const float* table;  // [half] frequencies then [half] amplitudes
    uint64_t head_width, dimension, half, offset;
    float scale;
    const uint64_t* advance;  // captured step: replay offset added to `offset`
};

// Segment `i` of the set with constant indices, so the fields stay in the
// kernel argument segment.
__device__ __forceinline__ GemvSeg pick(const GemvSet& set, int i) {
    if (i == 0) return set.seg[0];
    if (i == 1) return set.seg[1];
    return set.seg[2];
}

// A set's single input row normalised by RMSNorm inside the partial launch
// (the decode block's FFN RMSNorm): a[k] = src[k] * inv * gain[k], with inv
// from the row's chunk sums of squares (mhip::chunk_sumsq, written by the
// launch that produced the row) added in order -- the RMSNorm kernel's bits,
// for a prologue of `chunks` scalar reads instead of the whole row.
struct NormIn {
    const float* src;
    const float* chunk_ss;
    const float* gain;
    float eps;
    uint32_t chunks;
};

// Longest k slice a normalised input can have (its LDS staging).
constexpr uint64_t kNormSliceMax = 4096;

// NORM: 0, rows of A as stored; 1, the single row norm.src normalised.
template <int ROWS, class BT, bool STREAM, int CPL, int NORM>
__global__ __launch_bounds__(kGemvThreads) void gemv_set_partial_kernel(const float* __restrict__ A,
                                                                        uint64_t K, GemvSet set,
                                                                        NormIn norm) {
    const uint32_t b = blockIdx.x;
    const int i = (set.count > 2 && b >= set.seg[2].first_block) ? 2
                  : (set.count > 1 && b >= set.seg[1].first_block) ? 1 : 0;
    const GemvSeg s = pick(set, i);
    const uint32_t local = b - s.first_block;
    const uint64_t rb = blockIdx.y;  // row block of ROWS rows
    const BT* B = static_cast<const BT*>(s.b);
    float* partial = s.partial + rb * s.slices * ROWS * s.n;
    const uint32_t cg = local % s.col_groups, slice = local / s.col_groups;
    if constexpr (NORM == 0) {
        gemv_partial_body<ROWS, BT, STREAM, CPL>(StoredRows{A + rb * ROWS * K, K}, NoPrologue{}, B,
                                                 partial, nullptr, K, s.n, s.k_per_slice, cg, slice,
                                                 false, nullptr, 0);
    } else {
        static_assert(ROWS == 1, "a normalised input is one row");
        // The workgroup's k slice of the normalised row, staged in LDS once.
        __shared__ float sa[kNormSliceMax];
        const uint64_t k0 = static_cast<uint64_t>(slice) * s.k_per_slice;
        const uint64_t len = min(K, k0 + s.k_per_slice) - k0;
        auto scale = [&]() {
            float ss = 0.0f;
            for (uint32_t c = 0; c < norm.chunks; ++c) ss = ss + norm.chunk_ss[c];
            const float inv = mhip::inv_rms(ss, K, norm.eps);
            for (uint64_t j = threadIdx.x; j < len; j += kGemvThreads) {
                const float y = norm.src[k0 + j] * inv;
                sa[j] = norm.gain ? y * norm.gain[k0 + j] : y;
            }
            __syncthreads();
        };
        auto normed = [&](int, uint64_t k) { return sa[k - k0]; };
        gemv_partial_body<1, BT, STREAM, CPL>(normed, scale, B, partial, nullptr, K, s.n,
                                              s.k_per_slice, cg, slice, false, nullptr, 0);
    }
}

// The RoPE factors of one lane's 4 columns (two pairs): read before the
// reduction's partial sums are awaited, so they cost no round trip of their own.
struct RopeCoef {
    float f0, a0, f1, a1;  // frequency and amplitude of the two pairs
    uint64_t offset;
    bool on;               // the columns lie in the rotated dimensions
};

__device__ __forceinline__ RopeCoef rope_coef(const RopeEpi& e, uint64_t col) {
    RopeCoef c{};
    const uint64_t j = col % e.head_width;
    c.on = j < e.dimension;
    if (c.on) {
        const uint64_t p = j / 2;
        c.f0 = e.table[p];
        c.a0 = e.table[e.half + p];
        c.f1 = e.table[p + 1];
        c.a1 = e.table[e.half + p + 1];
    }
    c.offset = e.offset + (e.advance ? *e.advance : 0);
    return c;
}

__device__ __forceinline__ float4 rope_vec(const RopeCoef& c, float scale, uint64_t row, float4 v) {
    if (!c.on) return v;
    const float position = mhip::rope_position(c.offset, row, scale);
    float c0, s0, c1, s1;
    mhip::rope_freq_cs(position, c.f0, c.a0, &c0, &s0);
    mhip::rope_freq_cs(position, c.f1, c.a1, &c1, &s1);
    float4 r;
    mhip::rope_rotate(v.x, v.y, c0, s0, &r.x, &r.y);
    mhip::rope_rotate(v.z, v.w, c1, s1, &r.z, &r.w);
    return r;
}

template <int ROWS>
__global__ __launch_bounds__(kGemvThreads) void gemv_set_reduce_kernel(GemvSet set, int epilogue,
                                                                       RopeEpi rope_q,
                                                                       RopeEpi rope_k) {
    const uint32_t b = blockIdx.x;
    const int i = (set.count > 2 && b >= set.seg[2].first_group) ? 2
                  : (set.count > 1 && b >= set.seg[1].first_group) ? 1 : 0;
    const GemvSeg s = pick(set, i);
    const uint64_t rb = blockIdx.y;  // row block, as in gemv_set_partial_kernel
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t col = static_cast<uint64_t>(b - s.first_group) * kGemvCols + lane * 4;
    const bool live = col < s.n;
    float* out = s.out + rb * ROWS * s.n;
    if (epilogue == mhip::kGemvSiluMul) {
        // Gate (segment 0) and up (segment 1, the same columns) summed together.
        const GemvSeg u = pick(set, 1);
        const uint64_t advance = (wave == 0 && s.out_advance) ? *s.out_advance : 0;
        float4 v[2][ROWS];
        gemv_reduce_sum<ROWS, 2>({s.partial + rb * s.slices * ROWS * s.n,
                                  u.partial + rb * u.slices * ROWS * u.n},
                                 s.n, s.slices, col, live, v);
        if (wave != 0 || !live) return;
        out += advance * s.n;
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            float4 o;
            o.x = mhip::silu1(v[0][r].x) * v[1][r].x;
            o.y = mhip::silu1(v[0][r].y) * v[1][r].y;
            o.z = mhip::silu1(v[0][r].z) * v[1][r].z;
            o.w = mhip::silu1(v[0][r].w) * v[1][r].w;
            *reinterpret_cast<float4*>(out + r * s.n + col) = o;
        }
        return;
    }
    const bool rotate = epilogue == mhip::kGemvRopeQK && i < 2;
    RopeCoef coef{};
    uint64_t advance = 0;
    if (wave == 0 && live) {
        if (rotate) coef = rope_coef(i == 0 ? rope_q : rope_k, col);
        if (s.out_advance) advance = *s.out_advance;
    }
    float4 v[1][ROWS];
    gemv_reduce_sum<ROWS>({s.partial + rb * s.slices * ROWS * s.n}, s.n, s.slices, col, live, v);
    if (wave != 0 || !live) return;
    out += advance * s.n;
    const float scale = i == 0 ? rope_q.scale : rope_k.scale;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        float4 o = v[0][r];
        if (rotate) o = rope_vec(coef, scale, rb * ROWS + r, o);
        *reinterpret_cast<float4*>(out + r * s.n + col) = o;
    }
}

// Whether a GEMV reads its matrix non-temporally: one larger than an XCD's
// 4 MB L2 is streamed; a smaller one is kept in the caches across calls
// (the small blocks' weights), which saves a trip to HBM per launch.
bool gemv_streams_b(uint64_t bytes) { return bytes > (4ull << 20); }

// Split-k shape of a decode GEMV: about four workgroups per CU, each slice a
// multiple of 32 rows (four waves x eight rows in flight); one slice when
// the column groups alone fill the device.
void gemv_slicing(const mhip_ctx* ctx, uint64_t k, uint64_t n, uint64_t* slices_out,
                  uint64_t* k_per_slice_out) {
    const uint64_t col_groups = (n + kGemvCols - 1) / kGemvCols;
    const uint64_t target_blocks = static_cast<uint64_t>(ctx->compute_units ? ctx->compute_units : 256) * 4;
    uint64_t slices = (target_blocks + col_groups - 1) / col_groups;
    uint64_t k_per_slice = ((k + slices - 1) / slices + 31) / 32 * 32;
    if (k_per_slice < 32) k_per_slice = 32;
    slices = (k + k_per_slice - 1) / k_per_slice;
    if (slices <= 1) {
        slices = 1;
        k_per_slice = k;
    }
    *slices_out = slices;
    *k_per_slice_out = k_per_slice;
}

// Compact weights on up to 4 rows read 8 columns per lane (16-byte loads)
// when every row of B starts 16-byte aligned; otherwise 4.
template <int ROWS, class BT>
constexpr bool kGemvWideable = sizeof(BT) == 2 && ROWS <= 4;

template <int ROWS, class BT, int CPL>
void launch_gemv_partial(mhip_ctx* ctx, dim3 grid, bool stream, const float* a, const BT* b,
                         float* partial, float* c, uint64_t k, uint64_t n, uint64_t k_per_slice,
                         uint64_t slices, const float* addend, int mode) {
    if (stream)
        mhip::launch(ctx, (gemv_partial_kernel<ROWS, BT, true, CPL>), grid, dim3(kGemvThreads), 0, a,
                     b, partial, c, k, n, k_per_slice, static_cast<uint32_t>(slices), addend, mode);
    else
        mhip::launch(ctx, (gemv_partial_kernel<ROWS, BT, false, CPL>), grid, dim3(kGemvThreads), 0,
                     a, b, partial, c, k, n, k_per_slice, static_cast<uint32_t>(slices), addend,
                     mode);
}

// chunk_ss (one row, split k): the output's RMSNorm chunk sums too.
template <int ROWS, class BT>
mhip_status launch_gemv(mhip_ctx* ctx, const float* a, const BT* b, float* c, uint64_t k,
                        uint64_t n, const float* addend, int mode, uint64_t row_blocks = 1,
                        float* chunk_ss = nullptr) {
    const uint64_t col_groups = (n + kGemvCols - 1) / kGemvCols;  // of the reduction
    uint64_t slices, k_per_slice;
    gemv_slicing(ctx, k, n, &slices, &k_per_slice);
    float* partial = nullptr;
    if (slices > 1) {
        mhip_status st = workspace(ctx, row_blocks * slices * ROWS * n * sizeof(float), &partial);
        if (st != MHIP_OK) return st;
    }
    const bool stream = gemv_streams_b(k * n * sizeof(BT));
    bool wide = false;
    if constexpr (kGemvWideable<ROWS, BT>) wide = n % 8 == 0 && mhip::aligned16(b);
    const uint64_t part_groups = wide ? (n + 511) / 512 : col_groups;
    const dim3 grid(static_cast<unsigned>(part_groups), static_cast<unsigned>(slices),
                    static_cast<unsigned>(row_blocks));
    if constexpr (kGemvWideable<ROWS, BT>) {
        if (wide)
            launch_gemv_partial<ROWS, BT, 8>(ctx, grid, stream, a, b, partial, c, k, n, k_per_slice,
                                             slices, addend, mode);
        else
            launch_gemv_partial<ROWS, BT, 4>(ctx, grid, stream, a, b, partial, c, k, n, k_per_slice,
                                             slices, addend, mode);
    } else {
        launch_gemv_partial<ROWS, BT, 4>(ctx, grid, stream, a, b, partial, c, k, n, k_per_slice,
                                         slices, addend, mode);
    }
    mhip_status st = mhip::check_launch("matmul (decode partial sums)");
    if (st != MHIP_OK || slices == 1) return st;
    mhip::launch(ctx, gemv_reduce_kernel<ROWS>,
                 dim3(static_cast<unsigned>(col_groups), 1, static_cast<unsigned>(row_blocks)),
                 dim3(kGemvThreads), 0, partial, c, n, static_cast<uint32_t>(slices), addend, mode,
                 chunk_ss);
    return mhip::check_launch("matmul (decode reduction)");
}

template <int ROWS, class BT, int CPL, int NORM>
void launch_gemv_set_partial_n(mhip_ctx* ctx, dim3 grid, bool stream, const float* a, uint64_t k,
                               const GemvSet& set, const NormIn& norm) {
    if (stream)
        mhip::launch(ctx, (gemv_set_partial_kernel<ROWS, BT, true, CPL, NORM>), grid,
                     dim3(kGemvThreads), 0, a, k, set, norm);
    else
        mhip::launch(ctx, (gemv_set_partial_kernel<ROWS, BT, false, CPL, NORM>), grid,
                     dim3(kGemvThreads), 0, a, k, set, norm);
}

// `norm_mode` (NORM of gemv_set_partial_kernel) is nonzero only for one row.
template <int ROWS, class BT, int CPL>
void launch_gemv_set_partial(mhip_ctx* ctx, dim3 grid, bool stream, const float* a, uint64_t k,
                             const GemvSet& set, int norm_mode, const NormIn& norm) {
    if constexpr (ROWS == 1) {
        if (norm_mode == 1) return launch_gemv_set_partial_n<1, BT, CPL, 1>(ctx, grid, stream, a, k, set, norm);
    }
    launch_gemv_set_partial_n<ROWS, BT, CPL, 0>(ctx, grid, stream, a, k, set, norm);
}

// `wide`: the set's segments were planned with 8 columns per lane.
template <int ROWS, class BT>
mhip_status launch_gemv_set(mhip_ctx* ctx, const float* a, uint64_t k, GemvSet set, int epilogue,
                            const RopeEpi& rq, const RopeEpi& rk, uint32_t reduce_groups,
                            bool stream, bool wide, int norm_mode, const NormIn& norm,
                            uint32_t row_blocks = 1) {
    uint32_t blocks = 0;
    for (int i = 0; i < set.count; ++i) blocks += set.seg[i].col_groups * set.seg[i].slices;
    const dim3 grid(blocks, row_blocks);
    if constexpr (kGemvWideable<ROWS, BT>) {
        if (wide) launch_gemv_set_partial<ROWS, BT, 8>(ctx, grid, stream, a, k, set, norm_mode, norm);
        else launch_gemv_set_partial<ROWS, BT, 4>(ctx, grid, stream, a, k, set, norm_mode, norm);
    } else {
        if (wide) return MHIP_LAYOUT_UNSUPPORTED;
        launch_gemv_set_partial<ROWS, BT, 4>(ctx, grid, stream, a, k, set, norm_mode, norm);
    }
    mhip_status st = mhip::check_launch("decode projections (partial sums)");
    if (st != MHIP_OK) return st;
    mhip::launch(ctx, gemv_set_reduce_kernel<ROWS>, dim3(reduce_groups, row_blocks),
                 dim3(kGemvThreads), 0, set, epilogue, rq, rk);
    return mhip::check_launch("decode projections (reduction)");
}

template <class BT>
mhip_status dispatch_gemv(mhip_ctx* ctx, const float* a, const BT* b, float* c, uint64_t m,
                          uint64_t k, uint64_t n, const float* addend, int mode) {
    switch (m) {
        case 1: return launch_gemv<1, BT>(ctx, a, b, c, k, n, addend, mode);
        case 2: return launch_gemv<2, BT>(ctx, a, b, c, k, n, addend, mode);
        case 3: return launch_gemv<3, BT>(ctx, a, b, c, k, n, addend, mode);
        case 4: return launch_gemv<4, BT>(ctx, a, b, c, k, n, addend, mode);
        case 5: return launch_gemv<5, BT>(ctx, a, b, c, k, n, addend, mode);
        case 6: return launch_gemv<6, BT>(ctx, a, b, c, k, n, addend, mode);
        case 7: return launch_gemv<7, BT>(ctx, a, b, c, k, n, addend, mode);
        default: return launch_gemv<8, BT>(ctx, a, b, c, k, n, addend, mode);
    }
}

// Small products of 16-32 rows in one launch (no partial sums, no reduction
// launch): a workgroup of kSmallWaves waves owns a 32 x 32 tile of C. Wave w
// takes k range [w * kq, (w + 1) * kq) (kq a multiple of 8; the last ranges
// short or empty) and sums it with v_mfma_f32_32x32x2_f32 in the k order
// 8g + 4h + e of the MFMA tiles: lane half h feeds A[row][g + 4h + e] from one
// 16-byte load and B[g + 4h + e][col]. Loads go out two k groups at a time.
// The waves' partial tiles meet in LDS and wave r adds register row r over
// the waves in wave order. Each output's sum depends only on its own row and
// column, so any row subset of a product taking this path gives the same
// bits, and a set of products (the GEMV sets' epilogues) the bits of each.
constexpr int kSmallWaves = 16;
constexpr uint64_t kSmallMaxK = 1024;
static_assert(kSmallWaves == 16, "one register row of the 32 x 32 tile per wave");

// The tile's sums at (small_row(row0), col0 + lane % 32) for the calling
// wave, of A times each of the T matrices B[t] (same shape; T = 2 for a
// gate/up pair shares A's loads and issues both matrices' loads together).
// Every thread of the workgroup calls it (it synchronises).
template <class BT, int T>
__device__ __forceinline__ void small_tiles(const float* __restrict__ A,
                                            const BT* const (&B)[T], uint64_t M, uint64_t K,
                                            uint64_t N, uint64_t kq, uint64_t row0, uint64_t col0,
                                            float (*red)[16][64], float (&out)[T]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const uint64_t kb = wave * kq, ke = min(K, kb + kq);
    const uint64_t arow = row0 + l32, bcol = col0 + l32;
    const bool arow_ok = arow < M, bcol_ok = bcol < N;
    const float* ap = A + arow * K;
    v16f acc[T];
#pragma unroll
    for (int m = 0; m < T; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[m][r] = 0.0f;
    constexpr int kBatch = 2;  // k groups of 8 per batch of loads
    for (uint64_t g0 = kb; g0 < ke; g0 += 8 * kBatch) {
        float4 a4[kBatch];
        float bv[T][kBatch][4];
#pragma unroll
        for (int t = 0; t < kBatch; ++t) {
            const uint64_t kk = g0 + 8 * t + 4 * h;  // K % 4 == 0: all four or none
            a4[t] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (arow_ok && kk < ke) a4[t] = *reinterpret_cast<const float4*>(ap + kk);
#pragma unroll
            for (int m = 0; m < T; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    bv[m][t][e] = (bcol_ok && kk + e < ke) ? elem(B[m] + (kk + e) * N + bcol) : 0.0f;
        }
#pragma unroll
        for (int m = 0; m < T; ++m)
#pragma unroll
            for (int t = 0; t < kBatch; ++t) {
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[t].x, bv[m][t][0], acc[m], 0, 0, 0);
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[t].y, bv[m][t][1], acc[m], 0, 0, 0);
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[t].z, bv[m][t][2], acc[m], 0, 0, 0);
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[t].w, bv[m][t][3], acc[m], 0, 0, 0);
            }
    }
#pragma unroll
    for (int m = 0; m < T; ++m) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[m][r];
        __syncthreads();
        float v = red[0][wave][lane];
#pragma unroll
        for (int w = 1; w < kSmallWaves; ++w) v += red[w][wave][lane];
        out[m] = v;
        __syncthreads();  // `red` is written again
    }
}

template <class BT>
__device__ __forceinline__ float small_tile(const float* __restrict__ A, const BT* __restrict__ B,
                                            uint64_t M, uint64_t K, uint64_t N, uint64_t kq,
                                            uint64_t row0, uint64_t col0,
                                            float (*red)[16][64]) {
    const BT* const bs[1] = {B};
    float v[1];
    small_tiles<BT, 1>(A, bs, M, K, N, kq, row0, col0, red, v);
    return v[0];
}

// Register row r = wave of the tile holds row row0 + 8 (r / 4) + 4h + r % 4.
__device__ __forceinline__ uint64_t small_row(uint64_t row0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return row0 + 8 * (wave / 4) + 4 * (lane >> 5) + (wave % 4);
}

template <class BT>
__global__ __launch_bounds__(64 * kSmallWaves) void small_mfma_kernel(
    const float* __restrict__ A, const BT* __restrict__ B, float* __restrict__ C, uint64_t M,
    uint64_t K, uint64_t N, uint64_t kq, const float* __restrict__ addend, int addend_mode) {
    __shared__ float red[kSmallWaves][16][64];
    const uint64_t col0 = static_cast<uint64_t>(blockIdx.x) * 32;
    const uint64_t row0 = static_cast<uint64_t>(blockIdx.y) * 32;
    float v = small_tile<BT>(A, B, M, K, N, kq, row0, col0, red);
    const uint64_t row = small_row(row0), col = col0 + (threadIdx.x & 31);
    if (row >= M || col >= N) return;
    if (addend_mode == 1) v = v + addend[col];
    else if (addend_mode >= 2) v = apply_addend(v, addend[row * N + col], addend_mode);
    C[row * N + col] = v;
}

// A GEMV set (gemv_set_f32) of 16-32 rows on the small tiles: workgroup x
// takes a 32-column tile of one target (targets' tiles in order); with the
// silu-mul epilogue the workgroup sums the gate and up tiles of the same
// columns together and stores silu(gate) * up; with the RoPE epilogue targets 0
// and 1 rotate each interleaved pair (columns 2i, 2i + 1, in lanes l, l ^ 1)
// with the factors of the vector RoPE kernel. Each target's sums are those of
// small_mfma_kernel for it alone.
struct SmallSeg {
    const void* b;
    float* out;
    const uint64_t* out_advance;  // captured step: rows of `out` move by the replay offset
    uint64_t n;
    uint32_t first_tile;
};

struct SmallSet {
    SmallSeg seg[3];
    int count;
};

__device__ __forceinline__ SmallSeg pick(const SmallSet& set, int i) {
    if (i == 0) return set.seg[0];
    if (i == 1) return set.seg[1];
    return set.seg[2];
}

template <class BT>
__global__ __launch_bounds__(64 * kSmallWaves) void small_mfma_set_kernel(
    const float* __restrict__ A, uint64_t M, uint64_t K, uint64_t kq, SmallSet set, int epilogue,
    RopeEpi rope_q, RopeEpi rope_k) {
    __shared__ float red[kSmallWaves][16][64];
    const uint32_t b = blockIdx.x;
    const int i = (set.count > 2 && b >= set.seg[2].first_tile) ? 2
                  : (set.count > 1 && b >= set.seg[1].first_tile) ? 1 : 0;
    const SmallSeg s = pick(set, i);
    const int l32 = threadIdx.x & 31;
    const uint64_t col0 = static_cast<uint64_t>(b - s.first_tile) * 32;
    const uint64_t row0 = static_cast<uint64_t>(blockIdx.y) * 32;
    const uint64_t row = small_row(row0), col = col0 + l32;
    float v;
    if (epilogue == mhip::kGemvSiluMul) {
        // Gate (segment 0) and up (segment 1, the same columns) summed together.
        const BT* const bs[2] = {static_cast<const BT*>(s.b), static_cast<const BT*>(set.seg[1].b)};
        float gu[2];
        small_tiles<BT, 2>(A, bs, M, K, s.n, kq, row0, col0, red, gu);
        v = mhip::silu1(gu[0]) * gu[1];
    } else {
        v = small_tile<BT>(A, static_cast<const BT*>(s.b), M, K, s.n, kq, row0, col0, red);
    }
    if (epilogue == mhip::kGemvRopeQK && i < 2) {
        const float other = __shfl_xor(v, 1, 64);  // the pair's other column
        const RopeEpi& e = i == 0 ? rope_q : rope_k;
        const uint64_t j = col % e.head_width;
        if (j < e.dimension) {
            const uint64_t p = j / 2;
            const float position =
                mhip::rope_position(e.offset + (e.advance ? *e.advance : 0), row, e.scale);
            float c, sn;
            mhip::rope_freq_cs(position, e.table[p], e.table[e.half + p], &c, &sn);
            const bool even = (l32 & 1) == 0;
            float re, ro;
            mhip::rope_rotate(even ? v : other, even ? other : v, c, sn, &re, &ro);
            v = even ? re : ro;
        }
    }
    if (row >= M || col >= s.n) return;
    float* out = s.out + (s.out_advance ? *s.out_advance : 0) * s.n;
    out[row * s.n + col] = v;
}

// Whether a product of a few rows takes small_mfma_kernel: A's 16-byte loads
// need k % 4 == 0 and an aligned base; past kSmallMaxK the waves' 4-byte B
// loads make it slower than the row-blocked GEMV.
bool small_mfma_fits(uint64_t k, bool a_aligned) {
    return k % 4 == 0 && k <= kSmallMaxK && a_aligned;
}

template <class BT>
mhip_status launch_small_mfma(mhip_ctx* ctx, const float* a, const BT* b, float* c, uint64_t m,
                              uint64_t k, uint64_t n, const float* addend, int mode) {
    const uint64_t kq = (k + 8 * kSmallWaves - 1) / (8 * kSmallWaves) * 8;
    const dim3 grid(static_cast<unsigned>((n + 31) / 32), static_cast<unsigned>((m + 31) / 32));
    mhip::launch(ctx, small_mfma_kernel<BT>, grid, dim3(64 * kSmallWaves), 0, a, b, c, m, k, n, kq,
                 addend, mode);
    return mhip::check_launch("matmul (small MFMA tiles)");
}

template <class BT>
mhip_status launch_small_set(mhip_ctx* ctx, const float* a, uint64_t rows, uint64_t k,
                             const SmallSet& set, uint64_t tiles, int epilogue, const RopeEpi& rq,
                             const RopeEpi& rk) {
    const uint64_t kq = (k + 8 * kSmallWaves - 1) / (8 * kSmallWaves) * 8;
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>((rows + 31) / 32));
    mhip::launch(ctx, small_mfma_set_kernel<BT>, grid, dim3(64 * kSmallWaves), 0, a, rows, k, kq,
                 set, epilogue, rq, rk);
    return mhip::check_launch("GEMV set (small MFMA tiles)");
}

// Zero-inner-dimension product: C = 0 (+ addend).
__global__ void fill_addend_kernel(float* C, uint64_t M, uint64_t N, const float* addend,
                                   int mode) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= M * N) return;
    float v = 0.0f;
    if (mode == 1) v = v + addend[idx % N];
    else if (mode >= 2) v = apply_addend(v, addend[idx], mode);
    C[idx] = v;
}

// The shared body of the f32 and compact-weight matmuls: B as f32 or as bf16
// bit patterns; everything else (A, C, the addend, the arithmetic) is f32.
// The tile configurations, picked per shape by the time model (efficiencies
// measured with each configuration forced):
//  - kBig: 256 x 256 tiles, 8 waves of 64 x 128 (twice the MFMA work per byte
//    of LDS traffic): large products, 88 % of peak at 4096^3;
//  - kSmall: 128 x 128 tiles, 4 waves of 64 x 64, two workgroups per CU:
//    products whose tiles fill the CUs twice over (82 % at 4096^3);
//  - kMid: 128 x 128 tiles, 8 waves of 32 x 64: products with about one tile
//    (or k split) per CU, where the 4-wave kernel leaves each SIMD one wave
//    (83 % at 4096^3);
//  - kTiny: 64 x 64 tiles, 8 waves of 32 x 32 in two k groups, four-slice
//    steps: products of about one such tile per CU (1024^3: 256 tiles),
//    which then need no k split and no second launch (about 65 % of peak in
//    its steady state, measured per step with s_memtime at 1024^3).
enum class TileChoice { kBig, kSmall, kMid, kTiny };

using BigCfg = TileCfg<256, 256, 32, 64, 128, false, false>;
using SmallCfg = TileCfg<128, 128, 32, 64, 64, false, false>;
using MidCfg = TileCfg<128, 128, 32, 32, 64, false, false>;
using TinyCfg = TileCfg<64, 64, 32, 32, 32, false, false, 2>;

TileChoice choose_tiles(const mhip_ctx* ctx, uint64_t m, uint64_t k, uint64_t n) {
    const double t_big = gemm_seconds(ctx, m, k, n, 256, 256, 32, plan_per_cu<BigCfg>(), BigCfg::kWaves, 0.88);
    const double t_small =
        gemm_seconds(ctx, m, k, n, 128, 128, 32, plan_per_cu<SmallCfg>(), SmallCfg::kWaves, 0.82);
    const double t_mid = gemm_seconds(ctx, m, k, n, 128, 128, 32, plan_per_cu<MidCfg>(), MidCfg::kWaves, 0.83);
    const double t_tiny = gemm_seconds(ctx, m, k, n, 64, 64, 32, plan_per_cu<TinyCfg>(), TinyCfg::kWaves, 0.65);
    if (t_tiny < t_big && t_tiny < t_small && t_tiny < t_mid) return TileChoice::kTiny;
    if (t_big < t_small && t_big <= t_mid) return TileChoice::kBig;
    if (t_mid < t_small) return TileChoice::kMid;
    return TileChoice::kSmall;
}

// Which kernel path a product takes (the decode GEMV rules of matmul_impl,
// then the tile choice); `b_aligned`: B's base allows its vector loads.
mhip_matmul_plan plan_matmul(const mhip_ctx* ctx, uint64_t m, uint64_t k, uint64_t n, bool ta,
                             bool tb, bool b_aligned) {
    mhip_matmul_plan out{};
    if (m <= kGemvMaxRows && !ta && !tb && n % 4 == 0 && b_aligned) {
        uint64_t slices, per;
        gemv_slicing(ctx, k, n, &slices, &per);
        out.path = MHIP_MATMUL_PATH_GEMV;
        out.splits = static_cast<uint32_t>(slices);
        return out;
    }
    if (m <= 4 * kGemvMaxRows && m % kGemvMaxRows == 0 && m * k * n <= kGemvSmallProduct && !ta &&
        !tb && n % 4 == 0 && b_aligned) {
        if (small_mfma_fits(k, true)) {
            out.path = MHIP_MATMUL_PATH_SMALL_TILES;
            out.tile_m = out.tile_n = 32;
            out.waves = kSmallWaves;
            out.splits = 1;
            return out;
        }
        uint64_t slices, per;
        gemv_slicing(ctx, k, n, &slices, &per);
        out.path = MHIP_MATMUL_PATH_GEMV_ROW_BLOCKS;
        out.splits = static_cast<uint32_t>(slices);
        return out;
    }
    out.path = MHIP_MATMUL_PATH_TILES;
    uint64_t bm = 128, waves = SmallCfg::kWaves, per_cu = plan_per_cu<SmallCfg>();
    switch (choose_tiles(ctx, m, k, n)) {
        case TileChoice::kBig: bm = 256; waves = BigCfg::kWaves; per_cu = plan_per_cu<BigCfg>(); break;
        case TileChoice::kMid: waves = MidCfg::kWaves; per_cu = plan_per_cu<MidCfg>(); break;
        case TileChoice::kTiny: bm = 64; waves = TinyCfg::kWaves; per_cu = plan_per_cu<TinyCfg>(); break;
        case TileChoice::kSmall: break;
    }
    const GemmPlan p = plan_gemm(m, k, n, bm, bm, 32, per_cu * (ctx->compute_units ? ctx->compute_units : 256));
    out.tile_m = out.tile_n = static_cast<uint32_t>(bm);
    out.waves = static_cast<uint32_t>(waves);
    out.splits = p.stream ? 1u : static_cast<uint32_t>(p.splits);
    out.stream_k = p.stream ? 1u : 0u;
    return out;
}

template <class BT>
mhip_status matmul_impl(mhip_ctx* ctx, const float* a, const BT* b, float* out, uint64_t m,
                        uint64_t k, uint64_t n, int transpose_a, int transpose_b,
                        const float* addend, int addend_mode, bool gated = false) {
    MHIP_REQUIRE_CTX(ctx);
    if (gated ? addend_mode != 3 : (addend_mode < 0 || addend_mode > 2))
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul addend mode must be 0, 1 or 2");
    if (addend_mode != 0 && !addend)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul addend is null");
    if (m == 0 || n == 0) return MHIP_OK;
    if (!a || !b || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul: null buffer");
    if (k == 0) {
        mhip::launch(ctx, fill_addend_kernel, dim3(static_cast<unsigned>((m * n + 255) / 256)),
                     dim3(256), 0, out, m, n, addend, addend_mode);
        return mhip::check_launch("matmul (empty inner dimension)");
    }
    const bool ta = transpose_a != 0, tb = transpose_b != 0;
    // B's vector accesses (dwordx4 of f32, or 8 bytes of bf16) need rows of a
    // multiple of 4 elements and an aligned base.
    const uintptr_t b_align = sizeof(BT) == 4 ? 15u : 7u;
    const bool b_aligned = (reinterpret_cast<uintptr_t>(b) & b_align) == 0;
    if (m <= kGemvMaxRows && !ta && !tb && n % 4 == 0 && b_aligned)
        return dispatch_gemv<BT>(ctx, a, b, out, m, k, n, addend, addend_mode);
    // A few rows of a small product (up to 32 rows in blocks of 8, at most
    // 2^26 multiply-adds): one launch of small_mfma_kernel up to k = 1024,
    // else the GEMV's two short launches; both beat MFMA tiles that would be
    // three quarters padding and walk k serially.
    if (m <= 4 * kGemvMaxRows && m % kGemvMaxRows == 0 && m * k * n <= kGemvSmallProduct && !ta && !tb &&
        n % 4 == 0 && b_aligned) {
        if (small_mfma_fits(k, mhip::aligned16(a)))
            return launch_small_mfma<BT>(ctx, a, b, out, m, k, n, addend, addend_mode);
        return launch_gemv<kGemvMaxRows, BT>(ctx, a, b, out, k, n, addend, addend_mode, m / kGemvMaxRows);
    }
    const uint64_t lda = ta ? m : k, ldb = tb ? k : n;
    // Vector loads (and the direct loads into LDS, whose 32-bit offsets need
    // leading dimensions up to kDmaMaxLd).
    const bool vec = lda % 4 == 0 && ldb % 4 == 0 && mhip::aligned16(a) && b_aligned &&
                     lda <= kDmaMaxLd && ldb <= kDmaMaxLd;
    switch (choose_tiles(ctx, m, k, n)) {
        case TileChoice::kTiny:
            if (!ta && !tb)
                return launch_mfma<64, 64, 32, 32, 32, false, false, BT, 2>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            if (ta && !tb)
                return launch_mfma<64, 64, 32, 32, 32, true, false, BT, 2>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            if (!ta && tb)
                return launch_mfma<64, 64, 32, 32, 32, false, true, BT, 2>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            return launch_mfma<64, 64, 32, 32, 32, true, true, BT, 2>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
        case TileChoice::kBig:
            if (!ta && !tb)
                return launch_mfma<256, 256, 32, 64, 128, false, false, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            if (ta && !tb)
                return launch_mfma<256, 256, 32, 64, 128, true, false, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            if (!ta && tb)
                return launch_mfma<256, 256, 32, 64, 128, false, true, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            return launch_mfma<256, 256, 32, 64, 128, true, true, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
        case TileChoice::kMid:
            if (!ta && !tb)
                return launch_mfma<128, 128, 32, 32, 64, false, false, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            if (ta && !tb)
                return launch_mfma<128, 128, 32, 32, 64, true, false, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            if (!ta && tb)
                return launch_mfma<128, 128, 32, 32, 64, false, true, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
            return launch_mfma<128, 128, 32, 32, 64, true, true, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
        case TileChoice::kSmall:
            break;
    }
    if (!ta && !tb)
        return launch_mfma<128, 128, 32, 64, 64, false, false, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
    if (ta && !tb)
        return launch_mfma<128, 128, 32, 64, 64, true, false, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
    if (!ta && tb)
        return launch_mfma<128, 128, 32, 64, 64, false, true, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
    return launch_mfma<128, 128, 32, 64, 64, true, true, BT>(ctx, a, b, out, m, k, n, addend, addend_mode, vec);
}

}  // namespace

extern "C" mhip_status mhip_matmul_plan_f32(mhip_ctx* ctx, uint64_t m, uint64_t k, uint64_t n,
                                            int transpose_a, int transpose_b,
                                            mhip_matmul_plan* plan) {
    MHIP_REQUIRE_CTX(ctx);
    if (!plan) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "matmul plan: null output");
    *plan = plan_matmul(ctx, m, k, n, transpose_a != 0, transpose_b != 0, true);
    return MHIP_OK;
}

// The up product of a gated matmul (src/executor.rs:1484-1494): out =
// silu(gate) * (a . b), gate the [m, n] gate product, through the matmul's
// own kernels with the gate as an epilogue (addend mode 3), so it equals the
// product followed by silu-mul bit for bit, with no [m, n] temporary for the
// up product and no separate silu-mul launch.
mhip_status mhip::matmul_gated_f32(mhip_ctx* ctx, const float* a, const void* b, bool bf16,
                                   float* out, uint64_t m, uint64_t k, uint64_t n,
                                   bool transpose_a, bool transpose_b, const float* gate) {
    if (bf16)
        return matmul_impl<uint16_t>(ctx, a, static_cast<const uint16_t*>(b), out, m, k, n,
                                     transpose_a, transpose_b, gate, 3, true);
    return matmul_impl<float>(ctx, a, static_cast<const float*>(b), out, m, k, n, transpose_a,
                              transpose_b, gate, 3, true);
}

extern "C" mhip_status mhip_matmul_f32(mhip_ctx* ctx, const float* a, const float* b, float* out,
                                       uint64_t m, uint64_t k, uint64_t n, int transpose_a,
                                       int transpose_b, const float* addend, int addend_mode) {
    return matmul_impl<float>(ctx, a, b, out, m, k, n, transpose_a, transpose_b, addend, addend_mode);
}

// ---------------------------------------------------------------------------
// Allocation-free matmul: the partial sums in a fixed device array
// ---------------------------------------------------------------------------

// The scratch of mhip_matmul_f32_noalloc (split-k, stream-K and GEMV partial
// sums). Each GPU the library runs on holds its own copy until the process
// ends. On the host this name is a stand-in, not a device address: host code
// only ever uses the address hipGetSymbolAddress gives for a device.
static __device__ __align__(256) float scratch[MHIP_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kScratchDevices = 64;
std::mutex scratch_mutex;
float* scratch_address[kScratchDevices] = {};

}  // namespace

// The device address of `scratch` on the context's device: looked up once
// per device, with that device current, when the first context on it is
// created (or, if that failed, on the entry point's next call there).
mhip_status mhip::noalloc_scratch(mhip_ctx* ctx, float** out) {
    if (ctx->device < 0 || ctx->device >= kScratchDevices)
        return mhip::fail(MHIP_DEVICE_UNAVAILABLE, "allocation-free matmul: device ordinal out of range");
    std::lock_guard<std::mutex> lock(scratch_mutex);
    float*& address = scratch_address[ctx->device];
    if (!address) {
        // The caller's current device is put back afterwards.
        int previous = -1;
        hipError_t err = hipGetDevice(&previous);
        if (err == hipSuccess) err = hipSetDevice(ctx->device);
        void* p = nullptr;
        if (err == hipSuccess) err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (previous >= 0 && previous != ctx->device) (void)hipSetDevice(previous);
        if (err != hipSuccess) return mhip::from_hip(err, "locating the allocation-free matmul's scratch");
        address = static_cast<float*>(p);
    }
    if (out) *out = address;
    return MHIP_OK;
}

namespace {

// Points the context's matmul scratch at the fixed array for one call.
struct FixedScratch {
    mhip_ctx* ctx;
    FixedScratch(mhip_ctx* c, float* p) : ctx(c) {
        ctx->fixed_scratch = p;
        ctx->fixed_scratch_bytes = MHIP_NOALLOC_SCRATCH_BYTES;
    }
    ~FixedScratch() {
        ctx->fixed_scratch = nullptr;
        ctx->fixed_scratch_bytes = 0;
    }
};

}  // namespace

extern "C" mhip_status mhip_matmul_f32_noalloc(mhip_ctx* ctx, const float* a, const float* b,
                                               float* out, uint64_t m, uint64_t k, uint64_t n,
                                               int transpose_a, int transpose_b,
                                               const float* addend, int addend_mode) {
    MHIP_REQUIRE_CTX(ctx);
    float* p = nullptr;
    mhip_status st = mhip::noalloc_scratch(ctx, &p);
    if (st != MHIP_OK) return st;
    FixedScratch use(ctx, p);
    return matmul_impl<float>(ctx, a, b, out, m, k, n, transpose_a, transpose_b, addend, addend_mode);
}

extern "C" mhip_status mhip_matmul_bf16w_f32(mhip_ctx* ctx, const float* a, const uint16_t* b,
                                             float* out, uint64_t m, uint64_t k, uint64_t n,
                                             int transpose_a, int transpose_b, const float* addend,
                                             int addend_mode) {
    return matmul_impl<uint16_t>(ctx, a, b, out, m, k, n, transpose_a, transpose_b, addend,
                                 addend_mode);
}

namespace {

template <class BT>
mhip_status dispatch_gemv_set(mhip_ctx* ctx, const float* a, uint64_t rows, uint64_t k,
                              const GemvSet& set, int epilogue, const RopeEpi& rq,
                              const RopeEpi& rk, uint32_t g, bool stream, bool wide, int norm_mode,
                              const NormIn& norm) {
    switch (rows) {
        case 1: return launch_gemv_set<1, BT>(ctx, a, k, set, epilogue, rq, rk, g, stream, wide, norm_mode, norm);
        case 2: return launch_gemv_set<2, BT>(ctx, a, k, set, epilogue, rq, rk, g, stream, wide, 0, norm);
        case 3: return launch_gemv_set<3, BT>(ctx, a, k, set, epilogue, rq, rk, g, stream, wide, 0, norm);
        case 4: return launch_gemv_set<4, BT>(ctx, a, k, set, epilogue, rq, rk, g, stream, wide, 0, norm);
        case 5: return launch_gemv_set<5, BT>(ctx, a, k, set, epilogue, rq, rk, g, stream, wide, 0, norm);
        case 6: return launch_gemv_set<6, BT>(ctx, a, k, set, epilogue, rq, rk, g, stream, wide, 0, norm);
        case 7: return launch_gemv_set<7, BT>(ctx, a, k, set, epilogue, rq, rk, g, stream, wide, 0, norm);
        default:
            return launch_gemv_set<8, BT>(ctx, a, k, set, epilogue, rq, rk, g, stream, wide, 0, norm,
                                          static_cast<uint32_t>(rows / kGemvMaxRows));
    }
}

}  // namespace

namespace mhip {

mhip_status gemv_chunks_f32(mhip_ctx* ctx, const float* a, const void* b, float* out, uint64_t k,
                            uint64_t n, const float* addend, int addend_mode, bool bf16_weights,
                            float* chunk_ss) {
    MHIP_REQUIRE_CTX(ctx);
    // The one-row GEMV path of mhip_matmul_f32 with a split k (the chunk
    // sums come from its reduction launch).
    const uintptr_t b_align = bf16_weights ? 7u : 15u;
    if (!a || !b || !out || !chunk_ss || k == 0 || n % 4 != 0 || !aligned16(out) ||
        (reinterpret_cast<uintptr_t>(b) & b_align) != 0 || (addend_mode != 0 && !addend) ||
        addend_mode < 0 || addend_mode > 2)
        return MHIP_LAYOUT_UNSUPPORTED;
    uint64_t slices, k_per_slice;
    gemv_slicing(ctx, k, n, &slices, &k_per_slice);
    if (slices < 2) return MHIP_LAYOUT_UNSUPPORTED;
    return bf16_weights
               ? launch_gemv<1, uint16_t>(ctx, a, static_cast<const uint16_t*>(b), out, k, n, addend,
                                          addend_mode, 1, chunk_ss)
               : launch_gemv<1, float>(ctx, a, static_cast<const float*>(b), out, k, n, addend,
                                       addend_mode, 1, chunk_ss);
}

size_t gemv_merge_bytes(mhip_ctx* ctx, uint64_t heads, uint64_t d, uint64_t n, const void* b,
                        const float* out, bool bf16_weights) {
    const uintptr_t b_align = bf16_weights ? 7u : 15u;
    if (!ctx || !b || !out || !aligned16(out) || (reinterpret_cast<uintptr_t>(b) & b_align) != 0 ||
        heads == 0 || n == 0 || n % 4 != 0 || (d != 32 && d != 64 && d != 128 && d != 256))
        return 0;
    uint64_t slices, k_per_slice;
    gemv_slicing(ctx, heads * d, n, &slices, &k_per_slice);
    if (slices < 2 || k_per_slice > d || d % k_per_slice != 0) return 0;
    return (slices * n * sizeof(float) + 255) / 256 * 256;
}

namespace {

template <class BT, int CPL, int D4>
void launch_merge_partial(mhip_ctx* ctx, dim3 grid, bool stream, const DecodeChunks& r,
                          const BT* b, float* partial, uint64_t k, uint64_t n, uint64_t k_per_slice,
                          uint64_t slices) {
    if (stream)
        mhip::launch(ctx, (gemv_partial_merge_kernel<BT, true, CPL, D4>), grid, dim3(kGemvThreads),
                     0, r.part_o, r.part_ml, r.chunks, b, partial, k, n, k_per_slice,
                     static_cast<uint32_t>(slices));
    else
        mhip::launch(ctx, (gemv_partial_merge_kernel<BT, false, CPL, D4>), grid, dim3(kGemvThreads),
                     0, r.part_o, r.part_ml, r.chunks, b, partial, k, n, k_per_slice,
                     static_cast<uint32_t>(slices));
}

template <class BT, int CPL>
void launch_merge_partial_d(mhip_ctx* ctx, dim3 grid, bool stream, const DecodeChunks& r,
                            const BT* b, float* partial, uint64_t k, uint64_t n,
                            uint64_t k_per_slice, uint64_t slices) {
    switch (r.d) {
        case 32: return launch_merge_partial<BT, CPL, 8>(ctx, grid, stream, r, b, partial, k, n, k_per_slice, slices);
        case 64: return launch_merge_partial<BT, CPL, 16>(ctx, grid, stream, r, b, partial, k, n, k_per_slice, slices);
        case 128: return launch_merge_partial<BT, CPL, 32>(ctx, grid, stream, r, b, partial, k, n, k_per_slice, slices);
        default: return launch_merge_partial<BT, CPL, 64>(ctx, grid, stream, r, b, partial, k, n, k_per_slice, slices);
    }
}

// launch_gemv<1, BT>'s launches (same slicing, column groups, loads and
// reduction) with the merge kernel's partial launch.
template <class BT>
mhip_status launch_gemv_merge(mhip_ctx* ctx, const DecodeChunks& r, const BT* b, float* c,
                              uint64_t n, const float* addend, int mode, float* chunk_ss) {
    const uint64_t k = r.heads * r.d;
    const uint64_t col_groups = (n + kGemvCols - 1) / kGemvCols;
    uint64_t slices, k_per_slice;
    gemv_slicing(ctx, k, n, &slices, &k_per_slice);
    float* partial = r.extra;
    const bool stream = gemv_streams_b(k * n * sizeof(BT));
    bool wide = false;
    if constexpr (kGemvWideable<1, BT>) wide = n % 8 == 0 && mhip::aligned16(b);
    const uint64_t part_groups = wide ? (n + 511) / 512 : col_groups;
    const dim3 grid(static_cast<unsigned>(part_groups), static_cast<unsigned>(slices), 1);
    if constexpr (kGemvWideable<1, BT>) {
        if (wide)
            launch_merge_partial_d<BT, 8>(ctx, grid, stream, r, b, partial, k, n, k_per_slice, slices);
        else
            launch_merge_partial_d<BT, 4>(ctx, grid, stream, r, b, partial, k, n, k_per_slice, slices);
    } else {
        launch_merge_partial_d<BT, 4>(ctx, grid, stream, r, b, partial, k, n, k_per_slice, slices);
    }
    mhip_status st = mhip::check_launch("attention merge + output projection (partial sums)");
    if (st != MHIP_OK) return st;
    mhip::launch(ctx, gemv_reduce_kernel<1>, dim3(static_cast<unsigned>(col_groups), 1, 1),
                 dim3(kGemvThreads), 0, partial, c, n, static_cast<uint32_t>(slices), addend, mode,
                 chunk_ss);
    return mhip::check_launch("attention merge + output projection (reduction)");
}

}  // namespace

mhip_status gemv_merge_f32(mhip_ctx* ctx, const DecodeChunks& records, const void* b, float* out,
                           uint64_t n, const float* addend, int addend_mode, bool bf16_weights,
                           float* chunk_ss) {
    MHIP_REQUIRE_CTX(ctx);
    const size_t need = gemv_merge_bytes(ctx, records.heads, records.d, n, b, out, bf16_weights);
    if (need == 0 || records.extra_bytes < need || !records.extra || !records.part_o ||
        !records.part_ml || records.chunks == 0 || !chunk_ss || !aligned16(records.extra) ||
        (addend_mode != 0 && !addend) || addend_mode < 0 || addend_mode > 2)
        return MHIP_LAYOUT_UNSUPPORTED;
    return bf16_weights ? launch_gemv_merge<uint16_t>(ctx, records, static_cast<const uint16_t*>(b),
                                                      out, n, addend, addend_mode, chunk_ss)
                        : launch_gemv_merge<float>(ctx, records, static_cast<const float*>(b), out,
                                                   n, addend, addend_mode, chunk_ss);
}

mhip_status gemv_set_f32(mhip_ctx* ctx, const float* a, uint64_t rows, uint64_t k,
                         const GemvTarget* targets, int count, int epilogue,
                         const mhip_rope_params* rope, bool bf16_weights, const RowNorm* row_norm) {
    MHIP_REQUIRE_CTX(ctx);
    if (!targets || count < 1 || count > 3 || rows == 0 || k == 0) return MHIP_LAYOUT_UNSUPPORTED;
    if (!row_norm && !a) return MHIP_LAYOUT_UNSUPPORTED;
    NormIn norm{};
    int norm_mode = 0;
    if (row_norm) {
        // One row that the RMSNorm kernel would normalise with its vector
        // kernel (k % 4 == 0, at most 16384 floats, 16-byte aligned), so that
        // the chunk sums carry its order.
        const RowNorm& rn = *row_norm;
        int g = 0, vpt = 0;
        if (rows != 1 || k % 4 != 0 || !rn.src || !rn.chunk_ss || !(rn.eps > 0.0f) ||
            !aligned16(rn.src) || (rn.gain && !aligned16(rn.gain)) || !rms_layout(k / 4, &g, &vpt))
            return MHIP_LAYOUT_UNSUPPORTED;
        norm.src = rn.src;
        norm.chunk_ss = rn.chunk_ss;
        norm.gain = rn.gain;
        norm.eps = rn.eps;
        norm.chunks = static_cast<uint32_t>((k / 4 + 63) / 64);
        norm_mode = 1;
    }
    // Up to 8 rows, or up to 32 in blocks of 8 when every product is small
    // (as for the row-blocked matmul).
    if (rows > kGemvMaxRows) {
        if (rows > 4 * kGemvMaxRows || rows % kGemvMaxRows != 0) return MHIP_LAYOUT_UNSUPPORTED;
        for (int i = 0; i < count; ++i)
            if (rows * k * targets[i].n > kGemvSmallProduct) return MHIP_LAYOUT_UNSUPPORTED;
    }
    if (epilogue == kGemvSiluMul && (count != 2 || targets[0].n != targets[1].n))
        return MHIP_LAYOUT_UNSUPPORTED;
    if (epilogue == kGemvRopeQK && (count < 2 || !rope)) return MHIP_LAYOUT_UNSUPPORTED;
    GemvSet set{};
    set.count = count;
    bool stream = false;
    // Compact weights on up to 4 rows: 8 columns per lane when every matrix
    // allows 16-byte loads (as launch_gemv decides for one).
    bool wide = bf16_weights && rows <= 4;
    for (int i = 0; i < count; ++i)
        if (targets[i].n % 8 != 0 || !aligned16(targets[i].b)) wide = false;
    uint64_t floats = 0, blocks = 0, groups = 0;
    uint64_t offsets[3];
    for (int i = 0; i < count; ++i) {
        const GemvTarget& t = targets[i];
        const bool needs_out = !(epilogue == kGemvSiluMul && i == 1);
        const uintptr_t b_align = bf16_weights ? 7u : 15u;
        if (!t.b || t.n == 0 || t.n % 4 != 0 || (reinterpret_cast<uintptr_t>(t.b) & b_align) != 0 ||
            (needs_out && (!t.out || !aligned16(t.out))))
            return MHIP_LAYOUT_UNSUPPORTED;
        GemvSeg& g = set.seg[i];
        uint64_t slices, k_per_slice;
        gemv_slicing(ctx, k, t.n, &slices, &k_per_slice);
        g.b = t.b;
        g.out = t.out;
        g.out_advance = t.row_advances
                            ? advance_ptr(ctx, MHIP_ADVANCE_ROW_OFFSET, t.row_advance_limit)
                            : nullptr;
        g.n = t.n;
        g.k_per_slice = k_per_slice;
        g.col_groups = static_cast<uint32_t>((t.n + (wide ? 511 : 255)) / (wide ? 512 : 256));
        g.slices = static_cast<uint32_t>(slices);
        // The set streams its matrices when any of them is large.
        if (gemv_streams_b(k * t.n * (bf16_weights ? 2 : 4))) stream = true;
        g.first_block = static_cast<uint32_t>(blocks);
        g.first_group = static_cast<uint32_t>(groups);
        offsets[i] = floats;
        floats += (slices * rows * t.n + 63) / 64 * 64;
        blocks += g.col_groups * slices;
        // The reduction always takes 256 columns per workgroup.
        if (!(epilogue == kGemvSiluMul && i == 1)) groups += (t.n + kGemvCols - 1) / kGemvCols;
    }
    if (blocks >= (1ULL << 31)) return MHIP_LAYOUT_UNSUPPORTED;
    if (norm_mode)
        for (int i = 0; i < count; ++i)
            if (set.seg[i].k_per_slice > kNormSliceMax) return MHIP_LAYOUT_UNSUPPORTED;
    RopeEpi rq{}, rk{};
    if (epilogue == kGemvRopeQK) {
        for (int i = 0; i < 2; ++i) {
            const mhip_rope_params& p = rope[i];
            if (p.head_count == 0 || targets[i].n % p.head_count != 0) return MHIP_LAYOUT_UNSUPPORTED;
            const uint64_t hw = targets[i].n / p.head_count;
            if (p.half_split || p.dimension == 0 || p.dimension % 4 != 0 || p.dimension > hw ||
                hw % 4 != 0 || !(p.base > 0.0f) || !std::isfinite(p.base) || !(p.scale > 0.0f) ||
                !std::isfinite(p.scale) || (p.banded_factor > 0.0f && p.yarn_factor > 0.0f))
                return MHIP_LAYOUT_UNSUPPORTED;
            mhip_rope_params q = p;
            if (q.rotated_pairs > q.dimension / 2) q.rotated_pairs = q.dimension / 2;
            const float* table = nullptr;
            mhip_status st = rope_device_table(ctx, q, &table);
            if (st != MHIP_OK) return st;
            RopeEpi& e = i == 0 ? rq : rk;
            e.table = table;
            e.head_width = hw;
            e.dimension = q.dimension;
            e.half = q.dimension / 2;
            e.offset = q.position_offset;
            e.scale = q.scale;
            e.advance = advance_ptr(ctx, MHIP_ADVANCE_POSITION_OFFSET, UINT64_MAX);
        }
    }
    // 16-32 rows whose products take small_mfma_kernel as separate matmuls
    // take its set form (the same sums), in one launch.
    if (rows > kGemvMaxRows && norm_mode == 0 && small_mfma_fits(k, aligned16(a))) {
        SmallSet ss{};
        ss.count = count;
        uint64_t tiles = 0;
        for (int i = 0; i < count; ++i) {
            SmallSeg& g = ss.seg[i];
            g.b = targets[i].b;
            g.out = targets[i].out;
            g.out_advance = set.seg[i].out_advance;
            g.n = targets[i].n;
            if (epilogue == kGemvSiluMul && i == 1) {
                g.first_tile = UINT32_MAX;  // summed with the gate's tiles
                continue;
            }
            g.first_tile = static_cast<uint32_t>(tiles);
            tiles += (targets[i].n + 31) / 32;
        }
        return bf16_weights ? launch_small_set<uint16_t>(ctx, a, rows, k, ss, tiles, epilogue, rq, rk)
                            : launch_small_set<float>(ctx, a, rows, k, ss, tiles, epilogue, rq, rk);
    }
    void* scratch = nullptr;
    mhip_status st = workspace(ctx, floats * sizeof(float), &scratch);
    if (st != MHIP_OK) return st;
    float* partial = static_cast<float*>(scratch);
    for (int i = 0; i < count; ++i) set.seg[i].partial = partial + offsets[i];
    const uint32_t g = static_cast<uint32_t>(groups);
    return bf16_weights ? dispatch_gemv_set<uint16_t>(ctx, a, rows, k, set, epilogue, rq, rk, g, stream,
                                                      wide, norm_mode, norm)
                        : dispatch_gemv_set<float>(ctx, a, rows, k, set, epilogue, rq, rk, g, stream,
                                                   wide, norm_mode, norm);
}

}  // namespace mhip
