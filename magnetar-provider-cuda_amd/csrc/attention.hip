// Scaled dot-product attention with causal / sliding-window masks and grouped
// KV heads.
//
// Semantics are the reference's `attention_valued` (src/kernels.rs:6505-6884)
// defined by its three-pass kernel (src/kernels.cu:1868-1959): q [seq, H*d],
// k [kv_rows, Hkv*d], v [kv_rows, Hkv*vd]; kv_seq = key_count (<= kv_rows);
// query i sits at position qpos = (kv_seq - seq) + i and admits keys
// [lo, hi): hi = causal ? qpos + 1 : kv_seq, lo = qpos - (window - 1) when a
// window is set; weights are softmax(q.k * scale) over the admitted keys and
// the output row is their weighted mean of V rows (zeros if none). The
// reference has no batch dimension; here `batch` calls with fixed strides run
// in one launch and equal that many separate calls.
//
// Three kernels:
//  - prefill (head dims 64 and 128): fp32 MFMA flash attention. A workgroup
//    takes 128 queries of one (batch, head), four waves of 32, and walks the
//    admitted keys in 32-key tiles loaded straight into LDS (direct
//    global -> LDS loads, XOR-swizzled, double-buffered). Each wave computes S^T = K . Q^T with v_mfma_f32_32x32x2_f32
//    (Q^T lives in registers, pre-scaled by scale * log2 e), so every lane
//    owns one query column and 16 of the tile's keys: the online-softmax
//    max/sum need one exchange with lane l ^ 32. The accumulator registers
//    are then exactly the B operand of O^T = V^T . P^T, so the output stays
//    per-lane too. Probabilities are normalised per tile and the running
//    output rescaled, so it is always a convex combination of V rows and
//    never overflows (the reference's 1e38 known answer,
//    src/tests_conformance.rs:2215-2312).
//  - decode (one query row, head dim 4, 8, 16, ..., 256): split-KV. A
//    workgroup takes one (batch, KV head, key chunk) and the query heads
//    that share that KV head (up to 8; a larger group is split into slices
//    of 8, each reading the chunk), issues every K and V load of the chunk at once
//    (non-temporal dwordx4), keeps scores and probabilities in registers, and
//    writes the chunk's normalised output, max and weight sum; a second
//    kernel merges the chunks in a fixed order (deterministic).
//  - a generic kernel (any other shape): one wave per (query, head), online
//    softmax over 64-key chunks.
#include "common.hpp"
#include "decode_merge.hpp"
#include "internal.hpp"

#include <algorithm>
#include <cmath>

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
    const float* q;
    const float* k;
    const float* v;
    float* out;
    uint64_t seq, kv_seq, heads, kv_heads, d, vd;
    uint64_t offset;       // kv_seq - seq
    int causal;
    int64_t window;        // -1: none
    float qscale;          // scale * log2(e), applied to q
    uint64_t q_bs, k_bs, v_bs, o_bs;  // batch strides (floats)
    const uint64_t* advance;  // captured step: replay offset added to the key count
};

// A captured step's replay offset moves the key count, and with it the
// queries' positions (src/kernels.rs:1425-1435).
__device__ __forceinline__ void apply_advance(AttnArgs& a) {
    if (a.advance) {
        const uint64_t d = *a.advance;
        a.kv_seq += d;
        a.offset += d;
    }
}

// Admitted key range of the query at position qpos (src/kernels.cu:1909-1920).
__device__ __forceinline__ void key_range(const AttnArgs& a, uint64_t qpos, uint64_t* lo,
                                          uint64_t* hi) {
    uint64_t upper = a.causal ? qpos + 1 : a.kv_seq;
    if (upper > a.kv_seq) upper = a.kv_seq;
    uint64_t lower = 0;
    if (a.window >= 0) {
        const uint64_t w = static_cast<uint64_t>(a.window);
        const uint64_t back = w > 0 ? w - 1 : 0;
        lower = qpos > back ? qpos - back : 0;
        if (lower > upper) lower = upper;
    }
    *lo = lower;
    *hi = upper;
}

// ---------------------------------------------------------------------------
// Prefill: fp32 MFMA flash attention
// ---------------------------------------------------------------------------

template <int D, int VD>
struct PrefillCfg {
    static_assert(D >= 64 && VD >= 64, "rows of at least 16 chunks (the swizzle spans 16)");
    static constexpr int kBQ = 128;            // queries per workgroup (4 waves x 32)
    static constexpr int kBKV = 32;            // keys per tile
    static constexpr int kKTile = kBKV * D;    // floats; rows unpadded, 16-byte chunks swizzled
    static constexpr int kVTile = kBKV * VD;
    static constexpr int kLdsFloats = 2 * kKTile + 2 * kVTile;  // K and V, double-buffered apart
};

typedef __attribute__((address_space(3))) void lds_void_t;
// Word 3 of a raw (unformatted, unswizzled) buffer descriptor on gfx950.
constexpr int kRawBufferWord3 = 0x00020000;

// Rows [k0, k0 + 32) of a row-major [*, W] operand (leading dimension ld)
// into an LDS tile of 32 x W floats, by direct loads into LDS: one
// buffer_load_dwordx4 with the lds bit fills 1 KB of consecutive 16-byte
// slots, lane i slot i. Slot (row, c) holds the row's chunk c ^ (row & 15)
// (XOR swizzle instead of padding: 16-byte reads of one chunk position down
// 16 rows, which the LDS serves 16 lanes at a time over its 64 banks, and
// 4-byte reads across a row hit distinct banks). Rows at or past `rows`
// repeat row rows - 1 (finite data the caller masks out). Completion is
// tracked by vmcnt: wait for it before the tile's barrier.
//
// Each lane's byte offsets within a tile (row * ld + its chunk) are computed
// once; a tile's loads address the buffer that starts at g + k0 * ld with
// those 32-bit offsets. A tile spans 32 * ld * 4 bytes, below 2^32 (the
// launch checks ld). Buffer loads rather than global_load_lds: the compiler
// takes a pending global (FLAT) load into LDS for a possible LDS access and
// then waits for all of a wave's LDS reads at once (1129-1130 -> 1117-1124
// us at C4, the same bits).
template <int W>
struct TileDma {
    static constexpr int kChunksPerRow = W / 4;
    static constexpr int kInstrPerWave = 32 * W / 4 / 64 / 4;
    static_assert((kChunksPerRow & (kChunksPerRow - 1)) == 0 && kChunksPerRow >= 16,
                  "rows of a power-of-two number of chunks, at least 16");
    uint32_t off[kInstrPerWave];

    __device__ __forceinline__ TileDma(uint64_t ld, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < kInstrPerWave; ++j) {
            const int slot = (wave * kInstrPerWave + j) * 64 + lane;
            const int row = slot / kChunksPerRow;
            const int chunk = (slot % kChunksPerRow) ^ (row & 15);
            off[j] = static_cast<uint32_t>((row * ld + chunk * 4) * sizeof(float));
        }
    }

    __device__ __forceinline__ void load(const float* g, uint64_t ld, uint64_t k0, uint64_t rows,
                                         float* tile, int wave, int lane) const {
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(g + k0 * ld), 0,
            static_cast<int>(static_cast<uint32_t>(32 * ld * sizeof(float))), kRawBufferWord3);
        if (k0 + 32 <= rows) {
#pragma unroll
            for (int j = 0; j < kInstrPerWave; ++j) {
                const int slot0 = (wave * kInstrPerWave + j) * 64;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(tile + slot0 * 4), 16, off[j],
                                                         0, 0, 0);
            }
            return;
        }
        const uint32_t end = static_cast<uint32_t>(rows - 1 - k0);  // k0 < rows
        const uint32_t row_bytes = static_cast<uint32_t>(ld * sizeof(float));
#pragma unroll
        for (int j = 0; j < kInstrPerWave; ++j) {
            const int slot0 = (wave * kInstrPerWave + j) * 64;
            const uint32_t row = static_cast<uint32_t>(slot0 + lane) / kChunksPerRow;
            const uint32_t o = row > end ? off[j] - (row - end) * row_bytes : off[j];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(tile + slot0 * 4), 16, o, 0, 0, 0);
        }
    }
};

// S^T[key][query] of one tile: A = the K rows (lane -> key l32), B = Q^T.
template <int D>
__device__ __forceinline__ v16f tile_scores(const float* sk, const float (&qf)[D / 2], int l32,
                                            int half) {
    v16f s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
    const float* krow = sk + l32 * D;
    const int swz = l32 & 15;
#pragma unroll
    for (int t = 0; t < D / 2; t += 4) {
        const int chunk = (half * (D / 8) + t / 4) ^ swz;
        // A native vector read: read through HIP's float4 struct, the compiler
        // waited for the next tile's direct loads (vmcnt(0)) before the first
        // score read, though they fill the other buffer.
        const mhip::f32x4 kv = *reinterpret_cast<const mhip::f32x4*>(krow + chunk * 4);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[0], qf[t], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[1], qf[t + 1], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[2], qf[t + 2], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[3], qf[t + 3], s, 0, 0, 0);
    }
    return s;
}

// A wave's queries recomputed over their admitted keys only, on the VALU,
// after its tile loop: taken when an edge tile of the wave held a non-finite
// V value. In an edge tile a key one query of the wave masks can be one
// another admits; it enters the P . V MFMA at weight 0 for the first, and a
// non-finite V there turns that 0 into NaN, where the reference never reads
// the key (src/kernels.cu:1909-1920). Here each query visits only [lo, hi)
// (within the workgroup's key chunk), one key at a time: the score from this
// lane's half of Q^T (qf, pre-scaled to the log2 domain) and the other
// half's in lane l ^ 32, an online softmax, and this lane's outputs
// (register r of block vb: column vb*32 + 8*(r/4) + 4*half + r%4), so an
// admitted inf or NaN gives what the reference's sum gives and a masked one
// nothing. Slow (each query reads its keys from memory), and only for inputs
// with non-finite values next to a mask edge; the tile loop's accumulators
// are dead here, which keeps the kernel within its registers.
template <int D, int VD>
__device__ __forceinline__ void recompute_admitted(const float (&qf)[D / 2], const float* K,
                                                   uint64_t k_ld, const float* V, uint64_t v_ld,
                                                   uint64_t lo, uint64_t hi, int half,
                                                   v16f (&o)[VD / 32], float* m_out, float* l_out) {
#pragma unroll
    for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[vb][r] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    for (uint64_t j = lo; j < hi; ++j) {
        const float* krow = K + j * k_ld + half * (D / 2);
        float part = 0.0f;
#pragma unroll
        for (int t = 0; t < D / 2; t += 4) {
            const float4 k4 = *reinterpret_cast<const float4*>(krow + t);
            part += qf[t] * k4.x + qf[t + 1] * k4.y + qf[t + 2] * k4.z + qf[t + 3] * k4.w;
        }
        const float s = part + __shfl_xor(part, 32, 64);
        const float m_new = fmaxf(m, s);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m - m_use);
        const float w = __builtin_amdgcn_exp2f(s - m_use);
        l = l * alpha + w;
        const float* vrow = V + j * v_ld;
#pragma unroll
        for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 v4 = *reinterpret_cast<const float4*>(vrow + vb * 32 + 8 * g + 4 * half);
                o[vb][4 * g] = o[vb][4 * g] * alpha + w * v4.x;
                o[vb][4 * g + 1] = o[vb][4 * g + 1] * alpha + w * v4.y;
                o[vb][4 * g + 2] = o[vb][4 * g + 2] * alpha + w * v4.z;
                o[vb][4 * g + 3] = o[vb][4 * g + 3] * alpha + w * v4.w;
            }
        m = m_new;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[vb][r] *= inv;
    *m_out = m;
    *l_out = l;
}

// Short prefills, whose query tiles alone would leave most of the device
// idle, split the key range: chunk c of nchunks covers key tiles [c *
// chunk_tiles, (c + 1) * chunk_tiles) counted from key 0, and writes, per
// query, the chunk's normalised output, running max (log2 domain) and weight
// sum for attn_prefill_combine_kernel. The split depends on one sequence's
// shape only, so a batch still equals its separate calls.
struct PrefillSplit {
    uint32_t nchunks;      // 1: no split, the kernel writes the output itself
    uint32_t chunk_tiles;
    float* part_o;         // [batch * seq][heads][nchunks][VD]
    float* part_ml;        // [batch * seq][heads][nchunks][2]
};

// The workgroup walks its key tiles double-buffered in LDS, each tile loaded
// straight from global memory into LDS (no register staging), which keeps
// the kernel within 256 registers: two waves per SIMD, one from each of the
// two workgroups a CU holds, overlap each other's MFMA and softmax phases.
template <int D, int VD>
__global__ __launch_bounds__(256, 2) void attn_prefill_kernel(AttnArgs a, PrefillSplit sp) {
    apply_advance(a);
    using Cfg = PrefillCfg<D, VD>;
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int l32 = lane & 31, half = lane >> 5;

    // Heaviest (latest) query tiles first over the whole grid: under a causal
    // mask they see the most keys. Block ids are dealt round-robin to the 8
    // XCDs, so consecutive ids take the same query tile of different (batch,
    // head) pairs: every XCD gets an equal share of each weight class and runs
    // it heaviest first (ids of one head's query tiles, dealt to XCDs by
    // query tile, left XCDs with 2.4x the work of others).
    const uint64_t qtiles = (a.seq + Cfg::kBQ - 1) / Cfg::kBQ;
    const uint64_t chunk = blockIdx.x % sp.nchunks;
    const uint64_t pairs = gridDim.x / sp.nchunks / qtiles;
    const uint64_t bid = blockIdx.x / sp.nchunks;
    const uint64_t qt = qtiles - 1 - bid / pairs;
    const uint64_t bh = bid % pairs;
    const uint64_t head = bh % a.heads, b = bh / a.heads;
    const uint64_t kvh = head / (a.heads / a.kv_heads);

    const float* Q = a.q + b * a.q_bs + head * D;
    const float* K = a.k + b * a.k_bs + kvh * D;
    const float* V = a.v + b * a.v_bs + kvh * VD;
    float* O = a.out + b * a.o_bs + head * VD;
    const uint64_t q_ld = a.heads * D, k_ld = a.kv_heads * D, v_ld = a.kv_heads * VD,
                   o_ld = a.heads * VD;

    // This lane's query and its Q^T operand: Q[q][half * D/2 + t], t < D/2.
    const uint64_t q_first = qt * Cfg::kBQ;
    const uint64_t q = q_first + wave * 32 + l32;
    const bool q_live = q < a.seq;
    float qf[D / 2];
#pragma unroll
    for (int t = 0; t < D / 2; t += 4) {
        float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (q_live) v4 = *reinterpret_cast<const float4*>(Q + q * q_ld + half * (D / 2) + t);
        qf[t] = v4.x * a.qscale;
        qf[t + 1] = v4.y * a.qscale;
        qf[t + 2] = v4.z * a.qscale;
        qf[t + 3] = v4.w * a.qscale;
    }
    uint64_t q_lo = 0, q_hi = 0;
    if (q_live) key_range(a, a.offset + q, &q_lo, &q_hi);

    // Key range of the whole workgroup and of this wave (for skipping tiles),
    // and the keys every live query of the wave admits (tiles inside need no mask).
    const uint64_t q_last = min(a.seq, q_first + Cfg::kBQ) - 1;
    uint64_t blk_lo, blk_hi, tmp;
    key_range(a, a.offset + q_first, &blk_lo, &tmp);
    key_range(a, a.offset + q_last, &tmp, &blk_hi);
    const uint64_t w_first = q_first + wave * 32;
    const uint64_t w_last = min(a.seq, w_first + 32);
    uint64_t wave_lo = 0, wave_hi = 0, all_lo = 0, all_hi = 0;
    if (w_first < a.seq) {
        key_range(a, a.offset + w_first, &wave_lo, &all_hi);
        key_range(a, a.offset + w_last - 1, &all_lo, &wave_hi);
    }
    const uint64_t tile_begin = blk_lo / Cfg::kBKV * Cfg::kBKV;
    const int ntiles = blk_hi > tile_begin
                           ? static_cast<int>((blk_hi - tile_begin + Cfg::kBKV - 1) / Cfg::kBKV)
                           : 0;
    auto wave_in = [&](uint64_t k0) { return k0 < wave_hi && k0 + Cfg::kBKV > wave_lo; };
    // This query's admitted keys relative to the first tile (32-bit: the
    // caller keeps key counts below 2^31).
    const int rel_lo = static_cast<int>(q_lo > tile_begin ? q_lo - tile_begin : 0);
    const int rel_hi = static_cast<int>(q_hi > tile_begin ? q_hi - tile_begin : 0);

    float m = -INFINITY, l = 0.0f;
    v16f o[VD / 32];
#pragma unroll
    for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[vb][r] = 0.0f;

    float* const kbuf0 = lds;
    float* const vbuf0 = lds + 2 * Cfg::kKTile;
    auto kbuf = [&](int i) { return kbuf0 + (i & 1) * Cfg::kKTile; };
    auto vbuf = [&](int i) { return vbuf0 + (i & 1) * Cfg::kVTile; };
    const TileDma<D> kdma(k_ld, wave, lane);
    const TileDma<VD> vdma(v_ld, wave, lane);
    auto load_k = [&](uint64_t k0, float* dst) { kdma.load(K, k_ld, k0, a.kv_seq, dst, wave, lane); };
    auto load_v = [&](uint64_t k0, float* dst) { vdma.load(V, v_ld, k0, a.kv_seq, dst, wave, lane); };

    // V reads: key row `key`, column vb*32 + l32 sits in chunk
    // (vb*8 + l32/4) ^ (key & 15), and key & 15 = 8*((t/4) & 1) + 4*half +
    // t%4 for step t: block vb ^ ((t/4) & 1), chunk (l32/4) ^ (4*half + t%4).
    int vx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) vx[j] = (((l32 >> 2) ^ (4 * half + j)) << 2) + (l32 & 3);

    // This workgroup's tiles [i_begin, i_end) of the ntiles from tile_begin:
    // all of them, or the part inside its key chunk.
    int i_begin = 0, i_end = ntiles;
    if (sp.nchunks > 1) {
        const int64_t first = static_cast<int64_t>(tile_begin / Cfg::kBKV);
        const int64_t c0 = static_cast<int64_t>(chunk) * sp.chunk_tiles - first;
        i_begin = static_cast<int>(min<int64_t>(max<int64_t>(c0, 0), ntiles));
        i_end = static_cast<int>(min<int64_t>(max<int64_t>(c0 + sp.chunk_tiles, 0), ntiles));
    }

    // The j-th tile walked sits in buffer j & 1 (K and V); the next one is
    // loaded straight into the other buffer while it is used (that buffer
    // held the previous tile, whose readers all passed the previous barrier).
    bool redo = false;  // an edge tile of this wave held a non-finite V value
    if (i_end > i_begin) {
        load_k(tile_begin + static_cast<uint64_t>(i_begin) * Cfg::kBKV, kbuf(0));
        load_v(tile_begin + static_cast<uint64_t>(i_begin) * Cfg::kBKV, vbuf(0));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int i = i_begin; i < i_end; ++i) {
        const int j = i - i_begin;
        const int cur = j & 1;
        const uint64_t k0 = tile_begin + static_cast<uint64_t>(i) * Cfg::kBKV;
        if (i + 1 < i_end) {
            load_k(k0 + Cfg::kBKV, kbuf(cur ^ 1));
            load_v(k0 + Cfg::kBKV, vbuf(cur ^ 1));
        }
        if (wave_in(k0)) {
            // A tile every query of the wave admits whole needs no mask.
            const bool masked = !(k0 >= all_lo && k0 + Cfg::kBKV <= all_hi);
            const float* sv = vbuf(cur);
            // An edge tile checks its V for non-finite values (integer steps:
            // an all-ones exponent gives e + 1 = 256, so (e + 1) >> 8 is 1; no
            // compare masks to hold; four reads in flight), before the scores
            // while fewer registers are live. One found sends the wave to
            // recompute_admitted after the loop.
            if (masked) {
                uint32_t nonfinite = 0;
                const mhip::f32x4* tile4 = reinterpret_cast<const mhip::f32x4*>(sv);
#pragma unroll
                for (int j = 0; j < Cfg::kVTile / 4 / 64; ++j) {
                    const mhip::f32x4 v4 = tile4[j * 64 + lane];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        nonfinite |= (((__float_as_uint(v4[e]) >> 23) & 0xFFu) + 1u) >> 8;
                    if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
                }
                redo |= __builtin_amdgcn_ballot_w64(nonfinite != 0) != 0;
            }
            v16f s_cur = tile_scores<D>(kbuf(cur), qf, l32, half);
            // Register r holds key k0 + 8*(r/4) + 4*half + r%4 of query q; bit
            // j of `span` says whether tile key j is admitted.
            if (masked) {
                const int lo_r = min(max(rel_lo - i * Cfg::kBKV, 0), Cfg::kBKV);
                const int hi_r = min(max(rel_hi - i * Cfg::kBKV, 0), Cfg::kBKV);
                const uint64_t span = ((1ull << hi_r) - 1ull) & ~((1ull << lo_r) - 1ull);
                const uint32_t mine = static_cast<uint32_t>(span) >> (4 * half);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = 8 * (r / 4) + (r % 4);
                    s_cur[r] = (mine >> key) & 1u ? s_cur[r] : -INFINITY;
                }
            }
            float tile_max = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) tile_max = fmaxf(tile_max, s_cur[r]);
            tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32, 64));
            // Every lane runs the update (the MFMAs below need the whole wave);
            // a query with no admitted key yet keeps m = -inf, l = 0, o = 0.
            const float m_new = fmaxf(m, tile_max);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m - m_use);
            float psum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s_cur[r] = __builtin_amdgcn_exp2f(s_cur[r] - m_use);
                psum += s_cur[r];
            }
            psum += __shfl_xor(psum, 32, 64);
            const float l_new = l * alpha + psum;
            const float inv = l_new > 0.0f ? __builtin_amdgcn_rcpf(l_new) : 0.0f;
            // A tile that adds nothing for this query leaves its output as it was.
            const float keep = (psum == 0.0f && alpha == 1.0f) || l_new == 0.0f ? 1.0f : (l * alpha) * inv;
#pragma unroll
            for (int r = 0; r < 16; ++r) s_cur[r] *= inv;
#pragma unroll
            for (int vb = 0; vb < VD / 32; ++vb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) o[vb][r] *= keep;
                // O^T += V^T . P^T: step t pairs key 8*(t/4) + 4*half + t%4 with register t.
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const int key_row = 8 * (t / 4) + 4 * half + (t % 4);
                    const float v = sv[key_row * VD + (vb ^ ((t >> 2) & 1)) * 32 + vx[t % 4]];
                    o[vb] = __builtin_amdgcn_mfma_f32_32x32x2f32(v, s_cur[t], o[vb], 0, 0, 0);
                }
            }
            m = m_new;
            l = l_new;
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }

    if (redo) {
        // This workgroup's keys (its tiles [i_begin, i_end)), the query's range within them.
        const uint64_t c_lo = tile_begin + static_cast<uint64_t>(i_begin) * Cfg::kBKV;
        const uint64_t c_hi = tile_begin + static_cast<uint64_t>(i_end) * Cfg::kBKV;
        const uint64_t lo = max(q_lo, c_lo), hi = min(q_hi, c_hi);
        recompute_admitted<D, VD>(qf, K, k_ld, V, v_ld, lo, hi > lo ? hi : lo, half, o, &m, &l);
    }

    // Register r of block vb holds O[q][vb*32 + 8*(r/4) + 4*half + r%4].
    if (q_live && sp.nchunks > 1) {
        const uint64_t rec = ((b * a.seq + q) * a.heads + head) * sp.nchunks + chunk;
        float* po = sp.part_o + rec * VD;
#pragma unroll
        for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(po + vb * 32 + 8 * g + 4 * half) =
                    make_float4(o[vb][4 * g], o[vb][4 * g + 1], o[vb][4 * g + 2], o[vb][4 * g + 3]);
        if (half == 0) *reinterpret_cast<float2*>(sp.part_ml + 2 * rec) = make_float2(m, l);
    } else if (q_live) {
        float* orow = O + q * o_ld;
#pragma unroll
        for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(orow + vb * 32 + 8 * g + 4 * half) =
                    make_float4(o[vb][4 * g], o[vb][4 * g + 1], o[vb][4 * g + 2], o[vb][4 * g + 3]);
    }
}

// Chunk records of split attention live in the context's workspace.
mhip_status attention_workspace(mhip_ctx* ctx, size_t bytes, float** out) {
    void* p = nullptr;
    mhip_status st = mhip::workspace(ctx, bytes, &p);
    *out = static_cast<float*>(p);
    return st;
}

// Merges a split prefill's chunk records per (query row, head): out = sum_c
// w_c o_c with w_c = l_c 2^(m_c - M) / sum_c' l_c' 2^(m_c' - M), in chunk
// order; no admitted key in any chunk gives zeros. VD / 4 threads per (row,
// head), one float4 of the output each.
template <int VD>
__global__ __launch_bounds__(256) void attn_prefill_combine_kernel(AttnArgs a, uint64_t rows,
                                                                   PrefillSplit sp) {
    constexpr int kLanes = VD / 4;
    constexpr int kItems = 256 / kLanes;
    const uint64_t item = static_cast<uint64_t>(blockIdx.x) * kItems + threadIdx.x / kLanes;
    const int t = threadIdx.x % kLanes;
    if (item >= rows * a.heads) return;
    const uint64_t row = item / a.heads, head = item % a.heads;
    const uint64_t b = row / a.seq, q = row % a.seq;
    const float* ml = sp.part_ml + 2 * item * sp.nchunks;
    const float* po = sp.part_o + item * sp.nchunks * VD + 4 * t;
    float M = -INFINITY;
    for (uint32_t c = 0; c < sp.nchunks; ++c) M = fmaxf(M, ml[2 * c]);
    float total = 0.0f;
    if (M != -INFINITY)
        for (uint32_t c = 0; c < sp.nchunks; ++c)
            if (ml[2 * c + 1] > 0.0f) total += ml[2 * c + 1] * exp2f(ml[2 * c] - M);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (total > 0.0f) {
        const float inv_total = 1.0f / total;
        for (uint32_t c = 0; c < sp.nchunks; ++c) {
            const float l = ml[2 * c + 1];
            if (!(l > 0.0f)) continue;
            const float w = l * exp2f(ml[2 * c] - M) * inv_total;
            const float4 o = *reinterpret_cast<const float4*>(po + c * VD);
            acc.x += w * o.x; acc.y += w * o.y; acc.z += w * o.z; acc.w += w * o.w;
        }
    }
    *reinterpret_cast<float4*>(a.out + b * a.o_bs + q * (a.heads * VD) + head * VD + 4 * t) = acc;
}

// Key chunks for a prefill whose query tiles (per sequence) fill under the
// device's resident slots (two workgroups per CU): enough chunks of at
// least 4 key tiles to fill them, at most 16.
void prefill_split(const mhip_ctx* ctx, const AttnArgs& a, uint64_t qtiles, uint64_t kbkv,
                   uint32_t* nchunks, uint32_t* chunk_tiles) {
    *nchunks = 1;
    *chunk_tiles = 0;
    // A replayed key count may pass the captured one: chunks sized here from
    // the captured count would leave the later keys to no workgroup.
    if (a.advance) return;
    const uint64_t slots = 2 * static_cast<uint64_t>(ctx->compute_units ? ctx->compute_units : 256);
    const uint64_t per_sequence = a.heads * qtiles;
    const uint64_t kv_tiles = (a.kv_seq + kbkv - 1) / kbkv;
    if (per_sequence >= slots || kv_tiles < 8) return;
    uint64_t n = std::min<uint64_t>((slots + per_sequence - 1) / per_sequence, kv_tiles / 4);
    n = std::min<uint64_t>(n, 16);
    if (n < 2) return;
    const uint64_t per = (kv_tiles + n - 1) / n;
    *chunk_tiles = static_cast<uint32_t>(per);
    *nchunks = static_cast<uint32_t>((kv_tiles + per - 1) / per);
}

template <int D, int VD>
mhip_status launch_prefill(mhip_ctx* ctx, const AttnArgs& a, uint64_t batch) {
    using Cfg = PrefillCfg<D, VD>;
    const uint64_t qtiles = (a.seq + Cfg::kBQ - 1) / Cfg::kBQ;
    PrefillSplit sp{};
    prefill_split(ctx, a, qtiles, Cfg::kBKV, &sp.nchunks, &sp.chunk_tiles);
    const uint64_t blocks = batch * a.heads * qtiles * sp.nchunks;
    if (blocks >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention: too many query tiles");
    const uint64_t rows = batch * a.seq;
    if (sp.nchunks > 1) {
        const uint64_t records = rows * a.heads * sp.nchunks;
        float* part = nullptr;
        mhip_status st = attention_workspace(ctx, records * (VD + 2) * sizeof(float), &part);
        if (st != MHIP_OK) return st;
        sp.part_o = part;
        sp.part_ml = part + records * VD;
    }
    const size_t lds = Cfg::kLdsFloats * sizeof(float);
    static bool configured = false;
    if (!configured) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_prefill_kernel<D, VD>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        configured = true;
    }
    mhip::launch(ctx, (attn_prefill_kernel<D, VD>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                 lds, a, sp);
    mhip_status st = mhip::check_launch("attention (MFMA prefill)");
    if (st != MHIP_OK || sp.nchunks == 1) return st;
    const uint64_t items = rows * a.heads;
    constexpr uint64_t kItems = 256 / (VD / 4);
    mhip::launch(ctx, (attn_prefill_combine_kernel<VD>),
                 dim3(static_cast<unsigned>((items + kItems - 1) / kItems)), dim3(256), 0, a, rows,
                 sp);
    return mhip::check_launch("attention (prefill chunk merge)");
}

// ---------------------------------------------------------------------------
// Decode: split-KV over key chunks, all query heads of a KV head together
// ---------------------------------------------------------------------------

constexpr int kMaxGroup = 8;  // query heads per workgroup; larger groups take several

// Keys per chunk for head dim 4*D4: kDecodeSteps(D4) steps of 256/D4 keys
// (D4 lanes hold one key row, 64/D4 keys per wave, four waves). At D >= 16
// a chunk is 32 KB of K plus 32 KB of V.
// Calls whose default chunks give every CU 16 workgroups or more (many
// batch rows or heads, long caches) take twice the steps: half the
// workgroups and records (C4 decode, B8 KV 4096: 175 -> 171 us).
__host__ __device__ constexpr int decode_steps(int d4) { return d4 >= 4 ? 8 : 2 * d4; }
__host__ __device__ constexpr int decode_chunk(int d4, int steps) { return steps * 256 / d4; }
__host__ __device__ constexpr int decode_chunk(int d4) { return decode_chunk(d4, decode_steps(d4)); }

// One workgroup per (batch, KV head, key chunk). Every thread issues all of
// its K and V loads before any arithmetic (2 * kSteps dwordx4 in flight);
// scores, the chunk max and the probabilities stay in registers, and only
// the per-wave partial sums meet in LDS. Writes, per query head of the
// group, the chunk's output normalised by its own weight sum, plus the
// chunk max (log2 domain) and weight sum.
template <int D4, int GT, int STEPS>
__global__ __launch_bounds__(256) void attn_decode_partial_kernel(
    AttnArgs a, uint64_t key_base, uint64_t chunks, float* __restrict__ part_o,
    float* __restrict__ part_ml) {
    constexpr int kLPK = D4;              // lanes per key
    constexpr int kKPS = 64 / kLPK;       // keys per wave step
    constexpr int kKPW = 4 * kKPS;        // keys per workgroup step
    constexpr int kSteps = STEPS;
    constexpr int D = 4 * D4;
    __shared__ float4 sq[GT][D4];
    __shared__ float4 red[4][GT][D4];
    __shared__ float wm[4][GT], wl[4][GT];

    // (batch, KV head) varies fastest: workgroups in flight together read
    // whole K/V rows (all heads of the same keys) rather than one head's
    // 4*D-byte slice of many rows. A group of more than GT query heads is
    // taken GT heads at a time (head slice hs), each slice reading the chunk.
    const int group_all = static_cast<int>(a.heads / a.kv_heads);
    const int slices = (group_all + GT - 1) / GT;
    const uint64_t units = gridDim.x / chunks;
    const uint64_t c_idx = blockIdx.x / units;
    const uint64_t unit = blockIdx.x % units;
    const uint64_t pairs = units / static_cast<uint64_t>(slices);
    const int hs = static_cast<int>(unit / pairs);
    const uint64_t bkv = unit % pairs;
    const uint64_t kvh = bkv % a.kv_heads, b = bkv / a.kv_heads;
    const int group = min(GT, group_all - hs * GT);
    const uint64_t head0 = kvh * static_cast<uint64_t>(group_all) + static_cast<uint64_t>(hs) * GT;
    // The chunk's keys: [key_base + c * chunk, + chunk) inside the admitted
    // range of the query (at position offset; a replay may move it).
    apply_advance(a);
    uint64_t key_lo, key_hi;
    key_range(a, a.offset, &key_lo, &key_hi);
    const uint64_t c_base = key_base + c_idx * static_cast<uint64_t>(kSteps * kKPW);
    const uint64_t c_lo = max(c_base, key_lo);
    const uint64_t c_hi = min(c_base + static_cast<uint64_t>(kSteps * kKPW), key_hi);
    const int n = c_lo < c_hi ? static_cast<int>(c_hi - c_lo) : 0;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / kLPK, sl = lane % kLPK;
    const uint64_t k_ld = a.kv_heads * D;
    const float* K = a.k + b * a.k_bs + kvh * D + 4 * sl;
    const float* V = a.v + b * a.v_bs + kvh * D + 4 * sl;

    float4 kr[kSteps], vr[kSteps];
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
        const int j = u * kKPW + wave * kKPS + sub;
        kr[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        vr[u] = kr[u];
        if (j < n) {
            kr[u] = mhip::load_nt(reinterpret_cast<const float4*>(K + (c_lo + j) * k_ld));
            vr[u] = mhip::load_nt(reinterpret_cast<const float4*>(V + (c_lo + j) * k_ld));
        }
    }
    const float* Qb = a.q + b * a.q_bs + head0 * D;
    for (int i = threadIdx.x; i < group * D4; i += 256) {
        float4 q4 = *reinterpret_cast<const float4*>(Qb + 4 * static_cast<uint64_t>(i));
        q4.x *= a.qscale; q4.y *= a.qscale; q4.z *= a.qscale; q4.w *= a.qscale;
        sq[i / D4][i % D4] = q4;
    }
    __syncthreads();

    // Scores (log2 domain) and the chunk max per head.
    float s[GT][kSteps];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        if (g >= group) break;
        const float4 q4 = sq[g][sl];
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < kSteps; ++u) {
            float dot = kr[u].x * q4.x + kr[u].y * q4.y + kr[u].z * q4.z + kr[u].w * q4.w;
#pragma unroll
            for (int off = kLPK / 2; off >= 1; off >>= 1) dot += __shfl_xor(dot, off, 64);
            const int j = u * kKPW + wave * kKPS + sub;
            s[g][u] = j < n ? dot : -INFINITY;
            mx = fmaxf(mx, s[g][u]);
        }
#pragma unroll
        for (int off = kLPK; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        if (lane == 0) wm[wave][g] = mx;
    }
    __syncthreads();

    // Probabilities and the chunk's weight sum per head.
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        if (g >= group) break;
        const float m = fmaxf(fmaxf(wm[0][g], wm[1][g]), fmaxf(wm[2][g], wm[3][g]));
        float l = 0.0f;
#pragma unroll
        for (int u = 0; u < kSteps; ++u) {
            s[g][u] = m == -INFINITY ? 0.0f : exp2f(s[g][u] - m);
            l += s[g][u];
        }
#pragma unroll
        for (int off = kLPK; off < 64; off <<= 1) l += __shfl_xor(l, off, 64);
        if (lane == 0) wl[wave][g] = l;
    }
    __syncthreads();

    // Weighted V rows with normalised probabilities: every partial sum is a
    // convex combination of V rows, so none overflows.
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        if (g >= group) break;
        const float l = (wl[0][g] + wl[1][g]) + (wl[2][g] + wl[3][g]);
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < kSteps; ++u) {
            const float p = s[g][u] * inv;
            acc.x += p * vr[u].x;
            acc.y += p * vr[u].y;
            acc.z += p * vr[u].z;
            acc.w += p * vr[u].w;
        }
#pragma unroll
        for (int off = kLPK; off < 64; off <<= 1) {
            acc.x += __shfl_xor(acc.x, off, 64);
            acc.y += __shfl_xor(acc.y, off, 64);
            acc.z += __shfl_xor(acc.z, off, 64);
            acc.w += __shfl_xor(acc.w, off, 64);
        }
        if (sub == 0) red[wave][g][sl] = acc;
    }
    __syncthreads();

    const uint64_t bh0 = b * a.heads + head0;
    for (int i = threadIdx.x; i < group * D4; i += 256) {
        const int g = i / D4, t = i % D4;
        float4 o = red[0][g][t];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const float4 r = red[w][g][t];
            o.x += r.x; o.y += r.y; o.z += r.z; o.w += r.w;
        }
        const float l = (wl[0][g] + wl[1][g]) + (wl[2][g] + wl[3][g]);
        const uint64_t rec = (bh0 + g) * chunks + c_idx;
        *reinterpret_cast<float4*>(part_o + rec * D + 4 * t) = o;
        if (t == 0) {
            const float m = fmaxf(fmaxf(wm[0][g], wm[1][g]), fmaxf(wm[2][g], wm[3][g]));
            *reinterpret_cast<float2*>(part_ml + 2 * rec) = make_float2(m, l);
        }
    }
}

// Merges the chunk records of one (batch, head) (mhip::merge_decode_chunks,
// whose fixed order every run repeats) and writes its output row.
template <int D4>
__global__ __launch_bounds__(256) void attn_decode_combine_kernel(
    AttnArgs a, uint64_t chunks, const float* __restrict__ part_o,
    const float* __restrict__ part_ml) {
    constexpr int D = 4 * D4;
    const uint64_t bh = blockIdx.x;
    const uint64_t head = bh % a.heads, b = bh / a.heads;
    const float4 v = mhip::merge_decode_chunks<D4>(part_ml + 2 * bh * chunks, part_o + bh * chunks * D,
                                                   chunks, 0, D4);
    if (threadIdx.x < D4)
        *reinterpret_cast<float4*>(a.out + b * a.o_bs + head * D + 4 * threadIdx.x) = v;
}

// Keys [lo, hi) in chunks of STEPS steps. `keep`: leave the chunk records
// for the caller's merge (no combine launch) and reserve `keep->extra_bytes`
// more of the workspace for it.
template <int D4, int GT, int STEPS>
mhip_status launch_decode_chunks(mhip_ctx* ctx, const AttnArgs& a, uint64_t batch, uint64_t kv_rows,
                                 bool bounded, mhip::DecodeChunks* keep, uint64_t lo, uint64_t hi) {
    constexpr int D = 4 * D4;
    constexpr uint64_t kChunk = decode_chunk(D4, STEPS);
    uint64_t chunks = (hi - lo + kChunk - 1) / kChunk;
    if (chunks == 0) chunks = 1;
    const uint64_t slices = (a.heads / a.kv_heads + GT - 1) / GT;
    const uint64_t units = batch * a.kv_heads * slices;
    if (units * chunks >= (1ULL << 31))
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention decode: too many key chunks");
    const uint64_t records = batch * a.heads * chunks;
    // A call bounded by a key count sizes the scratch for every row of K/V
    // (at the shorter chunks, the most records), so a step captured later at
    // the same shape never needs to grow it.
    constexpr uint64_t kShortChunk = decode_chunk(D4);
    const uint64_t reserve = bounded ? batch * a.heads * std::max<uint64_t>(1, (kv_rows + kShortChunk - 1) / kShortChunk)
                                     : records;
    float* part = nullptr;
    const uint64_t record_floats = (std::max(records, reserve) * (D + 2) + 63) / 64 * 64;
    const size_t extra = keep ? keep->extra_bytes : 0;
    mhip_status st = attention_workspace(ctx, record_floats * sizeof(float) + extra, &part);
    if (st != MHIP_OK) return st;
    float* part_o = part;
    float* part_ml = part + records * D;
    mhip::launch(ctx, (attn_decode_partial_kernel<D4, GT, STEPS>),
                 dim3(static_cast<unsigned>(units * chunks)), dim3(256), 0, a, lo, chunks, part_o,
                 part_ml);
    st = mhip::check_launch("attention (decode chunks)");
    if (st != MHIP_OK) return st;
    if (keep) {
        keep->part_o = part_o;
        keep->part_ml = part_ml;
        keep->chunks = chunks;
        keep->extra = part + record_floats;
        return MHIP_OK;
    }
    mhip::launch(ctx, attn_decode_combine_kernel<D4>, dim3(static_cast<unsigned>(batch * a.heads)),
                 dim3(256), 0, a, chunks, part_o, part_ml);
    return mhip::check_launch("attention (decode combine)");
}

template <int D4, int GT>
mhip_status launch_decode_group(mhip_ctx* ctx, const AttnArgs& a, uint64_t batch,
                                uint64_t kv_rows, bool bounded, mhip::DecodeChunks* keep) {
    // The one query (seq == 1) sits at position kv_seq - 1 in every batch
    // row and head, so the admitted key range is the same for all of them.
    // A captured call whose key count advances covers every row of K/V; its
    // workgroups find their keys from the replayed count.
    uint64_t lo = 0, hi = kv_rows;
    if (!a.advance) {
        uint64_t upper = a.causal ? a.offset + 1 : a.kv_seq;
        if (upper > a.kv_seq) upper = a.kv_seq;
        uint64_t lower = 0;
        if (a.window >= 0) {
            const uint64_t w = static_cast<uint64_t>(a.window);
            const uint64_t back = w > 0 ? w - 1 : 0;
            lower = a.offset > back ? a.offset - back : 0;
            if (lower > upper) lower = upper;
        }
        lo = lower;
        hi = upper;
    }
    constexpr int kSteps = decode_steps(D4);
    if constexpr (D4 >= 4 && GT <= 2) {
        // The choice follows the capacity for a bounded call, so its eager
        // run and a capture of it take the same chunks.
        const uint64_t span = bounded ? kv_rows : hi - lo;
        const uint64_t slices = (a.heads / a.kv_heads + GT - 1) / GT;
        const uint64_t wgs = batch * a.kv_heads * slices * ((span + decode_chunk(D4) - 1) / decode_chunk(D4));
        const uint64_t cus = ctx->compute_units ? ctx->compute_units : 256;
        if (wgs >= 16 * cus)
            return launch_decode_chunks<D4, GT, 2 * kSteps>(ctx, a, batch, kv_rows, bounded, keep, lo, hi);
    }
    return launch_decode_chunks<D4, GT, kSteps>(ctx, a, batch, kv_rows, bounded, keep, lo, hi);
}

template <int D4>
mhip_status launch_decode(mhip_ctx* ctx, const AttnArgs& a, uint64_t batch, uint64_t kv_rows,
                          bool bounded, mhip::DecodeChunks* keep = nullptr) {
    const uint64_t group = a.heads / a.kv_heads;
    if (group == 1) return launch_decode_group<D4, 1>(ctx, a, batch, kv_rows, bounded, keep);
    if (group == 2) return launch_decode_group<D4, 2>(ctx, a, batch, kv_rows, bounded, keep);
    if (group <= 4) return launch_decode_group<D4, 4>(ctx, a, batch, kv_rows, bounded, keep);
    return launch_decode_group<D4, kMaxGroup>(ctx, a, batch, kv_rows, bounded, keep);
}

// ---------------------------------------------------------------------------
// Generic: one wave per (batch, query, head)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void attn_generic_kernel(AttnArgs a, uint64_t total) {
    apply_advance(a);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t item = static_cast<uint64_t>(blockIdx.x) * 4 + wave;
    if (item >= total) return;
    const uint64_t head = item % a.heads;
    const uint64_t qi = (item / a.heads) % a.seq;
    const uint64_t b = item / (a.heads * a.seq);
    const uint64_t kvh = head / (a.heads / a.kv_heads);
    const float* qrow = a.q + b * a.q_bs + qi * a.heads * a.d + head * a.d;
    const float* K = a.k + b * a.k_bs + kvh * a.d;
    const float* V = a.v + b * a.v_bs + kvh * a.vd;
    const uint64_t k_ld = a.kv_heads * a.d, v_ld = a.kv_heads * a.vd;
    float* orow = a.out + b * a.o_bs + qi * a.heads * a.vd + head * a.vd;
    uint64_t lo, hi;
    key_range(a, a.offset + qi, &lo, &hi);
    constexpr int kMaxCols = 4;  // value columns per lane: vd <= 256
    float acc[kMaxCols] = {0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    for (uint64_t k0 = lo; k0 < hi; k0 += 64) {
        const uint64_t key = k0 + lane;
        float s = -INFINITY;
        if (key < hi) {
            float dot = 0.0f;
            for (uint64_t t = 0; t < a.d; ++t) dot += qrow[t] * K[key * k_ld + t];
            s = dot * a.qscale;
        }
        float mx = s;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        const float m_new = fmaxf(m, mx);
        const float p = exp2f(s - m_new);
        float sum = p;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
        const float alpha = exp2f(m - m_new);
        const float l_new = l * alpha + sum;
        const float inv = 1.0f / l_new;
        const float keep = l * alpha * inv;
        const float p_hat = p * inv;
        const int nk = static_cast<int>(min<uint64_t>(64, hi - k0));
#pragma unroll
        for (int c = 0; c < kMaxCols; ++c) acc[c] *= keep;
        for (int j = 0; j < nk; ++j) {
            const float pj = __shfl(p_hat, j, 64);
#pragma unroll
            for (int c = 0; c < kMaxCols; ++c) {
                const uint64_t col = lane + 64 * c;
                if (col < a.vd) acc[c] += pj * V[(k0 + j) * v_ld + col];
            }
        }
        m = m_new;
        l = l_new;
    }
    for (int c = 0; c < kMaxCols; ++c) {
        const uint64_t col = lane + 64 * c;
        if (col < a.vd) orow[col] = acc[c];
    }
}

}  // namespace

namespace {

// The checks and kernel arguments of mhip_attention_f32; *empty when there
// is no query row (nothing to do).
mhip_status prepare_attention(mhip_ctx* ctx, const float* q, const float* k, const float* v,
                              float* out, const mhip_attention_params* p, AttnArgs* args,
                              uint64_t* batch_out, bool* empty) {
    *empty = false;
    if (!p) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention: null params");
    const uint64_t H = p->head_count, Hkv = p->kv_head_count, d = p->head_dimension;
    const uint64_t vd = p->value_dimension ? p->value_dimension : d;
    if (H == 0 || d == 0 || Hkv == 0 || vd == 0)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "head_count, kv_head_count, and head_dimension must all be positive");
    if (H % Hkv != 0)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "head_count " + std::to_string(H) +
                              " must be an exact multiple of kv_head_count " + std::to_string(Hkv));
    if (p->window_size == 0)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "window_size must be positive; a zero window admits no keys");
    if (p->window_size > 0 && !p->causal)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "window_size is only defined for causal attention");
    if (p->kv_seq_len > p->kv_rows)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "key_count " + std::to_string(p->kv_seq_len) + " exceeds the " +
                              std::to_string(p->kv_rows) + " rows of K/V");
    if (p->seq_len > p->kv_seq_len)
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED,
                          "q sequence length " + std::to_string(p->seq_len) +
                              " cannot exceed k/v sequence length " + std::to_string(p->kv_seq_len));
    if (!(p->scale <= 0.0f) && !std::isfinite(p->scale))
        return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention scale must be finite and positive");
    const uint64_t batch = p->batch ? p->batch : 1;
    *batch_out = batch;
    if (p->seq_len == 0) {
        *empty = true;
        return MHIP_OK;
    }
    if (!q || !k || !v || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention: null buffer");

    AttnArgs& a = *args;
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.seq = p->seq_len;
    a.kv_seq = p->kv_seq_len;
    a.heads = H;
    a.kv_heads = Hkv;
    a.d = d;
    a.vd = vd;
    a.offset = p->kv_seq_len - p->seq_len;
    a.causal = p->causal ? 1 : 0;
    a.window = p->window_size > 0 ? p->window_size : -1;
    const float scale = p->scale > 0.0f ? p->scale : 1.0f / std::sqrt(static_cast<float>(d));
    a.qscale = scale * kLog2e;
    // A captured call bounded by an explicit key count advances it with the
    // replay offset (one query row; several rows replay only at offset 0).
    a.advance = nullptr;
    if (p->bounded_key_count) {
        if (p->seq_len == 1)
            a.advance = mhip::advance_ptr(ctx, MHIP_ADVANCE_KEY_COUNT, p->kv_rows - p->kv_seq_len);
        else
            (void)mhip::advance_ptr(ctx, MHIP_ADVANCE_KEY_COUNT, 0);
    }
    a.q_bs = p->q_batch_stride ? p->q_batch_stride : p->seq_len * H * d;
    a.k_bs = p->kv_batch_stride ? p->kv_batch_stride : p->kv_rows * Hkv * d;
    a.v_bs = p->v_batch_stride ? p->v_batch_stride : p->kv_rows * Hkv * vd;
    a.o_bs = p->out_batch_stride ? p->out_batch_stride : p->seq_len * H * vd;
    return MHIP_OK;
}

bool decode_aligned(const AttnArgs& a) {
    return mhip::aligned16(a.q) && mhip::aligned16(a.k) && mhip::aligned16(a.v) &&
           mhip::aligned16(a.out) && a.q_bs % 4 == 0 && a.k_bs % 4 == 0 && a.v_bs % 4 == 0 &&
           a.o_bs % 4 == 0;
}

}  // namespace

namespace mhip {

mhip_status attention_decode_chunks_f32(mhip_ctx* ctx, const float* q, const float* k,
                                        const float* v, const mhip_attention_params* p,
                                        DecodeChunks* out) {
    MHIP_REQUIRE_CTX(ctx);
    if (!out || !p || p->seq_len != 1 || (p->batch && p->batch != 1)) return MHIP_LAYOUT_UNSUPPORTED;
    AttnArgs a;
    uint64_t batch = 1;
    bool empty = false;
    // No output row is written: the records' consumer merges them. Any
    // aligned address stands in for the output in the checks.
    mhip_status st = prepare_attention(ctx, q, k, v, const_cast<float*>(q), p, &a, &batch, &empty);
    if (st != MHIP_OK) return st;
    const uint64_t d = a.d;
    if (empty || !decode_aligned(a) || a.vd != d || d % 4 != 0 || d > 256 || p->kv_seq_len == 0)
        return MHIP_LAYOUT_UNSUPPORTED;
    out->heads = a.heads;
    out->d = d;
    const bool bounded = p->bounded_key_count != 0;
    switch (d / 4) {
        case 1: return launch_decode<1>(ctx, a, 1, p->kv_rows, bounded, out);
        case 2: return launch_decode<2>(ctx, a, 1, p->kv_rows, bounded, out);
        case 4: return launch_decode<4>(ctx, a, 1, p->kv_rows, bounded, out);
        case 8: return launch_decode<8>(ctx, a, 1, p->kv_rows, bounded, out);
        case 16: return launch_decode<16>(ctx, a, 1, p->kv_rows, bounded, out);
        case 32: return launch_decode<32>(ctx, a, 1, p->kv_rows, bounded, out);
        case 64: return launch_decode<64>(ctx, a, 1, p->kv_rows, bounded, out);
        default: return MHIP_LAYOUT_UNSUPPORTED;
    }
}

}  // namespace mhip

extern "C" mhip_status mhip_attention_f32(mhip_ctx* ctx, const float* q, const float* k,
                                          const float* v, float* out,
                                          const mhip_attention_params* p) {
    MHIP_REQUIRE_CTX(ctx);
    AttnArgs a;
    uint64_t batch = 1;
    bool empty = false;
    mhip_status pst = prepare_attention(ctx, q, k, v, out, p, &a, &batch, &empty);
    if (pst != MHIP_OK || empty) return pst;
    const uint64_t H = a.heads, d = a.d, vd = a.vd;

    const bool aligned = decode_aligned(a);
    if (aligned && p->seq_len == 1 && vd == d && d % 4 == 0 && d <= 256 && p->kv_seq_len > 0) {
        mhip_status st = MHIP_CAPTURE_UNSUPPORTED;
        switch (d / 4) {
            case 1: st = launch_decode<1>(ctx, a, batch, p->kv_rows, p->bounded_key_count != 0); break;
            case 2: st = launch_decode<2>(ctx, a, batch, p->kv_rows, p->bounded_key_count != 0); break;
            case 4: st = launch_decode<4>(ctx, a, batch, p->kv_rows, p->bounded_key_count != 0); break;
            case 8: st = launch_decode<8>(ctx, a, batch, p->kv_rows, p->bounded_key_count != 0); break;
            case 16: st = launch_decode<16>(ctx, a, batch, p->kv_rows, p->bounded_key_count != 0); break;
            case 32: st = launch_decode<32>(ctx, a, batch, p->kv_rows, p->bounded_key_count != 0); break;
            case 64: st = launch_decode<64>(ctx, a, batch, p->kv_rows, p->bounded_key_count != 0); break;
            default: break;
        }
        if (st != MHIP_CAPTURE_UNSUPPORTED) return st;  // else: no decode kernel for this d
    }
    // The MFMA kernel's key arithmetic is 32-bit, and so are its byte
    // offsets within a 32-row K or V tile.
    const bool small_keys = p->kv_rows < (1ULL << 31) && a.kv_heads * std::max(d, vd) < (1ULL << 25);
    if (aligned && small_keys && vd == d && d == 128) return launch_prefill<128, 128>(ctx, a, batch);
    if (aligned && small_keys && vd == d && d == 64) return launch_prefill<64, 64>(ctx, a, batch);
    if (vd > 256) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention value dimension above 256");
    const uint64_t total = batch * p->seq_len * H;
    if (total / 4 >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention: too many rows");
    mhip::launch(ctx, attn_generic_kernel, dim3(static_cast<unsigned>((total + 3) / 4)), dim3(256),
                 0, a, total);
    return mhip::check_launch("attention (generic)");
}
