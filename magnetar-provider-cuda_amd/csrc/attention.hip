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
//    admitted keys in 32-key tiles staged in LDS (double-buffered through
//    registers). Each wave computes S^T = K . Q^T with v_mfma_f32_32x32x2_f32
//    (Q^T lives in registers, pre-scaled by scale * log2 e), so every lane
//    owns one query column and 16 of the tile's keys: the online-softmax
//    max/sum need one exchange with lane l ^ 32. The accumulator registers
//    are then exactly the B operand of O^T = V^T . P^T, so the output stays
//    per-lane too. Probabilities are normalised per tile and the running
//    output rescaled, so it is always a convex combination of V rows and
//    never overflows (the reference's 1e38 known answer,
//    src/tests_conformance.rs:2215-2312).
//  - decode (one query row, any head dim that is a multiple of 4 up to 256):
//    split-KV. A workgroup takes one (batch, KV head, key chunk) and all the
//    query heads that share that KV head, streams K and V once with dwordx4
//    loads, and writes the chunk's normalised output, max and weight sum; a
//    second kernel merges chunks in chunk order (deterministic).
//  - a generic kernel (any other shape): one wave per (query, head), online
//    softmax over 64-key chunks.
#include "common.hpp"

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
};

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
    static constexpr int kBQ = 128;            // queries per workgroup (4 waves x 32)
    static constexpr int kBKV = 32;            // keys per tile
    static constexpr int kSK = D + 4;          // LDS row stride of K (dwordx4 aligned)
    static constexpr int kSV = VD + 4;
    static constexpr int kTile = kBKV * kSK + kBKV * kSV;
    static constexpr int kLdsFloats = 2 * kTile;
    static constexpr int kKChunks = kBKV * D / 4 / 256;   // dwordx4 per thread
    static constexpr int kVChunks = kBKV * VD / 4 / 256;
    static_assert(kBKV * D % 1024 == 0 && kBKV * VD % 1024 == 0, "tile must split over 256 threads");
};

template <int D, int VD>
__global__ __launch_bounds__(256, (D > 64 ? 1 : 2)) void attn_prefill_kernel(AttnArgs a) {
    using Cfg = PrefillCfg<D, VD>;
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, half = lane >> 5;

    // Heaviest (latest) query tiles first: under a causal mask they see the most keys.
    const uint64_t qtiles = (a.seq + Cfg::kBQ - 1) / Cfg::kBQ;
    const uint64_t bid = blockIdx.x;
    const uint64_t qt = qtiles - 1 - bid % qtiles;
    const uint64_t bh = bid / qtiles;
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

    // Key range of the whole workgroup and of this wave (for skipping tiles).
    const uint64_t q_last = min(a.seq, q_first + Cfg::kBQ) - 1;
    uint64_t blk_lo, blk_hi, tmp;
    key_range(a, a.offset + q_first, &blk_lo, &tmp);
    key_range(a, a.offset + q_last, &tmp, &blk_hi);
    const uint64_t w_first = q_first + wave * 32;
    const uint64_t w_last = min(a.seq, w_first + 32);
    uint64_t wave_lo = 0, wave_hi = 0;
    if (w_first < a.seq) {
        key_range(a, a.offset + w_first, &wave_lo, &tmp);
        key_range(a, a.offset + w_last - 1, &tmp, &wave_hi);
    }
    const uint64_t tile_begin = blk_lo / Cfg::kBKV * Cfg::kBKV;

    float m = -INFINITY, l = 0.0f;
    v16f o[VD / 32];
#pragma unroll
    for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[vb][r] = 0.0f;

    float4 rk[Cfg::kKChunks], rv[Cfg::kVChunks];
    auto load = [&](uint64_t k0) {
#pragma unroll
        for (int i = 0; i < Cfg::kKChunks; ++i) {
            const int c = threadIdx.x + i * 256;
            const int row = c / (D / 4), col = (c % (D / 4)) * 4;
            const uint64_t key = k0 + row;
            rk[i] = key < a.kv_seq ? *reinterpret_cast<const float4*>(K + key * k_ld + col)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < Cfg::kVChunks; ++i) {
            const int c = threadIdx.x + i * 256;
            const int row = c / (VD / 4), col = (c % (VD / 4)) * 4;
            const uint64_t key = k0 + row;
            rv[i] = key < a.kv_seq ? *reinterpret_cast<const float4*>(V + key * v_ld + col)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store = [&](int buf) {
        float* sk = lds + buf * Cfg::kTile;
        float* sv = sk + Cfg::kBKV * Cfg::kSK;
#pragma unroll
        for (int i = 0; i < Cfg::kKChunks; ++i) {
            const int c = threadIdx.x + i * 256;
            *reinterpret_cast<float4*>(sk + (c / (D / 4)) * Cfg::kSK + (c % (D / 4)) * 4) = rk[i];
        }
#pragma unroll
        for (int i = 0; i < Cfg::kVChunks; ++i) {
            const int c = threadIdx.x + i * 256;
            *reinterpret_cast<float4*>(sv + (c / (VD / 4)) * Cfg::kSV + (c % (VD / 4)) * 4) = rv[i];
        }
    };

    if (tile_begin < blk_hi) {
        load(tile_begin);
        store(0);
    }
    __syncthreads();
    int buf = 0;
    for (uint64_t k0 = tile_begin; k0 < blk_hi; k0 += Cfg::kBKV, buf ^= 1) {
        const bool more = k0 + Cfg::kBKV < blk_hi;
        if (more) load(k0 + Cfg::kBKV);
        if (k0 < wave_hi && k0 + Cfg::kBKV > wave_lo) {
            const float* sk = lds + buf * Cfg::kTile;
            const float* sv = sk + Cfg::kBKV * Cfg::kSK;
            // S^T[key][query] for the tile: A = K rows (lane -> key l32), B = Q^T.
            v16f s;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.0f;
            const float* krow = sk + l32 * Cfg::kSK + half * (D / 2);
#pragma unroll
            for (int t = 0; t < D / 2; t += 4) {
                const float4 kv = *reinterpret_cast<const float4*>(krow + t);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[t], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[t + 1], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[t + 2], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[t + 3], s, 0, 0, 0);
            }
            // Register r holds key k0 + 8*(r/4) + 4*half + r%4 of query q.
            float tile_max = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint64_t key = k0 + 8 * (r / 4) + 4 * half + (r % 4);
                const bool ok = q_live && key >= q_lo && key < q_hi;
                s[r] = ok ? s[r] : -INFINITY;
                tile_max = fmaxf(tile_max, s[r]);
            }
            tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32, 64));
            // Every lane runs the update (the MFMAs below need the whole wave);
            // a query with no admitted key yet keeps m = -inf, l = 0, o = 0.
            const float m_new = fmaxf(m, tile_max);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = exp2f(m - m_use);
            float psum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = exp2f(s[r] - m_use);
                psum += s[r];
            }
            psum += __shfl_xor(psum, 32, 64);
            const float l_new = l * alpha + psum;
            const float inv = l_new > 0.0f ? 1.0f / l_new : 0.0f;
            // A tile that adds nothing for this query leaves its output as it was.
            const float keep = (psum == 0.0f && alpha == 1.0f) || l_new == 0.0f ? 1.0f : (l * alpha) * inv;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] *= inv;
#pragma unroll
            for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[vb][r] *= keep;
            // O^T += V^T . P^T: step t pairs key 8*(t/4) + 4*half + t%4 with register t.
#pragma unroll
            for (int vb = 0; vb < VD / 32; ++vb) {
                const float* vcol = sv + vb * 32 + l32;
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const int key = 8 * (t / 4) + 4 * half + (t % 4);
                    o[vb] = __builtin_amdgcn_mfma_f32_32x32x2f32(vcol[key * Cfg::kSV], s[t],
                                                                o[vb], 0, 0, 0);
                }
            }
            m = m_new;
            l = l_new;
        }
        if (more) store(buf ^ 1);
        __syncthreads();
    }

    // Register r of block vb holds O[q][vb*32 + 8*(r/4) + 4*half + r%4].
    if (q_live) {
        float* orow = O + q * o_ld;
#pragma unroll
        for (int vb = 0; vb < VD / 32; ++vb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(orow + vb * 32 + 8 * g + 4 * half) =
                    make_float4(o[vb][4 * g], o[vb][4 * g + 1], o[vb][4 * g + 2], o[vb][4 * g + 3]);
    }
}

template <int D, int VD>
mhip_status launch_prefill(mhip_ctx* ctx, const AttnArgs& a, uint64_t batch) {
    using Cfg = PrefillCfg<D, VD>;
    const uint64_t blocks = batch * a.heads * ((a.seq + Cfg::kBQ - 1) / Cfg::kBQ);
    if (blocks >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention: too many query tiles");
    const size_t lds = Cfg::kLdsFloats * sizeof(float);
    static bool configured = false;
    if (!configured) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_prefill_kernel<D, VD>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        configured = true;
    }
    hipLaunchKernelGGL((attn_prefill_kernel<D, VD>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), lds, ctx->stream, a);
    return mhip::check_launch("attention (MFMA prefill)");
}

// ---------------------------------------------------------------------------
// Decode: split-KV over key chunks, all query heads of a KV head together
// ---------------------------------------------------------------------------

constexpr int kMaxGroup = 8;

// Partial record per (batch, head, chunk): [0..vd) normalised output, then max, sum.
template <int D4>  // D / 4: lanes per key row
__global__ __launch_bounds__(256) void attn_decode_partial_kernel(AttnArgs a, uint64_t chunk,
                                                                  uint64_t chunks,
                                                                  float* __restrict__ part) {
    constexpr int kLPK = D4;            // lanes per key
    constexpr int kKPS = 64 / kLPK;     // keys per wave step
    constexpr int D = 4 * D4;
    extern __shared__ float lds[];      // q [G][D], scores [G][chunk], red [4*kKPS][G][D]
    const uint64_t group = a.heads / a.kv_heads;
    const uint64_t c_idx = blockIdx.x % chunks;
    const uint64_t bkv = blockIdx.x / chunks;
    const uint64_t kvh = bkv % a.kv_heads, b = bkv / a.kv_heads;
    const uint64_t k_begin = c_idx * chunk;
    const uint64_t k_end = min(a.kv_seq, k_begin + chunk);
    const uint64_t qpos = a.offset;  // the one query row: seq == 1
    uint64_t lo, hi;
    key_range(a, qpos, &lo, &hi);
    const uint64_t c_lo = max(lo, k_begin), c_hi = min(hi, k_end);
    const int n = c_lo < c_hi ? static_cast<int>(c_hi - c_lo) : 0;

    float* sq = lds;                                   // [group][D]
    float* ss = lds + group * D;                       // [group][chunk]
    float* sred = ss + group * chunk;                  // [4*kKPS][group][D]
    const float* Qb = a.q + b * a.q_bs;
    for (uint64_t i = threadIdx.x; i < group * D; i += 256) {
        const uint64_t g = i / D, t = i % D;
        sq[i] = Qb[(kvh * group + g) * D + t] * a.qscale;
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / kLPK, sl = lane % kLPK;
    const float* K = a.k + b * a.k_bs + kvh * D;
    const float* V = a.v + b * a.v_bs + kvh * D;
    const uint64_t k_ld = a.kv_heads * D;

    // Scores: key j of the chunk handled by (wave, sub) = j % (4*kKPS).
    for (int j0 = 0; j0 < n; j0 += 4 * kKPS) {
        const int j = j0 + wave * kKPS + sub;
        float4 kv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j < n) kv = *reinterpret_cast<const float4*>(K + (c_lo + j) * k_ld + 4 * sl);
        for (uint64_t g = 0; g < group; ++g) {
            const float4 qv = *reinterpret_cast<const float4*>(sq + g * D + 4 * sl);
            float dot = kv.x * qv.x + kv.y * qv.y + kv.z * qv.z + kv.w * qv.w;
#pragma unroll
            for (int off = kLPK / 2; off >= 1; off >>= 1) dot += __shfl_xor(dot, off, 64);
            if (sl == 0 && j < n) ss[g * chunk + j] = dot;
        }
    }
    __syncthreads();
    // Per head: max and weight sum over the chunk (one wave per head).
    __shared__ float stat_m[kMaxGroup], stat_l[kMaxGroup];
    for (uint64_t g = wave; g < group; g += 4) {
        float mx = -INFINITY;
        for (int j = lane; j < n; j += 64) mx = fmaxf(mx, ss[g * chunk + j]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float sum = 0.0f;
        for (int j = lane; j < n; j += 64) {
            const float p = exp2f(ss[g * chunk + j] - mx);
            ss[g * chunk + j] = p;
            sum += p;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int j = lane; j < n; j += 64) ss[g * chunk + j] *= inv;
        if (lane == 0) {
            stat_m[g] = mx;
            stat_l[g] = sum;
        }
    }
    __syncthreads();
    // Weighted mean of V rows: lane sl owns columns [4sl, 4sl+4).
    float4 acc[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j0 = 0; j0 < n; j0 += 4 * kKPS) {
        const int j = j0 + wave * kKPS + sub;
        if (j < n) {
            const float4 vv = *reinterpret_cast<const float4*>(V + (c_lo + j) * k_ld + 4 * sl);
#pragma unroll
            for (int g = 0; g < kMaxGroup; ++g) {
                if (g < static_cast<int>(group)) {
                    const float p = ss[g * chunk + j];
                    acc[g].x += p * vv.x;
                    acc[g].y += p * vv.y;
                    acc[g].z += p * vv.z;
                    acc[g].w += p * vv.w;
                }
            }
        }
    }
    const int slot = wave * kKPS + sub;
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
        if (g < static_cast<int>(group))
            *reinterpret_cast<float4*>(sred + (slot * group + g) * D + 4 * sl) = acc[g];
    __syncthreads();
    const uint64_t rec = D + 2;
    for (uint64_t i = threadIdx.x; i < group * D; i += 256) {
        const uint64_t g = i / D, t = i % D;
        float v = 0.0f;
        for (int s2 = 0; s2 < 4 * kKPS; ++s2) v += sred[(s2 * group + g) * D + t];
        float* dst = part + (((b * a.heads) + kvh * group + g) * chunks + c_idx) * rec;
        dst[t] = v;
        if (t == 0) {
            dst[D] = stat_m[g];
            dst[D + 1] = stat_l[g];
        }
    }
}

// Merges the chunk records of one (batch, head) in chunk order.
__global__ __launch_bounds__(256) void attn_decode_combine_kernel(AttnArgs a, uint64_t chunks,
                                                                  const float* __restrict__ part) {
    const uint64_t bh = blockIdx.x;
    const uint64_t head = bh % a.heads, b = bh / a.heads;
    const uint64_t D = a.vd, rec = D + 2;
    const float* p = part + bh * chunks * rec;
    float mx = -INFINITY;
    for (uint64_t c = 0; c < chunks; ++c) mx = fmaxf(mx, p[c * rec + D]);
    float total = 0.0f;
    if (mx != -INFINITY)
        for (uint64_t c = 0; c < chunks; ++c) total += p[c * rec + D + 1] * exp2f(p[c * rec + D] - mx);
    float* orow = a.out + b * a.o_bs + head * D;
    for (uint64_t t = threadIdx.x; t < D; t += 256) {
        float v = 0.0f;
        if (total > 0.0f) {
            for (uint64_t c = 0; c < chunks; ++c) {
                const float w = p[c * rec + D + 1] * exp2f(p[c * rec + D] - mx) / total;
                if (w > 0.0f) v += w * p[c * rec + t];
            }
        }
        orow[t] = v;
    }
}

template <int D4>
mhip_status launch_decode(mhip_ctx* ctx, const AttnArgs& a, uint64_t batch) {
    constexpr int D = 4 * D4;
    const uint64_t group = a.heads / a.kv_heads;
    const uint64_t units = batch * a.kv_heads;
    const uint64_t target = static_cast<uint64_t>(ctx->compute_units ? ctx->compute_units : 256) * 4;
    uint64_t chunks = (target + units - 1) / units;
    uint64_t chunk = (a.kv_seq + chunks - 1) / chunks;
    chunk = (chunk + 63) / 64 * 64;
    if (chunk < 64) chunk = 64;
    // Keep scores + reduction scratch within 64 KiB of LDS.
    const uint64_t red = static_cast<uint64_t>(4 * (64 / D4)) * group * D;
    while (chunk > 64 && (group * D + group * chunk + red) * 4 > 65536) chunk -= 64;
    if ((group * D + group * chunk + red) * 4 > 65536) return MHIP_CAPTURE_UNSUPPORTED;  // caller falls back
    chunks = (a.kv_seq + chunk - 1) / chunk;
    if (chunks == 0) chunks = 1;
    const uint64_t rec = D + 2;
    const size_t bytes = batch * a.heads * chunks * rec * sizeof(float);
    if (ctx->workspace_bytes < bytes) {
        if (ctx->workspace) {
            (void)hipStreamSynchronize(ctx->stream);
            (void)hipFree(ctx->workspace);
            ctx->workspace = nullptr;
            ctx->workspace_bytes = 0;
        }
        hipError_t err = hipMalloc(&ctx->workspace, bytes);
        if (err != hipSuccess) return mhip::from_hip(err, "allocating the attention workspace");
        ctx->workspace_bytes = bytes;
    }
    float* part = static_cast<float*>(ctx->workspace);
    const size_t lds = (group * D + group * chunk + red) * sizeof(float);
    hipLaunchKernelGGL(attn_decode_partial_kernel<D4>, dim3(static_cast<unsigned>(units * chunks)),
                       dim3(256), lds, ctx->stream, a, chunk, chunks, part);
    mhip_status st = mhip::check_launch("attention (decode chunks)");
    if (st != MHIP_OK) return st;
    hipLaunchKernelGGL(attn_decode_combine_kernel, dim3(static_cast<unsigned>(batch * a.heads)),
                       dim3(256), 0, ctx->stream, a, chunks, part);
    return mhip::check_launch("attention (decode combine)");
}

// ---------------------------------------------------------------------------
// Generic: one wave per (batch, query, head)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void attn_generic_kernel(AttnArgs a, uint64_t total) {
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

extern "C" mhip_status mhip_attention_f32(mhip_ctx* ctx, const float* q, const float* k,
                                          const float* v, float* out,
                                          const mhip_attention_params* p) {
    MHIP_REQUIRE_CTX(ctx);
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
    if (p->seq_len == 0) return MHIP_OK;
    if (!q || !k || !v || !out) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention: null buffer");

    AttnArgs a;
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
    a.q_bs = p->q_batch_stride ? p->q_batch_stride : p->seq_len * H * d;
    a.k_bs = p->kv_batch_stride ? p->kv_batch_stride : p->kv_rows * Hkv * d;
    a.v_bs = p->v_batch_stride ? p->v_batch_stride : p->kv_rows * Hkv * vd;
    a.o_bs = p->out_batch_stride ? p->out_batch_stride : p->seq_len * H * vd;

    const bool aligned = mhip::aligned16(q) && mhip::aligned16(k) && mhip::aligned16(v) &&
                         mhip::aligned16(out) && a.q_bs % 4 == 0 && a.k_bs % 4 == 0 &&
                         a.v_bs % 4 == 0 && a.o_bs % 4 == 0;
    if (aligned && p->seq_len == 1 && vd == d && d % 4 == 0 && d <= 256 && H / Hkv <= kMaxGroup &&
        p->kv_seq_len > 0) {
        mhip_status st = MHIP_CAPTURE_UNSUPPORTED;
        switch (d / 4) {
            case 1: st = launch_decode<1>(ctx, a, batch); break;
            case 2: st = launch_decode<2>(ctx, a, batch); break;
            case 4: st = launch_decode<4>(ctx, a, batch); break;
            case 8: st = launch_decode<8>(ctx, a, batch); break;
            case 16: st = launch_decode<16>(ctx, a, batch); break;
            case 32: st = launch_decode<32>(ctx, a, batch); break;
            case 64: st = launch_decode<64>(ctx, a, batch); break;
            default: break;
        }
        if (st != MHIP_CAPTURE_UNSUPPORTED) return st;  // else: no decode kernel fits
    }
    if (aligned && vd == d && d == 128) return launch_prefill<128, 128>(ctx, a, batch);
    if (aligned && vd == d && d == 64) return launch_prefill<64, 64>(ctx, a, batch);
    if (vd > 256) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention value dimension above 256");
    const uint64_t total = batch * p->seq_len * H;
    if (total / 4 >= (1ULL << 31)) return mhip::fail(MHIP_SHAPE_UNSUPPORTED, "attention: too many rows");
    hipLaunchKernelGGL(attn_generic_kernel, dim3(static_cast<unsigned>((total + 3) / 4)), dim3(256),
                       0, ctx->stream, a, total);
    return mhip::check_launch("attention (generic)");
}
