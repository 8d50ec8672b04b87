// A Llama-style decoder block chained device-resident over the C ABI's
// Kernels, with an in-place KV cache.
//
// The reference composes this chain in the Runtime (no single function;
// closest: src/tests_hardware_hot_path.rs:339-526 and
// benches/kernel_chaining.rs:59-89): embedding -> rmsnorm -> Q/K/V matmuls ->
// rope (Q with H heads, K with Hkv heads) -> causal attention -> output matmul
// + residual -> rmsnorm -> gate/up matmuls -> silu * up -> down matmul +
// residual. Decode appends K/V rows at `position` (`kv-write`,
// src/kernels.rs:2278-2325) and attends to `position + seq` keys
// (`key_count`). Here the K and V projections are written straight into
// their cache rows and rotated in place, so the append costs no copy, and the
// residual adds ride in the matmul epilogues (matmul-residual, bit-identical
// to matmul + add). For decode (up to 8 rows, or up to 32 in blocks of 8 when
// the products are small) the Q/K/V and gate/up projections each run as one
// fused GEMV set whose reduction applies RoPE or silu * up, and the embedding
// row is normalised as it is gathered; for one token the attention merge and
// the FFN RMSNorm also ride in the GEMV launches that consume them. Every
// fusion is bit-identical to the separate calls. All launches go on the
// context's stream; nothing waits.
#include <cstring>
#include <string>

#include "internal.hpp"
#include "magnetar_hip.h"

namespace {

struct Layout {
    uint64_t x, h, q, a, x2, h2, g, u, css;  // float offsets into the workspace
    uint64_t floats;
};

Layout layout(const mhip_block_config& c, uint64_t seq) {
    Layout l{};
    uint64_t off = 0;
    auto take = [&](uint64_t n) {
        uint64_t at = off;
        off += (n + 63) / 64 * 64;  // 256-byte aligned slices
        return at;
    };
    l.x = take(seq * c.hidden);
    l.h = take(seq * c.hidden);
    l.q = take(seq * c.heads * c.head_dim);
    l.a = take(seq * c.heads * c.head_dim);
    l.x2 = take(seq * c.hidden);
    l.h2 = take(seq * c.hidden);
    l.g = take(seq * c.ffn);
    l.u = take(seq * c.ffn);
    l.css = take((c.hidden + 255) / 256);  // one token's RMSNorm chunk sums
    l.floats = off;
    return l;
}

}  // namespace

extern "C" {

uint64_t mhip_block_workspace_bytes(const mhip_block_config* cfg, uint64_t seq) {
    if (!cfg) return 0;
    return layout(*cfg, seq).floats * sizeof(float);
}

mhip_status mhip_block_forward(mhip_ctx* ctx, const mhip_block_config* cfg,
                               const mhip_block_weights* w, const float* ids, uint64_t seq,
                               uint64_t position, float* k_cache, float* v_cache,
                               uint64_t cache_rows, void* workspace, uint64_t workspace_bytes,
                               float* out) {
    if (!ctx) return MHIP_DEVICE_UNAVAILABLE;
    if (!cfg || !w || !ids || !k_cache || !v_cache || !workspace || !out)
        return MHIP_SHAPE_UNSUPPORTED;
    const mhip_block_config& c = *cfg;
    if (c.heads == 0 || c.kv_heads == 0 || c.heads % c.kv_heads != 0 || c.head_dim == 0 ||
        c.heads * c.head_dim != c.hidden || seq == 0 || position + seq > cache_rows)
        return MHIP_SHAPE_UNSUPPORTED;
    const Layout l = layout(c, seq);
    if (workspace_bytes < l.floats * sizeof(float)) return MHIP_SHAPE_UNSUPPORTED;
    float* ws = static_cast<float*>(workspace);
    float *x = ws + l.x, *h = ws + l.h, *q = ws + l.q, *a = ws + l.a, *x2 = ws + l.x2,
          *h2 = ws + l.h2, *g = ws + l.g, *u = ws + l.u, *css = ws + l.css;
    const uint64_t kv_dim = c.kv_heads * c.head_dim;
    float* k_rows = k_cache + position * kv_dim;
    float* v_rows = v_cache + position * kv_dim;
    if (c.weight_format != MHIP_WEIGHTS_F32 && c.weight_format != MHIP_WEIGHTS_BF16)
        return MHIP_DTYPE_UNSUPPORTED;
    const bool bf16 = c.weight_format == MHIP_WEIGHTS_BF16;
    // A weight matrix product, f32 or compact bf16 weights.
    auto mm = [&](const float* lhs, const float* weight, float* dst, uint64_t m, uint64_t k,
                  uint64_t n, const float* addend, int mode) {
        return bf16 ? mhip_matmul_bf16w_f32(ctx, lhs, reinterpret_cast<const uint16_t*>(weight),
                                            dst, m, k, n, 0, 0, addend, mode)
                    : mhip_matmul_f32(ctx, lhs, weight, dst, m, k, n, 0, 0, addend, mode);
    };
    mhip_status st;
#define MHIP_TRY(call)                 \
    do {                               \
        if ((st = (call)) != MHIP_OK) \
            return st;                 \
    } while (0)
    mhip_rope_params rope[2];
    mhip_rope_params_default(&rope[0], c.head_dim, c.heads);
    rope[0].base = c.rope_base;
    rope[0].position_offset = position;
    rope[1] = rope[0];
    rope[1].head_count = c.kv_heads;
    // Decode (a few rows, or a few blocks of 8 rows of a small block): Q, K, V
    // as one set of GEMVs with RoPE applied where
    // their split-k sums are added. Otherwise three matmuls and two RoPE calls.
    // In a captured step whose row offset advances, the K/V rows written
    // follow the replay offset (the rows left below them bound it).
    const uint64_t rows_left = cache_rows - (position + seq);
    mhip::GemvTarget qkv[3] = {{w->wq, c.heads * c.head_dim, q},
                               {w->wk, kv_dim, k_rows, true, rows_left},
                               {w->wv, kv_dim, v_rows, true, rows_left}};
    // Embedding + RMSNorm in one pass where the row fits the fused kernel.
    st = mhip::embed_rmsnorm_f32(ctx, w->embedding, c.vocab, c.hidden, ids, seq, w->attn_norm,
                                 c.eps, x, h, bf16);
    if (st == MHIP_LAYOUT_UNSUPPORTED) {
        MHIP_TRY(bf16 ? mhip_embedding_bf16w_f32(ctx, reinterpret_cast<const uint16_t*>(w->embedding),
                                                 c.vocab, c.hidden, ids, seq, x)
                      : mhip_embedding_f32(ctx, w->embedding, c.vocab, c.hidden, ids, seq, x));
        MHIP_TRY(mhip_rmsnorm_f32(ctx, x, w->attn_norm, h, seq, c.hidden, 0, c.eps));
    } else if (st != MHIP_OK) {
        return st;
    }
    st = mhip::gemv_set_f32(ctx, h, seq, c.hidden, qkv, 3, mhip::kGemvRopeQK, rope, bf16);
    if (st == MHIP_LAYOUT_UNSUPPORTED) {
        // The separate matmuls write fixed rows of the cache.
        if (mhip::capture_advancing(ctx) & MHIP_ADVANCE_ROW_OFFSET)
            return mhip::forbid_in_capture(ctx, "a K/V append that the fused projections cannot take with an advancing row offset");
        MHIP_TRY(mm(h, w->wq, q, seq, c.hidden, c.heads * c.head_dim, nullptr, 0));
        MHIP_TRY(mm(h, w->wk, k_rows, seq, c.hidden, kv_dim, nullptr, 0));
        MHIP_TRY(mm(h, w->wv, v_rows, seq, c.hidden, kv_dim, nullptr, 0));
        MHIP_TRY(mhip_rope_f32(ctx, q, q, seq, c.heads * c.head_dim, &rope[0]));
        MHIP_TRY(mhip_rope_f32(ctx, k_rows, k_rows, seq, kv_dim, &rope[1]));
    } else if (st != MHIP_OK) {
        return st;
    }
    mhip_attention_params ap;
    std::memset(&ap, 0, sizeof(ap));
    ap.seq_len = seq;
    ap.kv_rows = cache_rows;
    ap.kv_seq_len = position + seq;
    ap.head_count = c.heads;
    ap.kv_head_count = c.kv_heads;
    ap.head_dimension = c.head_dim;
    ap.value_dimension = c.head_dim;
    ap.causal = 1;
    ap.bounded_key_count = 1;
    ap.window_size = -1;
    ap.batch = 1;
    // One token: attention leaves its key-chunk records and the O
    // projection's partial launch merges them (no merge launch); the O
    // reduction also writes x2's RMSNorm chunk sums, and the gate/up launch
    // normalises x2 from them (no RMSNorm launch). Otherwise attention,
    // matmul-residual and RMSNorm as separate calls.
    bool have_chunks = false;
    if (seq == 1) {
        mhip::DecodeChunks rec;
        rec.extra_bytes = mhip::gemv_merge_bytes(ctx, c.heads, c.head_dim, c.hidden, w->wo, x2, bf16);
        st = rec.extra_bytes ? mhip::attention_decode_chunks_f32(ctx, q, k_cache, v_cache, &ap, &rec)
                             : MHIP_LAYOUT_UNSUPPORTED;
        if (st == MHIP_OK) {
            // The records are in flight: no fallback from here on.
            MHIP_TRY(mhip::gemv_merge_f32(ctx, rec, w->wo, x2, c.hidden, x, 2, bf16, css));
            have_chunks = true;
        } else if (st != MHIP_LAYOUT_UNSUPPORTED) {
            return st;
        }
    }
    if (!have_chunks) {
        MHIP_TRY(mhip_attention_f32(ctx, q, k_cache, v_cache, a, &ap));
        st = MHIP_LAYOUT_UNSUPPORTED;
        if (seq == 1)
            st = mhip::gemv_chunks_f32(ctx, a, w->wo, x2, c.heads * c.head_dim, c.hidden, x, 2, bf16, css);
        if (st == MHIP_LAYOUT_UNSUPPORTED)
            MHIP_TRY(mm(a, w->wo, x2, seq, c.heads * c.head_dim, c.hidden, x, 2));
        else if (st != MHIP_OK)
            return st;
        have_chunks = st == MHIP_OK && seq == 1;
    }
    // Decode (as for Q/K/V): gate and up as one set of GEMVs whose reduction writes
    // silu(gate) * up. Otherwise the gate matmul, then the up matmul with
    // silu(gate) applied to each finished sum.
    const mhip::GemvTarget gate_up[2] = {{w->w_gate, c.ffn, g}, {w->w_up, c.ffn, nullptr}};
    st = MHIP_LAYOUT_UNSUPPORTED;
    if (have_chunks) {
        mhip::RowNorm n{};
        n.src = x2;
        n.chunk_ss = css;
        n.gain = w->ffn_norm;
        n.eps = c.eps;
        st = mhip::gemv_set_f32(ctx, nullptr, 1, c.hidden, gate_up, 2, mhip::kGemvSiluMul, nullptr,
                                bf16, &n);
        if (st != MHIP_OK && st != MHIP_LAYOUT_UNSUPPORTED) return st;
    }
    if (st == MHIP_LAYOUT_UNSUPPORTED) {
        MHIP_TRY(mhip_rmsnorm_f32(ctx, x2, w->ffn_norm, h2, seq, c.hidden, 0, c.eps));
        st = mhip::gemv_set_f32(ctx, h2, seq, c.hidden, gate_up, 2, mhip::kGemvSiluMul, nullptr, bf16);
    }
    if (st == MHIP_LAYOUT_UNSUPPORTED) {
        // The gate product, then the up product gated by it as it is
        // stored (the bits of the two products and silu-mul).
        MHIP_TRY(mm(h2, w->w_gate, u, seq, c.hidden, c.ffn, nullptr, 0));
        MHIP_TRY(mhip::matmul_gated_f32(ctx, h2, w->w_up, bf16, g, seq, c.hidden, c.ffn, false,
                                        false, u));
    } else if (st != MHIP_OK) {
        return st;
    }
    MHIP_TRY(mm(g, w->w_down, out, seq, c.ffn, c.hidden, x2, 2));
#undef MHIP_TRY
    return MHIP_OK;
}

}  // extern "C"
