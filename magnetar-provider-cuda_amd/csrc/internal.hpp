// Fused entry points used inside the library (the decoder block), not part
// of the C ABI. Host-only declarations: includable from g++-built sources.
//
// Each one computes exactly what the separate ABI calls it replaces compute
// -- same kernels' arithmetic, same split-k slicing, same summation order --
// so a chain that uses them is bit-identical to the unfused chain; only the
// launches (and the intermediate HBM round trips) go away.
#pragma once

#include <cstdint>

#include "magnetar_hip.h"

namespace mhip {

// out = mhip_embedding_f32(table, ids) and h = mhip_rmsnorm_f32(out, weight,
// eps) in one launch: the table row is read once, normalised from registers
// and written to both. An invalid id raises MHIP_FLAG_EMBEDDING_INVALID_ID
// and leaves that row of both outputs unwritten, as the embedding does.
// Requires dim % 4 == 0, 16-byte aligned buffers and dim <= 16384; returns
// MHIP_LAYOUT_UNSUPPORTED otherwise (the caller then runs the two calls).
// `table` is f32, or bf16 bit patterns when `bf16_table`.
mhip_status embed_rmsnorm_f32(mhip_ctx* ctx, const void* table, uint64_t vocab, uint64_t dim,
                              const float* ids, uint64_t rows, const float* weight, float eps,
                              float* out, float* h, bool bf16_table = false);

// One decode projection: out[rows, n] = a[rows, k] . b[k, n]; b is f32, or
// bf16 bit patterns when the set's weights are compact.
struct GemvTarget {
    const void* b;
    uint64_t n;
    float* out;
    // While capturing with MHIP_ADVANCE_ROW_OFFSET: the rows written move
    // down by the replay offset (a KV cache append), by at most this many.
    bool row_advances = false;
    uint64_t row_advance_limit = 0;
};

// Epilogues applied where the split-k partial sums are added up.
enum GemvEpilogue : int {
    kGemvPlain = 0,    // every target stored as is
    kGemvRopeQK = 1,   // targets 0 and 1 rotated by `rope[0]`, `rope[1]` (Q, K); 2 plain (V)
    kGemvSiluMul = 2,  // targets[0].out = silu(a.b0) * (a.b1); b0, b1 of equal shape
};

// Up to three projections of the same input `a` (rows <= 8) in two
// launches: one over every target's k-slices, one that adds each target's
// slices and applies the epilogue. Equal to mhip_matmul_f32 per target
// followed by mhip_rope_f32 / mhip_silu_mul_f32, bit for bit. Returns
// MHIP_LAYOUT_UNSUPPORTED when a target does not fit the decode GEMV
// (n % 4, alignment, rows > 8) or the rope parameters are not the vector
// interleaved form; the caller then runs the separate calls.
//
// With `norm` (one row only), the input is not `a` but the row norm.src
// normalised inside the partial launch: times its RMSNorm scale (from the
// row's chunk sums of squares, norm.chunk_ss, as gemv_chunks_f32 writes them)
// and gain -- the bits of mhip_rmsnorm_f32 followed by the set.
struct RowNorm {
    const float* src;
    const float* chunk_ss;
    const float* gain = nullptr;
    float eps = 0.0f;
};
mhip_status gemv_set_f32(mhip_ctx* ctx, const float* a, uint64_t rows, uint64_t k,
                         const GemvTarget* targets, int count, int epilogue,
                         const mhip_rope_params* rope, bool bf16_weights = false,
                         const RowNorm* norm = nullptr);

// out[m, n] = silu(gate) * (a . b): mhip_matmul_f32 (or the compact-weight
// matmul, `bf16`) with the gate applied to each finished sum, equal to the
// product followed by mhip_silu_mul_f32(gate, product) bit for bit. gate is
// [m, n] (the gate product); out must not overlap it.
mhip_status matmul_gated_f32(mhip_ctx* ctx, const float* a, const void* b, bool bf16, float* out,
                             uint64_t m, uint64_t k, uint64_t n, bool transpose_a,
                             bool transpose_b, const float* gate);

// out[1, n] = a[1, k] . b[k, n] (+ addend as mhip_matmul_f32's addend_mode),
// exactly the one-row decode GEMV of mhip_matmul_f32 (b f32, or bf16 bits
// when `bf16_weights`), that also writes the RMSNorm chunk sums of squares of
// `out` (mhip::chunk_sumsq; ceil(n / 256) floats) to chunk_ss. Returns
// MHIP_LAYOUT_UNSUPPORTED when that GEMV would not split k (the chunk sums
// come from its reduction launch) or the operands do not fit it.
mhip_status gemv_chunks_f32(mhip_ctx* ctx, const float* a, const void* b, float* out, uint64_t k,
                            uint64_t n, const float* addend, int addend_mode, bool bf16_weights,
                            float* chunk_ss);

// Single-query decode attention (mhip_attention_f32 with seq_len 1, batch 1)
// launched without its merge: the key-chunk records are left in the
// context's workspace for a consumer that merges them itself, followed by
// `extra_bytes` of workspace for that consumer (`extra`). Returns
// MHIP_LAYOUT_UNSUPPORTED, with nothing launched, for any call that
// mhip_attention_f32 would not run on its split-KV decode kernels.
struct DecodeChunks {
    size_t extra_bytes = 0;   // in
    const float* part_o = nullptr;   // [heads][chunks][d]: chunk outputs
    const float* part_ml = nullptr;  // [heads][chunks][2]: chunk max and weight sum
    uint64_t chunks = 0, heads = 0, d = 0;
    float* extra = nullptr;
};
mhip_status attention_decode_chunks_f32(mhip_ctx* ctx, const float* q, const float* k,
                                        const float* v, const mhip_attention_params* p,
                                        DecodeChunks* out);

// The output projection of one decode token over attention's chunk records:
// out[n] = merge(records)[k] . b[k, n] (+ addend), k = heads * d, with the
// merge done inside the GEMV's partial launch (each workgroup merges its k
// slice of one head) instead of a merge launch. Bit-identical to
// mhip_attention_f32 followed by gemv_chunks_f32 (whose chunk sums it also
// writes). gemv_merge_bytes gives the workspace it needs (the records'
// `extra`), or 0 when the shapes do not fit: a k slice must lie within one
// head (the GEMV's slice length divides d), the GEMV must split k, and `b`
// and `out` must be aligned for it.
size_t gemv_merge_bytes(mhip_ctx* ctx, uint64_t heads, uint64_t d, uint64_t n, const void* b,
                        const float* out, bool bf16_weights);
mhip_status gemv_merge_f32(mhip_ctx* ctx, const DecodeChunks& records, const void* b, float* out,
                           uint64_t n, const float* addend, int addend_mode, bool bf16_weights,
                           float* chunk_ss);

// While capturing: records that `what` cannot be captured and returns
// MHIP_CAPTURE_UNSUPPORTED; MHIP_OK otherwise.
mhip_status forbid_in_capture(mhip_ctx* ctx, const char* what);

// The MHIP_ADVANCE_* bits of the capture in progress (0 when not capturing).
uint32_t capture_advancing(const mhip_ctx* ctx);

}  // namespace mhip
