/*
 * CPU oracle for the Magnetar MI355X Provider's hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * CPU Provider's (`ReferenceCpuExecutor`, crate `magnetar-provider-cpu`)
 * semantics for the required-now Kernel set, as the reference CUDA Provider
 * documents and mirrors them. Only `tests/`, `__graft_entry__.smoke()` and
 * `bench.py`'s `cpu_baseline` leg may load it, and only as the checker or the
 * timed CPU baseline. The product path never calls it.
 *
 * Every function states the reference file:line it follows (paths are into
 * astorise/Magnetar-provider-CUDA). Arithmetic is plain IEEE-754 binary32 in
 * the reference's order: this file is built with -ffp-contract=off and
 * without fast-math so no operation is fused or reassociated.
 *
 * Status codes are the `mhip_status` values of include/magnetar_hip.h.
 */
#ifndef MAGNETAR_ORACLE_H
#define MAGNETAR_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_SHAPE_UNSUPPORTED = 1,
    ORC_EXECUTION_FAILED = 4,
};

/* ---- deterministic generators (reference test fixtures) ---- */
void orc_hashed_values(float* out, uint64_t len, uint64_t seed);
void orc_values(float* out, uint64_t count, uint64_t seed);
void orc_attention_values(float* out, uint64_t len, uint64_t seed);
void orc_uniform(float* out, uint64_t len, uint64_t seed, float lo, float hi);
void orc_normal(float* out, uint64_t len, uint64_t seed, float mean, float std);
void orc_token_ids(float* out, uint64_t len, uint64_t seed, uint64_t vocab);

/* ---- half-precision codec ---- */
float orc_f16_to_f32(uint16_t bits);
float orc_bf16_to_f32(uint16_t bits);
uint16_t orc_f32_to_f16(float value);
uint16_t orc_f32_to_bf16(float value);
void orc_encode_f16(const float* in, uint16_t* out, uint64_t n);
void orc_encode_bf16(const float* in, uint16_t* out, uint64_t n);
void orc_decode_f16(const uint16_t* in, float* out, uint64_t n);
void orc_decode_bf16(const uint16_t* in, float* out, uint64_t n);
/* op: 0 add, 1 mul; dtype: 0 f16, 1 bf16 */
void orc_half_binary(const uint16_t* a, const uint16_t* b, uint16_t* out, uint64_t n,
                     int dtype, int op);

/* ---- f32 elementwise ---- */
void orc_add(const float* a, const float* b, float* out, uint64_t n);
int  orc_bias_add(const float* a, const float* bias, float* out, uint64_t cols, uint64_t n);
void orc_mul(const float* a, const float* b, float* out, uint64_t n);
void orc_mul_scalar(const float* a, const float* b, float* out, uint64_t n);
void orc_silu(const float* x, float* out, uint64_t n);
void orc_silu_mul(const float* gate, const float* up, float* out, uint64_t n);
void orc_scale(const float* x, float* out, float factor, uint64_t n);

/* ---- gather / rows ---- */
int orc_embedding(const float* table, uint64_t vocab, uint64_t dim, const float* ids,
                  uint64_t num_ids, float* out);
int orc_rmsnorm(const float* in, const float* weight, float* out, uint64_t rows,
                uint64_t cols, uint64_t weight_row_stride, float eps);
int orc_softmax_rows(const float* in, float* out, uint64_t rows, uint64_t cols);

/* RoPE per-pair frequency (and amplitude) table; the kernel-side formula. */
typedef struct {
    float base;
    float scale;
    uint64_t dimension;
    uint64_t position_offset;
    uint64_t head_count;
    uint32_t half_split;       /* 0 interleaved (2p, 2p+1), 1 half-split (p, p+half) */
    uint64_t rotated_pairs;    /* pairs >= this keep angle 0 (partial rotary) */
    float banded_factor;       /* 0 disables banded scaling */
    float low_freq_factor;
    float high_freq_factor;
    float original_context_length;
    float yarn_factor;         /* 0 disables YaRN */
    float yarn_low;
    float yarn_high;
    float amplitude;           /* YaRN attention factor, 1 otherwise */
} orc_rope_params;

void orc_rope_frequencies(const orc_rope_params* p, float* freq, float* amp);
int orc_rope(const float* in, float* out, uint64_t rows, uint64_t cols,
             const orc_rope_params* p);

/* ---- matmul ---- */
/* addend_mode: 0 none, 1 row bias [n], 2 full residual [m, n] */
int orc_matmul(const float* a, const float* b, float* out, uint64_t m, uint64_t k,
               uint64_t n, int transpose_a, int transpose_b, const float* addend,
               int addend_mode);
/* Rows [row_begin, row_end) of the plain (untransposed) product only: the
 * bounded CPU-baseline sample. */
void orc_matmul_rows(const float* a, const float* b, float* out, uint64_t row_begin,
                     uint64_t row_end, uint64_t k, uint64_t n);

/* ---- attention ---- */
typedef struct {
    uint64_t seq_len;
    uint64_t kv_rows;          /* rows held by k and v */
    uint64_t kv_seq_len;       /* key_count, <= kv_rows */
    uint64_t head_count;
    uint64_t kv_head_count;
    uint64_t head_dimension;
    uint64_t value_dimension;
    int causal;
    int64_t window_size;       /* -1: no window */
    float scale;               /* <= 0: 1/sqrt(head_dimension) */
} orc_attention_params;

int orc_attention(const float* q, const float* k, const float* v, float* out,
                  const orc_attention_params* p);
/* Heads [head_begin, head_end) only: the bounded CPU-baseline sample. */
int orc_attention_heads(const float* q, const float* k, const float* v, float* out,
                        const orc_attention_params* p, uint64_t head_begin,
                        uint64_t head_end);

/* Greedy next-token selection (src/kernels.cu:1808-1866): the column of the
 * largest score / temperature (score when temperature is 0) among finite
 * scores outside the [start, end) pairs of `ranges`; ties to the lowest
 * column. -1 when none is eligible. Restated as an ascending scan with a
 * strict comparison, not the reference's key encoding. */
int64_t orc_greedy_select(const float* row, uint64_t cols, const uint64_t* ranges,
                          uint32_t range_count, float temperature);

#ifdef __cplusplus
}
#endif
#endif
