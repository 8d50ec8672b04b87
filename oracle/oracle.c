/*
 * CPU oracle for the Magnetar MI355X Provider's hot path -- TEST
 * INFRASTRUCTURE ONLY (the checker and the timed CPU baseline; never the
 * product). Declarations and the build rules are in oracle.h.
 *
 * Citations are file:line into the reference repository
 * astorise/Magnetar-provider-CUDA. The reference's true oracle,
 * `magnetar_provider_cpu::*` (crate magnetar-provider-cpu 1.0.0, path
 * dependency ../cpu, revision unpinned in Cargo.lock:909-916), is not
 * available; this file restates the semantics the reference's CUDA kernels
 * document as mirroring it, in the order those kernels give ("k ascending",
 * src/kernels.cu:1262-1264; the three-pass attention, src/kernels.cu:1868-1959).
 *
 * Pinning (how each function is checked beyond restating it) lives in
 * tests/test_oracle.py; parity status per function is listed in the header
 * comment of that file.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* Generators                                                              */
/* ---------------------------------------------------------------------- */

/* splitmix64 step, src/tests_conformance.rs:2116-2128. */
static uint64_t splitmix_next(uint64_t* state) {
    *state += 0x9e3779b97f4a7c15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

static uint64_t splitmix_seed(uint64_t seed) {
    return 0x9e3779b97f4a7c15ULL ^ (seed * 0xbf58476d1ce4e5b9ULL);
}

/* `hashed_values`: [-0.5, 0.5) from the top 24 bits, src/tests_conformance.rs:2116-2128. */
void orc_hashed_values(float* out, uint64_t len, uint64_t seed) {
    uint64_t state = splitmix_seed(seed);
    for (uint64_t i = 0; i < len; i++) {
        uint64_t z = splitmix_next(&state);
        out[i] = (float)(z >> 40) / (float)(1ULL << 24) - 0.5f;
    }
}

/* `values`: (((i*7919 + seed*104729) % 2001) - 1000) * 1e-4, src/tests_conformance.rs:298-302. */
void orc_values(float* out, uint64_t count, uint64_t seed) {
    for (uint64_t i = 0; i < count; i++) {
        out[i] = ((float)((i * 7919 + seed * 104729) % 2001) - 1000.0f) * 1e-4f;
    }
}

/* `attention_values`: ((i*7919 + seed*104729) % 2003) / 2003 - 0.5, src/tests_conformance.rs:2131-2135. */
void orc_attention_values(float* out, uint64_t len, uint64_t seed) {
    for (uint64_t i = 0; i < len; i++) {
        out[i] = (float)((i * 7919 + seed * 104729) % 2003) / 2003.0f - 0.5f;
    }
}

/* Benchmark inputs (the BASELINE configs): splitmix64 uniforms on [lo, hi). */
void orc_uniform(float* out, uint64_t len, uint64_t seed, float lo, float hi) {
    uint64_t state = splitmix_seed(seed);
    for (uint64_t i = 0; i < len; i++) {
        double u = (double)(splitmix_next(&state) >> 11) * (1.0 / 9007199254740992.0);
        out[i] = (float)((double)lo + ((double)hi - (double)lo) * u);
    }
}

/* Box-Muller normals over splitmix64 uniforms in (0, 1]. */
void orc_normal(float* out, uint64_t len, uint64_t seed, float mean, float std) {
    uint64_t state = splitmix_seed(seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t i = 0; i < len; i += 2) {
        double u1 = ((double)(splitmix_next(&state) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(splitmix_next(&state) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)((double)mean + (double)std * r * cos(two_pi * u2));
        if (i + 1 < len) {
            out[i + 1] = (float)((double)mean + (double)std * r * sin(two_pi * u2));
        }
    }
}

/* Token ids ~U[0, vocab) stored as f32 (the embedding's id dtype, src/kernels.rs:3833-3840). */
void orc_token_ids(float* out, uint64_t len, uint64_t seed, uint64_t vocab) {
    uint64_t state = splitmix_seed(seed);
    for (uint64_t i = 0; i < len; i++) {
        out[i] = (float)(splitmix_next(&state) % vocab);
    }
}

/* ---------------------------------------------------------------------- */
/* Half-precision codec: src/half_precision.rs:14-125                      */
/* ---------------------------------------------------------------------- */

static inline float bits_to_f32(uint32_t bits) {
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint32_t f32_to_bits(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    return bits;
}

/* Exact binary16 -> binary32, src/half_precision.rs:14-37. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exponent = (h >> 10) & 0x1F;
    uint32_t mantissa = h & 0x3FF;
    uint32_t magnitude;
    if (exponent == 0) {
        if (mantissa == 0) {
            magnitude = 0;
        } else {
            /* Subnormal: normalise the significand. */
            uint32_t shift = 0;
            while ((mantissa & 0x400) == 0) {
                mantissa <<= 1;
                shift++;
            }
            mantissa &= 0x3FF;
            magnitude = ((127 - 15 - shift + 1) << 23) | (mantissa << 13);
        }
    } else if (exponent == 0x1F) {
        magnitude = (0xFFu << 23) | (mantissa << 13);
    } else {
        magnitude = ((exponent - 15 + 127) << 23) | (mantissa << 13);
    }
    return bits_to_f32(sign | magnitude);
}

/* Exact bfloat16 -> binary32, src/half_precision.rs:39-42. */
float orc_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

/* Round-to-nearest-even binary32 -> binary16, src/half_precision.rs:46-108. */
uint16_t orc_f32_to_f16(float value) {
    uint32_t bits = f32_to_bits(value);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    uint32_t mant = bits & 0x007FFFFF;
    int32_t exp32 = (int32_t)((bits >> 23) & 0xFF);
    if (exp32 == 0xFF) {
        if (mant == 0) return sign | 0x7C00;
        uint16_t payload = (uint16_t)(mant >> 13);
        return sign | 0x7C00 | (payload ? payload : 1);
    }
    int32_t unbiased = exp32 - 127;
    if (unbiased > 15) return sign | 0x7C00;
    if (unbiased < -14) {
        uint32_t significand = exp32 == 0 ? mant : (mant | 0x00800000u);
        if (significand == 0) return sign;
        uint32_t shift = (uint32_t)(-(unbiased + 1));
        if (shift >= 32) return sign;
        uint32_t halfway = 1u << (shift - 1);
        uint32_t result = significand >> shift;
        uint32_t rem = significand & ((1u << shift) - 1);
        if (rem > halfway || (rem == halfway && (result & 1u))) result++;
        return sign | (uint16_t)result;
    }
    uint32_t mant10 = mant >> 13;
    uint32_t rem = mant & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (mant10 & 1u))) mant10++;
    uint32_t exp16 = (uint32_t)(unbiased + 15);
    if (mant10 == 0x400) {
        if (exp16 + 1 >= 0x1F) return sign | 0x7C00;
        return sign | (uint16_t)((exp16 + 1) << 10);
    }
    return sign | (uint16_t)((exp16 << 10) | mant10);
}

/* Round-to-nearest-even binary32 -> bfloat16 with the NaN rule, src/half_precision.rs:110-125. */
uint16_t orc_f32_to_bf16(float value) {
    uint32_t bits = f32_to_bits(value);
    if (isnan(value)) {
        uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
        uint16_t mant7 = (uint16_t)((bits >> 16) & 0x7F);
        return sign | 0x7F80 | (mant7 ? mant7 : 0x40);
    }
    uint32_t bias = 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + bias) >> 16);
}

void orc_encode_f16(const float* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}
void orc_encode_bf16(const float* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}
void orc_decode_f16(const uint16_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}
void orc_decode_bf16(const uint16_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}

/* `add_f16_kernel` & co.: decode, one f32 operation, RNE encode,
 * src/kernels.cu:2913-2939; the reference's exact model of it is
 * src/tests_conformance.rs:2334-2347, which computes `op(x, y)` in the host's
 * compiled f32 arithmetic.
 *
 * A NaN result's bits are this build's convention, stated rather than left to
 * the host's ALU: a NaN operand's payload, quieted, the FIRST operand's when
 * both are NaN; a NaN made from non-NaN operands (inf - inf, 0 * inf) is the
 * negative default quiet NaN 0xFFC00000. What the ISA fixes is narrower: with
 * both operands NaN, x86 SSE returns the first SOURCE register's NaN, and which
 * operand a compiler puts there depends on code generation (clang -O2 scalar
 * code, Rust's backend, gives the first operand; gcc -O3 and numpy's vector
 * loops can give the second). The reference's outputs therefore do not pin the
 * survivor of NaN op NaN; the tests accept either operand's quieted payload
 * there and are bit-exact everywhere else. */
static float nan_rule(float x, float y, float r) {
    uint32_t bits;
    if (!isnan(r)) return r;
    if (isnan(x)) memcpy(&bits, &x, 4), bits |= 0x00400000u;
    else if (isnan(y)) memcpy(&bits, &y, 4), bits |= 0x00400000u;
    else bits = 0xFFC00000u;
    memcpy(&r, &bits, 4);
    return r;
}

void orc_half_binary(const uint16_t* a, const uint16_t* b, uint16_t* out, uint64_t n,
                     int dtype, int op) {
    for (uint64_t i = 0; i < n; i++) {
        float x = dtype ? orc_bf16_to_f32(a[i]) : orc_f16_to_f32(a[i]);
        float y = dtype ? orc_bf16_to_f32(b[i]) : orc_f16_to_f32(b[i]);
        float r = nan_rule(x, y, op ? x * y : x + y);
        out[i] = dtype ? orc_f32_to_bf16(r) : orc_f32_to_f16(r);
    }
}

/* ---------------------------------------------------------------------- */
/* f32 elementwise                                                         */
/* ---------------------------------------------------------------------- */

/* `add_kernel`, src/kernels.cu:30-35; dispatch src/kernels.rs:2956-2975. */
void orc_add(const float* a, const float* b, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = a[i] + b[i];
}

/* `bias_add_kernel`, src/kernels.cu:1091-1096; checks src/kernels.rs:2977-3000. */
int orc_bias_add(const float* a, const float* bias, float* out, uint64_t cols, uint64_t n) {
    if (cols == 0 || n % cols != 0) return ORC_SHAPE_UNSUPPORTED;
    for (uint64_t i = 0; i < n; i++) out[i] = a[i] + bias[i % cols];
    return ORC_OK;
}

/* `mul_kernel`, src/kernels.cu:55-60. */
void orc_mul(const float* a, const float* b, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = a[i] * b[i];
}

/* `mul_scalar_kernel`, src/kernels.cu:112-117; chosen at src/executor.rs:1923-1932. */
void orc_mul_scalar(const float* a, const float* b, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = a[i] * b[0];
}

/* `silu_kernel`: v * (1 / (1 + expf(-v))), src/kernels.cu:73-79. */
void orc_silu(const float* x, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        float v = x[i];
        out[i] = v * (1.0f / (1.0f + expf(-v)));
    }
}

/* `silu_mul_kernel`: silu(gate) * up, same expression order, src/kernels.cu:64-71. */
void orc_silu_mul(const float* gate, const float* up, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        float v = gate[i];
        float activated = v * (1.0f / (1.0f + expf(-v)));
        out[i] = activated * up[i];
    }
}

/* `scale_kernel`: x * factor, src/kernels.cu:95-101 (the embedding's `scale`,
 * src/executor.rs:1509-1516). */
void orc_scale(const float* x, float* out, float factor, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = x[i] * factor;
}

/* ---------------------------------------------------------------------- */
/* Embedding gather                                                        */
/* ---------------------------------------------------------------------- */

/* `embedding_lookup_kernel`, src/kernels.cu:127-176; the failure is
 * src/kernels.rs:3984-3997 (ShapeUnsupported, rows of invalid ids unwritten).
 * An id is valid iff id >= 0, id == floor(id) and id < vocab. */
int orc_embedding(const float* table, uint64_t vocab, uint64_t dim, const float* ids,
                  uint64_t num_ids, float* out) {
    int status = ORC_OK;
    for (uint64_t r = 0; r < num_ids; r++) {
        float raw = ids[r];
        if (raw < 0.0f || raw != floorf(raw) || (double)raw >= (double)vocab) {
            status = ORC_SHAPE_UNSUPPORTED;
            continue;
        }
        uint64_t id = (uint64_t)raw;
        memcpy(out + r * dim, table + id * dim, dim * sizeof(float));
    }
    return status;
}

/* ---------------------------------------------------------------------- */
/* Row reductions                                                          */
/* ---------------------------------------------------------------------- */

/* `rmsnorm_kernel`: inv = 1/sqrtf(sum(x^2)/cols + eps), y = x*inv*w,
 * src/kernels.cu:1098-1138; checks src/kernels.rs:4013-4085. The sum of
 * squares runs ascending in f32 (the CPU Provider's order). */
int orc_rmsnorm(const float* in, const float* weight, float* out, uint64_t rows,
                uint64_t cols, uint64_t weight_row_stride, float eps) {
    if (cols == 0 || !(eps > 0.0f)) return ORC_SHAPE_UNSUPPORTED;
    for (uint64_t r = 0; r < rows; r++) {
        const float* x = in + r * cols;
        float sum = 0.0f;
        for (uint64_t i = 0; i < cols; i++) sum += x[i] * x[i];
        float inv = 1.0f / sqrtf(sum / (float)cols + eps);
        float* y = out + r * cols;
        if (weight) {
            const float* w = weight + r * weight_row_stride;
            for (uint64_t i = 0; i < cols; i++) y[i] = x[i] * inv * w[i];
        } else {
            for (uint64_t i = 0; i < cols; i++) y[i] = x[i] * inv;
        }
    }
    return ORC_OK;
}

/* `softmax_rows_kernel`, src/kernels.cu:1232-1260: max by fmaxf (NaN-ignoring);
 * a non-finite max fails the call (src/kernels.rs:4371-4378, ExecutionFailed);
 * sum of expf(x - max) ascending; y = expf(x - max) / sum. */
int orc_softmax_rows(const float* in, float* out, uint64_t rows, uint64_t cols) {
    int status = ORC_OK;
    for (uint64_t r = 0; r < rows; r++) {
        const float* x = in + r * cols;
        float m = -INFINITY;
        for (uint64_t i = 0; i < cols; i++) m = fmaxf(m, x[i]);
        if (!isfinite(m)) {
            status = ORC_EXECUTION_FAILED;
            continue;
        }
        float sum = 0.0f;
        for (uint64_t i = 0; i < cols; i++) sum += expf(x[i] - m);
        float* y = out + r * cols;
        for (uint64_t i = 0; i < cols; i++) y[i] = expf(x[i] - m) / sum;
    }
    return status;
}

/* ---------------------------------------------------------------------- */
/* RoPE                                                                    */
/* ---------------------------------------------------------------------- */

/* Per-pair frequency and amplitude, the f32 operations of `rope_kernel`,
 * src/kernels.cu:1197-1221: powf(base, -2p/dimension), then the banded
 * scaling, then YaRN's blend; pairs at or past `rotated_pairs` get frequency
 * 0 and amplitude 1 (angle 0: pass-through). */
void orc_rope_frequencies(const orc_rope_params* p, float* freq, float* amp) {
    uint64_t half = p->dimension / 2;
    for (uint64_t pair = 0; pair < half; pair++) {
        float frequency = powf(p->base, -2.0f * (float)pair / (float)p->dimension);
        if (p->banded_factor > 0.0f) {
            float wavelength = 6.283185307179586f / frequency;
            if (wavelength < p->original_context_length / p->high_freq_factor) {
                /* high frequencies kept */
            } else if (wavelength > p->original_context_length / p->low_freq_factor) {
                frequency = frequency / p->banded_factor;
            } else {
                float smooth = (p->original_context_length / wavelength - p->low_freq_factor) /
                               (p->high_freq_factor - p->low_freq_factor);
                frequency = (1.0f - smooth) * frequency / p->banded_factor + smooth * frequency;
            }
        }
        if (p->yarn_factor > 0.0f) {
            float high = p->yarn_low == p->yarn_high ? p->yarn_high + 0.001f : p->yarn_high;
            float ramp = ((float)pair - p->yarn_low) / (high - p->yarn_low);
            ramp = fminf(fmaxf(ramp, 0.0f), 1.0f);
            float interpolated = frequency / p->yarn_factor;
            frequency = interpolated * ramp + frequency * (1.0f - ramp);
        }
        int rotated = pair < p->rotated_pairs;
        freq[pair] = rotated ? frequency : 0.0f;
        amp[pair] = rotated ? p->amplitude : 1.0f;
    }
}

/* `rope_kernel`, src/kernels.cu:1147-1229; checks src/kernels.rs:4224-4320.
 * Per (row, head, pair): pos = (float)(offset + row) * scale,
 * angle = pos * freq[pair], s = sinf(angle)*amp, c = cosf(angle)*amp,
 * o1 = a*c - b*s, o2 = a*s + b*c. Columns past `dimension` in each head copy
 * through. */
int orc_rope(const float* in, float* out, uint64_t rows, uint64_t cols,
             const orc_rope_params* p) {
    if (p->head_count == 0 || cols % p->head_count != 0) return ORC_SHAPE_UNSUPPORTED;
    uint64_t head_width = cols / p->head_count;
    if (p->dimension == 0 || p->dimension % 2 != 0 || p->dimension > head_width)
        return ORC_SHAPE_UNSUPPORTED;
    if (!isfinite(p->base) || p->base <= 0.0f || !isfinite(p->scale) || p->scale <= 0.0f)
        return ORC_SHAPE_UNSUPPORTED;
    uint64_t half = p->dimension / 2;
    float freq[4096], amp[4096];
    if (half > 4096) return ORC_SHAPE_UNSUPPORTED;
    orc_rope_frequencies(p, freq, amp);
    memcpy(out, in, rows * cols * sizeof(float));
    for (uint64_t r = 0; r < rows; r++) {
        float position = (float)(p->position_offset + r) * p->scale;
        for (uint64_t h = 0; h < p->head_count; h++) {
            uint64_t base_col = r * cols + h * head_width;
            for (uint64_t pair = 0; pair < half; pair++) {
                float angle = position * freq[pair];
                float s = sinf(angle) * amp[pair];
                float c = cosf(angle) * amp[pair];
                uint64_t first = p->half_split ? base_col + pair : base_col + 2 * pair;
                uint64_t second = p->half_split ? base_col + pair + half : base_col + 2 * pair + 1;
                float a = in[first];
                float b = in[second];
                out[first] = a * c - b * s;
                out[second] = a * s + b * c;
            }
        }
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Matmul                                                                  */
/* ---------------------------------------------------------------------- */

/* `matmul_kernel`'s definition: f32 accumulation over k ascending, then the
 * fused addend added to the finished sum, src/kernels.cu:1262-1306;
 * strides and checks src/kernels.rs:5518-5580. */
int orc_matmul(const float* a, const float* b, float* out, uint64_t m, uint64_t k,
               uint64_t n, int transpose_a, int transpose_b, const float* addend,
               int addend_mode) {
    uint64_t a_row = transpose_a ? 1 : k, a_inner = transpose_a ? m : 1;
    uint64_t b_inner = transpose_b ? 1 : n, b_col = transpose_b ? k : 1;
    /* Loop-interchanged so B streams by rows: every out[r][c] still starts at
     * 0.0f and adds a[r][i] * b[i][c] for i ascending, one f32 rounding each. */
    for (uint64_t r = 0; r < m; r++) {
        float* o = out + r * n;
        for (uint64_t c = 0; c < n; c++) o[c] = 0.0f;
        for (uint64_t i = 0; i < k; i++) {
            float av = a[r * a_row + i * a_inner];
            const float* brow = b + i * b_inner;
            if (b_col == 1) {
                for (uint64_t c = 0; c < n; c++) o[c] += av * brow[c];
            } else {
                for (uint64_t c = 0; c < n; c++) o[c] += av * brow[c * b_col];
            }
        }
        if (addend_mode == 1) {
            for (uint64_t c = 0; c < n; c++) o[c] = o[c] + addend[c];
        } else if (addend_mode == 2) {
            for (uint64_t c = 0; c < n; c++) o[c] = o[c] + addend[r * n + c];
        }
    }
    return ORC_OK;
}

/* The same sums for a row range, loop-interchanged so B streams by rows:
 * each output still accumulates k ascending in f32, so the values are the
 * same as orc_matmul's. */
void orc_matmul_rows(const float* a, const float* b, float* out, uint64_t row_begin,
                     uint64_t row_end, uint64_t k, uint64_t n) {
    for (uint64_t r = row_begin; r < row_end; r++) {
        float* o = out + (r - row_begin) * n;
        for (uint64_t c = 0; c < n; c++) o[c] = 0.0f;
        for (uint64_t i = 0; i < k; i++) {
            float av = a[r * k + i];
            const float* brow = b + i * n;
            for (uint64_t c = 0; c < n; c++) o[c] += av * brow[c];
        }
    }
}

/* ---------------------------------------------------------------------- */
/* Attention                                                               */
/* ---------------------------------------------------------------------- */

/* The key range one query admits, src/kernels.cu:1909-1920. */
static void key_range(const orc_attention_params* p, uint64_t qpos, uint64_t* lo, uint64_t* hi) {
    uint64_t upper = p->causal ? qpos + 1 : p->kv_seq_len;
    uint64_t lower = 0;
    if (p->window_size >= 0) {
        uint64_t window = (uint64_t)p->window_size;
        uint64_t back = window > 0 ? window - 1 : 0;
        lower = qpos > back ? qpos - back : 0;
        if (lower > upper) lower = upper;
    }
    *lo = lower;
    *hi = upper;
}

/* `attention_kernel`, the defining three-pass form, src/kernels.cu:1868-1959;
 * validation src/kernels.rs:6533-6628. Rows: q [seq, H*d], k [kv_rows, Hkv*d],
 * v [kv_rows, Hkv*vd]; out [seq, H*vd]. qpos = (kv_seq - seq) + i. */
int orc_attention_heads(const float* q, const float* k, const float* v, float* out,
                        const orc_attention_params* p, uint64_t head_begin,
                        uint64_t head_end) {
    uint64_t H = p->head_count, Hkv = p->kv_head_count, d = p->head_dimension;
    uint64_t vd = p->value_dimension;
    if (H == 0 || Hkv == 0 || d == 0 || vd == 0 || H % Hkv != 0) return ORC_SHAPE_UNSUPPORTED;
    if (p->kv_seq_len > p->kv_rows || p->seq_len > p->kv_seq_len) return ORC_SHAPE_UNSUPPORTED;
    if (p->window_size == 0 || (p->window_size > 0 && !p->causal)) return ORC_SHAPE_UNSUPPORTED;
    uint64_t group = H / Hkv;
    uint64_t q_dim = H * d, kv_dim = Hkv * d, v_dim = Hkv * vd;
    uint64_t offset = p->kv_seq_len - p->seq_len;
    float scale = p->scale > 0.0f ? p->scale : 1.0f / sqrtf((float)d);
    for (uint64_t h = head_begin; h < head_end; h++) {
        uint64_t kvh = h / group;
        for (uint64_t i = 0; i < p->seq_len; i++) {
            uint64_t lo, hi;
            key_range(p, offset + i, &lo, &hi);
            const float* qr = q + i * q_dim + h * d;
            float m = -INFINITY;
            for (uint64_t j = lo; j < hi; j++) {
                const float* kr = k + j * kv_dim + kvh * d;
                float dot = 0.0f;
                for (uint64_t t = 0; t < d; t++) dot += qr[t] * kr[t];
                m = fmaxf(m, dot * scale);
            }
            float sum = 0.0f;
            for (uint64_t j = lo; j < hi; j++) {
                const float* kr = k + j * kv_dim + kvh * d;
                float dot = 0.0f;
                for (uint64_t t = 0; t < d; t++) dot += qr[t] * kr[t];
                sum += expf(dot * scale - m);
            }
            float* o = out + (i * H + h) * vd;
            for (uint64_t t = 0; t < vd; t++) o[t] = 0.0f;
            for (uint64_t j = lo; j < hi; j++) {
                const float* kr = k + j * kv_dim + kvh * d;
                float dot = 0.0f;
                for (uint64_t t = 0; t < d; t++) dot += qr[t] * kr[t];
                float w = expf(dot * scale - m) / sum;
                const float* vr = v + j * v_dim + kvh * vd;
                for (uint64_t t = 0; t < vd; t++) o[t] += w * vr[t];
            }
        }
    }
    return ORC_OK;
}

int orc_attention(const float* q, const float* k, const float* v, float* out,
                  const orc_attention_params* p) {
    return orc_attention_heads(q, k, v, out, p, 0, p->head_count);
}

/* src/kernels.cu:1808-1866 (greedy_select_kernel's contract). */
int64_t orc_greedy_select(const float* row, uint64_t cols, const uint64_t* ranges,
                          uint32_t range_count, float temperature) {
    int64_t best = -1;
    float best_value = 0.0f;
    for (uint64_t i = 0; i < cols; ++i) {
        float value = row[i];
        if (!isfinite(value)) continue;
        int excluded = 0;
        for (uint32_t r = 0; r < range_count; ++r)
            if (i >= ranges[2 * r] && i < ranges[2 * r + 1]) excluded = 1;
        if (excluded) continue;
        if (temperature != 0.0f) value = value / temperature;
        if (best < 0 || value > best_value) {
            best = (int64_t)i;
            best_value = value;
        }
    }
    return best;
}
