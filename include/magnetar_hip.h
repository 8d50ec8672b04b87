/*
 * magnetar_hip.h -- the C ABI of the Magnetar MI355X (gfx950) Provider.
 *
 * This is the drop-in boundary for the reference's hot path: the f32
 * required-now Kernel set plus the f16/bf16 add/mul path that the reference
 * CUDA Provider dispatches from `CudaExecutor::run_invocation_with_offer`
 * (src/executor.rs:1422-2027) to `CudaKernels` launch wrappers
 * (src/kernels.rs) over cudarc. Every entry point is plain C: device pointers,
 * sizes and small POD parameter structs; no C++ or torch types cross it.
 *
 * Conventions
 *  - Every function returns an `mhip_status`. On failure a redacted,
 *    thread-local diagnostic is available from `mhip_last_error_detail()`
 *    (never a native pointer or handle; src/error.rs:44-52).
 *  - Kernel entry points enqueue on the context's single in-order HIP stream
 *    and return before the device finishes (the reference's one-stream model,
 *    src/kernels.rs:796-827). `mhip_download` and `mhip_sync` wait.
 *  - Data-dependent failures (an invalid embedding id, a softmax row with no
 *    finite entry) are recorded in a device flag word and reported by
 *    `mhip_check_flags`, which waits; the chained path checks once at the end
 *    instead of after every call.
 *  - All f32 tensors are contiguous row-major.
 */
#ifndef MAGNETAR_HIP_H
#define MAGNETAR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error categories: one-to-one with `CudaErrorCode` (src/error.rs:15-42). */
typedef enum {
    MHIP_OK = 0,
    MHIP_SHAPE_UNSUPPORTED = 1,
    MHIP_DTYPE_UNSUPPORTED = 2,
    MHIP_LAYOUT_UNSUPPORTED = 3,
    MHIP_EXECUTION_FAILED = 4,
    MHIP_OUT_OF_DEVICE_MEMORY = 5,
    MHIP_COMPILATION_FAILED = 6,
    MHIP_DRIVER_FAILED = 7,
    MHIP_DEVICE_UNAVAILABLE = 8,
    MHIP_CAPTURE_UNSUPPORTED = 9
} mhip_status;

/* Half-precision storage formats (`CudaHalfDType`, src/kernels.rs:191-251). */
typedef enum { MHIP_F16 = 0, MHIP_BF16 = 1 } mhip_half_dtype;

typedef struct mhip_ctx mhip_ctx;

/* Device metadata (`cuda_device_descriptor`, src/device.rs:41-74). */
typedef struct {
    int ordinal;
    char name[256];
    char architecture[64];      /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    uint64_t total_memory;
    uint64_t free_memory;
    uint32_t compute_units;
    uint32_t wavefront_size;
    uint64_t lds_per_workgroup;
    int pressure;               /* 0 low, 1 moderate, 2 high, 3 saturated, -1 unknown
                                   (buckets at free ratio 0.5/0.2/0.05, src/device.rs:81-92) */
} mhip_device_info;

/* Flag bits reported by mhip_check_flags. */
#define MHIP_FLAG_EMBEDDING_INVALID_ID 1u
#define MHIP_FLAG_SOFTMAX_NON_FINITE 2u

/* ---- diagnostics ------------------------------------------------------ */
const char* mhip_last_error_detail(void);
const char* mhip_status_name(mhip_status status);
const char* mhip_version(void);

/* ---- context and device (src/provider.rs:119-179) ---------------------- */
/* Number of visible HIP devices; 0 (and MHIP_OK) when there is no driver or GPU. */
mhip_status mhip_device_count(int* count);
/* Binds device `ordinal`; MHIP_DEVICE_UNAVAILABLE (never a crash) when absent. */
mhip_status mhip_ctx_create(int ordinal, mhip_ctx** out);
mhip_status mhip_ctx_destroy(mhip_ctx* ctx);
mhip_status mhip_device_query(mhip_ctx* ctx, mhip_device_info* info);

/* ---- buffers (CudaDeviceBuffer, src/kernels.rs:253-379, :1630-1665, :2118-2164) */
mhip_status mhip_alloc(mhip_ctx* ctx, size_t bytes, void** device_ptr);
mhip_status mhip_free(mhip_ctx* ctx, void* device_ptr);
mhip_status mhip_upload(mhip_ctx* ctx, void* device_dst, const void* host_src, size_t bytes);
/* Waits for the stream, then copies. */
mhip_status mhip_download(mhip_ctx* ctx, void* host_dst, const void* device_src, size_t bytes);
mhip_status mhip_copy(mhip_ctx* ctx, void* device_dst, const void* device_src, size_t bytes);
mhip_status mhip_zero(mhip_ctx* ctx, void* device_dst, size_t bytes);
mhip_status mhip_sync(mhip_ctx* ctx);
/* Waits, reads and clears the flag word; returns MHIP_SHAPE_UNSUPPORTED for an
 * invalid embedding id (src/kernels.rs:3984-3997) or MHIP_EXECUTION_FAILED for
 * a softmax row with no finite entry (src/kernels.rs:4371-4378). `flags` may be
 * NULL. */
mhip_status mhip_check_flags(mhip_ctx* ctx, uint32_t* flags);

/* Stream timing with HIP events on the context's stream. */
mhip_status mhip_timer_start(mhip_ctx* ctx);
/* Records the stop event, waits for it, returns elapsed milliseconds. */
mhip_status mhip_timer_stop(mhip_ctx* ctx, float* elapsed_ms);

/* ---- f32 elementwise (src/kernels.rs:2956-3118, :3227-3252, :4492-4523) ---- */
/* out[i] = a[i] + b[i]                         add_kernel, src/kernels.cu:30-35 */
mhip_status mhip_add_f32(mhip_ctx* ctx, const float* a, const float* b, float* out, uint64_t n);
/* out[i] = a[i] + bias[i % cols]; n % cols == 0  bias_add_kernel, src/kernels.cu:1091-1096 */
mhip_status mhip_bias_add_f32(mhip_ctx* ctx, const float* a, const float* bias, float* out,
                              uint64_t cols, uint64_t n);
/* out[i] = a[i] * b[i]                         mul_kernel, src/kernels.cu:55-60 */
mhip_status mhip_mul_f32(mhip_ctx* ctx, const float* a, const float* b, float* out, uint64_t n);
/* out[i] = a[i] * b[0]                         mul_scalar_kernel, src/kernels.cu:112-117 */
mhip_status mhip_mul_scalar_f32(mhip_ctx* ctx, const float* a, const float* b, float* out,
                                uint64_t n);
/* out[i] = x * (1 / (1 + expf(-x)))            silu_kernel, src/kernels.cu:73-79 */
mhip_status mhip_silu_f32(mhip_ctx* ctx, const float* x, float* out, uint64_t n);
/* out[i] = silu(gate[i]) * up[i]               silu_mul_kernel, src/kernels.cu:64-71 */
mhip_status mhip_silu_mul_f32(mhip_ctx* ctx, const float* gate, const float* up, float* out,
                              uint64_t n);
/* out[i] = x[i] * factor                       scale_kernel, src/kernels.cu:95-101 */
mhip_status mhip_scale_f32(mhip_ctx* ctx, const float* x, float* out, float factor, uint64_t n);

/* ---- half precision on 2-byte buffers (src/kernels.rs:2172-2266, src/kernels.cu:2806-2939) */
/* out = enc(dec(a) op dec(b)), op in f32, RNE encode; bit-exact. */
mhip_status mhip_add_half(mhip_ctx* ctx, const uint16_t* a, const uint16_t* b, uint16_t* out,
                          uint64_t n, mhip_half_dtype dtype);
mhip_status mhip_mul_half(mhip_ctx* ctx, const uint16_t* a, const uint16_t* b, uint16_t* out,
                          uint64_t n, mhip_half_dtype dtype);
/* f32 <-> half on the device: the upload_half / download_half codec
 * (src/kernels.rs:2172-2219, src/half_precision.rs:14-125) without the host trip. */
mhip_status mhip_encode_half(mhip_ctx* ctx, const float* in, uint16_t* out, uint64_t n,
                             mhip_half_dtype dtype);
mhip_status mhip_decode_half(mhip_ctx* ctx, const uint16_t* in, float* out, uint64_t n,
                             mhip_half_dtype dtype);

/* ---- embedding gather (src/kernels.rs:3833-3997, src/kernels.cu:127-176) ---- */
/* out[r, :] = table[ids[r], :] for f32 ids that are in-range non-negative
 * integers; an invalid id leaves its row unwritten and sets
 * MHIP_FLAG_EMBEDDING_INVALID_ID. */
mhip_status mhip_embedding_f32(mhip_ctx* ctx, const float* table, uint64_t vocab, uint64_t dim,
                               const float* ids, uint64_t num_ids, float* out);

/* ---- row reductions ----------------------------------------------------- */
/* y = x * (1/sqrtf(mean(x^2) + eps)) * w; `weight` NULL for scale 1;
 * weight_row_stride 0 (broadcast row) or cols (per-row).
 * rmsnorm_kernel, src/kernels.cu:1098-1138; src/kernels.rs:4013-4104 */
mhip_status mhip_rmsnorm_f32(mhip_ctx* ctx, const float* in, const float* weight, float* out,
                             uint64_t rows, uint64_t cols, uint64_t weight_row_stride,
                             float eps);
/* Row softmax; a row whose max is not finite sets MHIP_FLAG_SOFTMAX_NON_FINITE.
 * softmax_rows_kernel, src/kernels.cu:1232-1260; src/kernels.rs:4357-4386 */
mhip_status mhip_softmax_rows_f32(mhip_ctx* ctx, const float* in, float* out, uint64_t rows,
                                  uint64_t cols);

/* ---- RoPE (rope_kernel, src/kernels.cu:1147-1229; src/kernels.rs:4224-4355) ---- */
typedef struct {
    float base;                     /* > 0, finite (default 10000) */
    float scale;                    /* > 0, finite (default 1) */
    uint64_t dimension;             /* even, <= head width */
    uint64_t position_offset;
    uint64_t head_count;            /* divides cols */
    uint32_t half_split;            /* 0 interleaved (2p, 2p+1); 1 half-split (p, p + dim/2) */
    uint64_t rotated_pairs;         /* partial rotary: pairs >= this pass through; clamp to dim/2 */
    float banded_factor;            /* 0 disables banded frequency scaling */
    float low_freq_factor;
    float high_freq_factor;
    float original_context_length;
    float yarn_factor;              /* 0 disables YaRN */
    float yarn_low;                 /* YaRN correction range */
    float yarn_high;
    float amplitude;                /* YaRN attention factor; 1 otherwise */
} mhip_rope_params;
/* Fills `p` with the reference defaults for `dimension` and `head_count`. */
void mhip_rope_params_default(mhip_rope_params* p, uint64_t dimension, uint64_t head_count);
mhip_status mhip_rope_f32(mhip_ctx* ctx, const float* in, float* out, uint64_t rows,
                          uint64_t cols, const mhip_rope_params* params);

/* ---- matmul (src/kernels.rs:4388-4436, :5518-5789; src/kernels.cu:1262-1693) ---- */
/* out[m, n] = A . B with A [m, k] (or [k, m] stored when transpose_a) and
 * B [k, n] (or [n, k] when transpose_b), f32 accumulation; addend_mode 1 adds
 * addend[col] (matmul-bias), 2 adds addend[row * n + col] (matmul-residual)
 * to the finished sum. fp32 MFMA tiles for m > 8; an HBM-streaming split-k
 * kernel for m <= 8 (decode), whose partial sums use a grow-only workspace
 * owned by the context. */
mhip_status mhip_matmul_f32(mhip_ctx* ctx, const float* a, const float* b, float* out,
                            uint64_t m, uint64_t k, uint64_t n, int transpose_a,
                            int transpose_b, const float* addend, int addend_mode);

/* Which kernel path mhip_matmul_f32 takes for an m x k x n product with
 * 16-byte aligned operands. No counterpart in the reference: a diagnostic for
 * tests (that a case exercises the path it is written for) and tuning.
 * path: the split-k GEMV (m <= 8), row blocks of 8 on the GEMV (16-32 rows of
 * a small product with k > 1024), one launch of 32 x 32 MFMA tiles with k
 * split over the workgroup's waves (16-32 rows of a small product, k <= 1024,
 * k % 4 == 0), or MFMA tiles of tile_m x tile_n with `waves` waves per
 * workgroup. splits: k slices of the GEMV, or k splits of the tiles (1: none);
 * stream_k: 1 when (tile, k slice) runs are dealt to the workgroups. */
enum {
    MHIP_MATMUL_PATH_GEMV = 0,
    MHIP_MATMUL_PATH_GEMV_ROW_BLOCKS = 1,
    MHIP_MATMUL_PATH_TILES = 2,
    MHIP_MATMUL_PATH_SMALL_TILES = 3
};
typedef struct {
    uint32_t path;
    uint32_t tile_m, tile_n, waves;
    uint32_t splits;
    uint32_t stream_k;
} mhip_matmul_plan;
mhip_status mhip_matmul_plan_f32(mhip_ctx* ctx, uint64_t m, uint64_t k, uint64_t n,
                                 int transpose_a, int transpose_b, mhip_matmul_plan* plan);

/* ---- attention (src/kernels.rs:6505-7078; src/kernels.cu:1868-2787) ---- */
typedef struct {
    uint64_t seq_len;           /* query rows */
    uint64_t kv_rows;           /* rows held by k and v */
    uint64_t kv_seq_len;        /* key_count: keys in use, <= kv_rows (kv_rows when absent) */
    uint64_t head_count;
    uint64_t kv_head_count;     /* divides head_count (grouped-query attention) */
    uint64_t head_dimension;
    uint64_t value_dimension;   /* V and output width per head; 0 means head_dimension */
    int causal;
    int64_t window_size;        /* sliding window (causal only); -1 none, 0 rejected */
    float scale;                /* factor on q.k; <= 0 means 1/sqrt(head_dimension) */
    /* Batched extension: `batch` independent calls with these element strides
     * (0: densely packed); the reference has no batch dimension. */
    uint64_t batch;
    uint64_t q_batch_stride;
    uint64_t kv_batch_stride;
    uint64_t v_batch_stride;
    uint64_t out_batch_stride;
    /* 1 when kv_seq_len came from an explicit key count (the executor's
     * `key_count` attribute): a captured call may then advance it. */
    uint32_t bounded_key_count;
} mhip_attention_params;
/* q [seq, H*d], k [kv_rows, Hkv*d], v [kv_rows, Hkv*vd] -> out [seq, H*vd].
 * Query i sits at position (kv_seq_len - seq_len) + i; a causal query admits
 * keys up to its own position, a window of w the last w of them. Softmax of
 * q.k * scale over the admitted keys weights V rows; no admitted key gives 0.
 * fp32 MFMA flash prefill for head dims 64/128, split-KV decode for one query
 * row (workspace owned by the context), a generic kernel otherwise. */
mhip_status mhip_attention_f32(mhip_ctx* ctx, const float* q, const float* k, const float* v,
                               float* out, const mhip_attention_params* params);

/* Allocation-free matmul. No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments, paths and results
 * as mhip_matmul_f32 (bit for bit), but the split-k / stream-K / GEMV partial
 * sums go to a fixed device array of MHIP_NOALLOC_SCRATCH_BYTES that the
 * library holds on each GPU it runs on until the process ends, instead of
 * the context's grow-only workspace; it calls no hipMalloc or hipFree. A
 * product whose partial sums need more returns MHIP_SHAPE_UNSUPPORTED (the
 * detail names the bytes needed). Every context on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (different streams or
 * contexts) race; calls ordered on one stream do not. */
#define MHIP_NOALLOC_SCRATCH_BYTES (128ull << 20)
mhip_status mhip_matmul_f32_noalloc(mhip_ctx* ctx, const float* a, const float* b, float* out,
                                    uint64_t m, uint64_t k, uint64_t n, int transpose_a,
                                    int transpose_b, const float* addend, int addend_mode);

/* Compact bf16 weights (execute-native-half-precision, src/kernels.rs:1665-1723):
 * the matmul with b given as bf16 bit patterns ([k, n], or [n, k] when
 * transpose_b) and the embedding lookup with a bf16 table. Each widens the
 * weight exactly (a bf16 value is an f32 with zero low bits) and computes in
 * f32, so the result equals mhip_matmul_f32 / mhip_embedding_f32 on the
 * widened weight bit for bit, reading half the weight bytes. */
mhip_status mhip_matmul_bf16w_f32(mhip_ctx* ctx, const float* a, const uint16_t* b, float* out,
                                  uint64_t m, uint64_t k, uint64_t n, int transpose_a,
                                  int transpose_b, const float* addend, int addend_mode);
mhip_status mhip_embedding_bf16w_f32(mhip_ctx* ctx, const uint16_t* table, uint64_t vocab,
                                     uint64_t dim, const float* ids, uint64_t num_ids, float* out);

/* Greedy next-token selection (src/kernels.rs:4437-4488): the column of
 * logits row `row` ([rows, cols]) with the largest score / temperature (score
 * as is when temperature is 0) among finite scores outside the `range_count`
 * excluded [start, end) pairs in `excluded` (host memory, 2 * range_count
 * values); ties go to the lowest column. *column = -1 when no column is
 * eligible. One kernel launch; the answer arrives in a pinned host word of
 * the context and the call synchronises the context's stream. Calls on one
 * context must not overlap (they share that word and the device key). */
mhip_status mhip_greedy_select_f32(mhip_ctx* ctx, const float* logits, uint64_t rows,
                                   uint64_t cols, uint64_t row, const uint64_t* excluded,
                                   uint32_t range_count, float temperature, int64_t* column);

/* kv-write (src/kernels.rs:2270-2325): store [capacity, width] rows
 * [row_offset, row_offset + count) = rows [count, width], in place; other rows
 * unchanged. An overrun is ShapeUnsupported and writes nothing. */
mhip_status mhip_kv_write_f32(mhip_ctx* ctx, float* store, uint64_t capacity, uint64_t width,
                              const float* rows, uint64_t count, uint64_t row_offset);

/* ---- step capture and replay (src/kernels.rs:1019-1349, src/executor.rs:177-336) ----
 * Between mhip_capture_begin and mhip_capture_end, the context's launches are
 * recorded (kernel, grid, argument values) instead of running; a replay
 * re-issues them in order on the context's stream (hipGraphLaunch of the same
 * launches measured 4.6-7 us slower per step here). A launch whose attribute is
 * named in `advancing` adds the replay offset given to mhip_graph_launch:
 * RoPE's position_offset, attention's key count (one query row, and only when
 * the caller sets mhip_attention_params.bounded_key_count) and kv-write's
 * row_offset. Each such launch bounds the offset (the key count and the rows
 * written must stay inside K/V and the store). Nothing that allocates,
 * transfers, clears memory or synchronises can be captured: such a call
 * returns CaptureUnsupported and fails the capture (mhip_capture_end then
 * reports the first reason). Multi-row attention replays only at offset 0. */
typedef enum {
    MHIP_ADVANCE_POSITION_OFFSET = 1,
    MHIP_ADVANCE_KEY_COUNT = 2,
    MHIP_ADVANCE_ROW_OFFSET = 4
} mhip_advancing;
typedef struct mhip_graph mhip_graph;
mhip_status mhip_capture_begin(mhip_ctx* ctx, uint32_t advancing);
/* Instantiates the recorded step; *max_offset is the largest replay offset
 * every advancing launch allows. Does not run it. */
mhip_status mhip_capture_end(mhip_ctx* ctx, mhip_graph** out, uint64_t* max_offset);
mhip_status mhip_capture_abort(mhip_ctx* ctx);
int mhip_capture_active(const mhip_ctx* ctx);
/* Runs the step with every advancing attribute increased by `offset`
 * (ShapeUnsupported beyond the bound). Its launches set failure flags as
 * eager calls do: a flag stays set, whichever call or replay set it, until
 * mhip_check_flags reads and clears it. */
mhip_status mhip_graph_launch(mhip_graph* graph, uint64_t offset);
uint64_t mhip_graph_max_offset(const mhip_graph* graph);
mhip_status mhip_graph_destroy(mhip_graph* graph);

/* ---- decoder block, chained device-resident (src/tests_hardware_hot_path.rs:339-526) ---- */
/* Block weight storage: f32, or compact bf16 bit patterns for the matrices
 * (embedding, wq, wk, wv, wo, w_gate, w_up, w_down; norms stay f32). */
typedef enum { MHIP_WEIGHTS_F32 = 0, MHIP_WEIGHTS_BF16 = 1 } mhip_weight_format;

typedef struct {
    uint64_t hidden;            /* = heads * head_dim */
    uint64_t heads;
    uint64_t kv_heads;
    uint64_t head_dim;
    uint64_t ffn;               /* SwiGLU intermediate width */
    uint64_t vocab;
    float eps;                  /* RMSNorm epsilon */
    float rope_base;            /* RoPE theta */
    uint32_t weight_format;     /* mhip_weight_format */
} mhip_block_config;

/* Device pointers, row-major: embedding [vocab, hidden]; attn_norm and
 * ffn_norm [hidden]; wq [hidden, H*hd], wk and wv [hidden, Hkv*hd],
 * wo [H*hd, hidden]; w_gate and w_up [hidden, ffn]; w_down [ffn, hidden].
 * f32, except that the matrices hold bf16 bit patterns (2 bytes each, the
 * pointer reinterpreted) under MHIP_WEIGHTS_BF16. */
typedef struct {
    const float* embedding;
    const float* attn_norm;
    const float* wq;
    const float* wk;
    const float* wv;
    const float* wo;
    const float* ffn_norm;
    const float* w_gate;
    const float* w_up;
    const float* w_down;
} mhip_block_weights;

/* Workspace bytes mhip_block_forward needs for `seq` tokens. */
uint64_t mhip_block_workspace_bytes(const mhip_block_config* cfg, uint64_t seq);
/* One block over `seq` tokens (ids: f32 token ids on the device) at positions
 * position .. position+seq-1: embedding -> rmsnorm -> q/k/v -> rope ->
 * K/V written into cache rows [position, position+seq) -> causal attention over
 * position+seq keys -> o-proj + residual -> rmsnorm -> silu(gate) * up ->
 * down + residual -> out [seq, hidden]. k_cache / v_cache: [cache_rows,
 * kv_heads*head_dim]. Enqueues only; an invalid id is reported by
 * mhip_check_flags. */
mhip_status mhip_block_forward(mhip_ctx* ctx, const mhip_block_config* cfg,
                               const mhip_block_weights* weights, const float* ids, uint64_t seq,
                               uint64_t position, float* k_cache, float* v_cache,
                               uint64_t cache_rows, void* workspace, uint64_t workspace_bytes,
                               float* out);

/* ======================================================================== */
/* Executor: the `CudaExecutor`-shaped ProviderExecutionApi (src/executor.rs) */
/* ======================================================================== */
/* Tensors are device-resident buffers keyed by resource id (src/executor.rs:101);
 * invocations name a Kernel and its inputs/outputs by id, with typed
 * attributes, and run eagerly on submit (src/executor.rs:2191-2241). No device
 * pointer ever crosses this part of the interface. */

typedef struct mhip_executor mhip_executor;

typedef enum { MHIP_DTYPE_F32 = 0, MHIP_DTYPE_F16 = 1, MHIP_DTYPE_BF16 = 2 } mhip_dtype;

/* `KernelError` categories (src/error.rs:97-133 plus the executor's own). */
typedef enum {
    MHIP_KERNEL_OK = 0,
    MHIP_KERNEL_SHAPE_UNSUPPORTED = 1,
    MHIP_KERNEL_DTYPE_UNSUPPORTED = 2,
    MHIP_KERNEL_LAYOUT_UNSUPPORTED = 3,
    MHIP_KERNEL_DEVICE_UNSUPPORTED = 4,
    MHIP_KERNEL_OUT_OF_DEVICE_MEMORY = 5,
    MHIP_KERNEL_EXECUTION_FAILED = 6,
    MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED = 7,
    MHIP_KERNEL_NOT_FOUND = 8,
    MHIP_KERNEL_TIMEOUT = 9,
    /* replay_step only: StepReplayError::Invalidated (src/executor.rs:272-336) */
    MHIP_STEP_REPLAY_INVALIDATED = 10
} mhip_kernel_error;

/* `OperatorAttributeValue` (src/executor.rs:1141-1185). */
typedef enum {
    MHIP_ATTR_FLOAT = 0,
    MHIP_ATTR_INTEGER = 1,
    MHIP_ATTR_BOOLEAN = 2,
    MHIP_ATTR_STRING = 3,
    MHIP_ATTR_DTYPE = 4
} mhip_attr_kind;

typedef struct {
    const char* key;
    int kind;               /* mhip_attr_kind */
    double f;
    int64_t i;
    int b;
    const char* s;
    int dtype;              /* mhip_dtype */
} mhip_attribute;

typedef struct {
    const char* id;
    int dtype;              /* mhip_dtype of the descriptor */
    const uint64_t* shape;
    int rank;
} mhip_tensor_ref;

typedef struct {
    const char* invocation_id;
    const char* kernel_name;
    const mhip_tensor_ref* inputs;
    int input_count;
    const mhip_tensor_ref* outputs;
    int output_count;
    const mhip_attribute* attributes;
    int attribute_count;
    int64_t deadline_millis;   /* -1: none; 0 fails with MHIP_KERNEL_TIMEOUT */
} mhip_invocation;

/* `KernelObservation` kinds (src/executor.rs:1082-1100, :1197-1231). */
typedef enum {
    MHIP_OBS_DISPATCH_STARTED = 0,
    MHIP_OBS_DISPATCH_COMPLETED = 1,
    MHIP_OBS_DISPATCH_FAILED = 2,
    MHIP_OBS_TIMEOUT = 3
} mhip_observation_kind;

typedef struct {
    int kind;               /* mhip_observation_kind */
    char kernel[64];
    char invocation[64];
    int error;              /* mhip_kernel_error for DISPATCH_FAILED */
} mhip_observation;

mhip_status mhip_executor_create(mhip_ctx* ctx, const char* device_id, const char* provider_name,
                                 mhip_executor** out);
mhip_status mhip_executor_destroy(mhip_executor* ex);
/* The detail text of the calling thread's last executor failure. */
const char* mhip_executor_last_detail(void);

/* write_tensor / write_weight_tensor (src/executor.rs:394-418): `data` holds
 * f32 values for MHIP_DTYPE_F32, 2-byte bit patterns for F16/BF16. */
mhip_kernel_error mhip_executor_write_tensor(mhip_executor* ex, const char* id,
                                             const uint64_t* shape, int rank, int dtype,
                                             const void* data, size_t bytes);
/* f32 host values stored as `dtype`, encoded RNE on the device (upload_half,
 * src/kernels.rs:2172-2197). */
mhip_kernel_error mhip_executor_write_tensor_values(mhip_executor* ex, const char* id,
                                                    const uint64_t* shape, int rank, int dtype,
                                                    const float* values);
mhip_kernel_error mhip_executor_write_zeroed_tensor(mhip_executor* ex, const char* id,
                                                    const uint64_t* shape, int rank, int dtype);
/* write_weight_tensor (src/executor.rs:384-399, src/kernels.rs:1665-1723):
 * `values` (f32) stored compact as bf16 bit patterns when the tensor is a
 * matrix of at least 65536 values that are all exact bf16 values (*compact =
 * 1), else as f32. Lossless either way: reads return the same f32 values.
 * Kernels read compact weights directly where the reference does (matmul,
 * matmul-bias, matmul-residual: b; gated-matmul: gate, up; embedding:
 * table); any other use stores the weight as f32 first, for good. */
mhip_kernel_error mhip_executor_write_weight_tensor(mhip_executor* ex, const char* id,
                                                    const uint64_t* shape, int rank,
                                                    const float* values, int* compact);
/* KV store precisions (KvStorePrecision: F32, Tq4, Tq3). */
typedef enum { MHIP_KV_F32 = 0, MHIP_KV_TQ4 = 1, MHIP_KV_TQ3 = 2 } mhip_kv_precision;
/* write_zeroed_kv_store (src/executor.rs:560-602): a zeroed f32 store of
 * `shape` under `id`, *stored = 1. The quantized TurboQuant precisions are not
 * provided by this build: *stored = 0 and nothing is written (the caller keeps
 * an f32 store). */
mhip_kernel_error mhip_executor_write_zeroed_kv_store(mhip_executor* ex, const char* id,
                                                      const uint64_t* shape, int rank,
                                                      int precision, uint64_t head_dimension,
                                                      int* stored);
/* read_tensor (src/executor.rs:430-434): the stored bytes, waiting for the device. */
mhip_kernel_error mhip_executor_read_tensor(mhip_executor* ex, const char* id, void* dst,
                                            size_t capacity, size_t* written);
/* The stored values decoded to f32 (download_half, src/kernels.rs:2203-2219). */
mhip_kernel_error mhip_executor_read_tensor_values(mhip_executor* ex, const char* id, float* dst,
                                                   size_t capacity);
/* read_tensor_rows (src/executor.rs:2392-2414): rows of a rank >= 1 f32 tensor. */
mhip_kernel_error mhip_executor_read_tensor_rows(mhip_executor* ex, const char* id,
                                                 uint64_t row_begin, uint64_t row_count,
                                                 float* dst, size_t capacity);
/* resident_shape: rank and dtype too; shape holds up to 8 dims. */
mhip_kernel_error mhip_executor_resident_shape(mhip_executor* ex, const char* id, uint64_t* shape,
                                               int* rank, int* dtype);
mhip_kernel_error mhip_executor_release_tensor(mhip_executor* ex, const char* id);
mhip_kernel_error mhip_executor_copy_tensor(mhip_executor* ex, const char* src, const char* dst);
uint64_t mhip_executor_tensor_count(mhip_executor* ex);

/* submit_kernel / complete_kernel (src/executor.rs:2322-2330, :2222-2241):
 * submit runs the invocation eagerly and parks its result under `handle`;
 * complete returns that result (MHIP_KERNEL_OK or the failure) exactly once. */
mhip_kernel_error mhip_executor_submit_kernel(mhip_executor* ex, const mhip_invocation* inv,
                                              uint64_t* handle);
mhip_kernel_error mhip_executor_complete_kernel(mhip_executor* ex, uint64_t handle);
/* submit + complete in one call. */
mhip_kernel_error mhip_executor_execute(mhip_executor* ex, const mhip_invocation* inv);
/* MAGNETAR_HIP_SYNC_NODES equivalent: wait for the device after each dispatch. */
/* select_greedy_column (src/executor.rs:2549-2564): greedy selection on the
 * stored logits resource; *column = -1 when none is eligible. */
mhip_kernel_error mhip_executor_select_greedy_column(mhip_executor* ex, const char* logits,
                                                     uint64_t row, const uint64_t* excluded,
                                                     uint32_t range_count, float temperature,
                                                     int64_t* column);

/* Step capture (src/executor.rs:177-336): the invocations between begin and
 * end are recorded as a launch sequence (see mhip_capture_begin); `advancing`
 * names the attributes a replay offset increases ("position_offset",
 * "key_count", "row_offset"). end instantiates the step, runs it once and
 * writes its id ("<provider>:step-capture:<n>"). replay_step writes each
 * input's f32 values into the buffer the step read and runs it at `offset`:
 * MHIP_STEP_REPLAY_INVALIDATED when a captured resource has another buffer
 * now, an input was not read by the step or the offset leaves the bounds;
 * MHIP_KERNEL_EXECUTION_FAILED for an invalid embedding id. */
int mhip_executor_supports_step_capture(mhip_executor* ex);
mhip_kernel_error mhip_executor_begin_step_capture(mhip_executor* ex, const char* const* advancing,
                                                   int count);
mhip_kernel_error mhip_executor_end_step_capture(mhip_executor* ex, char* id_out, size_t capacity);
mhip_kernel_error mhip_executor_abort_step_capture(mhip_executor* ex);
mhip_kernel_error mhip_executor_replay_step(mhip_executor* ex, const char* id, uint64_t offset,
                                            const char* const* input_ids,
                                            const float* const* input_values,
                                            const uint64_t* input_lengths, int input_count);
mhip_kernel_error mhip_executor_release_step_capture(mhip_executor* ex, const char* id);
mhip_status mhip_executor_set_sync_nodes(mhip_executor* ex, int enabled);
/* Deferred device checks (no counterpart in the reference, which reads the
 * failure flags after every embedding and softmax dispatch,
 * src/kernels.rs:3946-3968 and :4360; that stays the default). Enabled, those
 * dispatches return without waiting for the device, and the flags are read
 * once at the next tensor read, greedy selection, step-capture start,
 * mhip_executor_check or disable. A failure found there is returned by that
 * call, in the dispatch's category, naming the first unchecked dispatch; the
 * failing dispatch's output has been written by then. For executor-driven
 * chains that should not pay one host round trip per lookup. */
mhip_kernel_error mhip_executor_set_deferred_checks(mhip_executor* ex, int enabled);
mhip_kernel_error mhip_executor_check(mhip_executor* ex);
/* The observation log (last 4096 entries, src/executor.rs:82). */
uint64_t mhip_executor_observation_count(mhip_executor* ex);
mhip_status mhip_executor_observation(mhip_executor* ex, uint64_t index, mhip_observation* out);

/* ======================================================================== */
/* Provider facade and Kernel advertisements (src/provider.rs, advertisements.rs) */
/* ======================================================================== */

typedef enum {
    MHIP_HEALTH_AVAILABLE = 0,
    MHIP_HEALTH_DEGRADED = 1,
    MHIP_HEALTH_UNAVAILABLE = 2
} mhip_health;

typedef struct mhip_provider mhip_provider;

typedef struct {
    char name[128];
    char version[32];
    char vendor[64];
    char description[160];
} mhip_provider_metadata;

typedef struct {
    char id[32];                /* "hip:<ordinal>" */
    char name[256];
    char architecture[64];
    uint64_t memory_capacity;
    uint32_t compute_units;
    int pressure;               /* as mhip_device_info.pressure */
} mhip_device_descriptor;

/* Never fails for lack of hardware: with no device the provider reports
 * MHIP_HEALTH_UNAVAILABLE, zero devices and zero advertisements. */
mhip_status mhip_provider_create(int ordinal, const char* provider_name, mhip_provider** out);
mhip_status mhip_provider_destroy(mhip_provider* p);
mhip_status mhip_provider_metadata_get(mhip_provider* p, mhip_provider_metadata* out);
int mhip_provider_health(mhip_provider* p);
int mhip_provider_device_count(mhip_provider* p);
mhip_status mhip_provider_device(mhip_provider* p, int index, mhip_device_descriptor* out);
/* The provider's executor (NULL unless healthy); owned by the provider. */
mhip_executor* mhip_provider_executor(mhip_provider* p);
mhip_status mhip_provider_initialize(mhip_provider* p);
mhip_status mhip_provider_shutdown(mhip_provider* p);

typedef struct {
    char name[48];              /* Kernel name, e.g. "matmul", "add-half" */
    char operator_name[48];     /* portable Operator, e.g. "add" for "add-half" */
    char operator_family[32];   /* LinearAlgebra, Tensor, Activation, ... */
    uint32_t input_dtypes;      /* bit (1 << mhip_dtype) per accepted dtype */
    uint32_t output_dtypes;
    int rank;                   /* required rank, 0 when any */
    char features[256];         /* comma-separated optional forms honoured */
    char conformance_profile[32];
    char family[16];            /* implementation family: "Hip" */
    char device_id[32];
    char provider[128];
} mhip_advertisement;

int mhip_provider_advertisement_count(mhip_provider* p);
mhip_status mhip_provider_advertisement(mhip_provider* p, int index, mhip_advertisement* out);

#ifdef __cplusplus
}
#endif
#endif /* MAGNETAR_HIP_H */
