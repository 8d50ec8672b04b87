// The executor: device-resident tensors keyed by resource id and the
// name -> Kernel dispatch of the reference's `CudaExecutor`
// (src/executor.rs:91-2565), over the C ABI's kernel entry points.
//
// What is kept from the reference, and where:
//  - attribute parsing and defaults (src/executor.rs:1141-1185, :1422-2027);
//  - shape validation and its messages (src/kernels.rs, per Kernel below);
//  - the overwritten output's buffer offered back to the Kernel, and put back
//    when the dispatch fails (src/executor.rs:1268-1321);
//  - deadline 0 -> KernelTimeout; observations (src/executor.rs:1191-1233);
//  - eager submit, result parked until complete (src/executor.rs:2191-2241).
// What differs: f16/bf16 tensors stay 2-byte on the device and add-half /
// mul-half read and write them there (the reference round-trips through the
// host, src/executor.rs:1970-2013).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <optional>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "internal.hpp"
#include "magnetar_hip.h"

namespace {

thread_local std::string g_detail;

using Shape = std::vector<uint64_t>;

struct KernelFailure {
    mhip_kernel_error code;
    std::string detail;
};

[[noreturn]] void raise(mhip_kernel_error code, const std::string& detail) {
    throw KernelFailure{code, detail};
}

// CudaError -> KernelError (src/error.rs:97-133).
mhip_kernel_error map_status(mhip_status st) {
    switch (st) {
        case MHIP_OK: return MHIP_KERNEL_OK;
        case MHIP_SHAPE_UNSUPPORTED: return MHIP_KERNEL_SHAPE_UNSUPPORTED;
        case MHIP_DTYPE_UNSUPPORTED: return MHIP_KERNEL_DTYPE_UNSUPPORTED;
        case MHIP_LAYOUT_UNSUPPORTED: return MHIP_KERNEL_LAYOUT_UNSUPPORTED;
        case MHIP_DEVICE_UNAVAILABLE: return MHIP_KERNEL_DEVICE_UNSUPPORTED;
        case MHIP_OUT_OF_DEVICE_MEMORY: return MHIP_KERNEL_OUT_OF_DEVICE_MEMORY;
        default: return MHIP_KERNEL_EXECUTION_FAILED;
    }
}

void check(mhip_status st) {
    if (st != MHIP_OK) raise(map_status(st), mhip_last_error_detail());
}

std::string fmt_shape(const Shape& s) {
    std::ostringstream o;
    o << "[";
    for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
    o << "]";
    return o.str();
}

uint64_t numel(const Shape& s) {
    uint64_t n = 1;
    for (uint64_t d : s) n *= d;
    return n;
}

size_t dtype_size(int dtype) { return dtype == MHIP_DTYPE_F32 ? 4 : 2; }

const char* dtype_name(int dtype) {
    switch (dtype) {
        case MHIP_DTYPE_F32: return "Float32";
        case MHIP_DTYPE_F16: return "Float16";
        case MHIP_DTYPE_BF16: return "BrainFloat16";
    }
    return "Unknown";
}

// One device allocation with its shape and dtype (`CudaDeviceBuffer`,
// src/kernels.rs:253-379).
struct Buffer {
    mhip_ctx* ctx = nullptr;
    void* ptr = nullptr;
    size_t bytes = 0;
    Shape shape;
    int dtype = MHIP_DTYPE_F32;
    // An f32 weight stored compact as bf16 bit patterns (write_weight_tensor,
    // src/kernels.rs:1665-1723): 2 bytes per value, widened exactly on read.
    bool compact = false;

    Buffer(mhip_ctx* c, size_t nbytes, Shape s, int dt) : ctx(c), bytes(nbytes), shape(std::move(s)), dtype(dt) {
        check(mhip_alloc(ctx, bytes, &ptr));
    }
    ~Buffer() {
        if (ptr) mhip_free(ctx, ptr);
    }
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;
    float* f() const { return static_cast<float*>(ptr); }
    uint16_t* h() const { return static_cast<uint16_t*>(ptr); }
};
using BufferPtr = std::unique_ptr<Buffer>;

struct Attr {
    int kind = MHIP_ATTR_FLOAT;
    double f = 0.0;
    int64_t i = 0;
    bool b = false;
    std::string s;
    int dtype = MHIP_DTYPE_F32;

    std::string debug() const {
        std::ostringstream o;
        switch (kind) {
            case MHIP_ATTR_FLOAT: o << "Float(" << f << ")"; break;
            case MHIP_ATTR_INTEGER: o << "Integer(" << i << ")"; break;
            case MHIP_ATTR_BOOLEAN: o << "Boolean(" << (b ? "true" : "false") << ")"; break;
            case MHIP_ATTR_STRING: o << "String(\"" << s << "\")"; break;
            default: o << "DType(" << dtype_name(dtype) << ")"; break;
        }
        return o.str();
    }
};

struct TensorRef {
    std::string id;
    int dtype = MHIP_DTYPE_F32;
    Shape shape;
};

struct Invocation {
    std::string id;
    std::string kernel;
    std::vector<TensorRef> inputs, outputs;
    std::map<std::string, Attr> attrs;
    int64_t deadline = -1;
};

// ---- attribute readers (src/executor.rs:1141-1185) ----
float attr_float(const Invocation& inv, const char* key, float dflt) {
    auto it = inv.attrs.find(key);
    if (it != inv.attrs.end() && it->second.kind == MHIP_ATTR_FLOAT) return static_cast<float>(it->second.f);
    return dflt;
}

std::optional<float> attr_float_opt(const Invocation& inv, const char* key) {
    auto it = inv.attrs.find(key);
    if (it == inv.attrs.end()) return std::nullopt;
    if (it->second.kind == MHIP_ATTR_FLOAT) return static_cast<float>(it->second.f);
    raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, std::string(key) + " " + it->second.debug() + " must be a float");
}

std::optional<uint64_t> attr_integer(const Invocation& inv, const char* key) {
    auto it = inv.attrs.find(key);
    if (it != inv.attrs.end() && it->second.kind == MHIP_ATTR_INTEGER && it->second.i >= 0)
        return static_cast<uint64_t>(it->second.i);
    return std::nullopt;
}

bool attr_bool(const Invocation& inv, const char* key, bool dflt) {
    auto it = inv.attrs.find(key);
    if (it != inv.attrs.end() && it->second.kind == MHIP_ATTR_BOOLEAN) return it->second.b;
    return dflt;
}

const Attr* attr(const Invocation& inv, const char* key) {
    auto it = inv.attrs.find(key);
    return it == inv.attrs.end() ? nullptr : &it->second;
}

// A positive integer attribute, absent -> nullopt, anything else refused.
std::optional<uint64_t> attr_positive(const Invocation& inv, const char* key, const char* what) {
    const Attr* a = attr(inv, key);
    if (!a) return std::nullopt;
    if (a->kind == MHIP_ATTR_INTEGER && a->i > 0) return static_cast<uint64_t>(a->i);
    raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED,
          std::string(what) + " " + key + " " + a->debug() + " must be a positive integer");
}

struct Observation {
    int kind;
    std::string kernel, invocation;
    int error;
};

}  // namespace

// What a step capture read and wrote (src/executor.rs:339-380): each
// resource's buffer as captured, and the vocabulary of every embedding
// lookup's ids, which a replay checks on the host.
struct Recording {
    std::map<std::string, std::pair<void*, size_t>> resources;
    std::map<std::string, uint64_t> embedding_ids;
    bool has_embedding = false;
};

struct CapturedStep {
    mhip_graph* graph = nullptr;
    Recording recording;
};

struct mhip_executor {
    mhip_ctx* ctx = nullptr;
    std::unique_ptr<Recording> capture;  // while a step capture is recording
    std::map<std::string, CapturedStep> captures;
    uint64_t next_capture = 0;
    std::string device_id, provider_name;
    std::mutex mu;
    std::map<std::string, BufferPtr> storage;
    std::map<uint64_t, std::pair<mhip_kernel_error, std::string>> results;
    uint64_t next_handle = 1;
    std::deque<Observation> observations;
    bool sync_nodes = false;
    // Deferred device checks: the failure flags of embedding and softmax are
    // read at the next materialisation (a tensor read, a greedy selection,
    // a capture's start or an explicit check) instead of after each dispatch.
    bool deferred_checks = false;
    std::string pending_check;  // the first dispatch not yet checked
    uint64_t pending_count = 0;
    // The gate product of gated-matmul's matmul path, reused by every call
    // (stream order makes that safe) and grown when a call needs more; an
    // outgrown buffer that a captured step may still use stays allocated
    // until the executor is destroyed.
    BufferPtr gate_product;
    std::vector<BufferPtr> retired_gate_products;

    static constexpr size_t kObservationCapacity = 4096;

    // The failure-flag check after a dispatch that can raise one: now (the
    // reference's order, src/kernels.rs:3946-3968 and :4360), or noted for
    // flush_checks when checks are deferred.
    void device_check(const Invocation& inv) {
        if (deferred_checks) {
            if (pending_count++ == 0)
                pending_check = "'" + inv.kernel + "' invocation '" + inv.id + "'";
            return;
        }
        mhip_status st = mhip_check_flags(ctx, nullptr);
        if (st != MHIP_OK) raise(map_status(st), mhip_last_error_detail());
    }

    // Reads the flags once for every deferred check; a failure names the
    // first unchecked dispatch and how many share the check.
    void flush_checks() {
        if (pending_count == 0) return;
        const std::string first = pending_check;
        const uint64_t count = pending_count;
        pending_check.clear();
        pending_count = 0;
        mhip_status st = mhip_check_flags(ctx, nullptr);
        if (st != MHIP_OK)
            raise(map_status(st), std::string(mhip_last_error_detail()) +
                                      " (deferred check of " + std::to_string(count) +
                                      " dispatch(es) from " + first + ")");
    }

    void observe(int kind, const Invocation& inv, int error = 0) {
        observations.push_back({kind, inv.kernel, inv.id, error});
        if (observations.size() > 2 * kObservationCapacity)
            observations.erase(observations.begin(),
                               observations.begin() + (observations.size() - kObservationCapacity));
    }

    Buffer& get(const Invocation& inv, size_t index) {
        if (index >= inv.inputs.size())
            raise(MHIP_KERNEL_EXECUTION_FAILED, "missing input at index " + std::to_string(index));
        auto it = storage.find(inv.inputs[index].id);
        if (it == storage.end())
            raise(MHIP_KERNEL_EXECUTION_FAILED,
                  "no materialized data for input resource " + inv.inputs[index].id);
        return *it->second;
    }

    // The output allocation: the offered buffer when its size matches
    // (`alloc_output`, src/kernels.rs:2342-2355), else a fresh one.
    BufferPtr alloc_output(BufferPtr& offered, const Shape& shape, int dtype) {
        const size_t bytes = numel(shape) * dtype_size(dtype);
        if (offered && offered->bytes == bytes && !offered->compact) {
            BufferPtr out = std::move(offered);
            out->shape = shape;
            out->dtype = dtype;
            return out;
        }
        return std::make_unique<Buffer>(ctx, bytes, shape, dtype);
    }

    static void require_f32(const Buffer& b, const char* what) {
        if (b.dtype != MHIP_DTYPE_F32)
            raise(MHIP_KERNEL_DTYPE_UNSUPPORTED,
                  std::string(what) + " reads f32 operands, got " + dtype_name(b.dtype));
    }

    static std::pair<uint64_t, uint64_t> rows_cols(const Buffer& b) {
        if (b.shape.size() != 2)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "expected rank-2 tensor, got shape " + fmt_shape(b.shape));
        return {b.shape[0], b.shape[1]};
    }

    // ---- Kernels (src/kernels.rs wrappers) ----

    BufferPtr op_add(const Buffer& a, const Buffer& b, BufferPtr& offered) {
        require_f32(a, "add");
        require_f32(b, "add");
        if (a.shape == b.shape) {
            BufferPtr out = alloc_output(offered, a.shape, MHIP_DTYPE_F32);
            check(mhip_add_f32(ctx, a.f(), b.f(), out->f(), numel(a.shape)));
            return out;
        }
        if (a.shape.empty()) raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "add expects at least one dimension");
        const uint64_t cols = a.shape.back();
        if (!(b.shape == Shape{cols} || b.shape == Shape{1, cols}))
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "add expects b to match a's shape " + fmt_shape(a.shape) + " or broadcast as [" +
                      std::to_string(cols) + "]/[1, " + std::to_string(cols) + "], got " +
                      fmt_shape(b.shape));
        BufferPtr out = alloc_output(offered, a.shape, MHIP_DTYPE_F32);
        check(mhip_bias_add_f32(ctx, a.f(), b.f(), out->f(), cols, numel(a.shape)));
        return out;
    }

    BufferPtr op_mul(const Buffer& a, const Buffer& b, BufferPtr& offered) {
        require_f32(a, "mul");
        require_f32(b, "mul");
        // A [1] second operand multiplies every element (src/executor.rs:1923-1932).
        if (b.shape == Shape{1} && a.shape != b.shape) {
            BufferPtr out = alloc_output(offered, a.shape, MHIP_DTYPE_F32);
            check(mhip_mul_scalar_f32(ctx, a.f(), b.f(), out->f(), numel(a.shape)));
            return out;
        }
        if (a.shape != b.shape)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "shape mismatch: " + fmt_shape(a.shape) + " vs " + fmt_shape(b.shape));
        BufferPtr out = alloc_output(offered, a.shape, MHIP_DTYPE_F32);
        check(mhip_mul_f32(ctx, a.f(), b.f(), out->f(), numel(a.shape)));
        return out;
    }

    BufferPtr op_silu(const Buffer& x, BufferPtr& offered) {
        require_f32(x, "silu");
        BufferPtr out = alloc_output(offered, x.shape, MHIP_DTYPE_F32);
        check(mhip_silu_f32(ctx, x.f(), out->f(), numel(x.shape)));
        return out;
    }

    BufferPtr op_silu_mul(const Buffer& g, const Buffer& u, BufferPtr& offered) {
        require_f32(g, "silu-mul");
        require_f32(u, "silu-mul");
        if (g.shape != u.shape)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "shape mismatch: " + fmt_shape(g.shape) + " vs " + fmt_shape(u.shape));
        BufferPtr out = alloc_output(offered, g.shape, MHIP_DTYPE_F32);
        check(mhip_silu_mul_f32(ctx, g.f(), u.f(), out->f(), numel(g.shape)));
        return out;
    }

    // src/kernels.rs:3833-3997; `scale` in place (src/executor.rs:1502-1518).
    BufferPtr op_embedding(const Invocation& inv, const Buffer& table, const Buffer& ids,
                           BufferPtr& offered) {
        auto [vocab, dim] = rows_cols(table);
        require_f32(table, "the embedding lookup's table");
        require_f32(ids, "the embedding lookup's ids");
        const std::optional<float> factor = attr_float_opt(inv, "scale");
        const uint64_t num = numel(ids.shape);
        BufferPtr out = alloc_output(offered, Shape{num, dim}, MHIP_DTYPE_F32);
        check(table.compact
                  ? mhip_embedding_bf16w_f32(ctx, table.h(), vocab, dim, ids.f(), num, out->f())
                  : mhip_embedding_f32(ctx, table.f(), vocab, dim, ids.f(), num, out->f()));
        if (capture) {
            // A captured step checks its ids on the host at each replay and
            // the flag after its first run.
            capture->has_embedding = true;
            capture->embedding_ids[inv.inputs[1].id] = vocab;
        } else {
            device_check(inv);
        }
        if (factor) check(mhip_scale_f32(ctx, out->f(), out->f(), *factor, num * dim));
        return out;
    }

    // src/executor.rs:1519-1562, src/kernels.rs:4013-4104.
    BufferPtr op_rmsnorm(const Invocation& inv, BufferPtr& offered) {
        const Buffer& input = get(inv, 0);
        const Buffer* weight = inv.inputs.size() == 1 ? nullptr : &get(inv, 1);
        if (const Attr* ws = attr(inv, "with_scale"); ws && ws->kind == MHIP_ATTR_BOOLEAN &&
                                                     ws->b != (weight != nullptr))
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED,
                  std::string("rmsnorm with_scale ") + (ws->b ? "true" : "false") +
                      " contradicts its " + std::to_string(inv.inputs.size()) + " input(s)");
        auto hc = attr_positive(inv, "head_count", "rmsnorm");
        auto hd = attr_positive(inv, "head_dimension", "rmsnorm");
        if (hc.has_value() != hd.has_value())
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "rmsnorm head_count and head_dimension go together");
        const float eps = attr_float(inv, "epsilon", 1e-6f);
        require_f32(input, "rmsnorm");
        if (weight) require_f32(*weight, "rmsnorm");
        if (input.shape.empty())
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "RMSNorm expects at least one dimension");
        const uint64_t row_width = input.shape.back();
        uint64_t cols = row_width;
        if (hc) {
            if (*hc * *hd != row_width)
                raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                      "RMSNorm's " + std::to_string(*hc) + " heads of " + std::to_string(*hd) +
                          " do not tile rows of " + std::to_string(row_width));
            cols = *hd;
        }
        const uint64_t len = numel(input.shape);
        if (cols == 0 || len % cols != 0)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "RMSNorm data length " + std::to_string(len) +
                      " is not divisible by hidden dimension " + std::to_string(cols));
        const uint64_t rows = len / cols;
        uint64_t stride = 0;
        if (weight) {
            if (weight->shape == Shape{cols} || weight->shape == Shape{1, cols}) {
                stride = 0;
            } else if (!hc && (weight->shape == input.shape || weight->shape == Shape{rows, cols})) {
                stride = cols;
            } else {
                raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                      "RMSNorm weight shape must be [" + std::to_string(cols) + "], [1, " +
                          std::to_string(cols) + "], input shape " + fmt_shape(input.shape) +
                          ", or [" + std::to_string(rows) + ", " + std::to_string(cols) +
                          "], got " + fmt_shape(weight->shape));
            }
        }
        if (!(eps > 0.0f)) raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "RMSNorm epsilon must be positive");
        BufferPtr out = alloc_output(offered, input.shape, MHIP_DTYPE_F32);
        check(mhip_rmsnorm_f32(ctx, input.f(), weight ? weight->f() : nullptr, out->f(), rows, cols,
                               stride, eps));
        return out;
    }

    // src/executor.rs:1563-1666, src/kernels.rs:4224-4355.
    BufferPtr op_rope(const Invocation& inv, BufferPtr& offered) {
        const Buffer& input = get(inv, 0);
        mhip_rope_params p;
        const float base = attr_float(inv, "base", 10000.0f);
        const float scale = attr_float(inv, "scale", 1.0f);
        auto dimension = attr_integer(inv, "dimension");
        if (!dimension) raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "dimension");
        if (const Attr* pm = attr(inv, "position_mode"); pm && pm->kind == MHIP_ATTR_STRING &&
                                                        pm->s != "sequential")
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "position_mode '" + pm->s + "' is not implemented");
        uint64_t offset = 0;
        if (const Attr* po = attr(inv, "position_offset")) {
            if (po->kind != MHIP_ATTR_INTEGER)
                raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "position_offset must be an integer");
            if (po->i < 0)
                raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED,
                      "position_offset " + std::to_string(po->i) + " must not be negative");
            offset = static_cast<uint64_t>(po->i);
        }
        const uint64_t head_count = attr_integer(inv, "head_count").value_or(1);
        uint32_t half_split = 0;
        if (const Attr* rp = attr(inv, "rotation_pairing")) {
            if (rp->kind != MHIP_ATTR_STRING)
                raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "rotation_pairing must be a string");
            if (rp->s == "interleaved") half_split = 0;
            else if (rp->s == "half_split") half_split = 1;
            else raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "rotation_pairing '" + rp->s + "' is not implemented");
        }
        mhip_rope_params_default(&p, *dimension, head_count);
        p.base = base;
        p.scale = scale;
        p.position_offset = offset;
        p.half_split = half_split;
        apply_frequency_scaling(inv, *dimension, base, &p);
        if (const Attr* prf = attr(inv, "partial_rotary_factor")) {
            if (!(prf->kind == MHIP_ATTR_FLOAT && prf->f > 0.0 && prf->f <= 1.0))
                raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED,
                      "partial_rotary_factor " + prf->debug() + " must be a float in (0, 1]");
            p.rotated_pairs = static_cast<uint64_t>(std::floor(prf->f * static_cast<double>(*dimension) / 2.0));
        }
        require_f32(input, "rope");
        auto [rows, cols] = rows_cols(input);
        BufferPtr out = alloc_output(offered, input.shape, MHIP_DTYPE_F32);
        check(mhip_rope_f32(ctx, input.f(), out->f(), rows, cols, &p));
        return out;
    }

    // Banded (Llama-3 style) and YaRN frequency scaling. The reference reads
    // them with magnetar_core's `RopeYarnFrequencyScaling::from_attributes` /
    // `RopeBandedFrequencyScaling::from_attributes` (absent here); this
    // restates them: `frequency_scaling` names the scheme, YaRN wins.
    // YaRN's correction range is the published one (find_correction_dim of
    // beta_fast / beta_slow, floored / ceiled when `truncate`, clamped to
    // [0, dimension/2 - 1]), computed in f64 like the reference's.
    static void apply_frequency_scaling(const Invocation& inv, uint64_t dimension, float base,
                                        mhip_rope_params* p) {
        const Attr* fs = attr(inv, "frequency_scaling");
        if (!fs) return;
        if (fs->kind != MHIP_ATTR_STRING)
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "frequency_scaling must be a string");
        auto num = [&](const char* key, double dflt) -> double {
            const Attr* a = attr(inv, key);
            if (!a) return dflt;
            if (a->kind == MHIP_ATTR_FLOAT) return a->f;
            if (a->kind == MHIP_ATTR_INTEGER) return static_cast<double>(a->i);
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, std::string(key) + " " + a->debug() + " must be a number");
        };
        const double factor = num("factor", 0.0);
        if (!(factor > 0.0) || !std::isfinite(factor))
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "frequency scaling factor must be positive");
        const double ctx_len = num("original_context_length", 0.0);
        if (!(ctx_len > 0.0))
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "original_context_length must be positive");
        if (fs->s == "yarn") {
            const double beta_fast = num("beta_fast", 32.0), beta_slow = num("beta_slow", 1.0);
            const bool truncate = attr_bool(inv, "truncate", true);
            auto corr = [&](double rotations) {
                return static_cast<double>(dimension) * std::log(ctx_len / (rotations * 2.0 * 3.14159265358979323846)) /
                       (2.0 * std::log(static_cast<double>(base)));
            };
            double low = corr(beta_fast), high = corr(beta_slow);
            if (truncate) {
                low = std::floor(low);
                high = std::ceil(high);
            }
            low = std::max(low, 0.0);
            high = std::min(high, static_cast<double>(dimension) - 1.0);
            p->yarn_factor = static_cast<float>(factor);
            p->yarn_low = static_cast<float>(low);
            p->yarn_high = static_cast<float>(high);
            p->amplitude = static_cast<float>(num("attention_factor", 1.0));
        } else if (fs->s == "banded") {
            const double low = num("low_freq_factor", 1.0), high = num("high_freq_factor", 4.0);
            if (!(low > 0.0 && high > low))
                raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED,
                      "banded scaling needs 0 < low_freq_factor < high_freq_factor");
            p->banded_factor = static_cast<float>(factor);
            p->low_freq_factor = static_cast<float>(low);
            p->high_freq_factor = static_cast<float>(high);
            p->original_context_length = static_cast<float>(ctx_len);
        } else {
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED,
                  "frequency_scaling '" + fs->s + "' is not implemented");
        }
    }

    // src/kernels.rs:4357-4386.
    BufferPtr op_softmax(const Invocation& inv, const Buffer& x, BufferPtr& offered) {
        // Its failure check reads the device (src/kernels.rs:4360).
        check(mhip::forbid_in_capture(ctx, "softmax"));
        require_f32(x, "softmax");
        auto [rows, cols] = rows_cols(x);
        BufferPtr out = alloc_output(offered, x.shape, MHIP_DTYPE_F32);
        check(mhip_softmax_rows_f32(ctx, x.f(), out->f(), rows, cols));
        device_check(inv);
        return out;
    }

    // matmul / matmul-bias / matmul-residual (src/kernels.rs:5518-5580).
    BufferPtr op_matmul(const Invocation& inv, int addend_mode, BufferPtr& offered) {
        const Buffer& a = get(inv, 0);
        const Buffer& b = get(inv, 1);
        const Buffer* addend = addend_mode ? &get(inv, 2) : nullptr;
        const bool ta = attr_bool(inv, "transpose_a", false);
        const bool tb = attr_bool(inv, "transpose_b", false);
        require_f32_accumulation(inv);
        auto [m, k, n] = matmul_dims(a, b, ta, tb);
        if (addend_mode == 1 && !(addend->shape == Shape{n} || addend->shape == Shape{1, n}))
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "matmul-bias bias shape must be [" + std::to_string(n) + "] or [1, " +
                      std::to_string(n) + "], got " + fmt_shape(addend->shape));
        if (addend_mode == 2 && addend->shape != Shape{m, n})
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "matmul-residual residual shape must be [" + std::to_string(m) + ", " +
                      std::to_string(n) + "], got " + fmt_shape(addend->shape));
        require_f32(a, "matmul's a");
        require_f32(b, "matmul's b");
        if (addend) require_f32(*addend, "a fused matmul's addend");
        BufferPtr out = alloc_output(offered, Shape{m, n}, MHIP_DTYPE_F32);
        check(matmul(a, b, out->f(), m, k, n, ta, tb, addend ? addend->f() : nullptr, addend_mode));
        return out;
    }

    // A product whose b is an f32 or a compact weight.
    mhip_status matmul(const Buffer& a, const Buffer& b, float* out, uint64_t m, uint64_t k,
                       uint64_t n, bool ta, bool tb, const float* addend, int mode) {
        if (b.compact)
            return mhip_matmul_bf16w_f32(ctx, a.f(), b.h(), out, m, k, n, ta, tb, addend, mode);
        return mhip_matmul_f32(ctx, a.f(), b.f(), out, m, k, n, ta, tb, addend, mode);
    }

    static std::tuple<uint64_t, uint64_t, uint64_t> matmul_dims(const Buffer& a, const Buffer& b,
                                                                bool ta, bool tb) {
        auto [ar, ac] = rows_cols(a);
        auto [br, bc] = rows_cols(b);
        const uint64_t m = ta ? ac : ar, k = ta ? ar : ac;
        const uint64_t k2 = tb ? bc : br, n = tb ? br : bc;
        if (k != k2)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "matmul inner dimension mismatch: " + std::to_string(k) + " vs " + std::to_string(k2));
        return {m, k, n};
    }

    // src/executor.rs:1238-1249.
    static void require_f32_accumulation(const Invocation& inv) {
        if (const Attr* acc = attr(inv, "accumulation_dtype");
            acc && acc->kind == MHIP_ATTR_DTYPE && acc->dtype != MHIP_DTYPE_F32)
            raise(MHIP_KERNEL_DTYPE_UNSUPPORTED,
                  std::string("the HIP Provider only accumulates in f32; requested ") +
                      dtype_name(acc->dtype));
    }

    // gated-matmul: silu(a . gate) * (a . up), as the two matmuls and
    // silu-mul it fuses (src/executor.rs:1484-1494). A few rows (decode) run
    // as one GEMV set whose reduction writes silu(gate) * up: no temporaries,
    // bit-identical to the two matmuls and silu-mul.
    BufferPtr op_gated_matmul(const Invocation& inv, BufferPtr& offered) {
        const Buffer& a = get(inv, 0);
        const Buffer& gate = get(inv, 1);
        const Buffer& up = get(inv, 2);
        const bool ta = attr_bool(inv, "transpose_a", false);
        const bool tb = attr_bool(inv, "transpose_b", false);
        require_f32_accumulation(inv);
        auto [m, k, n] = matmul_dims(a, gate, ta, tb);
        auto [m2, k2, n2] = matmul_dims(a, up, ta, tb);
        (void)k2;
        if (m2 != m || n2 != n)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "gated-matmul gate " + fmt_shape(gate.shape) + " and up " + fmt_shape(up.shape) +
                      " disagree");
        require_f32(a, "gated-matmul");
        require_f32(gate, "gated-matmul");
        require_f32(up, "gated-matmul");
        if (!ta && !tb && gate.compact == up.compact && m > 0 && n > 0 && k > 0) {
            BufferPtr out = alloc_output(offered, Shape{m, n}, MHIP_DTYPE_F32);
            const mhip::GemvTarget t[2] = {{gate.ptr, n, out->f()}, {up.ptr, n, nullptr}};
            const mhip_status st =
                mhip::gemv_set_f32(ctx, a.f(), m, k, t, 2, mhip::kGemvSiluMul, nullptr, gate.compact);
            if (st == MHIP_OK) return out;
            if (st != MHIP_LAYOUT_UNSUPPORTED) check(st);
            offered = std::move(out);  // reused below
        }
        // The gate product, then the up product with silu(gate) applied to
        // each finished sum as it is stored.
        const size_t bytes = std::max<size_t>(m * n * 4, 4);
        if (!gate_product || gate_product->bytes < bytes) {
            BufferPtr grown = std::make_unique<Buffer>(ctx, bytes, Shape{m, n}, MHIP_DTYPE_F32);
            if (gate_product) {
                if (captures.empty()) {
                    check(mhip_sync(ctx));  // earlier calls may still use it
                    gate_product.reset();
                } else {
                    retired_gate_products.push_back(std::move(gate_product));
                }
            }
            gate_product = std::move(grown);
        }
        BufferPtr out = alloc_output(offered, Shape{m, n}, MHIP_DTYPE_F32);
        check(matmul(a, gate, gate_product->f(), m, k, n, ta, tb, nullptr, 0));
        check(mhip::matmul_gated_f32(ctx, a.f(), up.ptr, up.compact, out->f(), m, k, n, ta, tb,
                                     gate_product->f()));
        return out;
    }

    // src/executor.rs:1667-1796, src/kernels.rs:6505-6628.
    BufferPtr op_attention(const Invocation& inv, BufferPtr& offered) {
        const Buffer& q = get(inv, 0);
        const Buffer& k = get(inv, 1);
        const Buffer& v = get(inv, 2);
        auto head_count = attr_integer(inv, "head_count");
        if (!head_count) raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "head_count");
        auto head_dim = attr_integer(inv, "head_dimension");
        if (!head_dim) raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "head_dimension");
        auto kv_heads = attr_integer(inv, "kv_head_count");
        auto window = attr_integer(inv, "window_size");
        const bool causal = attr_bool(inv, "causal", false);
        if (const Attr* mk = attr(inv, "attention_mask_kind"); mk && mk->kind == MHIP_ATTR_STRING) {
            bool expected;
            if (mk->s == "causal") expected = true;
            else if (mk->s == "bidirectional") expected = false;
            else raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "attention_mask_kind '" + mk->s + "' is not implemented");
            if (expected != causal)
                raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED,
                      "attention_mask_kind '" + mk->s + "' is inconsistent with causal=" +
                          (causal ? "true" : "false"));
        }
        auto key_count = attr_integer(inv, "key_count");
        auto scale = attr_float_opt(inv, "scale");
        auto value_dim = attr_positive(inv, "value_head_dimension", "attention");
        for (const char* unsupported : {"value_head_stride", "latent_kv_width"})
            if (attr(inv, unsupported))
                raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED,
                      std::string("attention ") + unsupported + " is not implemented by this Provider");
        require_f32(q, "attention");
        require_f32(k, "attention");
        require_f32(v, "attention");
        const uint64_t H = *head_count, d = *head_dim;
        const uint64_t vd = value_dim.value_or(d);
        if (vd == d && k.shape != v.shape)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "shape mismatch: " + fmt_shape(k.shape) + " vs " + fmt_shape(v.shape));
        if (scale && !(std::isfinite(*scale) && *scale > 0.0f)) {
            std::ostringstream o;
            o << "attention scale " << *scale << " must be finite and positive";
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, o.str());
        }
        const uint64_t Hkv = kv_heads.value_or(H);
        if (H == 0 || d == 0 || Hkv == 0 || vd == 0)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "head_count, kv_head_count, and head_dimension must all be positive");
        if (H % Hkv != 0)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "head_count " + std::to_string(H) + " must be an exact multiple of kv_head_count " +
                      std::to_string(Hkv));
        if (window && *window == 0)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "window_size must be positive; a zero window admits no keys");
        if (window && !causal)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "window_size is only defined for causal attention");
        auto [seq, q_dim] = rows_cols(q);
        auto [kv_rows, kv_dim] = rows_cols(k);
        const uint64_t kv_seq = key_count.value_or(kv_rows);
        if (kv_seq > kv_rows)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "key_count " + std::to_string(kv_seq) + " exceeds the " + std::to_string(kv_rows) +
                      " rows of K/V");
        if (seq > kv_seq)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "q sequence length " + std::to_string(seq) + " cannot exceed k/v sequence length " +
                      std::to_string(kv_seq));
        if (H * d != q_dim)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "head_count * head_dimension must equal q row width " + std::to_string(q_dim) +
                      ", got " + std::to_string(H) + " * " + std::to_string(d));
        if (Hkv * d != kv_dim)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "kv_head_count * head_dimension must equal k/v row width " + std::to_string(kv_dim) +
                      ", got " + std::to_string(Hkv) + " * " + std::to_string(d));
        auto [v_rows, v_dim] = rows_cols(v);
        if (v_rows != kv_rows || Hkv * vd != v_dim)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "v must hold " + std::to_string(kv_rows) + " rows of kv_head_count * value_dimension = " +
                      std::to_string(Hkv) + " * " + std::to_string(vd) + ", got " + fmt_shape(v.shape));
        mhip_attention_params p{};
        p.seq_len = seq;
        p.kv_rows = kv_rows;
        p.kv_seq_len = kv_seq;
        p.head_count = H;
        p.kv_head_count = Hkv;
        p.head_dimension = d;
        p.value_dimension = vd;
        p.causal = causal;
        p.window_size = window ? static_cast<int64_t>(*window) : -1;
        p.scale = scale.value_or(0.0f);
        p.batch = 1;
        p.bounded_key_count = key_count.has_value() ? 1 : 0;
        BufferPtr out = alloc_output(offered, Shape{seq, H * vd}, MHIP_DTYPE_F32);
        check(mhip_attention_f32(ctx, q.f(), k.f(), v.f(), out->f(), &p));
        return out;
    }

    // concat along rows (src/kernels.rs:3058-3101): b's rows after a's.
    BufferPtr op_concat(const Invocation& inv, BufferPtr& offered) {
        const Buffer& a = get(inv, 0);
        const Buffer& b = get(inv, 1);
        if (const Attr* ax = attr(inv, "axis"); ax && !(ax->kind == MHIP_ATTR_STRING && ax->s == "rows"))
            raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "concat axis must be 'rows'");
        require_f32(a, "concat");
        require_f32(b, "concat");
        if (a.shape.empty()) raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "concat expects a to have at least one dimension");
        if (b.shape.empty()) raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "concat expects b to have at least one dimension");
        if (Shape(a.shape.begin() + 1, a.shape.end()) != Shape(b.shape.begin() + 1, b.shape.end()))
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "concat expects a and b to share trailing dimensions, got " + fmt_shape(a.shape) +
                      " and " + fmt_shape(b.shape));
        Shape shape = a.shape;
        shape[0] = a.shape[0] + b.shape[0];
        BufferPtr out = alloc_output(offered, shape, MHIP_DTYPE_F32);
        check(mhip_copy(ctx, out->ptr, a.ptr, a.bytes));
        check(mhip_copy(ctx, static_cast<char*>(out->ptr) + a.bytes, b.ptr, b.bytes));
        return out;
    }

    // add-half / mul-half on 2-byte device buffers (src/executor.rs:1970-2013).
    BufferPtr op_half(const Invocation& inv, bool mul, BufferPtr& offered) {
        check(mhip::forbid_in_capture(ctx, "a half-precision Kernel"));
        const Buffer& a = get(inv, 0);
        const Buffer& b = get(inv, 1);
        const int dtype = inv.inputs[0].dtype;
        if (dtype != MHIP_DTYPE_F16 && dtype != MHIP_DTYPE_BF16)
            raise(MHIP_KERNEL_DTYPE_UNSUPPORTED,
                  std::string("add-half/mul-half take Float16 or BrainFloat16, got ") + dtype_name(dtype));
        if (a.shape != b.shape)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "shape mismatch: " + fmt_shape(a.shape) + " vs " + fmt_shape(b.shape));
        const mhip_half_dtype hd = dtype == MHIP_DTYPE_F16 ? MHIP_F16 : MHIP_BF16;
        const uint64_t n = numel(a.shape);
        // Operands stored as f32 are encoded on the device first; operands of
        // the other half format are refused.
        std::unique_ptr<Buffer> ta, tb;
        auto as_half = [&](const Buffer& x, std::unique_ptr<Buffer>& tmp) -> const uint16_t* {
            if (x.dtype == dtype) return x.h();
            if (x.dtype != MHIP_DTYPE_F32)
                raise(MHIP_KERNEL_DTYPE_UNSUPPORTED,
                      std::string("operand stored as ") + dtype_name(x.dtype) + ", expected " + dtype_name(dtype));
            tmp = std::make_unique<Buffer>(ctx, n * 2, x.shape, dtype);
            check(mhip_encode_half(ctx, x.f(), tmp->h(), n, hd));
            return tmp->h();
        };
        const uint16_t* ha = as_half(a, ta);
        const uint16_t* hb = as_half(b, tb);
        const int out_dtype = inv.outputs.empty() ? dtype : inv.outputs[0].dtype;
        if (out_dtype == dtype) {
            BufferPtr out = alloc_output(offered, a.shape, dtype);
            check(mul ? mhip_mul_half(ctx, ha, hb, out->h(), n, hd) : mhip_add_half(ctx, ha, hb, out->h(), n, hd));
            if (ta || tb) check(mhip_sync(ctx));
            return out;
        }
        if (out_dtype != MHIP_DTYPE_F32)
            raise(MHIP_KERNEL_DTYPE_UNSUPPORTED, "add-half/mul-half output must be its input dtype or Float32");
        Buffer tmp(ctx, n * 2, a.shape, dtype);
        check(mul ? mhip_mul_half(ctx, ha, hb, tmp.h(), n, hd) : mhip_add_half(ctx, ha, hb, tmp.h(), n, hd));
        BufferPtr out = alloc_output(offered, a.shape, MHIP_DTYPE_F32);
        check(mhip_decode_half(ctx, tmp.h(), out->f(), n, hd));
        check(mhip_sync(ctx));
        return out;
    }

    // src/executor.rs:1422-2027.
    BufferPtr dispatch(const Invocation& inv, BufferPtr& offered) {
        const std::string& name = inv.kernel;
        if (name == "matmul") return op_matmul(inv, 0, offered);
        if (name == "matmul-bias") return op_matmul(inv, 1, offered);
        if (name == "matmul-residual") return op_matmul(inv, 2, offered);
        if (name == "gated-matmul") return op_gated_matmul(inv, offered);
        if (name == "silu-mul") return op_silu_mul(get(inv, 0), get(inv, 1), offered);
        if (name == "embedding") return op_embedding(inv, get(inv, 0), get(inv, 1), offered);
        if (name == "rmsnorm") return op_rmsnorm(inv, offered);
        if (name == "rope") return op_rope(inv, offered);
        if (name == "attention") return op_attention(inv, offered);
        if (name == "softmax") return op_softmax(inv, get(inv, 0), offered);
        if (name == "silu") return op_silu(get(inv, 0), offered);
        if (name == "add") return op_add(get(inv, 0), get(inv, 1), offered);
        if (name == "mul") return op_mul(get(inv, 0), get(inv, 1), offered);
        if (name == "concat") return op_concat(inv, offered);
        if (name == "residual-add") return op_add(get(inv, 0), get(inv, 1), offered);
        if (name == "add-half") return op_half(inv, false, offered);
        if (name == "mul-half") return op_half(inv, true, offered);
        raise(MHIP_KERNEL_NOT_FOUND, name);
    }

    BufferPtr clone(const Buffer& b) {
        BufferPtr copy = std::make_unique<Buffer>(ctx, b.bytes, b.shape, b.dtype);
        copy->compact = b.compact;
        check(mhip_copy(ctx, copy->ptr, b.ptr, b.bytes));
        return copy;
    }

    // kv-write (src/executor.rs:1366-1420, src/kernels.rs:2270-2325): rows
    // into the store's own buffer when the output is the store (a KV
    // history), otherwise into a copy stored under the output. The store goes
    // back under the output id either way; a failed write leaves its rows.
    void run_kv_write(const Invocation& inv) {
        expand_compact_inputs(inv);
        const std::optional<uint64_t> row_offset = attr_integer(inv, "row_offset");
        if (!row_offset) raise(MHIP_KERNEL_ATTRIBUTE_UNSUPPORTED, "row_offset");
        if (inv.inputs.size() < 1) raise(MHIP_KERNEL_EXECUTION_FAILED, "missing input at index 0");
        if (inv.inputs.size() < 2) raise(MHIP_KERNEL_EXECUTION_FAILED, "missing input at index 1");
        if (inv.outputs.empty()) raise(MHIP_KERNEL_EXECUTION_FAILED, "missing output at index 0");
        const std::string& store_id = inv.inputs[0].id;
        const std::string& rows_id = inv.inputs[1].id;
        const std::string& out_id = inv.outputs[0].id;
        auto it = storage.find(store_id);
        if (it == storage.end())
            raise(MHIP_KERNEL_EXECUTION_FAILED, "no materialized data for input resource " + store_id);
        BufferPtr store;
        if (out_id == store_id) {
            store = std::move(it->second);
            storage.erase(it);
        } else {
            store = clone(*it->second);
        }
        std::string error;
        mhip_kernel_error code = MHIP_KERNEL_OK;
        try {
            auto rit = storage.find(rows_id);
            if (rit == storage.end())
                raise(MHIP_KERNEL_EXECUTION_FAILED, "no materialized data for input resource " + rows_id);
            const Buffer& rows = *rit->second;
            require_f32(*store, "kv-write");
            require_f32(rows, "kv-write");
            const auto [capacity, width] = rows_cols(*store);
            const auto [count, row_width] = rows_cols(rows);
            if (row_width != width)
                raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "kv-write rows have width " +
                                                         std::to_string(row_width) + ", the store " +
                                                         std::to_string(width));
            check(mhip_kv_write_f32(ctx, store->f(), capacity, width, rows.f(), count, *row_offset));
        } catch (const KernelFailure& f) {
            code = f.code;
            error = f.detail;
        }
        storage[out_id] = std::move(store);
        if (code != MHIP_KERNEL_OK) raise(code, error);
    }

    // The same values as a compact buffer, stored as f32 (widened on the
    // device).
    BufferPtr expand(const Buffer& b) {
        const uint64_t n = numel(b.shape);
        BufferPtr f = std::make_unique<Buffer>(ctx, n * 4, b.shape, MHIP_DTYPE_F32);
        check(mhip_decode_half(ctx, b.h(), f->f(), n, MHIP_BF16));
        return f;
    }

    // expand_unsupported_compact_inputs (src/executor.rs:1323-1364): every
    // compact input is stored as f32 for good unless the Kernel reads it
    // compact -- the matmul family's b, gated-matmul's gate and up, the
    // embedding lookup's table.
    void expand_compact_inputs(const Invocation& inv) {
        const std::string& name = inv.kernel;
        auto reads_compact = [&](size_t index) {
            if (name == "matmul" || name == "matmul-bias" || name == "matmul-residual") return index == 1;
            if (name == "gated-matmul") return index == 1 || index == 2;
            if (name == "embedding") return index == 0;
            return false;
        };
        for (size_t i = 0; i < inv.inputs.size(); ++i) {
            auto it = storage.find(inv.inputs[i].id);
            if (reads_compact(i) || it == storage.end() || !it->second->compact) continue;
            try {
                it->second = expand(*it->second);
            } catch (const KernelFailure& f) {
                raise(MHIP_KERNEL_EXECUTION_FAILED,
                      "expanding compact input " + std::to_string(i) + " of " + name + ": " + f.detail);
            }
        }
    }

    // run_invocation_uncaptured (src/executor.rs:1268-1321): the overwritten
    // output's buffer is offered unless an input reads it; on failure it is
    // put back so the resource keeps its value.
    void run(const Invocation& inv) {
        expand_compact_inputs(inv);
        if (inv.kernel == "kv-write") {
            run_kv_write(inv);
            record(inv);
            if (sync_nodes && !capture) check(mhip_sync(ctx));
            return;
        }
        if (inv.outputs.empty())
            raise(MHIP_KERNEL_EXECUTION_FAILED, "missing output at index 0");
        const std::string& out_id = inv.outputs[0].id;
        BufferPtr offered;
        bool read_by_input = false;
        for (const auto& in : inv.inputs) read_by_input |= in.id == out_id;
        if (!read_by_input) {
            auto it = storage.find(out_id);
            if (it != storage.end()) {
                offered = std::move(it->second);
                storage.erase(it);
            }
        }
        try {
            BufferPtr out = dispatch(inv, offered);
            storage[out_id] = std::move(out);
        } catch (...) {
            if (offered) storage[out_id] = std::move(offered);
            throw;
        }
        record(inv);
        if (sync_nodes && !capture) check(mhip_sync(ctx));
    }

    // Notes the buffers a captured invocation read and wrote.
    void record(const Invocation& inv) {
        if (!capture) return;
        auto note = [&](const TensorRef& r) {
            auto it = storage.find(r.id);
            if (it != storage.end()) capture->resources[r.id] = {it->second->ptr, it->second->bytes};
        };
        for (const auto& r : inv.inputs) note(r);
        for (const auto& r : inv.outputs) note(r);
    }

    // execute_invocation (src/executor.rs:1191-1233).
    std::pair<mhip_kernel_error, std::string> execute(const Invocation& inv) {
        observe(MHIP_OBS_DISPATCH_STARTED, inv);
        if (inv.deadline == 0) {
            observe(MHIP_OBS_TIMEOUT, inv);
            return {MHIP_KERNEL_TIMEOUT, "deadline of 0 ms"};
        }
        try {
            run(inv);
            observe(MHIP_OBS_DISPATCH_COMPLETED, inv);
            return {MHIP_KERNEL_OK, ""};
        } catch (const KernelFailure& f) {
            observe(MHIP_OBS_DISPATCH_FAILED, inv, f.code);
            return {f.code, f.detail};
        }
    }
};

namespace {

Invocation convert(const mhip_invocation* c) {
    Invocation inv;
    inv.id = c->invocation_id ? c->invocation_id : "";
    inv.kernel = c->kernel_name ? c->kernel_name : "";
    auto refs = [](const mhip_tensor_ref* r, int count) {
        std::vector<TensorRef> out;
        for (int i = 0; i < count; ++i) {
            TensorRef t;
            t.id = r[i].id ? r[i].id : "";
            t.dtype = r[i].dtype;
            if (r[i].shape) t.shape.assign(r[i].shape, r[i].shape + r[i].rank);
            out.push_back(std::move(t));
        }
        return out;
    };
    inv.inputs = refs(c->inputs, c->input_count);
    inv.outputs = refs(c->outputs, c->output_count);
    for (int i = 0; i < c->attribute_count; ++i) {
        const mhip_attribute& a = c->attributes[i];
        Attr v;
        v.kind = a.kind;
        v.f = a.f;
        v.i = a.i;
        v.b = a.b != 0;
        v.s = a.s ? a.s : "";
        v.dtype = a.dtype;
        inv.attrs[a.key ? a.key : ""] = v;
    }
    inv.deadline = c->deadline_millis;
    return inv;
}

mhip_kernel_error finish(mhip_kernel_error code, const std::string& detail) {
    g_detail = detail;
    return code;
}

template <class F>
mhip_kernel_error guarded(F&& f) {
    try {
        f();
        return finish(MHIP_KERNEL_OK, "");
    } catch (const KernelFailure& e) {
        return finish(e.code, e.detail);
    } catch (const std::exception& e) {
        return finish(MHIP_KERNEL_EXECUTION_FAILED, e.what());
    }
}

Shape make_shape(const uint64_t* shape, int rank) {
    if (rank < 0 || rank > 8) raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "tensor rank must be 0..8");
    return shape ? Shape(shape, shape + rank) : Shape();
}

void check_dtype(int dtype) {
    if (dtype != MHIP_DTYPE_F32 && dtype != MHIP_DTYPE_F16 && dtype != MHIP_DTYPE_BF16)
        raise(MHIP_KERNEL_DTYPE_UNSUPPORTED, "unknown dtype " + std::to_string(dtype));
}

}  // namespace

extern "C" {

mhip_status mhip_executor_create(mhip_ctx* ctx, const char* device_id, const char* provider_name,
                                 mhip_executor** out) {
    if (!out) return MHIP_SHAPE_UNSUPPORTED;
    *out = nullptr;
    if (!ctx) return MHIP_DEVICE_UNAVAILABLE;
    auto* ex = new mhip_executor();
    ex->ctx = ctx;
    ex->device_id = device_id ? device_id : "hip:0";
    ex->provider_name = provider_name ? provider_name : "magnetar:provider/hip";
    if (const char* env = std::getenv("MAGNETAR_HIP_SYNC_NODES")) ex->sync_nodes = std::strcmp(env, "1") == 0;
    *out = ex;
    return MHIP_OK;
}

mhip_status mhip_executor_destroy(mhip_executor* ex) {
    if (!ex) return MHIP_OK;
    {
        std::lock_guard<std::mutex> lock(ex->mu);
        if (ex->capture) {
            mhip_capture_abort(ex->ctx);
            ex->capture.reset();
        }
        for (auto& entry : ex->captures) mhip_graph_destroy(entry.second.graph);
        ex->captures.clear();
        mhip_sync(ex->ctx);
        ex->storage.clear();
        ex->gate_product.reset();
        ex->retired_gate_products.clear();
    }
    delete ex;
    return MHIP_OK;
}

const char* mhip_executor_last_detail(void) { return g_detail.c_str(); }

mhip_kernel_error mhip_executor_write_tensor(mhip_executor* ex, const char* id, const uint64_t* shape,
                                             int rank, int dtype, const void* data, size_t bytes) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        check_dtype(dtype);
        Shape s = make_shape(shape, rank);
        const size_t want = numel(s) * dtype_size(dtype);
        if (bytes != want)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  std::to_string(bytes) + " bytes cannot fill a " + dtype_name(dtype) + " tensor of shape " +
                      fmt_shape(s));
        std::lock_guard<std::mutex> lock(ex->mu);
        auto buf = std::make_unique<Buffer>(ex->ctx, want, s, dtype);
        if (want) check(mhip_upload(ex->ctx, buf->ptr, data, want));
        ex->storage[id] = std::move(buf);
    });
}

mhip_kernel_error mhip_executor_write_tensor_values(mhip_executor* ex, const char* id,
                                                    const uint64_t* shape, int rank, int dtype,
                                                    const float* values) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        check_dtype(dtype);
        Shape s = make_shape(shape, rank);
        const uint64_t n = numel(s);
        std::lock_guard<std::mutex> lock(ex->mu);
        auto buf = std::make_unique<Buffer>(ex->ctx, n * dtype_size(dtype), s, dtype);
        if (dtype == MHIP_DTYPE_F32) {
            if (n) check(mhip_upload(ex->ctx, buf->ptr, values, n * 4));
        } else if (n) {
            Buffer staging(ex->ctx, n * 4, s, MHIP_DTYPE_F32);
            check(mhip_upload(ex->ctx, staging.ptr, values, n * 4));
            check(mhip_encode_half(ex->ctx, staging.f(), buf->h(), n,
                                   dtype == MHIP_DTYPE_F16 ? MHIP_F16 : MHIP_BF16));
            check(mhip_sync(ex->ctx));
        }
        ex->storage[id] = std::move(buf);
    });
}

mhip_kernel_error mhip_executor_write_zeroed_tensor(mhip_executor* ex, const char* id,
                                                    const uint64_t* shape, int rank, int dtype) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        check_dtype(dtype);
        Shape s = make_shape(shape, rank);
        std::lock_guard<std::mutex> lock(ex->mu);
        auto buf = std::make_unique<Buffer>(ex->ctx, numel(s) * dtype_size(dtype), s, dtype);
        check(mhip_zero(ex->ctx, buf->ptr, buf->bytes));
        ex->storage[id] = std::move(buf);
    });
}

mhip_kernel_error mhip_executor_write_zeroed_kv_store(mhip_executor* ex, const char* id,
                                                      const uint64_t* shape, int rank,
                                                      int precision, uint64_t head_dimension,
                                                      int* stored) {
    (void)head_dimension;  // used by the quantized stores only
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        if (stored) *stored = 0;
        if (precision != MHIP_KV_F32) return;
        Shape s = make_shape(shape, rank);
        std::lock_guard<std::mutex> lock(ex->mu);
        auto buf = std::make_unique<Buffer>(ex->ctx, numel(s) * 4, s, MHIP_DTYPE_F32);
        check(mhip_zero(ex->ctx, buf->ptr, buf->bytes));
        ex->storage[id] = std::move(buf);
        if (stored) *stored = 1;
    });
}

namespace {

// Downloads `count` values of a compact buffer from value `first` on and
// widens them to f32 on the host.
void download_widened(mhip_ctx* ctx, const Buffer& b, uint64_t first, uint64_t count, float* dst) {
    std::vector<uint16_t> bits(count);
    if (count) check(mhip_download(ctx, bits.data(), b.h() + first, count * 2));
    for (uint64_t i = 0; i < count; ++i) {
        const uint32_t u = static_cast<uint32_t>(bits[i]) << 16;
        std::memcpy(dst + i, &u, 4);
    }
}

}  // namespace

mhip_kernel_error mhip_executor_write_weight_tensor(mhip_executor* ex, const char* id,
                                                    const uint64_t* shape, int rank,
                                                    const float* values, int* compact) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        if (compact) *compact = 0;
        Shape s = make_shape(shape, rank);
        const uint64_t n = numel(s);
        if (n && !values) raise(MHIP_KERNEL_EXECUTION_FAILED, "null values");
        // Compact when a matrix of at least 65536 values holds only exact bf16
        // values (src/kernels.rs:1672-1690); lossless either way.
        bool exact = s.size() == 2 && n >= (1u << 16);
        for (uint64_t i = 0; exact && i < n; ++i) {
            uint32_t u;
            std::memcpy(&u, values + i, 4);
            exact = (u & 0xFFFFu) == 0;
        }
        std::lock_guard<std::mutex> lock(ex->mu);
        if (!exact) {
            auto buf = std::make_unique<Buffer>(ex->ctx, n * 4, s, MHIP_DTYPE_F32);
            if (n) check(mhip_upload(ex->ctx, buf->ptr, values, n * 4));
            ex->storage[id] = std::move(buf);
            return;
        }
        auto buf = std::make_unique<Buffer>(ex->ctx, n * 2, s, MHIP_DTYPE_F32);
        buf->compact = true;
        // Converted and uploaded a chunk at a time, bounding the host copy.
        constexpr uint64_t kChunk = 1u << 20;
        std::vector<uint16_t> bits(std::min<uint64_t>(n, kChunk));
        for (uint64_t first = 0; first < n; first += kChunk) {
            const uint64_t count = std::min<uint64_t>(kChunk, n - first);
            for (uint64_t i = 0; i < count; ++i) {
                uint32_t u;
                std::memcpy(&u, values + first + i, 4);
                bits[i] = static_cast<uint16_t>(u >> 16);
            }
            check(mhip_upload(ex->ctx, buf->h() + first, bits.data(), count * 2));
        }
        ex->storage[id] = std::move(buf);
        if (compact) *compact = 1;
    });
}

mhip_kernel_error mhip_executor_read_tensor(mhip_executor* ex, const char* id, void* dst,
                                            size_t capacity, size_t* written) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        std::lock_guard<std::mutex> lock(ex->mu);
        ex->flush_checks();
        auto it = ex->storage.find(id);
        if (it == ex->storage.end())
            raise(MHIP_KERNEL_EXECUTION_FAILED, std::string("no materialized data for resource ") + id);
        const Buffer& b = *it->second;
        if (b.compact) {
            const uint64_t n = numel(b.shape);
            if (capacity < n * 4)
                raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "destination holds " + std::to_string(capacity) +
                                                         " bytes, tensor has " + std::to_string(n * 4));
            download_widened(ex->ctx, b, 0, n, static_cast<float*>(dst));
            if (written) *written = n * 4;
            return;
        }
        if (capacity < b.bytes)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "destination holds " + std::to_string(capacity) +
                                                     " bytes, tensor has " + std::to_string(b.bytes));
        check(mhip_download(ex->ctx, dst, b.ptr, b.bytes));
        if (written) *written = b.bytes;
    });
}

mhip_kernel_error mhip_executor_read_tensor_values(mhip_executor* ex, const char* id, float* dst,
                                                   size_t capacity) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        std::lock_guard<std::mutex> lock(ex->mu);
        ex->flush_checks();
        auto it = ex->storage.find(id);
        if (it == ex->storage.end())
            raise(MHIP_KERNEL_EXECUTION_FAILED, std::string("no materialized data for resource ") + id);
        const Buffer& b = *it->second;
        const uint64_t n = numel(b.shape);
        if (capacity < n)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "destination holds " + std::to_string(capacity) +
                                                     " values, tensor has " + std::to_string(n));
        if (b.compact) {
            download_widened(ex->ctx, b, 0, n, dst);
        } else if (b.dtype == MHIP_DTYPE_F32) {
            check(mhip_download(ex->ctx, dst, b.ptr, n * 4));
        } else {
            Buffer tmp(ex->ctx, n * 4, b.shape, MHIP_DTYPE_F32);
            check(mhip_decode_half(ex->ctx, b.h(), tmp.f(), n,
                                   b.dtype == MHIP_DTYPE_F16 ? MHIP_F16 : MHIP_BF16));
            check(mhip_download(ex->ctx, dst, tmp.ptr, n * 4));
        }
    });
}

mhip_kernel_error mhip_executor_read_tensor_rows(mhip_executor* ex, const char* id,
                                                 uint64_t row_begin, uint64_t row_count, float* dst,
                                                 size_t capacity) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        std::lock_guard<std::mutex> lock(ex->mu);
        ex->flush_checks();
        auto it = ex->storage.find(id);
        if (it == ex->storage.end())
            raise(MHIP_KERNEL_EXECUTION_FAILED, std::string("no materialized data for resource ") + id);
        const Buffer& b = *it->second;
        if (b.dtype != MHIP_DTYPE_F32) raise(MHIP_KERNEL_DTYPE_UNSUPPORTED, "row reads take f32 tensors");
        if (b.shape.empty()) raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "row reads need at least one dimension");
        const uint64_t rows = b.shape[0];
        const uint64_t width = rows ? numel(b.shape) / rows : 0;
        if (row_begin > rows || row_count > rows - row_begin)
            raise(MHIP_KERNEL_SHAPE_UNSUPPORTED,
                  "rows [" + std::to_string(row_begin) + ", " + std::to_string(row_begin + row_count) +
                      ") are outside the " + std::to_string(rows) + " rows");
        if (capacity < row_count * width) raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "destination too small");
        if (b.compact)
            download_widened(ex->ctx, b, row_begin * width, row_count * width, dst);
        else
            check(mhip_download(ex->ctx, dst, b.f() + row_begin * width, row_count * width * 4));
    });
}

mhip_kernel_error mhip_executor_resident_shape(mhip_executor* ex, const char* id, uint64_t* shape,
                                               int* rank, int* dtype) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        std::lock_guard<std::mutex> lock(ex->mu);
        auto it = ex->storage.find(id);
        if (it == ex->storage.end())
            raise(MHIP_KERNEL_EXECUTION_FAILED, std::string("no materialized data for resource ") + id);
        const Buffer& b = *it->second;
        if (rank) *rank = static_cast<int>(b.shape.size());
        if (dtype) *dtype = b.dtype;
        if (shape)
            for (size_t i = 0; i < b.shape.size() && i < 8; ++i) shape[i] = b.shape[i];
    });
}

mhip_kernel_error mhip_executor_release_tensor(mhip_executor* ex, const char* id) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        std::lock_guard<std::mutex> lock(ex->mu);
        auto it = ex->storage.find(id);
        if (it != ex->storage.end()) {
            mhip_sync(ex->ctx);  // kernels may still read it
            ex->storage.erase(it);
        }
    });
}

mhip_kernel_error mhip_executor_copy_tensor(mhip_executor* ex, const char* src, const char* dst) {
    return guarded([&] {
        if (!ex || !src || !dst) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        std::lock_guard<std::mutex> lock(ex->mu);
        auto it = ex->storage.find(src);
        if (it == ex->storage.end())
            raise(MHIP_KERNEL_EXECUTION_FAILED, std::string("no materialized data for resource ") + src);
        const Buffer& b = *it->second;
        auto copy = std::make_unique<Buffer>(ex->ctx, b.bytes, b.shape, b.dtype);
        copy->compact = b.compact;
        check(mhip_copy(ex->ctx, copy->ptr, b.ptr, b.bytes));
        ex->storage[dst] = std::move(copy);
    });
}

uint64_t mhip_executor_tensor_count(mhip_executor* ex) {
    if (!ex) return 0;
    std::lock_guard<std::mutex> lock(ex->mu);
    return ex->storage.size();
}

mhip_kernel_error mhip_executor_submit_kernel(mhip_executor* ex, const mhip_invocation* inv,
                                              uint64_t* handle) {
    if (!ex || !inv) return finish(MHIP_KERNEL_EXECUTION_FAILED, "null executor or invocation");
    Invocation v = convert(inv);
    std::lock_guard<std::mutex> lock(ex->mu);
    auto result = ex->execute(v);
    const uint64_t h = ex->next_handle++;
    ex->results[h] = result;
    if (handle) *handle = h;
    return finish(MHIP_KERNEL_OK, "");
}

mhip_kernel_error mhip_executor_complete_kernel(mhip_executor* ex, uint64_t handle) {
    if (!ex) return finish(MHIP_KERNEL_EXECUTION_FAILED, "null executor");
    std::lock_guard<std::mutex> lock(ex->mu);
    auto it = ex->results.find(handle);
    if (it == ex->results.end())
        return finish(MHIP_KERNEL_EXECUTION_FAILED, "unknown execution handle " + std::to_string(handle));
    auto result = it->second;
    ex->results.erase(it);
    return finish(result.first, result.second);
}

mhip_kernel_error mhip_executor_execute(mhip_executor* ex, const mhip_invocation* inv) {
    uint64_t handle = 0;
    mhip_kernel_error e = mhip_executor_submit_kernel(ex, inv, &handle);
    if (e != MHIP_KERNEL_OK) return e;
    return mhip_executor_complete_kernel(ex, handle);
}

mhip_kernel_error mhip_executor_set_deferred_checks(mhip_executor* ex, int enabled) {
    return guarded([&] {
        if (!ex) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor");
        std::lock_guard<std::mutex> lock(ex->mu);
        ex->deferred_checks = enabled != 0;
        if (!enabled) ex->flush_checks();
    });
}

mhip_kernel_error mhip_executor_check(mhip_executor* ex) {
    return guarded([&] {
        if (!ex) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor");
        std::lock_guard<std::mutex> lock(ex->mu);
        ex->flush_checks();
    });
}

mhip_status mhip_executor_set_sync_nodes(mhip_executor* ex, int enabled) {
    if (!ex) return MHIP_SHAPE_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(ex->mu);
    ex->sync_nodes = enabled != 0;
    return MHIP_OK;
}

uint64_t mhip_executor_observation_count(mhip_executor* ex) {
    if (!ex) return 0;
    std::lock_guard<std::mutex> lock(ex->mu);
    return ex->observations.size();
}

mhip_status mhip_executor_observation(mhip_executor* ex, uint64_t index, mhip_observation* out) {
    if (!ex || !out) return MHIP_SHAPE_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(ex->mu);
    if (index >= ex->observations.size()) return MHIP_SHAPE_UNSUPPORTED;
    const Observation& o = ex->observations[index];
    std::memset(out, 0, sizeof(*out));
    out->kind = o.kind;
    std::snprintf(out->kernel, sizeof(out->kernel), "%s", o.kernel.c_str());
    std::snprintf(out->invocation, sizeof(out->invocation), "%s", o.invocation.c_str());
    out->error = o.error;
    return MHIP_OK;
}

mhip_kernel_error mhip_executor_select_greedy_column(mhip_executor* ex, const char* logits,
                                                     uint64_t row, const uint64_t* excluded,
                                                     uint32_t range_count, float temperature,
                                                     int64_t* column) {
    return guarded([&] {
        if (!ex || !logits || !column) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor, id or result");
        *column = -1;
        std::lock_guard<std::mutex> lock(ex->mu);
        ex->flush_checks();
        auto it = ex->storage.find(logits);
        if (it == ex->storage.end())
            raise(MHIP_KERNEL_EXECUTION_FAILED, std::string("no materialized data for resource ") + logits);
        const Buffer& b = *it->second;
        mhip_executor::require_f32(b, "greedy selection's logits");
        if (b.shape.empty()) raise(MHIP_KERNEL_SHAPE_UNSUPPORTED, "logits have no columns");
        const uint64_t cols = b.shape.back();
        const uint64_t rows = cols ? numel(b.shape) / cols : 0;
        check(mhip_greedy_select_f32(ex->ctx, b.f(), rows, cols, row, excluded, range_count,
                                     temperature, column));
    });
}

// ---- step capture (src/executor.rs:177-336) ----

int mhip_executor_supports_step_capture(mhip_executor* ex) { return ex ? 1 : 0; }

mhip_kernel_error mhip_executor_begin_step_capture(mhip_executor* ex, const char* const* advancing,
                                                   int count) {
    return guarded([&] {
        if (!ex) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor");
        std::lock_guard<std::mutex> lock(ex->mu);
        if (ex->capture) raise(MHIP_KERNEL_EXECUTION_FAILED, "a step capture is already in progress");
        ex->flush_checks();
        uint32_t bits = 0;
        for (int i = 0; i < count; ++i) {
            const std::string name = advancing && advancing[i] ? advancing[i] : "";
            if (name == "position_offset") bits |= MHIP_ADVANCE_POSITION_OFFSET;
            else if (name == "key_count") bits |= MHIP_ADVANCE_KEY_COUNT;
            else if (name == "row_offset") bits |= MHIP_ADVANCE_ROW_OFFSET;
        }
        mhip_status st = mhip_capture_begin(ex->ctx, bits);
        if (st != MHIP_OK) raise(MHIP_KERNEL_EXECUTION_FAILED, mhip_last_error_detail());
        ex->capture = std::make_unique<Recording>();
    });
}

// Instantiates the recorded step and runs it once, so its results are
// available; writes the step's id to `id_out`.
mhip_kernel_error mhip_executor_end_step_capture(mhip_executor* ex, char* id_out, size_t capacity) {
    return guarded([&] {
        if (!ex) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor");
        std::lock_guard<std::mutex> lock(ex->mu);
        if (!ex->capture) raise(MHIP_KERNEL_EXECUTION_FAILED, "no step capture is in progress");
        std::unique_ptr<Recording> recording = std::move(ex->capture);
        mhip_graph* graph = nullptr;
        uint64_t max_offset = 0;
        mhip_status st = mhip_capture_end(ex->ctx, &graph, &max_offset);
        if (st != MHIP_OK) raise(MHIP_KERNEL_EXECUTION_FAILED, mhip_last_error_detail());
        st = mhip_graph_launch(graph, 0);
        if (st == MHIP_OK && recording->has_embedding) st = mhip_check_flags(ex->ctx, nullptr);
        if (st != MHIP_OK) {
            const std::string detail = mhip_last_error_detail();
            mhip_graph_destroy(graph);
            raise(MHIP_KERNEL_EXECUTION_FAILED, detail);
        }
        const std::string id = ex->provider_name + ":step-capture:" + std::to_string(ex->next_capture++);
        ex->captures[id] = CapturedStep{graph, std::move(*recording)};
        if (id_out && capacity) std::snprintf(id_out, capacity, "%s", id.c_str());
    });
}

mhip_kernel_error mhip_executor_abort_step_capture(mhip_executor* ex) {
    return guarded([&] {
        if (!ex) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor");
        std::lock_guard<std::mutex> lock(ex->mu);
        ex->capture.reset();
        mhip_capture_abort(ex->ctx);
    });
}

// Runs a captured step again with every advancing attribute increased by
// `offset`, after writing `inputs` into the buffers the step reads. A step
// whose buffers moved, or an input it never read, is Invalidated; an invalid
// embedding id fails the replay before anything runs.
mhip_kernel_error mhip_executor_replay_step(mhip_executor* ex, const char* id, uint64_t offset,
                                            const char* const* input_ids,
                                            const float* const* input_values,
                                            const uint64_t* input_lengths, int input_count) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        std::lock_guard<std::mutex> lock(ex->mu);
        auto it = ex->captures.find(id);
        if (it == ex->captures.end())
            raise(MHIP_STEP_REPLAY_INVALIDATED, std::string("no step capture '") + id + "'");
        CapturedStep& step = it->second;
        const uint64_t bound = mhip_graph_max_offset(step.graph);
        if (offset > bound)
            raise(MHIP_STEP_REPLAY_INVALIDATED, "offset " + std::to_string(offset) +
                                                    " leaves the captured bounds (at most " +
                                                    std::to_string(bound) + ")");
        for (const auto& [resource, where] : step.recording.resources) {
            auto s = ex->storage.find(resource);
            if (s == ex->storage.end() || s->second->ptr != where.first || s->second->bytes != where.second)
                raise(MHIP_STEP_REPLAY_INVALIDATED,
                      "resource '" + resource + "' no longer has its captured storage");
        }
        for (int i = 0; i < input_count; ++i) {
            const std::string resource = input_ids[i] ? input_ids[i] : "";
            if (!step.recording.resources.count(resource))
                raise(MHIP_STEP_REPLAY_INVALIDATED,
                      "input '" + resource + "' was not read by the captured step");
            auto vocab = step.recording.embedding_ids.find(resource);
            if (vocab != step.recording.embedding_ids.end()) {
                for (uint64_t j = 0; j < input_lengths[i]; ++j) {
                    const float value = input_values[i][j];
                    if (!(value >= 0.0f && value == std::floor(value) &&
                          static_cast<double>(value) < static_cast<double>(vocab->second)))
                        raise(MHIP_KERNEL_EXECUTION_FAILED,
                              "embedding lookup id is not a valid in-range non-negative integer");
                }
            }
        }
        for (int i = 0; i < input_count; ++i) {
            Buffer& buffer = *ex->storage[input_ids[i]];
            if (buffer.dtype != MHIP_DTYPE_F32 || input_lengths[i] * 4 != buffer.bytes)
                raise(MHIP_KERNEL_EXECUTION_FAILED,
                      std::string("replay input '") + input_ids[i] + "' has " +
                          std::to_string(input_lengths[i]) + " values, its buffer " +
                          std::to_string(buffer.bytes / 4));
            check(mhip_upload(ex->ctx, buffer.ptr, input_values[i], buffer.bytes));
        }
        check(mhip_graph_launch(step.graph, offset));
    });
}

mhip_kernel_error mhip_executor_release_step_capture(mhip_executor* ex, const char* id) {
    return guarded([&] {
        if (!ex || !id) raise(MHIP_KERNEL_EXECUTION_FAILED, "null executor or id");
        std::lock_guard<std::mutex> lock(ex->mu);
        auto it = ex->captures.find(id);
        if (it == ex->captures.end()) return;
        mhip_graph_destroy(it->second.graph);
        ex->captures.erase(it);
        // Gate buffers outgrown while a capture could read them are freed
        // once no capture is left, after the replays in flight have ended.
        if (ex->captures.empty() && !ex->retired_gate_products.empty()) {
            check(mhip_sync(ex->ctx));
            ex->retired_gate_products.clear();
        }
    });
}

}  // extern "C"
