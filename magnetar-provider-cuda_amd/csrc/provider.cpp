// Provider facade, device descriptor and Kernel advertisements.
//
// Mirrors `CudaProvider` (src/provider.rs:76-324): construction never fails
// for lack of hardware (no driver or device -> Unavailable, zero devices, zero
// advertisements); a device whose executor cannot be built -> Degraded.
// Advertisements follow `cuda_kernel_advertisements` (src/advertisements.rs:
// 140-289) for the Kernels this Provider implements: f32 in/out, contiguous
// layout, device memory, timeout-only cancellation, rank 2 for matmul / rope /
// attention / softmax (src/advertisements.rs:57-80), and the half-precision
// add/mul Kernels under the `add` / `mul` Operators (:109-132).
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "magnetar_hip.h"

namespace {

constexpr const char* kDefaultName = "magnetar:provider/hip";
constexpr const char* kVersion = "0.1.0";
constexpr const char* kVendor = "magnetar";
constexpr const char* kDescription =
    "GPU-executing Provider for AMD Instinct MI355X (gfx950) with hand-written HIP kernels";
constexpr const char* kProfile = "hip-conformance-v1";
constexpr const char* kFamily = "Hip";

constexpr uint32_t kF32 = 1u << MHIP_DTYPE_F32;
constexpr uint32_t kHalf = (1u << MHIP_DTYPE_F16) | (1u << MHIP_DTYPE_BF16);

struct AdvertSpec {
    const char* name;
    const char* op;
    const char* family;
    uint32_t dtypes;
    int rank;
    const char* features;
};

// Feature strings name the optional operator forms each Kernel honours.
const AdvertSpec kAdverts[] = {
    {"matmul", "matmul", "LinearAlgebra", kF32, 2, ""},
    {"matmul-bias", "matmul-bias", "LinearAlgebra", kF32, 0, ""},
    {"matmul-residual", "matmul-residual", "LinearAlgebra", kF32, 0, ""},
    {"silu-mul", "silu-mul", "Activation", kF32, 0, ""},
    {"gated-matmul", "gated-matmul", "LinearAlgebra", kF32, 0, ""},
    {"embedding", "embedding", "Tensor", kF32, 0, "embedding-scale"},
    {"rmsnorm", "rmsnorm", "Normalization", kF32, 0, "rmsnorm-per-head,rmsnorm-without-weight"},
    {"rope", "rope", "PositionEncoding", kF32, 2,
     "rope-banded-frequency-scaling,rope-partial-rotary,rope-yarn-frequency-scaling"},
    {"attention", "attention", "Attention", kF32, 2,
     "key-count,attention-scale,attention-value-head-dimension"},
    {"softmax", "softmax", "Activation", kF32, 2, ""},
    {"silu", "silu", "Activation", kF32, 0, ""},
    {"add", "add", "Tensor", kF32, 0, ""},
    {"mul", "mul", "Tensor", kF32, 0, ""},
    {"concat", "concat", "Tensor", kF32, 0, ""},
    {"kv-write", "kv-write", "Tensor", kF32, 2, ""},
    {"residual-add", "residual-add", "Tensor", kF32, 0, ""},
    {"add-half", "add", "Tensor", kHalf, 0, ""},
    {"mul-half", "mul", "Tensor", kHalf, 0, ""},
};
constexpr int kAdvertCount = sizeof(kAdverts) / sizeof(kAdverts[0]);

}  // namespace

struct mhip_provider {
    std::string name;
    int ordinal = 0;
    mhip_ctx* ctx = nullptr;
    mhip_executor* executor = nullptr;
    bool has_device = false;
    mhip_device_descriptor device{};
};

extern "C" {

mhip_status mhip_provider_create(int ordinal, const char* provider_name, mhip_provider** out) {
    if (!out) return MHIP_SHAPE_UNSUPPORTED;
    auto* p = new mhip_provider();
    p->name = provider_name ? provider_name : kDefaultName;
    p->ordinal = ordinal;
    // Discovery: any failure is the "no hardware" outcome, never an error.
    if (mhip_ctx_create(ordinal, &p->ctx) == MHIP_OK) {
        mhip_device_info info;
        if (mhip_device_query(p->ctx, &info) == MHIP_OK) {
            p->has_device = true;
            std::snprintf(p->device.id, sizeof(p->device.id), "hip:%d", ordinal);
            std::snprintf(p->device.name, sizeof(p->device.name), "%s",
                          info.name[0] ? info.name : "AMD Instinct GPU");
            std::snprintf(p->device.architecture, sizeof(p->device.architecture), "%s",
                          info.architecture);
            p->device.memory_capacity = info.total_memory;
            p->device.compute_units = info.compute_units;
            p->device.pressure = info.pressure;
            if (mhip_executor_create(p->ctx, p->device.id, p->name.c_str(), &p->executor) != MHIP_OK)
                p->executor = nullptr;
        } else {
            mhip_ctx_destroy(p->ctx);
            p->ctx = nullptr;
        }
    }
    *out = p;
    return MHIP_OK;
}

mhip_status mhip_provider_destroy(mhip_provider* p) {
    if (!p) return MHIP_OK;
    if (p->executor) mhip_executor_destroy(p->executor);
    if (p->ctx) mhip_ctx_destroy(p->ctx);
    delete p;
    return MHIP_OK;
}

mhip_status mhip_provider_metadata_get(mhip_provider* p, mhip_provider_metadata* out) {
    if (!p || !out) return MHIP_SHAPE_UNSUPPORTED;
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", p->name.c_str());
    std::snprintf(out->version, sizeof(out->version), "%s", kVersion);
    std::snprintf(out->vendor, sizeof(out->vendor), "%s", kVendor);
    std::snprintf(out->description, sizeof(out->description), "%s", kDescription);
    return MHIP_OK;
}

// src/provider.rs:262-279.
int mhip_provider_health(mhip_provider* p) {
    if (!p || !p->has_device) return MHIP_HEALTH_UNAVAILABLE;
    return p->executor ? MHIP_HEALTH_AVAILABLE : MHIP_HEALTH_DEGRADED;
}

int mhip_provider_device_count(mhip_provider* p) { return p && p->has_device ? 1 : 0; }

mhip_status mhip_provider_device(mhip_provider* p, int index, mhip_device_descriptor* out) {
    if (!p || !out || !p->has_device || index != 0) return MHIP_SHAPE_UNSUPPORTED;
    *out = p->device;
    if (p->ctx) {
        mhip_device_info info;
        if (mhip_device_query(p->ctx, &info) == MHIP_OK) out->pressure = info.pressure;
    }
    return MHIP_OK;
}

mhip_executor* mhip_provider_executor(mhip_provider* p) { return p ? p->executor : nullptr; }

mhip_status mhip_provider_initialize(mhip_provider* p) { return p ? MHIP_OK : MHIP_SHAPE_UNSUPPORTED; }
mhip_status mhip_provider_shutdown(mhip_provider* p) {
    if (!p) return MHIP_SHAPE_UNSUPPORTED;
    return p->ctx ? mhip_sync(p->ctx) : MHIP_OK;
}

// No Device discovered means no Kernel can run anywhere: no advertisements
// (src/provider.rs:288-296).
int mhip_provider_advertisement_count(mhip_provider* p) {
    return p && p->has_device ? kAdvertCount : 0;
}

mhip_status mhip_provider_advertisement(mhip_provider* p, int index, mhip_advertisement* out) {
    if (!p || !out || !p->has_device || index < 0 || index >= kAdvertCount) return MHIP_SHAPE_UNSUPPORTED;
    const AdvertSpec& a = kAdverts[index];
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", a.name);
    std::snprintf(out->operator_name, sizeof(out->operator_name), "%s", a.op);
    std::snprintf(out->operator_family, sizeof(out->operator_family), "%s", a.family);
    out->input_dtypes = a.dtypes;
    out->output_dtypes = a.dtypes;
    out->rank = a.rank;
    std::snprintf(out->features, sizeof(out->features), "%s", a.features);
    std::snprintf(out->conformance_profile, sizeof(out->conformance_profile), "%s", kProfile);
    std::snprintf(out->family, sizeof(out->family), "%s", kFamily);
    std::snprintf(out->device_id, sizeof(out->device_id), "%s", p->device.id);
    std::snprintf(out->provider, sizeof(out->provider), "%s", p->name.c_str());
    return MHIP_OK;
}

}  // extern "C"
