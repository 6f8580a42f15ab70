// Score-mod and runtime planning (include/onednn_flash/score_mod_plan.hpp,
// runtime_plan.hpp). The reference planner (src/onednn_flash/
// score_mod_plan.cpp:115-182, runtime_plan.cpp:77-200) decides between oneDNN
// post-ops and its reference tiles; here the same decisions and signature
// strings are kept for that case, and a HIP plan is made when a GPU is
// present: fp32/bf16/fp16 inputs, scale, same-shape or row-broadcast bias,
// generated ALiBi and a soft-cap all lower into the fused attention kernel.

#include "onednn_flash/runtime_plan.hpp"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <limits>
#include <mutex>
#include <sstream>

namespace onednn_flash {

const char* to_string(DataType value) {
    switch (value) {
        case DataType::F32: return "f32";
        case DataType::BF16: return "bf16";
        case DataType::F16: return "f16";
        case DataType::Unsupported: return "unsupported";
    }
    return "unknown";
}

const char* to_string(ScoreModKind value) {
    switch (value) {
        case ScoreModKind::None: return "none";
        case ScoreModKind::Scale: return "scale";
        case ScoreModKind::AdditiveBias: return "additive_bias";
        case ScoreModKind::ScaleAdditiveBias: return "scale_additive_bias";
        case ScoreModKind::Unsupported: return "unsupported";
    }
    return "unknown";
}

const char* to_string(BiasKind value) {
    switch (value) {
        case BiasKind::None: return "none";
        case BiasKind::SameShapeTile: return "same_shape_tile";
        case BiasKind::BroadcastRow: return "broadcast_row";
        case BiasKind::BroadcastCol: return "broadcast_col";
        case BiasKind::AlibiGenerated: return "alibi_generated";
        case BiasKind::Unsupported: return "unsupported";
    }
    return "unknown";
}

const char* to_string(LoweringStatus value) {
    switch (value) {
        case LoweringStatus::LoweredToOneDnnPostOps: return "lowered_to_onednn_post_ops";
        case LoweringStatus::PartiallyLowered: return "partially_lowered";
        case LoweringStatus::OneDNNFlashEpilogue: return "onednn_flash_epilogue";
        case LoweringStatus::ReferenceFallback: return "reference_fallback";
        case LoweringStatus::Unsupported: return "unsupported";
        case LoweringStatus::LoweredToHipKernel: return "lowered_to_hip_kernel";
    }
    return "unknown";
}

const char* to_string(FallbackReason value) {
    switch (value) {
        case FallbackReason::None: return "none";
        case FallbackReason::OneDnnDisabled: return "onednn_disabled";
        case FallbackReason::OneDnnUnavailable: return "onednn_unavailable";
        case FallbackReason::UnsupportedDType: return "unsupported_dtype";
        case FallbackReason::UnsupportedShape: return "unsupported_shape";
        case FallbackReason::UnsupportedScoreMod: return "unsupported_score_mod";
        case FallbackReason::UnsupportedBlockMask: return "unsupported_block_mask";
        case FallbackReason::UnsupportedPostOp: return "unsupported_post_op";
        case FallbackReason::UnsupportedBiasLayout: return "unsupported_bias_layout";
        case FallbackReason::UnsupportedBroadcast: return "unsupported_broadcast";
        case FallbackReason::UnsupportedEdgeTile: return "unsupported_edge_tile";
        case FallbackReason::NumericalSafetyFallback: return "numerical_safety_fallback";
        case FallbackReason::DebugForcedReference: return "debug_forced_reference";
        case FallbackReason::HipUnavailable: return "hip_unavailable";
        case FallbackReason::HipDisabled: return "hip_disabled";
    }
    return "unknown";
}

const char* to_string(BlockMaskKind value) {
    switch (value) {
        case BlockMaskKind::None: return "none";
        case BlockMaskKind::Causal: return "causal";
        case BlockMaskKind::Unsupported: return "unsupported";
    }
    return "unknown";
}

const char* to_string(QkBackendKind value) {
    switch (value) {
        case QkBackendKind::Reference: return "reference";
        case QkBackendKind::OneDnnMatmul: return "onednn_matmul";
        case QkBackendKind::OneDnnBrgemmBaseline: return "onednn_brgemm_baseline";
        case QkBackendKind::Hip: return "hip";
    }
    return "unknown";
}

const char* to_string(QkLayoutKind value) {
    switch (value) {
        case QkLayoutKind::RowMajorKStrided: return "row_major_k_strided";
        case QkLayoutKind::CopiedTransposedK: return "copied_transposed_k";
        case QkLayoutKind::BrgemmTransformedKBaseline: return "brgemm_transformed_k_baseline";
    }
    return "unknown";
}

namespace {

std::string unsupported_signature(FallbackReason reason) {
    return std::string("unsupported:") + to_string(reason);
}

// "none" | "scale:<dtype>" | "[scale_]additive_bias:<bias kind>:<dtype>"
std::string score_mod_signature(ScoreModKind kind, BiasKind bias, DataType dtype) {
    switch (kind) {
        case ScoreModKind::None: return "none";
        case ScoreModKind::Scale: return std::string("scale:") + to_string(dtype);
        case ScoreModKind::AdditiveBias:
        case ScoreModKind::ScaleAdditiveBias:
            return std::string(to_string(kind)) + ':' + to_string(bias) + ':' + to_string(dtype);
        case ScoreModKind::Unsupported: break;
    }
    return unsupported_signature(FallbackReason::UnsupportedScoreMod);
}

ScoreModPlan base_score_mod_plan(ScoreModKind kind, DataType dtype, bool has_scale, float scale,
                                 BiasKind bias) {
    ScoreModPlan p;
    p.kind = kind;
    p.dtype = dtype;
    p.has_scale = has_scale;
    p.scale_value = has_scale ? scale : 1.0f;
    p.bias_kind = bias;
    p.has_bias = bias != BiasKind::None;
    return p;
}

void mark_fallback(ScoreModPlan& p, LoweringStatus status, FallbackReason reason) {
    p.lowering_status = status;
    p.fallback_reason = reason;
    p.signature = unsupported_signature(reason);
}

bool shape_is_valid(const RuntimePlanInput& in) {
    return in.batch > 0 && in.heads > 0 && in.query_length > 0 && in.key_length > 0 &&
           in.head_dim > 0 && in.value_dim > 0;
}

bool all_f32(const RuntimePlanInput& in) {
    return in.q_dtype == DataType::F32 && in.k_dtype == DataType::F32 &&
           in.v_dtype == DataType::F32 && in.out_dtype == DataType::F32;
}

// The HIP kernels take one input type for Q, K and V; the output is fp32 or
// that type.
bool hip_dtypes_ok(const RuntimePlanInput& in) {
    const DataType t = in.q_dtype;
    const bool input_ok = t == DataType::F32 || t == DataType::BF16 || t == DataType::F16;
    return input_ok && in.k_dtype == t && in.v_dtype == t &&
           (in.out_dtype == t || in.out_dtype == DataType::F32);
}

std::string shape_signature(const RuntimePlanInput& in) {
    std::ostringstream oss;
    oss << 'b' << in.batch << 'h' << in.heads << 'm' << in.query_length << 'n' << in.key_length
        << 'd' << in.head_dim << "dv" << in.value_dim;
    return oss.str();
}

std::string dtype_signature(const RuntimePlanInput& in) {
    std::ostringstream oss;
    oss << 'q' << to_string(in.q_dtype) << 'k' << to_string(in.k_dtype) << 'v'
        << to_string(in.v_dtype) << 'o' << to_string(in.out_dtype);
    return oss.str();
}

void finish_plan(RuntimePlan& plan) {
    plan.requires_mask_tile_generator = plan.block_mask_plan.requires_mask_tile_generator;
    plan.requires_onednn_flash_epilogue =
        plan.requires_mask_tile_generator ||
        plan.score_mod_plan.lowering_status == LoweringStatus::OneDNNFlashEpilogue;
    std::ostringstream sig;
    sig << shape_signature(plan.input) << '|' << dtype_signature(plan.input) << '|'
        << plan.score_mod_plan.signature << '|' << plan.block_mask_plan.signature << '|'
        << to_string(plan.qk_backend) << '|' << to_string(plan.qk_layout);
    plan.runtime_plan_signature = sig.str();
    std::ostringstream dbg;
    dbg << "RuntimePlan{backend=" << to_string(plan.qk_backend)
        << ", layout=" << to_string(plan.qk_layout)
        << ", score_mod=" << plan.score_mod_plan.signature
        << ", block_mask=" << plan.block_mask_plan.signature
        << ", fallback=" << to_string(plan.fallback_reason) << '}';
    plan.debug_summary = dbg.str();
}

}  // namespace

ScoreModPlan make_score_mod_plan(ScoreModKind requested_kind, DataType dtype, bool has_scale,
                                 float scale_value, BiasKind requested_bias_kind,
                                 bool one_dnn_post_ops_available) {
    ScoreModPlan p = base_score_mod_plan(requested_kind, dtype, has_scale, scale_value,
                                         requested_bias_kind);
    if (dtype != DataType::F32) {
        p.kind = ScoreModKind::Unsupported;
        mark_fallback(p, LoweringStatus::ReferenceFallback, FallbackReason::UnsupportedDType);
        return p;
    }
    if (requested_kind == ScoreModKind::Unsupported) {
        mark_fallback(p, LoweringStatus::ReferenceFallback, FallbackReason::UnsupportedScoreMod);
        return p;
    }
    if (p.has_bias && requested_bias_kind != BiasKind::SameShapeTile) {
        const bool broadcast = requested_bias_kind == BiasKind::BroadcastRow ||
                               requested_bias_kind == BiasKind::BroadcastCol;
        mark_fallback(p, LoweringStatus::OneDNNFlashEpilogue,
                      broadcast ? FallbackReason::UnsupportedBroadcast
                                : FallbackReason::UnsupportedBiasLayout);
        return p;
    }
    const bool post_ops = one_dnn_post_ops_available || requested_kind == ScoreModKind::None;
    p.lowering_status = post_ops ? LoweringStatus::LoweredToOneDnnPostOps
                                 : LoweringStatus::OneDNNFlashEpilogue;
    p.fallback_reason = post_ops ? FallbackReason::None : FallbackReason::UnsupportedPostOp;
    p.signature = score_mod_signature(requested_kind, requested_bias_kind, dtype);
    return p;
}

ScoreModPlan make_hip_score_mod_plan(ScoreModKind requested_kind, DataType dtype, bool has_scale,
                                     float scale_value, BiasKind requested_bias_kind,
                                     float softcap) {
    ScoreModPlan p = base_score_mod_plan(requested_kind, dtype, has_scale, scale_value,
                                         requested_bias_kind);
    p.has_softcap = softcap > 0.0f;
    p.softcap_value = p.has_softcap ? softcap : 0.0f;
    if (dtype != DataType::F32 && dtype != DataType::BF16 && dtype != DataType::F16) {
        p.kind = ScoreModKind::Unsupported;
        mark_fallback(p, LoweringStatus::ReferenceFallback, FallbackReason::UnsupportedDType);
        return p;
    }
    if (requested_kind == ScoreModKind::Unsupported || !(softcap >= 0.0f)) {
        mark_fallback(p, LoweringStatus::ReferenceFallback, FallbackReason::UnsupportedScoreMod);
        return p;
    }
    switch (requested_bias_kind) {
        case BiasKind::None:
        case BiasKind::SameShapeTile:
        case BiasKind::BroadcastRow:
        case BiasKind::AlibiGenerated:
            break;
        case BiasKind::BroadcastCol:
            mark_fallback(p, LoweringStatus::ReferenceFallback, FallbackReason::UnsupportedBroadcast);
            return p;
        case BiasKind::Unsupported:
            mark_fallback(p, LoweringStatus::ReferenceFallback, FallbackReason::UnsupportedBiasLayout);
            return p;
    }
    p.lowering_status = LoweringStatus::LoweredToHipKernel;
    p.fallback_reason = FallbackReason::None;
    p.signature = score_mod_signature(requested_kind, requested_bias_kind, dtype);
    if (p.has_softcap) {
        char buf[48];
        std::snprintf(buf, sizeof buf, ":softcap=%g", static_cast<double>(softcap));
        p.signature += buf;
    }
    return p;
}

BlockMaskPlan make_block_mask_plan(BlockMaskKind requested_kind, int query_length, int key_length) {
    (void)query_length;
    BlockMaskPlan p;
    p.kind = requested_kind;
    if (requested_kind == BlockMaskKind::None) {
        p.signature = "none";
        return p;
    }
    if (requested_kind == BlockMaskKind::Causal) {
        p.has_boundary_tiles = true;
        // Top-left causal masks (q, k) with k > q; some key tile lies wholly
        // above the diagonal of some query tile as soon as such a pair exists,
        // i.e. when there are at least two keys. (The reference writes
        // key_length > query_length here, which the attention loop's own
        // causal skipping does not follow.)
        p.can_skip_tiles = key_length > 1;
        p.requires_mask_tile_generator = true;
        p.signature = "causal";
        return p;
    }
    p.kind = BlockMaskKind::Unsupported;
    p.fallback_reason = FallbackReason::UnsupportedBlockMask;
    p.signature = "unsupported:unsupported_block_mask";
    return p;
}

MaskTileDescriptor make_causal_mask_tile_descriptor(int q_start, int k_start, int q_size, int k_size) {
    MaskTileDescriptor d;
    d.required = true;
    d.q_start = q_start;
    d.k_start = k_start;
    d.q_size = q_size;
    d.k_size = k_size;
    d.masked_value = -std::numeric_limits<float>::infinity();
    // Row q of the tile has every key masked iff k_start > q; the first row is
    // the most masked one. (The reference compares with the last row,
    // q_start + q_size - 1, which is the condition for every row being masked.)
    d.all_masked_row_possible = k_start > q_start;
    return d;
}

RuntimePlan make_runtime_plan(const RuntimePlanInput& input, bool one_dnn_available,
                              bool one_dnn_post_ops_available, bool hip_available) {
    RuntimePlan plan;
    plan.input = input;
    const bool valid_shape = shape_is_valid(input);
    plan.block_mask_plan =
        make_block_mask_plan(input.requested_block_mask, input.query_length, input.key_length);

    const bool use_hip = input.enable_hip && hip_available && !input.force_reference &&
                         valid_shape && hip_dtypes_ok(input);
    if (use_hip) {
        plan.score_mod_plan =
            make_hip_score_mod_plan(input.requested_score_mod, input.q_dtype, input.has_scale,
                                    input.scale_value, input.requested_bias_kind, input.softcap);
        if (plan.score_mod_plan.fallback_reason != FallbackReason::None)
            plan.fallback_reason = plan.score_mod_plan.fallback_reason;
        else
            plan.fallback_reason = plan.block_mask_plan.fallback_reason;
        if (plan.fallback_reason == FallbackReason::None) {
            plan.qk_backend = QkBackendKind::Hip;
            plan.qk_lowering_status = LoweringStatus::LoweredToHipKernel;
        } else {
            plan.qk_backend = QkBackendKind::Reference;
            plan.qk_lowering_status = LoweringStatus::ReferenceFallback;
        }
        plan.qk_layout = QkLayoutKind::RowMajorKStrided;
        plan.uses_onednn_post_ops = false;
        finish_plan(plan);
        return plan;
    }

    // The reference's decision (runtime_plan.cpp:112-182), unchanged.
    const bool dtypes_ok = all_f32(input);
    const bool use_onednn = input.enable_onednn && one_dnn_available && !input.force_reference &&
                            valid_shape && dtypes_ok;
    plan.score_mod_plan = make_score_mod_plan(input.requested_score_mod, input.q_dtype,
                                              input.has_scale, input.scale_value,
                                              input.requested_bias_kind,
                                              use_onednn && one_dnn_post_ops_available);
    if (!valid_shape) plan.fallback_reason = FallbackReason::UnsupportedShape;
    else if (!dtypes_ok) plan.fallback_reason = FallbackReason::UnsupportedDType;
    else if (input.force_reference) plan.fallback_reason = FallbackReason::DebugForcedReference;
    else if (!input.enable_onednn) plan.fallback_reason = FallbackReason::OneDnnDisabled;
    else if (!one_dnn_available) plan.fallback_reason = FallbackReason::OneDnnUnavailable;
    else if (plan.score_mod_plan.fallback_reason != FallbackReason::None)
        plan.fallback_reason = plan.score_mod_plan.fallback_reason;
    else plan.fallback_reason = plan.block_mask_plan.fallback_reason;

    const bool lowered = use_onednn &&
                         plan.score_mod_plan.lowering_status == LoweringStatus::LoweredToOneDnnPostOps &&
                         plan.block_mask_plan.fallback_reason == FallbackReason::None;
    plan.qk_backend = lowered ? QkBackendKind::OneDnnMatmul : QkBackendKind::Reference;
    plan.qk_layout = QkLayoutKind::RowMajorKStrided;
    plan.qk_lowering_status = lowered ? LoweringStatus::LoweredToOneDnnPostOps
                                      : LoweringStatus::ReferenceFallback;
    plan.uses_onednn_post_ops = lowered && input.requested_score_mod != ScoreModKind::None;
    finish_plan(plan);
    return plan;
}

RuntimePlan make_runtime_plan(const RuntimePlanInput& input, bool one_dnn_available,
                              bool one_dnn_post_ops_available) {
    return make_runtime_plan(input, one_dnn_available, one_dnn_post_ops_available,
                             hip_backend_available());
}

RuntimePlanCacheKey make_runtime_plan_cache_key(const RuntimePlan& plan) {
    RuntimePlanCacheKey key;
    key.semantic_shape = shape_signature(plan.input);
    key.dtype_signature = dtype_signature(plan.input);
    key.score_mod_signature = plan.score_mod_plan.signature;
    key.block_mask_signature = plan.block_mask_plan.signature;
    std::ostringstream policy;
    policy << "force_reference=" << (plan.input.force_reference ? "true" : "false")
           << ";enable_onednn=" << (plan.input.enable_onednn ? "true" : "false")
           << ";backend=" << to_string(plan.qk_backend) << ";layout=" << to_string(plan.qk_layout);
    key.policy_signature = policy.str();
    return key;
}

bool hip_backend_available() {
    static std::once_flag once;
    static bool available = false;
    std::call_once(once, [] {
        int n = 0;
        available = hipGetDeviceCount(&n) == hipSuccess && n > 0;
    });
    return available;
}

}  // namespace onednn_flash
