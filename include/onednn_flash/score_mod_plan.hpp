#pragma once

// Score-modification planning, same names, values and signature strings as
// the reference's include/onednn_flash/score_mod_plan.hpp:1-82. Additions
// (appended so that existing enumerator values keep their integers):
// DataType::F16, LoweringStatus::LoweredToHipKernel,
// FallbackReason::HipUnavailable / HipDisabled, the soft-cap fields of
// ScoreModPlan, and an overload of make_score_mod_plan that plans for this
// library's HIP kernels.

#include <string>

namespace onednn_flash {

enum class DataType {
    F32,
    BF16,
    Unsupported,
    F16,
};

enum class ScoreModKind {
    None,
    Scale,
    AdditiveBias,
    ScaleAdditiveBias,
    Unsupported,
};

enum class BiasKind {
    None,
    SameShapeTile,
    BroadcastRow,
    BroadcastCol,
    AlibiGenerated,
    Unsupported,
};

enum class LoweringStatus {
    LoweredToOneDnnPostOps,
    PartiallyLowered,
    OneDNNFlashEpilogue,
    ReferenceFallback,
    Unsupported,
    LoweredToHipKernel,
};

enum class FallbackReason {
    None,
    OneDnnDisabled,
    OneDnnUnavailable,
    UnsupportedDType,
    UnsupportedShape,
    UnsupportedScoreMod,
    UnsupportedBlockMask,
    UnsupportedPostOp,
    UnsupportedBiasLayout,
    UnsupportedBroadcast,
    UnsupportedEdgeTile,
    NumericalSafetyFallback,
    DebugForcedReference,
    HipUnavailable,
    HipDisabled,
};

struct ScoreModPlan {
    ScoreModKind kind{ScoreModKind::None};
    DataType dtype{DataType::F32};

    bool has_scale{false};
    float scale_value{1.0f};

    BiasKind bias_kind{BiasKind::None};
    bool has_bias{false};

    LoweringStatus lowering_status{LoweringStatus::LoweredToOneDnnPostOps};
    FallbackReason fallback_reason{FallbackReason::None};

    std::string signature{"none"};

    // cap * tanh(score / cap) after scale and bias (HIP kernels only)
    bool has_softcap{false};
    float softcap_value{0.0f};
};

const char* to_string(DataType value);
const char* to_string(ScoreModKind value);
const char* to_string(BiasKind value);
const char* to_string(LoweringStatus value);
const char* to_string(FallbackReason value);

// Reference planner (src/onednn_flash/score_mod_plan.cpp:115-182): fp32 only,
// same-shape bias lowered to oneDNN post-ops when they are available.
ScoreModPlan make_score_mod_plan(ScoreModKind requested_kind,
                                 DataType dtype,
                                 bool has_scale,
                                 float scale_value,
                                 BiasKind requested_bias_kind,
                                 bool one_dnn_post_ops_available);

// Planner for the HIP attention kernels: fp32/bf16/fp16; scale, same-shape or
// row-broadcast bias (shape [1,n]: a dense bias with a zero query stride),
// generated ALiBi, and a soft-cap, all lowered into the fused kernel.
// BroadcastCol (shape [m,1]) would need a zero key stride, which the dense
// bias path does not take: UnsupportedBroadcast, as in the reference.
ScoreModPlan make_hip_score_mod_plan(ScoreModKind requested_kind,
                                     DataType dtype,
                                     bool has_scale,
                                     float scale_value,
                                     BiasKind requested_bias_kind,
                                     float softcap);

}  // namespace onednn_flash
