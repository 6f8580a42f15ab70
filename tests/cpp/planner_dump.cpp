// Prints the planner's decisions over a grid of inputs, one line per case, so
// that two builds of the planner can be compared line by line: this library's
// (built with -DOFH_PLANNER, planning with no GPU present so that only the
// reference's decision chain runs) and the reference's own
// src/onednn_flash/{score_mod_plan,runtime_plan}.cpp compiled by oracle/Makefile.
// Only names both headers share are used.
//
// Line kinds:  S <inputs> | <ScoreModPlan>       make_score_mod_plan
//              B <inputs> | <BlockMaskPlan>      make_block_mask_plan
//              T <inputs> | <MaskTileDescriptor> make_causal_mask_tile_descriptor
//              R <inputs> | <RuntimePlan> | <RuntimePlanCacheKey>
// Fields are "name=value" separated by ';'.
// With --hip (this library's build only) it prints instead
//              H <inputs> | <RuntimePlan>        planning with a GPU present,
// over inputs that include fp16 and a soft-cap.

#include <cstdio>
#include <string>

#include "onednn_flash/runtime_plan.hpp"
#include "onednn_flash/score_mod_plan.hpp"

using namespace onednn_flash;

namespace {

std::string b(bool v) { return v ? "1" : "0"; }

std::string f(float v) {
    char buf[32];
    std::snprintf(buf, sizeof buf, "%.9g", static_cast<double>(v));
    return buf;
}

std::string score_mod(const ScoreModPlan& p) {
    return std::string("kind=") + to_string(p.kind) + ";dtype=" + to_string(p.dtype) +
           ";has_scale=" + b(p.has_scale) + ";scale=" + f(p.scale_value) +
           ";bias_kind=" + to_string(p.bias_kind) + ";has_bias=" + b(p.has_bias) +
           ";lowering=" + to_string(p.lowering_status) + ";fallback=" + to_string(p.fallback_reason) +
           ";signature=" + p.signature;
}

std::string block_mask(const BlockMaskPlan& p) {
    return std::string("kind=") + to_string(p.kind) + ";boundary=" + b(p.has_boundary_tiles) +
           ";can_skip_tiles=" + b(p.can_skip_tiles) + ";generator=" + b(p.requires_mask_tile_generator) +
           ";fallback=" + to_string(p.fallback_reason) + ";signature=" + p.signature;
}

RuntimePlan plan(const RuntimePlanInput& in, bool onednn, bool post_ops) {
#ifdef OFH_PLANNER
    return make_runtime_plan(in, onednn, post_ops, /*hip_available=*/false);
#else
    return make_runtime_plan(in, onednn, post_ops);
#endif
}

const DataType kDtypes[] = {DataType::F32, DataType::BF16, DataType::Unsupported};
const ScoreModKind kKinds[] = {ScoreModKind::None, ScoreModKind::Scale, ScoreModKind::AdditiveBias,
                               ScoreModKind::ScaleAdditiveBias, ScoreModKind::Unsupported};
const BiasKind kBiases[] = {BiasKind::None,          BiasKind::SameShapeTile, BiasKind::BroadcastRow,
                            BiasKind::BroadcastCol,  BiasKind::AlibiGenerated, BiasKind::Unsupported};
const BlockMaskKind kMasks[] = {BlockMaskKind::None, BlockMaskKind::Causal, BlockMaskKind::Unsupported};

#ifdef OFH_PLANNER
int dump_hip() {
    const DataType dsets[][4] = {{DataType::F32, DataType::F32, DataType::F32, DataType::F32},
                                 {DataType::BF16, DataType::BF16, DataType::BF16, DataType::BF16},
                                 {DataType::BF16, DataType::BF16, DataType::BF16, DataType::F32},
                                 {DataType::F16, DataType::F16, DataType::F16, DataType::F16},
                                 {DataType::F16, DataType::F16, DataType::F16, DataType::F32},
                                 {DataType::F32, DataType::F32, DataType::F32, DataType::BF16},
                                 {DataType::BF16, DataType::F16, DataType::BF16, DataType::BF16},
                                 {DataType::Unsupported, DataType::F32, DataType::F32, DataType::F32}};
    const int shapes[][2] = {{128, 128}, {0, 64}};
    for (const auto& sh : shapes)
        for (const auto& ds : dsets)
            for (ScoreModKind kind : kKinds)
                for (BiasKind bias : kBiases)
                    for (BlockMaskKind m : kMasks)
                        for (int force = 0; force < 2; ++force)
                            for (int enable_hip = 0; enable_hip < 2; ++enable_hip)
                                for (float cap : {0.0f, 30.0f}) {
                                    RuntimePlanInput in;
                                    in.batch = 2;
                                    in.heads = 4;
                                    in.query_length = sh[0];
                                    in.key_length = sh[1];
                                    in.head_dim = 128;
                                    in.value_dim = 128;
                                    in.q_dtype = ds[0];
                                    in.k_dtype = ds[1];
                                    in.v_dtype = ds[2];
                                    in.out_dtype = ds[3];
                                    in.requested_score_mod = kind;
                                    in.has_scale = true;
                                    in.scale_value = 0.125f;
                                    in.requested_bias_kind = bias;
                                    in.requested_block_mask = m;
                                    in.force_reference = force != 0;
                                    in.enable_hip = enable_hip != 0;
                                    in.softcap = cap;
                                    const RuntimePlan p = make_runtime_plan(in, false, false, true);
                                    std::printf(
                                        "H m=%d;n=%d;dtypes=%s,%s,%s,%s;kind=%s;bias=%s;mask=%s;"
                                        "force_reference=%d;enable_hip=%d;softcap=%s | %s | %s | "
                                        "backend=%s;lowering=%s;fallback=%s;signature=%s\n",
                                        sh[0], sh[1], to_string(ds[0]), to_string(ds[1]), to_string(ds[2]),
                                        to_string(ds[3]), to_string(kind), to_string(bias), to_string(m),
                                        force, enable_hip, f(cap).c_str(), score_mod(p.score_mod_plan).c_str(),
                                        block_mask(p.block_mask_plan).c_str(), to_string(p.qk_backend),
                                        to_string(p.qk_lowering_status), to_string(p.fallback_reason),
                                        p.runtime_plan_signature.c_str());
                                }
    return 0;
}
#endif

}  // namespace

int main(int argc, char** argv) {
#ifdef OFH_PLANNER
    if (argc > 1 && std::string(argv[1]) == "--hip") return dump_hip();
#else
    (void)argc;
    (void)argv;
#endif
    // make_score_mod_plan over every requested combination.
    for (DataType dt : kDtypes)
        for (ScoreModKind kind : kKinds)
            for (int has_scale = 0; has_scale < 2; ++has_scale)
                for (BiasKind bias : kBiases)
                    for (int post_ops = 0; post_ops < 2; ++post_ops) {
                        const ScoreModPlan p = make_score_mod_plan(kind, dt, has_scale != 0, 0.125f,
                                                                   bias, post_ops != 0);
                        std::printf("S dtype=%s;kind=%s;has_scale=%d;bias=%s;post_ops=%d | %s\n",
                                    to_string(dt), to_string(kind), has_scale, to_string(bias),
                                    post_ops, score_mod(p).c_str());
                    }

    // make_block_mask_plan.
    const int lengths[][2] = {{1, 1}, {1, 64}, {64, 1}, {64, 64}, {64, 128}, {128, 64}};
    for (BlockMaskKind m : kMasks)
        for (const auto& l : lengths)
            std::printf("B kind=%s;m=%d;n=%d | %s\n", to_string(m), l[0], l[1],
                        block_mask(make_block_mask_plan(m, l[0], l[1])).c_str());

    // make_causal_mask_tile_descriptor over tiles around the diagonal.
    for (int qs = 0; qs <= 64; qs += 32)
        for (int ks = 0; ks <= 96; ks += 16)
            for (int qz : {1, 16, 32})
                for (int kz : {1, 32}) {
                    const MaskTileDescriptor d = make_causal_mask_tile_descriptor(qs, ks, qz, kz);
                    std::printf("T q_start=%d;k_start=%d;q_size=%d;k_size=%d | required=%s;q_start=%d;"
                                "k_start=%d;q_size=%d;k_size=%d;masked_value=%s;all_masked_row_possible=%s\n",
                                qs, ks, qz, kz, b(d.required).c_str(), d.q_start, d.k_start, d.q_size,
                                d.k_size, f(d.masked_value).c_str(), b(d.all_masked_row_possible).c_str());
                }

    // make_runtime_plan + make_runtime_plan_cache_key.
    const int shapes[][6] = {{1, 1, 64, 64, 32, 32}, {2, 4, 128, 256, 64, 48}, {1, 1, 0, 64, 32, 32}};
    const DataType dsets[][4] = {{DataType::F32, DataType::F32, DataType::F32, DataType::F32},
                                 {DataType::BF16, DataType::BF16, DataType::BF16, DataType::BF16},
                                 {DataType::F32, DataType::F32, DataType::F32, DataType::BF16},
                                 {DataType::Unsupported, DataType::F32, DataType::F32, DataType::F32}};
    // force_reference, enable_onednn, one_dnn_available, one_dnn_post_ops_available
    const int policies[][4] = {{0, 1, 1, 1}, {0, 1, 1, 0}, {0, 1, 0, 0}, {0, 0, 1, 1}, {1, 1, 1, 1}};
    for (const auto& s : shapes)
        for (const auto& ds : dsets)
            for (ScoreModKind kind : kKinds)
                for (int has_scale = 0; has_scale < 2; ++has_scale)
                    for (BiasKind bias : kBiases)
                        for (BlockMaskKind m : kMasks)
                            for (const auto& pol : policies) {
                                RuntimePlanInput in;
                                in.batch = s[0];
                                in.heads = s[1];
                                in.query_length = s[2];
                                in.key_length = s[3];
                                in.head_dim = s[4];
                                in.value_dim = s[5];
                                in.q_dtype = ds[0];
                                in.k_dtype = ds[1];
                                in.v_dtype = ds[2];
                                in.out_dtype = ds[3];
                                in.requested_score_mod = kind;
                                in.has_scale = has_scale != 0;
                                in.scale_value = 0.125f;
                                in.requested_bias_kind = bias;
                                in.requested_block_mask = m;
                                in.force_reference = pol[0] != 0;
                                in.enable_onednn = pol[1] != 0;
                                const RuntimePlan p = plan(in, pol[2] != 0, pol[3] != 0);
                                const RuntimePlanCacheKey key = make_runtime_plan_cache_key(p);
                                std::printf(
                                    "R shape=%dx%dx%dx%dx%dx%d;dtypes=%s,%s,%s,%s;kind=%s;has_scale=%d;"
                                    "bias=%s;mask=%s;force_reference=%d;enable_onednn=%d;onednn=%d;"
                                    "post_ops=%d | %s | %s | backend=%s;layout=%s;lowering=%s;"
                                    "uses_post_ops=%s;epilogue=%s;generator=%s;fallback=%s;"
                                    "signature=%s;debug=%s | shape=%s;dtype=%s;score_mod=%s;"
                                    "block_mask=%s;policy=%s\n",
                                    s[0], s[1], s[2], s[3], s[4], s[5], to_string(ds[0]), to_string(ds[1]),
                                    to_string(ds[2]), to_string(ds[3]), to_string(kind), has_scale,
                                    to_string(bias), to_string(m), pol[0], pol[1], pol[2], pol[3],
                                    score_mod(p.score_mod_plan).c_str(), block_mask(p.block_mask_plan).c_str(),
                                    to_string(p.qk_backend), to_string(p.qk_layout),
                                    to_string(p.qk_lowering_status), b(p.uses_onednn_post_ops).c_str(),
                                    b(p.requires_onednn_flash_epilogue).c_str(),
                                    b(p.requires_mask_tile_generator).c_str(), to_string(p.fallback_reason),
                                    p.runtime_plan_signature.c_str(), p.debug_summary.c_str(),
                                    key.semantic_shape.c_str(), key.dtype_signature.c_str(),
                                    key.score_mod_signature.c_str(), key.block_mask_signature.c_str(),
                                    key.policy_signature.c_str());
                            }
    return 0;
}
