#pragma once

// QK score tile with post-ops, same names and signatures as the reference's
// src/onednn_flash/qk_score_tile_internal.hpp:1-63 (kept under the same file
// name so that its callers, e.g. benchmarks/bench_qk_postops.cpp, build
// unchanged). Q, K, score and bias are host fp32 buffers; the scores are
// computed on the GPU by the exact-order kernel (one fp32 rounding per product
// and per partial sum, k ascending, then * scale, then + bias), which gives
// the reference's results bit for bit whatever backend the plan names.
// Device-resident callers use ofh_qk_score_tile (onednn_flash_hip.h).

#include <cstddef>
#include <string>

#include "onednn_flash/runtime_plan.hpp"
#include "onednn_flash/tile_kernel.hpp"

namespace onednn_flash {

struct QkScoreTilePostOpsInput {
    const float* additive_bias{nullptr};
    std::size_t additive_bias_stride_m{0};
    std::size_t additive_bias_stride_n{1};
};

struct QkScoreTileDebugInfo {
    QkBackendKind backend{QkBackendKind::Reference};
    LoweringStatus lowering_status{LoweringStatus::ReferenceFallback};
    FallbackReason fallback_reason{FallbackReason::None};
    bool used_onednn_post_ops{false};
    std::string message;
};

enum class QkScoreTileSyncMode {
    WaitAfterExecute,
    DeferUntilExplicitWait,
};

struct QkScoreTileExecuteOptions {
    QkScoreTileSyncMode sync_mode{QkScoreTileSyncMode::WaitAfterExecute};
};

// Per-thread counters. This library keeps one device staging buffer per host
// thread in place of the reference's oneDNN primitive cache: a "hit" is a call
// that reused it, a "miss" one that had to grow it, a "rebind" a call whose
// host pointers differ from the previous call's, cache_size the buffers held.
struct QkScoreTileCacheStats {
    std::size_t primitive_cache_hits{0};
    std::size_t primitive_cache_misses{0};
    std::size_t memory_handle_rebinds{0};
    std::size_t immediate_waits{0};
    std::size_t deferred_waits{0};
    std::size_t cache_size{0};
};

// Waits for this thread's deferred calls (the name is the reference's).
void qk_score_tile_wait_for_onednn();

QkScoreTileCacheStats qk_score_tile_get_cache_stats();

void qk_score_tile_reset_cache_stats();

void qk_score_tile_inplace_with_options(const float* q,
                                        const float* k,
                                        float* score,
                                        const StridedMatmulShape& shape,
                                        const RuntimePlan& plan,
                                        const QkScoreTilePostOpsInput& post_ops,
                                        const QkScoreTileExecuteOptions& execute_options,
                                        QkScoreTileDebugInfo* debug = nullptr);

void qk_score_tile_inplace(const float* q,
                           const float* k,
                           float* score,
                           const StridedMatmulShape& shape,
                           const RuntimePlan& plan,
                           const QkScoreTilePostOpsInput& post_ops,
                           QkScoreTileDebugInfo* debug = nullptr);

}  // namespace onednn_flash
