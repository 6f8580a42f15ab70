// QK score tile with post-ops on host buffers (qk_score_tile_internal.hpp):
// validation with the reference's messages (src/onednn_flash/qk_score_tile.cpp:
// 16-26, 36-47), staging into a per-thread device buffer, the exact-order
// HIP score kernel through the C ABI, and the copy back. Immediate calls wait
// for the result; deferred calls leave it queued on this thread's stream until
// qk_score_tile_wait_for_onednn().

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "onednn_flash/qk_score_tile_internal.hpp"
#include "onednn_flash_hip.h"

namespace onednn_flash {
namespace {

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

struct QkContext {
    void* buffer{nullptr};
    std::size_t bytes{0};
    int device{-1};
    hipStream_t stream{nullptr};
    bool pending{false};
    const void* last_ptrs[4]{nullptr, nullptr, nullptr, nullptr};
    QkScoreTileCacheStats stats;

    ~QkContext() {
        // Process teardown: release quietly (the runtime may already be gone).
        if (stream != nullptr) (void)hipStreamSynchronize(stream);
        if (buffer != nullptr) (void)hipFree(buffer);
        if (stream != nullptr) (void)hipStreamDestroy(stream);
    }

    // Stream and staging buffer of at least `need` bytes on the current device.
    void prepare(std::size_t need) {
        int dev = 0;
        check_hip(hipGetDevice(&dev), "hipGetDevice");
        if (dev != device) {
            if (stream != nullptr) {
                check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
                pending = false;
                (void)hipFree(buffer);
                (void)hipStreamDestroy(stream);
                buffer = nullptr;
                bytes = 0;
                stream = nullptr;
            }
            check_hip(hipStreamCreate(&stream), "hipStreamCreate");
            device = dev;
        }
        if (buffer != nullptr && bytes >= need) {
            ++stats.primitive_cache_hits;
            return;
        }
        ++stats.primitive_cache_misses;
        if (buffer != nullptr) {
            check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
            check_hip(hipFree(buffer), "hipFree");
            buffer = nullptr;
            bytes = 0;
        }
        check_hip(hipMalloc(&buffer, need), "hipMalloc");
        bytes = need;
    }
};

QkContext& context() {
    thread_local QkContext ctx;
    return ctx;
}

std::size_t round_up(std::size_t x) { return (x + 255) & ~std::size_t(255); }

// Elements spanned by a strided [rows, cols] view.
std::size_t extent(std::size_t rows, std::size_t cols, std::size_t s_row, std::size_t s_col) {
    return (rows - 1) * s_row + (cols - 1) * s_col + 1;
}

void set_debug(QkScoreTileDebugInfo* debug, const std::string& message) {
    if (debug == nullptr) return;
    debug->backend = QkBackendKind::Hip;
    debug->lowering_status = LoweringStatus::LoweredToHipKernel;
    debug->fallback_reason = FallbackReason::None;
    debug->used_onednn_post_ops = false;
    debug->message = message;
}

}  // namespace

void qk_score_tile_wait_for_onednn() {
    QkContext& ctx = context();
    if (ctx.pending) {
        check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
        ctx.pending = false;
        ++ctx.stats.deferred_waits;
    }
}

QkScoreTileCacheStats qk_score_tile_get_cache_stats() {
    QkScoreTileCacheStats s = context().stats;
    s.cache_size = context().buffer != nullptr ? 1 : 0;
    return s;
}

void qk_score_tile_reset_cache_stats() {
    QkContext& ctx = context();
    ctx.stats = QkScoreTileCacheStats{};
}

void qk_score_tile_inplace_with_options(const float* q,
                                        const float* k,
                                        float* score,
                                        const StridedMatmulShape& shape,
                                        const RuntimePlan& plan,
                                        const QkScoreTilePostOpsInput& post_ops,
                                        const QkScoreTileExecuteOptions& execute_options,
                                        QkScoreTileDebugInfo* debug) {
    if (shape.m == 0 || shape.n == 0 || shape.k == 0)
        throw std::invalid_argument("QK score tile dimensions must be non-zero");
    if (q == nullptr || k == nullptr || score == nullptr)
        throw std::invalid_argument("QK score tile pointers must be non-null");
    const ScoreModPlan& sm = plan.score_mod_plan;
    if (sm.has_bias && post_ops.additive_bias == nullptr)
        throw std::invalid_argument("QK score tile additive bias pointer is required by plan");

    const std::size_t na = extent(shape.m, shape.k, shape.a_stride_m, shape.a_stride_k);
    const std::size_t nb = extent(shape.k, shape.n, shape.b_stride_k, shape.b_stride_n);
    const std::size_t nc = extent(shape.m, shape.n, shape.c_stride_m, shape.c_stride_n);
    const std::size_t nbias =
        sm.has_bias ? extent(shape.m, shape.n, post_ops.additive_bias_stride_m,
                             post_ops.additive_bias_stride_n)
                    : 0;
    const std::size_t off_b = round_up(na * 4), off_c = off_b + round_up(nb * 4);
    const std::size_t off_bias = off_c + round_up(nc * 4);

    QkContext& ctx = context();
    const void* ptrs[4] = {q, k, score, post_ops.additive_bias};
    for (int i = 0; i < 4; ++i) {
        if (ptrs[i] != ctx.last_ptrs[i]) {
            ++ctx.stats.memory_handle_rebinds;
            break;
        }
    }
    for (int i = 0; i < 4; ++i) ctx.last_ptrs[i] = ptrs[i];
    ctx.prepare(off_bias + round_up(nbias * 4));
    char* base = static_cast<char*>(ctx.buffer);
    hipStream_t s = ctx.stream;

    check_hip(hipMemcpyAsync(base, q, na * 4, hipMemcpyHostToDevice, s), "hipMemcpyAsync(q)");
    check_hip(hipMemcpyAsync(base + off_b, k, nb * 4, hipMemcpyHostToDevice, s), "hipMemcpyAsync(k)");
    // A strided score view keeps the caller's values between its elements.
    const bool dense_c = shape.c_stride_n == 1 && shape.c_stride_m == shape.n;
    if (!dense_c)
        check_hip(hipMemcpyAsync(base + off_c, score, nc * 4, hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync(score)");
    if (sm.has_bias)
        check_hip(hipMemcpyAsync(base + off_bias, post_ops.additive_bias, nbias * 4,
                                 hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync(bias)");

    ofh_qk_score_params p;
    ofh_qk_score_params_init(&p);
    p.batch = 1;
    p.m = (int64_t)shape.m;
    p.n = (int64_t)shape.n;
    p.k = (int64_t)shape.k;
    p.a_stride_m = (int64_t)shape.a_stride_m;
    p.a_stride_k = (int64_t)shape.a_stride_k;
    p.b_stride_k = (int64_t)shape.b_stride_k;
    p.b_stride_n = (int64_t)shape.b_stride_n;
    p.c_stride_m = (int64_t)shape.c_stride_m;
    p.c_stride_n = (int64_t)shape.c_stride_n;
    p.dtype = OFH_DTYPE_F32;
    p.has_scale = sm.has_scale ? 1 : 0;
    p.scale = sm.scale_value;
    if (sm.has_bias) {
        p.bias = reinterpret_cast<const float*>(base + off_bias);
        p.bias_stride_m = (int64_t)post_ops.additive_bias_stride_m;
        p.bias_stride_n = (int64_t)post_ops.additive_bias_stride_n;
    }
    p.softcap = sm.has_softcap ? sm.softcap_value : 0.0f;
    p.algorithm = OFH_QK_EXACT;
    const int rc = ofh_qk_score_tile(&p, base, base + off_b, reinterpret_cast<float*>(base + off_c), s);
    if (rc == OFH_ERROR_INVALID_ARGUMENT) throw std::invalid_argument(ofh_last_error());
    if (rc != OFH_SUCCESS) throw std::runtime_error(ofh_last_error());
    check_hip(hipMemcpyAsync(score, base + off_c, nc * 4, hipMemcpyDeviceToHost, s),
              "hipMemcpyAsync(score)");

    const bool defer = execute_options.sync_mode == QkScoreTileSyncMode::DeferUntilExplicitWait;
    std::string message = "qk_score_tile: HIP exact-order kernel";
    if (plan.qk_backend != QkBackendKind::Hip)
        message += std::string(" (plan asked for ") + to_string(plan.qk_backend) + ")";
    if (defer) {
        ctx.pending = true;
        message += ", deferred stream wait";
    } else {
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        ctx.pending = false;
        ++ctx.stats.immediate_waits;
    }
    set_debug(debug, message);
}

void qk_score_tile_inplace(const float* q,
                           const float* k,
                           float* score,
                           const StridedMatmulShape& shape,
                           const RuntimePlan& plan,
                           const QkScoreTilePostOpsInput& post_ops,
                           QkScoreTileDebugInfo* debug) {
    qk_score_tile_inplace_with_options(q, k, score, shape, plan, post_ops,
                                       QkScoreTileExecuteOptions{}, debug);
}

}  // namespace onednn_flash
