// QK score tile + post-ops microbenchmark on the GPU, the counterpart of the
// reference's benchmarks/bench_qk_postops.cpp: the same shapes, score cases
// (none / scale 0.125 / scale + same-shape bias), sin inputs and inline fp32
// checking loop, and the same JSON record schema
// (onednn_flash.cpp_qk_postops_benchmark.v4, bench_qk_postops.cpp:327-379)
// with fields appended for the device measurements.
//
// Requested backends:
//   hip_host          qk_score_tile_inplace_with_options on host buffers, one
//                     call per tile as the reference's loop (includes the PCIe
//                     copies; sync modes immediate / deferred)
//   hip_device_exact  ofh_qk_score_tile, whole batch in one call on
//                     device-resident fp32 inputs (bit-exact kernel)
//   hip_device_mfma   ofh_qk_score_tile on device-resident bf16 inputs
//                     (matrix-core kernel; checked against the fp32 upcast)
//   cpu_loop          the checking loop itself, the reference's CPU reference
//                     path (shapes up to 128 x 128 only)
// Shapes: the reference's three; --large adds 32 heads of 1024^2 and of
// 4096^2 with d = 128 (device-resident backends only); --large-only runs just those.
// time_ms* are wall-clock per batch (as the reference); device_time_ms_* come
// from HIP events around the device-resident calls.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include "onednn_flash/qk_score_tile_internal.hpp"
#include "onednn_flash/runtime_plan.hpp"
#include "onednn_flash_hip.h"

namespace of = onednn_flash;

namespace {

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

struct ShapeCase {
    int batch, heads;
    std::size_t m, n, d, dv;
};

struct ScoreCase {
    const char* name;
    of::ScoreModKind kind;
    bool has_scale;
    float scale;
    bool has_bias;
};

struct Stats {
    double mean{0}, median{0}, p90{0}, min{0}, max{0}, stddev{0};
};

Stats summarize(std::vector<double> v) {
    Stats s;
    if (v.empty()) return s;
    s.mean = std::accumulate(v.begin(), v.end(), 0.0) / (double)v.size();
    double var = 0.0;
    for (double x : v) var += (x - s.mean) * (x - s.mean);
    s.stddev = std::sqrt(var / (double)v.size());
    std::sort(v.begin(), v.end());
    const std::size_t mid = v.size() / 2;
    s.median = v.size() % 2 ? v[mid] : 0.5 * (v[mid - 1] + v[mid]);
    const std::size_t rank = (std::size_t)std::ceil(0.9 * (double)v.size());
    s.p90 = v[std::min(v.size() - 1, rank == 0 ? 0 : rank - 1)];
    s.min = v.front();
    s.max = v.back();
    return s;
}

struct Record {
    ShapeCase shape;
    std::string requested_backend, actual_backend, qk_layout, score_mod, sync_mode, lowering_status,
        fallback_reason, dtype;
    bool used_onednn_post_ops{false};
    float max_abs_diff{0};
    bool checked_all_rows{true};
    Stats wall, device;
    bool has_device{false};
    double flops{0}, bytes{0};
    int warmup{0}, repeat{0};
    of::QkScoreTileCacheStats cache;
};

std::vector<float> make_values(std::size_t n, float offset) {
    std::vector<float> v(n);
    for (std::size_t i = 0; i < n; ++i) v[i] = std::sin(static_cast<float>(i) * 0.017f + offset) * 0.25f;
    return v;
}

// Round to bfloat16 (nearest even); returns the bits, and the fp32 upcast in place.
std::vector<uint16_t> to_bf16(std::vector<float>& x) {
    std::vector<uint16_t> bits(x.size());
    for (std::size_t i = 0; i < x.size(); ++i) {
        uint32_t u;
        std::memcpy(&u, &x[i], 4);
        u += 0x7FFFu + ((u >> 16) & 1u);
        bits[i] = (uint16_t)(u >> 16);
        const uint32_t back = (uint32_t)bits[i] << 16;
        std::memcpy(&x[i], &back, 4);
    }
    return bits;
}

// The reference microbench's inline expected-value loop (bench_qk_postops.cpp:
// 201-220), over every row or every `row_step`-th row.
void expected_scores(const ShapeCase& sh, const ScoreCase& sc, const std::vector<float>& q,
                     const std::vector<float>& k, const std::vector<float>& bias, std::vector<float>& out,
                     std::size_t row_step) {
    const std::size_t tiles = (std::size_t)sh.batch * sh.heads;
    for (std::size_t t = 0; t < tiles; ++t) {
        const float* qt = q.data() + t * sh.m * sh.d;
        const float* kt = k.data() + t * sh.n * sh.d;
        for (std::size_t i = 0; i < sh.m; i += row_step)
            for (std::size_t j = 0; j < sh.n; ++j) {
                float value = 0.0f;
                for (std::size_t kk = 0; kk < sh.d; ++kk) value += qt[i * sh.d + kk] * kt[j * sh.d + kk];
                if (sc.has_scale) value *= sc.scale;
                if (sc.has_bias) value += bias[t * sh.m * sh.n + i * sh.n + j];
                out[t * sh.m * sh.n + i * sh.n + j] = value;
            }
    }
}

float max_diff_rows(const ShapeCase& sh, const std::vector<float>& a, const std::vector<float>& b,
                    std::size_t row_step) {
    float d = 0.0f;
    const std::size_t tiles = (std::size_t)sh.batch * sh.heads;
    for (std::size_t t = 0; t < tiles; ++t)
        for (std::size_t i = 0; i < sh.m; i += row_step)
            for (std::size_t j = 0; j < sh.n; ++j) {
                const std::size_t x = t * sh.m * sh.n + i * sh.n + j;
                d = std::max(d, std::fabs(a[x] - b[x]));
            }
    return d;
}

of::RuntimePlan make_plan(const ShapeCase& sh, const ScoreCase& sc) {
    of::RuntimePlanInput in;
    in.batch = sh.batch;
    in.heads = sh.heads;
    in.query_length = (int)sh.m;
    in.key_length = (int)sh.n;
    in.head_dim = (int)sh.d;
    in.value_dim = (int)sh.dv;
    in.requested_score_mod = sc.kind;
    in.has_scale = sc.has_scale;
    in.scale_value = sc.scale;
    in.requested_bias_kind = sc.has_bias ? of::BiasKind::SameShapeTile : of::BiasKind::None;
    return of::make_runtime_plan(in, false, false);
}

Record base_record(const ShapeCase& sh, const ScoreCase& sc, const of::RuntimePlan& plan, int warmup,
                   int repeat) {
    Record r;
    r.shape = sh;
    r.qk_layout = of::to_string(plan.qk_layout);
    r.score_mod = plan.score_mod_plan.signature;
    r.warmup = warmup;
    r.repeat = repeat;
    const double tiles = (double)sh.batch * sh.heads;
    r.flops = 2.0 * tiles * (double)sh.m * sh.n * sh.d;
    return r;
}

Record run_host(const ShapeCase& sh, const ScoreCase& sc, bool defer, int warmup, int repeat) {
    const auto plan = make_plan(sh, sc);
    Record r = base_record(sh, sc, plan, warmup, repeat);
    r.requested_backend = "hip_host";
    r.sync_mode = defer ? "defer_until_record_end" : "wait_after_execute";
    r.dtype = "f32";
    const std::size_t tiles = (std::size_t)sh.batch * sh.heads;
    const auto q = make_values(tiles * sh.m * sh.d, 0.1f);
    const auto k = make_values(tiles * sh.n * sh.d, 0.7f);
    const auto bias = make_values(tiles * sh.m * sh.n, 1.3f);
    std::vector<float> expected(tiles * sh.m * sh.n, 0.0f), actual(expected.size(), 0.0f);
    expected_scores(sh, sc, q, k, bias, expected, 1);
    const of::StridedMatmulShape st{sh.m, sh.n, sh.d, sh.d, 1, 1, sh.d, sh.n, 1};
    of::QkScoreTileExecuteOptions opts;
    if (defer) opts.sync_mode = of::QkScoreTileSyncMode::DeferUntilExplicitWait;
    of::QkScoreTileDebugInfo debug;
    auto once = [&]() {
        std::fill(actual.begin(), actual.end(), 0.0f);
        for (std::size_t t = 0; t < tiles; ++t) {
            of::QkScoreTilePostOpsInput post;
            post.additive_bias = sc.has_bias ? bias.data() + t * sh.m * sh.n : nullptr;
            post.additive_bias_stride_m = sh.n;
            post.additive_bias_stride_n = 1;
            of::qk_score_tile_inplace_with_options(q.data() + t * sh.m * sh.d, k.data() + t * sh.n * sh.d,
                                                   actual.data() + t * sh.m * sh.n, st, plan, post, opts,
                                                   &debug);
        }
        if (defer) of::qk_score_tile_wait_for_onednn();
    };
    for (int i = 0; i < warmup; ++i) once();
    of::qk_score_tile_reset_cache_stats();
    std::vector<double> ms;
    for (int i = 0; i < repeat; ++i) {
        const auto t0 = std::chrono::steady_clock::now();
        once();
        ms.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
    }
    r.wall = summarize(ms);
    r.cache = of::qk_score_tile_get_cache_stats();
    r.actual_backend = of::to_string(debug.backend);
    r.lowering_status = of::to_string(debug.lowering_status);
    r.fallback_reason = of::to_string(debug.fallback_reason);
    r.used_onednn_post_ops = debug.used_onednn_post_ops;
    r.max_abs_diff = max_diff_rows(sh, expected, actual, 1);
    r.bytes = 4.0 * tiles * ((double)sh.m * sh.d + (double)sh.n * sh.d + (double)sh.m * sh.n * (sc.has_bias ? 2 : 1));
    return r;
}

Record run_device(const ShapeCase& sh, const ScoreCase& sc, bool bf16, int warmup, int repeat) {
    const auto plan = make_plan(sh, sc);
    Record r = base_record(sh, sc, plan, warmup, repeat);
    r.requested_backend = bf16 ? "hip_device_mfma" : "hip_device_exact";
    r.actual_backend = "hip";
    r.sync_mode = "stream_ordered";
    r.lowering_status = "lowered_to_hip_kernel";
    r.fallback_reason = "none";
    r.dtype = bf16 ? "bf16" : "f32";
    const std::size_t tiles = (std::size_t)sh.batch * sh.heads;
    auto q = make_values(tiles * sh.m * sh.d, 0.1f);
    auto k = make_values(tiles * sh.n * sh.d, 0.7f);
    const auto bias = make_values(tiles * sh.m * sh.n, 1.3f);
    std::vector<uint16_t> qb, kb;
    if (bf16) {
        qb = to_bf16(q);
        kb = to_bf16(k);
    }
    const std::size_t esz = bf16 ? 2 : 4;
    void *dq = nullptr, *dk = nullptr, *dc = nullptr, *dbias = nullptr;
    const std::size_t nc = tiles * sh.m * sh.n;
    hip_ok(hipMalloc(&dq, q.size() * esz), "hipMalloc");
    hip_ok(hipMalloc(&dk, k.size() * esz), "hipMalloc");
    hip_ok(hipMalloc(&dc, nc * 4), "hipMalloc");
    hip_ok(hipMemcpy(dq, bf16 ? (const void*)qb.data() : (const void*)q.data(), q.size() * esz,
                     hipMemcpyHostToDevice), "hipMemcpy");
    hip_ok(hipMemcpy(dk, bf16 ? (const void*)kb.data() : (const void*)k.data(), k.size() * esz,
                     hipMemcpyHostToDevice), "hipMemcpy");
    if (sc.has_bias) {
        hip_ok(hipMalloc(&dbias, nc * 4), "hipMalloc");
        hip_ok(hipMemcpy(dbias, bias.data(), nc * 4, hipMemcpyHostToDevice), "hipMemcpy");
    }
    ofh_qk_score_params p;
    ofh_qk_score_params_init(&p);
    p.batch = (int64_t)tiles;
    p.m = (int64_t)sh.m;
    p.n = (int64_t)sh.n;
    p.k = (int64_t)sh.d;
    p.a_stride_m = (int64_t)sh.d;
    p.a_stride_k = 1;
    p.a_stride_batch = (int64_t)(sh.m * sh.d);
    p.b_stride_k = 1;
    p.b_stride_n = (int64_t)sh.d;
    p.b_stride_batch = (int64_t)(sh.n * sh.d);
    p.c_stride_m = (int64_t)sh.n;
    p.c_stride_n = 1;
    p.c_stride_batch = (int64_t)(sh.m * sh.n);
    p.dtype = bf16 ? OFH_DTYPE_BF16 : OFH_DTYPE_F32;
    p.has_scale = sc.has_scale;
    p.scale = sc.scale;
    if (sc.has_bias) {
        p.bias = (const float*)dbias;
        p.bias_stride_m = (int64_t)sh.n;
        p.bias_stride_n = 1;
        p.bias_stride_batch = (int64_t)(sh.m * sh.n);
    }
    p.algorithm = bf16 ? OFH_QK_MFMA : OFH_QK_EXACT;
    hipStream_t s;
    hip_ok(hipStreamCreate(&s), "hipStreamCreate");
    hipEvent_t e0, e1;
    hip_ok(hipEventCreate(&e0), "hipEventCreate");
    hip_ok(hipEventCreate(&e1), "hipEventCreate");
    auto call = [&]() {
        if (ofh_qk_score_tile(&p, dq, dk, (float*)dc, s) != OFH_SUCCESS)
            throw std::runtime_error(ofh_last_error());
    };
    for (int i = 0; i < warmup; ++i) call();
    hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    std::vector<double> wall, dev;
    for (int i = 0; i < repeat; ++i) {
        const auto t0 = std::chrono::steady_clock::now();
        hip_ok(hipEventRecord(e0, s), "hipEventRecord");
        call();
        hip_ok(hipEventRecord(e1, s), "hipEventRecord");
        hip_ok(hipEventSynchronize(e1), "hipEventSynchronize");
        wall.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
        float ms = 0.0f;
        hip_ok(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        dev.push_back(ms);
    }
    r.wall = summarize(wall);
    r.device = summarize(dev);
    r.has_device = true;
    std::vector<float> actual(nc), expected(nc, 0.0f);
    hip_ok(hipMemcpy(actual.data(), dc, nc * 4, hipMemcpyDeviceToHost), "hipMemcpy");
    // Large tiles: check every 61st row (a prime stride crosses every block row).
    const std::size_t step = sh.m * sh.n * sh.d * tiles > (std::size_t)1 << 28 ? 61 : 1;
    r.checked_all_rows = step == 1;
    expected_scores(sh, sc, q, k, bias, expected, step);
    r.max_abs_diff = max_diff_rows(sh, expected, actual, step);
    r.bytes = (double)tiles * ((double)(sh.m + sh.n) * sh.d * esz + (double)sh.m * sh.n * 4 * (sc.has_bias ? 2 : 1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(s);
    (void)hipFree(dq);
    (void)hipFree(dk);
    (void)hipFree(dc);
    if (dbias) (void)hipFree(dbias);
    return r;
}

Record run_cpu_loop(const ShapeCase& sh, const ScoreCase& sc, int warmup, int repeat) {
    const auto plan = make_plan(sh, sc);
    Record r = base_record(sh, sc, plan, warmup, repeat);
    r.requested_backend = "cpu_loop";
    r.actual_backend = "cpu";
    r.sync_mode = "wait_after_execute";
    r.lowering_status = "reference_fallback";
    r.fallback_reason = "none";
    r.dtype = "f32";
    const std::size_t tiles = (std::size_t)sh.batch * sh.heads;
    const auto q = make_values(tiles * sh.m * sh.d, 0.1f);
    const auto k = make_values(tiles * sh.n * sh.d, 0.7f);
    const auto bias = make_values(tiles * sh.m * sh.n, 1.3f);
    std::vector<float> out(tiles * sh.m * sh.n);
    for (int i = 0; i < warmup; ++i) expected_scores(sh, sc, q, k, bias, out, 1);
    std::vector<double> ms;
    for (int i = 0; i < repeat; ++i) {
        const auto t0 = std::chrono::steady_clock::now();
        expected_scores(sh, sc, q, k, bias, out, 1);
        ms.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
    }
    r.wall = summarize(ms);
    r.bytes = 4.0 * tiles * ((double)sh.m * sh.d + (double)sh.n * sh.d + (double)sh.m * sh.n * (sc.has_bias ? 2 : 1));
    return r;
}

void ensure_parent(const std::string& path) {
    const std::filesystem::path p(path);
    if (p.has_parent_path()) std::filesystem::create_directories(p.parent_path());
}

void write_json(const std::string& path, const std::vector<Record>& recs, const std::string& device) {
    ensure_parent(path);
    std::ofstream out(path);
    if (!out) throw std::runtime_error("failed to open JSON output: " + path);
    out << std::fixed << std::setprecision(6);
    out << "{\n";
    out << "  \"schema\": \"onednn_flash.cpp_qk_postops_benchmark.v4\",\n";
    out << "  \"benchmark_level\": \"cpp_qk_score_tile\",\n";
    out << "  \"git_commit\": \"unknown\",\n";
    out << "  \"one_dnn_version\": \"not_built\",\n";
    out << "  \"device\": \"" << device << "\",\n";
    out << "  \"interpretation_boundary\": \"QK score tile benchmark only; device_time_ms_* are HIP-event "
           "times of device-resident calls, time_ms_* wall clock per batch.\",\n";
    out << "  \"records\": [\n";
    for (std::size_t i = 0; i < recs.size(); ++i) {
        const Record& r = recs[i];
        out << "    {\n";
        out << "      \"shape\": {\"batch\": " << r.shape.batch << ", \"heads\": " << r.shape.heads
            << ", \"m\": " << r.shape.m << ", \"n\": " << r.shape.n << ", \"head_dim\": " << r.shape.d
            << ", \"value_dim\": " << r.shape.dv << "},\n";
        out << "      \"requested_backend\": \"" << r.requested_backend << "\",\n";
        out << "      \"actual_backend\": \"" << r.actual_backend << "\",\n";
        out << "      \"qk_layout\": \"" << r.qk_layout << "\",\n";
        out << "      \"score_mod\": \"" << r.score_mod << "\",\n";
        out << "      \"sync_mode\": \"" << r.sync_mode << "\",\n";
        out << "      \"lowering_status\": \"" << r.lowering_status << "\",\n";
        out << "      \"fallback_reason\": \"" << r.fallback_reason << "\",\n";
        out << "      \"used_onednn_post_ops\": " << (r.used_onednn_post_ops ? "true" : "false") << ",\n";
        out << "      \"max_abs_diff\": " << r.max_abs_diff << ",\n";
        out << "      \"time_ms\": " << r.wall.mean << ",\n";
        out << "      \"time_ms_mean\": " << r.wall.mean << ",\n";
        out << "      \"time_ms_median\": " << r.wall.median << ",\n";
        out << "      \"time_ms_p90\": " << r.wall.p90 << ",\n";
        out << "      \"time_ms_min\": " << r.wall.min << ",\n";
        out << "      \"time_ms_max\": " << r.wall.max << ",\n";
        out << "      \"time_ms_stddev\": " << r.wall.stddev << ",\n";
        out << "      \"warmup\": " << r.warmup << ",\n";
        out << "      \"repeat\": " << r.repeat << ",\n";
        out << "      \"cache_stats\": {\n";
        out << "        \"primitive_cache_hits\": " << r.cache.primitive_cache_hits << ",\n";
        out << "        \"primitive_cache_misses\": " << r.cache.primitive_cache_misses << ",\n";
        out << "        \"memory_handle_rebinds\": " << r.cache.memory_handle_rebinds << ",\n";
        out << "        \"immediate_waits\": " << r.cache.immediate_waits << ",\n";
        out << "        \"deferred_waits\": " << r.cache.deferred_waits << ",\n";
        out << "        \"cache_size\": " << r.cache.cache_size << "\n";
        out << "      },\n";
        out << "      \"dtype\": \"" << r.dtype << "\",\n";
        out << "      \"checked_all_rows\": " << (r.checked_all_rows ? "true" : "false") << ",\n";
        const double t = r.has_device ? r.device.median : r.wall.median;
        if (r.has_device) {
            out << "      \"device_time_ms_mean\": " << r.device.mean << ",\n";
            out << "      \"device_time_ms_median\": " << r.device.median << ",\n";
            out << "      \"device_time_ms_p90\": " << r.device.p90 << ",\n";
            out << "      \"device_time_ms_min\": " << r.device.min << ",\n";
        }
        out << "      \"gflop_per_s\": " << (t > 0 ? r.flops / (t * 1e6) : 0.0) << ",\n";
        out << "      \"gb_per_s\": " << (t > 0 ? r.bytes / (t * 1e6) : 0.0) << "\n";
        out << "    }" << (i + 1 == recs.size() ? "\n" : ",\n");
    }
    out << "  ]\n}\n";
}

void write_csv(const std::string& path, const std::vector<Record>& recs) {
    ensure_parent(path);
    std::ofstream out(path);
    if (!out) throw std::runtime_error("failed to open CSV output: " + path);
    out << "batch,heads,m,n,head_dim,value_dim,requested_backend,actual_backend,qk_layout,score_mod,"
           "sync_mode,lowering_status,fallback_reason,used_onednn_post_ops,max_abs_diff,time_ms,"
           "time_ms_mean,time_ms_median,time_ms_p90,time_ms_min,time_ms_max,time_ms_stddev,warmup,"
           "repeat,cache_hits,cache_misses,handle_rebinds,immediate_waits,deferred_waits,cache_size,"
           "dtype,device_time_ms_median,gflop_per_s,gb_per_s\n";
    out << std::fixed << std::setprecision(6);
    for (const Record& r : recs) {
        const double t = r.has_device ? r.device.median : r.wall.median;
        out << r.shape.batch << ',' << r.shape.heads << ',' << r.shape.m << ',' << r.shape.n << ','
            << r.shape.d << ',' << r.shape.dv << ',' << r.requested_backend << ',' << r.actual_backend << ','
            << r.qk_layout << ',' << r.score_mod << ',' << r.sync_mode << ',' << r.lowering_status << ','
            << r.fallback_reason << ',' << (r.used_onednn_post_ops ? "true" : "false") << ','
            << r.max_abs_diff << ',' << r.wall.mean << ',' << r.wall.mean << ',' << r.wall.median << ','
            << r.wall.p90 << ',' << r.wall.min << ',' << r.wall.max << ',' << r.wall.stddev << ','
            << r.warmup << ',' << r.repeat << ',' << r.cache.primitive_cache_hits << ','
            << r.cache.primitive_cache_misses << ',' << r.cache.memory_handle_rebinds << ','
            << r.cache.immediate_waits << ',' << r.cache.deferred_waits << ',' << r.cache.cache_size << ','
            << r.dtype << ',' << (r.has_device ? r.device.median : 0.0) << ','
            << (t > 0 ? r.flops / (t * 1e6) : 0.0) << ',' << (t > 0 ? r.bytes / (t * 1e6) : 0.0) << '\n';
    }
}

}  // namespace

int main(int argc, char** argv) {
    std::string json_path = "results/qk_postops/cpp-qk-postops.json";
    std::string csv_path = "results/qk_postops/cpp-qk-postops.csv";
    int warmup = 2, repeat = 5;
    bool include_deferred = false, large = false, large_only = false;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--output-json" && i + 1 < argc) json_path = argv[++i];
        else if (a == "--output-csv" && i + 1 < argc) csv_path = argv[++i];
        else if (a == "--warmup" && i + 1 < argc) warmup = std::stoi(argv[++i]);
        else if (a == "--repeat" && i + 1 < argc) repeat = std::stoi(argv[++i]);
        else if (a == "--include-deferred-wait") include_deferred = true;
        else if (a == "--large") large = true;
        else if (a == "--large-only") large = large_only = true;
        else {
            std::cerr << "Unknown argument: " << a << "\n";
            return 2;
        }
    }
    if (warmup < 0 || repeat <= 0) {
        std::cerr << "--warmup must be non-negative and --repeat positive\n";
        return 2;
    }
    try {
        int dev = 0;
        hip_ok(hipGetDevice(&dev), "hipGetDevice");
        hipDeviceProp_t prop;
        hip_ok(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
        std::vector<ShapeCase> shapes{{1, 1, 64, 64, 32, 32}, {1, 1, 128, 128, 64, 64}, {1, 4, 128, 128, 64, 64}};
        if (large_only) shapes.clear();
        const std::size_t reference_shapes = shapes.size();
        if (large) {
            shapes.push_back({1, 32, 1024, 1024, 128, 128});
            shapes.push_back({1, 32, 4096, 4096, 128, 128});
        }
        const ScoreCase cases[] = {{"none", of::ScoreModKind::None, false, 1.0f, false},
                                   {"scale", of::ScoreModKind::Scale, true, 0.125f, false},
                                   {"scale_additive_bias", of::ScoreModKind::ScaleAdditiveBias, true, 0.125f, true}};
        std::vector<Record> recs;
        for (std::size_t si = 0; si < shapes.size(); ++si) {
            const ShapeCase& sh = shapes[si];
            const bool small = si < reference_shapes;
            for (const ScoreCase& sc : cases) {
                std::cerr << "shape " << sh.batch << "x" << sh.heads << "x" << sh.m << "x" << sh.n << "x" << sh.d
                          << " " << sc.name << "\n";
                if (small) {
                    recs.push_back(run_cpu_loop(sh, sc, warmup, repeat));
                    recs.push_back(run_host(sh, sc, false, warmup, repeat));
                    if (include_deferred) recs.push_back(run_host(sh, sc, true, warmup, repeat));
                }
                recs.push_back(run_device(sh, sc, false, warmup, repeat));
                recs.push_back(run_device(sh, sc, true, warmup, repeat));
            }
        }
        write_json(json_path, recs, prop.name);
        write_csv(csv_path, recs);
        for (const Record& r : recs) {
            std::printf("%dx%dx%zux%zux%zu %-20s %-18s %-5s max_abs_diff %-10.3g wall %.4f ms", r.shape.batch,
                        r.shape.heads, r.shape.m, r.shape.n, r.shape.d, r.score_mod.c_str(),
                        r.requested_backend.c_str(), r.dtype.c_str(), r.max_abs_diff, r.wall.median);
            if (r.has_device)
                std::printf("  device %.4f ms  %.1f GB/s  %.1f GFLOP/s", r.device.median,
                            r.bytes / (r.device.median * 1e6), r.flops / (r.device.median * 1e6));
            std::printf("\n");
        }
    } catch (const std::exception& e) {
        std::cerr << "bench_qk_postops: " << e.what() << "\n";
        return 1;
    }
    return 0;
}
