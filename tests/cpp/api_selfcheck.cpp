// Self-check of the C++ API (include/onednn_flash/*.hpp) on the GPU, the
// counterpart of the reference's benchmarks/bench_attention.cpp:33-160: every
// attention entry point against standard_attention on M=N=128, D=64, causal,
// scale 1/8, inputs sin(0.013 i + {0.1, 1.3, 2.7}) * 0.25, max-abs <= 1e-5.
// Also exercises the batched and raw-pointer entries, BlockMask, ScoreBiasFn,
// per-head ALiBi, the tile-GEMM seam and the error contract, and the QK score
// tile with post-ops on the reference microbench's cases
// (benchmarks/bench_qk_postops.cpp:186-231,441-447), bit for bit against its
// inline fp32 loop (build with -ffp-contract=off). Exit code 0 = pass.

#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "onednn_flash/attention.hpp"
#include "onednn_flash/backend.hpp"
#include "onednn_flash/batched_attention.hpp"
#include "onednn_flash/qk_score_tile_internal.hpp"
#include "onednn_flash/runtime_plan.hpp"

namespace of = onednn_flash;

static std::vector<float> sin_values(std::size_t n, float offset) {
    std::vector<float> v(n);
    for (std::size_t i = 0; i < n; ++i) v[i] = std::sin(static_cast<float>(i) * 0.013f + offset) * 0.25f;
    return v;
}

static int failures = 0;
static void expect(bool ok, const char* what, double value) {
    std::printf("%-48s %s (%.3g)\n", what, ok ? "ok" : "FAIL", value);
    if (!ok) ++failures;
}

template <typename E, typename Fn>
static void expect_throw(Fn&& fn, const char* what) {
    bool thrown = false;
    try {
        fn();
    } catch (const E&) {
        thrown = true;
    } catch (...) {
    }
    expect(thrown, what, thrown ? 1.0 : 0.0);
}

// QK score tile: shapes x score cases x sync modes of the reference microbench.
static void qk_score_checks() {
    struct Shape { int batch, heads; std::size_t m, n, d; };
    struct Case { const char* name; of::ScoreModKind kind; bool has_scale; bool has_bias; };
    const Shape shapes[] = {{1, 1, 64, 64, 32}, {1, 1, 128, 128, 64}, {1, 4, 128, 128, 64}};
    const Case cases[] = {{"none", of::ScoreModKind::None, false, false},
                          {"scale", of::ScoreModKind::Scale, true, false},
                          {"scale_additive_bias", of::ScoreModKind::ScaleAdditiveBias, true, true}};
    bool all_exact = true, all_hip = true;
    for (const Shape& sh : shapes) {
        const std::size_t tiles = static_cast<std::size_t>(sh.batch) * sh.heads;
        std::vector<float> q(tiles * sh.m * sh.d), k(tiles * sh.n * sh.d), bias(tiles * sh.m * sh.n);
        for (std::size_t i = 0; i < q.size(); ++i) q[i] = std::sin(static_cast<float>(i) * 0.017f + 0.1f) * 0.25f;
        for (std::size_t i = 0; i < k.size(); ++i) k[i] = std::sin(static_cast<float>(i) * 0.017f + 0.7f) * 0.25f;
        for (std::size_t i = 0; i < bias.size(); ++i) bias[i] = std::sin(static_cast<float>(i) * 0.017f + 1.3f) * 0.25f;
        for (const Case& c : cases) {
            of::RuntimePlanInput in;
            in.batch = sh.batch;
            in.heads = sh.heads;
            in.query_length = static_cast<int>(sh.m);
            in.key_length = static_cast<int>(sh.n);
            in.head_dim = static_cast<int>(sh.d);
            in.value_dim = static_cast<int>(sh.d);
            in.requested_score_mod = c.kind;
            in.has_scale = c.has_scale;
            in.scale_value = 0.125f;
            in.requested_bias_kind = c.has_bias ? of::BiasKind::SameShapeTile : of::BiasKind::None;
            const of::RuntimePlan plan = of::make_runtime_plan(in, false, false);
            all_hip = all_hip && plan.qk_backend == of::QkBackendKind::Hip;
            std::vector<float> expected(tiles * sh.m * sh.n);
            for (std::size_t t = 0; t < tiles; ++t)
                for (std::size_t i = 0; i < sh.m; ++i)
                    for (std::size_t j = 0; j < sh.n; ++j) {
                        float value = 0.0f;
                        for (std::size_t kk = 0; kk < sh.d; ++kk)
                            value += q[(t * sh.m + i) * sh.d + kk] * k[(t * sh.n + j) * sh.d + kk];
                        if (c.has_scale) value *= 0.125f;
                        if (c.has_bias) value += bias[(t * sh.m + i) * sh.n + j];
                        expected[(t * sh.m + i) * sh.n + j] = value;
                    }
            const of::StridedMatmulShape st{sh.m, sh.n, sh.d, sh.d, 1, 1, sh.d, sh.n, 1};
            for (int defer = 0; defer < 2; ++defer) {
                std::vector<float> actual(expected.size(), 0.0f);
                of::QkScoreTileExecuteOptions opts;
                if (defer) opts.sync_mode = of::QkScoreTileSyncMode::DeferUntilExplicitWait;
                of::QkScoreTileDebugInfo debug;
                for (std::size_t t = 0; t < tiles; ++t) {
                    of::QkScoreTilePostOpsInput post;
                    post.additive_bias = c.has_bias ? bias.data() + t * sh.m * sh.n : nullptr;
                    post.additive_bias_stride_m = sh.n;
                    post.additive_bias_stride_n = 1;
                    of::qk_score_tile_inplace_with_options(q.data() + t * sh.m * sh.d,
                                                           k.data() + t * sh.n * sh.d,
                                                           actual.data() + t * sh.m * sh.n, st, plan,
                                                           post, opts, &debug);
                }
                if (defer) of::qk_score_tile_wait_for_onednn();
                const bool exact = std::memcmp(actual.data(), expected.data(), expected.size() * 4) == 0;
                all_exact = all_exact && exact && debug.backend == of::QkBackendKind::Hip &&
                            debug.lowering_status == of::LoweringStatus::LoweredToHipKernel;
                if (!exact)
                    std::printf("  qk_score_tile %dx%dx%zux%zux%zu %s defer=%d: max diff %g\n", sh.batch,
                                sh.heads, sh.m, sh.n, sh.d, c.name, defer, of::max_abs_diff(actual, expected));
            }
        }
    }
    expect(all_hip, "make_runtime_plan picks the HIP backend", all_hip ? 1.0 : 0.0);
    expect(all_exact, "qk_score_tile_inplace: 18 records bit-exact", all_exact ? 1.0 : 0.0);

    // cache and wait counters
    of::qk_score_tile_reset_cache_stats();
    std::vector<float> q(64 * 32, 0.5f), k(64 * 32, 0.25f), s(64 * 64);
    of::RuntimePlanInput in;
    in.query_length = in.key_length = 64;
    in.head_dim = in.value_dim = 32;
    const of::RuntimePlan plan = of::make_runtime_plan(in, false, false);
    const of::StridedMatmulShape st{64, 64, 32, 32, 1, 1, 32, 64, 1};
    for (int i = 0; i < 3; ++i) of::qk_score_tile_inplace(q.data(), k.data(), s.data(), st, plan, {});
    of::QkScoreTileExecuteOptions deferred;
    deferred.sync_mode = of::QkScoreTileSyncMode::DeferUntilExplicitWait;
    of::qk_score_tile_inplace_with_options(q.data(), k.data(), s.data(), st, plan, {}, deferred);
    of::qk_score_tile_wait_for_onednn();
    const auto stats = of::qk_score_tile_get_cache_stats();
    expect(stats.immediate_waits == 3 && stats.deferred_waits == 1 && stats.cache_size == 1 &&
               stats.primitive_cache_hits + stats.primitive_cache_misses == 4,
           "qk_score_tile cache stats", static_cast<double>(stats.primitive_cache_hits));
    expect(s[0] == 4.0f, "qk_score_tile value 32*0.5*0.25", s[0]);

    // error contract (qk_score_tile.cpp:16-26,36-47)
    expect_throw<std::invalid_argument>([&] {
        of::qk_score_tile_inplace(q.data(), k.data(), s.data(), of::StridedMatmulShape{0, 64, 32, 32, 1, 1, 32, 64, 1},
                                  plan, {});
    }, "qk_score_tile zero dims throws invalid_argument");
    expect_throw<std::invalid_argument>([&] {
        of::qk_score_tile_inplace(nullptr, k.data(), s.data(), st, plan, {});
    }, "qk_score_tile null pointer throws invalid_argument");
    expect_throw<std::invalid_argument>([&] {
        of::RuntimePlanInput bin = in;
        bin.requested_score_mod = of::ScoreModKind::AdditiveBias;
        bin.requested_bias_kind = of::BiasKind::SameShapeTile;
        of::qk_score_tile_inplace(q.data(), k.data(), s.data(), st, of::make_runtime_plan(bin, false, false), {});
    }, "qk_score_tile missing bias throws invalid_argument");
}

int main() {
    const of::AttentionShape shape{128, 128, 64, 64};
    const auto q = sin_values(shape.query_tokens * shape.head_dim, 0.1f);
    const auto k = sin_values(shape.key_tokens * shape.head_dim, 1.3f);
    const auto v = sin_values(shape.key_tokens * shape.value_dim, 2.7f);
    const of::AttentionOptions options{1.0f / std::sqrt(static_cast<float>(shape.head_dim)), true, 32};

    const auto standard = of::standard_attention(q, k, v, shape, options);
    auto tile_opts = options;
    tile_opts.query_block_size = 16;
    expect(of::max_abs_diff(standard, of::flash_attention_tiled(q, k, v, shape, options)) <= 1e-5f,
           "flash_attention_tiled vs standard", of::max_abs_diff(standard, of::flash_attention_tiled(q, k, v, shape, options)));
    const double d_q = of::max_abs_diff(standard, of::flash_attention_q_tile(q, k, v, shape, tile_opts));
    expect(d_q <= 1e-5, "flash_attention_q_tile vs standard", d_q);
    const double d_qkpv = of::max_abs_diff(standard, of::flash_attention_qk_pv_tile(q, k, v, shape, tile_opts));
    expect(d_qkpv <= 1e-5, "flash_attention_qk_pv_tile vs standard", d_qkpv);
    const double d_run = of::max_abs_diff(standard, of::run_attention(of::AttentionBackendKind::FlashMfmaHip, q, k, v, shape, options));
    expect(d_run <= 1e-5, "run_attention(FlashMfmaHip) vs standard", d_run);

    std::vector<float> out_ws(shape.query_tokens * shape.value_dim, -1.0f);
    of::AttentionWorkspace ws;
    of::flash_attention_qk_pv_tile_ws(q.data(), k.data(), v.data(), out_ws.data(), shape, tile_opts, ws);
    void* const first_buffer = ws.device_buffer;
    of::flash_attention_qk_pv_tile_ws(q.data(), k.data(), v.data(), out_ws.data(), shape, tile_opts, ws);
    expect(ws.device_buffer == first_buffer, "workspace reused without reallocation", 0.0);
    {
        // the reference's public tile buffers, sized by resize() as there
        of::AttentionWorkspace w2;
        w2.resize(32, 64, 16, 8);
        const bool sizes = w2.q_tile.size() == 32 * 16 && w2.k_tile_t.size() == 16 * 64 && w2.v_tile.size() == 64 * 8 &&
                           w2.score_tile.size() == 32 * 64 && w2.p_tile.size() == 32 * 64 &&
                           w2.pv_tile.size() == 32 * 8 && w2.acc.size() == 32 * 8 && w2.running_max.size() == 32 &&
                           w2.running_sum.size() == 32 && w2.old_scales.size() == 32 && w2.new_maxes.size() == 32 &&
                           w2.block_sums.size() == 32 && w2.row_has_valid.size() == 32;
        w2.q_tile[5] = 3.0f;
        of::AttentionWorkspace w3 = w2;  // copy: host buffers, no shared device memory
        const bool copied = w3.q_tile.size() == w2.q_tile.size() && w3.q_tile[5] == 3.0f &&
                            w3.device_buffer == nullptr && w2.device_buffer != nullptr;
        of::AttentionWorkspace w4 = std::move(w2);  // move: both, and the source gives up its device memory
        const bool moved = w4.q_tile.size() == 32 * 16 && w4.device_buffer != nullptr && w2.device_buffer == nullptr;
        expect(sizes && copied && moved, "workspace tile buffers, copy and move", sizes + 2.0 * copied + 4.0 * moved);
    }
    expect(of::max_abs_diff(standard, out_ws) <= 1e-5f, "flash_attention_qk_pv_tile_ws vs standard",
           of::max_abs_diff(standard, out_ws));

    // batched: two heads with different data == two single-head calls
    const of::BatchedAttentionShape bshape{1, 2, 128, 128, 64, 64};
    std::vector<float> bq(q), bk(k), bv(v);
    const auto q2 = sin_values(q.size(), 0.5f), k2 = sin_values(k.size(), 0.9f), v2 = sin_values(v.size(), 1.7f);
    bq.insert(bq.end(), q2.begin(), q2.end());
    bk.insert(bk.end(), k2.begin(), k2.end());
    bv.insert(bv.end(), v2.begin(), v2.end());
    std::vector<float> bout(2 * 128 * 64);
    of::flash_attention_batched_qk_pv_tile(bq.data(), bk.data(), bv.data(), bout.data(), bshape, options);
    const auto second = of::standard_attention(q2, k2, v2, shape, options);
    const std::vector<float> h0(bout.begin(), bout.begin() + 128 * 64), h1(bout.begin() + 128 * 64, bout.end());
    expect(of::max_abs_diff(h0, standard) <= 1e-5f && of::max_abs_diff(h1, second) <= 1e-5f,
           "batched entry vs per-head standard", std::max(of::max_abs_diff(h0, standard), of::max_abs_diff(h1, second)));

    // BlockMask + ScoreBiasFn (ALiBi through the callback) vs per-head ALiBi slopes
    of::BlockMask bm;
    bm.query_block_size = 32;
    bm.key_block_size = 32;
    bm.query_blocks = 4;
    bm.key_blocks = 4;
    bm.allowed = {1, 0, 0, 0, 1, 1, 0, 0, 0, 1, 1, 0, 1, 0, 1, 1};
    auto mopts = options;
    mopts.block_mask = &bm;
    mopts.score_bias = [](std::size_t qi, std::size_t kj) {
        return 0.25f * static_cast<float>(static_cast<long>(kj) - static_cast<long>(qi));
    };
    const auto std_mask = of::standard_attention(q, k, v, shape, mopts);
    const auto fl_mask = of::flash_attention_tiled(q, k, v, shape, mopts);
    expect(of::max_abs_diff(std_mask, fl_mask) <= 1e-5f, "block mask + score_bias: flash vs standard",
           of::max_abs_diff(std_mask, fl_mask));
    {   // the callback runs only for pairs that the block mask and the causal rule let through
        size_t calls = 0, masked_calls = 0;
        auto copts = mopts;
        copts.causal = true;
        copts.score_bias = [&](std::size_t qi, std::size_t kj) {
            ++calls;
            if (kj > qi || !bm.allows(qi, kj)) ++masked_calls;
            return 0.0f;
        };
        (void)of::flash_attention_tiled(q, k, v, shape, copts);
        size_t unmasked = 0;
        for (std::size_t qi = 0; qi < shape.query_tokens; ++qi)
            for (std::size_t kj = 0; kj <= qi && kj < shape.key_tokens; ++kj) unmasked += bm.allows(qi, kj) ? 1 : 0;
        expect(masked_calls == 0 && calls == unmasked, "score_bias evaluated on unmasked pairs only",
               (float)masked_calls);
        // a dense bias beyond 2 GiB is refused before any device work
        of::AttentionShape big = shape;
        big.query_tokens = big.key_tokens = 32768;
        auto bopts = options;
        bopts.score_bias = [](std::size_t, std::size_t) { return 0.0f; };
        bool refused = false;
        try {
            (void)of::flash_attention_tiled(std::vector<float>(big.query_tokens * big.head_dim),
                                            std::vector<float>(big.key_tokens * big.head_dim),
                                            std::vector<float>(big.key_tokens * big.value_dim), big, bopts);
        } catch (const std::invalid_argument& e) {
            refused = std::string(e.what()).find("exceeds 2 GiB") != std::string::npos;
        }
        expect(refused, "score_bias over 2 GiB refused", 0.0f);
    }
    auto aopts = options;
    aopts.block_mask = &bm;
    aopts.alibi_slopes = {0.25f};
    const auto fl_alibi = of::flash_attention_tiled(q, k, v, shape, aopts);
    expect(of::max_abs_diff(std_mask, fl_alibi) <= 1e-5f, "alibi_slopes == ALiBi ScoreBiasFn",
           of::max_abs_diff(std_mask, fl_alibi));
    expect(bm.allows(40, 10) && !bm.allows(10, 40) && !bm.allows(500, 0), "BlockMask::allows", 0.0);

    // tile-GEMM seam: C = A x B and the strided K^T view
    const of::MatmulShape ms{5, 7, 3};
    std::vector<float> a(15), b(21);
    for (int i = 0; i < 15; ++i) a[i] = 0.5f * i - 3.0f;
    for (int i = 0; i < 21; ++i) b[i] = 0.25f * i - 2.0f;
    const auto c = of::matmul_tile(of::TileKernelKind::HipMfma, a, b, ms);
    std::vector<float> c_ref(35);
    for (int i = 0; i < 5; ++i)
        for (int j = 0; j < 7; ++j) {
            float s = 0.0f;
            for (int kk = 0; kk < 3; ++kk) s += a[i * 3 + kk] * b[kk * 7 + j];
            c_ref[i * 7 + j] = s;
        }
    expect(std::memcmp(c.data(), c_ref.data(), 35 * 4) == 0, "matmul_tile (bit-exact)",
           of::max_abs_diff(c, c_ref));
    std::vector<float> kt(7 * 3);  // K[7,3] row-major, read as B = K^T [3,7]
    for (int j = 0; j < 7; ++j)
        for (int kk = 0; kk < 3; ++kk) kt[j * 3 + kk] = b[kk * 7 + j];
    std::vector<float> cs(35, 0.0f);
    of::matmul_tile_strided_inplace(of::TileKernelKind::Reference, a.data(), kt.data(), cs.data(),
                                    of::StridedMatmulShape{5, 7, 3, 3, 1, 1, 3, 7, 1});
    expect(std::memcmp(cs.data(), c.data(), 35 * 4) == 0, "matmul_tile_strided_inplace (bit-exact)",
           of::max_abs_diff(cs, c));

    qk_score_checks();

    // error contract
    expect_throw<std::invalid_argument>([&] { of::standard_attention(q, k, std::vector<float>(3), shape, options); },
                                        "V size mismatch throws invalid_argument");
    expect_throw<std::invalid_argument>([&] {
        auto o = options;
        o.key_block_size = 0;
        of::flash_attention_tiled(q, k, v, shape, o);
    }, "key_block_size 0 throws invalid_argument");
    expect_throw<std::invalid_argument>([&] {
        of::BlockMask bad = bm;
        bad.allowed.pop_back();
        auto o = options;
        o.block_mask = &bad;
        of::standard_attention(q, k, v, shape, o);
    }, "bad BlockMask throws invalid_argument");
    expect_throw<std::runtime_error>([&] {
        // the MFMA kernels serve head dims up to 256
        of::run_attention(of::AttentionBackendKind::FlashMfmaHip, sin_values(128 * 264, 0.f), sin_values(128 * 264, 1.f),
                          sin_values(128 * 264, 2.f), of::AttentionShape{128, 128, 264, 264}, options);
    }, "unsupported MFMA shape throws runtime_error");

    std::printf("%s\n", failures == 0 ? "ALL OK" : "FAILURES");
    return failures == 0 ? 0 : 1;
}
