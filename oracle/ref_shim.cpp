// C entry points over the reference's own attention library, compiled from the
// reference sources where they lie (oracle/Makefile). TEST INFRASTRUCTURE
// ONLY: used to write golden vectors, to cross-check the oracle restatement,
// and as the "reference" CPU baseline. Nothing shipped links it.
//
// Every function returns 0 on success and -1 when the reference threw; the
// exception text is available from ref_last_error().

#include <cstddef>
#include <cstdint>
#include <exception>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "onednn_flash/attention.hpp"
#include "onednn_flash/batched_attention.hpp"
#include "onednn_flash/qk_score_tile_internal.hpp"

namespace {

thread_local std::string g_err;

struct RefCase {
    std::size_t M, N, D, Dv;
    float scale;
    int causal;
    std::size_t q_bs, k_bs;
    const std::uint8_t* mask;  // may be null
    std::size_t mqbs, mkbs, mqb, mkb;
    float alibi_slope;         // used when has_alibi
    int has_alibi;
};

onednn_flash::AttentionOptions make_options(const RefCase& c, onednn_flash::BlockMask& bm) {
    onednn_flash::AttentionOptions o;
    o.scale = c.scale;
    o.causal = c.causal != 0;
    o.key_block_size = c.k_bs;
    o.query_block_size = c.q_bs;
    if (c.mask != nullptr) {
        bm.query_block_size = c.mqbs;
        bm.key_block_size = c.mkbs;
        bm.query_blocks = c.mqb;
        bm.key_blocks = c.mkb;
        bm.allowed.assign(c.mask, c.mask + c.mqb * c.mkb);
        o.block_mask = &bm;
    }
    if (c.has_alibi) {
        const float slope = c.alibi_slope;
        o.score_bias = [slope](std::size_t qi, std::size_t kj) {
            return slope * static_cast<float>(static_cast<std::int64_t>(kj) -
                                              static_cast<std::int64_t>(qi));
        };
    }
    return o;
}

template <typename Fn>
int guarded(Fn&& fn) {
    try {
        fn();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_err.c_str(); }

// variant: 0 standard_attention, 1 flash_attention_tiled, 2 flash_attention_q_tile,
// 3 flash_attention_qk_pv_tile, 4 flash_attention_qk_pv_tile_ws (StridedK).
int ref_attention_head(int variant, const float* q, const float* k, const float* v, float* out,
                       std::size_t M, std::size_t N, std::size_t D, std::size_t Dv, float scale,
                       int causal, std::size_t q_bs, std::size_t k_bs, const std::uint8_t* mask,
                       std::size_t mqbs, std::size_t mkbs, std::size_t mqb, std::size_t mkb,
                       int has_alibi, float alibi_slope) {
    return guarded([&]() {
        const RefCase c{M, N, D, Dv, scale, causal, q_bs, k_bs, mask, mqbs, mkbs, mqb, mkb,
                        alibi_slope, has_alibi};
        onednn_flash::BlockMask bm;
        const auto options = make_options(c, bm);
        const onednn_flash::AttentionShape shape{M, N, D, Dv};
        if (variant == 4) {
            onednn_flash::AttentionWorkspace ws;
            onednn_flash::flash_attention_qk_pv_tile_ws(q, k, v, out, shape, options, ws);
            return;
        }
        const std::vector<float> qv(q, q + M * D), kv(k, k + N * D), vv(v, v + N * Dv);
        std::vector<float> r;
        switch (variant) {
            case 0: r = onednn_flash::standard_attention(qv, kv, vv, shape, options); break;
            case 1: r = onednn_flash::flash_attention_tiled(qv, kv, vv, shape, options); break;
            case 2: r = onednn_flash::flash_attention_q_tile(qv, kv, vv, shape, options); break;
            case 3: r = onednn_flash::flash_attention_qk_pv_tile(qv, kv, vv, shape, options); break;
            default: throw std::invalid_argument("unknown variant");
        }
        for (std::size_t i = 0; i < r.size(); ++i) out[i] = r[i];
    });
}

// flash_attention_batched_qk_pv_tile over an explicit list of flat heads of
// contiguous [B,H,*,*] tensors, one head per call, heads split across
// `threads` host threads (the reference keeps a thread_local workspace per
// thread, batched_attention.cpp:37). out is [nheads, M, Dv]. alibi_slopes is
// indexed by head_idx % heads when non-null.
int ref_flash_batched_heads(const float* q, const float* k, const float* v, float* out,
                            std::size_t heads, std::size_t M, std::size_t N, std::size_t D,
                            std::size_t Dv, float scale, int causal, std::size_t q_bs,
                            std::size_t k_bs, const std::uint8_t* mask, std::size_t mqbs,
                            std::size_t mkbs, std::size_t mqb, std::size_t mkb,
                            const float* alibi_slopes, const std::size_t* head_idx,
                            std::size_t nheads, int threads) {
    std::vector<std::string> errors(static_cast<std::size_t>(threads > 0 ? threads : 1));
    const std::size_t nt = errors.size();
    auto worker = [&](std::size_t w) {
        try {
            for (std::size_t i = w; i < nheads; i += nt) {
                const std::size_t bh = head_idx[i];
                const RefCase c{M, N, D, Dv, scale, causal, q_bs, k_bs, mask, mqbs, mkbs, mqb, mkb,
                                alibi_slopes ? alibi_slopes[bh % heads] : 0.0f,
                                alibi_slopes != nullptr};
                onednn_flash::BlockMask bm;
                const auto options = make_options(c, bm);
                const onednn_flash::BatchedAttentionShape shape{1, 1, M, N, D, Dv};
                onednn_flash::flash_attention_batched_qk_pv_tile(
                    q + bh * M * D, k + bh * N * D, v + bh * N * Dv, out + i * M * Dv, shape,
                    options);
            }
        } catch (const std::exception& e) {
            errors[w] = e.what();
        }
    };
    std::vector<std::thread> pool;
    for (std::size_t w = 1; w < nt; ++w) pool.emplace_back(worker, w);
    worker(0);
    for (auto& t : pool) t.join();
    for (const auto& e : errors) {
        if (!e.empty()) {
            g_err = e;
            return -1;
        }
    }
    return 0;
}

// qk_score_tile_inplace (src/onednn_flash/qk_score_tile.cpp:404-418) on one
// strided fp32 tile, with the plan make_runtime_plan gives for a build without
// oneDNN (the reference tile product plus reference post-ops). bias may be null.
int ref_qk_score_tile(const float* q, const float* k, float* score, std::size_t m, std::size_t n,
                      std::size_t kdim, std::size_t a_sm, std::size_t a_sk, std::size_t b_sk,
                      std::size_t b_sn, std::size_t c_sm, std::size_t c_sn, int has_scale,
                      float scale, const float* bias, std::size_t bias_sm, std::size_t bias_sn) {
    return guarded([&]() {
        onednn_flash::RuntimePlanInput in;
        in.query_length = static_cast<int>(m);
        in.key_length = static_cast<int>(n);
        in.head_dim = static_cast<int>(kdim);
        in.value_dim = static_cast<int>(kdim);
        in.has_scale = has_scale != 0;
        in.scale_value = scale;
        if (bias != nullptr) {
            in.requested_score_mod = has_scale ? onednn_flash::ScoreModKind::ScaleAdditiveBias
                                               : onednn_flash::ScoreModKind::AdditiveBias;
            in.requested_bias_kind = onednn_flash::BiasKind::SameShapeTile;
        } else {
            in.requested_score_mod = has_scale ? onednn_flash::ScoreModKind::Scale
                                               : onednn_flash::ScoreModKind::None;
        }
        const auto plan = onednn_flash::make_runtime_plan(in, false, false);
        onednn_flash::QkScoreTilePostOpsInput post_ops;
        post_ops.additive_bias = bias;
        post_ops.additive_bias_stride_m = bias_sm;
        post_ops.additive_bias_stride_n = bias_sn;
        const onednn_flash::StridedMatmulShape shape{m, n, kdim, a_sm, a_sk, b_sk, b_sn, c_sm, c_sn};
        onednn_flash::qk_score_tile_inplace(q, k, score, shape, plan, post_ops);
    });
}

}  // extern "C"
