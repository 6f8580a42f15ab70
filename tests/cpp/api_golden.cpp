// Runs every C++ API entry point (include/onednn_flash/*.hpp) on one golden
// case and writes their outputs, so that tests/test_gpu_cpp_api.py can compare
// them with the compiled reference's outputs stored in tests/golden/*.npz
// (written by tests/golden/make_golden.py from src/onednn_flash/attention.cpp).
//
// Usage: api_golden <case.bin> <out.bin>
//
// case.bin, little-endian: int64 M, N, D, Dv, causal, has_mask, mask_qbs,
// mask_kbs, mask_qb, mask_kb, has_alibi, ntiles, then ntiles (q_bs, k_bs)
// int64 pairs; float32 scale, alibi_slope; float32 q[M*D], k[N*D], v[N*Dv];
// uint8 mask[mask_qb*mask_kb] when has_mask.
//
// out.bin: float32 blocks of M*Dv values, in this order:
//   standard_attention, flash_attention_tiled (key_block_size = k_bs of tile 0),
//   flash_attention_q_tile (tile 0), flash_attention_qk_pv_tile (tile 0),
//   flash_attention_qk_pv_tile_ws for every tile, flash_attention_batched_qk_pv_tile
//   (one head), run_attention(StandardReference), run_attention(FlashTiledReference),
//   run_attention(FlashMfmaHip) (the MFMA kernel, also for head dims that are not
//   a multiple of 32 and D != Dv), and, when the case has an ALiBi slope, flash_attention_tiled with the slope
//   as per-head alibi_slopes instead of the ScoreBiasFn.
// Exit code 0 when every call returned; the values are judged by the caller.

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <vector>

#include "onednn_flash/attention.hpp"
#include "onednn_flash/backend.hpp"
#include "onednn_flash/batched_attention.hpp"

namespace of = onednn_flash;

namespace {

template <typename T>
bool read_n(std::FILE* f, T* dst, std::size_t n) {
    return std::fread(dst, sizeof(T), n, f) == n;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s case.bin out.bin\n", argv[0]);
        return 2;
    }
    std::FILE* f = std::fopen(argv[1], "rb");
    if (f == nullptr) {
        std::perror(argv[1]);
        return 2;
    }
    int64_t hdr[12];
    if (!read_n(f, hdr, 12)) return 2;
    const std::size_t M = hdr[0], N = hdr[1], D = hdr[2], Dv = hdr[3];
    const bool causal = hdr[4] != 0, has_mask = hdr[5] != 0, has_alibi = hdr[10] != 0;
    const std::size_t ntiles = hdr[11];
    std::vector<int64_t> tiles(2 * ntiles);
    float sc[2];
    if (!read_n(f, tiles.data(), tiles.size()) || !read_n(f, sc, 2) || ntiles == 0) return 2;
    std::vector<float> q(M * D), k(N * D), v(N * Dv);
    if (!read_n(f, q.data(), q.size()) || !read_n(f, k.data(), k.size()) || !read_n(f, v.data(), v.size()))
        return 2;
    of::BlockMask bm;
    if (has_mask) {
        bm.query_block_size = hdr[6];
        bm.key_block_size = hdr[7];
        bm.query_blocks = hdr[8];
        bm.key_blocks = hdr[9];
        bm.allowed.resize(bm.query_blocks * bm.key_blocks);
        if (!read_n(f, bm.allowed.data(), bm.allowed.size())) return 2;
    }
    std::fclose(f);

    const of::AttentionShape shape{M, N, D, Dv};
    of::AttentionOptions opt;
    opt.scale = sc[0];
    opt.causal = causal;
    opt.key_block_size = tiles[1];
    opt.query_block_size = tiles[0];
    if (has_mask) opt.block_mask = &bm;
    const float slope = sc[1];
    if (has_alibi)
        opt.score_bias = [slope](std::size_t qi, std::size_t kj) {
            return slope * static_cast<float>(static_cast<long>(kj) - static_cast<long>(qi));
        };

    std::vector<std::vector<float>> outs;
    try {
        outs.push_back(of::standard_attention(q, k, v, shape, opt));
        outs.push_back(of::flash_attention_tiled(q, k, v, shape, opt));
        outs.push_back(of::flash_attention_q_tile(q, k, v, shape, opt));
        outs.push_back(of::flash_attention_qk_pv_tile(q, k, v, shape, opt));
        of::AttentionWorkspace ws;
        for (std::size_t t = 0; t < ntiles; ++t) {
            of::AttentionOptions o = opt;
            o.query_block_size = tiles[2 * t];
            o.key_block_size = tiles[2 * t + 1];
            std::vector<float> out(M * Dv, 0.0f);
            of::flash_attention_qk_pv_tile_ws(q.data(), k.data(), v.data(), out.data(), shape, o, ws);
            outs.push_back(out);
        }
        std::vector<float> bout(M * Dv, 0.0f);
        of::flash_attention_batched_qk_pv_tile(q.data(), k.data(), v.data(), bout.data(),
                                               of::BatchedAttentionShape{1, 1, M, N, D, Dv}, opt);
        outs.push_back(bout);
        outs.push_back(of::run_attention(of::AttentionBackendKind::StandardReference, q, k, v, shape, opt));
        outs.push_back(of::run_attention(of::AttentionBackendKind::FlashTiledReference, q, k, v, shape, opt));
        // demands the MFMA kernel (throws where none serves the head dims)
        outs.push_back(of::run_attention(of::AttentionBackendKind::FlashMfmaHip, q, k, v, shape, opt));
        if (has_alibi) {
            of::AttentionOptions o = opt;
            o.score_bias = nullptr;
            o.alibi_slopes = {slope};
            outs.push_back(of::flash_attention_tiled(q, k, v, shape, o));
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "api_golden: %s\n", e.what());
        return 1;
    }
    std::FILE* o = std::fopen(argv[2], "wb");
    if (o == nullptr) {
        std::perror(argv[2]);
        return 2;
    }
    for (const auto& x : outs) {
        if (x.size() != M * Dv || std::fwrite(x.data(), 4, x.size(), o) != x.size()) return 1;
    }
    std::fclose(o);
    std::printf("api_golden: %zu outputs of %zu x %zu\n", outs.size(), M, Dv);
    return 0;
}
