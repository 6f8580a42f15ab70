#pragma once

// Public attention API of the reference (include/onednn_flash/attention.hpp:1-87),
// same names, signatures and argument meaning; every function here computes
// on the GPU (gfx950). Additions are appended at the END of AttentionOptions
// so that aggregate initialisation {scale, causal, key_block_size} keeps working.
//
// Errors: std::invalid_argument for bad shapes/arguments (as the reference),
// std::runtime_error for HIP failures and for what the GPU cannot run.

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

#include "onednn_flash/attention_workspace.hpp"
#include "onednn_flash/tile_kernel.hpp"

namespace onednn_flash {

struct AttentionShape {
    std::size_t query_tokens;
    std::size_t key_tokens;
    std::size_t head_dim;
    std::size_t value_dim;
};

struct BlockMask {
    std::size_t query_block_size = 1;
    std::size_t key_block_size = 1;
    std::size_t query_blocks = 0;
    std::size_t key_blocks = 0;
    // Row-major [query_blocks, key_blocks]; non-zero allows the block.
    std::vector<std::uint8_t> allowed;

    bool allows(std::size_t query_index, std::size_t key_index) const;
};

// Additive bias(query_index, key_index). It is host code: the GPU entry points
// evaluate it once per (query, key) into a dense bias tensor before launching.
using ScoreBiasFn = std::function<float(std::size_t query_index, std::size_t key_index)>;

enum class QkTileLayout {
    CopiedTransposed,
    StridedK,
    BrgemmTransformedK,
};

struct AttentionOptions {
    float scale = 1.0f;
    bool causal = false;
    std::size_t key_block_size = 64;    // advisory on the GPU (kernel tiles are fixed)
    std::size_t query_block_size = 1;   // advisory on the GPU
    TileKernelKind qk_tile_kernel = TileKernelKind::Reference;
    TileKernelKind pv_tile_kernel = TileKernelKind::Reference;
    QkTileLayout qk_tile_layout = QkTileLayout::StridedK;
    const BlockMask* block_mask = nullptr;
    ScoreBiasFn score_bias = nullptr;

    // --- additions (no counterpart in the reference) ---
    // Per-head ALiBi: bias alibi_slopes[h] * (key_index - query_index); empty = none.
    // Mutually exclusive with score_bias.
    std::vector<float> alibi_slopes;
    // tanh soft-cap applied after scale + bias: softcap * tanh(s / softcap); <= 0 = off.
    float softcap = 0.0f;
};

std::vector<float> standard_attention(const std::vector<float>& q, const std::vector<float>& k,
                                      const std::vector<float>& v, const AttentionShape& shape,
                                      const AttentionOptions& options);

std::vector<float> flash_attention_tiled(const std::vector<float>& q, const std::vector<float>& k,
                                         const std::vector<float>& v, const AttentionShape& shape,
                                         const AttentionOptions& options);

std::vector<float> flash_attention_q_tile(const std::vector<float>& q, const std::vector<float>& k,
                                          const std::vector<float>& v, const AttentionShape& shape,
                                          const AttentionOptions& options);

std::vector<float> flash_attention_qk_pv_tile(const std::vector<float>& q,
                                              const std::vector<float>& k,
                                              const std::vector<float>& v,
                                              const AttentionShape& shape,
                                              const AttentionOptions& options);

float max_abs_diff(const std::vector<float>& a, const std::vector<float>& b);

// Raw host pointers, one head; repeated calls with the same workspace
// allocate nothing. Rows without any valid key are written as 0.
void flash_attention_qk_pv_tile_ws(const float* q, const float* k, const float* v, float* output,
                                   const AttentionShape& shape, const AttentionOptions& options,
                                   AttentionWorkspace& ws);

}  // namespace onednn_flash
