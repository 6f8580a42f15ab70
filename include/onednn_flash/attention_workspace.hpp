#pragma once

// AttentionWorkspace (reference include/onednn_flash/attention_workspace.hpp:16-47):
// buffers sized once and reused so that repeated calls allocate nothing. Here
// the buffers are device memory that stages the host tensors of the
// raw-pointer entry points; resize() only grows them.

#include <cstddef>
#include <cstdint>
#include <vector>

namespace onednn_flash {

struct AttentionWorkspace {
    AttentionWorkspace() = default;
    // Copies take the host tile buffers; the copy gets its own device staging
    // area on first use (device memory is never shared between workspaces).
    AttentionWorkspace(const AttentionWorkspace& other);
    AttentionWorkspace& operator=(const AttentionWorkspace& other);
    AttentionWorkspace(AttentionWorkspace&& other) noexcept;
    AttentionWorkspace& operator=(AttentionWorkspace&& other) noexcept;
    ~AttentionWorkspace();

    // Host tile buffers of the reference's CPU flash loop, the same public
    // members sized by resize() as there (q_block x head_dim and so on); the
    // GPU kernels do not use them, code that reads or sizes them keeps working.
    std::vector<float> q_tile;      // [q_block, head_dim]
    std::vector<float> k_tile_t;    // [head_dim, k_block]
    std::vector<float> v_tile;      // [k_block, value_dim]
    std::vector<float> score_tile;  // [q_block, k_block]
    std::vector<float> p_tile;      // [q_block, k_block]
    std::vector<float> pv_tile;     // [q_block, value_dim]
    std::vector<float> running_max;  // [q_block]
    std::vector<float> running_sum;  // [q_block]
    std::vector<float> acc;          // [q_block, value_dim]
    std::vector<float> old_scales;   // [q_block]
    std::vector<float> new_maxes;    // [q_block]
    std::vector<float> block_sums;   // [q_block]
    std::vector<std::uint8_t> row_has_valid;  // [q_block]

    // Same signature as the reference: sizes the host tile buffers above for
    // one tile of the given size and grows the device staging area to match.
    void resize(std::size_t q_block_size, std::size_t k_block_size, std::size_t head_dim,
                std::size_t value_dim);

    // Grows the device staging area to at least `bytes`.
    void reserve_device_bytes(std::size_t bytes);

    void* device_buffer = nullptr;  // device staging area
    std::size_t device_bytes = 0;
    int device = -1;
};

}  // namespace onednn_flash
