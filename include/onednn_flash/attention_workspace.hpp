#pragma once

// AttentionWorkspace (reference include/onednn_flash/attention_workspace.hpp:16-47):
// buffers sized once and reused so that repeated calls allocate nothing. Here
// the buffers are device memory that stages the host tensors of the
// raw-pointer entry points; resize() only grows them.

#include <cstddef>
#include <cstdint>

namespace onednn_flash {

struct AttentionWorkspace {
    AttentionWorkspace() = default;
    AttentionWorkspace(const AttentionWorkspace&) = delete;
    AttentionWorkspace& operator=(const AttentionWorkspace&) = delete;
    AttentionWorkspace(AttentionWorkspace&& other) noexcept;
    AttentionWorkspace& operator=(AttentionWorkspace&& other) noexcept;
    ~AttentionWorkspace();

    // Same signature as the reference. Makes room for one tile of the given
    // size; kept for source compatibility (the GPU path sizes itself).
    void resize(std::size_t q_block_size, std::size_t k_block_size, std::size_t head_dim,
                std::size_t value_dim);

    // Grows the device staging area to at least `bytes`.
    void reserve_device_bytes(std::size_t bytes);

    void* device_buffer = nullptr;  // device staging area
    std::size_t device_bytes = 0;
    int device = -1;
};

}  // namespace onednn_flash
