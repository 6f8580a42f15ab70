#pragma once

// Batched entry of the reference (include/onednn_flash/batched_attention.hpp:1-33)
// plus its device-memory counterpart.

#include <cstddef>

#include "onednn_flash/attention.hpp"

namespace onednn_flash {

struct BatchedAttentionShape {
    std::size_t batch;
    std::size_t heads;
    std::size_t query_tokens;
    std::size_t key_tokens;
    std::size_t head_dim;
    std::size_t value_dim;
};

// Flat row-major host tensors Q[B,H,M,D], K[B,H,N,D], V[B,H,N,Dv], O[B,H,M,Dv].
// Computed on the current GPU in fp32 through a per-thread workspace (no
// allocation after the first call of a given size); synchronous.
void flash_attention_batched_qk_pv_tile(const float* q, const float* k, const float* v, float* out,
                                        const BatchedAttentionShape& shape,
                                        const AttentionOptions& options);

// --- addition: device tensors ---
enum class DeviceDType { F32, BF16, F16 };

// Same layout, device pointers, element type `dtype` for q/k/v and `out_dtype`
// (dtype or F32) for out; asynchronous on `stream` (a hipStream_t, nullptr =
// default stream). options.block_mask and a ScoreBiasFn are host objects: they
// are uploaded (evaluated) per call; use the C ABI (onednn_flash_hip.h) with
// device-resident masks and biases to avoid that.
void flash_attention_batched_device(const void* q, const void* k, const void* v, void* out,
                                    const BatchedAttentionShape& shape,
                                    const AttentionOptions& options, DeviceDType dtype,
                                    DeviceDType out_dtype, void* stream);

}  // namespace onednn_flash
