#pragma once

// Backend dispatch of the reference (include/onednn_flash/backend.hpp:1-21).
// Both reference enumerators run on the GPU here: StandardReference is the
// exact two-pass (rowwise) kernel, FlashTiledReference the flash kernel
// (MFMA where the shape allows it). FlashMfmaHip requests the MFMA kernel and
// throws std::runtime_error if the shape is not supported by it.

#include <vector>

#include "onednn_flash/attention.hpp"

namespace onednn_flash {

enum class AttentionBackendKind {
    StandardReference,
    FlashTiledReference,
    FlashMfmaHip,
};

const char* backend_name(AttentionBackendKind kind);

std::vector<float> run_attention(AttentionBackendKind kind, const std::vector<float>& q,
                                 const std::vector<float>& k, const std::vector<float>& v,
                                 const AttentionShape& shape, const AttentionOptions& options);

}  // namespace onednn_flash
