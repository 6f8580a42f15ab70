#pragma once

// Tile-GEMM seam of the reference (include/onednn_flash/tile_kernel.hpp:1-74),
// same names and signatures. In this library the QK^T and PV tiles of the
// attention kernels run on MFMA inside the fused kernel; these standalone
// entry points run one fp32 tile product on the GPU for callers of the seam.

#include <cstddef>
#include <vector>

namespace onednn_flash {

struct MatmulShape {
    std::size_t m;
    std::size_t n;
    std::size_t k;
};

struct StridedMatmulShape {
    std::size_t m;
    std::size_t n;
    std::size_t k;
    std::size_t a_stride_m;
    std::size_t a_stride_k;
    std::size_t b_stride_k;
    std::size_t b_stride_n;
    std::size_t c_stride_m;
    std::size_t c_stride_n;
};

// Reference, OneDnn and OneDnnBrgemm keep their meaning as option values
// (they are accepted and all run on the GPU here); HipMfma names this
// library's MFMA tiles explicitly.
enum class TileKernelKind {
    Reference,
    OneDnn,
    OneDnnBrgemm,
    HipMfma,
};

const char* tile_kernel_name(TileKernelKind kind);

// Row-major C[m,n] = A[m,k] x B[k,n] on host buffers (GPU computes, fp32).
void matmul_tile_inplace(TileKernelKind kind, const float* a, const float* b, float* c,
                         const MatmulShape& shape);

// Strided views of A, B and C (e.g. K^T read from row-major K without a copy).
void matmul_tile_strided_inplace(TileKernelKind kind, const float* a, const float* b, float* c,
                                 const StridedMatmulShape& shape);

std::vector<float> matmul_tile(TileKernelKind kind, const std::vector<float>& a,
                               const std::vector<float>& b, const MatmulShape& shape);

std::vector<float> matmul_tile_reference(const std::vector<float>& a, const std::vector<float>& b,
                                         const MatmulShape& shape);

void matmul_tile_reference_inplace(const float* a, const float* b, float* c,
                                   const MatmulShape& shape);

}  // namespace onednn_flash
