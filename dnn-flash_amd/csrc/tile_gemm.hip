// Standalone fp32 tile product C = A x B over strided views, the GPU body of
// the reference's tile-GEMM seam (src/onednn_flash/tile_kernel.cpp:49-86):
// one thread per output element, k ascending. The attention kernels do not
// use it (their tiles run on MFMA inside the fused kernel).

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ofh {
namespace {

__global__ __launch_bounds__(256) void tile_gemm_kernel(const float* __restrict__ a,
                                                        const float* __restrict__ b,
                                                        float* __restrict__ c, int m, int n, int k,
                                                        int64_t asm_, int64_t ask, int64_t bsk,
                                                        int64_t bsn, int64_t csm, int64_t csn) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)m * n) return;
    const int i = (int)(idx / n), j = (int)(idx - (int64_t)i * n);
    float sum = 0.0f;
    for (int kk = 0; kk < k; ++kk) sum += a[i * asm_ + kk * ask] * b[kk * bsk + j * bsn];
    c[i * csm + j * csn] = sum;
}

}  // namespace

hipError_t launch_tile_gemm(const float* a, const float* b, float* c, int m, int n, int k,
                            int64_t asm_, int64_t ask, int64_t bsk, int64_t bsn, int64_t csm,
                            int64_t csn, hipStream_t s) {
    const int64_t total = (int64_t)m * n;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(tile_gemm_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a,
                       b, c, m, n, k, asm_, ask, bsk, bsn, csm, csn);
    return hipGetLastError();
}

}  // namespace ofh
