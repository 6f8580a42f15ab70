// C++ API of the reference (include/onednn_flash/{attention,batched_attention,
// backend,tile_kernel,attention_workspace}.hpp), implemented over the C ABI:
// host tensors are staged into a reused device workspace, the HIP kernels
// run, the result is copied back. No attention arithmetic happens on the host.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "onednn_flash/attention.hpp"
#include "onednn_flash/backend.hpp"
#include "onednn_flash/batched_attention.hpp"
#include "onednn_flash/tile_kernel.hpp"
#include "onednn_flash_hip.h"

namespace ofh {
hipError_t launch_tile_gemm(const float* a, const float* b, float* c, int m, int n, int k,
                            int64_t asm_, int64_t ask, int64_t bsk, int64_t bsn, int64_t csm,
                            int64_t csn, hipStream_t s);
}

namespace onednn_flash {
namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void throw_status(int rc) {
    if (rc == OFH_SUCCESS) return;
    const std::string msg = ofh_last_error();
    if (rc == OFH_ERROR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

// validate_inputs of the reference (attention.cpp:18-38), same messages.
void validate_vectors(const std::vector<float>& q, const std::vector<float>& k,
                      const std::vector<float>& v, const AttentionShape& s) {
    if (q.size() != s.query_tokens * s.head_dim) throw std::invalid_argument("Q size does not match shape");
    if (k.size() != s.key_tokens * s.head_dim) throw std::invalid_argument("K size does not match shape");
    if (v.size() != s.key_tokens * s.value_dim) throw std::invalid_argument("V size does not match shape");
    if (s.query_tokens == 0 || s.key_tokens == 0 || s.head_dim == 0 || s.value_dim == 0)
        throw std::invalid_argument("Attention dimensions must be non-zero");
}

// The checks BlockMask::allows repeats per element (attention.cpp:71-79), done once.
void validate_mask(const BlockMask& m) {
    if (m.query_block_size == 0 || m.key_block_size == 0)
        throw std::invalid_argument("BlockMask block sizes must be non-zero");
    if (m.query_blocks == 0 || m.key_blocks == 0)
        throw std::invalid_argument("BlockMask dimensions must be non-zero");
    if (m.allowed.size() != m.query_blocks * m.key_blocks)
        throw std::invalid_argument("BlockMask allowed bitmap size does not match dimensions");
}

size_t round_up(size_t x) { return (x + 255) & ~size_t(255); }

// Dense fp32 bias [M, N] for a host score_bias callback, shared by every head:
// the callback runs once per pair that the causal rule and the block mask let
// through, the pairs the reference evaluates it for (masked_out before the
// bias, attention.cpp:101-107); masked pairs hold 0 and are never used. The
// array is staged to the device, so its size is capped at kMaxHostBiasBytes.
constexpr size_t kMaxHostBiasBytes = size_t(1) << 31;

std::vector<float> expand_score_bias(const AttentionOptions& o, size_t M, size_t N) {
    std::vector<float> dense;
    if (!o.score_bias) return dense;
    if (M > kMaxHostBiasBytes / 4 / N)
        throw std::invalid_argument("score_bias: the dense [" + std::to_string(M) + " x " + std::to_string(N) +
                                    "] fp32 bias exceeds 2 GiB; use alibi_slopes or the C API with a "
                                    "device bias tensor");
    dense.assign(M * N, 0.0f);
    const BlockMask* bm = o.block_mask;  // validated by the caller
    for (size_t i = 0; i < M; ++i) {
        const size_t jend = o.causal ? std::min(N, i + 1) : N;
        const size_t qb = bm ? i / bm->query_block_size : 0;
        if (bm && qb >= bm->query_blocks) continue;  // the whole row is masked
        float* row = dense.data() + i * N;
        for (size_t j = 0; j < jend; ++j) {
            if (bm) {
                const size_t kb = j / bm->key_block_size;
                if (kb >= bm->key_blocks || bm->allowed[qb * bm->key_blocks + kb] == 0) continue;
            }
            row[j] = o.score_bias(i, j);
        }
    }
    return dense;
}

// One fp32 attention call on host tensors [B*H, T, *] through `ws`.
void run_host(const float* q, const float* k, const float* v, float* out, size_t B, size_t H,
              const AttentionShape& s, const AttentionOptions& o, int algorithm,
              AttentionWorkspace& ws) {
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
        throw std::invalid_argument("attention pointers must be non-null");
    const size_t M = s.query_tokens, N = s.key_tokens, D = s.head_dim, Dv = s.value_dim;
    if (B == 0 || H == 0 || M == 0 || N == 0 || D == 0 || Dv == 0)
        throw std::invalid_argument("Attention dimensions must be non-zero");
    if (o.block_mask != nullptr) validate_mask(*o.block_mask);
    if (o.score_bias && !o.alibi_slopes.empty())
        throw std::invalid_argument("score_bias and alibi_slopes are mutually exclusive");
    if (!o.alibi_slopes.empty() && o.alibi_slopes.size() != H)
        throw std::invalid_argument("alibi_slopes must hold one slope per head");

    const std::vector<float> dense = expand_score_bias(o, M, N);

    const size_t nq = B * H * M * D, nk = B * H * N * D, nv = B * H * N * Dv, no = B * H * M * Dv;
    const size_t nmask = o.block_mask ? o.block_mask->allowed.size() : 0;
    const size_t off_k = round_up(nq * 4), off_v = off_k + round_up(nk * 4);
    const size_t off_o = off_v + round_up(nv * 4), off_m = off_o + round_up(no * 4);
    const size_t off_b = off_m + round_up(nmask), off_s = off_b + round_up(dense.size() * 4);

    ofh_attention_params p;
    ofh_attention_params_init(&p);
    p.batch = B;
    p.heads = H;
    p.query_tokens = M;
    p.key_tokens = N;
    p.head_dim = D;
    p.value_dim = Dv;
    p.dtype = OFH_DTYPE_F32;
    p.out_dtype = OFH_DTYPE_F32;
    p.scale = o.scale;
    p.causal = o.causal ? 1 : 0;
    p.algorithm = algorithm;
    if (nmask) {
        p.mask_allowed = o.block_mask->allowed.data();  // host pointer: only the sizes are read here
        p.mask_query_block_size = o.block_mask->query_block_size;
        p.mask_key_block_size = o.block_mask->key_block_size;
        p.mask_query_blocks = o.block_mask->query_blocks;
        p.mask_key_blocks = o.block_mask->key_blocks;
    }
    // the attention workspace (tile lists, key-split partial rows) lives in this
    // thread's buffer too, so that concurrent threads never share one
    size_t ws_bytes = 0;
    throw_status(ofh_attention_workspace_bytes(&p, &ws_bytes));
    const size_t off_w = off_s + round_up(o.alibi_slopes.size() * 4);
    const size_t total = off_w + round_up(ws_bytes);
    ws.reserve_device_bytes(total);
    char* base = static_cast<char*>(ws.device_buffer);

    hip_check(hipMemcpy(base, q, nq * 4, hipMemcpyHostToDevice), "hipMemcpy(q)");
    hip_check(hipMemcpy(base + off_k, k, nk * 4, hipMemcpyHostToDevice), "hipMemcpy(k)");
    hip_check(hipMemcpy(base + off_v, v, nv * 4, hipMemcpyHostToDevice), "hipMemcpy(v)");

    if (nmask) {
        hip_check(hipMemcpy(base + off_m, o.block_mask->allowed.data(), nmask, hipMemcpyHostToDevice),
                  "hipMemcpy(mask)");
        p.mask_allowed = reinterpret_cast<const uint8_t*>(base + off_m);
    }
    if (!dense.empty()) {
        hip_check(hipMemcpy(base + off_b, dense.data(), dense.size() * 4, hipMemcpyHostToDevice),
                  "hipMemcpy(bias)");
        p.bias_kind = OFH_BIAS_DENSE;
        p.bias = reinterpret_cast<const float*>(base + off_b);
    } else if (!o.alibi_slopes.empty()) {
        hip_check(hipMemcpy(base + off_s, o.alibi_slopes.data(), H * 4, hipMemcpyHostToDevice),
                  "hipMemcpy(slopes)");
        p.bias_kind = OFH_BIAS_ALIBI;
        p.alibi_slopes = reinterpret_cast<const float*>(base + off_s);
    }
    p.softcap = o.softcap > 0.0f ? o.softcap : 0.0f;
    throw_status(ofh_attention_fwd(&p, base, base + off_k, base + off_v, base + off_o,
                                   ws_bytes ? base + off_w : nullptr, ws_bytes, nullptr));
    hip_check(hipMemcpy(out, base + off_o, no * 4, hipMemcpyDeviceToHost), "hipMemcpy(out)");
}

AttentionWorkspace& thread_workspace() {
    thread_local AttentionWorkspace ws;
    return ws;
}

std::vector<float> run_vectors(const std::vector<float>& q, const std::vector<float>& k,
                               const std::vector<float>& v, const AttentionShape& s,
                               const AttentionOptions& o, int algorithm) {
    validate_vectors(q, k, v, s);
    std::vector<float> out(s.query_tokens * s.value_dim, 0.0f);
    run_host(q.data(), k.data(), v.data(), out.data(), 1, 1, s, o, algorithm, thread_workspace());
    return out;
}

}  // namespace

// ---------------------------------------------------------------------------
// AttentionWorkspace

namespace {
// the host tile buffers, member by member (copy or move)
template <typename Src>
void assign_host_tiles(AttentionWorkspace& d, Src&& s) {
    d.q_tile = std::forward<Src>(s).q_tile;
    d.k_tile_t = std::forward<Src>(s).k_tile_t;
    d.v_tile = std::forward<Src>(s).v_tile;
    d.score_tile = std::forward<Src>(s).score_tile;
    d.p_tile = std::forward<Src>(s).p_tile;
    d.pv_tile = std::forward<Src>(s).pv_tile;
    d.running_max = std::forward<Src>(s).running_max;
    d.running_sum = std::forward<Src>(s).running_sum;
    d.acc = std::forward<Src>(s).acc;
    d.old_scales = std::forward<Src>(s).old_scales;
    d.new_maxes = std::forward<Src>(s).new_maxes;
    d.block_sums = std::forward<Src>(s).block_sums;
    d.row_has_valid = std::forward<Src>(s).row_has_valid;
}
}  // namespace

AttentionWorkspace::AttentionWorkspace(const AttentionWorkspace& other) { assign_host_tiles(*this, other); }

AttentionWorkspace& AttentionWorkspace::operator=(const AttentionWorkspace& other) {
    if (this != &other) assign_host_tiles(*this, other);  // the device staging area stays this workspace's own
    return *this;
}

AttentionWorkspace::AttentionWorkspace(AttentionWorkspace&& other) noexcept
    : device_buffer(other.device_buffer), device_bytes(other.device_bytes), device(other.device) {
    assign_host_tiles(*this, std::move(other));
    other.device_buffer = nullptr;
    other.device_bytes = 0;
    other.device = -1;
}

AttentionWorkspace& AttentionWorkspace::operator=(AttentionWorkspace&& other) noexcept {
    if (this != &other) {
        if (device_buffer != nullptr) (void)hipFree(device_buffer);
        assign_host_tiles(*this, std::move(other));
        device_buffer = other.device_buffer;
        device_bytes = other.device_bytes;
        device = other.device;
        other.device_buffer = nullptr;
        other.device_bytes = 0;
        other.device = -1;
    }
    return *this;
}

AttentionWorkspace::~AttentionWorkspace() {
    if (device_buffer != nullptr) (void)hipFree(device_buffer);
}

void AttentionWorkspace::resize(std::size_t q_block_size, std::size_t k_block_size,
                                std::size_t head_dim, std::size_t value_dim) {
    q_tile.resize(q_block_size * head_dim);
    k_tile_t.resize(head_dim * k_block_size);
    v_tile.resize(k_block_size * value_dim);
    score_tile.resize(q_block_size * k_block_size);
    p_tile.resize(q_block_size * k_block_size);
    pv_tile.resize(q_block_size * value_dim);
    for (auto* row : {&running_max, &running_sum, &old_scales, &new_maxes, &block_sums}) row->resize(q_block_size);
    acc.resize(q_block_size * value_dim);
    row_has_valid.resize(q_block_size);
    reserve_device_bytes(4 * (q_block_size * head_dim + k_block_size * (head_dim + value_dim) +
                              q_block_size * value_dim));
}

void AttentionWorkspace::reserve_device_bytes(std::size_t bytes) {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (device_buffer != nullptr && device == dev && device_bytes >= bytes) return;
    if (device_buffer != nullptr) {
        hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        hip_check(hipFree(device_buffer), "hipFree");
        device_buffer = nullptr;
        device_bytes = 0;
    }
    hip_check(hipMalloc(&device_buffer, std::max<std::size_t>(bytes, 256)), "hipMalloc");
    device_bytes = std::max<std::size_t>(bytes, 256);
    device = dev;
}

// ---------------------------------------------------------------------------
// attention.hpp

bool BlockMask::allows(std::size_t query_index, std::size_t key_index) const {
    validate_mask(*this);
    const std::size_t qb = query_index / query_block_size;
    const std::size_t kb = key_index / key_block_size;
    if (qb >= query_blocks || kb >= key_blocks) return false;
    return allowed[qb * key_blocks + kb] != 0;
}

std::vector<float> standard_attention(const std::vector<float>& q, const std::vector<float>& k,
                                      const std::vector<float>& v, const AttentionShape& shape,
                                      const AttentionOptions& options) {
    return run_vectors(q, k, v, shape, options, OFH_ALGO_ROWWISE);
}

std::vector<float> flash_attention_tiled(const std::vector<float>& q, const std::vector<float>& k,
                                         const std::vector<float>& v, const AttentionShape& shape,
                                         const AttentionOptions& options) {
    if (options.key_block_size == 0) throw std::invalid_argument("key_block_size must be non-zero");
    return run_vectors(q, k, v, shape, options, OFH_ALGO_AUTO);
}

std::vector<float> flash_attention_q_tile(const std::vector<float>& q, const std::vector<float>& k,
                                          const std::vector<float>& v, const AttentionShape& shape,
                                          const AttentionOptions& options) {
    if (options.key_block_size == 0) throw std::invalid_argument("key_block_size must be non-zero");
    if (options.query_block_size == 0) throw std::invalid_argument("query_block_size must be non-zero");
    return run_vectors(q, k, v, shape, options, OFH_ALGO_AUTO);
}

std::vector<float> flash_attention_qk_pv_tile(const std::vector<float>& q,
                                              const std::vector<float>& k,
                                              const std::vector<float>& v,
                                              const AttentionShape& shape,
                                              const AttentionOptions& options) {
    if (options.key_block_size == 0) throw std::invalid_argument("key_block_size must be non-zero");
    if (options.query_block_size == 0) throw std::invalid_argument("query_block_size must be non-zero");
    return run_vectors(q, k, v, shape, options, OFH_ALGO_AUTO);
}

float max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
    if (a.size() != b.size()) throw std::invalid_argument("Cannot compare vectors with different sizes");
    float diff = 0.0f;
    for (std::size_t i = 0; i < a.size(); ++i) diff = std::max(diff, std::fabs(a[i] - b[i]));
    return diff;
}

void flash_attention_qk_pv_tile_ws(const float* q, const float* k, const float* v, float* output,
                                   const AttentionShape& shape, const AttentionOptions& options,
                                   AttentionWorkspace& ws) {
    if (q == nullptr || k == nullptr || v == nullptr || output == nullptr)
        throw std::invalid_argument("attention pointers must be non-null");
    if (shape.query_tokens == 0 || shape.key_tokens == 0 || shape.head_dim == 0 || shape.value_dim == 0)
        throw std::invalid_argument("Attention dimensions must be non-zero");
    if (options.key_block_size == 0) throw std::invalid_argument("key_block_size must be non-zero");
    if (options.query_block_size == 0) throw std::invalid_argument("query_block_size must be non-zero");
    run_host(q, k, v, output, 1, 1, shape, options, OFH_ALGO_AUTO, ws);
}

// ---------------------------------------------------------------------------
// batched_attention.hpp

void flash_attention_batched_qk_pv_tile(const float* q, const float* k, const float* v, float* out,
                                        const BatchedAttentionShape& shape,
                                        const AttentionOptions& options) {
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
        throw std::invalid_argument("batched attention input/output pointers must be non-null");
    if (shape.batch == 0 || shape.heads == 0 || shape.query_tokens == 0 || shape.key_tokens == 0 ||
        shape.head_dim == 0 || shape.value_dim == 0)
        throw std::invalid_argument("batched attention dimensions must be non-zero");
    const AttentionShape inner{shape.query_tokens, shape.key_tokens, shape.head_dim, shape.value_dim};
    run_host(q, k, v, out, shape.batch, shape.heads, inner, options, OFH_ALGO_AUTO, thread_workspace());
}

void flash_attention_batched_device(const void* q, const void* k, const void* v, void* out,
                                    const BatchedAttentionShape& shape,
                                    const AttentionOptions& options, DeviceDType dtype,
                                    DeviceDType out_dtype, void* stream) {
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
        throw std::invalid_argument("batched attention input/output pointers must be non-null");
    if (shape.batch == 0 || shape.heads == 0 || shape.query_tokens == 0 || shape.key_tokens == 0 ||
        shape.head_dim == 0 || shape.value_dim == 0)
        throw std::invalid_argument("batched attention dimensions must be non-zero");
    const AttentionOptions& o = options;
    if (o.block_mask != nullptr) validate_mask(*o.block_mask);
    if (o.score_bias && !o.alibi_slopes.empty())
        throw std::invalid_argument("score_bias and alibi_slopes are mutually exclusive");
    if (!o.alibi_slopes.empty() && o.alibi_slopes.size() != shape.heads)
        throw std::invalid_argument("alibi_slopes must hold one slope per head");
    const size_t M = shape.query_tokens, N = shape.key_tokens;
    const std::vector<float> dense = expand_score_bias(o, M, N);
    const size_t nmask = o.block_mask ? o.block_mask->allowed.size() : 0;
    const size_t off_b = round_up(nmask), off_s = off_b + round_up(dense.size() * 4);
    const size_t total = off_s + round_up(o.alibi_slopes.size() * 4);
    thread_local AttentionWorkspace aux;
    aux.reserve_device_bytes(total);
    char* base = static_cast<char*>(aux.device_buffer);
    hipStream_t s = static_cast<hipStream_t>(stream);

    auto to_ofh = [](DeviceDType d) {
        return d == DeviceDType::BF16 ? OFH_DTYPE_BF16 : d == DeviceDType::F16 ? OFH_DTYPE_F16 : OFH_DTYPE_F32;
    };
    ofh_attention_params p;
    ofh_attention_params_init(&p);
    p.batch = shape.batch;
    p.heads = shape.heads;
    p.query_tokens = M;
    p.key_tokens = N;
    p.head_dim = shape.head_dim;
    p.value_dim = shape.value_dim;
    p.dtype = to_ofh(dtype);
    p.out_dtype = to_ofh(out_dtype);
    p.scale = o.scale;
    p.causal = o.causal ? 1 : 0;
    // The staging buffer is reused by the next call on this thread: order the
    // uploads on the caller's stream and wait for them before returning.
    if (nmask) {
        hip_check(hipMemcpyAsync(base, o.block_mask->allowed.data(), nmask, hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync(mask)");
        p.mask_allowed = reinterpret_cast<const uint8_t*>(base);
        p.mask_query_block_size = o.block_mask->query_block_size;
        p.mask_key_block_size = o.block_mask->key_block_size;
        p.mask_query_blocks = o.block_mask->query_blocks;
        p.mask_key_blocks = o.block_mask->key_blocks;
    }
    if (!dense.empty()) {
        hip_check(hipMemcpyAsync(base + off_b, dense.data(), dense.size() * 4, hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync(bias)");
        p.bias_kind = OFH_BIAS_DENSE;
        p.bias = reinterpret_cast<const float*>(base + off_b);
    } else if (!o.alibi_slopes.empty()) {
        hip_check(hipMemcpyAsync(base + off_s, o.alibi_slopes.data(), o.alibi_slopes.size() * 4,
                                 hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync(slopes)");
        p.bias_kind = OFH_BIAS_ALIBI;
        p.alibi_slopes = reinterpret_cast<const float*>(base + off_s);
    }
    p.softcap = o.softcap > 0.0f ? o.softcap : 0.0f;
    throw_status(ofh_attention_fwd(&p, q, k, v, out, nullptr, 0, stream));
    if (nmask || !dense.empty() || !o.alibi_slopes.empty())
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

// ---------------------------------------------------------------------------
// backend.hpp

const char* backend_name(AttentionBackendKind kind) {
    switch (kind) {
        case AttentionBackendKind::StandardReference: return "standard_reference";
        case AttentionBackendKind::FlashTiledReference: return "flash_tiled_reference";
        case AttentionBackendKind::FlashMfmaHip: return "flash_mfma_hip";
    }
    return "unknown";
}

std::vector<float> run_attention(AttentionBackendKind kind, const std::vector<float>& q,
                                 const std::vector<float>& k, const std::vector<float>& v,
                                 const AttentionShape& shape, const AttentionOptions& options) {
    switch (kind) {
        case AttentionBackendKind::StandardReference:
            return standard_attention(q, k, v, shape, options);
        case AttentionBackendKind::FlashTiledReference:
            return flash_attention_tiled(q, k, v, shape, options);
        case AttentionBackendKind::FlashMfmaHip:
            validate_vectors(q, k, v, shape);
            {
                std::vector<float> out(shape.query_tokens * shape.value_dim, 0.0f);
                run_host(q.data(), k.data(), v.data(), out.data(), 1, 1, shape, options,
                         OFH_ALGO_FLASH_MFMA, thread_workspace());
                return out;
            }
    }
    throw std::invalid_argument("Unknown attention backend kind");
}

// ---------------------------------------------------------------------------
// tile_kernel.hpp: one fp32 tile product on the GPU.

const char* tile_kernel_name(TileKernelKind kind) {
    switch (kind) {
        case TileKernelKind::Reference: return "reference";
        case TileKernelKind::OneDnn: return "onednn";
        case TileKernelKind::OneDnnBrgemm: return "onednn_brgemm";
        case TileKernelKind::HipMfma: return "hip_mfma";
    }
    return "unknown";
}

void matmul_tile_strided_inplace(TileKernelKind kind, const float* a, const float* b, float* c,
                                 const StridedMatmulShape& s) {
    if (kind != TileKernelKind::Reference && kind != TileKernelKind::OneDnn &&
        kind != TileKernelKind::OneDnnBrgemm && kind != TileKernelKind::HipMfma)
        throw std::invalid_argument("Unknown tile kernel kind");
    if (s.m == 0 || s.n == 0 || s.k == 0) throw std::invalid_argument("matmul dimensions must be non-zero");
    if (a == nullptr || b == nullptr || c == nullptr) throw std::invalid_argument("matmul pointers must be non-null");
    const size_t na = (s.m - 1) * s.a_stride_m + (s.k - 1) * s.a_stride_k + 1;
    const size_t nb = (s.k - 1) * s.b_stride_k + (s.n - 1) * s.b_stride_n + 1;
    const size_t nc = (s.m - 1) * s.c_stride_m + (s.n - 1) * s.c_stride_n + 1;
    AttentionWorkspace& ws = thread_workspace();
    const size_t off_b = round_up(na * 4), off_c = off_b + round_up(nb * 4);
    ws.reserve_device_bytes(off_c + round_up(nc * 4));
    char* base = static_cast<char*>(ws.device_buffer);
    hip_check(hipMemcpy(base, a, na * 4, hipMemcpyHostToDevice), "hipMemcpy(a)");
    hip_check(hipMemcpy(base + off_b, b, nb * 4, hipMemcpyHostToDevice), "hipMemcpy(b)");
    // C may be a strided view: start from the caller's contents so that
    // elements outside the view are preserved.
    hip_check(hipMemcpy(base + off_c, c, nc * 4, hipMemcpyHostToDevice), "hipMemcpy(c)");
    hip_check(ofh::launch_tile_gemm(reinterpret_cast<const float*>(base),
                                    reinterpret_cast<const float*>(base + off_b),
                                    reinterpret_cast<float*>(base + off_c), (int)s.m, (int)s.n,
                                    (int)s.k, (int64_t)s.a_stride_m, (int64_t)s.a_stride_k,
                                    (int64_t)s.b_stride_k, (int64_t)s.b_stride_n,
                                    (int64_t)s.c_stride_m, (int64_t)s.c_stride_n, nullptr),
              "tile GEMM launch");
    hip_check(hipMemcpy(c, base + off_c, nc * 4, hipMemcpyDeviceToHost), "hipMemcpy(c)");
}

void matmul_tile_inplace(TileKernelKind kind, const float* a, const float* b, float* c,
                         const MatmulShape& s) {
    matmul_tile_strided_inplace(kind, a, b, c, StridedMatmulShape{s.m, s.n, s.k, s.k, 1, s.n, 1, s.n, 1});
}

void matmul_tile_reference_inplace(const float* a, const float* b, float* c, const MatmulShape& s) {
    matmul_tile_inplace(TileKernelKind::Reference, a, b, c, s);
}

std::vector<float> matmul_tile_reference(const std::vector<float>& a, const std::vector<float>& b,
                                         const MatmulShape& s) {
    if (s.m == 0 || s.n == 0 || s.k == 0) throw std::invalid_argument("matmul dimensions must be non-zero");
    if (a.size() != s.m * s.k) throw std::invalid_argument("A size does not match matmul shape");
    if (b.size() != s.k * s.n) throw std::invalid_argument("B size does not match matmul shape");
    std::vector<float> c(s.m * s.n, 0.0f);
    matmul_tile_reference_inplace(a.data(), b.data(), c.data(), s);
    return c;
}

std::vector<float> matmul_tile(TileKernelKind kind, const std::vector<float>& a,
                               const std::vector<float>& b, const MatmulShape& s) {
    if (s.m == 0 || s.n == 0 || s.k == 0) throw std::invalid_argument("matmul dimensions must be non-zero");
    if (a.size() != s.m * s.k) throw std::invalid_argument("A size does not match matmul shape");
    if (b.size() != s.k * s.n) throw std::invalid_argument("B size does not match matmul shape");
    std::vector<float> c(s.m * s.n, 0.0f);
    matmul_tile_inplace(kind, a.data(), b.data(), c.data(), s);
    return c;
}

}  // namespace onednn_flash
