// Exact two-pass softmax attention, one query row per wavefront, any head_dim
// and value_dim: the GPU counterpart of standard_attention
// (src/onednn_flash/attention.cpp:88-137 of the reference). Pass 1 finds the
// row max over valid keys; pass 2 recomputes the scores, forms
// p = exp(s - max), the denominator and sum_k p_k * V[k]. Scores are never
// stored: they are recomputed rather than materialised. Used for
// OFH_ALGO_ROWWISE and for shapes the MFMA flash kernels do not take
// (D != Dv, D not in {64, 128}, unaligned rows).
//
// Lanes own keys during the score passes (each lane one key, the query row
// broadcast from LDS) and own output columns during accumulation (each of
// the 64 probabilities of a key chunk is broadcast with a scalar read-lane),
// so V reads are coalesced along the row.

#include "ofh_kernels.h"

namespace ofh {
namespace {

constexpr int kRowsPerBlock = 4;   // one wavefront per query row
constexpr int kMaxD = 1024;        // query row staged in LDS (fp32)
constexpr int kAccPerLane = 8;     // output columns per lane per pass-2 sweep (512 per sweep)

template <typename T>
__device__ __forceinline__ float to_f32(T x) {
    return (float)x;
}

__device__ __forceinline__ bool row_masked(const FwdArgs& a, int qi, int kj) {
    if (a.causal && kj > qi) return true;
    if (a.mask != nullptr) {
        const int qb = qi / a.mask_qbs, kb = kj / a.mask_kbs;
        if (qb >= a.mask_qb || kb >= a.mask_kb) return true;
        return a.mask[(int64_t)qb * a.mask_kb + kb] == 0;
    }
    return false;
}

template <typename T>
__device__ __forceinline__ float row_score(const FwdArgs& a, const float* qs, const T* krow,
                                           int qi, int kj, float slope, const float* bias_row) {
    float dot = 0.0f;
    for (int d = 0; d < a.D; ++d) dot += qs[d] * to_f32(krow[d]);
    float s = dot * a.scale;
    if (a.bias_kind == BIAS_ALIBI) s += slope * (float)(kj - qi);
    else if (a.bias_kind == BIAS_DENSE) s += bias_row[kj];
    if (a.softcap > 0.0f) s = a.softcap * tanhf(s / a.softcap);
    return s;
}

template <typename T>
__global__ __launch_bounds__(64 * kRowsPerBlock) void rowwise_fwd_kernel(FwdArgs a) {
    __shared__ float qs_all[kRowsPerBlock][kMaxD];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t row_id = (int64_t)blockIdx.x * kRowsPerBlock + w;
    const bool valid = row_id < (int64_t)a.B * a.H * a.M;  // wave-uniform
    const int qi = valid ? (int)(row_id % a.M) : 0;
    const int bh = valid ? (int)(row_id / a.M) : 0;
    const int b = bh / a.H, h = bh - b * a.H;
    const T* Qp = (const T*)a.q + b * a.q_sb + h * a.q_sh + (int64_t)qi * a.q_sm;
    const T* Kp = (const T*)a.k + b * a.k_sb + h * a.k_sh;
    const T* Vp = (const T*)a.v + b * a.v_sb + h * a.v_sh;
    float* qs = qs_all[w];
    if (valid) {
        for (int d = lane; d < a.D; d += 64) qs[d] = to_f32(Qp[d]);
    }
    __syncthreads();
    if (!valid) return;

    const float slope = a.bias_kind == BIAS_ALIBI ? a.alibi[h] : 0.0f;
    const float* bias_row = a.bias_kind == BIAS_DENSE
                                ? a.bias + b * a.bias_sb + h * a.bias_sh + (int64_t)qi * a.bias_sm
                                : nullptr;

    // Pass 1: row max over valid keys.
    float mx = -__builtin_huge_valf();
    bool any = false;
    for (int k0 = 0; k0 < a.N; k0 += 64) {
        const int kj = k0 + lane;
        if (kj < a.N && !row_masked(a, qi, kj)) {
            const float s = row_score(a, qs, Kp + (int64_t)kj * a.k_sn, qi, kj, slope, bias_row);
            mx = fmaxf(mx, s);
            any = true;
        }
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    any = __any(any);

    // Pass 2, in sweeps of 64*kAccPerLane output columns. The probability of
    // key k0+jj is broadcast from lane jj with a scalar read-lane.
    for (int dv0 = 0; dv0 < a.Dv; dv0 += 64 * kAccPerLane) {
        float acc[kAccPerLane];
        for (int t = 0; t < kAccPerLane; ++t) acc[t] = 0.0f;
        float denom = 0.0f;
        if (any) {
            for (int k0 = 0; k0 < a.N; k0 += 64) {
                const int kj = k0 + lane;
                float p = 0.0f;
                if (kj < a.N && !row_masked(a, qi, kj)) {
                    const float s = row_score(a, qs, Kp + (int64_t)kj * a.k_sn, qi, kj, slope, bias_row);
                    p = expf(s - mx);
                }
                denom += p;
                const int kn = min(64, a.N - k0);
                for (int jj = 0; jj < kn; ++jj) {
                    const float pj = __builtin_bit_cast(
                        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), jj));
                    if (pj == 0.0f) continue;  // uniform
                    const T* vrow = Vp + (int64_t)(k0 + jj) * a.v_sn;
                    for (int t = 0; t < kAccPerLane; ++t) {
                        const int d = dv0 + lane + 64 * t;
                        if (d < a.Dv) acc[t] += pj * to_f32(vrow[d]);
                    }
                }
            }
        }
        for (int off = 32; off > 0; off >>= 1) denom += __shfl_xor(denom, off);
        const float inv = (any && denom > 0.0f) ? 1.0f / denom : 0.0f;
        for (int t = 0; t < kAccPerLane; ++t) {
            const int d = dv0 + lane + 64 * t;
            if (d >= a.Dv) continue;
            const float val = acc[t] * inv;
            const int64_t off = b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_sm + d;
            if (a.out_f32) ((float*)a.o)[off] = val;
            else ((T*)a.o)[off] = (T)val;
        }
    }
}

}  // namespace

hipError_t launch_rowwise(const FwdArgs& a, int dtype, hipStream_t s) {
    if (a.D > kMaxD) return hipErrorInvalidValue;
    const int64_t rows = (int64_t)a.B * a.H * a.M;
    const int64_t grid = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    if (grid <= 0) return hipSuccess;
    const dim3 g((unsigned)grid), blk(64 * kRowsPerBlock);
    switch (dtype) {
        case DT_F32: hipLaunchKernelGGL(rowwise_fwd_kernel<float>, g, blk, 0, s, a); break;
        case DT_BF16: hipLaunchKernelGGL(rowwise_fwd_kernel<__bf16>, g, blk, 0, s, a); break;
        case DT_F16: hipLaunchKernelGGL(rowwise_fwd_kernel<_Float16>, g, blk, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Block-mask tile lists: for each query tile of the flash kernel, the ordered
// list of key tiles that hold at least one allowed (query, key) pair. Each
// entry also says, per 32-row slice of the query tile (one wavefront of the
// attention kernel), whether the slice has an allowed pair at all (else that
// wavefront skips the tile) and whether the mask allows all of its pairs
// (else it masks element-wise). Built before the attention launch, so skipped
// tiles issue no loads at all. One workgroup of four wavefronts per query
// tile, 256 key tiles per round; the list is compacted in key order with a
// per-wavefront ballot and a prefix over the wavefronts' counts.
namespace {

constexpr int kListWaves = 4;

__global__ __launch_bounds__(64 * kListWaves) void tile_list_kernel(TileListArgs a) {
    const int qt = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    __shared__ int wave_counts[kListWaves];
    const int q0 = qt * a.block_m;
    const int slices = a.block_m / 32;
    int count = 0;
    for (int base = 0; base < a.num_k_tiles; base += 64 * kListWaves) {
        const int kt = base + tid;
        unsigned any_bits = 0, full_bits = 0;
        if (kt < a.num_k_tiles) {
            const int k0 = kt * a.block_n;
            const int k1 = min(a.N, k0 + a.block_n);
            for (int w = 0; w < slices; ++w) {
                const int s0 = q0 + 32 * w, s1 = min(a.M, s0 + 32);
                if (s0 >= s1) continue;
                bool any, all;
                classify_mask_slice(a.mask, a.mask_qbs, a.mask_kbs, a.mask_qb, a.mask_kb, a.causal, s0, s1,
                                    k0, k1, any, all);
                any_bits |= (any ? 1u : 0u) << w;
                full_bits |= (all ? 1u : 0u) << w;
            }
        }
        const unsigned long long bal = __ballot(any_bits != 0);
        if (lane == 0) wave_counts[wave] = __popcll(bal);
        __syncthreads();
        int before = count, total = count;
        for (int w = 0; w < kListWaves; ++w) {
            before += w < wave ? wave_counts[w] : 0;
            total += wave_counts[w];
        }
        if (any_bits != 0)
            a.entries[(int64_t)qt * a.num_k_tiles + before + __popcll(bal & ((1ull << lane) - 1ull))] =
                list_entry(kt, any_bits, full_bits);
        __syncthreads();  // wave_counts is rewritten in the next round
        count = total;
    }
    if (tid == 0) a.counts[qt] = count;
}

}  // namespace

hipError_t launch_tile_lists(const TileListArgs& a, hipStream_t s) {
    if (a.num_q_tiles <= 0) return hipSuccess;
    hipLaunchKernelGGL(tile_list_kernel, dim3(a.num_q_tiles), dim3(64 * kListWaves), 0, s, a);
    return hipGetLastError();
}

}  // namespace ofh
