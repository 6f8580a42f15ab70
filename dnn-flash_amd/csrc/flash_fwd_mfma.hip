// Flash-style attention forward on gfx950 matrix cores.
//
// Replaces the CPU loop nest of flash_attention_qk_pv_tile_ws
// (src/onednn_flash/attention.cpp:486-695 of the reference) and its batched
// driver (src/onednn_flash/batched_attention.cpp:9-49): one workgroup owns a
// 128-row query block of one (batch, head); K/V stream through LDS in tiles
// of 64 keys (32 for fp32); QK^T and PV run on MFMA; the online-softmax
// recurrence (running max, rescaled running sum, rescaled accumulator,
// attention.cpp:628-673) lives in registers; the N x N score matrix is never
// formed.
//
// Layout trick. Scores are computed transposed, S^T = K * Q^T, with K as the
// MFMA A operand and Q as the B operand. In the 32x32 accumulator layout lane
// l then holds 16 scores of ONE query (column l%32), so the row max, the row
// sum and the accumulator rescale are per-lane scalars, and the only
// cross-lane step per tile is one exchange between the two 32-lane halves
// for the max. The output is accumulated transposed as well, O^T = V^T * P^T:
// the B operand P^T is exactly the lane's own probabilities (no shuffle), and
// V^T is read from a transposed copy of the V tile kept in LDS.
//
// The accumulator row r = 8i + 4g + j (lane half g = l/32, register 4i+j)
// is fed from A-operand row r, and A rows are permuted by kappa(r) =
// 16(i>>1) + 8g + 4(i&1) + j. With that permutation, registers [8c, 8c+8) of
// lane half g hold 8 consecutive positions 16c + 8g + t, which is what the
// next MFMA wants in a lane (k-slots 8g..8g+7 of a 16-wide chunk), and what
// a 16-byte store of the output wants.

#include "ofh_kernels.h"

namespace ofh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ int kappa(int r) {
    return ((r >> 4) << 4) | (((r >> 2) & 1) << 3) | (((r >> 3) & 1) << 2) | (r & 3);
}

// Position (within a 32-row block) held by accumulator register e of lane half g.
__device__ __forceinline__ int acc_pos(int e, int g) { return ((e >> 3) << 4) + (g << 3) + (e & 7); }

template <typename T>
struct Mfma16;
template <>
struct Mfma16<__bf16> {
    typedef bf16x8 v8;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma16<_Float16> {
    typedef f16x8 v8;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

// Workgroup id -> (flat head, query tile). Workgroups are handed to the 8 XCDs
// round-robin, so when B*H is a multiple of 8 the heads are partitioned over
// XCDs (all query tiles of a head run on one XCD and share its L2 for K/V),
// and each XCD walks its heads one after another. Causal query tiles run
// heaviest (longest key range) first.
__device__ __forceinline__ void map_work(int id, int BH, int nqt, int causal, int& bh, int& qt) {
    int t;
    if ((BH & 7) == 0) {
        const int xcd = id & 7, j = id >> 3;
        const int hl = j / nqt;
        t = j - hl * nqt;
        bh = hl * 8 + xcd;
    } else {
        bh = id % BH;
        t = id / BH;
    }
    qt = causal ? nqt - 1 - t : t;
}

// masked_out (attention.cpp:54-62) plus the key-range bound of a ragged last tile.
__device__ __forceinline__ bool elem_masked(const FwdArgs& a, int qi, int kj) {
    if (kj >= a.N) return true;
    if (a.causal && kj > qi) return true;
    if (a.mask != nullptr) {
        const int qb = qi / a.mask_qbs, kb = kj / a.mask_kbs;
        if (qb >= a.mask_qb || kb >= a.mask_kb) return true;
        return a.mask[(int64_t)qb * a.mask_kb + kb] == 0;
    }
    return false;
}

// tanh(y) = 1 - 2 / (exp(2y) + 1): saturates to +-1 for large |y| (exp2 -> inf / 0).
__device__ __forceinline__ float tanh_exp(float y) {
    const float e = __builtin_amdgcn_exp2f(y * (2.0f * kLog2e));
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}

// Scale, additive bias, soft-cap; result in log2 units for exp2.
__device__ __forceinline__ float general_score(const FwdArgs& a, float s, int qi, int kj,
                                               float slope, const float* bias_row) {
    float t = s * a.scale;
    if (a.bias_kind == BIAS_ALIBI) {
        t += slope * (float)(kj - qi);
    } else if (a.bias_kind == BIAS_DENSE) {
        t += bias_row[kj];
    }
    if (a.softcap > 0.0f) t = a.softcap * tanh_exp(t * a.inv_softcap);
    return t * kLog2e;
}

// One K/V tile of online softmax on the 32x32 accumulator blocks `s` (NB
// blocks of 32 keys), in place: raw dot products in, probabilities out.
// Returns alpha, the factor the accumulator must be rescaled by.
template <int NB, bool GENERAL>
__device__ __forceinline__ float online_softmax_tile(const FwdArgs& a, f32x16 (&s)[NB], bool need_mask,
                                                     int my_q, int k0, int g, float slope,
                                                     const float* bias_row, float& m_run,
                                                     float& l_run) {
    float mx = kNegInf;
    if (!GENERAL && !need_mask) {
#pragma unroll
        for (int sb = 0; sb < NB; ++sb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                s[sb][e] *= a.scale_log2;
                mx = fmaxf(mx, s[sb][e]);
            }
        }
    } else {
        const bool row_out = GENERAL && my_q >= a.M;
#pragma unroll
        for (int sb = 0; sb < NB; ++sb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int kj = k0 + 32 * sb + acc_pos(e, g);
                const bool msk = row_out || (need_mask && elem_masked(a, my_q, kj));
                float x = kNegInf;
                if (!msk) {
                    x = GENERAL ? general_score(a, s[sb][e], my_q, kj, slope, bias_row)
                                : s[sb][e] * a.scale_log2;
                }
                s[sb][e] = x;
                mx = fmaxf(mx, x);
            }
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == kNegInf) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float lsum = 0.0f;
#pragma unroll
    for (int sb = 0; sb < NB; ++sb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float p = __builtin_amdgcn_exp2f(s[sb][e] - m_use);
            s[sb][e] = p;
            lsum += p;
        }
    }
    l_run = l_run * alpha + lsum;
    return alpha;
}

// ---------------------------------------------------------------------------
// bf16 / fp16 inputs, fp32 accumulate: v_mfma_f32_32x32x16_{bf16,f16}.

template <typename T, int D, bool GENERAL>
__global__ __launch_bounds__(kThreads) void flash_fwd_mfma16_kernel(FwdArgs a) {
    using M16 = Mfma16<T>;
    using v8 = typename M16::v8;
    constexpr int BN = kBlockN;
    constexpr int KSTR = D + 8;   // K tile row stride in LDS (elements): 16-byte pad
    constexpr int VSTR = BN + 8;  // V^T tile row stride in LDS (elements)
    constexpr int KTILE = BN * KSTR;
    constexpr int VTILE = D * VSTR;
    constexpr int STAGE = KTILE + VTILE;
    constexpr int CHUNKS = BN * D / 8;        // 16-byte chunks per K (or V) tile
    constexpr int CPT = CHUNKS / kThreads;    // chunks per thread
    constexpr int NDC = D / 8;                // 16-byte chunks per row
    constexpr int NKG = BN / CPT;             // key groups of the V transposition
    static_assert(CHUNKS % kThreads == 0, "tile must split evenly over the workgroup");
    static_assert(CPT == 2 || CPT == 4, "V transposition handles 2 or 4 keys per thread");
    static_assert(NKG * NDC == kThreads, "V transposition covers the tile");

    __shared__ __attribute__((aligned(16))) unsigned short lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, r = lane & 31;

    int bh, qt;
    map_work(blockIdx.x, a.B * a.H, a.num_q_tiles, a.causal, bh, qt);
    const int b = bh / a.H, h = bh - b * a.H;
    const T* __restrict__ Qp = (const T*)a.q + b * a.q_sb + h * a.q_sh;
    const T* __restrict__ Kp = (const T*)a.k + b * a.k_sb + h * a.k_sh;
    const T* __restrict__ Vp = (const T*)a.v + b * a.v_sb + h * a.v_sh;
    const int q0 = qt * kBlockM;
    const int qw0 = q0 + wave * kQueriesPerWave;
    const int my_q = qw0 + r;

    // Q^T fragments (B operand of S^T = K Q^T): lane holds Q[my_q][16c + 8g .. +7].
    v8 qf[D / 16];
    {
        const T* qrow = Qp + (int64_t)my_q * a.q_sm + 8 * g;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            u32x4 u = {0u, 0u, 0u, 0u};
            if (my_q < a.M) u = *(const u32x4*)(qrow + 16 * c);
            qf[c] = __builtin_bit_cast(v8, u);
        }
    }

    int ntiles;
    const int* list = nullptr;
    if (a.tile_counts != nullptr) {
        ntiles = a.tile_counts[qt];
        list = a.tile_entries + (int64_t)qt * a.num_k_tiles;
    } else {
        const int kend = a.causal ? min(a.N, q0 + kBlockM) : a.N;
        ntiles = (kend + BN - 1) / BN;
    }

    u32x4 kreg[CPT], vreg[CPT];
    const int vkg = tid % NKG, vdc = tid / NKG;
    auto load_tile = [&](int kt) {
        const int k0 = kt * BN;
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int ci = tid + kThreads * u;
            const int row = ci / NDC, cc = ci % NDC;
            const int kj = k0 + row;
            kreg[u] = u32x4{0u, 0u, 0u, 0u};
            if (kj < a.N) kreg[u] = *(const u32x4*)(Kp + (int64_t)kj * a.k_sn + 8 * cc);
        }
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int kj = k0 + vkg * CPT + u;
            vreg[u] = u32x4{0u, 0u, 0u, 0u};
            if (kj < a.N) vreg[u] = *(const u32x4*)(Vp + (int64_t)kj * a.v_sn + 8 * vdc);
        }
    };
    auto store_tile = [&](int buf) {
        unsigned short* Ks = lds + buf * STAGE;
        unsigned short* Vs = Ks + KTILE;
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int ci = tid + kThreads * u;
            const int row = ci / NDC, cc = ci % NDC;
            *(u32x4*)(Ks + row * KSTR + 8 * cc) = kreg[u];
        }
        // V^T: element e of this thread's 8-wide d chunk, CPT consecutive keys.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int w = e >> 1;
            unsigned short* dst = Vs + (8 * vdc + e) * VSTR + vkg * CPT;
            if constexpr (CPT == 4) {
                const unsigned x0 = vreg[0][w], x1 = vreg[1][w], x2 = vreg[2][w], x3 = vreg[3][w];
                u32x2 val;
                if (e & 1) {
                    val[0] = (x0 >> 16) | (x1 & 0xffff0000u);
                    val[1] = (x2 >> 16) | (x3 & 0xffff0000u);
                } else {
                    val[0] = (x0 & 0xffffu) | (x1 << 16);
                    val[1] = (x2 & 0xffffu) | (x3 << 16);
                }
                *(u32x2*)dst = val;
            } else {
                const unsigned x0 = vreg[0][w], x1 = vreg[1][w];
                const unsigned val = (e & 1) ? ((x0 >> 16) | (x1 & 0xffff0000u))
                                             : ((x0 & 0xffffu) | (x1 << 16));
                *(unsigned*)dst = val;
            }
        }
    };
    auto tile_at = [&](int it, bool& partial) -> int {
        if (list != nullptr) {
            const int e = list[it];
            partial = (e & 1) != 0;
            return e >> 1;
        }
        partial = false;
        return it;
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int db = 0; db < D / 32; ++db) o[db] = f32x16{};
    float m_run = kNegInf, l_run = 0.0f;
    const float slope = (GENERAL && a.bias_kind == BIAS_ALIBI) ? a.alibi[h] : 0.0f;
    const float* bias_row = nullptr;
    if (GENERAL && a.bias_kind == BIAS_DENSE && my_q < a.M)
        bias_row = a.bias + b * a.bias_sb + h * a.bias_sh + (int64_t)my_q * a.bias_sm;

    if (ntiles > 0) {
        bool p0;
        load_tile(tile_at(0, p0));
        store_tile(0);
    }
    __syncthreads();

    for (int it = 0; it < ntiles; ++it) {
        bool partial;
        const int kt = tile_at(it, partial);
        if (it + 1 < ntiles) {
            bool pn;
            load_tile(tile_at(it + 1, pn));
        }
        const unsigned short* Ks = lds + (it & 1) * STAGE;
        const unsigned short* Vs = Ks + KTILE;
        const int k0 = kt * BN;
        const bool active = !(a.causal && k0 > qw0 + kQueriesPerWave - 1);
        if (active) {
            const bool need_mask = list != nullptr
                                       ? partial
                                       : ((k0 + BN > a.N) || (a.causal && k0 + BN - 1 > qw0));
            f32x16 s[BN / 32];
#pragma unroll
            for (int sb = 0; sb < BN / 32; ++sb) {
                s[sb] = f32x16{};
                const unsigned short* krow = Ks + (32 * sb + kappa(r)) * KSTR + 8 * g;
#pragma unroll
                for (int c = 0; c < D / 16; ++c) {
                    const v8 af = __builtin_bit_cast(v8, *(const u32x4*)(krow + 16 * c));
                    s[sb] = M16::mma(af, qf[c], s[sb]);
                }
            }
            const float alpha = online_softmax_tile<BN / 32, GENERAL>(
                a, s, need_mask, my_q, k0, g, slope, bias_row, m_run, l_run);
#pragma unroll
            for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
            v8 pf[BN / 16];
#pragma unroll
            for (int c = 0; c < BN / 16; ++c) {
#pragma unroll
                for (int t = 0; t < 8; ++t) pf[c][t] = (T)s[c >> 1][8 * (c & 1) + t];
            }
#pragma unroll
            for (int db = 0; db < D / 32; ++db) {
                const unsigned short* vrow = Vs + (32 * db + kappa(r)) * VSTR + 8 * g;
#pragma unroll
                for (int c = 0; c < BN / 16; ++c) {
                    const v8 af = __builtin_bit_cast(v8, *(const u32x4*)(vrow + 16 * c));
                    o[db] = M16::mma(af, pf[c], o[db]);
                }
            }
        }
        if (it + 1 < ntiles) store_tile((it + 1) & 1);
        __syncthreads();
    }

    // Normalise; rows that saw no valid key have l = 0 and are written as 0.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (my_q < a.M) {
        if (a.out_f32) {
            float* orow = (float*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)my_q * a.o_sm + 8 * g;
#pragma unroll
            for (int db = 0; db < D / 32; ++db) {
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    f32x4 lo, hi;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        lo[t] = o[db][8 * cc + t] * inv;
                        hi[t] = o[db][8 * cc + 4 + t] * inv;
                    }
                    *(f32x4*)(orow + 32 * db + 16 * cc) = lo;
                    *(f32x4*)(orow + 32 * db + 16 * cc + 4) = hi;
                }
            }
        } else {
            T* orow = (T*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)my_q * a.o_sm + 8 * g;
#pragma unroll
            for (int db = 0; db < D / 32; ++db) {
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    v8 val;
#pragma unroll
                    for (int t = 0; t < 8; ++t) val[t] = (T)(o[db][8 * cc + t] * inv);
                    *(u32x4*)(orow + 32 * db + 16 * cc) = __builtin_bit_cast(u32x4, val);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fp32 inputs: v_mfma_f32_32x32x2_f32. Each MFMA consumes one element per lane
// and operand, so K and V stay row-major in LDS (no transposition): the
// reduction index d of S^T is split as d = g*D/2 + s over the two lane halves,
// and each PV step takes the two keys that the lane halves hold in register u.

constexpr int kBlockNF32 = 32;

template <int D, bool GENERAL>
__global__ __launch_bounds__(kThreads) void flash_fwd_mfma32_kernel(FwdArgs a) {
    constexpr int BN = kBlockNF32;
    constexpr int KSTR = D + 4;  // floats; conflict-free 16-byte reads of rows kappa(r)
    constexpr int VSTR = D + 4;  // floats; lane halves read rows 8 apart -> opposite bank halves
    constexpr int KTILE = BN * KSTR;
    constexpr int STAGE = 2 * KTILE;
    constexpr int CHUNKS = BN * D / 4;
    constexpr int CPT = CHUNKS / kThreads;
    constexpr int NDC = D / 4;
    static_assert(CHUNKS % kThreads == 0, "tile must split evenly over the workgroup");

    __shared__ __attribute__((aligned(16))) float lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, r = lane & 31;

    int bh, qt;
    map_work(blockIdx.x, a.B * a.H, a.num_q_tiles, a.causal, bh, qt);
    const int b = bh / a.H, h = bh - b * a.H;
    const float* __restrict__ Qp = (const float*)a.q + b * a.q_sb + h * a.q_sh;
    const float* __restrict__ Kp = (const float*)a.k + b * a.k_sb + h * a.k_sh;
    const float* __restrict__ Vp = (const float*)a.v + b * a.v_sb + h * a.v_sh;
    const int q0 = qt * kBlockM;
    const int qw0 = q0 + wave * kQueriesPerWave;
    const int my_q = qw0 + r;

    float qf[D / 2];
    {
        const float* qrow = Qp + (int64_t)my_q * a.q_sm + g * (D / 2);
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
            f32x4 u = {0.f, 0.f, 0.f, 0.f};
            if (my_q < a.M) u = *(const f32x4*)(qrow + 4 * c);
#pragma unroll
            for (int t = 0; t < 4; ++t) qf[4 * c + t] = u[t];
        }
    }

    int ntiles;
    const int* list = nullptr;
    if (a.tile_counts != nullptr) {
        ntiles = a.tile_counts[qt];
        list = a.tile_entries + (int64_t)qt * a.num_k_tiles;
    } else {
        const int kend = a.causal ? min(a.N, q0 + kBlockM) : a.N;
        ntiles = (kend + BN - 1) / BN;
    }

    f32x4 kreg[CPT], vreg[CPT];
    auto load_tile = [&](int kt) {
        const int k0 = kt * BN;
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int ci = tid + kThreads * u;
            const int row = ci / NDC, cc = ci % NDC;
            const int kj = k0 + row;
            kreg[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            vreg[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (kj < a.N) {
                kreg[u] = *(const f32x4*)(Kp + (int64_t)kj * a.k_sn + 4 * cc);
                vreg[u] = *(const f32x4*)(Vp + (int64_t)kj * a.v_sn + 4 * cc);
            }
        }
    };
    auto store_tile = [&](int buf) {
        float* Ks = lds + buf * STAGE;
        float* Vs = Ks + KTILE;
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int ci = tid + kThreads * u;
            const int row = ci / NDC, cc = ci % NDC;
            *(f32x4*)(Ks + row * KSTR + 4 * cc) = kreg[u];
            *(f32x4*)(Vs + row * VSTR + 4 * cc) = vreg[u];
        }
    };
    auto tile_at = [&](int it, bool& partial) -> int {
        if (list != nullptr) {
            const int e = list[it];
            partial = (e & 1) != 0;
            return e >> 1;
        }
        partial = false;
        return it;
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int db = 0; db < D / 32; ++db) o[db] = f32x16{};
    float m_run = kNegInf, l_run = 0.0f;
    const float slope = (GENERAL && a.bias_kind == BIAS_ALIBI) ? a.alibi[h] : 0.0f;
    const float* bias_row = nullptr;
    if (GENERAL && a.bias_kind == BIAS_DENSE && my_q < a.M)
        bias_row = a.bias + b * a.bias_sb + h * a.bias_sh + (int64_t)my_q * a.bias_sm;

    if (ntiles > 0) {
        bool p0;
        load_tile(tile_at(0, p0));
        store_tile(0);
    }
    __syncthreads();

    for (int it = 0; it < ntiles; ++it) {
        bool partial;
        const int kt = tile_at(it, partial);
        if (it + 1 < ntiles) {
            bool pn;
            load_tile(tile_at(it + 1, pn));
        }
        const float* Ks = lds + (it & 1) * STAGE;
        const float* Vs = Ks + KTILE;
        const int k0 = kt * BN;
        const bool active = !(a.causal && k0 > qw0 + kQueriesPerWave - 1);
        if (active) {
            const bool need_mask = list != nullptr
                                       ? partial
                                       : ((k0 + BN > a.N) || (a.causal && k0 + BN - 1 > qw0));
            f32x16 s[1];
            s[0] = f32x16{};
            const float* krow = Ks + kappa(r) * KSTR + g * (D / 2);
#pragma unroll
            for (int c = 0; c < D / 8; ++c) {
                const f32x4 kv = *(const f32x4*)(krow + 4 * c);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    s[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[t], qf[4 * c + t], s[0], 0, 0, 0);
            }
            const float alpha = online_softmax_tile<1, GENERAL>(a, s, need_mask, my_q, k0, g, slope,
                                                                bias_row, m_run, l_run);
#pragma unroll
            for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const float* vrow = Vs + acc_pos(u, g) * VSTR + r;
#pragma unroll
                for (int db = 0; db < D / 32; ++db)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * db], s[0][u], o[db], 0, 0, 0);
            }
        }
        if (it + 1 < ntiles) store_tile((it + 1) & 1);
        __syncthreads();
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (my_q < a.M) {
        float* orow = (float*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)my_q * a.o_sm + 4 * g;
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f32x4 val;
#pragma unroll
                for (int j = 0; j < 4; ++j) val[j] = o[db][4 * i + j] * inv;
                *(f32x4*)(orow + 32 * db + 8 * i) = val;
            }
        }
    }
}

template <typename K>
hipError_t launch(K kernel, const FwdArgs& a, hipStream_t s) {
    const int64_t grid = (int64_t)a.B * a.H * a.num_q_tiles;
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_flash_mfma(const FwdArgs& a, int dtype, bool general_mod, hipStream_t s) {
#define OFH_DISPATCH_GM(KERNEL, ...)                                   \
    return general_mod ? launch(KERNEL<__VA_ARGS__, true>, a, s)        \
                       : launch(KERNEL<__VA_ARGS__, false>, a, s)
    if (dtype == DT_BF16) {
        if (a.D == 64) { OFH_DISPATCH_GM(flash_fwd_mfma16_kernel, __bf16, 64); }
        if (a.D == 128) { OFH_DISPATCH_GM(flash_fwd_mfma16_kernel, __bf16, 128); }
    } else if (dtype == DT_F16) {
        if (a.D == 64) { OFH_DISPATCH_GM(flash_fwd_mfma16_kernel, _Float16, 64); }
        if (a.D == 128) { OFH_DISPATCH_GM(flash_fwd_mfma16_kernel, _Float16, 128); }
    } else if (dtype == DT_F32) {
        if (a.D == 64) { OFH_DISPATCH_GM(flash_fwd_mfma32_kernel, 64); }
        if (a.D == 128) { OFH_DISPATCH_GM(flash_fwd_mfma32_kernel, 128); }
    }
#undef OFH_DISPATCH_GM
    return hipErrorInvalidValue;
}

const char* flash_mfma_kernel_name(int dtype, int D, bool general_mod) {
    static const char* names[3][2][2] = {
        {{"flash_fwd_mfma32_kernel<64,plain>", "flash_fwd_mfma32_kernel<64,general>"},
         {"flash_fwd_mfma32_kernel<128,plain>", "flash_fwd_mfma32_kernel<128,general>"}},
        {{"flash_fwd_mfma16_kernel<bf16,64,plain>", "flash_fwd_mfma16_kernel<bf16,64,general>"},
         {"flash_fwd_mfma16_kernel<bf16,128,plain>", "flash_fwd_mfma16_kernel<bf16,128,general>"}},
        {{"flash_fwd_mfma16_kernel<f16,64,plain>", "flash_fwd_mfma16_kernel<f16,64,general>"},
         {"flash_fwd_mfma16_kernel<f16,128,plain>", "flash_fwd_mfma16_kernel<f16,128,general>"}},
    };
    if (dtype < 0 || dtype > 2 || (D != 64 && D != 128)) return "none";
    return names[dtype][D == 128][general_mod ? 1 : 0];
}

int flash_mfma_block_n(int dtype) { return dtype == DT_F32 ? kBlockNF32 : kBlockN; }

}  // namespace ofh
