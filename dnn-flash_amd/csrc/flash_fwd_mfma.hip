// Flash-style attention forward on gfx950 matrix cores.
//
// Replaces the CPU loop nest of flash_attention_qk_pv_tile_ws
// (src/onednn_flash/attention.cpp:486-695 of the reference) and its batched
// driver (src/onednn_flash/batched_attention.cpp:9-49): one workgroup owns a
// query block of one (batch, head) (256 rows for bf16/fp16, 128 with a
// block mask or for fp32), each wavefront 32 of its rows; K/V stream through
// LDS in tiles of 64 or 128 keys; QK^T and PV run on MFMA; the
// online-softmax recurrence (running max, rescaled running sum, rescaled
// accumulator, attention.cpp:628-673) lives in registers; the N x N score
// matrix is never formed.
//
// Layout trick. Scores are computed transposed, S^T = K * Q^T, with K as the
// MFMA A operand and Q as the B operand. In the 32x32 accumulator layout lane
// l then holds 16 scores of ONE query (column l%32), so the row max, the row
// sum and the accumulator rescale are per-lane scalars, and the only
// cross-lane step per tile is one exchange between the two 32-lane halves
// for the max. The output is accumulated transposed as well, O^T = V^T * P^T:
// the B operand P^T is exactly the lane's own probabilities (no shuffle). In
// the 16-bit kernels the V^T A-operand fragments come from the row-major V
// tile in LDS through the transposing ds_read_b64_tr_b16; the fp32 kernel
// reads V row-major (one element per lane and operand).
//
// The accumulator row r = 8i + 4g + j (lane half g = l/32, register 4i+j)
// is fed from A-operand row r, and A rows are permuted by kappa(r) =
// 16(i>>1) + 8g + 4(i&1) + j. With that permutation, registers [8c, 8c+8) of
// lane half g hold 8 consecutive positions 16c + 8g + t, which is what the
// next MFMA wants in a lane (k-slots 8g..8g+7 of a 16-wide chunk), and what
// a 16-byte store of the output wants.

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <vector>

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

// s_waitcnt vmcnt(0): every vector-memory load issued so far has returned
// (and every store has completed: gfx9 counts both in vmcnt). Issued once
// before the tile loop, it tells the compiler's wait-count tracking that the
// Q fragments are resident on every path into the loop; without it the loop
// waits on them (and so on every load issued after them, i.e. the K/V
// prefetch) at each use.
__device__ __forceinline__ void wait_vm_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt vmcnt(N): at most N vector-memory operations still outstanding
// (they complete in issue order, so every older one has completed).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

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

// Causal attention without a block mask: workgroup id -> (flat head, query
// tiles nqt-1-p and p). The heavy tile runs first, then the light one, so
// every workgroup does the same number of tile steps (no tail of short
// workgroups) and both tiles share the head's K/V in one XCD's L2. qt_b is
// -1 when p is the middle tile of an odd count.
__device__ __forceinline__ void map_work_pair(int id, int BH, int nqt, int& bh, int& qt_a, int& qt_b) {
    const int np = (nqt + 1) / 2;
    int p;
    if ((BH & 7) == 0) {
        const int xcd = id & 7, j = id >> 3;
        const int hl = j / np;
        p = j - hl * np;
        bh = hl * 8 + xcd;
    } else {
        bh = id % BH;
        p = id / BH;
    }
    qt_a = nqt - 1 - p;
    qt_b = (p != qt_a) ? p : -1;
}

// Query tiles of this workgroup: one, or a causal pair (see map_work_pair).
__device__ __forceinline__ int work_tiles(const FwdArgs& a, bool paired, int& bh, int (&qts)[2]) {
    if (paired) {
        map_work_pair(blockIdx.x, a.B * a.H, a.num_q_tiles, bh, qts[0], qts[1]);
        return qts[1] >= 0 ? 2 : 1;
    }
    map_work(blockIdx.x, a.B * a.H, a.num_q_tiles, a.causal, bh, qts[0]);
    return 1;
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
// Key split (FwdArgs::num_splits > 1). Query tile qt has steps(qt) K/V tile
// steps; splits [0, active(qt)) of it run, split s over steps
// [s*range, (s+1)*range), range = split_range(steps(qt)). With one active split, split 0 writes O
// directly. Otherwise every active split writes its unnormalised partial rows
// (O_s, m_s, l_s) and the rows are merged with the log-sum-exp rule of
// attention.cpp:661-674 applied across splits:
//   m* = max_s m_s,  O = sum_s 2^(m_s - m*) O_s / sum_s 2^(m_s - m*) l_s.
// Rows that saw no valid key in any split (l = 0) are written as 0.

// Steps per split of a query tile with `steps` K/V tile steps.
__device__ __forceinline__ int split_range(const FwdArgs& a, int steps) {
    return a.pair_split ? max(1, (steps + a.num_splits - 1) / a.num_splits) : a.split_tiles;
}
__device__ __forceinline__ int split_active(const FwdArgs& a, int steps) {
    const int range = split_range(a, steps);
    return max(1, min(a.num_splits, (steps + range - 1) / range));
}

// Folds partial (m2, l2, o2) into (m, l, o); maxima in log2 units.
__device__ __forceinline__ void lse_fold(float& m, float& l, f32x4& o, float m2, float l2, f32x4 o2) {
    const float mg = fmaxf(m, m2);
    const float mu = mg == kNegInf ? 0.0f : mg;
    const float w1 = __builtin_amdgcn_exp2f(m - mu), w2 = __builtin_amdgcn_exp2f(m2 - mu);  // 0 for -inf
    l = l * w1 + l2 * w2;
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] = o[t] * w1 + o2[t] * w2;
    m = mg;
}

// Partial rows merged inside the launch that writes them (split_counters set)
// are stored and loaded with agent-scope atomics: each access is coherent
// across the XCDs' L2 caches by itself, so no L2 writeback or invalidation
// (an agent-scope fence) is needed, which would cost every other workgroup on
// the XCD its cached K/V tiles. Partial rows merged by a second launch use
// plain accesses (the launch boundary makes them visible).
__device__ __forceinline__ void put_partial(float* p, float v, bool coherent) {
    if (coherent) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}
__device__ __forceinline__ void put_partial4(float* p, f32x4 v, bool coherent) {
    if (coherent) {
#pragma unroll
        for (int t = 0; t < 4; ++t) __hip_atomic_store(p + t, v[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        *(f32x4*)p = v;
    }
}
template <bool COHERENT>
__device__ __forceinline__ float get_partial(const float* p) {
    if (COHERENT) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *p;
}
template <bool COHERENT>
__device__ __forceinline__ f32x4 get_partial4(const float* p) {
    if (COHERENT) {
        f32x4 v;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = __hip_atomic_load(p + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return v;
    }
    return *(const f32x4*)p;
}

// Merges columns [4c, 4c+4) of partial row prow over splits s0, s0+sstep, ...
// below `active`, four splits per group so that their loads are in flight
// together; the running max is raised per group.
template <bool COHERENT>
__device__ __forceinline__ void merge_partials(const FwdArgs& a, int64_t prow, int c, int s0, int sstep,
                                               int active, float& m, float& l, f32x4& acc) {
    const int64_t stride = (int64_t)a.B * a.H * a.M;
    constexpr int G = 4;
    for (int s = s0; s < active; s += G * sstep) {
        float ms[G], ls[G];
        f32x4 os[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const bool ok = s + j * sstep < active;
            const int64_t r = (int64_t)(ok ? s + j * sstep : s) * stride + prow;
            // (plain float loads: element 1 of a loaded u32x2 passed through
            // __builtin_bit_cast was read as element 0 by this compiler)
            ms[j] = ok ? get_partial<COHERENT>(a.part_ml + 2 * r) : kNegInf;
            ls[j] = get_partial<COHERENT>(a.part_ml + 2 * r + 1);
            os[j] = get_partial4<COHERENT>(a.part_o + r * a.Dv + 4 * c);
        }
        float mg = m;
#pragma unroll
        for (int j = 0; j < G; ++j) mg = fmaxf(mg, ms[j]);
        const float mu = mg == kNegInf ? 0.0f : mg;
        const float keep = __builtin_amdgcn_exp2f(m - mu);  // 0 while m is -inf
        l *= keep;
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] *= keep;
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const float w = __builtin_amdgcn_exp2f(ms[j] - mu);  // 0 for splits past `active`
            l += w * ls[j];
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[t] += w * os[j][t];
        }
        m = mg;
    }
}

// Writes columns [4c, 4c+4) of O row `row` of head bh, normalised by l.
template <typename T>
__device__ __forceinline__ void store_merged(const FwdArgs& a, int bh, int row, int c, float l, f32x4 acc) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int b = bh / a.H, h = bh - b * a.H;
    const int64_t off = b * a.o_sb + h * a.o_sh + (int64_t)row * a.o_sm + 4 * c;
    if (sizeof(T) == 4 || a.out_f32) {
        *(f32x4*)((float*)a.o + off) = acc * inv;
    } else if constexpr (sizeof(T) == 2) {
        typedef T v4 __attribute__((ext_vector_type(4)));
        v4 val;
#pragma unroll
        for (int t = 0; t < 4; ++t) val[t] = (T)(acc[t] * inv);
        *(v4*)((T*)a.o + off) = val;
    }
}

// Counts this workgroup in its query tile's arrival counter once the partial
// rows of every thread are stored (agent-scope atomic stores, complete when
// vmcnt reaches 0); true in the workgroup that arrives last, to which the
// partial rows of all splits of the tile are then visible through agent-scope
// atomic loads. That workgroup sets the counter back to zero for the next
// call on the stream. Every thread calls it; `flag` is one int of LDS.
__device__ __forceinline__ bool split_arrive(unsigned* ctr, int active, int* flag) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the partial-row stores stay above the wait
    wait_vm_loads();                          // vmcnt(0): this thread's stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev + 1 == (unsigned)active;
        if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last ? 1 : 0;
    }
    __syncthreads();
    return *flag != 0;
}

// Merge of the `rows` rows from q0 of head bh by one workgroup of NTHREADS
// threads: a thread per (row, 4-column chunk); when there are fewer such
// items than threads (few rows), the splits are shared out over groups of
// threads whose results are folded through `red` (6 * NTHREADS floats of LDS).
template <typename T, int NTHREADS>
__device__ void merge_split_rows(const FwdArgs& a, int bh, int q0, int rows, int active, float* red) {
    const int chunks = a.Dv >> 2;
    const int items = rows * chunks;
    const int t = threadIdx.x;
    if (items >= NTHREADS) {
        for (int item = t; item < items; item += NTHREADS) {
            const int rr = item / chunks, c = item - rr * chunks;
            float m = kNegInf, l = 0.0f;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            merge_partials<true>(a, (int64_t)bh * a.M + q0 + rr, c, 0, 1, active, m, l, acc);
            store_merged<T>(a, bh, q0 + rr, c, l, acc);
        }
        return;
    }
    const int groups = min(active, NTHREADS / items);
    const int item = t % items, grp = t / items;
    const bool mine = grp < groups;
    const int rr = item / chunks, c = item - rr * chunks;
    float m = kNegInf, l = 0.0f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (mine) merge_partials<true>(a, (int64_t)bh * a.M + q0 + rr, c, grp, groups, active, m, l, acc);
    if (mine && grp > 0) {
        float* e = red + 6 * (grp * items + item);
        e[0] = m;
        e[1] = l;
#pragma unroll
        for (int j = 0; j < 4; ++j) e[2 + j] = acc[j];
    }
    __syncthreads();
    if (grp == 0) {
        for (int j = 1; j < groups; ++j) {
            const float* e = red + 6 * (j * items + item);
            lse_fold(m, l, acc, e[0], e[1], f32x4{e[2], e[3], e[4], e[5]});
        }
        store_merged<T>(a, bh, q0 + rr, c, l, acc);
    }
}

// ---------------------------------------------------------------------------
// bf16 / fp16 inputs, fp32 accumulate: v_mfma_f32_32x32x16_{bf16,f16}.
//
// Every wavefront owns 32 query rows. K/V tiles are staged one tile ahead
// by global_load_lds_dwordx4 copies straight into LDS (no staging registers,
// no LDS store instructions). With the plain scale and no block mask a
// staged tile is 128 keys (two 64-key compute steps at D=128), otherwise 64.
// Loads are unconditional: rows past the end are clamped to the last row,
// their V zeroed and their scores masked, so no exec-masked branch breaks
// the compiler's wait counting.
//
// LDS layout (TileLayout): both tiles row-major [key][d], unpadded, with the
// 16-byte chunks of a row XOR-swizzled so that the K A-operand reads
// (ds_read_b128) and the V reads (ds_read_b64_tr_b16, which deliver V^T
// fragments directly, so V is never transposed in a separate pass) are free
// of bank conflicts at one XOR per read.
//
// Workgroup schedule (every 16-bit call): lockstep. All wavefronts run S,
// softmax and PV of a tile between two barriers; double-buffered LDS.
// Without a block-mask list the workgroup has 8 wavefronts (256 query rows);
// with one it has 4 (128 rows), which wastes fewer partial tiles on fine
// masks.
//
// Online softmax with lazy rescaling: the running max m that probabilities
// are taken against is raised only when a tile's max exceeds it by more than
// kRescaleSlack (log2 units), so p <= 2^8 and the O/l rescale (a wave-uniform
// branch) runs on a few tiles per row instead of every tile. The result is
// exact in real arithmetic: O and l share the same stale max.

constexpr int kBlockN16 = 64;      // keys per K/V tile (16-bit kernels) ...
constexpr int kBlockN16Wide = 128; // ... and for D = 64 without score_mod or block mask
constexpr float kRescaleSlack = 8.0f;
constexpr float kSumBound = 256.0f;  // 2^kRescaleSlack
constexpr int kFragAhead = 4;  // LDS fragment reads in flight ahead of the MFMAs (plain scale)

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

// Score modification of a 16-bit kernel instantiation: the plain scale, or
// any mix of ALiBi / dense bias / soft-cap selected per call.
enum ScoreMod { MOD_PLAIN = 0, MOD_GENERAL = 1 };


// One 16-byte global -> LDS copy per lane (lane L writes lds + 16 L; lds is
// wave-uniform). Written as assembly so that the compiler does not make LDS
// reads of the other stage wait for it; completion is awaited explicitly
// (wait_vm_loads) before the barrier that publishes the tile. M0 is restored.
__device__ __forceinline__ void dma16(const void* g, unsigned lds) {
    unsigned save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(save) : "v"(g), "s"(lds) : "memory");
}

// K and V tiles in LDS: row-major [key][d], unpadded (each global -> LDS
// copy instruction writes 1 KB of consecutive LDS). Chunk c (16 bytes) of row
// r sits at position c ^ kswz(r) (K) or c ^ vswz(r) (V), which keeps both
// read patterns free of bank conflicts (measured with SQ_LDS_BANK_CONFLICT):
// K fragments read rows kappa(0..15) at one chunk per 16 lanes; V^T fragments
// are transposing reads of 4 rows x 2 chunks per 16 lanes. For D = 64 two rows
// share a 256-byte bank line, hence row >> 1.
//
// Head dims that are not powers of two (96, 160, 192, 224) XOR only inside
// aligned groups of chunks that divide the row (see kswz), and their reads add
// per-lane bases to compile-time offsets instead of XORing the address.
template <int D, int BN>
struct TileLayout {
    static constexpr int RB = D * 2;              // bytes of one K/V row
    static constexpr int CPR = D / 8;             // 16-byte chunks per row
    static constexpr bool POW2 = (D & (D - 1)) == 0;
    static_assert(D % 32 == 0 && D >= 32 && D <= 256, "head dims of the 16-bit kernels: multiples of 32 up to 256");
    // Both swizzles must repeat every 8 rows or less at D = 256 (every 16 at
    // D = 128, 32 at D = 64, 64 at D = 32): a copy lane reuses one swizzled
    // chunk offset for the rows DSTEP = 64 * wavefronts / CPR apart that it
    // copies (8 rows with 4 wavefronts at D = 256). The V swizzle must also
    // repeat every 4 rows: a V^T fragment is two transposing reads 4 rows
    // apart at one lane offset.
    //
    // Rows that are not a power of two wide (D = 96, 160, 192, 224): a
    // 16-byte K read serves 16 lanes at a time, rows kappa(0..15) at one
    // chunk, and with 12, 20 or 28 chunks per row those rows start on only 4
    // distinct 16-byte bank groups (2 at 24 chunks). The chunk index is XORed
    // inside aligned groups of KG chunks (KG divides the row): by (row>>2)&3
    // (KG = 4), so the 16 rows cover the 16 bank groups, or by (row>>1)&7 at
    // D = 192 (KG = 8). A V^T read serves rows 4 apart in 64-byte runs, which
    // already fall on distinct banks except at D = 192 (rows 384 bytes apart):
    // there chunks are XORed with 4 on (row>>1)&1.
    static constexpr int KG = POW2 ? 1 : (D == 192 ? 8 : 4);
    static_assert(POW2 || CPR % KG == 0, "the K swizzle group divides the row");
    static __device__ __forceinline__ int kswz(int row) {
        if (!POW2) return D == 192 ? (row >> 1) & 7 : (row >> 2) & 3;
        if (D == 256) return row & 7;
        if (D == 128) return row & 15;
        if (D == 64) return (row >> 1) & 7;
        return (row >> 2) & 3;  // D = 32: four rows share a bank line
    }
    static __device__ __forceinline__ int vswz(int row) {
        if (!POW2) return D == 192 ? 4 * ((row >> 1) & 1) : 0;
        if (D >= 128) return 4 * (row & 3);
        if (D == 64) return 4 * ((row >> 1) & 1);
        return 0;  // D = 32: a row is one 32-column block
    }
    static constexpr int KSTR = RB;
    static constexpr int VSTR = RB;
    static constexpr int KTILE = BN * KSTR;
    static constexpr int VTILE = BN * VSTR;
    static constexpr int STAGE = KTILE + VTILE;   // K tile then V tile
};

// max over both 32-lane halves (lane l and l^32 hold the same query row)
__device__ __forceinline__ float half_swap_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                                    __builtin_bit_cast(unsigned, x), false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}

template <typename T>
struct Dot2;
template <>
struct Dot2<__bf16> {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ float sum2(v2 a, float acc) {
        return __builtin_amdgcn_fdot2_f32_bf16(a, v2{(__bf16)1.0f, (__bf16)1.0f}, acc, false);
    }
};
template <>
struct Dot2<_Float16> {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ float sum2(v2 a, float acc) {
        return __builtin_amdgcn_fdot2(a, v2{(_Float16)1.0f, (_Float16)1.0f}, acc, false);
    }
};

// Position of accumulator register e of sub-block sb within a 64-key tile,
// relative to the lane half's first key (8g): 32sb + 16(e>>3) + (e&7).
__device__ __forceinline__ constexpr int tile_pos(int sb, int e) { return 32 * sb + 16 * (e >> 3) + (e & 7); }

// The per-wavefront state and the tile operations of one 32-row wavefront.
// A "tile step" is identified by its entry: the key tile index, or with a
// block-mask list (LIST) the list entry (key tile + per-slice bits).
template <typename T, int D, int MOD, bool LIST, int NTHREADS, int BN_, int SB = 1, int DVK = D>
struct Wave32 {
    // DVK: value columns the kernel computes (a multiple of 32 up to D; O and
    // PV cover only those, the K side and the LDS rows stay D wide)
    static_assert(DVK % 32 == 0 && DVK <= D, "value columns: a multiple of 32 up to D");
    using T_ = T;
    using M16 = Mfma16<T>;
    using v8 = typename M16::v8;
    // K/V staged by global -> LDS copies in every kernel without a block-mask
    // list (register staging with one)
    using L = TileLayout<D, BN_ * SB>;
    static constexpr int BN = BN_;
    static constexpr int SN = BN_ * SB;                 // keys per staged tile
    static constexpr int CPT = SN * L::CPR / NTHREADS;  // 16-byte chunks per thread per tile
    static_assert(CPT >= 1 && SN * L::CPR % NTHREADS == 0, "tile must split evenly");

    const FwdArgs& a;
    unsigned char* smem;
    const T* Kp;
    const T* Vp;
    int tid, g, h, b, wave;
    int qw0, my_q;
    int ntiles;
    const int* list;
    v8 qf[D / 16];
    f32x16 o[DVK / 32];
    f32x16 s[BN / 32];
    v8 pf[BN / 16];
    float m_run, l_run;
    float slope;
    float alibi_step[8];  // soft-capped ALiBi: 2^(slope c_b t), t = 0..7 (wave-uniform)
    const float* bias_row;
    // LDS read lane offsets
    int k_lane_off, v_lane_off;
    // rows that are not a power of two wide: per-lane bases of the swizzled
    // chunk pairs (K) and 32-column blocks (V at D = 192), the rest of the
    // offset is a compile-time immediate
    int k_base[L::POW2 ? 1 : L::KG / 2];
    int v_base[L::POW2 ? 1 : 2];
    // K/V copies: lane offsets (elements) of its chunk in rows dma_row0 + u*DSTEP
    // when a copy instruction covers whole rows (64 * wavefronts divisible by
    // the chunks per row: every power-of-two D); otherwise each instruction's
    // row and chunk are derived from its slot index.
    static constexpr bool UNIFORM_COPY = (64 * (NTHREADS / 64)) % L::CPR == 0;
    static constexpr int DSTEP = UNIFORM_COPY ? 64 * (NTHREADS / 64) / L::CPR : 0;
    static_assert(!UNIFORM_COPY || !L::POW2 ||
                      DSTEP % (D == 256 ? 8 : D == 128 ? 16 : D == 64 ? 32 : 64) == 0,
                  "the K/V swizzles must repeat within the rows one copy lane covers");
    static_assert(UNIFORM_COPY || !L::POW2, "power-of-two rows are copied by whole-row instructions");
    static_assert(L::POW2 || !UNIFORM_COPY, "rows that are not a power of two wide are copied slot by slot");
    int dma_row0, dma_koff, dma_voff;
    // K fragment c (chunks 2c, 2c+1) and V^T block db at the lane's read offsets
    __device__ __forceinline__ int k_off(int c) const {
        if constexpr (L::POW2) return k_lane_off ^ (32 * c);
        // chunk (2c + g) ^ s = (2c & ~(KG-1)) + ((2c & (KG-1)) ^ (g ^ s))
        else return k_base[c % (L::KG / 2)] + 16 * ((2 * c) & ~(L::KG - 1));
    }
    __device__ __forceinline__ int v_off(int db) const {
        if constexpr (L::POW2) return v_lane_off ^ (64 * db);
        else if constexpr (D == 192) return v_base[db & 1] + 64 * (db & ~1);
        else return v_lane_off + 64 * db;
    }

    __device__ __forceinline__ Wave32(const FwdArgs& args, unsigned char* sm, int bh, int q0, int wv)
        : a(args), smem(sm), wave(wv) {
        tid = threadIdx.x;
        const int lane = tid & 63;
        g = lane >> 5;
        const int r = lane & 31;
        b = bh / a.H;
        h = bh - b * a.H;
        const T* Qp = (const T*)a.q + b * a.q_sb + h * a.q_sh;
        Kp = (const T*)a.k + b * a.k_sb + h * a.k_sh;
        Vp = (const T*)a.v + b * a.v_sb + h * a.v_sh;
        qw0 = q0 + wave * kQueriesPerWave;
        my_q = qw0 + r;
        // Q^T fragments (B operand of S^T = K Q^T): lane holds Q[my_q][16c + 8g .. +7].
        // Rows past the end read the last row; their results are never stored.
        // Columns at or past a.D (the kernel's D is the head dim rounded up) are zero.
        const T* qrow = Qp + (int64_t)min(my_q, a.M - 1) * a.q_sm + 8 * g;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            u32x4 u = {0u, 0u, 0u, 0u};
            if (16 * c + 8 * g < a.D) u = *(const u32x4*)(qrow + 16 * c);
            qf[c] = __builtin_bit_cast(v8, u);
        }
#pragma unroll
        for (int db = 0; db < DVK / 32; ++db) o[db] = f32x16{};
        m_run = kNegInf;
        l_run = 0.0f;
        slope = 0.0f;
        bias_row = nullptr;
        if (MOD == MOD_GENERAL) {
            if (a.bias_kind == BIAS_ALIBI) slope = a.alibi[h];
            const float sl8 = slope * (2.0f * kLog2e) * a.inv_softcap;
#pragma unroll
            for (int t = 0; t < 8; ++t)
                alibi_step[t] = __builtin_bit_cast(
                    float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, __builtin_amdgcn_exp2f(sl8 * (float)t))));
            if (a.bias_kind == BIAS_DENSE)
                bias_row = a.bias + b * a.bias_sb + h * a.bias_sh + (int64_t)min(my_q, a.M - 1) * a.bias_sm;
        }
        // K: A-operand row kappa(r) of a 32-key block, chunk 2c+g. V (transposed
        // reads): input lane j of a 16-lane group reads key (j/4) of a 4-key
        // group at d-chunk cmap(j%4) of the group's 16 columns; cmap = {0,2,1,3}
        // applies kappa to the output rows.
        const int G = lane >> 4, j = lane & 15;
        const int v_dquad = 16 * (G & 1) + 4 * ((j & 1) * 2 + ((j >> 1) & 1));  // d offset within 32
        // K chunk 2c+g of row kappa(r) sits at 32 (c ^ kh) + 16 gl: read at k_lane_off ^ 32c
        const int ksw = L::kswz(kappa(r));
        k_lane_off = kappa(r) * L::KSTR + 16 * ((g ^ ksw) & 1) + 32 * (ksw >> 1);
        if constexpr (!L::POW2) {
#pragma unroll
            for (int jj = 0; jj < L::KG / 2; ++jj) k_base[jj] = kappa(r) * L::KSTR + 16 * ((2 * jj) ^ (g ^ ksw));
        }
        // V chunk (v_dquad>>3) + 4 db of row 8g + j/4 sits at chunk + 4 (db ^ rq): read at v_lane_off ^ 64 db
        const int rq = L::vswz(8 * g + (j >> 2)) >> 2;
        v_lane_off = L::KTILE + (8 * g + (j >> 2)) * L::VSTR + (v_dquad >> 3) * 16 + (v_dquad & 4) * 2 + 64 * rq;
        if constexpr (!L::POW2) {
            const int vb0 = L::KTILE + (8 * g + (j >> 2)) * L::VSTR + (v_dquad >> 3) * 16 + (v_dquad & 4) * 2;
            v_base[0] = vb0 + 64 * rq;
            v_base[1] = vb0 + 64 * (1 ^ rq);
        }
        // copies: wave instruction u covers 16-byte slots 64 (u NWAVES + wave) + lane
        const int slot0 = 64 * wave + lane;
        dma_row0 = slot0 / L::CPR;
        const int pos = slot0 % L::CPR;
        dma_koff = dma_row0 * (int)a.k_sn + 8 * src_chunk(pos ^ L::kswz(dma_row0), a.D);
        dma_voff = dma_row0 * (int)a.v_sn + 8 * src_chunk(pos ^ L::vswz(dma_row0), a.Dv);
    }

    // Source chunk of the 16-byte chunk c of a K/V row whose real width is
    // `width` elements (the kernel's D may round the head dims up): chunks at
    // or past the real width repeat the row's last real chunk, finite data
    // that meets the zero Q columns (K) or fills O^T rows that are never
    // stored (V).
    static __device__ __forceinline__ int src_chunk(int c, int width) { return min(c, (width >> 3) - 1); }

    // Entry of tile step `it` (a global load with a list: issue it early).
    __device__ __forceinline__ int entry(int it) const { return LIST ? list[it] : it; }
    __device__ __forceinline__ int tile_of(int e) const { return LIST ? list_tile(e) : e; }
    __device__ __forceinline__ bool tile_active(int e) const {
        if (LIST) return list_any(e, wave);
        return qw0 < a.M && !(a.causal && e * BN > qw0 + kQueriesPerWave - 1);
    }
    // causal diagonal or ragged end inside the tile
    __device__ __forceinline__ bool tile_crosses(int kt) const {
        return (kt * BN + BN > a.N) || (a.causal && kt * BN + BN - 1 > qw0);
    }

    // Global -> LDS copy of staged tile kt into `stage_off` (asynchronous).
    // Rows past N read row N-1; zero_tail clears their V rows once landed.
    __device__ __forceinline__ void copy_tile(int kt, int stage_off) {
        const int k0 = kt * SN;
        const T* kt_base = Kp + (int64_t)k0 * a.k_sn;
        const T* vt_base = Vp + (int64_t)k0 * a.v_sn;
        const unsigned lds0 = (unsigned)(uintptr_t)smem + stage_off + 1024 * wave;
        constexpr int NW = NTHREADS / 64;
        if constexpr (!UNIFORM_COPY) {
            // slot 64 (u NW + wave) + lane: row slot / CPR, position slot % CPR
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                const int slot = 64 * (u * NW + wave) + (tid & 63);
                const int row = slot / L::CPR, pos = slot - row * L::CPR;
                const int rr = min(k0 + row, a.N - 1) - k0;
                dma16(kt_base + (int64_t)rr * a.k_sn + 8 * src_chunk(pos ^ L::kswz(row), a.D), lds0 + 1024 * NW * u);
                dma16(vt_base + (int64_t)rr * a.v_sn + 8 * src_chunk(pos ^ L::vswz(row), a.Dv),
                      lds0 + L::KTILE + 1024 * NW * u);
            }
            return;
        }
        if (k0 + SN <= a.N) {
            const T* kp = kt_base + dma_koff;
            const T* vp = vt_base + dma_voff;
            const int64_t kstep = (int64_t)DSTEP * a.k_sn, vstep = (int64_t)DSTEP * a.v_sn;
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                dma16(kp, lds0 + 1024 * NW * u);
                dma16(vp, lds0 + L::KTILE + 1024 * NW * u);
                kp += kstep;
                vp += vstep;
            }
        } else {
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                const int row = min(k0 + dma_row0 + u * DSTEP, a.N - 1) - k0 - dma_row0;
                dma16(kt_base + (int64_t)row * a.k_sn + dma_koff, lds0 + 1024 * NW * u);
                dma16(vt_base + (int64_t)row * a.v_sn + dma_voff, lds0 + L::KTILE + 1024 * NW * u);
            }
        }
    }
    __device__ __forceinline__ void zero_tail(int kt, int stage_off) {
        const int k0 = kt * SN;
        if (k0 + SN <= a.N) return;
        constexpr int NW = NTHREADS / 64;
        const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int row = UNIFORM_COPY ? dma_row0 + u * DSTEP : (64 * (u * NW + wave) + (tid & 63)) / L::CPR;
            if (k0 + row >= a.N)
                *(u32x4*)(smem + stage_off + L::KTILE + 1024 * wave + 1024 * NW * u + 16 * (tid & 63)) = zero;
        }
    }

    // S^T = K Q^T for the tile in LDS stage `stage_off`.
    __device__ __forceinline__ void qk(int stage_off, int sub = 0) {
        // Fragments are read kFragAhead MFMAs ahead of their use; the
        // scheduling fences keep the compiler from sinking each read next to
        // its MFMA (it otherwise keeps two in flight).
        constexpr int NF = (BN / 32) * (D / 16);
        const lds_u8* kbs = (const lds_u8*)smem + stage_off + sub * BN * L::KSTR;
        auto rd = [&](int i) {
            const int sb = i / (D / 16), c = i % (D / 16);
            return __builtin_bit_cast(v8, *(const lds_u32x4*)(kbs + 32 * sb * L::KSTR + k_off(c)));
        };
        v8 f[kFragAhead];
#pragma unroll
        for (int i = 0; i < kFragAhead; ++i) f[i] = rd(i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int sb = 0; sb < BN / 32; ++sb) s[sb] = f32x16{};
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            s[i / (D / 16)] = M16::mma(f[i % kFragAhead], qf[i % (D / 16)], s[i / (D / 16)]);
            if (i + kFragAhead < NF) f[i % kFragAhead] = rd(i + kFragAhead);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // O^T += V^T P^T for the tile in LDS stage `stage_off` (A operand from two
    // transposed 4-key reads).
    __device__ __forceinline__ void pv(int stage_off, int sub = 0) {
        const lds_u8* vbs = (const lds_u8*)smem + stage_off + sub * BN * L::VSTR;
        auto vfrag = [&](int c, int db) {
            const int off = v_off(db);
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vbs + (16 * c) * L::VSTR + off));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vbs + (16 * c + 4) * L::VSTR + off));
            return __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        };
        // V^T fragments kFragAhead MFMAs ahead (see qk)
        constexpr int NF = (DVK / 32) * (BN / 16);
        v8 f[kFragAhead];
#pragma unroll
        for (int i = 0; i < kFragAhead; ++i) f[i] = vfrag(i % (BN / 16), i / (BN / 16));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            o[i / (BN / 16)] = M16::mma(f[i % kFragAhead], pf[i % (BN / 16)], o[i / (BN / 16)]);
            if (i + kFragAhead < NF)
                f[i % kFragAhead] = vfrag((i + kFragAhead) % (BN / 16), (i + kFragAhead) / (BN / 16));
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Scores in log2 units with the call's score_mod: scale, then ALiBi
    // slope*(key - query) or a dense bias, then cap*tanh(x/cap). Constants are
    // folded so ALiBi costs two FMAs per score and the soft-cap an exp2, an
    // add and a reciprocal:
    //   u = 2 log2e t / cap, tanh = 1 - 2/(2^u + 1), x = log2e cap tanh
    //     = cap_hi + cap_m2 * r with r = 1/(2^u + 1), cap_hi = log2e cap,
    //   cap_m2 = -2 log2e cap < 0;
    // with a soft-cap s is left holding r (the softmax takes the row max from
    // min r and folds cap_hi + cap_m2 * r into its exp2 argument).
    template <int BIAS, bool CAP>
    __device__ __forceinline__ void score_mod_tile(int k0) {
        const float c_s = CAP ? a.scale * (2.0f * kLog2e) * a.inv_softcap : a.scale_log2;
        const float c_b = CAP ? (2.0f * kLog2e) * a.inv_softcap : kLog2e;
        const float sl = slope * c_b;
        const float base = sl * (float)(k0 + 8 * g - my_q);
        float bvals[BN / 2];
        if (BIAS == BIAS_DENSE) {
            const float* br = bias_row + k0 + 8 * g;
            if (k0 + BN <= a.N) {
#pragma unroll
                for (int q4 = 0; q4 < BN / 8; ++q4) {
                    const f32x4 v = *(const f32x4*)(br + 16 * (q4 >> 1) + 4 * (q4 & 1));
#pragma unroll
                    for (int t = 0; t < 4; ++t) bvals[4 * q4 + t] = v[t];
                }
            } else {
#pragma unroll
                for (int sb = 0; sb < BN / 32; ++sb)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        bvals[16 * sb + e] = bias_row[min(k0 + 8 * g + tile_pos(sb, e), a.N - 1)];
            }
        }
        if constexpr (BIAS == BIAS_ALIBI && CAP) {
            // 2^u = 2^(c_s s + base_j) * 2^(sl t) with key 8-group base_j and t = key & 7: the ALiBi step
            // inside a group rides on the "+ 1" of the soft-cap as a multiply-add
#pragma unroll
            for (int sb = 0; sb < BN / 32; ++sb)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const float bj = __builtin_fmaf(sl, (float)(32 * sb + 16 * hh), base);
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(s[sb][8 * hh + t], c_s, bj));
                        s[sb][8 * hh + t] = __builtin_amdgcn_rcpf(__builtin_fmaf(x, alibi_step[t], 1.0f));
                    }
                }
            return;
        }
#pragma unroll
        for (int sb = 0; sb < BN / 32; ++sb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                float u;
                if (BIAS == BIAS_ALIBI)
                    u = __builtin_fmaf(s[sb][e], c_s, __builtin_fmaf(sl, (float)tile_pos(sb, e), base));
                else if (BIAS == BIAS_DENSE)
                    u = __builtin_fmaf(s[sb][e], c_s, bvals[16 * sb + e] * c_b);
                else
                    u = s[sb][e] * c_s;
                // with a soft-cap, s keeps r = 1 / (2^u + 1): the log2 score is
                // cap_hi + cap_m2 * r, formed inside the softmax's exp2 argument
                if (CAP) u = __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(u) + 1.0f);
                s[sb][e] = u;
            }
    }
    __device__ __forceinline__ void general_scores(int k0) {
        const bool cap = a.softcap > 0.0f;
        if (a.bias_kind == BIAS_ALIBI) {
            if (cap) score_mod_tile<BIAS_ALIBI, true>(k0);
            else score_mod_tile<BIAS_ALIBI, false>(k0);
        } else if (a.bias_kind == BIAS_DENSE) {
            if (cap) score_mod_tile<BIAS_DENSE, true>(k0);
            else score_mod_tile<BIAS_DENSE, false>(k0);
        } else {
            if (cap) score_mod_tile<BIAS_NONE, true>(k0);
            else score_mod_tile<BIAS_NONE, false>(k0);
        }
    }

    // Masked scores -> `masked` (-inf, or +inf for soft-capped scores held as
    // r). Causal / ragged end: key k0+8g+pos is valid iff pos < lim. With a
    // block mask whose blocks cut the slice: per element.
    __device__ __forceinline__ void apply_mask(int e_ent, int k0, float masked = kNegInf) {
        if (LIST && !list_full(e_ent, wave)) {
            // masked_out (attention.cpp:54-62) per element, branch-free: the
            // bitmap bytes are read at clamped indices and combined by selects
            const int qb = my_q / a.mask_qbs;
            const bool row_ok = qb < a.mask_qb;
            const uint8_t* mrow = a.mask + (int64_t)min(qb, a.mask_qb - 1) * a.mask_kb;
            const int klim = a.causal ? min(a.N - 1, my_q) : a.N - 1;  // last valid key
            // 8 consecutive keys at a time: their bitmap bytes are loaded together
#pragma unroll
            for (int q8 = 0; q8 < BN / 16; ++q8) {
                const int sb = q8 >> 1, e0 = 8 * (q8 & 1);
                unsigned char byte[8];
                int kbs[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    kbs[t] = min(k0 + 8 * g + tile_pos(sb, e0 + t), a.N - 1) / a.mask_kbs;
                    byte[t] = mrow[min(kbs[t], a.mask_kb - 1)];
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int kj = k0 + 8 * g + tile_pos(sb, e0 + t);
                    const bool ok = row_ok & (kj <= klim) & (kbs[t] < a.mask_kb) & (byte[t] != 0);
                    s[sb][e0 + t] = ok ? s[sb][e0 + t] : masked;
                }
            }
            return;
        }
        const int lim = (a.causal ? min(a.N, my_q + 1) : a.N) - k0 - 8 * g;
#pragma unroll
        for (int sb = 0; sb < BN / 32; ++sb)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                if (tile_pos(sb, e) >= lim) s[sb][e] = masked;
    }

    // Online softmax of the scores in s (tile step with entry e_ent): running
    // max with lazy rescale of O and l, probabilities packed into pf, row sum.
    __device__ __forceinline__ void softmax(int e_ent) {
        const int kt = tile_of(e_ent);
        const int k0 = kt * BN;
        const bool need_mask = tile_crosses(kt) || (LIST && !list_full(e_ent, wave));
        float mx = kNegInf;
        const bool raw = MOD == MOD_PLAIN && !need_mask;  // s still holds raw dot products
        // 128-key tiles (D <= 64, no list): p is taken against the running max
        // first, without the tile's max. A row sum of at most 2^kRescaleSlack
        // proves every p <= 2^kRescaleSlack, the bound the lazy rescale keeps,
        // so the result is the one the max would have given (the max raises
        // nothing then). Otherwise (a larger sum, inf or NaN) the tile is redone
        // below with its max. Measured +5-6 % at D = 32 and 64; at D = 96 and
        // 128 (64-key tiles) the same code measured slower (3-6 %).
        if (D <= 64 && !LIST && raw && __builtin_amdgcn_ballot_w64(m_run == kNegInf) == 0) {
            float fsum = 0.0f;
#pragma unroll
            for (int c = 0; c < BN / 16; ++c) {
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    pf[c][t] = (T)__builtin_amdgcn_exp2f(
                        __builtin_fmaf(s[c >> 1][8 * (c & 1) + t], a.scale_log2, -m_run));
#pragma unroll
                for (int t = 0; t < 8; t += 2)
                    fsum = Dot2<T>::sum2(typename Dot2<T>::v2{pf[c][t], pf[c][t + 1]}, fsum);
            }
            if (__builtin_amdgcn_ballot_w64(!(fsum <= kSumBound)) == 0) {
                l_run += fsum;
                return;
            }
        }
        const bool capped = MOD == MOD_GENERAL && a.softcap > 0.0f;  // uniform
        const float cap_hi = a.softcap * kLog2e, cap_m2 = -2.0f * a.softcap * kLog2e;
        if (raw) {
            if (a.scale_log2 >= 0.0f) {
#pragma unroll
                for (int sb = 0; sb < BN / 32; ++sb)
#pragma unroll
                    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[sb][e]);
                mx *= a.scale_log2;
            } else {
                float mn = __builtin_huge_valf();
#pragma unroll
                for (int sb = 0; sb < BN / 32; ++sb)
#pragma unroll
                    for (int e = 0; e < 16; ++e) mn = fminf(mn, s[sb][e]);
                mx = mn * a.scale_log2;
            }
        } else if (capped) {
            general_scores(k0);  // s = r, log2 score cap_hi + cap_m2 * r, decreasing in r
            if (need_mask) apply_mask(e_ent, k0, __builtin_huge_valf());
            float mn = __builtin_huge_valf();
#pragma unroll
            for (int sb = 0; sb < BN / 32; ++sb)
#pragma unroll
                for (int e = 0; e < 16; ++e) mn = fminf(mn, s[sb][e]);
            mx = __builtin_fmaf(mn, cap_m2, cap_hi);  // -inf when every score is masked
        } else {
            if (MOD == MOD_GENERAL) {
                general_scores(k0);
            } else {
#pragma unroll
                for (int sb = 0; sb < BN / 32; ++sb) s[sb] *= a.scale_log2;
            }
            if (need_mask) apply_mask(e_ent, k0);
#pragma unroll
            for (int sb = 0; sb < BN / 32; ++sb)
#pragma unroll
                for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[sb][e]);
        }
        mx = half_swap_max(mx);

        // Lazy rescale (wave-uniform branch).
        const bool raise = mx > m_run + kRescaleSlack;
        if (__builtin_amdgcn_ballot_w64(raise) != 0) {
            // lanes that do not raise keep their max and scale by exactly 1
            // (their m_run may be -inf: -inf - -inf must not reach exp2)
            const float alpha = raise ? __builtin_amdgcn_exp2f(m_run - mx) : 1.0f;
            m_run = raise ? mx : m_run;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < DVK / 32; ++db) o[db] *= alpha;
        }
        const float m_use = (m_run == kNegInf) ? 0.0f : m_run;

        if (raw) {
#pragma unroll
            for (int c = 0; c < BN / 16; ++c)
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    pf[c][t] = (T)__builtin_amdgcn_exp2f(
                        __builtin_fmaf(s[c >> 1][8 * (c & 1) + t], a.scale_log2, -m_use));
        } else if (capped) {
            const float c0 = cap_hi - m_use;
#pragma unroll
            for (int c = 0; c < BN / 16; ++c)
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    pf[c][t] = (T)__builtin_amdgcn_exp2f(__builtin_fmaf(s[c >> 1][8 * (c & 1) + t], cap_m2, c0));
        } else {
#pragma unroll
            for (int c = 0; c < BN / 16; ++c)
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    pf[c][t] = (T)__builtin_amdgcn_exp2f(s[c >> 1][8 * (c & 1) + t] - m_use);
        }
        float lsum = 0.0f;
#pragma unroll
        for (int c = 0; c < BN / 16; ++c)
#pragma unroll
            for (int t = 0; t < 8; t += 2)
                lsum = Dot2<T>::sum2(typename Dot2<T>::v2{pf[c][t], pf[c][t + 1]}, lsum);
        l_run += lsum;
    }

    // Key split: the unnormalised rows and (m, l) of split `split`.
    __device__ __forceinline__ void store_partial(int split) {
        const float l_tot = l_run + __shfl_xor(l_run, 32);
        if (my_q >= a.M) return;
        const int64_t prow = ((int64_t)split * a.B * a.H + (int64_t)b * a.H + h) * a.M + my_q;
        float* po = a.part_o + prow * a.Dv + 8 * g;
        const bool coh = a.split_counters != nullptr;
#pragma unroll
        for (int db = 0; db < DVK / 32; ++db) {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                if (32 * db + 16 * cc + 8 * g >= a.Dv) continue;  // past the value dim
                f32x4 lo, hi;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    lo[t] = o[db][8 * cc + t];
                    hi[t] = o[db][8 * cc + 4 + t];
                }
                put_partial4(po + 32 * db + 16 * cc, lo, coh);
                put_partial4(po + 32 * db + 16 * cc + 4, hi, coh);
            }
        }
        if (g == 0) {
            put_partial(a.part_ml + 2 * prow, m_run, coh);
            put_partial(a.part_ml + 2 * prow + 1, l_tot, coh);
        }
    }

    // Normalise and store; rows that saw no valid key have l = 0 and are written as 0.
    __device__ __forceinline__ void store_output() {
        const float l_tot = l_run + __shfl_xor(l_run, 32);
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        if (my_q >= a.M) return;
        if (a.out_f32) {
            float* orow = (float*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)my_q * a.o_sm + 8 * g;
#pragma unroll
            for (int db = 0; db < DVK / 32; ++db) {
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    if (32 * db + 16 * cc + 8 * g >= a.Dv) continue;  // past the value dim
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
            for (int db = 0; db < DVK / 32; ++db) {
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    if (32 * db + 16 * cc + 8 * g >= a.Dv) continue;  // past the value dim
                    v8 val;
#pragma unroll
                    for (int t = 0; t < 8; ++t) val[t] = (T)(o[db][8 * cc + t] * inv);
                    *(u32x4*)(orow + 32 * db + 16 * cc) = __builtin_bit_cast(u32x4, val);
                }
            }
        }
    }
};

// Tile steps of the workgroup's query block: their number and, with a block
// mask, the list of entries.
__device__ __forceinline__ void tile_range(const FwdArgs& a, int qt, int block_m, int block_n,
                                           int& ntiles, const int*& list) {
    list = nullptr;
    if (a.tile_counts != nullptr) {
        ntiles = a.tile_counts[qt];
        list = a.tile_entries + (int64_t)qt * a.num_k_tiles;
    } else {
        const int q0 = qt * block_m;
        const int kend = a.causal ? min(a.N, q0 + block_m) : a.N;
        ntiles = (kend + block_n - 1) / block_n;
    }
}

// All wavefronts run S, softmax and PV of a tile step between two barriers;
// double-buffered LDS. The copies of tile it+1 go into the free stage at the
// start of step it and are awaited before the barrier that ends it, so their
// latency hides behind a whole step. With a list, entries are loaded two
// steps ahead of their use.
// End of a query tile (or of its key split `split` of `active`): O, or the
// partial rows followed by the merge in the split workgroup that arrives last.
template <typename W, int NTHREADS, bool SPLIT>
__device__ __forceinline__ void finish_qtile(const FwdArgs& a, W& w, unsigned char* smem, int bh, int qt,
                                             int q0, int block_m, int split, int active) {
    if (!SPLIT || active <= 1) {
        w.store_output();
        return;
    }
    w.store_partial(split);
    if (a.split_counters == nullptr) return;  // merged by combine_splits_kernel
    __syncthreads();                          // LDS below is reused
    int* flag = (int*)(smem + 24 * NTHREADS);
    if (split_arrive(a.split_counters + (int64_t)bh * a.num_q_tiles + qt, active, flag))
        merge_split_rows<typename W::T_, NTHREADS>(a, bh, q0, min(block_m, a.M - q0), active, (float*)smem);
}

typedef __attribute__((address_space(3))) int lds_int;

// Block-mask list of query tile q0 built by its own workgroup, in LDS: the key
// tiles (in order) that hold a pair allowed by the mask and the causal rule
// for some 32-row slice, each with per-slice any/all bits (list_entry), the
// list the tile_list kernel builds in global memory (rowwise_fwd.hip). One key
// tile per thread and round; compacted with a per-wavefront ballot and a
// prefix over the wavefronts' counts. Returns the entry count (uniform).
template <int NWAVES>
__device__ int build_tile_list_lds(const FwdArgs& a, int q0, int block_n, lds_int* list, lds_int* wave_counts) {
    constexpr int NT = NWAVES * 64;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int count = 0;
    // The mask-block rows of each slice are the same for every thread (the
    // query tile is the workgroup's); only the key tile differs. They are
    // formed once, and by shifts where the block sizes are powers of two
    // (the common case; a division costs some twenty VALU instructions).
    const bool pow2 = (a.mask_qbs & (a.mask_qbs - 1)) == 0 && (a.mask_kbs & (a.mask_kbs - 1)) == 0;  // uniform
    const int lq = __builtin_ctz((unsigned)a.mask_qbs), lk = __builtin_ctz((unsigned)a.mask_kbs);
    int sq0[NWAVES], sq1[NWAVES], se[NWAVES];
    bool one_qb = true;  // every slice within one mask-block row (uniform)
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) {
        const int s0 = q0 + kQueriesPerWave * w, s1 = min(a.M, s0 + kQueriesPerWave);
        se[w] = s1;
        sq0[w] = s0 < s1 ? (pow2 ? s0 >> lq : s0 / a.mask_qbs) : 1;
        sq1[w] = s0 < s1 ? (pow2 ? (s1 - 1) >> lq : (s1 - 1) / a.mask_qbs) : 0;  // empty slice: no rows
        one_qb = one_qb && sq0[w] >= sq1[w];
    }
    for (int base = 0; base < a.num_k_tiles; base += NT) {
        const int kt = base + tid;
        unsigned any_bits = 0, full_bits = 0;
        if (kt < a.num_k_tiles) {
            const int k0 = kt * block_n, k1 = min(a.N, k0 + block_n);
            const int kb0 = pow2 ? k0 >> lk : k0 / a.mask_kbs;
            const int kb1 = pow2 ? (k1 - 1) >> lk : (k1 - 1) / a.mask_kbs;
            if (one_qb && kb0 == kb1) {
                // One mask byte per slice (the common case: blocks no smaller
                // than a slice and a key tile), all requested before any is
                // used: the loops below would wait for each in turn. Same
                // rule as classify_mask_blocks.
                unsigned char mb[NWAVES];
#pragma unroll
                for (int w = 0; w < NWAVES; ++w)
                    mb[w] = a.mask[(int64_t)min(sq0[w], a.mask_qb - 1) * a.mask_kb + min(kb0, a.mask_kb - 1)];
#pragma unroll
                for (int w = 0; w < NWAVES; ++w) {
                    const int qe = min(se[w], (sq0[w] + 1) * a.mask_qbs);
                    const bool allowed = sq0[w] <= sq1[w] && sq0[w] < a.mask_qb && kb0 < a.mask_kb && mb[w] != 0;
                    const bool any = allowed && (!a.causal || k0 <= qe - 1);
                    any_bits |= (any ? 1u : 0u) << w;
                    full_bits |= (allowed ? 1u : 0u) << w;
                }
            } else {
#pragma unroll
                for (int w = 0; w < NWAVES; ++w) {
                    if (sq0[w] > sq1[w]) continue;
                    bool any, all;
                    classify_mask_blocks(a.mask, a.mask_qbs, a.mask_kbs, a.mask_qb, a.mask_kb, a.causal, se[w],
                                         k0, sq0[w], sq1[w], kb0, kb1, any, all);
                    any_bits |= (any ? 1u : 0u) << w;
                    full_bits |= (all ? 1u : 0u) << w;
                }
            }
        }
        const unsigned long long bal = __ballot(any_bits != 0);
        if (lane == 0) wave_counts[wave] = __popcll(bal);
        __syncthreads();
        int before = count, total = count;
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) {
            const int c = wave_counts[w];
            before += w < wave ? c : 0;
            total += c;
        }
        if (any_bits != 0) list[before + __popcll(bal & ((1ull << lane) - 1ull))] = list_entry(kt, any_bits, full_bits);
        __syncthreads();  // wave_counts is rewritten in the next round
        count = total;
    }
    return count;
}

// Stages of the LDS-list schedule: tiles it+1 .. it+NSTAGE-1 are in flight
// while tile it is computed (three stages up to D = 64, two above, where a
// stage is 32 KB or more).
template <int D>
constexpr int lds_list_stages() { return D <= 64 ? 3 : 2; }
constexpr int kLdsListCountsBytes = 64;  // per-wavefront counts, then the list

// Block-mask query tile with its list in LDS (one workgroup per query tile,
// no key split): the list is built first (mask reads only, before any K/V
// load), then the K/V tiles of its entries stream through a ring of
// NSTAGE stages, NSTAGE-1 tiles ahead of the one being computed. The list is
// read from LDS, so the only vector-memory operations in the loop are the
// tile copies (2 CPT per thread and tile) and the wait before each barrier
// leaves the younger tiles' copies in flight.
template <typename W, int NWAVES, int MOD>
__device__ __forceinline__ void lds_list_qtile(const FwdArgs& a, unsigned char* smem, int bh, int qt, int q0,
                                               int wave) {
    using L = typename W::L;
    constexpr int D = L::CPR * 8;
    constexpr int NSTAGE = lds_list_stages<D>();
    constexpr int VM_PER_TILE = 2 * W::CPT;
    static_assert(W::SN == W::BN, "one compute step per list entry");
    lds_int* counts = (lds_int*)(smem + NSTAGE * L::STAGE);
    lds_int* lst = counts + kLdsListCountsBytes / 4;
    const int ntiles = build_tile_list_lds<NWAVES>(a, q0, W::BN, lst, counts);
    W w(a, smem, bh, q0, wave);
    if (ntiles == 0) {  // uniform over the workgroup
        w.store_output();
        return;
    }
    auto tile_of = [](int e) { return list_tile(e); };
    w.copy_tile(tile_of(lst[0]), 0);
    if (NSTAGE > 2 && ntiles > 1) {
        w.copy_tile(tile_of(lst[1]), L::STAGE);
        wait_vm<VM_PER_TILE>();  // tile 0 (and the Q fragments) landed; tile 1 in flight
    } else {
        wait_vm_loads();
    }
    w.zero_tail(tile_of(lst[0]), 0);
    __syncthreads();
    int stage = 0;
    for (int it = 0; it < ntiles; ++it) {
        const int ahead = it + NSTAGE - 1;  // tile copied during this step
        int astage = stage + (NSTAGE - 1) * L::STAGE;
        if (astage >= NSTAGE * L::STAGE) astage -= NSTAGE * L::STAGE;
        if (ahead < ntiles) w.copy_tile(tile_of(lst[ahead]), astage);
        const int e = lst[it];
        if (w.tile_active(e)) {
            if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(1);
            w.qk(stage);
            if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(0);
            w.softmax(e);
            if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(1);
            w.pv(stage);
            if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(0);
        }
        // tile it+1 must have landed; the copies of tile it+2 may stay in flight
        if (NSTAGE > 2 && it + 2 < ntiles) wait_vm<VM_PER_TILE>();
        else wait_vm_loads();
        int nstage = stage + L::STAGE;
        if (nstage >= NSTAGE * L::STAGE) nstage = 0;
        if (it + 1 < ntiles) w.zero_tail(tile_of(lst[it + 1]), nstage);
        __syncthreads();
        stage = nstage;
    }
    w.store_output();
}

template <typename T, int D, int MOD, bool LIST, int NWAVES, int BN, int SB, bool SPLIT, int DVK = D>
__device__ __forceinline__ void lockstep_qtile(const FwdArgs& a, unsigned char* smem, int bh, int qt,
                                               int split = 0) {
    constexpr int NTHREADS = NWAVES * 64;
    constexpr int BLOCK_M = NWAVES * kQueriesPerWave;
    static_assert(!LIST || NWAVES <= kListSlices, "list entries carry one bit per wavefront");
    using W = Wave32<T, D, MOD, LIST, NTHREADS, BN, SB, DVK>;
    using L = typename W::L;
    static_assert(2 * L::STAGE >= 24 * NTHREADS + 4, "split merge scratch fits in the LDS stages");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q0 = qt * BLOCK_M;
    if constexpr (!LIST) {
        // SB compute steps of BN keys per staged tile of SB*BN keys (one
        // barrier per staged tile); no list. Tile
        // st+1 is copied global -> LDS (no registers) into the free stage at
        // the start of step st and awaited before the barrier that ends it.
        static_assert(!LIST, "LDS copies: no list");
        const int kend = a.causal ? min(a.N, q0 + BLOCK_M) : a.N;
        const int nst = (kend + W::SN - 1) / W::SN;      // staged tiles
        const int active = SPLIT ? split_active(a, nst) : 1;
        if (split >= active) return;                     // uniform over the workgroup
        const int range = SPLIT ? split_range(a, nst) : nst;
        const int st0 = SPLIT ? split * range : 0;
        const int st1 = SPLIT ? min(nst, st0 + range) : nst;
        W w(a, smem, bh, q0, wave);
        if (st0 >= st1) {  // uniform over the workgroup
            finish_qtile<W, NTHREADS, SPLIT>(a, w, smem, bh, qt, q0, BLOCK_M, split, active);
            return;
        }
        // (returning early keeps every path into the loop through the wait
        // below, so the compiler sees the Q fragments resident in the loop)
        w.copy_tile(st0, 0);
        wait_vm_loads();
        w.zero_tail(st0, 0);
        __syncthreads();
        for (int st = st0; st < st1; ++st) {
            const int stage = ((st - st0) & 1) * L::STAGE;
            const int nstage = ((st - st0 + 1) & 1) * L::STAGE;
            if (st + 1 < st1) w.copy_tile(st + 1, nstage);
#pragma unroll
            for (int j = 0; j < SB; ++j) {
                const int e = st * SB + j;               // BN-key compute tile
                if (e * BN < kend && w.tile_active(e)) {
                    // Plain scale: matrix phases at wave priority 1 and the
                    // softmax at 0, so that a wavefront ready for MFMAs issues
                    // first when the two wavefronts of a SIMD drift apart
                    // (measured +1-2 %; with a score_mod the longer softmax is
                    // better left at equal priority).
                    if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(1);
                    w.qk(stage, j);
                    if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(0);
                    w.softmax(e);
                    if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(1);
                    w.pv(stage, j);
                    if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(0);
                }
            }
            wait_vm_loads();
            if (st + 1 < st1) w.zero_tail(st + 1, nstage);
            __syncthreads();
        }
        finish_qtile<W, NTHREADS, SPLIT>(a, w, smem, bh, qt, q0, BLOCK_M, split, active);
        return;
    }
    if constexpr (LIST) {
        if (a.tile_counts == nullptr) {  // list built in LDS (no key split)
            lds_list_qtile<W, NWAVES, MOD>(a, smem, bh, qt, q0, wave);
            return;
        }
    }
    int ntiles;
    const int* list;
    tile_range(a, qt, BLOCK_M, BN, ntiles, list);
    const int active = SPLIT ? split_active(a, ntiles) : 1;
    if (split >= active) return;  // uniform over the workgroup
    const int range = SPLIT ? split_range(a, ntiles) : ntiles;
    const int it0 = SPLIT ? split * range : 0;
    const int it1 = SPLIT ? min(ntiles, it0 + range) : ntiles;
    W w(a, smem, bh, q0, wave);
    w.ntiles = ntiles;
    w.list = list;
    // entry it+1 is copied during step it
    if (it0 >= it1) {
        finish_qtile<W, NTHREADS, SPLIT>(a, w, smem, bh, qt, q0, BLOCK_M, split, active);
        return;
    }
    int e_cur = w.entry(it0);
    int e_nxt = it0 + 1 < it1 ? w.entry(it0 + 1) : 0;
    w.copy_tile(w.tile_of(e_cur), 0);
    wait_vm_loads();
    w.zero_tail(w.tile_of(e_cur), 0);
    __syncthreads();
    for (int it = it0; it < it1; ++it) {
        const int stage = ((it - it0) & 1) * L::STAGE;
        const int nstage = ((it - it0 + 1) & 1) * L::STAGE;
        if (it + 1 < it1) w.copy_tile(w.tile_of(e_nxt), nstage);
        const int e_nn = it + 2 < it1 ? w.entry(it + 2) : 0;
        if (w.tile_active(e_cur)) {
            if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(1);
            w.qk(stage);
            if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(0);
            w.softmax(e_cur);
            if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(1);
            w.pv(stage);
            if (MOD == MOD_PLAIN) __builtin_amdgcn_s_setprio(0);
        }
        wait_vm_loads();
        if (it + 1 < it1) w.zero_tail(w.tile_of(e_nxt), nstage);
        __syncthreads();
        e_cur = e_nxt;
        e_nxt = e_nn;
    }
    finish_qtile<W, NTHREADS, SPLIT>(a, w, smem, bh, qt, q0, BLOCK_M, split, active);
}

// Workgroups per CU the register budget is sized for: one of 8 wavefronts,
// two of 4, or one of 4 from D = 160 up (one wavefront per SIMD, so the O
// accumulators can use the accumulation registers). The plain-scale
// block-mask kernels at D <= 64 fit three of 4 (at most 168 VGPRs: 163 at
// D = 64, 128 at D = 32, no spills; their LDS, three 16 KB stages and the
// list, fits three workgroups too). On the fp16 block-sparse workload the
// third wavefront per SIMD measured within 1 % of two (+0.1 to +0.6 % with
// the timing order alternated). With a score_mod the same bound spills, so
// those keep two.
constexpr int lockstep_min_blocks(int D, int nwaves, int mod, bool list) {
    return nwaves == 8 ? 1 : D >= 160 ? 1 : (list && mod == MOD_PLAIN && D <= 64) ? 3 : 2;
}

// SPLIT (query tiles not paired): the kernel may run a key split; calls with
// one split take the instantiation without it, whose loop then keeps the
// split's values out of its scalar registers (fewer spilled to vector lanes).
template <typename T, int D, int MOD, bool LIST, int NWAVES, bool PAIRED, int BN = kBlockN16, int SB = 1,
          bool SPLIT = true, int DVK = D>
__global__ __launch_bounds__(NWAVES * 64, lockstep_min_blocks(D, NWAVES, MOD, LIST)) void flash_fwd_lockstep_kernel(FwdArgs a) {
    using L = TileLayout<D, BN * SB>;
    // block-mask kernels: LDS sized at launch (list_kernel_lds_bytes)
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn_smem[];
    __shared__ __attribute__((aligned(16))) unsigned char st_smem[LIST ? 16 : 2 * L::STAGE];
    unsigned char* smem = LIST ? dyn_smem : st_smem;
    int bh, qts[2];
    if (!PAIRED) {  // key split s: workgroups [s * tiles, (s+1) * tiles)
        const int tiles = a.B * a.H * a.num_q_tiles;
        const int split = (int)blockIdx.x / tiles;
        map_work((int)blockIdx.x - split * tiles, a.B * a.H, a.num_q_tiles, a.causal, bh, qts[0]);
        lockstep_qtile<T, D, MOD, LIST, NWAVES, BN, SB, SPLIT, DVK>(a, smem, bh, qts[0], split);
        return;
    }
    // (paired query tiles are never split)
    const int n = work_tiles(a, PAIRED, bh, qts);
    lockstep_qtile<T, D, MOD, LIST, NWAVES, BN, SB, false, DVK>(a, smem, bh, qts[0]);
    if (n > 1) {
        __syncthreads();  // LDS stages are reused
        lockstep_qtile<T, D, MOD, LIST, NWAVES, BN, SB, false, DVK>(a, smem, bh, qts[1]);
    }
}

// Block-mask calls whose lists are built in LDS (no key split, no global
// list): the LDS-list path of the lockstep kernel as a kernel of its own, so
// that its loop does not share registers with the global-list path.
template <typename T, int D, int MOD>
__global__ __launch_bounds__(256, lockstep_min_blocks(D, 4, MOD, true)) void flash_fwd_lds_list_kernel(FwdArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn_smem[];
    using W = Wave32<T, D, MOD, true, 256, kBlockN16, 1>;
    int bh, qt;
    map_work((int)blockIdx.x, a.B * a.H, a.num_q_tiles, a.causal, bh, qt);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    lds_list_qtile<W, 4, MOD>(a, dyn_smem, bh, qt, qt * 4 * kQueriesPerWave, wave);
}

// Causal query tile pairs with a key split (FwdArgs::pair_split): workgroup s
// of the pair (nqt-1-p, p) runs split s of both tiles, each tile cut into
// num_splits ranges of its own length, so every workgroup runs about
// (steps(nqt-1-p) + steps(p)) / num_splits staged tiles. A kernel of its own,
// so that the paired kernel without a split keeps its code.
template <typename T, int D, int MOD, int NWAVES, int BN = kBlockN16, int SB = 1>
__global__ __launch_bounds__(NWAVES * 64, lockstep_min_blocks(D, NWAVES, MOD, false)) void flash_fwd_pair_split_kernel(FwdArgs a) {
    using L = TileLayout<D, BN * SB>;
    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * L::STAGE];
    const int pairs = a.B * a.H * ((a.num_q_tiles + 1) / 2);
    const int split = (int)blockIdx.x / pairs;
    int bh, qa, qb;
    map_work_pair((int)blockIdx.x - split * pairs, a.B * a.H, a.num_q_tiles, bh, qa, qb);
    lockstep_qtile<T, D, MOD, false, NWAVES, BN, SB, true>(a, smem, bh, qa, split);
    if (qb >= 0) {
        __syncthreads();  // LDS stages are reused
        lockstep_qtile<T, D, MOD, false, NWAVES, BN, SB, true>(a, smem, bh, qb, split);
    }
}

// ---------------------------------------------------------------------------
// fp32 inputs: v_mfma_f32_32x32x2_f32. Each MFMA consumes one element per lane
// and operand, so K and V stay row-major in LDS (no transposition): the
// reduction index d of S^T is split as d = g*D/2 + s over the two lane halves,
// and each PV step takes the two keys that the lane halves hold in register u.
// With a key split (FwdArgs::num_splits > 1) the workgroups of a query tile
// each run a range of its K/V tile steps and write partial rows, which
// combine_splits_kernel merges. Causal calls split with FwdArgs::pair_split:
// workgroup s of the pair (nqt-1-p, p) runs split s of both query tiles, each
// tile cut into num_splits ranges of its own length, so a workgroup runs
// about (steps(nqt-1-p) + steps(p)) / num_splits steps whatever p is (with
// one range length for all tiles the longest tile's ranges set the time).

constexpr int kBlockNF32 = 32;  // keys per accumulator block of the fp32 kernel
constexpr int kTilesF32 = 2;    // blocks per K/V tile: 64 keys per barrier (+3 to +5 % over one block)
constexpr int kWaves32 = 4;
constexpr int kThreads32 = kWaves32 * 64;
constexpr int kBlockM32 = kWaves32 * kQueriesPerWave;  // 128

template <int D, int NB>
struct Mfma32Tiles {
    static constexpr int BN = kBlockNF32 * NB;  // NB blocks of 32 keys per K/V tile
    static constexpr int KSTR = D + 4;  // floats; conflict-free 16-byte reads of rows kappa(r)
    static constexpr int VSTR = D + 4;  // floats; lane halves read rows 8 apart -> opposite bank halves
    static constexpr int KTILE = BN * KSTR;
    static constexpr int STAGE = 2 * KTILE;
};

// Query tile qt of head bh, key split `split` (the whole key range without
// one), on the workgroup's LDS `lds` (2 * STAGE floats).
template <int D, bool GENERAL, int NB, bool LISTS = true>
__device__ __forceinline__ void mfma32_qtile(const FwdArgs& a, float* lds, int bh, int qt, int split) {
    using TL = Mfma32Tiles<D, NB>;
    constexpr int BN = TL::BN;
    constexpr int KSTR = TL::KSTR;
    constexpr int VSTR = TL::VSTR;
    constexpr int KTILE = TL::KTILE;
    constexpr int STAGE = TL::STAGE;
    constexpr int CHUNKS = BN * D / 4;
    constexpr int CPT = CHUNKS / kThreads32;
    constexpr int NDC = D / 4;
    static_assert(CHUNKS % kThreads32 == 0, "tile must split evenly over the workgroup");

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, r = lane & 31;
    const int b = bh / a.H, h = bh - b * a.H;
    const float* __restrict__ Qp = (const float*)a.q + b * a.q_sb + h * a.q_sh;
    const float* __restrict__ Kp = (const float*)a.k + b * a.k_sb + h * a.k_sh;
    const float* __restrict__ Vp = (const float*)a.v + b * a.v_sb + h * a.v_sh;
    const int q0 = qt * kBlockM32;
    const int qw0 = q0 + wave * kQueriesPerWave;
    const int my_q = qw0 + r;

    // Q^T operand: lane holds Q[my_q][g*D/2 + s]; rows past M and columns at
    // or past a.D (the kernel's D is the head dim rounded up) are zero
    float qf[D / 2];
    {
        const float* qrow = Qp + (int64_t)my_q * a.q_sm + g * (D / 2);
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
            f32x4 u = {0.f, 0.f, 0.f, 0.f};
            if (my_q < a.M && g * (D / 2) + 4 * c < a.D) u = *(const f32x4*)(qrow + 4 * c);
#pragma unroll
            for (int t = 0; t < 4; ++t) qf[4 * c + t] = u[t];
        }
    }

    int ntiles;
    const int* list = nullptr;
    if (LISTS && a.tile_counts != nullptr) {
        ntiles = a.tile_counts[qt];
        list = a.tile_entries + (int64_t)qt * a.num_k_tiles;
    } else {
        const int kend = a.causal ? min(a.N, q0 + kBlockM32) : a.N;
        ntiles = (kend + BN - 1) / BN;
    }
    // tile steps [it0, it1) of this workgroup's key split
    const int active = split_active(a, ntiles);
    if (split >= active) return;  // uniform over the workgroup
    const int range = split_range(a, ntiles);
    const int it0 = split * range;
    const int it1 = min(ntiles, it0 + range);

    f32x4 kreg[CPT], vreg[CPT];
    auto load_tile = [&](int kt) {
        const int k0 = kt * BN;
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int ci = tid + kThreads32 * u;
            const int row = ci / NDC, cc = ci % NDC;
            const int kj = k0 + row;
            kreg[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            vreg[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            // columns past the head dims stay zero
            if (kj < a.N && 4 * cc < a.D) kreg[u] = *(const f32x4*)(Kp + (int64_t)kj * a.k_sn + 4 * cc);
            if (kj < a.N && 4 * cc < a.Dv) vreg[u] = *(const f32x4*)(Vp + (int64_t)kj * a.v_sn + 4 * cc);
        }
    };
    auto store_tile = [&](int buf) {
        float* Ks = lds + buf * STAGE;
        float* Vs = Ks + KTILE;
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int ci = tid + kThreads32 * u;
            const int row = ci / NDC, cc = ci % NDC;
            *(f32x4*)(Ks + row * KSTR + 4 * cc) = kreg[u];
            *(f32x4*)(Vs + row * VSTR + 4 * cc) = vreg[u];
        }
    };
    auto tile_at = [&](int it, int& ent) -> int {
        if (list != nullptr) {
            ent = list[it];
            return list_tile(ent);
        }
        ent = 0;
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

    if (it0 < it1) {
        int e0;
        load_tile(tile_at(it0, e0));
    }
    wait_vm_loads();
    if (it0 < it1) store_tile(0);
    __syncthreads();

    for (int it = it0; it < it1; ++it) {
        int ent;
        const int kt = tile_at(it, ent);
        if (it + 1 < it1) {
            int en;
            load_tile(tile_at(it + 1, en));
        }
        const float* Ks = lds + ((it - it0) & 1) * STAGE;
        const float* Vs = Ks + KTILE;
        const int k0 = kt * BN;
        const bool active = list != nullptr ? list_any(ent, wave)
                                            : !(a.causal && k0 > qw0 + kQueriesPerWave - 1);
        if (active) {
            const bool need_mask = ((k0 + BN > a.N) || (a.causal && k0 + BN - 1 > qw0)) ||
                                   (list != nullptr && !list_full(ent, wave));
            f32x16 s[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) s[b] = f32x16{};
            const float* krow = Ks + kappa(r) * KSTR + g * (D / 2);
#pragma unroll
            for (int c = 0; c < D / 8; ++c) {
                f32x4 kv[NB];
#pragma unroll
                for (int b = 0; b < NB; ++b) kv[b] = *(const f32x4*)(krow + 32 * b * KSTR + 4 * c);
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        s[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[b][t], qf[4 * c + t], s[b], 0, 0, 0);
            }
            const float alpha = online_softmax_tile<NB, GENERAL>(a, s, need_mask, my_q, k0, g, slope,
                                                                 bias_row, m_run, l_run);
#pragma unroll
            for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const float* vrow = Vs + (32 * b + acc_pos(u, g)) * VSTR + r;
#pragma unroll
                    for (int db = 0; db < D / 32; ++db)
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * db], s[b][u], o[db], 0, 0, 0);
                }
        }
        if (it + 1 < it1) store_tile((it + 1 - it0) & 1);
        __syncthreads();
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
    if (active > 1) {
        // partial row: unnormalised O and (m, l), merged by the last split to arrive
        if (my_q < a.M) {
            const int64_t prow = ((int64_t)split * a.B * a.H + bh) * a.M + my_q;
            float* po = a.part_o + prow * a.Dv + 4 * g;
            const bool coh = a.split_counters != nullptr;
#pragma unroll
            for (int db = 0; db < D / 32; ++db) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (32 * db + 8 * i + 4 * g >= a.Dv) continue;  // past the value dim
                    f32x4 val;
#pragma unroll
                    for (int j = 0; j < 4; ++j) val[j] = o[db][4 * i + j];
                    put_partial4(po + 32 * db + 8 * i, val, coh);
                }
            }
            if (g == 0) {
                put_partial(a.part_ml + 2 * prow, m_run, coh);
                put_partial(a.part_ml + 2 * prow + 1, l_tot, coh);
            }
        }
        if (a.split_counters == nullptr) return;  // merged by combine_splits_kernel
        __syncthreads();                          // LDS below is reused
        static_assert(2 * STAGE * 4 >= 24 * kThreads32 + 4, "split merge scratch fits in the LDS stages");
        int* flag = (int*)(lds + 6 * kThreads32);
        if (split_arrive(a.split_counters + (int64_t)bh * a.num_q_tiles + qt, active, flag))
            merge_split_rows<float, kThreads32>(a, bh, q0, min(kBlockM32, a.M - q0), active, lds);
        return;
    }
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (my_q < a.M) {
        float* orow = (float*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)my_q * a.o_sm + 4 * g;
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (32 * db + 8 * i + 4 * g >= a.Dv) continue;  // past the value dim
                f32x4 val;
#pragma unroll
                for (int j = 0; j < 4; ++j) val[j] = o[db][4 * i + j] * inv;
                *(f32x4*)(orow + 32 * db + 8 * i) = val;
            }
        }
    }
}

// PAIRS_ONLY: causal calls without a block mask, which always run query tile
// pairs: an instantiation without the unpaired and list paths, whose values
// then stay out of its scalar registers (57 -> 10 spilled at D = 64; +1 %).
template <int D, bool GENERAL, int NB = 1, bool PAIRS_ONLY = false>
__global__ __launch_bounds__(kThreads32) void flash_fwd_mfma32_kernel(FwdArgs a) {
    __shared__ __attribute__((aligned(16))) float lds[2 * Mfma32Tiles<D, NB>::STAGE];
    if (PAIRS_ONLY || a.pair_split) {  // causal query tile pairs, split s of both tiles
        const int pairs = a.B * a.H * ((a.num_q_tiles + 1) / 2);
        const int split = (int)blockIdx.x / pairs;
        int bh, qa, qb;
        map_work_pair((int)blockIdx.x - split * pairs, a.B * a.H, a.num_q_tiles, bh, qa, qb);
        mfma32_qtile<D, GENERAL, NB, !PAIRS_ONLY>(a, lds, bh, qa, split);
        if (qb >= 0) {
            __syncthreads();  // LDS stages are reused
            mfma32_qtile<D, GENERAL, NB, !PAIRS_ONLY>(a, lds, bh, qb, split);
        }
        return;
    }
    int bh, qt;
    const int tiles_per_split = a.B * a.H * a.num_q_tiles;
    const int split = (int)blockIdx.x / tiles_per_split;
    map_work((int)blockIdx.x - split * tiles_per_split, a.B * a.H, a.num_q_tiles, a.causal, bh, qt);
    mfma32_qtile<D, GENERAL, NB>(a, lds, bh, qt, split);
}

// fp32 calls with few query rows (latency-bound: fewer 128-row query tiles
// than CUs). A workgroup of four wavefronts covers one 32-row query block and
// the wavefronts take its 32-key tiles in turn (wavefront w: steps it0 + w,
// it0 + w + 4, ...), so four times as many wavefronts share the work as in
// the 128-row kernel. Each keeps its own running (m, l, O) and reads its K and
// V tiles straight from global memory into the MFMA operand registers (no LDS
// staging, no barrier in the loop); at the end the four states are folded
// through LDS with the log-sum-exp rule (attention.cpp:661-674). Key splits
// across workgroups, and their merge, are those of the 128-row kernel.
template <int D, bool GENERAL>
__global__ __launch_bounds__(kThreads32) void flash_fwd_f32_rows32_kernel(FwdArgs a) {
    constexpr int NO = D / 2;  // O floats per lane
    constexpr int FS = NO + 2;  // folded floats per lane: O, m, l
    __shared__ __attribute__((aligned(16))) float fold[3 * FS * 64];
    static_assert(3 * FS * 64 >= 6 * kThreads32 + 1, "split merge scratch fits in the fold buffer");

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, r = lane & 31;
    int bh, qt;
    const int tiles_per_split = a.B * a.H * a.num_q_tiles;
    const int split = (int)blockIdx.x / tiles_per_split;
    map_work((int)blockIdx.x - split * tiles_per_split, a.B * a.H, a.num_q_tiles, a.causal, bh, qt);
    const int b = bh / a.H, h = bh - b * a.H;
    const float* __restrict__ Qp = (const float*)a.q + b * a.q_sb + h * a.q_sh;
    const float* __restrict__ Kp = (const float*)a.k + b * a.k_sb + h * a.k_sh;
    const float* __restrict__ Vp = (const float*)a.v + b * a.v_sb + h * a.v_sh;
    const int q0 = qt * kRowsF32;
    const int my_q = q0 + r;

    const int kend = a.causal ? min(a.N, q0 + kRowsF32) : a.N;
    const int ntiles = (kend + kBlockNF32 - 1) / kBlockNF32;
    const int active = split_active(a, ntiles);
    if (split >= active) return;  // uniform over the workgroup
    const int it0 = split * a.split_tiles;
    const int it1 = min(ntiles, it0 + a.split_tiles);

    // Q^T operand: lane holds Q[my_q][g*D/2 + s] (rows past M: zero)
    float qf[D / 2];
    {
        const float* qrow = Qp + (int64_t)min(my_q, a.M - 1) * a.q_sm + g * (D / 2);
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
            f32x4 u = {0.f, 0.f, 0.f, 0.f};
            // columns at or past a.D (the kernel's D rounds the head dim up) are zero
            if (g * (D / 2) + 4 * c < a.D) u = *(const f32x4*)(qrow + 4 * c);
            if (my_q >= a.M) u = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) qf[4 * c + t] = u[t];
        }
    }
    f32x16 o[D / 32];
#pragma unroll
    for (int db = 0; db < D / 32; ++db) o[db] = f32x16{};
    float m_run = kNegInf, l_run = 0.0f;
    const float slope = (GENERAL && a.bias_kind == BIAS_ALIBI) ? a.alibi[h] : 0.0f;
    const float* bias_row = nullptr;
    if (GENERAL && a.bias_kind == BIAS_DENSE && my_q < a.M)
        bias_row = a.bias + b * a.bias_sb + h * a.bias_sh + (int64_t)my_q * a.bias_sm;

    // K/V operand registers of tile it (A operands of S^T = K Q^T and of
    // O^T += V^T P^T): K[k0 + kappa(r)][g*D/2 + s] and V[k0 + acc_pos(u, g)][r + 32 db].
    // Rows past N read row N-1 (their scores are masked) and V past N is zero.
    // Up to D = 64 the next tile of the wavefront is loaded while this one is
    // computed (registers allow two sets).
    constexpr bool PREFETCH = D <= 64;
    struct KV {
        f32x4 k[D / 8];
        float v[16][D / 32];
    };
    auto load_kv = [&](int it, KV& t) {
        const int k0 = it * kBlockNF32;
        const float* krow = Kp + (int64_t)min(k0 + kappa(r), a.N - 1) * a.k_sn + g * (D / 2);
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
            t.k[c] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (g * (D / 2) + 4 * c < a.D) t.k[c] = *(const f32x4*)(krow + 4 * c);
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int kj = k0 + acc_pos(u, g);
            const float* vrow = Vp + (int64_t)min(kj, a.N - 1) * a.v_sn + r;
#pragma unroll
            for (int db = 0; db < D / 32; ++db) {
                float x = 0.0f;
                if (r + 32 * db < a.Dv) x = vrow[32 * db];
                t.v[u][db] = kj < a.N ? x : 0.0f;
            }
        }
    };
    auto compute = [&](int it, const KV& t) {
        const int k0 = it * kBlockNF32;
        f32x16 s[1] = {f32x16{}};
#pragma unroll
        for (int c = 0; c < D / 8; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                s[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(t.k[c][j], qf[4 * c + j], s[0], 0, 0, 0);
        const bool need_mask = (k0 + kBlockNF32 > a.N) || (a.causal && k0 + kBlockNF32 - 1 > q0);
        const float alpha =
            online_softmax_tile<1, GENERAL>(a, s, need_mask, my_q, k0, g, slope, bias_row, m_run, l_run);
#pragma unroll
        for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
#pragma unroll
        for (int u = 0; u < 16; ++u)
#pragma unroll
            for (int db = 0; db < D / 32; ++db)
                o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(t.v[u][db], s[0][u], o[db], 0, 0, 0);
    };
    if constexpr (PREFETCH) {
        KV cur, nxt;
        int it = it0 + wave;
        if (it < it1) load_kv(it, cur);
        for (; it < it1; it += kWaves32) {
            const bool more = it + kWaves32 < it1;
            if (more) load_kv(it + kWaves32, nxt);
            compute(it, cur);
            if (more) cur = nxt;
        }
    } else {
        for (int it = it0 + wave; it < it1; it += kWaves32) {
            KV cur;
            load_kv(it, cur);
            compute(it, cur);
        }
    }

    // Fold wavefronts 1-3 into wavefront 0 (the four hold the same rows in the
    // same lane layout); a wavefront that saw no tile has m = -inf, l = 0, O = 0.
    if (wave > 0) {
        float* f = fold + (wave - 1) * FS * 64 + lane;
#pragma unroll
        for (int i = 0; i < NO; ++i) f[64 * i] = o[i >> 4][i & 15];
        f[64 * NO] = m_run;
        f[64 * (NO + 1)] = l_run;
    }
    __syncthreads();
    if (wave == 0) {
        float mg = m_run;
#pragma unroll
        for (int w = 0; w < kWaves32 - 1; ++w) mg = fmaxf(mg, fold[w * FS * 64 + 64 * NO + lane]);
        const float mu = mg == kNegInf ? 0.0f : mg;
        const float w0 = __builtin_amdgcn_exp2f(m_run - mu);  // 0 while m_run is -inf
        l_run *= w0;
#pragma unroll
        for (int db = 0; db < D / 32; ++db) o[db] *= w0;
#pragma unroll
        for (int w = 0; w < kWaves32 - 1; ++w) {
            const float* f = fold + w * FS * 64 + lane;
            const float ww = __builtin_amdgcn_exp2f(f[64 * NO] - mu);
            l_run += ww * f[64 * (NO + 1)];
#pragma unroll
            for (int i = 0; i < NO; ++i) o[i >> 4][i & 15] += ww * f[64 * i];
        }
        m_run = mg;
    }
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    if (active > 1) {
        // partial row: unnormalised O and (m, l), merged by the last split to arrive
        const bool coh = a.split_counters != nullptr;
        if (wave == 0 && my_q < a.M) {
            const int64_t prow = ((int64_t)split * a.B * a.H + bh) * a.M + my_q;
            float* po = a.part_o + prow * a.Dv + 4 * g;
#pragma unroll
            for (int db = 0; db < D / 32; ++db) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (32 * db + 8 * i + 4 * g >= a.Dv) continue;  // past the value dim
                    f32x4 val;
#pragma unroll
                    for (int j = 0; j < 4; ++j) val[j] = o[db][4 * i + j];
                    put_partial4(po + 32 * db + 8 * i, val, coh);
                }
            }
            if (g == 0) {
                put_partial(a.part_ml + 2 * prow, m_run, coh);
                put_partial(a.part_ml + 2 * prow + 1, l_tot, coh);
            }
        }
        if (!coh) return;  // merged by combine_splits_kernel
        __syncthreads();   // the fold buffer below is reused
        int* flag = (int*)(fold + 6 * kThreads32);
        if (split_arrive(a.split_counters + (int64_t)bh * a.num_q_tiles + qt, active, flag))
            merge_split_rows<float, kThreads32>(a, bh, q0, min(kRowsF32, a.M - q0), active, fold);
        return;
    }
    if (wave == 0 && my_q < a.M) {
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        float* orow = (float*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)my_q * a.o_sm + 4 * g;
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (32 * db + 8 * i + 4 * g >= a.Dv) continue;  // past the value dim
                f32x4 val;
#pragma unroll
                for (int j = 0; j < 4; ++j) val[j] = o[db][4 * i + j] * inv;
                *(f32x4*)(orow + 32 * db + 8 * i) = val;
            }
        }
    }
}

// One 32-key tile of online softmax on two 16x16 score blocks (keys k0 + 16 kb
// + 4 kq + i of query my_q in register i of block kb), in place; the four
// lanes of a query (kq = 0..3) exchange their maxima. Returns alpha.
template <bool GENERAL>
__device__ __forceinline__ float online_softmax_16(const FwdArgs& a, f32x4 (&s)[2], bool need_mask, int my_q,
                                                   int k0, int kq, float slope, const float* bias_row,
                                                   float& m_run, float& l_run) {
    float mx = kNegInf;
    const bool row_out = GENERAL && my_q >= a.M;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kj = k0 + 16 * kb + 4 * kq + i;
            float x;
            if (!GENERAL && !need_mask) {
                x = s[kb][i] * a.scale_log2;
            } else {
                x = kNegInf;
                if (!(row_out || (need_mask && elem_masked(a, my_q, kj))))
                    x = GENERAL ? general_score(a, s[kb][i], my_q, kj, slope, bias_row) : s[kb][i] * a.scale_log2;
            }
            s[kb][i] = x;
            mx = fmaxf(mx, x);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == kNegInf) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float lsum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(s[kb][i] - m_use);
            s[kb][i] = p;
            lsum += p;
        }
    }
    l_run = l_run * alpha + lsum;
    return alpha;
}

// fp32 calls with few query rows and few keys: 16-row query blocks, one
// workgroup of sixteen wavefronts per block (one workgroup per CU), no key
// split, so no partial rows leave the CU. Wavefront w takes the block's
// 32-key tiles w, w + 16, ... on v_mfma_f32_16x16x4f32: its K tile copied
// into LDS, its V tile read straight into the operand registers, the block's
// Q rows read once per workgroup through LDS; the sixteen (m, l, O) states
// are folded through LDS with the log-sum-exp rule (attention.cpp:661-674).
//
// Operand layout (lane l: n = l % 16, kq = l / 16). The head dim is permuted
// inside each contraction, which leaves every sum unchanged:
//   S^T = K Q^T: instruction c = 4 cc + t (< D/4) contracts over d = 16 cc +
//     4 kq + t, so lane l holds K[key][16 cc + 4 kq, +4) and Q[q0 + n][16 cc
//     + 4 kq, +4) as one 16-byte chunk per cc (the four lanes of a row read
//     64 contiguous bytes); score block kb lands as
//     S^T[k0 + 16 kb + 4 kq + i][q0 + n] in register i.
//   O^T += V^T P^T: instruction (kb, i) contracts over keys k0 + 16 kb +
//     4 kq + i, whose probability is the lane's own register i of block kb;
//     output block db holds d = (D/16) m + db in row m, so lane l reads
//     V[key][(D/16) n, +D/16) in one load, and holds O[q0 + n][(D/4) kq, +D/4)
//     with d = (D/4) kq + e in element e = (D/16) i + db.
constexpr int kWavesRows16 = 16;
constexpr int kThreadsRows16 = kWavesRows16 * 64;

template <int D, bool GENERAL>
__global__ __launch_bounds__(kThreadsRows16) void flash_fwd_f32_rows16_kernel(FwdArgs a) {
    static_assert(D == 32 || D == 64, "16-row fp32 blocks: D = 32 or 64");
    constexpr int NC = D / 4;   // contraction floats per lane of S^T, O floats per lane
    constexpr int NDB = D / 16;  // 16-row blocks of O^T
    typedef float vrow_t __attribute__((ext_vector_type(NDB)));
    constexpr int QSTR = D + 4;  // LDS row stride of the Q block (16 rows at distinct banks)
    constexpr int CPR = D / 4;   // 16-byte chunks per K row
    constexpr int KT = kBlockNF32 * D;  // floats of one wavefront's K tile in LDS
    static_assert(64 * NC <= KT, "a wavefront's folded state fits in its K tile");
    // K tiles, one per wavefront (later its folded state); Q block; (m, l) per wavefront and query
    __shared__ __attribute__((aligned(16))) float k_lds[kWavesRows16 * KT];
    __shared__ float fold_ml[kWavesRows16 * 32];
    __shared__ __attribute__((aligned(16))) float q_lds[kRowsF32Narrow * QSTR];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, kq = lane >> 4;
    int bh, qt;
    map_work((int)blockIdx.x, a.B * a.H, a.num_q_tiles, a.causal, bh, qt);
    const int b = bh / a.H, h = bh - b * a.H;
    const float* __restrict__ Qp = (const float*)a.q + b * a.q_sb + h * a.q_sh;
    const float* __restrict__ Kp = (const float*)a.k + b * a.k_sb + h * a.k_sh;
    const float* __restrict__ Vp = (const float*)a.v + b * a.v_sb + h * a.v_sh;
    const int q0 = qt * kRowsF32Narrow;
    const int my_q = q0 + n;
    const int kend = a.causal ? min(a.N, q0 + kRowsF32Narrow) : a.N;
    const int ntiles = (kend + kBlockNF32 - 1) / kBlockNF32;

    // K tile it is copied into the wavefront's LDS tile (global -> LDS, 1 KB
    // of whole rows per instruction); chunk c of row r sits at slot
    // c ^ kswz(r), so that the operand reads (16 rows at one chunk per 16
    // lanes) meet distinct banks. V is read straight into the operand
    // registers once the K operands are consumed. Rows past N read row N-1
    // (their scores are masked, so their probabilities are exactly 0); K
    // chunks past D re-read the row's last chunk (Q is zero there), V columns
    // past Dv its last columns (those output rows are not stored).
    float* const kw = k_lds + wave * KT;
    auto kswz = [](int r) { return D == 64 ? (r & 15) : ((r >> 1) & 7); };
    auto load_k = [&](int it) {
        const unsigned base = (unsigned)(uintptr_t)kw;
#pragma unroll
        for (int j = 0; j < KT / 256; ++j) {
            const int sl = 64 * j + lane, r = sl / CPR, c = (sl % CPR) ^ kswz(r);
            dma16(Kp + (int64_t)min(it * kBlockNF32 + r, a.N - 1) * a.k_sn + min(4 * c, a.D - 4), base + 1024 * j);
        }
    };
    vrow_t vf[2][4];
    auto load_v = [&](int it) {
        const int vc = min(NDB * n, a.Dv - NDB);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                vf[kb][i] = *(const vrow_t*)(Vp + (int64_t)min(it * kBlockNF32 + 16 * kb + 4 * kq + i, a.N - 1) *
                                                       a.v_sn + vc);
    };
    // The Q block is read by the first 4 D threads (one 16-byte chunk each;
    // rows past M and chunks past D are zero), after which the wavefront's
    // first K tile is requested, and staged through LDS.
    f32x4 qv = {0.f, 0.f, 0.f, 0.f};
    const int qr = tid / (D / 4), qc = 4 * (tid - qr * (D / 4));
    if (tid < 4 * D) {
        qv = *(const f32x4*)(Qp + (int64_t)min(q0 + qr, a.M - 1) * a.q_sm + min(qc, a.D - 4));
        if (q0 + qr >= a.M || qc >= a.D) qv = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (wave < ntiles) load_k(wave);
    if (tid < 4 * D) *(f32x4*)(q_lds + qr * QSTR + qc) = qv;
    __syncthreads();
    float qf[NC];  // Q[my_q][16 cc + 4 kq + t] at 4 cc + t
#pragma unroll
    for (int cc = 0; cc < NC / 4; ++cc) {
        const f32x4 u = *(const f32x4*)(q_lds + n * QSTR + 16 * cc + 4 * kq);
#pragma unroll
        for (int t = 0; t < 4; ++t) qf[4 * cc + t] = u[t];
    }
    f32x4 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf, l_run = 0.0f;
    const float slope = (GENERAL && a.bias_kind == BIAS_ALIBI) ? a.alibi[h] : 0.0f;
    const float* bias_row = nullptr;
    if (GENERAL && a.bias_kind == BIAS_DENSE && my_q < a.M)
        bias_row = a.bias + b * a.bias_sb + h * a.bias_sh + (int64_t)my_q * a.bias_sm;

    for (int it = wave; it < ntiles; it += kWavesRows16) {
        const int k0 = it * kBlockNF32;
        if (it != wave) load_k(it);
        wait_vm_loads();  // this wavefront's K copy has landed
        f32x4 kf[2][NC / 4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int cc = 0; cc < NC / 4; ++cc)
                kf[kb][cc] = *(const f32x4*)(kw + (16 * kb + n) * D + 4 * ((4 * cc + kq) ^ kswz(16 * kb + n)));
        f32x4 s[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kb][c >> 2][c & 3], qf[c], s[kb], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_v(it);
        const bool need_mask = (k0 + kBlockNF32 > a.N) || (a.causal && k0 + kBlockNF32 - 1 > q0);
        const float alpha =
            online_softmax_16<GENERAL>(a, s, need_mask, my_q, k0, kq, slope, bias_row, m_run, l_run);
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db] *= alpha;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int db = 0; db < NDB; ++db)
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[kb][i][db], s[kb][i], o[db], 0, 0, 0);
    }

    // Every wavefront (one that saw no tile has m = -inf, l = 0, O = 0) leaves
    // its O in d order (in its K tile, whose reads are done) and the (m, l)
    // of its 16 queries in LDS.
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    {
        float* f = kw + lane * NC;
#pragma unroll
        for (int c = 0; c < NC / 4; ++c) {
            f32x4 val;
#pragma unroll
            for (int t = 0; t < 4; ++t) val[t] = o[(4 * c + t) % NDB][(4 * c + t) / NDB];
            *(f32x4*)(f + 4 * c) = val;
        }
        if (kq == 0) {
            fold_ml[wave * 32 + n] = m_run;
            fold_ml[wave * 32 + 16 + n] = l_run;
        }
    }
    __syncthreads();
    // Thread t folds 4 output columns: lane slot L = t / (NC / 4), chunk t % (NC / 4).
    if (tid < 64 * (NC / 4)) {
        const int L = tid / (NC / 4), c = tid - L * (NC / 4);
        const int qn = L & 15, kqL = L >> 4;
        float mg = kNegInf;
#pragma unroll
        for (int w = 0; w < kWavesRows16; ++w) mg = fmaxf(mg, fold_ml[w * 32 + qn]);
        const float mu = mg == kNegInf ? 0.0f : mg;
        float l = 0.0f;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < kWavesRows16; ++w) {
            const float ww = __builtin_amdgcn_exp2f(fold_ml[w * 32 + qn] - mu);  // 0 for m = -inf
            l += ww * fold_ml[w * 32 + 16 + qn];
            acc += ww * *(const f32x4*)(k_lds + w * KT + L * NC + 4 * c);
        }
        const int q = q0 + qn, d = NC * kqL + 4 * c;
        if (q < a.M && d < a.Dv) {
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            *(f32x4*)((float*)a.o + b * a.o_sb + h * a.o_sh + (int64_t)q * a.o_sm + d) = acc * inv;
        }
    }
}

// Merge of key-split partial rows in a launch of its own (no arrival
// counters). A workgroup merges `rows` consecutive rows of one head (a power
// of two, so they lie in one query tile): thread t takes (row, 4-column chunk)
// item t % (rows * chunks) and the splits grp, grp + groups, ... with
// grp = t / (rows * chunks), so that a row's splits are read by `groups`
// threads at once; the groups' results are folded through LDS. T is the
// input type (the output type unless out_f32).
template <typename T>
__global__ __launch_bounds__(256) void combine_splits_kernel(FwdArgs a, int rows, int groups) {
    __shared__ float red[6 * 256];
    const int chunks = a.Dv >> 2;
    const int per_head = (a.M + rows - 1) / rows;
    const int bh = (int)blockIdx.x / per_head;
    const int row0 = ((int)blockIdx.x - bh * per_head) * rows;
    const int qt = row0 / a.split_bm;
    int steps;
    if (a.tile_counts != nullptr) {
        steps = a.tile_counts[qt];
    } else {
        const int kend = a.causal ? min(a.N, (qt + 1) * a.split_bm) : a.N;
        steps = (kend + a.split_bn - 1) / a.split_bn;
    }
    const int active = split_active(a, steps);
    if (active <= 1) return;  // split 0 wrote these rows (uniform over the workgroup)
    const int items = rows * chunks;  // items * groups <= 256
    const int t = threadIdx.x;
    const int item = t % items, grp = t / items;
    const int rr = item / chunks, c = item - rr * chunks;
    const int row = row0 + rr;
    const int ng = min(groups, active);
    const bool mine = grp < ng && row < a.M;
    float m = kNegInf, l = 0.0f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (mine) merge_partials<false>(a, (int64_t)bh * a.M + row, c, grp, ng, active, m, l, acc);
    if (ng > 1) {
        if (mine && grp > 0) {
            float* e = red + 6 * t;
            e[0] = m;
            e[1] = l;
#pragma unroll
            for (int j = 0; j < 4; ++j) e[2 + j] = acc[j];
        }
        __syncthreads();
        if (mine && grp == 0)
            for (int j = 1; j < ng; ++j) {
                const float* e = red + 6 * (j * items + item);
                lse_fold(m, l, acc, e[0], e[1], f32x4{e[2], e[3], e[4], e[5]});
            }
    }
    if (mine && grp == 0) store_merged<T>(a, bh, row, c, l, acc);
}

template <typename K>
hipError_t launch(K kernel, int threads, const FwdArgs& a, hipStream_t s, bool paired = false, size_t lds = 0) {
    const int64_t grid = (int64_t)a.B * a.H * (paired ? (a.num_q_tiles + 1) / 2 : a.num_q_tiles) * a.num_splits;
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(threads), lds, s, a);
    return hipGetLastError();
}

}  // namespace

// 16-bit kernel workgroups: 8 wavefronts (256 query rows) without a
// block-mask list, 4 wavefronts (128 rows, finer skipping) with one, and 4
// wavefronts from D = 192 up (register file), except without score_mod at
// D = 192, where O (96 registers), Q (48) and a 64-key score tile fit two
// wavefronts per SIMD, and at D = 256 with 32-key compute steps (64 keys
// staged; 34-54 VGPRs spilled): 8 wavefronts there whenever the 4-wavefront
// grid (one workgroup per CU) would take more than one round of the CUs (B4
// H32 N4096, D = 192: 0.81 against 1.21 ms causal, 1.44 against 2.22 ms
// non-causal, bit-identical; D = 256: 1.41 against 1.45 ms causal, 2.59
// against 2.82 ms non-causal; bf16 B1 H24 N2048 D192 non-causal, 192
// workgroups of 8 against 384 of 4: 80 against 141 us), 4 on calls that one
// round holds (whose 4-wavefront grid or key split runs faster: bf16 causal
// B2 H16 N2048 D192 84 against 99 us with 8 wavefronts and a pair split, B1
// H8 N2048 43 against 59 us). The 8-wavefront grid then never takes a key
// split: it has more than half as many workgroups as CUs.
static bool eight_waves_wide(bool causal, int64_t bh, int64_t query_tokens) {
    const int64_t nqt4 = (query_tokens + 127) / 128;
    return bh * (causal ? (nqt4 + 1) / 2 : nqt4) > kComputeUnits;
}

// Causal calls without a block-mask list pair query tiles per workgroup.
static bool pairs_causal_tiles(bool causal, bool tile_list) { return causal && !tile_list; }

// Keys per staged K/V tile (one barrier each) of a 16-bit call: 128 without
// score_mod or block mask (half the barriers and tile stores per key), else 64
// (with a block mask a wider tile skips at a coarser grain; the score_mod
// kernel holds all fragments of a tile). At D = 64 the 128 keys are one compute
// step (+9 to +13 %); at D = 128, where S and P for 128 keys would spill, they
// are computed in two 64-key steps between the same barriers (+1 to +5 %).
// D = 32 stages 128 keys in every kernel without a block mask (a 64-key tile
// of 64-byte rows is fewer 16-byte chunks than the 8 wavefronts copy), as do
// D = 96 and 160 (their 64-key tiles do not split evenly over 512 threads);
// D > 160 runs 64-key tiles throughout, on 4 wavefronts (128 query rows) or,
// at D = 192 and 256 without score_mod, 8 (two 32-key compute steps per
// staged tile at D = 256).
static int block_n16(int D, bool general_mod, bool tile_list) {
    if (D > 160 || tile_list) return kBlockN16;
    if (D == 32 || D == 96 || D == 160) return kBlockN16Wide;
    return !general_mod ? kBlockN16Wide : kBlockN16;
}

// LDS of the 16-bit block-mask kernel (4 wavefronts, 64-key tiles): two
// stages with the tile_list kernel's global list, or lds_list_stages stages,
// the per-wavefront counts and the list itself with a list built in LDS.
template <int D>
static size_t list_kernel_lds_bytes_d(bool lds_list, int num_k_tiles) {
    using L = TileLayout<D, kBlockN16>;
    if (!lds_list) return 2 * (size_t)L::STAGE;
    return (size_t)lds_list_stages<D>() * L::STAGE + kLdsListCountsBytes + 4 * (size_t)num_k_tiles;
}

size_t list_kernel_lds_bytes(int D, bool lds_list, int num_k_tiles) {
    switch (D) {
        case 32: return list_kernel_lds_bytes_d<32>(lds_list, num_k_tiles);
        case 64: return list_kernel_lds_bytes_d<64>(lds_list, num_k_tiles);
        case 96: return list_kernel_lds_bytes_d<96>(lds_list, num_k_tiles);
        case 128: return list_kernel_lds_bytes_d<128>(lds_list, num_k_tiles);
        case 160: return list_kernel_lds_bytes_d<160>(lds_list, num_k_tiles);
        case 192: return list_kernel_lds_bytes_d<192>(lds_list, num_k_tiles);
        case 224: return list_kernel_lds_bytes_d<224>(lds_list, num_k_tiles);
        case 256: return list_kernel_lds_bytes_d<256>(lds_list, num_k_tiles);
        default: return 0;
    }
}

template <typename T, int D>
static hipError_t launch16(const FwdArgs& a, bool general_mod, hipStream_t s) {
    const bool list = a.mask != nullptr;
    const bool paired = pairs_causal_tiles(a.causal != 0, list) && a.num_splits == 1;
    if (list) {
        const size_t lds = list_kernel_lds_bytes(D, a.tile_counts == nullptr, a.num_k_tiles);
        if (a.tile_counts == nullptr && a.num_splits == 1)
            return general_mod ? launch(flash_fwd_lds_list_kernel<T, D, MOD_GENERAL>, 256, a, s, false, lds)
                               : launch(flash_fwd_lds_list_kernel<T, D, MOD_PLAIN>, 256, a, s, false, lds);
        return general_mod ? launch(flash_fwd_lockstep_kernel<T, D, MOD_GENERAL, true, 4, false>, 256, a, s, false, lds)
                           : launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, true, 4, false>, 256, a, s, false, lds);
    }
    const bool pair_split = a.pair_split != 0;
    if constexpr (D > 160) {
        if (general_mod) {
            if (pair_split) return launch(flash_fwd_pair_split_kernel<T, D, MOD_GENERAL, 4>, 256, a, s, true);
            return paired ? launch(flash_fwd_lockstep_kernel<T, D, MOD_GENERAL, false, 4, true>, 256, a, s, true)
                 : a.num_splits > 1 ? launch(flash_fwd_lockstep_kernel<T, D, MOD_GENERAL, false, 4, false>, 256, a, s)
                          : launch(flash_fwd_lockstep_kernel<T, D, MOD_GENERAL, false, 4, false, kBlockN16, 1, false>, 256, a, s);
        }
        if constexpr (D == 256) {  // 256-row query tiles: 8 wavefronts, 64 keys staged as two 32-key steps
            if (a.split_bm == 8 * kQueriesPerWave) {
                if (pair_split || a.num_splits > 1) return hipErrorInvalidValue;
                return paired ? launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, true, 32, 2>, 512, a, s, true)
                              : launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, false, 32, 2, false>, 512, a, s);
            }
        }
        if constexpr (D == 192) {  // 256-row query tiles: 8 wavefronts on 64-key tiles
            // (chosen only where its workgroups outnumber half the CUs, so never with a key split)
            if (a.split_bm == 8 * kQueriesPerWave) {
                if (pair_split || a.num_splits > 1) return hipErrorInvalidValue;
                if (a.Dv <= 128)  // value columns 128 (e.g. 192/128 query-key/value heads): PV over those only
                    return paired ? launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, true, kBlockN16, 1, true, 128>, 512, a, s, true)
                                  : launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, false, kBlockN16, 1, false, 128>, 512, a, s);
                return paired ? launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, true>, 512, a, s, true)
                              : launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, false, kBlockN16, 1, false>, 512, a, s);
            }
        }
        if (a.split_bm != 4 * kQueriesPerWave) return hipErrorInvalidValue;
        if (pair_split) return launch(flash_fwd_pair_split_kernel<T, D, MOD_PLAIN, 4>, 256, a, s, true);
        return paired ? launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 4, true>, 256, a, s, true)
             : a.num_splits > 1 ? launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 4, false>, 256, a, s)
                      : launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 4, false, kBlockN16, 1, false>, 256, a, s);
    } else {
        // score_mod: 64-key compute steps (two per staged tile at D = 32, 96, 160)
        constexpr int GSB = (D == 32 || (D & (D - 1)) != 0) ? 2 : 1;
        if (general_mod)
            return pair_split ? launch(flash_fwd_pair_split_kernel<T, D, MOD_GENERAL, 8, kBlockN16, GSB>, 512, a, s, true)
                 : paired ? launch(flash_fwd_lockstep_kernel<T, D, MOD_GENERAL, false, 8, true, kBlockN16, GSB>, 512, a, s, true)
                 : a.num_splits > 1 ? launch(flash_fwd_lockstep_kernel<T, D, MOD_GENERAL, false, 8, false, kBlockN16, GSB>, 512, a, s)
                          : launch(flash_fwd_lockstep_kernel<T, D, MOD_GENERAL, false, 8, false, kBlockN16, GSB, false>, 512, a, s);
        // D <= 64: 128-key tiles; D = 128: 128 keys staged per barrier, two 64-key compute steps
        constexpr int BN = D <= 64 ? kBlockN16Wide : kBlockN16;
        constexpr int SB = D <= 64 ? 1 : kBlockN16Wide / kBlockN16;
        if (pair_split) return launch(flash_fwd_pair_split_kernel<T, D, MOD_PLAIN, 8, BN, SB>, 512, a, s, true);
        return paired ? launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, true, BN, SB>, 512, a, s, true)
             : a.num_splits > 1 ? launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, false, BN, SB>, 512, a, s)
                      : launch(flash_fwd_lockstep_kernel<T, D, MOD_PLAIN, false, 8, false, BN, SB, false>, 512, a, s);
    }
}

// fp32 128-row query tiles: causal pairs without a block mask take the
// pairs-only instantiation. Above D = 128 a K/V tile is one block of 32 keys
// (two stages of 64-key tiles would not fit the LDS).
template <int D>
static hipError_t launch32(const FwdArgs& a, bool general_mod, hipStream_t s) {
    constexpr int NB = D > 128 ? 1 : kTilesF32;
    if (a.split_bn != kBlockNF32 * NB) return hipErrorInvalidValue;
    if (a.pair_split && a.tile_counts == nullptr)
        return general_mod ? launch(flash_fwd_mfma32_kernel<D, true, NB, true>, kThreads32, a, s, true)
                           : launch(flash_fwd_mfma32_kernel<D, false, NB, true>, kThreads32, a, s, true);
    return general_mod ? launch(flash_fwd_mfma32_kernel<D, true, NB>, kThreads32, a, s, a.pair_split != 0)
                       : launch(flash_fwd_mfma32_kernel<D, false, NB>, kThreads32, a, s, a.pair_split != 0);
}

hipError_t launch_flash_mfma(const FwdArgs& a, int dtype, bool general_mod, hipStream_t s) {
    // the kernel's head dim: D and Dv rounded up (the kernels zero-pad Q and
    // mask the stores past Dv)
    const int kd = flash_mfma_kernel_dim(dtype, a.D, a.Dv);
    if (dtype == DT_BF16 || dtype == DT_F16) {
        const bool f16 = dtype == DT_F16;
        switch (kd) {
            case 32: return f16 ? launch16<_Float16, 32>(a, general_mod, s) : launch16<__bf16, 32>(a, general_mod, s);
            case 64: return f16 ? launch16<_Float16, 64>(a, general_mod, s) : launch16<__bf16, 64>(a, general_mod, s);
            case 96: return f16 ? launch16<_Float16, 96>(a, general_mod, s) : launch16<__bf16, 96>(a, general_mod, s);
            case 128: return f16 ? launch16<_Float16, 128>(a, general_mod, s) : launch16<__bf16, 128>(a, general_mod, s);
            case 160: return f16 ? launch16<_Float16, 160>(a, general_mod, s) : launch16<__bf16, 160>(a, general_mod, s);
            case 192: return f16 ? launch16<_Float16, 192>(a, general_mod, s) : launch16<__bf16, 192>(a, general_mod, s);
            case 224: return f16 ? launch16<_Float16, 224>(a, general_mod, s) : launch16<__bf16, 224>(a, general_mod, s);
            case 256: return f16 ? launch16<_Float16, 256>(a, general_mod, s) : launch16<__bf16, 256>(a, general_mod, s);
            default: return hipErrorInvalidValue;
        }
    } else if (dtype == DT_F32) {
        if (a.split_bm == kRowsF32Narrow) {  // few query rows and keys: 16-row blocks, no key split
            if (a.tile_counts != nullptr || a.mask != nullptr || a.num_splits != 1) return hipErrorInvalidValue;
            switch (kd) {
                case 32: return general_mod ? launch(flash_fwd_f32_rows16_kernel<32, true>, kThreadsRows16, a, s)
                                            : launch(flash_fwd_f32_rows16_kernel<32, false>, kThreadsRows16, a, s);
                case 64: return general_mod ? launch(flash_fwd_f32_rows16_kernel<64, true>, kThreadsRows16, a, s)
                                            : launch(flash_fwd_f32_rows16_kernel<64, false>, kThreadsRows16, a, s);
                default: return hipErrorInvalidValue;
            }
        }
        if (a.split_bm == kRowsF32) {  // few query rows: 32-row blocks (no block mask)
            if (a.tile_counts != nullptr) return hipErrorInvalidValue;
            switch (kd) {
                case 32: return general_mod ? launch(flash_fwd_f32_rows32_kernel<32, true>, kThreads32, a, s)
                                            : launch(flash_fwd_f32_rows32_kernel<32, false>, kThreads32, a, s);
                case 64: return general_mod ? launch(flash_fwd_f32_rows32_kernel<64, true>, kThreads32, a, s)
                                            : launch(flash_fwd_f32_rows32_kernel<64, false>, kThreads32, a, s);
                case 96: return general_mod ? launch(flash_fwd_f32_rows32_kernel<96, true>, kThreads32, a, s)
                                            : launch(flash_fwd_f32_rows32_kernel<96, false>, kThreads32, a, s);
                case 128: return general_mod ? launch(flash_fwd_f32_rows32_kernel<128, true>, kThreads32, a, s)
                                             : launch(flash_fwd_f32_rows32_kernel<128, false>, kThreads32, a, s);
                default: return hipErrorInvalidValue;
            }
        }
        switch (kd) {
            case 32: return launch32<32>(a, general_mod, s);
            case 64: return launch32<64>(a, general_mod, s);
            case 96: return launch32<96>(a, general_mod, s);
            case 128: return launch32<128>(a, general_mod, s);
            case 160: return launch32<160>(a, general_mod, s);
            case 192: return launch32<192>(a, general_mod, s);
            case 224: return launch32<224>(a, general_mod, s);
            case 256: return launch32<256>(a, general_mod, s);
            default: break;
        }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_combine_splits(const FwdArgs& a, int dtype, hipStream_t s) {
    const int chunks = a.Dv / 4;
    if (a.B * a.H * a.M <= 0 || chunks <= 0 || chunks > 256 || a.split_bm <= 0) return hipErrorInvalidValue;
    // splits per row read in parallel: a thread keeps four splits' loads in
    // flight, so a group is added only while each would read more than four
    // (up to 8 groups: two rounds of four loads per thread for 64 splits);
    // rows per workgroup: a power of two dividing the query tile, with
    // rows * chunks * groups <= 256
    int groups = 1;
    while (groups < 8 && 4 * groups < a.num_splits && 2 * groups * chunks <= 256) groups *= 2;
    int rows = 1;
    while (2 * rows * chunks * groups <= 256 && 2 * rows <= a.split_bm && a.split_bm % (2 * rows) == 0) rows *= 2;
    const int64_t nblk = (int64_t)a.B * a.H * ((a.M + rows - 1) / rows);
    if (nblk > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)nblk);
    if (dtype == DT_F32 || a.out_f32) hipLaunchKernelGGL(combine_splits_kernel<float>, grid, dim3(256), 0, s, a, rows, groups);
    else if (dtype == DT_BF16) hipLaunchKernelGGL(combine_splits_kernel<__bf16>, grid, dim3(256), 0, s, a, rows, groups);
    else if (dtype == DT_F16) hipLaunchKernelGGL(combine_splits_kernel<_Float16>, grid, dim3(256), 0, s, a, rows, groups);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

namespace {
// Arrival counters of the single-launch key-split merge (see FwdArgs).
static __device__ __align__(256) unsigned split_counters[kSplitCounterSlots * kMaxSplitTiles];
std::mutex g_counter_mu;
std::map<int, unsigned*> g_counter_addr;  // device -> address of its copy of split_counters
}  // namespace

hipError_t split_counter_slot(int slot, unsigned** ptr) {
    if (slot < 0 || slot >= kSplitCounterSlots) return hipErrorInvalidValue;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_counter_mu);
    auto it = g_counter_addr.find(dev);
    if (it == g_counter_addr.end()) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(split_counters));
        if (e != hipSuccess) return e;
        it = g_counter_addr.emplace(dev, static_cast<unsigned*>(p)).first;
    }
    *ptr = it->second + (size_t)slot * kMaxSplitTiles;
    return hipSuccess;
}

bool flash_mfma_head_dim(int dtype, int D) {
    (void)dtype;  // every dtype: multiples of 32 up to 256
    return D % 32 == 0 && D >= 32 && D <= 256;
}

int flash_mfma_kernel_dim(int dtype, int D, int Dv) {
    const int unit = dtype == DT_F32 ? 4 : 8;  // elements per 16-byte row chunk
    if (D <= 0 || Dv <= 0 || D % unit != 0 || Dv % unit != 0) return 0;
    const int kd = (std::max(D, Dv) + 31) / 32 * 32;
    return flash_mfma_head_dim(dtype, kd) ? kd : 0;
}

const char* flash_mfma_kernel_name(int dtype, int D, bool general_mod, bool tile_list, int threads) {
    if (dtype < 0 || dtype > 2 || !flash_mfma_head_dim(dtype, D)) return "none";
    // [dtype][D / 32 - 1][score_mod][list][8 wavefronts]
    static const std::vector<std::string> names = [] {
        std::vector<std::string> v;
        const char* tn[3] = {"f32", "bf16", "f16"};
        for (int dt = 0; dt < 3; ++dt)
            for (int d = 32; d <= 256; d += 32)
                for (int mod = 0; mod < 2; ++mod)
                    for (int list = 0; list < 2; ++list)
                        for (int w8 = 0; w8 < 2; ++w8) {
                            std::string n;
                            if (dt == DT_F32) {
                                n = "flash_fwd_mfma32_kernel<" + std::to_string(d) + (mod ? ",general>" : ",plain>");
                            } else {
                                n = std::string("flash_fwd_lockstep_kernel<") + tn[dt] + "," + std::to_string(d) +
                                    (mod ? ",mod" : ",plain");
                                const bool pow2 = (d & (d - 1)) == 0;
                                if (list) n += ",list,4w>";
                                else if (d == 192 && !mod && w8) n += ",8w>";
                                else if (d == 256 && !mod && w8) n += ",8w,2x32keys>";
                                else if (d > 160) n += ",4w>";
                                else if (!mod && d <= 64) n += ",8w,128keys>";
                                else if (!mod) n += ",8w,2x64keys>";
                                else if (d == 32 || !pow2) n += ",8w,2x64keys>";
                                else n += ",8w>";
                            }
                            v.push_back(n);
                        }
        return v;
    }();
    const int di = D / 32 - 1;
    return names[((((size_t)dtype * 8 + di) * 2 + (general_mod ? 1 : 0)) * 2 + (tile_list ? 1 : 0)) * 2 +
                 (threads >= 512 ? 1 : 0)]
        .c_str();
}

MfmaTiles flash_mfma_tiles(int dtype, int D, bool general_mod, bool tile_list, bool causal, int64_t bh,
                           int64_t query_tokens) {
    if (dtype == DT_F32) return MfmaTiles{kBlockM32, kBlockNF32 * (D > 128 ? 1 : kTilesF32), kThreads32, false};
    const bool paired = pairs_causal_tiles(causal, tile_list);
    const int bn = block_n16(D, general_mod, tile_list);
    const bool four =
        tile_list || (D > 160 && !((D == 192 || D == 256) && !general_mod && eight_waves_wide(causal, bh, query_tokens)));
    if (four) return MfmaTiles{128, bn, 256, paired};
    return MfmaTiles{256, bn, 512, paired};
}

}  // namespace ofh
