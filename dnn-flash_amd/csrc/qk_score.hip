// QK score tile with post-ops on the device: S = (Q K^T) * scale + bias
// (+ soft-cap), for a batch of strided tiles.
//
// Follows the reference's QK score tile (src/onednn_flash/qk_score_tile.cpp:
// 48-69 post-ops after matmul_tile_strided_inplace, whose reference kernel
// sums over k sequentially in fp32, src/onednn_flash/tile_kernel.cpp:49-86).
// Every product and every partial sum is rounded once, in the same order, so
// fp32 results are bit-identical to the reference. 32x32 output blocks per
// workgroup; Q and K^T chunks of 32 along k are staged through LDS as fp32.
//
// For bf16/fp16 inputs a matrix-core variant computes the same scores with
// v_mfma_f32_32x32x16_{bf16,f16}: the products are exact in fp32 and only the
// summation order differs from the sequential sum (error within k * 2^-24 *
// sum_k |q k| per score). It needs rows contiguous along k and 16-byte aligned.

#include "ofh_kernels.h"

#include <algorithm>

namespace ofh {
namespace {

constexpr int kQkTile = 32;
constexpr int64_t kMaxGridZ = 65535;   // tiles per launch (grid z)

template <typename T>
__device__ __forceinline__ float to_f32(T x) { return (float)x; }

template <typename T>
__global__ __launch_bounds__(256) void qk_score_kernel(QkScoreArgs a) {
    // Products, sums, scale and bias are each rounded: no contraction to FMA.
#pragma clang fp contract(off)
    __shared__ float qs[kQkTile][kQkTile + 1];   // [row i][kk]
    __shared__ float ks[kQkTile][kQkTile + 1];   // [kk][col j]
    const int tid = threadIdx.x;
    const int tx = tid & 31, ty = tid >> 5;      // column, row group (8 groups of 4 rows)
    const int64_t bt = blockIdx.z;
    const int64_t i0 = (int64_t)blockIdx.y * kQkTile, j0 = (int64_t)blockIdx.x * kQkTile;
    const T* q = (const T*)a.q + bt * a.a_sb;
    const T* k = (const T*)a.k + bt * a.b_sb;
    const bool q_k_fast = a.a_sk <= a.a_sm, k_k_fast = a.b_sk <= a.b_sn;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t k0 = 0; k0 < a.K; k0 += kQkTile) {
        // Stage both chunks, zero outside the tile. Lanes walk whichever axis
        // has the smaller stride so that row-major Q [m,k] and K [n,k] (both
        // contiguous along k) are read with unit stride.
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = ty + 8 * u;
            if (q_k_fast) {
                const int64_t qi = i0 + r, qk = k0 + tx;
                qs[r][tx] = (qi < a.M && qk < a.K) ? to_f32(q[qi * a.a_sm + qk * a.a_sk]) : 0.0f;
            } else {
                const int64_t qi = i0 + tx, qk = k0 + r;
                qs[tx][r] = (qi < a.M && qk < a.K) ? to_f32(q[qi * a.a_sm + qk * a.a_sk]) : 0.0f;
            }
            if (k_k_fast) {
                const int64_t kk = k0 + tx, kj = j0 + r;
                ks[tx][r] = (kk < a.K && kj < a.N) ? to_f32(k[kk * a.b_sk + kj * a.b_sn]) : 0.0f;
            } else {
                const int64_t kk = k0 + r, kj = j0 + tx;
                ks[r][tx] = (kk < a.K && kj < a.N) ? to_f32(k[kk * a.b_sk + kj * a.b_sn]) : 0.0f;
            }
        }
        __syncthreads();
        const int kn = (int)min((int64_t)kQkTile, a.K - k0);
        for (int t = 0; t < kn; ++t) {
            const float b = ks[t][tx];
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[u] = acc[u] + qs[ty + 8 * u][t] * b;
        }
        __syncthreads();
    }
    const int64_t j = j0 + tx;
    if (j >= a.N) return;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t i = i0 + ty + 8 * u;
        if (i >= a.M) continue;
        float v = acc[u];
        if (a.has_scale) v = v * a.scale;
        if (a.bias != nullptr) v = v + a.bias[bt * a.bias_sb + i * a.bias_sm + j * a.bias_sn];
        if (a.softcap > 0.0f) v = a.softcap * tanhf(v / a.softcap);
        a.c[bt * a.c_sb + i * a.c_sm + j * a.c_sn] = v;
    }
}

typedef __bf16 qk_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 qk_f16x8 __attribute__((ext_vector_type(8)));
typedef float qk_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int qk_u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct QkMfma;
template <>
struct QkMfma<__bf16> {
    static __device__ __forceinline__ qk_f32x16 run(qk_u32x4 a, qk_u32x4 b, qk_f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(qk_bf16x8, a),
                                                       __builtin_bit_cast(qk_bf16x8, b), c, 0, 0, 0);
    }
};
template <>
struct QkMfma<_Float16> {
    static __device__ __forceinline__ qk_f32x16 run(qk_u32x4 a, qk_u32x4 b, qk_f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(qk_f16x8, a),
                                                      __builtin_bit_cast(qk_f16x8, b), c, 0, 0, 0);
    }
};

// 128x128 score block per workgroup, 4 wavefronts of 64x64 (2x2 MFMA tiles of
// 32x32). Operand lane layout of the 32x32x16 MFMA: lane l holds row (l & 31)
// of the A operand and column (l & 31) of the B operand, k elements
// 8*(l >> 5) .. +7 of the 16-wide step; output element e of lane l is row
// 8*(e >> 2) + 4*(l >> 5) + (e & 3), column l & 31. With A = K and B = Q^T
// the tile is S^T, so each lane owns runs of 4 consecutive keys of one query
// row: contiguous in the row-major score matrix.
constexpr int kMfmaBlock = 128;

// LDS of the matrix-core score kernel, 32 KB so that three workgroups fit a CU
// (their registers allow three). Unpadded rows (the DMA copies below write
// consecutive bytes) with XOR-swizzled 16-byte chunks, chosen so that every
// access pattern below touches 16 distinct bank groups per 16 lanes.
//
// Operands: per 64-wide k chunk, the workgroup's 128 Q rows and 128 K rows,
// 128 bytes each, copied global -> LDS by global_load_lds_dwordx4 (a
// wavefront writes 1 KB of consecutive LDS: eight rows). Chunk c of row r sits
// at position c ^ ((r >> 1) & 7): a fragment read takes 16 consecutive rows at
// one chunk, and rows r, r + 1 share a 256-byte bank line.
//
// Epilogue: each wavefront's 64x64 fp32 block in two passes of 32 rows x 256
// bytes, chunk c of row r at c ^ (r & 15); written 16 rows x one chunk per 16
// lanes, read back one row (16 chunks) per 16 lanes.
constexpr int kChunkK = 64;
constexpr int kRowBytes = kChunkK * 2;
constexpr int kOperandBytes = 2 * kMfmaBlock * kRowBytes;  // Q then K: 32 KB
constexpr int kStageBytes = 4 * 32 * 256;                  // 32 rows x 64 fp32 per wavefront: 32 KB
constexpr int kQkLdsBytes = kOperandBytes > kStageBytes ? kOperandBytes : kStageBytes;

typedef __attribute__((address_space(3))) unsigned char qk_lds_u8;
typedef __attribute__((address_space(3))) qk_u32x4 qk_lds_u32x4;

// One 16-byte global -> LDS copy per lane; `dst` is the wavefront's LDS base
// (lane L writes dst + 16 L).
__device__ __forceinline__ void dma16(const void* src, qk_lds_u8* dst) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}
__device__ __forceinline__ qk_u32x4 lds_read16(const qk_lds_u8* p) { return *(const qk_lds_u32x4*)p; }
typedef float qk_f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) qk_f32x4 qk_lds_f32x4;
__device__ __forceinline__ void lds_write_f4(qk_lds_u8* p, qk_f32x4 v) { *(qk_lds_f32x4*)p = v; }
__device__ __forceinline__ qk_f32x4 lds_read_f4(const qk_lds_u8* p) { return *(const qk_lds_f32x4*)p; }

template <typename T, bool CAP>
__global__ __launch_bounds__(256) void qk_score_mfma_kernel(QkScoreArgs a) {
    // Scale and bias are rounded separately, as the reference applies them.
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) unsigned char smem[kQkLdsBytes];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t bt = blockIdx.z;
    const int64_t qb0 = (int64_t)blockIdx.y * kMfmaBlock, kb0 = (int64_t)blockIdx.x * kMfmaBlock;
    const int64_t i0 = qb0 + (wave >> 1) * 64;
    const int64_t j0 = kb0 + (wave & 1) * 64;
    const T* q = (const T*)a.q + bt * a.a_sb;
    const T* k = (const T*)a.k + bt * a.b_sb;
    const int r = lane & 31, half = lane >> 5;
    qk_lds_u8* lds = (qk_lds_u8*)smem;
    // DMA copy of one k-chunk: wavefront w, step u copies rows 32u + 8w .. +7
    // of Q and of K; lane L writes row 32u + 8w + (L >> 3), position L & 7,
    // holding global chunk (L & 7) ^ ((row >> 1) & 7). Rows past M or N and
    // chunks past K read clamped in-range addresses; their values are never used.
    auto copy_chunk = [&](int64_t k0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int row = 32 * u + 8 * wave + (lane >> 3);
            const int c = (lane & 7) ^ ((row >> 1) & 7);
            const int64_t kc = (k0 + 8 * c < a.K) ? k0 + 8 * c : k0;
            const int64_t qi = min(qb0 + row, a.M - 1), kj = min(kb0 + row, a.N - 1);
            const int base = (32 * u + 8 * wave) * kRowBytes;
            dma16(q + qi * a.a_sm + kc, lds + base);
            dma16(k + kj * a.b_sn + kc, lds + kMfmaBlock * kRowBytes + base);
        }
    };
    // Fragment rows of this lane: Q (B operand) rows and K (A operand) rows.
    int qoff[2], koff[2], qsw[2], ksw[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int qr = (wave >> 1) * 64 + 32 * t + r, kr = (wave & 1) * 64 + 32 * t + r;
        qoff[t] = qr * kRowBytes;
        koff[t] = kMfmaBlock * kRowBytes + kr * kRowBytes;
        qsw[t] = (qr >> 1) & 7;
        ksw[t] = (kr >> 1) & 7;
    }
    qk_f32x16 acc[2][2];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[x][y][e] = 0.0f;
    const qk_u32x4 zero = {0u, 0u, 0u, 0u};
    for (int64_t k0 = 0; k0 < a.K; k0 += kChunkK) {
        copy_chunk(k0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's copies have landed
        __syncthreads();                      // ... and every other wavefront's
        const int steps = ((int)min((int64_t)kChunkK, a.K - k0) + 15) / 16;  // 16-wide k steps
        for (int st = 0; st < steps; ++st) {
            const int c = 2 * st + half;                     // 16-byte chunk of this lane
            const bool kin = k0 + 8 * c < a.K;               // K is a multiple of 8
            qk_u32x4 qa[2], kb[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                qa[t] = kin ? lds_read16(lds + qoff[t] + 16 * (c ^ qsw[t])) : zero;
                kb[t] = kin ? lds_read16(lds + koff[t] + 16 * (c ^ ksw[t])) : zero;
            }
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y) acc[x][y] = QkMfma<T>::run(kb[y], qa[x], acc[x][y]);
        }
        __syncthreads();  // the next chunk (or the epilogue) overwrites the operands
    }
    // acc[x][y] holds the transposed tile: lane column r is query i0+32x+r and
    // elements 4g..4g+3 are the four consecutive keys j0+32y+8g+4*half+0..3.
    // The block goes through LDS (two passes of 32 rows) so that the global
    // stores and bias loads are full 256-byte row segments: 16 lanes per row,
    // four rows per instruction.
    qk_lds_u8* st = lds + wave * 32 * 256;  // this wavefront's 32-row pass buffer
    const int col = 4 * (lane & 15);
    const int64_t jb = j0 + col;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
        // pass x: rows 32x .. 32x+31 of the wavefront's block
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int chunk = 8 * y + 2 * g + half;  // keys 32y + 8g + 4 half .. +3
                lds_write_f4(st + r * 256 + 16 * (chunk ^ (r & 15)),
                             qk_f32x4{acc[x][y][4 * g], acc[x][y][4 * g + 1], acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]});
            }
        __syncthreads();
#pragma unroll 4
        for (int it = 0; it < 8; ++it) {
            const int row = 4 * it + (lane >> 4);
            const int64_t i = i0 + 32 * x + row;
            if (i >= a.M || jb >= a.N) continue;
            const qk_f32x4 raw = lds_read_f4(st + row * 256 + 16 * ((lane & 15) ^ (row & 15)));
            float v[4] = {raw[0], raw[1], raw[2], raw[3]};
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = a.has_scale ? v[u] * a.scale : v[u];
            float* crow = a.c + bt * a.c_sb + i * a.c_sm;
            const float* brow = a.bias != nullptr ? a.bias + bt * a.bias_sb + i * a.bias_sm : nullptr;
            if (a.vec4 && jb + 3 < a.N) {
                if (brow != nullptr) {
                    const float4 b4 = *(const float4*)(brow + jb);
                    v[0] = v[0] + b4.x;
                    v[1] = v[1] + b4.y;
                    v[2] = v[2] + b4.z;
                    v[3] = v[3] + b4.w;
                }
                if (CAP)
#pragma unroll
                    for (int u = 0; u < 4; ++u) v[u] = a.softcap * tanhf(v[u] / a.softcap);
                *(float4*)(crow + jb) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int64_t j = jb + u;
                    if (j >= a.N) break;
                    float w = v[u];
                    if (brow != nullptr) w = w + brow[j * a.bias_sn];
                    if (CAP) w = a.softcap * tanhf(w / a.softcap);
                    crow[j * a.c_sn] = w;
                }
            }
        }
        __syncthreads();  // the next pass reuses the buffer
    }
}

// Score rows without a bias or soft-cap, K <= 128 (scores only need the scale):
// one workgroup per 128-row query block and run of `tpw` 128-key blocks.
// The query block's MFMA fragments stay in registers for the whole run; K
// block t+1 is copied global -> LDS into the second buffer while block t is
// multiplied and written, and the buffer block t was read from then stages
// its epilogue (the same 256-byte row segments as above). 64 KB of LDS, two
// workgroups per CU. A one-block workgroup serialises its copies, MFMAs and
// stores (0.59-0.65 ms for 32 heads x 4096^2 x 128, against 0.35 ms for the
// stores alone); streaming K blocks through two buffers overlaps them.
// Workgroups are numbered so that each XCD (workgroup n runs on XCD n mod 8)
// takes a contiguous range of query blocks, i.e. reads the Q and K of a few
// heads only. Same products and summation order as qk_score_mfma_kernel, so
// the scores are bit-identical. CH = 16-byte chunks per K row in LDS (K <= 8 CH).
constexpr int kRowBufBytes = 32 * 1024;   // one K block (128 rows x 16 CH bytes), or the epilogue staging

template <int CH>
__device__ __forceinline__ int row_swz(int row) {
    // chunk position XOR: 16 consecutive rows of a fragment read hit 16 distinct 16-byte bank groups
    return CH == 16 ? (row & 15) : CH == 8 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}

template <typename T, int CH>
__global__ __launch_bounds__(256, 2) void qk_score_mfma_rows_kernel(QkScoreArgs a, int64_t nqb, int64_t npieces,
                                                                    int tpw) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * kRowBufBytes];
    constexpr int RB = CH * 16;    // LDS bytes per K row
    constexpr int RPI = 64 / CH;   // K rows per wavefront copy instruction (1 KB of LDS)
    constexpr int STEPS = CH / 2;  // 16-wide k steps
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 31, half = lane >> 5;
    const int64_t total = gridDim.x, n = blockIdx.x, per = total / 8;
    const int64_t id = n < 8 * per ? (n % 8) * per + n / 8 : n;
    const int64_t piece = id % npieces;
    const int64_t qb = (id / npieces) % nqb;
    const int64_t bt = id / (npieces * nqb);
    const int64_t nkb = (a.N + kMfmaBlock - 1) / kMfmaBlock;
    const int64_t kb_begin = piece * tpw;
    const int64_t kb_end = min(nkb, kb_begin + tpw);
    const T* q = (const T*)a.q + bt * a.a_sb;
    const T* k = (const T*)a.k + bt * a.b_sb;
    qk_lds_u8* lds = (qk_lds_u8*)smem;
    const qk_u32x4 zero = {0u, 0u, 0u, 0u};
    const int64_t i0 = qb * kMfmaBlock + (wave >> 1) * 64;   // the wavefront's 64 query rows
    // B-operand fragments of the wavefront's query rows (rows past M clamped, chunks past K zero)
    qk_u32x4 qf[2][STEPS];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
        const int64_t qr = min(i0 + 32 * x + r, a.M - 1);
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int c = 2 * st + half;
            qf[x][st] = 8 * c < a.K ? *(const qk_u32x4*)(q + qr * a.a_sm + 8 * c) : zero;
        }
    }
    // K block kb -> LDS buffer buf: wavefront w, step u copies rows (4u + w) RPI .. +RPI-1; lane L
    // writes row (4u + w) RPI + L / CH, position L % CH, holding global chunk (L % CH) ^ row_swz(row).
    // Rows past N and chunks past K read clamped in-range addresses; their values are never used.
    // Lane offsets are 32-bit from the block's base (the launcher checks 128 b_sn fits).
    const int bsn = (int)a.b_sn;
    auto copy_k = [&](int64_t kb, int buf) {
        const T* kblk = k + kb * kMfmaBlock * a.b_sn;
        const int lim = (int)min((int64_t)kMfmaBlock - 1, a.N - 1 - kb * kMfmaBlock);
#pragma unroll
        for (int u = 0; u < CH / 2; ++u) {
            const int slot = 4 * u + wave;
            const int row = slot * RPI + lane / CH;
            const int c = (lane % CH) ^ row_swz<CH>(row);
            const int kc = 8 * c < a.K ? 8 * c : 0;
            dma16(kblk + (min(row, lim) * bsn + kc), lds + buf * kRowBufBytes + slot * 1024);
        }
    };
    int koff[2], ksw[2];
#pragma unroll
    for (int y = 0; y < 2; ++y) {
        const int kr = (wave & 1) * 64 + 32 * y + r;
        koff[y] = kr * RB;
        ksw[y] = row_swz<CH>(kr);
    }
    copy_k(kb_begin, 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the first K block and the Q fragments
    __syncthreads();
    for (int64_t kb = kb_begin; kb < kb_end; ++kb) {
        const int buf = (int)((kb - kb_begin) & 1);
        if (kb + 1 < kb_end) copy_k(kb + 1, buf ^ 1);
        qk_lds_u8* kl = lds + buf * kRowBufBytes;
        qk_f32x16 acc[2][2];
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[x][y][e] = 0.0f;
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int c = 2 * st + half;
            const bool kin = 8 * c < a.K;
            qk_u32x4 kf[2];
#pragma unroll
            for (int y = 0; y < 2; ++y) kf[y] = kin ? lds_read16(kl + koff[y] + 16 * (c ^ ksw[y])) : zero;
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y) acc[x][y] = QkMfma<T>::run(kf[y], qf[x][st], acc[x][y]);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): K block kb+1 has landed
        __syncthreads();                      // ... for every wavefront; buffer `kl` is free for staging
        // epilogue as in qk_score_mfma_kernel, with 32-bit lane offsets from the wavefront's
        // block (the launcher checks that 64 rows and 64 columns of strides fit)
        const int64_t j0 = kb * kMfmaBlock + (wave & 1) * 64;
        qk_lds_u8* stg = kl + wave * 32 * 256;
        const int col = 4 * (lane & 15);
        const int64_t jb = j0 + col;
        float* cw = a.c + bt * a.c_sb + i0 * a.c_sm + j0 * a.c_sn;
        const int csm = (int)a.c_sm, csn = (int)a.c_sn;
#pragma unroll
        for (int x = 0; x < 2; ++x) {
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int chunk = 8 * y + 2 * g + half;
                    lds_write_f4(stg + r * 256 + 16 * (chunk ^ (r & 15)),
                                 qk_f32x4{acc[x][y][4 * g], acc[x][y][4 * g + 1], acc[x][y][4 * g + 2],
                                          acc[x][y][4 * g + 3]});
                }
            __syncthreads();
            // two rows of stores per unrolled step: more would hoist every row's address out of
            // the K-block loop and leave too few registers for two wavefronts per SIMD
#pragma unroll 2
            for (int it = 0; it < 8; ++it) {
                const int row = 4 * it + (lane >> 4);
                const int rr = 32 * x + row;   // row in the wavefront's block
                if (i0 + rr >= a.M || jb >= a.N) continue;
                const qk_f32x4 raw = lds_read_f4(stg + row * 256 + 16 * ((lane & 15) ^ (row & 15)));
                float v[4] = {raw[0], raw[1], raw[2], raw[3]};
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = a.has_scale ? v[u] * a.scale : v[u];
                if (a.vec4 && jb + 3 < a.N) {
                    *(float4*)(cw + (rr * csm + col)) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        if (jb + u >= a.N) break;
                        cw[rr * csm + (col + u) * csn] = v[u];
                    }
                }
            }
            __syncthreads();  // the next pass (or the next K block's copy) reuses the buffer
        }
    }
}

// K blocks per workgroup of the row kernel: runs of 4, shorter where that would
// leave fewer than one round of workgroups (two per CU on 256 CUs), longer
// beyond 4096 workgroups. Measured on 32 heads x D 128: 1024^2 0.029 ms with 4
// (0.033 with 2, 0.040 with 1 or 8), 2048^2 0.124 ms with 4 (0.164 with 8 or
// 16), 4096^2 0.463-0.465 ms with 8 or 16 (0.513 with 32).
inline int64_t rows_blocks_per_workgroup(int64_t tiles, int64_t nkb) {
    int64_t tpw = tiles / 4096;
    if (tpw < 4) tpw = std::min<int64_t>(4, std::max<int64_t>(1, tiles / 512));
    return std::min(tpw, nkb);
}

}  // namespace

bool qk_score_mfma_supported(const QkScoreArgs& a, int dtype) {
    if (dtype != DT_BF16 && dtype != DT_F16) return false;
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return a.a_sk == 1 && a.b_sk == 1 && a.K % 8 == 0 && a.a_sm % 8 == 0 && a.b_sn % 8 == 0 &&
           a.a_sb % 8 == 0 && a.b_sb % 8 == 0 && al16(a.q) && al16(a.k);
}

hipError_t launch_qk_score_mfma(const QkScoreArgs& a, int dtype, hipStream_t s) {
    if (a.batch <= 0 || a.M <= 0 || a.N <= 0 || a.K <= 0) return hipSuccess;
    if (!qk_score_mfma_supported(a, dtype)) return hipErrorInvalidValue;
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const bool c_vec = a.c_sn == 1 && a.c_sm % 4 == 0 && a.c_sb % 4 == 0 && al16(a.c);
    const bool b_vec = a.bias == nullptr ||
                       (a.bias_sn == 1 && a.bias_sm % 4 == 0 && a.bias_sb % 4 == 0 && al16(a.bias));
    // Scores only (no bias, no soft-cap), K <= 128, lane offsets within 32 bits: the row kernel.
    const int64_t lim31 = int64_t(1) << 31;
    const bool rows = a.bias == nullptr && !(a.softcap > 0.0f) && a.K <= 128 &&
                      (kMfmaBlock - 1) * a.b_sn + a.K < lim31 && 63 * (a.c_sm + a.c_sn) + 4 < lim31 &&
                      a.b_sn >= 0 && a.c_sm >= 0 && a.c_sn >= 0;
    if (rows) {
        const int64_t nqb = (a.M + kMfmaBlock - 1) / kMfmaBlock, nkb = (a.N + kMfmaBlock - 1) / kMfmaBlock;
        const int64_t max_grid = (int64_t(1) << 31) - 1;
        for (int64_t b0 = 0; b0 < a.batch;) {
            QkScoreArgs x = a;
            x.vec4 = c_vec;
            x.batch = std::min<int64_t>(a.batch - b0, std::max<int64_t>(1, max_grid / (nqb * nkb)));
            x.q = (const char*)a.q + b0 * a.a_sb * 2;
            x.k = (const char*)a.k + b0 * a.b_sb * 2;
            x.c = a.c + b0 * a.c_sb;
            const int64_t tiles = x.batch * nqb * nkb;
            const int64_t tpw = rows_blocks_per_workgroup(tiles, nkb);
            const int64_t npieces = (nkb + tpw - 1) / tpw;
            const dim3 grid((unsigned)(x.batch * nqb * npieces));
            const int K = (int)a.K;
            if (dtype == DT_BF16) {
                if (K <= 32) hipLaunchKernelGGL((qk_score_mfma_rows_kernel<__bf16, 4>), grid, dim3(256), 0, s, x, nqb, npieces, (int)tpw);
                else if (K <= 64) hipLaunchKernelGGL((qk_score_mfma_rows_kernel<__bf16, 8>), grid, dim3(256), 0, s, x, nqb, npieces, (int)tpw);
                else hipLaunchKernelGGL((qk_score_mfma_rows_kernel<__bf16, 16>), grid, dim3(256), 0, s, x, nqb, npieces, (int)tpw);
            } else {
                if (K <= 32) hipLaunchKernelGGL((qk_score_mfma_rows_kernel<_Float16, 4>), grid, dim3(256), 0, s, x, nqb, npieces, (int)tpw);
                else if (K <= 64) hipLaunchKernelGGL((qk_score_mfma_rows_kernel<_Float16, 8>), grid, dim3(256), 0, s, x, nqb, npieces, (int)tpw);
                else hipLaunchKernelGGL((qk_score_mfma_rows_kernel<_Float16, 16>), grid, dim3(256), 0, s, x, nqb, npieces, (int)tpw);
            }
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            b0 += x.batch;
        }
        return hipSuccess;
    }
    for (int64_t b0 = 0; b0 < a.batch; b0 += kMaxGridZ) {
        QkScoreArgs x = a;
        x.vec4 = c_vec && b_vec;
        x.batch = std::min<int64_t>(kMaxGridZ, a.batch - b0);
        x.q = (const char*)a.q + b0 * a.a_sb * 2;
        x.k = (const char*)a.k + b0 * a.b_sb * 2;
        x.c = a.c + b0 * a.c_sb;
        if (a.bias != nullptr) x.bias = a.bias + b0 * a.bias_sb;
        const dim3 grid((unsigned)((a.N + kMfmaBlock - 1) / kMfmaBlock),
                        (unsigned)((a.M + kMfmaBlock - 1) / kMfmaBlock), (unsigned)x.batch);
        // The soft-cap epilogue is a separate instantiation: it needs many more
        // registers, which would lower the occupancy of the common case.
        const bool cap = a.softcap > 0.0f;
        if (dtype == DT_BF16) {
            if (cap) hipLaunchKernelGGL((qk_score_mfma_kernel<__bf16, true>), grid, dim3(256), 0, s, x);
            else hipLaunchKernelGGL((qk_score_mfma_kernel<__bf16, false>), grid, dim3(256), 0, s, x);
        } else {
            if (cap) hipLaunchKernelGGL((qk_score_mfma_kernel<_Float16, true>), grid, dim3(256), 0, s, x);
            else hipLaunchKernelGGL((qk_score_mfma_kernel<_Float16, false>), grid, dim3(256), 0, s, x);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_qk_score(const QkScoreArgs& a, int dtype, hipStream_t s) {
    if (a.batch <= 0 || a.M <= 0 || a.N <= 0 || a.K <= 0) return hipSuccess;
    const size_t esz = dtype == DT_F32 ? 4 : 2;
    for (int64_t b0 = 0; b0 < a.batch; b0 += kMaxGridZ) {
        QkScoreArgs x = a;
        x.batch = std::min<int64_t>(kMaxGridZ, a.batch - b0);
        x.q = (const char*)a.q + b0 * a.a_sb * esz;
        x.k = (const char*)a.k + b0 * a.b_sb * esz;
        x.c = a.c + b0 * a.c_sb;
        if (a.bias != nullptr) x.bias = a.bias + b0 * a.bias_sb;
        const dim3 grid((unsigned)((a.N + kQkTile - 1) / kQkTile),
                        (unsigned)((a.M + kQkTile - 1) / kQkTile), (unsigned)x.batch);
        switch (dtype) {
            case DT_F32: hipLaunchKernelGGL(qk_score_kernel<float>, grid, dim3(256), 0, s, x); break;
            case DT_BF16: hipLaunchKernelGGL(qk_score_kernel<__bf16>, grid, dim3(256), 0, s, x); break;
            case DT_F16: hipLaunchKernelGGL(qk_score_kernel<_Float16>, grid, dim3(256), 0, s, x); break;
            default: return hipErrorInvalidValue;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Plain strided fp32 tile product (the tile-GEMM seam,
// src/onednn_flash/tile_kernel.cpp:67-86): the score kernel with no post-ops.
hipError_t launch_tile_gemm(const float* a, const float* b, float* c, int m, int n, int k,
                            int64_t asm_, int64_t ask, int64_t bsk, int64_t bsn, int64_t csm,
                            int64_t csn, hipStream_t s) {
    QkScoreArgs x{};
    x.batch = 1;
    x.M = m;
    x.N = n;
    x.K = k;
    x.q = a;
    x.k = b;
    x.c = c;
    x.a_sm = asm_;
    x.a_sk = ask;
    x.b_sk = bsk;
    x.b_sn = bsn;
    x.c_sm = csm;
    x.c_sn = csn;
    return launch_qk_score(x, DT_F32, s);
}

}  // namespace ofh
