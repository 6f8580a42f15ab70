// Kernel-side argument block and launcher entry points shared by the HIP
// translation units of the library. Internal header: not installed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ofh {

enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
enum Bias : int { BIAS_NONE = 0, BIAS_ALIBI = 1, BIAS_DENSE = 2 };

// Every wavefront of the MFMA flash kernels owns 32 query rows (one 32-wide
// MFMA column block); the workgroup shape depends on the element type.
constexpr int kQueriesPerWave = 32;

// fp32 calls with fewer 128-row query tiles than this run 32-row query
// blocks, four wavefronts per block sharing its keys (flash_fwd_f32_rows32_kernel).
constexpr int kRowsF32 = 32;
constexpr int kRows32Below = 128;
// Of those, calls at D <= 64 whose 16-row blocks fit one round of the CUs
// (one workgroup each) and whose keys are at most kRows16MaxKeyTiles tiles of
// 32 (twice that where the blocks fill half the CUs) run 16-row blocks of
// sixteen wavefronts without a key split (flash_fwd_f32_rows16_kernel).
constexpr int kRowsF32Narrow = 16;
constexpr int kRows16MaxKeyTiles = 32;

struct MfmaTiles {
    int block_m;  // query rows per query tile
    int block_n;  // keys per K/V tile
    int threads;  // threads per workgroup
    bool paired;  // each workgroup runs query tiles nqt-1-p and p (causal)
};

// Everything a forward kernel needs, passed by value. Pointers are device
// pointers; strides are in elements; the last axis of every tensor is
// contiguous.
struct FwdArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    int64_t q_sb, q_sh, q_sm;
    int64_t k_sb, k_sh, k_sn;
    int64_t v_sb, v_sh, v_sn;
    int64_t o_sb, o_sh, o_sm;
    int B, H, M, N, D, Dv;
    float scale;       // score scale
    float scale_log2;  // scale * log2(e)
    int causal;
    // block mask
    const uint8_t* mask;
    int mask_qbs, mask_kbs, mask_qb, mask_kb;
    // per-query-tile lists of key tiles (block mask only)
    const int* tile_counts;   // [num_q_tiles]
    const int* tile_entries;  // [num_q_tiles, num_k_tiles], see list_entry()
    int num_q_tiles, num_k_tiles;
    // score_mod
    int bias_kind;
    const float* alibi;  // [H]
    const float* bias;
    int64_t bias_sb, bias_sh, bias_sm;
    float softcap;      // 0: off
    float inv_softcap;
    int out_f32;        // 1: O is fp32, else O has the input dtype
    // Key split: workgroup s of a query tile runs its K/V tile steps
    // [s*split_tiles, (s+1)*split_tiles). A query tile with steps(qt) steps has
    // active(qt) = max(1, min(num_splits, ceil(steps(qt) / split_tiles)))
    // splits; with one, split 0 writes O itself. Otherwise every active split
    // writes its unnormalised O rows and (m, l) per row to part_o / part_ml,
    // and the rows are merged into O: by the split workgroup that arrives last
    // (counted in split_counters, which it leaves at zero), or, with
    // split_counters null, by combine_splits_kernel in a second launch.
    // num_splits == 1: one workgroup per query tile.
    int num_splits;
    int split_tiles;
    // 1 (causal calls of the fp32 128-row kernel and of
    // flash_fwd_pair_split_kernel): workgroups take the causal query tile
    // pairs (nqt-1-p, p) of map_work_pair, and query tile qt's steps are cut
    // into num_splits ranges of ceil(steps(qt) / num_splits) steps
    // (split_tiles unused), so every workgroup runs about the same number of
    // steps; workgroup s of a pair runs split s of both tiles.
    int pair_split;
    int split_bm, split_bn;  // query rows per query tile and keys per K/V tile step (every call)
    float* part_o;           // [num_splits][B*H][M][Dv] fp32
    float* part_ml;          // [num_splits][B*H][M][2] fp32: running max (log2 units), row sum
    unsigned* split_counters;  // [B*H*num_q_tiles] arrival counters, zero between calls, or null
};

// Single-launch key-split merge: arrival counters live in a static device
// array of kSplitCounterSlots slots of kMaxSplitTiles counters per GPU. A slot
// is used by one stream at a time (calls on a stream run in order); every call
// leaves the counters it used at zero, the state the code object loads with.
constexpr int kSplitCounterSlots = 64;
constexpr int kMaxSplitTiles = 1024;
// Device address of counter slot `slot` on the current device (looked up once
// per device, then cached).
hipError_t split_counter_slot(int slot, unsigned** ptr);

// Block-mask tile list entry: the key tile index and, for each 32-row slice
// w of the query tile (one wavefront each, at most kListSlices), bit w: the
// slice holds a pair that the mask and the causal rule allow; bit 4+w: the
// mask allows every pair of the slice (causal and ragged-end masking is still
// applied element-wise by the attention kernel).
constexpr int kListSlices = 4;
__host__ __device__ inline int list_entry(int kt, unsigned any, unsigned full) {
    return (kt << 8) | (int)((full & 15u) << 4) | (int)(any & 15u);
}
__host__ __device__ inline int list_tile(int e) { return e >> 8; }
__host__ __device__ inline bool list_any(int e, int slice) { return ((e >> slice) & 1) != 0; }
__host__ __device__ inline bool list_full(int e, int slice) { return ((e >> (4 + slice)) & 1) != 0; }

// Rows [q0,q1) x keys [k0,k1) of a block-mask call, already clipped to the
// problem: any = some pair is allowed by the mask (blocks out of its range are
// disallowed) and by the causal rule; all = the mask allows every pair (causal
// masking is applied element-wise by the attention kernel either way).
__device__ inline void classify_mask_slice(const uint8_t* mask, int qbs, int kbs, int nqb, int nkb, int causal,
                                           int q0, int q1, int k0, int k1, bool& any, bool& all) {
    any = false;
    all = true;
    const int qb0 = q0 / qbs, qb1 = (q1 - 1) / qbs;
    const int kb0 = k0 / kbs, kb1 = (k1 - 1) / kbs;
    for (int qb = qb0; qb <= qb1; ++qb) {
        const int qe = min(q1, (qb + 1) * qbs);
        for (int kb = kb0; kb <= kb1; ++kb) {
            const int ks = max(k0, kb * kbs);
            const bool allowed = qb < nqb && kb < nkb && mask[(int64_t)qb * nkb + kb] != 0;
            // causal: some key of the block is <= some query of the block iff ks <= qe-1
            any = any || (allowed && (!causal || ks <= qe - 1));
            all = all && allowed;
        }
    }
}

// classify_mask_slice with the slice's and the key tile's mask-block ranges
// already formed: query blocks [qb0, qb1] of a slice ending at row q1
// (exclusive), key blocks [kb0, kb1] of a tile starting at key k0.
__device__ inline void classify_mask_blocks(const uint8_t* mask, int qbs, int kbs, int nqb, int nkb, int causal,
                                            int q1, int k0, int qb0, int qb1, int kb0, int kb1, bool& any,
                                            bool& all) {
    any = false;
    all = true;
    for (int qb = qb0; qb <= qb1; ++qb) {
        const int qe = min(q1, (qb + 1) * qbs);
        for (int kb = kb0; kb <= kb1; ++kb) {
            const int ks = max(k0, kb * kbs);
            const bool allowed = qb < nqb && kb < nkb && mask[(int64_t)qb * nkb + kb] != 0;
            any = any || (allowed && (!causal || ks <= qe - 1));
            all = all && allowed;
        }
    }
}

struct TileListArgs {
    int M, N, block_m, block_n, causal;
    const uint8_t* mask;
    int mask_qbs, mask_kbs, mask_qb, mask_kb;
    int num_q_tiles, num_k_tiles;
    int* counts;
    int* entries;
};

// Batched strided fp32 score tile S = (Q K^T) * scale + bias (+ soft-cap).
// Strides are in elements; b_* index the K^T view (kk, j); bias is fp32 or null.
struct QkScoreArgs {
    int64_t batch, M, N, K;
    const void* q;
    const void* k;
    float* c;
    int64_t a_sm, a_sk, a_sb;
    int64_t b_sk, b_sn, b_sb;
    int64_t c_sm, c_sn, c_sb;
    int has_scale;
    float scale;
    const float* bias;
    int64_t bias_sm, bias_sn, bias_sb;
    float softcap;
    int vec4;   // set by the launcher: 16-byte score (and bias) row runs are aligned
};

// Launchers; each returns the hipError_t of the launch.
hipError_t launch_flash_mfma(const FwdArgs& a, int dtype, bool general_mod, hipStream_t s);
hipError_t launch_rowwise(const FwdArgs& a, int dtype, hipStream_t s);
hipError_t launch_tile_lists(const TileListArgs& a, hipStream_t s);
// Merge of the key-split partial rows into O in a second launch (num_splits > 1,
// split_counters null); dtype is the input type.
hipError_t launch_combine_splits(const FwdArgs& a, int dtype, hipStream_t s);
hipError_t launch_qk_score(const QkScoreArgs& a, int dtype, hipStream_t s);
// Matrix-core score kernel for bf16/fp16 with unit k-strides and 16-byte rows.
bool qk_score_mfma_supported(const QkScoreArgs& a, int dtype);
hipError_t launch_qk_score_mfma(const QkScoreArgs& a, int dtype, hipStream_t s);

// LDS bytes of the 16-bit block-mask kernel: with lds_list the workgroup
// builds its query tile's list in LDS (no tile_list launch, no workspace).
size_t list_kernel_lds_bytes(int D, bool lds_list, int num_k_tiles);
constexpr int kLdsListMaxTiles = 4096;  // key tiles of a list built in LDS
// Head dims the MFMA kernels are built for: every multiple of 32 from 32 to
// 256 (fp32 above 128 on one-block K/V tiles of 32 keys).
bool flash_mfma_head_dim(int dtype, int D);
// Head dim of the MFMA kernel that serves a call with head dims (D, Dv): the
// larger rounded up to a multiple of 32 (the kernels zero-pad Q past D and
// leave the output columns past Dv unwritten), or 0 when none does: bf16/fp16
// need multiples of 8, fp32 multiples of 4 (16-byte row chunks), up to 256.
int flash_mfma_kernel_dim(int dtype, int D, int Dv);
// threads: the workgroup size of the tiling the call runs (flash_mfma_tiles).
const char* flash_mfma_kernel_name(int dtype, int D, bool general_mod, bool tile_list, int threads);
// Compute units of an MI355X.
constexpr int kComputeUnits = 256;
// Workgroup tiling of the MFMA kernel for a dtype and a call of bh heads
// (batch x heads) and query_tokens rows: 16-bit D = 192 and 256 without
// score_mod or block mask run 8 wavefronts (256 rows) where 4 (128 rows, one
// workgroup per CU) would take more than one round of the CUs, else 4.
MfmaTiles flash_mfma_tiles(int dtype, int head_dim, bool general_mod, bool tile_list, bool causal, int64_t bh,
                           int64_t query_tokens);

// Scratch of the allocation-free entry point: a static device array of
// kNoAllocScratchBytes per GPU. noalloc_scratch returns the current device's
// address of it (looked up once per device, then cached).
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
hipError_t noalloc_scratch(void** ptr);

}  // namespace ofh
