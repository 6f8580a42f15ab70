// C ABI of the attention forward library (include/onednn_flash_hip.h):
// argument validation with the reference's error texts, layout resolution,
// kernel choice, scratch management and the host-buffer convenience entry.

#include "onednn_flash_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "ofh_kernels.h"
#include "stream_key.h"

namespace {

thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

#define OFH_HIP_CHECK(expr)                                                                   \
    do {                                                                                      \
        const hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                                 \
            return set_error(OFH_ERROR_HIP, std::string(#expr " failed: ") + hipGetErrorString(e_)); \
    } while (0)

size_t elem_size(int dtype) { return dtype == OFH_DTYPE_F32 ? 4 : 2; }

struct Resolved {
    int64_t qs[3], ks[3], vs[3], os[3];
    int algorithm;       // OFH_ALGO_FLASH_MFMA or OFH_ALGO_ROWWISE
    bool general_mod;    // bias or soft-cap present
    bool tile_list;      // block-mask tile lists are used
    bool lds_list;       // ... built by each workgroup in LDS (no tile_list launch, no workspace)
    int block_m, block_n, threads;
    bool paired;         // causal query tiles run in pairs per workgroup
    int num_q_tiles, num_k_tiles;
    int key_splits;      // workgroups per query tile, each over a range of K/V tiles
    int split_tiles;     // K/V tile steps per split
    bool pair_split;     // causal: query tile pairs, each tile split in key_splits ranges of its own length
    int kdim;            // head dim of the MFMA kernel: max(D, Dv) rounded up to a multiple of 32
};

void contiguous_strides(int64_t out[3], const int64_t in[3], size_t H, size_t T, size_t last) {
    if (in[0] == 0 && in[1] == 0 && in[2] == 0) {
        out[2] = (int64_t)last;
        out[1] = (int64_t)(T * last);
        out[0] = (int64_t)(H * T * last);
    } else {
        out[0] = in[0];
        out[1] = in[1];
        out[2] = in[2];
    }
}

// All-zero bias strides mean one contiguous [M, N] bias shared by every
// (batch, head), the shape of the reference's ScoreBiasFn (attention.hpp:31).
void dense_bias_strides(const ofh_attention_params* p, int64_t out[3]) {
    if (p->bias_strides[0] == 0 && p->bias_strides[1] == 0 && p->bias_strides[2] == 0) {
        out[0] = 0;
        out[1] = 0;
        out[2] = (int64_t)p->key_tokens;
    } else {
        out[0] = p->bias_strides[0];
        out[1] = p->bias_strides[1];
        out[2] = p->bias_strides[2];
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Shape and option checks, with the reference's messages where it has one
// (batched_attention.cpp:15-21, attention.cpp:71-79).
int validate(const ofh_attention_params* p, bool check_ptrs, const void* q, const void* k,
             const void* v, const void* out) {
    if (p == nullptr) return set_error(OFH_ERROR_INVALID_ARGUMENT, "params must be non-null");
    if (p->struct_size != sizeof(ofh_attention_params))
        return set_error(OFH_ERROR_INVALID_ARGUMENT,
                         "ofh_attention_params.struct_size mismatch (call ofh_attention_params_init)");
    if (check_ptrs && (q == nullptr || k == nullptr || v == nullptr || out == nullptr))
        return set_error(OFH_ERROR_INVALID_ARGUMENT,
                         "batched attention input/output pointers must be non-null");
    if (p->batch == 0 || p->heads == 0 || p->query_tokens == 0 || p->key_tokens == 0 ||
        p->head_dim == 0 || p->value_dim == 0)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "batched attention dimensions must be non-zero");
    const size_t imax = (size_t)std::numeric_limits<int32_t>::max();
    if (p->batch > imax || p->heads > imax || p->query_tokens > imax || p->key_tokens > imax ||
        p->head_dim > imax || p->value_dim > imax || p->batch * p->heads > imax)
        return set_error(OFH_ERROR_UNSUPPORTED, "attention dimensions exceed the 32-bit index range");
    if (p->dtype < OFH_DTYPE_F32 || p->dtype > OFH_DTYPE_F16)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "unknown dtype");
    if (p->out_dtype != p->dtype && p->out_dtype != OFH_DTYPE_F32)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "out_dtype must equal dtype or be f32");
    if (!std::isfinite(p->scale))
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "scale must be finite");
    if (p->mask_allowed != nullptr) {
        if (p->mask_query_block_size == 0 || p->mask_key_block_size == 0)
            return set_error(OFH_ERROR_INVALID_ARGUMENT, "BlockMask block sizes must be non-zero");
        if (p->mask_query_blocks == 0 || p->mask_key_blocks == 0)
            return set_error(OFH_ERROR_INVALID_ARGUMENT, "BlockMask dimensions must be non-zero");
        if (p->mask_query_block_size > imax || p->mask_key_block_size > imax ||
            p->mask_query_blocks > imax || p->mask_key_blocks > imax)
            return set_error(OFH_ERROR_UNSUPPORTED, "BlockMask dimensions exceed the 32-bit index range");
    }
    if (p->bias_kind < OFH_BIAS_NONE || p->bias_kind > OFH_BIAS_DENSE)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "unknown bias kind");
    if (p->bias_kind == OFH_BIAS_ALIBI && p->alibi_slopes == nullptr)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "ALiBi bias needs per-head slopes");
    if (p->bias_kind == OFH_BIAS_DENSE && p->bias == nullptr)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "dense bias needs a bias tensor");
    if (!(p->softcap >= 0.0f) || !std::isfinite(p->softcap))
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "softcap must be finite and >= 0");
    if (p->algorithm < OFH_ALGO_AUTO || p->algorithm > OFH_ALGO_ROWWISE)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "unknown algorithm");
    if (p->max_key_splits < 0)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "max_key_splits must be >= 0");
    return OFH_SUCCESS;
}

// Key split. A call whose query tiles give fewer workgroups than kTarget
// leaves CUs idle and runs as long as its longest query tile: the decode and
// short-query shapes (M <= 256 rows per head) of the 16-bit kernels, small
// fp32 calls. Such calls run the K/V tile steps of each query tile in ranges
// of split_tiles steps (at least 64 keys) sized so that all ranges together
// fill about kTarget workgroups, then merge the partial rows. Causal 16-bit
// calls then run their query tiles unpaired. Without a mask the tile steps of
// query tile qt are known on the host; with a block mask the list can only
// remove steps, so the unmasked count is an upper bound.
// Workgroups that run at once per CU for the kernel the call takes (registers
// and LDS of the kernels in flash_fwd_mfma.hip): the 8-wavefront 16-bit
// kernels one, the 4-wavefront ones two up to D = 128 (three for the
// plain-scale block-mask kernels up to D = 64), the fp32 kernels two up to
// D = 64.
int workgroups_per_cu(const ofh_attention_params* p, const Resolved& r) {
    if (p->dtype == OFH_DTYPE_F32) return r.kdim <= 64 ? 2 : 1;
    if (r.threads >= 512) return 1;
    if (r.tile_list && !r.general_mod && r.kdim <= 64) return 3;
    return r.kdim < 160 ? 2 : 1;
}
using ofh::kComputeUnits;

// Key split for calls with fewer query tiles than the GPU runs at once: every
// query tile's K/V tile steps are cut into ranges of `per` steps, one
// workgroup each. The split count is the largest whose workgroups (those with
// steps to run) all fit in one round of the GPU's slots (CUs x workgroups per
// CU): a second round doubles the longest chain, and every extra split adds
// partial rows to store and merge. Measured (per call): bf16 decode B1 H8 M1
// N32768 D128 30.9 us with 32 splits against 36.0 with 64; bf16 causal B1 H8
// N4096 D128 61.3 us with 3 against 87.7 with 7; fp32 causal B2 H8 N2048 D64
// 126 us with 3 against 135 with 4.
void choose_key_splits(const ofh_attention_params* p, Resolved& r) {
    r.key_splits = 1;
    r.split_tiles = 1 << 30;
    r.pair_split = false;
    if (p->dtype == OFH_DTYPE_F32 && (r.paired || r.block_m == ofh::kRowsF32Narrow)) return;
    if (p->max_key_splits == 1) return;
    const bool rows32 = p->dtype == OFH_DTYPE_F32 && r.block_m == ofh::kRowsF32;
    const int64_t slots = kComputeUnits * workgroups_per_cu(p, r);
    const int kMaxSplits = p->max_key_splits > 1 ? std::min(p->max_key_splits, 64) : 64;
    const int64_t bh = (int64_t)p->batch * p->heads;
    // Causal calls without a block mask (fp32 on 128-row tiles, 16-bit):
    // query tiles p and nqt-1-p share a workgroup and every tile is cut into S
    // ranges of its own length, so all workgroups run about the same number of
    // steps; S is the largest count whose pairs fit one round of the slots.
    // fp32 takes it first: a common range length for all tiles (causal B2 H8
    // N2048 D64: 3 splits of 11 steps) left the shorter tiles' workgroups idle.
    // 16-bit calls take it only where the common ranges would not split (the
    // pairs alone then leave CUs idle: f16 causal B1 H8 N8192 D128 0.223 ->
    // 0.172 ms); where they do split, a second tile per workgroup (its
    // prologue, partial rows and a wider merge) measured slower (bf16 causal
    // B1 H8 N4096 D128: 3 common ranges 0.060 ms, 4 per-tile ranges 0.065).
    const bool pair_ok = !rows32 && p->causal && !r.tile_list;
    auto plan_pair_split = [&]() {
        const int64_t pairs = bh * ((r.num_q_tiles + 1) / 2);
        const int64_t kend = std::min<int64_t>((int64_t)p->key_tokens, (int64_t)r.num_q_tiles * r.block_m);
        const int64_t max_steps = (kend + r.block_n - 1) / r.block_n;
        const int64_t s = std::min<int64_t>({(int64_t)kMaxSplits, slots / std::max<int64_t>(pairs, 1), max_steps});
        if (s < 2) return false;
        r.paired = true;
        r.pair_split = true;
        r.key_splits = (int)s;
        r.split_tiles = 1 << 30;
        return true;
    };
    if (pair_ok && p->dtype == OFH_DTYPE_F32 && plan_pair_split()) return;
    const int64_t wgs = bh * (r.paired ? (r.num_q_tiles + 1) / 2 : r.num_q_tiles);
    if (wgs >= slots) return;
    // tile steps of each query tile (block_n keys each)
    std::vector<int> steps((size_t)r.num_q_tiles);
    int max_steps = 0;
    for (int qt = 0; qt < r.num_q_tiles; ++qt) {
        const int64_t kend = p->causal ? std::min<int64_t>((int64_t)p->key_tokens, (int64_t)(qt + 1) * r.block_m)
                                       : (int64_t)p->key_tokens;
        steps[(size_t)qt] = (int)((kend + r.block_n - 1) / r.block_n);
        max_steps = std::max(max_steps, steps[(size_t)qt]);
    }
    // at least 64 keys per split (128/256-row kernels), or a tile per
    // wavefront (32-row fp32 blocks)
    const int min_steps = rows32 ? 4 : std::max(1, 64 / r.block_n);
    const int most = std::min(kMaxSplits, std::max(1, max_steps / min_steps));
    auto per_of = [&](int n) { return (max_steps + n - 1) / n; };
    auto active = [&](int n) {
        const int per = per_of(n);
        int64_t a = 0;
        for (int st : steps) a += (st + per - 1) / per;
        return a * bh;
    };
    // largest split count in [1, most] whose active workgroups fit the slots
    // (active grows with the count)
    int lo = 1, hi = most;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (active(mid) <= slots) lo = mid;
        else hi = mid - 1;
    }
    const int per = per_of(lo);
    const int splits = (max_steps + per - 1) / per;
    if (splits <= 1) {
        if (pair_ok) plan_pair_split();
        return;
    }
    r.key_splits = splits;
    r.split_tiles = per;
    r.paired = false;
}

// 16-bit block-mask calls without a key split build each query tile's list
// in the workgroup's LDS when it fits (at most kLdsListMaxTiles key tiles).
void set_lds_list(const ofh_attention_params* p, Resolved& r) {
    r.lds_list = r.tile_list && p->dtype != OFH_DTYPE_F32 && r.key_splits == 1 &&
                 r.num_k_tiles <= ofh::kLdsListMaxTiles;
}

void no_key_split(const ofh_attention_params* p, Resolved& r) {
    r.key_splits = 1;
    r.split_tiles = 1 << 30;
    r.pair_split = false;
    // 32- and 16-row blocks: no pairing, no list
    if (p->dtype == OFH_DTYPE_F32 && (r.block_m == ofh::kRowsF32 || r.block_m == ofh::kRowsF32Narrow)) return;
    const ofh::MfmaTiles t = ofh::flash_mfma_tiles(p->dtype, r.kdim, r.general_mod, r.tile_list, p->causal != 0,
                                                   (int64_t)p->batch * p->heads, p->query_tokens);
    r.paired = t.paired;
    r.block_n = t.block_n;
    r.num_k_tiles = (int)((p->key_tokens + r.block_n - 1) / r.block_n);
    set_lds_list(p, r);
}

int resolve(const ofh_attention_params* p, const void* q, const void* k, const void* v,
            const void* out, Resolved& r) {
    contiguous_strides(r.qs, p->q_strides, p->heads, p->query_tokens, p->head_dim);
    contiguous_strides(r.ks, p->k_strides, p->heads, p->key_tokens, p->head_dim);
    contiguous_strides(r.vs, p->v_strides, p->heads, p->key_tokens, p->value_dim);
    contiguous_strides(r.os, p->o_strides, p->heads, p->query_tokens, p->value_dim);
    r.general_mod = p->bias_kind != OFH_BIAS_NONE || p->softcap > 0.0f;

    // The MFMA kernels read and write 16-byte row chunks.
    const size_t es = elem_size(p->dtype), oes = elem_size(p->out_dtype);
    auto strides_ok = [](const int64_t s[3], size_t esz) {
        for (int i = 0; i < 3; ++i)
            if (((s[i] * (int64_t)esz) & 15) != 0) return false;
        return true;
    };
    // Head dims that are not the kernel's own (not a multiple of 32, or D != Dv)
    // run on the kernel of max(D, Dv) rounded up to a multiple of 32.
    r.kdim = p->head_dim <= 256 && p->value_dim <= 256
                 ? ofh::flash_mfma_kernel_dim(p->dtype, (int)p->head_dim, (int)p->value_dim)
                 : 0;
    const bool mfma_ok = r.kdim > 0 &&
                         (p->dtype != OFH_DTYPE_F32 || p->out_dtype == OFH_DTYPE_F32) &&
                         aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                         strides_ok(r.qs, es) && strides_ok(r.ks, es) && strides_ok(r.vs, es) &&
                         strides_ok(r.os, oes) &&
                         // K/V staging keeps per-lane row offsets (row < 64) in 32 bits
                         std::llabs((long long)r.ks[2]) <= (1 << 24) && std::llabs((long long)r.vs[2]) <= (1 << 24);
    if (p->algorithm == OFH_ALGO_FLASH_MFMA && !mfma_ok)
        return set_error(OFH_ERROR_UNSUPPORTED,
                         "flash MFMA kernel needs head_dim and value_dim multiples of 4 (fp32) "
                         "or of 8 (bf16/fp16) up to 256, 16-byte "
                         "aligned rows and K/V token strides of at most 2^24 elements; use "
                         "OFH_ALGO_AUTO or OFH_ALGO_ROWWISE");
    if (p->algorithm == OFH_ALGO_ROWWISE || !mfma_ok) {
        r.algorithm = OFH_ALGO_ROWWISE;
        if (p->head_dim > 1024)
            return set_error(OFH_ERROR_UNSUPPORTED, "rowwise kernel supports head_dim <= 1024");
        r.tile_list = false;
        r.lds_list = false;
        r.paired = false;
        r.block_m = 1;
        r.block_n = 64;
        r.threads = 256;
        r.num_q_tiles = 0;
        r.num_k_tiles = 0;
        r.key_splits = 1;
        r.split_tiles = 1 << 30;
        r.pair_split = false;
        return OFH_SUCCESS;
    }
    r.algorithm = OFH_ALGO_FLASH_MFMA;
    const ofh::MfmaTiles tiles =
        ofh::flash_mfma_tiles(p->dtype, r.kdim, r.general_mod, p->mask_allowed != nullptr, p->causal != 0,
                              (int64_t)p->batch * p->heads, p->query_tokens);
    r.block_m = tiles.block_m;
    r.block_n = tiles.block_n;
    r.threads = tiles.threads;
    r.paired = tiles.paired;
    r.num_q_tiles = (int)((p->query_tokens + r.block_m - 1) / r.block_m);
    r.num_k_tiles = (int)((p->key_tokens + r.block_n - 1) / r.block_n);
    r.tile_list = p->mask_allowed != nullptr;
    // fp32 with few query tiles (latency-bound): 32-row query blocks whose
    // four wavefronts share the keys, 32-key tiles (built up to D = 128)
    if (p->dtype == OFH_DTYPE_F32 && !r.tile_list && r.kdim <= 128 &&
        (int64_t)p->batch * p->heads * r.num_q_tiles < ofh::kRows32Below) {
        r.block_m = ofh::kRowsF32;
        r.block_n = 32;
        r.paired = false;
        r.num_q_tiles = (int)((p->query_tokens + r.block_m - 1) / r.block_m);
        r.num_k_tiles = (int)((p->key_tokens + r.block_n - 1) / r.block_n);
        // ... and with few keys as well, 16-row blocks of sixteen wavefronts
        // that fold every key in the CU (no partial rows, no merge): up to 32
        // key tiles of 32 (two per wavefront), or 64 where the blocks fill
        // half the CUs. A wavefront's further tiles cost ~6 us each (loads not
        // overlapped), against split workgroups that spread them over the
        // CUs. Measured per call, 16-row blocks against 32-row blocks with the
        // key split (D = 64): N512 8.8-9.4 against 10.0-15.3 us at 1 to 128
        // blocks; N1024 15.0-15.4 against 14.9-16.2 at 4 to 32 blocks and
        // 15.4-16.6 against 28.2-32.7 at 128 to 256; N2048 27.5 against 34.9
        // at 128 blocks, 27.7 against 21.7 at 64 and 27.3 against 13.1 at 32;
        // N4096 51.8 against 50.0 at 128. Causal blocks see the keys up to
        // their last row only.
        const int64_t nqb16 = ((int64_t)p->query_tokens + ofh::kRowsF32Narrow - 1) / ofh::kRowsF32Narrow;
        const int64_t blocks16 = (int64_t)p->batch * p->heads * nqb16;
        const int64_t keys16 = p->causal ? std::min<int64_t>((int64_t)p->key_tokens, nqb16 * ofh::kRowsF32Narrow)
                                         : (int64_t)p->key_tokens;
        const int64_t tiles16 = (keys16 + 31) / 32;
        if (r.kdim <= 64 && blocks16 <= kComputeUnits &&
            (tiles16 <= ofh::kRows16MaxKeyTiles || (tiles16 <= 2 * ofh::kRows16MaxKeyTiles && 2 * blocks16 >= kComputeUnits))) {
            r.block_m = ofh::kRowsF32Narrow;
            r.threads = 1024;
            r.num_q_tiles = (int)((p->query_tokens + r.block_m - 1) / r.block_m);
        }
    }
    const int64_t grid = (int64_t)p->batch * p->heads * r.num_q_tiles;
    if (grid > std::numeric_limits<int32_t>::max())
        return set_error(OFH_ERROR_UNSUPPORTED, "grid exceeds 2^31 workgroups");
    if (r.tile_list && (int64_t)r.num_q_tiles * r.num_k_tiles > (int64_t)1 << 31)
        return set_error(OFH_ERROR_UNSUPPORTED, "block-mask tile list too large");
    if (r.tile_list && (r.block_m > ofh::kQueriesPerWave * ofh::kListSlices || r.num_k_tiles > (1 << 22)))
        return set_error(OFH_ERROR_UNSUPPORTED, "block-mask tile list entry cannot encode this tiling");
    choose_key_splits(p, r);
    set_lds_list(p, r);
    return OFH_SUCCESS;
}

size_t round256(size_t n) { return (n + 255) & ~size_t(255); }

// Workspace layout: [tile counts][tile entries] (block mask), then
// [partial O][partial (m, l)] (key split).
size_t list_bytes(const Resolved& r) {
    if (!r.tile_list || r.lds_list) return 0;
    return round256((size_t)r.num_q_tiles * 4) + (size_t)r.num_q_tiles * (size_t)r.num_k_tiles * 4;
}
size_t partial_rows(const ofh_attention_params* p, const Resolved& r) {
    return (size_t)r.key_splits * p->batch * p->heads * p->query_tokens;
}
// Arrival counters of the single-launch split merge: slot 0 serves the
// allocation-free entry point, slots 1.. one stream each (first come, first
// served; keyed as the scratch buffers are, see stream_key.h). A call that
// finds no free slot, or runs with OFH_SPLIT_MERGE=launch in the environment,
// merges in a second launch instead.
std::mutex g_counter_mu;
std::map<ofh::StreamKey, int> g_counter_slots;
int g_next_counter_slot = 1;

int split_counters_for(hipStream_t stream, bool noalloc, unsigned** out) {
    *out = nullptr;
    const char* env = std::getenv("OFH_SPLIT_MERGE");
    if (env != nullptr && std::strcmp(env, "launch") == 0) return OFH_SUCCESS;
    int slot = 0;
    if (!noalloc) {
        int dev = 0;
        OFH_HIP_CHECK(hipGetDevice(&dev));
        std::lock_guard<std::mutex> lock(g_counter_mu);
        const ofh::StreamKey key = ofh::stream_key(dev, stream);
        auto it = g_counter_slots.find(key);
        if (it == g_counter_slots.end()) {
            if (g_next_counter_slot >= ofh::kSplitCounterSlots) return OFH_SUCCESS;
            it = g_counter_slots.emplace(key, g_next_counter_slot++).first;
        }
        slot = it->second;
    }
    OFH_HIP_CHECK(ofh::split_counter_slot(slot, out));
    return OFH_SUCCESS;
}

// The workgroup that arrives last merges its query tile alone, so the merge
// is one CU's latency chain: measured, it beats a second launch only while
// the tile's partial rows are few (at most 64 KiB; single-row decode,
// B1 H8 N32768 D128: 35.8 us against 39.4 us) and loses on larger ones
// (fp32 B1 H4 N512 D64, 8 splits of 128 rows: 32.3 us against 18.1 us).
bool merge_in_launch(const ofh_attention_params* p, const Resolved& r) {
    if (r.key_splits <= 1) return false;
    const int64_t tile_floats = std::min<int64_t>(r.block_m, (int64_t)p->query_tokens) *
                                (int64_t)p->value_dim * r.key_splits;
    return (int64_t)p->batch * p->heads * r.num_q_tiles <= ofh::kMaxSplitTiles && tile_floats <= (1 << 14);
}

size_t workspace_bytes_for(const ofh_attention_params* p, const Resolved& r) {
    size_t n = list_bytes(r);
    if (r.key_splits > 1) n = round256(n) + round256(partial_rows(p, r) * p->value_dim * 4) + partial_rows(p, r) * 8;
    return n;
}

// Library-owned scratch, used when the caller passes no workspace.
//
// The first kDedicatedScratchStreams streams of a device (keyed by
// stream_key: hipStreamPerThread per host thread) get a buffer each. Calls on
// one stream run in stream order, so they can share its buffer; calls on
// different streams never share one. A dedicated buffer grows on demand (its
// stream synchronised, then the old buffer freed) and lives until the process
// ends: the footprint is, per stream, the largest need of a call on it (at
// least 1 MiB).
//
// Streams beyond those share one overflow buffer per device, ordered across
// streams by an event: a call waits (on the device, hipStreamWaitEvent) for
// the previous call that used the buffer and records the event after its own
// launches. Growing it waits (on the host) for that last user. So the
// library's scratch stays bounded by kDedicatedScratchStreams + 1 buffers per
// device however many streams a caller creates.
//
// A stream under graph capture never grows or frees anything: it may use its
// dedicated buffer when that already fits, which is then marked as held by a
// graph. A held buffer is never freed: when it must grow, a new buffer
// replaces it and the old one stays allocated until the process ends, since
// replays of the graph still address it. Calls that do not fit return
// OFH_ERROR_WORKSPACE_TOO_SMALL before touching the stream (key splits are
// dropped first, which leaves the result unchanged).
//
// The mutex is held from the lookup until the call's launches are queued
// (fwd_impl), so no buffer is grown while a launch that uses it is unqueued.
constexpr int kDedicatedScratchStreams = 16;

struct DeviceScratch {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool held_by_graph = false;
};
struct SharedScratch {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t last_use = nullptr;
    bool recorded = false;
};
std::mutex g_scratch_mu;
std::map<ofh::StreamKey, DeviceScratch> g_scratch;
std::map<int, SharedScratch> g_shared_scratch;
std::vector<void*> g_graph_held;  // replaced buffers that captured graphs still address

bool stream_capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(stream, &st) == hipSuccess && st == hipStreamCaptureStatusActive;
}

int dedicated_scratch_count(int dev) {
    int n = 0;
    for (const auto& kv : g_scratch) n += kv.first.device == dev ? 1 : 0;
    return n;
}

// Caller holds g_scratch_mu. Bytes a call on `stream` under graph capture may
// use without allocating: its dedicated buffer's (0 without one).
size_t capture_scratch_bytes_locked(hipStream_t stream) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    auto it = g_scratch.find(ofh::stream_key(dev, stream));
    return it == g_scratch.end() ? 0 : it->second.bytes;
}

// Caller holds g_scratch_mu until the call's launches are queued; when
// *shared is set, it then calls shared_scratch_release.
int library_scratch_locked(size_t bytes, hipStream_t stream, bool capturing, void** out,
                           SharedScratch** shared) {
    *shared = nullptr;
    int dev = 0;
    OFH_HIP_CHECK(hipGetDevice(&dev));
    const ofh::StreamKey key = ofh::stream_key(dev, stream);
    auto it = g_scratch.find(key);
    if (it == g_scratch.end() && !capturing && dedicated_scratch_count(dev) < kDedicatedScratchStreams)
        it = g_scratch.emplace(key, DeviceScratch{}).first;
    if (it != g_scratch.end()) {
        DeviceScratch& s = it->second;
        if (s.bytes < bytes) {
            if (capturing)
                return set_error(OFH_ERROR_WORKSPACE_TOO_SMALL,
                                 "a stream under graph capture cannot grow the library's scratch: pass a "
                                 "workspace of " + std::to_string(bytes) + " bytes");
            if (s.ptr != nullptr) {
                if (s.held_by_graph) {
                    g_graph_held.push_back(s.ptr);
                } else {
                    OFH_HIP_CHECK(hipStreamSynchronize(stream));  // earlier launches on this stream may still use it
                    OFH_HIP_CHECK(hipFree(s.ptr));
                }
                s.ptr = nullptr;
                s.bytes = 0;
                s.held_by_graph = false;
            }
            const size_t grown = std::max(bytes, (size_t)1 << 20);
            OFH_HIP_CHECK(hipMalloc(&s.ptr, grown));
            s.bytes = grown;
        }
        if (capturing) s.held_by_graph = true;
        *out = s.ptr;
        return OFH_SUCCESS;
    }
    if (capturing)
        return set_error(OFH_ERROR_WORKSPACE_TOO_SMALL,
                         "a stream under graph capture has no library scratch: pass a workspace of " +
                             std::to_string(bytes) + " bytes");
    SharedScratch& sh = g_shared_scratch[dev];
    if (sh.last_use == nullptr) OFH_HIP_CHECK(hipEventCreateWithFlags(&sh.last_use, hipEventDisableTiming));
    if (sh.bytes < bytes) {
        if (sh.ptr != nullptr) {
            if (sh.recorded) OFH_HIP_CHECK(hipEventSynchronize(sh.last_use));  // the last user has finished
            OFH_HIP_CHECK(hipFree(sh.ptr));
            sh.ptr = nullptr;
            sh.bytes = 0;
        }
        const size_t grown = std::max(bytes, (size_t)1 << 20);
        OFH_HIP_CHECK(hipMalloc(&sh.ptr, grown));
        sh.bytes = grown;
    }
    if (sh.recorded) OFH_HIP_CHECK(hipStreamWaitEvent(stream, sh.last_use, 0));
    *shared = &sh;
    *out = sh.ptr;
    return OFH_SUCCESS;
}

// After the launches that use the shared overflow buffer are queued.
int shared_scratch_release(SharedScratch* sh, hipStream_t stream) {
    OFH_HIP_CHECK(hipEventRecord(sh->last_use, stream));
    sh->recorded = true;
    return OFH_SUCCESS;
}

ofh::FwdArgs make_args(const ofh_attention_params* p, const Resolved& r, const void* q,
                       const void* k, const void* v, void* out) {
    ofh::FwdArgs a;
    std::memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = out;
    a.q_sb = r.qs[0]; a.q_sh = r.qs[1]; a.q_sm = r.qs[2];
    a.k_sb = r.ks[0]; a.k_sh = r.ks[1]; a.k_sn = r.ks[2];
    a.v_sb = r.vs[0]; a.v_sh = r.vs[1]; a.v_sn = r.vs[2];
    a.o_sb = r.os[0]; a.o_sh = r.os[1]; a.o_sm = r.os[2];
    a.B = (int)p->batch;
    a.H = (int)p->heads;
    a.M = (int)p->query_tokens;
    a.N = (int)p->key_tokens;
    a.D = (int)p->head_dim;
    a.Dv = (int)p->value_dim;
    a.scale = p->scale;
    a.scale_log2 = p->scale * 1.4426950408889634f;
    a.causal = p->causal ? 1 : 0;
    a.mask = p->mask_allowed;
    a.mask_qbs = (int)p->mask_query_block_size;
    a.mask_kbs = (int)p->mask_key_block_size;
    a.mask_qb = (int)p->mask_query_blocks;
    a.mask_kb = (int)p->mask_key_blocks;
    a.num_q_tiles = r.num_q_tiles;
    a.num_k_tiles = r.num_k_tiles;
    a.bias_kind = p->bias_kind;
    a.alibi = p->alibi_slopes;
    a.bias = p->bias;
    int64_t bs[3];
    dense_bias_strides(p, bs);
    a.bias_sb = bs[0];
    a.bias_sh = bs[1];
    a.bias_sm = bs[2];
    a.softcap = p->softcap;
    a.inv_softcap = p->softcap > 0.0f ? 1.0f / p->softcap : 0.0f;
    a.out_f32 = p->out_dtype == OFH_DTYPE_F32 ? 1 : 0;
    a.num_splits = 1;
    a.split_tiles = 1 << 30;
    return a;
}

int fwd_impl(const ofh_attention_params* p, const void* q, const void* k, const void* v,
             void* out, void* workspace, size_t workspace_bytes, hipStream_t stream,
             bool noalloc = false) {
    if (int rc = validate(p, true, q, k, v, out)) return rc;
    Resolved r;
    if (int rc = resolve(p, q, k, v, out, r)) return rc;
    ofh::FwdArgs a = make_args(p, r, q, k, v, out);
    if (r.algorithm == OFH_ALGO_ROWWISE) {
        OFH_HIP_CHECK(ofh::launch_rowwise(a, p->dtype, stream));
        return OFH_SUCCESS;
    }
    size_t need = workspace_bytes_for(p, r);
    void* ws = workspace;
    SharedScratch* shared = nullptr;  // set when ws is the device's shared overflow buffer
    // held until this call's launches are queued when it uses library scratch
    std::unique_lock<std::mutex> scratch_lock(g_scratch_mu, std::defer_lock);
    // Once this call holds the shared buffer, its event is recorded on every
    // way out (also after a failed launch, whose earlier launches may use the
    // buffer), before the lock is released: the next user waits for them.
    struct SharedRelease {
        SharedScratch** sh;
        hipStream_t stream;
        ~SharedRelease() {  // an error path: the call's own error message stays
            if (*sh != nullptr && hipEventRecord((*sh)->last_use, stream) == hipSuccess) (*sh)->recorded = true;
        }
    } shared_release{&shared, stream};
    if (need > 0) {
        if (ws == nullptr && noalloc)  // the allocation-free entry always passes its scratch
            return set_error(OFH_ERROR_WORKSPACE_TOO_SMALL, "allocation-free call without its scratch");
        if (ws == nullptr) {
            scratch_lock.lock();
            // A stream under graph capture cannot allocate: a key split whose
            // partial rows do not fit the stream's library scratch is dropped
            // (the split only spreads the work; the result is the same).
            const bool capturing = stream_capturing(stream);
            if (capturing && r.key_splits > 1 && capture_scratch_bytes_locked(stream) < need) {
                no_key_split(p, r);
                need = workspace_bytes_for(p, r);
            }
            if (need > 0)
                if (int rc = library_scratch_locked(need, stream, capturing, &ws, &shared)) return rc;
        } else if (workspace_bytes < need) {
            // The allocation-free entry drops a key split whose partial rows
            // do not fit its static scratch (the split only spreads the work).
            if (noalloc && r.key_splits > 1) {
                no_key_split(p, r);
                need = workspace_bytes_for(p, r);
            }
            if (workspace_bytes < need)
                return set_error(OFH_ERROR_WORKSPACE_TOO_SMALL,
                                 "workspace too small: need " + std::to_string(need) + " bytes");
            if (need == 0) ws = nullptr;
        }
    }
    if (r.tile_list && !r.lds_list) {
        const size_t counts_bytes = round256((size_t)r.num_q_tiles * 4);
        ofh::TileListArgs t;
        t.M = a.M;
        t.N = a.N;
        t.block_m = r.block_m;
        t.block_n = r.block_n;
        t.causal = a.causal;
        t.mask = a.mask;
        t.mask_qbs = a.mask_qbs;
        t.mask_kbs = a.mask_kbs;
        t.mask_qb = a.mask_qb;
        t.mask_kb = a.mask_kb;
        t.num_q_tiles = r.num_q_tiles;
        t.num_k_tiles = r.num_k_tiles;
        t.counts = static_cast<int*>(ws);
        t.entries = reinterpret_cast<int*>(static_cast<char*>(ws) + counts_bytes);
        OFH_HIP_CHECK(ofh::launch_tile_lists(t, stream));
        a.tile_counts = t.counts;
        a.tile_entries = t.entries;
    }
    a.num_splits = r.key_splits;
    a.split_tiles = r.split_tiles;
    a.pair_split = r.pair_split ? 1 : 0;
    a.split_bm = r.block_m;
    a.split_bn = r.block_n;
    if (r.key_splits > 1) {
        char* base = static_cast<char*>(ws) + round256(list_bytes(r));
        a.part_o = reinterpret_cast<float*>(base);
        a.part_ml = reinterpret_cast<float*>(base + round256(partial_rows(p, r) * p->value_dim * 4));
        if (merge_in_launch(p, r))
            if (int rc = split_counters_for(stream, noalloc, &a.split_counters)) return rc;
    }
    OFH_HIP_CHECK(ofh::launch_flash_mfma(a, p->dtype, r.general_mod, stream));
    if (r.key_splits > 1 && a.split_counters == nullptr)
        OFH_HIP_CHECK(ofh::launch_combine_splits(a, p->dtype, stream));
    if (shared != nullptr) {
        SharedScratch* sh = shared;
        shared = nullptr;  // recorded here, with its status checked
        return shared_scratch_release(sh, stream);
    }
    return OFH_SUCCESS;
}

// Per-host-thread device staging for ofh_attention_fwd_host (the counterpart
// of the reference's thread_local AttentionWorkspace, batched_attention.cpp:37).
struct HostStaging {
    int device = -1;
    void* buf = nullptr;
    size_t bytes = 0;
    ~HostStaging() {
        if (buf != nullptr) (void)hipFree(buf);
    }
};
thread_local HostStaging g_staging;

void f32_to_half_bits(const float* in, uint16_t* out, size_t n, int dtype) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t x;
        std::memcpy(&x, &in[i], 4);
        if (dtype == OFH_DTYPE_BF16) {
            if ((x & 0x7fffffffu) > 0x7f800000u) {
                out[i] = (uint16_t)((x >> 16) | 0x40u);
            } else {
                x += 0x7fffu + ((x >> 16) & 1u);
                out[i] = (uint16_t)(x >> 16);
            }
        } else {
            const _Float16 h = (_Float16)in[i];  // round-to-nearest-even
            std::memcpy(&out[i], &h, 2);
        }
    }
}

}  // namespace

extern "C" {

void ofh_attention_params_init(ofh_attention_params* p) {
    if (p == nullptr) return;
    std::memset(p, 0, sizeof(*p));
    p->struct_size = sizeof(ofh_attention_params);
    p->dtype = OFH_DTYPE_F32;
    p->out_dtype = OFH_DTYPE_F32;
    p->scale = 1.0f;
    p->algorithm = OFH_ALGO_AUTO;
}

int ofh_attention_workspace_bytes(const ofh_attention_params* p, size_t* bytes) {
    if (bytes == nullptr) return set_error(OFH_ERROR_INVALID_ARGUMENT, "bytes must be non-null");
    if (int rc = validate(p, false, nullptr, nullptr, nullptr, nullptr)) return rc;
    // Alignment is not known here; assume aligned buffers (the larger answer).
    static const char dummy[16] __attribute__((aligned(16))) = {0};
    Resolved r;
    if (int rc = resolve(p, dummy, dummy, dummy, dummy, r)) return rc;
    *bytes = workspace_bytes_for(p, r);
    return OFH_SUCCESS;
}

int ofh_attention_fwd(const ofh_attention_params* p, const void* q, const void* k, const void* v,
                      void* out, void* workspace, size_t workspace_bytes, void* stream) {
    return fwd_impl(p, q, k, v, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int ofh_attention_fwd_noalloc(const ofh_attention_params* p, const void* q, const void* k,
                              const void* v, void* out, void* stream) {
    if (int rc = validate(p, true, q, k, v, out)) return rc;
    Resolved r;
    if (int rc = resolve(p, q, k, v, out, r)) return rc;
    size_t need = r.algorithm == OFH_ALGO_FLASH_MFMA ? workspace_bytes_for(p, r) : 0;
    if (need > ofh::kNoAllocScratchBytes && r.key_splits > 1) {  // fwd_impl drops the split
        no_key_split(p, r);
        need = workspace_bytes_for(p, r);
    }
    if (need > ofh::kNoAllocScratchBytes)
        return set_error(OFH_ERROR_WORKSPACE_TOO_SMALL,
                         "ofh_attention_fwd_noalloc: this call needs " + std::to_string(need) +
                             " bytes of scratch; the allocation-free entry holds at most " +
                             std::to_string(ofh::kNoAllocScratchBytes) +
                             " (use ofh_attention_fwd with a workspace)");
    // The static arrays (scratch, split counters) are looked up on every call:
    // the first call on a device materialises them there, whether or not this
    // call needs them, so no later call changes the device's memory.
    void* ws = nullptr;
    OFH_HIP_CHECK(ofh::noalloc_scratch(&ws));
    unsigned* counters = nullptr;
    OFH_HIP_CHECK(ofh::split_counter_slot(0, &counters));
    // The scratch is always handed over: fwd_impl plans the call again (with
    // its key split) and drops the split there when it does not fit.
    return fwd_impl(p, q, k, v, out, ws, ofh::kNoAllocScratchBytes, static_cast<hipStream_t>(stream), true);
}

int ofh_attention_fwd_host(const ofh_attention_params* p, const float* q, const float* k,
                           const float* v, float* out) {
    if (int rc = validate(p, true, q, k, v, out)) return rc;
    for (int i = 0; i < 3; ++i) {
        if (p->q_strides[i] || p->k_strides[i] || p->v_strides[i] || p->o_strides[i])
            return set_error(OFH_ERROR_INVALID_ARGUMENT,
                             "host entry takes the contiguous reference layout (strides must be 0)");
    }
    const size_t B = p->batch, H = p->heads, M = p->query_tokens, N = p->key_tokens;
    const size_t D = p->head_dim, Dv = p->value_dim;
    const size_t es = elem_size(p->dtype);
    const size_t nq = B * H * M * D, nk = B * H * N * D, nv = B * H * N * Dv, no = B * H * M * Dv;
    auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
    const size_t mask_n = p->mask_allowed ? p->mask_query_blocks * p->mask_key_blocks : 0;
    size_t bias_n = 0;
    if (p->bias_kind == OFH_BIAS_DENSE) {
        // host dense bias: the strides address a host tensor; stage its full extent
        int64_t s[3];
        dense_bias_strides(p, s);
        bias_n = (size_t)((int64_t)(B - 1) * s[0] + (int64_t)(H - 1) * s[1] +
                          (int64_t)(M - 1) * s[2] + (int64_t)N);
    }
    const size_t alibi_n = p->bias_kind == OFH_BIAS_ALIBI ? H : 0;
    const size_t off_q = 0, off_k = off_q + up(nq * es), off_v = off_k + up(nk * es);
    const size_t off_o = off_v + up(nv * es), off_m = off_o + up(no * 4);
    const size_t off_b = off_m + up(mask_n), off_a = off_b + up(bias_n * 4);
    // this thread's own attention workspace (tile lists, key-split partial
    // rows), so that concurrent host threads never share one
    size_t ws_n = 0;
    {
        ofh_attention_params wp = *p;
        wp.out_dtype = OFH_DTYPE_F32;
        if (int rc = ofh_attention_workspace_bytes(&wp, &ws_n)) return rc;
    }
    const size_t off_w = off_a + up(alibi_n * 4);
    const size_t total = off_w + up(ws_n);

    int dev = 0;
    OFH_HIP_CHECK(hipGetDevice(&dev));
    HostStaging& st = g_staging;
    if (st.buf != nullptr && (st.device != dev || st.bytes < total)) {
        OFH_HIP_CHECK(hipFree(st.buf));
        st.buf = nullptr;
        st.bytes = 0;
    }
    if (st.buf == nullptr) {
        OFH_HIP_CHECK(hipMalloc(&st.buf, total));
        st.bytes = total;
        st.device = dev;
    }
    char* base = static_cast<char*>(st.buf);
    auto put = [&](size_t off, const float* src, size_t n) -> int {
        if (p->dtype == OFH_DTYPE_F32) {
            OFH_HIP_CHECK(hipMemcpy(base + off, src, n * 4, hipMemcpyHostToDevice));
        } else {
            std::vector<uint16_t> tmp(n);
            f32_to_half_bits(src, tmp.data(), n, p->dtype);
            OFH_HIP_CHECK(hipMemcpy(base + off, tmp.data(), n * 2, hipMemcpyHostToDevice));
        }
        return OFH_SUCCESS;
    };
    if (int rc = put(off_q, q, nq)) return rc;
    if (int rc = put(off_k, k, nk)) return rc;
    if (int rc = put(off_v, v, nv)) return rc;
    ofh_attention_params dp = *p;
    dp.out_dtype = OFH_DTYPE_F32;
    if (mask_n) {
        OFH_HIP_CHECK(hipMemcpy(base + off_m, p->mask_allowed, mask_n, hipMemcpyHostToDevice));
        dp.mask_allowed = reinterpret_cast<const uint8_t*>(base + off_m);
    }
    if (bias_n) {
        OFH_HIP_CHECK(hipMemcpy(base + off_b, p->bias, bias_n * 4, hipMemcpyHostToDevice));
        dp.bias = reinterpret_cast<const float*>(base + off_b);
    }
    if (alibi_n) {
        OFH_HIP_CHECK(hipMemcpy(base + off_a, p->alibi_slopes, alibi_n * 4, hipMemcpyHostToDevice));
        dp.alibi_slopes = reinterpret_cast<const float*>(base + off_a);
    }
    if (int rc = fwd_impl(&dp, base + off_q, base + off_k, base + off_v, base + off_o,
                          ws_n ? base + off_w : nullptr, ws_n, nullptr))
        return rc;
    OFH_HIP_CHECK(hipMemcpy(out, base + off_o, no * 4, hipMemcpyDeviceToHost));
    OFH_HIP_CHECK(hipDeviceSynchronize());
    return OFH_SUCCESS;
}

namespace {
const char* rows32_kernel_name(int D, bool general, bool narrow) {
    static const std::vector<std::string> names = [] {
        std::vector<std::string> v;
        for (int nr = 0; nr < 2; ++nr)
            for (int d = 32; d <= 128; d += 32)
                for (int gm = 0; gm < 2; ++gm)
                    v.push_back(std::string(nr ? "flash_fwd_f32_rows16_kernel<" : "flash_fwd_f32_rows32_kernel<") +
                                std::to_string(d) + (gm ? ",general>" : ",plain>"));
        return v;
    }();
    return names[(size_t)(narrow ? 8 : 0) + (size_t)(D / 32 - 1) * 2 + (general ? 1 : 0)].c_str();
}
}  // namespace

int ofh_attention_launch_info(const ofh_attention_params* p, ofh_launch_info* info) {
    if (info == nullptr) return set_error(OFH_ERROR_INVALID_ARGUMENT, "info must be non-null");
    if (int rc = validate(p, false, nullptr, nullptr, nullptr, nullptr)) return rc;
    static const char dummy[16] __attribute__((aligned(16))) = {0};
    Resolved r;
    if (int rc = resolve(p, dummy, dummy, dummy, dummy, r)) return rc;
    std::memset(info, 0, sizeof(*info));
    info->algorithm = r.algorithm;
    info->uses_tile_list = r.tile_list ? 1 : 0;
    const char* name;
    if (r.algorithm == OFH_ALGO_FLASH_MFMA) {
        info->block_m = r.block_m;
        info->block_n = r.block_n;
        info->threads = r.threads;
        info->workgroups = (int64_t)p->batch * p->heads * (r.paired ? (r.num_q_tiles + 1) / 2 : r.num_q_tiles) *
                           r.key_splits;
        info->key_splits = r.key_splits;
        info->merge_in_launch = merge_in_launch(p, r) ? 1 : 0;
        name = (p->dtype == OFH_DTYPE_F32 && (r.block_m == ofh::kRowsF32 || r.block_m == ofh::kRowsF32Narrow))
                   ? rows32_kernel_name(r.kdim, r.general_mod, r.block_m == ofh::kRowsF32Narrow)
                   : ofh::flash_mfma_kernel_name(p->dtype, r.kdim, r.general_mod, r.tile_list, r.threads);
        // 16-bit causal pairs with a key split run the same tiling in a kernel of their own
        static thread_local std::string pair_name;
        const std::string lockstep = "flash_fwd_lockstep_kernel";
        if (r.pair_split && p->dtype != OFH_DTYPE_F32 && std::string(name).compare(0, lockstep.size(), lockstep) == 0) {
            pair_name = "flash_fwd_pair_split_kernel" + std::string(name).substr(lockstep.size());
            name = pair_name.c_str();
        }
        // 16-bit D = 192 on 8 wavefronts with value_dim <= 128: PV over 128 value columns only
        if (p->dtype != OFH_DTYPE_F32 && r.kdim == 192 && r.threads >= 512 && p->value_dim <= 128 &&
            std::string(name).compare(0, lockstep.size(), lockstep) == 0) {
            pair_name = std::string(name);
            pair_name.insert(pair_name.size() - 1, ",v128");
            name = pair_name.c_str();
        }
        // 16-bit causal query tiles run in pairs per workgroup (nqt-1-p, p)
        if (r.paired && !r.pair_split && p->dtype != OFH_DTYPE_F32 &&
            std::string(name).compare(0, lockstep.size(), lockstep) == 0) {
            pair_name = std::string(name);
            pair_name.insert(pair_name.size() - 1, ",paired");
            name = pair_name.c_str();
        }
        // 16-bit block-mask calls with their lists built in LDS: a kernel of their own
        if (r.lds_list && p->dtype != OFH_DTYPE_F32 && std::string(name).compare(0, lockstep.size(), lockstep) == 0) {
            pair_name = "flash_fwd_lds_list_kernel" + std::string(name).substr(lockstep.size());
            name = pair_name.c_str();
        }
    } else {
        info->block_m = 1;
        info->block_n = 64;
        info->threads = 256;
        info->workgroups = ((int64_t)p->batch * p->heads * p->query_tokens + 3) / 4;
        info->key_splits = 1;
        name = "rowwise_fwd_kernel";
    }
    std::strncpy(info->kernel_name, name, sizeof(info->kernel_name) - 1);
    return OFH_SUCCESS;
}

int ofh_attention_useful_flops(const ofh_attention_params* p, double* flops) {
    if (flops == nullptr) return set_error(OFH_ERROR_INVALID_ARGUMENT, "flops must be non-null");
    if (int rc = validate(p, false, nullptr, nullptr, nullptr, nullptr)) return rc;
    const size_t M = p->query_tokens, N = p->key_tokens;
    double pairs = 0.0;
    for (size_t i = 0; i < M; ++i) {
        const size_t kmax = p->causal ? std::min(N, i + 1) : N;  // keys [0, kmax) pass causal
        if (p->mask_allowed == nullptr) {
            pairs += (double)kmax;
            continue;
        }
        const size_t qb = i / p->mask_query_block_size;
        if (qb >= p->mask_query_blocks) continue;
        const uint8_t* row = p->mask_allowed + qb * p->mask_key_blocks;
        for (size_t kb = 0; kb < p->mask_key_blocks; ++kb) {
            if (!row[kb]) continue;
            const size_t ks = kb * p->mask_key_block_size;
            const size_t ke = std::min(kmax, ks + p->mask_key_block_size);
            if (ke > ks) pairs += (double)(ke - ks);
        }
    }
    *flops = 2.0 * (double)(p->head_dim + p->value_dim) * pairs * (double)p->batch * (double)p->heads;
    return OFH_SUCCESS;
}

void ofh_qk_score_params_init(ofh_qk_score_params* p) {
    if (p == nullptr) return;
    std::memset(p, 0, sizeof(*p));
    p->struct_size = sizeof(*p);
    p->batch = 1;
    p->dtype = OFH_DTYPE_F32;
    p->scale = 1.0f;
    p->algorithm = OFH_QK_AUTO;
}

int ofh_qk_score_tile(const ofh_qk_score_params* p, const void* q, const void* k, float* score,
                      void* stream) {
    if (p == nullptr) return set_error(OFH_ERROR_INVALID_ARGUMENT, "params must be non-null");
    if (p->struct_size != sizeof(*p))
        return set_error(OFH_ERROR_INVALID_ARGUMENT,
                         "ofh_qk_score_params.struct_size mismatch (call ofh_qk_score_params_init)");
    if (p->m <= 0 || p->n <= 0 || p->k <= 0)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "QK score tile dimensions must be non-zero");
    if (q == nullptr || k == nullptr || score == nullptr)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "QK score tile pointers must be non-null");
    if (p->batch <= 0) return set_error(OFH_ERROR_INVALID_ARGUMENT, "QK score tile batch must be positive");
    const int64_t strides[] = {p->a_stride_m, p->a_stride_k, p->a_stride_batch, p->b_stride_k,
                               p->b_stride_n, p->b_stride_batch, p->c_stride_m, p->c_stride_n,
                               p->c_stride_batch, p->bias_stride_m, p->bias_stride_n,
                               p->bias_stride_batch};
    for (int64_t st : strides)
        if (st < 0) return set_error(OFH_ERROR_INVALID_ARGUMENT, "QK score tile strides must be non-negative");
    if (p->dtype != OFH_DTYPE_F32 && p->dtype != OFH_DTYPE_BF16 && p->dtype != OFH_DTYPE_F16)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "unknown dtype");
    if (!(std::isfinite(p->softcap) && p->softcap >= 0.0f))
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "softcap must be finite and >= 0");
    if (p->algorithm != OFH_QK_AUTO && p->algorithm != OFH_QK_EXACT && p->algorithm != OFH_QK_MFMA)
        return set_error(OFH_ERROR_INVALID_ARGUMENT, "unknown algorithm");
    // Grid: x over 32-column blocks, y over 32-row blocks (at most 65535).
    if ((p->m + 31) / 32 > 65535 || (p->n + 31) / 32 > std::numeric_limits<int32_t>::max())
        return set_error(OFH_ERROR_UNSUPPORTED, "QK score tile exceeds the grid range");

    ofh::QkScoreArgs a{};
    a.batch = p->batch;
    a.M = p->m;
    a.N = p->n;
    a.K = p->k;
    a.q = q;
    a.k = k;
    a.c = score;
    a.a_sm = p->a_stride_m;
    a.a_sk = p->a_stride_k;
    a.a_sb = p->a_stride_batch;
    a.b_sk = p->b_stride_k;
    a.b_sn = p->b_stride_n;
    a.b_sb = p->b_stride_batch;
    a.c_sm = p->c_stride_m;
    a.c_sn = p->c_stride_n;
    a.c_sb = p->c_stride_batch;
    a.has_scale = p->has_scale != 0;
    a.scale = p->scale;
    a.bias = p->bias;
    a.bias_sm = p->bias_stride_m;
    a.bias_sn = p->bias_stride_n;
    a.bias_sb = p->bias_stride_batch;
    a.softcap = p->softcap;

    const bool mfma_ok = ofh::qk_score_mfma_supported(a, p->dtype);
    if (p->algorithm == OFH_QK_MFMA && !mfma_ok)
        return set_error(OFH_ERROR_UNSUPPORTED,
                         "MFMA QK score tile needs bf16/fp16 rows contiguous along k, 16-byte "
                         "aligned, with k % 8 == 0");
    const bool use_mfma = p->algorithm == OFH_QK_MFMA || (p->algorithm == OFH_QK_AUTO && mfma_ok);
    hipStream_t s = static_cast<hipStream_t>(stream);
    OFH_HIP_CHECK(use_mfma ? ofh::launch_qk_score_mfma(a, p->dtype, s)
                           : ofh::launch_qk_score(a, p->dtype, s));
    return OFH_SUCCESS;
}

const char* ofh_last_error(void) { return g_last_error.c_str(); }

int ofh_abi_version(void) { return OFH_ABI_VERSION; }

}  // extern "C"
