/*
 * onednn_flash_hip.h - C ABI of the MI355X (gfx950) attention forward library.
 *
 * Plain C: POD parameters, device pointers and sizes, an int status code, and
 * a thread-local error string. No C++ exceptions cross this boundary and no
 * HIP or framework types appear in the signatures (the stream is passed as
 * void*, a hipStream_t or NULL for the default stream).
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   ofh_attention_fwd            flash_attention_batched_qk_pv_tile
 *                                (include/onednn_flash/batched_attention.hpp:26-31,
 *                                 src/onednn_flash/batched_attention.cpp:9-49) and,
 *                                per head, flash_attention_qk_pv_tile_ws
 *                                (src/onednn_flash/attention.cpp:486-695)
 *   ofh_attention_fwd_host       the same entry on host fp32 buffers, as the
 *                                TensorFlow CPU op calls it
 *                                (tensorflow_ops/onednn_flash_attention_op.cc:125-134)
 *   ofh_attention_workspace_bytes
 *                                AttentionWorkspace::resize
 *                                (src/onednn_flash/attention_workspace.cpp:5-20)
 *   OFH_ALGO_ROWWISE             standard_attention
 *                                (src/onednn_flash/attention.cpp:88-137)
 *   ofh_qk_score_tile            qk_score_tile_inplace
 *                                (src/onednn_flash/qk_score_tile.cpp:353-418)
 *   ofh_last_error               the what() text of the exceptions the reference
 *                                throws (std::invalid_argument / std::runtime_error)
 */
#ifndef ONEDNN_FLASH_HIP_H
#define ONEDNN_FLASH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: ofh_attention_params gained max_key_splits and ofh_launch_info gained
 * merge_in_launch (both appended). */
#define OFH_ABI_VERSION 2

/* Status codes. INVALID_ARGUMENT corresponds to the reference's
 * std::invalid_argument, the others to std::runtime_error. */
typedef enum ofh_status {
    OFH_SUCCESS = 0,
    OFH_ERROR_INVALID_ARGUMENT = 1,
    OFH_ERROR_UNSUPPORTED = 2,
    OFH_ERROR_HIP = 3,
    OFH_ERROR_WORKSPACE_TOO_SMALL = 4
} ofh_status;

/* Element type of Q, K, V and O in device memory. */
typedef enum ofh_dtype {
    OFH_DTYPE_F32 = 0,
    OFH_DTYPE_BF16 = 1,
    OFH_DTYPE_F16 = 2
} ofh_dtype;

/* Additive score bias, applied after the scale (attention.cpp:106-107, 619). */
typedef enum ofh_bias_kind {
    OFH_BIAS_NONE = 0,
    OFH_BIAS_ALIBI = 1, /* alibi_slopes[h] * (key_index - query_index) */
    OFH_BIAS_DENSE = 2  /* bias[b*sb + h*sh + q*sq + k], fp32 */
} ofh_bias_kind;

/* Which kernel family runs. AUTO picks the MFMA flash kernel when the shape
 * is supported (head_dim and value_dim multiples of 4 for fp32 and of 8 for
 * bf16/fp16, up to 256, D != Dv allowed: the kernel of max(D, Dv)
 * rounded up to 32 runs with the padding zeroed in place; 16-byte aligned
 * rows) and the rowwise kernel otherwise. ROWWISE is the exact two-pass
 * softmax of standard_attention, run on the GPU one query row per wavefront. */
typedef enum ofh_algorithm {
    OFH_ALGO_AUTO = 0,
    OFH_ALGO_FLASH_MFMA = 1,
    OFH_ALGO_ROWWISE = 2
} ofh_algorithm;

typedef struct ofh_attention_params {
    uint32_t struct_size; /* sizeof(ofh_attention_params), set by ofh_attention_params_init */

    /* BatchedAttentionShape (batched_attention.hpp:9-16). */
    size_t batch, heads, query_tokens, key_tokens, head_dim, value_dim;

    int32_t dtype;      /* ofh_dtype of q, k, v */
    int32_t out_dtype;  /* ofh_dtype of out: the input dtype or OFH_DTYPE_F32 */

    /* Element strides for the batch, head and token axes; the last axis is
     * contiguous. All zero means the reference layout: contiguous
     * Q[B,H,M,D], K[B,H,N,D], V[B,H,N,Dv], O[B,H,M,Dv] (batched_attention.hpp:18-22). */
    int64_t q_strides[3], k_strides[3], v_strides[3], o_strides[3];

    float scale; /* AttentionOptions::scale (attention.hpp:40); default 1.0 */
    int32_t causal; /* top-left aligned: key > query is masked (attention.cpp:54-57) */

    /* BlockMask (attention.hpp:20-29): device pointer to a row-major
     * [mask_query_blocks, mask_key_blocks] uint8 bitmap, non-zero = allowed.
     * NULL means no block mask. Blocks out of range are disallowed. */
    const uint8_t* mask_allowed;
    size_t mask_query_block_size, mask_key_block_size, mask_query_blocks, mask_key_blocks;

    /* score_mod, fused into the score tile before exponentiation. Order:
     * s*scale + bias, then softcap*tanh(./softcap) when softcap > 0. Masked
     * scores get neither. */
    int32_t bias_kind;           /* ofh_bias_kind */
    const float* alibi_slopes;   /* device [heads] */
    const float* bias;           /* device fp32, see bias_strides */
    int64_t bias_strides[3];     /* batch, head, query-row strides (elements); key stride 1.
                                    All zero: one contiguous [M, N] bias for every head. */
    float softcap;               /* <= 0: disabled */

    int32_t algorithm;           /* ofh_algorithm */

    /* Key split of the MFMA kernels (no counterpart in the reference, whose
     * CPU loop has no workgroups to fill): a call whose query tiles give fewer
     * workgroups than the GPU holds runs each query tile's keys as several
     * workgroups and merges their partial rows. 0: the library chooses
     * (ofh_launch_info.key_splits); 1: never split; n > 1: at most n splits. */
    int32_t max_key_splits;
} ofh_attention_params;

/* Fills defaults: struct_size, dtype f32, out_dtype f32, scale 1.0, everything
 * else zero (no mask, no bias, AUTO). */
void ofh_attention_params_init(ofh_attention_params* p);

/* Bytes of device scratch the forward call needs for these parameters: the
 * per-query-tile list of allowed key tiles when a block mask is given, and the
 * partial rows (unnormalised O, running max and sum) when a call with few
 * query tiles splits each query tile's keys over several workgroups (see
 * ofh_launch_info.key_splits); 0 otherwise. */
int ofh_attention_workspace_bytes(const ofh_attention_params* p, size_t* bytes);

/* Attention forward on device buffers, ordered on `stream` (asynchronous).
 * workspace may be NULL: the library then uses device scratch it owns.
 *  - The first 16 streams used on a device get a buffer each (calls passing
 *    hipStreamPerThread are keyed by host thread, since that handle names a
 *    different stream in every thread; every other handle, NULL included,
 *    names one stream). A buffer grows on demand: the first call on its
 *    stream that needs more synchronises that stream (hipStreamSynchronize),
 *    frees the old buffer and calls hipMalloc. Each buffer is at least 1 MiB
 *    and as large as the largest need of a call on its stream, and it lives
 *    until the process ends.
 *  - Further streams share one overflow buffer per device. Calls that use it
 *    are ordered across streams on the device (each waits for the previous
 *    user's event, hipStreamWaitEvent, and records its own), and growing it
 *    waits on the host for its last user. The scratch stays bounded by 17
 *    buffers per device however many streams are used.
 * Such calls may block the host or allocate, so callers that must not
 * (HIP graph capture, framework ops with their own allocator) pass a
 * workspace of ofh_attention_workspace_bytes bytes instead.
 * On a stream under graph capture with workspace NULL, nothing is allocated,
 * freed or synchronised: a key split that does not fit the stream's buffer is
 * dropped (same result, one workgroup per query tile), and a call that still
 * needs scratch its stream's buffer does not hold (block-mask tile lists)
 * fails with OFH_ERROR_WORKSPACE_TOO_SMALL before anything is queued. A
 * buffer a captured graph uses is never freed while the process runs (a later
 * call that needs more gets a new one), since replays still address it.
 * Replays of a graph share that buffer with calls on the stream it was
 * captured on, so they must not overlap each other or such calls.
 * A key split with few rows per query tile (ofh_launch_info.merge_in_launch)
 * merges its partial rows in the launch itself, counting arrivals in a
 * counter slot that the library keeps per stream (keyed as above) for up to
 * 63 streams (later streams merge in a second launch); a captured graph keeps
 * its stream's slot, with the same rule for overlapping replays.
 * Calls from several host threads are safe: a thread holds the library's lock
 * from choosing the buffer until its launches are queued, and calls on
 * different streams never share a buffer without device-side ordering.
 * Fully-masked query rows are written as zeros, as standard_attention leaves
 * them (attention.cpp:111-113). */
int ofh_attention_fwd(const ofh_attention_params* p, const void* q, const void* k,
                      const void* v, void* out, void* workspace, size_t workspace_bytes,
                      void* stream);

/* ofh_attention_fwd without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory inside the call (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Its scratch (block-mask tile lists,
 * key-split partial rows) is a static device array of 16 MiB (16777216 bytes)
 * that every GPU the library runs on holds until the process ends. A key
 * split whose partial rows do not fit is dropped (the call runs unsplit, with
 * the same result); calls that still need more scratch than that (block-mask
 * lists) fail with OFH_ERROR_WORKSPACE_TOO_SMALL before any launch. It calls no hipMalloc or
 * hipFree; the first call on a device looks up that device's address of the
 * array once. All calls on one GPU share the array: calls that overlap on one
 * GPU (other streams, other host threads without ordering) race on it and
 * must be serialised by the caller. */
int ofh_attention_fwd_noalloc(const ofh_attention_params* p, const void* q, const void* k,
                              const void* v, void* out, void* stream);

/* The same computation on host fp32 buffers (contiguous reference layout):
 * copies in, runs on the current device, copies out, synchronises. The dtype
 * field selects the precision the GPU computes in (inputs are rounded to it
 * with round-to-nearest-even); out is always fp32. The mask and the ALiBi
 * slopes / dense bias are host pointers here. Device staging buffers are kept
 * per host thread and reused (no allocation after the first call of a size). */
int ofh_attention_fwd_host(const ofh_attention_params* p, const float* q, const float* k,
                           const float* v, float* out);

/* Describes the launch that ofh_attention_fwd would make. */
typedef struct ofh_launch_info {
    int32_t algorithm;        /* OFH_ALGO_FLASH_MFMA or OFH_ALGO_ROWWISE */
    int32_t block_m;          /* queries per workgroup */
    int32_t block_n;          /* keys per K/V tile */
    int32_t threads;          /* threads per workgroup */
    int64_t workgroups;       /* grid size of the attention kernel */
    int32_t uses_tile_list;   /* 1 when a block-mask tile list is built first */
    int32_t key_splits;       /* workgroups per query tile, each over a range of K/V
                                 tiles, whose partial rows are then merged */
    char kernel_name[96];
    int32_t merge_in_launch;  /* key_splits > 1: 1 when the split workgroup that finishes
                                 last merges its query tile (few rows per tile; needs a free
                                 counter slot, see ofh_attention_fwd), 0 when a second
                                 kernel merges the partial rows */
} ofh_launch_info;

int ofh_attention_launch_info(const ofh_attention_params* p, ofh_launch_info* info);

/* Useful FLOPs of the call: 4*D*(unmasked (query,key) pairs)*B*H for D == Dv
 * (2*(D+Dv)*pairs*B*H in general), counted exactly on the host from the mask.
 * The mask pointer must be a host pointer here. */
int ofh_attention_useful_flops(const ofh_attention_params* p, double* flops);

/* ---------------------------------------------------------------------------
 * QK score tile with post-ops: S = (Q K^T) * scale + bias on the device, for a
 * batch of independent strided tiles. Replaces qk_score_tile_inplace
 * (src/onednn_flash/qk_score_tile.cpp:353-418, post-ops :48-69) on device
 * buffers. Element (i, kk) of tile b of Q is q[b*a_stride_batch + i*a_stride_m
 * + kk*a_stride_k]; K^T (the reference's B operand) element (kk, j) is
 * k[b*b_stride_batch + kk*b_stride_k + j*b_stride_n] (row-major K [n,k]:
 * b_stride_k = 1, b_stride_n = k); scores are fp32. Each score is the
 * reference's sequential-k fp32 sum (one rounding per product and per add),
 * then times scale, then plus bias (OFH_QK_EXACT): bit-exact with the
 * reference for fp32 inputs, and with the fp32 upcast of bf16/fp16 inputs.
 * OFH_QK_MFMA (bf16/fp16, rows contiguous along k, 16-byte aligned, k % 8 == 0)
 * runs on the matrix cores: products are exact, the summation order differs
 * (|error| <= k * 2^-24 * sum_k |q k| before scale and bias). AUTO picks MFMA
 * for 16-bit inputs that meet its layout rule and EXACT otherwise. */
typedef enum ofh_qk_algorithm {
    OFH_QK_AUTO = 0,
    OFH_QK_EXACT = 1,
    OFH_QK_MFMA = 2
} ofh_qk_algorithm;

typedef struct ofh_qk_score_params {
    uint32_t struct_size;
    int64_t batch;                         /* number of tiles */
    int64_t m, n, k;
    int64_t a_stride_m, a_stride_k, a_stride_batch;
    int64_t b_stride_k, b_stride_n, b_stride_batch;
    int64_t c_stride_m, c_stride_n, c_stride_batch;
    int32_t dtype;                         /* ofh_dtype of Q and K */
    int32_t has_scale;
    float scale;
    const float* bias;                     /* device pointer or NULL */
    int64_t bias_stride_m, bias_stride_n, bias_stride_batch;
    float softcap;                         /* 0: off; else cap*tanh(s/cap) last */
    int32_t algorithm;                     /* ofh_qk_algorithm */
} ofh_qk_score_params;

/* Defaults: one tile, fp32, AUTO, no scale (scale 1), no bias, sizes and
 * strides zero. */
void ofh_qk_score_params_init(ofh_qk_score_params* p);

/* Stream-ordered; returns OFH_SUCCESS or an error code (ofh_last_error()).
 * Errors: zero m, n or k -> "QK score tile dimensions must be non-zero";
 * null q, k or score -> "QK score tile pointers must be non-null"
 * (qk_score_tile.cpp:16-26). */
int ofh_qk_score_tile(const ofh_qk_score_params* p, const void* q, const void* k, float* score,
                      void* stream);

/* Thread-local text of the last error on this thread ("" if none). */
const char* ofh_last_error(void);

/* OFH_ABI_VERSION the library was built with. */
int ofh_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ONEDNN_FLASH_HIP_H */
