/*
 * CPU oracle for the Flash-style attention forward path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or
 * calls this code; the tests compare the HIP kernels with it, and bench.py
 * times it as the CPU baseline beside them.
 *
 * It restates, in plain C++ with the same floating-point operation order, the
 * reference's CPU attention (paths relative to the reference repository):
 *   - standard_attention            src/onednn_flash/attention.cpp:88-137
 *   - flash_attention_qk_pv_tile_ws src/onednn_flash/attention.cpp:486-695
 *   - flash_attention_batched_qk_pv_tile
 *                                   src/onednn_flash/batched_attention.cpp:9-49
 *   - strided/contiguous reference tile GEMMs
 *                                   src/onednn_flash/tile_kernel.cpp:49-86
 *   - masked_out / BlockMask::allows / score_bias
 *                                   src/onednn_flash/attention.cpp:54-86
 *   - the QK score tile with scale and bias post-ops
 *                                   src/onednn_flash/qk_score_tile.cpp:48-69
 * and extends it with what the reference does not have:
 *   - a per-head ALiBi bias slope_h*(k-q) (the reference ScoreBiasFn has no head
 *     index, include/onednn_flash/attention.hpp:31),
 *   - a tanh soft-cap  cap*tanh(x/cap)  applied after scale+bias on unmasked
 *     scores only,
 *   - RNE rounding to bf16 / fp16,
 *   - a portable counter-based normal generator.
 *
 * Parity pins (tests/test_oracle.py): golden vectors written by the compiled
 * reference (tests/golden/), closed forms (K=0 gives the mean of V, N=1 gives
 * V[0], a dominant score selects its V row, an all-ones mask equals no mask,
 * ALiBi slope*(k-q) equals slope*k under softmax), brute force in double
 * precision, and bit-level rounding cases checked against torch's casts.
 */
#ifndef ONEDNN_FLASH_ORACLE_H
#define ONEDNN_FLASH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORACLE_BIAS_NONE = 0,
    ORACLE_BIAS_ALIBI = 1, /* slope_h * (k - q) */
    ORACLE_BIAS_DENSE = 2  /* dense[q * N + k], shared by every head */
};

/* One attention problem over a batch of heads. Tensors are contiguous
 * Q[B,H,M,D], K[B,H,N,D], V[B,H,N,Dv], O[B,H,M,Dv] in fp32. */
typedef struct oracle_params {
    size_t batch, heads, query_tokens, key_tokens, head_dim, value_dim;
    float scale;
    int causal;
    /* BlockMask (attention.hpp:20-29); allowed == NULL means no block mask. */
    const uint8_t* mask_allowed;
    size_t mask_query_block_size, mask_key_block_size, mask_query_blocks, mask_key_blocks;
    int bias_kind;
    const float* alibi_slopes; /* [heads] for ORACLE_BIAS_ALIBI */
    const float* dense_bias;   /* [M*N] for ORACLE_BIAS_DENSE */
    float softcap;             /* <= 0: no soft-cap */
} oracle_params;

/* 0 on success, -1 on invalid arguments (message in oracle_last_error()). */
const char* oracle_last_error(void);

/* standard_attention over every head; fully-masked rows are written as 0. */
int oracle_standard_attention(const float* q, const float* k, const float* v, float* out,
                              const oracle_params* p);

/* standard_attention for a subset of (head, row) pairs: out_rows[i*Dv..] is
 * the output row rows[i] of flat head heads_idx[i] (= b*H + h). Rows are
 * independent, so a sampled row equals the full computation's row. */
int oracle_standard_attention_rows(const float* q, const float* k, const float* v,
                                   const oracle_params* p, const size_t* head_idx,
                                   const size_t* rows, size_t nrows, float* out_rows,
                                   int threads);

/* flash_attention_batched_qk_pv_tile with the reference-kernel GEMMs and the
 * StridedK QK layout, heads split over `threads` host threads (each with its
 * own workspace). Rows without any valid key are left untouched, as in the
 * reference (attention.cpp:680-682). */
int oracle_flash_batched(const float* q, const float* k, const float* v, float* out,
                         const oracle_params* p, size_t query_block_size,
                         size_t key_block_size, int threads);

/* Same as oracle_flash_batched on an explicit list of flat heads (for a
 * bounded CPU-baseline sample). out is laid out as [nheads, M, Dv]. */
int oracle_flash_heads(const float* q, const float* k, const float* v, float* out,
                       const oracle_params* p, const size_t* head_idx, size_t nheads,
                       size_t query_block_size, size_t key_block_size, int threads);

/* Round-to-nearest-even conversions. */
void oracle_f32_to_bf16(const float* in, uint16_t* out, size_t n);
void oracle_bf16_to_f32(const uint16_t* in, float* out, size_t n);
void oracle_f32_to_f16(const float* in, uint16_t* out, size_t n);
void oracle_f16_to_f32(const uint16_t* in, float* out, size_t n);

/* Counter-based N(mean, std) generator: element i depends only on (seed, i).
 * splitmix64 finaliser over (seed, i) -> two 53-bit uniforms -> Box-Muller
 * (cosine branch), computed in double, rounded to float. */
/* QK score tile with post-ops over a batch of strided tiles, as
 * qk_score_tile_inplace's reference path (src/onednn_flash/qk_score_tile.cpp:
 * 48-69 after matmul_tile_reference_strided_inplace, tile_kernel.cpp:67-86):
 *   s = sum_kk q[i,kk]*k[kk,j]  (fp32, kk ascending, one rounding per op)
 *   s = s*scale (if has_scale);  s = s + bias[i,j] (if bias);
 *   s = cap*tanh(s/cap) (if softcap > 0; an extension, not in the reference).
 * Strides are in elements; q index b*a_sb + i*a_sm + kk*a_sk, k index
 * b*b_sb + kk*b_sk + j*b_sn (the K^T view), score b*c_sb + i*c_sm + j*c_sn. */
typedef struct oracle_qk_shape {
    size_t batch, m, n, k;
    size_t a_sm, a_sk, a_sb, b_sk, b_sn, b_sb, c_sm, c_sn, c_sb;
    size_t bias_sm, bias_sn, bias_sb;
} oracle_qk_shape;

int oracle_qk_score_tile(const float* q, const float* k, float* score, const oracle_qk_shape* s,
                         int has_scale, float scale, const float* bias, float softcap);

void oracle_fill_normal(uint64_t seed, size_t n, float mean, float stddev, float* out,
                        int threads);
uint64_t oracle_splitmix64(uint64_t x);

#ifdef __cplusplus
}
#endif

#endif /* ONEDNN_FLASH_ORACLE_H */
