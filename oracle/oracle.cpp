// CPU oracle for the attention forward path. TEST INFRASTRUCTURE ONLY: the
// shipped library never links or calls it. The header (oracle.h) lists the
// reference functions this file restates and the checks that pin it.
//
// Build: g++ -O3 -std=c++17 -ffp-contract=off -fPIC -shared (oracle/Makefile).
// -ffp-contract=off keeps a*b+c as two roundings, as in the reference build
// (ISO C++17 without -march=native, CMakeLists.txt:4-8).

#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_last_error;

int fail(const char* msg) {
    g_last_error = msg;
    return -1;
}

// BlockMask::allows (attention.cpp:70-86). The size validation that the
// reference repeats on every call is done once in validate() instead.
inline bool mask_allows(const oracle_params& p, size_t qi, size_t kj) {
    const size_t qb = qi / p.mask_query_block_size;
    const size_t kb = kj / p.mask_key_block_size;
    if (qb >= p.mask_query_blocks || kb >= p.mask_key_blocks) {
        return false;
    }
    return p.mask_allowed[qb * p.mask_key_blocks + kb] != 0;
}

// masked_out (attention.cpp:54-62): top-left causal, then the block mask.
inline bool masked_out(const oracle_params& p, size_t qi, size_t kj) {
    if (p.causal && kj > qi) {
        return true;
    }
    if (p.mask_allowed != nullptr && !mask_allows(p, qi, kj)) {
        return true;
    }
    return false;
}

// score_bias (attention.cpp:64-66), with the per-head ALiBi extension.
inline float score_bias(const oracle_params& p, size_t head, size_t qi, size_t kj) {
    switch (p.bias_kind) {
        case ORACLE_BIAS_ALIBI: {
            const size_t h = head % p.heads;
            const float dist = static_cast<float>(static_cast<int64_t>(kj) -
                                                  static_cast<int64_t>(qi));
            return p.alibi_slopes[h] * dist;
        }
        case ORACLE_BIAS_DENSE:
            return p.dense_bias[qi * p.key_tokens + kj];
        default:
            return 0.0f;
    }
}

// Scale, bias (attention.cpp:106-107 / 619) and the soft-cap extension, which
// comes last, before exponentiation.
inline float finish_score(const oracle_params& p, float dot, float bias) {
    float s = dot * p.scale + bias;
    if (p.softcap > 0.0f) {
        s = p.softcap * std::tanh(s / p.softcap);
    }
    return s;
}

int validate(const oracle_params* p) {
    if (p == nullptr) return fail("params must be non-null");
    if (p->batch == 0 || p->heads == 0 || p->query_tokens == 0 || p->key_tokens == 0 ||
        p->head_dim == 0 || p->value_dim == 0) {
        return fail("attention dimensions must be non-zero");
    }
    if (p->mask_allowed != nullptr) {
        if (p->mask_query_block_size == 0 || p->mask_key_block_size == 0) {
            return fail("BlockMask block sizes must be non-zero");
        }
        if (p->mask_query_blocks == 0 || p->mask_key_blocks == 0) {
            return fail("BlockMask dimensions must be non-zero");
        }
    }
    if (p->bias_kind == ORACLE_BIAS_ALIBI && p->alibi_slopes == nullptr) {
        return fail("ALiBi bias needs per-head slopes");
    }
    if (p->bias_kind == ORACLE_BIAS_DENSE && p->dense_bias == nullptr) {
        return fail("dense bias needs a bias matrix");
    }
    if (p->bias_kind < 0 || p->bias_kind > 2) return fail("unknown bias kind");
    return 0;
}

// dot_row (attention.cpp:40-52): fp32, sequential over d.
inline float dot_row(const float* a, const float* b, size_t width) {
    float sum = 0.0f;
    for (size_t d = 0; d < width; ++d) {
        sum += a[d] * b[d];
    }
    return sum;
}

// One output row of standard_attention (attention.cpp:98-133). `scores` is a
// scratch row of key_tokens floats. Returns false when the row has no valid
// key (the caller leaves it at 0, attention.cpp:111-113).
bool standard_row(const oracle_params& p, size_t head, size_t qi, const float* q,
                  const float* k, const float* v, float* scores, float* out_row) {
    const size_t N = p.key_tokens, D = p.head_dim, Dv = p.value_dim;
    const float neg_inf = -std::numeric_limits<float>::infinity();
    float row_max = neg_inf;
    bool has_valid_key = false;
    for (size_t kj = 0; kj < N; ++kj) {
        if (masked_out(p, qi, kj)) {
            scores[kj] = neg_inf;
            continue;
        }
        scores[kj] = finish_score(p, dot_row(q + qi * D, k + kj * D, D),
                                  score_bias(p, head, qi, kj));
        row_max = std::max(row_max, scores[kj]);
        has_valid_key = true;
    }
    if (!has_valid_key) {
        for (size_t vd = 0; vd < Dv; ++vd) out_row[vd] = 0.0f;
        return false;
    }
    float denom = 0.0f;
    for (size_t kj = 0; kj < N; ++kj) {
        if (std::isinf(scores[kj]) && scores[kj] < 0.0f) continue;
        scores[kj] = std::exp(scores[kj] - row_max);
        denom += scores[kj];
    }
    for (size_t vd = 0; vd < Dv; ++vd) {
        float acc = 0.0f;
        for (size_t kj = 0; kj < N; ++kj) {
            if (std::isinf(scores[kj]) && scores[kj] < 0.0f) continue;
            acc += scores[kj] * v[kj * Dv + vd];
        }
        out_row[vd] = acc / denom;
    }
    return true;
}

// Per-thread tile buffers, the counterpart of AttentionWorkspace
// (attention_workspace.hpp:16-47, attention_workspace.cpp:5-20).
struct Workspace {
    std::vector<float> score_tile, p_tile, pv_tile, running_max, running_sum, acc,
        old_scales, new_maxes, block_sums;
    std::vector<uint8_t> row_has_valid;
    void resize(size_t q_bs, size_t k_bs, size_t Dv) {
        score_tile.resize(q_bs * k_bs);
        p_tile.resize(q_bs * k_bs);
        pv_tile.resize(q_bs * Dv);
        running_max.resize(q_bs);
        running_sum.resize(q_bs);
        acc.resize(q_bs * Dv);
        old_scales.resize(q_bs);
        new_maxes.resize(q_bs);
        block_sums.resize(q_bs);
        row_has_valid.resize(q_bs);
    }
};

// flash_attention_qk_pv_tile_ws for one head (attention.cpp:486-695) with the
// Reference tile kernels and the StridedK QK layout (attention.cpp:580-599,
// tile_kernel.cpp:49-86).
void flash_head(const oracle_params& p, size_t head, const float* q, const float* k,
                const float* v, float* output, size_t q_bs, size_t k_bs, Workspace& ws) {
    const size_t M = p.query_tokens, N = p.key_tokens, D = p.head_dim, Dv = p.value_dim;
    const float neg_inf = -std::numeric_limits<float>::infinity();
    ws.resize(q_bs, k_bs, Dv);

    for (size_t q_block_begin = 0; q_block_begin < M; q_block_begin += q_bs) {
        const size_t q_block_end = std::min(M, q_block_begin + q_bs);
        const size_t q_rows = q_block_end - q_block_begin;
        const float* q_tile = q + q_block_begin * D;

        for (size_t i = 0; i < q_rows; ++i) {
            ws.running_max[i] = neg_inf;
            ws.running_sum[i] = 0.0f;
            ws.row_has_valid[i] = 0;
        }
        std::fill(ws.acc.begin(), ws.acc.begin() + q_rows * Dv, 0.0f);

        for (size_t k_block_begin = 0; k_block_begin < N; k_block_begin += k_bs) {
            const size_t k_block_end = std::min(N, k_block_begin + k_bs);
            const size_t k_cols = k_block_end - k_block_begin;
            if (p.causal && k_block_begin >= q_block_end) break;

            // QK tile through the strided B view of row-major K (tile_kernel.cpp:68-86).
            const float* k_tile = k + k_block_begin * D;
            for (size_t i = 0; i < q_rows; ++i) {
                for (size_t j = 0; j < k_cols; ++j) {
                    float sum = 0.0f;
                    for (size_t kk = 0; kk < D; ++kk) {
                        sum += q_tile[i * D + kk] * k_tile[kk + j * D];
                    }
                    ws.score_tile[i * k_cols + j] = sum;
                }
            }

            for (size_t i = 0; i < q_rows; ++i) {
                ws.new_maxes[i] = ws.running_max[i];
                ws.block_sums[i] = 0.0f;
                ws.row_has_valid[i] = 0;
            }
            for (size_t lk = 0; lk < q_rows; ++lk) {
                const size_t qi = q_block_begin + lk;
                float block_max = neg_inf;
                for (size_t kk = 0; kk < k_cols; ++kk) {
                    const size_t kj = k_block_begin + kk;
                    float& score = ws.score_tile[lk * k_cols + kk];
                    if (masked_out(p, qi, kj)) {
                        score = neg_inf;
                        continue;
                    }
                    score = finish_score(p, score, score_bias(p, head, qi, kj));
                    block_max = std::max(block_max, score);
                    ws.row_has_valid[lk] = 1;
                }
                if (!ws.row_has_valid[lk]) continue;
                const float new_max = std::max(ws.running_max[lk], block_max);
                ws.new_maxes[lk] = new_max;
                ws.old_scales[lk] = std::isinf(ws.running_max[lk]) && ws.running_max[lk] < 0.0f
                                        ? 0.0f
                                        : std::exp(ws.running_max[lk] - new_max);
                for (size_t kk = 0; kk < k_cols; ++kk) {
                    const float score = ws.score_tile[lk * k_cols + kk];
                    if (std::isinf(score) && score < 0.0f) {
                        ws.p_tile[lk * k_cols + kk] = 0.0f;
                        continue;
                    }
                    const float weight = std::exp(score - new_max);
                    ws.p_tile[lk * k_cols + kk] = weight;
                    ws.block_sums[lk] += weight;
                }
            }

            // PV tile, contiguous reference GEMM (tile_kernel.cpp:49-66). Rows
            // without a valid key are skipped: the reference computes them from
            // stale P values and then discards them (attention.cpp:663-665).
            const float* v_tile = v + k_block_begin * Dv;
            for (size_t i = 0; i < q_rows; ++i) {
                if (!ws.row_has_valid[i]) continue;
                for (size_t j = 0; j < Dv; ++j) {
                    float sum = 0.0f;
                    for (size_t kk = 0; kk < k_cols; ++kk) {
                        sum += ws.p_tile[i * k_cols + kk] * v_tile[kk * Dv + j];
                    }
                    ws.pv_tile[i * Dv + j] = sum;
                }
            }

            for (size_t lk = 0; lk < q_rows; ++lk) {
                if (!ws.row_has_valid[lk]) continue;
                const float old_scale = ws.old_scales[lk];
                for (size_t vd = 0; vd < Dv; ++vd) {
                    ws.acc[lk * Dv + vd] = ws.acc[lk * Dv + vd] * old_scale + ws.pv_tile[lk * Dv + vd];
                }
                ws.running_sum[lk] = ws.running_sum[lk] * old_scale + ws.block_sums[lk];
                ws.running_max[lk] = ws.new_maxes[lk];
            }
        }

        for (size_t lk = 0; lk < q_rows; ++lk) {
            const size_t qi = q_block_begin + lk;
            if (ws.running_sum[lk] <= 0.0f) continue;  // left untouched (attention.cpp:680-682)
            const float inv = 1.0f / ws.running_sum[lk];
            for (size_t vd = 0; vd < Dv; ++vd) {
                output[qi * Dv + vd] = ws.acc[lk * Dv + vd] * inv;
            }
        }
    }
}

template <typename Fn>
void parallel_for(size_t count, int threads, Fn&& fn) {
    const size_t t = static_cast<size_t>(std::max(1, threads));
    if (t == 1 || count <= 1) {
        for (size_t i = 0; i < count; ++i) fn(i, 0);
        return;
    }
    const size_t nt = std::min(t, count);
    std::vector<std::thread> pool;
    pool.reserve(nt);
    for (size_t w = 0; w < nt; ++w) {
        pool.emplace_back([&, w]() {
            for (size_t i = w; i < count; i += nt) fn(i, w);
        });
    }
    for (auto& th : pool) th.join();
}

inline uint32_t f32_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
inline float bits_f32(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

extern "C" {

const char* oracle_last_error(void) { return g_last_error.c_str(); }

int oracle_standard_attention(const float* q, const float* k, const float* v, float* out,
                              const oracle_params* p) {
    if (int rc = validate(p)) return rc;
    if (!q || !k || !v || !out) return fail("attention pointers must be non-null");
    const size_t M = p->query_tokens, N = p->key_tokens, D = p->head_dim, Dv = p->value_dim;
    std::vector<float> scores(N);
    for (size_t bh = 0; bh < p->batch * p->heads; ++bh) {
        for (size_t qi = 0; qi < M; ++qi) {
            standard_row(*p, bh, qi, q + bh * M * D, k + bh * N * D, v + bh * N * Dv,
                         scores.data(), out + bh * M * Dv + qi * Dv);
        }
    }
    return 0;
}

int oracle_standard_attention_rows(const float* q, const float* k, const float* v,
                                   const oracle_params* p, const size_t* head_idx,
                                   const size_t* rows, size_t nrows, float* out_rows,
                                   int threads) {
    if (int rc = validate(p)) return rc;
    if (!q || !k || !v || !out_rows || !head_idx || !rows) return fail("pointers must be non-null");
    const size_t M = p->query_tokens, N = p->key_tokens, D = p->head_dim, Dv = p->value_dim;
    for (size_t i = 0; i < nrows; ++i) {
        if (head_idx[i] >= p->batch * p->heads || rows[i] >= M) return fail("row index out of range");
    }
    std::vector<std::vector<float>> scratch(static_cast<size_t>(std::max(1, threads)),
                                            std::vector<float>(N));
    parallel_for(nrows, threads, [&](size_t i, size_t w) {
        const size_t bh = head_idx[i];
        standard_row(*p, bh, rows[i], q + bh * M * D, k + bh * N * D, v + bh * N * Dv,
                     scratch[w].data(), out_rows + i * Dv);
    });
    return 0;
}

int oracle_flash_heads(const float* q, const float* k, const float* v, float* out,
                       const oracle_params* p, const size_t* head_idx, size_t nheads,
                       size_t query_block_size, size_t key_block_size, int threads) {
    if (int rc = validate(p)) return rc;
    if (!q || !k || !v || !out || !head_idx) return fail("attention pointers must be non-null");
    if (key_block_size == 0) return fail("key_block_size must be non-zero");
    if (query_block_size == 0) return fail("query_block_size must be non-zero");
    const size_t M = p->query_tokens, N = p->key_tokens, D = p->head_dim, Dv = p->value_dim;
    for (size_t i = 0; i < nheads; ++i) {
        if (head_idx[i] >= p->batch * p->heads) return fail("head index out of range");
    }
    std::vector<Workspace> ws(static_cast<size_t>(std::max(1, threads)));
    parallel_for(nheads, threads, [&](size_t i, size_t w) {
        const size_t bh = head_idx[i];
        flash_head(*p, bh, q + bh * M * D, k + bh * N * D, v + bh * N * Dv, out + i * M * Dv,
                   query_block_size, key_block_size, ws[w]);
    });
    return 0;
}

int oracle_flash_batched(const float* q, const float* k, const float* v, float* out,
                         const oracle_params* p, size_t query_block_size,
                         size_t key_block_size, int threads) {
    if (int rc = validate(p)) return rc;
    std::vector<size_t> heads(p->batch * p->heads);
    for (size_t i = 0; i < heads.size(); ++i) heads[i] = i;
    return oracle_flash_heads(q, k, v, out, p, heads.data(), heads.size(), query_block_size,
                              key_block_size, threads);
}

void oracle_f32_to_bf16(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t x = f32_bits(in[i]);
        if ((x & 0x7fffffffu) > 0x7f800000u) {
            out[i] = static_cast<uint16_t>((x >> 16) | 0x0040u);  // quiet NaN
            continue;
        }
        x += 0x7fffu + ((x >> 16) & 1u);
        out[i] = static_cast<uint16_t>(x >> 16);
    }
}

void oracle_bf16_to_f32(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = bits_f32(static_cast<uint32_t>(in[i]) << 16);
}

void oracle_f32_to_f16(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t x = f32_bits(in[i]);
        const uint32_t sign = (x >> 16) & 0x8000u;
        const uint32_t a = x & 0x7fffffffu;
        uint32_t h;
        if (a > 0x7f800000u) {
            h = 0x7e00u;                     // NaN
        } else if (a >= 0x47800000u) {
            h = 0x7c00u;                     // |x| >= 2^16 (and inf): overflow to inf
        } else if (a < 0x38800000u) {
            // below 2^-14: fp16 subnormal (or zero). x * 2^24 is exact here and
            // nearbyint rounds half to even in the default rounding mode.
            const float scaled = bits_f32(a) * 16777216.0f;
            h = static_cast<uint32_t>(std::nearbyint(scaled));  // 1024 encodes 2^-14
        } else {
            const uint32_t mant = a & 0x7fffffu;
            const uint32_t exp = a >> 23;
            h = ((exp - 112u) << 10) | (mant >> 13);
            const uint32_t rem = mant & 0x1fffu;
            if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;  // may carry to inf
        }
        out[i] = static_cast<uint16_t>(sign | h);
    }
}

void oracle_f16_to_f32(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t h = in[i];
        const uint32_t sign = (h & 0x8000u) << 16;
        const uint32_t exp = (h >> 10) & 0x1fu;
        const uint32_t mant = h & 0x3ffu;
        float f;
        if (exp == 0) {
            f = static_cast<float>(mant) * (1.0f / 16777216.0f);  // mant * 2^-24, exact
            f = bits_f32(f32_bits(f) | sign);
        } else if (exp == 31) {
            f = bits_f32(sign | 0x7f800000u | (mant << 13));
        } else {
            f = bits_f32(sign | ((exp + 112u) << 23) | (mant << 13));
        }
        out[i] = f;
    }
}

int oracle_qk_score_tile(const float* q, const float* k, float* score, const oracle_qk_shape* s,
                         int has_scale, float scale, const float* bias, float softcap) {
    if (s == nullptr) return fail("shape must be non-null");
    if (s->m == 0 || s->n == 0 || s->k == 0) return fail("QK score tile dimensions must be non-zero");
    if (q == nullptr || k == nullptr || score == nullptr)
        return fail("QK score tile pointers must be non-null");
    for (size_t b = 0; b < s->batch; ++b) {
        const float* qb = q + b * s->a_sb;
        const float* kb = k + b * s->b_sb;
        float* cb = score + b * s->c_sb;
        for (size_t i = 0; i < s->m; ++i) {
            for (size_t j = 0; j < s->n; ++j) {
                float sum = 0.0f;
                for (size_t kk = 0; kk < s->k; ++kk) sum += qb[i * s->a_sm + kk * s->a_sk] * kb[kk * s->b_sk + j * s->b_sn];
                if (has_scale) sum *= scale;
                if (bias != nullptr) sum += bias[b * s->bias_sb + i * s->bias_sm + j * s->bias_sn];
                if (softcap > 0.0f) sum = softcap * std::tanh(sum / softcap);
                cb[i * s->c_sm + j * s->c_sn] = sum;
            }
        }
    }
    return 0;
}

uint64_t oracle_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void oracle_fill_normal(uint64_t seed, size_t n, float mean, float stddev, float* out,
                        int threads) {
    const uint64_t base = oracle_splitmix64(seed);
    const double two_pi = 6.283185307179586476925286766559;
    const size_t chunk = 1u << 16;
    const size_t nchunks = (n + chunk - 1) / chunk;
    parallel_for(nchunks, threads, [&](size_t c, size_t) {
        const size_t end = std::min(n, (c + 1) * chunk);
        for (size_t i = c * chunk; i < end; ++i) {
            const uint64_t h1 = oracle_splitmix64(base + 2 * static_cast<uint64_t>(i));
            const uint64_t h2 = oracle_splitmix64(base + 2 * static_cast<uint64_t>(i) + 1);
            const double u1 = static_cast<double>((h1 >> 11) + 1) * (1.0 / 9007199254740992.0);
            const double u2 = static_cast<double>(h2 >> 11) * (1.0 / 9007199254740992.0);
            const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
            out[i] = static_cast<float>(static_cast<double>(mean) + static_cast<double>(stddev) * z);
        }
    });
}

}  // extern "C"
