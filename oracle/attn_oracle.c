/*
 * CPU oracle for the paged-attention path — TEST INFRASTRUCTURE ONLY.
 * Restates the reference's attention loops (src/model_q8.cpp) in plain C with
 * the same loop order, formulas and OpenMP decomposition; built with the
 * reference's flags (-O3 -ffast-math -fopenmp, AVX2 target).  Layouts and the
 * pin of each function are listed in attn_oracle.h.
 */
#include "attn_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define PAGE ORACLE_PAGE_TOKENS

static inline size_t page_floats(int n_layers, int kv_dim) {
    return (size_t)n_layers * PAGE * (size_t)kv_dim;
}

static inline int pick_threads(int n_threads) {
    return n_threads > 0 ? n_threads : omp_get_num_procs();
}

int oracle_max_threads(void) { return omp_get_num_procs(); }

/* src/model_q8.cpp:142-159 — max starts at (float)INT32_MIN, expf, sum, divide. */
void oracle_softmax(float* x, int size) {
    float max_val = (float)INT32_MIN;
    for (int i = 0; i < size; i++) {
        if (x[i] > max_val) max_val = x[i];
    }
    float sum = 0.0f;
    for (int i = 0; i < size; i++) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    for (int i = 0; i < size; i++) x[i] /= sum;
}

/*
 * src/model_q8.cpp:601-615 (decode; the same loop at :457-471 for prefill rows
 * and :262-274 for the single-sequence path): for each pair (j, j+1) of a row,
 * with hd_j = j % head_size, (fcr, fci) = freq[pos*(head_size/2) + hd_j/2],
 * q' = (q0*fcr - q1*fci, q0*fci + q1*fcr); the first kv_dim entries of k
 * rotate the same way.  Row r is at position positions[r].
 */
void oracle_rope(float* q, float* k, int rows, const int32_t* positions,
                 const float* freq_real, const float* freq_imag, int dim, int kv_dim,
                 int head_size) {
    for (int r = 0; r < rows; r++) {
        int pos = positions[r];
        float* qb = q + (size_t)r * dim;
        float* kb = k + (size_t)r * kv_dim;
        for (int j = 0; j < dim; j += 2) {
            int head_dim = j % head_size;
            float fcr = freq_real[pos * (head_size / 2) + (head_dim / 2)];
            float fci = freq_imag[pos * (head_size / 2) + (head_dim / 2)];
            float q0 = qb[j];
            float q1 = qb[j + 1];
            qb[j] = q0 * (fcr)-q1 * fci;
            qb[j + 1] = q0 * fci + q1 * fcr;
            if (j < kv_dim) {
                float k0 = kb[j];
                float k1 = kb[j + 1];
                kb[j] = k0 * fcr - k1 * fci;
                kb[j + 1] = k0 * fci + k1 * fcr;
            }
        }
    }
}

/* src/model_q8.cpp:616-623 — page = table[pos/16], row = pos%16, layer offset l*16*kv_dim. */
void oracle_kv_append_decode(float* k_pool, float* v_pool, int n_layers, int kv_dim, int layer,
                             const float* k, const float* v, const int32_t* tables, int max_pages,
                             const int32_t* positions, int batch) {
    const size_t pf = page_floats(n_layers, kv_dim);
    for (int b = 0; b < batch; b++) {
        int pos = positions[b];
        int phy_id = tables[(size_t)b * max_pages + pos / PAGE];
        int block_off = pos % PAGE;
        size_t layer_off = (size_t)layer * PAGE * kv_dim;
        memcpy(k_pool + phy_id * pf + layer_off + (size_t)block_off * kv_dim,
               k + (size_t)b * kv_dim, (size_t)kv_dim * sizeof(float));
        memcpy(v_pool + phy_id * pf + layer_off + (size_t)block_off * kv_dim,
               v + (size_t)b * kv_dim, (size_t)kv_dim * sizeof(float));
    }
}

/* src/model_q8.cpp:473-484 — scatter the chunk's K/V rows at start_pos+t. */
void oracle_kv_scatter_prefill(float* k_pool, float* v_pool, int n_layers, int kv_dim, int layer,
                               const float* k, const float* v, const int32_t* table,
                               int start_pos, int num_tokens) {
    const size_t pf = page_floats(n_layers, kv_dim);
    size_t layer_off = (size_t)layer * PAGE * kv_dim;
    for (int t = 0; t < num_tokens; t++) {
        int pos = start_pos + t;
        int phy_id = table[pos / PAGE];
        int block_off = pos % PAGE;
        memcpy(k_pool + phy_id * pf + layer_off + (size_t)block_off * kv_dim,
               k + (size_t)t * kv_dim, (size_t)kv_dim * sizeof(float));
        memcpy(v_pool + phy_id * pf + layer_off + (size_t)block_off * kv_dim,
               v + (size_t)t * kv_dim, (size_t)kv_dim * sizeof(float));
    }
}

/*
 * src/model_q8.cpp:625-662 — batched decode: per (b,h) scores over pages
 * 0..pos/16 (rows up to pos%16 on the last page), each divided by
 * sqrtf(head_size); softmax over pos+1 scores; then o = sum_t att[t]*v_t.
 * OpenMP collapse(2) over (b,h) as in the reference.  The reference's score
 * scratch s->attn[b][h][seq_len] is allocated here per call.
 */
int oracle_decode_batch(const float* k_pool, const float* v_pool, int n_layers, int kv_dim,
                        int layer, const float* q, float* out, const int32_t* tables,
                        int max_pages, const int32_t* positions, int batch, int n_heads,
                        int n_kv_heads, int head_dim, int n_threads) {
    if (batch <= 0) return 0;
    const int dim = n_heads * head_dim;
    const int kv_mul = n_heads / n_kv_heads;
    const size_t pf = page_floats(n_layers, kv_dim);
    int max_ctx = 0;
    for (int b = 0; b < batch; b++)
        if (positions[b] + 1 > max_ctx) max_ctx = positions[b] + 1;
    float* attn = (float*)malloc((size_t)batch * n_heads * max_ctx * sizeof(float));
    if (!attn) return -1;
#pragma omp parallel for collapse(2) num_threads(pick_threads(n_threads))
    for (int b = 0; b < batch; b++) {
        for (int h = 0; h < n_heads; h++) {
            int pos = positions[b];
            const int32_t* block_table = tables + (size_t)b * max_pages;
            const float* qh = q + (size_t)b * dim + (size_t)h * head_dim;
            float* att = attn + ((size_t)b * n_heads + h) * max_ctx;
            int kv_h = h / kv_mul;
            size_t layer_off = (size_t)layer * PAGE * kv_dim;
            int num_full_blocks = pos / PAGE;
            for (int blk = 0; blk <= num_full_blocks; blk++) {
                int phy_id = block_table[blk];
                int end_t_off = (blk == num_full_blocks) ? (pos % PAGE) : (PAGE - 1);
                const float* k_base = k_pool + phy_id * pf + layer_off + (size_t)kv_h * head_dim;
                for (int t_off = 0; t_off <= end_t_off; t_off++) {
                    const float* k = k_base + (size_t)t_off * kv_dim;
                    float raw_score = 0.0f;
                    for (int p = 0; p < head_dim; p++) raw_score += qh[p] * k[p];
                    att[blk * PAGE + t_off] = raw_score / sqrtf((float)head_dim);
                }
            }
            oracle_softmax(att, pos + 1);
            float* xb_out = out + (size_t)b * dim + (size_t)h * head_dim;
            for (int p = 0; p < head_dim; p++) xb_out[p] = 0.0f;
            for (int blk = 0; blk <= num_full_blocks; blk++) {
                int phy_id = block_table[blk];
                const float* v_base = v_pool + phy_id * pf + layer_off + (size_t)kv_h * head_dim;
                int end_t_offset = (blk == num_full_blocks) ? (pos % PAGE) : (PAGE - 1);
                for (int t_off = 0; t_off <= end_t_offset; t_off++) {
                    const float* v = v_base + (size_t)t_off * kv_dim;
                    float a = att[blk * PAGE + t_off];
                    for (int p = 0; p < head_dim; p++) xb_out[p] += a * v[p];
                }
            }
        }
    }
    free(attn);
    return 0;
}

/*
 * src/model_q8.cpp:290-347 — single-sequence decode with AVX2: the q.k dot is
 * an 8-wide _mm256_fmadd_ps chain followed by the reference's fixed
 * horizontal-sum sequence (:306-321); PV is an 8-wide FMA into the output row
 * (:329-346).  OpenMP over heads.  Requires head_dim % 8 == 0.
 */
int oracle_decode_single_avx2(const float* k_pool, const float* v_pool, int n_layers, int kv_dim,
                              int layer, const float* q, float* out, const int32_t* table,
                              int pos, int n_heads, int n_kv_heads, int head_dim, int n_threads) {
    if (head_dim % 8 != 0) return -2;
    const int kv_mul = n_heads / n_kv_heads;
    const size_t pf = page_floats(n_layers, kv_dim);
    float* attn = (float*)malloc((size_t)n_heads * (pos + 1) * sizeof(float));
    if (!attn) return -1;
    size_t layer_off = (size_t)layer * PAGE * kv_dim;
#pragma omp parallel for num_threads(pick_threads(n_threads))
    for (int h = 0; h < n_heads; h++) {
        const float* qh = q + (size_t)h * head_dim;
        float* att = attn + (size_t)h * (pos + 1);
        int kv_h = h / kv_mul;
        int num_full_blocks = pos >> 4;
        for (int b = 0; b <= num_full_blocks; b++) {
            int t_physical_id = table[b];
            int end_t_offset = (b == num_full_blocks) ? (pos & 15) : 15;
            const float* k_base = k_pool + t_physical_id * pf + layer_off + (size_t)kv_h * head_dim;
            for (int t_off = 0; t_off <= end_t_offset; t_off++) {
                const float* k = k_base + (size_t)t_off * kv_dim;
                __m256 sum_vec = _mm256_setzero_ps();
                for (int p = 0; p < head_dim; p += 8) {
                    __m256 vq = _mm256_loadu_ps(&qh[p]);
                    __m256 vk = _mm256_loadu_ps(&k[p]);
                    sum_vec = _mm256_fmadd_ps(vq, vk, sum_vec);
                }
                __m128 vlow = _mm256_castps256_ps128(sum_vec);
                __m128 vhigh = _mm256_extractf128_ps(sum_vec, 1);
                vlow = _mm_add_ps(vlow, vhigh);
                __m128 shuf = _mm_movehdup_ps(vlow);
                __m128 sums = _mm_add_ps(vlow, shuf);
                shuf = _mm_movehl_ps(shuf, sums);
                sums = _mm_add_ss(sums, shuf);
                float raw_score = _mm_cvtss_f32(sums);
                att[b * PAGE + t_off] = raw_score / sqrtf((float)head_dim);
            }
        }
        oracle_softmax(att, pos + 1);
        float* xb_head = out + (size_t)h * head_dim;
        for (int p = 0; p < head_dim; p++) xb_head[p] = 0.0f;
        for (int b = 0; b <= num_full_blocks; b++) {
            int t_physical_id = table[b];
            int end_t_offset = (b == num_full_blocks) ? (pos & 15) : 15;
            const float* v_base = v_pool + t_physical_id * pf + layer_off + (size_t)kv_h * head_dim;
            for (int t_off = 0; t_off <= end_t_offset; t_off++) {
                const float* v = v_base + (size_t)t_off * kv_dim;
                __m256 va = _mm256_set1_ps(att[b * PAGE + t_off]);
                for (int p = 0; p < head_dim; p += 8) {
                    __m256 v_xb = _mm256_loadu_ps(&xb_head[p]);
                    __m256 vv = _mm256_loadu_ps(&v[p]);
                    v_xb = _mm256_fmadd_ps(va, vv, v_xb);
                    _mm256_storeu_ps(&xb_head[p], v_xb);
                }
            }
        }
    }
    free(attn);
    return 0;
}

/*
 * src/model_q8.cpp:485-523 — causal prefill for one sequence: for each
 * (t,h), pos = start_pos + t, a per-key online softmax (m starts at -1e9f,
 * rescale acc and d by expf(m - s) when a larger score arrives, then
 * e = expf(s - m), d += e, acc += e*v), finally acc /= d.  Keys come from
 * the pages via the block table (prefix pages and the chunk's own rows).
 */
int oracle_prefill_chunk(const float* k_pool, const float* v_pool, int n_layers, int kv_dim,
                         int layer, const float* q, float* out, const int32_t* table,
                         int start_pos, int num_tokens, int n_heads, int n_kv_heads,
                         int head_dim, int n_threads) {
    const int dim = n_heads * head_dim;
    const int kv_mul = n_heads / n_kv_heads;
    const size_t pf = page_floats(n_layers, kv_dim);
    size_t layer_off = (size_t)layer * PAGE * kv_dim;
#pragma omp parallel for collapse(2) num_threads(pick_threads(n_threads))
    for (int t = 0; t < num_tokens; t++) {
        for (int h = 0; h < n_heads; h++) {
            int pos = start_pos + t;
            const float* qh = q + (size_t)t * dim + (size_t)h * head_dim;
            float* xb_out = out + (size_t)t * dim + (size_t)h * head_dim;
            int kv_h = h / kv_mul;
            for (int p = 0; p < head_dim; p++) xb_out[p] = 0.0f;
            float m_global = -1e9f;
            float d_global = 0.0f;
            int num_full_blocks = pos / PAGE;
            for (int b = 0; b <= num_full_blocks; b++) {
                int phy_id = table[b];
                int end_t_off = (b == num_full_blocks) ? (pos % PAGE) : (PAGE - 1);
                const float* k_base = k_pool + phy_id * pf + layer_off + (size_t)kv_h * head_dim;
                const float* v_base = v_pool + phy_id * pf + layer_off + (size_t)kv_h * head_dim;
                for (int t_off = 0; t_off <= end_t_off; t_off++) {
                    const float* k = k_base + (size_t)t_off * kv_dim;
                    float raw_score = 0.0f;
                    for (int p = 0; p < head_dim; p++) raw_score += qh[p] * k[p];
                    raw_score /= sqrtf((float)head_dim);
                    if (raw_score > m_global) {
                        float correction = expf(m_global - raw_score);
                        for (int p = 0; p < head_dim; p++) xb_out[p] *= correction;
                        d_global *= correction;
                        m_global = raw_score;
                    }
                    float exp_score = expf(raw_score - m_global);
                    d_global += exp_score;
                    const float* v = v_base + (size_t)t_off * kv_dim;
                    for (int p = 0; p < head_dim; p++) xb_out[p] += exp_score * v[p];
                }
            }
            for (int p = 0; p < head_dim; p++) xb_out[p] /= d_global;
        }
    }
    return 0;
}

/*
 * src/model_q8.cpp:189-222 — the non-paged ("version 1") attention over a
 * contiguous cache [layer][seq_len][kv_dim]; same two-pass math as decode.
 */
int oracle_contiguous_attention(const float* key_cache, const float* value_cache, int seq_len,
                                int kv_dim, int layer, const float* q, float* out, int pos,
                                int n_heads, int n_kv_heads, int head_dim, int n_threads) {
    const int kv_mul = n_heads / n_kv_heads;
    size_t offset = (size_t)layer * seq_len * kv_dim;
    float* attn = (float*)malloc((size_t)n_heads * (pos + 1) * sizeof(float));
    if (!attn) return -1;
#pragma omp parallel for num_threads(pick_threads(n_threads))
    for (int h = 0; h < n_heads; h++) {
        const float* qh = q + (size_t)h * head_dim;
        float* att = attn + (size_t)h * (pos + 1);
        int kv_h = h / kv_mul;
        for (int t = 0; t <= pos; t++) {
            const float* k = key_cache + offset + (size_t)t * kv_dim + (size_t)kv_h * head_dim;
            float score = 0.0f;
            for (int p = 0; p < head_dim; p++) score += qh[p] * k[p];
            score /= sqrtf((float)head_dim);
            att[t] = score;
        }
        oracle_softmax(att, pos + 1);
        float* xb = out + (size_t)h * head_dim;
        for (int p = 0; p < head_dim; p++) xb[p] = 0.0f;
        for (int t = 0; t <= pos; t++) {
            const float* v = value_cache + offset + (size_t)t * kv_dim + (size_t)kv_h * head_dim;
            float a = att[t];
            for (int p = 0; p < head_dim; p++) xb[p] += a * v[p];
        }
    }
    free(attn);
    return 0;
}
