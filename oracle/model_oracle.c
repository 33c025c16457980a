/*
 * CPU oracle for the model-level operations — TEST INFRASTRUCTURE ONLY.
 * A loop-for-loop C restatement of the reference's Q8 products with the same
 * AVX2 intrinsic sequence, so that a build with the reference's flags gives
 * the reference's bits.
 */
#include "model_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <string.h>

static float block_scale(const uint8_t* blk) {
    float s;
    memcpy(&s, blk, sizeof(float));
    return s;
}

/* Eight-lane horizontal sum in the reference's order (src/model_q8.cpp:117-123). */
static float hsum8(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    __m128 shuf = _mm_movehdup_ps(lo);
    __m128 sums = _mm_add_ps(lo, shuf);
    shuf = _mm_movehl_ps(shuf, sums);
    sums = _mm_add_ss(sums, shuf);
    return _mm_cvtss_f32(sums);
}

/* src/model_q8.cpp:92-125 (matmul, BlockQ8 overload): out[i] = w[i] . x. */
void oracle_q8_matmul(float* out, const float* x, const uint8_t* w, int n, int d, int n_threads) {
    const int nb = n / ORACLE_Q8_BLOCK;
#pragma omp parallel for num_threads(n_threads)
    for (int i = 0; i < d; i++) {
        __m256 sum = _mm256_setzero_ps();
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)i * nb + b) * ORACLE_Q8_BLOCK_BYTES;
            const int8_t* q = (const int8_t*)(blk + sizeof(float));
            const __m256 sv = _mm256_set1_ps(block_scale(blk));
            for (int c = 0; c < 4; c++) {
                const __m128i q8 = _mm_loadl_epi64((const __m128i*)(q + 8 * c));
                const __m256 wf = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q8)), sv);
                sum = _mm256_fmadd_ps(wf, _mm256_loadu_ps(x + b * ORACLE_Q8_BLOCK + 8 * c), sum);
            }
        }
        out[i] = hsum8(sum);
    }
}

/* src/model_q8.cpp:382-420 (matmul_bulk, BlockQ8 overload), including its
 * block loop's overwrite of out[b*d+i]: only the last block of a row stays. */
void oracle_q8_matmul_bulk(float* out, const float* x, const uint8_t* w, int batch, int n, int d,
                           int n_threads) {
    const int nb = n / ORACLE_Q8_BLOCK;
#pragma omp parallel for num_threads(n_threads)
    for (int i = 0; i < d; i++) {
        for (int b = 0; b < batch; b++) out[(size_t)b * d + i] = 0.0f;
        for (int blk_i = 0; blk_i < nb; blk_i++) {
            const uint8_t* blk = w + ((size_t)i * nb + blk_i) * ORACLE_Q8_BLOCK_BYTES;
            const int8_t* q = (const int8_t*)(blk + sizeof(float));
            const __m256 sv = _mm256_set1_ps(block_scale(blk));
            __m256 wf[4];
            for (int c = 0; c < 4; c++) {
                const __m128i q8 = _mm_loadl_epi64((const __m128i*)(q + 8 * c));
                wf[c] = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q8)), sv);
            }
            for (int b = 0; b < batch; b++) {
                __m256 sum = _mm256_setzero_ps();
                const float* xr = x + (size_t)b * n + blk_i * ORACLE_Q8_BLOCK;
                for (int c = 0; c < 4; c++) sum = _mm256_fmadd_ps(wf[c], _mm256_loadu_ps(xr + 8 * c), sum);
                out[(size_t)b * d + i] = hsum8(sum);
            }
        }
    }
}

/* src/model_q8.cpp:128-140 */
void oracle_rms_norm(float* out, const float* x, const float* weight, int size) {
    float ss = 0.0f;
    for (int i = 0; i < size; i++) ss += x[i] * x[i];
    ss /= size;
    ss += 1e-5f;
    ss = 1.0f / sqrtf(ss);
    for (int i = 0; i < size; i++) out[i] = weight[i] * (ss * x[i]);
}

/* src/model_q8.cpp:672-680 (forward_decode_batch's form; forward_paged and
 * forward_prefill_chunk multiply by hb2 in a second statement, same value) */
void oracle_swiglu(float* hb, const float* hb2, int n) {
    for (int i = 0; i < n; i++) {
        float val = hb[i];
        val *= (1.0f / (1.0f + expf(-val)));
        hb[i] = val * hb2[i];
    }
}

/* src/model_q8.cpp:80-90 (matmul, float weights) */
void oracle_f32_matmul(float* out, const float* x, const float* w, int n, int d, int n_threads) {
#pragma omp parallel for num_threads(n_threads)
    for (int i = 0; i < d; i++) {
        float val = 0.0f;
        for (int j = 0; j < n; j++) val += w[(size_t)i * n + j] * x[j];
        out[i] = val;
    }
}

/* src/model_q8.cpp:370-380 (matmul_bulk, float weights) */
void oracle_f32_matmul_bulk(float* out, const float* x, const float* w, int batch, int n, int d,
                            int n_threads) {
#pragma omp parallel for collapse(2) num_threads(n_threads)
    for (int b = 0; b < batch; b++) {
        for (int i = 0; i < d; i++) {
            float val = 0.0f;
            for (int j = 0; j < n; j++) val += x[(size_t)b * n + j] * w[(size_t)i * n + j];
            out[(size_t)b * d + i] = val;
        }
    }
}
