/*
 * CPU oracle for the model-level operations around the attention path —
 * TEST INFRASTRUCTURE ONLY (same rules as attn_oracle.h: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may call it).
 *
 * BlockQ8 layout (src/model_q8.cpp:28-32): per 32 consecutive weights of a
 * row, a float scale then 32 int8 (36 bytes, packed); a [d][n] matrix is d
 * rows of n/32 blocks.
 *
 * Pins (see tests/):
 *   oracle_q8_matmul       reference build golden vectors (matmul, bit-exact),
 *                          fp64 closed form sum_k float(q)*scale*x
 *   oracle_q8_matmul_bulk  reference build golden vectors (matmul_bulk,
 *                          bit-exact), closed form "last block only"
 *   oracle_rms_norm, oracle_swiglu, oracle_f32_matmul(_bulk)
 *                          reference build golden logits of forward_paged /
 *                          forward_decode_batch / forward_prefill_chunk through
 *                          oracle/model.py's forward passes; fp64 closed forms
 */
#ifndef NITRO_MODEL_ORACLE_H
#define NITRO_MODEL_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_Q8_BLOCK 32
#define ORACLE_Q8_BLOCK_BYTES 36

void oracle_q8_matmul(float* out, const float* x, const uint8_t* w, int n, int d, int n_threads);
void oracle_q8_matmul_bulk(float* out, const float* x, const uint8_t* w, int batch, int n, int d,
                           int n_threads);

/* src/model_q8.cpp:128-140 */
void oracle_rms_norm(float* out, const float* x, const float* weight, int size);
/* src/model_q8.cpp:672-680 over n values: hb = silu(hb) * hb2 */
void oracle_swiglu(float* hb, const float* hb2, int n);
/* src/model_q8.cpp:80-90 (matmul, float) and :370-380 (matmul_bulk, float) */
void oracle_f32_matmul(float* out, const float* x, const float* w, int n, int d, int n_threads);
void oracle_f32_matmul_bulk(float* out, const float* x, const float* w, int batch, int n, int d,
                            int n_threads);

#ifdef __cplusplus
}
#endif
#endif
