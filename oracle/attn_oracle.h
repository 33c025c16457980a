/*
 * CPU oracle for the paged-attention path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's attention loops, kept loop-for-loop
 * with src/model_q8.cpp so that it can stand in for the reference where the
 * reference cannot be called as a unit.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may link or call it, and only to check results
 * against (or as the timed CPU baseline); the shipped library never does.
 *
 * KV pool layout (src/pagedMemory.hpp:86-106, src/model_q8.cpp:284-287,620-623,639):
 *   pool[page][layer][tok 0..15][kv_dim], kv_dim = n_kv_heads * head_dim, fp32.
 *   Element (page, l, tok, kv_h, d) is at
 *     pool + page*L*16*kv_dim + l*16*kv_dim + tok*kv_dim + kv_h*head_dim + d.
 *
 * Block tables are int32 [B][max_pages]; positions are the reference's `pos`
 * (the slot written this step); attention covers keys 0..pos inclusive.
 *
 * Pins (where each function is checked, see tests/):
 *   oracle_softmax               closed form (fp64) + reference build golden vectors
 *   oracle_decode_batch          reference build golden vectors (forward_decode_batch), fp64 closed form
 *   oracle_decode_single_avx2    reference build golden vectors (forward_paged), fp64 closed form
 *   oracle_prefill_chunk         reference build golden vectors (forward_prefill_chunk), fp64 closed form
 *   oracle_contiguous_attention  reference build golden vectors (forward), paged == contiguous invariant
 *   oracle_kv_append_decode      reference build golden vectors (pool bytes after forward_decode_batch)
 *   oracle_kv_scatter_prefill    reference build golden vectors (pool bytes after forward_prefill_chunk)
 *   oracle_rope                  reference build golden vectors (q, k before/after RoPE in
 *                                forward_decode_batch, forward_paged, forward_prefill_chunk),
 *                                rotation invariants (norm of each pair, identity at angle 0)
 */
#ifndef NITRO_ATTN_ORACLE_H
#define NITRO_ATTN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_PAGE_TOKENS 16

void oracle_softmax(float* x, int size);

void oracle_kv_append_decode(float* k_pool, float* v_pool, int n_layers, int kv_dim, int layer,
                             const float* k, const float* v, const int32_t* tables, int max_pages,
                             const int32_t* positions, int batch);

void oracle_kv_scatter_prefill(float* k_pool, float* v_pool, int n_layers, int kv_dim, int layer,
                               const float* k, const float* v, const int32_t* table,
                               int start_pos, int num_tokens);

int oracle_decode_batch(const float* k_pool, const float* v_pool, int n_layers, int kv_dim,
                        int layer, const float* q, float* out, const int32_t* tables,
                        int max_pages, const int32_t* positions, int batch, int n_heads,
                        int n_kv_heads, int head_dim, int n_threads);

int oracle_decode_single_avx2(const float* k_pool, const float* v_pool, int n_layers, int kv_dim,
                              int layer, const float* q, float* out, const int32_t* table,
                              int pos, int n_heads, int n_kv_heads, int head_dim, int n_threads);

int oracle_prefill_chunk(const float* k_pool, const float* v_pool, int n_layers, int kv_dim,
                         int layer, const float* q, float* out, const int32_t* table,
                         int start_pos, int num_tokens, int n_heads, int n_kv_heads,
                         int head_dim, int n_threads);

int oracle_contiguous_attention(const float* key_cache, const float* value_cache, int seq_len,
                                int kv_dim, int layer, const float* q, float* out, int pos,
                                int n_heads, int n_kv_heads, int head_dim, int n_threads);

void oracle_rope(float* q, float* k, int rows, const int32_t* positions,
                 const float* freq_real, const float* freq_imag, int dim, int kv_dim,
                 int head_size);

int oracle_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
