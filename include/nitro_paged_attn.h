/*
 * nitro_paged_attn.h — C ABI of the MI355X (gfx950) paged-attention path for
 * NitroRAG's inference engine.
 *
 * The reference (nvivek17/NitroRAG) has no attention function of its own: its
 * attention is inlined in the forward passes of src/model_q8.cpp, and its page
 * bookkeeping lives in src/pagedMemory.hpp.  This header is the boundary a
 * maintainer binds in place of those regions.  Every entry point names the
 * reference code it replaces (file:line, relative to the reference checkout).
 *
 * Conventions
 *  - Every function returns an int status (NITRO_OK = 0).  Where the reference
 *    calls exit(1) (pool exhaustion, src/pagedMemory.hpp:96,117,212) this
 *    library returns a status instead; nitro_last_error() gives the message.
 *  - Device pointers are caller-owned fp32 buffers in HBM; `stream` is a
 *    hipStream_t passed as void* (NULL = the null stream).  Launches are
 *    asynchronous on that stream.  One host thread drives a pool at a time.
 *  - KV pool layout is the reference's (src/pagedMemory.hpp:86-106):
 *      pool[page][layer][tok 0..15][kv_dim], kv_dim = n_kv_heads * head_dim.
 *    Element (page, l, tok, kv_h, d) sits at
 *      base + page*L*16*kv_dim + l*16*kv_dim + tok*kv_dim + kv_h*head_dim + d.
 *  - A block table is the reference's Sequence::block_table: logical page i
 *    of a sequence is physical page table[i].  `pos` is the slot written this
 *    step; attention covers keys 0..pos inclusive (src/model_q8.cpp:634-638).
 */
#ifndef NITRO_PAGED_ATTN_H
#define NITRO_PAGED_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Page size in tokens — src/pagedMemory.hpp:9 (BLOCK_SIZE). */
#define NITRO_PAGE_TOKENS 16

enum {
    NITRO_OK = 0,
    NITRO_ERR_INVALID_ARGUMENT = 1, /* bad pointer, id, shape or layer */
    NITRO_ERR_UNSUPPORTED = 2,      /* head_dim not a multiple of 4 in [4, 256], n_heads % n_kv_heads != 0 */
    NITRO_ERR_DEVICE_ALLOC = 3,     /* hipMalloc failed (reference: src/pagedMemory.hpp:96) */
    NITRO_ERR_OUT_OF_PAGES = 4,     /* no free page and nothing evictable (src/pagedMemory.hpp:117,212) */
    NITRO_ERR_BAD_BLOCK_TABLE = 5,  /* page id outside the pool, or pos beyond the table */
    NITRO_ERR_HIP = 6,              /* a HIP runtime call failed */
    NITRO_ERR_NO_BATCH = 7          /* attention/append called before a batch was uploaded */
};

const char* nitro_status_string(int status);
/* Message of the last failure on the calling thread ("" if none). */
const char* nitro_last_error(void);

/* ======================= host page bookkeeping ============================
 * Bit-exact restatement of src/pagedMemory.hpp in C++ (no device memory):
 * LIFO free list, reference counts, FNV-1a prefix cache with parent/child
 * topology and leaf-first LRU eviction, per-sequence block tables.  Not
 * thread-safe: the reference calls Sequence::allocate_next_token from an
 * OpenMP loop (src/model_q8.cpp:578-582), a data race; callers of this
 * library allocate sequentially in batch order, which is what the reference
 * does with one thread.
 */
typedef struct nitro_block_manager nitro_block_manager; /* KVBlock_Manager + PrefixCacheManager */
typedef struct nitro_sequence nitro_sequence;           /* Sequence */

typedef struct nitro_block_info {
    int32_t num_tokens;
    int32_t ref_count;
    int32_t parent_id;
    int32_t child_count;
} nitro_block_info; /* KVBlock fields, src/pagedMemory.hpp:28-37 */

/* hash_block_state — src/pagedMemory.hpp:14-24 */
uint64_t nitro_hash_block_state(uint64_t parent_hash, const int32_t* tokens, int32_t n);

/* KVBlock_Manager::KVBlock_Manager + PrefixCacheManager::PrefixCacheManager —
 * src/pagedMemory.hpp:86-111, 163-167 (bookkeeping only; K/V live in a nitro_kvpool). */
int nitro_bm_create(int32_t total_blocks, nitro_block_manager** out);
int nitro_bm_destroy(nitro_block_manager* bm); /* ~KVBlock_Manager, :157-160 */
int nitro_bm_allocate_block(nitro_block_manager* bm, int32_t* id);                 /* :113-128 */
int nitro_bm_inc_ref_count(nitro_block_manager* bm, int32_t id);                   /* :129-132 */
int nitro_bm_free_block(nitro_block_manager* bm, int32_t id);                      /* :137-144 */
int nitro_bm_force_free_block(nitro_block_manager* bm, int32_t id);                /* :145-151 */
int nitro_bm_get_free_count(const nitro_block_manager* bm, int32_t* n);           /* :134-136 */
int nitro_bm_get_block(const nitro_block_manager* bm, int32_t id, nitro_block_info* out); /* :154-156 */
int nitro_bm_is_cached(const nitro_block_manager* bm, int32_t id, int32_t* cached); /* :168-170 */
int nitro_bm_check_cache(const nitro_block_manager* bm, uint64_t block_hash, int32_t* id); /* :187-192 */
int nitro_bm_insert_cache(nitro_block_manager* bm, uint64_t block_hash, int32_t id,
                          int32_t parent_id);                                      /* :193-205 */
int nitro_bm_evict_lru_block(nitro_block_manager* bm);                             /* :206-229 */
/* Introspection of the same state the reference keeps privately
 * (free_list order, evictable_leaves front->back, cache_map, reverse_map). */
int nitro_bm_free_list(const nitro_block_manager* bm, int32_t* ids, int32_t cap, int32_t* n);
int nitro_bm_evictable_leaves(const nitro_block_manager* bm, int32_t* ids, int32_t cap, int32_t* n);
int nitro_bm_cache_entries(const nitro_block_manager* bm, uint64_t* hashes, int32_t* ids,
                           int32_t cap, int32_t* n); /* sorted by hash */
int nitro_bm_reverse_entries(const nitro_block_manager* bm, int32_t* ids, uint64_t* hashes,
                             int32_t cap, int32_t* n); /* sorted by id */

/* Sequence — src/pagedMemory.hpp:233-285 */
int nitro_seq_create(int32_t seq_id, nitro_sequence** out);                        /* :240-244 */
int nitro_seq_destroy(nitro_sequence* seq);
int nitro_seq_allocate_next_token(nitro_sequence* seq, nitro_block_manager* bm, int32_t token); /* :245-264 */
int nitro_seq_flush_cache(nitro_sequence* seq, nitro_block_manager* bm);           /* :265-273 */
int nitro_seq_release(nitro_sequence* seq, nitro_block_manager* bm);               /* :274-283 */
/* Prefix-hit walk over full 16-token chunks of prompt[start..n): on a hit,
 * inc_ref_count + push the shared page + advance current_hash; stops at the
 * first miss.  require_empty_buffer=1 is the scheduler's variant
 * (src/pagedMemory.hpp:346-359), 0 is ingest_prompt's (src/model_q8.cpp:699-714).
 * *next receives the index of the first token not covered by a hit. */
int nitro_seq_prefix_walk(nitro_sequence* seq, nitro_block_manager* bm, const int32_t* prompt,
                          int32_t n, int32_t start, int32_t require_empty_buffer, int32_t* next);
/* Bookkeeping of ingest_prompt (src/model_q8.cpp:695-724): the walk (if
 * enabled), then allocate_next_token for every remaining token, as
 * forward_prefill_chunk does first (:428-430).  *count = logical_token_count. */
int nitro_seq_ingest_prompt(nitro_sequence* seq, nitro_block_manager* bm, const int32_t* prompt,
                            int32_t n, int32_t enable_prefix_caching, int32_t* count);
int nitro_seq_state(const nitro_sequence* seq, int32_t* logical_token_count,
                    uint64_t* current_hash, int32_t* buffered_tokens, int32_t* num_pages);
int nitro_seq_block_table(const nitro_sequence* seq, int32_t* pages, int32_t cap, int32_t* n);
int nitro_seq_token_buffer(const nitro_sequence* seq, int32_t* tokens, int32_t cap, int32_t* n);
/* Packs the block tables of `batch` sequences into a dense host array
 * tables[batch][max_pages] (unused entries 0), the form the device takes. */
int nitro_pack_block_tables(const nitro_sequence* const* seqs, int32_t batch, int32_t max_pages,
                            int32_t* tables);

/* ============================ device KV pool ============================== */
typedef struct nitro_kvpool nitro_kvpool;

/* Device K and V pools with the reference layout — replaces the
 * aligned_alloc pools of KVBlock_Manager (src/pagedMemory.hpp:86-111).
 * nitro_kvpool_create owns (hipMalloc, zero-filled) memory; nitro_kvpool_wrap
 * borrows two caller buffers of num_pages*num_layers*16*kv_dim floats each. */
int nitro_kvpool_create(int32_t num_pages, int32_t num_layers, int32_t kv_dim, nitro_kvpool** out);
int nitro_kvpool_wrap(float* k_pool, float* v_pool, int32_t num_pages, int32_t num_layers,
                      int32_t kv_dim, nitro_kvpool** out);
/* The non-paged cache of forward (src/model_q8.cpp:189-222): borrows the
 * RunState key_cache / value_cache, each [num_layers][seq_len][kv_dim] floats
 * (src/model_q8.cpp:54-70), as a pool of seq_len/16 pages per layer, page p of
 * a layer being its rows 16p..16p+15.  Under the identity block table
 * {0, 1, .., pos/16} the decode entry points below compute forward's attention
 * (:193-222) and nitro_kv_append its cache write (:189-191) at the same
 * addresses.  seq_len must be a multiple of 16 (NITRO_ERR_UNSUPPORTED). */
int nitro_kvpool_wrap_contiguous(float* key_cache, float* value_cache, int32_t seq_len,
                                 int32_t num_layers, int32_t kv_dim, nitro_kvpool** out);
int nitro_kvpool_destroy(nitro_kvpool* pool); /* ~KVBlock_Manager, src/pagedMemory.hpp:157-160 */
int nitro_kvpool_data(const nitro_kvpool* pool, float** k_pool, float** v_pool);
int nitro_kvpool_shape(const nitro_kvpool* pool, int32_t* num_pages, int32_t* num_layers,
                       int32_t* kv_dim);

/* ----------------------------- decode ------------------------------------
 * The decode batch of forward_decode_batch (src/model_q8.cpp:571-662):
 * host tables[batch][max_pages] and positions[batch] (pos_b = the sequence's
 * logical_token_count before this step's token, src/pagedMemory.hpp:334-341).
 * Validated on the host (every page id of pages 0..pos/16 inside the pool),
 * then copied to device memory owned by the pool, on `stream`.  Sequences whose
 * first pages (4 or more) are the same physical pages (prefix-cache hits) are
 * noted here.  MHA decode launches over such a batch read those shared rows
 * once per set of sequences instead of once per sequence when the batch's
 * K/V rows add up to at least 128 MB; below that, reading each sequence's
 * rows from the caches measured faster. */
int nitro_decode_batch_upload(nitro_kvpool* pool, const int32_t* tables, const int32_t* positions,
                              int32_t batch, int32_t max_pages, void* stream);

/* KV append for the decode batch — src/model_q8.cpp:616-623 (and the
 * single-sequence append :279-287): k, v are device [batch][kv_dim]; row
 * pos%16 of page table[pos/16] at `layer` receives them. */
int nitro_kv_append(nitro_kvpool* pool, int32_t layer, const float* k, const float* v, void* stream);

/* Batched paged-attention decode — src/model_q8.cpp:625-662 (batched) and
 * :290-347 (single sequence, batch = 1).  q, out: device [batch][n_heads*head_dim].
 * For each (b, h): softmax over keys 0..pos_b of q.k/sqrt(head_dim), times V,
 * with kv head h / (n_heads/n_kv_heads).  head_dim: any multiple of 4 from 4
 * to 256.  One kernel launch: long contexts are split over workgroups (sized
 * from the batch's context lengths, so the GPU fills with even work), each
 * keeps an online softmax, and the last workgroup of a (b, head) to finish
 * merges the splits' partials in split order.  The first launch for an
 * uploaded batch may also copy a small work list (host to device, on
 * `stream`), and a launch that needs more split-K workspace than the pool
 * holds allocates it (hipMalloc, hipMemset).  Not re-entrant per pool:
 * launches that overlap on one pool race on its workspace and counters. */
int nitro_paged_attn_decode(nitro_kvpool* pool, int32_t layer, const float* q, float* out,
                            int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, void* stream);

/* Allocation-free batched decode.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory at call time (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * result as nitro_paged_attn_decode, but the caller passes the batch as device
 * arrays — tables [batch][max_pages] int32 and positions [batch] int32 (the
 * slot written this step, attended inclusive) — and max_context, a host bound
 * with positions[b] + 1 <= max_context for every b (keys past it are not
 * attended; page ids are range-checked on the device, nothing else of the
 * device arrays is validated).  Nothing is uploaded or allocated: split-K
 * partials and arrival counters live in a fixed 8 MiB workspace, one copy per
 * GPU for the life of the process (65,536 counters of batch * n_heads / query
 * heads per workgroup, the rest partials); a launch that needs more is refused
 * with NITRO_ERR_INVALID_ARGUMENT.  Every launch leaves the counters at zero.
 * All calls on one GPU share that workspace: calls that overlap on one GPU (two
 * streams, two threads) race.  pages_private (0 or 1): 1 when no physical page
 * is read by two sequences of the batch, so K/V rows are read once and go
 * through non-temporal loads (as nitro_paged_attn_decode chooses from its
 * uploaded tables); 0 keeps them cacheable for prefix-shared pages (measured
 * 8% slower at B=64, ctx 4096, 32 x 128 when nothing is shared).  The result
 * is the same either way. */
int nitro_paged_attn_decode_static(nitro_kvpool* pool, int32_t layer, const float* q, float* out,
                                   const int32_t* tables, const int32_t* positions, int32_t batch,
                                   int32_t max_pages, int32_t max_context, int32_t n_heads, int32_t n_kv_heads,
                                   int32_t head_dim, int32_t pages_private, void* stream);

/* nitro_kv_append followed by nitro_paged_attn_decode, as forward_decode_batch
 * does them (src/model_q8.cpp:616-662): k, v device [batch][kv_dim] are written
 * at each sequence's pos and attended.  One launch when no other sequence of
 * the batch reads the page holding a sequence's pos (the row is then read from
 * k / v directly); otherwise the append and the decode launch in turn.  The
 * pool and output equal those of the two calls. */
int nitro_paged_attn_decode_append(nitro_kvpool* pool, int32_t layer, const float* q, const float* k,
                                   const float* v, float* out, int32_t n_heads, int32_t n_kv_heads,
                                   int32_t head_dim, void* stream);

/* ----------------------------- prefill -----------------------------------
 * A prefill batch of chunks, one per sequence — forward_prefill_chunk
 * (src/model_q8.cpp:424-523) over several sequences at once.  Sequence b's
 * chunk has num_tokens[b] tokens at positions start_pos[b] .. start_pos[b] +
 * num_tokens[b] - 1 (start_pos = logical_token_count before the chunk,
 * src/pagedMemory.hpp:379).  Q/K/V/out rows of all chunks are packed in batch
 * order: rows [off_b, off_b + num_tokens[b]) with off_b = sum of earlier
 * num_tokens.  Validated on the host like the decode batch. */
int nitro_prefill_batch_upload(nitro_kvpool* pool, const int32_t* tables, const int32_t* start_pos,
                               const int32_t* num_tokens, int32_t batch, int32_t max_pages,
                               void* stream);

/* KV scatter of the prefill batch — src/model_q8.cpp:473-484.
 * k, v: device [total_tokens][kv_dim]. */
int nitro_kv_append_prefill(nitro_kvpool* pool, int32_t layer, const float* k, const float* v,
                            void* stream);

/* Causal paged prefill attention — src/model_q8.cpp:485-523.  q, out: device
 * [total_tokens][n_heads*head_dim]; the token at pos attends keys 0..pos
 * (prefix-hit pages, earlier chunks and this chunk's own rows).  head_dim: any
 * multiple of 4 from 4 to 256 (32, 64 and 128 run on the matrix cores). */
int nitro_paged_attn_prefill(nitro_kvpool* pool, int32_t layer, const float* q, float* out,
                             int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, void* stream);

/* KV scatter and causal prefill attention of the batch in one call — the
 * reference's prefill layer step, src/model_q8.cpp:473-484 then :485-523
 * (nitro_kv_append_prefill followed by nitro_paged_attn_prefill, with the same
 * pool contents and output).  k, v: device [total_tokens][kv_dim].  With the
 * matrix-core kernel (head_dim 32, 64, 128), positions below 32768, and no
 * page that a chunk row lands on named by any other table entry (checked at
 * upload), one launch reads each chunk's keys from k / v (keys cached before
 * start_pos from the pool) and appends the chunk: fresh prompts, later chunks
 * of a chunked prefill, suffixes after prefix-cache hits.  Otherwise the
 * scatter and the attention run as two launches. */
int nitro_paged_attn_prefill_append(nitro_kvpool* pool, int32_t layer, const float* q, const float* k,
                                    const float* v, float* out, int32_t n_heads, int32_t n_kv_heads,
                                    int32_t head_dim, void* stream);

/* No counterpart in the reference: how many nitro_paged_attn_prefill_append
 * calls the pool has run, and how many of them ran as one launch. */
int nitro_kvpool_prefill_counts(nitro_kvpool* pool, int64_t* calls, int64_t* one_launch);

/* ------------------------------- RoPE --------------------------------------
 * RoPE fused with the KV append, as the reference does it in one loop: each
 * pair (j, j+1) of q (all heads) and of k (kv heads) is rotated in place by
 * (c, s) = (freq_real, freq_imag)[pos*(head_dim/2) + (j % head_dim)/2] —
 * q' = (q0*c - q1*s, q0*s + q1*c) — then the rotated k and the unrotated v
 * are appended at pos.  freq_real/freq_imag: device [seq_len][head_dim/2]
 * (the reference's freq_cis_real/imag); every position must be < seq_len. */
/* Decode batch — src/model_q8.cpp:601-623 (single sequence :262-287).
 * q [batch][n_heads*head_dim], k and v [batch][kv_dim]. */
int nitro_rope_kv_append(nitro_kvpool* pool, int32_t layer, float* q, float* k, const float* v,
                         const float* freq_real, const float* freq_imag, int32_t seq_len,
                         int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, void* stream);
/* Prefill batch rows — src/model_q8.cpp:451-484.  Rows packed as for
 * nitro_kv_append_prefill. */
int nitro_rope_kv_append_prefill(nitro_kvpool* pool, int32_t layer, float* q, float* k,
                                 const float* v, const float* freq_real, const float* freq_imag,
                                 int32_t seq_len, int32_t n_heads, int32_t n_kv_heads,
                                 int32_t head_dim, void* stream);

/* ------------------------- Q8_0 matrix product -----------------------------
 * out[b][i] = sum_k w[i][k] * x[b][k], b < batch, i < d, k < n, with w in the
 * reference's BlockQ8 layout (src/model_q8.cpp:28-32; scripts/quantize.py):
 * row i is n/32 blocks of {float scale; int8 q[32]} (36 bytes), weight
 * (i, 32j + t) = float(q_t) * scale_j.  x is fp32 [batch][n] (16-byte
 * aligned), out fp32 [batch][d]; all device pointers.  n % 32 == 0.
 *   NITRO_Q8_FULL_ROWS — matmul (src/model_q8.cpp:92-125), used by forward
 *     and forward_paged;
 *   NITRO_Q8_LAST_BLOCK — matmul_bulk (src/model_q8.cpp:382-420), used by
 *     forward_prefill_chunk and forward_decode_batch: its block loop stores
 *     each block's sum over the previous one, so only block n/32-1 of every
 *     row reaches out.
 * fp32 products and accumulation; the summation order differs from the
 * reference's 8-lane AVX2 order (results agree to fp32 rounding). */
#define NITRO_Q8_FULL_ROWS 0
#define NITRO_Q8_LAST_BLOCK 1
int nitro_q8_matmul(const void* w, const float* x, float* out, int32_t batch, int32_t n,
                    int32_t d, int32_t semantics, void* stream);

/* ------------------------ transformer step (model) -------------------------
 * The forward passes of src/model_q8.cpp around the attention path, on the
 * device: embedding, per layer rms_norm -> wq/wk/wv (Q8) -> RoPE + KV append
 * -> paged attention -> wo -> residual -> rms_norm -> w1, w3 -> SwiGLU -> w2
 * -> residual, then the final rms_norm and the fp32 classifier (wcls = the
 * embedding table, src/Server_Inference.cpp:69).
 *
 * nitro_model_create takes the reference's model file as bytes
 * (src/Server_Inference.cpp:45-69, written by scripts/quantize.py): a header
 * of 7 int32 {dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size,
 * seq_len}, then token_embedding_table f32, rms_att f32, wq wk wv wo Q8,
 * rms_ffn f32, w1 w2 w3 Q8, rms_final f32, freq_cis_real, freq_cis_imag f32.
 * The weights are copied to the device; the caller may free the blob.  The
 * pool used with a model must have n_layers layers and kv_dim =
 * n_kv_heads * dim / n_heads.  The first forward with more than 4 rows of
 * full-row products (NITRO_Q8_FULL_ROWS) allocates and builds a tile-layout
 * copy of the Q8 matrices (1.125 bytes per weight) that those products read;
 * a caller capturing such forwards into a graph runs one first.
 *
 * semantics selects the Q8 product (NITRO_Q8_*): forward_decode_batch and
 * forward_prefill_chunk compute their Q8 products with matmul_bulk
 * (NITRO_Q8_LAST_BLOCK reproduces them), forward_paged with matmul
 * (NITRO_Q8_FULL_ROWS).  The classifier is fp32 in both. */
typedef struct nitro_model nitro_model;
int nitro_model_create(const void* blob, uint64_t bytes, nitro_model** out);
int nitro_model_destroy(nitro_model* model);
/* config[7] = the header fields, in file order. */
int nitro_model_config(const nitro_model* model, int32_t* config);
/* forward_decode_batch (src/model_q8.cpp:571-694), forward_paged (:244-368)
 * with batch = 1: tokens[batch] (host), one per sequence of the uploaded
 * decode batch (nitro_decode_batch_upload, positions = the slots written
 * now; the caller has already run the host bookkeeping of
 * Sequence::allocate_next_token).  Writes logits[batch][vocab_size] (device). */
int nitro_forward_decode_batch(nitro_model* model, nitro_kvpool* pool, const int32_t* tokens,
                               int32_t batch, float* logits, int32_t semantics, void* stream);
/* forward_prefill_chunk (src/model_q8.cpp:424-557) for every chunk of the
 * uploaded prefill batch: tokens[total_rows] (host, chunks packed in batch
 * order).  Writes logits[chunks][vocab_size] (device) for the last token of
 * each chunk. */
int nitro_forward_prefill(nitro_model* model, nitro_kvpool* pool, const int32_t* tokens,
                          int32_t total_rows, float* logits, int32_t semantics, void* stream);

/* ======================== continuous scheduler ============================
 * Request + Continuous_Scheduler (src/pagedMemory.hpp:287-399) over a
 * block manager the caller keeps alive.  max_tokens_per_batch is the
 * reference's token budget per step (256 there); max_generated is its finish
 * length (20, hard-coded at :393).  Block ids, prefix-cache state, chunking
 * and finish decisions come out exactly as the reference's.  A step either
 * runs on the device (nitro_sched_step) or is split for a caller-supplied
 * forward: nitro_sched_plan, the caller's forwards, nitro_sched_commit.
 * After an error from plan or step (e.g. NITRO_ERR_OUT_OF_PAGES, where the
 * reference calls exit(1)) the scheduler must only be destroyed. */
typedef struct nitro_scheduler nitro_scheduler;
int nitro_sched_create(nitro_block_manager* bm, int32_t max_tokens_per_batch, int32_t max_generated,
                       nitro_scheduler** out);
int nitro_sched_destroy(nitro_scheduler* sched);
/* new Request(req_id, prompt) + add_request (:309-312); n > 0, ids unique.
 * Once limits are set (nitro_sched_set_limits, or bound from the model by
 * the first nitro_sched_step), a prompt holding a token outside [0, vocab)
 * or with n + max_generated - 1 > seq_len (its last decode would sit at
 * position seq_len or later) is refused with NITRO_ERR_INVALID_ARGUMENT;
 * the reference has no such limit and would index its pools out of bounds. */
int nitro_sched_add_request(nitro_scheduler* sched, int32_t req_id, const int32_t* prompt, int32_t n);
/* The model's seq_len and vocabulary size for admission (0 = no limit).
 * nitro_sched_step sets them from its model on every call, and first finishes
 * (with the tokens they have) requests queued earlier that the model cannot
 * run, instead of failing the step. */
int nitro_sched_set_limits(nitro_scheduler* sched, int32_t seq_len, int32_t vocab);
int nitro_sched_has_active_requests(const nitro_scheduler* sched, int32_t* active); /* :313-315 */
/* step (:316-378) up to its two forward calls, including the
 * allocate_next_token loops those forwards begin with (src/model_q8.cpp:
 * 428-430, then :578-582 in batch order).  prefill[4] = {request id or -1,
 * chunk length, start position, 1 if the chunk completes the prompt}; the
 * chunk is prompt[start, start + length).  The decode rows (running order)
 * go to decode_ids / decode_tokens / decode_positions (cap entries each, at
 * least the running batch's size; any may be NULL), their count to *n_decode. */
int nitro_sched_plan(nitro_scheduler* sched, int32_t* prefill, int32_t* decode_ids,
                     int32_t* decode_tokens, int32_t* decode_positions, int32_t cap,
                     int32_t* n_decode);
/* step (:380-397) after the forwards: argmax tokens of the prefill chunk
 * (used when it completed its prompt) and of the n decode rows. */
int nitro_sched_commit(nitro_scheduler* sched, int32_t prefill_token, const int32_t* decode_tokens,
                       int32_t n);
/* One whole step on the device: plan, then ONE forward over the prefill
 * chunk's rows and the decode rows together (each weight matrix is read once
 * for both; forward_prefill_chunk + forward_decode_batch, src/model_q8.cpp:
 * 424-557 and 571-694), the reference's argmax (:559-569) on the device,
 * the tokens back to the host, commit.  Block tables live on the device
 * (one row per request, rows updated with the pages each step adds).  The
 * first call binds the scheduler to `pool` (pages must cover the block
 * manager's); later calls must pass the same pool.  Synchronises `stream`. */
int nitro_sched_step(nitro_scheduler* sched, nitro_model* model, nitro_kvpool* pool,
                     int32_t semantics, void* stream);
/* Logits rows the last nitro_sched_step computed (host copy, rows x
 * vocab_size): the prefill chunk's last row first when it completed its
 * prompt, then the decode rows.  *rows receives their count. */
int nitro_sched_last_logits(const nitro_scheduler* sched, float* logits, int32_t cap_rows,
                            int32_t* rows);
/* argmax (src/model_q8.cpp:559-569) of each of `rows` rows of logits
 * (device, rows x vocab) into out (device, rows int32): the first index of the
 * largest value above 0.0, 0 when no value exceeds 0.0; NaN never wins. */
int nitro_argmax(const float* logits, int32_t rows, int32_t vocab, int32_t* out, void* stream);
/* Scheduler state as int32 words: [n, running ids] [n, waiting ids] [n requests],
 * then per request in the order added: id, prefill_idx, is_prefill_done,
 * is_finished, next_token_to_process, [n, generated], logical_token_count,
 * current_hash lo, hi, [n, token buffer], [n, block table]. */
int nitro_sched_state(const nitro_scheduler* sched, int32_t* words, int32_t cap, int32_t* n);
int nitro_sched_generated(const nitro_scheduler* sched, int32_t req_id, int32_t* tokens, int32_t cap,
                          int32_t* n);
/* status[6] = {prefill_idx, is_prefill_done, is_finished, next_token_to_process,
 * generated count, logical_token_count}. */
int nitro_sched_request_status(const nitro_scheduler* sched, int32_t req_id, int32_t* status);
/* Forgets a finished request that a later step has released. */
int nitro_sched_drop_request(nitro_scheduler* sched, int32_t req_id);

/* ============================== NitroRPC ==================================
 * The wire format of src/NitroRPC.hpp, host byte order (little-endian here):
 * an int vector is its int32 count then the int32 values (send_ints /
 * recv_ints, :39-56); a structured query is uint64 subset_mask, float32
 * range_min, float32 range_max, then dim float32 (recv_structured_query,
 * :58-67).  The encoders report the byte count in *bytes (and write when
 * `out` holds it); the decoder reports count and bytes consumed.  The fd
 * functions are send_all / recv_all (:19-37) over a connected socket. */
int nitro_rpc_encode_ints(const int32_t* data, int32_t n, uint8_t* out, uint64_t cap, uint64_t* bytes);
int nitro_rpc_decode_ints(const uint8_t* buf, uint64_t len, int32_t* out, int32_t cap, int32_t* n,
                          uint64_t* consumed);
int nitro_rpc_encode_structured_query(uint64_t subset_mask, float range_min, float range_max, const float* vec,
                                      int32_t dim, uint8_t* out, uint64_t cap, uint64_t* bytes);
int nitro_rpc_send_ints(int32_t fd, const int32_t* data, int32_t n);                 /* :39-46 */
int nitro_rpc_recv_ints(int32_t fd, int32_t* out, int32_t cap, int32_t* n);           /* :48-56 */
int nitro_rpc_recv_structured_query(int32_t fd, int32_t dim, uint64_t* subset_mask, float* range_min,
                                    float* range_max, float* vec);                   /* :58-67 */

/* The serving loop of src/Server_Inference.cpp:86-112 over connections the
 * caller has accepted: nitro_server_accept_fd reads the prompt (an int
 * vector of at most max_prompt_tokens) and adds it as request 0, 1, 2, ...
 * (req_counter, :27-34); each nitro_server_step runs one nitro_sched_step,
 * sends every request's new tokens as bare int32 values and closes the
 * connections of finished requests, whose requests it forgets once the
 * scheduler has released them.  *active = has_active_requests.
 * nitro_server_accept_fd takes the fd whatever it returns: a prompt the
 * scheduler refuses (nitro_sched_add_request: one the model cannot finish) or
 * that cannot be read fails the call, and the server has then closed the fd
 * without sending a token, which is what a client whose request the
 * scheduler refuses at a later step receives too. */
typedef struct nitro_server nitro_server;
int nitro_server_create(nitro_scheduler* sched, nitro_model* model, nitro_kvpool* pool, int32_t semantics,
                        int32_t max_prompt_tokens, nitro_server** out);
int nitro_server_destroy(nitro_server* server); /* closes connections still open */
int nitro_server_accept_fd(nitro_server* server, int32_t fd, int32_t* req_id);
int nitro_server_step(nitro_server* server, void* stream, int32_t* active);

/* ------------------------------ checks ------------------------------------
 * Kernels re-check every page id they dereference against the pool size and
 * skip (and record) any outside it instead of faulting.  This reads and
 * clears that record (synchronising the pool's last stream): *bad_pages = 0
 * when no kernel saw a bad id. */
int nitro_kvpool_take_device_errors(nitro_kvpool* pool, int32_t* bad_pages);

/* Decode launches this pool has run over its current and earlier batches
 * (nitro_paged_attn_decode, nitro_paged_attn_decode_append and the
 * scheduler step's attention), and how many of them took the shared-prefix
 * form, where sequences that begin with the same physical pages read those
 * rows once per set of members.  No counterpart in the reference, which
 * reads every sequence's pages on its own: it is for callers that check
 * whether their prefix-cache hits are shared on the GPU. */
int nitro_kvpool_decode_counts(nitro_kvpool* pool, int64_t* launches, int64_t* shared_prefix_launches);

#ifdef __cplusplus
}
#endif
#endif /* NITRO_PAGED_ATTN_H */
