// Driver around the reference's own source — TEST INFRASTRUCTURE ONLY.
//
// Built by oracle/Makefile into oracle/_ref/libnitro_ref.so, compiling
// src/model_q8.cpp (which includes src/pagedMemory.hpp) from where it lies
// under the reference checkout, with the reference's flags.  Nothing from the
// reference is copied here: this file only instantiates the reference's types
// and calls its functions so that tests/golden/make_golden.py can record
// golden vectors (block-manager traces, prefix-cache state, attention
// outputs of forward_decode_batch / forward_paged / forward_prefill_chunk /
// forward, scheduler steps, NitroRPC messages) and so that CPU tests can
// cross-check the oracle live.
//
// Attention outputs are observed through s->xb2 = wo . xb with wo the Q8
// identity.  forward_paged and forward use the full-row Q8 matmul, so all of
// xb is observable there.  forward_decode_batch and forward_prefill_chunk use
// matmul_bulk, whose block loop keeps only the last 32-column block
// (src/model_q8.cpp:390-417), so only the last 32 entries of each row of xb
// are observable through xb2 in those paths.
//
// The reference terminates the process on pool exhaustion
// (src/pagedMemory.hpp:96,117,212); here `exit` is turned into a C++
// exception so a trace can record the failure and continue.

#include <immintrin.h>
#include <omp.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <iomanip>
#include <iostream>
#include <list>
#include <queue>
#include <stdexcept>
#include <unordered_map>
#include <vector>

struct RefExit {
    int code;
};
#define exit(code) throw RefExit{code}
#define private public
#include "model_q8.cpp"
#undef private
#include "NitroRPC.hpp"
#undef exit

namespace {

uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
float uniform_pm1(uint64_t& s) {  // uniform in [-1, 1)
    return (float)((double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0) * 2.0 - 1.0);
}

struct World {
    Config_Transformer c{};
    Transformer_Weights w{};
    RunState s{};
    KVBlock_Manager* mem = nullptr;
    PrefixCacheManager* cache = nullptr;
    std::vector<Request*> reqs;  // slot -> request (owns its Sequence)
    std::vector<float> emb, rms1, rms2, rms3, fcr, fci;
    std::vector<BlockQ8> wq, wk, wv, wo, w1, w2, w3;
    int kv_dim = 0, head_size = 0, max_rows = 0, total_blocks = 0;
    std::vector<float> key_cache, value_cache;
    Continuous_Scheduler* sched = nullptr;
    std::vector<Request*> sched_reqs;  // in the order they were added
};

void fill_q8(std::vector<BlockQ8>& m, int rows, int cols, uint64_t& rng, float scale) {
    m.resize((size_t)rows * cols / Q_BLOCK_SIZE);
    for (auto& b : m) {
        b.scale = scale;
        for (int i = 0; i < Q_BLOCK_SIZE; i++) b.weights[i] = (int8_t)((int)(splitmix64(rng) % 255) - 127);
    }
}
void identity_q8(std::vector<BlockQ8>& m, int rows, int cols) {
    m.assign((size_t)rows * cols / Q_BLOCK_SIZE, BlockQ8{});
    int nb = cols / Q_BLOCK_SIZE;
    for (auto& b : m) {
        b.scale = 1.0f;
        std::memset(b.weights, 0, sizeof(b.weights));
    }
    for (int i = 0; i < rows && i < cols; i++) m[(size_t)i * nb + i / Q_BLOCK_SIZE].weights[i % Q_BLOCK_SIZE] = 1;
}

}  // namespace

extern "C" {

uint64_t ref_hash_block_state(uint64_t parent, const int* tokens, int n) {
    std::vector<int> t(tokens, tokens + n);
    return hash_block_state(parent, t);
}

void ref_set_threads(int n) { omp_set_num_threads(n); }

// The reference's Q8 products called as units (src/model_q8.cpp:92-125,
// :382-420); w is packed BlockQ8 rows.
void ref_q8_matmul(float* out, const float* x, const void* w, int n, int d) {
    matmul(out, const_cast<float*>(x), (BlockQ8*)const_cast<void*>(w), n, d);
}
void ref_q8_matmul_bulk(float* out, const float* x, const void* w, int batch, int n, int d) {
    matmul_bulk(out, const_cast<float*>(x), (BlockQ8*)const_cast<void*>(w), batch, n, d);
}

// A tiny Llama-shaped model around a KVBlock_Manager/PrefixCacheManager pair.
// dim and kv_dim must be multiples of 32 (Q8 blocks); RoPE tables are the
// identity rotation so K/V rows in the pool are exactly the computed k/v.
static void* build_world(int n_heads, int n_kv_heads, int head_size, int n_layers, int vocab,
                         int seq_len, int hidden_dim, int total_blocks, int max_rows, int max_seqs,
                         uint64_t seed, bool random_model, float out_scale);

void* ref_world_create(int n_heads, int n_kv_heads, int head_size, int n_layers, int vocab,
                       int seq_len, int total_blocks, int max_rows, int max_seqs, uint64_t seed) {
    return build_world(n_heads, n_kv_heads, head_size, n_layers, vocab, seq_len, 32, total_blocks,
                       max_rows, max_seqs, seed, false, 1.0f);
}

// A tiny model with every weight random (embedding U[-1,1), rms weights
// U[0.5,1.5), Q8 matrices with random int8 and per-block scales), and the
// usual RoPE tables (angle pos * 10000^(-2i/head_size), i < head_size/2) —
// for logits-level golden vectors of the forward passes.  out_scale multiplies
// the scales of wo and w2 (the two products added to the residual stream):
// above 1 the layers outweigh the token's own embedding in the tied
// classifier, so the argmax depends on the attention context.
void* ref_model_create(int n_heads, int n_kv_heads, int head_size, int n_layers, int vocab,
                       int seq_len, int hidden_dim, int total_blocks, int max_rows, int max_seqs,
                       uint64_t seed, float out_scale) {
    return build_world(n_heads, n_kv_heads, head_size, n_layers, vocab, seq_len, hidden_dim,
                       total_blocks, max_rows, max_seqs, seed, true, out_scale);
}

static void* build_world(int n_heads, int n_kv_heads, int head_size, int n_layers, int vocab,
                         int seq_len, int hidden_dim, int total_blocks, int max_rows, int max_seqs,
                         uint64_t seed, bool random_model, float out_scale) {
    World* W = new World();
    Config_Transformer& c = W->c;
    c.dim = n_heads * head_size;
    c.hidden_dim = hidden_dim;
    c.n_layers = n_layers;
    c.n_heads = n_heads;
    c.n_kv_heads = n_kv_heads;
    c.vocab_size = vocab;
    c.seq_len = seq_len;
    W->head_size = head_size;
    W->kv_dim = n_kv_heads * head_size;
    W->max_rows = max_rows;
    W->total_blocks = total_blocks;
    uint64_t rng = seed;
    W->emb.resize((size_t)vocab * c.dim);
    for (auto& x : W->emb) x = uniform_pm1(rng);
    W->rms1.assign((size_t)n_layers * c.dim, 1.0f);
    W->rms2.assign((size_t)n_layers * c.dim, 1.0f);
    W->rms3.assign(c.dim, 1.0f);
    W->fcr.assign((size_t)seq_len * head_size / 2, 1.0f);
    W->fci.assign((size_t)seq_len * head_size / 2, 0.0f);
    fill_q8(W->wq, n_layers * c.dim, c.dim, rng, 1.0f / 64);
    fill_q8(W->wk, n_layers * W->kv_dim, c.dim, rng, 1.0f / 64);
    fill_q8(W->wv, n_layers * W->kv_dim, c.dim, rng, 1.0f / 64);
    // wo = identity per layer
    W->wo.clear();
    for (int l = 0; l < n_layers; l++) {
        std::vector<BlockQ8> one;
        identity_q8(one, c.dim, c.dim);
        W->wo.insert(W->wo.end(), one.begin(), one.end());
    }
    fill_q8(W->w1, n_layers * c.hidden_dim, c.dim, rng, 1.0f / 64);
    fill_q8(W->w3, n_layers * c.hidden_dim, c.dim, rng, 1.0f / 64);
    fill_q8(W->w2, n_layers * c.dim, c.hidden_dim, rng, 0.0f);
    if (random_model) {
        for (auto& x : W->rms1) x = 1.0f + 0.5f * uniform_pm1(rng);
        for (auto& x : W->rms2) x = 1.0f + 0.5f * uniform_pm1(rng);
        for (auto& x : W->rms3) x = 1.0f + 0.5f * uniform_pm1(rng);
        auto rand_q8 = [&](std::vector<BlockQ8>& m, int rows, int cols) {
            fill_q8(m, rows, cols, rng, 1.0f);
            const float base = 1.0f / (127.0f * std::sqrt((float)cols));
            for (auto& b : m) b.scale = base * (1.0f + 0.5f * uniform_pm1(rng));
        };
        rand_q8(W->wq, n_layers * c.dim, c.dim);
        rand_q8(W->wk, n_layers * W->kv_dim, c.dim);
        rand_q8(W->wv, n_layers * W->kv_dim, c.dim);
        rand_q8(W->wo, n_layers * c.dim, c.dim);
        rand_q8(W->w1, n_layers * c.hidden_dim, c.dim);
        rand_q8(W->w3, n_layers * c.hidden_dim, c.dim);
        rand_q8(W->w2, n_layers * c.dim, c.hidden_dim);
        for (auto& b : W->wo) b.scale *= out_scale;
        for (auto& b : W->w2) b.scale *= out_scale;
        for (int pos = 0; pos < seq_len; pos++)
            for (int i = 0; i < head_size / 2; i++) {
                const double ang = pos * std::pow(10000.0, -2.0 * i / head_size);
                W->fcr[(size_t)pos * (head_size / 2) + i] = (float)std::cos(ang);
                W->fci[(size_t)pos * (head_size / 2) + i] = (float)std::sin(ang);
            }
    }
    Transformer_Weights& w = W->w;
    w.token_embedding_table = W->emb.data();
    w.rms_attn_weights = W->rms1.data();
    w.wq = W->wq.data();
    w.wk = W->wk.data();
    w.wv = W->wv.data();
    w.wo = W->wo.data();
    w.rms_ffn_weight = W->rms2.data();
    w.w1 = W->w1.data();
    w.w2 = W->w2.data();
    w.w3 = W->w3.data();
    w.freq_cis_real = W->fcr.data();
    w.freq_cis_imag = W->fci.data();
    w.rms_final_weight = W->rms3.data();
    w.wcls = W->emb.data();
    RunState& s = W->s;
    s.x = (float*)calloc((size_t)max_rows * c.dim, sizeof(float));
    s.xb = (float*)calloc((size_t)max_rows * c.dim, sizeof(float));
    s.xb2 = (float*)calloc((size_t)max_rows * c.dim, sizeof(float));
    s.hb = (float*)calloc((size_t)max_rows * c.hidden_dim, sizeof(float));
    s.hb2 = (float*)calloc((size_t)max_rows * c.hidden_dim, sizeof(float));
    s.q = (float*)calloc((size_t)max_rows * c.dim, sizeof(float));
    s.k = (float*)calloc((size_t)max_rows * W->kv_dim, sizeof(float));
    s.v = (float*)calloc((size_t)max_rows * W->kv_dim, sizeof(float));
    s.logits = (float*)calloc((size_t)max_rows * vocab, sizeof(float));
    s.attn = (float*)calloc((size_t)max_rows * n_heads * seq_len, sizeof(float));
    W->key_cache.assign((size_t)n_layers * seq_len * W->kv_dim, 0.0f);
    W->value_cache.assign((size_t)n_layers * seq_len * W->kv_dim, 0.0f);
    s.key_cache = W->key_cache.data();
    s.value_cache = W->value_cache.data();
    W->mem = new KVBlock_Manager(total_blocks, n_layers, W->kv_dim);
    W->cache = new PrefixCacheManager(*W->mem, total_blocks);
    W->reqs.assign(max_seqs, nullptr);
    return W;
}

// Writes the model in the reference's file layout (src/Server_Inference.cpp:45-69):
// 7 int32 header fields, then the weight sections in load order.  Returns the
// byte count; writes only when cap is large enough.
uint64_t ref_model_serialize(void* p, uint8_t* out, uint64_t cap) {
    World* W = (World*)p;
    const Config_Transformer& c = W->c;
    std::vector<uint8_t> b;
    auto put = [&](const void* src, size_t n) {
        const uint8_t* s = (const uint8_t*)src;
        b.insert(b.end(), s, s + n);
    };
    const int32_t h[7] = {c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size, c.seq_len};
    put(h, sizeof(h));
    put(W->emb.data(), W->emb.size() * 4);
    put(W->rms1.data(), W->rms1.size() * 4);
    put(W->wq.data(), W->wq.size() * sizeof(BlockQ8));
    put(W->wk.data(), W->wk.size() * sizeof(BlockQ8));
    put(W->wv.data(), W->wv.size() * sizeof(BlockQ8));
    put(W->wo.data(), W->wo.size() * sizeof(BlockQ8));
    put(W->rms2.data(), W->rms2.size() * 4);
    put(W->w1.data(), W->w1.size() * sizeof(BlockQ8));
    put(W->w2.data(), W->w2.size() * sizeof(BlockQ8));
    put(W->w3.data(), W->w3.size() * sizeof(BlockQ8));
    put(W->rms3.data(), W->rms3.size() * 4);
    put(W->fcr.data(), W->fcr.size() * 4);
    put(W->fci.data(), W->fci.size() * 4);
    if (b.size() <= cap) std::memcpy(out, b.data(), b.size());
    return b.size();
}

// Copies rows [0, rows) of s->logits (rows x vocab_size).
int ref_read_logits(void* p, int rows, float* out) {
    World* W = (World*)p;
    if (rows > W->max_rows) return 1;
    std::memcpy(out, W->s.logits, sizeof(float) * (size_t)rows * W->c.vocab_size);
    return 0;
}

void ref_world_destroy(void* p) {
    World* W = (World*)p;
    for (auto* r : W->reqs) delete r;
    for (auto* r : W->sched_reqs) delete r;
    delete W->sched;
    delete W->cache;
    delete W->mem;
    RunState& s = W->s;
    free(s.x); free(s.xb); free(s.xb2); free(s.hb); free(s.hb2);
    free(s.q); free(s.k); free(s.v); free(s.logits); free(s.attn);
    delete W;
}

// Replaces the RoPE tables (seq_len x head_size/2 each); the world is created
// with the identity rotation (real 1, imaginary 0).
int ref_world_set_rope(void* p, const float* real, const float* imag) {
    World* W = (World*)p;
    std::memcpy(W->fcr.data(), real, sizeof(float) * W->fcr.size());
    std::memcpy(W->fci.data(), imag, sizeof(float) * W->fci.size());
    return 0;
}

int ref_world_dims(void* p, int* out) {
    World* W = (World*)p;
    out[0] = W->c.dim;
    out[1] = W->kv_dim;
    out[2] = W->c.n_layers;
    out[3] = W->total_blocks;
    out[4] = (int)W->reqs.size();
    return 0;
}

// ---- block manager / prefix cache / sequence operations -------------------
// Returns 0 on success, 1 when the reference called exit().
enum {
    OP_ALLOC = 1, OP_INC = 2, OP_FREE = 3, OP_FORCE_FREE = 4, OP_CHECK = 5, OP_INSERT = 6,
    OP_EVICT = 7, OP_SEQ_NEW = 8, OP_SEQ_APPEND = 9, OP_SEQ_FLUSH = 10, OP_SEQ_RELEASE = 11,
    OP_INGEST = 12, OP_FREE_COUNT = 13, OP_IS_CACHED = 14
};

int ref_op(void* p, int op, int a, int b, uint64_t h, const int* toks, int ntoks, int64_t* result) {
    World* W = (World*)p;
    KVBlock_Manager& mem = *W->mem;
    PrefixCacheManager& cache = *W->cache;
    *result = 0;
    try {
        switch (op) {
            case OP_ALLOC: *result = mem.allocate_block(cache); break;
            case OP_INC: mem.inc_ref_count(a, cache); break;
            case OP_FREE: mem.free_block(a, cache); break;
            case OP_FORCE_FREE: mem.force_free_block(a); break;
            case OP_CHECK: *result = cache.check_cache(h); break;
            case OP_INSERT: cache.insert_cache(h, a, b); break;
            case OP_EVICT: cache.evict_lru_block(); break;
            case OP_FREE_COUNT: *result = mem.get_free_count(); break;
            case OP_IS_CACHED: *result = cache.is_cached(a) ? 1 : 0; break;
            case OP_SEQ_NEW: {
                delete W->reqs[a];
                std::vector<int> prompt(toks, toks + ntoks);
                W->reqs[a] = new Request(a, prompt);
                break;
            }
            case OP_SEQ_APPEND: W->reqs[a]->seq.allocate_next_token(b, mem, cache); break;
            case OP_SEQ_FLUSH: W->reqs[a]->seq.flush_cache(cache); break;
            case OP_SEQ_RELEASE: W->reqs[a]->seq.release(mem, cache); break;
            case OP_INGEST: {
                std::vector<int> prompt(toks, toks + ntoks);
                *result = ingest_prompt(prompt, W->reqs[a]->seq, mem, cache, &W->c, &W->w, &W->s, b != 0);
                break;
            }
            default: return 2;
        }
    } catch (const RefExit&) {
        return 1;
    }
    return 0;
}

// Serialises the bookkeeping state into an int32 stream:
//   free_list [n, ids...]; per block [ref_count, num_tokens, parent_id, child_count];
//   evictable_leaves front->back [n, ids...]; cache_map sorted by hash [n, (lo, hi, id)...];
//   reverse_map sorted by id [n, (id, lo, hi)...]; per sequence slot
//   [exists, logical_token_count, hash lo, hash hi, |buffer|, buffer..., |table|, table...].
int ref_snapshot(void* p, int32_t* buf, int cap) {
    World* W = (World*)p;
    std::vector<int32_t> o;
    KVBlock_Manager& mem = *W->mem;
    PrefixCacheManager& cache = *W->cache;
    o.push_back((int32_t)mem.free_list.size());
    for (int id : mem.free_list) o.push_back(id);
    for (auto& b : mem.blocks) {
        o.push_back(b.ref_count);
        o.push_back(b.num_tokens);
        o.push_back(b.parent_id);
        o.push_back(b.child_count);
    }
    o.push_back((int32_t)cache.evictable_leaves.size());
    for (int id : cache.evictable_leaves) o.push_back(id);
    std::vector<std::pair<uint64_t, int>> cm(cache.cache_map.begin(), cache.cache_map.end());
    std::sort(cm.begin(), cm.end());
    o.push_back((int32_t)cm.size());
    for (auto& e : cm) {
        o.push_back((int32_t)(uint32_t)(e.first & 0xffffffffu));
        o.push_back((int32_t)(uint32_t)(e.first >> 32));
        o.push_back(e.second);
    }
    std::vector<std::pair<int, uint64_t>> rm(cache.reverse_map.begin(), cache.reverse_map.end());
    std::sort(rm.begin(), rm.end());
    o.push_back((int32_t)rm.size());
    for (auto& e : rm) {
        o.push_back(e.first);
        o.push_back((int32_t)(uint32_t)(e.second & 0xffffffffu));
        o.push_back((int32_t)(uint32_t)(e.second >> 32));
    }
    for (auto* r : W->reqs) {
        if (!r) {
            o.push_back(0);
            continue;
        }
        Sequence& q = r->seq;
        o.push_back(1);
        o.push_back(q.logical_token_count);
        o.push_back((int32_t)(uint32_t)(q.current_hash & 0xffffffffu));
        o.push_back((int32_t)(uint32_t)(q.current_hash >> 32));
        o.push_back((int32_t)q.token_buffer.size());
        for (int t : q.token_buffer) o.push_back(t);
        o.push_back((int32_t)q.block_table.size());
        for (int t : q.block_table) o.push_back(t);
    }
    if ((int)o.size() > cap) return -(int)o.size();
    std::memcpy(buf, o.data(), o.size() * sizeof(int32_t));
    return (int)o.size();
}

// ---- forward passes (attention observed through xb2) ----------------------

int ref_decode_batch(void* p, const int* slots, const int* tokens, int B, int* positions_out) {
    World* W = (World*)p;
    std::vector<int> toks(tokens, tokens + B), pos(B);
    std::vector<Request*> rs(B);
    for (int b = 0; b < B; b++) {
        rs[b] = W->reqs[slots[b]];
        pos[b] = rs[b]->seq.logical_token_count;
        positions_out[b] = pos[b];
    }
    try {
        forward_decode_batch(toks, pos, rs, &W->c, &W->w, &W->s, *W->mem, *W->cache);
    } catch (const RefExit&) {
        return 1;
    }
    return 0;
}

int ref_forward_paged(void* p, int slot, int token, int* pos_out) {
    World* W = (World*)p;
    Sequence& q = W->reqs[slot]->seq;
    int pos = q.logical_token_count;
    *pos_out = pos;
    try {
        forward_paged(token, pos, &W->c, &W->w, &W->s, q, *W->mem, *W->cache);
    } catch (const RefExit&) {
        return 1;
    }
    return 0;
}

int ref_prefill_chunk(void* p, int slot, const int* tokens, int n, int* start_pos_out) {
    World* W = (World*)p;
    Sequence& q = W->reqs[slot]->seq;
    std::vector<int> toks(tokens, tokens + n);
    *start_pos_out = q.logical_token_count;
    try {
        forward_prefill_chunk(toks, q.logical_token_count, &W->c, &W->w, &W->s, q, *W->mem, *W->cache);
    } catch (const RefExit&) {
        return 1;
    }
    return 0;
}

int ref_forward_contiguous(void* p, int token, int pos) {
    World* W = (World*)p;
    forward(token, pos, &W->c, &W->w, &W->s);
    return 0;
}

// Copies rows [0, rows) of s->q, s->k, s->v (post-RoPE inputs of the last
// layer's attention) and s->xb2 (= wo . attention output).
int ref_read_rows(void* p, int rows, float* q, float* k, float* v, float* xb2) {
    World* W = (World*)p;
    if (rows > W->max_rows) return 1;
    std::memcpy(q, W->s.q, sizeof(float) * (size_t)rows * W->c.dim);
    std::memcpy(k, W->s.k, sizeof(float) * (size_t)rows * W->kv_dim);
    std::memcpy(v, W->s.v, sizeof(float) * (size_t)rows * W->kv_dim);
    std::memcpy(xb2, W->s.xb2, sizeof(float) * (size_t)rows * W->c.dim);
    return 0;
}

static size_t pool_floats(World* W) {
    return (size_t)W->total_blocks * W->c.n_layers * BLOCK_SIZE * W->kv_dim;
}

int ref_read_pool(void* p, float* k_pool, float* v_pool) {
    World* W = (World*)p;
    KVBlock_Manager& mem = *W->mem;
    std::memcpy(k_pool, mem.global_k_pool, sizeof(float) * pool_floats(W));
    std::memcpy(v_pool, mem.global_v_pool, sizeof(float) * pool_floats(W));
    return 0;
}

int ref_write_pool(void* p, const float* k_pool, const float* v_pool) {
    World* W = (World*)p;
    KVBlock_Manager& mem = *W->mem;
    std::memcpy(mem.global_k_pool, k_pool, sizeof(float) * pool_floats(W));
    std::memcpy(mem.global_v_pool, v_pool, sizeof(float) * pool_floats(W));
    return 0;
}

int ref_read_contiguous_cache(void* p, float* key_cache, float* value_cache) {
    World* W = (World*)p;
    std::memcpy(key_cache, W->key_cache.data(), sizeof(float) * W->key_cache.size());
    std::memcpy(value_cache, W->value_cache.data(), sizeof(float) * W->value_cache.size());
    return 0;
}

int ref_write_contiguous_cache(void* p, const float* key_cache, const float* value_cache) {
    World* W = (World*)p;
    std::memcpy(W->key_cache.data(), key_cache, sizeof(float) * W->key_cache.size());
    std::memcpy(W->value_cache.data(), value_cache, sizeof(float) * W->value_cache.size());
    return 0;
}

// ---- Continuous_Scheduler (src/pagedMemory.hpp:287-399) -------------------
// One scheduler over the world's model, block manager and prefix cache.  The
// budget member max_tokens_per_batch (256 in the reference) may be set so
// small models exercise chunked prefill; everything else is the reference's.

int ref_sched_create(void* p, int max_tokens_per_batch) {
    World* W = (World*)p;
    if (W->sched) return 1;
    W->sched = new Continuous_Scheduler();
    W->sched->max_tokens_per_batch = max_tokens_per_batch;
    return 0;
}

int ref_sched_add(void* p, int req_id, const int* prompt, int n) {
    World* W = (World*)p;
    if (!W->sched || n <= 0) return 1;
    Request* r = new Request(req_id, std::vector<int>(prompt, prompt + n));
    W->sched_reqs.push_back(r);
    W->sched->add_request(r);
    return 0;
}

int ref_sched_active(void* p) { return ((World*)p)->sched->has_active_requests() ? 1 : 0; }

// Returns 0, or 1 when the reference called exit() (pool exhausted).
int ref_sched_step(void* p) {
    World* W = (World*)p;
    try {
        W->sched->step(&W->c, &W->w, &W->s, *W->mem, *W->cache);
    } catch (const RefExit&) {
        return 1;
    }
    return 0;
}

// Serialises the scheduler into an int32 stream:
//   [n, running_batch ids...] [n, waiting_queue ids front->back...] [n_requests]
//   then per request, in the order added: [req_id, prefill_idx, is_prefill_done,
//   is_finished, next_token_to_process, |generated|, generated...,
//   logical_token_count, hash lo, hash hi, |buffer|, buffer..., |table|, table...].
// Returns the word count (negated when cap is too small).
int ref_sched_state(void* p, int32_t* buf, int cap) {
    World* W = (World*)p;
    std::vector<int32_t> o;
    o.push_back((int32_t)W->sched->running_batch.size());
    for (Request* r : W->sched->running_batch) o.push_back(r->req_id);
    std::queue<Request*> q = W->sched->waiting_queue;
    o.push_back((int32_t)q.size());
    for (; !q.empty(); q.pop()) o.push_back(q.front()->req_id);
    o.push_back((int32_t)W->sched_reqs.size());
    for (Request* r : W->sched_reqs) {
        o.push_back(r->req_id);
        o.push_back(r->prefill_idx);
        o.push_back(r->is_prefill_done ? 1 : 0);
        o.push_back(r->is_finished ? 1 : 0);
        o.push_back(r->next_token_to_process);
        o.push_back((int32_t)r->generated_tokens.size());
        for (int t : r->generated_tokens) o.push_back(t);
        const Sequence& q2 = r->seq;
        o.push_back(q2.logical_token_count);
        o.push_back((int32_t)(uint32_t)(q2.current_hash & 0xffffffffu));
        o.push_back((int32_t)(uint32_t)(q2.current_hash >> 32));
        o.push_back((int32_t)q2.token_buffer.size());
        for (int t : q2.token_buffer) o.push_back(t);
        o.push_back((int32_t)q2.block_table.size());
        for (int t : q2.block_table) o.push_back(t);
    }
    if ((int)o.size() > cap) return -(int)o.size();
    std::memcpy(buf, o.data(), o.size() * sizeof(int32_t));
    return (int)o.size();
}

// ---- NitroRPC (src/NitroRPC.hpp), over a connected socket ----------------
int ref_rpc_send_ints(int fd, const int* data, int n) {
    return NitroRPC::send_ints(fd, std::vector<int>(data, data + n)) ? 0 : 1;
}

// Returns the count received (or -1 on failure); copies at most cap values.
int ref_rpc_recv_ints(int fd, int* out, int cap) {
    std::vector<int> v;
    if (!NitroRPC::recv_ints(fd, v)) return -1;
    for (int i = 0; i < (int)v.size() && i < cap; i++) out[i] = v[i];
    return (int)v.size();
}

int ref_rpc_recv_structured_query(int fd, int dim, uint64_t* mask, float* lo, float* hi, float* vec) {
    StructuredQuery q;
    if (!NitroRPC::recv_structured_query(fd, q, dim)) return 1;
    *mask = q.subset_mask;
    *lo = q.range_min;
    *hi = q.range_max;
    for (int i = 0; i < dim; i++) vec[i] = q.vec[i];
    return 0;
}

int ref_block_table(void* p, int slot, int* out, int cap) {
    World* W = (World*)p;
    if (!W->reqs[slot]) return -1;
    auto& t = W->reqs[slot]->seq.block_table;
    if ((int)t.size() > cap) return -(int)t.size();
    for (size_t i = 0; i < t.size(); i++) out[i] = t[i];
    return (int)t.size();
}

}  // extern "C"
