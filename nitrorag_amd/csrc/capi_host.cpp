// C ABI of the host page bookkeeping (declared in include/nitro_paged_attn.h).
#include <algorithm>
#include <cstring>

#include "capi_common.hpp"
#include "nitro_paged_attn.h"
#include "paged_memory.hpp"

namespace nitro {
namespace {
thread_local std::string g_last_error;

template <class T>
void copy_out(const std::vector<T>& v, T* out, int32_t cap, int32_t* n) {
    require(n != nullptr, ERR_INVALID_ARGUMENT, "null count pointer");
    *n = (int32_t)v.size();
    require(cap >= (int32_t)v.size() || out == nullptr, ERR_INVALID_ARGUMENT,
            "output buffer too small (the required size is in *n)");
    if (out) std::copy(v.begin(), v.end(), out);
}
}  // namespace

void set_last_error(const std::string& msg) { g_last_error = msg; }
void clear_last_error() { g_last_error.clear(); }
}  // namespace nitro

using namespace nitro;

extern "C" {

const char* nitro_status_string(int status) {
    switch (status) {
        case NITRO_OK: return "ok";
        case NITRO_ERR_INVALID_ARGUMENT: return "invalid argument";
        case NITRO_ERR_UNSUPPORTED: return "unsupported shape";
        case NITRO_ERR_DEVICE_ALLOC: return "device allocation failed";
        case NITRO_ERR_OUT_OF_PAGES: return "out of pages";
        case NITRO_ERR_BAD_BLOCK_TABLE: return "bad block table";
        case NITRO_ERR_HIP: return "HIP runtime error";
        case NITRO_ERR_NO_BATCH: return "no batch uploaded";
        default: return "unknown status";
    }
}

const char* nitro_last_error(void) { return g_last_error.c_str(); }

uint64_t nitro_hash_block_state(uint64_t parent_hash, const int32_t* tokens, int32_t n) {
    if (n <= 0 || tokens == nullptr) return parent_hash;
    return hash_block_state(parent_hash, tokens, n);
}

int nitro_bm_create(int32_t total_blocks, nitro_block_manager** out) {
    return guarded([&] {
        require(out != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        *out = nullptr;
        require(total_blocks > 0, ERR_INVALID_ARGUMENT, "total_blocks must be positive");
        *out = new nitro_block_manager(total_blocks);
    });
}

int nitro_bm_destroy(nitro_block_manager* bm) {
    delete bm;
    return NITRO_OK;
}

#define BM_REQUIRE(bm) require((bm) != nullptr, ERR_INVALID_ARGUMENT, "null block manager")

int nitro_bm_allocate_block(nitro_block_manager* bm, int32_t* id) {
    return guarded([&] {
        BM_REQUIRE(bm);
        require(id != nullptr, ERR_INVALID_ARGUMENT, "null id pointer");
        *id = bm->bm.mem.allocate_block(bm->bm.cache);
    });
}

int nitro_bm_inc_ref_count(nitro_block_manager* bm, int32_t id) {
    return guarded([&] {
        BM_REQUIRE(bm);
        bm->bm.mem.inc_ref_count(id, bm->bm.cache);
    });
}

int nitro_bm_free_block(nitro_block_manager* bm, int32_t id) {
    return guarded([&] {
        BM_REQUIRE(bm);
        bm->bm.mem.free_block(id, bm->bm.cache);
    });
}

int nitro_bm_force_free_block(nitro_block_manager* bm, int32_t id) {
    return guarded([&] {
        BM_REQUIRE(bm);
        bm->bm.mem.force_free_block(id);
    });
}

int nitro_bm_get_free_count(const nitro_block_manager* bm, int32_t* n) {
    return guarded([&] {
        BM_REQUIRE(bm);
        require(n != nullptr, ERR_INVALID_ARGUMENT, "null count pointer");
        *n = bm->bm.mem.get_free_count();
    });
}

int nitro_bm_get_block(const nitro_block_manager* bm, int32_t id, nitro_block_info* out) {
    return guarded([&] {
        BM_REQUIRE(bm);
        require(out != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        const KVBlock& b = bm->bm.mem.get_block(id);
        out->num_tokens = b.num_tokens;
        out->ref_count = b.ref_count;
        out->parent_id = b.parent_id;
        out->child_count = b.child_count;
    });
}

int nitro_bm_is_cached(const nitro_block_manager* bm, int32_t id, int32_t* cached) {
    return guarded([&] {
        BM_REQUIRE(bm);
        require(cached != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        bm->bm.mem.check_id(id);
        *cached = bm->bm.cache.is_cached(id) ? 1 : 0;
    });
}

int nitro_bm_check_cache(const nitro_block_manager* bm, uint64_t block_hash, int32_t* id) {
    return guarded([&] {
        BM_REQUIRE(bm);
        require(id != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        *id = bm->bm.cache.check_cache(block_hash);
    });
}

int nitro_bm_insert_cache(nitro_block_manager* bm, uint64_t block_hash, int32_t id, int32_t parent_id) {
    return guarded([&] {
        BM_REQUIRE(bm);
        bm->bm.cache.insert_cache(block_hash, id, parent_id);
    });
}

int nitro_bm_evict_lru_block(nitro_block_manager* bm) {
    return guarded([&] {
        BM_REQUIRE(bm);
        bm->bm.cache.evict_lru_block();
    });
}

int nitro_bm_free_list(const nitro_block_manager* bm, int32_t* ids, int32_t cap, int32_t* n) {
    return guarded([&] {
        BM_REQUIRE(bm);
        copy_out(bm->bm.mem.free_ids(), ids, cap, n);
    });
}

int nitro_bm_evictable_leaves(const nitro_block_manager* bm, int32_t* ids, int32_t cap, int32_t* n) {
    return guarded([&] {
        BM_REQUIRE(bm);
        copy_out(bm->bm.cache.evictable_leaves_front_to_back(), ids, cap, n);
    });
}

int nitro_bm_cache_entries(const nitro_block_manager* bm, uint64_t* hashes, int32_t* ids,
                           int32_t cap, int32_t* n) {
    return guarded([&] {
        BM_REQUIRE(bm);
        require(n != nullptr, ERR_INVALID_ARGUMENT, "null count pointer");
        auto e = bm->bm.cache.cache_entries();
        *n = (int32_t)e.size();
        if (!hashes && !ids) return;
        require(cap >= (int32_t)e.size(), ERR_INVALID_ARGUMENT, "output buffer too small");
        for (size_t i = 0; i < e.size(); i++) {
            if (hashes) hashes[i] = e[i].first;
            if (ids) ids[i] = e[i].second;
        }
    });
}

int nitro_bm_reverse_entries(const nitro_block_manager* bm, int32_t* ids, uint64_t* hashes,
                             int32_t cap, int32_t* n) {
    return guarded([&] {
        BM_REQUIRE(bm);
        require(n != nullptr, ERR_INVALID_ARGUMENT, "null count pointer");
        auto e = bm->bm.cache.reverse_entries();
        *n = (int32_t)e.size();
        if (!hashes && !ids) return;
        require(cap >= (int32_t)e.size(), ERR_INVALID_ARGUMENT, "output buffer too small");
        for (size_t i = 0; i < e.size(); i++) {
            if (ids) ids[i] = e[i].first;
            if (hashes) hashes[i] = e[i].second;
        }
    });
}

// ------------------------------------------------------------------ Sequence
#define SEQ_REQUIRE(s) require((s) != nullptr, ERR_INVALID_ARGUMENT, "null sequence")

int nitro_seq_create(int32_t seq_id, nitro_sequence** out) {
    return guarded([&] {
        require(out != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        *out = new nitro_sequence(seq_id);
    });
}

int nitro_seq_destroy(nitro_sequence* seq) {
    delete seq;
    return NITRO_OK;
}

int nitro_seq_allocate_next_token(nitro_sequence* seq, nitro_block_manager* bm, int32_t token) {
    return guarded([&] {
        SEQ_REQUIRE(seq);
        BM_REQUIRE(bm);
        seq->seq.allocate_next_token(token, bm->bm.mem, bm->bm.cache);
    });
}

int nitro_seq_flush_cache(nitro_sequence* seq, nitro_block_manager* bm) {
    return guarded([&] {
        SEQ_REQUIRE(seq);
        BM_REQUIRE(bm);
        seq->seq.flush_cache(bm->bm.cache);
    });
}

int nitro_seq_release(nitro_sequence* seq, nitro_block_manager* bm) {
    return guarded([&] {
        SEQ_REQUIRE(seq);
        BM_REQUIRE(bm);
        seq->seq.release(bm->bm.mem, bm->bm.cache);
    });
}

int nitro_seq_prefix_walk(nitro_sequence* seq, nitro_block_manager* bm, const int32_t* prompt,
                          int32_t n, int32_t start, int32_t require_empty_buffer, int32_t* next) {
    return guarded([&] {
        SEQ_REQUIRE(seq);
        BM_REQUIRE(bm);
        require(next != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        require(n >= 0 && start >= 0 && (prompt != nullptr || n == 0), ERR_INVALID_ARGUMENT,
                "bad prompt");
        *next = seq->seq.prefix_walk(prompt, n, start, require_empty_buffer != 0, bm->bm.mem,
                                     bm->bm.cache);
    });
}

int nitro_seq_ingest_prompt(nitro_sequence* seq, nitro_block_manager* bm, const int32_t* prompt,
                            int32_t n, int32_t enable_prefix_caching, int32_t* count) {
    return guarded([&] {
        SEQ_REQUIRE(seq);
        BM_REQUIRE(bm);
        require(n >= 0 && (prompt != nullptr || n == 0), ERR_INVALID_ARGUMENT, "bad prompt");
        int p = 0;
        if (enable_prefix_caching) p = seq->seq.prefix_walk(prompt, n, 0, false, bm->bm.mem, bm->bm.cache);
        for (; p < n; p++) seq->seq.allocate_next_token(prompt[p], bm->bm.mem, bm->bm.cache);
        if (count) *count = seq->seq.logical_token_count;
    });
}

int nitro_seq_state(const nitro_sequence* seq, int32_t* logical_token_count, uint64_t* current_hash,
                    int32_t* buffered_tokens, int32_t* num_pages) {
    return guarded([&] {
        SEQ_REQUIRE(seq);
        if (logical_token_count) *logical_token_count = seq->seq.logical_token_count;
        if (current_hash) *current_hash = seq->seq.current_hash;
        if (buffered_tokens) *buffered_tokens = (int32_t)seq->seq.token_buffer.size();
        if (num_pages) *num_pages = (int32_t)seq->seq.block_table.size();
    });
}

int nitro_seq_block_table(const nitro_sequence* seq, int32_t* pages, int32_t cap, int32_t* n) {
    return guarded([&] {
        SEQ_REQUIRE(seq);
        copy_out(seq->seq.block_table, pages, cap, n);
    });
}

int nitro_seq_token_buffer(const nitro_sequence* seq, int32_t* tokens, int32_t cap, int32_t* n) {
    return guarded([&] {
        SEQ_REQUIRE(seq);
        copy_out(seq->seq.token_buffer, tokens, cap, n);
    });
}

int nitro_pack_block_tables(const nitro_sequence* const* seqs, int32_t batch, int32_t max_pages,
                            int32_t* tables) {
    return guarded([&] {
        require(seqs != nullptr && tables != nullptr && batch > 0 && max_pages > 0,
                ERR_INVALID_ARGUMENT, "bad arguments");
        for (int b = 0; b < batch; b++) {
            require(seqs[b] != nullptr, ERR_INVALID_ARGUMENT, "null sequence in batch");
            const auto& t = seqs[b]->seq.block_table;
            require((int)t.size() <= max_pages, ERR_BAD_BLOCK_TABLE,
                    "a block table is longer than max_pages");
            int32_t* row = tables + (size_t)b * max_pages;
            std::fill(row, row + max_pages, 0);
            std::copy(t.begin(), t.end(), row);
        }
    });
}

}  // extern "C"
