// Host page bookkeeping of the paged-attention path (C++17, no device code).
//
// Semantics follow the reference's src/pagedMemory.hpp:9-285 operation by
// operation, so block ids, reference counts, prefix-cache topology and
// eviction order come out bit-identical:
//   - a LIFO free list initialised to [0..N-1] (the first allocation is N-1);
//   - ref_count=1 on allocation, a page returns to the free list when its
//     count reaches 0 and it is not in the prefix cache;
//   - the prefix cache maps FNV-1a-64 chain hashes to pages, tracks
//     parent/child counts, keeps leaves (ref 0, no children) in an MRU-first
//     list and, when the free list is empty and fewer than 5% of pages are
//     free, evicts from the LRU end until 20% are free, cascading to parents.
// Differences from the reference, by design: failures throw nitro::Error
// (mapped to status codes at the C ABI) where the reference calls exit(1);
// ids are range-checked; the LRU list is intrusive (prev/next arrays) and the
// reverse map is a per-page array, which keep the same observable order and
// contents as the reference's std::list / unordered_map.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace nitro {

constexpr int BLOCK_SIZE = 16;  // src/pagedMemory.hpp:9
constexpr uint64_t FNV_OFFSET_BASIS = 14695981039346656037ULL;
constexpr uint64_t FNV_PRIME = 1099511628211ULL;

enum Status : int {
    OK = 0,
    ERR_INVALID_ARGUMENT = 1,
    ERR_UNSUPPORTED = 2,
    ERR_DEVICE_ALLOC = 3,
    ERR_OUT_OF_PAGES = 4,
    ERR_BAD_BLOCK_TABLE = 5,
    ERR_HIP = 6,
    ERR_NO_BATCH = 7,
};

class Error : public std::runtime_error {
  public:
    Error(Status s, const std::string& msg) : std::runtime_error(msg), status(s) {}
    Status status;
};

// FNV-1a 64 continued from parent_hash over each token's 4 little-endian
// bytes (src/pagedMemory.hpp:14-24).
uint64_t hash_block_state(uint64_t parent_hash, const int32_t* tokens, int n);

struct KVBlock {  // src/pagedMemory.hpp:28-37 (storage pointers live in the device pool)
    int32_t physical_id = 0;
    int32_t num_tokens = 0;
    int32_t ref_count = 0;
    int32_t parent_id = -1;
    int32_t child_count = 0;
};

class PrefixCacheManager;

class KVBlock_Manager {
  public:
    explicit KVBlock_Manager(int total_blocks);
    int allocate_block(PrefixCacheManager& cache_mgr);
    void inc_ref_count(int id, PrefixCacheManager& cache_mgr);
    int get_free_count() const { return (int)free_list.size(); }
    void free_block(int id, PrefixCacheManager& cache_mgr);
    void force_free_block(int id);
    KVBlock& get_block(int id);
    const KVBlock& get_block(int id) const;
    int total_blocks() const { return (int)blocks.size(); }
    const std::vector<int32_t>& free_ids() const { return free_list; }
    void check_id(int id) const;

  private:
    std::vector<KVBlock> blocks;
    std::vector<int32_t> free_list;
};

class PrefixCacheManager {
  public:
    PrefixCacheManager(KVBlock_Manager& mm, int total_blocks);
    void evaluate_evictability(int phy_id);
    void insert_cache(uint64_t block_hash, int physical_block_id, int parent_phy_id);
    void evict_lru_block();
    bool is_cached(int phy_id) const { return reverse_valid[phy_id] != 0; }
    int check_cache(uint64_t block_hash) const;

    std::vector<int32_t> evictable_leaves_front_to_back() const;
    std::vector<std::pair<uint64_t, int32_t>> cache_entries() const;    // sorted by hash
    std::vector<std::pair<int32_t, uint64_t>> reverse_entries() const;  // sorted by id

    KVBlock_Manager& mem_mgr;

  private:
    // evictable_leaves: intrusive doubly-linked list over page ids, head = front.
    void lru_push_front(int id);
    void lru_erase(int id);
    int lru_pop_back();

    std::unordered_map<uint64_t, int32_t> cache_map;
    std::vector<uint64_t> reverse_hash;
    std::vector<uint8_t> reverse_valid;
    std::vector<int32_t> lru_prev, lru_next;
    std::vector<uint8_t> in_lru;
    int lru_head = -1, lru_tail = -1;
    int min_free_blocks;
    int target_free_blocks;
};

struct Sequence {  // src/pagedMemory.hpp:233-285
    explicit Sequence(int id) : seq_id(id) {}
    void allocate_next_token(int token, KVBlock_Manager& manager, PrefixCacheManager& cache_mgr);
    void flush_cache(PrefixCacheManager& cache_mgr);
    void release(KVBlock_Manager& manager, PrefixCacheManager& cache_mgr);
    // Prefix-hit walk (src/pagedMemory.hpp:346-359 with require_empty_buffer,
    // src/model_q8.cpp:699-714 without); returns the first index not covered.
    int prefix_walk(const int32_t* prompt, int n, int start, bool require_empty_buffer,
                    KVBlock_Manager& manager, PrefixCacheManager& cache_mgr);

    int seq_id;
    std::vector<int32_t> block_table;
    int logical_token_count = 0;
    uint64_t current_hash = FNV_OFFSET_BASIS;
    std::vector<int32_t> token_buffer;
};

// KVBlock_Manager and its PrefixCacheManager, created and destroyed together.
struct BlockManager {
    explicit BlockManager(int total_blocks) : mem(total_blocks), cache(mem, total_blocks) {}
    KVBlock_Manager mem;
    PrefixCacheManager cache;
};

}  // namespace nitro
