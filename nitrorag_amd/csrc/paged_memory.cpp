// Host page bookkeeping — see paged_memory.hpp for the contract.
#include "paged_memory.hpp"

#include <algorithm>
#include <string>

namespace nitro {

uint64_t hash_block_state(uint64_t parent_hash, const int32_t* tokens, int n) {
    uint64_t h = parent_hash;
    for (int i = 0; i < n; i++) {
        const uint32_t t = (uint32_t)tokens[i];
        for (int byte = 0; byte < 4; byte++) {  // little-endian byte order of an int32
            h ^= (t >> (8 * byte)) & 0xffu;
            h *= FNV_PRIME;
        }
    }
    return h;
}

// ----------------------------------------------------------- KVBlock_Manager
KVBlock_Manager::KVBlock_Manager(int total_blocks) {
    if (total_blocks <= 0) throw Error(ERR_INVALID_ARGUMENT, "total_blocks must be positive");
    blocks.resize(total_blocks);
    free_list.reserve(total_blocks);
    for (int i = 0; i < total_blocks; i++) {
        blocks[i].physical_id = i;
        free_list.push_back(i);  // [0..N-1]; allocation pops from the back
    }
}

void KVBlock_Manager::check_id(int id) const {
    if (id < 0 || id >= (int)blocks.size())
        throw Error(ERR_INVALID_ARGUMENT, "page id " + std::to_string(id) + " outside [0, " +
                                              std::to_string(blocks.size()) + ")");
}

KVBlock& KVBlock_Manager::get_block(int id) {
    check_id(id);
    return blocks[id];
}

const KVBlock& KVBlock_Manager::get_block(int id) const {
    check_id(id);
    return blocks[id];
}

int KVBlock_Manager::allocate_block(PrefixCacheManager& cache_mgr) {
    if (free_list.empty()) {
        cache_mgr.evict_lru_block();
        if (free_list.empty()) throw Error(ERR_OUT_OF_PAGES, "out of pages: eviction failed");
    }
    int id = free_list.back();
    free_list.pop_back();
    KVBlock& b = blocks[id];
    b.ref_count = 1;
    b.num_tokens = 0;
    b.parent_id = -1;
    b.child_count = 0;
    return id;
}

void KVBlock_Manager::inc_ref_count(int id, PrefixCacheManager& cache_mgr) {
    get_block(id).ref_count++;
    cache_mgr.evaluate_evictability(id);
}

void KVBlock_Manager::free_block(int id, PrefixCacheManager& cache_mgr) {
    KVBlock& b = get_block(id);
    b.ref_count--;
    cache_mgr.evaluate_evictability(id);
    if (b.ref_count == 0 && !cache_mgr.is_cached(id)) {
        b.num_tokens = 0;
        free_list.push_back(id);
    }
}

void KVBlock_Manager::force_free_block(int id) {
    KVBlock& b = get_block(id);
    b.num_tokens = 0;
    b.ref_count = 0;
    b.parent_id = -1;
    b.child_count = 0;
    free_list.push_back(id);
}

// -------------------------------------------------------- PrefixCacheManager
PrefixCacheManager::PrefixCacheManager(KVBlock_Manager& mm, int total_blocks)
    : mem_mgr(mm),
      reverse_hash(total_blocks, 0),
      reverse_valid(total_blocks, 0),
      lru_prev(total_blocks, -1),
      lru_next(total_blocks, -1),
      in_lru(total_blocks, 0) {
    // 5% trigger, 20% target (src/pagedMemory.hpp:165-166), truncating casts as there.
    min_free_blocks = std::max(1, (int)(total_blocks * 0.05));
    target_free_blocks = std::max(2, (int)(total_blocks * 0.2));
    cache_map.reserve((size_t)total_blocks * 2);
}

void PrefixCacheManager::lru_push_front(int id) {
    lru_prev[id] = -1;
    lru_next[id] = lru_head;
    if (lru_head != -1) lru_prev[lru_head] = id;
    lru_head = id;
    if (lru_tail == -1) lru_tail = id;
    in_lru[id] = 1;
}

void PrefixCacheManager::lru_erase(int id) {
    int p = lru_prev[id], n = lru_next[id];
    if (p != -1) lru_next[p] = n; else lru_head = n;
    if (n != -1) lru_prev[n] = p; else lru_tail = p;
    lru_prev[id] = lru_next[id] = -1;
    in_lru[id] = 0;
}

int PrefixCacheManager::lru_pop_back() {
    int id = lru_tail;
    lru_erase(id);
    return id;
}

void PrefixCacheManager::evaluate_evictability(int phy_id) {
    if (!is_cached(phy_id)) return;
    const KVBlock& b = mem_mgr.get_block(phy_id);
    bool evictable = (b.ref_count == 0 && b.child_count == 0);
    bool listed = in_lru[phy_id] != 0;
    if (evictable && !listed)
        lru_push_front(phy_id);
    else if (!evictable && listed)
        lru_erase(phy_id);
}

int PrefixCacheManager::check_cache(uint64_t block_hash) const {
    auto it = cache_map.find(block_hash);
    return it == cache_map.end() ? -1 : it->second;
}

void PrefixCacheManager::insert_cache(uint64_t block_hash, int physical_block_id, int parent_phy_id) {
    mem_mgr.check_id(physical_block_id);
    if (parent_phy_id != -1) mem_mgr.check_id(parent_phy_id);
    cache_map[block_hash] = physical_block_id;
    reverse_hash[physical_block_id] = block_hash;
    reverse_valid[physical_block_id] = 1;
    KVBlock& b = mem_mgr.get_block(physical_block_id);
    b.parent_id = parent_phy_id;
    b.child_count = 0;
    if (parent_phy_id != -1) {
        mem_mgr.get_block(parent_phy_id).child_count++;
        evaluate_evictability(parent_phy_id);
    }
    evaluate_evictability(physical_block_id);
}

void PrefixCacheManager::evict_lru_block() {
    if (mem_mgr.get_free_count() >= min_free_blocks) return;
    while (mem_mgr.get_free_count() < target_free_blocks) {
        if (lru_tail == -1) {
            if (mem_mgr.get_free_count() > 0) break;
            throw Error(ERR_OUT_OF_PAGES, "out of pages: no evictable prefix-cache leaves left");
        }
        int evict_id = lru_pop_back();
        // A listed page is always cached; an absent entry would read as hash 0.
        uint64_t h = reverse_valid[evict_id] ? reverse_hash[evict_id] : 0;
        cache_map.erase(h);
        reverse_valid[evict_id] = 0;
        reverse_hash[evict_id] = 0;
        int parent_id = mem_mgr.get_block(evict_id).parent_id;
        if (parent_id != -1) {
            mem_mgr.get_block(parent_id).child_count--;
            evaluate_evictability(parent_id);
        }
        mem_mgr.force_free_block(evict_id);
    }
}

std::vector<int32_t> PrefixCacheManager::evictable_leaves_front_to_back() const {
    std::vector<int32_t> out;
    for (int id = lru_head; id != -1; id = lru_next[id]) out.push_back(id);
    return out;
}

std::vector<std::pair<uint64_t, int32_t>> PrefixCacheManager::cache_entries() const {
    std::vector<std::pair<uint64_t, int32_t>> out(cache_map.begin(), cache_map.end());
    std::sort(out.begin(), out.end());
    return out;
}

std::vector<std::pair<int32_t, uint64_t>> PrefixCacheManager::reverse_entries() const {
    std::vector<std::pair<int32_t, uint64_t>> out;
    for (int i = 0; i < (int)reverse_valid.size(); i++)
        if (reverse_valid[i]) out.emplace_back(i, reverse_hash[i]);
    return out;
}

// ------------------------------------------------------------------ Sequence
void Sequence::allocate_next_token(int token, KVBlock_Manager& manager, PrefixCacheManager& cache_mgr) {
    if ((int)token_buffer.size() == BLOCK_SIZE) {
        // The page filled by the previous 16 tokens enters the prefix cache
        // only now, when its successor token arrives (src/pagedMemory.hpp:247-254).
        current_hash = hash_block_state(current_hash, token_buffer.data(), BLOCK_SIZE);
        int finished = block_table.back();
        int parent = block_table.size() > 1 ? block_table[block_table.size() - 2] : -1;
        cache_mgr.insert_cache(current_hash, finished, parent);
        token_buffer.clear();
    }
    if (logical_token_count % BLOCK_SIZE == 0) block_table.push_back(manager.allocate_block(cache_mgr));
    if (block_table.empty()) throw Error(ERR_INVALID_ARGUMENT, "sequence has no page to append to");
    token_buffer.push_back(token);
    manager.get_block(block_table.back()).num_tokens++;
    logical_token_count++;
}

void Sequence::flush_cache(PrefixCacheManager& cache_mgr) {
    if ((int)token_buffer.size() == BLOCK_SIZE) {
        current_hash = hash_block_state(current_hash, token_buffer.data(), BLOCK_SIZE);
        int parent = block_table.size() > 1 ? block_table[block_table.size() - 2] : -1;
        cache_mgr.insert_cache(current_hash, block_table.back(), parent);
    }
}

void Sequence::release(KVBlock_Manager& manager, PrefixCacheManager& cache_mgr) {
    for (int id : block_table) manager.free_block(id, cache_mgr);
    block_table.clear();
    token_buffer.clear();
    logical_token_count = 0;
    current_hash = FNV_OFFSET_BASIS;
}

int Sequence::prefix_walk(const int32_t* prompt, int n, int start, bool require_empty_buffer,
                          KVBlock_Manager& manager, PrefixCacheManager& cache_mgr) {
    int p = start;
    while (p + BLOCK_SIZE <= n && (!require_empty_buffer || token_buffer.empty())) {
        uint64_t h = hash_block_state(current_hash, prompt + p, BLOCK_SIZE);
        int hit = cache_mgr.check_cache(h);
        if (hit == -1) break;
        manager.inc_ref_count(hit, cache_mgr);
        block_table.push_back(hit);
        logical_token_count += BLOCK_SIZE;
        current_hash = h;
        p += BLOCK_SIZE;
    }
    return p;
}

}  // namespace nitro
