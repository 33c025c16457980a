// Replays a block-manager op script through the shipped C++ page bookkeeping
// (nitrorag_amd/csrc/paged_memory.cpp) and prints per-op results and the final
// state.  Built by tests/test_host_sanitizers.py with AddressSanitizer and
// UndefinedBehaviorSanitizer; host code only.
//
// stdin: "total_blocks max_seqs n_ops", then one line per op:
//        "op a b hash n tok_1 .. tok_n"
// stdout: one line per op "status result", then "STATE" and the state as
//        whitespace-separated int32 words in the order the golden traces use
//        (free list, per-page counters, LRU front->back, cache map by hash,
//        reverse map by id, per sequence slot).
#include <cstdint>
#include <cstdio>
#include <iostream>
#include <memory>
#include <vector>

#include "paged_memory.hpp"

using nitro::Error;

int main() {
    int total = 0, max_seqs = 0, n_ops = 0;
    if (!(std::cin >> total >> max_seqs >> n_ops)) return 2;
    nitro::BlockManager bm(total);
    std::vector<std::unique_ptr<nitro::Sequence>> seqs(max_seqs);
    for (int i = 0; i < n_ops; i++) {
        int op, a, b, n;
        uint64_t h;
        std::cin >> op >> a >> b >> h >> n;
        std::vector<int32_t> toks(n);
        for (auto& t : toks) std::cin >> t;
        int status = 0;
        long long result = 0;
        try {
            switch (op) {
                case 1: result = bm.mem.allocate_block(bm.cache); break;
                case 2: bm.mem.inc_ref_count(a, bm.cache); break;
                case 3: bm.mem.free_block(a, bm.cache); break;
                case 4: bm.mem.force_free_block(a); break;
                case 5: result = bm.cache.check_cache(h); break;
                case 6: bm.cache.insert_cache(h, a, b); break;
                case 7: bm.cache.evict_lru_block(); break;
                case 8: seqs[a] = std::make_unique<nitro::Sequence>(a); break;
                case 9: seqs[a]->allocate_next_token(b, bm.mem, bm.cache); break;
                case 10: seqs[a]->flush_cache(bm.cache); break;
                case 11: seqs[a]->release(bm.mem, bm.cache); break;
                case 12: {
                    int p = b ? seqs[a]->prefix_walk(toks.data(), n, 0, false, bm.mem, bm.cache) : 0;
                    for (; p < n; p++) seqs[a]->allocate_next_token(toks[p], bm.mem, bm.cache);
                    result = seqs[a]->logical_token_count;
                    break;
                }
                case 13: result = bm.mem.get_free_count(); break;
                case 14: result = bm.cache.is_cached(a) ? 1 : 0; break;
                default: status = 2;
            }
        } catch (const Error& e) {
            if (e.status != nitro::ERR_OUT_OF_PAGES) throw;
            status = 1;
            result = 0;
        }
        std::printf("%d %lld\n", status, result);
    }
    std::vector<long long> w;
    const auto& fl = bm.mem.free_ids();
    w.push_back((long long)fl.size());
    w.insert(w.end(), fl.begin(), fl.end());
    for (int i = 0; i < total; i++) {
        const auto& b = bm.mem.get_block(i);
        w.insert(w.end(), {b.ref_count, b.num_tokens, b.parent_id, b.child_count});
    }
    auto lru = bm.cache.evictable_leaves_front_to_back();
    w.push_back((long long)lru.size());
    w.insert(w.end(), lru.begin(), lru.end());
    auto cm = bm.cache.cache_entries();
    w.push_back((long long)cm.size());
    for (auto& e : cm) w.insert(w.end(), {(long long)(e.first & 0xffffffffu), (long long)(e.first >> 32), e.second});
    auto rm = bm.cache.reverse_entries();
    w.push_back((long long)rm.size());
    for (auto& e : rm) w.insert(w.end(), {e.first, (long long)(e.second & 0xffffffffu), (long long)(e.second >> 32)});
    for (auto& s : seqs) {
        if (!s) {
            w.push_back(0);
            continue;
        }
        w.push_back(1);
        w.push_back(s->logical_token_count);
        w.push_back((long long)(s->current_hash & 0xffffffffu));
        w.push_back((long long)(s->current_hash >> 32));
        w.push_back((long long)s->token_buffer.size());
        w.insert(w.end(), s->token_buffer.begin(), s->token_buffer.end());
        w.push_back((long long)s->block_table.size());
        w.insert(w.end(), s->block_table.begin(), s->block_table.end());
    }
    std::printf("STATE");
    for (long long x : w) std::printf(" %lld", x);
    std::printf("\n");
    return 0;
}
