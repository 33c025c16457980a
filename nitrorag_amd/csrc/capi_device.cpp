// C ABI of the device KV pool, batch uploads and kernel launches
// (declared in include/nitro_paged_attn.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "capi_common.hpp"
#include "device_pool.hpp"
#include "nitro_paged_attn.h"

using namespace nitro;

namespace {

// Decode launch shape: waves resident per CU at the kernel's occupancy
// (4 waves/SIMD x 4 SIMDs), and the range of waves per workgroup.
constexpr int kDecodeWavesPerCU = 16;
constexpr int kDecodeMinWaves = 4;
constexpr int kDecodeMaxWaves = 16;

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

void require_pool(const nitro_kvpool* pool) {
    require(pool != nullptr, ERR_INVALID_ARGUMENT, "null pool");
}

void check_table_rows(const nitro_kvpool* pool, const int32_t* tables, int b, int max_pages,
                      int last_pos) {
    require(last_pos >= 0, ERR_BAD_BLOCK_TABLE, "negative position");
    const int last_page = last_pos >> 4;
    if (last_page >= max_pages)
        throw Error(ERR_BAD_BLOCK_TABLE, "sequence " + std::to_string(b) + ": position " +
                                             std::to_string(last_pos) + " needs page " +
                                             std::to_string(last_page) + " but max_pages is " +
                                             std::to_string(max_pages));
    const int32_t* row = tables + (size_t)b * max_pages;
    for (int i = 0; i <= last_page; i++)
        if (row[i] < 0 || row[i] >= pool->num_pages)
            throw Error(ERR_BAD_BLOCK_TABLE, "sequence " + std::to_string(b) + ": page id " +
                                                 std::to_string(row[i]) + " at logical page " +
                                                 std::to_string(i) + " is outside [0, " +
                                                 std::to_string(pool->num_pages) + ")");
}

// Scans the pages the batch reads.  Returns true when a page id occurs in the
// used part of more than one table row (a prefix shared through the prefix
// cache), or twice in one row: decode then keeps plain loads so that the
// page's lines stay cached for the other readers.  Also records whether every
// row's page at pos_b is read by that row alone (then the fused append may
// write it while the other rows read the pool).
bool any_page_shared(const nitro_kvpool* pool, DecodeBatch& d, const int32_t* tables,
                     const int32_t* positions, int batch, int max_pages) {
    if (d.page_mark.size() != (size_t)pool->num_pages || d.stamp == UINT32_MAX) {
        d.page_mark.assign(pool->num_pages, 0);
        d.page_multi.assign(pool->num_pages, 0);
        d.stamp = 0;
    }
    const uint32_t stamp = ++d.stamp;
    bool shared = false;
    for (int b = 0; b < batch; b++) {
        const int32_t* row = tables + (size_t)b * max_pages;
        for (int i = 0; i <= (positions[b] >> 4); i++) {
            uint32_t& m = d.page_mark[row[i]];  // ids were checked against the pool
            if (m == stamp) {
                shared = true;
                d.page_multi[row[i]] = stamp;
            }
            m = stamp;
        }
    }
    d.new_rows_private = true;
    for (int b = 0; b < batch && shared; b++)
        d.new_rows_private &= d.page_multi[tables[(size_t)b * max_pages + (positions[b] >> 4)]] != stamp;
    return shared;
}

// Shared prefixes: at least kPrefixMinPages pages, in whole multiples of
// kPrefixPageQuantum pages (64 rows: a whole number of decode tiles at every
// head size, so a sequence's own rows start on a tile).
constexpr int kPrefixMinPages = 4;
constexpr int kPrefixPageQuantum = 4;

// Groups of two or more sequences whose first pages are the same physical
// pages (prefix-cache hits): sequences with equal first page ids, and the
// longest run of pages all of them share, kept below every member's newest
// row (pos_b >= 16 * pages, so each member keeps at least that row as its own).
std::vector<DecodeBatch::PrefixGroup> find_prefix_groups(const int32_t* tables, const int32_t* positions,
                                                         int batch, int max_pages) {
    std::vector<DecodeBatch::PrefixGroup> groups;
    std::vector<std::pair<int32_t, int32_t>> first;  // (first page id, b)
    for (int b = 0; b < batch; b++)
        if (positions[b] >= BLOCK_SIZE * kPrefixMinPages) first.push_back({tables[(size_t)b * max_pages], b});
    std::sort(first.begin(), first.end());
    for (size_t i = 0; i < first.size();) {
        size_t j = i;
        while (j < first.size() && first[j].first == first[i].first) j++;
        if (j - i >= 2) {
            DecodeBatch::PrefixGroup g;
            int cap = max_pages;
            for (size_t k = i; k < j; k++) {
                g.members.push_back(first[k].second);
                cap = std::min(cap, positions[first[k].second] / BLOCK_SIZE);
            }
            const int32_t* row0 = tables + (size_t)g.members[0] * max_pages;
            int pages = 0;
            for (; pages < cap; pages++) {
                bool same = true;
                for (int m : g.members) same &= tables[(size_t)m * max_pages + pages] == row0[pages];
                if (!same) break;
            }
            g.pages = pages - pages % kPrefixPageQuantum;
            if (g.pages >= kPrefixMinPages) groups.push_back(std::move(g));
        }
        i = j;
    }
    return groups;
}

// Page sharing of a decode batch from the host's copy of its tables: whether
// any page is read by two rows, the prefix groups, and whether every row's
// own rows (past its group's shared pages) are read by that row alone.
void find_decode_groups(const nitro_kvpool* pool, DecodeBatch& d, const int32_t* tables, const int32_t* positions,
                        int batch, int max_pages) {
    d.shared_pages = any_page_shared(pool, d, tables, positions, batch, max_pages);
    d.groups = d.shared_pages ? find_prefix_groups(tables, positions, batch, max_pages)
                              : std::vector<DecodeBatch::PrefixGroup>{};
    d.own_rows_private = true;
    if (!d.groups.empty()) {
        std::vector<int> shared(batch, 0);
        for (const auto& g : d.groups)
            for (int b : g.members) shared[b] = g.pages;
        for (int b = 0; b < batch && d.own_rows_private; b++)
            for (int i = shared[b]; i <= (positions[b] >> 4); i++)
                if (d.page_multi[tables[(size_t)b * max_pages + i]] == d.stamp) {
                    d.own_rows_private = false;
                    break;
                }
    }
}

void check_shape(const nitro_kvpool* pool, int layer, int n_heads, int n_kv_heads, int head_dim) {
    require(layer >= 0 && layer < pool->num_layers, ERR_INVALID_ARGUMENT, "layer out of range");
    require(n_heads > 0 && n_kv_heads > 0, ERR_INVALID_ARGUMENT, "head counts must be positive");
    require(n_heads % n_kv_heads == 0, ERR_UNSUPPORTED, "n_heads must be a multiple of n_kv_heads");
    require(attention_head_dim(head_dim), ERR_UNSUPPORTED, "head_dim must be a multiple of 4 from 4 to 256");
    require(n_kv_heads * head_dim == pool->kv_dim, ERR_INVALID_ARGUMENT,
            "n_kv_heads * head_dim must equal the pool's kv_dim");
}

int env_int(const char* name, int fallback) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : fallback;
}

// Launch shape of one decode launch, chosen from the batch's context lengths.
struct DecodeShape {
    int qh = 1, waves = 4, tps = 1;  // query heads / waves per workgroup, tiles per split
};

// Waves resident per CU at the kernel's occupancy (16; 8 with several query
// heads per workgroup, which take twice the registers) and the waves per
// workgroup, 4..16.  Splits are sized so that every workgroup of the launch is
// resident in one dispatch round with as few tile rounds per wave as possible:
//  - a batch that fills the GPU at 4 waves per workgroup is not split (the
//    most waves per workgroup when the launch takes several dispatch rounds
//    anyway: each workgroup's waves stream one sequence's K/V together, which
//    measured 0.3-1% faster at B=64 ctx 4096 than 4 waves);
//  - otherwise, for W = 4, 8, 16 waves, the smallest split of W*R tiles whose
//    workgroups all fit; the W with the fewest rounds R wins, then the one
//    with the fewest splits.  Long sequences split into equal runs, short ones
//    not at all, and every split is at most R tile rounds per wave.  16 waves
//    are taken only when no sequence splits.
// ctx(b) gives sequence b's context length; nothing is allocated.
template <class Ctx>
DecodeShape plan_decode_shape(const nitro_kvpool* pool, int B, Ctx ctx, int n_heads, int n_kv_heads,
                              int head_dim) {
    DecodeShape sh;
    const int tile = decode_tile_rows(head_dim);
    auto tiles = [&](int b) { return (ctx(b) + tile - 1) / tile; };
    int max_n = 1;
    for (int b = 0; b < B; b++) max_n = std::max(max_n, tiles(b));
    const int kv_mul = n_heads / n_kv_heads;
    int qh = env_int("NITRO_DECODE_HEADS_PER_WG", 0);
    if (qh <= 0) {
        qh = 1;
        while (qh * 2 <= decode_max_heads_per_wg(head_dim) && kv_mul % (qh * 2) == 0) qh *= 2;
    }
    require(qh <= decode_max_heads_per_wg(head_dim) && kv_mul % qh == 0, ERR_INVALID_ARGUMENT,
            "NITRO_DECODE_HEADS_PER_WG must divide n_heads/n_kv_heads and fit the head_dim");
    sh.qh = qh;
    const long long cols = n_heads / qh;  // workgroups per item
    const int max_waves = qh == 1 ? kDecodeMaxWaves : kDecodeMaxWaves / 2;
    const long long target = (long long)(qh == 1 ? kDecodeWavesPerCU : kDecodeWavesPerCU / 2) *
                             std::max(pool->num_cus, 1);
    const int max_tps = (DECODE_MAX_SPLIT_PAGES - 2) * BLOCK_SIZE / tile;  // the LDS table slice
    auto items_for = [&](int tps) {
        long long k = 0;
        for (int b = 0; b < B; b++) k += (tiles(b) + tps - 1) / tps;
        return k;
    };
    const int env_waves = env_int("NITRO_DECODE_WAVES", 0);
    const int env_tps = env_int("NITRO_DECODE_SPLIT_TILES", 0);
    int waves = 0, tps = 0;
    if (env_waves <= 0 && env_tps <= 0) {
        if ((long long)B * cols * kDecodeMinWaves >= target) {
            waves = kDecodeMinWaves;
            if ((long long)B * cols * kDecodeMinWaves > target) {
                waves = max_waves;
                while (waves > kDecodeMinWaves && waves > max_n) waves /= 2;
            }
            tps = max_n;
        } else {
            long long best_rounds = LLONG_MAX, best_items = LLONG_MAX;
            for (int w = kDecodeMinWaves; w <= max_waves; w *= 2) {
                for (int rounds = 1;; rounds++) {
                    const int c = std::min(w * rounds, max_tps);
                    const long long k = items_for(c);
                    if (k * cols * w <= target || c >= max_n || c == max_tps) {
                        if (k * cols * w > target) break;  // this wave count never fits
                        // 16-wave workgroups only where nothing splits: four
                        // waves a SIMD merging partials measured 3-4% slower
                        // than 8-wave splits at one 32x128 sequence
                        if (w > 8 && k > B) break;
                        const long long r = (std::min(c, max_n) + w - 1) / w;
                        if (r < best_rounds || (r == best_rounds && k < best_items)) {
                            best_rounds = r;
                            best_items = k;
                            waves = w;
                            tps = c;
                        }
                        break;
                    }
                }
            }
            if (waves == 0) {  // unreachable: 4 waves fit in this branch
                waves = kDecodeMinWaves;
                tps = max_n;
            }
        }
    } else {
        waves = env_waves > 0 ? env_waves : kDecodeMinWaves;
        tps = env_tps > 0 ? env_tps : max_n;
    }
    sh.waves = std::max(kDecodeMinWaves, std::min(waves, max_waves));
    sh.tps = std::max(1, std::min(tps, max_tps));
    return sh;
}

// Launch fields shared by every decode entry point.
DecodeLaunch decode_launch_base(const nitro_kvpool* pool, int layer, const float* q, float* out, int n_heads,
                                int n_kv_heads, int head_dim, const DecodeShape& sh, bool shared_pages) {
    DecodeLaunch a{};
    a.q = q;
    a.out = out;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    a.bad_pages = pool->bad_pages.ptr;
    a.page_stride = pool->page_stride();
    a.layer_off = pool->layer_offset(layer);
    a.kv_dim = pool->kv_dim;
    a.n_heads = n_heads;
    a.kv_mul = n_heads / n_kv_heads;
    a.head_dim = head_dim;
    a.num_pages = pool->num_pages;
    a.tiles_per_split = sh.tps;
    a.pstride = (head_dim + 2 + 31) / 32 * 32;
    a.waves = sh.waves;
    a.heads_per_wg = sh.qh;
    // Non-temporal K/V loads when every K/V line is read once per launch:
    // one workgroup per KV head and no page shared between sequences.
    const int stream_env = env_int("NITRO_DECODE_STREAM", -1);
    a.stream_kv = stream_env >= 0 ? stream_env != 0 : (sh.qh == a.kv_mul && !shared_pages);
    const int remap_env = env_int("NITRO_DECODE_XCD_REMAP", -1);
    a.xcd_remap = remap_env >= 0 ? remap_env != 0 : sh.qh < a.kv_mul;
    a.qscale = (float)(1.4426950408889634 / std::sqrt((double)head_dim));
    return a;
}

// Shared prefixes (prefix-cache hits): the rows that every member of a group
// shares are streamed once per set of W members (W = waves per workgroup),
// not once per member.  The launch's work list puts member items first: a
// workgroup whose W waves each take one member of the set over the same
// chunk of shared rows (so they read each row at about the same time,
// through one L1), each wave writing its member's partial of the chunk.  The
// sequences' own rows follow as usual splits, and every (sequence, head)
// merges its partials, the member items' first, whoever arrives last.  The
// list rides in the kernel arguments; a batch whose list does not fit, or
// that groups query heads per workgroup (GQA), is launched as usual.

// Builds that list into d.arg_list for the uploaded batch; false when it does
// not fit the kernel arguments or the item fields.
bool plan_prefix(nitro_kvpool* pool, int n_heads, int n_kv_heads, int head_dim) {
    DecodeBatch& d = pool->decode;
    const int B = d.batch;
    const int tile = decode_tile_rows(head_dim);
    std::vector<int> shared_rows(B, 0), group(B, -1);
    for (size_t g = 0; g < d.groups.size(); g++)
        for (int b : d.groups[g].members) {
            shared_rows[b] = d.groups[g].pages * BLOCK_SIZE;
            group[b] = (int)g;
        }
    auto ctx = [&](int b) { return d.positions[b] + 1; };
    auto own = [&](int b) { return ctx(b) - shared_rows[b]; };
    const DecodeShape sh = plan_decode_shape(pool, B, own, n_heads, n_kv_heads, head_dim);
    if (sh.qh != 1) return false;
    const int max_tps = (DECODE_MAX_SPLIT_PAGES - 2) * BLOCK_SIZE / tile;
    const int W = sh.waves;
    auto sets = [&](const DecodeBatch::PrefixGroup& g) { return ((int)g.members.size() + W - 1) / W; };
    auto own_tiles = [&](int b) { return (ctx(b) + tile - 1) / tile - shared_rows[b] / tile; };
    auto splits = [&](int b) { return (own_tiles(b) + sh.tps - 1) / sh.tps; };
    long long main_items = 0;
    for (int b = 0; b < B; b++) main_items += splits(b);

    // Chunks of ch tiles of shared rows per member item, which its workgroup
    // stages one tile after another.  Shorter chunks mean more items and
    // more partials to merge, longer ones a longer workgroup: the shared rows
    // of the longest group in two chunks, at least a split's tiles per wave
    // and at most 256 rows, more when the list would not fit.  A chunk starts
    // on a page.  Measured on 48 sequences sharing 512 rows, 12 x 64: 23.2-23.4
    // us at 8 tiles (256 rows), 23.5 at 10, 24.1 at 12, 24.9 at 7, 25.9 at 16,
    // 26.9 at 4; 29.2 us reading every sequence's rows.  Over 1024 shared rows
    // at 12 x 64 and 2048 at 32 x 128 the best chunk was also 256 rows.
    int longest = 0;
    for (const auto& g : d.groups) longest = std::max(longest, g.pages * BLOCK_SIZE / tile);
    int ch = std::min(256 / tile, std::max((sh.tps + W - 1) / W, (longest + 1) / 2));
    if (env_int("NITRO_DECODE_PREFIX_CHUNK", 0) > 0) ch = env_int("NITRO_DECODE_PREFIX_CHUNK", 0);
    while ((ch * tile) % BLOCK_SIZE) ch++;
    if (ch > max_tps) return false;  // a chunk's pages must fit the table slice
    long long member_items = 0, entries = 0;
    for (;; ch *= 2) {
        member_items = entries = 0;
        for (const auto& g : d.groups) {
            member_items += (long long)sets(g) * ((g.pages * BLOCK_SIZE / tile + ch - 1) / ch);
            for (int k = 0; k < sets(g); k++) entries += (std::min(W, (int)g.members.size() - k * W) + 1) / 2;
        }
        if (member_items + main_items + entries <= DECODE_ARG_ITEMS) break;
        if (ch * 2 > max_tps) return false;
    }
    auto chunks_of = [&](int g) { return (d.groups[g].pages * BLOCK_SIZE / tile + ch - 1) / ch; };

    // Partial slots: per sequence its member parts, then its splits.
    std::vector<int> first_slot(B), parts(B);
    int slot0 = 0;
    for (int b = 0; b < B; b++) {
        parts[b] = (group[b] >= 0 ? chunks_of(group[b]) : 0) + splits(b);
        if (splits(b) > 255 || shared_rows[b] / tile >= (1 << 23) || parts[b] >= (1 << 15) || slot0 >= (1 << 16))
            return false;
        first_slot[b] = slot0;
        slot0 += parts[b];
    }

    // Member items {-1 - first entry, members | part << 8, first tile,
    // tiles}; entries {b, first slot | parts << 16, b', ...} after the items.
    int n = 0, at = (int)(member_items + main_items);
    for (size_t g = 0; g < d.groups.size(); g++) {
        const auto& members = d.groups[g].members;
        const int tiles = d.groups[g].pages * BLOCK_SIZE / tile;
        for (int k = 0; k < sets(d.groups[g]); k++) {
            const int count = std::min(W, (int)members.size() - k * W);
            const int base = at;
            for (int j = 0; j < count; j += 2) {
                const int b0 = members[k * W + j], b1 = members[k * W + std::min(j + 1, count - 1)];
                d.arg_list.item[at++] = make_int4(b0, first_slot[b0] | (parts[b0] << 16), b1,
                                                  first_slot[b1] | (parts[b1] << 16));
            }
            for (int c = 0; c < chunks_of((int)g); c++)
                d.arg_list.item[n++] =
                    make_int4(-1 - base, count | (c << 8), c * ch, std::min(ch, tiles - c * ch));
        }
    }
    // The splits of each sequence's own rows, longest first.  With the member
    // items the launch can hold more workgroups than the GPU runs at once;
    // the ones dispatched last start when the first finish, and short ones
    // there end the launch sooner (48 sequences sharing 512 rows, 12 x 64:
    // 22.8-23.4 us against 24.2-24.4 shortest first).
    std::vector<std::pair<int, int4>> order;  // (tiles, item)
    for (int b = 0; b < B; b++) {
        const int first_tile = shared_rows[b] / tile;
        for (int x = 0; x < splits(b); x++)
            order.push_back({std::min(sh.tps, own_tiles(b) - x * sh.tps),
                             make_int4(b, x | (first_tile << 8), first_slot[b] | (parts[b] << 16), ctx(b))});
    }
    std::stable_sort(order.begin(), order.end(), [](const auto& x, const auto& y) { return x.first > y.first; });
    for (const auto& o : order) d.arg_list.item[n++] = o.second;
    d.main_items = n;
    d.main_tps = sh.tps;
    d.main_waves = W;
    d.prefix_slots = slot0;
    d.work_generation = ~0ull;  // arg_list now holds this list, not the usual one
    return true;
}

// Whether the shared-prefix form is worth taking for the uploaded batch.  It
// cuts the rows the launch moves from L2 and HBM, but its member workgroups
// stage their chunk tile by tile, a longer chain than the usual splits: it
// pays where the usual launch is bound by the bytes it moves, not by that
// chain.  Measured (per launch, the form against the usual one): 32 sequences
// sharing 256 rows at 12 x 64 (51 MB of K/V rows in all) 8.0-8.9 vs 7.0 us in
// the continuous-batching run; 48 sharing 512 rows (236 MB) 22.6 vs 24.2 us
// warm, 26.7 vs 32.8 flushed; at 32 x 128, 16 sharing 2048 rows (1.1 GB)
// 38.3 vs 49.7 us, 64 sharing 1024 (2.5 GB) 157 vs 172 us, 32 sharing 256
// (272 MB) equal; 8 sharing 4096 (1.1 GB) 61 vs 52 us, the one loss above the
// threshold.
constexpr double kPrefixFormMinBytes = 128e6;
bool prefix_form_pays(const nitro_kvpool* pool) {
    const DecodeBatch& d = pool->decode;
    double rows = 0;
    for (int b = 0; b < d.batch; b++) rows += d.positions[b] + 1;
    return rows * pool->kv_dim * 2 * sizeof(float) >= kPrefixFormMinBytes;
}

// The shared-prefix form of a decode launch, when the batch has prefix
// groups and its list fits; false otherwise (nothing launched).
bool launch_decode_prefix(nitro_kvpool* pool, int layer, const float* q, float* out, const float* k_new,
                          const float* v_new, int n_heads, int n_kv_heads, int head_dim, hipStream_t s) {
    DecodeBatch& d = pool->decode;
    const int32_t key = (n_heads << 16) ^ (n_kv_heads << 9) ^ head_dim;
    if (d.prefix_generation != d.generation || d.prefix_heads != key ||
        (d.prefix_ok && d.work_generation == d.generation)) {  // arg_list since taken by the usual list
        d.prefix_generation = d.generation;
        d.prefix_heads = key;
        d.prefix_ok = plan_prefix(pool, n_heads, n_kv_heads, head_dim) ? 1 : 0;
    }
    if (!d.prefix_ok) return false;
    DecodeShape sh;
    sh.qh = 1;
    sh.waves = d.main_waves;
    sh.tps = d.main_tps;
    DecodeLaunch a = decode_launch_base(pool, layer, q, out, n_heads, n_kv_heads, head_dim, sh, true);
    pool->partials.reserve((size_t)d.prefix_slots * n_heads * a.pstride);
    if (pool->counters.reserve((size_t)d.batch * n_heads))
        hip_check(hipMemset(pool->counters.ptr, 0, pool->counters.count * sizeof(int32_t)), "hipMemset");
    a.tables = d.tables.ptr;
    a.positions = d.pos.ptr;
    a.partials = pool->partials.ptr;
    a.counters = pool->counters.ptr;
    a.batch = d.batch;
    a.max_pages = d.max_pages;
    a.num_splits = 0;
    a.arg_items = 1;
    a.members = 1;
    a.work_items = d.main_items;
    a.ctx_limit = d.max_pages * BLOCK_SIZE;
    a.k_new = k_new;
    a.v_new = v_new;
    // each row past the shared ones is read once when no such page is read
    // twice: non-temporal loads, as without sharing (the shared rows are
    // re-read by the member sets, through plain loads of the same kernel
    // only in that case: NITRO_DECODE_STREAM overrides)
    a.stream_kv = env_int("NITRO_DECODE_STREAM", -1) >= 0 ? env_int("NITRO_DECODE_STREAM", -1) != 0
                                                         : d.own_rows_private && a.kv_mul == 1;
    hip_check(launch_paged_attn_decode(a, s, &d.arg_list), "paged_attn_decode launch");
    pool->last_stream = s;
    return true;
}

// One decode launch over the pool's uploaded batch (k_new / v_new: the fused
// append, used by the caller only where it is safe).
void launch_decode(nitro_kvpool* pool, int layer, const float* q, float* out, const float* k_new,
                   const float* v_new, int n_heads, int n_kv_heads, int head_dim, hipStream_t s) {
    DecodeBatch& d = pool->decode;
    d.launches++;
    const int prefix_mode = env_int("NITRO_DECODE_PREFIX", 1);  // 0 off, 1 where it pays, 2 always
    if (!d.groups.empty() && prefix_mode != 0 && (prefix_mode == 2 || prefix_form_pays(pool)) &&
        launch_decode_prefix(pool, layer, q, out, k_new, v_new, n_heads, n_kv_heads, head_dim, s)) {
        d.prefix_launches++;
        return;
    }
    const int B = d.batch;
    auto ctx = [&](int b) { return d.positions[b] + 1; };
    const DecodeShape sh = plan_decode_shape(pool, B, ctx, n_heads, n_kv_heads, head_dim);
    const int tile = decode_tile_rows(head_dim);
    auto splits = [&](int b) { return ((ctx(b) + tile - 1) / tile + sh.tps - 1) / sh.tps; };
    int max_splits = 1;
    long long slots = 0;
    bool uniform = true;
    for (int b = 0; b < B; b++) {
        max_splits = std::max(max_splits, splits(b));
        slots += splits(b);
        uniform &= splits(b) == splits(0);
    }
    // A work list when sequences split unevenly and the list fits the kernel
    // arguments (NITRO_DECODE_WORK_LIST=0/1 forces it off/on where it fits);
    // otherwise items are implied by the block id.
    const int list_env = env_int("NITRO_DECODE_WORK_LIST", -1);
    bool use_list = (list_env >= 0 ? list_env != 0 : (max_splits > 1 && !uniform)) &&
                    slots <= DECODE_ARG_ITEMS;
    if (use_list &&
        (d.work_generation != d.generation || d.work_tile != tile || d.work_tps != sh.tps)) {
        // items {b, split, first partial slot of b, ctx}, shortest first (equal
        // sizes in batch order).  The planner sizes splits so that the whole
        // launch is resident at once; the order then only sets which loads
        // reach the memory queue first, and the short items' loads going
        // first measured 0.6% (mixed lengths) to 2% (shared prefixes) faster
        // than longest first.
        std::vector<std::pair<int, int4>> order;  // (tiles, item)
        order.reserve((size_t)slots);
        int slot0 = 0;
        for (int b = 0; b < B; b++) {
            const int nt = (ctx(b) + tile - 1) / tile;
            for (int x = 0; x < splits(b); x++)
                order.push_back({std::min(sh.tps, nt - x * sh.tps), make_int4(b, x, slot0 | (splits(b) << 16), ctx(b))});
            slot0 += splits(b);
        }
        std::stable_sort(order.begin(), order.end(),
                         [](const auto& x, const auto& y) { return x.first < y.first; });
        for (size_t i = 0; i < order.size(); i++) d.arg_list.item[i] = order[i].second;
        d.work_generation = d.generation;
        d.work_tile = tile;
        d.work_tps = sh.tps;
        d.work_items = (int32_t)order.size();
    }
    if (!use_list) slots = (long long)B * max_splits;
    DecodeLaunch a = decode_launch_base(pool, layer, q, out, n_heads, n_kv_heads, head_dim, sh, d.shared_pages);
    if (max_splits > 1) {
        pool->partials.reserve((size_t)slots * n_heads * a.pstride);
        if (pool->counters.reserve((size_t)B * (n_heads / sh.qh)))
            hip_check(hipMemset(pool->counters.ptr, 0, pool->counters.count * sizeof(int32_t)), "hipMemset");
    }
    a.tables = d.tables.ptr;
    a.positions = d.pos.ptr;
    a.work_items = use_list ? d.work_items : 0;
    a.arg_items = use_list ? 1 : 0;
    a.partials = pool->partials.ptr;
    a.counters = pool->counters.ptr;
    a.k_new = k_new;
    a.v_new = v_new;
    a.batch = B;
    a.max_pages = d.max_pages;
    a.num_splits = use_list ? 0 : max_splits;
    a.ctx_limit = use_list ? d.max_pages * BLOCK_SIZE
                           : std::min(d.max_pages * BLOCK_SIZE, max_splits * sh.tps * tile);
    hip_check(launch_paged_attn_decode(a, s, use_list ? &d.arg_list : nullptr), "paged_attn_decode launch");
    pool->last_stream = s;
}

}  // namespace

namespace nitro {

void set_device_decode_batch(nitro_kvpool* pool, int batch, int max_pages, const int32_t* positions,
                             bool shared_pages, int32_t** tables, int32_t** device_positions,
                             int32_t** device_slots) {
    require_pool(pool);
    require(batch > 0 && max_pages > 0, ERR_INVALID_ARGUMENT, "batch and max_pages must be positive");
    DecodeBatch& d = pool->decode;
    d.batch = 0;
    d.tables.reserve((size_t)batch * max_pages);
    d.pos.reserve(batch);
    d.slots.reserve(batch);
    *device_slots = d.slots.ptr;
    d.positions.assign(positions, positions + batch);
    d.shared_pages = shared_pages;
    d.groups.clear();  // no host tables to find them in
    d.new_rows_private = false;
    d.generation++;
    d.batch = batch;
    d.max_pages = max_pages;
    *tables = d.tables.ptr;
    *device_positions = d.pos.ptr;
}

void set_device_decode_groups(nitro_kvpool* pool, const int32_t* tables, int max_pages) {
    require_pool(pool);
    DecodeBatch& d = pool->decode;
    require(d.batch > 0 && max_pages == d.max_pages, ERR_INVALID_ARGUMENT,
            "the host tables must be the rows of the batch just set");
    for (int b = 0; b < d.batch; b++) check_table_rows(pool, tables, b, max_pages, d.positions[b]);
    find_decode_groups(pool, d, tables, d.positions.data(), d.batch, max_pages);
}

}  // namespace nitro

extern "C" {

// seq_len > 0: a borrowed contiguous cache [num_layers][seq_len][kv_dim]
// viewed as seq_len / 16 pages per layer (page p = rows 16p..16p+15).
static int make_pool(float* k, float* v, bool owned, int32_t num_pages, int32_t num_layers,
                     int32_t kv_dim, nitro_kvpool** out, int32_t seq_len = 0) {
    return guarded([&] {
        require(out != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        *out = nullptr;
        require(num_pages > 0 && num_layers > 0 && kv_dim > 0, ERR_INVALID_ARGUMENT,
                "pool dimensions must be positive");
        require(kv_dim % 4 == 0, ERR_UNSUPPORTED, "kv_dim must be a multiple of 4");
        nitro_kvpool* pool = new nitro_kvpool();
        try {
            hip_check(hipGetDevice(&pool->device), "hipGetDevice");
            hip_check(hipDeviceGetAttribute(&pool->num_cus, hipDeviceAttributeMultiprocessorCount,
                                            pool->device),
                      "hipDeviceGetAttribute");
            pool->num_pages = num_pages;
            pool->num_layers = num_layers;
            pool->kv_dim = kv_dim;
            pool->owned = owned;
            pool->page_elems = (int64_t)(seq_len > 0 ? 1 : num_layers) * BLOCK_SIZE * kv_dim;
            pool->layer_elems = (int64_t)(seq_len > 0 ? seq_len : BLOCK_SIZE) * kv_dim;
            const size_t bytes = (size_t)num_pages * num_layers * BLOCK_SIZE * kv_dim * sizeof(float);
            if (owned) {
                hip_check(hipMalloc((void**)&pool->k, bytes), "hipMalloc(K pool)");
                hip_check(hipMalloc((void**)&pool->v, bytes), "hipMalloc(V pool)");
                hip_check(hipMemset(pool->k, 0, bytes), "hipMemset");
                hip_check(hipMemset(pool->v, 0, bytes), "hipMemset");
            } else {
                require(k != nullptr && v != nullptr, ERR_INVALID_ARGUMENT, "null pool buffer");
                require(((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0, ERR_INVALID_ARGUMENT,
                        "pool buffers must be 16-byte aligned");
                pool->k = k;
                pool->v = v;
            }
            pool->bad_pages.reserve(1);
            hip_check(hipMemset(pool->bad_pages.ptr, 0, sizeof(int32_t)), "hipMemset");
            hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        } catch (...) {
            if (owned) {
                if (pool->k) (void)hipFree(pool->k);
                if (pool->v) (void)hipFree(pool->v);
            }
            delete pool;
            throw;
        }
        *out = pool;
    });
}

int nitro_kvpool_create(int32_t num_pages, int32_t num_layers, int32_t kv_dim, nitro_kvpool** out) {
    return make_pool(nullptr, nullptr, true, num_pages, num_layers, kv_dim, out);
}

int nitro_kvpool_wrap(float* k_pool, float* v_pool, int32_t num_pages, int32_t num_layers,
                      int32_t kv_dim, nitro_kvpool** out) {
    return make_pool(k_pool, v_pool, false, num_pages, num_layers, kv_dim, out);
}

int nitro_kvpool_wrap_contiguous(float* key_cache, float* value_cache, int32_t seq_len,
                                 int32_t num_layers, int32_t kv_dim, nitro_kvpool** out) {
    if (out) *out = nullptr;
    const int st = guarded([&] {
        require(seq_len > 0, ERR_INVALID_ARGUMENT, "seq_len must be positive");
        require(seq_len % BLOCK_SIZE == 0, ERR_UNSUPPORTED,
                "seq_len must be a multiple of 16 (whole pages per layer)");
    });
    if (st != NITRO_OK) return st;
    return make_pool(key_cache, value_cache, false, seq_len / BLOCK_SIZE, num_layers, kv_dim, out,
                     seq_len);
}

int nitro_kvpool_destroy(nitro_kvpool* pool) {
    if (!pool) return NITRO_OK;
    return guarded([&] {
        (void)hipDeviceSynchronize();
        if (pool->owned) {
            (void)hipFree(pool->k);
            (void)hipFree(pool->v);
        }
        delete pool;
    });
}

int nitro_kvpool_data(const nitro_kvpool* pool, float** k_pool, float** v_pool) {
    return guarded([&] {
        require_pool(pool);
        if (k_pool) *k_pool = pool->k;
        if (v_pool) *v_pool = pool->v;
    });
}

int nitro_kvpool_shape(const nitro_kvpool* pool, int32_t* num_pages, int32_t* num_layers,
                       int32_t* kv_dim) {
    return guarded([&] {
        require_pool(pool);
        if (num_pages) *num_pages = pool->num_pages;
        if (num_layers) *num_layers = pool->num_layers;
        if (kv_dim) *kv_dim = pool->kv_dim;
    });
}

int nitro_decode_batch_upload(nitro_kvpool* pool, const int32_t* tables, const int32_t* positions,
                              int32_t batch, int32_t max_pages, void* stream) {
    return guarded([&] {
        require_pool(pool);
        require(tables != nullptr && positions != nullptr, ERR_INVALID_ARGUMENT, "null array");
        require(batch > 0 && max_pages > 0, ERR_INVALID_ARGUMENT, "batch and max_pages must be positive");
        for (int b = 0; b < batch; b++) check_table_rows(pool, tables, b, max_pages, positions[b]);
        DecodeBatch& d = pool->decode;
        const size_t nt = (size_t)batch * max_pages;
        d.batch = 0;  // invalid until the copies are issued
        d.tables.reserve(nt);
        d.pos.reserve(batch);
        d.slots.reserve(batch);
        hipStream_t s = as_stream(stream);
        Staging& st = pool->decode_staging;
        int32_t* h = st.acquire(nt + 2 * (size_t)batch);
        std::memcpy(h, tables, nt * sizeof(int32_t));
        std::memcpy(h + nt, positions, batch * sizeof(int32_t));
        for (int b = 0; b < batch; b++)  // where each row's K/V goes (the fused RoPE/append reads it)
            h[nt + batch + b] = tables[(size_t)b * max_pages + positions[b] / BLOCK_SIZE] * BLOCK_SIZE +
                                positions[b] % BLOCK_SIZE;
        st.copy(d.tables.ptr, h, nt, s);
        st.copy(d.pos.ptr, h + nt, batch, s);
        st.copy(d.slots.ptr, h + nt + batch, batch, s);
        st.finish(s);
        d.positions.assign(positions, positions + batch);
        find_decode_groups(pool, d, tables, positions, batch, max_pages);
        d.generation++;
        d.batch = batch;
        d.max_pages = max_pages;
        pool->last_stream = s;
    });
}

int nitro_kv_append(nitro_kvpool* pool, int32_t layer, const float* k, const float* v, void* stream) {
    return guarded([&] {
        require_pool(pool);
        require(k != nullptr && v != nullptr, ERR_INVALID_ARGUMENT, "null k/v");
        require(layer >= 0 && layer < pool->num_layers, ERR_INVALID_ARGUMENT, "layer out of range");
        const DecodeBatch& d = pool->decode;
        require(d.batch > 0, ERR_NO_BATCH, "no decode batch uploaded");
        hipStream_t s = as_stream(stream);
        hip_check(launch_kv_append_decode(pool->k, pool->v, k, v, d.tables.ptr, d.pos.ptr, d.batch,
                                          d.max_pages, pool->kv_dim, pool->page_stride(),
                                          pool->layer_offset(layer), pool->num_pages,
                                          pool->bad_pages.ptr, s),
                  "kv_append launch");
        pool->last_stream = s;
    });
}

int nitro_paged_attn_decode(nitro_kvpool* pool, int32_t layer, const float* q, float* out,
                            int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, void* stream) {
    return guarded([&] {
        require_pool(pool);
        require(q != nullptr && out != nullptr, ERR_INVALID_ARGUMENT, "null q/out");
        check_shape(pool, layer, n_heads, n_kv_heads, head_dim);
        require(pool->decode.batch > 0, ERR_NO_BATCH, "no decode batch uploaded");
        launch_decode(pool, layer, q, out, nullptr, nullptr, n_heads, n_kv_heads, head_dim, as_stream(stream));
    });
}

int nitro_paged_attn_decode_static(nitro_kvpool* pool, int32_t layer, const float* q, float* out,
                                   const int32_t* tables, const int32_t* positions, int32_t batch,
                                   int32_t max_pages, int32_t max_context, int32_t n_heads, int32_t n_kv_heads,
                                   int32_t head_dim, int32_t pages_private, void* stream) {
    return guarded([&] {
        require_pool(pool);
        require(q != nullptr && out != nullptr && tables != nullptr && positions != nullptr,
                ERR_INVALID_ARGUMENT, "null q/out/tables/positions");
        require(pages_private == 0 || pages_private == 1, ERR_INVALID_ARGUMENT, "pages_private must be 0 or 1");
        check_shape(pool, layer, n_heads, n_kv_heads, head_dim);
        require(batch > 0 && max_pages > 0, ERR_INVALID_ARGUMENT, "batch and max_pages must be positive");
        require(max_context > 0 && max_context <= max_pages * BLOCK_SIZE, ERR_INVALID_ARGUMENT,
                "max_context must be in [1, max_pages * 16]");
        // Every sequence is planned at max_context, so the splits are uniform
        // and implied by the block id: no work list, nothing to upload.
        auto ctx = [&](int) { return (int)max_context; };
        const DecodeShape sh = plan_decode_shape(pool, batch, ctx, n_heads, n_kv_heads, head_dim);
        const int tile = decode_tile_rows(head_dim);
        const int splits = ((max_context + tile - 1) / tile + sh.tps - 1) / sh.tps;
        // page sharing is the caller's to say: plain (cacheable) K/V loads
        // unless no page is read twice
        DecodeLaunch a = decode_launch_base(pool, layer, q, out, n_heads, n_kv_heads, head_dim, sh, !pages_private);
        float* ws = nullptr;
        if (splits > 1) {
            const size_t counters = (size_t)batch * (n_heads / sh.qh);
            const size_t partial_floats = (size_t)batch * splits * n_heads * a.pstride;
            const size_t room = DECODE_STATIC_SCRATCH_BYTES / sizeof(float) - DECODE_STATIC_COUNTERS;
            if (counters > DECODE_STATIC_COUNTERS || partial_floats > room)
                throw Error(ERR_INVALID_ARGUMENT,
                            "this launch needs " + std::to_string(counters) + " counters and " +
                                std::to_string(partial_floats * sizeof(float)) +
                                " bytes of split-K partials; the static workspace holds " +
                                std::to_string(DECODE_STATIC_COUNTERS) + " and " +
                                std::to_string(room * sizeof(float)) + " (use nitro_paged_attn_decode)");
            hip_check(decode_static_scratch(&ws), "hipGetSymbolAddress(scratch)");
        }
        a.tables = tables;
        a.positions = positions;
        a.partials = ws ? ws + DECODE_STATIC_COUNTERS : nullptr;
        a.counters = reinterpret_cast<int32_t*>(ws);
        a.batch = batch;
        a.max_pages = max_pages;
        a.num_splits = splits;
        a.ctx_limit = std::min(max_context, splits * sh.tps * tile);
        hipStream_t s = as_stream(stream);
        hip_check(launch_paged_attn_decode(a, s), "paged_attn_decode launch");
        pool->last_stream = s;
    });
}

int nitro_paged_attn_decode_append(nitro_kvpool* pool, int32_t layer, const float* q, const float* k,
                                   const float* v, float* out, int32_t n_heads, int32_t n_kv_heads,
                                   int32_t head_dim, void* stream) {
    return guarded([&] {
        require_pool(pool);
        require(q != nullptr && out != nullptr && k != nullptr && v != nullptr, ERR_INVALID_ARGUMENT,
                "null q/k/v/out");
        check_shape(pool, layer, n_heads, n_kv_heads, head_dim);
        const DecodeBatch& d = pool->decode;
        require(d.batch > 0, ERR_NO_BATCH, "no decode batch uploaded");
        hipStream_t s = as_stream(stream);
        if (d.new_rows_private || !d.shared_pages) {
            launch_decode(pool, layer, q, out, k, v, n_heads, n_kv_heads, head_dim, s);
        } else {  // another row reads a page being appended to: append first
            hip_check(launch_kv_append_decode(pool->k, pool->v, k, v, d.tables.ptr, d.pos.ptr, d.batch,
                                              d.max_pages, pool->kv_dim, pool->page_stride(),
                                              pool->layer_offset(layer), pool->num_pages,
                                              pool->bad_pages.ptr, s),
                      "kv_append launch");
            launch_decode(pool, layer, q, out, nullptr, nullptr, n_heads, n_kv_heads, head_dim, s);
        }
    });
}

// Whether attention may read a prefill batch's chunk keys from the new rows
// (and the cached keys below each chunk from the pool) while the same launch
// writes the chunk rows into the pool: no page is written from two table
// entries, and no page a chunk row lands on is also a cached-key page of any
// sequence (the page of a chunk's first row may hold the chunk's own cached
// rows: those are other rows of the same entry).
static bool chunk_pages_private(const int32_t* tables, const int32_t* start_pos,
                                const int32_t* num_tokens, int batch, int max_pages) {
    std::unordered_map<int32_t, std::pair<int, int>> written;  // page -> (seq, table index)
    for (int b = 0; b < batch; b++) {
        if (num_tokens[b] == 0) continue;
        const int32_t* row = tables + (size_t)b * max_pages;
        for (int i = start_pos[b] >> 4; i <= (start_pos[b] + num_tokens[b] - 1) >> 4; i++) {
            const auto at = written.emplace(row[i], std::make_pair(b, i));
            if (!at.second) return false;
        }
    }
    // a cached key's page (below a chunk's first page) must not be one a
    // chunk row lands on
    for (int b = 0; b < batch; b++) {
        if (num_tokens[b] == 0) continue;
        const int32_t* row = tables + (size_t)b * max_pages;
        for (int i = 0; i < start_pos[b] >> 4; i++)
            if (written.count(row[i])) return false;
    }
    return true;
}

int nitro_prefill_batch_upload(nitro_kvpool* pool, const int32_t* tables, const int32_t* start_pos,
                               const int32_t* num_tokens, int32_t batch, int32_t max_pages,
                               void* stream) {
    return guarded([&] {
        require_pool(pool);
        require(tables != nullptr && start_pos != nullptr && num_tokens != nullptr,
                ERR_INVALID_ARGUMENT, "null array");
        require(batch > 0 && max_pages > 0, ERR_INVALID_ARGUMENT, "batch and max_pages must be positive");
        PrefillBatch& p = pool->prefill;
        p.batch = 0;
        std::vector<int32_t> row_off(batch);
        long long total = 0;
        int max_tokens = 0;
        for (int b = 0; b < batch; b++) {
            require(num_tokens[b] >= 0 && start_pos[b] >= 0, ERR_INVALID_ARGUMENT,
                    "negative start_pos or num_tokens");
            if (num_tokens[b] > 0) check_table_rows(pool, tables, b, max_pages, start_pos[b] + num_tokens[b] - 1);
            row_off[b] = (int32_t)total;
            total += num_tokens[b];
            max_tokens = std::max(max_tokens, num_tokens[b]);
        }
        require(total > 0 && total < (1LL << 30), ERR_INVALID_ARGUMENT, "bad total token count");
        const int bm = prefill_block_m(0);
        // Work items (seq, first query row), longest key range first: one list
        // of bm-row items and one of PREFILL_WIDE_ROWS-row items (the launch
        // takes the list its kernel serves).
        auto work_list = [&](int rows) {
            std::vector<std::pair<long long, std::pair<int, int>>> items;
            for (int b = 0; b < batch; b++)
                for (int q0 = 0; q0 < num_tokens[b]; q0 += rows) {
                    const int last = start_pos[b] + std::min(num_tokens[b], q0 + rows) - 1;
                    items.push_back({-(long long)last, {b, q0}});
                }
            std::stable_sort(items.begin(), items.end(),
                             [](const auto& x, const auto& y) { return x.first < y.first; });
            return items;
        };
        const auto items = work_list(bm);
        const auto wide = work_list(PREFILL_WIDE_ROWS);

        const size_t nt = (size_t)batch * max_pages;
        const size_t n_work = items.size() * 2, n_wide = wide.size() * 2;
        const size_t need = nt + 3 * (size_t)batch + 2 * (size_t)total + n_work + n_wide;
        hipStream_t s = as_stream(stream);
        Staging& st = pool->prefill_staging;
        int32_t* h = st.acquire(need);
        int32_t* h_tables = h;
        int32_t* h_start = h_tables + nt;
        int32_t* h_len = h_start + batch;
        int32_t* h_off = h_len + batch;
        int32_t* h_slots = h_off + batch;
        int32_t* h_row_pos = h_slots + total;
        int32_t* h_work = h_row_pos + total;
        int32_t* h_wide = h_work + n_work;
        std::memcpy(h_tables, tables, nt * sizeof(int32_t));
        std::memcpy(h_start, start_pos, batch * sizeof(int32_t));
        std::memcpy(h_len, num_tokens, batch * sizeof(int32_t));
        std::memcpy(h_off, row_off.data(), batch * sizeof(int32_t));
        for (int b = 0; b < batch; b++)
            for (int t = 0; t < num_tokens[b]; t++) {
                const int pos = start_pos[b] + t;
                h_slots[row_off[b] + t] = tables[(size_t)b * max_pages + (pos >> 4)] * BLOCK_SIZE + (pos & 15);
                h_row_pos[row_off[b] + t] = pos;
            }
        for (size_t i = 0; i < items.size(); i++) {
            h_work[2 * i] = items[i].second.first;
            h_work[2 * i + 1] = items[i].second.second;
        }
        for (size_t i = 0; i < wide.size(); i++) {
            h_wide[2 * i] = wide[i].second.first;
            h_wide[2 * i + 1] = wide[i].second.second;
        }
        p.tables.reserve(nt);
        p.d_start.reserve(batch);
        p.d_len.reserve(batch);
        p.d_row_off.reserve(batch);
        p.slots.reserve(total);
        p.row_pos.reserve(total);
        p.work.reserve(n_work);
        p.work_wide.reserve(n_wide);
        st.copy(p.tables.ptr, h_tables, nt, s);
        st.copy(p.d_start.ptr, h_start, batch, s);
        st.copy(p.d_len.ptr, h_len, batch, s);
        st.copy(p.d_row_off.ptr, h_off, batch, s);
        st.copy(p.slots.ptr, h_slots, total, s);
        st.copy(p.row_pos.ptr, h_row_pos, total, s);
        st.copy(p.work.ptr, h_work, n_work, s);
        st.copy(p.work_wide.ptr, h_wide, n_wide, s);
        st.finish(s);
        p.start_pos.assign(start_pos, start_pos + batch);
        p.num_tokens.assign(num_tokens, num_tokens + batch);
        p.row_off = row_off;
        p.total_rows = (int32_t)total;
        p.max_tokens = max_tokens;
        int max_pos = 0;
        for (int b = 0; b < batch; b++)
            if (num_tokens[b] > 0) max_pos = std::max(max_pos, start_pos[b] + num_tokens[b] - 1);
        p.max_pos = max_pos;
        p.append_in_launch = chunk_pages_private(tables, start_pos, num_tokens, batch, max_pages);
        p.append_mixed = false;
        for (int b = 0; b < batch; b++) p.append_mixed |= num_tokens[b] > 0 && start_pos[b] > 0;
        p.work_items = (int32_t)items.size();
        p.work_block_m = bm;
        p.work_items_wide = (int32_t)wide.size();
        p.max_pages = max_pages;
        p.batch = batch;
        pool->last_stream = s;
    });
}

int nitro_kv_append_prefill(nitro_kvpool* pool, int32_t layer, const float* k, const float* v,
                            void* stream) {
    return guarded([&] {
        require_pool(pool);
        require(k != nullptr && v != nullptr, ERR_INVALID_ARGUMENT, "null k/v");
        require(layer >= 0 && layer < pool->num_layers, ERR_INVALID_ARGUMENT, "layer out of range");
        const PrefillBatch& p = pool->prefill;
        require(p.batch > 0, ERR_NO_BATCH, "no prefill batch uploaded");
        hipStream_t s = as_stream(stream);
        hip_check(launch_kv_scatter_rows(pool->k, pool->v, k, v, p.slots.ptr, p.total_rows,
                                         pool->kv_dim, pool->page_stride(), pool->layer_offset(layer),
                                         pool->num_pages, pool->bad_pages.ptr, s),
                  "kv_scatter launch");
        pool->last_stream = s;
    });
}

static PrefillLaunch prefill_args(nitro_kvpool* pool, int32_t layer, const float* q, float* out,
                                  int32_t n_heads, int32_t n_kv_heads, int32_t head_dim) {
    require_pool(pool);
    require(q != nullptr && out != nullptr, ERR_INVALID_ARGUMENT, "null q/out");
    check_shape(pool, layer, n_heads, n_kv_heads, head_dim);
    const PrefillBatch& p = pool->prefill;
    require(p.batch > 0, ERR_NO_BATCH, "no prefill batch uploaded");
    PrefillLaunch a{};
    a.q = q;
    a.out = out;
    a.k_pool = pool->k;
    a.v_pool = pool->v;
    a.tables = p.tables.ptr;
    a.start_pos = p.d_start.ptr;
    a.num_tokens = p.d_len.ptr;
    a.row_off = p.d_row_off.ptr;
    a.work = p.work.ptr;
    a.bad_pages = pool->bad_pages.ptr;
    a.page_stride = pool->page_stride();
    a.layer_off = pool->layer_offset(layer);
    a.kv_dim = pool->kv_dim;
    a.n_heads = n_heads;
    a.kv_mul = n_heads / n_kv_heads;
    a.head_dim = head_dim;
    a.max_pages = p.max_pages;
    a.num_pages = pool->num_pages;
    a.work_items = p.work_items;
    a.max_pos = p.max_pos;
    a.qscale = (float)(1.4426950408889634 / std::sqrt((double)head_dim));
    // NITRO_PREFILL_KERNEL=valu / mfma32 selects the VALU / fp32 matrix-core
    // kernel (A/B counter comparisons).
    const char* kern = std::getenv("NITRO_PREFILL_KERNEL");
    a.kernel = !kern                                ? PREFILL_KERNEL_DEFAULT
               : std::strcmp(kern, "valu") == 0     ? PREFILL_KERNEL_VALU
               : std::strcmp(kern, "mfma32") == 0   ? PREFILL_KERNEL_MFMA_F32
                                                    : PREFILL_KERNEL_DEFAULT;
    a.item_rows = p.work_block_m;
    if (prefill_uses_wide_items(a.kernel, head_dim)) {
        a.work = p.work_wide.ptr;
        a.work_items = p.work_items_wide;
        a.item_rows = PREFILL_WIDE_ROWS;
    }
    return a;
}

int nitro_paged_attn_prefill(nitro_kvpool* pool, int32_t layer, const float* q, float* out,
                             int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, void* stream) {
    return guarded([&] {
        const PrefillLaunch a = prefill_args(pool, layer, q, out, n_heads, n_kv_heads, head_dim);
        hipStream_t s = as_stream(stream);
        hip_check(launch_paged_attn_prefill(a, s), "paged_attn_prefill launch");
        pool->last_stream = s;
    });
}

int nitro_paged_attn_prefill_append(nitro_kvpool* pool, int32_t layer, const float* q, const float* k,
                                    const float* v, float* out, int32_t n_heads, int32_t n_kv_heads,
                                    int32_t head_dim, void* stream) {
    return guarded([&] {
        PrefillLaunch a = prefill_args(pool, layer, q, out, n_heads, n_kv_heads, head_dim);
        require(k != nullptr && v != nullptr, ERR_INVALID_ARGUMENT, "null k/v");
        PrefillBatch& p = pool->prefill;
        hipStream_t s = as_stream(stream);
        p.append_launches++;
        // NITRO_PREFILL_APPEND=0: always the scatter, then attention (A/B)
        if (p.append_in_launch && prefill_appends_in_launch(a.kernel, head_dim, p.max_pos, a.page_stride) &&
            env_int("NITRO_PREFILL_APPEND", 1) != 0) {
            a.k_new = k;
            a.v_new = v;
            a.append_mixed = p.append_mixed ? 1 : 0;
            hip_check(launch_paged_attn_prefill(a, s), "paged_attn_prefill append launch");
            p.fused_launches++;
        } else {
            hip_check(launch_kv_scatter_rows(pool->k, pool->v, k, v, p.slots.ptr, p.total_rows,
                                             pool->kv_dim, pool->page_stride(), pool->layer_offset(layer),
                                             pool->num_pages, pool->bad_pages.ptr, s),
                      "kv_scatter launch");
            hip_check(launch_paged_attn_prefill(a, s), "paged_attn_prefill launch");
        }
        pool->last_stream = s;
    });
}

int nitro_kvpool_prefill_counts(nitro_kvpool* pool, int64_t* calls, int64_t* one_launch) {
    return guarded([&] {
        require_pool(pool);
        require(calls != nullptr && one_launch != nullptr, ERR_INVALID_ARGUMENT, "null output");
        *calls = (int64_t)pool->prefill.append_launches;
        *one_launch = (int64_t)pool->prefill.fused_launches;
    });
}

static void check_rope(const nitro_kvpool* pool, int layer, int n_heads, int n_kv_heads,
                       int head_dim, int seq_len, int max_pos, const void* q, const void* k,
                       const void* v, const void* fr, const void* fi) {
    require(q && k && v && fr && fi, ERR_INVALID_ARGUMENT, "null q/k/v or RoPE table");
    check_shape(pool, layer, n_heads, n_kv_heads, head_dim);
    require(seq_len > max_pos, ERR_INVALID_ARGUMENT, "a position lies beyond the RoPE tables");
}

int nitro_rope_kv_append(nitro_kvpool* pool, int32_t layer, float* q, float* k, const float* v,
                         const float* freq_real, const float* freq_imag, int32_t seq_len,
                         int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, void* stream) {
    return guarded([&] {
        require_pool(pool);
        const DecodeBatch& d = pool->decode;
        require(d.batch > 0, ERR_NO_BATCH, "no decode batch uploaded");
        int max_pos = 0;
        for (int p : d.positions) max_pos = std::max(max_pos, p);
        check_rope(pool, layer, n_heads, n_kv_heads, head_dim, seq_len, max_pos, q, k, v,
                   freq_real, freq_imag);
        hipStream_t s = as_stream(stream);
        hip_check(launch_rope_kv_append(pool->k, pool->v, q, k, v, freq_real, freq_imag,
                                        d.tables.ptr, d.pos.ptr, nullptr, nullptr, d.batch,
                                        d.max_pages, n_heads * head_dim, pool->kv_dim, head_dim,
                                        pool->page_stride(), pool->layer_offset(layer),
                                        pool->num_pages, pool->bad_pages.ptr, s),
                  "rope_kv_append launch");
        pool->last_stream = s;
    });
}

int nitro_rope_kv_append_prefill(nitro_kvpool* pool, int32_t layer, float* q, float* k,
                                 const float* v, const float* freq_real, const float* freq_imag,
                                 int32_t seq_len, int32_t n_heads, int32_t n_kv_heads,
                                 int32_t head_dim, void* stream) {
    return guarded([&] {
        require_pool(pool);
        const PrefillBatch& p = pool->prefill;
        require(p.batch > 0, ERR_NO_BATCH, "no prefill batch uploaded");
        check_rope(pool, layer, n_heads, n_kv_heads, head_dim, seq_len, p.max_pos, q, k, v,
                   freq_real, freq_imag);
        hipStream_t s = as_stream(stream);
        hip_check(launch_rope_kv_append(pool->k, pool->v, q, k, v, freq_real, freq_imag, nullptr,
                                        nullptr, p.slots.ptr, p.row_pos.ptr, p.total_rows,
                                        p.max_pages, n_heads * head_dim, pool->kv_dim, head_dim,
                                        pool->page_stride(), pool->layer_offset(layer),
                                        pool->num_pages, pool->bad_pages.ptr, s),
                  "rope_kv_append_prefill launch");
        pool->last_stream = s;
    });
}

int nitro_q8_matmul(const void* w, const float* x, float* out, int32_t batch, int32_t n, int32_t d,
                    int32_t semantics, void* stream) {
    return guarded([&] {
        require(w != nullptr && x != nullptr && out != nullptr, ERR_INVALID_ARGUMENT, "null pointer");
        require(batch > 0 && n > 0 && d > 0, ERR_INVALID_ARGUMENT, "batch, n and d must be positive");
        require(n % 32 == 0, ERR_INVALID_ARGUMENT, "n must be a multiple of 32 (Q8 block)");
        require(semantics == NITRO_Q8_FULL_ROWS || semantics == NITRO_Q8_LAST_BLOCK, ERR_INVALID_ARGUMENT,
                "semantics must be NITRO_Q8_FULL_ROWS or NITRO_Q8_LAST_BLOCK");
        require(reinterpret_cast<uintptr_t>(w) % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0,
                ERR_INVALID_ARGUMENT, "w must be 4-byte and x 16-byte aligned");
        hip_check(launch_q8_matmul(w, x, out, batch, n, d, semantics == NITRO_Q8_LAST_BLOCK,
                                   as_stream(stream)),
                  "q8_matmul launch");
    });
}

int nitro_kvpool_decode_counts(nitro_kvpool* pool, int64_t* launches, int64_t* shared_prefix_launches) {
    return guarded([&] {
        require_pool(pool);
        require(launches != nullptr && shared_prefix_launches != nullptr, ERR_INVALID_ARGUMENT,
                "null output pointer");
        *launches = (int64_t)pool->decode.launches;
        *shared_prefix_launches = (int64_t)pool->decode.prefix_launches;
    });
}

int nitro_kvpool_take_device_errors(nitro_kvpool* pool, int32_t* bad_pages) {
    return guarded([&] {
        require_pool(pool);
        require(bad_pages != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        hip_check(hipStreamSynchronize(pool->last_stream), "hipStreamSynchronize");
        int32_t v = 0;
        hip_check(hipMemcpy(&v, pool->bad_pages.ptr, sizeof(int32_t), hipMemcpyDeviceToHost), "hipMemcpy");
        hip_check(hipMemset(pool->bad_pages.ptr, 0, sizeof(int32_t)), "hipMemset");
        hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        *bad_pages = v;
    });
}

}  // extern "C"
