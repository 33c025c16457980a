// Batched paged-attention decode for gfx950 (MI355X).
//
// Computes, for every (sequence b, query head h), what the reference's
// forward_decode_batch attention computes (src/model_q8.cpp:625-662):
//   s_t = q_h . k_t / sqrt(hd) over keys t = 0..pos_b (pages via the block
//   table, kv head h / (H/Hkv)), p = softmax(s), o_h = sum_t p_t v_t.
//
// Design (bandwidth-bound: K and V are read exactly once per query head):
//  - Work items: a (sequence, split) pair covers a run of at most
//    `tiles_per_split` tiles of TILE consecutive context rows.  The grid is
//    items x KV heads x head sub-groups, one workgroup of W wavefronts each
//    (W = 4..16 per launch); waves take the item's tiles round-robin.  With
//    a work list the host hands out only real items (shortest first), and
//    long sequences are split into equal runs, so no workgroup streams more
//    than one split's tiles whatever the mix of context lengths.  The list
//    (up to DECODE_ARG_ITEMS items) rides in the kernel arguments; an item
//    may start past a sequence's shared rows (below).  Without
//    one, item i is split i % num_splits of sequence i / num_splits and
//    workgroups past a sequence's last split exit at once.
//  - Lane layout: LG = 8 lanes share one K/V row (16 for a 256-wide head) so
//    that every global_load_dwordx4 reads whole 128-byte lines; a lane holds
//    HDP/LG floats of each of its RL rows (columns c*4 + j*4*LG).  HDP is the
//    head size rounded up to 32, 64, 128 or 256: columns past the head size
//    are masked (loaded as zero, never stored).  The 64/LG row groups of a
//    wave take interleaved rows of a tile (64, 32, 16, 8 rows for HDP = 32,
//    64, 128, 256); all 16 K/V float4 loads of a tile are issued before use.
//  - q.k: HDP/LG FMAs per lane and row, then a DPP butterfly across LG lanes.
//  - Softmax in base 2 (q is pre-scaled by log2(e)/sqrt(hd)): a wave keeps one
//    running max (each tile's maximum is taken across the lane groups), and
//    every lane group its own running (sum, acc), so the groups' states just
//    add up at the end (DPP and permlane swaps).  Waves (through LDS), then
//    splits are merged with the usual rescaling.  No score scratch.
//  - Split-K merge in the same launch: a split writes (acc[hd], m, l) per
//    query head with device-coherent stores (global_store ... sc1, written
//    through the XCD's L2), waits for them (vmcnt(0)) and bumps its (b, head
//    group)'s arrival counter; the workgroup that arrives last reads every
//    split's partials with device-coherent loads, merges them in split order
//    (results do not depend on arrival order), writes the output and resets
//    the counter to zero for the next launch.  Nothing waits on another
//    workgroup, and no fence writes back or invalidates a whole L2 (agent-
//    scope release/acquire fences do both on gfx950; measured, those halved
//    throughput at two splits).  Why the publish holds without them: every
//    access to a partial is itself a relaxed agent-scope atomic, which the
//    AMDGPU backend lowers to global_store / global_load with sc1 (LLVM's
//    GFX942 memory-model table, which gfx950 follows), coherent across the
//    XCDs' L2s on its own.  Of an agent-scope release sequence (buffer_wbl2
//    sc1; s_waitcnt vmcnt(0); the releasing access) that leaves the wait:
//    the L2 write-back only serves non-atomic stores, and there are none
//    here.  Likewise the acquire's buffer_inv sc1 only serves non-atomic
//    loads.  What remains is the order the compiler emits: a workgroup-
//    scope fence (inside __syncthreads on the split path, explicit on the
//    member path; on gfx950 it emits at most a wait) keeps the stores above
//    the wait and the counter bump, and the merge's loads below it.
//  - Fused append (k_new / v_new given): row pos_b = ctx_b - 1 is read from
//    the new K/V rows instead of the pool, and the workgroup holding that
//    row (head sub-group 0 of the last split) writes them into the pool slot,
//    i.e. forward_decode_batch's memcpy (src/model_q8.cpp:616-623) and its
//    attention in one launch.  The host uses it only when no other row of the
//    batch reads that page.
//  - Shared prefixes (MEMBERS instances; the host finds sequences whose first
//    pages are the same physical pages): the work list starts with member
//    items, each a set of up to W member sequences over a chunk of the shared
//    rows.  Wave w takes member w and streams the whole chunk, so the
//    workgroup's waves read each shared row at about the same time through
//    one L1 and the row leaves L2 once per set, not once per sequence.  The
//    wave writes its member's partial and counts it in like a split.  The
//    sequences' own rows follow as ordinary split items.  Every (sequence,
//    head) then has partials from both, merged in slot order (member chunks
//    first) by whichever workgroup or wave arrives last.
//  - The item's block-table slice is staged in LDS once; page ids outside the
//    pool are counted in *bad_pages and their rows skipped (no fault).
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>

#include "device_pool.hpp"

// Workspace of the allocation-free decode entry (nitro_paged_attn_decode_static):
// arrival counters, then split-K partials.  Each GPU the library runs on holds
// its own copy until the process ends; zero at load, and every launch leaves
// its counters at zero again.  Host code never passes this name to a kernel
// (in host code it is a stand-in, not a device address): it takes the address
// from decode_static_scratch below.
static __device__ __align__(256) float scratch[nitro::DECODE_STATIC_SCRATCH_BYTES / sizeof(float)];

namespace nitro {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t decode_static_scratch(float** ptr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *ptr = g_scratch_ptr[dev];
    return hipSuccess;
}

namespace {

constexpr int MAX_WAVES = 16;
constexpr int MAX_THREADS = 64 * MAX_WAVES;

template <int HDP>
struct DecodeGeom {
    // LG lanes share a K/V row so that one load instruction reads whole
    // 128-byte lines (8 lanes x 16 B; 16 lanes for HDP=256, two lines).  Each
    // lane holds NF4 float4 of a row (columns c*4 + j*4*LG) for RL rows per
    // tile: RL*NF4 = 8 float4 of K and 8 of V in flight per lane.
    static constexpr int LG = HDP <= 128 ? 8 : 16;
    static constexpr int NF4 = HDP / (4 * LG);
    static constexpr int RL = 8 / NF4;
    static constexpr int GROUPS = 64 / LG;  // row groups per wave
    static constexpr int TILE = RL * GROUPS;
    static_assert(NF4 >= 1 && RL * NF4 == 8, "padded head size 32, 64, 128 or 256");
};

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over the LG consecutive lanes of a group (result in every lane).
template <int LG>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (LG >= 2) x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (LG >= 4) x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (LG >= 8) x += dpp_mov<0x141>(x);  // row_half_mirror: other quad of the 8
    if constexpr (LG >= 16) x += dpp_mov<0x140>(x); // row_mirror: other 8 of the 16
    return x;
}

__device__ __forceinline__ float dot4(float4 a, float4 b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    acc = fmaf(a.w, b.w, acc);
    return acc;
}

typedef float f4v __attribute__((ext_vector_type(4)));

// K/V row loads.  STREAM issues them non-temporal (global_load_dwordx4 ... nt):
// lines read once per launch are not kept in L2 / MALL, which raises the
// achievable streaming rate; plain loads keep lines that other workgroups read
// again (pages shared between sequences, query heads of one KV group).
template <bool STREAM>
__device__ __forceinline__ float4 load_kv(const float* p) {
    if constexpr (STREAM) {
        const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
        return make_float4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const float4*>(p);
    }
}

// 2^x for x <= 0 on v_exp_f32 directly: results below 2^-126 flush to zero
// (exp2f adds range handling for them), far below what an fp32 sum of
// weights up to 1 can hold.
__device__ __forceinline__ float exp2_nonpos(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float scale_of(float m, float m_new) {
    return m == -INFINITY ? 0.0f : exp2_nonpos(m - m_new);
}

// The two values of a lane pair (l, l ^ 16 with HALVES = false; l, l ^ 32
// with HALVES = true) via v_permlane16_swap / v_permlane32_swap of x with
// itself, which leave both in every lane.
template <bool HALVES>
__device__ __forceinline__ void pair_values(float x, float& a, float& b) {
    if constexpr (HALVES) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        a = __uint_as_float(r[0]);
        b = __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        a = __uint_as_float(r[0]);
        b = __uint_as_float(r[1]);
    }
}

// (l, acc) of a lane added to its pair's (both hold the same running max).
template <int NF4, bool HALVES>
__device__ __forceinline__ void sum_pair(float& l, float4 (&acc)[NF4]) {
    float a, b;
    pair_values<HALVES>(l, a, b);
    l = a + b;
#pragma unroll
    for (int j = 0; j < NF4; j++) {
        float x0, x1, y0, y1, z0, z1, w0, w1;
        pair_values<HALVES>(acc[j].x, x0, x1);
        pair_values<HALVES>(acc[j].y, y0, y1);
        pair_values<HALVES>(acc[j].z, z0, z1);
        pair_values<HALVES>(acc[j].w, w0, w1);
        acc[j] = make_float4(x0 + x1, y0 + y1, z0 + z1, w0 + w1);
    }
}

// Maximum of x over the lane groups of a wave (x is uniform within a group of
// LG lanes; the result is in every lane).
template <int LG>
__device__ __forceinline__ float wave_max(float x) {
    if constexpr (LG == 8) x = fmaxf(x, dpp_mov<0x128>(x));  // row_ror:8: the other group of the row
    float a, b;
    pair_values<false>(x, a, b);
    x = fmaxf(a, b);
    pair_values<true>(x, a, b);
    return fmaxf(a, b);
}

// Device-coherent accesses of the split-K partials and arrival counters:
// relaxed atomics at agent scope are global_store / global_load ... sc1 on
// gfx950 (written through to, and read from, the point where the XCDs'
// caches agree) with no whole-cache writeback or invalidate.
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima): this wave's
// stores have completed.
__device__ __forceinline__ void wait_vector_memory() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Split-K merge of one (sequence, query head h): its partials in slots
// slot0 .. slot0 + parts - 1, combined in slot order (so the result does not
// depend on arrival order), output columns first, first + stride, ... (a
// workgroup's or a wave's threads).  Every part's (m, l, acc[d]) loads go out
// together, MB parts at a time.
constexpr int MERGE_BATCH = 8;
template <int MB>
__device__ __forceinline__ void merge_parts(const DecodeLaunch& a, int slot0, int parts, int n_heads, int h, int hd,
                                            int first, int stride, size_t out_row) {
    for (int d = first; d < hd; d += stride) {
        float M = -INFINITY, L = 0.0f, A = 0.0f;
        for (int sp0 = 0; sp0 < parts; sp0 += MB) {
            float ms[MB], ls[MB], as[MB];
#pragma unroll
            for (int j = 0; j < MB; j++) {
                const int sp = min(sp0 + j, parts - 1);  // past the last part: a repeat, unused
                const float* part = a.partials + ((size_t)(slot0 + sp) * n_heads + h) * a.pstride;
                ms[j] = load_coherent(part + hd);
                ls[j] = load_coherent(part + hd + 1);
                as[j] = load_coherent(part + d);
            }
#pragma unroll
            for (int j = 0; j < MB; j++) {
                if (sp0 + j >= parts) break;
                const float mm = fmaxf(M, ms[j]);
                const float f = scale_of(M, mm), fs = scale_of(ms[j], mm);
                L = L * f + ls[j] * fs;
                A = A * f + as[j] * fs;
                M = mm;
            }
        }
        a.out[out_row * hd + d] = A / L;
    }
}

// QH query heads of one KV head per workgroup (QH = 1 for MHA): each K/V
// row is loaded once and scored against all QH queries.  QH > 1 needs about
// twice the registers, so those workgroups hold at most 8 waves.  FULL: the
// head size is HDP (no column masks).
//
// The scalars that locate a workgroup's item and its block-table slice come
// first in the argument list, so that the build preloads them into SGPRs
// (-mllvm -amdgpu-kernarg-preload-count=10): the table and position loads go
// out at once, while the loads of the other arguments are still in flight.
// flags: bit 0 XCD work order, bit 1 items from arg_items.  waves and
// nblocks stand for blockDim.x / 64 and gridDim.x, which are read from memory.
template <int HDP, int QH, bool STREAM, bool FULL, bool MEMBERS>
__global__ __launch_bounds__(QH == 1 ? MAX_THREADS : MAX_THREADS / 2) void paged_attn_decode_kernel(
    const int32_t* __restrict__ tables, const int32_t* __restrict__ positions, int32_t max_pages,
    int32_t num_splits, int32_t tiles_per_split, int32_t n_heads, int32_t kv_mul, int32_t flags,
    int32_t waves, int32_t nblocks, DecodeLaunch a, DecodeArgItems arg_items) {
    using G = DecodeGeom<HDP>;
    constexpr int LG = G::LG, NF4 = G::NF4, RL = G::RL, GROUPS = G::GROUPS, TILE = G::TILE;
    constexpr int MAXW = QH == 1 ? MAX_WAVES : MAX_WAVES / 2;
    __shared__ int32_t s_pages[DECODE_MAX_SPLIT_PAGES];
    // member items: one staged tile of K and V, rows STAGE_ROW floats apart
    // (32 floats of padding where that puts a wave's two rows of one 16-lane
    // read on different banks)
    constexpr int STAGE_ROW = HDP == 64 || HDP == 128 ? HDP + 32 : HDP;
    __shared__ __attribute__((aligned(16))) float s_stage_k[MEMBERS ? TILE * STAGE_ROW : 4];
    __shared__ __attribute__((aligned(16))) float s_stage_v[MEMBERS ? TILE * STAGE_ROW : 4];
    __shared__ float s_acc[MAXW][QH][HDP];
    __shared__ float s_m[MAXW][QH], s_l[MAXW][QH];
    __shared__ int s_last;
    const int hd = FULL ? HDP : a.head_dim;
    const int threads = waves * 64;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane / LG;
    const int c = lane % LG;

    // Work order: (item * Hkv + kv_h) * (kv_mul/QH) + r; the workgroup serves
    // query heads h0 .. h0+QH-1, h0 = kv_h*kv_mul + r*QH, so the workgroups
    // that read one K/V range are consecutive.  With xcd_remap, block ids are
    // dealt to the 8 XCDs round-robin, so XCD x takes the x-th contiguous
    // eighth of that order: workgroups sharing a K/V range run together on
    // one XCD and re-read it from its L2.
    int w = blockIdx.x;
    if ((flags & 1)) {
        const int n = nblocks, per = n >> 3, rem = n & 7;
        const int x = w & 7;
        w = x * per + min(x, rem) + (w >> 3);
    }
    const int hsubs = kv_mul / QH;
    const int n_kv = n_heads / kv_mul;
    const int r = w % hsubs;
    const int rest = w / hsubs;
    const int kv_h = rest % n_kv;
    const int item = rest / n_kv;
    const int hg = kv_h * hsubs + r;  // head group of the sequence (arrival counter)
    const int bh_in_seq = kv_h * kv_mul + r * QH;

    // The item: from the work list {b, split | first tile << 8, first partial
    // slot of b | partials of b << 16, ctx}, or implied by the block id (then
    // the position load goes out together with the block-table slice and q
    // below).  With MEMBERS the list may also hold member items (x < 0):
    // {-1 - first member entry, members | part << 8, first tile, tiles}, the
    // entries {b, first slot | partials << 16, b', ...} two to an int4.
    const bool listed = flags & 2;
    int b, split, pslot0, ctx = 0, first_tile = 0, parts_b = 0;
    bool member = false;
    int mem_count = 0, mem_part = 0, mem_b = 0, mem_slot = 0, mem_parts = 0, mem_tiles = 0;
    if (listed) {
        // the list rides in the kernel arguments: one scalar load of the
        // item precedes the table and q loads
        const int4 it = arg_items.item[item];
        member = MEMBERS && it.x < 0;
        if (member) {
            mem_count = it.y & 0xFF;
            mem_part = it.y >> 8;
            first_tile = it.z;
            mem_tiles = it.w;
            const int4 e0 = arg_items.item[-1 - it.x];  // member 0: its table row holds the shared pages
            b = e0.x;
            const int mine = min(wave, mem_count - 1);
            const int4 e = arg_items.item[-1 - it.x + mine / 2];
            mem_b = (mine & 1) ? e.z : e.x;
            const int sp = (mine & 1) ? e.w : e.y;
            mem_slot = sp & 0xFFFF;
            mem_parts = sp >> 16;
            split = 0;
            pslot0 = 0;
            ctx = (first_tile + mem_tiles) * TILE;
        } else {
            b = it.x;
            split = it.y & 0xFF;
            first_tile = it.y >> 8;
            pslot0 = it.z & 0xFFFF;
            parts_b = it.z >> 16;
            ctx = it.w;
        }
    } else {
        b = item / num_splits;
        split = item - b * num_splits;
        pslot0 = b * num_splits;
    }
    const int bh0 = b * n_heads + bh_in_seq;
    // The split's block-table slice is read speculatively over the split's
    // whole page range (clipped to the table row); only the entries below the
    // context length are validated and used.
    constexpr int TBL_PER_THREAD = DECODE_MAX_SPLIT_PAGES / 256;  // >= 4 waves per workgroup
    const int tile_begin = first_tile + split * tiles_per_split;
    const int page_begin = (tile_begin * TILE) >> 4;
    const int span = member ? mem_tiles : tiles_per_split;  // tiles of the item at most
    const int spec_end = min(max_pages, ((tile_begin + span) * TILE + 15) >> 4);
    const int32_t* trow = tables + (size_t)b * max_pages;
    int tv[TBL_PER_THREAD];
#pragma unroll
    for (int k = 0; k < TBL_PER_THREAD; k++) {
        const int i = threadIdx.x + k * threads;
        tv[k] = i < spec_end - page_begin ? trow[page_begin + i] : -1;
    }

    // The position (implied items), then the other arguments the prologue
    // and the first tile use, loaded here together: one round trip, which
    // overlaps the table loads above, rather than one where each is first
    // used.  (A vector load of the position measured slower.)
    if (!listed) ctx = positions[b] + 1;
    asm volatile("" ::"s"(a.q), "s"(a.qscale), "s"(a.ctx_limit), "s"(a.num_pages), "s"(a.k_pool), "s"(a.v_pool),
                 "s"(a.layer_off), "s"(a.page_stride), "s"(a.k_new), "s"(a.v_new), "s"(a.kv_dim));

    // q slices of this lane, pre-scaled to base-2 logits (columns past the
    // head size are zero).  A member item's wave takes its member's query.
    float4 qv[QH][NF4];
#pragma unroll
    for (int qi = 0; qi < QH; qi++) {
        const size_t qrow = member ? (size_t)mem_b * n_heads + bh_in_seq : (size_t)(bh0 + qi);
        const float* qp = a.q + qrow * hd;
#pragma unroll
        for (int j = 0; j < NF4; j++) {
            const int col = (c + j * LG) * 4;
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
            if (FULL || col < hd) t = *reinterpret_cast<const float4*>(qp + col);
            qv[qi][j] = make_float4(t.x * a.qscale, t.y * a.qscale, t.z * a.qscale, t.w * a.qscale);
        }
    }

    ctx = max(0, min(ctx, a.ctx_limit));  // a position past the table (or the splits) reads no further
    if (ctx == 0) {
        // A device position below 0 (implied items only: uploaded positions
        // are checked on the host, and listed items carry ctx >= 1): the
        // sequence has no keys.  Split 0 writes zeros for its query heads, and
        // one workgroup of the sequence counts it in *bad_pages, as a page id
        // outside the pool is counted.
        if (split == 0) {
            for (int i = threadIdx.x; i < QH * hd; i += threads) a.out[(size_t)bh0 * hd + i] = 0.0f;
            if (threadIdx.x == 0 && bh_in_seq == 0) atomicAdd(a.bad_pages, 1);
        }
        return;
    }
    const int n_tiles = (ctx + TILE - 1) / TILE;
    if (tile_begin >= n_tiles) return;  // uniform for the workgroup (implied items only)
    // the tiles this workgroup streams: a member item's whole chunk, or the
    // split's run
    const int tile_end = member ? first_tile + mem_tiles : min(n_tiles, tile_begin + tiles_per_split);
    // this sequence's splits, its partials in all (a listed item carries the
    // count, which includes the member items' partials of its shared rows;
    // those take the first slots), and this split's slot
    const int splits_b = (n_tiles - first_tile + tiles_per_split - 1) / tiles_per_split;
    const int parts = listed ? parts_b : splits_b;
    const int my_slot = pslot0 + parts - splits_b + split;

    // Used part of the slice -> LDS (page ids checked against the pool size).
    const int page_end = ((min(ctx, tile_end * TILE) - 1) >> 4) + 1;
#pragma unroll
    for (int k = 0; k < TBL_PER_THREAD; k++) {
        const int i = threadIdx.x + k * threads;
        if (i < page_end - page_begin) {
            int p = tv[k];
            if ((unsigned)p >= (unsigned)a.num_pages) {
                atomicAdd(a.bad_pages, 1);
                p = -1;
            }
            s_pages[i] = p;
        }
    }
    __syncthreads();

    const float* kbase = a.k_pool + a.layer_off + (size_t)kv_h * hd;
    const float* vbase = a.v_pool + a.layer_off + (size_t)kv_h * hd;
    // Fused append: the new row is read from k_new / v_new, and head
    // sub-group 0 of the last split writes it into its page slot.  Nothing in
    // the launch reads that slot (the row itself comes from k_new / v_new), so
    // its values are loaded here and stored once the tiles are done: the
    // copy's load latency stays off the tile loop.  (hd / 4 <= 64 <= threads:
    // one float4 of K and one of V per thread at most.)
    // (A member item's rows are all shared rows, older than any new row.)
    const bool fused = a.k_new && !member;
    const int new_row = fused ? ctx - 1 : -1;
    const float* knew = fused ? a.k_new + (size_t)b * a.kv_dim + (size_t)kv_h * hd : nullptr;
    const float* vnew = fused ? a.v_new + (size_t)b * a.kv_dim + (size_t)kv_h * hd : nullptr;
    const bool appends = fused && r == 0 && tile_end == n_tiles && (int)threadIdx.x < hd / 4;
    float4 k_app = make_float4(0.f, 0.f, 0.f, 0.f), v_app = k_app;
    if (appends) {
        k_app = reinterpret_cast<const float4*>(knew)[threadIdx.x];
        v_app = reinterpret_cast<const float4*>(vnew)[threadIdx.x];
    }

    float m[QH], l[QH];
    float4 acc[QH][NF4];
#pragma unroll
    for (int qi = 0; qi < QH; qi++) {
        m[qi] = -INFINITY;
        l[qi] = 0.0f;
#pragma unroll
        for (int j = 0; j < NF4; j++) acc[qi][j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    // One tile's rows of this lane (kr, vr; valid: the row is real) into the
    // running (m, l, acc) of each query.
    auto consume = [&](const float4 (&kr)[RL][NF4], const float4 (&vr)[RL][NF4], const bool (&valid)[RL]) {
#pragma unroll
        for (int qi = 0; qi < QH; qi++) {
            float s[RL];
            float mt = -INFINITY;
#pragma unroll
            for (int i = 0; i < RL; i++) {
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < NF4; j++) d = dot4(qv[qi][j], kr[i][j], d);
                d = group_sum<LG>(d);
                s[i] = valid[i] ? d : -INFINITY;
                mt = fmaxf(mt, s[i]);
            }
            const float m_new = fmaxf(m[qi], wave_max<LG>(mt));
            const float alpha = scale_of(m[qi], m_new);
            float p[RL];
            float psum = 0.0f;
#pragma unroll
            for (int i = 0; i < RL; i++) {
                p[i] = valid[i] ? exp2_nonpos(s[i] - m_new) : 0.0f;
                psum += p[i];
            }
            l[qi] = l[qi] * alpha + psum;
#pragma unroll
            for (int j = 0; j < NF4; j++) {
                float4 o = make_float4(acc[qi][j].x * alpha, acc[qi][j].y * alpha,
                                       acc[qi][j].z * alpha, acc[qi][j].w * alpha);
#pragma unroll
                for (int i = 0; i < RL; i++) {
                    o.x = fmaf(p[i], vr[i][j].x, o.x);
                    o.y = fmaf(p[i], vr[i][j].y, o.y);
                    o.z = fmaf(p[i], vr[i][j].z, o.z);
                    o.w = fmaf(p[i], vr[i][j].w, o.w);
                }
                acc[qi][j] = o;
            }
            m[qi] = m_new;
        }
    };

    if (MEMBERS && member) {
        // A member item: the workgroup stages each tile of the chunk in LDS,
        // and wave w scores its member against every row.  Each thread loads
        // its share of the next tile into registers while the waves work on
        // the current one.  Staged rows are STAGE_ROW floats apart, so that a
        // wave's 16-byte reads of one column slice hit distinct banks.
        constexpr int F4_ROW = HDP / 4;
        constexpr int SHARE = TILE * F4_ROW / 256;  // float4 of K (and of V) per thread, >= 4 waves
        float4 sk[SHARE], sv[SHARE];
        auto stage_load = [&](int t) {
#pragma unroll
            for (int k = 0; k < SHARE; k++) {
                const int f = threadIdx.x + k * threads;
                const int row = f / F4_ROW, col = (f % F4_ROW) * 4;
                const int abs_row = t * TILE + row;
                const int page = f < TILE * F4_ROW ? s_pages[(abs_row >> 4) - page_begin] : -1;
                sk[k] = sv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (page >= 0 && (FULL || col < hd)) {
                    const size_t off = (size_t)page * a.page_stride + (size_t)(abs_row & 15) * a.kv_dim + col;
                    sk[k] = *reinterpret_cast<const float4*>(kbase + off);
                    sv[k] = *reinterpret_cast<const float4*>(vbase + off);
                }
            }
        };
        // (At hd 128 and 256 the next tile's registers would spill: there the
        // tile is loaded after the previous one is consumed.)
        constexpr bool PREFETCH = HDP <= 64;
        if (PREFETCH) stage_load(tile_begin);
        for (int t = tile_begin; t < tile_end; t++) {
            __syncthreads();  // every wave is done with the previous tile
            if (!PREFETCH) stage_load(t);
#pragma unroll
            for (int k = 0; k < SHARE; k++) {
                const int f = threadIdx.x + k * threads;
                if (f < TILE * F4_ROW) {
                    const int at = (f / F4_ROW) * STAGE_ROW + (f % F4_ROW) * 4;
                    *reinterpret_cast<float4*>(&s_stage_k[at]) = sk[k];
                    *reinterpret_cast<float4*>(&s_stage_v[at]) = sv[k];
                }
            }
            __syncthreads();
            if (PREFETCH && t + 1 < tile_end) stage_load(t + 1);
            if (wave < mem_count) {
                float4 kr[RL][NF4], vr[RL][NF4];
                bool valid[RL];
                bool any = false;
#pragma unroll
                for (int i = 0; i < RL; i++) {
                    const int row = t * TILE + g + i * GROUPS;
                    valid[i] = s_pages[(row >> 4) - page_begin] >= 0;
                    any |= valid[i];
#pragma unroll
                    for (int j = 0; j < NF4; j++) {
                        const int at = (g + i * GROUPS) * STAGE_ROW + (c + j * LG) * 4;
                        kr[i][j] = *reinterpret_cast<const float4*>(&s_stage_k[at]);
                        vr[i][j] = *reinterpret_cast<const float4*>(&s_stage_v[at]);
                    }
                }
                if (__builtin_amdgcn_ballot_w64(any) != 0) consume(kr, vr, valid);
            }
        }
    } else {
        // Waves take the split's tiles in turn.
        for (int t = tile_begin + wave; t < tile_end; t += waves) {
            float4 kr[RL][NF4], vr[RL][NF4];
            bool valid[RL];
            bool any = false;
#pragma unroll
            for (int i = 0; i < RL; i++) {
                const int row = t * TILE + g + i * GROUPS;
                int page = row < ctx ? s_pages[(row >> 4) - page_begin] : -1;
                valid[i] = page >= 0;
                any |= valid[i];
                if (valid[i]) {
                    const size_t off = (size_t)page * a.page_stride + (size_t)(row & 15) * a.kv_dim;
                    const bool fresh = row == new_row;
                    const float* kp = fresh ? knew : kbase + off;
                    const float* vp = fresh ? vnew : vbase + off;
#pragma unroll
                    for (int j = 0; j < NF4; j++) {
                        const int col = (c + j * LG) * 4;
                        if (FULL || col < hd) {
                            kr[i][j] = load_kv<STREAM>(kp + col);
                            vr[i][j] = load_kv<STREAM>(vp + col);
                        } else {
                            kr[i][j] = vr[i][j] = make_float4(0.f, 0.f, 0.f, 0.f);
                        }
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < NF4; j++) {
                        kr[i][j] = make_float4(0.f, 0.f, 0.f, 0.f);
                        vr[i][j] = make_float4(0.f, 0.f, 0.f, 0.f);
                    }
                }
            }
            // The running maximum is shared by the whole wave (the max below
            // crosses lane groups), so a tile is skipped only when no lane of
            // the wave holds a valid row.
            if (__builtin_amdgcn_ballot_w64(any) == 0) continue;
            consume(kr, vr, valid);
        }
    }

    // Merge the lane groups of the wave (lanes with equal c, across g).  They
    // share the running maximum, so their (l, acc) just add up: on VALU
    // permutes, no LDS round trips, lane l ^ 8 by DPP row_ror:8 (LG = 8),
    // then l ^ 16 and l ^ 32 by gfx950's permlane16 / permlane32 swaps, each
    // of which hands a lane both values of its pair.  Every lane ends up with
    // the wave's (m, l, acc).
#pragma unroll
    for (int qi = 0; qi < QH; qi++) {
        if constexpr (LG == 8) {
            l[qi] += dpp_mov<0x128>(l[qi]);
#pragma unroll
            for (int j = 0; j < NF4; j++)
                acc[qi][j] = make_float4(acc[qi][j].x + dpp_mov<0x128>(acc[qi][j].x),
                                         acc[qi][j].y + dpp_mov<0x128>(acc[qi][j].y),
                                         acc[qi][j].z + dpp_mov<0x128>(acc[qi][j].z),
                                         acc[qi][j].w + dpp_mov<0x128>(acc[qi][j].w));
        }
        sum_pair<NF4, false>(l[qi], acc[qi]);  // rows of 16 lanes: l ^ 16
        sum_pair<NF4, true>(l[qi], acc[qi]);   // halves of 32 lanes: l ^ 32
        if (g == 0 && !member) {
#pragma unroll
            for (int j = 0; j < NF4; j++)
                *reinterpret_cast<float4*>(&s_acc[wave][qi][(c + j * LG) * 4]) = acc[qi][j];
            if (c == 0) {
                s_m[wave][qi] = m[qi];
                s_l[wave][qi] = l[qi];
            }
        }
    }
    if (member) {
        // A member item's wave owns its member's result over the chunk: it
        // writes that partial, then counts it in like a split, and merges
        // the sequence's partials if it arrives last.  (Uniform for the
        // workgroup; no workgroup barrier follows.)
        if (wave < mem_count) {
            float* part = a.partials + ((size_t)(mem_slot + mem_part) * n_heads + bh_in_seq) * a.pstride;
            if (g == 0) {
#pragma unroll
                for (int j = 0; j < NF4; j++) {
                    const int col = (c + j * LG) * 4;
                    if (FULL || col < hd) {
                        store_coherent(part + col, acc[0][j].x);
                        store_coherent(part + col + 1, acc[0][j].y);
                        store_coherent(part + col + 2, acc[0][j].z);
                        store_coherent(part + col + 3, acc[0][j].w);
                    }
                }
                if (c == 0) {
                    store_coherent(part + hd, m[0]);
                    store_coherent(part + hd + 1, l[0]);
                }
            }
            // The same publish as the split path's below: the fence keeps the
            // compiler from moving the partial stores past the wait and the
            // counter bump (it is the fence __syncthreads carries there), and
            // the one after the bump keeps the merge's loads below it.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            wait_vector_memory();
            int last = 0;
            if (lane == 0) {
                int* counter = a.counters + (size_t)mem_b * (n_heads / QH) + hg;
                const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last = before == mem_parts - 1;
                if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            if (__builtin_amdgcn_readfirstlane(last))
                merge_parts<MERGE_BATCH>(a, mem_slot, mem_parts, n_heads, bh_in_seq, hd, lane, 64,
                                          (size_t)mem_b * n_heads + bh_in_seq);
        }
        return;
    }
    __syncthreads();

    // Merge the waves: thread o owns output column o % hd of head o / hd
    // (every wave's values read from LDS at once, then added in wave order).
    for (int o = threadIdx.x; o < QH * hd; o += threads) {
        const int qi = o / hd, d = o - qi * hd;
        float mw[MAXW];
        float M = -INFINITY, L = 0.0f, A = 0.0f;
#pragma unroll
        for (int wv = 0; wv < MAXW; wv++) {
            mw[wv] = wv < waves ? s_m[wv][qi] : -INFINITY;
            M = fmaxf(M, mw[wv]);
        }
#pragma unroll
        for (int wv = 0; wv < MAXW; wv++) {
            if (wv < waves) {
                const float f = scale_of(mw[wv], M);
                L += s_l[wv][qi] * f;
                A += s_acc[wv][qi][d] * f;
            }
        }
        const int bh = bh0 + qi;
        if (parts == 1) {
            a.out[(size_t)bh * hd + d] = A / L;
        } else {
            float* part = a.partials + ((size_t)my_slot * n_heads + bh - b * n_heads) * a.pstride;
            store_coherent(part + d, A);
            if (d == 0) {
                store_coherent(part + hd, M);
                store_coherent(part + hd + 1, L);
            }
        }
    }
    if (appends) {
        const int page = s_pages[((ctx - 1) >> 4) - page_begin];
        if (page >= 0) {
            const size_t off = a.layer_off + (size_t)page * a.page_stride + (size_t)((ctx - 1) & 15) * a.kv_dim +
                               (size_t)kv_h * hd;
            reinterpret_cast<float4*>(a.k_pool + off)[threadIdx.x] = k_app;
            reinterpret_cast<float4*>(a.v_pool + off)[threadIdx.x] = v_app;
        }
    }
    if (parts == 1) return;  // uniform for the workgroup

    // Split-K: the last workgroup of this (b, head group) to arrive merges.
    wait_vector_memory();
    __syncthreads();
    if (threadIdx.x == 0) {
        int* counter = a.counters + (size_t)b * (n_heads / QH) + hg;
        const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = before == parts - 1;
        if (before == parts - 1) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
#pragma unroll
    for (int qi = 0; qi < QH; qi++)
        merge_parts<MERGE_BATCH>(a, pslot0, parts, n_heads, bh_in_seq + qi, hd, (int)threadIdx.x, threads,
                                 (size_t)(bh0 + qi));
}

}  // namespace

int decode_max_heads_per_wg(int head_dim) {
    const int hdp = decode_padded_head_dim(head_dim);
    return hdp <= 64 ? 8 : hdp == 128 ? 4 : 2;  // QH * HDP <= 512
}

int decode_padded_head_dim(int head_dim) {
    return head_dim <= 32 ? 32 : head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
}

int decode_tile_rows(int head_dim) {
    switch (decode_padded_head_dim(head_dim)) {
        case 32: return DecodeGeom<32>::TILE;
        case 64: return DecodeGeom<64>::TILE;
        case 128: return DecodeGeom<128>::TILE;
        default: return DecodeGeom<256>::TILE;
    }
}

template <int HDP, int QH>
static void launch_main(const DecodeLaunch& a, const DecodeArgItems& it, dim3 grid, hipStream_t stream) {
    const dim3 block(64 * a.waves);
    const int32_t flags = (a.xcd_remap ? 1 : 0) | (a.arg_items ? 2 : 0);
#define NITRO_DECODE_ARGS a.tables, a.positions, a.max_pages, a.num_splits, a.tiles_per_split, a.n_heads, a.kv_mul, \
                          flags, a.waves, (int32_t)grid.x, a, it
    if constexpr (QH == 1) {
        if (a.members) {  // the list holds member items (shared prefixes)
            if (a.head_dim != HDP)
                hipLaunchKernelGGL((paged_attn_decode_kernel<HDP, 1, false, false, true>), grid, block, 0, stream, NITRO_DECODE_ARGS);
            else if (a.stream_kv)
                hipLaunchKernelGGL((paged_attn_decode_kernel<HDP, 1, true, true, true>), grid, block, 0, stream, NITRO_DECODE_ARGS);
            else
                hipLaunchKernelGGL((paged_attn_decode_kernel<HDP, 1, false, true, true>), grid, block, 0, stream, NITRO_DECODE_ARGS);
            return;
        }
    }
    if (a.head_dim != HDP)  // padded head: plain loads
        hipLaunchKernelGGL((paged_attn_decode_kernel<HDP, QH, false, false, false>), grid, block, 0, stream, NITRO_DECODE_ARGS);
    else if (a.stream_kv)
        hipLaunchKernelGGL((paged_attn_decode_kernel<HDP, QH, true, true, false>), grid, block, 0, stream, NITRO_DECODE_ARGS);
    else
        hipLaunchKernelGGL((paged_attn_decode_kernel<HDP, QH, false, true, false>), grid, block, 0, stream, NITRO_DECODE_ARGS);
#undef NITRO_DECODE_ARGS
}

template <int HDP>
static hipError_t launch_hd(const DecodeLaunch& a, const DecodeArgItems& it, hipStream_t stream) {
    if (a.heads_per_wg < 1 || a.kv_mul % a.heads_per_wg != 0 || a.heads_per_wg > decode_max_heads_per_wg(HDP) ||
        (a.heads_per_wg > 1 && a.waves > MAX_WAVES / 2) || (a.members && (!a.arg_items || a.heads_per_wg != 1)))
        return hipErrorInvalidValue;
    const size_t items = a.arg_items ? (size_t)a.work_items : (size_t)a.batch * a.num_splits;
    const dim3 grid((unsigned)(items * (a.n_heads / a.heads_per_wg)));
    switch (a.heads_per_wg) {
        case 1: launch_main<HDP, 1>(a, it, grid, stream); break;
        case 2: launch_main<HDP, 2>(a, it, grid, stream); break;
        case 4:
            if constexpr (4 * HDP <= 512) launch_main<HDP, 4>(a, it, grid, stream);
            break;
        case 8:
            if constexpr (8 * HDP <= 512) launch_main<HDP, 8>(a, it, grid, stream);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_paged_attn_decode(const DecodeLaunch& a, hipStream_t stream, const DecodeArgItems* items) {
    static const DecodeArgItems none{};
    const DecodeArgItems& it = items ? *items : none;
    if (a.arg_items && (!items || a.work_items > DECODE_ARG_ITEMS)) return hipErrorInvalidValue;
    // >= 4 waves: the block-table slice (<= DECODE_MAX_SPLIT_PAGES entries) is
    // loaded at most 4 entries per thread.
    if (a.waves < 4 || a.waves > MAX_WAVES || a.head_dim < 4 || a.head_dim > 256 || a.head_dim % 4 ||
        a.pstride < a.head_dim + 2)
        return hipErrorInvalidValue;
    switch (decode_padded_head_dim(a.head_dim)) {
        case 32: return launch_hd<32>(a, it, stream);
        case 64: return launch_hd<64>(a, it, stream);
        case 128: return launch_hd<128>(a, it, stream);
        default: return launch_hd<256>(a, it, stream);
    }
}

}  // namespace nitro
