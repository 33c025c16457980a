// Device-side state behind a nitro_kvpool handle: the K/V pools, the
// uploaded decode / prefill batches, the split-K workspace and the device
// error counter.  Host code only (kernels take plain pointers).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "paged_memory.hpp"

namespace nitro {

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        // HIP also records the failure as the thread's last error, which the
        // next launch check (hipGetLastError) would report as its own: clear it.
        (void)hipGetLastError();
        throw Error(e == hipErrorOutOfMemory ? ERR_DEVICE_ALLOC : ERR_HIP,
                    std::string(what) + ": " + hipGetErrorString(e));
    }
}

// Capacity for a buffer that must hold n elements and holds `have`: at least
// twice what it had (and 1024 elements), so a buffer sized per step (batch
// rows, table pages, upload words) is reallocated a few times over a serving
// run rather than whenever it grows.  A reallocation frees the old block, and
// hipFree / hipHostFree wait for the device.
inline size_t grown_capacity(size_t n, size_t have) {
    const size_t twice = 2 * have > 1024 ? 2 * have : 1024;
    return n > twice ? n : twice;
}

// A device allocation that only grows (hipMalloc outside any capture).
template <class T>
struct DeviceBuffer {
    T* ptr = nullptr;
    size_t count = 0;
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer() { reset(); }
    void reset() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        count = 0;
    }
    // Ensures room for n elements; returns true when (re)allocated (contents
    // of a fresh allocation are undefined).  count is the capacity, which may
    // exceed n (grown_capacity).
    bool reserve(size_t n) {
        if (n <= count && ptr) return false;
        const size_t cap = grown_capacity(n, count);
        reset();
        hip_check(hipMalloc((void**)&ptr, cap * sizeof(T)), "hipMalloc");
        count = cap;
        return true;
    }
};

// Pinned host staging for uploads: reused once the copies that read it have
// completed (tracked with an event), so callers may free their arrays at once.
struct Staging {
    int32_t* host = nullptr;
    size_t count = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
    Staging() = default;
    Staging(const Staging&) = delete;
    Staging& operator=(const Staging&) = delete;
    ~Staging() {
        if (pending) (void)hipEventSynchronize(done);
        if (host) (void)hipHostFree(host);
        if (done) (void)hipEventDestroy(done);
    }
    int32_t* acquire(size_t n) {
        if (!done) hip_check(hipEventCreateWithFlags(&done, hipEventDisableTiming), "hipEventCreate");
        if (pending) {
            hip_check(hipEventSynchronize(done), "hipEventSynchronize");
            pending = false;
        }
        if (n > count || !host) {
            const size_t cap = grown_capacity(n, count);
            if (host) hip_check(hipHostFree(host), "hipHostFree");
            host = nullptr;
            count = 0;
            hip_check(hipHostMalloc((void**)&host, cap * sizeof(int32_t)), "hipHostMalloc");
            count = cap;
        }
        return host;
    }
    void copy(int32_t* dst, const int32_t* src, size_t n, hipStream_t s) {
        hip_check(hipMemcpyAsync(dst, src, n * sizeof(int32_t), hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync");
    }
    void finish(hipStream_t s) {
        hip_check(hipEventRecord(done, s), "hipEventRecord");
        pending = true;
    }
};

// A decode work list short enough to travel in the kernel arguments (fetched
// with the launch's other arguments, so no load precedes the table and q loads).
constexpr int DECODE_ARG_ITEMS = 200;
struct DecodeArgItems {
    int4 item[DECODE_ARG_ITEMS];
};

struct DecodeBatch {
    int32_t batch = 0, max_pages = 0;
    bool shared_pages = false;       // some page id is read by more than one sequence
    bool new_rows_private = false;   // no row's page at pos_b is read by another row
    std::vector<int32_t> positions;  // host copy (launch geometry)
    std::vector<uint32_t> page_mark, page_multi;  // per pool page: upload stamps (shared-page scan)
    uint32_t stamp = 0;
    uint64_t generation = 0;         // bumped by every new batch (work-list cache key)
    DeviceBuffer<int32_t> tables, pos;
    DeviceBuffer<int32_t> slots;     // per row: page * 16 + position % 16 (where its K/V row goes)
    // The decode work list last built for this batch, and what it was built for
    // (work_items = 0: longer than the kernel arguments hold).
    DecodeArgItems arg_list;
    uint64_t work_generation = ~0ull;
    int32_t work_tile = 0, work_tps = 0, work_items = 0;
    // Sequences whose first `pages` pages are the same physical pages
    // (prefix-cache hits), found at upload from the host tables.
    struct PrefixGroup {
        int32_t pages = 0;
        std::vector<int32_t> members;
    };
    std::vector<PrefixGroup> groups;
    bool own_rows_private = false;   // no page past a group's shared pages is read by two rows
    // The shared-prefix plan last built (see launch_decode_prefix; its list
    // is in arg_list) and what it was built for.
    uint64_t prefix_generation = ~0ull;
    int32_t prefix_heads = 0, prefix_ok = 0;
    int32_t main_tps = 0, main_waves = 0, main_items = 0, prefix_slots = 0;
    // Launches over uploaded or device-set batches so far, and how many took
    // the shared-prefix form (nitro_kvpool_decode_counts).
    uint64_t launches = 0, prefix_launches = 0;
};

struct PrefillBatch {
    int32_t batch = 0, max_pages = 0, total_rows = 0, max_tokens = 0;
    std::vector<int32_t> start_pos, num_tokens, row_off;
    DeviceBuffer<int32_t> tables, d_start, d_len, d_row_off;
    DeviceBuffer<int32_t> slots;      // per packed row: page*16 + row-in-page
    DeviceBuffer<int32_t> row_pos;    // per packed row: its position in the sequence
    DeviceBuffer<int32_t> work;       // per work item: (seq, first query) pairs
    int32_t work_items = 0;
    int32_t work_block_m = 0;         // query rows per work item the list was built for
    DeviceBuffer<int32_t> work_wide;  // the same for items of PREFILL_WIDE_ROWS rows
    int32_t work_items_wide = 0;
    int32_t max_pos = 0;              // largest position of any row
    // No table entry but a chunk row's own names the page that row lands on:
    // attention may then read the chunk's keys from the new rows (and older
    // keys from the pool) while the same launch writes the rows into the pool.
    bool append_in_launch = false;
    bool append_mixed = false;  // ... and some chunk starts after cached keys
    uint64_t append_launches = 0, fused_launches = 0;  // nitro_paged_attn_prefill_append calls / one-launch form
};

}  // namespace nitro

struct nitro_model;

struct nitro_kvpool {
    float* k = nullptr;
    float* v = nullptr;
    bool owned = false;
    int32_t num_pages = 0, num_layers = 0, kv_dim = 0;
    int device = 0;
    int num_cus = 256;  // compute units of the pool's device (launch geometry)
    hipStream_t last_stream = nullptr;
    nitro::DecodeBatch decode;
    nitro::PrefillBatch prefill;
    nitro::DeviceBuffer<float> partials;      // split-K (acc[hd], m, l) per (partial slot, head)
    nitro::DeviceBuffer<int32_t> counters;    // split-K arrivals per (b, head group), zero between launches
    nitro::DeviceBuffer<int32_t> bad_pages;   // [1] device error counter
    nitro::Staging decode_staging, prefill_staging;

    // Element strides every kernel addresses the pools with: row r of page p
    // in layer l starts at p * page_elems + l * layer_elems + r * kv_dim.
    // Paged pool [page][layer][16][kv_dim]: page_elems = L*16*kv_dim,
    // layer_elems = 16*kv_dim.  Contiguous cache [layer][seq_len][kv_dim]
    // (nitro_kvpool_wrap_contiguous): page_elems = 16*kv_dim, layer_elems =
    // seq_len*kv_dim, so page p of a layer is its rows 16p..16p+15.
    int64_t page_elems = 0, layer_elems = 0;
    int64_t page_stride() const { return page_elems; }
    int64_t layer_offset(int layer) const { return (int64_t)layer * layer_elems; }
};

namespace nitro {

// Kernel launchers (defined in the .hip files).
struct DecodeLaunch {
    const float* q;
    float* out;
    float* k_pool;  // written only by the fused append (k_new != nullptr)
    float* v_pool;
    const int32_t* tables;
    const int32_t* positions;
    // arg_items: the work list is the DecodeArgItems kernel argument, work_items
    // entries {b, split, first partial slot of b, ctx_b}, full items first;
    // otherwise item i is split i % num_splits of sequence i / num_splits
    // (context from positions).
    int32_t arg_items;
    int32_t work_items;
    float* partials;    // split-K (acc[hd], m, l) per (partial slot, head), pstride floats each
    int32_t* counters;  // per (b, head group): arrivals of the splits (zero between launches)
    const float* k_new;  // fused append: [batch][kv_dim] rows written at pos_b (nullptr: none)
    const float* v_new;
    int32_t* bad_pages;
    int64_t page_stride, layer_off;
    int32_t kv_dim, batch, n_heads, kv_mul, head_dim, max_pages, num_pages;
    int32_t tiles_per_split, num_splits;
    int32_t ctx_limit;  // contexts are clamped to this (the table's and the splits' reach)
    int32_t pstride;    // floats per partial, >= head_dim + 2
    int32_t waves;  // wavefronts per workgroup, 4..16
    int32_t stream_kv;  // non-temporal K/V loads (lines read once per launch)
    int32_t xcd_remap;  // keep the workgroups that read one K/V range on one XCD
    int32_t heads_per_wg;  // query heads of one KV head per workgroup (divides kv_mul)
    // Shared-prefix launch (heads_per_wg 1, work list in the arguments): the
    // list may hold member items, whose waves each take one sequence of a
    // prefix group over a chunk of its shared rows; see the decode kernel.
    int32_t members;
    float qscale;
};
// Head sizes attention takes: multiples of 4 up to 256 (kernels are built for
// 32, 64, 128 and 256 and mask the columns past a smaller head size).
inline bool attention_head_dim(int hd) { return hd >= 4 && hd <= 256 && hd % 4 == 0; }
// The kernel width a head size runs at (32, 64, 128 or 256).
int decode_padded_head_dim(int head_dim);
// Rows per decode tile for a head_dim (the unit split-K partitions).
int decode_tile_rows(int head_dim);
// Most query heads one decode workgroup serves for a head_dim (1, 2, 4 or 8).
int decode_max_heads_per_wg(int head_dim);
// Largest number of pages one split may cover (its block-table slice lives in LDS).
constexpr int DECODE_MAX_SPLIT_PAGES = 1024;
// The allocation-free decode entry's workspace: a file-scope device array of
// this many bytes, the first DECODE_STATIC_COUNTERS int32 arrival counters,
// the rest split-K partials.
constexpr size_t DECODE_STATIC_SCRATCH_BYTES = 8u << 20;
constexpr size_t DECODE_STATIC_COUNTERS = 65536;
// Address of that array on the current device (hipGetSymbolAddress on the
// first call per device, kept per device).
hipError_t decode_static_scratch(float** ptr);
hipError_t launch_paged_attn_decode(const DecodeLaunch& a, hipStream_t stream,
                                    const DecodeArgItems* items = nullptr);

hipError_t launch_kv_append_decode(float* k_pool, float* v_pool, const float* k, const float* v,
                                   const int32_t* tables, const int32_t* positions, int batch,
                                   int max_pages, int kv_dim, int64_t page_stride,
                                   int64_t layer_off, int num_pages, int32_t* bad_pages,
                                   hipStream_t stream);
// rms_norm folded into a Q8 product's input (weight == nullptr: none): the
// product reads the raw residual stream x and uses weight[k] * (inv * x[b][k])
// with inv = 1 / sqrtf(sum_p ss[p * ss_stride + b] / n + 1e-5).
struct Q8Norm {
    const float* weight = nullptr;
    const float* ss = nullptr;
    int nparts = 0, ss_stride = 0;
};
// Residual epilogue of a Q8 product into x: x += product, and per 16-row
// tile p of the output the sum of squares of each batch row's new entries
// goes to ss[p * ss_stride + b].
struct Q8Resid {
    float* ss = nullptr;
    int ss_stride = 0;
};
// RoPE and the K/V append folded into the wq/wk/wv product's epilogue
// (src/model_q8.cpp:594-617, 447-470): q and k are rotated with
// freq_real/imag[pos] of their batch row, q goes to its buffer, k and v
// straight into the pools at the row's slot (page * 16 + position % 16).
// Rows below `split` take position / slot from pos[0] / slot[0], the others
// from pos[1] / slot[1] at (row - split).  Page ids outside the pool are
// skipped and counted in bad_pages.
struct Q8Rope {
    const float* freq_real = nullptr;
    const float* freq_imag = nullptr;
    int head_dim = 0;
    float* k_pool = nullptr;
    float* v_pool = nullptr;
    int64_t page_stride = 0, layer_off = 0;
    int num_pages = 0;
    int32_t* bad_pages = nullptr;
    const int32_t* pos[2] = {nullptr, nullptr};
    const int32_t* slot[2] = {nullptr, nullptr};
    int split = 0;
};
// A Q8_0 matrix in the matrix-core tile layout: a record per (16-row tile,
// 32-k block) of 576 bytes, the 16 rows' block scales (floats) and then 64
// runs of 8 int8, run c holding weights 8*(c/16)..+8 of the block of row
// c%16 (one 8-byte load per lane of a wave is one 512-byte read); a tile's
// records in block order, tiles in row order; rows past d are zero.
// Products over more than 4 activation rows read this copy when given one.
struct Q8Tiled {
    const void* w[3] = {nullptr, nullptr, nullptr};
};
// Q8 products of up to this many activation rows run on VALU over the BlockQ8
// rows; products of more full rows read the tile layout when there is one.
constexpr int Q8_GEMV_MAX_BATCH = 4;
inline size_t q8_tiled_bytes(size_t d, size_t n) { return (d + 15) / 16 * (n / 32) * 576; }
// tiled = the tile layout of w (rows of BlockQ8, d x n)
hipError_t launch_q8_tile(const void* w, void* tiled, int d, int n, hipStream_t stream);
// Q8_0 matrix product (rows of BlockQ8, fp32 activations); last_block_only
// selects the reference's matmul_bulk semantics.
hipError_t launch_q8_matmul(const void* w, const float* x, float* out, int batch, int n, int d,
                            bool last_block_only, hipStream_t stream);
// x[b] += w . in[b] ([batch][d], in place) with the squares of the new x
// rows summed per 16 outputs into ss (ceil(d/16) partials per row, stride batch).
hipError_t launch_q8_residual(const void* w, const float* in, float* x, float* ss, int batch, int n, int d,
                              bool last_block_only, hipStream_t stream, const void* w_tiled = nullptr);
// wq/wk/wv sharing x and n: q = wq . rms_norm(x), k, v likewise, with the
// RoPE + K/V-append epilogue: q written to out_q [batch][dim], k and v to the
// pools (d = {dim, kv_dim, kv_dim}).
hipError_t launch_q8_qkv(const void* const* w, const float* x, float* out_q, const int* d, int batch, int n,
                         bool last_block_only, const Q8Norm& norm, const Q8Rope& rope, hipStream_t stream,
                         const Q8Tiled& tiled = Q8Tiled{});
// hb = silu(x . w1^T) * (x . w3^T), [batch][hidden] (src/model_q8.cpp:670-680).
hipError_t launch_q8_swiglu(const void* w1, const void* w3, const float* x, float* hb, int batch, int n,
                            int hidden, bool last_block_only, const Q8Norm& norm, hipStream_t stream,
                            const Q8Tiled& tiled = Q8Tiled{});
// Row-wise model kernels and the fp32 classifier product (model_kernels.hip).
// x[r] = table[tokens[r]]; with ss, ss[r] = the row's sum of squares (one
// partial per row for a following Q8Norm).
hipError_t launch_embed_rows(const float* table, const int32_t* tokens, float* x, int rows, int dim,
                             int vocab, int32_t* bad_tokens, float* ss, hipStream_t stream);
hipError_t launch_add_rmsnorm(float* x, const float* delta, const float* weight, float* out, int rows,
                              int dim, hipStream_t stream);
hipError_t launch_gather_last_rows(const float* x, const float* ffn, const int32_t* row_off,
                                  const int32_t* len, float* last, int chunks, int dim,
                                  hipStream_t stream);
hipError_t launch_swiglu(float* hb, const float* hb2, size_t n, hipStream_t stream);
hipError_t launch_f32_matmul(const float* w, const float* x, float* out, int batch, int n, int d,
                             hipStream_t stream);
// The classifier over rms_norm(x) with the norm folded in (nm as for the Q8
// products: weights, and the partial sums of squares the last residual
// product left): launched only where the flat kernel takes the batch
// (batch <= 4, batch * n <= 16384, n % 64 == 0); false (nothing launched)
// otherwise, and the caller normalises x and calls launch_f32_matmul.
bool launch_f32_matmul_norm(const float* w, const float* x, const Q8Norm& nm, float* out, int batch, int n, int d,
                            hipStream_t stream);
hipError_t launch_rope_kv_append(float* k_pool, float* v_pool, float* q, float* k, const float* v,
                                 const float* freq_real, const float* freq_imag,
                                 const int32_t* tables, const int32_t* positions,
                                 const int32_t* slots, const int32_t* row_pos, int rows,
                                 int max_pages, int dim, int kv_dim, int head_dim,
                                 int64_t page_stride, int64_t layer_off, int num_pages,
                                 int32_t* bad_pages, hipStream_t stream);
hipError_t launch_kv_scatter_rows(float* k_pool, float* v_pool, const float* k, const float* v,
                                  const int32_t* slots, int rows, int kv_dim, int64_t page_stride,
                                  int64_t layer_off, int num_pages, int32_t* bad_pages,
                                  hipStream_t stream);

// Continuous-scheduler step (scheduler_kernels.hip): resident block-table
// rows -> this step's decode tables, and the reference's argmax per row.
hipError_t launch_sched_tables(int32_t* store, int row_stride, const int32_t* desc, const int32_t* other,
                               int n_other, const int32_t* chunk_table, int32_t* tables, int32_t* positions,
                               int32_t* slots, int batch, int max_pages, hipStream_t stream);
hipError_t launch_argmax_rows(const float* logits, int32_t* next, int rows, int vocab, hipStream_t stream);

struct PrefillLaunch {
    const float* q;
    float* out;
    float* k_pool;  // read, and written by the appending form
    float* v_pool;
    // Appending form (bf16 matrix-core kernel only): the chunk's new K/V rows
    // [rows][kv_dim]; its keys are read from here and copied into the pool by
    // the same launch.  nullptr: every key is read from the pool.
    const float* k_new;
    const float* v_new;
    int32_t append_mixed;  // appending form: some chunk starts after cached keys (read from the pool)
    int32_t max_pos;  // largest position of the batch
    const int32_t* tables;
    const int32_t* start_pos;
    const int32_t* num_tokens;
    const int32_t* row_off;
    const int32_t* work;  // pairs (seq, first query row of the chunk)
    int32_t* bad_pages;
    int64_t page_stride, layer_off;
    int32_t kv_dim, n_heads, kv_mul, head_dim, max_pages, num_pages, work_items;
    float qscale;
    int32_t kernel;     // PREFILL_KERNEL_*: which form runs where several exist
    int32_t item_rows;  // query rows per work item of `work` (64, or PREFILL_WIDE_ROWS)
};
// Query rows per work item of the wide list (the default kernel at hd 128).
constexpr int32_t PREFILL_WIDE_ROWS = 128;
// Whether a launch of this kernel / head_dim takes the wide work list.
bool prefill_uses_wide_items(int32_t kernel, int32_t head_dim);
// Whether this kernel / head_dim has the appending form (PrefillLaunch::k_new)
// for a batch whose largest position is max_pos (its table rows fit in LDS).
bool prefill_appends_in_launch(int32_t kernel, int32_t head_dim, int32_t max_pos, int64_t page_stride);
constexpr int32_t PREFILL_KERNEL_DEFAULT = 0;   // bf16 matrix cores at fp32 accuracy (hd <= 128)
constexpr int32_t PREFILL_KERNEL_VALU = 1;      // fp32 VALU FMAs
constexpr int32_t PREFILL_KERNEL_MFMA_F32 = 2;  // fp32 matrix cores (v_mfma_f32_16x16x4_f32)
// Query rows per prefill work item.
int prefill_block_m(int head_dim);
hipError_t launch_paged_attn_prefill(const PrefillLaunch& a, hipStream_t stream);

}  // namespace nitro

namespace nitro {

// Makes pool->decode a batch whose tables [batch][max_pages] and positions
// the caller writes on the device (stream-ordered before the next launch);
// positions is the host copy (launch geometry).  Returns the device arrays.
void set_device_decode_batch(nitro_kvpool* pool, int batch, int max_pages, const int32_t* positions,
                             bool shared_pages, int32_t** tables, int32_t** device_positions,
                             int32_t** device_slots);
// Hands over the host's copy of that batch's tables ([batch][max_pages], the
// same rows the caller writes on the device) so that its decode launches can
// read shared prefixes once per member set, as after an upload.
void set_device_decode_groups(nitro_kvpool* pool, const int32_t* tables, int max_pages);

// One forward over prefill rows [0, prefill_rows) and decode rows
// [prefill_rows, prefill_rows + decode_rows), tokens on the device.  With
// prefill_as_decode the decode batch in pool->decode holds every row (a
// chunk row is a decode row at its own position over the chunk's table);
// otherwise the prefill rows are the one-sequence batch in pool->prefill and
// pool->decode holds the decode rows.  Logits and argmax go out for the
// decode rows, preceded by the prefill chunk's last row when prefill_logits.
void forward_mixed(nitro_model* m, nitro_kvpool* pool, const int32_t* tokens, int prefill_rows,
                   int decode_rows, bool prefill_as_decode, bool prefill_logits, float* logits,
                   int32_t* next, int semantics, hipStream_t stream);
// Dimensions the scheduler needs: {dim, vocab, seq_len, n_layers, kv_dim}.
void model_dims(const nitro_model* m, int32_t* dims);

}  // namespace nitro
