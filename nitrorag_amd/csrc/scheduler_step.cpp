// Device half of the continuous scheduler: nitro_sched_step and
// nitro_sched_last_logits (declared in include/nitro_paged_attn.h).
//
// One step = the host plan (scheduler.cpp), one upload of the step's small
// inputs, one forward over the prefill chunk's rows and the decode rows
// together, the argmax on the device, a read-back of one token per row, the
// host commit.  Block tables stay on the device: every request that holds
// pages owns a row of `store` (row_stride = pages of a full sequence) that
// receives only the entries its sequence gained this step; the decode
// kernels' dense [batch][max_pages] tables are written from those rows on
// the device (launch_sched_tables).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "capi_common.hpp"
#include "device_pool.hpp"
#include "nitro_paged_attn.h"
#include "scheduler.hpp"

namespace nitro {

struct SchedDevice {
    nitro_kvpool* pool = nullptr;
    nitro_model* model = nullptr;
    int device = 0;
    int row_stride = 0;                 // pages per resident row
    int rows = 0;                       // resident rows allocated
    std::vector<int> free_rows;         // LIFO
    DeviceBuffer<int32_t> store;        // [rows][row_stride]
    DeviceBuffer<int32_t> step_in;      // tokens, decode descriptors, other entries
    DeviceBuffer<float> logits;         // [out_rows][vocab]
    DeviceBuffer<int32_t> next;         // [out_rows]
    Staging staging;
    int32_t* readback = nullptr;        // pinned, next tokens
    size_t readback_count = 0;
    int last_rows = 0;
    int vocab = 0;
    std::vector<uint32_t> page_mark;    // shared-page scan stamps
    uint32_t stamp = 0;
    std::vector<int32_t> host_tables;   // the decode batch's tables, when pages are shared

    ~SchedDevice() {
        if (readback) (void)hipHostFree(readback);
    }

    int take_row(hipStream_t s) {
        if (free_rows.empty()) grow(std::max(16, 2 * rows), s);
        const int r = free_rows.back();
        free_rows.pop_back();
        return r;
    }

    void grow(int n, hipStream_t s) {
        DeviceBuffer<int32_t> bigger;
        bigger.reserve((size_t)n * row_stride);
        if (rows > 0)
            hip_check(hipMemcpyAsync(bigger.ptr, store.ptr, sizeof(int32_t) * (size_t)rows * row_stride,
                                     hipMemcpyDeviceToDevice, s),
                      "hipMemcpyAsync(resident tables)");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        std::swap(store.ptr, bigger.ptr);
        std::swap(store.count, bigger.count);
        for (int r = n - 1; r >= rows; r--) free_rows.push_back(r);
        rows = n;
    }
};

namespace {

// Prefill chunks of at most this many rows run as rows of the decode batch.
constexpr int PREFILL_AS_DECODE_MAX_ROWS = 32;

void free_device(SchedDevice* d) { delete d; }

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// True when some page appears in more than one decode row's table (prefix
// sharing): the decode kernel then keeps its K/V loads cacheable.
bool rows_share_pages(SchedDevice& d, const StepPlan& p, int num_pages) {
    if ((int)d.page_mark.size() < num_pages) d.page_mark.assign(num_pages, 0);
    if (++d.stamp == 0) {
        std::fill(d.page_mark.begin(), d.page_mark.end(), 0);
        d.stamp = 1;
    }
    for (const Request* r : p.decode)
        for (int32_t page : r->seq.block_table) {
            if (d.page_mark[page] == d.stamp) return true;
            d.page_mark[page] = d.stamp;
        }
    return false;
}

// Requests the model cannot run are finished with the tokens they have,
// before any state changes, instead of failing this and every later step:
// a running request that would decode at or past seq_len or whose next token
// lies outside the vocabulary; a queue head whose prompt holds a token outside
// the vocabulary or would decode past seq_len before it finishes (its prompt
// of n tokens ends at position n + max_generated - 2).  The reference has no
// such check (its pools would be indexed out of bounds).
void retire_unrunnable(ContinuousScheduler& h, SchedDevice& d, int seq_len, int vocab) {
    for (Request* r : h.running()) {
        if (r->is_finished) continue;
        if (r->seq.logical_token_count >= seq_len || r->next_token_to_process < 0 ||
            r->next_token_to_process >= vocab)
            r->is_finished = true;  // released at the start of this step's plan
    }
    while (const Request* head = h.waiting_head()) {
        bool ok = (long long)head->prompt_tokens.size() + h.max_generated() - 1 <= seq_len;
        for (int32_t t : head->prompt_tokens) ok &= t >= 0 && t < vocab;
        if (ok) break;
        Request* r = h.find(head->req_id);
        if (r->slot >= 0) d.free_rows.push_back(r->slot);  // a resident table row, if it had one
        r->slot = -1;
        r->pages_on_device = 0;
        h.reject_head();
    }
}

}  // namespace
}  // namespace nitro

using namespace nitro;

extern "C" {

int nitro_sched_step(nitro_scheduler* sched, nitro_model* model, nitro_kvpool* pool, int32_t semantics,
                     void* stream) {
    return guarded([&] {
        require(sched != nullptr && model != nullptr && pool != nullptr, ERR_INVALID_ARGUMENT, "null handle");
        require(semantics == NITRO_Q8_FULL_ROWS || semantics == NITRO_Q8_LAST_BLOCK, ERR_INVALID_ARGUMENT,
                "unknown Q8 semantics");
        ContinuousScheduler& h = sched->host;
        int32_t dims[5];
        model_dims(model, dims);
        const int vocab = dims[1], seq_len = dims[2];
        require(pool->num_layers == dims[3] && pool->kv_dim == dims[4], ERR_INVALID_ARGUMENT,
                "pool layers / kv_dim do not match the model");
        require(h.block_manager().mem.total_blocks() <= pool->num_pages, ERR_INVALID_ARGUMENT,
                "the block manager has more pages than the pool");
        hipStream_t s = as_stream(stream);
        if (!sched->dev) {
            auto* d = new SchedDevice();
            d->pool = pool;
            d->model = model;
            d->row_stride = (seq_len + BLOCK_SIZE - 1) / BLOCK_SIZE;
            d->vocab = vocab;
            hip_check(hipGetDevice(&d->device), "hipGetDevice");
            sched->dev = d;
            sched->dev_free = free_device;
        }
        SchedDevice& d = *sched->dev;
        require(d.pool == pool && d.model == model, ERR_INVALID_ARGUMENT,
                "a scheduler steps one model over one pool (those of its first step)");
        h.set_limits(seq_len, vocab);
        retire_unrunnable(h, d, seq_len, vocab);
        if (!h.has_active_requests()) return;

        const StepPlan& p = h.plan();
        // From here on a failure leaves the step planned: the scheduler can
        // only be destroyed (as after the reference's exit).
        for (Request* r : p.released) {
            if (r->slot >= 0) d.free_rows.push_back(r->slot);
            r->slot = -1;
            r->pages_on_device = 0;
        }
        const int P = (int)p.prefill_tokens.size(), B = (int)p.decode.size();
        // A short chunk rides in the decode batch: each of its rows is a decode
        // row at its own position over the chunk's table (one RoPE/append and
        // one attention launch per layer for all rows).  Long chunks keep the
        // prefill kernel, which reads each K/V page once for many query rows.
        const bool chunk_rows = P > 0 && P <= PREFILL_AS_DECODE_MAX_ROWS;
        const int R = (chunk_rows ? P : 0) + B;  // rows of the decode batch
        // New table entries: a decode row's single new page travels in its
        // descriptor, the rest in the `other` list.
        std::vector<int32_t> desc(4 * (size_t)R), other;
        std::vector<int32_t> positions(R);
        const int c0 = chunk_rows ? P : 0;  // first request row in the batch
        for (int i = 0; i < c0; i++) {
            desc[4 * i] = -1;
            desc[4 * i + 1] = positions[i] = p.prefill_start + i;
            desc[4 * i + 2] = -1;
            desc[4 * i + 3] = 0;
        }
        for (int b = 0; b < B; b++) {
            Request* r = p.decode[b];
            if (r->slot < 0) r->slot = d.take_row(s);
            const int n = (int)r->seq.block_table.size();
            require(n - r->pages_on_device <= 1 && n <= d.row_stride, ERR_BAD_BLOCK_TABLE,
                    "a decode row gained more than one page");
            int32_t* e = &desc[4 * (size_t)(c0 + b)];
            e[0] = r->slot;
            e[1] = positions[c0 + b] = p.decode_positions[b];
            e[2] = n > r->pages_on_device ? r->pages_on_device : -1;
            e[3] = n > r->pages_on_device ? r->seq.block_table[n - 1] : 0;
            r->pages_on_device = n;
        }
        for (Request* r : p.grown) {
            if (std::find(p.decode.begin(), p.decode.end(), r) != p.decode.end()) continue;
            if (r->slot < 0) r->slot = d.take_row(s);
            const int n = (int)r->seq.block_table.size();
            require(n <= d.row_stride, ERR_BAD_BLOCK_TABLE, "a block table is longer than seq_len allows");
            for (int j = r->pages_on_device; j < n; j++) {
                other.push_back(r->slot * d.row_stride + j);
                other.push_back(r->seq.block_table[j]);
            }
            r->pages_on_device = n;
        }
        const int n_other = (int)other.size() / 2;
        const int out_rows = B + (p.prefill_finishes ? 1 : 0);
        d.last_rows = 0;
        if (P + B == 0 && n_other == 0) {
            h.commit(0, nullptr, 0);
            return;
        }
        const std::vector<int32_t> no_table;
        const std::vector<int32_t>& chunk_table = chunk_rows ? p.prefill->seq.block_table : no_table;

        // One upload: tokens (prefill rows, then decode rows), descriptors,
        // other entries, the chunk's table.
        const size_t n_in = (size_t)P + B + desc.size() + other.size() + chunk_table.size();
        d.step_in.reserve(n_in);
        int32_t* hin = d.staging.acquire(n_in);
        int32_t* w = hin;
        w = std::copy(p.prefill_tokens.begin(), p.prefill_tokens.end(), w);
        w = std::copy(p.decode_tokens.begin(), p.decode_tokens.end(), w);
        w = std::copy(desc.begin(), desc.end(), w);
        w = std::copy(other.begin(), other.end(), w);
        std::copy(chunk_table.begin(), chunk_table.end(), w);
        d.staging.copy(d.step_in.ptr, hin, n_in, s);
        d.staging.finish(s);
        const int32_t* d_tokens = d.step_in.ptr;
        const int32_t* d_desc = d.step_in.ptr + P + B;
        const int32_t* d_other = d_desc + desc.size();
        const int32_t* d_chunk_table = d_other + other.size();

        int32_t* d_tables = nullptr;
        int32_t* d_positions = nullptr;
        int32_t* d_slots = nullptr;
        int max_pages = 1;
        if (R > 0) {
            for (int i = 0; i < R; i++) max_pages = std::max(max_pages, positions[i] / BLOCK_SIZE + 1);
            // chunk rows read one table (and may share prefix hits with decode rows)
            const bool shared = c0 > 0 || rows_share_pages(d, p, pool->num_pages);
            set_device_decode_batch(pool, R, max_pages, positions.data(), shared, &d_tables, &d_positions,
                                    &d_slots);
            if (shared && R > 1) {
                // The host holds every row's table too: sequences that begin
                // with the same pages (a shared prompt, the rows of one chunk)
                // then read those rows once per member set in each layer.
                d.host_tables.assign((size_t)R * max_pages, 0);
                for (int i = 0; i < R; i++) {
                    const std::vector<int32_t>& t =
                        i < c0 ? p.prefill->seq.block_table : p.decode[i - c0]->seq.block_table;
                    const int n = positions[i] / BLOCK_SIZE + 1;
                    require((int)t.size() >= n, ERR_BAD_BLOCK_TABLE, "a row's table ends before its position");
                    std::copy(t.begin(), t.begin() + n, d.host_tables.begin() + (size_t)i * max_pages);
                }
                set_device_decode_groups(pool, d.host_tables.data(), max_pages);
            }
        }
        hip_check(launch_sched_tables(d.store.ptr, d.row_stride, d_desc, d_other, n_other, d_chunk_table,
                                      d_tables, d_positions, d_slots, R, max_pages, s),
                  "sched_tables launch");
        if (P > 0 && !chunk_rows) {
            const std::vector<int32_t>& t = p.prefill->seq.block_table;
            const int32_t start = p.prefill_start, len = P;
            require(nitro_prefill_batch_upload(pool, t.data(), &start, &len, 1, (int32_t)t.size(), stream) ==
                        NITRO_OK,
                    ERR_INVALID_ARGUMENT, nitro_last_error());
        }
        if (P + B > 0) {
            d.logits.reserve((size_t)std::max(out_rows, 1) * vocab);
            d.next.reserve(std::max(out_rows, 1));
            forward_mixed(model, pool, d_tokens, P, B, chunk_rows, p.prefill_finishes, d.logits.ptr, d.next.ptr,
                          semantics, s);
        }
        if ((size_t)out_rows > d.readback_count) {
            const size_t cap = grown_capacity(out_rows, d.readback_count);
            if (d.readback) hip_check(hipHostFree(d.readback), "hipHostFree");
            d.readback = nullptr;
            d.readback_count = 0;
            hip_check(hipHostMalloc((void**)&d.readback, sizeof(int32_t) * cap), "hipHostMalloc");
            d.readback_count = cap;
        }
        if (out_rows > 0)
            hip_check(hipMemcpyAsync(d.readback, d.next.ptr, sizeof(int32_t) * out_rows, hipMemcpyDeviceToHost, s),
                      "hipMemcpyAsync(next tokens)");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        pool->last_stream = s;
        d.last_rows = out_rows;
        const int first = p.prefill_finishes ? 1 : 0;
        h.commit(first ? d.readback[0] : 0, d.readback + first, B);
    });
}

int nitro_argmax(const float* logits, int32_t rows, int32_t vocab, int32_t* out, void* stream) {
    return guarded([&] {
        require(logits != nullptr && out != nullptr, ERR_INVALID_ARGUMENT, "null pointer");
        require(rows >= 0 && vocab > 0, ERR_INVALID_ARGUMENT, "rows must be >= 0 and vocab > 0");
        hip_check(launch_argmax_rows(logits, out, rows, vocab, as_stream(stream)), "argmax launch");
    });
}

int nitro_sched_last_logits(const nitro_scheduler* sched, float* logits, int32_t cap_rows, int32_t* rows) {
    return guarded([&] {
        require(sched != nullptr && rows != nullptr, ERR_INVALID_ARGUMENT, "null pointer");
        const SchedDevice* d = sched->dev;
        *rows = d ? d->last_rows : 0;
        if (!d || d->last_rows == 0 || logits == nullptr) return;
        require(cap_rows >= d->last_rows, ERR_INVALID_ARGUMENT, "output buffer too small (rows in *rows)");
        hip_check(hipMemcpy(logits, d->logits.ptr, sizeof(float) * (size_t)d->last_rows * d->vocab,
                            hipMemcpyDeviceToHost),
                  "hipMemcpy(logits)");
    });
}

}  // extern "C"
