// Host half of the continuous scheduler and its C ABI (declared in
// include/nitro_paged_attn.h).  Statement-level correspondence with
// src/pagedMemory.hpp:303-399 is noted inline.
#include "scheduler.hpp"

#include <algorithm>
#include <string>

#include "capi_common.hpp"
#include "nitro_paged_attn.h"

namespace nitro {

ContinuousScheduler::ContinuousScheduler(BlockManager& bm, int max_tokens_per_batch, int max_generated)
    : bm_(bm), budget_(max_tokens_per_batch), max_generated_(max_generated) {
    require(max_tokens_per_batch > 0, ERR_INVALID_ARGUMENT, "max_tokens_per_batch must be positive");
    require(max_generated > 0, ERR_INVALID_ARGUMENT, "max_generated must be positive");
}

Request& ContinuousScheduler::add_request(int req_id, const int32_t* prompt, int n) {
    require(prompt != nullptr && n > 0, ERR_INVALID_ARGUMENT, "a request needs a non-empty prompt");
    require(find(req_id) == nullptr, ERR_INVALID_ARGUMENT, "request id already in use");
    require(!planned_, ERR_INVALID_ARGUMENT, "a planned step has not been committed");
    if (seq_len_ > 0 && (long long)n + max_generated_ - 1 > seq_len_)
        throw Error(ERR_INVALID_ARGUMENT, "a prompt of " + std::to_string(n) + " tokens plus " +
                                              std::to_string(max_generated_) + " generated ones does not fit " +
                                              "the model's seq_len of " + std::to_string(seq_len_));
    if (vocab_ > 0)
        for (int i = 0; i < n; i++)
            require(prompt[i] >= 0 && prompt[i] < vocab_, ERR_INVALID_ARGUMENT,
                    "prompt token outside the vocabulary");
    requests_.push_back(std::make_unique<Request>(req_id, prompt, n));
    Request* r = requests_.back().get();
    r->next_token_to_process = r->prompt_tokens[0];  // :310
    waiting_.push_back(r);                             // :311
    return *r;
}

void ContinuousScheduler::set_limits(int seq_len, int vocab) {
    require(seq_len >= 0 && vocab >= 0, ERR_INVALID_ARGUMENT, "limits must not be negative");
    seq_len_ = seq_len;
    vocab_ = vocab;
}

const StepPlan& ContinuousScheduler::plan() {
    require(!planned_, ERR_INVALID_ARGUMENT, "the previous step has not been committed");
    KVBlock_Manager& mem = bm_.mem;
    PrefixCacheManager& cache = bm_.cache;
    StepPlan& p = plan_;
    p = StepPlan();
    // :317-326 release what finished last step (erase keeps the order)
    std::vector<Request*> kept;
    kept.reserve(running_.size());
    for (Request* r : running_) {
        if (r->is_finished) {
            r->seq.release(mem, cache);
            p.released.push_back(r);
        } else {
            kept.push_back(r);
        }
    }
    running_.swap(kept);
    int budget = budget_;  // :327
    // :332-340 one decode row per running request
    for (Request* r : running_) {
        if (r->is_prefill_done) {
            p.decode_tokens.push_back(r->next_token_to_process);
            p.decode_positions.push_back(r->seq.logical_token_count);
            p.decode.push_back(r);
            budget -= 1;
        }
    }
    // :341-377 at most one prefill chunk, from the queue head
    if (!waiting_.empty() && budget > 0) {
        Request* r = waiting_.front();
        const int n = (int)r->prompt_tokens.size();
        const size_t pages_before = r->seq.block_table.size();
        r->prefill_idx = r->seq.prefix_walk(r->prompt_tokens.data(), n, r->prefill_idx,
                                            /*require_empty_buffer=*/true, mem, cache);  // :346-359
        if (r->seq.block_table.size() != pages_before) p.grown.push_back(r);
        const int remaining = n - r->prefill_idx;
        const int chunk = std::min(remaining, budget);
        if (chunk > 0) {
            p.prefill_tokens.assign(r->prompt_tokens.begin() + r->prefill_idx,
                                    r->prompt_tokens.begin() + r->prefill_idx + chunk);
            p.prefill = r;
        }
        if (r->prefill_idx + chunk == n) {
            r->is_prefill_done = true;
            running_.push_back(r);
            waiting_.pop_front();
        } else {
            r->prefill_idx += chunk;
        }
    }
    // forward_prefill_chunk's allocations (src/model_q8.cpp:428-430), then
    // forward_decode_batch's (:578-582)
    if (p.prefill) {
        Sequence& q = p.prefill->seq;
        p.prefill_start = q.logical_token_count;
        p.prefill_finishes = p.prefill->is_prefill_done;
        const size_t pages_before = q.block_table.size();
        for (int32_t t : p.prefill_tokens) q.allocate_next_token(t, mem, cache);
        if (q.block_table.size() != pages_before &&
            (p.grown.empty() || p.grown.back() != p.prefill))
            p.grown.push_back(p.prefill);
    }
    for (size_t b = 0; b < p.decode.size(); b++) {
        Sequence& q = p.decode[b]->seq;
        const size_t pages_before = q.block_table.size();
        q.allocate_next_token(p.decode_tokens[b], mem, cache);
        if (q.block_table.size() != pages_before) p.grown.push_back(p.decode[b]);
    }
    planned_ = true;
    return p;
}

void ContinuousScheduler::commit(int32_t prefill_token, const int32_t* decode_tokens, int n) {
    require(planned_, ERR_INVALID_ARGUMENT, "no planned step to commit");
    StepPlan& p = plan_;
    require(n == (int)p.decode.size(), ERR_INVALID_ARGUMENT, "one token per decode row is required");
    require(n == 0 || decode_tokens != nullptr, ERR_INVALID_ARGUMENT, "null decode tokens");
    // :380-386
    if (p.prefill && p.prefill_finishes) {
        p.prefill->next_token_to_process = prefill_token;
        p.prefill->generated_tokens.push_back(prefill_token);
    }
    // :387-397
    for (int b = 0; b < n; b++) {
        Request* r = p.decode[b];
        r->next_token_to_process = decode_tokens[b];
        r->generated_tokens.push_back(decode_tokens[b]);
        if ((int)r->generated_tokens.size() >= max_generated_) r->is_finished = true;
    }
    planned_ = false;
}

Request* ContinuousScheduler::find(int req_id) {
    for (auto& r : requests_)
        if (r->req_id == req_id) return r.get();
    return nullptr;
}

const Request* ContinuousScheduler::find(int req_id) const {
    for (auto& r : requests_)
        if (r->req_id == req_id) return r.get();
    return nullptr;
}

void ContinuousScheduler::reject_head() {
    require(!planned_, ERR_INVALID_ARGUMENT, "a planned step has not been committed");
    require(!waiting_.empty(), ERR_INVALID_ARGUMENT, "no queued request");
    Request* r = waiting_.front();
    waiting_.pop_front();
    if (!r->seq.block_table.empty()) r->seq.release(bm_.mem, bm_.cache);
    r->is_finished = true;
}

bool ContinuousScheduler::droppable(int req_id) const {
    const Request* r = find(req_id);
    if (!r || !r->is_finished || planned_) return false;
    return std::find(waiting_.begin(), waiting_.end(), r) == waiting_.end() &&
           std::find(running_.begin(), running_.end(), r) == running_.end();
}

void ContinuousScheduler::drop(int req_id) {
    require(!planned_, ERR_INVALID_ARGUMENT, "a planned step has not been committed");
    auto it = std::find_if(requests_.begin(), requests_.end(),
                           [&](const std::unique_ptr<Request>& r) { return r->req_id == req_id; });
    require(it != requests_.end(), ERR_INVALID_ARGUMENT, "unknown request id");
    require(droppable(req_id), ERR_INVALID_ARGUMENT,
            "only a finished request that a later step has released can be dropped");
    requests_.erase(it);
}

std::vector<int32_t> ContinuousScheduler::state_words() const {
    std::vector<int32_t> o;
    o.push_back((int32_t)running_.size());
    for (const Request* r : running_) o.push_back(r->req_id);
    o.push_back((int32_t)waiting_.size());
    for (const Request* r : waiting_) o.push_back(r->req_id);
    o.push_back((int32_t)requests_.size());
    for (const auto& up : requests_) {
        const Request& r = *up;
        o.push_back(r.req_id);
        o.push_back(r.prefill_idx);
        o.push_back(r.is_prefill_done ? 1 : 0);
        o.push_back(r.is_finished ? 1 : 0);
        o.push_back(r.next_token_to_process);
        o.push_back((int32_t)r.generated_tokens.size());
        o.insert(o.end(), r.generated_tokens.begin(), r.generated_tokens.end());
        o.push_back(r.seq.logical_token_count);
        o.push_back((int32_t)(uint32_t)(r.seq.current_hash & 0xffffffffu));
        o.push_back((int32_t)(uint32_t)(r.seq.current_hash >> 32));
        o.push_back((int32_t)r.seq.token_buffer.size());
        o.insert(o.end(), r.seq.token_buffer.begin(), r.seq.token_buffer.end());
        o.push_back((int32_t)r.seq.block_table.size());
        o.insert(o.end(), r.seq.block_table.begin(), r.seq.block_table.end());
    }
    return o;
}

}  // namespace nitro

using namespace nitro;

namespace {

template <class T>
void copy_out(const std::vector<T>& v, T* out, int32_t cap, int32_t* n) {
    require(n != nullptr, ERR_INVALID_ARGUMENT, "null count pointer");
    *n = (int32_t)v.size();
    require(cap >= (int32_t)v.size() || out == nullptr, ERR_INVALID_ARGUMENT,
            "output buffer too small (the required size is in *n)");
    if (out) std::copy(v.begin(), v.end(), out);
}

void require_sched(const nitro_scheduler* s) { require(s != nullptr, ERR_INVALID_ARGUMENT, "null scheduler"); }

}  // namespace

extern "C" {

int nitro_sched_create(nitro_block_manager* bm, int32_t max_tokens_per_batch, int32_t max_generated,
                       nitro_scheduler** out) {
    return guarded([&] {
        require(out != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        *out = nullptr;
        require(bm != nullptr, ERR_INVALID_ARGUMENT, "null block manager");
        *out = new nitro_scheduler(bm, bm->bm, max_tokens_per_batch, max_generated);
    });
}

int nitro_sched_destroy(nitro_scheduler* s) {
    if (!s) return OK;
    return guarded([&] { delete s; });
}

int nitro_sched_add_request(nitro_scheduler* s, int32_t req_id, const int32_t* prompt, int32_t n) {
    return guarded([&] {
        require_sched(s);
        s->host.add_request(req_id, prompt, n);
    });
}

int nitro_sched_set_limits(nitro_scheduler* s, int32_t seq_len, int32_t vocab) {
    return guarded([&] {
        require_sched(s);
        s->host.set_limits(seq_len, vocab);
    });
}

int nitro_sched_has_active_requests(const nitro_scheduler* s, int32_t* active) {
    return guarded([&] {
        require_sched(s);
        require(active != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        *active = s->host.has_active_requests() ? 1 : 0;
    });
}

int nitro_sched_plan(nitro_scheduler* s, int32_t* prefill, int32_t* decode_ids, int32_t* decode_tokens,
                     int32_t* decode_positions, int32_t cap, int32_t* n_decode) {
    return guarded([&] {
        require_sched(s);
        require(prefill != nullptr && n_decode != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        require(s->host.running().size() <= (size_t)std::max(cap, 0) ||
                    (decode_ids == nullptr && decode_tokens == nullptr && decode_positions == nullptr),
                ERR_INVALID_ARGUMENT, "decode arrays shorter than the running batch");
        const StepPlan& p = s->host.plan();
        prefill[0] = p.prefill ? p.prefill->req_id : -1;
        prefill[1] = (int32_t)p.prefill_tokens.size();
        prefill[2] = p.prefill_start;
        prefill[3] = p.prefill_finishes ? 1 : 0;
        const int B = (int)p.decode.size();
        *n_decode = B;
        for (int b = 0; b < B; b++) {
            if (decode_ids) decode_ids[b] = p.decode[b]->req_id;
            if (decode_tokens) decode_tokens[b] = p.decode_tokens[b];
            if (decode_positions) decode_positions[b] = p.decode_positions[b];
        }
    });
}

int nitro_sched_commit(nitro_scheduler* s, int32_t prefill_token, const int32_t* decode_tokens, int32_t n) {
    return guarded([&] {
        require_sched(s);
        s->host.commit(prefill_token, decode_tokens, n);
    });
}

int nitro_sched_state(const nitro_scheduler* s, int32_t* words, int32_t cap, int32_t* n) {
    return guarded([&] {
        require_sched(s);
        copy_out(s->host.state_words(), words, cap, n);
    });
}

int nitro_sched_generated(const nitro_scheduler* s, int32_t req_id, int32_t* tokens, int32_t cap, int32_t* n) {
    return guarded([&] {
        require_sched(s);
        const Request* r = s->host.find(req_id);
        require(r != nullptr, ERR_INVALID_ARGUMENT, "unknown request id");
        copy_out(r->generated_tokens, tokens, cap, n);
    });
}

int nitro_sched_request_status(const nitro_scheduler* s, int32_t req_id, int32_t* status) {
    return guarded([&] {
        require_sched(s);
        require(status != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        const Request* r = s->host.find(req_id);
        require(r != nullptr, ERR_INVALID_ARGUMENT, "unknown request id");
        status[0] = r->prefill_idx;
        status[1] = r->is_prefill_done ? 1 : 0;
        status[2] = r->is_finished ? 1 : 0;
        status[3] = r->next_token_to_process;
        status[4] = (int32_t)r->generated_tokens.size();
        status[5] = r->seq.logical_token_count;
    });
}

int nitro_sched_drop_request(nitro_scheduler* s, int32_t req_id) {
    return guarded([&] {
        require_sched(s);
        s->host.drop(req_id);
    });
}

}  // extern "C"
