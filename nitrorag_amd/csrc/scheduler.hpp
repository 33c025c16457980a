// Host half of the continuous scheduler (C++17, no device code).
//
// Request and Continuous_Scheduler of the reference (src/pagedMemory.hpp:
// 287-399) with the two forward calls split out of step():
//   plan()   does everything step() does before forward_prefill_chunk and
//            forward_decode_batch — release the requests that finished, one
//            decode row per running request, admission of the queue head with
//            its prefix-cache walk and a chunk sized by the token budget — and
//            then the allocate_next_token calls those two forwards begin with
//            (src/model_q8.cpp:428-430, then :578-582 in batch order, which is
//            what the reference does with one OpenMP thread);
//   commit() applies the argmax tokens of the two forwards (:380-397).
// Block ids, prefix-cache state, chunking and finish decisions therefore come
// out exactly as the reference's.  The device half (the mixed prefill +
// decode forward over device-resident block tables) is in scheduler_step.cpp.
#pragma once

#include <cstdint>
#include <deque>
#include <memory>
#include <vector>

#include "paged_memory.hpp"

namespace nitro {

struct Request {  // src/pagedMemory.hpp:287-300
    Request(int id, const int32_t* prompt, int n) : req_id(id), prompt_tokens(prompt, prompt + n), seq(id) {}
    int req_id;
    std::vector<int32_t> prompt_tokens;
    std::vector<int32_t> generated_tokens;
    int prefill_idx = 0;
    bool is_prefill_done = false;
    bool is_finished = false;
    int32_t next_token_to_process = -1;
    Sequence seq;
    // Device half: row of the device-resident block tables and how many of
    // seq.block_table's entries that row already holds.
    int slot = -1;
    int pages_on_device = 0;
};

// The forward work of one step: at most one prefill chunk and the decode rows
// in running order, plus the requests released at its start.
struct StepPlan {
    Request* prefill = nullptr;
    std::vector<int32_t> prefill_tokens;
    int prefill_start = 0;
    bool prefill_finishes = false;  // the chunk completes the prompt (its argmax is used)
    std::vector<Request*> decode;
    std::vector<int32_t> decode_tokens, decode_positions;
    std::vector<Request*> released;
    // Requests whose block tables grew this step (prefix hits or allocations).
    std::vector<Request*> grown;
};

class ContinuousScheduler {
  public:
    ContinuousScheduler(BlockManager& bm, int max_tokens_per_batch, int max_generated);
    ContinuousScheduler(const ContinuousScheduler&) = delete;
    ContinuousScheduler& operator=(const ContinuousScheduler&) = delete;

    // add_request (:309-312): the first token to process is prompt[0].
    // With limits set, a prompt holding a token outside [0, vocab) or whose
    // generation would decode at or past seq_len (its last decode sits at
    // position n + max_generated - 2) is refused; the reference has no limit.
    Request& add_request(int req_id, const int32_t* prompt, int n);
    // The model's seq_len and vocabulary size (0 = no limit).
    void set_limits(int seq_len, int vocab);
    bool has_active_requests() const { return !waiting_.empty() || !running_.empty(); }  // :313-315
    // The queue head (the only request plan() may prefill), or null.
    const Request* waiting_head() const { return waiting_.empty() ? nullptr : waiting_.front(); }
    const std::vector<Request*>& running() const { return running_; }

    const StepPlan& plan();
    // prefill_token is used when the plan's chunk finishes its prompt;
    // decode_tokens has one entry per decode row.
    void commit(int32_t prefill_token, const int32_t* decode_tokens, int n);
    bool planned() const { return planned_; }

    // Takes the queue head out of the queue unserved: it is marked finished
    // with the tokens it has (none) and any pages it holds are released.  For
    // a request the model cannot run (the reference has no such check).
    void reject_head();
    // Forgets a request that has finished and been released.
    void drop(int req_id);
    // True when drop(req_id) would succeed: finished and in no queue.
    bool droppable(int req_id) const;
    Request* find(int req_id);
    const Request* find(int req_id) const;

    // running ids, waiting ids, then per request (in the order added): id,
    // prefill_idx, done, finished, next token, generated tokens, token count,
    // hash (lo, hi), token buffer, block table — each list length-prefixed.
    std::vector<int32_t> state_words() const;

    BlockManager& block_manager() { return bm_; }
    int max_tokens_per_batch() const { return budget_; }
    int max_generated() const { return max_generated_; }

  private:
    BlockManager& bm_;
    int budget_, max_generated_;
    int seq_len_ = 0, vocab_ = 0;
    std::deque<Request*> waiting_;
    std::vector<Request*> running_;
    std::vector<std::unique_ptr<Request>> requests_;
    StepPlan plan_;
    bool planned_ = false;
};

}  // namespace nitro

namespace nitro {
struct SchedDevice;  // device-resident tables and step buffers (scheduler_step.cpp)
}

struct nitro_block_manager;

// The C ABI handle: the host scheduler over a caller-owned block manager, and
// the device half, created by the first nitro_sched_step.
struct nitro_scheduler {
    nitro_scheduler(nitro_block_manager* h, nitro::BlockManager& bm, int budget, int max_generated)
        : bm_handle(h), host(bm, budget, max_generated) {}
    ~nitro_scheduler() {
        if (dev && dev_free) dev_free(dev);
    }
    nitro_block_manager* bm_handle;
    nitro::ContinuousScheduler host;
    nitro::SchedDevice* dev = nullptr;
    void (*dev_free)(nitro::SchedDevice*) = nullptr;
};
