// Shared helpers of the C ABI: status mapping and the per-thread last error.
#pragma once

#include <exception>
#include <new>
#include <string>

#include "paged_memory.hpp"

namespace nitro {

void set_last_error(const std::string& msg);
void clear_last_error();

// Runs `body` and converts nitro::Error / std::bad_alloc / anything else into
// a status code, recording the message for nitro_last_error().
template <class F>
int guarded(F&& body) {
    try {
        clear_last_error();
        body();
        return OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.status;
    } catch (const std::bad_alloc&) {
        set_last_error("host allocation failed");
        return ERR_INVALID_ARGUMENT;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return ERR_INVALID_ARGUMENT;
    }
}

inline void require(bool ok, Status s, const char* msg) {
    if (!ok) throw Error(s, msg);
}

}  // namespace nitro

// The bookkeeping handles of the C ABI (opaque to callers).
struct nitro_block_manager {
    explicit nitro_block_manager(int n) : bm(n) {}
    nitro::BlockManager bm;
};

struct nitro_sequence {
    explicit nitro_sequence(int id) : seq(id) {}
    nitro::Sequence seq;
};
