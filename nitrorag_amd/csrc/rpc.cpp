// NitroRPC wire format and the serving loop around the continuous scheduler
// (declared in include/nitro_paged_attn.h).
//
// Wire format (src/NitroRPC.hpp:39-67), host byte order (little-endian here):
//   int vector         int32 count, then count int32 values;
//   structured query   uint64 subset_mask, float32 range_min, float32
//                      range_max (16 bytes), then dim float32 values.
// The serving loop follows src/Server_Inference.cpp:86-112: a connection
// sends one int vector (the prompt) and becomes a request; every step the
// request's newly generated tokens go back as bare int32 values, and its
// connection is closed once it has finished.  Differences by design: the
// tokens are actually sent (the reference's flag `just_generated_new_token`
// is never set, so it sends none), a prompt longer than the caller's limit is
// refused instead of resizing to any length the peer names, and send uses
// MSG_NOSIGNAL so a vanished client is an error status, not SIGPIPE.
#include <sys/socket.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <string>
#include <vector>

#include "capi_common.hpp"
#include "nitro_paged_attn.h"
#include "scheduler.hpp"

namespace nitro {
namespace {

void send_all(int fd, const void* p, size_t n) {  // NitroRPC::send_all, :19-27
    const char* b = static_cast<const char*>(p);
    size_t done = 0;
    while (done < n) {
        const ssize_t k = ::send(fd, b + done, n - done, MSG_NOSIGNAL);
        if (k < 0 && errno == EINTR) continue;
        if (k <= 0) throw Error(ERR_INVALID_ARGUMENT, std::string("send failed: ") + std::strerror(errno));
        done += (size_t)k;
    }
}

void recv_all(int fd, void* p, size_t n) {  // NitroRPC::recv_all, :29-37
    char* b = static_cast<char*>(p);
    size_t done = 0;
    while (done < n) {
        const ssize_t k = ::recv(fd, b + done, n - done, 0);
        if (k < 0 && errno == EINTR) continue;
        if (k == 0) throw Error(ERR_INVALID_ARGUMENT, "connection closed before the message ended");
        if (k < 0) throw Error(ERR_INVALID_ARGUMENT, std::string("recv failed: ") + std::strerror(errno));
        done += (size_t)k;
    }
}

int32_t recv_count(int fd, int32_t cap) {
    int32_t n = 0;
    recv_all(fd, &n, sizeof(n));
    if (n < 0 || n > cap) throw Error(ERR_INVALID_ARGUMENT, "int vector of " + std::to_string(n) + " values; the limit is " + std::to_string(cap));
    return n;
}

}  // namespace
}  // namespace nitro

using namespace nitro;

struct nitro_server {
    nitro_scheduler* sched = nullptr;
    nitro_model* model = nullptr;
    nitro_kvpool* pool = nullptr;
    int32_t semantics = NITRO_Q8_LAST_BLOCK;
    int32_t max_prompt = 0;
    int32_t next_id = 0;  // req_counter, src/Server_Inference.cpp:27
    struct Conn {
        int32_t req_id;
        int fd;
        size_t sent = 0;
        bool closed = false;
    };
    std::vector<Conn> conns;
};

extern "C" {

int nitro_rpc_encode_ints(const int32_t* data, int32_t n, uint8_t* out, uint64_t cap, uint64_t* bytes) {
    return guarded([&] {
        require(bytes != nullptr && n >= 0 && (n == 0 || data != nullptr), ERR_INVALID_ARGUMENT, "bad arguments");
        *bytes = 4 + 4 * (uint64_t)n;
        if (!out) return;
        require(cap >= *bytes, ERR_INVALID_ARGUMENT, "output buffer too small (the size is in *bytes)");
        std::memcpy(out, &n, 4);
        if (n) std::memcpy(out + 4, data, 4 * (size_t)n);
    });
}

int nitro_rpc_decode_ints(const uint8_t* buf, uint64_t len, int32_t* out, int32_t cap, int32_t* n,
                          uint64_t* consumed) {
    return guarded([&] {
        require(buf != nullptr && n != nullptr && consumed != nullptr, ERR_INVALID_ARGUMENT, "null pointer");
        require(len >= 4, ERR_INVALID_ARGUMENT, "message shorter than its count");
        int32_t k;
        std::memcpy(&k, buf, 4);
        require(k >= 0, ERR_INVALID_ARGUMENT, "negative count");
        require(len >= 4 + 4 * (uint64_t)k, ERR_INVALID_ARGUMENT, "message shorter than its count says");
        *n = k;
        *consumed = 4 + 4 * (uint64_t)k;
        if (!out) return;
        require(k <= cap, ERR_INVALID_ARGUMENT, "output buffer too small (the count is in *n)");
        if (k) std::memcpy(out, buf + 4, 4 * (size_t)k);
    });
}

int nitro_rpc_encode_structured_query(uint64_t subset_mask, float range_min, float range_max, const float* vec,
                                      int32_t dim, uint8_t* out, uint64_t cap, uint64_t* bytes) {
    return guarded([&] {
        require(bytes != nullptr && dim >= 0 && (dim == 0 || vec != nullptr), ERR_INVALID_ARGUMENT, "bad arguments");
        *bytes = 16 + 4 * (uint64_t)dim;
        if (!out) return;
        require(cap >= *bytes, ERR_INVALID_ARGUMENT, "output buffer too small (the size is in *bytes)");
        std::memcpy(out, &subset_mask, 8);
        std::memcpy(out + 8, &range_min, 4);
        std::memcpy(out + 12, &range_max, 4);
        if (dim) std::memcpy(out + 16, vec, 4 * (size_t)dim);
    });
}

int nitro_rpc_send_ints(int32_t fd, const int32_t* data, int32_t n) {
    return guarded([&] {
        require(n >= 0 && (n == 0 || data != nullptr), ERR_INVALID_ARGUMENT, "bad arguments");
        std::vector<uint8_t> msg(4 + 4 * (size_t)n);  // one send, as one message
        std::memcpy(msg.data(), &n, 4);
        if (n) std::memcpy(msg.data() + 4, data, 4 * (size_t)n);
        send_all(fd, msg.data(), msg.size());
    });
}

int nitro_rpc_recv_ints(int32_t fd, int32_t* out, int32_t cap, int32_t* n) {
    return guarded([&] {
        require(n != nullptr && (out != nullptr || cap == 0), ERR_INVALID_ARGUMENT, "null pointer");
        const int32_t k = recv_count(fd, cap);
        if (k) recv_all(fd, out, 4 * (size_t)k);
        *n = k;
    });
}

int nitro_rpc_recv_structured_query(int32_t fd, int32_t dim, uint64_t* subset_mask, float* range_min,
                                    float* range_max, float* vec) {
    return guarded([&] {
        require(subset_mask && range_min && range_max && dim >= 0 && (vec || dim == 0), ERR_INVALID_ARGUMENT,
                "bad arguments");
        uint8_t meta[16];
        recv_all(fd, meta, 16);
        std::memcpy(subset_mask, meta, 8);
        std::memcpy(range_min, meta + 8, 4);
        std::memcpy(range_max, meta + 12, 4);
        if (dim) recv_all(fd, vec, 4 * (size_t)dim);
    });
}

int nitro_server_create(nitro_scheduler* sched, nitro_model* model, nitro_kvpool* pool, int32_t semantics,
                        int32_t max_prompt_tokens, nitro_server** out) {
    return guarded([&] {
        require(out != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        *out = nullptr;
        require(sched && model && pool, ERR_INVALID_ARGUMENT, "null handle");
        require(semantics == NITRO_Q8_FULL_ROWS || semantics == NITRO_Q8_LAST_BLOCK, ERR_INVALID_ARGUMENT,
                "unknown Q8 semantics");
        require(max_prompt_tokens > 0, ERR_INVALID_ARGUMENT, "max_prompt_tokens must be positive");
        auto* s = new nitro_server();
        s->sched = sched;
        s->model = model;
        s->pool = pool;
        s->semantics = semantics;
        s->max_prompt = max_prompt_tokens;
        *out = s;
    });
}

int nitro_server_destroy(nitro_server* server) {
    if (!server) return OK;
    return guarded([&] {
        for (auto& c : server->conns)
            if (!c.closed) ::close(c.fd);
        delete server;
    });
}

int nitro_server_accept_fd(nitro_server* server, int32_t fd, int32_t* req_id) {
    // The fd is the server's from the call on.  A prompt it refuses (add_request
    // refuses one the model cannot finish) or cannot read is answered as a
    // request the scheduler refuses later is: no tokens, and the connection
    // closed.
    const int st = guarded([&] {
        require(server != nullptr && req_id != nullptr, ERR_INVALID_ARGUMENT, "null pointer");
        // tcp_listener_thread (src/Server_Inference.cpp:28-35): the prompt, then a request
        std::vector<int32_t> prompt(server->max_prompt);
        const int32_t n = recv_count(fd, server->max_prompt);
        if (n) recv_all(fd, prompt.data(), 4 * (size_t)n);
        server->conns.reserve(server->conns.size() + 1);  // nothing throws once the request is in
        const int32_t id = server->next_id;
        server->sched->host.add_request(id, prompt.data(), n);
        server->next_id++;
        server->conns.push_back({id, fd});
        *req_id = id;
    });
    if (st != NITRO_OK && fd >= 0) ::close(fd);
    return st;
}

int nitro_server_step(nitro_server* server, void* stream, int32_t* active) {
    return guarded([&] {
        require(server != nullptr && active != nullptr, ERR_INVALID_ARGUMENT, "null pointer");
        ContinuousScheduler& h = server->sched->host;
        *active = 0;
        // Forget what is over: a closed connection whose request has finished
        // and been released by the scheduler (so neither list grows with the
        // number of requests served).
        std::vector<nitro_server::Conn> kept;
        kept.reserve(server->conns.size());
        for (const auto& c : server->conns) {
            if (c.closed && h.droppable(c.req_id)) {
                h.drop(c.req_id);
                continue;
            }
            kept.push_back(c);
        }
        server->conns.swap(kept);
        if (!h.has_active_requests()) return;
        require(nitro_sched_step(server->sched, server->model, server->pool, server->semantics, stream) == NITRO_OK,
                ERR_INVALID_ARGUMENT, nitro_last_error());
        // src/Server_Inference.cpp:101-109: new tokens out, finished connections closed
        for (auto& c : server->conns) {
            if (c.closed) continue;
            const Request* r = h.find(c.req_id);
            if (!r) continue;
            const auto& gen = r->generated_tokens;
            if (gen.size() > c.sent) {
                try {
                    send_all(c.fd, gen.data() + c.sent, 4 * (gen.size() - c.sent));
                    c.sent = gen.size();
                } catch (const Error&) {  // the client went away: stop serving it
                    ::close(c.fd);
                    c.closed = true;
                    continue;
                }
            }
            if (r->is_finished) {
                ::close(c.fd);
                c.closed = true;
            }
        }
        *active = h.has_active_requests() ? 1 : 0;
    });
}

}  // extern "C"
