// Drives the shipped scheduler and NitroRPC host code (nitrorag_amd/csrc/
// scheduler.cpp, rpc.cpp, with paged_memory.cpp and capi_host.cpp) for the
// AddressSanitizer + UndefinedBehaviorSanitizer replay in
// tests/test_host_sanitizers.py.  Host code only: the device step is replaced
// by a test double (nitro_sched_step below) that plans, picks deterministic
// tokens and commits.
//
// usage: host_driver_sched_rpc sched|rpc|server   (commands on stdin)
//
// sched: "S total_blocks budget max_generated", then per step
//        "T n_arrivals n_next", n_arrivals lines "rid n tok_1 .. tok_n", one
//        line "rid tok rid tok ..." (the token each request commits this step,
//        teacher-forced from a reference trace); after each step prints
//        "STATE <scheduler state words>" and "BM <block-manager words>".
// rpc:   lines "ENC n v..", "DEC hex", "RECV cap hex", "TRUNC cap hex",
//        "SQ dim mask_lo mask_hi min_bits max_bits v_bits..": one result line each.
// server: no input; serves clients over socket pairs, prints one line each.
#include <sys/socket.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "capi_common.hpp"
#include "nitro_paged_attn.h"
#include "scheduler.hpp"

using namespace nitro;

namespace {

int32_t fake_token(int req_id, size_t generated) { return (int32_t)((req_id * 7 + generated * 3) % 97 + 1); }

}  // namespace

// Test double of the device step: the host plan, deterministic tokens, commit.
extern "C" int nitro_sched_step(nitro_scheduler* s, nitro_model*, nitro_kvpool*, int32_t, void*) {
    return guarded([&] {
        require(s != nullptr, ERR_INVALID_ARGUMENT, "null scheduler");
        ContinuousScheduler& h = s->host;
        if (!h.has_active_requests()) return;
        const StepPlan& p = h.plan();
        const int32_t pt = p.prefill ? fake_token(p.prefill->req_id, p.prefill->generated_tokens.size()) : 0;
        std::vector<int32_t> dt;
        for (const Request* r : p.decode) dt.push_back(fake_token(r->req_id, r->generated_tokens.size()));
        h.commit(pt, dt.data(), (int)dt.size());
    });
}

namespace {

std::vector<long long> bm_words(nitro_block_manager* bm, int total) {
    std::vector<long long> w;
    std::vector<int32_t> ids(total);
    int32_t n = 0;
    nitro_bm_free_list(bm, ids.data(), total, &n);
    w.push_back(n);
    w.insert(w.end(), ids.begin(), ids.begin() + n);
    for (int i = 0; i < total; i++) {
        nitro_block_info b;
        nitro_bm_get_block(bm, i, &b);
        w.insert(w.end(), {b.ref_count, b.num_tokens, b.parent_id, b.child_count});
    }
    nitro_bm_evictable_leaves(bm, ids.data(), total, &n);
    w.push_back(n);
    w.insert(w.end(), ids.begin(), ids.begin() + n);
    std::vector<uint64_t> hashes(total);
    nitro_bm_cache_entries(bm, hashes.data(), ids.data(), total, &n);
    w.push_back(n);
    for (int i = 0; i < n; i++)
        w.insert(w.end(), {(long long)(hashes[i] & 0xffffffffu), (long long)(hashes[i] >> 32), ids[i]});
    nitro_bm_reverse_entries(bm, ids.data(), hashes.data(), total, &n);
    w.push_back(n);
    for (int i = 0; i < n; i++)
        w.insert(w.end(), {ids[i], (long long)(hashes[i] & 0xffffffffu), (long long)(hashes[i] >> 32)});
    return w;
}

int run_sched() {
    std::string tag;
    int total = 0, budget = 0, max_gen = 0;
    if (!(std::cin >> tag >> total >> budget >> max_gen) || tag != "S") return 2;
    nitro_block_manager* bm = nullptr;
    nitro_scheduler* s = nullptr;
    if (nitro_bm_create(total, &bm) || nitro_sched_create(bm, budget, max_gen, &s)) return 3;
    std::vector<int32_t> all_ids;
    while (std::cin >> tag && tag == "T") {
        int n_arr = 0, n_next = 0;
        std::cin >> n_arr >> n_next;
        for (int i = 0; i < n_arr; i++) {
            int rid = 0, n = 0;
            std::cin >> rid >> n;
            std::vector<int32_t> toks(n);
            for (auto& t : toks) std::cin >> t;
            if (nitro_sched_add_request(s, rid, toks.data(), n)) return 4;
            all_ids.push_back(rid);
        }
        std::map<int, int32_t> next;
        for (int i = 0; i < n_next; i++) {
            int rid = 0, tok = 0;
            std::cin >> rid >> tok;
            next[rid] = tok;
        }
        int32_t pre[4], n_dec = 0;
        std::vector<int32_t> ids(all_ids.size() + 1);
        if (nitro_sched_plan(s, pre, ids.data(), nullptr, nullptr, (int32_t)ids.size(), &n_dec)) return 5;
        std::vector<int32_t> dt(n_dec);
        for (int b = 0; b < n_dec; b++) dt[b] = next.at(ids[b]);
        const int32_t pt = pre[0] >= 0 ? next.at(pre[0]) : 0;
        if (nitro_sched_commit(s, pt, dt.data(), n_dec)) return 6;
        int32_t n = 0;
        nitro_sched_state(s, nullptr, 0, &n);
        std::vector<int32_t> words(n);
        nitro_sched_state(s, words.data(), n, &n);
        std::printf("STATE");
        for (int32_t x : words) std::printf(" %d", x);
        std::printf("\nBM");
        for (long long x : bm_words(bm, total)) std::printf(" %lld", x);
        std::printf("\n");
    }
    for (int32_t rid : all_ids)
        if (nitro_sched_drop_request(s, rid)) return 7;  // every request finished and was released
    int32_t n = 0;
    nitro_sched_state(s, nullptr, 0, &n);
    std::printf("FINAL %d\n", n);
    nitro_sched_destroy(s);
    nitro_bm_destroy(bm);
    return 0;
}

std::vector<uint8_t> from_hex(const std::string& h) {
    std::vector<uint8_t> b(h.size() / 2);
    for (size_t i = 0; i < b.size(); i++) b[i] = (uint8_t)std::stoi(h.substr(2 * i, 2), nullptr, 16);
    return b;
}

std::string to_hex(const uint8_t* p, size_t n) {
    static const char* d = "0123456789abcdef";
    std::string s;
    for (size_t i = 0; i < n; i++) {
        s += d[p[i] >> 4];
        s += d[p[i] & 15];
    }
    return s;
}

// Bytes written to one end of a socket pair, the other end returned (the
// writer closed when `close_writer`).
int feed(const std::vector<uint8_t>& bytes, bool close_writer, int* writer) {
    int sv[2];
    if (socketpair(AF_UNIX, SOCK_STREAM, 0, sv)) return -1;
    if (!bytes.empty() && send(sv[1], bytes.data(), bytes.size(), 0) != (ssize_t)bytes.size()) return -1;
    if (close_writer) {
        ::close(sv[1]);
        *writer = -1;
    } else {
        *writer = sv[1];
    }
    return sv[0];
}

int run_rpc() {
    std::string line;
    while (std::getline(std::cin, line)) {
        std::istringstream in(line);
        std::string kind;
        in >> kind;
        if (kind == "ENC") {
            int n = 0;
            in >> n;
            std::vector<int32_t> v(n);
            for (auto& x : v) in >> x;
            uint64_t bytes = 0;
            nitro_rpc_encode_ints(v.data(), n, nullptr, 0, &bytes);
            std::vector<uint8_t> out(bytes);
            const int st = nitro_rpc_encode_ints(v.data(), n, out.data(), out.size(), &bytes);
            // and the same through send_ints / recv_ints over a socket pair
            int sv[2];
            socketpair(AF_UNIX, SOCK_STREAM, 0, sv);
            const int st_send = nitro_rpc_send_ints(sv[1], v.data(), n);
            std::vector<int32_t> back(n + 1);
            int32_t got = -1;
            const int st_recv = nitro_rpc_recv_ints(sv[0], back.data(), n + 1, &got);
            ::close(sv[0]);
            ::close(sv[1]);
            bool same = got == n && std::equal(v.begin(), v.end(), back.begin());
            std::printf("ENC %d %s %d %d %d\n", st, to_hex(out.data(), out.size()).c_str(), st_send, st_recv,
                        same ? 1 : 0);
        } else if (kind == "DEC") {
            std::string hex;
            in >> hex;
            const std::vector<uint8_t> b = from_hex(hex);
            int32_t n = 0;
            uint64_t used = 0;
            int st = nitro_rpc_decode_ints(b.data(), b.size(), nullptr, 0, &n, &used);
            std::printf("DEC %d", st);
            if (st == NITRO_OK) {
                std::vector<int32_t> v(n > 0 ? n : 1);
                st = nitro_rpc_decode_ints(b.data(), b.size(), v.data(), n, &n, &used);
                std::printf(" %d %d %llu", st, n, (unsigned long long)used);
                for (int i = 0; i < n; i++) std::printf(" %d", v[i]);
            }
            std::printf("\n");
        } else if (kind == "RECV" || kind == "TRUNC") {
            int cap = 0;
            std::string hex;
            in >> cap >> hex;
            int writer = -1;
            const int fd = feed(from_hex(hex == "-" ? "" : hex), kind == "TRUNC", &writer);
            std::vector<int32_t> v(cap > 0 ? cap : 1);
            int32_t n = -1;
            const int st = nitro_rpc_recv_ints(fd, v.data(), cap, &n);
            std::printf("%s %d", kind.c_str(), st);
            if (st == NITRO_OK) {
                std::printf(" %d", n);
                for (int i = 0; i < n; i++) std::printf(" %d", v[i]);
            }
            std::printf("\n");
            ::close(fd);
            if (writer >= 0) ::close(writer);
        } else if (kind == "SQ") {
            int dim = 0;
            uint32_t mlo = 0, mhi = 0, lo_bits = 0, hi_bits = 0;
            in >> dim >> mlo >> mhi >> lo_bits >> hi_bits;
            std::vector<float> vec(dim);
            for (auto& x : vec) {
                uint32_t u = 0;
                in >> u;
                std::memcpy(&x, &u, 4);
            }
            float rmin, rmax;
            std::memcpy(&rmin, &lo_bits, 4);
            std::memcpy(&rmax, &hi_bits, 4);
            const uint64_t mask = ((uint64_t)mhi << 32) | mlo;
            uint64_t bytes = 0;
            std::vector<uint8_t> out(16 + 4 * (size_t)dim);
            const int st = nitro_rpc_encode_structured_query(mask, rmin, rmax, dim ? vec.data() : nullptr, dim,
                                                             out.data(), out.size(), &bytes);
            int writer = -1;
            const int fd = feed(out, true, &writer);
            uint64_t m2 = 0;
            float a = 0, b = 0;
            std::vector<float> v2(dim > 0 ? dim : 1);
            const int st2 = nitro_rpc_recv_structured_query(fd, dim, &m2, &a, &b, v2.data());
            ::close(fd);
            const bool same = m2 == mask && a == rmin && b == rmax &&
                              (dim == 0 || std::memcmp(v2.data(), vec.data(), 4 * (size_t)dim) == 0);
            std::printf("SQ %d %s %d %d\n", st, to_hex(out.data(), out.size()).c_str(), st2, same ? 1 : 0);
        }
    }
    return 0;
}

int run_server() {
    nitro_block_manager* bm = nullptr;
    nitro_scheduler* s = nullptr;
    nitro_server* srv = nullptr;
    const int32_t max_gen = 5;
    if (nitro_bm_create(64, &bm) || nitro_sched_create(bm, 32, max_gen, &s) || nitro_sched_set_limits(s, 64, 100))
        return 3;
    // the device step is the test double: model and pool are never touched
    if (nitro_server_create(s, reinterpret_cast<nitro_model*>(1), reinterpret_cast<nitro_kvpool*>(1),
                            NITRO_Q8_LAST_BLOCK, 128, &srv))
        return 4;
    struct Client {
        std::vector<int32_t> prompt;
        int fd = -1, rid = -1, status = 0;
        bool truncated = false;  // sends its count, part of the prompt, then shuts down
    };
    std::vector<Client> clients(6);
    for (int i = 0; i < 40; i++) clients[0].prompt.push_back(i % 90 + 1);
    clients[1].prompt = std::vector<int32_t>(61, 3);  // 61 + 4 > 64: cannot finish
    clients[2].prompt = {5, 6, 7};
    clients[3].prompt = {5, 100};                     // a token outside the vocabulary
    for (int i = 0; i < 60; i++) clients[4].prompt.push_back(i % 50 + 2);  // 60 + 4 = 64: fits
    clients[5].prompt = {8, 9, 10, 11};
    clients[5].truncated = true;                      // the server cannot read its prompt
    for (auto& c : clients) {
        int sv[2];
        socketpair(AF_UNIX, SOCK_STREAM, 0, sv);
        if (c.truncated) {
            const int32_t head[3] = {(int32_t)c.prompt.size(), c.prompt[0], c.prompt[1]};
            if (::send(sv[1], head, sizeof head, MSG_NOSIGNAL) != (ssize_t)sizeof head) return 6;
            ::shutdown(sv[1], SHUT_WR);
        } else {
            nitro_rpc_send_ints(sv[1], c.prompt.data(), (int32_t)c.prompt.size());
        }
        int32_t rid = -1;
        c.status = nitro_server_accept_fd(srv, sv[0], &rid);  // the fd is the server's
        c.rid = rid;
        c.fd = sv[1];
    }
    int32_t active = 1, steps = 0;
    while (active && steps < 200) {
        if (nitro_server_step(srv, nullptr, &active)) return 5;
        steps++;
    }
    nitro_server_step(srv, nullptr, &active);  // forgets what the last step released
    for (auto& c : clients) {
        std::vector<int32_t> got;
        int32_t x;
        ssize_t k;
        while ((k = recv(c.fd, &x, 4, MSG_WAITALL)) == 4) got.push_back(x);
        bool ok = c.status != NITRO_OK || (int)got.size() == max_gen;
        for (size_t i = 0; ok && i < got.size(); i++) ok = got[i] == fake_token(c.rid, i);
        std::printf("CLIENT %d %d %zu %d\n", c.status, c.rid, got.size(), ok ? 1 : 0);
        ::close(c.fd);
    }
    int32_t n = 0;
    nitro_sched_state(s, nullptr, 0, &n);
    std::vector<int32_t> words(n);
    nitro_sched_state(s, words.data(), n, &n);
    std::printf("REQUESTS %d STEPS %d\n", words.size() > 2 ? words[2] : -1, steps);
    nitro_server_destroy(srv);
    nitro_sched_destroy(s);
    nitro_bm_destroy(bm);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "";
    if (mode == "sched") return run_sched();
    if (mode == "rpc") return run_rpc();
    if (mode == "server") return run_server();
    return 2;
}
