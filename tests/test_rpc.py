"""NitroRPC wire format (nitro_rpc_*) against the reference's own
src/NitroRPC.hpp, recorded over socket pairs in tests/golden/rpc.json: the
bytes send_ints writes, and what recv_ints / recv_structured_query decode.
Host code only, plus the serving loop's intake (nitro_server_accept_fd)."""
import ctypes
import json
import os
import socket

import numpy as np
import pytest

import nitrorag_amd as na
from nitrorag_amd import _native as N

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rpc.json")
_u8p = ctypes.POINTER(ctypes.c_uint8)


@pytest.fixture(scope="module")
def cases():
    with open(GOLDEN) as f:
        return json.load(f)


def encode_ints(vals):
    a = np.asarray(vals, np.int32)
    nbytes = ctypes.c_uint64()
    N.call("nitro_rpc_encode_ints", a.ctypes.data_as(N._i32p), a.size, None, 0, ctypes.byref(nbytes))
    out = np.zeros(nbytes.value, np.uint8)
    N.call("nitro_rpc_encode_ints", a.ctypes.data_as(N._i32p), a.size, out.ctypes.data_as(_u8p), out.size,
           ctypes.byref(nbytes))
    return out.tobytes()


def decode_ints(wire):
    buf = np.frombuffer(wire, np.uint8).copy()
    n, used = ctypes.c_int32(), ctypes.c_uint64()
    N.call("nitro_rpc_decode_ints", buf.ctypes.data_as(_u8p), buf.size, None, 0, ctypes.byref(n), ctypes.byref(used))
    out = np.zeros(max(1, n.value), np.int32)
    N.call("nitro_rpc_decode_ints", buf.ctypes.data_as(_u8p), buf.size, out.ctypes.data_as(N._i32p), out.size,
           ctypes.byref(n), ctypes.byref(used))
    return out[:n.value].tolist(), used.value


def test_int_vectors_match_reference_bytes(cases):
    for c in cases:
        if c["kind"] == "send_ints":
            wire = bytes.fromhex(c["wire"])
            assert encode_ints(c["values"]) == wire
            assert decode_ints(wire) == (c["values"], len(wire))
            # and over a socket, as send_ints / recv_ints
            a, b = socket.socketpair()
            arr = np.asarray(c["values"], np.int32)
            N.call("nitro_rpc_send_ints", a.fileno(), arr.ctypes.data_as(N._i32p), arr.size)
            got = b.recv(1 << 16)
            while len(got) < len(wire):
                got += b.recv(1 << 16)
            assert got == wire
            a.close(), b.close()
        if c["kind"] == "recv_ints":
            a, b = socket.socketpair()
            b.sendall(bytes.fromhex(c["wire"]))
            out = np.zeros(max(1, c["count"]), np.int32)
            n = ctypes.c_int32()
            N.call("nitro_rpc_recv_ints", a.fileno(), out.ctypes.data_as(N._i32p), out.size, ctypes.byref(n))
            assert n.value == c["count"] and out[:n.value].tolist() == c["values"]
            a.close(), b.close()


def test_truncated_message_fails_like_the_reference(cases):
    c = [c for c in cases if c["kind"] == "recv_ints_truncated"][0]
    assert c["count"] == -1  # the reference reports failure
    a, b = socket.socketpair()
    b.sendall(bytes.fromhex(c["wire"]))
    b.close()
    out = np.zeros(8, np.int32)
    n = ctypes.c_int32()
    assert N.lib().nitro_rpc_recv_ints(a.fileno(), out.ctypes.data_as(N._i32p), 8, ctypes.byref(n)) == N.INVALID_ARGUMENT
    a.close()
    short = bytes.fromhex(c["wire"])
    with pytest.raises(na.NitroError):
        decode_ints(short)


def test_structured_queries_match_reference(cases):
    for c in cases:
        if c["kind"] != "recv_structured_query":
            continue
        dim, wire = c["dim"], bytes.fromhex(c["wire"])
        vec = np.asarray(c["vec"], np.float32)
        nbytes = ctypes.c_uint64()
        out = np.zeros(16 + 4 * dim, np.uint8)
        N.call("nitro_rpc_encode_structured_query", c["subset_mask"], c["range_min"], c["range_max"],
               vec.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), dim, out.ctypes.data_as(_u8p), out.size,
               ctypes.byref(nbytes))
        assert out.tobytes() == wire
        a, b = socket.socketpair()
        b.sendall(wire)
        m, lo, hi = ctypes.c_uint64(), ctypes.c_float(), ctypes.c_float()
        got = np.zeros(max(dim, 1), np.float32)
        N.call("nitro_rpc_recv_structured_query", a.fileno(), dim, ctypes.byref(m), ctypes.byref(lo),
               ctypes.byref(hi), got.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        a.close(), b.close()
        assert (m.value, lo.value, hi.value) == (c["subset_mask"], np.float32(c["range_min"]),
                                                 np.float32(c["range_max"]))
        assert np.array_equal(got[:dim], vec)


def closed_without_a_token(sock) -> bool:
    """The peer closed the connection before sending anything: end of stream,
    or a reset where the closing side still held unread bytes of ours."""
    sock.settimeout(10)
    try:
        return sock.recv(64) == b""
    except ConnectionResetError:
        return True


def test_oversize_count_is_refused():
    """The reference resizes to whatever count the peer names; here a count
    above the caller's limit is an error and nothing more is read."""
    a, b = socket.socketpair()
    b.sendall(np.asarray([1 << 30], np.int32).tobytes())
    out = np.zeros(4, np.int32)
    n = ctypes.c_int32()
    assert N.lib().nitro_rpc_recv_ints(a.fileno(), out.ctypes.data_as(N._i32p), 4, ctypes.byref(n)) == N.INVALID_ARGUMENT
    a.close(), b.close()


def test_server_intake_numbers_requests_like_the_reference():
    """tcp_listener_thread (src/Server_Inference.cpp:27-35): each connection's
    prompt becomes request 0, 1, 2, ... in the scheduler's waiting queue."""
    from oracle import scheduler as sc

    bm = na.BlockManager(16)
    sched = na.ContinuousScheduler(bm, 256, 20)
    srv = ctypes.c_void_p()
    N.call("nitro_server_create", sched.handle, ctypes.c_void_p(1), ctypes.c_void_p(1), 1, 64, ctypes.byref(srv))
    prompts = [[5, 6, 7], [9], list(range(40))]
    pairs = []
    for i, p in enumerate(prompts):
        a, b = socket.socketpair()
        b.sendall(np.asarray([len(p)] + p, np.int32).tobytes())
        rid = ctypes.c_int32()
        N.call("nitro_server_accept_fd", srv, os.dup(a.fileno()), ctypes.byref(rid))
        assert rid.value == i
        pairs.append((a, b))
    st = sc.decode_state(sched.state_words())
    assert st["waiting"] == [0, 1, 2] and [r["next"] for r in st["requests"]] == [5, 9, 0]
    # a prompt over the limit is refused and adds nothing; the server closes
    # the connection without sending a token
    a, b = socket.socketpair()
    b.sendall(np.asarray([65] + [1] * 65, np.int32).tobytes())
    rid = ctypes.c_int32()
    assert N.lib().nitro_server_accept_fd(srv, a.detach(), ctypes.byref(rid)) == N.INVALID_ARGUMENT
    assert sc.decode_state(sched.state_words())["waiting"] == [0, 1, 2]
    assert closed_without_a_token(b)
    b.close()
    N.call("nitro_server_destroy", srv)  # closes the three duplicated descriptors
    for x, y in pairs:
        x.close(), y.close()


def test_server_refuses_prompts_the_model_cannot_finish():
    """With the model's limits set on the scheduler, a prompt of n tokens is
    admitted only if its last decode (position n + max_generated - 2) lies
    below seq_len and every token is in the vocabulary; a refused prompt adds
    no request and takes no request id, and its client sees the connection
    closed with no token (what a request refused at a later step receives)."""
    from oracle import scheduler as sc

    bm = na.BlockManager(16)
    sched = na.ContinuousScheduler(bm, 256, 20)
    sched.set_limits(64, 100)
    srv = ctypes.c_void_p()
    N.call("nitro_server_create", sched.handle, ctypes.c_void_p(1), ctypes.c_void_p(1), 1, 128, ctypes.byref(srv))
    cases = [(list(range(1, 46)), True),        # 45 + 19 = 64 <= 64: the last decode sits at 63
             (list(range(1, 47)), False),       # 46 + 19 = 65 > 64
             ([3, 100, 4], False),              # token outside the vocabulary
             ([-1], False),
             ([99], True)]
    pairs, want_ids = [], []
    for prompt, ok in cases:
        a, b = socket.socketpair()
        b.sendall(np.asarray([len(prompt)] + prompt, np.int32).tobytes())
        rid = ctypes.c_int32(-7)
        fd = a.detach()  # the server's from the call on
        st = N.lib().nitro_server_accept_fd(srv, fd, ctypes.byref(rid))
        if ok:
            assert st == N.OK and rid.value == len(want_ids)
            want_ids.append(rid.value)
        else:
            assert st == N.INVALID_ARGUMENT and rid.value == -7
            assert closed_without_a_token(b)  # closed by the server, no token sent
        pairs.append((a, b))
    st = sc.decode_state(sched.state_words())
    assert st["waiting"] == want_ids
    # the scheduler's own entry point applies the same limits
    with pytest.raises(N.NitroError):
        sched.add_request(50, list(range(1, 47)))
    sched.add_request(50, list(range(1, 46)))
    N.call("nitro_server_destroy", srv)
    for x, y in pairs:
        x.close(), y.close()
