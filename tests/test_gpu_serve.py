"""GPU end to end through the serving loop (nitro_server_*): clients on
socket pairs send their prompts in the NitroRPC wire format, the server steps
the device scheduler, and each client reads its generated tokens back as
int32 values until the server closes the connection.  The tokens must be the
ones the reference's own scheduler generated for the same requests
(tests/golden/sched_traces.*, scenario with five users and one shared
prompt)."""
import ctypes
import socket
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    yield
    torch.cuda.synchronize()


def test_served_tokens_match_reference_scheduler(golden_sched, golden_model):
    import nitrorag_amd as na
    from nitrorag_amd import _native as N
    from nitrorag_amd.q8 import LAST_BLOCK
    from oracle import scheduler as sc
    from oracle.model import scale_residual_outputs

    meta, traces = golden_sched
    tr = [t for t in traces if t.name == "shared_prompt"][0]
    blob, _, _ = golden_model
    model = na.Model(scale_residual_outputs(blob, meta["out_scale"]))
    pool = na.KVPool(tr.total_blocks, model.n_layers, model.kv_dim)
    bm = na.BlockManager(tr.total_blocks)
    sched = na.ContinuousScheduler(bm, tr.budget, meta["max_generated"])
    srv = ctypes.c_void_p()
    N.call("nitro_server_create", sched.handle, model.handle, pool.handle, LAST_BLOCK, 1024, ctypes.byref(srv))
    clients = []
    for rid, prompt in tr.arrivals[0]:
        a, b = socket.socketpair()
        b.sendall(np.asarray([len(prompt)] + list(prompt), np.int32).tobytes())
        got = ctypes.c_int32()
        N.call("nitro_server_accept_fd", srv, a.detach(), ctypes.byref(got))
        assert got.value == rid
        clients.append(b)
    print(f"serving {len(clients)} clients", flush=True)
    sys.stdout.flush()
    steps, active = 0, ctypes.c_int32(1)
    while active.value:
        N.call("nitro_server_step", srv, None, ctypes.byref(active))
        steps += 1
        assert steps <= tr.steps + 1
    final = {r["req_id"]: r for r in sc.decode_state(tr.state(tr.steps - 1))["requests"]}
    for rid, b in enumerate(clients):
        data = b""
        while True:
            chunk = b.recv(1 << 16)
            if not chunk:  # the server closed the connection after the last token
                break
            data += chunk
        b.close()
        assert np.frombuffer(data, np.int32).tolist() == final[rid]["generated"], rid
    N.call("nitro_server_destroy", srv)
    assert pool.take_device_errors() == 0


def test_unrunnable_requests_do_not_wedge_the_server(golden_sched, golden_model):
    """A prompt that cannot finish inside the model's seq_len (128 for the tiny
    model: n + 20 - 1 > 128) is refused at accept once the first step has bound
    the limits; one queued before that is finished unserved (its connection
    closes with no tokens) instead of failing every later step.  The client
    beside them is served the reference scheduler's tokens, and the server
    forgets every finished request once it has been released."""
    import nitrorag_amd as na
    from nitrorag_amd import _native as N
    from nitrorag_amd.q8 import LAST_BLOCK
    from oracle import scheduler as sc
    from oracle.model import scale_residual_outputs

    meta, traces = golden_sched
    tr = [t for t in traces if t.name == "shared_prompt"][0]
    blob, _, _ = golden_model
    model = na.Model(scale_residual_outputs(blob, meta["out_scale"]))
    pool = na.KVPool(tr.total_blocks, model.n_layers, model.kv_dim)
    bm = na.BlockManager(tr.total_blocks)
    sched = na.ContinuousScheduler(bm, tr.budget, meta["max_generated"])
    srv = ctypes.c_void_p()
    N.call("nitro_server_create", sched.handle, model.handle, pool.handle, LAST_BLOCK, 1024, ctypes.byref(srv))

    def connect(prompt):
        a, b = socket.socketpair()
        b.sendall(np.asarray([len(prompt)] + list(prompt), np.int32).tobytes())
        rid = ctypes.c_int32(-1)
        fd = a.detach()
        st = N.lib().nitro_server_accept_fd(srv, fd, ctypes.byref(rid))
        return st, rid.value, fd, b

    long_prompt = [7] * 110  # 110 + 19 = 129 > 128
    rid0, prompt0 = tr.arrivals[0][0]
    st, r, _, c_long = connect(long_prompt)  # no step has run: no limits yet, admitted
    assert st == N.OK and r == 0
    st, r, _, c_ok = connect(prompt0)
    assert st == N.OK and r == 1
    print("stepping with an unrunnable request queued first", flush=True)
    sys.stdout.flush()
    active, steps = ctypes.c_int32(1), 0
    N.call("nitro_server_step", srv, None, ctypes.byref(active))
    steps += 1
    assert sched.request_status(0)["is_finished"] == 1 and sched.request_status(0)["generated"] == 0
    st, r, fd, c_refused = connect(long_prompt)  # limits are bound now: refused at accept
    assert st == N.INVALID_ARGUMENT
    c_refused.settimeout(10)
    try:  # the server closed it with no token sent (a reset if it left bytes unread)
        assert c_refused.recv(64) == b""
    except ConnectionResetError:
        pass
    c_refused.close()
    while active.value:
        N.call("nitro_server_step", srv, None, ctypes.byref(active))
        steps += 1
        assert steps <= 64

    def read_all(sock):
        data = b""
        while True:
            chunk = sock.recv(1 << 16)
            if not chunk:
                return np.frombuffer(data, np.int32).tolist()
            data += chunk

    assert read_all(c_long) == []
    # request 1 ran alone, so its tokens are those of a one-user run of the same
    # prompt: the oracle scheduler over the oracle forward gives them
    got = read_all(c_ok)
    assert len(got) == meta["max_generated"]
    one = na.ContinuousScheduler(na.BlockManager(tr.total_blocks), tr.budget, meta["max_generated"])
    one.add_request(0, prompt0)
    pool2 = na.KVPool(tr.total_blocks, model.n_layers, model.kv_dim)
    while one.has_active_requests():
        one.step(model, pool2, LAST_BLOCK)
    assert got == one.generated(0)
    # one more step releases nothing new; every finished request is forgotten
    N.call("nitro_server_step", srv, None, ctypes.byref(active))
    assert sc.decode_state(sched.state_words())["requests"] == []
    c_long.close(), c_ok.close()
    N.call("nitro_server_destroy", srv)
    assert pool.take_device_errors() == 0
