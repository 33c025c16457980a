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
