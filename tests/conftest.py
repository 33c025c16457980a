import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden_attention():
    with open(os.path.join(GOLDEN, "attention.json")) as f:
        meta = json.load(f)
    arrays = np.load(os.path.join(GOLDEN, "attention.npz"))
    cases = {}
    for m in meta:
        name = m["name"]
        cases[name] = (m, {k.split("/", 1)[1]: arrays[k] for k in arrays.files
                           if k.startswith(name + "/")})
    return cases


@pytest.fixture(scope="session")
def golden_traces():
    with open(os.path.join(GOLDEN, "block_manager_traces.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def golden_fnv():
    with open(os.path.join(GOLDEN, "fnv.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def golden_q8():
    with open(os.path.join(GOLDEN, "q8_matmul.json")) as f:
        meta = json.load(f)
    arrays = np.load(os.path.join(GOLDEN, "q8_matmul.npz"))
    return {name: (m, {k.split("/", 1)[1]: arrays[k] for k in arrays.files
                       if k.startswith(name + "/")})
            for name, m in meta.items()}


@pytest.fixture(scope="session")
def golden_model():
    blob = np.fromfile(os.path.join(GOLDEN, "model_tiny.bin"), dtype=np.uint8)
    with open(os.path.join(GOLDEN, "model_forward.json")) as f:
        meta = json.load(f)
    arrays = np.load(os.path.join(GOLDEN, "model_forward.npz"))
    return blob, meta, {k: arrays[k] for k in arrays.files}


class SchedTrace:
    """One scenario of tests/golden/sched_traces.*: per-step scheduler state
    words, block-manager snapshot words and the top logits the step left."""

    def __init__(self, meta, arrays):
        self.meta = meta
        self.name = meta["name"]
        self.total_blocks = meta["total_blocks"]
        self.budget = meta["max_tokens_per_batch"]
        self.steps = meta["steps"]
        self.arrivals = {int(k): [(rid, list(p)) for rid, p in v] for k, v in meta["arrivals"].items()}
        a = {k.split("/", 1)[1]: arrays[k] for k in arrays.files if k.startswith(self.name + "/")}
        self._a = a
        self._row_off = np.concatenate([[0], np.cumsum(a["rows"])])

    def state(self, t):
        o = self._a["state_off"]
        return self._a["state"][o[t]:o[t + 1]].tolist()

    def bm(self, t):
        o = self._a["bm_off"]
        return self._a["bm"][o[t]:o[t + 1]].tolist()

    def kind(self, t):
        """0: no forward, 1: decode rows, 2: the prefill chunk's last row."""
        return int(self._a["kind"][t])

    def top(self, t):
        r0, r1 = self._row_off[t], self._row_off[t + 1]
        return self._a["top_idx"][r0:r1], self._a["top_val"][r0:r1]


@pytest.fixture(scope="session")
def golden_sched():
    with open(os.path.join(GOLDEN, "sched_traces.json")) as f:
        meta = json.load(f)
    arrays = np.load(os.path.join(GOLDEN, "sched_traces.npz"))
    return meta, [SchedTrace(m, arrays) for m in meta["scenarios"]]
