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
