import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "lfm3-1.7b-mi50_amd")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs through the HIP C-ABI library)")


def load_host():
    """The package directory name is not a Python identifier; load its host module by path."""
    name = "dspark_amd_host"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "dspark.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def rope_numpy(base, pairs, D, positions):
    """Engine.buildRope (internal/model/engine.go:428-461) restated in numpy: inv[i] = 1 / float32(pow(base,
    float32(2 i) / D)) for i < pairs (0 beyond), f = float64(float32(p) * inv[i]), fp16 RNE of float32(cos f) and
    float32(sin f). cos and sin are Python's math module's (the C library routines the library's table builder calls;
    numpy's vectorised cos may differ in the last double bit from CPU to CPU)."""
    import math
    import numpy as np
    inv = np.zeros(D // 2, np.float32)
    for i in range(pairs):
        ex = np.float32(2 * i) / np.float32(D)
        inv[i] = np.float32(1.0) / np.float32(math.pow(base, float(ex)))
    p = np.arange(positions, dtype=np.float32)[:, None]
    f = (p * inv[None, :]).astype(np.float32).astype(np.float64)
    flat = f.ravel()
    cos = np.fromiter(map(math.cos, flat), np.float64, flat.size).reshape(f.shape)
    sin = np.fromiter(map(math.sin, flat), np.float64, flat.size).reshape(f.shape)
    return np.concatenate([cos.astype(np.float32).astype(np.float16), sin.astype(np.float32).astype(np.float16)],
                          axis=1).view(np.uint16)


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def kats():
    """Known-answer vectors held by the reference's own tests (tests/golden/reference_kats.json)."""
    import json
    with open(os.path.join(ROOT, "tests", "golden", "reference_kats.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def golden():
    """Seeded oracle vectors (tests/golden/vectors.npz, written by tests/golden/make_vectors.py)."""
    import numpy as np
    with np.load(os.path.join(ROOT, "tests", "golden", "vectors.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def host():
    return load_host()
