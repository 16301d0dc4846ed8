import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libbs_hip.so")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip-free guard: a gpu-marked test on a machine without a GPU is an error, not a skip."""
    if not gpu_available():
        pytest.fail("no GPU visible; run gpu tests on the MI355X box (-m gpu)")
    import torch
    torch.cuda.init()
    return True


def load_fastscan_golden(seed):
    """records of oracle/_ref/ref_fastscan (see oracle/ref_fastscan_main.inc)"""
    buf = open(os.path.join(GOLDEN, f"fastscan_s{seed}.bin"), "rb").read()
    off = 0
    out = []

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(buf, dtype=dtype, count=count, offset=off).copy()
        off += a.nbytes
        return a

    while off < len(buf):
        dim, pdim, nn, degree = take(np.int32, 4)
        dseed = int(take(np.uint32, 1)[0])
        exact = np.float32(take(np.float32, 1)[0])
        wpp = pdim // 32
        rec = dict(dim=int(dim), pdim=int(pdim), nn=int(nn), degree=int(degree), seed=dseed, exact=exact)
        rec["query"] = take(np.float32, dim)
        rec["signs"] = take(np.float32, pdim)
        rec["nbrs"] = take(np.uint32, nn * wpp)
        rec["factors"] = take(np.float32, 3 * degree)
        rec["codes"] = take(np.uint8, pdim)
        rec["low"], rec["width"] = take(np.float32, 2)
        rec["sum_q"] = int(take(np.int32, 1)[0])
        rec["raw"] = take(np.uint32, nn)
        rec["est"] = take(np.float32, nn)
        out.append(rec)
    return out


def load_cpucli(name):
    z = np.load(os.path.join(GOLDEN, f"cpucli_{name}.npz"), allow_pickle=False)
    meta = json.load(open(os.path.join(GOLDEN, f"cpucli_{name}.json")))
    return {k: z[k] for k in z.files}, meta


@pytest.fixture(scope="session")
def golden_sets():
    return {n: load_cpucli(n) for n in ("d32", "d100")}
