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


TREE_SETS = ("d32r8", "d100r16", "d64r48")


def load_rqtree(name):
    """the RaBitQ special case where the GPU search and the reference cpu_cli agree id for id
    (tests/golden/make_golden.py, rqtree_*)"""
    z = np.load(os.path.join(GOLDEN, f"rqtree_{name}.npz"), allow_pickle=False)
    meta = json.load(open(os.path.join(GOLDEN, f"rqtree_{name}.json")))
    return {k: z[k] for k in z.files}, meta


# ---------------------------------------------------------------------------------------
# Bloom filter restated from the reference (filter_bloom.cuh:25-38,104-120 and the row loop
# of gpu_search_warp.cuh:203-205) in Python integers, independent of the oracle and the kernel
# ---------------------------------------------------------------------------------------
INVALID_ID = 0xFFFFFFFF
_M32 = 0xFFFFFFFF


def _mix(x):
    # filter_bloom.cuh:25-38: x ^= x >> 16; x *= 0x45d9f3b; x ^= x >> 16 (32-bit arithmetic)
    x ^= x >> 16
    x = (x * 0x45D9F3B) & _M32
    return x ^ (x >> 16)


def bloom_bits(key, cap):
    b = max(5, (cap - 1).bit_length())
    mask = (1 << b) - 1
    return [_mix(key) & mask, _mix((key * 0x9E3779B9) & _M32) & mask, _mix((key * 0x517CC1B7) & _M32) & mask]


def bloom_simulate(cap, batches):
    """the reference's row filter (gpu_search_warp.cuh:203-205 with filter_bloom.cuh:104-120):
    rounds of 32 consecutive keys; each round tests against the bits of all earlier rounds,
    then sets its keys' bits; a key held twice in one round is new once (first index)"""
    bitset = set()
    new = np.zeros(batches.shape, np.uint32)
    for b in range(batches.shape[0]):
        row = [int(k) for k in batches[b]]
        for r0 in range(0, len(row), 32):
            seen_absent = set()
            for i in range(r0, min(r0 + 32, len(row))):
                k = row[i]
                if k == INVALID_ID:
                    continue
                absent = not all(h in bitset for h in bloom_bits(k, cap))
                if absent and k not in seen_absent:
                    new[b, i] = 1
                if absent:
                    seen_absent.add(k)
            for i in range(r0, min(r0 + 32, len(row))):
                if row[i] != INVALID_ID:
                    bitset.update(bloom_bits(row[i], cap))
    return new, bitset


