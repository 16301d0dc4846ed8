"""Host tools: file formats, index construction, synthetic inputs, ground truth.

Thin numpy wrappers over libbs_host.so (include/bs_host.h); each function names the
reference host code it stands in for.
"""
from __future__ import annotations

import ctypes as C
import math
import os
from typing import Tuple

import numpy as np

from . import _lib


def _err(what: str):
    msg = _lib.host().bs_host_last_error().decode(errors="replace")
    raise IOError(f"{what}: {msg}")


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _take(ptr: C.c_void_p, count: int, dtype) -> np.ndarray:
    """copy a library-allocated buffer into numpy and free it"""
    if count == 0 or not ptr.value:
        if ptr.value:
            _lib.host().bs_host_free(ptr)
        return np.empty(0, dtype=dtype)
    nbytes = count * np.dtype(dtype).itemsize
    buf = (C.c_char * nbytes).from_address(ptr.value)
    out = np.frombuffer(buf, dtype=dtype, count=count).copy()
    _lib.host().bs_host_free(ptr)
    return out


# ---- formats (include/data_loader.hpp, include/cpu_graph.hpp, include/rabitq.hpp) -----

def read_fvecs(path: str) -> np.ndarray:
    return _read_vecs(path, 0, np.float32)


def read_ivecs(path: str) -> np.ndarray:
    return _read_vecs(path, 1, np.int32)


def _read_vecs(path, is_int, dtype):
    ptr, n, d = C.c_void_p(), C.c_uint64(), C.c_uint32()
    if _lib.host().bs_read_vecs(path.encode(), is_int, C.byref(ptr), C.byref(n), C.byref(d)):
        _err("read " + path)
    return _take(ptr, n.value * d.value, dtype).reshape(n.value, d.value)


def write_fvecs(path: str, a: np.ndarray):
    a = np.ascontiguousarray(a, dtype=np.float32)
    if _lib.host().bs_write_vecs(path.encode(), 0, _p(a), a.shape[0], a.shape[1]):
        _err("write " + path)


def write_ivecs(path: str, a: np.ndarray):
    a = np.ascontiguousarray(a, dtype=np.int32)
    if _lib.host().bs_write_vecs(path.encode(), 1, _p(a), a.shape[0], a.shape[1]):
        _err("write " + path)


def read_graph(path: str) -> np.ndarray:
    ptr, n, deg = C.c_void_p(), C.c_uint64(), C.c_uint32()
    if _lib.host().bs_read_graph(path.encode(), C.byref(ptr), C.byref(n), C.byref(deg)):
        _err("read " + path)
    return _take(ptr, n.value * deg.value, np.uint32).reshape(n.value, deg.value)


def write_graph(path: str, edges: np.ndarray):
    e = np.ascontiguousarray(edges, dtype=np.uint32)
    if _lib.host().bs_write_graph(path.encode(), _p(e), e.shape[0], e.shape[1]):
        _err("write " + path)


def read_codebook(path: str, n: int, dim: int, degree: int):
    """returns entry, codes (n, degree*wpp) u32, factors (n, 3*degree) f32, signs (pdim,) f32"""
    entry, pdim = C.c_uint32(), C.c_uint32()
    pc, pf, ps = C.c_void_p(), C.c_void_p(), C.c_void_p()
    if _lib.host().bs_read_codebook(path.encode(), n, dim, degree, C.byref(entry), C.byref(pc), C.byref(pf),
                                    C.byref(ps), C.byref(pdim)):
        _err("read " + path)
    wpp = pdim.value // 32
    codes = _take(pc, n * degree * wpp, np.uint32).reshape(n, degree * wpp)
    factors = _take(pf, n * 3 * degree, np.float32).reshape(n, 3 * degree)
    signs = _take(ps, pdim.value, np.float32)
    return entry.value, codes, factors, signs


def write_codebook(path, vecs, edges, entry, codes, factors, signs):
    vecs = np.ascontiguousarray(vecs, dtype=np.float32)
    edges = np.ascontiguousarray(edges, dtype=np.uint32)
    codes = np.ascontiguousarray(codes, dtype=np.uint32)
    factors = np.ascontiguousarray(factors, dtype=np.float32)
    signs = np.ascontiguousarray(signs, dtype=np.float32)
    if _lib.host().bs_write_codebook(path.encode(), _p(vecs), _p(edges), vecs.shape[0], vecs.shape[1],
                                     edges.shape[1], entry, _p(codes), _p(factors), _p(signs), signs.shape[0]):
        _err("write " + path)


# ---- search pre/post steps (src/gpu_cli.cu:28-83) -----------------------------------------

def entry_point(vecs: np.ndarray) -> int:
    v = np.ascontiguousarray(vecs, dtype=np.float32)
    return int(_lib.host().bs_entry_point(_p(v), v.shape[0], v.shape[1]))


def recall(pred: np.ndarray, gt: np.ndarray) -> Tuple[float, int]:
    """gpu_cli recall: dedup, skip 0xFFFFFFFF, divide by nq*min(K, gt_k); (recall, duplicates)"""
    p = np.ascontiguousarray(pred, dtype=np.uint32)
    g = np.ascontiguousarray(gt, dtype=np.int32)
    dups = C.c_uint64()
    r = _lib.host().bs_recall(_p(p), p.shape[0], p.shape[1], _p(g), g.shape[1], C.byref(dups))
    return float(r), int(dups.value)


# ---- synthetic inputs ------------------------------------------------------------------

def gen_mixture(n, dim, centres, lo, hi, sigma, clamp_min=0.0, seed_c=101, seed_x=202) -> np.ndarray:
    out = np.empty((n, dim), dtype=np.float32)
    cm = -math.inf if clamp_min is None else clamp_min
    if _lib.host().bs_gen_mixture(_p(out), n, dim, centres, lo, hi, sigma, cm, seed_c, seed_x):
        _err("gen_mixture")
    return out


def gen_normalized(n, dim, seed) -> np.ndarray:
    out = np.empty((n, dim), dtype=np.float32)
    if _lib.host().bs_gen_normalized(_p(out), n, dim, seed):
        _err("gen_normalized")
    return out


def groundtruth(base, queries, k, threads=0) -> np.ndarray:
    b = np.ascontiguousarray(base, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    out = np.empty((q.shape[0], k), dtype=np.int32)
    if _lib.host().bs_groundtruth(_p(b), b.shape[0], _p(q), q.shape[0], b.shape[1], k, _p(out), threads):
        _err("groundtruth")
    return out


def groundtruth_refine(base, queries, cand, k, threads=0) -> np.ndarray:
    b = np.ascontiguousarray(base, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    c = np.ascontiguousarray(cand, dtype=np.int64)
    out = np.empty((q.shape[0], k), dtype=np.int32)
    if _lib.host().bs_groundtruth_refine(_p(b), b.shape[0], _p(q), q.shape[0], b.shape[1], _p(c), c.shape[1], k,
                                         _p(out), threads):
        _err("groundtruth_refine")
    return out


# ---- index construction ----------------------------------------------------------------

def build_vamana(vecs, degree=32, beam_width=128, alpha=2.0, seed=1234, exact=True, threads=0,
                 verbose=False) -> np.ndarray:
    v = np.ascontiguousarray(vecs, dtype=np.float32)
    edges = np.empty((v.shape[0], degree), dtype=np.uint32)
    if _lib.host().bs_build_vamana(_p(v), v.shape[0], v.shape[1], degree, beam_width, alpha, seed,
                                   1 if exact else 0, threads, _p(edges), 1 if verbose else 0):
        _err("build_vamana")
    return edges


def build_rabitq(vecs, edges, seed=12345, threads=0):
    """returns entry, codes (n, degree*wpp), factors (n, 3*degree), signs (pdim,)"""
    v = np.ascontiguousarray(vecs, dtype=np.float32)
    e = np.ascontiguousarray(edges, dtype=np.uint32)
    n, dim = v.shape
    deg = e.shape[1]
    pdim = int(_lib.host().bs_rabitq_padded_dim(dim))
    wpp = pdim // 32
    codes = np.empty((n, deg * wpp), dtype=np.uint32)
    factors = np.empty((n, 3 * deg), dtype=np.float32)
    signs = np.empty(pdim, dtype=np.float32)
    entry = C.c_uint32()
    if _lib.host().bs_build_rabitq(_p(v), _p(e), n, dim, deg, seed, threads, _p(codes), _p(factors), _p(signs),
                                   C.byref(entry)):
        _err("build_rabitq")
    return int(entry.value), codes, factors, signs


def padded_dim(dim: int) -> int:
    return int(_lib.host().bs_rabitq_padded_dim(dim))
