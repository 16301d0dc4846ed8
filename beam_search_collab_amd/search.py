"""Host-side mirror of the reference's GPU search interface (src/gpu_cli.cu).

Names follow the reference: GPUGraph (gpu_graph.cuh:81-146) owns the device copy of
the graph, attach_rabitq() plays GPURabitq (rabitq.cuh:67-110), the config classes are
GPUBaseSearchCfg / GPURabitqSearchCfg (gpu_search_base.cuh:17-23,
gpu_search_rabitq.cuh:21-26) and run_base / run_warp / run_rabitq dispatch the modes
like src/gpu_cli.cu:140-349.  Every call goes through libbs_hip.so; configuration errors
raise ValueError with the library's message (the reference prints it and exits 1).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np

from . import _lib

BS_BASE, BS_GROUP, BS_GROUP_BLOOM, BS_RABITQ = 0, 1, 2, 3
INVALID_ID = 0xFFFFFFFF

# gpu_cli "mode" strings (src/gpu_cli.cu:460-477)
MODES = {
    "base": (BS_BASE, 1),
    "warp1": (BS_GROUP, 1), "warp2": (BS_GROUP, 2), "warp4": (BS_GROUP, 4), "warp8": (BS_GROUP, 8),
    "bwarp1": (BS_GROUP_BLOOM, 1), "bwarp2": (BS_GROUP_BLOOM, 2), "bwarp4": (BS_GROUP_BLOOM, 4),
    "bwarp8": (BS_GROUP_BLOOM, 8),
    "rabitq": (BS_RABITQ, 1),
}


class BeamSearchError(RuntimeError):
    pass


def _check(rc: int, what: str):
    if rc != 0:
        msg = _lib.hip().bs_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise BeamSearchError(f"{what} failed ({rc}): {msg}")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


@dataclass
class GPUBaseSearchCfg:
    topk_size: int = 256
    filter_capacity: int = 1024
    entry_point: int = 0
    max_iterations: int = 1024
    reset_interval: int = 16


@dataclass
class GPURabitqSearchCfg:
    topk_size: int = 256
    filter_capacity: int = 1024
    entry_point: int = 0
    max_iterations: int = 1024


class GPUGraph:
    """Device-resident graph (vectors + fixed-degree adjacency) on the current GPU."""

    def __init__(self, vecs: np.ndarray, edges: np.ndarray):
        vecs = np.ascontiguousarray(vecs, dtype=np.float32)
        edges = np.ascontiguousarray(edges, dtype=np.uint32)
        if vecs.ndim != 2 or edges.ndim != 2 or vecs.shape[0] != edges.shape[0]:
            raise ValueError("vecs must be n x dim and edges n x degree")
        self.n, self.dim = vecs.shape
        self.degree = edges.shape[1]
        self._vecs = vecs  # host rows, for the exact fallback of groundtruth()
        self.padded_dim = 0
        h = C.c_void_p()
        _check(_lib.hip().bs_index_create(_ptr(vecs), _ptr(edges), self.n, self.dim, self.degree, C.byref(h)),
               "bs_index_create")
        self._h = h

    def attach_rabitq(self, codes: np.ndarray, factors: np.ndarray, signs: np.ndarray):
        codes = np.ascontiguousarray(codes, dtype=np.uint32)
        factors = np.ascontiguousarray(factors, dtype=np.float32)
        signs = np.ascontiguousarray(signs, dtype=np.float32)
        pdim = signs.shape[0]
        _check(_lib.hip().bs_index_attach_rabitq(self._h, _ptr(codes), _ptr(factors), _ptr(signs), pdim),
               "bs_index_attach_rabitq")
        self.padded_dim = pdim

    def entry_point(self) -> int:
        """compute_entry_point (src/gpu_cli.cu:55-83) on the device: same node as host.entry_point."""
        e = C.c_uint32(0)
        _check(_lib.hip().bs_index_entry_point(self._h, C.byref(e)), "bs_index_entry_point")
        return int(e.value)

    def build_rabitq(self, seed: int = 12345):
        """build_rabitq (src/build_rabitq.cpp) on the device from the uploaded graph:
        (entry, codes, factors, signs), byte-identical to host.build_rabitq."""
        pdim = 1
        while pdim < self.dim:
            pdim <<= 1
        wpp = pdim // 32
        codes = np.empty((self.n, self.degree * wpp), dtype=np.uint32)
        factors = np.empty((self.n, 3 * self.degree), dtype=np.float32)
        signs = np.empty(pdim, dtype=np.float32)
        e = C.c_uint32(0)
        _check(_lib.hip().bs_index_build_rabitq(self._h, seed, _ptr(codes), _ptr(factors), _ptr(signs), C.byref(e)),
               "bs_index_build_rabitq")
        return int(e.value), codes, factors, signs

    def set_query_order(self, mode: int):
        """0 off, 1 on for batches of >= 4096 queries (default), 2 always (bs_index_set_query_order)."""
        _check(_lib.hip().bs_index_set_query_order(self._h, mode), "bs_index_set_query_order")

    def label_costs(self) -> np.ndarray:
        """the expected search cost per pivot label calibrated at index creation
        (bs_index_label_costs), 256 floats"""
        out = np.empty(256, np.float32)
        _check(_lib.hip().bs_index_label_costs(self._h, _ptr(out)), "bs_index_label_costs")
        return out

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            _lib.hip().bs_index_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def search(self, queries: np.ndarray, K: int, mode: str = "base",
               cfg: Optional[object] = None, with_dists: bool = False) -> Tuple[np.ndarray, Optional[np.ndarray], dict]:
        """Search host queries; returns (ids nq x K, dists or None, stats)."""
        if mode not in MODES:
            raise ValueError(f"Unknown mode: {mode}")
        m, ny = MODES[mode]
        if cfg is None:
            cfg = GPURabitqSearchCfg() if m == BS_RABITQ else GPUBaseSearchCfg()
        c = make_cfg(m, ny, K, cfg)
        q = np.ascontiguousarray(queries, dtype=np.float32)
        if q.ndim != 2 or q.shape[1] != self.dim:
            raise ValueError(f"queries must be nq x {self.dim}")
        nq = q.shape[0]
        res = np.empty((nq, K), dtype=np.uint32)
        d = np.empty((nq, K), dtype=np.float32) if with_dists else None
        st = _lib.Stats()
        _check(_lib.hip().bs_search(self._h, C.byref(c), _ptr(q), nq, _ptr(res),
                                    _ptr(d) if d is not None else None, C.byref(st)), "bs_search")
        return res, d, st.as_dict()

    def groundtruth(self, queries: np.ndarray, k: int = 100, exact_fallback: bool = True) -> np.ndarray:
        """Exact k nearest rows (int32, -1 past the last row) by fp64 distance, ties by id.
        Matrix-core candidates with a per-query certificate; the queries without one are
        recomputed on the host (bs_groundtruth) unless exact_fallback is False, in which
        case their rows are -2."""
        q = np.ascontiguousarray(queries, dtype=np.float32)
        if q.ndim != 2 or q.shape[1] != self.dim:
            raise ValueError(f"queries must be nq x {self.dim}")
        nq = q.shape[0]
        out = np.empty((nq, k), dtype=np.int32)
        unc = np.zeros(nq, dtype=np.uint8)
        nu = C.c_uint64(0)
        _check(_lib.hip().bs_index_groundtruth(self._h, _ptr(q), nq, k, _ptr(out), _ptr(unc), C.byref(nu)),
               "bs_index_groundtruth")
        bad = np.nonzero(unc)[0]
        if len(bad):
            if exact_fallback:
                from . import host
                out[bad] = host.groundtruth(self._vecs, q[bad], k)
            else:
                out[bad] = -2
        return out

    def search_device(self, d_queries: int, nq: int, d_results: int, K: int, mode: str, cfg,
                      d_dists: int = 0, d_per_query: int = 0, stream: int = 0, sync: bool = False) -> dict:
        """Search device-resident buffers (raw device pointers, e.g. torch data_ptr())."""
        m, ny = MODES[mode]
        c = make_cfg(m, ny, K, cfg)
        st = _lib.Stats()
        _check(_lib.hip().bs_search_device(self._h, C.byref(c), C.c_void_p(d_queries), nq, C.c_void_p(d_results),
                                           C.c_void_p(d_dists) if d_dists else None,
                                           C.c_void_p(d_per_query) if d_per_query else None,
                                           C.c_void_p(stream) if stream else None, 1 if sync else 0, C.byref(st)),
               "bs_search_device")
        return st.as_dict()


    def search_device_noalloc(self, d_queries: int, nq: int, d_results: int, K: int, mode: str, cfg,
                              d_dists: int = 0, d_per_query: int = 0, stream: int = 0):
        """bs_search_device_noalloc: the same search, asynchronous on `stream`, allocating
        nothing (its scheduling workspace is a static device array; at most 262144 queries)."""
        m, ny = MODES[mode]
        c = make_cfg(m, ny, K, cfg)
        _check(_lib.hip().bs_search_device_noalloc(self._h, C.byref(c), C.c_void_p(d_queries), nq,
                                                   C.c_void_p(d_results), C.c_void_p(d_dists) if d_dists else None,
                                                   C.c_void_p(d_per_query) if d_per_query else None,
                                                   C.c_void_p(stream) if stream else None),
               "bs_search_device_noalloc")


def build_vamana_device(vecs: np.ndarray, degree: int = 32, beam_width: int = 128, alpha: float = 2.0,
                        seed: int = 1234, verbose: bool = False) -> np.ndarray:
    """build_graph (src/build_graph.cpp) on the device: the reference's graph, edge for
    edge (host.build_vamana with exact=True gives the same rows)."""
    v = np.ascontiguousarray(vecs, dtype=np.float32)
    if v.ndim != 2:
        raise ValueError("vecs must be n x dim")
    n, dim = v.shape
    edges = np.empty((n, degree), dtype=np.uint32)
    _check(_lib.hip().bs_build_vamana_device(_ptr(v), n, dim, degree, beam_width, alpha, seed, _ptr(edges),
                                             1 if verbose else 0), "bs_build_vamana_device")
    return edges


def make_cfg(mode: int, ny: int, K: int, cfg) -> _lib.SearchCfg:
    c = _lib.SearchCfg()
    c.mode = mode
    c.queries_per_group = ny
    c.K = K
    c.topk_size = cfg.topk_size
    c.filter_capacity = cfg.filter_capacity
    c.entry_point = cfg.entry_point
    c.max_iterations = cfg.max_iterations
    c.reset_interval = getattr(cfg, "reset_interval", 0)
    return c


# src/gpu_cli.cu:264-284 run_base, :209-234 run_warp<NY, Filter>, :319-349 run_rabitq<1>
def run_base(graph: GPUGraph, cfg: GPUBaseSearchCfg, queries: np.ndarray, K: int):
    return graph.search(queries, K, "base", cfg)


def run_warp(graph: GPUGraph, cfg: GPUBaseSearchCfg, queries: np.ndarray, K: int, ny: int = 1, bloom: bool = False):
    return graph.search(queries, K, ("bwarp" if bloom else "warp") + str(ny), cfg)


def run_rabitq(graph: GPUGraph, cfg: GPURabitqSearchCfg, queries: np.ndarray, K: int):
    return graph.search(queries, K, "rabitq", cfg)


# ---- primitive entry points ------------------------------------------------------

def debug_l2(graph: GPUGraph, queries: np.ndarray, qi: np.ndarray, ni: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(queries, dtype=np.float32)
    qi = np.ascontiguousarray(qi, dtype=np.uint32)
    ni = np.ascontiguousarray(ni, dtype=np.uint32)
    out = np.empty(qi.shape[0], dtype=np.float32)
    _check(_lib.hip().bs_debug_l2(graph.handle, _ptr(q), q.shape[0], _ptr(qi), _ptr(ni), qi.shape[0], _ptr(out)),
           "bs_debug_l2")
    return out


def debug_fastscan(query, signs, dim, seed, codes_nbr, factors, nn, degree, exact):
    pdim = 1
    while pdim < dim:
        pdim <<= 1
    query = np.ascontiguousarray(query, dtype=np.float32)
    signs = np.ascontiguousarray(signs, dtype=np.float32)
    codes_nbr = np.ascontiguousarray(codes_nbr, dtype=np.uint32)
    factors = np.ascontiguousarray(factors, dtype=np.float32)
    codes = np.empty(pdim, dtype=np.uint8)
    scal = np.empty(2, dtype=np.float32)
    sumq = np.empty(1, dtype=np.int32)
    raw = np.empty(nn, dtype=np.uint32)
    est = np.empty(nn, dtype=np.float32)
    _check(_lib.hip().bs_debug_fastscan(_ptr(query), _ptr(signs), dim, seed, _ptr(codes_nbr), _ptr(factors), nn,
                                        degree, float(exact), _ptr(codes), _ptr(scal), _ptr(sumq), _ptr(raw),
                                        _ptr(est)), "bs_debug_fastscan")
    return codes, float(scal[0]), float(scal[1]), int(sumq[0]), raw, est


def debug_beam(topk, keys, picks, pick_run):
    keys = np.ascontiguousarray(keys, dtype=np.uint64)
    nbatch, bsize = keys.shape
    picked = np.empty((nbatch, picks), dtype=np.uint32)
    beam = np.empty(topk, dtype=np.uint64)
    _check(_lib.hip().bs_debug_beam(topk, _ptr(keys), nbatch, bsize, picks, int(pick_run), _ptr(picked),
                                    _ptr(beam)), "bs_debug_beam")
    return picked, beam


def debug_sort(keys):
    keys = np.ascontiguousarray(keys, dtype=np.uint64)
    out = np.empty_like(keys)
    _check(_lib.hip().bs_debug_sort(_ptr(keys), keys.shape[0], _ptr(out)), "bs_debug_sort")
    return out


def debug_cost_order(signal):
    """(qmap, bucket) of the RaBitQ launch order for per-query cost signals (bs_debug_cost_order)"""
    signal = np.ascontiguousarray(signal, dtype=np.float32)
    n = signal.shape[0]
    qmap = np.empty(n, np.uint32)
    bucket = np.empty(n, np.uint32)
    _check(_lib.hip().bs_debug_cost_order(_ptr(signal), n, _ptr(qmap), _ptr(bucket)), "bs_debug_cost_order")
    return qmap, bucket


def debug_label_order(labels, lcost, g, X):
    """qmap of the base-family query order for given labels and per-label costs (None: plain label
    order); bs_debug_label_order"""
    labels = np.ascontiguousarray(labels, dtype=np.uint32)
    n = labels.shape[0]
    qmap = np.empty(n, np.uint32)
    lc = None if lcost is None else np.ascontiguousarray(lcost, dtype=np.float32)
    _check(_lib.hip().bs_debug_label_order(_ptr(labels), _ptr(lc) if lc is not None else None, n, g, X, _ptr(qmap)),
           "bs_debug_label_order")
    return qmap


def debug_mfma32(A, B):
    A = np.ascontiguousarray(A, dtype=np.float32).reshape(32, 2)
    B = np.ascontiguousarray(B, dtype=np.float32).reshape(2, 32)
    D = np.empty((32, 32), dtype=np.float32)
    _check(_lib.hip().bs_debug_mfma32(_ptr(A), _ptr(B), _ptr(D)), "bs_debug_mfma32")
    return D


def debug_filter(bloom, capacity, keys, qkeys):
    keys = np.ascontiguousarray(keys, dtype=np.uint32)
    qkeys = np.ascontiguousarray(qkeys, dtype=np.uint32)
    nbatch, bsize = keys.shape
    out_new = np.empty_like(keys)
    out_c = np.empty(qkeys.shape[0], dtype=np.uint32)
    _check(_lib.hip().bs_debug_filter(int(bloom), capacity, _ptr(keys), nbatch, bsize, _ptr(out_new), _ptr(qkeys),
                                      qkeys.shape[0], _ptr(out_c)), "bs_debug_filter")
    return out_new, out_c


def make_keys(dists: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """(orderable(dist) << 32) | (id << 1): the beam's key for unexpanded entries."""
    b = np.ascontiguousarray(dists, dtype=np.float32).view(np.uint32).astype(np.uint64)
    neg = (b & 0x80000000) != 0
    o = np.where(neg, (~b) & 0xFFFFFFFF, b | 0x80000000)
    return (o << np.uint64(32)) | ((np.asarray(ids, dtype=np.uint64) & 0x7FFFFFFF) << np.uint64(1))
