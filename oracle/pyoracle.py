"""ctypes bindings of oracle/bin/libbs_oracle.so (TEST INFRASTRUCTURE).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module,
as the checker.  The product path never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# BS_ORACLE_LIB / BS_ORACLE_MUTANT_LIB name other builds (the sanitizer build: make sanitize-check)
LIB_PATH = os.environ.get("BS_ORACLE_LIB") or os.path.join(HERE, "bin", "libbs_oracle.so")
REF_DIR = os.path.join(HERE, "_ref")

BASE_HASH, BASE_BLOOM, RABITQ_GPU, BASE_CPUREF, RABITQ_CPUREF = 0, 1, 2, 3, 4
L2_SEQ, L2_WAVE = 0, 1
EMPTY_KEY = 0xFFFFFFFFFFFFFFFF
INVALID_ID = 0xFFFFFFFF


class Index(C.Structure):
    _fields_ = [("vecs", C.c_void_p), ("edges", C.c_void_p), ("n", C.c_uint64), ("dim", C.c_int),
                ("degree", C.c_int), ("codes", C.c_void_p), ("factors", C.c_void_p), ("signs", C.c_void_p),
                ("padded_dim", C.c_int)]


class Cfg(C.Structure):
    _fields_ = [("mode", C.c_int), ("l2_kind", C.c_int), ("K", C.c_uint32), ("topk_size", C.c_uint32),
                ("filter_capacity", C.c_uint32), ("entry_point", C.c_uint32), ("max_iterations", C.c_int32),
                ("reset_interval", C.c_int32)]


class Stats(C.Structure):
    _fields_ = [("iterations", C.c_uint64), ("expansions", C.c_uint64), ("dist_evals", C.c_uint64),
                ("est_evals", C.c_uint64), ("rerank_evals", C.c_uint64)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: make -C oracle")
        L = C.CDLL(LIB_PATH)
        vp, u32, u64, i32, f32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32, C.c_float
        sig = {
            "orc_orderable": (u32, [f32]),
            "orc_make_key": (u64, [f32, u32, C.c_int]),
            "orc_l2_seq": (f32, [vp, vp, C.c_int]),
            "orc_l2_wave": (f32, [vp, vp, C.c_int]),
            "orc_l2_wave_lanes": (f32, [vp, vp, C.c_int]),
            "orc_padded_dim": (C.c_int, [C.c_int]),
            "orc_dither_hash": (u32, [u32, u32]),
            "orc_quantize_dither": (None, [vp, vp, C.c_int, u32, vp, vp, vp, vp]),
            "orc_quantize_round": (None, [vp, vp, C.c_int, vp, vp, vp, vp]),
            "orc_raw_dot": (u32, [vp, vp, C.c_int]),
            "orc_estimate": (f32, [u32, i32, f32, f32, f32, f32, f32, f32]),
            "orc_filter_run": (C.c_int, [C.c_int, u32, vp, C.c_int, C.c_int, vp, vp, C.c_int, vp]),
            "orc_bloom_hashes": (None, [u32, u32, vp]),
            "orc_base_state": (C.c_int, [C.POINTER(Index), C.POINTER(Cfg), vp, i32, vp, vp, vp]),
            "orc_beam_run": (C.c_int, [u32, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp]),
            "orc_search": (C.c_int, [C.POINTER(Index), C.POINTER(Cfg), vp, u64, vp, vp, vp]),
            "orc_entry_point": (u32, [vp, u64, C.c_int]),
            "orc_recall": (C.c_double, [vp, u64, C.c_int, vp, C.c_int, C.POINTER(u64)]),
            "orc_groundtruth": (None, [vp, u64, vp, u64, C.c_int, C.c_int, vp]),
        }
        for k, (r, a) in sig.items():
            f = getattr(L, k)
            f.restype, f.argtypes = r, a
        _lib = L
    return _lib


MUTANT_PATH = os.environ.get("BS_ORACLE_MUTANT_LIB") or os.path.join(HERE, "bin", "libbs_oracle_mutant.so")
MUTANT_SEEN_AT_ENTRY, MUTANT_REEXPAND, MUTANT_NO_DEDUP = 1, 2, 3
_mlib = None


def mutant_search(index, queries, K, mutant, topk, entry, max_it=1024, cap=1024):
    """ORC_RABITQ_GPU of the oracle built with a planted mistake (bs_oracle.c, ORC_MUTANTS):
    for tests that show a fixture tells the mistake apart"""
    global _mlib
    if _mlib is None:
        if not os.path.exists(MUTANT_PATH):
            raise ImportError(f"{MUTANT_PATH} missing: make -C oracle")
        _mlib = C.CDLL(MUTANT_PATH)
        _mlib.orc_search.restype = C.c_int
        _mlib.orc_search.argtypes = [C.POINTER(Index), C.POINTER(Cfg), C.c_void_p, C.c_uint64, C.c_void_p,
                                     C.c_void_p, C.c_void_p]
    C.c_int.in_dll(_mlib, "orc_mutant").value = int(mutant)
    return index.search(queries, K, RABITQ_GPU, topk, entry, max_it, cap, 0, L2_WAVE, _lib_handle=_mlib)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def l2_wave(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().orc_l2_wave(_p(a), _p(b), a.shape[0])


def l2_wave_lanes(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().orc_l2_wave_lanes(_p(a), _p(b), a.shape[0])


def l2_seq(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().orc_l2_seq(_p(a), _p(b), a.shape[0])


def quantize(query, signs, dim, seed=0, dither=True):
    pdim = lib().orc_padded_dim(dim)
    q = np.ascontiguousarray(query, np.float32)
    s = np.ascontiguousarray(signs, np.float32)
    codes = np.empty(pdim, np.uint8)
    low, width, sq = C.c_float(), C.c_float(), C.c_int32()
    if dither:
        lib().orc_quantize_dither(_p(q), _p(s), dim, seed, _p(codes), C.byref(low), C.byref(width), C.byref(sq))
    else:
        lib().orc_quantize_round(_p(q), _p(s), dim, _p(codes), C.byref(low), C.byref(width), C.byref(sq))
    return codes, low.value, width.value, sq.value


def raw_dot(codes, nbr_words, pdim):
    c = np.ascontiguousarray(codes, np.uint8)
    w = np.ascontiguousarray(nbr_words, np.uint32)
    return lib().orc_raw_dot(_p(c), _p(w), pdim)


def estimate(raw, sum_q, width, low, tx, fdq, fvq, exact):
    return lib().orc_estimate(raw, sum_q, width, low, tx, fdq, fvq, exact)


def filter_run(bloom, capacity, keys, qkeys):
    keys = np.ascontiguousarray(keys, np.uint32)
    qkeys = np.ascontiguousarray(qkeys, np.uint32)
    nb, bs = keys.shape
    out_new = np.empty_like(keys)
    out_c = np.empty(qkeys.shape[0], np.uint32)
    lib().orc_filter_run(int(bloom), capacity, _p(keys), nb, bs, _p(out_new), _p(qkeys), qkeys.shape[0], _p(out_c))
    return out_new, out_c


def bloom_hashes(capacity, key):
    h = np.empty(3, np.uint32)
    lib().orc_bloom_hashes(capacity, key, _p(h))
    return [int(x) for x in h]


def beam_run(topk, keys, picks, pick_run):
    keys = np.ascontiguousarray(keys, np.uint64)
    nb, bs = keys.shape
    picked = np.empty((nb, picks), np.uint32)
    beam = np.empty(topk, np.uint64)
    lib().orc_beam_run(topk, _p(keys), nb, bs, picks, int(pick_run), _p(picked), _p(beam))
    return picked, beam


class OracleIndex:
    def __init__(self, vecs, edges, codes=None, factors=None, signs=None):
        self.vecs = np.ascontiguousarray(vecs, np.float32)
        self.edges = np.ascontiguousarray(edges, np.uint32)
        self.codes = None if codes is None else np.ascontiguousarray(codes, np.uint32)
        self.factors = None if factors is None else np.ascontiguousarray(factors, np.float32)
        self.signs = None if signs is None else np.ascontiguousarray(signs, np.float32)
        ix = Index()
        ix.vecs, ix.edges = self.vecs.ctypes.data, self.edges.ctypes.data
        ix.n, ix.dim, ix.degree = self.vecs.shape[0], self.vecs.shape[1], self.edges.shape[1]
        if self.codes is not None:
            ix.codes, ix.factors, ix.signs = self.codes.ctypes.data, self.factors.ctypes.data, self.signs.ctypes.data
            ix.padded_dim = self.signs.shape[0]
        self.ix = ix

    def search(self, queries, K, mode, topk, entry, max_it=1024, cap=1024, reset=16, l2=L2_WAVE, _lib_handle=None):
        q = np.ascontiguousarray(queries, np.float32)
        nq = q.shape[0]
        c = Cfg(mode, l2, K, topk, cap, entry, max_it, reset)
        res = np.empty((nq, K), np.uint32)
        d = np.empty((nq, K), np.float32)
        st = (Stats * nq)()
        rc = (_lib_handle or lib()).orc_search(C.byref(self.ix), C.byref(c), _p(q), nq, _p(res), _p(d), C.cast(st, C.c_void_p))
        if rc != 0:
            raise ValueError("orc_search failed")
        stats = np.array([[s.iterations, s.expansions, s.dist_evals, s.est_evals, s.rerank_evals] for s in st],
                         dtype=np.uint64).reshape(nq, 5)
        return res, d, stats


    def base_state(self, query, mode, topk, entry, cap, reset, stop_iter, K=10, max_it=1024, l2=L2_WAVE):
        """beam keys and filter contents of one base/bwarp query after iteration stop_iter's
        merge and reset (hash: the stored ids; Bloom: the bit words)"""
        q = np.ascontiguousarray(query, np.float32)
        c = Cfg(mode, l2, K, topk, cap, entry, max_it, reset)
        beam = np.full(topk, EMPTY_KEY, np.uint64)
        filt = np.empty(max(cap, 32) * 2, np.uint32)
        nf = C.c_uint32(0)
        if lib().orc_base_state(C.byref(self.ix), C.byref(c), _p(q), stop_iter, _p(beam), _p(filt), C.byref(nf)) != 0:
            raise ValueError("orc_base_state failed")
        return beam, filt[: nf.value].copy()


def entry_point(vecs):
    v = np.ascontiguousarray(vecs, np.float32)
    return int(lib().orc_entry_point(_p(v), v.shape[0], v.shape[1]))


def groundtruth(base, queries, k):
    b = np.ascontiguousarray(base, np.float32)
    q = np.ascontiguousarray(queries, np.float32)
    out = np.empty((q.shape[0], k), np.int32)
    lib().orc_groundtruth(_p(b), b.shape[0], _p(q), q.shape[0], b.shape[1], k, _p(out))
    return out


def recall(pred, gt):
    p = np.ascontiguousarray(pred, np.uint32)
    g = np.ascontiguousarray(gt, np.int32)
    d = C.c_uint64()
    r = lib().orc_recall(_p(p), p.shape[0], p.shape[1], _p(g), g.shape[1], C.byref(d))
    return r, d.value
