"""Oracle fastscan (quantizer, raw sums, estimate) against the reference's own host
restatement of GPU fastscan (unittest/test_fastscan.cu:54-145), via committed golden
vectors, plus closed forms."""
import numpy as np
import pytest

from conftest import load_fastscan_golden
from oracle import pyoracle as po


@pytest.mark.parametrize("seed", [42, 123])
def test_quantize_raw_estimate_match_reference_golden(seed):
    recs = load_fastscan_golden(seed)
    assert len(recs) == 48
    dims = {r["dim"] for r in recs}
    assert any(d & (d - 1) for d in dims), "non-power-of-two dims covered"
    for r in recs:
        codes, low, width, sq = po.quantize(r["query"], r["signs"], r["dim"], r["seed"], dither=True)
        assert np.array_equal(codes, r["codes"])
        assert np.float32(low).tobytes() == r["low"].tobytes()
        assert np.float32(width).tobytes() == r["width"].tobytes()
        assert sq == r["sum_q"]
        wpp = r["pdim"] // 32
        for n in range(r["nn"]):
            raw = po.raw_dot(r["codes"], r["nbrs"][n * wpp:(n + 1) * wpp], r["pdim"])
            assert raw == r["raw"][n]
            deg = r["degree"]
            est = po.estimate(raw, r["sum_q"], float(r["width"]), float(r["low"]), float(r["factors"][n]),
                              float(r["factors"][deg + n]), float(r["factors"][2 * deg + n]), float(r["exact"]))
            assert np.float32(est).tobytes() == r["est"][n].tobytes()


def test_raw_dot_closed_form():
    rng = np.random.default_rng(5)
    for pdim in (32, 64, 128, 1024):
        codes = rng.integers(0, 64, pdim).astype(np.uint8)
        words = rng.integers(0, 2**32, pdim // 32, dtype=np.uint64).astype(np.uint32)
        bits = np.unpackbits(words.view(np.uint8), bitorder="little")[:pdim]
        assert po.raw_dot(codes, words, pdim) == int((bits.astype(np.int64) * codes).sum())


def test_quantizer_codes_track_rotation():
    """codes ~ (r - low)/width within one dither step; the extremes map to 0 and 63;
    sum_q is the code sum.  r = H (signs * q) with H the Sylvester-Hadamard matrix."""
    rng = np.random.default_rng(9)
    for dim in (32, 100, 128, 960):
        pdim = po.lib().orc_padded_dim(dim)
        q = rng.standard_normal(dim).astype(np.float32)
        s = np.where(rng.integers(0, 2, pdim) > 0, 1.0, -1.0).astype(np.float32)
        H = np.array([[1.0]])
        while H.shape[0] < pdim:
            H = np.block([[H, H], [H, -H]])
        x = np.zeros(pdim)
        x[:dim] = q.astype(np.float64) * s[:dim]
        r = H @ x
        codes, low, width, sq = po.quantize(q, s, dim, 0, dither=True)
        assert abs(low - r.min()) <= 1e-4 * max(1.0, abs(r.min()))
        assert abs(width - (r.max() - r.min()) / 63) <= 1e-4 * width
        t = (r - r.min()) / ((r.max() - r.min()) / 63)
        assert np.all(codes >= np.floor(t) - 1) and np.all(codes <= np.ceil(t) + 1)
        assert codes[np.argmin(r)] == 0 and codes[np.argmax(r)] in (62, 63)
        assert sq == int(codes.astype(np.int64).sum())


def test_dither_hash_is_the_reference_mixer():
    # values of the two-round 0x45d9f3b mixer (fastscan.cuh:125-134) for small inputs,
    # computed by hand-expansion of the integer recurrence in Python's arbitrary precision
    def mix(a, b):
        a ^= b
        a ^= a >> 16
        a = (a * 0x45D9F3B) & 0xFFFFFFFF
        a ^= a >> 16
        a = (a * 0x45D9F3B) & 0xFFFFFFFF
        a ^= a >> 16
        return a
    for a, b in [(0, 0), (0, 1), (0, 127), (12345, 7), (0xFFFFFFFF, 3)]:
        assert po.lib().orc_dither_hash(a, b) == mix(a, b)
    assert po.lib().orc_dither_hash(0, 0) == 0


def test_l2_orders_against_fp64_and_integers():
    """orc_l2_wave (the kernels' lane order), orc_l2_wave_lanes (its one-chunk-per-lane form,
    the RaBitQ search with narrow codes) and orc_l2_seq (the reference CPU's sequential sum):
    within 1e-5 relative of an fp64 sum, and exact when every partial sum is an integer below
    2^24 (then every order gives the same float); the two lane orders are different orders
    (they differ in the last bits on some inputs of more than 4 dims)"""
    rng = np.random.default_rng(4)
    differ = 0
    for dim in (1, 3, 16, 25, 32, 100, 128, 200, 384, 960, 1024):
        for _ in range(20):
            a = rng.standard_normal(dim).astype(np.float32) * 10
            b = rng.standard_normal(dim).astype(np.float32) * 10
            want = float(((a.astype(np.float64) - b.astype(np.float64)) ** 2).sum())
            assert abs(po.l2_wave(a, b) - want) <= 1e-5 * want
            assert abs(po.l2_wave_lanes(a, b) - want) <= 1e-5 * want
            assert abs(po.l2_seq(a, b) - want) <= 1e-5 * want
            differ += po.l2_wave(a, b) != po.l2_wave_lanes(a, b)
            ai = rng.integers(0, 16, dim).astype(np.float32)
            bi = rng.integers(0, 16, dim).astype(np.float32)
            exact = int(((ai.astype(np.int64) - bi.astype(np.int64)) ** 2).sum())
            assert po.l2_wave(ai, bi) == exact and po.l2_seq(ai, bi) == exact
            assert po.l2_wave_lanes(ai, bi) == exact
        if dim <= 4:  # one chunk: both forms are the same sum
            assert all(po.l2_wave(x, y) == po.l2_wave_lanes(x, y)
                       for x, y in ((rng.standard_normal(dim).astype(np.float32),
                                     rng.standard_normal(dim).astype(np.float32)) for _ in range(5)))
    assert differ > 20
