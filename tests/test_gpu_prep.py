"""Index preparation on the MI355X: the entry point of compute_entry_point
(src/gpu_cli.cu:55-83) computed on the device equals the host restatement (bs_entry_point,
itself pinned to the reference's fixture entries) node for node."""
import numpy as np
import pytest

from beam_search_collab_amd import host, search

pytestmark = pytest.mark.gpu


def gpu_entry(base):
    g = search.GPUGraph(base, np.zeros((base.shape[0], 1), np.uint32))
    try:
        return g.entry_point()
    finally:
        g.close()


@pytest.mark.parametrize("name", ["d32", "d100"])
def test_entry_point_reference_fixture(gpu, golden_sets, name):
    arrays, _ = golden_sets[name]
    assert gpu_entry(arrays["base"]) == int(arrays["entry"])


@pytest.mark.parametrize("n,dim", [(1, 8), (2, 3), (257, 1), (5000, 16), (5000, 100), (70001, 128), (3000, 960),
                                   (513, 1024)])
def test_entry_point_matches_host(gpu, n, dim):
    rng = np.random.default_rng(n + dim)
    base = (rng.standard_normal((n, dim)) * 30 + 50).astype(np.float32)
    assert gpu_entry(base) == host.entry_point(base)
    mix = host.gen_mixture(n, dim, 8, 0.0, 128.0, 12.0, 0.0, 3, 4)
    assert gpu_entry(mix) == host.entry_point(mix)


def test_entry_point_ties_and_non_finite_rows(gpu):
    # identical rows: the first one
    assert gpu_entry(np.ones((300, 20), np.float32)) == 0
    # the nearest row repeated: the first copy wins (strict <)
    rng = np.random.default_rng(1)
    base = rng.standard_normal((1000, 24)).astype(np.float32)
    e = host.entry_point(base)
    base2 = np.concatenate([base[:e], base[e:e + 1], base[e:]])  # duplicate at e and e + 1
    assert host.entry_point(base2) == e
    assert gpu_entry(base2) == e
    # rows with inf / nan never win (dist < best fails), as on the host
    base3 = base.copy()
    base3[::7, 3] = np.inf
    base3[5, 0] = np.nan
    assert gpu_entry(base3) == host.entry_point(base3)


def _graph(n, dim, degree, seed, kind="mixture"):
    if kind == "mixture":
        base = host.gen_mixture(n, dim, 8, 0.0, 128.0, 12.0, 0.0, seed, seed + 1)
    else:
        base = host.gen_normalized(n, dim, seed)
    edges = host.build_vamana(base, degree, 2 * degree, 1.2, 7, exact=False, threads=0)
    return base, edges


@pytest.mark.parametrize("n,dim,degree,kind", [(3000, 17, 8, "mixture"), (3000, 30, 16, "normalized"),
                                               (5000, 100, 32, "normalized"), (5000, 128, 32, "mixture"),
                                               (2000, 200, 24, "mixture"), (1500, 960, 32, "mixture"),
                                               (1000, 1024, 12, "normalized")])
def test_device_rabitq_codebook_is_byte_identical(gpu, n, dim, degree, kind):
    """bs_index_build_rabitq equals the host builder (itself byte-identical to the reference
    build_rabitq) in every code word, factor bit, sign and the medoid, with absent edges"""
    base, edges = _graph(n, dim, degree, dim + degree, kind)
    edges[::5, -1] = 0xFFFFFFFF
    edges[7, :] = 0xFFFFFFFF
    g = search.GPUGraph(base, edges)
    try:
        for seed in (12345, 3):
            e_d, c_d, f_d, s_d = g.build_rabitq(seed)
            e_h, c_h, f_h, s_h = host.build_rabitq(base, edges, seed)
            assert e_d == e_h
            assert np.array_equal(c_d, c_h)
            assert s_d.tobytes() == s_h.tobytes()
            bad = np.nonzero(f_d.view(np.uint32) != f_h.view(np.uint32))
            assert len(bad[0]) == 0, (dim, seed, bad[0][:5], bad[1][:5])
    finally:
        g.close()


@pytest.mark.parametrize("name", ["d32", "d100"])
def test_device_rabitq_codebook_reference_file(gpu, name):
    """the codebook file written from the device build has the sha256 of the reference
    build_rabitq's file for the same graph"""
    import hashlib, json, os, tempfile
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    meta = json.load(open(os.path.join(golden, f"build_{name}.json")))
    spec = meta["spec"]
    if spec["kind"] == "mixture":
        base = host.gen_mixture(spec["n"], spec["dim"], spec["centres"], 0.0, 128.0, 12.0, 0.0, 101, 202)
    else:
        base = host.gen_normalized(spec["n"], spec["dim"], 202)
    bg = meta["build_graph"]
    edges = host.build_vamana(base, bg["degree"], bg["beam"], bg["alpha"], bg["seed"], exact=True, threads=4)
    g = search.GPUGraph(base, edges)
    try:
        entry, codes, factors, signs = g.build_rabitq(meta["build_rabitq"]["seed"])
    finally:
        g.close()
    d = tempfile.mkdtemp()
    host.write_codebook(f"{d}/cb.bin", base, edges, entry, codes, factors, signs)
    assert hashlib.sha256(open(f"{d}/cb.bin", "rb").read()).hexdigest() == meta["codebook_sha256"]


@pytest.mark.parametrize("n,dim,degree,beam,alpha,kind", [
    (1, 8, 4, 8, 1.2, "mixture"), (7, 5, 4, 8, 1.0, "normalized"), (300, 24, 8, 16, 1.2, "mixture"),
    (3000, 32, 16, 32, 2.0, "mixture"), (4000, 100, 32, 64, 1.2, "normalized"),
    (5000, 128, 32, 128, 2.0, "mixture"), (2500, 48, 64, 100, 1.5, "normalized"),
    (1500, 200, 24, 256, 2.0, "mixture"), (1200, 17, 128, 128, 1.2, "mixture")])
def test_device_vamana_is_the_reference_graph(gpu, n, dim, degree, beam, alpha, kind):
    """bs_build_vamana_device gives the host exact builder's rows (the host builder is
    byte-identical to the reference build_graph), including tiny n, odd dims, degree 128
    and beams that are not a multiple of 64"""
    if kind == "mixture":
        base = host.gen_mixture(n, dim, 6, 0.0, 50.0, 4.0, 0.0, n + dim, degree)
    else:
        base = host.gen_normalized(n, dim, n + degree)
    for seed in (7, 1234):
        want = host.build_vamana(base, degree, beam, alpha, seed, exact=True, threads=0)
        got = search.build_vamana_device(base, degree, beam, alpha, seed)
        bad = np.nonzero((got != want).any(1))[0]
        assert len(bad) == 0, (n, dim, degree, seed, len(bad), bad[:5], got[bad[0]], want[bad[0]])


def test_device_vamana_duplicate_points(gpu):
    """repeated rows give equal distances: ties resolved by node id as the reference does"""
    rng = np.random.default_rng(4)
    base = rng.integers(0, 4, (2000, 16)).astype(np.float32)
    want = host.build_vamana(base, 12, 32, 1.2, 5, exact=True, threads=0)
    got = search.build_vamana_device(base, 12, 32, 1.2, 5)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("name", ["d32", "d100"])
def test_device_vamana_reference_file(gpu, name):
    """the graph file written from the device build has the sha256 of the reference
    build_graph's file"""
    import hashlib, json, os, tempfile
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    meta = json.load(open(os.path.join(golden, f"build_{name}.json")))
    spec = meta["spec"]
    if spec["kind"] == "mixture":
        base = host.gen_mixture(spec["n"], spec["dim"], spec["centres"], 0.0, 128.0, 12.0, 0.0, 101, 202)
    else:
        base = host.gen_normalized(spec["n"], spec["dim"], 202)
    bg = meta["build_graph"]
    edges = search.build_vamana_device(base, bg["degree"], bg["beam"], bg["alpha"], bg["seed"])
    d = tempfile.mkdtemp()
    host.write_graph(f"{d}/g.bin", edges)
    assert hashlib.sha256(open(f"{d}/g.bin", "rb").read()).hexdigest() == meta["graph_sha256"]
