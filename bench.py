"""Benchmark of the GPU graph beam search on one MI355X.

Workload (synthetic, seeded): 1M x 128 fp32 base from a 64-centre Gaussian mixture
(centres ~U[0,128], sigma 12, clamped >= 0), 10k queries drawn the same way, degree-32
Vamana graph (beam 128, alpha 2.0, seed 1234), base mode K=100, topk_size=256,
filter_capacity=1024, reset_interval=16, max_iterations=1024.  A "step" is one search of
all 10k queries with the queries already resident in HBM.

    python bench.py [--gpus 1] [--steps 5] [--warmup 1] [--n 1000000] [--nq 10000]
                    [--mode base] [--topk 256] [--K 100] [--no-cpu]

Prints one JSON line (see the repository contract) with `roofline` (algorithmic bytes of
the search kernel / its average launch time, HIP events on the launch stream) and
`cpu_baseline` (the reference cpu_cli, built from the reference sources into oracle/_ref,
on a bounded query sample on this host's cores; the oracle port when _ref is absent).
"""
import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--nq", type=int, default=10_000)
    ap.add_argument("--dim", type=int, default=128)
    ap.add_argument("--degree", type=int, default=32)
    ap.add_argument("--mode", default="base")
    ap.add_argument("--topk", type=int, default=256)
    ap.add_argument("--K", type=int, default=100)
    ap.add_argument("--cap", type=int, default=1024)
    ap.add_argument("--reset", type=int, default=16)
    ap.add_argument("--max-it", type=int, default=1024)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-procs", type=int, default=0)
    ap.add_argument("--cpu-queries", type=int, default=400, help="queries per CPU process")
    ap.add_argument("--sweep", default="", help="comma list of topk values to sweep (extra lines on stderr)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="run one elementwise copy of this many MiB first (HBM-counter calibration under rocprofv3)")
    return ap.parse_args()


def gt_gpu(base_t, q_t, k, margin=28):
    """exact top-k: fp32 GEMM candidates on the GPU, exact fp64 re-scoring on the host"""
    import numpy as np
    import torch
    from beam_search_collab_amd import host
    nq = q_t.shape[0]
    kk = k + margin
    bn = (base_t * base_t).sum(1)
    cand = torch.empty((nq, kk), dtype=torch.int64, device=q_t.device)
    for i in range(0, nq, 1024):
        q = q_t[i:i + 1024]
        best_d = None
        best_i = None
        for j in range(0, base_t.shape[0], 262144):
            b = base_t[j:j + 262144]
            d = bn[j:j + 262144][None, :] - 2.0 * (q @ b.T)
            v, ix = torch.topk(d, kk, dim=1, largest=False)
            ix = ix + j
            if best_d is None:
                best_d, best_i = v, ix
            else:
                cd = torch.cat([best_d, v], 1)
                ci = torch.cat([best_i, ix], 1)
                v2, sel = torch.topk(cd, kk, dim=1, largest=False)
                best_d, best_i = v2, torch.gather(ci, 1, sel)
        cand[i:i + 1024] = best_i
    return host.groundtruth_refine(base_t.cpu().numpy(), q_t.cpu().numpy(), cand.cpu().numpy(), k)


def cpu_baseline(files, nq_total, args, entry_line_check=None):
    """reference cpu_cli on P query shards in parallel processes, one core each"""
    import numpy as np
    from beam_search_collab_amd import host
    from oracle import pyoracle as po
    ref = os.path.join(po.REF_DIR, "cpu_cli")
    P = args.cpu_procs or min(16, os.cpu_count() or 1)
    per = min(args.cpu_queries, nq_total // P)
    q = host.read_fvecs(files["query"])
    gt = host.read_ivecs(files["gt"])
    shards = []
    for p in range(P):
        qs = q[p * per:(p + 1) * per]
        qf = os.path.join(files["dir"], f"q_shard{p}.fvecs")
        gf = os.path.join(files["dir"], f"gt_shard{p}.ivecs")
        host.write_fvecs(qf, qs)
        host.write_ivecs(gf, gt[p * per:(p + 1) * per])
        shards.append((qf, gf))
    if os.path.exists(ref):
        procs = []
        for p, (qf, gf) in enumerate(shards):
            cfg = {"data": {"graph": files["graph"], "base": files["base"], "query": qf, "gt": gf},
                   "search": {"mode": "base", "K": args.K, "topk_size": args.topk,
                              "max_iterations": args.max_it}}
            cmd = [ref]
            if _has_taskset():
                cmd = ["taskset", "-c", str(p % (os.cpu_count() or 1))] + cmd
            pr = subprocess.Popen(cmd, stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
            pr.stdin.write(json.dumps(cfg))
            pr.stdin.close()
            procs.append(pr)
        times, recalls = [], []
        for pr in procs:
            out = pr.stdout.read()
            pr.wait()
            if pr.returncode != 0:
                raise RuntimeError("cpu_cli failed: " + pr.stderr.read()[-400:])
            for line in out.splitlines():
                if "time:" in line:
                    times.append(float(line.split("time:")[1].split("ms")[0]))
                if line.startswith("recall@"):
                    recalls.append(float(line.split(":")[1]))
        qps_all = P * per / (max(times) / 1000.0)
        qps_1 = per / (sum(times) / len(times) / 1000.0)
        return {"value": round(qps_all, 1), "unit": "queries/s", "cores": P, "kind": "reference",
                "sample": f"{P} processes x {per} queries of the same 10k-query workload (one core each, "
                          f"taskset), reference cpu_cli base mode built from source, search time only",
                "one_core_qps": round(qps_1, 1), "recall_at_K": round(sum(recalls) / len(recalls), 4)}
    # oracle port (single thread) when the reference binary is absent
    base = host.read_fvecs(files["base"])
    edges = host.read_graph(files["graph"])
    oi = po.OracleIndex(base, edges)
    t = time.time()
    oi.search(q[:per], args.K, po.BASE_CPUREF, args.topk, files["entry"], args.max_it, args.cap, 0, po.L2_SEQ)
    dt = time.time() - t
    return {"value": round(per / dt, 1), "unit": "queries/s", "cores": 1, "kind": "port",
            "sample": f"{per} queries, CPU oracle restatement of cpu_search_base.hpp, one thread"}


def kernel_name(args):
    tr = 1 if args.topk <= 64 else 2 if args.topk <= 128 else 4 if args.topk <= 256 else 8
    cr = 1 if args.degree <= 64 else 2
    qm = 1 if (args.dim + 3) // 4 <= 64 else 4
    mode = {"base": 0, "bwarp": 1, "rabitq": 2}.get(args.mode.rstrip("0123456789"), 0)
    return f"bsd::search_kernel<{tr}, {cr}, {qm}, {mode}>"


def measured_traffic(args):
    """HBM bytes per launch of the search kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE / WRITE_SIZE scaled by a 1 GiB copy), for the default workload only."""
    default = (args.n, args.nq, args.dim, args.degree, args.mode, args.topk, args.K, args.cap, args.reset) == \
        (1_000_000, 10_000, 128, 32, "base", 256, 100, 1024, 16)
    path = os.path.join(ROOT, "profiles", "search_kernel_base_1Mx128_traffic.json")
    if not default or not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)["traffic_bytes"]


def _has_taskset():
    from shutil import which
    return which("taskset") is not None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the search shards "
              "by queries (independent units, no exchange between GPUs), so N GPUs run N disjoint query "
              "shards of the same replicated index", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from beam_search_collab_amd import host, search

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    dev = torch.device("cuda:0")
    t0 = time.time()
    base = host.gen_mixture(args.n, args.dim, 64, 0.0, 128.0, 12.0, 0.0, 101, 202)
    queries = host.gen_mixture(args.nq, args.dim, 64, 0.0, 128.0, 12.0, 0.0, 101, 303)
    log(f"data {args.n}x{args.dim}, {args.nq} queries: {time.time() - t0:.1f}s")
    t1 = time.time()
    edges = host.build_vamana(base, args.degree, 128, 2.0, 1234, exact=False, verbose=True)
    log(f"Vamana graph R={args.degree}: {time.time() - t1:.1f}s")
    t1 = time.time()
    base_t = torch.from_numpy(base).to(dev)
    q_t = torch.from_numpy(queries).to(dev)
    gt = gt_gpu(base_t, q_t, 100)
    del base_t
    torch.cuda.empty_cache()
    log(f"ground truth top-100: {time.time() - t1:.1f}s")
    entry = host.entry_point(base)
    if args.calib_copy_mib:
        # a plain read-once/write-once kernel of known size: rocprofv3 --pmc FETCH_SIZE /
        # WRITE_SIZE on it gives the counter-to-bytes factor used for the search kernel
        x = torch.ones(args.calib_copy_mib << 18, dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        torch.add(x, 1.0, out=y)
        torch.cuda.synchronize()
        log(f"calibration copy: {args.calib_copy_mib} MiB read + {args.calib_copy_mib} MiB written")
        del x, y
    g = search.GPUGraph(base, edges)
    cfg = search.GPUBaseSearchCfg(args.topk, args.cap, entry, args.max_it, args.reset)
    nq, K = args.nq, args.K
    res_t = torch.empty((nq, K), dtype=torch.int32, device=dev)
    pq_t = torch.zeros((nq, 5), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def step(per_query=0):
        g.search_device(q_t.data_ptr(), nq, res_t.data_ptr(), K, args.mode, cfg, d_per_query=per_query,
                        stream=stream)

    for _ in range(args.warmup):
        step(pq_t.data_ptr())
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    tt = time.time()
    for s in range(args.steps):
        ev[s][0].record()
        step()
        ev[s][1].record()
    torch.cuda.synchronize()
    wall = time.time() - tt
    kms = [a.elapsed_time(b) for a, b in ev]
    ms_per_step = wall * 1000.0 / args.steps
    avg_kernel_ms = sum(kms) / len(kms)
    ids = res_t.cpu().numpy().view(np.uint32)
    r_k, dups = host.recall(ids, gt)
    r_10, _ = host.recall(ids[:, :10], gt[:, :10])
    pq = pq_t.cpu().numpy().astype(np.int64)
    E, D = int(pq[:, 1].sum()), int(pq[:, 2].sum())
    d, R = args.dim, args.degree
    # base/warp byte model: B_q = 4d + E*4R + D*4d + 4K (query, adjacency rows, gathered
    # vectors, results), summed over the launch's queries
    bytes_launch = nq * (4 * d + 4 * K) + E * 4 * R + D * 4 * d
    achieved = bytes_launch / (avg_kernel_ms / 1000.0) / 1e9
    qps = nq / (ms_per_step / 1000.0)
    log(f"search: {ms_per_step:.2f} ms/step, kernel {avg_kernel_ms:.2f} ms, {qps:.0f} QPS, "
        f"recall@{K} {r_k:.4f} recall@10 {r_10:.4f}, E/q {E / nq:.1f} D/q {D / nq:.1f}, "
        f"{achieved:.0f} GB/s algorithmic")

    for tk in [int(x) for x in args.sweep.split(",") if x]:
        c2 = search.GPUBaseSearchCfg(tk, args.cap, entry, args.max_it, args.reset)
        k2 = min(K, tk)
        r2 = torch.empty((nq, k2), dtype=torch.int32, device=dev)
        st = g.search_device(q_t.data_ptr(), nq, r2.data_ptr(), k2, args.mode, c2, stream=stream, sync=True)
        st = g.search_device(q_t.data_ptr(), nq, r2.data_ptr(), k2, args.mode, c2, stream=stream, sync=True)
        i2 = r2.cpu().numpy().view(np.uint32)
        log(f"sweep topk={tk}: kernel {st['kernel_ms']:.2f} ms, {nq / st['kernel_ms'] * 1000:.0f} QPS, "
            f"recall@10 {host.recall(i2[:, :10], gt[:, :10])[0]:.4f}")

    cpu = None
    if not args.no_cpu:
        t1 = time.time()
        tmp = tempfile.mkdtemp(prefix="bs_bench_")
        files = {"dir": tmp, "base": f"{tmp}/base.fvecs", "graph": f"{tmp}/graph.bin", "query": f"{tmp}/q.fvecs",
                 "gt": f"{tmp}/gt.ivecs", "entry": entry}
        host.write_fvecs(files["base"], base)
        host.write_graph(files["graph"], edges)
        host.write_fvecs(files["query"], queries)
        host.write_ivecs(files["gt"], gt)
        cpu = cpu_baseline(files, nq, args)
        for f in os.listdir(tmp):
            os.remove(os.path.join(tmp, f))
        os.rmdir(tmp)
        log(f"cpu baseline: {cpu} ({time.time() - t1:.1f}s)")

    traffic = measured_traffic(args)
    out = {
        "metric": "QPS @ recall@10>=0.95, 1Mx128 fp32, 1 MI355X; achieved HBM GB/s",
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded 64-centre Gaussian mixture, built in-run)",
        "config": {"workload": f"base-mode graph beam search, {args.n}x{args.dim} fp32, {nq} queries, "
                               f"degree-{R} Vamana (beam 128, alpha 2.0, seed 1234)",
                   "mode": args.mode, "K": K, "topk_size": args.topk, "filter_capacity": args.cap,
                   "reset_interval": args.reset, "max_iterations": args.max_it,
                   "recall_at_10": round(r_10, 4), f"recall_at_{K}": round(r_k, 4), "duplicates": dups,
                   "expansions_per_query": round(E / nq, 2), "dist_evals_per_query": round(D / nq, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": kernel_name(args), "avg_launch_ms": round(avg_kernel_ms, 3),
                     "bytes_per_launch": bytes_launch},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
