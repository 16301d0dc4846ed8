/*
 * bs_hip.h -- C-ABI of the MI355X (gfx950) graph beam search: libbs_hip.so.
 *
 * This is the drop-in boundary for the reference's GPU search path.  The reference has
 * no FFI of its own: its boundary is C++ templates inside src/gpu_cli.cu
 *   host  run_base / run_warp<NY,Filter> / run_rabitq<NY>   (src/gpu_cli.cu:140-349)
 *   ->    kernel_{base,warp,rabitq}_search<<<...>>>          (src/gpu_cli.cu:87-136)
 *   ->    Searcher::search(query, results, K)                (gpu_search_base.cuh:65,
 *                                                             gpu_search_warp.cuh:54,
 *                                                             gpu_search_rabitq.cuh:65)
 * with the device-resident index of GPUGraph / GPURabitq (gpu_graph.cuh:81-146,
 * rabitq.cuh:67-110).  The entry points below replace exactly that layer; a C++ host
 * (gpu_cli), Python (ctypes) or any other FFI binds them.  No HIP or torch types
 * appear in the signatures: streams are passed as void* (a hipStream_t, or NULL for the
 * null stream).
 *
 * Conventions
 *   - return 0 on success, a negative BS_E* code on error; bs_last_error() returns the
 *     text of the calling thread's last error.  No C++ exception crosses the ABI.
 *   - calls on one bs_index must be externally serialised; separate indexes are
 *     independent.
 *   - results are node ids in ascending (distance, id) order, 0xFFFFFFFF where fewer
 *     than K nodes were found (the reference writes the K results in descending order,
 *     topk_shared.cuh:420-429; the CPU reference cpu_cli writes them ascending).
 */
#ifndef BS_HIP_H
#define BS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BS_OK 0
#define BS_EINVAL (-1)  /* bad argument / unsupported configuration          */
#define BS_EHIP (-2)    /* a HIP runtime call failed                          */
#define BS_ENOMEM (-3)  /* device or host allocation failed                   */
#define BS_ENODEV (-4)  /* no usable gfx950 device                            */

typedef struct bs_index_s* bs_index;

/* Search modes (src/gpu_cli.cu:427-477 "mode"):
 *   BS_BASE        "base"    one query per workgroup, hash filter
 *   BS_GROUP       "warpN"   N = queries_per_group queries per workgroup, hash filter
 *   BS_GROUP_BLOOM "bwarpN"  as BS_GROUP with the Bloom visit filter
 *   BS_RABITQ      "rabitq"  RaBitQ estimates + exact rerank (needs bs_index_attach_rabitq)
 * Every mode runs one query per 64-lane wavefront.  base/warpN give identical results
 * (same semantics); they differ only in how many wavefronts share a workgroup. */
typedef enum { BS_BASE = 0, BS_GROUP = 1, BS_GROUP_BLOOM = 2, BS_RABITQ = 3 } bs_mode;

/* GPUBaseSearchCfg (gpu_search_base.cuh:17-23) / GPURabitqSearchCfg
 * (gpu_search_rabitq.cuh:21-26) plus the mode and K of gpu_cli's JSON "search" object
 * (src/gpu_cli.cu:414-452). */
typedef struct {
    int32_t mode;               /* bs_mode                                             */
    uint32_t queries_per_group; /* wavefronts (queries) per workgroup: 1,2,4,8; 0 -> 1  */
    uint32_t K;                 /* results per query (>= 1, <= topk_size)              */
    uint32_t topk_size;         /* beam slots, 1..4096 (see the limits below)          */
    uint32_t filter_capacity;   /* hash slots / Bloom bits (rounded up to a power of 2)*/
    uint32_t entry_point;       /* start node (< n)                                    */
    int32_t max_iterations;     /* >= 0                                                */
    int32_t reset_interval;     /* forgettable-filter reset period; 0 = never (>= 0)   */
} bs_search_cfg;

/* Limits against the reference: degree 1..256 and dim 1..1024 as gpu_cli (gpu_cli.cu:208-233,
 * 340-347).  topk_size 1..4096 (any value, not only multiples of 32): the beam is held in the
 * wavefront's registers, 64 keys per register, in 1..16 registers up to 1024 keys and in 32 or
 * 64 above (the RaBitQ expanded set in the wavefront's LDS slice); the reference's
 * SharedBitonicTopK (topk_shared.cuh:272-331) takes multiples of 32 in shared memory, bounded by
 * the shared memory per block.  Beams above 4096 are refused with BS_EINVAL.  With topk_size >=
 * filter_capacity a base search admits no new nodes once its table is full, as the reference's
 * forgettable filter does: such beams want a larger filter_capacity (at most 65536). */

/* Work counters summed over the queries of one call (the byte model of the roofline:
 * base  B_q = 4d + E*4R + D*4d + 4K;
 * rabitq B_q = 4d + 4pdim + E*(4R + 4R*wpp + 12R + 4d) + T_r*4d + 4K). */
typedef struct {
    double kernel_ms;       /* search kernel time (HIP events on the launch stream)     */
    uint64_t iterations;    /* beam-loop iterations                                    */
    uint64_t expansions;    /* E: adjacency rows (rabitq: node records) read           */
    uint64_t dist_evals;    /* D: exact L2 evaluations during the search               */
    uint64_t est_evals;     /* RaBitQ estimates                                        */
    uint64_t rerank_evals;  /* T_r: exact L2 evaluations of the final rerank           */
} bs_stats;

/* Upload a graph: vecs n*dim f32, edges n*degree u32 (ids < n or 0xFFFFFFFF).
 * Replaces GPUGraph(const CPUGraph&) (gpu_graph.cuh:81-146).  Validates every edge on
 * the host.  dim 1..1024, degree 1..256 (the reference gpu_cli's range), n < 2^31.  Also
 * prepares the query scheduling: 256 pivot rows, and the expected search cost per pivot
 * region (about 7 ms at 1M x 128: the entry point and a base search of 16384 index rows;
 * without it, which a failure there leaves, the scheduling uses the plain label order). */
int bs_index_create(const float* vecs, const uint32_t* edges, uint64_t n, uint32_t dim,
                    uint32_t degree, bs_index* out);

/* Attach RaBitQ data: codes n*degree*(padded_dim/32) u32, factors n*3*degree f32
 * (tx | fdq | fvq per node), signs padded_dim f32.  Replaces GPURabitq(const
 * CPURabitqData&) (rabitq.cuh:67-110).  padded_dim must be pow2ceil(dim) and >= 32. */
int bs_index_attach_rabitq(bs_index idx, const uint32_t* codes, const float* factors,
                           const float* signs, uint32_t padded_dim);

/* Search nq host-resident queries (nq*dim f32); results (host, nq*K u32) and optional
 * dists (host, nq*K f32, NULL allowed) are written.  Replaces one timed launch of
 * run_base / run_warp / run_rabitq (src/gpu_cli.cu:140-349) including the query upload
 * and result download of gpu_cli main (src/gpu_cli.cu:399-421,481). stats nullable; with
 * stats the per-query counters are collected too (see bs_search_device).
 * The device staging buffers belong to the index: they grow to the largest call and are
 * reused (freed by bs_index_destroy). */
int bs_search(bs_index idx, const bs_search_cfg* cfg, const float* queries, uint64_t nq,
              uint32_t* results, float* dists, bs_stats* stats);

/* Same search with device-resident buffers (queries nq*dim f32, results nq*K u32,
 * dists nq*K f32 or NULL, per_query nq*5 u32 counters {iterations, expansions,
 * dist_evals, est_evals, rerank_evals} or NULL), launched on `stream` (hipStream_t or
 * NULL).  Allocates no device memory.  Asynchronous unless sync != 0; with sync != 0
 * stats (nullable) gets kernel_ms and, when per_query is given, the summed counters.
 * Results never depend on per_query; in rabitq mode it costs an expanded-set lookup of
 * every neighbour (to count est_evals), which the search itself needs only for the
 * neighbours below the beam's last key, so pass NULL where counters are not wanted. */
int bs_search_device(bs_index idx, const bs_search_cfg* cfg, const float* d_queries,
                     uint64_t nq, uint32_t* d_results, float* d_dists, uint32_t* d_per_query,
                     void* stream, int sync, bs_stats* stats);

/* bs_search_device without allocation.  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The query-scheduling workspace (labels, launch map,
 * bucket counters) is a static device array of 2 MiB + 2 KiB per GPU, held until the process
 * ends, instead of the index's; the call allocates nothing and records no event.  At most
 * 262144 queries per call (the workspace's size; larger nq is rejected with BS_EINVAL).
 * Asynchronous on `stream`; buffers as for bs_search_device.  Every call on one GPU shares
 * the array: calls that overlap on one GPU (other streams, other threads) race; calls in
 * order on one stream do not.  The current device must be the index's.  A call may be
 * recorded into a HIP graph (stream capture) and replayed: it issues kernel launches only
 * (the array's address is looked up once per device by bs_index_create, and the bucket
 * counters are cleared by a kernel, not a memset); tested with three replays of a captured
 * scheduled call against bs_search_device. */
int bs_search_device_noalloc(bs_index idx, const bs_search_cfg* cfg, const float* d_queries,
                             uint64_t nq, uint32_t* d_results, float* d_dists,
                             uint32_t* d_per_query, void* stream);

/* Query scheduling (no counterpart in the reference, whose launches run query i in
 * block i, src/gpu_cli.cu:94-95,111-112,128-129).  Queries are independent, so their order
 * changes no result; it changes where their gathers hit and when the launch ends.  With
 * scheduling on, a base / warp / bwarp launch first labels each query with its nearest of
 * 256 pivot rows (fixed at bs_index_create), sorts the queries by label and gives each XCD
 * a contiguous run of them, so queries that walk the same region share that XCD's L2; inside
 * a run (launches of up to 65536 queries) the labels go by descending expected cost, which
 * bs_index_create calibrates once (16384 index rows searched in base mode from the
 * reference's entry point, iterations averaged per label).  A
 * RaBitQ launch is ordered longest first by predicted cost instead: a pilot search (topk
 * 16, 12 iterations, K 1) gives each query the exact distance of the best row it reaches,
 * and the queries run in descending order of it (the launch of several rounds then ends
 * with short queries).  Results, distances and per-query counters are written at each
 * query's own row as before.  mode 0: off;
 * 1 (default): on for calls with nq >= 4096; 2: on for every call.  Scheduled calls run
 * in launches of at most 262144 queries and share a workspace of the index; a call made
 * on another stream waits for the previous scheduled call on the device. */
int bs_index_set_query_order(bs_index idx, int mode);

/* The expected search cost per pivot label that bs_index_create calibrated (mean iterations of
 * the calibration search's queries of each label; labels without one get the mean of all):
 * out[256] (host).  BS_EINVAL when the index has none (the calibration failed), in which case
 * the base-family order is the plain label order.  No counterpart in the reference. */
int bs_index_label_costs(bs_index idx, float* out);

/* The search entry point of the uploaded index, computed on the device: compute_entry_point
 * (src/gpu_cli.cu:55-83) -- the float centroid accumulated row by row, then the first row of
 * least float squared distance to it -- with the same float roundings, so *entry equals
 * bs_entry_point (bs_host.h) on the same vectors.  Synchronous; allocates 4*dim + 8 bytes. */
int bs_index_entry_point(bs_index idx, uint32_t* entry);

/* The RaBitQ codebook of the uploaded index, computed on the device: build_rabitq
 * (src/build_rabitq.cpp:59-99,138-264) -- sign table from mt19937_64(seed), per edge the
 * residual of the rotated vectors, its 1-bit code and the factors (tx | fdq | fvq), entry =
 * medoid with a double centroid -- byte-identical to bs_build_rabitq (bs_host.h).  Host
 * outputs: codes n*degree*(pdim/32) u32, factors n*3*degree f32, signs pdim f32, entry.
 * The float work runs on the device; the factor products the reference forms in long
 * double are finished on the host.  Synchronous; allocates work buffers (rotations
 * n*pdim f32, codes, 16 B per edge).  dim > 16. */
int bs_index_build_rabitq(bs_index idx, uint32_t seed, uint32_t* codes, float* factors, float* signs,
                          uint32_t* entry);

/* Vamana graph construction on the device: build_graph (src/build_graph.cpp:95-392) with
 * the same insertion order (mt19937(seed) shuffle), batches, beam rule, sequential float
 * distances, dedupe_and_prune and mirrored-edge order, so edges_out (host, n*degree u32,
 * rows padded with node 0) equals the reference's graph (bs_build_vamana with exact != 0,
 * bs_host.h).  vecs: host n*dim f32.  degree 1..128, beam_width 1..1024, alpha >= 1.
 * Synchronous; allocates its work buffers (the visited bitmaps of up to 2 GiB, lists,
 * visit lists and sort space).  Fails with BS_EINVAL if a search expands more than
 * max(1024, 4*beam_width) nodes.  verbose != 0 prints progress to stderr. */
int bs_build_vamana_device(const float* vecs, uint64_t n, uint32_t dim, uint32_t degree, uint32_t beam_width,
                           float alpha, uint32_t seed, uint32_t* edges_out, int verbose);

/* Device pointers of the uploaded index (for tests and profilers). */
int bs_index_info(bs_index idx, uint64_t* n, uint32_t* dim, uint32_t* degree,
                  uint32_t* padded_dim, int* has_rabitq);

void bs_index_destroy(bs_index idx);
const char* bs_last_error(void);

/* ---- exact ground truth (no counterpart in the reference, whose ground truth comes from
 * HDF5 files, script/unpack.py:56-81) ---------------------------------------------------
 * The k nearest rows of the index (k <= 128, dim <= 256) to each of nq queries by exact
 * distance: fp64 squared differences summed in dimension order, ties by id -- the order of
 * bs_groundtruth (bs_host.h).  Candidates come from fp32 matrix-core dot products; each
 * query carries a certificate that no row outside its candidates can be among the k nearest.
 * out: nq*k int32 (-1 where fewer than k rows exist).  uncertified: nq bytes (1 = no
 * certificate: recompute that query, e.g. with bs_groundtruth) or NULL; n_uncertified
 * (nullable) gets their number.  Synchronous; allocates device work buffers. */
int bs_index_groundtruth(bs_index idx, const float* queries, uint64_t nq, uint32_t k, int32_t* out,
                         uint8_t* uncertified, uint64_t* n_uncertified);
/* The same on device buffers (queries nq*dim f32, out nq*k int32, uncertified nq u8 or
 * NULL), launched on `stream` (hipStream_t or NULL), synchronous at return. */
int bs_index_groundtruth_device(bs_index idx, const float* d_queries, uint64_t nq, uint32_t k,
                                int32_t* d_out, uint8_t* d_uncertified, void* stream,
                                uint64_t* n_uncertified);

/* ---- primitive entry points (parity tests of the device building blocks) ----------
 * Each runs the same device functions the search kernels use, on one wavefront per
 * instance.  All buffers are host memory. */

/* L2 of pairs (query qi[p], node ni[p]) with the search kernels' wave64 order.
 * Replaces l2_warp (l2.cuh:26-40). */
int bs_debug_l2(bs_index idx, const float* queries, uint64_t nq, const uint32_t* qi,
                const uint32_t* ni, uint64_t npairs, float* out);

/* Quantize one query (sign flip, WHT, dithered 6-bit codes, seed) and estimate nn
 * neighbours: codes_nbr nn*(pdim/32) u32, factors 3*degree f32 (tx|fdq|fvq, nn <= 128,
 * nn <= degree).  The raw sums take the search kernel's path for the layout: pdim <= 128
 * with nn <= 64 two lanes per neighbour, pdim <= 128 with nn > 64 a neighbour per lane
 * and register, pdim > 128 pdim/128 lanes per neighbour.  Outputs: codes_out pdim u8, scal_out {low, width} f32, sum_q_out,
 * raw_out nn u32, est_out nn f32.  Replaces RabitqQuantizer::quantize + RabitQFastScan
 * (fastscan.cuh:151-369). */
int bs_debug_fastscan(const float* query, const float* signs, uint32_t dim, uint32_t seed,
                      const uint32_t* codes_nbr, const float* factors, uint32_t nn,
                      uint32_t degree, float exact, uint8_t* codes_out, float* scal_out,
                      int32_t* sum_q_out, uint32_t* raw_out, float* est_out);

/* Beam harness: topk slots; nbatch batches of bsize (<= 256) candidate keys
 * ((orderable(dist) << 32) | (id << 1), 0xFFFF...FF = no candidate) merged in order;
 * after each batch `picks` picks (pick_run = 1: the rabitq rule for identical keys).
 * picked nbatch*picks ids (0xFFFFFFFF = nothing to pick), beam_out topk keys.
 * Replaces SharedBitonicTopK / RegBitonicTopK merge + pick (topk_shared.cuh:272-380,
 * topk_reg.cuh). */
int bs_debug_beam(uint32_t topk, const uint64_t* keys, uint32_t nbatch, uint32_t bsize,
                  uint32_t picks, int pick_run, uint32_t* picked, uint64_t* beam_out);

/* Full sort of n (<= 1024) keys ascending (the rerank sorter; replaces the bitonic
 * re-sort of topk_shared.cuh:384-416). */
int bs_debug_sort(const uint64_t* keys, uint32_t n, uint64_t* out);

/* The cost order of RaBitQ query scheduling on n (<= 262144) signals (host f32, larger =
 * expected to run longer): qmap[p] = the query at launch position p (longest first), bucket[q]
 * = query q's bucket (0 = largest; 256 buckets over mean +- 2 standard deviations of the
 * finite signals within 3 standard deviations of the mean of all finite signals; NaN and
 * values above the range in bucket 0, values below it in bucket 255).  No counterpart in the
 * reference (its launches run query i in block i). */
int bs_debug_cost_order(const float* signal, uint64_t n, uint32_t* qmap, uint32_t* bucket);

/* The placement of the base-family query order for n (<= 65536) queries with the given pivot
 * labels (host, < 256), g queries per workgroup (1..8) and X XCDs (1..32): qmap[p] = the query
 * at launch position p.  Workgroup b runs on XCD b mod X; XCD x gets the x-th contiguous run
 * of the queries sorted by label.  lcost (host, 256 expected costs per label, or NULL): inside
 * each run the labels go by descending cost, ties in label order.  No counterpart in the
 * reference (its launches run query i in block i). */
int bs_debug_label_order(const uint32_t* labels, const float* lcost, uint64_t n, uint32_t g, uint32_t X,
                         uint32_t* qmap);

/* One v_mfma_f32_32x32x2f32 product: A 32x2 and B 2x32 row-major in, D = A B 32x32
 * row-major out, read back through the accumulator layout the ground-truth kernel uses. */
int bs_debug_mfma32(const float* A, const float* B, float* D);

/* Visit filters: nbatch lane-parallel batches of bsize (<= 64) inserts (0xFFFFFFFF =
 * idle lane), then nquery contains().  bloom = 0: HashFilter (filter_hash.cuh),
 * 1: BloomFilter (filter_bloom.cuh). */
int bs_debug_filter(int bloom, uint32_t capacity, const uint32_t* keys, uint32_t nbatch,
                    uint32_t bsize, uint32_t* out_new, const uint32_t* qkeys, uint32_t nquery,
                    uint32_t* out_contains);

/* The instrumented build (libbs_hip_phase.so, `make phase`; not this library) exports four
 * readers of its clocks besides every entry point above, for measurement only:
 *   int bs_phase_read(unsigned long long out[16], int reset);       RaBitQ loop phase sums
 *   int bs_phase_read_base(unsigned long long out[16], int reset);  base loop phase sums
 *   int bs_query_clock_read(unsigned long long* out, uint64_t n);   start, end, hardware id
 *                                                                   of queries 0..n-1 (<= 65536)
 *   int bs_query_clock_read_rabitq(unsigned long long* out, uint64_t n);  the same, narrow-code
 *                                                                   RaBitQ launches
 * Slots of the phase sums: 0-5 the loop's phases, 6 the end of the query, 8 expansions,
 * 9 iterations, 10 queries. */

#ifdef __cplusplus
}
#endif
#endif
