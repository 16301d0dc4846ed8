/*
 * bs_host.h -- host-side (CPU) C-ABI of the MI355X beam-search framework:
 * file formats, index construction and input preparation.
 *
 * These are the host tools that sit on either side of the GPU search path
 * (include/bs_hip.h).  Each entry point replaces a piece of the reference's host
 * C++; the reference function is cited next to each declaration.
 *
 * Conventions: 0 = success, negative = error (bs_host_last_error() gives the text);
 * all arrays are caller-owned, row major, little endian; ids are uint32, 0xFFFFFFFF
 * marks "no node".  Functions that return allocated buffers hand back pointers that
 * must be released with bs_host_free().
 */
#ifndef BS_HOST_H
#define BS_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BS_HOST_OK 0
#define BS_HOST_EINVAL (-1)
#define BS_HOST_EIO (-2)
#define BS_HOST_ENOMEM (-3)

const char* bs_host_last_error(void);
void bs_host_free(void* p);

/* ---- file formats ------------------------------------------------------- */

/* fvecs / ivecs: per row int32 dim + dim payload words.
 * Replaces read_fvecs / read_ivecs (include/data_loader.hpp:9-45), adding size
 * validation (a ragged or truncated file is an error instead of garbage rows). */
int bs_read_vecs(const char* path, int is_int, void** data, uint64_t* n, uint32_t* dim);
/* write_fvecs / write_ivecs (include/data_loader.hpp:47-65) */
int bs_write_vecs(const char* path, int is_int, const void* data, uint64_t n, uint32_t dim);

/* graph.bin: int32 n, int32 degree, uint32 edges[n*degree].
 * CPUGraph::load edge part (include/cpu_graph.hpp:125-145); build_graph.cpp:142-154. */
int bs_read_graph(const char* path, uint32_t** edges, uint64_t* n, uint32_t* degree);
int bs_write_graph(const char* path, const uint32_t* edges, uint64_t n, uint32_t degree);

/* codebook.bin: uint32 entry; n rows [dim f32 | degree*wpp u32 codes |
 * 3*degree f32 factors (tx | fdq | fvq) | degree u32 ids]; pdim f32 signs.
 * load_rabitq_codebook (include/rabitq.hpp:49-97) extracts codes/factors/signs; this
 * reader also validates the file size (the reference does not, rabitq.hpp:75-90). */
int bs_read_codebook(const char* path, uint64_t n, uint32_t dim, uint32_t degree,
                     uint32_t* entry, uint32_t** codes, float** factors, float** signs,
                     uint32_t* padded_dim);
int bs_write_codebook(const char* path, const float* vecs, const uint32_t* edges, uint64_t n,
                      uint32_t dim, uint32_t degree, uint32_t entry, const uint32_t* codes,
                      const float* factors, const float* signs, uint32_t padded_dim);

/* ---- host pre/post steps of the search CLI ------------------------------- */

/* compute_entry_point (src/gpu_cli.cu:55-83): float centroid, nearest row. */
uint32_t bs_entry_point(const float* vecs, uint64_t n, uint32_t dim);

/* compute_recall (src/gpu_cli.cu:28-51): dedup, skip 0xFFFFFFFF,
 * divide by nq*min(K, gt_k).  dups (nullable) receives the duplicate count. */
double bs_recall(const uint32_t* pred, uint64_t nq, uint32_t K, const int32_t* gt,
                 uint32_t gt_k, uint64_t* dups);

/* ---- input preparation --------------------------------------------------- */

/* Seeded synthetic data (no reference counterpart: the reference downloads
 * ann-benchmarks sets, script/download_dataset.sh).  Counter-based: row i of stream
 * `seed` is the same whatever the thread count.
 *   mixture:    `centres` centres ~U[lo,hi]^dim (stream seed_c), each row = a uniformly
 *               chosen centre + sigma*N(0,1) per coordinate, clamped >= clamp_min
 *               (pass -INFINITY for no clamp).
 *   normalized: N(0,1) per coordinate, then scaled to unit L2 norm. */
int bs_gen_mixture(float* out, uint64_t n, uint32_t dim, uint32_t centres, float lo, float hi,
                   float sigma, float clamp_min, uint64_t seed_c, uint64_t seed_x);
int bs_gen_normalized(float* out, uint64_t n, uint32_t dim, uint64_t seed);

/* Exact ground truth: k nearest by double-accumulated (q-b)^2, ties by id.
 * (reference: groundtruth from HDF5, script/unpack.py:56-81) */
int bs_groundtruth(const float* base, uint64_t n, const float* queries, uint64_t nq,
                   uint32_t dim, uint32_t k, int32_t* out, int threads);
/* Same result from a candidate superset: for each query the ncand candidate ids
 * (e.g. an approximate GPU top list) are re-scored exactly and the k best kept. */
int bs_groundtruth_refine(const float* base, uint64_t n, const float* queries, uint64_t nq,
                          uint32_t dim, const int64_t* cand, uint32_t ncand, uint32_t k,
                          int32_t* out, int threads);

/* ---- index construction -------------------------------------------------- */

/* Batched incremental Vamana (src/build_graph.cpp:260-392): insertion order
 * std::shuffle(mt19937(seed)); batches [start, min(2*start, start + 2% n)); per point a
 * beam search of width beam_width from order[0] collects the expanded nodes, which are
 * deduplicated and alpha-pruned (build_graph.cpp:156-208); reverse edges are added after
 * each batch and over-full lists re-pruned; rows shorter than degree are padded with 0.
 * exact = 1 reproduces the reference's sequential float distances (same graph bytes);
 * exact = 0 uses a vectorized distance (same algorithm, different rounding).
 * edges_out: n*degree. */
int bs_build_vamana(const float* vecs, uint64_t n, uint32_t dim, uint32_t degree,
                    uint32_t beam_width, float alpha, uint32_t seed, int exact, int threads,
                    uint32_t* edges_out, int verbose);

/* RaBitQ per-edge codebook (src/build_rabitq.cpp:103-264): signs = +-1/sqrt(pdim) from
 * mt19937_64(seed); per edge (u,v): residual of the rotated vectors, 1-bit codes, factors
 * (tx, fdq, fvq); entry point = medoid with a double centroid.
 * codes_out: n*degree*(pdim/32), factors_out: n*3*degree, signs_out: pdim. */
int bs_build_rabitq(const float* vecs, const uint32_t* edges, uint64_t n, uint32_t dim,
                    uint32_t degree, uint32_t seed, int threads, uint32_t* codes_out,
                    float* factors_out, float* signs_out, uint32_t* entry_out);

uint32_t bs_rabitq_padded_dim(uint32_t dim);

#ifdef __cplusplus
}
#endif
#endif
