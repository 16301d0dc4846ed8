/*
 * bs_oracle.h -- CPU restatement of the reference graph beam search (TEST INFRASTRUCTURE).
 *
 * This library is the checker for the HIP search path.  Only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 * The product path (libbs_hip.so, gpu_cli) never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Two families of
 * search semantics are restated:
 *   - "cpuref": the reference CPU search (include/cpu_search_base.hpp,
 *     include/cpu_search_rabitq.hpp), pinned bit-exactly against the reference
 *     cpu_cli built from source into oracle/_ref;
 *   - "gpu": the reference GPU search (include/gpu_search_{base,warp,rabitq}.cuh)
 *     made deterministic: (dist, id) total order, defined filter-insert order, the
 *     wave64 L2 reduction order of the HIP kernels.  It is the bit-exact model the
 *     HIP kernels are compared against.
 *
 * Parity status of each part (what pins it) is listed in the header of bs_oracle.c.
 */
#ifndef BS_ORACLE_H
#define BS_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_EMPTY_KEY 0xFFFFFFFFFFFFFFFFull
#define ORC_INVALID_ID 0xFFFFFFFFu

/* search modes */
enum {
    ORC_BASE_HASH = 0,     /* gpu_search_base/warp with HashFilter (forgettable)      */
    ORC_BASE_BLOOM = 1,    /* gpu_search_warp with BloomFilter (bwarp*)                */
    ORC_RABITQ_GPU = 2,    /* gpu_search_rabitq (expanded-set, dithered quantizer)     */
    ORC_BASE_CPUREF = 3,   /* cpu_search_base.hpp                                      */
    ORC_RABITQ_CPUREF = 4  /* cpu_search_rabitq.hpp                                    */
};

/* L2 reduction orders */
enum {
    ORC_L2_SEQ = 0,   /* sequential float sum (reference CPU, cpu_search_base.hpp:29-37) */
    ORC_L2_WAVE = 1   /* this build's wave64 lane-partial + xor-butterfly order          */
};

typedef struct {
    const float* vecs;      /* n * dim, row major */
    const uint32_t* edges;  /* n * degree */
    uint64_t n;
    int dim;
    int degree;
    /* rabitq (optional) */
    const uint32_t* codes;   /* n * degree * wpp */
    const float* factors;    /* n * 3 * degree   */
    const float* signs;      /* pdim             */
    int padded_dim;
} orc_index;

typedef struct {
    int mode;
    int l2_kind;
    uint32_t K;
    uint32_t topk_size;
    uint32_t filter_capacity;
    uint32_t entry_point;
    int32_t max_iterations;
    int32_t reset_interval;   /* 0 = never reset */
} orc_cfg;

typedef struct {
    uint64_t iterations;   /* loop iterations executed                      */
    uint64_t expansions;   /* adjacency rows (or rabitq records) read       */
    uint64_t dist_evals;   /* exact L2 evaluations during the search        */
    uint64_t est_evals;    /* RaBitQ estimates                              */
    uint64_t rerank_evals; /* exact L2 evaluations in the final rerank      */
} orc_stats;

/* ---- keys ---- */
uint32_t orc_orderable(float f);
uint64_t orc_make_key(float dist, uint32_t id, int expanded);

/* ---- L2 ---- */
float orc_l2_seq(const float* a, const float* b, int dim);
float orc_l2_wave(const float* a, const float* b, int dim);
float orc_l2_wave_lanes(const float* a, const float* b, int dim);
void orc_l2_wave_shape(int dim, int* group, int* per_lane);

/* ---- fastscan (fastscan.cuh; unittest/test_fastscan.cu:54-145) ---- */
int orc_padded_dim(int dim);
uint32_t orc_dither_hash(uint32_t a, uint32_t b);
void orc_quantize_dither(const float* query, const float* signs, int dim, uint32_t seed,
                         uint8_t* codes, float* low, float* width, int32_t* sum_q);
void orc_quantize_round(const float* query, const float* signs, int dim,
                        uint8_t* codes, float* low, float* width, int32_t* sum_q);
uint32_t orc_raw_dot(const uint8_t* codes, const uint32_t* nbr, int pdim);
float orc_estimate(uint32_t raw, int32_t sum_q, float width, float low,
                   float tx, float fdq, float fvq, float exact);

/* ---- visit filters ---- */
/* Runs nbatch batches of bsize lane-parallel inserts (keys == 0xFFFFFFFF are idle lanes;
 * a Bloom batch is inserted in rounds of 32 keys), writes the insert result per key, then
 * answers nquery contains() queries. */
int orc_filter_run(int bloom, uint32_t capacity, const uint32_t* keys, int nbatch, int bsize,
                   uint32_t* out_new, const uint32_t* qkeys, int nquery, uint32_t* out_contains);
/* the three bit positions of `key` in a Bloom filter of `capacity` bits (filter_bloom.cuh:25-38) */
void orc_bloom_hashes(uint32_t capacity, uint32_t key, uint32_t* h);

/* ---- beam primitive harness ---- */
/* topk slots; nbatch batches of bsize candidate keys merged in order; after each batch
 * `picks` picks (pick_run=1: rabitq run rule).  picked[nbatch*picks], final beam[topk]. */
int orc_beam_run(uint32_t topk, const uint64_t* keys, int nbatch, int bsize, int picks,
                 int pick_run, uint32_t* picked, uint64_t* beam_out);

/* ---- searches ---- */
int orc_search(const orc_index* idx, const orc_cfg* cfg, const float* queries, uint64_t nq,
               uint32_t* results, float* dists, orc_stats* stats);
/* base / bwarp loop state of one query at iteration stop_iter, after that iteration's merge
 * and reset, before its pick: beam_out[topk] keys; filter_out = the hash table's stored ids
 * (n_filter of them, table order) or the Bloom words (n_filter words). */
int orc_base_state(const orc_index* idx, const orc_cfg* cfg, const float* query, int32_t stop_iter,
                   uint64_t* beam_out, uint32_t* filter_out, uint32_t* n_filter);

/* ---- host pre/post steps (src/gpu_cli.cu:28-83) ---- */
uint32_t orc_entry_point(const float* vecs, uint64_t n, int dim);
double orc_recall(const uint32_t* pred, uint64_t nq, int K, const int32_t* gt, int gt_k,
                  uint64_t* dups);
void orc_groundtruth(const float* base, uint64_t n, const float* queries, uint64_t nq, int dim,
                     int k, int32_t* out);

#ifdef __cplusplus
}
#endif
#endif
