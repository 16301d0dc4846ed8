/*
 * bs_oracle.c -- CPU restatement of the reference graph beam search.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, as the checker.  The product path never calls it.
 * Build: oracle/Makefile (gcc -O2 -std=c11 -ffp-contract=off; no -march, so float
 * arithmetic is exactly the IEEE single-precision sequence written here).
 *
 * What pins each part (checked by tests/test_oracle_*.py):
 *   orc_quantize_dither / orc_raw_dot / orc_estimate / orc_padded_dim / orc_dither_hash
 *       golden vectors written by the reference's own host functions
 *       (unittest/test_fastscan.cu:54-145, compiled into oracle/_ref/ref_fastscan),
 *       committed under tests/golden/fastscan_*.bin; plus closed forms (raw sum is the
 *       integer sum of selected codes; codes follow the Sylvester-Hadamard rotation).
 *   orc_l2_seq       reference cpu_cli ids (bit-exact) through ORC_BASE_CPUREF.
 *   orc_l2_wave, orc_l2_wave_lanes
 *                    fp64 sum within 1e-5 relative; exact on integer-valued inputs
 *                    (every partial sum is an exactly representable integer); the two
 *                    orders differ in the last bits (tests/test_oracle_semantics.py).
 *   ORC_BASE_CPUREF, ORC_RABITQ_CPUREF
 *                    result ids of the reference cpu_cli (oracle/_ref/cpu_cli) on
 *                    synthetic sets, committed under tests/golden/cpucli_*.npz.
 *   ORC_BASE_HASH    equals ORC_BASE_CPUREF (ids, distances, expansions) when the table
 *                    cannot fill between resets, with reset_interval 0, 1, 4 and 16
 *                    (tests/test_oracle_semantics.py); after every reset the table holds
 *                    exactly the beam ids (orc_base_state snapshots).
 *   ORC_BASE_BLOOM   bit positions against hand-computed values and a Python restatement of
 *                    filter_bloom.cuh:25-38; the 32-key round rule against that restatement
 *                    and a closed-form pair (a key whose bits an earlier round set is not
 *                    new); reduces to ORC_BASE_HASH when the filter has no false positives.
 *   ORC_RABITQ_GPU   ids, order and distances of the reference cpu_cli rabitq search on the
 *                    inputs where the two searches must coincide (fdq = fvq = 0, a tree padded
 *                    with self-loops, integer vectors; tests/golden/rqtree_*); the
 *                    expanded-set re-entry, the skip of a node expanded before, node-0
 *                    padding, evictions, the rerank and the dedup flush by a 9-node search
 *                    traced by hand (tests/test_rabitq_hand_trace.py: ids, distances and
 *                    every counter as literals), which each planted mistake of the
 *                    ORC_MUTANTS build fails; properties and recall elsewhere.
 *   orc_entry_point  reference cpu_cli "entry=" line (bit-exact id).
 *   orc_beam_run, orc_filter_run
 *                    closed forms of the reference unit tests (shuffled 0..n-1 keep the
 *                    smallest topk; picks never repeat; set semantics against a brute
 *                    force set).
 */
#include "bs_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* keys: (orderable(dist) << 32) | (id << 1) | expanded                       */
/* The reference orders beam entries by distance only on the GPU             */
/* (topk_shared.cuh:463,499; topk_reg.cuh:323) and by (dist, node) on the CPU */
/* (cpu_search_base.hpp:48-51).  The keys give the CPU's total order; the    */
/* expanded mark (the reference's id MSB, topk_shared.cuh:370) is the LSB.   */
/* ------------------------------------------------------------------------- */
uint32_t orc_orderable(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

uint64_t orc_make_key(float dist, uint32_t id, int expanded) {
    return ((uint64_t)orc_orderable(dist) << 32) | ((uint64_t)(id & 0x7FFFFFFFu) << 1) |
           (uint64_t)(expanded ? 1 : 0);
}

static inline uint32_t key_id(uint64_t k) { return (uint32_t)((k >> 1) & 0x7FFFFFFFu); }

static inline float key_dist(uint64_t k) {
    uint32_t o = (uint32_t)(k >> 32);
    uint32_t b = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static int cmp_u64(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x > y) - (x < y);
}

/* ------------------------------------------------------------------------- */
/* L2                                                                        */
/* ------------------------------------------------------------------------- */

/* cpu_search_base.hpp:29-37, cpu_search_rabitq.hpp:147-155, gpu_cli.cu:70-76:
 * sequential single-precision sum of (q - v)^2, separate multiply and add. */
float orc_l2_seq(const float* a, const float* b, int dim) {
    float sum = 0.0f;
    for (int d = 0; d < dim; ++d) {
        const float diff = a[d] - b[d];
        sum += diff * diff;
    }
    return sum;
}

/* The HIP kernels' L2 order (the reference's l2_warp, l2.cuh:26-40, is a lane-strided
 * partial sum plus a shuffle tree; this build's wave64 form is restated here):
 * rows are zero-padded to dpad = roundup(dim, 4) floats = `chunks` float4 chunks; a row
 * is handled by G = pow2ceil(chunks)/4 lanes (1 <= G <= 64); lane l accumulates the
 * chunks j = l, l+G, l+2G, ... and within a chunk the 4 components in order, each with
 * one fused multiply-add p = fma(diff, diff, p); the G partials are then combined by an
 * xor butterfly p_l += p_{l^s}, s = 1, 2, 4, ..., G/2.  Padded components add exactly 0. */
void orc_l2_wave_shape(int dim, int* group, int* per_lane) {
    int chunks = (dim + 3) / 4;
    int p = 1;
    while (p < chunks) p <<= 1;
    int g = p >= 4 ? p / 4 : 1;
    if (g > 64) g = 64;
    *group = g;
    *per_lane = (chunks + g - 1) / g;
}

/* the same order for a given lane count G per row (QR = ceil(chunks / G) chunks per lane) */
static float l2_wave_g(const float* a, const float* b, int dim, int G) {
    int chunks = (dim + 3) / 4;
    int QR = (chunks + G - 1) / G;
    float P[64], Q[64];
    for (int l = 0; l < G; ++l) {
        float p = 0.0f;
        for (int k = 0; k < QR; ++k) {
            int j = l + k * G;
            if (j >= chunks) continue;
            for (int c = 0; c < 4; ++c) {
                int i = 4 * j + c;
                if (i >= dim) continue;
                float diff = a[i] - b[i];
                p = fmaf(diff, diff, p);
            }
        }
        P[l] = p;
    }
    for (int s = 1; s < G; s <<= 1) {
        for (int l = 0; l < G; ++l) Q[l] = P[l] + P[l ^ s];
        memcpy(P, Q, sizeof(float) * (size_t)G);
    }
    return P[0];
}

float orc_l2_wave(const float* a, const float* b, int dim) {
    int G, QR;
    orc_l2_wave_shape(dim, &G, &QR);
    return l2_wave_g(a, b, dim, G);
}

/* The one-chunk-per-lane form the RaBitQ search with narrow codes (padded dim <= 128) uses
 * for the distances of its loop (the entry point and each expanded node; the final rerank
 * keeps orc_l2_wave): G = pow2ceil(chunks) lanes (at most 64), one chunk each, the same
 * butterfly over G lanes. */
float orc_l2_wave_lanes(const float* a, const float* b, int dim) {
    int chunks = (dim + 3) / 4;
    int g = 1;
    while (g < chunks) g <<= 1;
    if (g > 64) g = 64;
    return l2_wave_g(a, b, dim, g);
}

static float l2_of(int kind, const float* a, const float* b, int dim) {
    return kind == ORC_L2_SEQ ? orc_l2_seq(a, b, dim) : orc_l2_wave(a, b, dim);
}

/* the RaBitQ GPU search's loop distances: one chunk per lane with narrow codes (pdim <= 128) */
static float l2_rq(int kind, int pdim, const float* a, const float* b, int dim) {
    if (kind == ORC_L2_WAVE && pdim <= 128) return orc_l2_wave_lanes(a, b, dim);
    return l2_of(kind, a, b, dim);
}

/* ------------------------------------------------------------------------- */
/* fastscan                                                                  */
/* ------------------------------------------------------------------------- */

/* fastscan.cuh:119-124, rabitq.hpp:58-59 */
int orc_padded_dim(int dim) {
    int p = 1;
    while (p < dim) p <<= 1;
    return p;
}

/* fastscan.cuh:125-134 */
uint32_t orc_dither_hash(uint32_t a, uint32_t b) {
    a ^= b;
    a ^= a >> 16;
    a *= 0x45d9f3bu;
    a ^= a >> 16;
    a *= 0x45d9f3bu;
    a ^= a >> 16;
    return a;
}

/* fastscan.cuh:136-139 */
static float uniform_01(uint32_t h) { return (float)(h & 0xFFFFFFu) / 16777216.0f; }

/* build_rabitq.cpp:19-30, cpu_search_rabitq.hpp:155-163, fastscan.cuh:165-179 */
static void wht(float* x, int n) {
    for (int len = 1; len < n; len <<= 1)
        for (int i = 0; i < n; i += len << 1)
            for (int j = 0; j < len; ++j) {
                float u = x[i + j], v = x[i + j + len];
                x[i + j] = u + v;
                x[i + j + len] = u - v;
            }
}

static void rotate(const float* q, const float* signs, int dim, int pdim, float* rot) {
    for (int d = 0; d < dim; ++d) rot[d] = q[d] * signs[d];
    for (int d = dim; d < pdim; ++d) rot[d] = 0.0f;
    wht(rot, pdim);
}

/* std::min / std::max as the reference CPU code uses them */
static inline float smin(float a, float b) { return (b < a) ? b : a; }
static inline float smax(float a, float b) { return (a < b) ? b : a; }

/* fastscan.cuh:151-247 (GPU quantizer) == unittest/test_fastscan.cu:88-120:
 * c_i = clamp(floor((r_i - low) * (1/width) + u_i), 0, 63), u_i = uniform(hash(seed, i)). */
void orc_quantize_dither(const float* query, const float* signs, int dim, uint32_t seed,
                         uint8_t* codes, float* low, float* width, int32_t* sum_q) {
    int pdim = orc_padded_dim(dim);
    float* rot = (float*)malloc(sizeof(float) * (size_t)pdim);
    rotate(query, signs, dim, pdim, rot);
    float lo = rot[0], hi = rot[0];
    for (int d = 1; d < pdim; ++d) {
        lo = smin(lo, rot[d]);
        hi = smax(hi, rot[d]);
    }
    float w = (hi - lo) / 63.0f;
    float inv_w = 1.0f / w;
    int32_t s = 0;
    for (int d = 0; d < pdim; ++d) {
        float x = (rot[d] - lo) * inv_w;
        float u = uniform_01(orc_dither_hash(seed, (uint32_t)d));
        int q = (int)floorf(x + u);
        if (q < 0) q = 0;
        if (q > 63) q = 63;
        codes[d] = (uint8_t)q;
        s += q;
    }
    *low = lo;
    *width = w;
    *sum_q = s;
    free(rot);
}

/* cpu_search_rabitq.hpp:120-144 (CPU quantizer, no dither, no clamp):
 * c_i = (uint8_t) lroundf((r_i - low) * (1/width) + 0.5f). */
void orc_quantize_round(const float* query, const float* signs, int dim,
                        uint8_t* codes, float* low, float* width, int32_t* sum_q) {
    int pdim = orc_padded_dim(dim);
    float* rot = (float*)malloc(sizeof(float) * (size_t)pdim);
    rotate(query, signs, dim, pdim, rot);
    float lo = rot[0], hi = rot[0];
    for (int d = 1; d < pdim; ++d) {
        lo = smin(lo, rot[d]);
        hi = smax(hi, rot[d]);
    }
    float w = (hi - lo) / (float)((1 << 6) - 1);
    float inv_w = 1.0f / w;
    int32_t s = 0;
    for (int d = 0; d < pdim; ++d) {
        uint8_t v = (uint8_t)lroundf((rot[d] - lo) * inv_w + 0.5f);
        codes[d] = v;
        s += v;
    }
    *low = lo;
    *width = w;
    *sum_q = s;
    free(rot);
}

/* fastscan.cuh:346-355 == test_fastscan.cu:122-133 == cpu_search_rabitq.hpp:172-176:
 * raw = sum of codes[d] over the dims whose bit is set; bit d is bit d%32 of word d/32. */
uint32_t orc_raw_dot(const uint8_t* codes, const uint32_t* nbr, int pdim) {
    uint32_t s = 0;
    for (int d = 0; d < pdim; ++d)
        if ((nbr[d >> 5] >> (d & 31)) & 1u) s += codes[d];
    return s;
}

/* fastscan.cuh:361-366 == test_fastscan.cu:135-145:
 * est = tx + exact + fdq * width * ip + fvq * low, ip = 2 raw - sum_q;
 * FLT_MAX when tx == FLT_MAX or est is not finite.  No contraction. */
float orc_estimate(uint32_t raw, int32_t sum_q, float width, float low,
                   float tx, float fdq, float fvq, float exact) {
    float ip = (float)((int32_t)(raw << 1) - sum_q);
    float est = tx + exact + fdq * width * ip + fvq * low;
    if (tx == FLT_MAX || !isfinite(est)) est = FLT_MAX;
    return est;
}

/* ------------------------------------------------------------------------- */
/* visit filters                                                             */
/* ------------------------------------------------------------------------- */

static unsigned log2_ceil(unsigned n) {
    if (n <= 1) return 0;
    unsigned p = 1, b = 0;
    while (p < n) {
        p <<= 1;
        b++;
    }
    return b;
}

/* HashFilter (filter_hash.cuh:11-99): open addressing, h = (k ^ (k >> bitlen)) & mask,
 * linear probe, empty = 0xFFFFFFFF, insert -> 1 if new, 0 if present or the table is
 * full.  The reference inserts lane-parallel with atomicCAS; membership is independent
 * of the insert order unless the table fills, so the defined order here is sequential
 * in lane (neighbour) order. */
typedef struct {
    uint32_t* t;
    uint32_t size, mask, bitlen, occupied;
} hashf;

static void hash_init(hashf* h, uint32_t cap) {
    h->bitlen = log2_ceil(cap);
    h->size = 1u << h->bitlen;
    h->mask = h->size - 1;
    h->t = (uint32_t*)malloc(sizeof(uint32_t) * h->size);
    memset(h->t, 0xFF, sizeof(uint32_t) * h->size);
    h->occupied = 0;
}
static void hash_clear(hashf* h) {
    memset(h->t, 0xFF, sizeof(uint32_t) * h->size);
    h->occupied = 0;
}
static void hash_free(hashf* h) { free(h->t); }

static uint32_t hash_insert(hashf* h, uint32_t k) {
    uint32_t idx = (k ^ (k >> h->bitlen)) & h->mask;
    for (uint32_t i = 0; i < h->size; ++i) {
        if (h->t[idx] == 0xFFFFFFFFu) {
            h->t[idx] = k;
            h->occupied++;
            return 1;
        }
        if (h->t[idx] == k) return 0;
        idx = (idx + 1) & h->mask;
    }
    return 0;
}

static uint32_t hash_contains(const hashf* h, uint32_t k) {
    uint32_t idx = (k ^ (k >> h->bitlen)) & h->mask;
    for (uint32_t i = 0; i < h->size; ++i) {
        if (h->t[idx] == k) return 1;
        if (h->t[idx] == 0xFFFFFFFFu) return 0;
        idx = (idx + 1) & h->mask;
    }
    return 0;
}

/* BloomFilter (filter_bloom.cuh:13-131): 2^max(5, log2ceil(cap)) bits, k = 3 hashes.
 * The reference's warp filters a row in rounds of 32 neighbours (gpu_search_warp.cuh:203-205,
 * lane stride BX = 32); each lane tests its key's three bits, then sets them
 * (test-then-atomicOr, filter_bloom.cuh:104-120), so a round sees the bits of the earlier
 * rounds, and two lanes of one round holding the same key can both see "new" (a race).
 * Defined rule here: bloom_insert_batch is one round -- a key is new iff not all of its
 * bits were set before the round and it is the first occurrence of its value in the
 * round; then all bits of all keys of the round are set.  bloom_insert_rounds splits a
 * row into rounds of 32. */
typedef struct {
    uint32_t* w;
    uint32_t bitlen, mask, words;
} bloomf;

static void bloom_init(bloomf* b, uint32_t cap) {
    unsigned bl = log2_ceil(cap);
    if (bl < 5) bl = 5;
    b->bitlen = bl;
    b->mask = (bl >= 32) ? 0xFFFFFFFFu : ((1u << bl) - 1);
    b->words = 1u << (bl - 5);
    b->w = (uint32_t*)calloc(b->words, sizeof(uint32_t));
}
static void bloom_clear(bloomf* b) { memset(b->w, 0, sizeof(uint32_t) * b->words); }
static void bloom_free(bloomf* b) { free(b->w); }

/* filter_bloom.cuh:25-38 */
static void bloom_hashes(const bloomf* b, uint32_t key, uint32_t h[3]) {
    uint32_t a = key;
    a ^= a >> 16;
    a *= 0x45d9f3bu;
    a ^= a >> 16;
    h[0] = a & b->mask;
    uint32_t c = key * 0x9e3779b9u;
    c ^= c >> 16;
    c *= 0x45d9f3bu;
    c ^= c >> 16;
    h[1] = c & b->mask;
    uint32_t e = key * 0x517cc1b7u;
    e ^= e >> 16;
    e *= 0x45d9f3bu;
    e ^= e >> 16;
    h[2] = e & b->mask;
}

static int bloom_test(const bloomf* b, uint32_t key) {
    uint32_t h[3];
    bloom_hashes(b, key, h);
    for (int i = 0; i < 3; ++i)
        if (!((b->w[h[i] >> 5] >> (h[i] & 31)) & 1u)) return 0;
    return 1;
}

static void bloom_set(bloomf* b, uint32_t key) {
    uint32_t h[3];
    bloom_hashes(b, key, h);
    for (int i = 0; i < 3; ++i) b->w[h[i] >> 5] |= 1u << (h[i] & 31);
}

/* batch insert; keys == 0xFFFFFFFF are idle lanes (result 0) */
static void bloom_insert_batch(bloomf* b, const uint32_t* keys, int m, uint32_t* out) {
    for (int i = 0; i < m; ++i) {
        out[i] = 0;
        if (keys[i] == ORC_INVALID_ID) continue;
        int first = 1;
        for (int j = 0; j < i; ++j)
            if (keys[j] == keys[i]) {
                first = 0;
                break;
            }
        out[i] = (first && !bloom_test(b, keys[i])) ? 1u : 0u;
    }
    for (int i = 0; i < m; ++i)
        if (keys[i] != ORC_INVALID_ID) bloom_set(b, keys[i]);
}

/* a row of m keys in rounds of 32 (gpu_search_warp.cuh:203-205) */
static void bloom_insert_rounds(bloomf* b, const uint32_t* keys, int m, uint32_t* out) {
    for (int r0 = 0; r0 < m; r0 += 32) bloom_insert_batch(b, keys + r0, (m - r0 < 32) ? m - r0 : 32, out + r0);
}

void orc_bloom_hashes(uint32_t capacity, uint32_t key, uint32_t* h) {
    bloomf b;
    bloom_init(&b, capacity);
    bloom_hashes(&b, key, h);
    bloom_free(&b);
}

static void hash_insert_batch(hashf* h, const uint32_t* keys, int m, uint32_t* out) {
    for (int i = 0; i < m; ++i) out[i] = (keys[i] == ORC_INVALID_ID) ? 0u : hash_insert(h, keys[i]);
}

int orc_filter_run(int bloom, uint32_t capacity, const uint32_t* keys, int nbatch, int bsize,
                   uint32_t* out_new, const uint32_t* qkeys, int nquery, uint32_t* out_contains) {
    if (bloom) {
        bloomf b;
        bloom_init(&b, capacity);
        for (int i = 0; i < nbatch; ++i)
            bloom_insert_rounds(&b, keys + (size_t)i * bsize, bsize, out_new + (size_t)i * bsize);
        for (int i = 0; i < nquery; ++i) out_contains[i] = (uint32_t)bloom_test(&b, qkeys[i]);
        bloom_free(&b);
    } else {
        hashf h;
        hash_init(&h, capacity);
        for (int i = 0; i < nbatch; ++i)
            hash_insert_batch(&h, keys + (size_t)i * bsize, bsize, out_new + (size_t)i * bsize);
        for (int i = 0; i < nquery; ++i) out_contains[i] = hash_contains(&h, qkeys[i]);
        hash_free(&h);
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* beam (TopKBuffer contract, topk.cuh:16-49)                                 */
/* sorted ascending keys; empty slots are ORC_EMPTY_KEY (their LSB is set, so  */
/* they never look "unexpanded").                                             */
/* ------------------------------------------------------------------------- */
typedef struct {
    uint64_t* k;
    uint64_t* tmp;
    uint32_t T;
} beam_t;

static void beam_init(beam_t* b, uint32_t T, uint32_t maxcand) {
    b->T = T;
    b->k = (uint64_t*)malloc(sizeof(uint64_t) * T);
    b->tmp = (uint64_t*)malloc(sizeof(uint64_t) * (T + maxcand));
    for (uint32_t i = 0; i < T; ++i) b->k[i] = ORC_EMPTY_KEY;
}
static void beam_free(beam_t* b) {
    free(b->k);
    free(b->tmp);
}

/* merge (topk_shared.cuh:272-331): keep the T smallest of beam U candidates. */
static void beam_merge(beam_t* b, uint64_t* cand, uint32_t c) {
    if (c == 0) return;
    qsort(cand, c, sizeof(uint64_t), cmp_u64);
    uint32_t i = 0, j = 0, o = 0;
    while (o < b->T) {
        if (j < c && (i >= b->T || cand[j] < b->k[i]))
            b->tmp[o++] = cand[j++];
        else
            b->tmp[o++] = b->k[i++];
    }
    memcpy(b->k, b->tmp, sizeof(uint64_t) * b->T);
}

/* pick<1> (topk_shared.cuh:335-380; cpu_search_base.hpp:53-59): the smallest
 * unexpanded entry is marked expanded and returned.  run = 1 (duplicates possible, the
 * rabitq beam): of a run of identical keys the last one is marked, so the beam stays
 * sorted.  Returns ORC_INVALID_ID when every valid entry is expanded. */
static uint32_t beam_pick(beam_t* b, int run) {
    for (uint32_t p = 0; p < b->T; ++p) {
        if (b->k[p] & 1ull) continue;
        uint32_t q = p;
        if (run)
            while (q + 1 < b->T && b->k[q + 1] == b->k[p]) q++;
        b->k[q] |= 1ull;
        return key_id(b->k[q]);
    }
    return ORC_INVALID_ID;
}

int orc_beam_run(uint32_t topk, const uint64_t* keys, int nbatch, int bsize, int picks,
                 int pick_run, uint32_t* picked, uint64_t* beam_out) {
    beam_t b;
    beam_init(&b, topk, (uint32_t)bsize);
    uint64_t* cand = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(bsize > 0 ? bsize : 1));
    for (int i = 0; i < nbatch; ++i) {
        uint32_t c = 0;
        for (int j = 0; j < bsize; ++j) {
            uint64_t k = keys[(size_t)i * bsize + j];
            if (k != ORC_EMPTY_KEY) cand[c++] = k;
        }
        beam_merge(&b, cand, c);
        for (int p = 0; p < picks; ++p) picked[(size_t)i * picks + p] = beam_pick(&b, pick_run);
    }
    memcpy(beam_out, b.k, sizeof(uint64_t) * topk);
    free(cand);
    beam_free(&b);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* searches                                                                  */
/* ------------------------------------------------------------------------- */

static void write_beam_out(const beam_t* b, uint32_t K, uint32_t* res, float* dists) {
    for (uint32_t i = 0; i < K; ++i) {
        uint64_t k = (i < b->T) ? b->k[i] : ORC_EMPTY_KEY;
        res[i] = (k == ORC_EMPTY_KEY) ? ORC_INVALID_ID : key_id(k);
        if (dists) dists[i] = (k == ORC_EMPTY_KEY) ? FLT_MAX : key_dist(k);
    }
}

/* gpu_search_base.cuh:120-247 (base, one block per query) and
 * gpu_search_warp.cuh:122-238 (warpN / bwarpN, one warp per query): the same loop:
 *   merge candidates -> (every reset_interval iterations: clear the filter and re-insert
 *   the beam ids) -> pick the best unexpanded -> insert its neighbours into the filter,
 *   new ones become candidates with exact L2.  A final merge catches the last
 *   candidates when the loop ran out of iterations. */
static void search_base_gpu(const orc_index* ix, const orc_cfg* cfg, const float* q,
                            uint32_t* res, float* dists, orc_stats* st, int32_t stop_iter,
                            uint64_t* beam_snap, uint32_t* filt_snap, uint32_t* n_snap) {
    const int R = ix->degree, dim = ix->dim;
    const int bloom = cfg->mode == ORC_BASE_BLOOM;
    beam_t b;
    beam_init(&b, cfg->topk_size, (uint32_t)R);
    hashf h;
    bloomf bf;
    if (bloom) bloom_init(&bf, cfg->filter_capacity);
    else hash_init(&h, cfg->filter_capacity);
    uint64_t* cand = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)R);
    uint32_t* flags = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)R);
    uint32_t nc = 0;

    const uint32_t ep = cfg->entry_point;
    cand[nc++] = orc_make_key(l2_of(cfg->l2_kind, q, ix->vecs + (size_t)ep * dim, dim), ep, 0);
    st->dist_evals++;
    if (bloom) bloom_set(&bf, ep);
    else hash_insert(&h, ep);

    for (int32_t iter = 0; iter < cfg->max_iterations; ++iter) {
        st->iterations++;
        beam_merge(&b, cand, nc);
        nc = 0;
        if (cfg->reset_interval > 0 && (iter + 1) % cfg->reset_interval == 0) {
            /* forgettable reset (gpu_search_base.cuh:173-181): clear, then re-insert the beam
             * ids walking the reference's descending buffer from position 0 (the largest key
             * first), one at a time; a table smaller than the beam keeps the first ones. */
            if (bloom) bloom_clear(&bf);
            else hash_clear(&h);
            for (uint32_t i = b.T; i-- > 0;) {
                if (b.k[i] == ORC_EMPTY_KEY) continue;
                if (bloom) bloom_set(&bf, key_id(b.k[i]));
                else hash_insert(&h, key_id(b.k[i]));
            }
        }
        if (iter == stop_iter) {
            if (beam_snap) memcpy(beam_snap, b.k, sizeof(uint64_t) * b.T);
            if (filt_snap) {
                uint32_t nf = 0;
                if (bloom) {
                    memcpy(filt_snap, bf.w, sizeof(uint32_t) * bf.words);
                    nf = bf.words;
                } else {
                    for (uint32_t s = 0; s < h.size; ++s)
                        if (h.t[s] != ORC_INVALID_ID) filt_snap[nf++] = h.t[s];
                }
                if (n_snap) *n_snap = nf;
            }
            break;
        }
        uint32_t p = beam_pick(&b, 0);
        if (p == ORC_INVALID_ID) break;
        st->expansions++;
        const uint32_t* row = ix->edges + (size_t)p * R;
        if (bloom) bloom_insert_rounds(&bf, row, R, flags);
        else hash_insert_batch(&h, row, R, flags);
        for (int i = 0; i < R; ++i) {
            if (row[i] == ORC_INVALID_ID || !flags[i]) continue;
            float d = l2_of(cfg->l2_kind, q, ix->vecs + (size_t)row[i] * dim, dim);
            st->dist_evals++;
            cand[nc++] = orc_make_key(d, row[i], 0);
        }
    }
    beam_merge(&b, cand, nc);
    write_beam_out(&b, cfg->K, res, dists);
    free(cand);
    free(flags);
    if (bloom) bloom_free(&bf);
    else hash_free(&h);
    beam_free(&b);
}

int orc_base_state(const orc_index* ix, const orc_cfg* cfg, const float* query, int32_t stop_iter,
                   uint64_t* beam_out, uint32_t* filter_out, uint32_t* n_filter) {
    if (!ix || !cfg || (cfg->mode != ORC_BASE_HASH && cfg->mode != ORC_BASE_BLOOM) || stop_iter < 0) return -1;
    orc_stats st = {0, 0, 0, 0, 0};
    uint32_t* res = (uint32_t*)malloc(sizeof(uint32_t) * cfg->K);
    search_base_gpu(ix, cfg, query, res, NULL, &st, stop_iter, beam_out, filter_out, n_filter);
    free(res);
    return 0;
}

/* cpu_search_base.hpp:22-82: seen set that never forgets, sort by (dist, node),
 * expand the first unexpanded, push every unseen neighbour, truncate to topk.
 * (The reference computes distance(child) for child == UINT32_MAX, out of bounds;
 * such entries are skipped here.) */
static void search_base_cpuref(const orc_index* ix, const orc_cfg* cfg, const float* q,
                               uint32_t* res, float* dists, orc_stats* st) {
    const int R = ix->degree, dim = ix->dim;
    beam_t b;
    beam_init(&b, cfg->topk_size, (uint32_t)R);
    hashf seen;
    uint64_t bound = 2ull * (1ull + (uint64_t)(cfg->max_iterations > 0 ? cfg->max_iterations : 0) * (uint64_t)R);
    if (bound > (1ull << 30)) bound = 1ull << 30;
    hash_init(&seen, (uint32_t)bound);
    uint64_t* cand = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)R);
    const uint32_t ep = cfg->entry_point;
    uint64_t e = orc_make_key(l2_of(cfg->l2_kind, q, ix->vecs + (size_t)ep * dim, dim), ep, 0);
    st->dist_evals++;
    beam_merge(&b, &e, 1);
    hash_insert(&seen, ep);
    for (int32_t iter = 0; iter < cfg->max_iterations; ++iter) {
        st->iterations++;
        uint32_t p = beam_pick(&b, 0);
        if (p == ORC_INVALID_ID) break;
        st->expansions++;
        const uint32_t* row = ix->edges + (size_t)p * R;
        uint32_t nc = 0;
        for (int i = 0; i < R; ++i) {
            if (row[i] == ORC_INVALID_ID) continue;
            if (!hash_insert(&seen, row[i])) continue;
            float d = l2_of(cfg->l2_kind, q, ix->vecs + (size_t)row[i] * dim, dim);
            st->dist_evals++;
            cand[nc++] = orc_make_key(d, row[i], 0);
        }
        beam_merge(&b, cand, nc);
    }
    write_beam_out(&b, cfg->K, res, dists);
    free(cand);
    hash_free(&seen);
    beam_free(&b);
}

/* gpu_search_rabitq.cuh:191-340: dithered quantizer (seed 0, :206); exact-L2 entry;
 * loop: pick -> insert into the expanded set, skip the iteration if already expanded
 * (:250-252) -> neighbours not yet expanded get the per-edge estimate (a node may
 * re-enter the beam through another parent) -> merge.  Then exact-L2 rerank of every
 * beam slot (:315-317), sort, and a dedup flush from the smallest (:320-339) that
 * accepts at most `filter size` distinct ids. */
#ifdef ORC_MUTANTS
/* Planted mistakes, built only into bin/libbs_oracle_mutant.so: the tests check that a
 * fixture fails each of them (a fixture that a plausible misreading passes pins nothing).
 *   1  a node is seen once it enters the beam (cpu_search_rabitq.hpp:128-133) instead of
 *      once it is expanded: no second estimate through another parent
 *   2  a picked node that was expanded before is expanded again (no skip, :250-252)
 *   3  the flush writes duplicate ids (no dedup, :320-339) */
int orc_mutant = 0;
#define MUTANT(k) (orc_mutant == (k))
#else
#define MUTANT(k) 0
#endif

static void search_rabitq_gpu(const orc_index* ix, const orc_cfg* cfg, const float* q,
                              uint32_t* res, float* dists, orc_stats* st) {
    const int R = ix->degree, dim = ix->dim;
    const int pdim = ix->padded_dim, wpp = pdim / 32;
    uint8_t* codes = (uint8_t*)malloc((size_t)pdim);
    float low, width;
    int32_t sum_q;
    orc_quantize_dither(q, ix->signs, dim, 0u, codes, &low, &width, &sum_q);

    beam_t b;
    beam_init(&b, cfg->topk_size, (uint32_t)R);
    hashf h;
    hash_init(&h, cfg->filter_capacity);
    uint64_t* cand = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(R > (int)b.T ? R : (int)b.T));
    const uint32_t ep = cfg->entry_point;
    uint64_t e = orc_make_key(l2_rq(cfg->l2_kind, pdim, q, ix->vecs + (size_t)ep * dim, dim), ep, 0);
    st->dist_evals++;
    beam_merge(&b, &e, 1);
    hashf seen; /* mutant 1 only */
    hash_init(&seen, MUTANT(1) ? 1u << 20 : 1u);
    if (MUTANT(1)) hash_insert(&seen, ep);

    for (int32_t iter = 0; iter < cfg->max_iterations; ++iter) {
        st->iterations++;
        uint32_t p = beam_pick(&b, 1);
        if (p == ORC_INVALID_ID) break;
        if (!hash_insert(&h, p) && !MUTANT(2)) continue;
        st->expansions++;
        float exact = l2_rq(cfg->l2_kind, pdim, q, ix->vecs + (size_t)p * dim, dim);
        st->dist_evals++;
        const uint32_t* row = ix->edges + (size_t)p * R;
        const uint32_t* pc = ix->codes + (size_t)p * R * wpp;
        const float* fac = ix->factors + (size_t)p * 3 * R;
        uint32_t nc = 0;
        for (int i = 0; i < R; ++i) {
            uint32_t child = row[i];
            if (child == ORC_INVALID_ID || hash_contains(&h, child)) continue;
            if (MUTANT(1) && !hash_insert(&seen, child)) continue;
            uint32_t raw = orc_raw_dot(codes, pc + (size_t)i * wpp, pdim);
            float est = orc_estimate(raw, sum_q, width, low, fac[i], fac[R + i], fac[2 * R + i], exact);
            st->est_evals++;
            cand[nc++] = orc_make_key(est, child, 0);
        }
        beam_merge(&b, cand, nc);
    }

    /* rerank */
    uint32_t nv = 0;
    for (uint32_t i = 0; i < b.T; ++i) {
        if (b.k[i] == ORC_EMPTY_KEY) continue;
        uint32_t id = key_id(b.k[i]);
        cand[nv++] = orc_make_key(l2_of(cfg->l2_kind, q, ix->vecs + (size_t)id * dim, dim), id, 0);
        st->rerank_evals++;
    }
    qsort(cand, nv, sizeof(uint64_t), cmp_u64);
    /* dedup flush: identical ids carry identical exact distances, so duplicates are
     * adjacent; the flush's hash set (cap = filter size) accepts at most h.size ids. */
    uint32_t written = 0, distinct = 0, prev = ORC_INVALID_ID;
    for (uint32_t i = 0; i < nv && written < cfg->K; ++i) {
        uint32_t id = key_id(cand[i]);
        if (id == prev && !MUTANT(3)) continue;
        prev = id;
        if (distinct >= h.size) continue;
        distinct++;
        res[written] = id;
        if (dists) dists[written] = key_dist(cand[i]);
        written++;
    }
    for (; written < cfg->K; ++written) {
        res[written] = ORC_INVALID_ID;
        if (dists) dists[written] = FLT_MAX;
    }
    free(codes);
    free(cand);
    hash_free(&h);
    hash_free(&seen);
    beam_free(&b);
}

/* cpu_search_rabitq.hpp:115-237 */
static void search_rabitq_cpuref(const orc_index* ix, const orc_cfg* cfg, const float* q,
                                 uint32_t* res, float* dists, orc_stats* st) {
    const int R = ix->degree, dim = ix->dim;
    const int pdim = ix->padded_dim, wpp = pdim / 32;
    uint8_t* codes = (uint8_t*)malloc((size_t)pdim);
    float low, width;
    int32_t sum_q;
    orc_quantize_round(q, ix->signs, dim, codes, &low, &width, &sum_q);

    beam_t b;
    beam_init(&b, cfg->topk_size, (uint32_t)R);
    hashf seen;
    uint64_t bound = 2ull * (1ull + (uint64_t)(cfg->max_iterations > 0 ? cfg->max_iterations : 0) * (uint64_t)R);
    if (bound > (1ull << 30)) bound = 1ull << 30;
    hash_init(&seen, (uint32_t)bound);
    uint64_t* cand = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(R > (int)b.T ? R : (int)b.T));
    const uint32_t ep = cfg->entry_point;
    uint64_t e = orc_make_key(l2_of(cfg->l2_kind, q, ix->vecs + (size_t)ep * dim, dim), ep, 0);
    st->dist_evals++;
    beam_merge(&b, &e, 1);
    hash_insert(&seen, ep);
    for (int32_t iter = 0; iter < cfg->max_iterations; ++iter) {
        st->iterations++;
        uint32_t p = beam_pick(&b, 0);
        if (p == ORC_INVALID_ID) break;
        st->expansions++;
        float exact = l2_of(cfg->l2_kind, q, ix->vecs + (size_t)p * dim, dim);
        st->dist_evals++;
        const uint32_t* row = ix->edges + (size_t)p * R;
        const uint32_t* pc = ix->codes + (size_t)p * R * wpp;
        const float* fac = ix->factors + (size_t)p * 3 * R;
        uint32_t nc = 0;
        for (int i = 0; i < R; ++i) {
            uint32_t child = row[i];
            if (child == ORC_INVALID_ID) continue;
            if (!hash_insert(&seen, child)) continue;
            float est;
            if (fac[i] == FLT_MAX) {
                est = FLT_MAX;
            } else {
                uint32_t raw = orc_raw_dot(codes, pc + (size_t)i * wpp, pdim);
                float ip = (float)((int32_t)(raw << 1) - sum_q);
                est = fac[i] + exact + fac[R + i] * width * ip + fac[2 * R + i] * low;
                if (!isfinite(est)) est = FLT_MAX;
            }
            st->est_evals++;
            cand[nc++] = orc_make_key(est, child, 0);
        }
        beam_merge(&b, cand, nc);
    }
    uint32_t nv = 0;
    for (uint32_t i = 0; i < b.T; ++i) {
        if (b.k[i] == ORC_EMPTY_KEY) continue;
        uint32_t id = key_id(b.k[i]);
        cand[nv++] = orc_make_key(l2_of(cfg->l2_kind, q, ix->vecs + (size_t)id * dim, dim), id, 0);
        st->rerank_evals++;
    }
    qsort(cand, nv, sizeof(uint64_t), cmp_u64);
    for (uint32_t i = 0; i < cfg->K; ++i) {
        res[i] = (i < nv) ? key_id(cand[i]) : ORC_INVALID_ID;
        if (dists) dists[i] = (i < nv) ? key_dist(cand[i]) : FLT_MAX;
    }
    free(codes);
    free(cand);
    hash_free(&seen);
    beam_free(&b);
}

int orc_search(const orc_index* ix, const orc_cfg* cfg, const float* queries, uint64_t nq,
               uint32_t* results, float* dists, orc_stats* stats) {
    if (!ix || !cfg || cfg->topk_size == 0 || cfg->K == 0) return -1;
    if ((cfg->mode == ORC_RABITQ_GPU || cfg->mode == ORC_RABITQ_CPUREF) && !ix->codes) return -1;
    for (uint64_t i = 0; i < nq; ++i) {
        orc_stats st = {0, 0, 0, 0, 0};
        const float* q = queries + i * (uint64_t)ix->dim;
        uint32_t* r = results + i * cfg->K;
        float* d = dists ? dists + i * cfg->K : NULL;
        switch (cfg->mode) {
        case ORC_BASE_HASH:
        case ORC_BASE_BLOOM: search_base_gpu(ix, cfg, q, r, d, &st, -1, NULL, NULL, NULL); break;
        case ORC_BASE_CPUREF: search_base_cpuref(ix, cfg, q, r, d, &st); break;
        case ORC_RABITQ_GPU: search_rabitq_gpu(ix, cfg, q, r, d, &st); break;
        case ORC_RABITQ_CPUREF: search_rabitq_cpuref(ix, cfg, q, r, d, &st); break;
        default: return -1;
        }
        if (stats) stats[i] = st;
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* host pre/post steps                                                       */
/* ------------------------------------------------------------------------- */

/* gpu_cli.cu:55-83 == cpu_cli.cpp:35-62: float centroid accumulated as
 * c[d] += row[d] * (1/n) in row order, then the first row with the smallest
 * sequential float distance to it. */
uint32_t orc_entry_point(const float* vecs, uint64_t n, int dim) {
    float* c = (float*)calloc((size_t)dim, sizeof(float));
    float inv = 1.0f / (float)n;
    for (uint64_t i = 0; i < n; ++i) {
        const float* row = vecs + i * (uint64_t)dim;
        for (int d = 0; d < dim; ++d) c[d] += row[d] * inv;
    }
    uint32_t best = 0;
    float bd = FLT_MAX;
    for (uint64_t i = 0; i < n; ++i) {
        const float* row = vecs + i * (uint64_t)dim;
        float s = 0.0f;
        for (int d = 0; d < dim; ++d) {
            float diff = row[d] - c[d];
            s += diff * diff;
        }
        if (s < bd) {
            bd = s;
            best = (uint32_t)i;
        }
    }
    free(c);
    return best;
}

/* gpu_cli.cu:28-51: per query, skip -1, count and skip duplicates, count hits in the
 * first gt_k ground-truth ids; recall = hits / (nq * min(K, gt_k)). */
double orc_recall(const uint32_t* pred, uint64_t nq, int K, const int32_t* gt, int gt_k,
                  uint64_t* dups) {
    uint64_t correct = 0, nd = 0;
    for (uint64_t i = 0; i < nq; ++i) {
        const uint32_t* p = pred + i * (uint64_t)K;
        const int32_t* g = gt + i * (uint64_t)gt_k;
        for (int j = 0; j < K; ++j) {
            if (p[j] == ORC_INVALID_ID) continue;
            int dup = 0;
            for (int t = 0; t < j; ++t)
                if (p[t] == p[j]) {
                    dup = 1;
                    break;
                }
            if (dup) {
                nd++;
                continue;
            }
            for (int t = 0; t < gt_k; ++t)
                if ((uint32_t)g[t] == p[j]) {
                    correct++;
                    break;
                }
        }
    }
    if (dups) *dups = nd;
    int m = K < gt_k ? K : gt_k;
    return (double)correct / ((double)nq * (double)m);
}

/* exact ground truth: double accumulation of (q - b)^2, k smallest by (dist, id) */
typedef struct {
    double d;
    uint32_t id;
} dpair;
static int cmp_dpair(const void* a, const void* b) {
    const dpair* x = (const dpair*)a;
    const dpair* y = (const dpair*)b;
    if (x->d != y->d) return x->d < y->d ? -1 : 1;
    return (x->id > y->id) - (x->id < y->id);
}

void orc_groundtruth(const float* base, uint64_t n, const float* queries, uint64_t nq, int dim,
                     int k, int32_t* out) {
    dpair* all = (dpair*)malloc(sizeof(dpair) * (size_t)n);
    for (uint64_t i = 0; i < nq; ++i) {
        const float* q = queries + i * (uint64_t)dim;
        for (uint64_t j = 0; j < n; ++j) {
            const float* v = base + j * (uint64_t)dim;
            double s = 0.0;
            for (int d = 0; d < dim; ++d) {
                double diff = (double)q[d] - (double)v[d];
                s += diff * diff;
            }
            all[j].d = s;
            all[j].id = (uint32_t)j;
        }
        qsort(all, (size_t)n, sizeof(dpair), cmp_dpair);
        for (int t = 0; t < k; ++t) out[i * (uint64_t)k + t] = (t < (int)n) ? (int32_t)all[t].id : -1;
    }
    free(all);
}
