// Search kernels: one query per 64-lane wavefront, NY wavefronts per workgroup.
//
// MODE_HASH / MODE_BLOOM restate gpu_search_base.cuh:120-247 and
// gpu_search_warp.cuh:122-238 (the "base", "warpN" and "bwarpN" modes: the same loop,
// only the visit filter differs); MODE_RABITQ restates gpu_search_rabitq.cuh:191-340.
// The deterministic semantics (tie order, filter batch rules) are restated on the CPU
// by oracle/bs_oracle.c.
#pragma once
#include "bs_device.hpp"

namespace bsd {

// MODE_RABITQ: codes of at most 4 words per neighbour (pdim <= 128), one neighbour per
// lane; MODE_RABITQ_WIDE: longer codes, a neighbour spread over pdim / 128 lanes.
enum { MODE_HASH = 0, MODE_BLOOM = 1, MODE_RABITQ = 2, MODE_RABITQ_WIDE = 3 };

struct SearchParams {
    const float* vecs;      // n * dstride (zero-padded rows)
    const uint32_t* edges;  // n * R
    const uint32_t* recs;   // rabitq node records, n * rec_words
    const float* signs;     // pdim
    const float* queries;   // nq * dim
    uint32_t* results;      // nq * K
    float* dists;           // nq * K or null
    uint32_t* per_query;    // nq * 5 or null: iterations, expansions, dist, est, rerank
    const uint32_t* qmap;   // nq: launch position -> query, or null (identity)
    uint64_t nq;
    uint32_t dim, dstride, R, K, T;
    uint32_t filter_bits;     // bloom: log2 bits
    uint32_t filter_slots;    // hash: slots (a multiple of 4)
    uint32_t filter_cap;      // hash: keys the table accepts (the reference's slot count)
    uint32_t entry;
    int32_t max_it, reset;
    uint32_t pdim, wpp, rec_words, rec_ids, rec_fac, rec_codes;  // record offsets (words)
    QuadShape Q;            // code layout of a record (quad_shape(wpp, R))
    uint32_t lds_wave;      // bytes of LDS per wavefront
    uint32_t off_filter, off_scratch, off_cand;  // byte offsets inside the wave slice
    uint32_t off_planes;    // rabitq: the query's bit planes (outside the merge scratch)
    uint32_t off_pend;      // rabitq, beams of more than 256: the deferred merge's append staging (64 keys, in the merge scratch)
    uint32_t coop;          // base mode: wavefronts per query (1, 2, 4); 1 otherwise
    uint32_t off_coop;      // word where the first wavefront posts the row count
    L2Shape L;
};

// Per-phase clocks of the RaBitQ and base loops, compiled only into the instrumented library
// (make phase: -DBS_PHASE_CLOCKS, libbs_hip_phase.so, read by bs_phase_read for the RaBitQ
// instances and bs_phase_read_base for the hash-filter ones, each translation unit holding
// its own sums): s_memtime at the phase boundaries, summed per query and added to
// bs_phase_clock at the query's end (slots 0-5 the loop's phases, 6 the final flush, rerank
// and results, 8 expansions, 9 iterations, 10 queries).  In the library itself every call
// below is empty.
#ifdef BS_PHASE_CLOCKS
static __device__ unsigned long long bs_phase_clock[16];
#endif
struct PhaseClock {
#ifdef BS_PHASE_CLOCKS
    uint64_t t = 0, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    __device__ __forceinline__ void start() { t = __builtin_amdgcn_s_memtime(); }
    __device__ __forceinline__ void mark(int i) {
        const uint64_t n = __builtin_amdgcn_s_memtime();
        acc[i] += n - t;
        t = n;
    }
    __device__ __forceinline__ void flush(uint32_t n_exp, uint32_t n_iter) {
        if (lane_id() != 0) return;
        for (int i = 0; i < 8; ++i) atomicAdd(&bs_phase_clock[i], static_cast<unsigned long long>(acc[i]));
        atomicAdd(&bs_phase_clock[8], static_cast<unsigned long long>(n_exp));
        atomicAdd(&bs_phase_clock[9], static_cast<unsigned long long>(n_iter));
        atomicAdd(&bs_phase_clock[10], 1ull);
    }
#else
    __device__ __forceinline__ void start() {}
    __device__ __forceinline__ void mark(int) {}
    __device__ __forceinline__ void flush(uint32_t, uint32_t) {}
#endif
};

// Per-query clocks of the same instrumented build (bs_query_clock_read): for query q < 65536
// of the last launch, its start and end (s_memrealtime: 100 MHz, one counter for the whole
// device) and the wavefront's hardware id (HW_ID, XCC_ID in the upper word), written by the
// query's first wavefront.  The launch's timeline: concurrency, the drain after the last
// query starts, the XCD and CU each query ran on.
#ifdef BS_PHASE_CLOCKS
constexpr uint32_t QUERY_CLOCK_MAX = 65536;
static __device__ unsigned long long bs_query_clock[QUERY_CLOCK_MAX * 3];
#endif
struct QueryClock {
#ifdef BS_PHASE_CLOCKS
    uint64_t t0 = 0;
    __device__ __forceinline__ void start() { t0 = __builtin_amdgcn_s_memrealtime(); }
    __device__ __forceinline__ void finish(uint64_t qid, bool writer) {
        const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
        if (!writer || qid >= QUERY_CLOCK_MAX) return;
        const uint64_t hw = static_cast<uint64_t>(__builtin_amdgcn_s_getreg((31 << 11) | 4)) |
                            (static_cast<uint64_t>(__builtin_amdgcn_s_getreg((31 << 11) | 20)) << 32);
        bs_query_clock[qid * 3 + 0] = t0;
        bs_query_clock[qid * 3 + 1] = t1;
        bs_query_clock[qid * 3 + 2] = hw;
    }
#else
    __device__ __forceinline__ void start() {}
    __device__ __forceinline__ void finish(uint64_t, bool) {}
#endif
};

// Register budget per instance, matched to what the LDS slice allows anyway: RaBitQ beams
// up to 256 (about 7 KB of LDS per wavefront) are compiled for 5 wavefronts per SIMD (at most
// 96 VGPRs); the loops with beams up to 256 and two passes of rows in flight (Bloom over rows
// of up to 128 dims, hash over rows of up to 64) get 4 (128 VGPRs, no spills).  RaBitQ beams
// of 513..768 keys with narrow codes get 4 as well (left alone they take 3 per SIMD, against
// 4 for 8 registers): 1M x 128, 10k queries, topk 704 6.52 -> 6.39 ms, 768 6.94 -> 6.77; 16
// registers lose with it (9.19 -> 10.3 ms).
template <int TR, int CR, int MODE, int PB>
constexpr int min_waves_per_simd() {
    if (MODE == MODE_RABITQ && CR == 1 && (TR == 10 || TR == 12)) return 4;
    return (CR != 1 || TR > 4) ? 1 : MODE == MODE_RABITQ ? 5 : PB == 2 ? 4 : 1;
}

template <int TR, int CR, int QMAX, int MODE, int PB>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(min_waves_per_simd<TR, CR, MODE, PB>(), 8)))
search_kernel(const SearchParams p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const uint32_t lane = lane_id();
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t coop = p.coop;  // > 1: the workgroup's wavefronts share one query
    const uint64_t pos = coop > 1 ? static_cast<uint64_t>(blockIdx.x)
                                  : static_cast<uint64_t>(blockIdx.x) * (blockDim.x >> 6) + wave;
    if (pos >= p.nq) return;
    const uint64_t qid = p.qmap ? uniform(p.qmap[pos]) : pos;
    if (qid >= p.nq) return;
    QueryClock qclk;
    qclk.start();

    char* my = smem + static_cast<size_t>(coop > 1 ? 0u : wave) * p.lds_wave;
    uint64_t* scratch = reinterpret_cast<uint64_t*>(my + p.off_scratch);
    uint32_t* cand_ids = reinterpret_cast<uint32_t*>(my + p.off_cand);
    float* cand_d = reinterpret_cast<float*>(my + p.off_cand) + 64 * CR;
    // the merge's sorted candidates and slot bitmap reuse the candidate staging area
    // (free once the keys are in registers), which has room for 64*CR + max(TR, 8) keys
    uint64_t* merge_aux = reinterpret_cast<uint64_t*>(my + p.off_cand);

    const L2Shape L = p.L;
    const uint32_t lig = lane & (L.G - 1);
    const float* qv = p.queries + qid * p.dim;
    float4 q[QMAX];
    load_query<QMAX>(qv, p.dim, lig, L, q);

    const uint32_t T = p.T;
    uint64_t beam[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) beam[r] = EMPTY_KEY;

    uint32_t n_iter = 0, n_exp = 0, n_dist = 0, n_est = 0, n_rr = 0;
    BeamState st = {0u};  // the pick's scan start

    if constexpr (MODE == MODE_HASH || MODE == MODE_BLOOM) {
        // ------------------------------------------------------------------ base
        const float* vbase = p.vecs;
        const uint64_t vstride = p.dstride;
        uint32_t* batch = reinterpret_cast<uint32_t*>(my + p.off_coop);
        if (coop > 1 && wave != 0) {
            // helper wavefront: wait for a posted batch of candidate ids, compute its
            // share of their distances, repeat until the first wavefront posts INVALID
            for (;;) {
                __syncthreads();
                const uint32_t c = *batch;
                if (c == INVALID) break;
                const uint32_t lo = c * wave / coop, hi = c * (wave + 1) / coop;
                if (hi > lo) l2_rows<QMAX, PB>(q, vbase, vstride, cand_ids + lo, cand_d + lo, hi - lo, L);
                __syncthreads();
            }
            return;
        }

        HashLds hf;
        BloomLds bf;
        if constexpr (MODE == MODE_HASH) {
            hf.t = reinterpret_cast<uint32_t*>(my + p.off_filter);
            hf.size = p.filter_slots;
            hf.cap = p.filter_cap;
            hf.clear();
        } else {
            bf.w = reinterpret_cast<uint32_t*>(my + p.off_filter);
            bf.bits = p.filter_bits;
            bf.words = 1u << (p.filter_bits - 5);
            bf.mask = (p.filter_bits >= 32) ? 0xFFFFFFFFu : ((1u << p.filter_bits) - 1);
            bf.clear();
        }
        // seed: the entry point is the only candidate (gpu_search_base.cuh:142-152)
        uint64_t ck[CR];
        uint64_t cm[CR];
#pragma unroll
        for (int rc = 0; rc < CR; ++rc) {
            ck[rc] = EMPTY_KEY;
            cm[rc] = 0;
        }
        {
            const float d0 = l2_one<QMAX>(q, vbase + static_cast<uint64_t>(p.entry) * vstride, L);
            ck[0] = (lane == 0) ? make_key(d0, p.entry) : EMPTY_KEY;
            cm[0] = 1ull;
            n_dist = 1;
            if constexpr (MODE == MODE_HASH) {
                hf.insert1(p.entry);
            } else {
                if (lane == 0) bf.set_lane(p.entry);
                wave_sync();
            }
        }
        int32_t until_reset = p.reset;
        PhaseClock clk;  // instrumented build: 0 merge, 1 re-fill, 2 pick, 3 list + filter, 4 L2, 5 keys
        clk.start();
        // The neighbour list of the predicted next parent is requested before the merge,
        // so its HBM round trip overlaps merge, refill and pick: after the merge the
        // smallest unexpanded key is the smaller of the beam's next unexpanded key and the
        // smallest merged candidate.  The list is used only when the pick returns that node.
        uint32_t pre = INVALID;
        uint32_t pre_child[CR];
        uint64_t next_key = EMPTY_KEY;

        for (int32_t iter = 0; iter < p.max_it; ++iter) {
            ++n_iter;
            // merge candidates into the beam
            bool any = false;
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) any = any || (cm[rc] != 0);
            if (any) beam_merge<TR, CR, (CR == 1)>(beam, ck, cm, T, scratch, merge_aux, st);
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) cm[rc] = 0;
            clk.mark(0);

            // forgettable filter: clear and re-insert the beam ids (gpu_search_base.cuh:173-181)
            // in the reference's order, its descending buffer from position 0 (largest key
            // first).  Every beam id was admitted by the table and the table admits at most
            // `cap` ids between resets, so the beam never holds more ids than the table
            // accepts: the order cannot change which ids are kept.
            if (p.reset > 0 && --until_reset == 0) {
                until_reset = p.reset;
                if constexpr (MODE == MODE_HASH) {
                    hf.clear();
#pragma unroll
                    for (int r = TR - 1; r >= 0; --r) {
                        const uint32_t id = (beam[r] == EMPTY_KEY) ? INVALID : key_id(beam[r]);
                        hf.insert_batch<true>(id);
                    }
                } else {
                    bf.clear();
#pragma unroll
                    for (int r = 0; r < TR; ++r)
                        if (beam[r] != EMPTY_KEY) bf.set_lane(key_id(beam[r]));
                    wave_sync();
                }
            }
            clk.mark(1);

            // pick the best unexpanded node
            const uint32_t parent = beam_pick<TR, false>(beam, st, &next_key);
            if (parent == INVALID) break;
            ++n_exp;
            clk.mark(2);

            // expand: neighbours through the filter
            uint32_t child[CR], isnew[CR];
            if (parent == pre) {
#pragma unroll
                for (int rc = 0; rc < CR; ++rc) child[rc] = pre_child[rc];
            } else {
                const uint32_t* row = p.edges + static_cast<uint64_t>(parent) * p.R;
#pragma unroll
                for (int rc = 0; rc < CR; ++rc) {
                    const uint32_t i = static_cast<uint32_t>(rc) * 64u + lane;
                    child[rc] = row[i < p.R ? i : 0u];
                }
            }
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) {
                const uint32_t i = static_cast<uint32_t>(rc) * 64u + lane;
                child[rc] = (i < p.R) ? child[rc] : INVALID;
            }
            if constexpr (MODE == MODE_HASH) {
#pragma unroll
                for (int rc = 0; rc < CR; ++rc) isnew[rc] = hf.insert_batch(child[rc]);
            } else {
                bf.insert_batch<CR>(child, isnew);
            }
            // compact the new neighbours into the LDS id list
            uint32_t c = 0;
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) {
                const uint64_t m = ballot(isnew[rc] != 0);
                if (isnew[rc]) cand_ids[c + bsw::lanes_below(m)] = child[rc];
                c += static_cast<uint32_t>(__builtin_popcountll(m));
            }
            wave_sync();
            clk.mark(3);
            if (c == 0) continue;
            n_dist += c;
            if (coop > 1) {
                if (lane == 0) *batch = c;
                __syncthreads();  // batch posted
                const uint32_t hi = c / coop;
                if (hi > 0) l2_rows<QMAX, PB>(q, vbase, vstride, cand_ids, cand_d, hi, L);
                __syncthreads();  // every share of cand_d written
            } else {
                l2_rows<QMAX, PB>(q, vbase, vstride, cand_ids, cand_d, c, L);
            }
            clk.mark(4);
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) {
                const uint32_t j = static_cast<uint32_t>(rc) * 64u + lane;
                const bool v = j < c;
                ck[rc] = v ? make_key(cand_d[j], cand_ids[j]) : EMPTY_KEY;
                cm[rc] = ballot(v);
            }
            wave_sync();
            {
                const uint64_t c0 = wave_min_key<CR>(ck);
                const uint64_t nk = c0 < next_key ? c0 : next_key;
                pre = nk == EMPTY_KEY ? INVALID : key_id(nk);
                if (pre != INVALID) {
                    const uint32_t* row = p.edges + static_cast<uint64_t>(pre) * p.R;
#pragma unroll
                    for (int rc = 0; rc < CR; ++rc) {
                        const uint32_t i = static_cast<uint32_t>(rc) * 64u + lane;
                        pre_child[rc] = row[i < p.R ? i : 0u];
                    }
                }
            }
            clk.mark(5);
        }
        clk.mark(6);
        if (coop > 1) {  // release the helper wavefronts
            if (lane == 0) *batch = INVALID;
            __syncthreads();
        }
        {
            bool any = false;
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) any = any || (cm[rc] != 0);
            if (any) beam_merge<TR, CR, (CR == 1)>(beam, ck, cm, T, scratch, merge_aux, st);
        }
        // flush the K smallest, ascending
        uint32_t* out = p.results + qid * p.K;
        float* dout = p.dists ? p.dists + qid * p.K : nullptr;
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            const uint32_t e = static_cast<uint32_t>(r) * 64u + lane;
            if (e < p.K) {
                out[e] = (beam[r] == EMPTY_KEY) ? INVALID : key_id(beam[r]);
                if (dout) dout[e] = (beam[r] == EMPTY_KEY) ? FLT_MAX : key_dist(beam[r]);
            }
        }
        clk.mark(6);
        clk.flush(n_exp, n_iter);
    } else {
        // ---------------------------------------------------------------- rabitq
        HashLds hf;
        hf.t = reinterpret_cast<uint32_t*>(my + p.off_filter);
        hf.size = p.filter_slots;
        hf.cap = p.filter_cap;
        const uint32_t wpp = p.wpp;
        const uint64_t rstride = p.rec_words;
        const float* rbase = reinterpret_cast<const float*>(p.recs);

        constexpr bool WIDE = MODE == MODE_RABITQ_WIDE;
        const QuadShape S = p.Q;
        const uint32_t qi = lane & (S.qpn - 1), nl = lane >> S.qshift;

        // quantize the query.  Wide layout: the lane's plane words stay in registers;
        // narrow layout: the 24 words all lanes share stay in LDS (planes4, outside the
        // merge scratch) and are re-read per expansion.
        uint4 pl[6];
        QuantOut qo;
        uint32_t* planes4 = reinterpret_cast<uint32_t*>(my + p.off_planes);
        {
            float* qscr = reinterpret_cast<float*>(scratch);
            uint32_t* planes = reinterpret_cast<uint32_t*>(my + p.off_scratch + 4u * p.pdim);
            qo = quantize(qv, p.signs, p.dim, p.pdim, 0u, qscr, planes, nullptr);
            if constexpr (WIDE) lane_plane_quads(planes, wpp, S, pl);
            else store_planes4(planes, wpp, planes4);
        }
        hf.clear();

        // entry point with its exact distance (gpu_search_rabitq.cuh:210-223)
        {
            const float d0 = l2_one<QMAX>(q, rbase + static_cast<uint64_t>(p.entry) * rstride, L);
            n_dist = 1;
            uint64_t ck[1] = {lane == 0 ? make_key(d0, p.entry) : EMPTY_KEY};
            uint64_t cm[1] = {1ull};
            beam_merge<TR, 1>(beam, ck, cm, T, scratch, merge_aux, st);
        }
        uint32_t* rawbuf = cand_ids;
        // Beams of more than 256 keys defer the merge: candidates wait in a list of up to 64
        // keys (pending_add); 1M x 128, 10k queries: topk 768 8.87 -> 8.11 ms, 512 6.11 ->
        // 5.95, while smaller beams lose (256 2.67 -> 2.73, 128 1.47 -> 1.61)
        constexpr bool DEFER = TR >= 8;
        // the list's append staging shares the merge scratch (live only between pending_add's
        // compaction and its read-back, when no merge runs)
        PendingList pd = {DEFER ? reinterpret_cast<uint64_t*>(my + p.off_pend) : nullptr, 0u, EMPTY_KEY,
                          DEFER ? beam_last<TR>(beam, T) : EMPTY_KEY};
        uint32_t picks = 0;
        PhaseClock clk;
        clk.start();

        for (int32_t iter = 0; iter < p.max_it; ++iter) {
            ++n_iter;
            // the pick is wave-uniform; readfirstlane puts it in a scalar register (the
            // compiler may leave it in a vector one), so that the record's addresses below
            // are scalar bases with per-lane offsets
            const uint32_t parent = uniform(DEFER ? pending_pick<TR, true>(beam, st, pd, T, scratch, merge_aux, picks)
                                                  : beam_pick<TR, true>(beam, st));
            clk.mark(0);
            if (parent == INVALID) break;
            const uint32_t* rec = p.recs + static_cast<uint64_t>(parent) * rstride;
            const float* fac = reinterpret_cast<const float*>(rec + p.rec_fac);
            const uint32_t* codes = rec + p.rec_codes;
            // Every load of the record -- neighbour ids, factors, the parent's vector and
            // (the first four passes of) the codes -- is issued before any result is used,
            // so an expansion costs one HBM round trip.  Indices are clamped, not masked.
            uint32_t child[CR];
            float ftx[CR], ffd[CR], ffv[CR];
            // byte offsets from the record, a wave-uniform base (bsw::load_off; a record is a
            // few KB)
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) {
                const uint32_t i = static_cast<uint32_t>(rc) * 64u + lane;
                const uint32_t ic = i < p.R ? i : 0u;
                child[rc] = bsw::load_off<uint32_t>(rec, 4u * (p.rec_ids + ic));
                ftx[rc] = bsw::load_off<float>(fac, 4u * ic);
                ffd[rc] = bsw::load_off<float>(fac, 4u * (p.R + ic));
                ffv[rc] = bsw::load_off<float>(fac, 4u * (2u * p.R + ic));
            }
            float4 pv[1][QMAX];
            {
                const float* const rows[1] = {reinterpret_cast<const float*>(rec)};
                l2_load<QMAX, 1, true>(rows, lig, L, pv);
            }
            constexpr int NC = WIDE ? 4 : CR;
            uint4 cw[NC];
            // narrow codes with one candidate register: two lanes per neighbour (load_code_halves)
            constexpr bool HALVES = !WIDE && CR == 1;
            CodeHalves ch;
            if constexpr (HALVES) {
                ch = load_code_halves(codes, p.R, S);
            } else {
#pragma unroll
                for (int t = 0; t < NC; ++t) {
                    const uint32_t nb = WIDE ? static_cast<uint32_t>(t) * S.npp + nl : static_cast<uint32_t>(t) * 64u + lane;
                    cw[t] = load_quad(codes, nb, p.R, qi, S);
                }
            }
            // The expanded set is probed while the record is in flight: the loads of a node
            // already expanded (gpu_search_rabitq.cuh:249-252; 7.5% of the picks at config C)
            // are wasted, the probe's LDS latency of every other pick is hidden.
            const bool fresh_parent = hf.insert1(parent) != 0u;
            clk.mark(1);
            if (!fresh_parent) continue;
            ++n_exp;

            // the home groups of the neighbours' expanded-set sequences, read now so that the
            // lookups below do not wait for the LDS (the parent's insert above is visible)
            uint4 hg[CR];
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) hg[rc] = hf.home_group(child[rc]);
            // exact distance of the parent
            float pe[1];
            l2_accum<QMAX, 1>(q, pv, lig, L, pe);
            const float exact = __uint_as_float(readlane(__float_as_uint(bsw::group_sum(pe[0], L.G)), 0));
            ++n_dist;
            clk.mark(2);
            // fastscan sums of the neighbours
            uint32_t raw[CR];
            if constexpr (WIDE) {
                const uint4(&c0)[4] = reinterpret_cast<const uint4(&)[4]>(cw);
                raw_sums_wide(pl, codes, p.R, S, c0, rawbuf);
#pragma unroll
                for (int rc = 0; rc < CR; ++rc) {
                    const uint32_t i = static_cast<uint32_t>(rc) * 64u + lane;
                    raw[rc] = rawbuf[i < p.R ? i : 0u];
                }
            } else if constexpr (HALVES) {
                raw[0] = raw_halves(planes4, ch, p.R);
            } else {
#pragma unroll
                for (int b = 0; b < 6; ++b) pl[b] = reinterpret_cast<const uint4*>(planes4)[b];
#pragma unroll
                for (int rc = 0; rc < CR; ++rc) raw[rc] = raw_quad(pl, cw[rc < NC ? rc : 0]);
            }
            clk.mark(3);
            // Only neighbours below the beam's last key can enter it (the merge drops the
            // others first), so only they are looked up in the expanded set.  The estimate
            // counter (neighbours not yet expanded: the reference's estimates) needs every
            // neighbour's lookup; it is made only when per-query counters are requested.
            uint64_t ck[CR], cm[CR];
            uint32_t nv = 0;
            const uint64_t thr_k = DEFER ? pd.thr : beam_last<TR>(beam, T);
            const bool count_all = p.per_query != nullptr;
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) {
                const uint32_t i = static_cast<uint32_t>(rc) * 64u + lane;
                const uint64_t ok = ballot(i < p.R && child[rc] != INVALID);
                const float est = estimate(raw[rc], qo.sum_q, qo.width, qo.low, ftx[rc], ffd[rc], ffv[rc], exact);
                const uint64_t key = make_key(est, child[rc]);
                const uint64_t below = ok & ballot(key < thr_k);
                const uint64_t probe = count_all ? ok : below;
                const uint64_t fresh = probe ? probe & ~hf.contains_mask(child[rc], probe, hg[rc]) : 0ull;
                ck[rc] = bsw::lane_in(below & fresh) ? key : EMPTY_KEY;
                cm[rc] = below & fresh;
                nv += static_cast<uint32_t>(__builtin_popcountll(fresh));
            }
            wave_sync();
            n_est += nv;
            clk.mark(4);
            if constexpr (DEFER) pending_add<TR, CR>(beam, ck, cm, pd, T, scratch, merge_aux, st);
            else beam_merge<TR, CR>(beam, ck, cm, T, scratch, merge_aux, st);
            clk.mark(5);
        }
        if constexpr (DEFER) pending_flush<TR>(beam, pd, T, scratch, merge_aux, st);

        // exact rerank of every beam slot (gpu_search_rabitq.cuh:314-317)
        uint32_t* ids = reinterpret_cast<uint32_t*>(scratch);
        float* rd = reinterpret_cast<float*>(scratch) + 64 * TR;
        uint32_t nvb = 0;
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            const uint32_t e = static_cast<uint32_t>(r) * 64u + lane;
            // an empty slot names row 0: the gather below reads the first nvb ids, which
            // are all valid while the beam is sorted (empty keys last); should that order
            // ever break, the rerank reads a wrong row instead of one outside the index
            ids[e] = (beam[r] == EMPTY_KEY) ? 0u : key_id(beam[r]);
            nvb += static_cast<uint32_t>(__builtin_popcountll(ballot(beam[r] != EMPTY_KEY)));
        }
        wave_sync();
        // the valid entries are the first nvb (the beam is sorted, empty keys last)
        if constexpr (QMAX == 1) {
            // narrow codes: the loop's one-chunk-per-lane rows fit one row per pass per 32
            // lanes; the rerank's many rows go 4 chunks per lane (8 rows of 128 dims per pass,
            // the base search's order), with the query reloaded in that layout
            const L2Shape L4 = l2_shape(p.dim);
            float4 q4[4];
            load_query<4>(qv, p.dim, lane & (L4.G - 1), L4, q4);
            l2_rows<4, 2>(q4, rbase, rstride, ids, rd, nvb, L4);
        } else {
            l2_rows<QMAX, PB>(q, rbase, rstride, ids, rd, nvb, L);
        }
        n_rr += nvb;
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            const uint32_t e = static_cast<uint32_t>(r) * 64u + lane;
            beam[r] = (e < nvb) ? make_key(rd[e], ids[e]) : EMPTY_KEY;
        }
        wave_sync();
        sort_beam<TR>(beam, scratch);

        // dedup flush from the smallest (gpu_search_rabitq.cuh:319-339): identical ids
        // carry identical exact distances and are adjacent; the flush's hash set accepts
        // at most `cap` distinct ids (the reference's slot count).
        uint32_t* out = p.results + qid * p.K;
        float* dout = p.dists ? p.dists + qid * p.K : nullptr;
        const uint32_t limit = (p.K < hf.cap) ? p.K : hf.cap;
        uint32_t written = 0;
        uint32_t prev_last = INVALID;  // id of element 64*r - 1
        uint32_t wpos[TR];
        bool keep[TR];
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            const uint32_t id = (beam[r] == EMPTY_KEY) ? INVALID : key_id(beam[r]);
            uint32_t prv = bsw::prev_lane(id);
            if (lane == 0) prv = prev_last;
            keep[r] = (id != INVALID) && (id != prv);
            const uint64_t km = ballot(keep[r]);
            wpos[r] = written + bsw::lanes_below(km);
            written += static_cast<uint32_t>(__builtin_popcountll(km));
            prev_last = readlane(id, 63);
        }
        const uint32_t nw = written < limit ? written : limit;
        for (uint32_t e = nw + lane; e < p.K; e += 64) {
            out[e] = INVALID;
            if (dout) dout[e] = FLT_MAX;
        }
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            if (keep[r] && wpos[r] < nw) {
                out[wpos[r]] = key_id(beam[r]);
                if (dout) dout[wpos[r]] = key_dist(beam[r]);
            }
        }
        clk.mark(6);
        clk.flush(n_exp, n_iter);
    }

    qclk.finish(qid, lane == 0 && (coop <= 1 || wave == 0));
    if (p.per_query && lane == 0) {
        uint32_t* pq = p.per_query + qid * 5;
        pq[0] = n_iter;
        pq[1] = n_exp;
        pq[2] = n_dist;
        pq[3] = n_est;
        pq[4] = n_rr;
    }
}

}  // namespace bsd
