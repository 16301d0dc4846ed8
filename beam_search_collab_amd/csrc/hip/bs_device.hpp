// Device building blocks of the wave64 graph beam search (gfx950).
//
// One query runs on one 64-lane wavefront.  State per query:
//   beam     T = 64*TR keys in VGPRs, sorted ascending, element e = r*64 + lane
//            (register-major); key = (orderable(dist) << 32) | (id << 1) | expanded
//   filter   visit filter in the wave's LDS slice (hash table or Bloom bits)
//   query    the lane's float4 chunks of the query in VGPRs (L2 layout below)
// Replaces the reference's TopKBuffer / VisitFilter / l2_warp / RabitQFastScan
// (topk.cuh:16-49, visit_filter.cuh:10-30, l2.cuh:26-40, fastscan.cuh:19-369).
#pragma once
#include "wave.hpp"

#include <float.h>
#include <stdint.h>

namespace bsd {

using bsw::ballot;
using bsw::lane_id;
using bsw::readlane;
using bsw::readlane64;
using bsw::uniform;
using bsw::wave_sync;

constexpr uint64_t EMPTY_KEY = ~0ull;
constexpr uint32_t INVALID = 0xFFFFFFFFu;

// ---------------------------------------------------------------------------
// keys: total order (dist, id, expanded).  The reference compares distances only
// (topk_shared.cuh:463,499, ties unordered) and marks expansion in the id MSB
// (topk_shared.cuh:370); here the CPU reference's (dist, node) order
// (cpu_search_base.hpp:48-51) is the key order and the mark is the key's LSB.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_dist(uint64_t k) {
    const uint32_t o = static_cast<uint32_t>(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ uint64_t make_key(float d, uint32_t id) {
    return (static_cast<uint64_t>(orderable(d)) << 32) | (static_cast<uint64_t>(id & 0x7FFFFFFFu) << 1);
}
__device__ __forceinline__ uint32_t key_id(uint64_t k) { return static_cast<uint32_t>(k >> 1) & 0x7FFFFFFFu; }

// ---------------------------------------------------------------------------
// beam merge: keep the T smallest of (beam U candidates).
// Replaces SharedBitonicTopK::merge / RegBitonicTopK::merge (topk_shared.cuh:272-331).
// Candidates live in registers ck[CR] (candidate index j = rc*64 + lane), `cmask[rc]`
// says which lanes hold one.  Final positions:
//   beam element e moves to e + #(candidates < beam[e]);
//   candidate j moves to #(beam <= cand_j) + #(candidates before j in (key, index)).
// These positions are a permutation of 0..T+c-1; the first T form the new beam.
// A candidate whose key is >= the beam's last key (EMPTY while the beam is not full)
// lands at position >= T and is evicted (ties go after beam entries), so it is dropped
// first.  The beam stays sorted (a mark sets a key's LSB: beam_pick marks the last of a
// run of identical keys).  Two ways to the same result:
//  - rank loop: each remaining candidate kj is broadcast once and compared with every beam
//    register (the compare mask is the ballot): the elements above kj shift by one;
//  - sorted merge (CR = 1, SORTED, at least merge_sort_min<TR>() candidates): the candidates are
//    compacted and bitonic-sorted across lanes, each finds its rank in the beam by a
//    binary search of an LDS copy, the occupied output slots are marked in a bitmap and
//    every output slot gathers its key from the candidate or the beam copy.
// Identical keys are indistinguishable, so the two orders of equal candidates agree.
// LDS: scratch = 64*TR + 1 keys (the last one a dump slot), aux = 64 + TR keys.
// ---------------------------------------------------------------------------
// What merge and pick keep besides the registers: `first`, a lower bound on the register
// that holds the first unexpanded key (0 always is one).  (Finding a candidate's register
// from the registers' last keys instead of comparing it with every register was measured
// slower for every beam size once the large RaBitQ beams defer their merges: 1M x 128, 10k
// queries, rabitq topk 600 5.91 -> 5.60 ms, 768 7.69 -> 6.77, 1024 11.0 -> 9.19 ms without
// it; base topk 1024 unchanged.)
struct BeamState {
    uint32_t first;
};

template <int TR>
__device__ __forceinline__ BeamState beam_state(const uint64_t (&)[TR]) {
    BeamState st;
    st.first = 0;
    return st;
}

// Beams of more than 16 registers (topk 1025..4096): 32 and 64 registers of 64-bit keys.
// A register index that is not a compile-time constant is a register-indexed move, and the
// largest register tuple it can address is 32 dwords (16 keys); an array indexed that way
// beyond that size goes to scratch memory whole.  So every access to a register chosen at
// run time goes through beam_reg / beam_mark, which for the large beams combine all
// registers under a uniform mask (about 4 TR instructions) and keep the beam in VGPRs.  The
// masks are ANDs rather than selects: the compiler folds a chain of selects among array
// elements into a load from a selected address, which is the run-time index again.

// register r of the beam (wave-uniform r: a register-indexed move, s_set_gpr_idx)
template <int TR>
__device__ __forceinline__ uint64_t beam_reg(const uint64_t (&beam)[TR], uint32_t r) {
    if constexpr (TR <= 16) {
        return beam[r];
    } else {
        uint64_t v = 0;
#pragma unroll
        for (int i = 0; i < TR; ++i) v |= beam[i] & (0ull - static_cast<uint64_t>(r == static_cast<uint32_t>(i)));
        return v;
    }
}

// set the mark (key LSB) of the lanes of lm in register r (wave-uniform r)
template <int TR>
__device__ __forceinline__ void beam_mark(uint64_t (&beam)[TR], uint32_t r, uint64_t lm) {
    if constexpr (TR <= 16) {
        beam[r] |= bsw::lane_in(lm) ? 1ull : 0ull;
    } else {
        const uint64_t bit = bsw::lane_in(lm) ? 1ull : 0ull;
#pragma unroll
        for (int i = 0; i < TR; ++i) beam[i] |= bit & static_cast<uint64_t>(r == static_cast<uint32_t>(i));
    }
}

// The rank loop costs ~2 TR + 6 instructions per candidate, the sorted merge ~250 plus LDS
// latency: the crossover.
template <int TR>
__device__ __forceinline__ constexpr uint32_t merge_sort_min() {
    return TR >= 16 ? 3u : TR >= 8 ? 5u : 8u;
}

// EMPTY in the slots at T and beyond (only when T < 64*TR: the gathers above fill
// every register, the registers past T first)
template <int TR>
__device__ __forceinline__ void beam_clear_tail(uint64_t (&beam)[TR], uint32_t T) {
    if (T >= 64u * TR) return;
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint32_t b = static_cast<uint32_t>(r) * 64u;
        const uint64_t live = b >= T ? 0ull : (T - b >= 64u ? ~0ull : (1ull << (T - b)) - 1ull);
        beam[r] = bsw::lane_in(live) ? beam[r] : EMPTY_KEY;
    }
}

// lanes whose index has bit s clear (s a power of two; s = 64: every lane)
__host__ __device__ constexpr uint64_t lanes_bit_clear(uint32_t s) {
    return s == 1    ? 0x5555555555555555ull
           : s == 2  ? 0x3333333333333333ull
           : s == 4  ? 0x0F0F0F0F0F0F0F0Full
           : s == 8  ? 0x00FF00FF00FF00FFull
           : s == 16 ? 0x0000FFFF0000FFFFull
           : s == 32 ? 0x00000000FFFFFFFFull
                     : ~0ull;
}

// ascending bitonic sort of the first P = pow2ceil(n) lanes (lanes beyond hold EMPTY).
// A lane keeps the smaller of its key and its partner's where bit s and bit k of its
// index agree: a constant lane mask.
__device__ __forceinline__ uint64_t sort_lanes(uint64_t v, uint32_t n) {
#pragma unroll
    for (uint32_t k = 2; k <= 64; k <<= 1) {
        if (k / 2 >= n) break;
#pragma unroll
        for (uint32_t s = k >> 1; s >= 1; s >>= 1) {
            const uint64_t p = bsw::xor_lane64_rt(v, s);
            const uint64_t keep_min = ~(lanes_bit_clear(s) ^ lanes_bit_clear(k));
            const uint64_t lt = ballot(p < v);
            v = bsw::lane_in(~(keep_min ^ lt)) ? p : v;
        }
    }
    return v;
}

template <int TR>
__device__ __forceinline__ void beam_merge_sorted(uint64_t (&beam)[TR], uint64_t ck, uint64_t cmask, uint32_t n,
                                                  uint32_t T, uint64_t* B, uint64_t* aux, BeamState& st) {
    const uint32_t lane = lane_id();
    uint64_t* C = aux;       // 64 sorted candidates
    uint64_t* M = aux + 64;  // TR words: bit s = output slot s holds a candidate
    // compact the candidates to C[0..n), copy the beam to B, clear the bitmap
    if (bsw::lane_in(cmask)) C[bsw::lanes_below(cmask)] = ck;
#pragma unroll
    for (int r = 0; r < TR; ++r) B[static_cast<uint32_t>(r) * 64u + lane] = beam[r];
    if (lane < static_cast<uint32_t>(TR)) M[lane] = 0ull;
    wave_sync();
    uint64_t c = lane < n ? C[lane] : EMPTY_KEY;
    c = sort_lanes(c, n);
    // rank in the beam: #(beam <= c).  Registers hold sorted runs of 64, so the run is
    // chosen from the registers' last keys, then 6 halving steps inside it.
    uint32_t lo = 0;
#pragma unroll
    for (int r = 0; r < TR - 1; ++r) lo += (readlane64(beam[r], 63) <= c) ? 64u : 0u;
#pragma unroll
    for (uint32_t step = 32; step >= 1; step >>= 1)
        if (B[lo + step - 1] <= c) lo += step;
    const uint32_t pos = lane + lo;
    st.first = min(st.first, uniform(pos) >> 6);  // lane 0: the smallest candidate
    C[lane] = c;  // sorted (EMPTY past n)
    {
        // every lane ors a word (0 unless it places a candidate): no divergent branch
        const bool place = lane < n && pos < T;
        __hip_atomic_fetch_or(&M[place ? (pos >> 6) : 0u], place ? 1ull << (pos & 63u) : 0ull, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_WAVEFRONT);
    }
    wave_sync();
    uint32_t before = 0;  // candidates in the slots of earlier registers
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint64_t mw = bsw::uniform64(M[r]);
        const uint32_t s = static_cast<uint32_t>(r) * 64u + lane;
        const uint32_t ob = before + bsw::lanes_below(mw);
        // both reads unconditional (a conditional LDS read becomes an exec-mask branch)
        const uint64_t vc = C[min(ob, 63u)];
        const uint64_t vb = B[s - ob];
        beam[r] = bsw::lane_in(mw) ? vc : vb;
        before += static_cast<uint32_t>(__builtin_popcountll(mw));
    }
    beam_clear_tail<TR>(beam, T);
    wave_sync();
}

template <int TR, int CR, bool SORTED = true>
__device__ __forceinline__ void beam_merge(uint64_t (&beam)[TR], const uint64_t (&ck)[CR],
                                           const uint64_t (&cmask_in)[CR], uint32_t T,
                                           uint64_t* lds_scratch, uint64_t* lds_aux, BeamState& st) {
    const uint32_t lane = lane_id();
    const uint64_t thr = readlane64(beam_reg<TR>(beam, (T - 1) >> 6), (T - 1) & 63u);
    uint64_t cmask[CR];
    uint32_t n = 0;
#pragma unroll
    for (int rc = 0; rc < CR; ++rc) {
        cmask[rc] = cmask_in[rc] & ballot(ck[rc] < thr);
        n += static_cast<uint32_t>(__builtin_popcountll(cmask[rc]));
    }
    if (n == 0) return;
    if constexpr (CR == 1 && SORTED) {
        if (n >= merge_sort_min<TR>()) {
            beam_merge_sorted<TR>(beam, ck[0], cmask[0], n, T, lds_scratch, lds_aux, st);
            return;
        }
    }
    // lp[r]: per-lane shift of register r, by every smaller candidate
    uint32_t lp[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) lp[r] = 0;
    uint32_t cpos[CR];
#pragma unroll
    for (int rc = 0; rc < CR; ++rc) cpos[rc] = 0;
    uint32_t minle = 64u * TR;  // the smallest candidate's slot: its beam rank

#pragma unroll
    for (int rj = 0; rj < CR; ++rj) {
        uint64_t m = cmask[rj];
        while (m) {
            const uint32_t lj = static_cast<uint32_t>(__builtin_ctzll(m));
            m &= m - 1;
            const uint64_t kj = readlane64(ck[rj], lj);
            uint32_t ngt = 0;  // #(beam > kj)
#pragma unroll
            for (int r = 0; r < TR; ++r) {
                const uint64_t lt = ballot(kj < beam[r]);
                lp[r] += bsw::lane_in(lt) ? 1u : 0u;
                ngt += static_cast<uint32_t>(__builtin_popcountll(lt));
            }
            const uint32_t le = 64u * TR - ngt;  // #(beam <= kj)
            minle = min(minle, le);
#pragma unroll
            for (int rc = 0; rc < CR; ++rc) {
                // lanes whose candidate index (rc * 64 + lane) is above candidate j's
                const uint64_t above = rc < rj ? 0ull : rc > rj ? ~0ull : ~((2ull << lj) - 1ull);
                const bool before = (kj < ck[rc]) || (kj == ck[rc] && bsw::lane_in(above));
                cpos[rc] += before ? 1u : 0u;
                if (rc == rj) cpos[rc] += bsw::lane_in(1ull << lj) ? le : 0u;
            }
        }
    }
    // unconditional scatter and gather (a conditional LDS access becomes an exec-mask
    // branch).  Positions are a permutation of the beam's 64*TR slots and the candidates;
    // keys landing at 64*TR or beyond go to the dump slot 64*TR, those landing in
    // [T, 64*TR) are overwritten with EMPTY after the gather (beam_clear_tail).
    constexpr uint32_t DUMP = 64u * TR;
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint32_t bpos = static_cast<uint32_t>(r) * 64u + lane + lp[r];
        lds_scratch[min(bpos, DUMP)] = beam[r];
    }
#pragma unroll
    for (int rc = 0; rc < CR; ++rc) lds_scratch[bsw::lane_in(cmask[rc]) ? min(cpos[rc], DUMP) : DUMP] = ck[rc];
    wave_sync();
#pragma unroll
    for (int r = 0; r < TR; ++r) beam[r] = lds_scratch[static_cast<uint32_t>(r) * 64u + lane];
    beam_clear_tail<TR>(beam, T);
    st.first = min(st.first, minle >> 6);
    wave_sync();
}

// ---------------------------------------------------------------------------
// pick<1> (topk_shared.cuh:335-380): mark the smallest unexpanded entry and return its
// id (INVALID if none).  RUN = true (the rabitq beam may hold identical keys): of a run
// of identical keys the last one is marked, which keeps the beam sorted.
// ---------------------------------------------------------------------------

// st.first: keys only move to later slots, so the bound holds until a merge places a
// candidate before it (beam_merge lowers it); the pick scans from it and leaves it at the
// register where it found its key.
// next_key (optional): the unexpanded key that follows the picked one in the beam
// (EMPTY_KEY if none), for a prediction of the following pick.
// beam_pick in two steps, for the deferred merge's pick (pending_pick): the beam's smallest
// unexpanded key (EMPTY_KEY if none), not marked; `at` = its slot 64 r + l, `row_out` = the
// register r itself, st.first advances to it.
template <int TR>
__device__ __forceinline__ uint64_t beam_peek(const uint64_t (&beam)[TR], BeamState& st, uint32_t& at,
                                              uint64_t& row_out) {
    uint32_t pr = st.first;
    uint64_t row, mp;
    for (;;) {
        if (pr >= static_cast<uint32_t>(TR)) {
            st.first = pr;
            at = 64u * TR;
            row_out = EMPTY_KEY;
            return EMPTY_KEY;
        }
        row = beam_reg<TR>(beam, pr);
        mp = ballot((static_cast<uint32_t>(row) & 1u) == 0u);
        if (mp != 0) break;
        ++pr;
    }
    st.first = pr;
    const uint32_t pl = static_cast<uint32_t>(__builtin_ctzll(mp));
    at = 64u * pr + pl;
    row_out = row;
    return readlane64(row, pl);
}

template <int TR, bool RUN>
__device__ __forceinline__ uint32_t beam_pick(uint64_t (&beam)[TR], BeamState& st, uint64_t* next_key = nullptr) {
    // the first register holding an unexpanded key, its first such lane
    uint32_t pr = st.first;
    uint64_t row, mp;
    for (;;) {
        if (pr >= static_cast<uint32_t>(TR)) {
            st.first = pr;
            return INVALID;
        }
        row = beam_reg<TR>(beam, pr);
        mp = ballot((static_cast<uint32_t>(row) & 1u) == 0u);
        if (mp != 0) break;
        ++pr;
    }
    st.first = pr;
    const uint32_t pl = static_cast<uint32_t>(__builtin_ctzll(mp));
    const uint64_t kp = readlane64(row, pl);
    if (next_key) {
        uint64_t nk = EMPTY_KEY;
        const uint64_t mp2 = mp & (mp - 1u);
        if (mp2 != 0) {
            nk = readlane64(row, static_cast<uint32_t>(__builtin_ctzll(mp2)));
        } else {
            for (uint32_t r = pr + 1; r < static_cast<uint32_t>(TR); ++r) {
                const uint64_t row2 = beam_reg<TR>(beam, r);
                const uint64_t m2 = ballot((static_cast<uint32_t>(row2) & 1u) == 0u);
                if (m2 != 0) {
                    nk = readlane64(row2, static_cast<uint32_t>(__builtin_ctzll(m2)));
                    break;
                }
            }
        }
        *next_key = nk;
    }
    uint32_t qr = pr, ql = pl;
    if constexpr (RUN) {
        // identical keys are rare: look at the next element first, scan only if it repeats
        uint64_t nxt = EMPTY_KEY;
        if (pl < 63u) nxt = readlane64(row, pl + 1u);
        else if (pr + 1u < static_cast<uint32_t>(TR)) nxt = readlane64(beam_reg<TR>(beam, pr + 1u), 0u);
        if (nxt == kp) {
#pragma unroll
            for (int r = 0; r < TR; ++r) {
                const uint64_t mm = ballot(beam[r] == kp);
                if (static_cast<uint32_t>(r) >= pr && mm != 0) {
                    qr = static_cast<uint32_t>(r);
                    ql = 63u - static_cast<uint32_t>(__builtin_clzll(mm));
                }
            }
        }
    }
    // set the mark (key LSB) of element (qr, ql)
    beam_mark<TR>(beam, qr, 1ull << ql);
    return key_id(kp);
}

// exact 64-bit minimum of v over the wave (every lane active): the upper words' minimum by
// a butterfly in rows of 16 and the rows' results, then, when more than one lane holds that
// upper word, the lower words' minimum among them
__device__ __forceinline__ uint64_t wave_min64(uint64_t v) {
    const uint32_t vh = static_cast<uint32_t>(v >> 32);
    uint32_t h = vh;
    h = min(h, bsw::xor_lane<1>(h));
    h = min(h, bsw::xor_lane<2>(h));
    h = min(h, bsw::partner<4>(h));
    h = min(h, bsw::partner<8>(h));
    const uint32_t m = min(min(readlane(h, 0), readlane(h, 16)), min(readlane(h, 32), readlane(h, 48)));
    const uint64_t at = ballot(vh == m);
    const uint32_t l0 = static_cast<uint32_t>(__builtin_ctzll(at));
    if ((at & (at - 1u)) == 0) return (static_cast<uint64_t>(m) << 32) | readlane(static_cast<uint32_t>(v), l0);
    uint32_t lo = bsw::lane_in(at) ? static_cast<uint32_t>(v) : 0xFFFFFFFFu;
    lo = min(lo, bsw::xor_lane<1>(lo));
    lo = min(lo, bsw::xor_lane<2>(lo));
    lo = min(lo, bsw::partner<4>(lo));
    lo = min(lo, bsw::partner<8>(lo));
    const uint32_t ml = min(min(readlane(lo, 0), readlane(lo, 16)), min(readlane(lo, 32), readlane(lo, 48)));
    return (static_cast<uint64_t>(m) << 32) | ml;
}

// ---------------------------------------------------------------------------
// Deferred merge.  The beam must hold the T smallest keys merged so far, and a key
// evicted once never returns (the T-th key only falls).  So candidates need not enter
// the beam at once: those below the beam's last key are appended to a pending list of up
// to 64 keys (one per lane), which is merged into the beam (beam_merge) when it would overflow
// and whenever the beam itself is needed (filter re-fill, rerank, results).  The T
// smallest of (beam U list) are exactly the T smallest keys merged so far (a key the beam
// evicted or the list refused has at least T smaller keys).  The pick takes the smallest
// unmarked key u of beam and list: u is among the T smallest iff fewer than T keys of the
// union are smaller, and those are all marked, so the count is needed only once T picks
// have been made.  Identical keys are indistinguishable, so which copy of a key carries a
// mark does not matter -- except when a key is held unmarked more than once (RaBitQ): the
// immediate merge may have evicted some of those copies, so such a pick merges the list
// first (pending_pick).  With that rule every pick, merge and result is the one of an
// immediate merge (checked against the oracle, which merges at once).
// ---------------------------------------------------------------------------
struct PendingList {
    uint64_t* k;   // 64 key slots in the wave's LDS, the staging area of appends
    uint32_t n;    // keys held
    uint64_t v;    // the list itself: key `lane` in lane `lane` (< n), EMPTY_KEY above
    uint64_t thr;  // the beam's last key (slot T - 1), kept current by the functions below,
                   // the only ones that change the beam while the list is in use
};

// the beam's key in slot T - 1 (EMPTY_KEY while the beam is not full)
template <int TR>
__device__ __forceinline__ uint64_t beam_last(const uint64_t (&beam)[TR], uint32_t T) {
    return readlane64(beam_reg<TR>(beam, (T - 1) >> 6), (T - 1) & 63u);
}

template <int TR>
__device__ __forceinline__ void pending_flush(uint64_t (&beam)[TR], PendingList& pd, uint32_t T, uint64_t* scratch,
                                              uint64_t* aux, BeamState& st) {
    if (pd.n == 0) return;
    const uint64_t ck[1] = {pd.v};
    const uint64_t cm[1] = {pd.n >= 64u ? ~0ull : (1ull << pd.n) - 1ull};
    beam_merge<TR, 1>(beam, ck, cm, T, scratch, aux, st);
    pd.n = 0;
    pd.v = EMPTY_KEY;
    pd.thr = beam_last<TR>(beam, T);
}

// candidates ck (lanes cm, every one below the beam's last key: the caller has filtered
// them against it) into the list; a full list is merged first, and candidates that do not
// fit even then are merged directly
template <int TR, int CR>
__device__ __forceinline__ void pending_add(uint64_t (&beam)[TR], const uint64_t (&ck)[CR], const uint64_t (&cm)[CR],
                                            PendingList& pd, uint32_t T, uint64_t* scratch, uint64_t* aux,
                                            BeamState& st) {
    uint64_t ok[CR];
    uint32_t n = 0;
#pragma unroll
    for (int rc = 0; rc < CR; ++rc) {
        ok[rc] = cm[rc];
        n += static_cast<uint32_t>(__builtin_popcountll(ok[rc]));
    }
    if (n == 0) return;
    if (pd.n + n > 64u) {
        pending_flush<TR>(beam, pd, T, scratch, aux, st);
        n = 0;
#pragma unroll
        for (int rc = 0; rc < CR; ++rc) {
            ok[rc] &= ballot(ck[rc] < pd.thr);
            n += static_cast<uint32_t>(__builtin_popcountll(ok[rc]));
        }
        if (n == 0) return;
        if (n > 64u) {
            beam_merge<TR, CR>(beam, ck, ok, T, scratch, aux, st);
            pd.thr = beam_last<TR>(beam, T);
            return;
        }
    }
    // the new keys are compacted through the LDS slots above the list's end; the slots
    // below it are stale (marks are set in the register copy only) and not read
    const uint32_t n0 = pd.n;
    uint32_t at = n0;
#pragma unroll
    for (int rc = 0; rc < CR; ++rc) {
        if (bsw::lane_in(ok[rc])) pd.k[at + bsw::lanes_below(ok[rc])] = ck[rc];
        at += static_cast<uint32_t>(__builtin_popcountll(ok[rc]));
    }
    pd.n = at;
    wave_sync();
    const uint32_t lane = lane_id();
    const uint64_t r = pd.k[lane];
    pd.v = lane < n0 ? pd.v : (lane < at ? r : EMPTY_KEY);
}

// pick over beam and list (the beam_pick of an immediately merged beam); picks = marks
// made so far, counted here.  With RUN, a key held unmarked more than once is picked from
// the merged beam: the immediate merge may have evicted some of its copies, and which
// copies are left decides which one carries the mark, so the list is merged first.
template <int TR, bool RUN>
__device__ __forceinline__ uint32_t pending_pick(uint64_t (&beam)[TR], BeamState& st, PendingList& pd, uint32_t T,
                                                 uint64_t* scratch, uint64_t* aux, uint32_t& picks) {
    const uint32_t lane = lane_id();
    const uint64_t v = pd.v;
    uint32_t at;
    uint64_t row;
    const uint64_t ub = beam_peek<TR>(beam, st, at, row);
    // the list's smallest unmarked key, wanted only when it is <= ub: the lanes whose
    // unmarked key is <= ub say whether it is, and with one such lane the key is its key
    // (1M x 128, 10k queries, rabitq topk 512 3.72 -> 3.66 ms, 768 5.88 -> 5.84)
    uint64_t pmin = EMPTY_KEY;
    if (pd.n > 0) {
        const uint64_t um = (v & 1ull) ? EMPTY_KEY : v;
        // (when ub is EMPTY every lane qualifies and pmin is the plain minimum, EMPTY if the
        // list holds no unmarked key)
        const uint64_t le = ballot(um <= ub);
        if (le != 0)
            pmin = (le & (le - 1u)) == 0 ? readlane64(um, static_cast<uint32_t>(__builtin_ctzll(le))) : wave_min64(um);
    }
    const bool from_list = pmin <= ub && pmin != EMPTY_KEY;
    const uint64_t u = from_list ? pmin : ub;
    if (u == EMPTY_KEY) return INVALID;
    // a pick from the beam: the key after it, read once for the duplicate check and the mark
    // (the beam's unmarked copies of u follow it)
    uint64_t kn = EMPTY_KEY;
    if (RUN && !from_list) {
        // in the register beam_peek read unless u is its last lane
        const uint32_t nx = at + 1u;
        if ((nx & 63u) != 0u) kn = readlane64(row, nx & 63u);
        else if (nx < 64u * TR) kn = readlane64(beam_reg<TR>(beam, nx >> 6), 0u);
    }
    if constexpr (RUN) {
        if (pd.n > 0) {
            const bool dup = from_list ? (ub == u || __builtin_popcountll(ballot(v == u)) >= 2) : kn == u;
            if (dup) {
                pending_flush<TR>(beam, pd, T, scratch, aux, st);
                const uint32_t id = beam_pick<TR, true>(beam, st);
                pd.thr = beam_last<TR>(beam, T);  // the mark may have been slot T - 1's
                picks += id != INVALID ? 1u : 0u;
                return id;
            }
        }
    }
    if (picks >= T) {
        // u must be among the T smallest of beam U list
        uint32_t below = 0;
#pragma unroll
        for (int r = 0; r < TR; ++r) below += static_cast<uint32_t>(__builtin_popcountll(ballot(beam[r] < u)));
        below += static_cast<uint32_t>(__builtin_popcountll(ballot(v < u)));
        if (below >= T) return INVALID;
    }
    ++picks;
    // The slot to mark, (mr, ml), with ml = 64 for a pick from the list: one register-indexed
    // write on every path.  A write on some paths only made the compiler copy the whole
    // beam (its registers as one 32-register tuple) to another tuple and back at the join:
    // 32 64-bit moves per mark at 10 registers.
    uint32_t mr = 0, ml = 64;
    if (from_list) {
        const uint32_t l = static_cast<uint32_t>(__builtin_ctzll(ballot(v == u)));
        pd.v = v | (lane == l ? 1ull : 0ull);
    } else {
        mr = at >> 6;
        ml = at & 63u;
        if (RUN && kn == u) {
            // of a run of identical keys the last one is marked (the beam stays sorted)
#pragma unroll
            for (int r = 0; r < TR; ++r) {
                const uint64_t mm = ballot(beam[r] == ub);
                if (static_cast<uint32_t>(r) >= (at >> 6) && mm != 0) {
                    mr = static_cast<uint32_t>(r);
                    ml = 63u - static_cast<uint32_t>(__builtin_clzll(mm));
                }
            }
        }
    }
    const uint64_t lm = ml < 64u ? (1ull << ml) : 0ull;
    beam_mark<TR>(beam, mr, lm);
    if (ml < 64u && 64u * mr + ml == T - 1u) pd.thr |= 1ull;
    return key_id(u);
}

// The smallest key held by the lanes of k[0..CR) (EMPTY_KEY if none), for the prediction
// of the next pick: after a merge the smallest unexpanded key is the smaller of the beam's
// next unexpanded key (beam_pick's next_key) and the smallest merged candidate.  The upper
// words are reduced exactly; among keys sharing the smallest upper word the lowest lane's
// is returned.
template <int CR>
__device__ __forceinline__ uint64_t wave_min_key(const uint64_t (&k)[CR]) {
    uint64_t v = k[0];
#pragma unroll
    for (int rc = 1; rc < CR; ++rc) v = k[rc] < v ? k[rc] : v;
    const uint32_t vh = static_cast<uint32_t>(v >> 32);
    uint32_t h = vh;
    h = min(h, bsw::xor_lane<1>(h));
    h = min(h, bsw::xor_lane<2>(h));
    h = min(h, bsw::partner<4>(h));
    h = min(h, bsw::partner<8>(h));
    const uint32_t m = min(min(readlane(h, 0), readlane(h, 16)), min(readlane(h, 32), readlane(h, 48)));
    return readlane64(v, static_cast<uint32_t>(__builtin_ctzll(ballot(vh == m))));
}

// ---------------------------------------------------------------------------
// bitonic sort of the 64*TR register-major keys, ascending (the rerank re-sort,
// topk_shared.cuh:384-416).  Partners at distance >= 64 are other registers of the same
// lane; closer partners are cross-lane exchanges (DPP / swizzle / bpermute).
// ---------------------------------------------------------------------------
template <int TR>
__device__ __forceinline__ void bitonic_sort(uint64_t (&v)[TR]) {
    const uint32_t lane = lane_id();
    constexpr uint32_t N = 64u * TR;
#pragma unroll
    for (uint32_t k = 2; k <= N; k <<= 1) {
#pragma unroll
        for (uint32_t s = k >> 1; s >= 1; s >>= 1) {
            if (s >= 64) {
                const uint32_t rs = s / 64u;
#pragma unroll
                for (uint32_t r = 0; r < TR; ++r) {
                    if ((r & rs) == 0) {
                        const uint32_t r2 = r | rs;
                        const uint32_t e = r * 64u + lane;
                        const bool asc = (e & k) == 0;
                        const uint64_t a = v[r], b = v[r2];
                        const bool sw = asc ? (b < a) : (a < b);
                        v[r] = sw ? b : a;
                        v[r2] = sw ? a : b;
                    }
                }
            } else {
#pragma unroll
                for (uint32_t r = 0; r < TR; ++r) {
                    const uint64_t p = bsw::xor_lane64_rt(v[r], s);
                    const uint32_t e = r * 64u + lane;
                    const bool asc = (e & k) == 0;
                    const bool lower = (lane & s) == 0;
                    const bool keep_min = (lower == asc);
                    const uint64_t mn = p < v[r] ? p : v[r];
                    const uint64_t mx = p < v[r] ? v[r] : p;
                    v[r] = keep_min ? mn : mx;
                }
            }
        }
    }
}

// The same network for beams of more than 16 registers (2048 and 4096 keys), run in LDS:
// unrolled over registers it is more code than the compiler will unroll, and a loop over
// registers indexes them at run time.  The keys go to S[0, 64 TR) register-major, every step
// of the network makes its 32 TR compare-exchanges 64 at a time, and the keys come back.
template <int TR>
__device__ __forceinline__ void sort_beam_lds(uint64_t (&v)[TR], uint64_t* S) {
    static_assert((TR & (TR - 1)) == 0, "the bitonic network sorts a power of two of keys");
    const uint32_t lane = lane_id();
    constexpr uint32_t N = 64u * TR;
#pragma unroll
    for (int r = 0; r < TR; ++r) S[static_cast<uint32_t>(r) * 64u + lane] = v[r];
    wave_sync();
#pragma unroll 1
    for (uint32_t k = 2; k <= N; k <<= 1) {
#pragma unroll 1
        for (uint32_t j = k >> 1; j >= 1; j >>= 1) {
            // pair i: elements a (bit j clear) and a + j; ascending where bit k of a is clear
#pragma unroll 4
            for (uint32_t i = lane; i < N / 2; i += 64) {
                const uint32_t a = ((i & ~(j - 1u)) << 1) | (i & (j - 1u));
                const uint64_t x = S[a], y = S[a + j];
                const bool sw = (a & k) == 0 ? (y < x) : (x < y);
                S[a] = sw ? y : x;
                S[a + j] = sw ? x : y;
            }
            wave_sync();
        }
    }
#pragma unroll
    for (int r = 0; r < TR; ++r) v[r] = S[static_cast<uint32_t>(r) * 64u + lane];
    wave_sync();
}

// the same for any register count: counts that are not a power of two sort in the next
// power of two, padded with EMPTY keys (which sort last); beams of more than 16 registers
// sort in S (64 TR keys of LDS; unused otherwise)
template <int TR>
__device__ __forceinline__ void sort_beam(uint64_t (&v)[TR], uint64_t* S) {
    if constexpr (TR > 16) {
        sort_beam_lds<TR>(v, S);
    } else if constexpr ((TR & (TR - 1)) == 0) {
        bitonic_sort<TR>(v);
    } else {
        constexpr int P = 16;  // the register counts that are not a power of two: 10 and 12
        static_assert(TR < P, "padded to 16 registers");
        uint64_t w[P];
#pragma unroll
        for (int r = 0; r < P; ++r) w[r] = r < TR ? v[r] : EMPTY_KEY;
        bitonic_sort<P>(w);
#pragma unroll
        for (int r = 0; r < TR; ++r) v[r] = w[r];
    }
}

// ---------------------------------------------------------------------------
// visit filters in the wave's LDS slice
// ---------------------------------------------------------------------------

// HashFilter (filter_hash.cuh:11-99): an LDS set of node ids with linear probing, empty =
// 0xFFFFFFFF, that refuses keys once `cap` are stored (the reference's table has cap =
// 2^ceil(log2 capacity) slots).  Membership does not depend on where keys sit, so the table
// may have more slots than cap (shorter probe runs).  A key's probe sequence is the slots
// from its home slot on; it sits in the first empty slot of its sequence at insertion and
// slots never empty, so a lookup stops at the key (present) or an empty slot (absent).
// Inserts go slot by slot (a compare-and-swap returns the slot's key); lookups read 4 slots
// (16 B, one ds_read_b128) per step.  `occ` counts occupied slots (wave-uniform).  The
// table has any multiple of 4 slots (sized to the LDS the wavefront's residency leaves), so
// the home slot is a multiplicative hash scaled to [0, size) rather than the reference's
// power-of-two mask; where a key sits never changes a result.
struct HashLds {
    uint32_t* t;
    uint32_t size;  // slots, a multiple of 4
    uint32_t cap;   // keys accepted
    uint32_t occ;

    __device__ __forceinline__ uint32_t home(uint32_t k) const {
        return static_cast<uint32_t>((static_cast<uint64_t>(k * 0x9E3779B1u) * size) >> 32);
    }
    __device__ __forceinline__ uint32_t next(uint32_t i) const { return i + 1 == size ? 0u : i + 1; }
    __device__ __forceinline__ uint32_t add(uint32_t i, uint32_t d) const {  // d < size
        return i + d >= size ? i + d - size : i + d;
    }

    __device__ __forceinline__ void clear() {
        const uint32_t lane = lane_id();
        uint4* t4 = reinterpret_cast<uint4*>(t);
        const uint4 e = make_uint4(INVALID, INVALID, INVALID, INVALID);
        for (uint32_t i = lane; i < (size >> 2); i += 64) t4[i] = e;
        occ = 0;
        wave_sync();
    }

    // one key, sequential semantics, all lanes cooperate: probe 64 consecutive slots per
    // step, first slot that holds k (present) or is empty (insert there).
    // returns 1 if newly inserted; 0 if present or the table is full.
    __device__ __forceinline__ uint32_t insert1(uint32_t k) {
        if (occ >= cap) return 0u;  // full: present or rejected, 0 either way
        const uint32_t lane = lane_id();
        const uint32_t h = home(k);
        for (uint32_t base = 0; base < size; base += 64) {
            const uint32_t off = base + lane;
            const uint32_t idx = add(h, off < size ? off : 0u);
            const uint32_t s = t[idx];  // lanes past the table read the home slot, masked below
            const uint64_t in = size - base >= 64u ? ~0ull : (1ull << (size - base)) - 1ull;
            const uint64_t hit = ballot(s == k) & in;
            const uint64_t any = hit | (ballot(s == INVALID) & in);
            if (any) {
                const uint32_t first = static_cast<uint32_t>(__builtin_ctzll(any));
                if ((hit >> first) & 1ull) return 0u;
                if (bsw::lane_in(1ull << first)) t[idx] = k;
                wave_sync();
                occ += 1;
                return 1u;
            }
        }
        return 0u;
    }

    // Lanes of `active` whose key is in the table.  Every lane of the wave takes part: the
    // probe runs group by group for the whole wave, with the lanes still searching kept in
    // a mask, until each of them has met its key or an empty slot.  A key's sequence starts
    // at its home slot: the slots before it in its group of 4 are not in the sequence (they
    // end it, after a full turn).
    // The first group (home_group, read ahead by the caller so that its LDS latency hides
    // behind other work) is passed in.
    __device__ __forceinline__ uint4 home_group(uint32_t k) const {
        return reinterpret_cast<const uint4*>(t)[home(k) >> 2];
    }
    __device__ __forceinline__ uint64_t contains_mask(uint32_t k, uint64_t active) const {
        return contains_mask(k, active, home_group(k));
    }
    __device__ __forceinline__ uint64_t contains_mask(uint32_t k, uint64_t active, uint4 v) const {
        const uint4* t4 = reinterpret_cast<const uint4*>(t);
        const uint32_t s0 = home(k);
        const uint32_t nq = size >> 2;
        uint32_t q = s0 >> 2;
        const uint32_t f = s0 & 3u;
        const uint64_t f0 = ballot(f == 0u), f1 = ballot(f <= 1u), f2 = ballot(f <= 2u);
        uint64_t hit = (ballot(v.x == k) & f0) | (ballot(v.y == k) & f1) | (ballot(v.z == k) & f2) | ballot(v.w == k);
        const uint64_t emp = (ballot(v.x == INVALID) & f0) | (ballot(v.y == INVALID) & f1) |
                             (ballot(v.z == INVALID) & f2) | ballot(v.w == INVALID);
        uint64_t found = hit & active;
        uint64_t pending = active & ~(hit | emp);
        for (uint32_t i = 0; pending != 0 && i < nq; ++i) {
            q = q + 1 == nq ? 0u : q + 1;
            v = t4[q];
            hit = ballot(v.x == k) | ballot(v.y == k) | ballot(v.z == k) | ballot(v.w == k);
            // INVALID is the largest word: a group holds an empty slot iff its maximum is INVALID
            const uint64_t e = ballot(max(max(v.x, v.y), max(v.z, v.w)) == INVALID);
            found |= hit & pending;
            pending &= ~(hit | e);
        }
        return found;
    }

    // lane-parallel batch (one key per lane, INVALID = idle).  Sequential semantics in
    // lane order (DESC: from lane 63 down): when the batch cannot fill the table, every
    // lane inserts concurrently with LDS compare-and-swap (membership does not depend on the
    // order); otherwise the keys are inserted one by one in that order.  Returns 1 for
    // newly inserted keys.
    template <bool DESC = false>
    __device__ __forceinline__ uint32_t insert_batch(uint32_t k) {
        const uint32_t lane = lane_id();
        const bool valid = k != INVALID;
        const uint64_t vm = ballot(valid);
        const uint32_t nv = static_cast<uint32_t>(__builtin_popcountll(vm));
        uint32_t isnew = 0;
        // A full table accepts nothing and every key already present reports 0, so the
        // batch changes nothing (filter_hash.cuh:78-86 probes all slots to the same end).
        if (nv == 0 || occ >= cap) return 0;
        if (occ + nv <= cap) {
            uint32_t idx = home(k);
            bool done = !valid;
            for (uint32_t step = 0; step <= size; ++step) {
                if (ballot(!done) == 0) break;
                if (!done) {
                    const uint32_t old = atomicCAS(&t[idx], INVALID, k);
                    if (old == INVALID) {
                        isnew = 1;
                        done = true;
                    } else if (old == k) {
                        done = true;
                    } else {
                        idx = next(idx);
                    }
                }
            }
            wave_sync();
            occ += static_cast<uint32_t>(__builtin_popcountll(ballot(isnew != 0)));
        } else {
            // one key at a time until the table fills; the keys after that all report 0
            uint64_t m = vm;
            while (m && occ < cap) {
                const uint32_t l = DESC ? 63u - static_cast<uint32_t>(__builtin_clzll(m))
                                        : static_cast<uint32_t>(__builtin_ctzll(m));
                m &= ~(1ull << l);
                const uint32_t r = insert1(readlane(k, l));
                if (lane == l) isnew = r;
            }
        }
        return isnew;
    }
};

// BloomFilter (filter_bloom.cuh:13-131): 2^max(5, bits) bits, three hashes.  The
// reference's warp filters a row in rounds of 32 neighbours (gpu_search_warp.cuh:203-205,
// lane stride BX = 32), each lane testing its key's bits and then setting them
// (filter_bloom.cuh:104-120), so a round's keys see the bits of every earlier round.
// Within a round the test-then-atomicOr races for a key held twice; the rule here: a key
// is new iff its bits were not all set before its round and it is the first index of the
// round holding that value.
struct BloomLds {
    uint32_t* w;
    uint32_t bits, words, mask;

    __device__ __forceinline__ void hashes(uint32_t key, uint32_t& h0, uint32_t& h1, uint32_t& h2) const {
        uint32_t a = key;
        a ^= a >> 16;
        a *= 0x45d9f3bu;
        a ^= a >> 16;
        h0 = a & mask;
        uint32_t b = key * 0x9e3779b9u;
        b ^= b >> 16;
        b *= 0x45d9f3bu;
        b ^= b >> 16;
        h1 = b & mask;
        uint32_t c = key * 0x517cc1b7u;
        c ^= c >> 16;
        c *= 0x45d9f3bu;
        c ^= c >> 16;
        h2 = c & mask;
    }

    __device__ __forceinline__ void clear() {
        const uint32_t lane = lane_id();
        for (uint32_t i = lane; i < words; i += 64) w[i] = 0u;
        wave_sync();
    }

    __device__ __forceinline__ bool test_lane(uint32_t k) const {
        uint32_t h0, h1, h2;
        hashes(k, h0, h1, h2);
        return ((w[h0 >> 5] >> (h0 & 31)) & 1u) && ((w[h1 >> 5] >> (h1 & 31)) & 1u) &&
               ((w[h2 >> 5] >> (h2 & 31)) & 1u);
    }

    __device__ __forceinline__ void set_lane(uint32_t k) {
        uint32_t h0, h1, h2;
        hashes(k, h0, h1, h2);
        atomicOr(&w[h0 >> 5], 1u << (h0 & 31));
        atomicOr(&w[h1 >> 5], 1u << (h1 & 31));
        atomicOr(&w[h2 >> 5], 1u << (h2 & 31));
    }

    // keys k[rc] (rc-th register, index rc*64 + lane); returns new flags per register.
    // Rounds of 32 indices in index order: register rc's lanes 0-31, then its lanes 32-63.
    template <int CR>
    __device__ __forceinline__ void insert_batch(const uint32_t (&k)[CR], uint32_t (&isnew)[CR]) {
        const uint32_t lane = lane_id();
        const bool upper = lane >= 32u;
#pragma unroll
        for (int rc = 0; rc < CR; ++rc) {
            isnew[rc] = 0u;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const bool valid = (upper == (h == 1)) && k[rc] != INVALID;
                if (ballot(valid) == 0) continue;
                const bool absent = valid && !test_lane(k[rc]);
                // first occurrence among the round's absent keys: a key equal to one of them
                // hashes to the same bits, so it is absent too, and only absent keys can be new
                uint64_t m = ballot(absent);
                bool dup = false;
                while (m) {
                    const uint32_t lj = static_cast<uint32_t>(__builtin_ctzll(m));
                    m &= m - 1;
                    dup = dup || (k[rc] == readlane(k[rc], lj) && lj < lane);
                }
                wave_sync();  // every test of the round reads the bits before any is set
                if (valid) set_lane(k[rc]);
                isnew[rc] = (absent && !dup) ? 1u : isnew[rc];
                wave_sync();
            }
        }
    }
};

// ---------------------------------------------------------------------------
// L2 (l2.cuh:26-40, rebuilt for wave64).  Rows are zero-padded to a multiple of 4
// floats; a row is handled by G lanes (G = min(64, pow2ceil(dim/4))), lane `lig` of a
// group accumulates chunks lig, lig+G, ... with one fma per component, and the group
// sums its partials with an xor butterfly.  The same order is restated on the CPU
// (orc_l2_wave in oracle/bs_oracle.c).
// ---------------------------------------------------------------------------
struct L2Shape {
    uint32_t G, gshift, QR, chunks, rpp;  // rpp = rows per pass = 64 / G
};

// Row layout for `dim`: chunks = dim/4 float4 chunks; G = pow2ceil(chunks)/4 lanes per row
// (1 <= G <= 64), so each lane holds QR = ceil(chunks/G) <= 4 chunks (for dim <= 1024) and a
// 64-lane pass covers 64/G rows.  Four chunks per lane keep the butterfly short (log2 G
// steps per pass) and put 64/G rows of loads in flight per pass.
// Passes in flight for l2_rows: about `rows` rows per batch, 2..8 passes (at most 128
// VGPRs of loads; a row of dim > 256 spans 32 or 64 lanes, so one pass holds only 1-2
// rows).  The search asks for 16 rows, or 32 for hash-filter searches over rows of up to
// 128 dims (a degree-32 neighbour list in one HBM round trip).
__host__ __device__ inline int l2_passes_in_flight(const L2Shape& L, uint32_t rows = 16) {
    const uint32_t pb = rows / L.rpp;
    return pb <= 2u ? 2 : pb >= 8u ? 8 : static_cast<int>(pb);
}

__host__ __device__ inline L2Shape l2_shape(uint32_t dim) {
    L2Shape L;
    L.chunks = (dim + 3) / 4;
    uint32_t p = 1;
    while (p < L.chunks) p <<= 1;
    L.G = p >= 4 ? p / 4 : 1;
    if (L.G > 64) L.G = 64;
    L.gshift = 0;
    while ((1u << L.gshift) < L.G) ++L.gshift;
    L.QR = (L.chunks + L.G - 1) / L.G;
    L.rpp = 64 / L.G;
    return L;
}

// The shape with one chunk per lane: G = pow2ceil(chunks) lanes per row (at most 64), so
// QR = 1 for rows of up to 256 dims.  Used by the RaBitQ search with narrow codes (dim <= 128)
// in its loop, which computes one row at a time (the entry point, then each expanded node's
// exact distance): the whole wavefront on one row takes a quarter of the instructions of the
// 4-chunk shape, whose 8 lane groups would each repeat the same row.  Its final rerank of many
// rows keeps the 4-chunk shape.  (orc_l2_wave_lanes in oracle/bs_oracle.c.)
__host__ __device__ inline L2Shape l2_shape_lanes(uint32_t dim) {
    L2Shape L;
    L.chunks = (dim + 3) / 4;
    uint32_t p = 1;
    while (p < L.chunks) p <<= 1;
    L.G = p > 64 ? 64 : p;
    L.gshift = 0;
    while ((1u << L.gshift) < L.G) ++L.gshift;
    L.QR = (L.chunks + L.G - 1) / L.G;
    L.rpp = 64 / L.G;
    return L;
}

// Loads of PB rows (one row per lane group per pass), issued without waiting.  Every
// load is unconditional -- chunks outside the row are redirected to chunk 0 of the same
// row (l2_accum zeroes their difference) -- so all PB*QMAX loads of a lane are in flight
// together (a conditional load would be followed by its own wait before the next one
// issues).  rows[t] must point at a valid row for every lane (inactive groups pass row 0).
// UNIFORM: every lane's rows[t] is the same (a picked node's record), loaded from a scalar base.
template <int QMAX, int PB, bool UNIFORM = false>
__device__ __forceinline__ void l2_load(const float* const (&rows)[PB], uint32_t lig, const L2Shape& L,
                                        float4 (&v)[PB][QMAX]) {
#pragma unroll
    for (int t = 0; t < PB; ++t) {
        const float4* r4 = reinterpret_cast<const float4*>(rows[t]);
#pragma unroll
        for (int kk = 0; kk < QMAX; ++kk) {
            const uint32_t j = lig + static_cast<uint32_t>(kk) * L.G;
            const bool ok = static_cast<uint32_t>(kk) < L.QR && j < L.chunks;
            if constexpr (UNIFORM) v[t][kk] = bsw::load_off<float4>(r4, (ok ? j : 0u) << 4);
            else v[t][kk] = r4[ok ? j : 0u];
        }
    }
}

// Lane partial sums of squared differences of the rows loaded by l2_load, in chunk order
// with explicit fma (the order the oracle's wave L2 restates).
template <int QMAX, int PB>
__device__ __forceinline__ void l2_accum(const float4 (&q)[QMAX], const float4 (&v)[PB][QMAX], uint32_t lig,
                                         const L2Shape& L, float (&p)[PB]) {
    const bool full = L.QR * L.G == L.chunks && L.QR == static_cast<uint32_t>(QMAX);
#pragma unroll
    for (int t = 0; t < PB; ++t) {
        float acc = 0.0f;
#pragma unroll
        for (int kk = 0; kk < QMAX; ++kk) {
            const uint32_t j = lig + static_cast<uint32_t>(kk) * L.G;
            const bool ok = full || (static_cast<uint32_t>(kk) < L.QR && j < L.chunks);
            float d0 = q[kk].x - v[t][kk].x, d1 = q[kk].y - v[t][kk].y, d2 = q[kk].z - v[t][kk].z,
                  d3 = q[kk].w - v[t][kk].w;
            if (!ok) d0 = d1 = d2 = d3 = 0.0f;
            acc = __builtin_fmaf(d0, d0, acc);
            acc = __builtin_fmaf(d1, d1, acc);
            acc = __builtin_fmaf(d2, d2, acc);
            acc = __builtin_fmaf(d3, d3, acc);
        }
        p[t] = acc;
    }
}

template <int QMAX, int PB>
__device__ __forceinline__ void l2_partials(const float4 (&q)[QMAX], const float* const (&rows)[PB], uint32_t lig,
                                            const L2Shape& L, float (&p)[PB]) {
    float4 v[PB][QMAX];
    l2_load<QMAX, PB>(rows, lig, L, v);
    l2_accum<QMAX, PB>(q, v, lig, L, p);
}

// query chunks of this lane: chunk j = lig + k*G, components beyond dim are 0
template <int QMAX>
__device__ __forceinline__ void load_query(const float* qv, uint32_t dim, uint32_t lig, const L2Shape& L,
                                           float4 (&q)[QMAX]) {
#pragma unroll
    for (int kk = 0; kk < QMAX; ++kk) {
        const uint32_t j = lig + static_cast<uint32_t>(kk) * L.G;
        float c[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t i = 4u * j + static_cast<uint32_t>(t);
            c[t] = (static_cast<uint32_t>(kk) < L.QR && j < L.chunks && i < dim) ? qv[i] : 0.0f;
        }
        q[kk] = make_float4(c[0], c[1], c[2], c[3]);
    }
}

// Distances of `cnt` rows whose ids are in lds_ids[0..cnt), written to lds_d[0..cnt).
// Rows are `stride` floats apart.  Passes of rpp rows, PB passes (PB * QMAX float4 loads
// per lane) in flight before the first reduction.
template <int QMAX, int PB>
__device__ __forceinline__ void l2_rows(const float4 (&q)[QMAX], const float* base, uint64_t stride,
                                        const uint32_t* lds_ids, float* lds_d, uint32_t cnt,
                                        const L2Shape& L) {
    const uint32_t lane = lane_id();
    const uint32_t g = lane >> L.gshift, lig = lane & (L.G - 1);
    for (uint32_t j0 = 0; j0 < cnt; j0 += PB * L.rpp) {
        const float* rows[PB];
#pragma unroll
        for (int t = 0; t < PB; ++t) {
            const uint32_t j = j0 + static_cast<uint32_t>(t) * L.rpp + g;
            const uint32_t id = (j < cnt) ? lds_ids[j] : 0u;
            rows[t] = base + static_cast<uint64_t>(id) * stride;
        }
        float p[PB];
        l2_partials<QMAX, PB>(q, rows, lig, L, p);
#pragma unroll
        for (int t = 0; t < PB; ++t) {
            const float s = bsw::group_sum(p[t], L.G);
            const uint32_t j = j0 + static_cast<uint32_t>(t) * L.rpp + g;
            if (lig == 0 && j < cnt) lds_d[j] = s;
        }
    }
    wave_sync();
}

// L2 of one row, result in every lane
template <int QMAX>
__device__ __forceinline__ float l2_one(const float4 (&q)[QMAX], const float* row, const L2Shape& L) {
    const uint32_t lig = lane_id() & (L.G - 1);
    const float* const rows[1] = {row};
    float p[1];
    l2_partials<QMAX, 1>(q, rows, lig, L, p);
    const float r = bsw::group_sum(p[0], L.G);
    return __uint_as_float(readlane(__float_as_uint(r), 0));
}

// ---------------------------------------------------------------------------
// RaBitQ query quantization (fastscan.cuh:151-247) and bit planes (:292-329).
// scratch: pdim floats of the wave's LDS; planes: 6*wpp words of LDS.
// ---------------------------------------------------------------------------
struct QuantOut {
    float low, width;
    int32_t sum_q;
};

__device__ __forceinline__ uint32_t dither_hash(uint32_t a, uint32_t b) {
    a ^= b;
    a ^= a >> 16;
    a *= 0x45d9f3bu;
    a ^= a >> 16;
    a *= 0x45d9f3bu;
    a ^= a >> 16;
    return a;
}

__device__ __forceinline__ QuantOut quantize(const float* qv, const float* signs, uint32_t dim,
                                             uint32_t pdim, uint32_t seed, float* scratch,
                                             uint32_t* planes, uint8_t* codes_out) {
    const uint32_t lane = lane_id();
    for (uint32_t i = lane; i < pdim; i += 64) scratch[i] = (i < dim) ? __fmul_rn(qv[i], signs[i]) : 0.0f;
    wave_sync();
    uint32_t lshift = 0;
    for (uint32_t len = 1; len < pdim; len <<= 1, ++lshift) {
        for (uint32_t pi = lane; pi < (pdim >> 1); pi += 64) {
            const uint32_t blk = pi >> lshift, j = pi & (len - 1);
            const uint32_t i1 = (blk << (lshift + 1)) + j, i2 = i1 + len;
            const float u = scratch[i1], v = scratch[i2];
            scratch[i1] = __fadd_rn(u, v);
            scratch[i2] = __fsub_rn(u, v);
        }
        wave_sync();
    }
    float mn = FLT_MAX, mx = -FLT_MAX;
    for (uint32_t i = lane; i < pdim; i += 64) {
        const float v = scratch[i];
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    }
    mn = bsw::wave_min(mn);
    mx = bsw::wave_max(mx);
    const float low = __uint_as_float(uniform(__float_as_uint(mn)));
    const float high = __uint_as_float(uniform(__float_as_uint(mx)));
    const float width = __fdiv_rn(__fsub_rn(high, low), 63.0f);
    const float inv_w = __fdiv_rn(1.0f, width);
    uint32_t lsum = 0;
    // codes are written back into scratch as words (one code per word) and into planes
    for (uint32_t i0 = 0; i0 < pdim; i0 += 64) {
        const uint32_t i = i0 + lane;
        uint32_t c = 0;
        if (i < pdim) {
            const float x = __fmul_rn(__fsub_rn(scratch[i], low), inv_w);
            const float u = static_cast<float>(dither_hash(seed, i) & 0xFFFFFFu) * (1.0f / 16777216.0f);
            int qi = static_cast<int>(floorf(__fadd_rn(x, u)));
            qi = qi < 0 ? 0 : (qi > 63 ? 63 : qi);
            c = static_cast<uint32_t>(qi);
            lsum += c;
            if (codes_out) codes_out[i] = static_cast<uint8_t>(c);
        }
#pragma unroll
        for (int b = 0; b < 6; ++b) {
            const uint64_t m = ballot(((c >> b) & 1u) != 0u);
            const uint32_t w0 = i0 >> 5;
            if (lane == 0) planes[b * (pdim >> 5) + w0] = static_cast<uint32_t>(m);
            if (lane == 0 && i0 + 32 < pdim) planes[b * (pdim >> 5) + w0 + 1] = static_cast<uint32_t>(m >> 32);
        }
    }
    wave_sync();
    const uint32_t s = bsw::group_sum_u32(lsum, 64);
    QuantOut o;
    o.low = low;
    o.width = width;
    o.sum_q = static_cast<int32_t>(uniform(s));
    return o;
}

// est = tx + exact + fdq * width * ip + fvq * low, ip = 2 raw - sum_q; FLT_MAX when
// tx == FLT_MAX or not finite (fastscan.cuh:361-366).  Evaluated in exactly that order
// with no contraction.
__device__ __forceinline__ float estimate(uint32_t raw, int32_t sum_q, float width, float low, float tx,
                                          float fdq, float fvq, float exact) {
    const float ip = static_cast<float>(static_cast<int32_t>(raw << 1) - sum_q);
    const float a = __fadd_rn(tx, exact);
    const float b = __fmul_rn(__fmul_rn(fdq, width), ip);
    const float c = __fmul_rn(fvq, low);
    float est = __fadd_rn(__fadd_rn(a, b), c);
    if (tx == FLT_MAX || !__builtin_isfinite(est)) est = FLT_MAX;
    return est;
}

// ---------------------------------------------------------------------------
// Fastscan sums in the quad layout.  In a node record the codes of one neighbour are
// cws = max(wpp, 4) words (words >= wpp are zero), so a lane reads four code words of
// one neighbour with one 16-byte load.  Lane l works on quad l % qpn (qpn = cws / 4) of
// neighbour pass * npp + l / qpn (npp = 64 / qpn).  With wpp <= 4 ("narrow", pdim <= 128)
// a lane holds a whole neighbour and every lane uses the same plane words; otherwise
// ("wide") the qpn partial sums of a neighbour are combined by an xor butterfly (exact
// integer adds).
// ---------------------------------------------------------------------------
struct QuadShape {
    uint32_t cws, qpn, qshift, npp, passes;
};

__host__ __device__ inline QuadShape quad_shape(uint32_t wpp, uint32_t R) {
    QuadShape S;
    S.cws = wpp < 4 ? 4u : wpp;
    S.qpn = S.cws / 4;
    S.qshift = 0;
    while ((1u << S.qshift) < S.qpn) ++S.qshift;
    S.npp = 64u / S.qpn;
    S.passes = (R + S.npp - 1) / S.npp;
    return S;
}

// the lane's plane words: pl[b] = words 4 * (lane % qpn) .. +3 of plane b (0 beyond wpp),
// from the planes quantize() left in LDS
__device__ __forceinline__ void lane_plane_quads(const uint32_t* planes, uint32_t wpp, const QuadShape& S,
                                                 uint4 (&pl)[6]) {
    const uint32_t qi = lane_id() & (S.qpn - 1);
#pragma unroll
    for (int b = 0; b < 6; ++b) {
        uint32_t w4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t w = 4u * qi + static_cast<uint32_t>(k);
            w4[k] = (w < wpp) ? planes[static_cast<uint32_t>(b) * wpp + w] : 0u;
        }
        pl[b] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
    wave_sync();
}

// Narrow layout: the 6 x 4 plane words every lane uses, padded to 4 words per plane
// (planes4[4b + k]), kept in LDS for the whole query and re-read per expansion.
__device__ __forceinline__ void store_planes4(const uint32_t* planes, uint32_t wpp, uint32_t* planes4) {
    const uint32_t lane = lane_id();
    if (lane < 24u) {
        const uint32_t b = lane >> 2, k = lane & 3u;
        planes4[lane] = (k < wpp) ? planes[b * wpp + k] : 0u;
    }
    wave_sync();
}

// the four code words of quad `qi` of neighbour nb (nb >= R reads neighbour 0: every
// load is issued unconditionally; the caller ignores the result)
__device__ __forceinline__ uint4 load_quad(const uint32_t* codes, uint32_t nb, uint32_t R, uint32_t qi,
                                           const QuadShape& S) {
    const uint32_t n = nb < R ? nb : 0u;
    return *reinterpret_cast<const uint4*>(codes + static_cast<uint64_t>(n) * S.cws + 4u * qi);
}

// Narrow codes (pdim <= 128, cws = 4 words per neighbour) with one candidate register
// (R <= 64): two lanes per neighbour, so the popcounts of a 32-neighbour row run on every
// lane.  Lane l takes words 2 (l / 32) and 2 (l / 32) + 1 of neighbour l % 32 (and of
// neighbour 32 + l % 32 when R > 32) in one 8-byte load; the two halves of a neighbour's
// raw sum meet across lanes l and l + 32.  Loads are issued unconditionally (neighbours
// >= R read neighbour 0; the caller ignores those lanes).
struct CodeHalves {
    uint2 a, b;
};

__device__ __forceinline__ CodeHalves load_code_halves(const uint32_t* codes, uint32_t R, const QuadShape& S) {
    const uint32_t lane = lane_id();
    const uint32_t nb = lane & 31u, w = 2u * (lane >> 5);
    // byte offsets from the record's codes, a wave-uniform base (bsw::load_off)
    CodeHalves h;
    h.a = bsw::load_off<uint2>(codes, 4u * ((nb < R ? nb : 0u) * S.cws + w));
    h.b = make_uint2(0u, 0u);
    if (R > 32u) h.b = bsw::load_off<uint2>(codes, 4u * ((nb + 32u < R ? nb + 32u : 0u) * S.cws + w));
    return h;
}

// raw sum of neighbour `lane` from the halves and the 24 shared plane words (planes4, LDS)
__device__ __forceinline__ uint32_t raw_halves(const uint32_t* planes4, const CodeHalves& h, uint32_t R) {
    const uint32_t lane = lane_id();
    const uint32_t* pw = planes4 + 2u * (lane >> 5);
    uint2 w[6];
#pragma unroll
    for (int b = 0; b < 6; ++b) w[b] = *reinterpret_cast<const uint2*>(pw + 4 * b);
    auto half_sum = [&](uint2 c) __attribute__((always_inline)) {
        uint32_t r = 0;
#pragma unroll
        for (int b = 0; b < 6; ++b) {
            uint32_t n = static_cast<uint32_t>(__builtin_popcount(w[b].x & c.x));
            n += static_cast<uint32_t>(__builtin_popcount(w[b].y & c.y));
            r += n << b;
        }
        return r;
    };
    // v_permlane32_swap(a, b) leaves (a's lower half, b's lower half) in result 0 and (a's
    // upper half, b's upper half) in result 1: their sum holds neighbour l's two halves in
    // lane l < 32 and neighbour 32 + (l - 32)'s in lane l >= 32
    const uint32_t ra = half_sum(h.a);
    const uint32_t rb = R > 32u ? half_sum(h.b) : ra;
    const auto r = __builtin_amdgcn_permlane32_swap(ra, rb, false, false);
    return r[0] + r[1];
}

// raw = sum_b 2^b * popcount(plane_b & code) over the four words of a quad
__device__ __forceinline__ uint32_t raw_quad(const uint4 (&pl)[6], uint4 c) {
    uint32_t r = 0;
#pragma unroll
    for (int b = 0; b < 6; ++b) {
        uint32_t n = static_cast<uint32_t>(__builtin_popcount(pl[b].x & c.x));
        n += static_cast<uint32_t>(__builtin_popcount(pl[b].y & c.y));
        n += static_cast<uint32_t>(__builtin_popcount(pl[b].z & c.z));
        n += static_cast<uint32_t>(__builtin_popcount(pl[b].w & c.w));
        r += n << b;
    }
    return r;
}

// Wide layout: raw sums of neighbours [0, R) into rawbuf (LDS).  c0 holds the lane's
// quads of passes 0..3, issued by the caller together with its other loads; later
// passes are loaded here, four at a time.
__device__ __forceinline__ void raw_sums_wide(const uint4 (&pl)[6], const uint32_t* codes, uint32_t R,
                                              const QuadShape& S, const uint4 (&c0)[4], uint32_t* rawbuf) {
    const uint32_t lane = lane_id();
    const uint32_t qi = lane & (S.qpn - 1), nl = lane >> S.qshift;
    uint4 c[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) c[t] = c0[t];
    for (uint32_t t0 = 0; t0 < S.passes; t0 += 4) {
        if (t0 > 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) c[t] = load_quad(codes, (t0 + static_cast<uint32_t>(t)) * S.npp + nl, R, qi, S);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t nb = (t0 + static_cast<uint32_t>(t)) * S.npp + nl;
            const uint32_t s = bsw::group_sum_u32(raw_quad(pl, c[t]), S.qpn);
            if (qi == 0 && nb < R) rawbuf[nb] = s;
        }
    }
    wave_sync();
}

}  // namespace bsd
