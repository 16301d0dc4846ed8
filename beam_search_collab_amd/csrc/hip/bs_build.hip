// Vamana graph construction on the device: the batched incremental builder of
// build_graph (src/build_graph.cpp:95-392), node for node and edge for edge.
//
// The reference inserts the points of a random order in batches (1, 2, 4, ... up to 2% of
// n per batch).  Every point of a batch searches the graph as it stood before the batch,
// keeps the nodes it expanded, and dedupes / prunes them to its out-list; then the
// batch's edges are mirrored into their targets' lists in batch order, and every list
// longer than the degree is pruned again.  All of it is deterministic, so the device runs
// the same steps in parallel where the reference does:
//   vb_search      a wavefront per point of the batch: the greedy beam search (beam of
//                  beam_width (dist, node) keys in registers, a per-search visited bitmap
//                  in HBM, every candidate pushed in list order under the reference's
//                  rule "size < width or dist < tail"), the expanded nodes appended to
//                  the point's visit list;
//   (sort)         the visit lists by (dist, node) (segmented radix sort);
//   vb_prune       a wavefront per list: dedupe_and_prune (build_graph.cpp:156-208) --
//                  skip the node itself and repeated ids, then two passes (alpha 1, then
//                  alpha) keeping a candidate unless alpha * d(candidate, kept) <= its
//                  distance for a kept node;
//   vb_rev_*       the mirrored edges as 64-bit keys (target << 32 | batch position),
//                  radix-sorted, so each target's new entries arrive in the reference's
//                  append order; lists that stay within the degree get them appended,
//                  the others are gathered, sorted and pruned;
//   vb_final       a wavefront per node: the final dedupe (sort by (dist, node)) and the
//                  edge row, padded with node 0 as the reference pads.
// Distances are the reference's sequential float sums (build_graph.cpp:95-102), one lane
// per pair, so every comparison sees the reference's values.
#include "bs_hip.h"
#include "bs_device.hpp"

#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <numeric>
#include <random>
#include <string>
#include <vector>

void bs_internal_set_error(const std::string& msg);
int bs_internal_exception();

namespace bvb {

using namespace bsw;
using bsd::EMPTY_KEY;
using bsd::INVALID;

// list entries are (dist, node) keys: orderable(dist) << 32 | node
__device__ __forceinline__ uint64_t lkey(float d, uint32_t id) {
    return (static_cast<uint64_t>(bsd::orderable(d)) << 32) | id;
}
__device__ __forceinline__ float lkey_dist(uint64_t k) { return bsd::key_dist(k); }

// build_graph.cpp:95-102: sum += diff * diff in dimension order (rows are 16-B aligned)
__device__ __forceinline__ float l2_seq(const float* a, const float* b, uint32_t dim) {
    float s = 0.0f;
    uint32_t i = 0;
    for (; i + 4 <= dim; i += 4) {
        const float4 x = *reinterpret_cast<const float4*>(a + i);
        const float4 y = *reinterpret_cast<const float4*>(b + i);
        float d = x.x - y.x;
        s = s + d * d;
        d = x.y - y.y;
        s = s + d * d;
        d = x.z - y.z;
        s = s + d * d;
        d = x.w - y.w;
        s = s + d * d;
    }
    for (; i < dim; ++i) {
        const float d = a[i] - b[i];
        s = s + d * d;
    }
    return s;
}

struct Graph {
    const float* vecs;  // n * dstride
    uint32_t dstride, dim, deg;
    uint64_t n;
    uint32_t* lid;      // n * deg
    float* ldist;       // n * deg
    uint32_t* lcnt;     // n
};

// key of element e of the register-major beam (e uniform)
template <int TR>
__device__ __forceinline__ uint64_t beam_at(const uint64_t (&beam)[TR], uint32_t e) {
    const uint32_t r = e >> 6;
    uint64_t row = beam[0];
#pragma unroll
    for (int k = 1; k < TR; ++k) row = (r == static_cast<uint32_t>(k)) ? beam[k] : row;
    return readlane64(row, e & 63u);
}

// push of one candidate key (LSB 0 = unexpanded) into the sorted beam of sz <= cap keys:
// sorted insert, then truncation to cap (build_graph.cpp:45-89 BeamQueue::push)
template <int TR>
__device__ __forceinline__ void beam_insert(uint64_t (&beam)[TR], uint32_t& sz, uint32_t cap, uint64_t ck) {
    const uint32_t lane = lane_id();
    uint32_t pos = 0;
#pragma unroll
    for (int r = 0; r < TR; ++r) pos += static_cast<uint32_t>(__builtin_popcountll(ballot(beam[r] < ck)));
    uint64_t carry[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) carry[r] = r == 0 ? EMPTY_KEY : readlane64(beam[r - 1], 63);
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint32_t e = static_cast<uint32_t>(r) * 64u + lane;
        const uint32_t plo = prev_lane(static_cast<uint32_t>(beam[r]));
        const uint32_t phi = prev_lane(static_cast<uint32_t>(beam[r] >> 32));
        uint64_t prv = (static_cast<uint64_t>(phi) << 32) | plo;
        if (lane == 0) prv = carry[r];
        uint64_t v = e < pos ? beam[r] : (e == pos ? ck : prv);
        beam[r] = e < cap ? v : EMPTY_KEY;
    }
    sz = sz + 1 < cap ? sz + 1 : cap;
}

// The greedy search of one point (build_graph.cpp:284-312), a wavefront per point.
// out: the expanded nodes as list keys in expansion order (at most outcap; *overflow set
// beyond); vis: this search's visited bitmap (cleared by the host before the batch).
template <int TR>
__global__ void __launch_bounds__(256) vb_search(const Graph G, const uint32_t* order, uint64_t start, uint64_t count,
                                                 uint32_t L, uint64_t* outk, uint32_t* outn, uint32_t outcap,
                                                 uint32_t* vis, uint64_t vis_words, uint32_t* overflow) {
    const uint32_t lane = lane_id();
    const uint64_t j = static_cast<uint64_t>(blockIdx.x) * 4 + uniform(threadIdx.x >> 6);
    if (j >= count) return;
    const uint32_t target = order[start + j];
    const uint32_t ep = order[0];
    const float* trow = G.vecs + static_cast<uint64_t>(target) * G.dstride;
    uint32_t* vb = vis + j * vis_words;
    uint64_t* out = outk + j * outcap;
    uint64_t beam[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) beam[r] = EMPTY_KEY;
    uint32_t sz = 0;
    {
        const float d0 = l2_seq(G.vecs + static_cast<uint64_t>(ep) * G.dstride, trow, G.dim);
        beam_insert<TR>(beam, sz, L, bsd::make_key(d0, ep));
        if (lane == 0) vb[ep >> 5] |= 1u << (ep & 31u);
    }
    uint32_t nout = 0;
    for (;;) {
        // the first unexpanded entry: its key, then its mark
        uint32_t pr = TR;
        uint64_t mp = 0;
#pragma unroll
        for (int r = TR - 1; r >= 0; --r) {
            const uint64_t m = ballot((static_cast<uint32_t>(beam[r]) & 1u) == 0u && beam[r] != EMPTY_KEY);
            pr = m != 0 ? static_cast<uint32_t>(r) : pr;
            mp = m != 0 ? m : mp;
        }
        if (pr == static_cast<uint32_t>(TR)) break;
        const uint32_t pl = static_cast<uint32_t>(__builtin_ctzll(mp));
        const uint64_t kp = beam_at<TR>(beam, pr * 64u + pl);
#pragma unroll
        for (int r = 0; r < TR; ++r)
            if (pr == static_cast<uint32_t>(r)) beam[r] |= (lane == pl) ? 1ull : 0ull;
        const uint32_t cur = bsd::key_id(kp);
        if (nout == outcap) {
            if (lane == 0) atomicOr(overflow, 1u);
            break;
        }
        if (lane == 0) out[nout] = lkey(bsd::key_dist(kp), cur);
        ++nout;
        // neighbours in list order; a neighbour not visited before joins the frontier
        const uint32_t cnt = G.lcnt[cur];
        for (uint32_t k0 = 0; k0 < cnt; k0 += 64) {
            const uint32_t k = k0 + lane;
            uint32_t nb = INVALID;
            bool fresh = false;
            if (k < cnt) {
                nb = G.lid[static_cast<uint64_t>(cur) * G.deg + k];
                const uint32_t bit = 1u << (nb & 31u);
                fresh = (atomicOr(&vb[nb >> 5], bit) & bit) == 0u;
            }
            float d = 0.0f;
            if (fresh) d = l2_seq(G.vecs + static_cast<uint64_t>(nb) * G.dstride, trow, G.dim);
            const uint64_t ck = fresh ? bsd::make_key(d, nb) : EMPTY_KEY;
            uint64_t m = ballot(fresh);
            if (sz == L && m) {
                // a full beam's last entry only moves closer, so a candidate at or beyond it
                // now is refused at its turn as well: only the others go through the pushes
                const float dl = bsd::key_dist(beam_at<TR>(beam, L - 1));
                m &= ballot(fresh && d < dl);
            }
            while (m) {
                const uint32_t l = static_cast<uint32_t>(__builtin_ctzll(m));
                m &= m - 1;
                const uint64_t c = readlane64(ck, l);
                // push if the beam has room or the distance is below the last entry's
                bool take = sz < L;
                if (!take) take = bsd::key_dist(c) < bsd::key_dist(beam_at<TR>(beam, sz - 1));
                if (take) beam_insert<TR>(beam, sz, L, c);
            }
        }
    }
    if (lane == 0) outn[j] = nout;
}

// dedupe_and_prune (build_graph.cpp:156-208) of one sorted list of list keys, a
// wavefront per list; the result becomes node src's list.  keys are rewritten in place
// (the deduplicated prefix).  kept: LDS, deg entries per wavefront.
__device__ void prune_list(const Graph& G, uint64_t* keys, uint32_t n, uint32_t src, float alpha, uint64_t* kept) {
    const uint32_t lane = lane_id();
    // dedupe: skip src and an id equal to the last kept one (in place, order kept)
    uint32_t nu = 0, last = INVALID;
    for (uint32_t i0 = 0; i0 < n; i0 += 64) {
        const uint32_t i = i0 + lane;
        const uint64_t k = i < n ? keys[i] : EMPTY_KEY;
        const uint32_t id = static_cast<uint32_t>(k);
        const bool valid = i < n && id != src;
        const uint64_t vm = ballot(valid);
        // id of the closest valid element before this lane (or the carried last)
        const uint64_t below = vm & ((1ull << lane) - 1ull);
        const uint32_t src_lane = below ? 63u - static_cast<uint32_t>(__builtin_clzll(below)) : lane;
        const uint32_t pid = static_cast<uint32_t>(
            __builtin_amdgcn_ds_bpermute(static_cast<int>(src_lane << 2), static_cast<int>(id)));
        const uint32_t prev = below ? pid : last;
        const bool keep = valid && id != prev;
        const uint64_t km = ballot(keep);
        wave_sync();
        if (keep) keys[nu + lanes_below(km)] = k;
        nu += static_cast<uint32_t>(__builtin_popcountll(km));
        if (vm) last = readlane(id, 63u - static_cast<uint32_t>(__builtin_clzll(vm)));
        wave_sync();
    }
    __threadfence_block();
    uint32_t* lid = G.lid + static_cast<uint64_t>(src) * G.deg;
    float* ld = G.ldist + static_cast<uint64_t>(src) * G.deg;
    if (nu <= G.deg) {
        for (uint32_t i = lane; i < nu; i += 64) {
            const uint64_t k = keys[i];
            lid[i] = static_cast<uint32_t>(k);
            ld[i] = lkey_dist(k);
        }
        if (lane == 0) G.lcnt[src] = nu;
        return;
    }
    uint32_t kc = 0;
    const float alphas[2] = {1.0f, alpha};
    const uint32_t h = lane >> 5, l = lane & 31u;
    for (int pass = 0; pass < 2; ++pass) {
        const float a = alphas[pass];
        uint32_t i = 0;
        while (i < nu && kc < G.deg) {
            if (kc <= 32) {
                // Two candidates per step: lanes 0-31 test e_i and lanes 32-63 test e_(i+1)
                // against the kept set (one kept node per lane), so all lanes are busy.  When
                // e_i is kept, e_(i+1) is also tested against e_i before it can be kept, so
                // every decision is the one-at-a-time loop's, on the same distances.
                const bool two = i + 1 < nu;
                const uint64_t e = keys[two ? i + h : i];
                bool hit = false;
                if (l < kc && (h == 0 || two)) {
                    const float* erow = G.vecs + static_cast<uint64_t>(static_cast<uint32_t>(e)) * G.dstride;
                    const uint32_t kid = static_cast<uint32_t>(kept[l]);
                    hit = a * l2_seq(erow, G.vecs + static_cast<uint64_t>(kid) * G.dstride, G.dim) <= lkey_dist(e);
                }
                const uint64_t bm = ballot(hit);
                const uint64_t e0 = readlane64(e, 0), e1 = readlane64(e, 32);
                bool dom1 = (bm >> 32) != 0ull;
                if ((bm & 0xFFFFFFFFull) == 0ull) {
                    if (lane == 0) kept[kc] = e0;
                    ++kc;
                    wave_sync();
                    if (two && kc < G.deg && !dom1) {
                        const float d = l2_seq(G.vecs + static_cast<uint64_t>(static_cast<uint32_t>(e1)) * G.dstride,
                                               G.vecs + static_cast<uint64_t>(static_cast<uint32_t>(e0)) * G.dstride, G.dim);
                        dom1 = a * d <= lkey_dist(e1);
                    }
                }
                if (two && kc < G.deg && !dom1) {
                    if (lane == 0) kept[kc] = e1;
                    ++kc;
                    wave_sync();
                }
                i += two ? 2 : 1;
                continue;
            }
            // more than 32 kept: one candidate, a kept node per lane in chunks of 64
            const uint64_t e = keys[i];
            const uint32_t eid = static_cast<uint32_t>(e);
            const float ed = lkey_dist(e);
            const float* erow = G.vecs + static_cast<uint64_t>(eid) * G.dstride;
            bool dom = false;
            for (uint32_t k0 = 0; k0 < kc && !dom; k0 += 64) {
                bool hit = false;
                if (k0 + lane < kc) {
                    const uint32_t kid = static_cast<uint32_t>(kept[k0 + lane]);
                    const float dk = l2_seq(erow, G.vecs + static_cast<uint64_t>(kid) * G.dstride, G.dim);
                    hit = a * dk <= ed;
                }
                dom = ballot(hit) != 0;
            }
            if (!dom) {
                if (lane == 0) kept[kc] = e;
                ++kc;
                wave_sync();
            }
            ++i;
        }
    }
    for (uint32_t i = lane; i < kc; i += 64) {
        const uint64_t k = kept[i];
        lid[i] = static_cast<uint32_t>(k);
        ld[i] = lkey_dist(k);
    }
    if (lane == 0) G.lcnt[src] = kc;
}

// the batch's visit lists: job j = (sorted keys at j * outcap, outn[j] keys, order[start + j])
__global__ void __launch_bounds__(256) vb_prune_targets(const Graph G, uint64_t* keys, const uint32_t* outn,
                                                        uint32_t outcap, const uint32_t* order, uint64_t start,
                                                        uint64_t count, float alpha) {
    __shared__ uint64_t kept_s[4][128];
    const uint32_t w = uniform(threadIdx.x >> 6);
    const uint64_t j = static_cast<uint64_t>(blockIdx.x) * 4 + w;
    if (j >= count) return;
    prune_list(G, keys + j * outcap, outn[j], order[start + j], alpha, kept_s[w]);
}

// mirrored edges: record (j, k) of the batch -> key (target << 32 | j * deg + k), or ~0
__global__ void __launch_bounds__(256) vb_rev_keys(const Graph G, const uint32_t* order, uint64_t start,
                                                   uint64_t count, uint64_t* rk, unsigned long long* nvalid) {
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= count * G.deg) return;
    const uint64_t j = t / G.deg;
    const uint32_t k = static_cast<uint32_t>(t - j * G.deg);
    const uint32_t src = order[start + j];
    uint64_t key = ~0ull;
    if (k < G.lcnt[src]) {
        key = (static_cast<uint64_t>(G.lid[static_cast<uint64_t>(src) * G.deg + k]) << 32) | static_cast<uint32_t>(t);
        atomicAdd(nvalid, 1ull);
    }
    rk[t] = key;
}

// targets of the mirrored edges: every first record of a target registers (target,
// begin, end) -- end by binary search for the next target
__global__ void __launch_bounds__(256) vb_rev_heads(const uint64_t* rk, uint64_t m, uint4* heads,
                                                    unsigned int* nheads) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= m) return;
    const uint32_t dst = static_cast<uint32_t>(rk[i] >> 32);
    if (i > 0 && static_cast<uint32_t>(rk[i - 1] >> 32) == dst) return;
    uint64_t lo = i + 1, hi = m;  // first index with a larger target
    while (lo < hi) {
        const uint64_t mid = (lo + hi) / 2;
        if (static_cast<uint32_t>(rk[mid] >> 32) == dst) lo = mid + 1;
        else hi = mid;
    }
    const unsigned int h = atomicAdd(nheads, 1u);
    heads[h] = make_uint4(dst, static_cast<uint32_t>(i), static_cast<uint32_t>(lo), 0u);
}

// apply the mirrored edges of one target (a wavefront each): append when the list stays
// within the degree, else gather old + new list keys for the sort and prune
__global__ void __launch_bounds__(256) vb_rev_apply(const Graph G, const uint64_t* rk, const uint4* heads,
                                                    unsigned int nheads, const uint32_t* order, uint64_t start,
                                                    uint64_t* big, unsigned long long* bigtotal, uint4* bigjobs,
                                                    unsigned int* nbig) {
    const uint32_t lane = lane_id();
    const uint64_t h = static_cast<uint64_t>(blockIdx.x) * 4 + uniform(threadIdx.x >> 6);
    if (h >= nheads) return;
    const uint4 hd = heads[h];
    const uint32_t dst = hd.x, b = hd.y, app = hd.z - hd.y;
    const uint32_t old = G.lcnt[dst];
    uint32_t* lid = G.lid + static_cast<uint64_t>(dst) * G.deg;
    float* ld = G.ldist + static_cast<uint64_t>(dst) * G.deg;
    auto rec = [&](uint32_t k, uint32_t& src, float& d) __attribute__((always_inline)) {
        const uint32_t t = static_cast<uint32_t>(rk[b + k]);
        const uint32_t j = t / G.deg, kk = t - j * G.deg;
        src = order[start + j];
        d = G.ldist[static_cast<uint64_t>(src) * G.deg + kk];
    };
    if (old + app <= G.deg) {
        for (uint32_t k = lane; k < app; k += 64) {
            uint32_t src;
            float d;
            rec(k, src, d);
            lid[old + k] = src;
            ld[old + k] = d;
        }
        if (lane == 0) G.lcnt[dst] = old + app;
        return;
    }
    const uint32_t tot = old + app;
    unsigned long long off = 0;
    if (lane == 0) off = atomicAdd(bigtotal, static_cast<unsigned long long>(tot));
    off = readlane64(off, 0);
    for (uint32_t k = lane; k < tot; k += 64) {
        uint64_t key;
        if (k < old) {
            key = lkey(ld[k], lid[k]);
        } else {
            uint32_t src;
            float d;
            rec(k - old, src, d);
            key = lkey(d, src);
        }
        big[off + k] = key;
    }
    if (lane == 0) {
        const unsigned int q = atomicAdd(nbig, 1u);
        bigjobs[q] = make_uint4(dst, static_cast<uint32_t>(off), static_cast<uint32_t>(off >> 32), tot);
    }
}

__global__ void __launch_bounds__(256) vb_big_offsets(const uint4* bigjobs, unsigned int nbig, uint64_t* begin,
                                                      uint64_t* end) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= nbig) return;
    const uint4 jb = bigjobs[i];
    const uint64_t off = (static_cast<uint64_t>(jb.z) << 32) | jb.y;
    begin[i] = off;
    end[i] = off + jb.w;
}

__global__ void __launch_bounds__(256) vb_prune_big(const Graph G, uint64_t* keys, const uint4* bigjobs,
                                                    unsigned int nbig, float alpha) {
    __shared__ uint64_t kept_s[4][128];
    const uint32_t w = uniform(threadIdx.x >> 6);
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 4 + w;
    if (i >= nbig) return;
    const uint4 jb = bigjobs[i];
    const uint64_t off = (static_cast<uint64_t>(jb.z) << 32) | jb.y;
    prune_list(G, keys + off, jb.w, jb.x, alpha, kept_s[w]);
}

// the final dedupe_and_prune of every node (build_graph.cpp:382-390): its list (at most
// deg <= 128 entries) sorted by (dist, node), the node itself and repeats skipped, the row
// padded with node 0
template <int TR>
__global__ void __launch_bounds__(256) vb_final(const Graph G, uint32_t* edges_out) {
    const uint32_t lane = lane_id();
    const uint64_t u = static_cast<uint64_t>(blockIdx.x) * 4 + uniform(threadIdx.x >> 6);
    if (u >= G.n) return;
    const uint32_t cnt = G.lcnt[u];
    uint64_t v[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint32_t e = static_cast<uint32_t>(r) * 64u + lane;
        v[r] = e < cnt ? lkey(G.ldist[u * G.deg + e], G.lid[u * G.deg + e]) : EMPTY_KEY;
    }
    bsd::bitonic_sort<TR>(v);
    uint32_t nu = 0, last = INVALID;
    uint32_t* row = edges_out + u * G.deg;
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint32_t id = static_cast<uint32_t>(v[r]);
        const bool valid = v[r] != EMPTY_KEY && id != static_cast<uint32_t>(u);
        const uint64_t vm = ballot(valid);
        const uint64_t below = vm & ((1ull << lane) - 1ull);
        const uint32_t src_lane = below ? 63u - static_cast<uint32_t>(__builtin_clzll(below)) : lane;
        const uint32_t pid = static_cast<uint32_t>(
            __builtin_amdgcn_ds_bpermute(static_cast<int>(src_lane << 2), static_cast<int>(id)));
        const uint32_t prev = below ? pid : last;
        const bool keep = valid && id != prev;
        const uint64_t km = ballot(keep);
        const uint32_t p = nu + lanes_below(km);
        if (keep && p < G.deg) row[p] = id;
        nu += static_cast<uint32_t>(__builtin_popcountll(km));
        if (vm) last = readlane(id, 63u - static_cast<uint32_t>(__builtin_clzll(vm)));
    }
    for (uint32_t e = nu + lane; e < G.deg; e += 64) row[e] = 0u;
}

}  // namespace bvb

namespace {

int vfail(int code, const std::string& msg) {
    bs_internal_set_error(msg);
    return code;
}

template <typename F>
hipError_t launch_tr(uint32_t TR, F&& f) {
    switch (TR) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 8: f(std::integral_constant<int, 8>{}); break;
    default: f(std::integral_constant<int, 16>{}); break;
    }
    return hipGetLastError();
}

struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    template <typename T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

}  // namespace

extern "C" int bs_build_vamana_device(const float* vecs, uint64_t n, uint32_t dim, uint32_t degree,
                                      uint32_t beam_width, float alpha, uint32_t seed, uint32_t* edges_out,
                                      int verbose) try {
    if (!vecs || !edges_out) return vfail(BS_EINVAL, "vecs and edges_out must be given");
    if (n == 0) return vfail(BS_EINVAL, "base dataset is empty");
    if (n > 0x7FFFFFFFull) return vfail(BS_EINVAL, "at most 2^31-1 points");
    if (dim == 0 || dim > 4096) return vfail(BS_EINVAL, "dim must be in 1..4096");
    if (degree == 0 || degree > 128) return vfail(BS_EINVAL, "degree must be in 1..128");
    if (beam_width == 0 || beam_width > 1024) return vfail(BS_EINVAL, "beam width must be in 1..1024");
    if (!(alpha >= 1.0f)) return vfail(BS_EINVAL, "alpha must be at least 1.0");
    const auto t0 = std::chrono::steady_clock::now();
    const uint32_t dstride = (dim + 3) & ~3u;
    const uint32_t TR = beam_width <= 64 ? 1 : beam_width <= 128 ? 2 : beam_width <= 256 ? 4 : beam_width <= 512 ? 8 : 16;
    const uint32_t outcap = std::max<uint32_t>(1024u, 4u * beam_width);

    // insertion order (build_graph.cpp:268-272)
    std::vector<uint32_t> order(n);
    std::iota(order.begin(), order.end(), 0u);
    std::mt19937 gen(seed);
    std::shuffle(order.begin(), order.end(), gen);
    const uint64_t batch_bound = std::max<uint64_t>(1, static_cast<uint64_t>(0.02 * static_cast<double>(n)));
    const uint64_t max_batch = std::min<uint64_t>(batch_bound, n);
    // searches in flight: bounded by the visited bitmaps (at most 2 GiB)
    const uint64_t vis_words = (n + 31) / 32;
    const uint64_t slots = std::max<uint64_t>(1, std::min<uint64_t>(max_batch, (2ull << 30) / (vis_words * 4)));

    DevBuf d_vecs, d_lid, d_ld, d_lcnt, d_order, d_vis, d_outk, d_outs, d_outn, d_flag, d_rk, d_rks, d_heads, d_nh,
        d_nvalid, d_big, d_bigs, d_bigtot, d_bigjobs, d_nbig, d_beg, d_end, d_segb, d_sege, d_edges, d_tmp;
    auto alloc = [&](DevBuf& b, size_t bytes) { return hipMalloc(&b.p, std::max<size_t>(bytes, 8)) == hipSuccess; };
    const uint64_t mrec = max_batch * degree;
    const uint64_t bigcap = mrec * (static_cast<uint64_t>(degree) + 1);
    if (!alloc(d_vecs, n * dstride * 4ull) || !alloc(d_lid, n * degree * 4ull) || !alloc(d_ld, n * degree * 4ull) ||
        !alloc(d_lcnt, n * 4ull) || !alloc(d_order, n * 4ull) || !alloc(d_vis, slots * vis_words * 4ull) ||
        !alloc(d_outk, slots * outcap * 8ull) || !alloc(d_outs, slots * outcap * 8ull) || !alloc(d_outn, slots * 4ull) ||
        !alloc(d_flag, 4) || !alloc(d_rk, mrec * 8ull) || !alloc(d_rks, mrec * 8ull) || !alloc(d_heads, mrec * 16ull) ||
        !alloc(d_nh, 4) || !alloc(d_nvalid, 8) || !alloc(d_big, bigcap * 8ull) || !alloc(d_bigs, bigcap * 8ull) ||
        !alloc(d_bigtot, 8) || !alloc(d_bigjobs, mrec * 16ull) || !alloc(d_nbig, 4) || !alloc(d_beg, mrec * 8ull) ||
        !alloc(d_end, mrec * 8ull) || !alloc(d_segb, slots * 8ull) || !alloc(d_sege, slots * 8ull) ||
        !alloc(d_edges, n * degree * 4ull))
        return vfail(BS_ENOMEM, "hipMalloc of the graph-construction buffers failed");

    hipError_t e = hipSuccess;
    if (dstride == dim) {
        e = hipMemcpy(d_vecs.p, vecs, n * dim * 4ull, hipMemcpyHostToDevice);
    } else {
        e = hipMemset(d_vecs.p, 0, n * dstride * 4ull);
        if (e == hipSuccess)
            e = hipMemcpy2D(d_vecs.p, dstride * 4ull, vecs, dim * 4ull, dim * 4ull, n, hipMemcpyHostToDevice);
    }
    if (e == hipSuccess) e = hipMemcpy(d_order.p, order.data(), n * 4ull, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(d_lcnt.p, 0, n * 4ull);
    if (e == hipSuccess) e = hipMemset(d_flag.p, 0, 4);
    if (e != hipSuccess) return vfail(BS_EHIP, std::string("graph construction upload: ") + hipGetErrorString(e));

    bvb::Graph G{d_vecs.as<float>(), dstride, dim, degree, n, d_lid.as<uint32_t>(), d_ld.as<float>(),
                 d_lcnt.as<uint32_t>()};
    const uint32_t* ord = d_order.as<uint32_t>();

    if (slots * outcap > 0x7FFFFFFFull || bigcap > 0x7FFFFFFFull || mrec > 0xFFFFFFFFull)
        return vfail(BS_EINVAL, "batch too large for the device sorts (n or beam width too large)");
    // hipCUB work space, sized for the largest of the three sorts
    size_t tmp_bytes = 0;
    {
        size_t b1 = 0, b2 = 0, b3 = 0;
        e = hipcub::DeviceSegmentedRadixSort::SortKeys(nullptr, b1, d_outk.as<uint64_t>(), d_outs.as<uint64_t>(),
                                                   static_cast<int>(std::min<uint64_t>(slots * outcap, 0x7FFFFFFF)),
                                                   static_cast<int>(slots), d_segb.as<uint64_t>(),
                                                   d_sege.as<uint64_t>());
        if (e == hipSuccess)
            e = hipcub::DeviceRadixSort::SortKeys(nullptr, b2, d_rk.as<uint64_t>(), d_rks.as<uint64_t>(),
                                                  static_cast<int>(mrec));
        if (e == hipSuccess)
            e = hipcub::DeviceSegmentedRadixSort::SortKeys(nullptr, b3, d_big.as<uint64_t>(), d_bigs.as<uint64_t>(),
                                                   static_cast<int>(std::min<uint64_t>(bigcap, 0x7FFFFFFF)),
                                                   static_cast<int>(mrec), d_beg.as<uint64_t>(),
                                                   d_end.as<uint64_t>());
        if (e != hipSuccess) return vfail(BS_EHIP, std::string("sort sizing: ") + hipGetErrorString(e));
        tmp_bytes = std::max({b1, b2, b3});
        if (!alloc(d_tmp, tmp_bytes)) return vfail(BS_ENOMEM, "hipMalloc of the sort work space failed");
    }

    uint64_t start = 1;
    double last_print = 0.0;
    std::vector<uint64_t> segb(slots), sege(slots);
    std::vector<uint32_t> outn(slots);
    while (start < n) {
        const uint64_t end = std::min(std::min(start * 2, start + batch_bound), n);
        // 1. searches and visit-list prunes, `slots` points at a time
        for (uint64_t s0 = start; e == hipSuccess && s0 < end; s0 += slots) {
            const uint64_t cnt = std::min(slots, end - s0);
            e = hipMemsetAsync(d_vis.p, 0, cnt * vis_words * 4ull, nullptr);
            if (e != hipSuccess) break;
            const dim3 wg(static_cast<uint32_t>((cnt + 3) / 4));
            e = launch_tr(TR, [&](auto trc) {
                constexpr int T = decltype(trc)::value;
                hipLaunchKernelGGL(bvb::vb_search<T>, wg, dim3(256), 0, nullptr, G, ord, s0, cnt, beam_width,
                                   d_outk.as<uint64_t>(), d_outn.as<uint32_t>(), outcap, d_vis.as<uint32_t>(),
                                   vis_words, d_flag.as<uint32_t>());
            });
            if (e != hipSuccess) break;
            uint32_t flag = 0;
            e = hipMemcpy(outn.data(), d_outn.p, cnt * 4ull, hipMemcpyDeviceToHost);
            if (e == hipSuccess) e = hipMemcpy(&flag, d_flag.p, 4, hipMemcpyDeviceToHost);
            if (e != hipSuccess) break;
            if (flag) return vfail(BS_EINVAL, "a search expanded more than " + std::to_string(outcap) + " nodes");
            for (uint64_t j = 0; j < cnt; ++j) {
                segb[j] = j * outcap;
                sege[j] = j * outcap + outn[j];
            }
            e = hipMemcpy(d_segb.p, segb.data(), cnt * 8ull, hipMemcpyHostToDevice);
            if (e == hipSuccess) e = hipMemcpy(d_sege.p, sege.data(), cnt * 8ull, hipMemcpyHostToDevice);
            if (e == hipSuccess)
                e = hipcub::DeviceSegmentedRadixSort::SortKeys(d_tmp.p, tmp_bytes, d_outk.as<uint64_t>(),
                                                               d_outs.as<uint64_t>(), static_cast<int>(cnt * outcap),
                                                               static_cast<int>(cnt), d_segb.as<uint64_t>(),
                                                               d_sege.as<uint64_t>());
            if (e != hipSuccess) break;
            hipLaunchKernelGGL(bvb::vb_prune_targets, wg, dim3(256), 0, nullptr, G, d_outs.as<uint64_t>(),
                               d_outn.as<uint32_t>(), outcap, ord, s0, cnt, alpha);
            e = hipGetLastError();
        }
        if (e != hipSuccess) break;
        // 2. mirrored edges in batch order
        const uint64_t bcnt = end - start, m = bcnt * degree;
        e = hipMemsetAsync(d_nvalid.p, 0, 8, nullptr);
        if (e == hipSuccess) e = hipMemsetAsync(d_nh.p, 0, 4, nullptr);
        if (e == hipSuccess) e = hipMemsetAsync(d_nbig.p, 0, 4, nullptr);
        if (e == hipSuccess) e = hipMemsetAsync(d_bigtot.p, 0, 8, nullptr);
        if (e != hipSuccess) break;
        hipLaunchKernelGGL(bvb::vb_rev_keys, dim3(static_cast<uint32_t>((m + 255) / 256)), dim3(256), 0, nullptr, G,
                           ord, start, bcnt, d_rk.as<uint64_t>(), d_nvalid.as<unsigned long long>());
        e = hipGetLastError();
        if (e == hipSuccess)
            e = hipcub::DeviceRadixSort::SortKeys(d_tmp.p, tmp_bytes, d_rk.as<uint64_t>(), d_rks.as<uint64_t>(),
                                                  static_cast<int>(m));
        unsigned long long mv = 0;
        if (e == hipSuccess) e = hipMemcpy(&mv, d_nvalid.p, 8, hipMemcpyDeviceToHost);
        if (e != hipSuccess) break;
        if (mv) {
            hipLaunchKernelGGL(bvb::vb_rev_heads, dim3(static_cast<uint32_t>((mv + 255) / 256)), dim3(256), 0, nullptr,
                               d_rks.as<uint64_t>(), static_cast<uint64_t>(mv), d_heads.as<uint4>(),
                               d_nh.as<unsigned int>());
            unsigned int nh = 0, nbig = 0;
            e = hipGetLastError();
            if (e == hipSuccess) e = hipMemcpy(&nh, d_nh.p, 4, hipMemcpyDeviceToHost);
            if (e != hipSuccess) break;
            hipLaunchKernelGGL(bvb::vb_rev_apply, dim3((nh + 3) / 4), dim3(256), 0, nullptr, G, d_rks.as<uint64_t>(),
                               d_heads.as<uint4>(), nh, ord, start, d_big.as<uint64_t>(),
                               d_bigtot.as<unsigned long long>(), d_bigjobs.as<uint4>(), d_nbig.as<unsigned int>());
            e = hipGetLastError();
            if (e == hipSuccess) e = hipMemcpy(&nbig, d_nbig.p, 4, hipMemcpyDeviceToHost);
            if (e != hipSuccess) break;
            if (nbig) {
                unsigned long long tot = 0;
                e = hipMemcpy(&tot, d_bigtot.p, 8, hipMemcpyDeviceToHost);
                if (e != hipSuccess) break;
                hipLaunchKernelGGL(bvb::vb_big_offsets, dim3((nbig + 255) / 256), dim3(256), 0, nullptr,
                                   d_bigjobs.as<uint4>(), nbig, d_beg.as<uint64_t>(), d_end.as<uint64_t>());
                e = hipGetLastError();
                if (e == hipSuccess)
                    e = hipcub::DeviceSegmentedRadixSort::SortKeys(d_tmp.p, tmp_bytes, d_big.as<uint64_t>(),
                                                                   d_bigs.as<uint64_t>(), static_cast<int>(tot),
                                                                   static_cast<int>(nbig), d_beg.as<uint64_t>(),
                                                                   d_end.as<uint64_t>());
                if (e != hipSuccess) break;
                hipLaunchKernelGGL(bvb::vb_prune_big, dim3((nbig + 3) / 4), dim3(256), 0, nullptr, G,
                                   d_bigs.as<uint64_t>(), d_bigjobs.as<uint4>(), nbig, alpha);
                e = hipGetLastError();
                if (e != hipSuccess) break;
            }
        }
        if (verbose) {
            e = hipDeviceSynchronize();
            const double el = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            if (end == n || el - last_print >= 5.0) {
                std::fprintf(stderr, "  build_graph (device): %llu / %llu points inserted, %.1fs\n",
                             static_cast<unsigned long long>(end), static_cast<unsigned long long>(n), el);
                last_print = el;
            }
        }
        start = end;
    }
    if (e == hipSuccess) {
        e = launch_tr(degree <= 64 ? 1 : 2, [&](auto trc) {
            constexpr int T = decltype(trc)::value;
            hipLaunchKernelGGL(bvb::vb_final<T>, dim3(static_cast<uint32_t>((n + 3) / 4)), dim3(256), 0, nullptr, G,
                               d_edges.as<uint32_t>());
        });
    }
    if (e == hipSuccess) e = hipMemcpy(edges_out, d_edges.p, n * degree * 4ull, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return vfail(BS_EHIP, std::string("graph construction: ") + hipGetErrorString(e));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}
