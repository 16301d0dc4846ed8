// Batched incremental Vamana graph construction (host, OpenMP).
//
// Same algorithm, parameters, insertion order and tie rules as the reference builder
// (src/build_graph.cpp:260-392); see bs_build_vamana in include/bs_host.h.  The data
// structures are this build's own: a fixed-capacity sorted beam with a cursor on the
// first unexpanded entry, per-thread epoch-stamped visited arrays, distances computed
// four at a time (each one still a sequential float sum, so results are identical to
// the reference's one-at-a-time loop in exact mode).
#include "bs_host.h"
#include "host_common.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <random>
#include <utility>
#include <vector>

#include <immintrin.h>
#include <omp.h>

namespace {

using Edge = std::pair<float, uint32_t>;  // (distance to the row's node, neighbour)

struct Ctx {
    const float* v;
    uint32_t dim;
    bool exact;
    bool avx2;
    const float* row(uint32_t i) const { return v + static_cast<uint64_t>(i) * dim; }
};

// ---- distances -------------------------------------------------------------

// build_graph.cpp:95-102: sum += diff * diff, sequentially (exact mode).
inline float l2_seq(const float* a, const float* b, uint32_t dim) {
    float s = 0.0f;
    for (uint32_t i = 0; i < dim; ++i) {
        const float d = a[i] - b[i];
        s += d * d;
    }
    return s;
}

// four independent sequential sums, interleaved for instruction-level parallelism
inline void l2_seq4(const float* q, const float* r0, const float* r1, const float* r2,
                    const float* r3, uint32_t dim, float* out) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    for (uint32_t i = 0; i < dim; ++i) {
        const float a = q[i];
        const float d0 = r0[i] - a, d1 = r1[i] - a, d2 = r2[i] - a, d3 = r3[i] - a;
        s0 += d0 * d0;
        s1 += d1 * d1;
        s2 += d2 * d2;
        s3 += d3 * d3;
    }
    out[0] = s0;
    out[1] = s1;
    out[2] = s2;
    out[3] = s3;
}

__attribute__((target("avx2,fma"))) float l2_avx2(const float* a, const float* b, uint32_t dim) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    uint32_t i = 0;
    for (; i + 16 <= dim; i += 16) {
        __m256 d0 = _mm256_sub_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i));
        __m256 d1 = _mm256_sub_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8));
        acc0 = _mm256_fmadd_ps(d0, d0, acc0);
        acc1 = _mm256_fmadd_ps(d1, d1, acc1);
    }
    for (; i + 8 <= dim; i += 8) {
        __m256 d0 = _mm256_sub_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i));
        acc0 = _mm256_fmadd_ps(d0, d0, acc0);
    }
    acc0 = _mm256_add_ps(acc0, acc1);
    __m128 lo = _mm256_castps256_ps128(acc0), hi = _mm256_extractf128_ps(acc0, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
    float r = _mm_cvtss_f32(s);
    for (; i < dim; ++i) {
        const float d = a[i] - b[i];
        r += d * d;
    }
    return r;
}

inline float dist(const Ctx& c, uint32_t x, uint32_t y) {
    return (!c.exact && c.avx2) ? l2_avx2(c.row(x), c.row(y), c.dim) : l2_seq(c.row(x), c.row(y), c.dim);
}

// distances from node q to nodes ids[0..m)
inline void dist_many(const Ctx& c, uint32_t q, const uint32_t* ids, size_t m, float* out) {
    const float* qr = c.row(q);
    size_t i = 0;
    if (c.exact || !c.avx2) {
        for (; i + 4 <= m; i += 4)
            l2_seq4(qr, c.row(ids[i]), c.row(ids[i + 1]), c.row(ids[i + 2]), c.row(ids[i + 3]), c.dim, out + i);
        for (; i < m; ++i) out[i] = l2_seq(c.row(ids[i]), qr, c.dim);
    } else {
        for (; i < m; ++i) out[i] = l2_avx2(c.row(ids[i]), qr, c.dim);
    }
}

// ---- beam (build_graph.cpp:45-89 BeamQueue semantics) -------------------------

struct Item {
    float d;
    uint32_t node;
    bool expanded;
};

inline bool item_less(float da, uint32_t na, float db, uint32_t nb) {
    return da != db ? da < db : na < nb;
}

struct Beam {
    std::vector<Item> it;
    size_t cap = 0, sz = 0, first = 0;  // first = index of the first unexpanded item
    void reset(size_t c) {
        cap = c;
        it.resize(c + 1);
        sz = 0;
        first = 0;
    }
    // push of a node not present (the visited set guarantees it): sorted insert by
    // (dist, node), then truncate to capacity.
    void push(uint32_t node, float d) {
        size_t lo = 0, hi = sz;
        while (lo < hi) {
            size_t mid = (lo + hi) / 2;
            if (item_less(it[mid].d, it[mid].node, d, node)) lo = mid + 1;
            else hi = mid;
        }
        std::memmove(&it[lo + 1], &it[lo], (sz - lo) * sizeof(Item));
        it[lo] = {d, node, false};
        ++sz;
        if (lo <= first) first = lo;
        if (sz > cap) sz = cap;
        if (first > sz) first = sz;
    }
    bool has_unexpanded() const { return first < sz; }
    float tail() const { return it[sz - 1].d; }
    void advance() {
        while (first < sz && it[first].expanded) ++first;
    }
};

// ---- dedupe_and_prune (build_graph.cpp:156-208) -------------------------------

void dedupe_and_prune(const Ctx& c, std::vector<Edge>& nb, uint32_t src, uint32_t degree,
                      float alpha, std::vector<Edge>& uniq, std::vector<float>& dtmp,
                      std::vector<uint32_t>& itmp) {
    if (nb.empty()) return;
    std::sort(nb.begin(), nb.end(), [](const Edge& a, const Edge& b) {
        return a.first != b.first ? a.first < b.first : a.second < b.second;
    });
    uniq.clear();
    uint32_t last = 0xFFFFFFFFu;
    for (const Edge& e : nb) {
        if (e.second == src) continue;
        if (e.second == last) continue;
        uniq.push_back(e);
        last = e.second;
    }
    if (uniq.size() <= degree) {
        nb.swap(uniq);
        return;
    }
    std::vector<Edge> pruned;
    pruned.reserve(degree);
    const float alphas[2] = {1.0f, alpha};
    for (int pass = 0; pass < 2; ++pass) {
        const float a = alphas[pass];
        for (const Edge& e : uniq) {
            if (pruned.size() == degree) break;
            // distances from e.second to every kept node, then the first dominating one
            itmp.resize(pruned.size());
            for (size_t k = 0; k < pruned.size(); ++k) itmp[k] = pruned[k].second;
            dtmp.resize(pruned.size());
            bool dominated = false;
            size_t k0 = 0;
            while (k0 < pruned.size() && !dominated) {
                size_t m = std::min<size_t>(8, pruned.size() - k0);
                dist_many(c, e.second, itmp.data() + k0, m, dtmp.data() + k0);
                for (size_t k = k0; k < k0 + m; ++k)
                    if (a * dtmp[k] <= e.first) {
                        dominated = true;
                        break;
                    }
                k0 += m;
            }
            if (!dominated) pruned.push_back(e);
        }
    }
    nb.swap(pruned);
}

}  // namespace

extern "C" int bs_build_vamana(const float* vecs, uint64_t n, uint32_t dim, uint32_t degree,
                               uint32_t beam_width, float alpha, uint32_t seed, int exact,
                               int threads, uint32_t* edges_out, int verbose) try {
    if (n == 0) return bsh::fail(BS_HOST_EINVAL, "base dataset is empty");
    if (degree == 0 || beam_width == 0) return bsh::fail(BS_HOST_EINVAL, "degree and beam width must be positive");
    if (!(alpha >= 1.0f)) return bsh::fail(BS_HOST_EINVAL, "alpha must be at least 1.0");
    if (n > 0x7FFFFFFFull) return bsh::fail(BS_HOST_EINVAL, "at most 2^31-1 points");
    const int T = bsh::n_threads(threads);
    Ctx c{vecs, dim, exact != 0, __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")};
    const auto t0 = std::chrono::steady_clock::now();

    std::vector<uint32_t> order(n);
    std::iota(order.begin(), order.end(), 0u);
    std::mt19937 gen(seed);
    std::shuffle(order.begin(), order.end(), gen);

    std::vector<std::vector<Edge>> graph(n);
    const uint64_t batch_bound = std::max<uint64_t>(1, static_cast<uint64_t>(0.02 * static_cast<double>(n)));

    // per-thread scratch
    struct Scratch {
        std::vector<uint32_t> stamp;
        uint32_t epoch = 0;
        Beam beam;
        std::vector<uint32_t> frontier;
        std::vector<float> fd;
        std::vector<Edge> uniq;
        std::vector<float> dtmp;
        std::vector<uint32_t> itmp;
    };
    std::vector<Scratch> scr(T);
    for (auto& s : scr) s.stamp.assign(n, 0);

    uint64_t start = 1;
    double last_print = 0.0;
    while (start < n) {
        const uint64_t end = std::min(std::min(start * 2, start + batch_bound), n);
#pragma omp parallel for schedule(dynamic, 1) num_threads(T)
        for (int64_t ii = static_cast<int64_t>(start); ii < static_cast<int64_t>(end); ++ii) {
            Scratch& s = scr[omp_get_thread_num()];
            if (++s.epoch == 0) {
                std::fill(s.stamp.begin(), s.stamp.end(), 0u);
                s.epoch = 1;
            }
            const uint32_t target = order[static_cast<uint64_t>(ii)];
            Beam& beam = s.beam;
            beam.reset(beam_width);
            beam.push(order[0], dist(c, order[0], target));
            s.stamp[order[0]] = s.epoch;
            std::vector<Edge>& out = graph[target];
            while (beam.has_unexpanded()) {
                Item& item = beam.it[beam.first];
                const Item cur = item;
                out.emplace_back(cur.d, cur.node);
                item.expanded = true;
                beam.advance();
                s.frontier.clear();
                for (const Edge& nbe : graph[cur.node]) {
                    if (s.stamp[nbe.second] != s.epoch) {
                        s.stamp[nbe.second] = s.epoch;
                        s.frontier.push_back(nbe.second);
                    }
                }
                s.fd.resize(s.frontier.size());
                dist_many(c, target, s.frontier.data(), s.frontier.size(), s.fd.data());
                for (size_t f = 0; f < s.frontier.size(); ++f) {
                    if (beam.sz < beam.cap || s.fd[f] < beam.tail()) beam.push(s.frontier[f], s.fd[f]);
                }
            }
            dedupe_and_prune(c, out, target, degree, alpha, s.uniq, s.dtmp, s.itmp);
        }
        for (uint64_t i = start; i < end; ++i) {
            const uint32_t src = order[i];
            for (const Edge& e : graph[src]) graph[e.second].emplace_back(e.first, src);
        }
#pragma omp parallel for schedule(dynamic, 256) num_threads(T)
        for (int64_t u = 0; u < static_cast<int64_t>(n); ++u) {
            if (graph[u].size() > degree) {
                Scratch& s = scr[omp_get_thread_num()];
                dedupe_and_prune(c, graph[u], static_cast<uint32_t>(u), degree, alpha, s.uniq, s.dtmp, s.itmp);
            }
        }
        if (verbose) {
            const double el = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            if (end == n || el - last_print >= 5.0) {
                std::fprintf(stderr, "  build_graph: %llu / %llu points inserted, %.1fs\n",
                             static_cast<unsigned long long>(end), static_cast<unsigned long long>(n), el);
                last_print = el;
            }
        }
        start = end;
    }
#pragma omp parallel for schedule(dynamic, 256) num_threads(T)
    for (int64_t u = 0; u < static_cast<int64_t>(n); ++u) {
        Scratch& s = scr[omp_get_thread_num()];
        dedupe_and_prune(c, graph[u], static_cast<uint32_t>(u), degree, alpha, s.uniq, s.dtmp, s.itmp);
        const size_t lim = std::min<size_t>(graph[u].size(), degree);
        uint32_t* row = edges_out + static_cast<uint64_t>(u) * degree;
        for (size_t j = 0; j < degree; ++j) row[j] = j < lim ? graph[u][j].second : 0u;
    }
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}
