// Host-side C-ABI: file formats, entry point, recall, synthetic inputs, ground truth.
// Declarations and reference citations: include/bs_host.h.
#include "bs_host.h"
#include "host_common.hpp"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <fstream>
#include <new>
#include <string>
#include <unordered_set>
#include <vector>

#include <omp.h>

namespace bsh {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int n_threads(int threads) { return threads > 0 ? threads : omp_get_max_threads(); }

int exception_code() {
    try {
        throw;
    } catch (const std::bad_alloc&) {
        return fail(BS_HOST_ENOMEM, "host memory allocation failed");
    } catch (const std::exception& e) {
        return fail(BS_HOST_EIO, std::string("internal error: ") + e.what());
    } catch (...) {
        return fail(BS_HOST_EIO, "internal error");
    }
}

}  // namespace bsh

using bsh::fail;

extern "C" const char* bs_host_last_error(void) { return bsh::g_err.c_str(); }
extern "C" void bs_host_free(void* p) { std::free(p); }

// ---------------------------------------------------------------------------
// formats
// ---------------------------------------------------------------------------

extern "C" int bs_read_vecs(const char* path, int is_int, void** data, uint64_t* n,
                            uint32_t* dim) try {
    std::ifstream in(path, std::ios::binary);
    if (!in) return fail(BS_HOST_EIO, std::string("cannot open ") + path);
    in.seekg(0, std::ios::end);
    const uint64_t size = static_cast<uint64_t>(in.tellg());
    in.seekg(0, std::ios::beg);
    if (size == 0) {
        *data = nullptr;
        *n = 0;
        *dim = 0;
        return BS_HOST_OK;
    }
    int32_t d = 0;
    in.read(reinterpret_cast<char*>(&d), 4);
    if (!in || d <= 0) return fail(BS_HOST_EIO, std::string("bad vecs header in ") + path);
    const uint64_t stride = 4ull + 4ull * static_cast<uint64_t>(d);
    if (size % stride != 0)
        return fail(BS_HOST_EIO, std::string("vecs file size is not a multiple of its row size: ") + path);
    const uint64_t rows = size / stride;
    char* buf = static_cast<char*>(std::malloc(rows * 4ull * d));
    if (!buf) return fail(BS_HOST_ENOMEM, "out of host memory");
    in.seekg(0, std::ios::beg);
    // read in blocks of rows
    const uint64_t block = std::max<uint64_t>(1, (64ull << 20) / stride);
    std::vector<char> tmp(block * stride);
    for (uint64_t r0 = 0; r0 < rows; r0 += block) {
        const uint64_t m = std::min(block, rows - r0);
        in.read(tmp.data(), static_cast<std::streamsize>(m * stride));
        if (!in) {
            std::free(buf);
            return fail(BS_HOST_EIO, std::string("short read in ") + path);
        }
        for (uint64_t i = 0; i < m; ++i) {
            int32_t di;
            std::memcpy(&di, tmp.data() + i * stride, 4);
            if (di != d) {
                std::free(buf);
                return fail(BS_HOST_EIO, std::string("ragged vecs row in ") + path);
            }
            std::memcpy(buf + (r0 + i) * 4ull * d, tmp.data() + i * stride + 4, 4ull * d);
        }
    }
    (void)is_int;
    *data = buf;
    *n = rows;
    *dim = static_cast<uint32_t>(d);
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

extern "C" int bs_write_vecs(const char* path, int is_int, const void* data, uint64_t n,
                             uint32_t dim) try {
    (void)is_int;
    std::ofstream out(path, std::ios::binary);
    if (!out) return fail(BS_HOST_EIO, std::string("cannot create ") + path);
    const int32_t d = static_cast<int32_t>(dim);
    const char* p = static_cast<const char*>(data);
    const uint64_t stride = 4ull + 4ull * dim;
    const uint64_t block = std::max<uint64_t>(1, (64ull << 20) / stride);
    std::vector<char> tmp(block * stride);
    for (uint64_t r0 = 0; r0 < n; r0 += block) {
        const uint64_t m = std::min(block, n - r0);
        for (uint64_t i = 0; i < m; ++i) {
            std::memcpy(tmp.data() + i * stride, &d, 4);
            std::memcpy(tmp.data() + i * stride + 4, p + (r0 + i) * 4ull * dim, 4ull * dim);
        }
        out.write(tmp.data(), static_cast<std::streamsize>(m * stride));
    }
    if (!out) return fail(BS_HOST_EIO, std::string("write failed: ") + path);
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

extern "C" int bs_read_graph(const char* path, uint32_t** edges, uint64_t* n, uint32_t* degree) try {
    std::ifstream in(path, std::ios::binary);
    if (!in) return fail(BS_HOST_EIO, std::string("cannot open graph file: ") + path);
    in.seekg(0, std::ios::end);
    const uint64_t size = static_cast<uint64_t>(in.tellg());
    in.seekg(0, std::ios::beg);
    int32_t h[2] = {0, 0};
    in.read(reinterpret_cast<char*>(h), 8);
    if (!in || h[0] < 0 || h[1] <= 0) return fail(BS_HOST_EIO, std::string("bad graph header: ") + path);
    const uint64_t cnt = static_cast<uint64_t>(h[0]) * static_cast<uint64_t>(h[1]);
    if (size != 8 + 4 * cnt) return fail(BS_HOST_EIO, std::string("graph file size does not match its header: ") + path);
    uint32_t* e = static_cast<uint32_t*>(std::malloc(std::max<uint64_t>(4, 4 * cnt)));
    if (!e) return fail(BS_HOST_ENOMEM, "out of host memory");
    in.read(reinterpret_cast<char*>(e), static_cast<std::streamsize>(4 * cnt));
    if (!in) {
        std::free(e);
        return fail(BS_HOST_EIO, std::string("short read: ") + path);
    }
    *edges = e;
    *n = static_cast<uint64_t>(h[0]);
    *degree = static_cast<uint32_t>(h[1]);
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

extern "C" int bs_write_graph(const char* path, const uint32_t* edges, uint64_t n, uint32_t degree) try {
    std::ofstream out(path, std::ios::binary);
    if (!out) return fail(BS_HOST_EIO, std::string("cannot create ") + path);
    int32_t h[2] = {static_cast<int32_t>(n), static_cast<int32_t>(degree)};
    out.write(reinterpret_cast<const char*>(h), 8);
    out.write(reinterpret_cast<const char*>(edges), static_cast<std::streamsize>(4 * n * degree));
    if (!out) return fail(BS_HOST_EIO, std::string("write failed: ") + path);
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

extern "C" uint32_t bs_rabitq_padded_dim(uint32_t dim) {
    uint32_t p = 1;
    while (p < dim) p <<= 1;
    return p;
}

extern "C" int bs_read_codebook(const char* path, uint64_t n, uint32_t dim, uint32_t degree,
                                uint32_t* entry, uint32_t** codes, float** factors,
                                float** signs, uint32_t* padded_dim) try {
    const uint32_t pdim = bs_rabitq_padded_dim(dim);
    if (pdim < 32) return fail(BS_HOST_EINVAL, "rabitq needs a padded dim >= 32 (dim > 16)");
    const uint32_t wpp = pdim / 32;
    const uint64_t code_off = dim, factor_off = code_off + uint64_t(wpp) * degree,
                   nbr_off = factor_off + 3ull * degree, row = nbr_off + degree;
    std::ifstream in(path, std::ios::binary);
    if (!in) return fail(BS_HOST_EIO, std::string("cannot open codebook: ") + path);
    in.seekg(0, std::ios::end);
    const uint64_t size = static_cast<uint64_t>(in.tellg());
    in.seekg(0, std::ios::beg);
    const uint64_t expect = 4 + 4 * (n * row + pdim);
    if (size != expect)
        return fail(BS_HOST_EIO, "codebook size " + std::to_string(size) + " != expected " +
                                     std::to_string(expect) + " for n/dim/degree of the graph");
    uint32_t ep = 0;
    in.read(reinterpret_cast<char*>(&ep), 4);
    uint32_t* c = static_cast<uint32_t*>(std::malloc(std::max<uint64_t>(4, 4 * n * degree * wpp)));
    float* f = static_cast<float*>(std::malloc(std::max<uint64_t>(4, 12 * n * degree)));
    float* s = static_cast<float*>(std::malloc(4ull * pdim));
    if (!c || !f || !s) {
        std::free(c);
        std::free(f);
        std::free(s);
        return fail(BS_HOST_ENOMEM, "out of host memory");
    }
    const uint64_t block = std::max<uint64_t>(1, (64ull << 20) / (4 * row));
    std::vector<uint32_t> tmp(block * row);
    for (uint64_t r0 = 0; r0 < n; r0 += block) {
        const uint64_t m = std::min(block, n - r0);
        in.read(reinterpret_cast<char*>(tmp.data()), static_cast<std::streamsize>(4 * m * row));
        for (uint64_t i = 0; i < m; ++i) {
            const uint32_t* r = tmp.data() + i * row;
            std::memcpy(c + (r0 + i) * degree * wpp, r + code_off, 4ull * degree * wpp);
            std::memcpy(f + (r0 + i) * 3 * degree, r + factor_off, 12ull * degree);
        }
    }
    in.read(reinterpret_cast<char*>(s), 4ll * pdim);
    if (!in) {
        std::free(c);
        std::free(f);
        std::free(s);
        return fail(BS_HOST_EIO, std::string("short read: ") + path);
    }
    *entry = ep;
    *codes = c;
    *factors = f;
    *signs = s;
    *padded_dim = pdim;
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

extern "C" int bs_write_codebook(const char* path, const float* vecs, const uint32_t* edges,
                                 uint64_t n, uint32_t dim, uint32_t degree, uint32_t entry,
                                 const uint32_t* codes, const float* factors, const float* signs,
                                 uint32_t padded_dim) try {
    const uint32_t wpp = padded_dim / 32;
    const uint64_t code_off = dim, factor_off = code_off + uint64_t(wpp) * degree,
                   nbr_off = factor_off + 3ull * degree, row = nbr_off + degree;
    std::ofstream out(path, std::ios::binary);
    if (!out) return fail(BS_HOST_EIO, std::string("cannot create ") + path);
    out.write(reinterpret_cast<const char*>(&entry), 4);
    std::vector<uint32_t> r(row);
    for (uint64_t i = 0; i < n; ++i) {
        std::memcpy(r.data(), vecs + i * dim, 4ull * dim);
        std::memcpy(r.data() + code_off, codes + i * degree * wpp, 4ull * degree * wpp);
        std::memcpy(r.data() + factor_off, factors + i * 3 * degree, 12ull * degree);
        std::memcpy(r.data() + nbr_off, edges + i * degree, 4ull * degree);
        out.write(reinterpret_cast<const char*>(r.data()), static_cast<std::streamsize>(4 * row));
    }
    out.write(reinterpret_cast<const char*>(signs), 4ll * padded_dim);
    if (!out) return fail(BS_HOST_EIO, std::string("write failed: ") + path);
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

// ---------------------------------------------------------------------------
// entry point and recall (src/gpu_cli.cu:28-83)
// ---------------------------------------------------------------------------

extern "C" uint32_t bs_entry_point(const float* vecs, uint64_t n, uint32_t dim) {
    // Sequential on purpose: the centroid is accumulated row after row in float, as the
    // reference does, so the chosen node is the reference's.
    std::vector<float> c(dim, 0.0f);
    const float inv = 1.0f / static_cast<float>(n);
    for (uint64_t i = 0; i < n; ++i) {
        const float* row = vecs + i * dim;
        for (uint32_t d = 0; d < dim; ++d) c[d] += row[d] * inv;
    }
    // The nearest-row scan is order independent except for ties (first index wins):
    // parallel chunks, then the smallest (dist, index).
    const int T = bsh::n_threads(0);
    std::vector<float> bd(T, FLT_MAX);
    std::vector<uint64_t> bi(T, 0);
#pragma omp parallel num_threads(T)
    {
        const int t = omp_get_thread_num();
        float best = FLT_MAX;
        uint64_t besti = 0;
#pragma omp for schedule(static)
        for (int64_t i = 0; i < static_cast<int64_t>(n); ++i) {
            const float* row = vecs + static_cast<uint64_t>(i) * dim;
            float s = 0.0f;
            for (uint32_t d = 0; d < dim; ++d) {
                const float diff = row[d] - c[d];
                s += diff * diff;
            }
            if (s < best) {
                best = s;
                besti = static_cast<uint64_t>(i);
            }
        }
        bd[t] = best;
        bi[t] = besti;
    }
    float best = FLT_MAX;
    uint64_t besti = 0;
    for (int t = 0; t < T; ++t)
        if (bd[t] < best || (bd[t] == best && bi[t] < besti)) {
            best = bd[t];
            besti = bi[t];
        }
    return static_cast<uint32_t>(besti);
}

extern "C" double bs_recall(const uint32_t* pred, uint64_t nq, uint32_t K, const int32_t* gt,
                            uint32_t gt_k, uint64_t* dups) {
    uint64_t correct = 0, nd = 0;
    for (uint64_t i = 0; i < nq; ++i) {
        std::unordered_set<int32_t> g(gt + i * gt_k, gt + (i + 1) * gt_k);
        std::unordered_set<uint32_t> seen;
        for (uint32_t j = 0; j < K; ++j) {
            const uint32_t p = pred[i * K + j];
            if (p == 0xFFFFFFFFu) continue;
            if (!seen.insert(p).second) {
                nd++;
                continue;
            }
            if (g.count(static_cast<int32_t>(p))) correct++;
        }
    }
    if (dups) *dups = nd;
    const uint32_t m = std::min(K, gt_k);
    return static_cast<double>(correct) / (static_cast<double>(nq) * m);
}

// ---------------------------------------------------------------------------
// synthetic data
// ---------------------------------------------------------------------------

namespace {

// SplitMix64 finaliser as a counter-based generator: word(stream, counter).
inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
inline uint64_t word(uint64_t stream, uint64_t ctr) { return mix64(mix64(stream) ^ mix64(ctr * 0xD1B54A32D192ED03ull + 1)); }
// uniform in [0,1) with 53 random bits
inline double unif(uint64_t w) { return static_cast<double>(w >> 11) * (1.0 / 9007199254740992.0); }

// Box-Muller (the two-output form): two uniforms -> two independent N(0,1).
inline void box_muller(uint64_t w1, uint64_t w2, double& z0, double& z1) {
    const double u1 = 1.0 - unif(w1);  // (0,1]
    const double u2 = unif(w2);
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double t = 6.283185307179586476925 * u2;
    z0 = r * std::cos(t);
    z1 = r * std::sin(t);
}

void gaussian_row(uint64_t stream, uint64_t row, uint32_t dim, double* z) {
    const uint64_t base = row * (static_cast<uint64_t>(dim) + 2);
    for (uint32_t d = 0; d < dim; d += 2) {
        double a, b;
        box_muller(word(stream, base + d), word(stream, base + d + 1), a, b);
        z[d] = a;
        if (d + 1 < dim) z[d + 1] = b;
    }
}

}  // namespace

extern "C" int bs_gen_mixture(float* out, uint64_t n, uint32_t dim, uint32_t centres, float lo,
                              float hi, float sigma, float clamp_min, uint64_t seed_c,
                              uint64_t seed_x) try {
    if (centres == 0 || dim == 0) return fail(BS_HOST_EINVAL, "centres and dim must be positive");
    std::vector<float> C(static_cast<size_t>(centres) * dim);
    for (uint64_t i = 0; i < C.size(); ++i)
        C[i] = static_cast<float>(lo + (static_cast<double>(hi) - lo) * unif(word(seed_c, i)));
#pragma omp parallel
    {
        std::vector<double> z(dim + 1);
#pragma omp for schedule(static)
        for (int64_t i = 0; i < static_cast<int64_t>(n); ++i) {
            const uint64_t r = static_cast<uint64_t>(i);
            const uint32_t c = static_cast<uint32_t>(word(seed_x ^ 0x5EEDC0DEull, r) % centres);
            gaussian_row(seed_x, r, dim, z.data());
            float* o = out + r * dim;
            for (uint32_t d = 0; d < dim; ++d) {
                float v = static_cast<float>(C[static_cast<size_t>(c) * dim + d] + static_cast<double>(sigma) * z[d]);
                o[d] = v < clamp_min ? clamp_min : v;
            }
        }
    }
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

extern "C" int bs_gen_normalized(float* out, uint64_t n, uint32_t dim, uint64_t seed) try {
#pragma omp parallel
    {
        std::vector<double> z(dim + 1);
#pragma omp for schedule(static)
        for (int64_t i = 0; i < static_cast<int64_t>(n); ++i) {
            const uint64_t r = static_cast<uint64_t>(i);
            gaussian_row(seed, r, dim, z.data());
            double s = 0.0;
            for (uint32_t d = 0; d < dim; ++d) s += z[d] * z[d];
            const double inv = s > 0 ? 1.0 / std::sqrt(s) : 0.0;
            for (uint32_t d = 0; d < dim; ++d) out[r * dim + d] = static_cast<float>(z[d] * inv);
        }
    }
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

// ---------------------------------------------------------------------------
// ground truth
// ---------------------------------------------------------------------------

namespace {
struct DP {
    double d;
    uint32_t id;
    bool operator<(const DP& o) const { return d != o.d ? d < o.d : id < o.id; }
};
inline double l2d(const float* a, const float* b, uint32_t dim) {
    double s = 0.0;
    for (uint32_t i = 0; i < dim; ++i) {
        const double diff = static_cast<double>(a[i]) - static_cast<double>(b[i]);
        s += diff * diff;
    }
    return s;
}
}  // namespace

extern "C" int bs_groundtruth(const float* base, uint64_t n, const float* queries, uint64_t nq,
                              uint32_t dim, uint32_t k, int32_t* out, int threads) try {
    if (k == 0) return fail(BS_HOST_EINVAL, "k must be positive");
#pragma omp parallel num_threads(bsh::n_threads(threads))
    {
        std::vector<DP> heap;
        heap.reserve(k + 1);
#pragma omp for schedule(dynamic, 4)
        for (int64_t qi = 0; qi < static_cast<int64_t>(nq); ++qi) {
            const float* q = queries + static_cast<uint64_t>(qi) * dim;
            heap.clear();
            for (uint64_t j = 0; j < n; ++j) {
                DP e{l2d(q, base + j * dim, dim), static_cast<uint32_t>(j)};
                if (heap.size() < k) {
                    heap.push_back(e);
                    std::push_heap(heap.begin(), heap.end());
                } else if (e < heap.front()) {
                    std::pop_heap(heap.begin(), heap.end());
                    heap.back() = e;
                    std::push_heap(heap.begin(), heap.end());
                }
            }
            std::sort(heap.begin(), heap.end());
            for (uint32_t t = 0; t < k; ++t)
                out[static_cast<uint64_t>(qi) * k + t] = t < heap.size() ? static_cast<int32_t>(heap[t].id) : -1;
        }
    }
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}

extern "C" int bs_groundtruth_refine(const float* base, uint64_t n, const float* queries,
                                     uint64_t nq, uint32_t dim, const int64_t* cand,
                                     uint32_t ncand, uint32_t k, int32_t* out, int threads) try {
    if (k == 0 || ncand < k) return fail(BS_HOST_EINVAL, "need ncand >= k > 0");
#pragma omp parallel num_threads(bsh::n_threads(threads))
    {
        std::vector<DP> v;
        v.reserve(ncand);
#pragma omp for schedule(static)
        for (int64_t qi = 0; qi < static_cast<int64_t>(nq); ++qi) {
            const float* q = queries + static_cast<uint64_t>(qi) * dim;
            v.clear();
            for (uint32_t c = 0; c < ncand; ++c) {
                const int64_t id = cand[static_cast<uint64_t>(qi) * ncand + c];
                if (id < 0 || static_cast<uint64_t>(id) >= n) continue;
                v.push_back({l2d(q, base + static_cast<uint64_t>(id) * dim, dim), static_cast<uint32_t>(id)});
            }
            std::sort(v.begin(), v.end());
            v.erase(std::unique(v.begin(), v.end(), [](const DP& a, const DP& b) { return a.id == b.id; }), v.end());
            for (uint32_t t = 0; t < k; ++t)
                out[static_cast<uint64_t>(qi) * k + t] = t < v.size() ? static_cast<int32_t>(v[t].id) : -1;
        }
    }
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}
