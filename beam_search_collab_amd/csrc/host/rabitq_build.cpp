// RaBitQ per-edge codebook construction (host, OpenMP).
//
// Same arithmetic as the reference builder (src/build_rabitq.cpp:19-264) so the codebook
// is byte-identical: float WHT rotation of signs * vector, float residual and norms,
// long double for the factor products.  This build rotates every node once and reuses
// the rotation for all edges that touch it (the reference recomputes the neighbour's
// rotation per edge; the values are the same).
#include "bs_host.h"
#include "host_common.hpp"

#include <cfloat>
#include <cmath>
#include <cstring>
#include <limits>
#include <random>
#include <vector>

#include <omp.h>

namespace {

// build_rabitq.cpp:19-30
void wht(float* x, uint32_t n) {
    for (uint32_t len = 1; len < n; len <<= 1)
        for (uint32_t i = 0; i < n; i += len << 1)
            for (uint32_t j = 0; j < len; ++j) {
                const float u = x[i + j], v = x[i + j + len];
                x[i + j] = u + v;
                x[i + j + len] = u - v;
            }
}

}  // namespace

extern "C" int bs_build_rabitq(const float* vecs, const uint32_t* edges, uint64_t n, uint32_t dim,
                               uint32_t degree, uint32_t seed, int threads, uint32_t* codes_out,
                               float* factors_out, float* signs_out, uint32_t* entry_out) try {
    const uint32_t pdim = bs_rabitq_padded_dim(dim);
    if (pdim < 32) return bsh::fail(BS_HOST_EINVAL, "rabitq needs a padded dim >= 32 (dim > 16)");
    const uint32_t wpp = pdim / 32;
    const int T = bsh::n_threads(threads);

    // signs (build_rabitq.cpp:138-145)
    {
        std::mt19937_64 gen(seed);
        std::uniform_int_distribution<int> coin(0, 1);
        const float scale = 1.0f / std::sqrt(static_cast<float>(pdim));
        for (uint32_t i = 0; i < pdim; ++i) signs_out[i] = static_cast<float>(2 * coin(gen) - 1) * scale;
    }

    // medoid entry point (build_rabitq.cpp:59-99): double centroid, nearest row;
    // ties resolved to the smallest index.
    {
        std::vector<double> cen(dim, 0.0);
        for (uint64_t i = 0; i < n; ++i)
            for (uint32_t d = 0; d < dim; ++d) cen[d] += vecs[i * dim + d];
        for (uint32_t d = 0; d < dim; ++d) cen[d] /= static_cast<double>(n);
        std::vector<double> bd(T, std::numeric_limits<double>::max());
        std::vector<uint64_t> bi(T, 0);
#pragma omp parallel num_threads(T)
        {
            const int t = omp_get_thread_num();
#pragma omp for schedule(static)
            for (int64_t i = 0; i < static_cast<int64_t>(n); ++i) {
                double s = 0.0;
                for (uint32_t d = 0; d < dim; ++d) {
                    const double diff = vecs[static_cast<uint64_t>(i) * dim + d] - cen[d];
                    s += diff * diff;
                }
                if (s < bd[t]) {
                    bd[t] = s;
                    bi[t] = static_cast<uint64_t>(i);
                }
            }
        }
        double best = std::numeric_limits<double>::max();
        uint64_t besti = 0;
        for (int t = 0; t < T; ++t)
            if (bd[t] < best || (bd[t] == best && bi[t] < besti)) {
                best = bd[t];
                besti = bi[t];
            }
        *entry_out = static_cast<uint32_t>(besti);
    }

    // rotations of every node: rot = WHT(signs * [v, 0...])
    std::vector<float> rot(n * static_cast<uint64_t>(pdim));
#pragma omp parallel for schedule(static) num_threads(T)
    for (int64_t i = 0; i < static_cast<int64_t>(n); ++i) {
        float* r = rot.data() + static_cast<uint64_t>(i) * pdim;
        const float* v = vecs + static_cast<uint64_t>(i) * dim;
        for (uint32_t d = 0; d < dim; ++d) r[d] = v[d] * signs_out[d];
        for (uint32_t d = dim; d < pdim; ++d) r[d] = 0.0f;
        wht(r, pdim);
    }

    // per-edge codes and factors (build_rabitq.cpp:178-259)
    const float fac_norm = 1.0f / std::sqrt(static_cast<float>(dim));
#pragma omp parallel num_threads(T)
    {
        std::vector<float> res(pdim);
#pragma omp for schedule(dynamic, 64)
        for (int64_t ui = 0; ui < static_cast<int64_t>(n); ++ui) {
            const uint64_t u = static_cast<uint64_t>(ui);
            const float* ur = rot.data() + u * pdim;
            uint32_t* cw = codes_out + u * degree * wpp;
            std::memset(cw, 0, 4ull * degree * wpp);
            float* tx = factors_out + u * 3 * degree;
            float* dq = tx + degree;
            float* vq = dq + degree;
            for (uint32_t i = 0; i < degree; ++i) {
                const uint32_t v = edges[u * degree + i];
                if (v == 0xFFFFFFFFu) {
                    tx[i] = FLT_MAX;
                    dq[i] = 0.0f;
                    vq[i] = 0.0f;
                    continue;
                }
                const float* vr = rot.data() + static_cast<uint64_t>(v) * pdim;
                float sqr_r = 0.0f;
                for (uint32_t d = 0; d < dim; ++d) {
                    res[d] = vr[d] - ur[d];
                    sqr_r += res[d] * res[d];
                }
                const float r_norm = std::sqrt(sqr_r) + 1e-10f;
                int bin_sum = 0;
                uint32_t* code = cw + static_cast<uint64_t>(i) * wpp;
                for (uint32_t d = 0; d < dim; ++d) {
                    if (res[d] > 0.0f) {
                        code[d >> 5] |= 1u << (d & 31);
                        ++bin_sum;
                    }
                }
                float fx0 = 0.0f, fx1 = 0.0f;
                for (uint32_t d = 0; d < dim; ++d) {
                    const float sv = (res[d] > 0.0f) ? 1.0f : -1.0f;
                    fx0 += res[d] * sv * fac_norm;
                    fx1 += ur[d] * sv;
                }
                fx0 /= r_norm;
                fx1 *= fac_norm;
                const long double x_x0 = static_cast<long double>(r_norm) / fx0;
                tx[i] = static_cast<float>(static_cast<long double>(r_norm) * r_norm + 2.0L * x_x0 * fx1);
                dq[i] = static_cast<float>(-2.0L * x_x0 * fac_norm);
                vq[i] = dq[i] * static_cast<float>(2 * bin_sum - static_cast<int>(dim));
            }
        }
    }
    return BS_HOST_OK;
} catch (...) {
    return bsh::exception_code();
}
