// C-ABI of libbs_hip.so: index residency, search dispatch, primitive entry points.
// Declarations and reference citations: include/bs_hip.h.
#include "bs_hip.h"
#include "bs_launch.hpp"
#include "bs_order.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cstdio>
#include <cstring>
#include <exception>
#include <mutex>
#include <new>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define HIP_TRY(call)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return fail(BS_EHIP, std::string(#call) + " failed: " + hipGetErrorString(e_));  \
    } while (0)

uint32_t log2_ceil(uint32_t v) {
    uint32_t b = 0;
    while ((1ull << b) < v) ++b;
    return b;
}

int check_device() {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, dev));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(BS_ENODEV, std::string("libbs_hip.so is built for gfx950 (MI355X); device is ") + prop.gcnArchName);
    if (prop.warpSize != 64) return fail(BS_ENODEV, "wavefront size 64 required");
    return BS_OK;
}

}  // namespace

struct bs_index_s {
    int device = 0;
    uint64_t n = 0;
    uint32_t dim = 0, dstride = 0, degree = 0;
    float* d_vecs = nullptr;
    uint32_t* d_edges = nullptr;
    // rabitq node records: [vec dstride | ids R | tx R | fdq R | fvq R | codes R*wpp],
    // rounded up to 32 words (128 B)
    uint32_t pdim = 0, wpp = 0, rec_words = 0, rec_ids = 0, rec_fac = 0, rec_codes = 0;
    uint32_t* d_recs = nullptr;
    float* d_signs = nullptr;
    size_t max_lds = 65536;
    size_t lds_cu = 65536;  // LDS per compute unit (shared by its resident workgroups)
    uint32_t cus = 256;  // compute units of the device
    uint32_t xcds = 1;   // XCDs of the device (workgroup b runs on XCD b mod xcds)
    // query scheduling (bs_order.hip): pivots, labels, launch map, for up to ORDER_CHUNK
    // queries per search launch; ws_free orders launches that share the workspace
    int order_mode = 1;
    float* d_pivT = nullptr;
    float* d_pnorm = nullptr;
    uint32_t* d_ows = nullptr;  // key[ORDER_CHUNK] | qmap[ORDER_CHUNK] | hist[P] | cursor[P]
    hipEvent_t ws_free = nullptr;
    // expected cost per label for the base-family label order (calibrate_labels), or null
    float* d_lcost = nullptr;
    // device staging of bs_search (host buffers): grows to the largest call, reused after
    void* d_stage = nullptr;
    size_t stage_bytes = 0;
};

namespace {
constexpr uint64_t ORDER_CHUNK = 1u << 18;  // queries per ordered search launch
constexpr uint64_t ORDER_MIN_NQ = 4096;     // mode 1 orders launches of at least this many
// LDS is handed to workgroups in 512-B granules (measured on gfx950: a 10848-B workgroup
// is resident 14 times per CU, not the 15 that 160 KB / 10848 B suggests)
constexpr uint32_t LDS_GRANULE = 512;

// Pivots for query scheduling: ORDER_P rows spread evenly over the index (all rows when
// n is smaller), re-ordered by a greedy nearest-neighbour tour so that consecutive
// labels are near in space.  Returns the transposed pivots and their squared norms.
void make_pivots(const float* vecs, uint64_t n, uint32_t dim, std::vector<float>& pivT, std::vector<float>& pnorm) {
    const uint32_t P = bso::ORDER_P;
    const uint32_t m = static_cast<uint32_t>(std::min<uint64_t>(P, n));
    std::vector<uint64_t> rows(m);
    for (uint32_t i = 0; i < m; ++i) rows[i] = static_cast<uint64_t>(i) * n / m;
    std::vector<uint32_t> tour;
    std::vector<char> used(m, 0);
    uint32_t cur = 0;
    used[0] = 1;
    tour.push_back(0);
    while (tour.size() < m) {
        const float* a = vecs + rows[cur] * dim;
        double best = DBL_MAX;
        uint32_t bi = 0;
        for (uint32_t j = 0; j < m; ++j) {
            if (used[j]) continue;
            const float* b = vecs + rows[j] * dim;
            double d = 0;
            for (uint32_t k = 0; k < dim; ++k) {
                const double t = static_cast<double>(a[k]) - b[k];
                d += t * t;
            }
            if (d < best) {
                best = d;
                bi = j;
            }
        }
        used[bi] = 1;
        tour.push_back(bi);
        cur = bi;
    }
    pivT.assign(static_cast<size_t>((dim + 15) & ~15u) * P, 0.0f);  // rows for whole blocks of 16
    pnorm.assign(P, 1e30f);  // unused slots never win
    for (uint32_t t = 0; t < m; ++t) {
        const float* v = vecs + rows[tour[t]] * dim;
        double nn = 0;
        for (uint32_t k = 0; k < dim; ++k) {
            pivT[static_cast<size_t>(k) * P + t] = v[k];
            nn += static_cast<double>(v[k]) * v[k];
        }
        pnorm[t] = static_cast<float>(nn);
    }
}
// the device address of bs_search_device_noalloc's static workspace (defined below)
int noalloc_workspace(int dev, uint32_t** out);
// the label costs of the base-family query order (defined below)
void calibrate_labels(bs_index ix);
}  // namespace

extern "C" const char* bs_last_error(void) { return g_err.c_str(); }

// helpers for the primitive entry points (bs_debug.hip)
int bs_internal_vecs(bs_index ix, const float** vecs, uint32_t* dstride) {
    if (!ix) return fail(BS_EINVAL, "null index");
    *vecs = ix->d_vecs;
    *dstride = ix->dstride;
    return BS_OK;
}
int bs_internal_edges(bs_index ix, const uint32_t** edges) {
    if (!ix) return fail(BS_EINVAL, "null index");
    *edges = ix->d_edges;
    return BS_OK;
}
void bs_internal_set_error(const std::string& msg) { g_err = msg; }
// Inside a catch handler: the error code and text for the exception in flight (every
// entry point catches all exceptions; none crosses the C-ABI).
int bs_internal_exception() {
    try {
        throw;
    } catch (const std::bad_alloc&) {
        return fail(BS_ENOMEM, "host memory allocation failed");
    } catch (const std::exception& e) {
        return fail(BS_EHIP, std::string("internal error: ") + e.what());
    } catch (...) {
        return fail(BS_EHIP, "internal error");
    }
}

extern "C" int bs_index_create(const float* vecs, const uint32_t* edges, uint64_t n, uint32_t dim,
                               uint32_t degree, bs_index* out) try {
    if (!out) return fail(BS_EINVAL, "out is null");
    *out = nullptr;
    if (!vecs || !edges) return fail(BS_EINVAL, "vecs and edges must be given");
    if (n == 0 || n > 0x7FFFFFFFull) return fail(BS_EINVAL, "need 0 < n < 2^31");
    if (dim == 0 || dim > 1024) return fail(BS_EINVAL, "dim must be in 1..1024");
    if (degree == 0 || degree > 256) return fail(BS_EINVAL, "degree must be in 1..256");
    // every neighbour id must address a node (the kernels gather rows without bounds checks)
    for (uint64_t i = 0, cnt = n * degree; i < cnt; ++i) {
        const uint32_t e = edges[i];
        if (e != 0xFFFFFFFFu && e >= n)
            return fail(BS_EINVAL, "edge " + std::to_string(i) + " points to node " + std::to_string(e) +
                                       " >= n = " + std::to_string(n));
    }
    int rc = check_device();
    if (rc) return rc;
    int device = 0;
    HIP_TRY(hipGetDevice(&device));
    {
        // bs_search_device_noalloc's workspace address on this device, looked up here, at
        // set-up, so that no later call (one under graph capture, say) makes the lookup
        uint32_t* ws = nullptr;
        rc = noalloc_workspace(device, &ws);
        if (rc) return rc;
    }
    bs_index_s* ix = new bs_index_s();
    ix->n = n;
    ix->dim = dim;
    ix->dstride = (dim + 3) & ~3u;
    ix->degree = degree;
    ix->device = device;
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, ix->device) == hipSuccess && lds > 0)
        ix->max_lds = static_cast<size_t>(lds);
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, ix->device) == hipSuccess &&
        lds > 0)
        ix->lds_cu = static_cast<size_t>(lds);
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ix->device) == hipSuccess && cus > 0)
        ix->cus = static_cast<uint32_t>(cus);
    int xcds = 0;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, ix->device) == hipSuccess && xcds > 0)
        ix->xcds = std::min<uint32_t>(static_cast<uint32_t>(xcds), bso::ORDER_MAX_X);
    const size_t vbytes = n * ix->dstride * sizeof(float);
    if (hipMalloc(&ix->d_vecs, vbytes) != hipSuccess) {
        delete ix;
        return fail(BS_ENOMEM, "hipMalloc of the vectors failed");
    }
    if (hipMalloc(&ix->d_edges, n * degree * sizeof(uint32_t)) != hipSuccess) {
        (void)hipFree(ix->d_vecs);
        delete ix;
        return fail(BS_ENOMEM, "hipMalloc of the edges failed");
    }
    hipError_t e = hipSuccess;
    if (ix->dstride == dim) {
        e = hipMemcpy(ix->d_vecs, vecs, vbytes, hipMemcpyHostToDevice);
    } else {
        e = hipMemset(ix->d_vecs, 0, vbytes);
        if (e == hipSuccess)
            e = hipMemcpy2D(ix->d_vecs, ix->dstride * sizeof(float), vecs, dim * sizeof(float), dim * sizeof(float),
                            n, hipMemcpyHostToDevice);
    }
    if (e == hipSuccess) e = hipMemcpy(ix->d_edges, edges, n * degree * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        std::vector<float> pivT, pnorm;
        make_pivots(vecs, n, dim, pivT, pnorm);
        const size_t ows = (2 * ORDER_CHUNK + 2 * bso::ORDER_P) * sizeof(uint32_t);
        e = hipMalloc(&ix->d_pivT, pivT.size() * sizeof(float));
        if (e == hipSuccess) e = hipMalloc(&ix->d_pnorm, pnorm.size() * sizeof(float));
        if (e == hipSuccess) e = hipMalloc(&ix->d_ows, ows);
        if (e == hipSuccess) e = hipMemcpy(ix->d_pivT, pivT.data(), pivT.size() * sizeof(float), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(ix->d_pnorm, pnorm.data(), pnorm.size() * sizeof(float), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemset(ix->d_ows, 0, ows);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ix->ws_free, hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        bs_index_destroy(ix);
        return fail(BS_EHIP, std::string("upload failed: ") + hipGetErrorString(e));
    }
    calibrate_labels(ix);
    *out = ix;
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

// Node records [vec dstride | ids R | tx R | fdq R | fvq R | codes R*cws | 0...] (rw words),
// a thread per word.  vecs/edges/factors/codes/recs point at the chunk's first node.
__global__ void __launch_bounds__(256) assemble_records(const float* vecs, const uint32_t* edges,
                                                        const float* factors, const uint32_t* codes, uint64_t m,
                                                        uint32_t dstride, uint32_t R, uint32_t wpp, uint32_t cws,
                                                        uint32_t rw, uint32_t* recs) {
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= m * rw) return;
    const uint64_t u = t / rw;
    const uint32_t w = static_cast<uint32_t>(t - u * rw);
    const uint32_t ids = dstride, fac = ids + R, cod = fac + 3 * R;
    uint32_t v = 0;
    if (w < ids) {
        v = __float_as_uint(vecs[u * dstride + w]);
    } else if (w < fac) {
        v = edges[u * R + (w - ids)];
    } else if (w < cod) {
        v = __float_as_uint(factors[u * 3 * R + (w - fac)]);
    } else if (w - cod < R * cws) {
        const uint32_t j = (w - cod) / cws, k = (w - cod) % cws;
        v = k < wpp ? codes[(u * R + j) * wpp + k] : 0u;
    }
    recs[t] = v;
}

extern "C" int bs_index_attach_rabitq(bs_index ix, const uint32_t* codes, const float* factors,
                                      const float* signs, uint32_t padded_dim) try {
    if (!ix || !codes || !factors || !signs) return fail(BS_EINVAL, "null argument");
    uint32_t p = 1;
    while (p < ix->dim) p <<= 1;
    if (padded_dim != p) return fail(BS_EINVAL, "padded_dim must be pow2ceil(dim) = " + std::to_string(p));
    if (padded_dim < 32 || padded_dim > 2048) return fail(BS_EINVAL, "padded_dim must be in 32..2048");
    const uint32_t R = ix->degree, wpp = padded_dim / 32;
    const uint32_t cws = bsd::quad_shape(wpp, R).cws;  // code words per neighbour, >= 4
    uint32_t rw = ix->dstride + R + 3 * R + R * cws;
    rw = (rw + 31) & ~31u;
    if (ix->d_recs) {
        (void)hipFree(ix->d_recs);
        ix->d_recs = nullptr;
    }
    if (ix->d_signs) {
        (void)hipFree(ix->d_signs);
        ix->d_signs = nullptr;
    }
    if (hipMalloc(&ix->d_recs, ix->n * static_cast<size_t>(rw) * 4) != hipSuccess)
        return fail(BS_ENOMEM, "hipMalloc of the rabitq records failed");
    HIP_TRY(hipMalloc(&ix->d_signs, padded_dim * sizeof(float)));
    HIP_TRY(hipMemcpy(ix->d_signs, signs, padded_dim * sizeof(float), hipMemcpyHostToDevice));
    ix->pdim = padded_dim;
    ix->wpp = wpp;
    ix->rec_words = rw;
    ix->rec_ids = ix->dstride;
    ix->rec_fac = ix->rec_ids + R;
    ix->rec_codes = ix->rec_fac + 3 * R;
    // upload codes and factors in chunks of nodes; a kernel writes the chunk's records from
    // them and the resident vectors and edges
    const uint64_t chunk = std::max<uint64_t>(1, (256ull << 20) / (4ull * R * (wpp + 3)));
    const uint64_t m0 = std::min(chunk, ix->n);
    uint32_t* d_codes = nullptr;
    float* d_fac = nullptr;
    if (hipMalloc(&d_codes, m0 * R * wpp * 4ull) != hipSuccess || hipMalloc(&d_fac, m0 * 3ull * R * 4ull) != hipSuccess) {
        if (d_codes) (void)hipFree(d_codes);
        return fail(BS_ENOMEM, "hipMalloc of the record staging buffers failed");
    }
    hipError_t e = hipSuccess;
    for (uint64_t r0 = 0; e == hipSuccess && r0 < ix->n; r0 += chunk) {
        const uint64_t m = std::min(chunk, ix->n - r0);
        e = hipMemcpy(d_codes, codes + r0 * R * wpp, m * R * wpp * 4ull, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d_fac, factors + r0 * 3ull * R, m * 3ull * R * 4ull, hipMemcpyHostToDevice);
        if (e != hipSuccess) break;
        const uint64_t words = m * rw;
        hipLaunchKernelGGL(assemble_records, dim3(static_cast<uint32_t>((words + 255) / 256)), dim3(256), 0, nullptr,
                           ix->d_vecs + r0 * ix->dstride, ix->d_edges + r0 * R, d_fac, d_codes, m, ix->dstride, R, wpp,
                           cws, rw, ix->d_recs + r0 * rw);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    (void)hipFree(d_codes);
    (void)hipFree(d_fac);
    if (e != hipSuccess) return fail(BS_EHIP, std::string("rabitq record assembly: ") + hipGetErrorString(e));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

extern "C" int bs_index_info(bs_index ix, uint64_t* n, uint32_t* dim, uint32_t* degree,
                             uint32_t* padded_dim, int* has_rabitq) try {
    if (!ix) return fail(BS_EINVAL, "null index");
    if (n) *n = ix->n;
    if (dim) *dim = ix->dim;
    if (degree) *degree = ix->degree;
    if (padded_dim) *padded_dim = ix->pdim;
    if (has_rabitq) *has_rabitq = ix->d_recs != nullptr;
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

extern "C" void bs_index_destroy(bs_index ix) {
    if (!ix) return;
    if (ix->d_vecs) (void)hipFree(ix->d_vecs);
    if (ix->d_edges) (void)hipFree(ix->d_edges);
    if (ix->d_recs) (void)hipFree(ix->d_recs);
    if (ix->d_signs) (void)hipFree(ix->d_signs);
    if (ix->ws_free) {
        (void)hipEventSynchronize(ix->ws_free);
        (void)hipEventDestroy(ix->ws_free);
    }
    if (ix->d_pivT) (void)hipFree(ix->d_pivT);
    if (ix->d_pnorm) (void)hipFree(ix->d_pnorm);
    if (ix->d_ows) (void)hipFree(ix->d_ows);
    if (ix->d_lcost) (void)hipFree(ix->d_lcost);
    if (ix->d_stage) (void)hipFree(ix->d_stage);
    delete ix;
}

extern "C" int bs_index_label_costs(bs_index ix, float* out) try {
    if (!ix || !out) return fail(BS_EINVAL, "null argument");
    if (!ix->d_lcost) return fail(BS_EINVAL, "the index has no calibrated label costs");
    HIP_TRY(hipMemcpy(out, ix->d_lcost, bso::ORDER_P * sizeof(float), hipMemcpyDeviceToHost));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

extern "C" int bs_index_set_query_order(bs_index ix, int mode) try {
    if (!ix) return fail(BS_EINVAL, "null index");
    if (mode < 0 || mode > 2) return fail(BS_EINVAL, "query order mode must be 0, 1 or 2");
    ix->order_mode = mode;
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

namespace {

struct Plan {
    bsd::SearchParams p;
    int TR, CR, PB, mode;
    uint32_t g;
    dim3 grid, block;
    size_t lds;
};

// validate the configuration and fill the kernel parameters
int make_plan(bs_index ix, const bs_search_cfg* cfg, uint64_t nq, Plan& pl) {
    if (!ix || !cfg) return fail(BS_EINVAL, "null argument");
    const int mode = cfg->mode;
    if (mode < BS_BASE || mode > BS_RABITQ) return fail(BS_EINVAL, "unknown mode " + std::to_string(mode));
    if (mode == BS_RABITQ && !ix->d_recs) return fail(BS_EINVAL, "rabitq mode needs bs_index_attach_rabitq first");
    const uint32_t T = cfg->topk_size;
    if (T == 0 || T > 4096) return fail(BS_EINVAL, "topk_size must be in 1..4096");
    if (cfg->K == 0) return fail(BS_EINVAL, "K must be >= 1");
    if (mode != BS_RABITQ && T < cfg->K)
        return fail(BS_EINVAL, "topk_size (" + std::to_string(T) + ") must be >= K (" + std::to_string(cfg->K) + ")");
    if (cfg->K > 4096) return fail(BS_EINVAL, "K must be <= 4096");
    if (cfg->entry_point >= ix->n) return fail(BS_EINVAL, "entry_point out of range");
    if (cfg->max_iterations < 0) return fail(BS_EINVAL, "max_iterations must be >= 0");
    if (cfg->reset_interval < 0) return fail(BS_EINVAL, "reset_interval must be >= 0");
    uint32_t ny = cfg->queries_per_group ? cfg->queries_per_group : 1;
    if (ny != 1 && ny != 2 && ny != 4 && ny != 8) return fail(BS_EINVAL, "queries_per_group must be 1, 2, 4 or 8");
    const uint32_t cap = cfg->filter_capacity;
    if (cap > (1u << 16) && mode != BS_GROUP_BLOOM) return fail(BS_EINVAL, "filter_capacity must be <= 65536");
    if (cap > (1u << 22)) return fail(BS_EINVAL, "filter_capacity must be <= 2^22");

    pl.mode = mode;
    // RaBitQ beams of 513..640 and 641..768 keys get 10 and 12 registers (the recall@10 0.95
    // point of config C is topk 640: 1M x 128, 10k queries, 6.31 ms with 12 registers)
    pl.TR = T <= 64 ? 1 : T <= 128 ? 2 : T <= 256 ? 4 : T <= 512 ? 8
          : (T <= 640 && mode == BS_RABITQ) ? 10 : (T <= 768 && mode == BS_RABITQ) ? 12
          : T <= 1024 ? 16 : T <= 2048 ? 32 : 64;
    pl.CR = ix->degree <= 64 ? 1 : ix->degree <= 128 ? 2 : 4;
    // RaBitQ with narrow codes (dim <= 128): one chunk per lane (bsd::l2_shape_lanes)
    const bool narrow_rq = mode == BS_RABITQ && ix->wpp <= 4;
    bsd::L2Shape L = narrow_rq ? bsd::l2_shape_lanes(ix->dim) : bsd::l2_shape(ix->dim);
    if (L.QR > (narrow_rq ? 1u : 4u)) return fail(BS_EINVAL, "dim too large");
    // 32 rows per batch for the hash-filter loop over rows of up to 128 dims: 1M x 128,
    // degree 32: topk 256 4.58 -> 4.49 ms, topk 128 2.54 -> 2.39, topk 512 9.75 -> 8.66
    // (with the larger visit filter below); the Bloom loop keeps 16 (its wavefronts per CU
    // drop from 16 to 12 for nothing: bwarp1 5.46 -> 6.41 ms)
    pl.PB = bsd::l2_passes_in_flight(L, (mode == BS_BASE || mode == BS_GROUP) && L.rpp >= 8u ? 32u : 16u);

    bsd::SearchParams& p = pl.p;
    std::memset(&p, 0, sizeof(p));
    p.vecs = ix->d_vecs;
    p.edges = ix->d_edges;
    p.recs = ix->d_recs;
    p.signs = ix->d_signs;
    p.nq = nq;
    p.dim = ix->dim;
    p.dstride = ix->dstride;
    p.R = ix->degree;
    p.K = cfg->K;
    p.T = T;
    p.entry = cfg->entry_point;
    p.max_it = cfg->max_iterations;
    p.reset = cfg->reset_interval;
    p.L = L;
    // The hash filters (visit filter, RaBitQ expanded set) refuse keys as the reference's
    // table of 2^ceil(log2 capacity) slots does, but get more slots when the workgroup's LDS
    // allows it: probe runs at the same occupancy are shorter, the results are the same.
    // The visit filter fills up between resets: it gets at least twice the slots (config B:
    // 5.0 -> 4.8 ms, topk 512: 20.1 -> 10.9 ms), and up to four times as many as the LDS
    // left by the instance's register-limited residency holds (config B with 32-row L2
    // batches: 2048 slots 4.54 ms, 2624 slots 4.43 ms; smaller tables that admit more
    // wavefronts lost: 1344 slots at 20 wavefronts per CU 5.0 ms).  The slice budget rounds
    // to 512 B, while gfx950 allocates LDS in 1280-B granules (slices of 12640 B fit 12 per
    // CU, of 12896 B 11), so config B's 2624-slot table (13152 B) holds 11 wavefronts per CU
    // of the 12 its registers allow; a table small enough for 12 measured slower (2496 slots,
    // 12 per CU: 4.19-4.27 ms against 4.09-4.14 for 2560-2816 slots at 11, 4.13-4.16 for
    // 3072 at 10, 4.5 for 3328 at 9; identical results throughout).  The RaBitQ expanded set
    // ends with about one key per beam slot and gets 5T/3 slots within [cap, 2 cap] (topk
    // 768: 2048 slots 14.0 ms, 1280 slots 12.8 ms: fewer slots, more wavefronts per CU).
    uint32_t scratch = 512u * pl.TR + 16u;  // the beam and the merge's dump slot
    if (mode == BS_RABITQ) {
        p.pdim = ix->pdim;
        p.wpp = ix->wpp;
        p.rec_words = ix->rec_words;
        p.rec_ids = ix->rec_ids;
        p.rec_fac = ix->rec_fac;
        p.rec_codes = ix->rec_codes;
        p.Q = bsd::quad_shape(ix->wpp, ix->degree);
        // quantizer workspace (4 pdim B) and merge scratch overlap; the bit planes
        // (6 planes of max(wpp, 4) words) follow both and live for the whole query
        const uint32_t planes_at = std::max(scratch, 4u * ix->pdim);
        scratch = planes_at + 24u * std::max(ix->wpp, 4u);
        p.off_planes = planes_at;  // relative to off_scratch until the layout is fixed below
    }
    const uint32_t planes_rel = p.off_planes;
    auto al = [](uint32_t v) { return (v + 15u) & ~15u; };
    auto layout = [&](uint32_t filter_bytes) {
        p.off_filter = 0;
        p.off_scratch = al(filter_bytes);
        p.off_cand = p.off_scratch + al(scratch);
        if (mode == BS_RABITQ) p.off_planes = planes_rel + p.off_scratch;
        p.off_coop = p.off_cand + 64u * pl.CR * 8u + 8u * std::max(pl.TR, 8);  // after the merge's slot bitmap
        p.lds_wave = al(p.off_coop + 4u);
        // the deferred merge's append staging (64 keys) reuses the merge scratch: it is
        // written and read back inside pending_add, where no merge is running
        if (mode == BS_RABITQ && pl.TR >= 8) p.off_pend = p.off_scratch;
    };
    if (mode == BS_GROUP_BLOOM) {
        uint32_t b = log2_ceil(cap);
        if (b < 5) b = 5;
        p.filter_bits = b;
        p.filter_cap = 0;
        layout((1u << (b - 5)) * 4);
    } else {
        const uint32_t b = log2_ceil(cap);
        p.filter_cap = 1u << b;
        const uint32_t base_slots = std::max(4u, p.filter_cap);
        if (mode != BS_RABITQ) {
            p.filter_slots = b < 11 ? base_slots * 2u : base_slots;
            layout(0);
            const uint32_t other = p.lds_wave;  // the slice without the filter
            int wg = 0;                          // workgroups per CU the registers allow
            if (bsd::launch_search_hash(p, pl.TR, pl.CR, pl.PB, dim3(1), dim3(64 * ny), 0, nullptr, &wg) ==
                    hipSuccess &&
                wg > 0) {
                const uint32_t per_wave = static_cast<uint32_t>((ix->lds_cu / static_cast<size_t>(wg)) &
                                                                ~static_cast<size_t>(LDS_GRANULE - 1)) / ny;
                const uint32_t fit = per_wave > other ? (per_wave - other) / 4u / 64u * 64u : 0u;
                if (fit > p.filter_slots) p.filter_slots = std::min(fit, 4u * base_slots);
            }
        } else {
            // the expanded set holds about one key per beam slot: 5T/3 slots (a multiple of
            // 64), at least cap and at most 2 cap, and no more than the LDS that the
            // instance's register-limited residency leaves (fewer slots rather than fewer
            // wavefronts per CU)
            const uint64_t want = (5ull * T / 3 + 63) / 64 * 64;
            p.filter_slots = static_cast<uint32_t>(std::min<uint64_t>(2ull * base_slots, std::max<uint64_t>(base_slots, want)));
            layout(0);
            const uint32_t other = p.lds_wave;
            int wg = 0;
            const hipError_t oe =
                ix->wpp <= 4 ? bsd::launch_search_rabitq(p, pl.TR, pl.CR, pl.PB, dim3(1), dim3(64), 0, nullptr, &wg)
                             : bsd::launch_search_rabitq_wide(p, pl.TR, pl.CR, pl.PB, dim3(1), dim3(64), 0, nullptr, &wg);
            if (oe == hipSuccess && wg > 0) {
                const uint32_t per_wave =
                    static_cast<uint32_t>((ix->lds_cu / static_cast<size_t>(wg)) & ~static_cast<size_t>(LDS_GRANULE - 1));
                const uint32_t fit = per_wave > other ? (per_wave - other) / 4u / 64u * 64u : 0u;
                if (fit < p.filter_slots) p.filter_slots = std::max(base_slots, fit);
            }
        }
        layout(p.filter_slots * 4u);
        if (static_cast<size_t>(p.lds_wave) * ny > ix->max_lds && p.filter_slots > base_slots) {
            p.filter_slots = base_slots;
            layout(p.filter_slots * 4u);
        }
    }
    // base mode with too few queries to give every SIMD 4 wavefronts: 2 or 4 wavefronts
    // share one query (the reference's block-per-query base kernel); they split the
    // distance rows of each expansion, the rest of the loop runs on the first wavefront.
    // Beams of 256 and more keep the first wavefront busy longer per expansion, so there
    // the split is sized to keep every query resident (the instance's measured occupancy:
    // 1M x 960, 1k queries, topk 256, 2 waves/SIMD: 4 wavefronts per query 8.2 ms, 2 per
    // query 6.8 ms); smaller beams gain more from helpers than they lose to a second round
    // of queries (topk 64 on the same data: 2.0 ms against 2.3 ms).
    p.coop = 1;
    if (mode == BS_BASE) {
        uint64_t slots = 16ull * ix->cus;
        if (pl.TR >= 4) {
            int w = 0;
            if (bsd::launch_search_hash(p, pl.TR, pl.CR, pl.PB, dim3(1), dim3(64), p.lds_wave, nullptr, &w) ==
                    hipSuccess &&
                w > 0)
                slots = static_cast<uint64_t>(w) * ix->cus;
        }
        if (nq * 4 <= slots) p.coop = 4;
        else if (nq * 2 <= slots) p.coop = 2;
    }
    pl.lds = static_cast<size_t>(p.lds_wave) * ny;
    if (pl.lds > ix->max_lds)
        return fail(BS_EINVAL, "LDS per workgroup " + std::to_string(pl.lds) + " B exceeds the device limit " +
                                   std::to_string(ix->max_lds) + " B (lower filter_capacity or queries_per_group)");
    pl.block = dim3(64 * (p.coop > 1 ? p.coop : ny));
    pl.g = p.coop > 1 ? 1u : ny;  // queries per workgroup
    const uint64_t groups = (nq + pl.g - 1) / pl.g;
    if (groups > 0x7FFFFFFFull) return fail(BS_EINVAL, "too many queries for one launch");
    pl.grid = dim3(static_cast<uint32_t>(groups));
    return BS_OK;
}

hipError_t launch(const Plan& pl, hipStream_t s) {
    switch (pl.mode) {
    case BS_GROUP_BLOOM: return bsd::launch_search_bloom(pl.p, pl.TR, pl.CR, pl.PB, pl.grid, pl.block, pl.lds, s);
    case BS_RABITQ:
        if (pl.p.wpp <= 4) return bsd::launch_search_rabitq(pl.p, pl.TR, pl.CR, pl.PB, pl.grid, pl.block, pl.lds, s);
        return bsd::launch_search_rabitq_wide(pl.p, pl.TR, pl.CR, pl.PB, pl.grid, pl.block, pl.lds, s);
    default: return bsd::launch_search_hash(pl.p, pl.TR, pl.CR, pl.PB, pl.grid, pl.block, pl.lds, s);
    }
}

// Expected cost per pivot label, for the base-family label order (order_one_cost: inside each
// XCD's run of labels the costliest go first).  CAL_ROWS rows of the index (evenly spaced
// ids) are searched as queries in base mode (topk CAL_T, K 1, filter 1024, reset 16) from the
// reference's entry point (compute_entry_point), and their iterations averaged per label: a
// property of the index's regions, independent of the queries later searched.  Config B
// (1M x 128, 10k queries, topk 256), launch by the label order 4.26 ms, with the labels of
// each run by these costs 4.05 ms (by the mean cost of the searched queries themselves 4.01;
// Spearman +0.91 between the two); the calibration takes ~6 ms once per index.  Any failure
// leaves d_lcost null, i.e. the plain label order.
constexpr uint32_t CAL_ROWS = 16384, CAL_T = 64;
void calibrate_labels(bs_index ix) {
    uint32_t entry = 0;
    if (bs_index_entry_point(ix, &entry) != BS_OK) return;
    const uint32_t m = static_cast<uint32_t>(std::min<uint64_t>({CAL_ROWS, ix->n, (8ull << 20) / ix->dim}));
    float* q = nullptr;
    float* lc = nullptr;
    uint32_t *key = nullptr, *res = nullptr, *pq = nullptr;
    hipError_t e = hipMalloc(&q, static_cast<size_t>(m) * ix->dim * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&key, m * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&res, m * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&pq, static_cast<size_t>(m) * 5 * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&lc, bso::ORDER_P * sizeof(float));
    if (e == hipSuccess) e = bso::launch_gather_rows(ix->d_vecs, ix->dstride, ix->dim, ix->n, m, q, nullptr);
    if (e == hipSuccess) {
        bso::OrderParams o;
        std::memset(&o, 0, sizeof(o));
        o.queries = q;
        o.nq = m;
        o.dim = ix->dim;
        o.pivT = ix->d_pivT;
        o.pnorm = ix->d_pnorm;
        o.key = key;
        e = bso::launch_labels(o, nullptr);
    }
    if (e == hipSuccess) {
        bs_search_cfg c;
        std::memset(&c, 0, sizeof(c));
        c.mode = BS_BASE;
        c.K = 1;
        c.topk_size = CAL_T;
        c.filter_capacity = 1024;
        c.entry_point = entry;
        c.max_iterations = 1024;
        c.reset_interval = 16;
        c.queries_per_group = 1;
        Plan pl;
        e = make_plan(ix, &c, m, pl) == BS_OK ? hipSuccess : hipErrorInvalidValue;
        if (e == hipSuccess) {
            pl.p.queries = q;
            pl.p.results = res;
            pl.p.per_query = pq;
            e = launch(pl, nullptr);
        }
    }
    if (e == hipSuccess) e = bso::launch_label_cost(key, pq, m, lc, nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    for (void* b : {static_cast<void*>(q), static_cast<void*>(key), static_cast<void*>(res), static_cast<void*>(pq)})
        if (b) (void)hipFree(b);
    if (e == hipSuccess) {
        ix->d_lcost = lc;
    } else {
        if (lc) (void)hipFree(lc);
        (void)hipGetLastError();  // the plain label order stays; the error is not the caller's
    }
}

// RaBitQ launches are ordered by predicted cost, longest first, instead of by label.  A
// query's iteration count varies (config C, topk 600, 10k queries: p50 640, p99 916, max
// 1024) and a launch of several rounds ends with its last-started long queries; locality
// gains nothing there (labels 5.65 ms, query order 5.44, measured costs longest-first 4.43).
// The signal is the exact distance of the best row a short search finds (PILOT_T keys,
// PILOT_IT iterations): Spearman +0.61 with the full search's iterations at config C (+0.74
// with 24 iterations, which order the launch no better: 4.64 ms either way; pilot 0.087 ms
// against 0.139).
constexpr uint32_t PILOT_T = 16, PILOT_IT = 12, PILOT_CAP = 64;

// The pilot search of one chunk: K = 1, distances into key[0..m) as floats (the cost order
// reads them there), ids into qmap[0..m) (overwritten by the launch map).
hipError_t launch_pilot(bs_index ix, const Plan& pl, const float* queries, uint64_t m, uint32_t* ows, hipStream_t s) {
    bs_search_cfg pc;
    std::memset(&pc, 0, sizeof(pc));
    pc.mode = BS_RABITQ;
    pc.K = 1;
    pc.topk_size = PILOT_T;
    pc.filter_capacity = PILOT_CAP;
    pc.entry_point = pl.p.entry;
    pc.max_iterations = PILOT_IT;
    pc.queries_per_group = 1;
    Plan pp;
    if (make_plan(ix, &pc, m, pp) != BS_OK) return hipErrorInvalidValue;
    pp.p.queries = queries;
    pp.p.results = ows + ORDER_CHUNK;
    pp.p.dists = reinterpret_cast<float*>(ows);
    pp.p.per_query = nullptr;
    pp.p.qmap = nullptr;
    return launch(pp, s);
}

// The search in launches of at most ORDER_CHUNK queries, each preceded by the query
// scheduling kernels that fill its launch map in `ows` (key[ORDER_CHUNK] | qmap[ORDER_CHUNK] |
// hist[P] | cursor[P], hist zero on entry): labels for base and group modes, the pilot
// search and cost order for RaBitQ.  guard: the workspace is the index's, shared by calls
// on any stream, so a launch waits for the previous one to have read it.
hipError_t launch_ordered(bs_index ix, Plan pl, uint64_t nq, hipStream_t s, uint32_t* ows, bool guard) {
    const bsd::SearchParams all = pl.p;
    const uint32_t g = pl.g, X = ix->xcds;
    const bool cost = pl.mode == BS_RABITQ;
    hipError_t e = guard ? hipStreamWaitEvent(s, ix->ws_free, 0) : hipSuccess;
    for (uint64_t c0 = 0; e == hipSuccess && c0 < nq; c0 += ORDER_CHUNK) {
        const uint64_t m = std::min(ORDER_CHUNK, nq - c0);
        bso::OrderParams o;
        std::memset(&o, 0, sizeof(o));
        o.queries = all.queries + c0 * all.dim;
        o.nq = m;
        o.dim = all.dim;
        o.pivT = ix->d_pivT;
        o.pnorm = ix->d_pnorm;
        o.key = ows;
        o.qmap = ows + ORDER_CHUNK;
        o.hist = o.qmap + ORDER_CHUNK;
        o.cursor = o.hist + bso::ORDER_P;
        o.g = g;
        o.X = X;
        o.lcost = ix->d_lcost;
        bso::order_starts(o, m);
        if (cost) {
            e = launch_pilot(ix, pl, o.queries, m, ows, s);
            if (e == hipSuccess) e = bso::launch_cost_order(o, s);
        } else {
            e = bso::launch_order(o, s);
        }
        if (e != hipSuccess) break;
        pl.p.queries = all.queries + c0 * all.dim;
        pl.p.results = all.results + c0 * all.K;
        pl.p.dists = all.dists ? all.dists + c0 * all.K : nullptr;
        pl.p.per_query = all.per_query ? all.per_query + c0 * 5 : nullptr;
        pl.p.qmap = o.qmap;
        pl.p.nq = m;
        pl.grid = dim3(static_cast<uint32_t>((m + g - 1) / g));
        e = launch(pl, s);
    }
    if (e == hipSuccess && guard) e = hipEventRecord(ix->ws_free, s);
    return e;
}

}  // namespace

extern "C" int bs_search_device(bs_index ix, const bs_search_cfg* cfg, const float* d_queries, uint64_t nq,
                                uint32_t* d_results, float* d_dists, uint32_t* d_per_query, void* stream,
                                int sync, bs_stats* stats) try {
    Plan pl;
    int rc = make_plan(ix, cfg, nq, pl);
    if (rc) return rc;
    if (nq == 0) {
        if (stats) std::memset(stats, 0, sizeof(*stats));
        return BS_OK;
    }
    if (!d_queries || !d_results) return fail(BS_EINVAL, "queries and results must be given");
    pl.p.queries = d_queries;
    pl.p.results = d_results;
    pl.p.dists = d_dists;
    pl.p.per_query = d_per_query;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (sync) {
        HIP_TRY(hipEventCreate(&e0));
        HIP_TRY(hipEventCreate(&e1));
        HIP_TRY(hipEventRecord(e0, s));
    }
    const bool order = ix->order_mode == 2 || (ix->order_mode == 1 && nq >= ORDER_MIN_NQ);
    hipError_t le = order ? launch_ordered(ix, pl, nq, s, ix->d_ows, true) : launch(pl, s);
    if (le != hipSuccess) {
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        return fail(BS_EHIP, std::string("search launch failed: ") + hipGetErrorString(le));
    }
    if (sync) {
        HIP_TRY(hipEventRecord(e1, s));
        HIP_TRY(hipEventSynchronize(e1));
        float ms = 0;
        HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        if (stats) {
            std::memset(stats, 0, sizeof(*stats));
            stats->kernel_ms = ms;
            if (d_per_query) {
                std::vector<uint32_t> pq(nq * 5);
                HIP_TRY(hipMemcpy(pq.data(), d_per_query, nq * 5 * 4, hipMemcpyDeviceToHost));
                for (uint64_t i = 0; i < nq; ++i) {
                    stats->iterations += pq[i * 5 + 0];
                    stats->expansions += pq[i * 5 + 1];
                    stats->dist_evals += pq[i * 5 + 2];
                    stats->est_evals += pq[i * 5 + 3];
                    stats->rerank_evals += pq[i * 5 + 4];
                }
            }
        }
    }
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

extern "C" int bs_search(bs_index ix, const bs_search_cfg* cfg, const float* queries, uint64_t nq,
                         uint32_t* results, float* dists, bs_stats* stats) try {
    Plan pl;
    int rc = make_plan(ix, cfg, nq, pl);
    if (rc) return rc;
    if (nq == 0) {
        if (stats) std::memset(stats, 0, sizeof(*stats));
        return BS_OK;
    }
    if (!queries || !results) return fail(BS_EINVAL, "queries and results must be given");
    // queries | results | dists | per-query counters, each 256-B aligned, in the index's
    // staging buffer (calls on one index are serialised and this one is synchronous)
    auto al = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
    const size_t qb = nq * ix->dim * sizeof(float), rb = nq * cfg->K * sizeof(uint32_t), pb = nq * 5 * 4;
    const size_t need = al(qb) + al(rb) + (dists ? al(rb) : 0) + al(pb);
    if (need > ix->stage_bytes) {
        if (ix->d_stage) (void)hipFree(ix->d_stage);
        ix->d_stage = nullptr;
        ix->stage_bytes = 0;
        if (hipMalloc(&ix->d_stage, need) != hipSuccess) {
            ix->d_stage = nullptr;
            return fail(BS_ENOMEM, "hipMalloc of the query staging buffer failed");
        }
        ix->stage_bytes = need;
    }
    char* base = static_cast<char*>(ix->d_stage);
    float* dq = reinterpret_cast<float*>(base);
    uint32_t* dr = reinterpret_cast<uint32_t*>(base + al(qb));
    float* dd = dists ? reinterpret_cast<float*>(base + al(qb) + al(rb)) : nullptr;
    uint32_t* dp = reinterpret_cast<uint32_t*>(base + al(qb) + al(rb) + (dists ? al(rb) : 0));
    hipError_t e = hipMemcpy(dq, queries, qb, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(BS_EHIP, std::string("query upload failed: ") + hipGetErrorString(e));
    bs_stats st;
    // per-query counters only when the caller asks for statistics (they cost the RaBitQ loop
    // an expanded-set lookup of every neighbour)
    rc = bs_search_device(ix, cfg, dq, nq, dr, dd, stats ? dp : nullptr, nullptr, 1, &st);
    if (rc == BS_OK) {
        e = hipMemcpy(results, dr, rb, hipMemcpyDeviceToHost);
        if (e == hipSuccess && dists) e = hipMemcpy(dists, dd, rb, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = fail(BS_EHIP, std::string("result download failed: ") + hipGetErrorString(e));
    }
    if (rc == BS_OK && stats) *stats = st;
    return rc;
} catch (...) {
    return bs_internal_exception();
}

// ---------------------------------------------------------------------------------------
// bs_search_device_noalloc: bs_search_device whose query-scheduling workspace is a static
// device array instead of the index's, so that a call allocates nothing (for callers that
// cannot allocate: code under HIP graph capture, serving loops, harnesses that forbid it).
// ---------------------------------------------------------------------------------------
// key[ORDER_CHUNK] | qmap[ORDER_CHUNK] | hist[ORDER_P] | cursor[ORDER_P]: 2 MiB + 2 KiB,
// one copy per GPU for the life of the process.  Host code never uses this name as an
// address: the device address comes from hipGetSymbolAddress (noalloc_workspace).
constexpr size_t NOALLOC_WORDS = 2 * ORDER_CHUNK + 2 * bso::ORDER_P;
static __device__ __align__(256) uint32_t scratch[NOALLOC_WORDS];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
uint32_t* g_scratch_ptr[MAX_DEVICES] = {};

// this device's address of `scratch`, looked up once per device with that device current
// (bs_index_create makes the first lookup for its device)
int noalloc_workspace(int dev, uint32_t** out) {
    if (dev < 0 || dev >= MAX_DEVICES) return fail(BS_EINVAL, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(BS_EHIP, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<uint32_t*>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return BS_OK;
}

// fill kernel for the histogram (no memset node, so the call can be captured in a graph)
__global__ void __launch_bounds__(256) clear_words(uint32_t* w, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) w[i] = 0u;
}

}  // namespace

extern "C" int bs_search_device_noalloc(bs_index ix, const bs_search_cfg* cfg, const float* d_queries, uint64_t nq,
                                        uint32_t* d_results, float* d_dists, uint32_t* d_per_query,
                                        void* stream) try {
    if (nq > ORDER_CHUNK)
        return fail(BS_EINVAL, "bs_search_device_noalloc: nq = " + std::to_string(nq) + " exceeds the " +
                                   std::to_string(ORDER_CHUNK) + " queries its static workspace holds; split the batch");
    Plan pl;
    int rc = make_plan(ix, cfg, nq, pl);
    if (rc) return rc;
    if (nq == 0) return BS_OK;
    if (!d_queries || !d_results) return fail(BS_EINVAL, "queries and results must be given");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != ix->device)
        return fail(BS_EINVAL, "the index lives on device " + std::to_string(ix->device) + ", the current device is " +
                                   std::to_string(dev));
    pl.p.queries = d_queries;
    pl.p.results = d_results;
    pl.p.dists = d_dists;
    pl.p.per_query = d_per_query;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool order = ix->order_mode == 2 || (ix->order_mode == 1 && nq >= ORDER_MIN_NQ);
    hipError_t le = hipSuccess;
    if (order) {
        uint32_t* ws = nullptr;
        rc = noalloc_workspace(dev, &ws);
        if (rc) return rc;
        // the histogram must start at zero; the previous call's contents stay otherwise
        hipLaunchKernelGGL(clear_words, dim3((bso::ORDER_P + 255) / 256), dim3(256), 0, s, ws + 2 * ORDER_CHUNK,
                           bso::ORDER_P);
        le = hipGetLastError();
        if (le == hipSuccess) le = launch_ordered(ix, pl, nq, s, ws, false);
    } else {
        le = launch(pl, s);
    }
    if (le != hipSuccess) return fail(BS_EHIP, std::string("search launch failed: ") + hipGetErrorString(le));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}
