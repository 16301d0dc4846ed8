// Query scheduling for cache locality.
//
// Queries are independent (no query reads another's state: src/gpu_cli.cu:94-95,111-112,
// 128-129), so the order in which a launch runs them changes only where their gathers
// hit.  Two queries near each other in space walk overlapping parts of the graph; run
// on the same XCD at about the same time, the second finds much of what it reads in
// that XCD's L2.  Before a search launch, each query is labelled with its nearest of
// 256 pivot rows (kept in a nearest-neighbour tour order, so neighbouring labels are
// near in space), the labels are bucket-sorted, and the sorted list is cut into one
// contiguous run per XCD.  Workgroup b runs on XCD b mod X (the dispatcher's
// round-robin), so position p of the launch (workgroup p / g, g queries per
// workgroup) is given the next query of its XCD's run.  The search kernel reads
// qmap[p] for its query and writes results at that query's own row.
#include "bs_order.hpp"
#include "wave.hpp"

namespace bso {

using namespace bsw;

// launches of up to ONE_WG queries are ordered in one workgroup after the labels (order_one,
// cost_order_one): LDS counts and placement instead of global atomics and more launches
constexpr uint64_t ONE_WG = 65536;

// The one-workgroup kernels read their queries' keys in batches of KCH loads per thread, all
// issued before any is used (a few global round trips per pass instead of one per query the
// thread handles); nothing per query stays in registers between passes (64 queries per
// thread would not fit), what a later pass needs goes back to the key array.
constexpr int KPT = static_cast<int>(ONE_WG / 1024);  // queries per thread at most
constexpr int KCH = 16;                               // loads in flight per thread

// v[j] = key of query t + 1024 (c + j) (fill for queries past nq)
__device__ __forceinline__ void load_batch(const OrderParams& o, int c, uint32_t fill, uint32_t (&v)[KCH]) {
    const uint64_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
        const uint64_t q = t + 1024ull * static_cast<uint32_t>(c + j);
        v[j] = q < o.nq ? o.key[q] : fill;
    }
}

__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Matrix-core labelling: a workgroup of 4 wavefronts takes 32 queries; wavefront w forms
// the 32 x 64 block of dot products with pivots [64w, 64w + 64) as two 32 x 32 tiles of
// v_mfma_f32_32x32x2f32 (A: lane l holds query l % 32 at dimension k0 + l / 32; B: lane l
// holds pivot l % 32 of the tile at the same dimension; accumulator register r of lane l
// is query 8(r / 4) + 4(l / 32) + r % 4, pivot l % 32).  Each query's best pivot of the
// block is found by an xor butterfly within the lane half, the four blocks meet in LDS.
__global__ void __launch_bounds__(256) order_key(const OrderParams o) {
    __shared__ uint64_t best_s[4][32];
    const uint32_t lane = lane_id(), half = lane >> 5, l32 = lane & 31u;
    const uint32_t w = uniform(threadIdx.x >> 6);
    const uint64_t q0 = static_cast<uint64_t>(blockIdx.x) * 32;
    const uint64_t qr = q0 + l32 < o.nq ? q0 + l32 : o.nq - 1;
    const float* qp = o.queries + qr * o.dim;
    const float* pp = o.pivT + 64 * w + l32;
    const uint32_t dim16 = (o.dim + 15) & ~15u;  // pivT has dim16 rows (those past dim zero)
    f32x16 acc0 = {}, acc1 = {};
    for (uint32_t kb = 0; kb < dim16; kb += 16) {
        float a[8], b0[8], b1[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {  // all loads of 8 k-steps before their products
            const uint32_t k = kb + 2 * u + half;
            const float av = qp[k < o.dim ? k : o.dim - 1];  // unconditional load, then select
            a[u] = k < o.dim ? av : 0.0f;
            b0[u] = pp[static_cast<size_t>(k) * ORDER_P];
            b1[u] = pp[static_cast<size_t>(k) * ORDER_P + 32];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u], b0[u], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u], b1[u], acc1, 0, 0, 0);
        }
    }
    const uint32_t p0 = 64 * w + l32, p1 = p0 + 32;
    const float n0 = o.pnorm[p0], n1 = o.pnorm[p1];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        // |p|^2 - 2 q.p orders the pivots as |q - p|^2 does; ties go to the lower index
        const uint64_t k0v = (static_cast<uint64_t>(orderable(__builtin_fmaf(-2.0f, acc0[r], n0))) << 32) | p0;
        const uint64_t k1v = (static_cast<uint64_t>(orderable(__builtin_fmaf(-2.0f, acc1[r], n1))) << 32) | p1;
        uint64_t b = k0v < k1v ? k0v : k1v, t;
        t = xor_lane64<1>(b); b = t < b ? t : b;
        t = xor_lane64<2>(b); b = t < b ? t : b;
        t = xor_lane64<4>(b); b = t < b ? t : b;
        t = xor_lane64<8>(b); b = t < b ? t : b;
        t = xor_lane64<16>(b); b = t < b ? t : b;
        if (l32 == static_cast<uint32_t>(r)) best_s[w][8 * (r / 4) + 4 * half + r % 4] = b;
    }
    __syncthreads();
    if (w == 0 && lane < 32 && q0 + lane < o.nq) {
        uint64_t b = best_s[0][lane];
#pragma unroll
        for (int v = 1; v < 4; ++v) b = best_s[v][lane] < b ? best_s[v][lane] : b;
        const uint32_t label = static_cast<uint32_t>(b) & (ORDER_P - 1);
        o.key[q0 + lane] = label;
        if (o.nq > ONE_WG) atomicAdd(&o.hist[label], 1u);  // below, order_one counts in LDS
    }
}

// One workgroup of ORDER_P threads: bucket starts by an exclusive scan of the label
// counts; the counts are cleared for the next launch.
__global__ void __launch_bounds__(ORDER_P) order_scan(const OrderParams o) {
    __shared__ uint32_t s[ORDER_P];
    const uint32_t t = threadIdx.x;
    const uint32_t c = o.hist[t];
    s[t] = c;
    __syncthreads();
    for (uint32_t d = 1; d < ORDER_P; d <<= 1) {
        const uint32_t v = t >= d ? s[t - d] : 0u;
        __syncthreads();
        s[t] += v;
        __syncthreads();
    }
    o.cursor[t] = s[t] - c;
    o.hist[t] = 0u;
}

// launch position of the query of label-order rank r: XCD x's run starts at rank start[x];
// XCD x runs workgroups x, x + X, ... of g queries each
__device__ __forceinline__ uint64_t order_pos(const OrderParams& o, uint32_t r) {
    uint32_t x = 0;
    while (x + 1 < o.X && o.start[x + 1] <= r) ++x;
    const uint32_t j = r - o.start[x];
    const uint64_t b = x + static_cast<uint64_t>(o.X) * (j / o.g);
    return b * o.g + j % o.g;
}

// Thread per query: its rank in label order, then its launch position.
__global__ void __launch_bounds__(256) order_place(const OrderParams o) {
    const uint64_t q = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (q >= o.nq) return;
    const uint64_t pos = order_pos(o, atomicAdd(&o.cursor[o.key[q]], 1u));
    if (pos < o.nq) o.qmap[pos] = static_cast<uint32_t>(q);
}

// Cost order.  A launch of several rounds of queries ends when its last-started queries do,
// so the queries expected to run longest go first.  key[q] holds the signal as a float;
// the 256 buckets span mean +- 2 standard deviations of the finite signals, taken over
// those within 3 standard deviations of the mean of all of them (so that a few far values
// do not squeeze the rest into a few buckets); bucket 0 = largest.
// One workgroup: the range, kept in cursor[0..1] as float bits until order_scan.
template <uint32_t NT>
__device__ __forceinline__ void cost_moments(const OrderParams& o, double clo, double chi, double* s1, double* s2,
                                             double* sn, double& mu, double& sd) {
    const uint32_t t = threadIdx.x;
    double a = 0.0, b = 0.0, n = 0.0;
    for (uint64_t q = t; q < o.nq; q += NT) {
        const double d = __uint_as_float(o.key[q]);
        if (d >= clo && d <= chi) {  // false for NaN
            a += d;
            b += d * d;
            n += 1.0;
        }
    }
    s1[t] = a;
    s2[t] = b;
    sn[t] = n;
    __syncthreads();
    for (uint32_t h = NT / 2; h > 0; h >>= 1) {
        if (t < h) {
            s1[t] += s1[t + h];
            s2[t] += s2[t + h];
            sn[t] += sn[t + h];
        }
        __syncthreads();
    }
    mu = sn[0] > 0.0 ? s1[0] / sn[0] : 0.0;
    const double var = sn[0] > 0.0 ? s2[0] / sn[0] - mu * mu : 0.0;
    sd = var > 0.0 ? sqrt(var) : 0.0;
    __syncthreads();
}

// the bucket range [lo, hi) of the signals (every thread of the workgroup gets it)
template <uint32_t NT>
__device__ __forceinline__ void cost_bounds(const OrderParams& o, double* s1, double* s2, double* sn, float& lo,
                                            float& hi) {
    const double fmax = 3.4028234663852886e38;
    double mu, sd;
    cost_moments<NT>(o, -fmax, fmax, s1, s2, sn, mu, sd);
    cost_moments<NT>(o, mu - 3.0 * sd, mu + 3.0 * sd, s1, s2, sn, mu, sd);
    lo = static_cast<float>(mu - 2.0 * sd);
    hi = static_cast<float>(mu + 2.0 * sd);
    if (!(hi > lo)) hi = lo + 1.0f;
}

// the bucket of signal d: above the range, infinite or NaN first (0), below it last
__device__ __forceinline__ uint32_t cost_bucket(float d, float lo, float hi) {
    uint32_t b = 0;
    if (d <= lo) {
        b = ORDER_P - 1;
    } else if (d < hi) {
        const float f = (hi - d) / (hi - lo) * static_cast<float>(ORDER_P);
        b = f >= static_cast<float>(ORDER_P - 1) ? ORDER_P - 1 : f >= 0.0f ? static_cast<uint32_t>(f) : 0u;
    }
    return b;
}

__global__ void __launch_bounds__(256) cost_range(const OrderParams o) {
    __shared__ double s1[256], s2[256], sn[256];
    float lo, hi;
    cost_bounds<256>(o, s1, s2, sn, lo, hi);
    if (threadIdx.x == 0) {
        o.cursor[0] = __float_as_uint(lo);
        o.cursor[1] = __float_as_uint(hi);
    }
}

// Thread per query: its bucket (in place of the signal) and the bucket counts.
__global__ void __launch_bounds__(256) cost_key(const OrderParams o) {
    const uint64_t q = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (q >= o.nq) return;
    const uint32_t b = cost_bucket(__uint_as_float(o.key[q]), __uint_as_float(o.cursor[0]), __uint_as_float(o.cursor[1]));
    o.key[q] = b;
    atomicAdd(&o.hist[b], 1u);
}

// The whole cost order in one workgroup, for launches of up to ONE_WG queries: range,
// buckets and counts in LDS, the scan, the placement (4 launches and their global atomics
// took 0.07 ms at 10k queries), with the signals in registers.  key[q] gets the bucket;
// hist and cursor are left untouched.
// cost_moments over the launch's signals, read in batches
__device__ __forceinline__ void batch_moments(const OrderParams& o, double clo, double chi, double* s1, double* s2,
                                              double* sn, double& mu, double& sd) {
    const uint32_t t = threadIdx.x;
    double a = 0.0, b = 0.0, n = 0.0;
#pragma unroll 1
    for (int c = 0; c < KPT && t + 1024ull * c < o.nq; c += KCH) {
        uint32_t v[KCH];
        load_batch(o, c, 0x7FC00000u, v);  // NaN past nq: not counted
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const double d = __uint_as_float(v[j]);
            if (d >= clo && d <= chi) {  // false for NaN
                a += d;
                b += d * d;
                n += 1.0;
            }
        }
    }
    s1[t] = a;
    s2[t] = b;
    sn[t] = n;
    __syncthreads();
    for (uint32_t h = 512; h > 0; h >>= 1) {
        if (t < h) {
            s1[t] += s1[t + h];
            s2[t] += s2[t + h];
            sn[t] += sn[t + h];
        }
        __syncthreads();
    }
    mu = sn[0] > 0.0 ? s1[0] / sn[0] : 0.0;
    const double var = sn[0] > 0.0 ? s2[0] / sn[0] - mu * mu : 0.0;
    sd = var > 0.0 ? sqrt(var) : 0.0;
    __syncthreads();
}

__global__ void __launch_bounds__(1024) cost_order_one(const OrderParams o) {
    __shared__ double s1[1024], s2[1024], sn[1024];
    __shared__ uint32_t cnt[ORDER_P], cur[ORDER_P];
    const uint32_t t = threadIdx.x;
    const double fmax = 3.4028234663852886e38;
    double mu, sd;
    batch_moments(o, -fmax, fmax, s1, s2, sn, mu, sd);
    batch_moments(o, mu - 3.0 * sd, mu + 3.0 * sd, s1, s2, sn, mu, sd);
    const float lo = static_cast<float>(mu - 2.0 * sd);
    float hi = static_cast<float>(mu + 2.0 * sd);
    if (!(hi > lo)) hi = lo + 1.0f;
    if (t < ORDER_P) cnt[t] = 0u;
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < KPT && t + 1024ull * c < o.nq; c += KCH) {
        uint32_t v[KCH];
        load_batch(o, c, 0u, v);
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const uint64_t q = t + 1024ull * (c + j);
            if (q < o.nq) {
                const uint32_t b = cost_bucket(__uint_as_float(v[j]), lo, hi);
                o.key[q] = b;
                atomicAdd(&cnt[b], 1u);
            }
        }
    }
    __syncthreads();
    if (t == 0) {
        uint32_t a = 0;
        for (uint32_t b = 0; b < ORDER_P; ++b) {
            cur[b] = a;
            a += cnt[b];
        }
    }
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < KPT && t + 1024ull * c < o.nq; c += KCH) {
        uint32_t v[KCH];
        load_batch(o, c, 0u, v);
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const uint64_t q = t + 1024ull * (c + j);
            if (q < o.nq) o.qmap[atomicAdd(&cur[v[j]], 1u)] = static_cast<uint32_t>(q);
        }
    }
}

hipError_t launch_cost_order(const OrderParams& o, hipStream_t s) {
    OrderParams c = o;
    c.X = 1;
    c.start[0] = 0;
    if (c.nq <= ONE_WG) {
        hipLaunchKernelGGL(cost_order_one, dim3(1), dim3(1024), 0, s, c);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(cost_range, dim3(1), dim3(256), 0, s, c);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(cost_key, dim3(static_cast<uint32_t>((c.nq + 255) / 256)), dim3(256), 0, s, c);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(order_scan, dim3(1), dim3(ORDER_P), 0, s, c);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(order_place, dim3(static_cast<uint32_t>((c.nq + 255) / 256)), dim3(256), 0, s, c);
    return hipGetLastError();
}

// order_scan and order_place in one workgroup, with the label counts in LDS (launches of up to
// ONE_WG queries; order_key then leaves hist alone)
__global__ void __launch_bounds__(1024) order_one(const OrderParams o) {
    __shared__ uint32_t cnt[ORDER_P], cur[ORDER_P];
    const uint32_t t = threadIdx.x;
    if (t < ORDER_P) cnt[t] = 0u;
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < KPT && t + 1024ull * c < o.nq; c += KCH) {
        uint32_t v[KCH];
        load_batch(o, c, 0u, v);
#pragma unroll
        for (int j = 0; j < KCH; ++j)
            if (t + 1024ull * (c + j) < o.nq) atomicAdd(&cnt[v[j]], 1u);
    }
    __syncthreads();
    if (t == 0) {
        uint32_t a = 0;
        for (uint32_t b = 0; b < ORDER_P; ++b) {
            cur[b] = a;
            a += cnt[b];
        }
    }
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < KPT && t + 1024ull * c < o.nq; c += KCH) {
        uint32_t v[KCH];
        load_batch(o, c, 0u, v);
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const uint64_t q = t + 1024ull * (c + j);
            if (q < o.nq) {
                const uint64_t pos = order_pos(o, atomicAdd(&cur[v[j]], 1u));
                if (pos < o.nq) o.qmap[pos] = static_cast<uint32_t>(q);
            }
        }
    }
}

// order_one with per-label expected costs.  Each XCD still gets its contiguous run of the
// label order (the same queries, so the same locality in its L2), but inside the run the
// labels go by descending expected cost (ties in label, i.e. tour, order): a launch of
// several rounds then ends with each XCD's cheapest regions instead of wherever its run
// happens to end.  A query's key in registers carries its XCD in bits 8+ between the passes.
__global__ void __launch_bounds__(1024) order_one_cost(const OrderParams o) {
    __shared__ uint32_t cnt[ORDER_P], cur[ORDER_P], lrank[ORDER_P], byrank[ORDER_P];
    __shared__ float cost[ORDER_P];
    __shared__ uint32_t off[ORDER_MAX_X * ORDER_P];
    const uint32_t t = threadIdx.x, X = o.X;
    if (t < ORDER_P) {
        cnt[t] = 0u;
        const float c = o.lcost[t];
        cost[t] = c - c == 0.0f ? c : 0.0f;  // finite, so that the ranks below are a permutation
    }
    for (uint32_t i = t; i < X * ORDER_P; i += 1024) off[i] = 0u;
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < KPT && t + 1024ull * c < o.nq; c += KCH) {
        uint32_t v[KCH];
        load_batch(o, c, 0u, v);
#pragma unroll
        for (int j = 0; j < KCH; ++j)
            if (t + 1024ull * (c + j) < o.nq) atomicAdd(&cnt[v[j]], 1u);
    }
    if (t < ORDER_P) {
        uint32_t r = 0;
        const float c = cost[t];
        for (uint32_t j = 0; j < ORDER_P; ++j) r += (cost[j] > c || (cost[j] == c && j < t)) ? 1u : 0u;
        lrank[t] = r;
    }
    __syncthreads();
    if (t < ORDER_P) byrank[lrank[t]] = t;
    if (t == 0) {
        uint32_t a = 0;
        for (uint32_t b = 0; b < ORDER_P; ++b) {
            cur[b] = a;
            a += cnt[b];
        }
    }
    __syncthreads();
    // each query's XCD: the run its rank in the label order falls in (kept in key bits 8+)
#pragma unroll 1
    for (int c = 0; c < KPT && t + 1024ull * c < o.nq; c += KCH) {
        uint32_t v[KCH];
        load_batch(o, c, 0u, v);
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const uint64_t q = t + 1024ull * (c + j);
            if (q < o.nq) {
                const uint32_t l = v[j];
                const uint32_t r = atomicAdd(&cur[l], 1u);
                uint32_t x = 0;
                while (x + 1 < X && o.start[x + 1] <= r) ++x;
                o.key[q] = l | (x << 8);
                atomicAdd(&off[x * ORDER_P + l], 1u);
            }
        }
    }
    __syncthreads();
    // inside each run, the labels in rank order
    if (t < X) {
        uint32_t a = 0;
        for (uint32_t k = 0; k < ORDER_P; ++k) {
            const uint32_t l = byrank[k];
            const uint32_t n = off[t * ORDER_P + l];
            off[t * ORDER_P + l] = a;
            a += n;
        }
    }
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < KPT && t + 1024ull * c < o.nq; c += KCH) {
        uint32_t v[KCH];
        load_batch(o, c, 0u, v);
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
            const uint64_t q = t + 1024ull * (c + j);
            if (q < o.nq) {
                const uint32_t l = v[j] & (ORDER_P - 1), x = v[j] >> 8;
                const uint32_t i = atomicAdd(&off[x * ORDER_P + l], 1u);
                const uint64_t pos = (x + static_cast<uint64_t>(X) * (i / o.g)) * o.g + i % o.g;
                if (pos < o.nq) o.qmap[pos] = static_cast<uint32_t>(q);
                o.key[q] = l;
            }
        }
    }
}

__global__ void __launch_bounds__(1024) label_cost(const uint32_t* labels, const uint32_t* per_query, uint32_t n,
                                                   float* lcost) {
    __shared__ uint32_t sum[ORDER_P], cnt[ORDER_P];
    __shared__ unsigned long long all;
    const uint32_t t = threadIdx.x;
    if (t < ORDER_P) sum[t] = cnt[t] = 0u;
    if (t == 0) all = 0ull;
    __syncthreads();
    for (uint32_t i = t; i < n; i += 1024) {
        const uint32_t l = labels[i] & (ORDER_P - 1), it = per_query[static_cast<uint64_t>(i) * 5];
        atomicAdd(&sum[l], it);
        atomicAdd(&cnt[l], 1u);
        atomicAdd(&all, static_cast<unsigned long long>(it));
    }
    __syncthreads();
    if (t < ORDER_P) {
        const float mean = n ? static_cast<float>(static_cast<double>(all) / n) : 0.0f;
        lcost[t] = cnt[t] ? static_cast<float>(static_cast<double>(sum[t]) / cnt[t]) : mean;
    }
}

__global__ void __launch_bounds__(256) gather_rows(const float* vecs, uint32_t dstride, uint32_t dim, uint64_t n,
                                                   uint32_t m, float* out) {
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (e >= static_cast<uint64_t>(m) * dim) return;
    const uint64_t i = e / dim, k = e - i * dim;
    out[e] = vecs[(i * n / m) * dstride + k];
}

hipError_t launch_place(const OrderParams& o, hipStream_t s) {
    if (o.nq > ONE_WG) return hipErrorInvalidValue;
    if (o.lcost) hipLaunchKernelGGL(order_one_cost, dim3(1), dim3(1024), 0, s, o);
    else hipLaunchKernelGGL(order_one, dim3(1), dim3(1024), 0, s, o);
    return hipGetLastError();
}

hipError_t launch_labels(const OrderParams& o, hipStream_t s) {
    if (o.nq > ONE_WG) return hipErrorInvalidValue;
    hipLaunchKernelGGL(order_key, dim3(static_cast<uint32_t>((o.nq + 31) / 32)), dim3(256), 0, s, o);
    return hipGetLastError();
}

hipError_t launch_label_cost(const uint32_t* labels, const uint32_t* per_query, uint32_t n, float* lcost,
                             hipStream_t s) {
    hipLaunchKernelGGL(label_cost, dim3(1), dim3(1024), 0, s, labels, per_query, n, lcost);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const float* vecs, uint32_t dstride, uint32_t dim, uint64_t n, uint32_t m, float* out,
                              hipStream_t s) {
    const uint64_t total = static_cast<uint64_t>(m) * dim;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(gather_rows, dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256), 0, s, vecs, dstride,
                       dim, n, m, out);
    return hipGetLastError();
}

hipError_t launch_order(const OrderParams& o, hipStream_t s) {
    hipLaunchKernelGGL(order_key, dim3(static_cast<uint32_t>((o.nq + 31) / 32)), dim3(256), 0, s, o);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (o.nq <= ONE_WG) {
        if (o.lcost) hipLaunchKernelGGL(order_one_cost, dim3(1), dim3(1024), 0, s, o);
        else hipLaunchKernelGGL(order_one, dim3(1), dim3(1024), 0, s, o);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(order_scan, dim3(1), dim3(ORDER_P), 0, s, o);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(order_place, dim3(static_cast<uint32_t>((o.nq + 255) / 256)), dim3(256), 0, s, o);
    return hipGetLastError();
}

}  // namespace bso
