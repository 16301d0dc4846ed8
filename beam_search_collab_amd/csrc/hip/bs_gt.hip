// Exact brute-force k nearest neighbours on the GPU (the ground truth the recall of a
// search is scored against).  The reference has no such tool (its ground truth comes
// from HDF5 files, script/unpack.py:56-81); this is the one dense contraction near the
// search path, so it runs on the matrix cores.
//
//   gt_norms    |b_j|^2 in fp32 and max_j |b_j|^2
//   gt_select   32 queries x 32 rows per v_mfma_f32_32x32x2f32 step: a_j = |b_j|^2 - 2 q.b_j
//               (fp32), the 128 smallest (a_j, j) per (query, row split) kept in HBM with a
//               per-query threshold in registers and an LDS append buffer; each split
//               publishes its 128th value per query (an upper bound of the query's 128th
//               value over all rows) and filters by the least bound published
//   gt_refine   merge the splits' lists, exact fp64 distances of the 128 candidates summed
//               in dimension order (the host bs_groundtruth's arithmetic), order by
//               (distance, id), and a certificate: every other row j has
//               a_j >= a_C (the 128th approximate value), and |a_j + |q|^2 - d_j| <= eps, so
//               when the k-th exact distance is below a_C + |q|^2 - eps no other row can
//               be among the k nearest.  Uncertified queries are reported, not guessed.
#include "bs_hip.h"
#include "bs_device.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>

int bs_internal_vecs(bs_index idx, const float** vecs, uint32_t* dstride);
void bs_internal_set_error(const std::string& msg);
int bs_internal_exception();

namespace bsg {

using bsd::EMPTY_KEY;
using bsd::orderable;
using bsw::ballot;
using bsw::lane_id;
using bsw::readlane;
using bsw::readlane64;
using bsw::wave_sync;

constexpr uint32_t C = 128;           // candidates kept per (query, split)
constexpr uint32_t BUF = 128;         // LDS append slots per query
constexpr uint32_t FLUSH = BUF - 32;  // a buffer is merged once it holds this many keys
constexpr uint32_t LDS_WAVE = 32 * BUF * 8 + 128 * 8 + 72 * 8;  // append buffers, merge scratch

typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256) gt_norms(const float* vecs, uint64_t n, uint32_t dim, uint32_t dstride,
                                                float* bn, uint32_t* bmax_bits) {
    const uint64_t j = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    float s = 0.0f;
    if (j < n) {
        const float* r = vecs + j * dstride;
        for (uint32_t i = 0; i < dim; ++i) s = __builtin_fmaf(r[i], r[i], s);
        bn[j] = s;
    }
    s = bsw::wave_max(s);  // s >= 0, so the float order is the bit order
    if (lane_id() == 0) atomicMax(bmax_bits, __float_as_uint(s));
}

// D (32 x 32) element of accumulator register r in this lane: row (query) 8(r/4) + 4(lane/32)
// + r%4, column (base row) lane % 32 -- the v_mfma_f32_32x32x2f32 output layout, checked by
// bs_debug_mfma32.
__device__ __forceinline__ uint32_t acc_row(int r, uint32_t half) {
    return 8u * static_cast<uint32_t>(r / 4) + 4u * half + static_cast<uint32_t>(r % 4);
}

template <int KP>
__global__ void __launch_bounds__(256) gt_select(const float* vecs, uint32_t dstride, const float* bn, uint64_t n,
                                                 const float* queries, uint32_t dim, uint64_t nq, uint32_t nsplit,
                                                 uint64_t split_rows, uint64_t* topc, uint32_t* tshare) {
    constexpr int H = KP / 2;  // dimensions per lane half
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const uint32_t lane = lane_id(), wave = threadIdx.x >> 6, half = lane >> 5, l32 = lane & 31u;
    const uint64_t w = static_cast<uint64_t>(blockIdx.x) * 4 + wave;
    const uint64_t nqb = (nq + 31) / 32;
    if (w >= nqb * nsplit) return;
    // consecutive wavefronts take consecutive query blocks of the same row split, so the
    // wavefronts resident together stream the same base tiles and share them through L2
    const uint64_t qb = w % nqb, s = w / nqb;
    const uint64_t r0 = s * split_rows;
    const uint64_t r1 = std::min<uint64_t>(n, r0 + split_rows);

    char* my = smem + static_cast<size_t>(wave) * LDS_WAVE;
    uint64_t* buf = reinterpret_cast<uint64_t*>(my);
    uint64_t* mscr = reinterpret_cast<uint64_t*>(my + 32 * BUF * 8);
    uint64_t* maux = mscr + 128;

    // A operand: lane (l32, half) holds query qb*32 + l32, dimensions half*H + t
    float a[H];
    {
        const uint64_t qi = qb * 32 + l32;
        const float* qv = queries + std::min<uint64_t>(qi, nq - 1) * dim;
#pragma unroll
        for (int t = 0; t < H; ++t) {  // all loads first (clamped), then the zeroing
            const uint32_t d = half * H + static_cast<uint32_t>(t);
            a[t] = qv[d < dim ? d : 0u];
        }
#pragma unroll
        for (int t = 0; t < H; ++t) {
            const uint32_t d = half * H + static_cast<uint32_t>(t);
            if (qi >= nq || d >= dim) a[t] = 0.0f;
        }
    }
    // per accumulator register, the threshold of its query: the largest value its list
    // keeps (a float compare passes a superset of the list's key order)
    float tau[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) tau[r] = __builtin_inff();
    // lane i < 32 holds the number of keys in query i's append buffer
    uint32_t cnt = 0;
    // queries whose list has been written to HBM (each lane re-reads only what it wrote)
    uint32_t written = 0;

    // B operand: lane (l32, half) holds row tile + l32 (clamped), dimensions half*H + t
    auto load_tile = [&](uint64_t tile, float4 (&b)[H / 4], float& bnj) __attribute__((always_inline)) {
        const uint64_t j = std::min<uint64_t>(tile + l32, n - 1);
        const float4* row = reinterpret_cast<const float4*>(vecs + j * dstride);
        // chunks past the row read chunk 0 instead: the query operand is 0 in those
        // dimensions, so they add nothing, and no load waits on a condition
#pragma unroll
        for (int c = 0; c < H / 4; ++c) {
            const uint32_t c4 = half * (H / 4) + static_cast<uint32_t>(c);
            b[c] = row[4u * c4 < dstride ? c4 : 0u];
        }
        bnj = bn[j];
    };

    // merge every query buffer holding at least `need` keys into its top-C list
    auto compact = [&](uint32_t need) __attribute__((always_inline)) {
        const uint32_t mycnt = lane < 32 ? cnt : 0u;
        uint64_t todo = ballot(lane < 32 && mycnt >= need);
        while (todo) {
            const uint32_t i = static_cast<uint32_t>(__builtin_ctzll(todo));
            todo &= todo - 1;
            const uint32_t c = readlane(mycnt, i);
            const uint64_t qi = qb * 32 + i;
            if (qi < nq) {
                uint64_t* top = topc + (qi * nsplit + s) * C;
                uint64_t beam[2] = {EMPTY_KEY, EMPTY_KEY};
                const uint32_t shared = tshare[qi];  // issued with the list: one round trip
                if ((written >> i) & 1u) {
                    beam[0] = top[lane];
                    beam[1] = top[64 + lane];
                }
                written |= 1u << i;
                // one HBM round trip of the list per flush, then the buffer in runs of 64
                bsd::BeamState st = bsd::beam_state<2>(beam);
                for (uint32_t b0 = 0; b0 < c; b0 += 64) {
                    uint64_t ck[1] = {b0 + lane < c ? buf[i * BUF + b0 + lane] : EMPTY_KEY};
                    uint64_t cm[1] = {ballot(b0 + lane < c)};
                    bsd::beam_merge<2, 1, true>(beam, ck, cm, C, mscr, maux, st);
                }
                top[lane] = beam[0];
                top[64 + lane] = beam[1];
                const uint64_t last = readlane64(beam[1], 63);
                // this split's C-th value bounds the query's C-th value over all rows from
                // above; publish it, and filter by the least bound any split has published
                if (last != EMPTY_KEY && lane == 0) atomicMin(&tshare[qi], static_cast<uint32_t>(last >> 32));
                const uint32_t tk = std::min(last == EMPTY_KEY ? ~0u : static_cast<uint32_t>(last >> 32), shared);
                const float nt = tk == ~0u ? __builtin_inff() : bsd::key_dist(static_cast<uint64_t>(tk) << 32);
                const uint32_t rr = 4u * (i / 8u) + (i % 4u), hh = (i / 4u) & 1u;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (static_cast<uint32_t>(r) == rr && half == hh) tau[r] = nt;
            }
            if (lane == i) cnt = 0;
            wave_sync();
        }
    };

    auto step = [&](uint64_t tile, const float4 (&b)[H / 4], float bnj) __attribute__((always_inline)) {
        // one accumulator: a 32x32x2 f32 step occupies the matrix pipe as long as its
        // result takes, so the dependent chain costs no extra issue slots
        f32x16 acc = {};
#pragma unroll
        for (int c = 0; c < H / 4; ++c) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[4 * c + 0], b[c].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[4 * c + 1], b[c].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[4 * c + 2], b[c].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[4 * c + 3], b[c].w, acc, 0, 0, 0);
        }
        const uint64_t j = tile + l32;
        const bool whole = tile + 32 <= r1;  // wave-uniform: only a split's last tile is partial
        // Accumulator register r holds, in each lane half h, the 32 rows of one query
        // acc_row(r, h), so a register's survivors append to at most two buffers: their
        // slots come from the ballot (mbcnt within the half), not from LDS atomics.  First
        // every a_j and the survivors (independent, so they issue back to back), then the
        // wave-uniform branches, only for groups of four registers holding a survivor.
        float av[16];
        uint32_t okb = 0;
        const bool in = whole || j < r1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            av[r] = __builtin_fmaf(-2.0f, acc[r], bnj);
            okb |= (in && av[r] <= tau[r]) ? 1u << r : 0u;
        }
        const uint64_t any = ballot(okb != 0u);
        bool appended = false;
        if (any) {
            appended = true;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if (!ballot(((okb >> (4 * g)) & 15u) != 0u)) continue;
#pragma unroll
                for (int r = 4 * g; r < 4 * g + 4; ++r) {
                    const bool ok = (okb >> r) & 1u;
                    const uint64_t m = ballot(ok);
                    if (!m) continue;
                    const uint32_t m0 = static_cast<uint32_t>(m), m1 = static_cast<uint32_t>(m >> 32);
                    const uint32_t i0 = acc_row(r, 0), i1 = acc_row(r, 1);
                    const uint32_t c0 = readlane(cnt, i0), c1 = readlane(cnt, i1);  // < FLUSH: see below
                    if (ok) {
                        const uint32_t pos = half ? c1 + __builtin_amdgcn_mbcnt_hi(m1, 0u) : c0 + __builtin_amdgcn_mbcnt_lo(m0, 0u);
                        const uint32_t i = half ? i1 : i0;
                        buf[i * BUF + pos] = (static_cast<uint64_t>(orderable(av[r])) << 32) | static_cast<uint32_t>(j);
                    }
                    cnt += lane == i0 ? static_cast<uint32_t>(__builtin_popcount(m0)) : 0u;
                    cnt += lane == i1 ? static_cast<uint32_t>(__builtin_popcount(m1)) : 0u;
                }
            }
        }
        if (appended) {
            wave_sync();
            compact(FLUSH);  // every buffer holds < FLUSH keys before the next 32 rows arrive
        }
    };

    float4 bA[H / 4], bB[H / 4];
    float nA = 0.0f, nB = 0.0f;
    load_tile(r0, bA, nA);
    for (uint64_t tile = r0; tile < r1; tile += 64) {
        load_tile(tile + 32, bB, nB);  // rows past the split are loaded (clamped) and ignored
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of this tile's products
        step(tile, bA, nA);
        if (tile + 32 >= r1) break;
        load_tile(tile + 64, bA, nA);
        __builtin_amdgcn_sched_barrier(0);
        step(tile + 32, bB, nB);
    }
    compact(1);
    for (uint32_t i = 0; i < 32; ++i) {  // a list with no key at all is still written
        const uint64_t qi = qb * 32 + i;
        if (!((written >> i) & 1u) && qi < nq) {
            topc[(qi * nsplit + s) * C + lane] = EMPTY_KEY;
            topc[(qi * nsplit + s) * C + 64 + lane] = EMPTY_KEY;
        }
    }
}

// one wavefront per query: merge the split lists, exact fp64 re-score, order, certify
__global__ void __launch_bounds__(256) gt_refine(const float* vecs, uint32_t dstride, uint64_t n, const float* queries,
                                                 uint32_t dim, uint64_t nq, uint32_t nsplit, const uint64_t* topc,
                                                 uint32_t k, float bmax2, int32_t* out, uint8_t* unc,
                                                 unsigned long long* n_unc) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const uint32_t lane = lane_id(), wave = threadIdx.x >> 6;
    const uint64_t qi = static_cast<uint64_t>(blockIdx.x) * 4 + wave;
    if (qi >= nq) return;
    uint64_t* mscr = reinterpret_cast<uint64_t*>(smem) + static_cast<size_t>(wave) * 200;
    uint64_t* maux = mscr + 128;

    const uint64_t* lists = topc + qi * nsplit * C;
    uint64_t beam[2] = {lists[lane], lists[64 + lane]};
    bsd::BeamState st = bsd::beam_state<2>(beam);
    for (uint32_t s = 1; s < nsplit; ++s) {
        uint64_t ck[2] = {lists[s * C + lane], lists[s * C + 64 + lane]};
        uint64_t cm[2] = {ballot(ck[0] != EMPTY_KEY), ballot(ck[1] != EMPTY_KEY)};
        bsd::beam_merge<2, 2, false>(beam, ck, cm, C, mscr, maux, st);
    }
    const uint64_t kc = readlane64(beam[1], 63);  // the C-th approximate key

    // exact distances, dimension order, fp64 (bs_groundtruth's l2d)
    const float* qv = queries + qi * dim;
    double dd[2];
    uint32_t id[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        id[r] = beam[r] == EMPTY_KEY ? 0xFFFFFFFFu : static_cast<uint32_t>(beam[r]);
        const float* row = vecs + static_cast<uint64_t>(id[r] == 0xFFFFFFFFu ? 0u : id[r]) * dstride;
        double acc = 0.0;
        for (uint32_t i = 0; i < dim; ++i) {
            const double diff = __dsub_rn(static_cast<double>(qv[i]), static_cast<double>(row[i]));
            acc = __dadd_rn(acc, __dmul_rn(diff, diff));
        }
        dd[r] = id[r] == 0xFFFFFFFFu ? __builtin_inf() : acc;
    }
    // rank of each candidate in (distance, id) order
    uint32_t rank[2] = {0, 0};
    for (uint32_t e = 0; e < C; ++e) {
        const uint64_t vb = readlane64(static_cast<uint64_t>(__double_as_longlong(e < 64 ? dd[0] : dd[1])), e & 63u);
        const uint32_t ve = readlane(e < 64 ? id[0] : id[1], e & 63u);
        const double de = __longlong_as_double(static_cast<long long>(vb));
#pragma unroll
        for (int r = 0; r < 2; ++r) rank[r] += (de < dd[r] || (de == dd[r] && ve < id[r])) ? 1u : 0u;
    }
    // valid candidates take ranks 0..nvalid-1; the slots from nvalid to k get -1
    int32_t* o = out + qi * k;
    const uint32_t nvalid = static_cast<uint32_t>(__builtin_popcountll(ballot(id[0] != 0xFFFFFFFFu)) +
                                                  __builtin_popcountll(ballot(id[1] != 0xFFFFFFFFu)));
    for (uint32_t t = nvalid + lane; t < k; t += 64) o[t] = -1;
#pragma unroll
    for (int r = 0; r < 2; ++r)
        if (id[r] != 0xFFFFFFFFu && rank[r] < k) o[rank[r]] = static_cast<int32_t>(id[r]);

    // certificate
    bool ok = true;
    if (kc != EMPTY_KEY && k <= C) {
        double dk = 0.0;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint64_t m = ballot(rank[r] == k - 1);
            if (m) dk = __longlong_as_double(static_cast<long long>(
                           readlane64(static_cast<uint64_t>(__double_as_longlong(dd[r])), __builtin_ctzll(m))));
        }
        double qn2 = 0.0;
        for (uint32_t i = 0; i < dim; ++i) qn2 += static_cast<double>(qv[i]) * static_cast<double>(qv[i]);
        const double ac = static_cast<double>(bsd::key_dist(kc));
        const double qb = __builtin_sqrt(qn2) + __builtin_sqrt(static_cast<double>(bmax2));
        const double eps = 2.0 * (dim + 3) * 0x1p-24 * qb * qb;
        ok = dk < ac + qn2 - eps;
    }
    if (lane == 0) {
        if (unc) unc[qi] = ok ? 0 : 1;
        if (!ok) atomicAdd(n_unc, 1ull);
    }
}

// v_mfma_f32_32x32x2f32 layout check: A 32x2, B 2x32 given row-major; D 32x32 row-major
__global__ void __launch_bounds__(64) dbg_mfma32(const float* A, const float* B, float* D) {
    const uint32_t lane = lane_id(), half = lane >> 5, l32 = lane & 31u;
    f32x16 acc = {};
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(A[l32 * 2 + half], B[half * 32 + l32], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) D[acc_row(r, half) * 32 + l32] = acc[r];
}

}  // namespace bsg

namespace {
int gfail(int code, const std::string& msg) {
    bs_internal_set_error(msg);
    return code;
}
#define GTRY(call)                                                                                    \
    do {                                                                                              \
        hipError_t e_ = (call);                                                                       \
        if (e_ != hipSuccess) return gfail(BS_EHIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

template <int KP>
hipError_t launch_select(dim3 g, hipStream_t s, const float* vecs, uint32_t dstride, const float* bn, uint64_t n,
                         const float* q, uint32_t dim, uint64_t nq, uint32_t nsplit, uint64_t split_rows,
                         uint64_t* topc, uint32_t* tshare) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(bsg::gt_select<KP>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 4 * bsg::LDS_WAVE);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(bsg::gt_select<KP>, g, dim3(256), 4 * bsg::LDS_WAVE, s, vecs, dstride, bn, n, q, dim, nq,
                       nsplit, split_rows, topc, tshare);
    return hipGetLastError();
}
}  // namespace

extern "C" int bs_index_groundtruth_device(bs_index idx, const float* d_queries, uint64_t nq, uint32_t k,
                                           int32_t* d_out, uint8_t* d_uncertified, void* stream,
                                           uint64_t* n_uncertified) try {
    const float* vecs = nullptr;
    uint32_t dstride = 0;
    int rc = bs_internal_vecs(idx, &vecs, &dstride);
    if (rc) return rc;
    uint64_t n = 0;
    uint32_t dim = 0;
    rc = bs_index_info(idx, &n, &dim, nullptr, nullptr, nullptr);
    if (rc) return rc;
    if (k == 0 || k > bsg::C) return gfail(BS_EINVAL, "k must be in 1..128");
    if (dim > 256) return gfail(BS_EINVAL, "the device ground truth supports dim <= 256");
    if (nq == 0) return BS_OK;
    if (!d_queries || !d_out) return gfail(BS_EINVAL, "queries and output must be given");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int KP = dim <= 64 ? 64 : dim <= 128 ? 128 : dim <= 192 ? 192 : 256;
    const uint64_t nqb = (nq + 31) / 32;
    // about 4096 wavefronts in flight: split the rows among them (>= 32 rows each)
    uint64_t nsplit = std::max<uint64_t>(1, std::min<uint64_t>(256, 4096 / nqb));
    uint64_t split_rows = ((n + nsplit - 1) / nsplit + 31) / 32 * 32;
    nsplit = (n + split_rows - 1) / split_rows;

    float* bn = nullptr;
    uint32_t* bmax = nullptr;
    uint64_t* topc = nullptr;
    uint32_t* tshare = nullptr;
    unsigned long long* nunc = nullptr;
    auto release = [&]() {
        if (bn) (void)hipFree(bn);
        if (bmax) (void)hipFree(bmax);
        if (topc) (void)hipFree(topc);
        if (tshare) (void)hipFree(tshare);
        if (nunc) (void)hipFree(nunc);
    };
    if (hipMalloc(&bn, n * sizeof(float)) != hipSuccess || hipMalloc(&bmax, 4) != hipSuccess ||
        hipMalloc(&topc, nq * nsplit * bsg::C * 8) != hipSuccess || hipMalloc(&nunc, 8) != hipSuccess ||
        hipMalloc(&tshare, nq * 4) != hipSuccess) {
        release();
        return gfail(BS_ENOMEM, "hipMalloc of the ground-truth work buffers failed");
    }
    hipError_t e = hipMemsetAsync(bmax, 0, 4, s);
    if (e == hipSuccess) e = hipMemsetAsync(nunc, 0, 8, s);
    if (e == hipSuccess) e = hipMemsetAsync(tshare, 0xFF, nq * 4, s);  // no bound published yet
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsg::gt_norms, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, vecs, n, dim,
                           dstride, bn, bmax);
        e = hipGetLastError();
    }
    uint32_t bmax_host = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&bmax_host, bmax, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    float bmax2 = 0.0f;
    std::memcpy(&bmax2, &bmax_host, 4);
    if (e == hipSuccess) {
        const dim3 g(static_cast<uint32_t>((nqb * nsplit + 3) / 4));
        switch (KP) {
        case 64: e = launch_select<64>(g, s, vecs, dstride, bn, n, d_queries, dim, nq, nsplit, split_rows, topc, tshare); break;
        case 128: e = launch_select<128>(g, s, vecs, dstride, bn, n, d_queries, dim, nq, nsplit, split_rows, topc, tshare); break;
        case 192: e = launch_select<192>(g, s, vecs, dstride, bn, n, d_queries, dim, nq, nsplit, split_rows, topc, tshare); break;
        default: e = launch_select<256>(g, s, vecs, dstride, bn, n, d_queries, dim, nq, nsplit, split_rows, topc, tshare); break;
        }
    }
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsg::gt_refine, dim3(static_cast<uint32_t>((nq + 3) / 4)), dim3(256), 4 * 200 * 8, s, vecs,
                           dstride, n, d_queries, dim, nq, static_cast<uint32_t>(nsplit), topc, k,
                           bmax2, d_out, d_uncertified, nunc);
        e = hipGetLastError();
    }
    unsigned long long nu = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&nu, nunc, 8, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    release();
    if (e != hipSuccess) return gfail(BS_EHIP, std::string("ground truth: ") + hipGetErrorString(e));
    if (n_uncertified) *n_uncertified = nu;
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

extern "C" int bs_index_groundtruth(bs_index idx, const float* queries, uint64_t nq, uint32_t k, int32_t* out,
                                    uint8_t* uncertified, uint64_t* n_uncertified) try {
    if (nq == 0) {
        if (n_uncertified) *n_uncertified = 0;
        return BS_OK;
    }
    uint32_t dim = 0;
    int rc = bs_index_info(idx, nullptr, &dim, nullptr, nullptr, nullptr);
    if (rc) return rc;
    if (!queries || !out) return gfail(BS_EINVAL, "queries and output must be given");
    float* dq = nullptr;
    int32_t* dout = nullptr;
    uint8_t* dunc = nullptr;
    auto release = [&]() {
        if (dq) (void)hipFree(dq);
        if (dout) (void)hipFree(dout);
        if (dunc) (void)hipFree(dunc);
    };
    if (hipMalloc(&dq, nq * dim * 4) != hipSuccess || hipMalloc(&dout, nq * k * 4) != hipSuccess ||
        hipMalloc(&dunc, nq) != hipSuccess) {
        release();
        return gfail(BS_ENOMEM, "hipMalloc of the ground-truth buffers failed");
    }
    if (hipMemcpy(dq, queries, nq * dim * 4, hipMemcpyHostToDevice) != hipSuccess) {
        release();
        return gfail(BS_EHIP, "query upload failed");
    }
    rc = bs_index_groundtruth_device(idx, dq, nq, k, dout, dunc, nullptr, n_uncertified);
    if (rc == BS_OK) {
        hipError_t e = hipMemcpy(out, dout, nq * k * 4, hipMemcpyDeviceToHost);
        if (e == hipSuccess && uncertified) e = hipMemcpy(uncertified, dunc, nq, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = gfail(BS_EHIP, std::string("result download failed: ") + hipGetErrorString(e));
    }
    release();
    return rc;
} catch (...) {
    return bs_internal_exception();
}

extern "C" int bs_debug_mfma32(const float* A, const float* B, float* D) try {
    float *dA = nullptr, *dB = nullptr, *dD = nullptr;
    auto release = [&]() {
        if (dA) (void)hipFree(dA);
        if (dB) (void)hipFree(dB);
        if (dD) (void)hipFree(dD);
    };
    if (hipMalloc(&dA, 64 * 4) != hipSuccess || hipMalloc(&dB, 64 * 4) != hipSuccess ||
        hipMalloc(&dD, 1024 * 4) != hipSuccess) {
        release();
        return gfail(BS_ENOMEM, "hipMalloc failed");
    }
    hipError_t e = hipMemcpy(dA, A, 64 * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dB, B, 64 * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsg::dbg_mfma32, dim3(1), dim3(64), 0, nullptr, dA, dB, dD);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(D, dD, 1024 * 4, hipMemcpyDeviceToHost);
    release();
    if (e != hipSuccess) return gfail(BS_EHIP, std::string("mfma check: ") + hipGetErrorString(e));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}
