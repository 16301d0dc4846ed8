// Primitive entry points: run the search kernels' device building blocks on small
// inputs so the parity tests can check each block against the CPU oracle.
#include "bs_hip.h"
#include "bs_device.hpp"
#include "bs_order.hpp"

#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

struct bs_index_s;  // opaque here; only its device pointers are needed (via bs_index_info)

namespace {

// errors of this file go through bs_last_error() as well
int dfail(int code, const std::string& msg);

template <class T>
struct DevBuf {
    T* p = nullptr;
    size_t n = 0;
    hipError_t alloc(size_t count) {
        n = count;
        return hipMalloc(&p, std::max<size_t>(1, count) * sizeof(T));
    }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

#define DTRY(call)                                                                             \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess) return dfail(BS_EHIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

}  // namespace

// shared with bs_api.hip: index device pointers
extern "C" int bs_index_info(bs_index idx, uint64_t* n, uint32_t* dim, uint32_t* degree, uint32_t* padded_dim,
                             int* has_rabitq);
int bs_internal_vecs(bs_index idx, const float** vecs, uint32_t* dstride);
void bs_internal_set_error(const std::string& msg);
int bs_internal_exception();

namespace {
int dfail(int code, const std::string& msg) {
    bs_internal_set_error(msg);
    return code;
}

}  // namespace

// ---------------------------------------------------------------------------
// L2 pairs: one wavefront per pair
// ---------------------------------------------------------------------------
template <int QMAX>
__global__ void __launch_bounds__(256) dbg_l2_kernel(const float* vecs, uint32_t dstride, const float* queries,
                                                     uint32_t dim, const uint32_t* qi, const uint32_t* ni,
                                                     uint64_t npairs, bsd::L2Shape L, float* out) {
    const uint64_t pr = static_cast<uint64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (pr >= npairs) return;
    const uint32_t lane = bsd::lane_id();
    float4 q[QMAX];
    bsd::load_query<QMAX>(queries + static_cast<uint64_t>(qi[pr]) * dim, dim, lane & (L.G - 1), L, q);
    const float d = bsd::l2_one<QMAX>(q, vecs + static_cast<uint64_t>(ni[pr]) * dstride, L);
    if (lane == 0) out[pr] = d;
}

extern "C" int bs_debug_l2(bs_index idx, const float* queries, uint64_t nq, const uint32_t* qi,
                           const uint32_t* ni, uint64_t npairs, float* out) try {
    uint64_t n = 0;
    uint32_t dim = 0, degree = 0;
    int rc = bs_index_info(idx, &n, &dim, &degree, nullptr, nullptr);
    if (rc) return rc;
    if (npairs && (!queries || !qi || !ni || !out)) return dfail(BS_EINVAL, "queries, qi, ni and out must be given");
    for (uint64_t i = 0; i < npairs; ++i)
        if (qi[i] >= nq || ni[i] >= n) return dfail(BS_EINVAL, "pair index out of range");
    if (npairs == 0) return BS_OK;
    const float* vecs = nullptr;
    uint32_t dstride = 0;
    bs_internal_vecs(idx, &vecs, &dstride);
    DevBuf<float> dq, dout;
    DevBuf<uint32_t> dqi, dni;
    DTRY(dq.alloc(nq * dim));
    DTRY(dout.alloc(npairs));
    DTRY(dqi.alloc(npairs));
    DTRY(dni.alloc(npairs));
    DTRY(hipMemcpy(dq.p, queries, nq * dim * 4, hipMemcpyHostToDevice));
    DTRY(hipMemcpy(dqi.p, qi, npairs * 4, hipMemcpyHostToDevice));
    DTRY(hipMemcpy(dni.p, ni, npairs * 4, hipMemcpyHostToDevice));
    const bsd::L2Shape L = bsd::l2_shape(dim);
    const dim3 grid(static_cast<uint32_t>((npairs + 3) / 4)), block(256);
    hipLaunchKernelGGL(dbg_l2_kernel<4>, grid, block, 0, nullptr, vecs, dstride, dq.p, dim, dqi.p, dni.p, npairs, L,
                       dout.p);
    DTRY(hipGetLastError());
    DTRY(hipMemcpy(out, dout.p, npairs * 4, hipMemcpyDeviceToHost));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

// ---------------------------------------------------------------------------
// fastscan: quantize one query and estimate nn neighbours (one wavefront)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64) dbg_fastscan_kernel(const float* query, const float* signs, uint32_t dim,
                                                          uint32_t pdim, uint32_t seed, const uint32_t* codes_nbr,
                                                          const float* factors, uint32_t nn, uint32_t degree,
                                                          float exact, uint8_t* codes_out, float* scal_out,
                                                          int32_t* sumq_out, uint32_t* raw_out, float* est_out) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    float* scr = reinterpret_cast<float*>(smem);
    uint32_t* planes = reinterpret_cast<uint32_t*>(smem + 4u * pdim);
    uint32_t* rawbuf = planes + 6u * (pdim / 32u);
    const uint32_t lane = bsd::lane_id();
    const uint32_t wpp = pdim / 32u;
    const bsd::QuantOut qo = bsd::quantize(query, signs, dim, pdim, seed, scr, planes, codes_out);
    // codes_nbr: nn neighbours of cws = max(wpp, 4) words each (the record layout).  The
    // search kernel's paths: narrow codes with nn <= 64 (one candidate register) two lanes
    // per neighbour; narrow codes with nn > 64 a neighbour per lane and register; wide codes
    // pdim / 128 lanes per neighbour.
    const bsd::QuadShape S = bsd::quad_shape(wpp, nn);
    uint4 pl[6];
    if (S.qpn == 1) {
        // narrow: the shared plane words go through LDS as in the search kernel
        uint32_t* planes4 = reinterpret_cast<uint32_t*>(smem + ((4u * pdim + 24u * wpp + 512u + 15u) & ~15u));
        bsd::store_planes4(planes, wpp, planes4);
        if (nn <= 64u) {
            const bsd::CodeHalves h = bsd::load_code_halves(codes_nbr, nn, S);
            const uint32_t r = bsd::raw_halves(planes4, h, nn);
            if (lane < nn) rawbuf[lane] = r;
        } else {
#pragma unroll
            for (int b = 0; b < 6; ++b) pl[b] = reinterpret_cast<const uint4*>(planes4)[b];
#pragma unroll
            for (uint32_t rc = 0; rc < 2; ++rc) {
                const uint32_t nb = rc * 64u + lane;
                const uint32_t r = bsd::raw_quad(pl, bsd::load_quad(codes_nbr, nb, nn, 0u, S));
                if (nb < nn) rawbuf[nb] = r;
            }
        }
        bsd::wave_sync();
    } else {
        bsd::lane_plane_quads(planes, wpp, S, pl);
        const uint32_t qi = lane & (S.qpn - 1), nl = lane >> S.qshift;
        uint4 c0[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) c0[t] = bsd::load_quad(codes_nbr, static_cast<uint32_t>(t) * S.npp + nl, nn, qi, S);
        bsd::raw_sums_wide(pl, codes_nbr, nn, S, c0, rawbuf);
    }
    for (uint32_t j = lane; j < nn; j += 64) {
        const uint32_t raw = rawbuf[j];
        raw_out[j] = raw;
        est_out[j] = bsd::estimate(raw, qo.sum_q, qo.width, qo.low, factors[j], factors[degree + j],
                                   factors[2 * degree + j], exact);
    }
    if (lane == 0) {
        scal_out[0] = qo.low;
        scal_out[1] = qo.width;
        *sumq_out = qo.sum_q;
    }
}

extern "C" int bs_debug_fastscan(const float* query, const float* signs, uint32_t dim, uint32_t seed,
                                 const uint32_t* codes_nbr, const float* factors, uint32_t nn, uint32_t degree,
                                 float exact, uint8_t* codes_out, float* scal_out, int32_t* sum_q_out,
                                 uint32_t* raw_out, float* est_out) try {
    uint32_t pdim = 1;
    while (pdim < dim) pdim <<= 1;
    if (pdim < 32 || pdim > 2048) return dfail(BS_EINVAL, "padded dim must be in 32..2048");
    if (!query || !signs || !codes_out || !scal_out || !sum_q_out || (nn && (!codes_nbr || !factors || !raw_out || !est_out)))
        return dfail(BS_EINVAL, "null buffer");
    if (nn == 0 || nn > 128 || nn > degree) return dfail(BS_EINVAL, "need 1 <= nn <= min(128, degree)");
    const uint32_t wpp = pdim / 32;
    DevBuf<float> dq, ds, dfac, dscal, dest;
    DevBuf<uint32_t> dcodes, draw;
    DevBuf<uint8_t> dco;
    DevBuf<int32_t> dsum;
    DTRY(dq.alloc(dim));
    DTRY(ds.alloc(pdim));
    DTRY(dfac.alloc(3 * degree));
    DTRY(dscal.alloc(2));
    DTRY(dest.alloc(nn));
    const uint32_t cws = bsd::quad_shape(wpp, nn).cws;
    std::vector<uint32_t> padded(static_cast<size_t>(nn) * cws, 0u);
    for (uint32_t j = 0; j < nn; ++j)
        for (uint32_t w = 0; w < wpp; ++w) padded[static_cast<size_t>(j) * cws + w] = codes_nbr[static_cast<size_t>(j) * wpp + w];
    DTRY(dcodes.alloc(padded.size()));
    DTRY(draw.alloc(nn));
    DTRY(dco.alloc(pdim));
    DTRY(dsum.alloc(1));
    DTRY(hipMemcpy(dq.p, query, dim * 4, hipMemcpyHostToDevice));
    DTRY(hipMemcpy(ds.p, signs, pdim * 4, hipMemcpyHostToDevice));
    DTRY(hipMemcpy(dfac.p, factors, 3 * degree * 4, hipMemcpyHostToDevice));
    DTRY(hipMemcpy(dcodes.p, padded.data(), padded.size() * 4, hipMemcpyHostToDevice));
    const size_t lds = ((4u * pdim + 24u * wpp + 4u * 128u + 15u) & ~15u) + 96u;
    hipLaunchKernelGGL(dbg_fastscan_kernel, dim3(1), dim3(64), lds, nullptr, dq.p, ds.p, dim, pdim, seed, dcodes.p,
                       dfac.p, nn, degree, exact, dco.p, dscal.p, dsum.p, draw.p, dest.p);
    DTRY(hipGetLastError());
    DTRY(hipMemcpy(codes_out, dco.p, pdim, hipMemcpyDeviceToHost));
    DTRY(hipMemcpy(scal_out, dscal.p, 8, hipMemcpyDeviceToHost));
    DTRY(hipMemcpy(sum_q_out, dsum.p, 4, hipMemcpyDeviceToHost));
    DTRY(hipMemcpy(raw_out, draw.p, nn * 4, hipMemcpyDeviceToHost));
    DTRY(hipMemcpy(est_out, dest.p, nn * 4, hipMemcpyDeviceToHost));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

// ---------------------------------------------------------------------------
// beam harness: merges and picks on one wavefront
// ---------------------------------------------------------------------------
template <int TR, int CR, bool RUN>
__global__ void __launch_bounds__(64) dbg_beam_kernel(uint32_t T, const uint64_t* keys, uint32_t nbatch,
                                                      uint32_t bsize, uint32_t picks, uint32_t* picked,
                                                      uint64_t* beam_out) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    uint64_t* scratch = reinterpret_cast<uint64_t*>(smem);
    const uint32_t lane = bsd::lane_id();
    uint64_t beam[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) beam[r] = bsd::EMPTY_KEY;
    bsd::BeamState st = {0u};  // kept by merge and pick
    for (uint32_t b = 0; b < nbatch; ++b) {
        uint64_t ck[CR], cm[CR];
#pragma unroll
        for (int rc = 0; rc < CR; ++rc) {
            const uint32_t j = static_cast<uint32_t>(rc) * 64u + lane;
            ck[rc] = (j < bsize) ? keys[static_cast<uint64_t>(b) * bsize + j] : bsd::EMPTY_KEY;
            cm[rc] = bsd::ballot(ck[rc] != bsd::EMPTY_KEY);
        }
        bsd::beam_merge<TR, CR>(beam, ck, cm, T, scratch, scratch + 64 * TR + 2, st);
        for (uint32_t k = 0; k < picks; ++k) {
            const uint32_t id = bsd::beam_pick<TR, RUN>(beam, st);
            if (lane == 0) picked[static_cast<uint64_t>(b) * picks + k] = id;
        }
    }
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint32_t e = static_cast<uint32_t>(r) * 64u + lane;
        if (e < T) beam_out[e] = beam[r];
    }
}

template <int TR, int CR>
static void launch_beam(int run, uint32_t T, const uint64_t* k, uint32_t nb, uint32_t bs, uint32_t picks,
                        uint32_t* pk, uint64_t* bo) {
    const size_t lds = 512u * TR + 16u + 8u * (64u + (TR > 8 ? TR : 8));  // merge scratch (+ dump slot) + aux
    if (run)
        hipLaunchKernelGGL((dbg_beam_kernel<TR, CR, true>), dim3(1), dim3(64), lds, nullptr, T, k, nb, bs, picks, pk, bo);
    else
        hipLaunchKernelGGL((dbg_beam_kernel<TR, CR, false>), dim3(1), dim3(64), lds, nullptr, T, k, nb, bs, picks, pk,
                           bo);
}

template <int TR>
static void launch_beam_c(int CR, int run, uint32_t T, const uint64_t* k, uint32_t nb, uint32_t bs, uint32_t picks,
                          uint32_t* pk, uint64_t* bo) {
    if (CR == 1) launch_beam<TR, 1>(run, T, k, nb, bs, picks, pk, bo);
    else launch_beam<TR, 2>(run, T, k, nb, bs, picks, pk, bo);
}

extern "C" int bs_debug_beam(uint32_t topk, const uint64_t* keys, uint32_t nbatch, uint32_t bsize, uint32_t picks,
                             int pick_run, uint32_t* picked, uint64_t* beam_out) try {
    if (topk == 0 || topk > 4096) return dfail(BS_EINVAL, "topk must be in 1..4096");
    if (bsize == 0 || bsize > 128) return dfail(BS_EINVAL, "bsize must be in 1..128");
    if (!beam_out || (nbatch && !keys) || (nbatch && picks && !picked)) return dfail(BS_EINVAL, "null buffer");
    DevBuf<uint64_t> dk, db;
    DevBuf<uint32_t> dp;
    const size_t nk = static_cast<size_t>(nbatch) * bsize;
    DTRY(dk.alloc(nk));
    DTRY(db.alloc(topk));
    DTRY(dp.alloc(static_cast<size_t>(nbatch) * picks));
    if (nk) DTRY(hipMemcpy(dk.p, keys, nk * 8, hipMemcpyHostToDevice));
    // the search kernel's beam sizes, with the RaBitQ ones (10 and 12 registers) above 512
    const int TR = topk <= 64 ? 1 : topk <= 128 ? 2 : topk <= 256 ? 4 : topk <= 512 ? 8 : topk <= 640 ? 10
                 : topk <= 768 ? 12 : topk <= 1024 ? 16 : topk <= 2048 ? 32 : 64;
    const int CR = bsize <= 64 ? 1 : 2;
    switch (TR) {
    case 1: launch_beam_c<1>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    case 2: launch_beam_c<2>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    case 4: launch_beam_c<4>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    case 8: launch_beam_c<8>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    case 10: launch_beam_c<10>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    case 12: launch_beam_c<12>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    case 16: launch_beam_c<16>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    case 32: launch_beam_c<32>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    default: launch_beam_c<64>(CR, pick_run, topk, dk.p, nbatch, bsize, picks, dp.p, db.p); break;
    }
    DTRY(hipGetLastError());
    DTRY(hipMemcpy(beam_out, db.p, topk * 8, hipMemcpyDeviceToHost));
    if (nbatch * picks) DTRY(hipMemcpy(picked, dp.p, static_cast<size_t>(nbatch) * picks * 4, hipMemcpyDeviceToHost));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

// ---------------------------------------------------------------------------
// sort
// ---------------------------------------------------------------------------
template <int TR>
__global__ void __launch_bounds__(64) dbg_sort_kernel(const uint64_t* keys, uint32_t n, uint64_t* out) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const uint32_t lane = bsd::lane_id();
    uint64_t v[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint32_t e = static_cast<uint32_t>(r) * 64u + lane;
        v[r] = e < n ? keys[e] : bsd::EMPTY_KEY;
    }
    bsd::sort_beam<TR>(v, reinterpret_cast<uint64_t*>(smem));  // the rerank's sort
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const uint32_t e = static_cast<uint32_t>(r) * 64u + lane;
        if (e < n) out[e] = v[r];
    }
}

extern "C" int bs_debug_sort(const uint64_t* keys, uint32_t n, uint64_t* out) try {
    if (n == 0) return BS_OK;
    if (n > 4096) return dfail(BS_EINVAL, "n must be <= 4096");
    if (!keys || !out) return dfail(BS_EINVAL, "keys and out must be given");
    DevBuf<uint64_t> dk, dout;
    DTRY(dk.alloc(n));
    DTRY(dout.alloc(n));
    DTRY(hipMemcpy(dk.p, keys, n * 8, hipMemcpyHostToDevice));
    if (n <= 64) hipLaunchKernelGGL(dbg_sort_kernel<1>, dim3(1), dim3(64), 0, nullptr, dk.p, n, dout.p);
    else if (n <= 128) hipLaunchKernelGGL(dbg_sort_kernel<2>, dim3(1), dim3(64), 0, nullptr, dk.p, n, dout.p);
    else if (n <= 256) hipLaunchKernelGGL(dbg_sort_kernel<4>, dim3(1), dim3(64), 0, nullptr, dk.p, n, dout.p);
    else if (n <= 512) hipLaunchKernelGGL(dbg_sort_kernel<8>, dim3(1), dim3(64), 0, nullptr, dk.p, n, dout.p);
    else if (n <= 1024) hipLaunchKernelGGL(dbg_sort_kernel<16>, dim3(1), dim3(64), 0, nullptr, dk.p, n, dout.p);
    else if (n <= 2048) hipLaunchKernelGGL(dbg_sort_kernel<32>, dim3(1), dim3(64), 32 * 512, nullptr, dk.p, n, dout.p);
    else hipLaunchKernelGGL(dbg_sort_kernel<64>, dim3(1), dim3(64), 64 * 512, nullptr, dk.p, n, dout.p);
    DTRY(hipGetLastError());
    DTRY(hipMemcpy(out, dout.p, n * 8, hipMemcpyDeviceToHost));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

// ---------------------------------------------------------------------------
// cost order of the RaBitQ query scheduling
// ---------------------------------------------------------------------------
extern "C" int bs_debug_cost_order(const float* signal, uint64_t n, uint32_t* qmap, uint32_t* bucket) try {
    if (n == 0) return BS_OK;
    if (n > (1u << 18)) return dfail(BS_EINVAL, "n must be <= 262144");
    if (!signal || !qmap || !bucket) return dfail(BS_EINVAL, "signal, qmap and bucket must be given");
    DevBuf<uint32_t> key, map, hist, cursor;
    DTRY(key.alloc(n));
    DTRY(map.alloc(n));
    DTRY(hist.alloc(bso::ORDER_P));
    DTRY(cursor.alloc(bso::ORDER_P));
    DTRY(hipMemcpy(key.p, signal, n * 4, hipMemcpyHostToDevice));
    DTRY(hipMemset(hist.p, 0, bso::ORDER_P * 4));
    DTRY(hipMemset(map.p, 0xFF, n * 4));
    bso::OrderParams o;
    std::memset(&o, 0, sizeof(o));
    o.nq = n;
    o.key = key.p;
    o.qmap = map.p;
    o.hist = hist.p;
    o.cursor = cursor.p;
    o.g = 1;
    o.X = 1;
    DTRY(bso::launch_cost_order(o, nullptr));
    DTRY(hipMemcpy(qmap, map.p, n * 4, hipMemcpyDeviceToHost));
    DTRY(hipMemcpy(bucket, key.p, n * 4, hipMemcpyDeviceToHost));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

extern "C" int bs_debug_label_order(const uint32_t* labels, const float* lcost, uint64_t n, uint32_t g, uint32_t X,
                                    uint32_t* qmap) try {
    if (n == 0) return BS_OK;
    if (n > 65536) return dfail(BS_EINVAL, "n must be <= 65536");
    if (g == 0 || g > 8 || X == 0 || X > bso::ORDER_MAX_X) return dfail(BS_EINVAL, "g must be in 1..8, X in 1..32");
    if (!labels || !qmap) return dfail(BS_EINVAL, "labels and qmap must be given");
    for (uint64_t i = 0; i < n; ++i)
        if (labels[i] >= bso::ORDER_P) return dfail(BS_EINVAL, "labels must be < 256");
    DevBuf<uint32_t> key, map;
    DevBuf<float> lc;
    DTRY(key.alloc(n));
    DTRY(map.alloc(n));
    DTRY(hipMemcpy(key.p, labels, n * 4, hipMemcpyHostToDevice));
    DTRY(hipMemset(map.p, 0xFF, n * 4));
    if (lcost) {
        DTRY(lc.alloc(bso::ORDER_P));
        DTRY(hipMemcpy(lc.p, lcost, bso::ORDER_P * 4, hipMemcpyHostToDevice));
    }
    bso::OrderParams o;
    std::memset(&o, 0, sizeof(o));
    o.nq = n;
    o.key = key.p;
    o.qmap = map.p;
    o.lcost = lcost ? lc.p : nullptr;
    o.g = g;
    o.X = X;
    bso::order_starts(o, n);
    DTRY(bso::launch_place(o, nullptr));
    DTRY(hipMemcpy(qmap, map.p, n * 4, hipMemcpyDeviceToHost));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

// ---------------------------------------------------------------------------
// visit filters
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64) dbg_filter_kernel(int bloom, uint32_t bits, const uint32_t* keys,
                                                        uint32_t nbatch, uint32_t bsize, uint32_t* out_new,
                                                        const uint32_t* qkeys, uint32_t nquery,
                                                        uint32_t* out_contains) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const uint32_t lane = bsd::lane_id();
    if (!bloom) {
        bsd::HashLds h;
        h.t = reinterpret_cast<uint32_t*>(smem);
        h.size = (1u << bits) >= 4u ? (1u << bits) : 4u;
        h.cap = 1u << bits;
        h.clear();
        for (uint32_t b = 0; b < nbatch; ++b) {
            const uint32_t k = lane < bsize ? keys[static_cast<uint64_t>(b) * bsize + lane] : bsd::INVALID;
            const uint32_t r = h.insert_batch(k);
            if (lane < bsize) out_new[static_cast<uint64_t>(b) * bsize + lane] = r;
        }
        for (uint32_t i0 = 0; i0 < nquery; i0 += 64) {
            const uint32_t i = i0 + lane;
            const uint64_t act = bsd::ballot(i < nquery);
            const uint64_t in = h.contains_mask(i < nquery ? qkeys[i] : bsd::INVALID, act);
            if (i < nquery) out_contains[i] = bsw::lane_in(in) ? 1u : 0u;
        }
    } else {
        bsd::BloomLds f;
        f.w = reinterpret_cast<uint32_t*>(smem);
        f.bits = bits;
        f.words = 1u << (bits - 5);
        f.mask = bits >= 32 ? 0xFFFFFFFFu : ((1u << bits) - 1);
        f.clear();
        for (uint32_t b = 0; b < nbatch; ++b) {
            uint32_t k[1] = {lane < bsize ? keys[static_cast<uint64_t>(b) * bsize + lane] : bsd::INVALID};
            uint32_t r[1];
            f.insert_batch<1>(k, r);
            if (lane < bsize) out_new[static_cast<uint64_t>(b) * bsize + lane] = r[0];
        }
        for (uint32_t i = lane; i < nquery; i += 64) out_contains[i] = f.test_lane(qkeys[i]) ? 1u : 0u;
    }
}

extern "C" int bs_debug_filter(int bloom, uint32_t capacity, const uint32_t* keys, uint32_t nbatch, uint32_t bsize,
                               uint32_t* out_new, const uint32_t* qkeys, uint32_t nquery, uint32_t* out_contains) try {
    if (bsize == 0 || bsize > 64) return dfail(BS_EINVAL, "bsize must be in 1..64");
    if ((nbatch && (!keys || !out_new)) || (nquery && (!qkeys || !out_contains))) return dfail(BS_EINVAL, "null buffer");
    uint32_t bits = 0;
    while ((1ull << bits) < capacity) ++bits;
    size_t lds;
    if (bloom) {
        if (bits < 5) bits = 5;
        lds = (size_t(1) << (bits - 5)) * 4;
    } else {
        lds = std::max<size_t>(16, (size_t(1) << bits) * 4);
    }
    if (lds > 65536) return dfail(BS_EINVAL, "capacity too large for the primitive test");
    DevBuf<uint32_t> dk, dn, dq, dc;
    const size_t nk = static_cast<size_t>(nbatch) * bsize;
    DTRY(dk.alloc(nk));
    DTRY(dn.alloc(nk));
    DTRY(dq.alloc(nquery));
    DTRY(dc.alloc(nquery));
    if (nk) DTRY(hipMemcpy(dk.p, keys, nk * 4, hipMemcpyHostToDevice));
    if (nquery) DTRY(hipMemcpy(dq.p, qkeys, nquery * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(dbg_filter_kernel, dim3(1), dim3(64), lds, nullptr, bloom, bits, dk.p, nbatch, bsize, dn.p,
                       dq.p, nquery, dc.p);
    DTRY(hipGetLastError());
    if (nk) DTRY(hipMemcpy(out_new, dn.p, nk * 4, hipMemcpyDeviceToHost));
    if (nquery) DTRY(hipMemcpy(out_contains, dc.p, nquery * 4, hipMemcpyDeviceToHost));
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}
