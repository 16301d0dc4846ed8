// Index preparation on the device: the search entry point and the RaBitQ codebook.
//
// compute_entry_point (src/gpu_cli.cu:55-83): a float centroid accumulated row after row
// (centroid[d] += row[d] * inv, inv = 1 / n), then the first row of least float squared
// distance to it (diff = row[d] - centroid[d]; dist += diff * diff, dimensions in order;
// a row replaces the best only if dist < best, starting from FLT_MAX and row 0).  The
// float roundings of both loops are reproduced exactly, so the node is the reference's.
//
// build_rabitq (src/build_rabitq.cpp:59-99,138-264): the same two steps in double for the
// codebook's medoid, every node's rotation WHT(signs * [v, 0...]) once, then a thread per
// edge for the residual, its 1-bit code and the float parts of its factors, in the
// reference's operation order; the three factor products, which the reference forms in
// long double, are finished on the host.
#include "bs_hip.h"
#include "wave.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

int bs_internal_vecs(bs_index idx, const float** vecs, uint32_t* dstride);
int bs_internal_edges(bs_index idx, const uint32_t** edges);
void bs_internal_set_error(const std::string& msg);
int bs_internal_exception();

namespace bsp {

using namespace bsw;

constexpr uint32_t EP_COLS = 16;                        // dimensions per workgroup
constexpr uint32_t EP_ROWS = 1024;                      // rows per LDS chunk
constexpr uint32_t EP_S = EP_ROWS + 4;                  // floats per column of a chunk (see entry_centroid)
constexpr uint32_t EP_THREADS = 1024;                   // wavefront 0 adds, the other 15 stage rows
constexpr uint32_t EP_STAGERS = EP_THREADS / 64 - 1;
constexpr uint32_t EP_GROUPS = EP_ROWS / 16;            // 16-row groups per chunk
constexpr uint32_t EP_GPW = (EP_GROUPS + EP_STAGERS - 1) / EP_STAGERS;  // groups per staging wavefront
constexpr size_t EP_LDS = (2 * EP_COLS * EP_S + 32) * sizeof(float);  // two chunks + 32 spare: 128.6 KB

__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// LDS reads issued outside the compiler's view, for a software pipeline it would otherwise
// restructure.  The compiler does not count them, so every result is claimed through
// lgkm_wait (at most N LDS operations of this wavefront still outstanding, the register
// tied to the wait so no use moves above it) or lgkm_drain before it is read or its
// registers are reused.  LDS returns in issue order, so waiting down to N completes all
// but the N most recent of these reads (scalar loads the compiler has in flight only make
// the wait longer).  The compiler must not copy such a register before its wait: the
// generated code reads each one in place, and the entry-point tests compare the centroid's
// node bit for bit with the host restatement.
__device__ __forceinline__ uint32_t lds_address(const float* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) float*)p));
}
using f32x4 = float __attribute__((ext_vector_type(4)));
template <int OFF>
__device__ __forceinline__ void lds_read_b128(f32x4& v, uint32_t addr) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
}
template <int N>
__device__ __forceinline__ void lgkm_wait(f32x4& a, f32x4& b, f32x4& c, f32x4& d) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N) : "memory");
}
__device__ __forceinline__ void lgkm_drain(f32x4 (&w)[8]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7])
                 :
                 : "memory");
}

// The centroid is one dependent chain of n additions per dimension, so the only
// parallelism is across dimensions, and a wavefront's chain costs the same whatever the
// number of its lanes that take part (about 6 cycles per dependent v_add).  Workgroup x
// owns the 16 dimensions [16x, 16x + 16) (so a 128-dimensional set keeps 8 CUs busy and
// each CU needs only 64 bytes per row); its first wavefront adds (dimension = lane % 16),
// one v_add per row and one ds_read_b128 per four rows, while the other 15 wavefronts keep
// it fed.  Chunks of EP_ROWS rows are stored column-major in LDS (a column's rows
// contiguous, columns EP_S floats apart, so 16 lanes hit 16 distinct 4-bank groups), two chunks in LDS and two
// more in flight in the stagers' registers: loads are issued two chunks ahead, so their
// latency overlaps two chunks of additions.  A stager lane (r, k) = (lane / 16, lane % 16)
// loads rows 4r..4r+3 of a 16-row group in column k, one row per load instruction (a
// wavefront instruction covers 4 rows x 64 bytes), and stores them with one ds_write_b128.
// In float mode the stagers form the products row[d] * inv, so the chain is additions only.
//   float:  c += row[d] * inv                       (compute_entry_point)
//   double: c += (double)row[d], then c / n         (find_medoid)
template <typename T>
__global__ void __launch_bounds__(EP_THREADS) entry_centroid(const float* vecs, uint64_t n, uint32_t dim,
                                                            uint32_t dstride, float inv, T* cent,
                                                            unsigned long long* best) {
    extern __shared__ __attribute__((aligned(16))) float buf[];  // [2][EP_COLS][EP_S], 32 spare
    const uint32_t lane = lane_id(), wave = uniform(threadIdx.x >> 6);
    const uint32_t k = lane & (EP_COLS - 1), rq = lane / EP_COLS;
    const uint32_t col = blockIdx.x * EP_COLS + k;
    const uint64_t nchunk = (n + EP_ROWS - 1) / EP_ROWS;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        // float: the key (FLT_MAX, row 0); double: the distance bits of DBL_MAX
        if constexpr (sizeof(T) == 4) *best = static_cast<unsigned long long>(orderable(FLT_MAX)) << 32;
        else *best = static_cast<unsigned long long>(__double_as_longlong(DBL_MAX));
    }
    // stager wavefront w (1..15) owns the 16-row groups g = (w - 1) + 15 j of every chunk
    const uint32_t sw = wave - 1;
    float ra[EP_GPW * 4], rb[EP_GPW * 4];
    // Every load is issued unconditionally (a fixed number per chunk, so the compiler waits
    // for exactly the older chunk), with rows past n clamped to n - 1 and columns past dim to
    // dim - 1: the adding wavefront never reads those rows nor writes those columns.
    const uint32_t coff = (col < dim ? col : dim - 1) * 4u;
    const uint32_t rowbytes = dstride * 4u;  // dstride <= 1024: a chunk spans at most 4 MB
    auto load = [&](uint64_t c, float (&r)[EP_GPW * 4]) __attribute__((always_inline)) {
        const uint64_t row0 = std::min<uint64_t>(c * EP_ROWS, n - 1);
        const uint32_t last = static_cast<uint32_t>(std::min<uint64_t>(n - 1 - row0, EP_ROWS - 1));
        const char* base = reinterpret_cast<const char*>(vecs + row0 * dstride) + coff;
#pragma unroll
        for (uint32_t j = 0; j < EP_GPW; ++j) {
            const uint32_t g = sw + j * EP_STAGERS;
#pragma unroll
            for (uint32_t t = 0; t < 4; ++t) {
                const uint32_t rr = std::min(16 * g + 4 * rq + t, last);
                r[4 * j + t] = *reinterpret_cast<const float*>(base + static_cast<uint64_t>(rr) * rowbytes);
            }
        }
    };
    auto store = [&](uint32_t h, const float (&r)[EP_GPW * 4]) __attribute__((always_inline)) {
        float* dst = buf + (h * EP_COLS + k) * EP_S + 4 * rq;
#pragma unroll
        for (uint32_t j = 0; j < EP_GPW; ++j) {
            const uint32_t g = sw + j * EP_STAGERS;
            if (g < EP_GROUPS) {
                float4 v = make_float4(r[4 * j], r[4 * j + 1], r[4 * j + 2], r[4 * j + 3]);
                if constexpr (sizeof(T) == 4) v = make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv);
                *reinterpret_cast<float4*>(dst + 16 * g) = v;
            }
        }
    };
    T s = 0;
    // The adding wavefront keeps eight ds_read_b128 (32 rows) in flight: each half block
    // of 16 rows is added, then its registers take the 16 rows 32 rows further on.  All 64 lanes
    // run the chain (lanes 16-63 repeat lanes 0-15: a partly masked wavefront adds slower).  The compiler turns such a
    // rotation of plain loads back into load-then-use blocks (one LDS latency per 32 rows),
    // so the reads are issued by lds_read_b128 and waited for by lgkm_wait; the reads of
    // the last block run past the column's rows into the next column or the 32 spare floats
    // at the end of the buffer, and are drained, never added.
    auto consume = [&](uint64_t c, uint32_t h) __attribute__((always_inline)) {
        const float* src = buf + (h * EP_COLS + k) * EP_S;
        const uint32_t rows = static_cast<uint32_t>(n - c * EP_ROWS < EP_ROWS ? n - c * EP_ROWS : EP_ROWS);
        const uint32_t nblk = rows / 32;
        uint32_t addr = lds_address(src);
        f32x4 w[8];
        lds_read_b128<0>(w[0], addr);
        lds_read_b128<16>(w[1], addr);
        lds_read_b128<32>(w[2], addr);
        lds_read_b128<48>(w[3], addr);
        lds_read_b128<64>(w[4], addr);
        lds_read_b128<80>(w[5], addr);
        lds_read_b128<96>(w[6], addr);
        lds_read_b128<112>(w[7], addr);
        for (uint32_t b = 0; b < nblk; ++b) {
            addr += 128;
#define BSP_ADD(v)                                  \
    s = s + static_cast<T>(v.x);                    \
    s = s + static_cast<T>(v.y);                    \
    s = s + static_cast<T>(v.z);                    \
    s = s + static_cast<T>(v.w);
            lgkm_wait<4>(w[0], w[1], w[2], w[3]);
            BSP_ADD(w[0]) BSP_ADD(w[1]) BSP_ADD(w[2]) BSP_ADD(w[3])
            lds_read_b128<0>(w[0], addr);
            lds_read_b128<16>(w[1], addr);
            lds_read_b128<32>(w[2], addr);
            lds_read_b128<48>(w[3], addr);
            lgkm_wait<4>(w[4], w[5], w[6], w[7]);
            BSP_ADD(w[4]) BSP_ADD(w[5]) BSP_ADD(w[6]) BSP_ADD(w[7])
            lds_read_b128<64>(w[4], addr);
            lds_read_b128<80>(w[5], addr);
            lds_read_b128<96>(w[6], addr);
            lds_read_b128<112>(w[7], addr);
#undef BSP_ADD
        }
        lgkm_drain(w);
        for (uint32_t r = 32 * nblk; r < rows; ++r) s = s + static_cast<T>(src[r]);
    };
    // prologue: chunk 0 into LDS half 0, chunk 1 held in rb, chunk 2 in flight into ra
    if (wave != 0) {
        load(0, ra);
        load(1, rb);
        store(0, ra);
        load(2, ra);
    }
    __syncthreads();
    // chunk c is in LDS half c & 1; while it is added, the stagers store chunk c + 1 into
    // the other half and issue the loads of chunk c + 3 into the registers they freed
    // (past the last chunk the stagers go on storing into the half that is not being read
    // and loading clamped rows; nothing reads them)
    for (uint64_t c = 0; c < nchunk; c += 2) {
        if (wave == 0) {
            consume(c, 0);
        } else {
            store(1, rb);
            load(c + 3, rb);
        }
        __syncthreads();
        if (c + 1 >= nchunk) break;
        if (wave == 0) {
            consume(c + 1, 1);
        } else {
            store(0, ra);
            load(c + 4, ra);
        }
        __syncthreads();
    }
    if constexpr (sizeof(T) == 8) s = s / static_cast<double>(n);
    if (wave == 0 && lane < EP_COLS && col < dim) cent[col] = s;
}

// Distance of every row to the centroid in dimension order, as the reference's loops form it
// (float: diff = row[d] - c[d], dist += diff * diff; double: the same with row[d] widened).
// A wavefront owns 64 rows, a lane one row's dependent chain of dim steps.  Its rows pass
// through a wavefront-private LDS tile of 64 rows x 64 dimensions: loaded coalesced (16
// lanes per row, a float4 each, 4 rows per load instruction, every tile's loads in flight
// together), stored row-major with rows EP_TS floats apart (16 lanes of a b128 phase hit 16
// distinct 4-bank groups), then each lane reads its own row back one float4 at a time.
//   float:  the least (orderable dist, row) with dist < FLT_MAX by a 64-bit atomic minimum
//   double: every row's dist, and the least distance bits (non-negative doubles order as
//           their bit patterns); medoid_index then takes the least row at that distance
constexpr uint32_t EP_TS = 64 + 4;
constexpr size_t ND_LDS = 4 * 64 * EP_TS * sizeof(float);  // four wavefronts' tiles

template <typename T>
__global__ void __launch_bounds__(256) row_dist(const float* vecs, uint64_t n, uint32_t dim, uint32_t dstride,
                                                const T* cent, T* dist, unsigned long long* best) {
    __shared__ T c[1024];
    extern __shared__ __attribute__((aligned(16))) float tiles[];
    for (uint32_t k = threadIdx.x; k < dim; k += 256) c[k] = cent[k];
    __syncthreads();
    const uint32_t lane = lane_id(), wave = uniform(threadIdx.x >> 6);
    const uint64_t r0 = (static_cast<uint64_t>(blockIdx.x) * 4 + wave) * 64;
    if (r0 >= n) return;  // wavefront-uniform: no barrier follows
    float* tile = tiles + wave * 64 * EP_TS;
    // loader role: row r0 + 4 i + lane / 16 (clamped to n - 1), columns 4 (lane % 16) + 0..3
    const uint32_t lr = lane >> 4, lc = (lane & 15u) * 4;
    const uint64_t i = r0 + lane;
    T s = 0;
    for (uint32_t d0 = 0; d0 < dim; d0 += 64) {
        f32x4 v[16];
#pragma unroll
        for (uint32_t t = 0; t < 16; ++t) {
            const uint64_t row = std::min<uint64_t>(r0 + 4 * t + lr, n - 1);
            // columns at or past dim are never added; they read column 0 of the row
            const uint32_t cc = d0 + lc < dim ? d0 + lc : 0u;
            v[t] = *reinterpret_cast<const f32x4*>(vecs + row * dstride + cc);
        }
        wave_sync();  // the previous tile's reads are done before it is overwritten
#pragma unroll
        for (uint32_t t = 0; t < 16; ++t) *reinterpret_cast<f32x4*>(tile + (4 * t + lr) * EP_TS + lc) = v[t];
        wave_sync();
        const float* mine = tile + lane * EP_TS;
        const uint32_t cols = dim - d0 < 64 ? dim - d0 : 64;
        uint32_t k = 0;
        for (; k + 4 <= cols; k += 4) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(mine + k);
            T e = static_cast<T>(x.x) - c[d0 + k];
            s = s + e * e;
            e = static_cast<T>(x.y) - c[d0 + k + 1];
            s = s + e * e;
            e = static_cast<T>(x.z) - c[d0 + k + 2];
            s = s + e * e;
            e = static_cast<T>(x.w) - c[d0 + k + 3];
            s = s + e * e;
        }
        for (; k < cols; ++k) {
            const T e = static_cast<T>(mine[k]) - c[d0 + k];
            s = s + e * e;
        }
    }
    unsigned long long key = ~0ull;
    if (i < n) {
        if constexpr (sizeof(T) == 4) {
            if (s < FLT_MAX) key = (static_cast<unsigned long long>(orderable(s)) << 32) | i;
        } else {
            dist[i] = s;
            if (s < DBL_MAX) key = static_cast<unsigned long long>(__double_as_longlong(s));
        }
    }
    unsigned long long t;
    t = xor_lane64<1>(key); key = t < key ? t : key;
    t = xor_lane64<2>(key); key = t < key ? t : key;
    t = xor_lane64<4>(key); key = t < key ? t : key;
    t = xor_lane64<8>(key); key = t < key ? t : key;
    t = xor_lane64<16>(key); key = t < key ? t : key;
    t = xor_lane64<32>(key); key = t < key ? t : key;
    if (lane == 0 && key != ~0ull) atomicMin(best, key);
}

__global__ void __launch_bounds__(256) medoid_index(uint64_t n, const double* dist, const unsigned long long* best,
                                                    uint32_t* index) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    const unsigned long long b = *best;  // still DBL_MAX: no row qualified
    if (i < n && b != static_cast<unsigned long long>(__double_as_longlong(DBL_MAX)) &&
        static_cast<unsigned long long>(__double_as_longlong(dist[i])) == b)
        atomicMin(index, static_cast<uint32_t>(i));
}

// rotate_vector (build_rabitq.cpp:19-55): r = WHT(signs * [v, 0...]), one wavefront per
// node in LDS.  Stage len pairs (a, a + len) for a with bit len clear; the pairs of a
// stage are disjoint, so any lane order gives the sequential loop's values.
__global__ void __launch_bounds__(256) rq_rotate(const float* vecs, uint32_t dstride, uint64_t n, uint32_t dim,
                                                 uint32_t pdim, const float* signs, float* rot) {
    extern __shared__ float sh[];
    const uint32_t lane = lane_id(), w = uniform(threadIdx.x >> 6);
    const uint64_t u = static_cast<uint64_t>(blockIdx.x) * 4 + w;
    if (u >= n) return;
    float* x = sh + w * pdim;
    for (uint32_t d = lane; d < pdim; d += 64) x[d] = d < dim ? vecs[u * dstride + d] * signs[d] : 0.0f;
    wave_sync();
    for (uint32_t len = 1; len < pdim; len <<= 1) {
        for (uint32_t t = lane; t < pdim / 2; t += 64) {
            const uint32_t a = (t / len) * 2 * len + (t % len), b = a + len;
            const float xa = x[a], xb = x[b];
            x[a] = xa + xb;
            x[b] = xa - xb;
        }
        wave_sync();
    }
    for (uint32_t d = lane; d < pdim; d += 64) rot[u * pdim + d] = x[d];
}

// Thread per edge (build_rabitq.cpp:217-256): residual = v_rot - u_rot over the first
// dim components; sqr_r, the code bits, bin_sum, fac_x0 and fac_x1 accumulate in
// dimension order as in the reference's loops.  out: (r_norm, fac_x0 / r_norm,
// fac_x1 * fac_norm, bin_sum); an absent neighbour gets bin_sum = -1.
__global__ void __launch_bounds__(256) rq_edges(const float* rot, const uint32_t* edges, uint64_t ne, uint32_t R,
                                                uint32_t dim, uint32_t pdim, uint32_t wpp, float fac_norm,
                                                uint32_t* codes, float4* out) {
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (e >= ne) return;
    const uint32_t v = edges[e];
    uint32_t* cw = codes + e * wpp;
    if (v == 0xFFFFFFFFu) {
        for (uint32_t w = 0; w < wpp; ++w) cw[w] = 0u;
        out[e] = make_float4(0.0f, 0.0f, 0.0f, __int_as_float(-1));
        return;
    }
    const float4* ur = reinterpret_cast<const float4*>(rot + (e / R) * pdim);
    const float4* vr = reinterpret_cast<const float4*>(rot + static_cast<uint64_t>(v) * pdim);
    float sqr = 0.0f, fx0 = 0.0f, fx1 = 0.0f;
    int bin_sum = 0;
    uint32_t word = 0;
    for (uint32_t d4 = 0; d4 * 4 < dim; ++d4) {
        const float4 a = vr[d4], b = ur[d4];
        const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = d4 * 4 + j;
            if (d < dim) {
                const float res = av[j] - bv[j];
                sqr = sqr + res * res;
                const bool pos = res > 0.0f;
                word |= pos ? (1u << (d & 31u)) : 0u;
                bin_sum += pos ? 1 : 0;
                const float sv = pos ? 1.0f : -1.0f;
                fx0 = fx0 + res * sv * fac_norm;
                fx1 = fx1 + bv[j] * sv;
            }
            if (d < dim && (d & 31u) == 31u) {
                cw[d >> 5] = word;
                word = 0;
            }
        }
    }
    for (uint32_t w = (dim + 31) / 32; w < wpp; ++w) cw[w] = 0u;
    if (dim & 31u) cw[dim >> 5] = word;
    const float r_norm = sqrtf(sqr) + 1e-10f;
    out[e] = make_float4(r_norm, fx0 / r_norm, fx1 * fac_norm, __int_as_float(bin_sum));
}

}  // namespace bsp

namespace {
int pfail(int code, const std::string& msg) {
    bs_internal_set_error(msg);
    return code;
}
}  // namespace

extern "C" int bs_index_entry_point(bs_index idx, uint32_t* entry) try {
    if (!entry) return pfail(BS_EINVAL, "entry is null");
    const float* vecs = nullptr;
    uint32_t dstride = 0;
    int rc = bs_internal_vecs(idx, &vecs, &dstride);
    if (rc) return rc;
    uint64_t n = 0;
    uint32_t dim = 0;
    rc = bs_index_info(idx, &n, &dim, nullptr, nullptr, nullptr);
    if (rc) return rc;
    float* cent = nullptr;
    unsigned long long* best = nullptr;
    if (hipMalloc(&cent, dim * sizeof(float)) != hipSuccess || hipMalloc(&best, sizeof(*best)) != hipSuccess) {
        if (cent) (void)hipFree(cent);
        return pfail(BS_ENOMEM, "hipMalloc of the entry-point buffers failed");
    }
    const float inv = 1.0f / static_cast<float>(n);
    const size_t lds = bsp::EP_LDS;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(bsp::entry_centroid<float>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::entry_centroid<float>, dim3((dim + bsp::EP_COLS - 1) / bsp::EP_COLS), dim3(bsp::EP_THREADS), lds, nullptr, vecs, n,
                           dim, dstride, inv, cent, best);
        e = hipGetLastError();
    }
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(bsp::row_dist<float>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bsp::ND_LDS));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::row_dist<float>, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), bsp::ND_LDS,
                           nullptr, vecs, n, dim, dstride, cent, nullptr, best);
        e = hipGetLastError();
    }
    unsigned long long key = 0;
    if (e == hipSuccess) e = hipMemcpy(&key, best, sizeof(key), hipMemcpyDeviceToHost);
    (void)hipFree(cent);
    (void)hipFree(best);
    if (e != hipSuccess) return pfail(BS_EHIP, std::string("entry point: ") + hipGetErrorString(e));
    *entry = static_cast<uint32_t>(key & 0xFFFFFFFFull);
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}

extern "C" int bs_index_build_rabitq(bs_index idx, uint32_t seed, uint32_t* codes_out, float* factors_out,
                                     float* signs_out, uint32_t* entry_out) try {
    if (!codes_out || !factors_out || !signs_out || !entry_out) return pfail(BS_EINVAL, "null output");
    const float* vecs = nullptr;
    const uint32_t* edges = nullptr;
    uint32_t dstride = 0;
    int rc = bs_internal_vecs(idx, &vecs, &dstride);
    if (rc) return rc;
    rc = bs_internal_edges(idx, &edges);
    if (rc) return rc;
    uint64_t n = 0;
    uint32_t dim = 0, R = 0;
    rc = bs_index_info(idx, &n, &dim, &R, nullptr, nullptr);
    if (rc) return rc;
    uint32_t pdim = 1;
    while (pdim < dim) pdim <<= 1;
    if (pdim < 32) return pfail(BS_EINVAL, "rabitq needs a padded dim >= 32 (dim > 16)");
    const uint32_t wpp = pdim / 32;
    const uint64_t ne = n * R;

    // signs (build_rabitq.cpp:138-145): mt19937_64(seed), a fair coin per padded dimension
    {
        std::mt19937_64 gen(seed);
        std::uniform_int_distribution<int> coin(0, 1);
        const float scale = 1.0f / std::sqrt(static_cast<float>(pdim));
        for (uint32_t i = 0; i < pdim; ++i) signs_out[i] = static_cast<float>(2 * coin(gen) - 1) * scale;
    }
    const float fac_norm = 1.0f / std::sqrt(static_cast<float>(dim));

    float* d_signs = nullptr;
    float* d_rot = nullptr;
    uint32_t* d_codes = nullptr;
    float4* d_out = nullptr;
    double* d_cent = nullptr;
    double* d_dist = nullptr;
    unsigned long long* d_best = nullptr;
    uint32_t* d_index = nullptr;
    auto release = [&]() {
        if (d_signs) (void)hipFree(d_signs);
        if (d_rot) (void)hipFree(d_rot);
        if (d_codes) (void)hipFree(d_codes);
        if (d_out) (void)hipFree(d_out);
        if (d_cent) (void)hipFree(d_cent);
        if (d_dist) (void)hipFree(d_dist);
        if (d_best) (void)hipFree(d_best);
        if (d_index) (void)hipFree(d_index);
    };
    if (hipMalloc(&d_signs, pdim * sizeof(float)) != hipSuccess || hipMalloc(&d_rot, n * pdim * sizeof(float)) != hipSuccess ||
        hipMalloc(&d_codes, ne * wpp * sizeof(uint32_t)) != hipSuccess || hipMalloc(&d_out, ne * sizeof(float4)) != hipSuccess ||
        hipMalloc(&d_cent, dim * sizeof(double)) != hipSuccess || hipMalloc(&d_dist, n * sizeof(double)) != hipSuccess ||
        hipMalloc(&d_best, sizeof(unsigned long long)) != hipSuccess || hipMalloc(&d_index, sizeof(uint32_t)) != hipSuccess) {
        release();
        return pfail(BS_ENOMEM, "hipMalloc of the codebook work buffers failed");
    }
    std::vector<float4> st(ne);
    const uint32_t init_index = 0xFFFFFFFFu;
    hipError_t e = hipMemcpy(d_signs, signs_out, pdim * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d_index, &init_index, sizeof(init_index), hipMemcpyHostToDevice);
    // medoid (find_medoid, build_rabitq.cpp:59-99) in double
    const size_t lds = bsp::EP_LDS;
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(bsp::entry_centroid<double>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::entry_centroid<double>, dim3((dim + bsp::EP_COLS - 1) / bsp::EP_COLS), dim3(bsp::EP_THREADS), lds, nullptr,
                           vecs, n, dim, dstride, 0.0f, d_cent, d_best);
        e = hipGetLastError();
    }
    const dim3 rows_grid(static_cast<uint32_t>((n + 255) / 256));
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(bsp::row_dist<double>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bsp::ND_LDS));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::row_dist<double>, rows_grid, dim3(256), bsp::ND_LDS, nullptr, vecs, n, dim, dstride,
                           d_cent, d_dist, d_best);
        e = hipGetLastError();
    }
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::medoid_index, rows_grid, dim3(256), 0, nullptr, n, d_dist, d_best, d_index);
        e = hipGetLastError();
    }
    // rotations, then the edges
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::rq_rotate, dim3(static_cast<uint32_t>((n + 3) / 4)), dim3(256),
                           4 * pdim * sizeof(float), nullptr, vecs, dstride, n, dim, pdim, d_signs, d_rot);
        e = hipGetLastError();
    }
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::rq_edges, dim3(static_cast<uint32_t>((ne + 255) / 256)), dim3(256), 0, nullptr, d_rot,
                           edges, ne, R, dim, pdim, wpp, fac_norm, d_codes, d_out);
        e = hipGetLastError();
    }
    uint32_t medoid = 0;
    if (e == hipSuccess) e = hipMemcpy(&medoid, d_index, sizeof(medoid), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(codes_out, d_codes, ne * wpp * sizeof(uint32_t), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(st.data(), d_out, ne * sizeof(float4), hipMemcpyDeviceToHost);
    release();
    if (e != hipSuccess) return pfail(BS_EHIP, std::string("rabitq codebook: ") + hipGetErrorString(e));
    *entry_out = medoid == 0xFFFFFFFFu ? 0u : medoid;  // no row below DBL_MAX: row 0, as the reference

    // the factor products in long double (build_rabitq.cpp:250-256), on the host threads
    auto finish = [&](uint64_t u0, uint64_t u1) {
        for (uint64_t u = u0; u < u1; ++u) {
            float* tx = factors_out + u * 3 * R;
            float* dq = tx + R;
            float* vq = dq + R;
            for (uint32_t i = 0; i < R; ++i) {
                const float4 t = st[u * R + i];
                const int bin_sum = __builtin_bit_cast(int, t.w);
                if (bin_sum < 0) {
                    tx[i] = FLT_MAX;
                    dq[i] = 0.0f;
                    vq[i] = 0.0f;
                    continue;
                }
                const float r_norm = t.x, fx0 = t.y, fx1 = t.z;
                const long double x_x0 = static_cast<long double>(r_norm) / fx0;
                tx[i] = static_cast<float>(static_cast<long double>(r_norm) * r_norm + 2.0L * x_x0 * fx1);
                dq[i] = static_cast<float>(-2.0L * x_x0 * fac_norm);
                vq[i] = dq[i] * static_cast<float>(2 * bin_sum - static_cast<int>(dim));
            }
        }
    };
    const uint32_t T = std::max(1u, std::min(32u, std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (uint32_t t = 0; t < T; ++t) pool.emplace_back(finish, n * t / T, n * (t + 1) / T);
    for (auto& th : pool) th.join();
    return BS_OK;
} catch (...) {
    return bs_internal_exception();
}
