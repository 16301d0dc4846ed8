// Index preparation on the device: the search entry point.
//
// compute_entry_point (src/gpu_cli.cu:55-83): a float centroid accumulated row after row
// (centroid[d] += row[d] * inv, inv = 1 / n), then the first row of least float squared
// distance to it (diff = row[d] - centroid[d]; dist += diff * diff, dimensions in order;
// a row replaces the best only if dist < best, starting from FLT_MAX and row 0).  The
// float roundings of both loops are reproduced exactly, so the node is the reference's.
#include "bs_hip.h"
#include "wave.hpp"

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstring>
#include <string>

int bs_internal_vecs(bs_index idx, const float** vecs, uint32_t* dstride);
void bs_internal_set_error(const std::string& msg);

namespace bsp {

using namespace bsw;

constexpr uint32_t EP_ROWS = 256;    // rows per LDS chunk (64 columns each: 64 KB)
constexpr uint32_t EP_THREADS = 1024;

__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The centroid is one dependent chain of n additions per dimension, so the only
// parallelism is across dimensions: workgroup x owns dimensions [64x, 64x + 64), its
// first wavefront adds (lane = dimension) while the other 15 wavefronts stream the next
// chunk of rows into the other half of a double buffer in LDS.
__global__ void __launch_bounds__(EP_THREADS) entry_centroid(const float* vecs, uint64_t n, uint32_t dim,
                                                            uint32_t dstride, float inv, float* cent,
                                                            unsigned long long* best) {
    extern __shared__ float buf[];  // [2][EP_ROWS][64]
    const uint32_t lane = lane_id(), wave = uniform(threadIdx.x >> 6);
    const uint32_t col0 = blockIdx.x * 64;
    const uint64_t nchunk = (n + EP_ROWS - 1) / EP_ROWS;
    if (blockIdx.x == 0 && threadIdx.x == 0)
        *best = static_cast<unsigned long long>(orderable(FLT_MAX)) << 32;  // (FLT_MAX, row 0)
    // stage chunk c into buffer half h with threads [t0, EP_THREADS)
    auto stage = [&](uint64_t c, uint32_t h, uint32_t t0) __attribute__((always_inline)) {
        float* dst = buf + h * (EP_ROWS * 64);
        const uint64_t r0 = c * EP_ROWS;
        for (uint32_t e = threadIdx.x - t0; e < EP_ROWS * 64; e += EP_THREADS - t0) {
            const uint32_t r = e >> 6, k = e & 63u;
            const uint64_t row = r0 + r;
            float v = 0.0f;
            if (row < n && col0 + k < dim) v = vecs[row * dstride + col0 + k];
            dst[e] = v;
        }
    };
    stage(0, 0, 0);
    __syncthreads();
    float s = 0.0f;
    for (uint64_t c = 0; c < nchunk; ++c) {
        const uint32_t h = static_cast<uint32_t>(c & 1);
        if (wave == 0) {
            const float* src = buf + h * (EP_ROWS * 64) + lane;
            const uint32_t rows = static_cast<uint32_t>(n - c * EP_ROWS < EP_ROWS ? n - c * EP_ROWS : EP_ROWS);
#pragma unroll 16
            for (uint32_t r = 0; r < rows; ++r) s = s + src[r * 64] * inv;
        } else if (c + 1 < nchunk) {
            stage(c + 1, h ^ 1u, 64);
        }
        __syncthreads();
    }
    if (wave == 0 && col0 + lane < dim) cent[col0 + lane] = s;
}

// Thread per row: its float distance in dimension order, then the least (dist, row) of
// the rows with dist < FLT_MAX by one 64-bit atomic minimum per wavefront.
__global__ void __launch_bounds__(256) entry_nearest(const float* vecs, uint64_t n, uint32_t dim,
                                                     uint32_t dstride, const float* cent,
                                                     unsigned long long* best) {
    __shared__ float c[1024];
    for (uint32_t k = threadIdx.x; k < dim; k += 256) c[k] = cent[k];
    __syncthreads();
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    unsigned long long key = ~0ull;
    if (i < n) {
        const float4* row = reinterpret_cast<const float4*>(vecs + i * dstride);
        float s = 0.0f;
        uint32_t k = 0;
        for (; k + 4 <= dim; k += 4) {
            const float4 v = row[k >> 2];
            float d = v.x - c[k];
            s = s + d * d;
            d = v.y - c[k + 1];
            s = s + d * d;
            d = v.z - c[k + 2];
            s = s + d * d;
            d = v.w - c[k + 3];
            s = s + d * d;
        }
        for (; k < dim; ++k) {
            const float d = vecs[i * dstride + k] - c[k];
            s = s + d * d;
        }
        if (s < FLT_MAX) key = (static_cast<unsigned long long>(orderable(s)) << 32) | i;
    }
    unsigned long long t;
    t = xor_lane64<1>(key); key = t < key ? t : key;
    t = xor_lane64<2>(key); key = t < key ? t : key;
    t = xor_lane64<4>(key); key = t < key ? t : key;
    t = xor_lane64<8>(key); key = t < key ? t : key;
    t = xor_lane64<16>(key); key = t < key ? t : key;
    t = xor_lane64<32>(key); key = t < key ? t : key;
    if (lane_id() == 0 && key != ~0ull) atomicMin(best, key);
}

}  // namespace bsp

namespace {
int pfail(int code, const std::string& msg) {
    bs_internal_set_error(msg);
    return code;
}
}  // namespace

extern "C" int bs_index_entry_point(bs_index idx, uint32_t* entry) {
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
    const size_t lds = 2 * bsp::EP_ROWS * 64 * sizeof(float);
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(bsp::entry_centroid),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::entry_centroid, dim3((dim + 63) / 64), dim3(bsp::EP_THREADS), lds, nullptr, vecs, n,
                           dim, dstride, inv, cent, best);
        e = hipGetLastError();
    }
    if (e == hipSuccess) {
        hipLaunchKernelGGL(bsp::entry_nearest, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, nullptr,
                           vecs, n, dim, dstride, cent, best);
        e = hipGetLastError();
    }
    unsigned long long key = 0;
    if (e == hipSuccess) e = hipMemcpy(&key, best, sizeof(key), hipMemcpyDeviceToHost);
    (void)hipFree(cent);
    (void)hipFree(best);
    if (e != hipSuccess) return pfail(BS_EHIP, std::string("entry point: ") + hipGetErrorString(e));
    *entry = static_cast<uint32_t>(key & 0xFFFFFFFFull);
    return BS_OK;
}
