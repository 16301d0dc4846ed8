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
        atomicAdd(&o.hist[label], 1u);
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

// Thread per query: its rank in label order, then its launch position.
__global__ void __launch_bounds__(256) order_place(const OrderParams o) {
    const uint64_t q = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (q >= o.nq) return;
    const uint32_t r = atomicAdd(&o.cursor[o.key[q]], 1u);
    uint32_t x = 0;
    while (x + 1 < o.X && o.start[x + 1] <= r) ++x;
    const uint32_t j = r - o.start[x];
    const uint64_t b = x + static_cast<uint64_t>(o.X) * (j / o.g);
    const uint64_t pos = b * o.g + j % o.g;
    if (pos < o.nq) o.qmap[pos] = static_cast<uint32_t>(q);
}

hipError_t launch_order(const OrderParams& o, hipStream_t s) {
    hipLaunchKernelGGL(order_key, dim3(static_cast<uint32_t>((o.nq + 31) / 32)), dim3(256), 0, s, o);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(order_scan, dim3(1), dim3(ORDER_P), 0, s, o);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(order_place, dim3(static_cast<uint32_t>((o.nq + 255) / 256)), dim3(256), 0, s, o);
    return hipGetLastError();
}

}  // namespace bso
