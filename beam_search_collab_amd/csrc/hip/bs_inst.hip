// Explicit search-kernel instances for one mode (BS_INST_MODE = 0 hash, 1 bloom,
// 2 rabitq, 3 rabitq with wide codes), compiled once per mode so the instances build in
// parallel.
#include "bs_launch.hpp"

#ifndef BS_INST_MODE
#error "BS_INST_MODE must be defined"
#endif

namespace bsd {

// occ != null: no launch; *occ = the instance's resident wavefronts per CU (one-wavefront
// workgroups with `lds` bytes of LDS each)
template <int TR, int CR, int QMAX, int PB>
static hipError_t launch_one(const SearchParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t s, int* occ) {
    auto k = search_kernel<TR, CR, QMAX, BS_INST_MODE, PB>;
    if (occ) return hipOccupancyMaxActiveBlocksPerMultiprocessor(occ, k, 64, lds);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, grid, block, lds, s, p);
    return hipGetLastError();
}

template <int TR, int CR>
static hipError_t launch_p(const SearchParams& p, int PB, dim3 g, dim3 b, size_t lds, hipStream_t s, int* occ) {
    // every dim <= 1024 fits 4 float4 chunks per lane (bsd::l2_shape).  Narrow RaBitQ codes
    // mean dim <= 128, computed with one chunk per lane (bsd::l2_shape_lanes: 2-8 rows per
    // pass), 8 passes in flight; wide codes mean dim > 128, hence PB >= 4.
    if constexpr (BS_INST_MODE == 2) {
        (void)PB;
        return launch_one<TR, CR, 1, 8>(p, g, b, lds, s, occ);
    } else if constexpr (BS_INST_MODE == 3) {
        return PB == 4 ? launch_one<TR, CR, 4, 4>(p, g, b, lds, s, occ) : launch_one<TR, CR, 4, 8>(p, g, b, lds, s, occ);
    } else {
        switch (PB) {
        case 2: return launch_one<TR, CR, 4, 2>(p, g, b, lds, s, occ);
        case 4: return launch_one<TR, CR, 4, 4>(p, g, b, lds, s, occ);
        default: return launch_one<TR, CR, 4, 8>(p, g, b, lds, s, occ);
        }
    }
}

template <int TR>
static hipError_t launch_c(const SearchParams& p, int CR, int PB, dim3 g, dim3 b, size_t lds, hipStream_t s,
                           int* occ) {
    // degree <= 64, <= 128, <= 256 (gpu_cli.cu:208-233)
    return CR == 1   ? launch_p<TR, 1>(p, PB, g, b, lds, s, occ)
           : CR == 2 ? launch_p<TR, 2>(p, PB, g, b, lds, s, occ)
                     : launch_p<TR, 4>(p, PB, g, b, lds, s, occ);
}

static hipError_t launch_any(const SearchParams& p, int TR, int CR, int PB, dim3 g, dim3 b, size_t lds,
                             hipStream_t s, int* occ) {
    switch (TR) {
    case 1: return launch_c<1>(p, CR, PB, g, b, lds, s, occ);
    case 2: return launch_c<2>(p, CR, PB, g, b, lds, s, occ);
    case 4: return launch_c<4>(p, CR, PB, g, b, lds, s, occ);
    case 8: return launch_c<8>(p, CR, PB, g, b, lds, s, occ);
#if BS_INST_MODE >= 2
    case 10: return launch_c<10>(p, CR, PB, g, b, lds, s, occ);  // rabitq beams of 513..640
    case 12: return launch_c<12>(p, CR, PB, g, b, lds, s, occ);  // rabitq beams of 641..768
#endif
    case 16: return launch_c<16>(p, CR, PB, g, b, lds, s, occ);
    case 32: return launch_c<32>(p, CR, PB, g, b, lds, s, occ);  // beams of 1025..2048
    default: return launch_c<64>(p, CR, PB, g, b, lds, s, occ);  // beams of 2049..4096
    }
}

#if BS_INST_MODE == 0
#ifdef BS_PHASE_CLOCKS
// the instrumented library's clock sums of the hash-filter (base, warp) instances
// (PhaseClock): out[0..16) as bs_phase_clock holds them; reset != 0 clears them afterwards
extern "C" int bs_phase_read_base(unsigned long long* out, int reset) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(bs_phase_clock), sizeof(unsigned long long) * 16) != hipSuccess) return 1;
    if (reset) {
        const unsigned long long z[16] = {};
        if (hipMemcpyToSymbol(HIP_SYMBOL(bs_phase_clock), z, sizeof(z)) != hipSuccess) return 2;
    }
    return 0;
}
// the instrumented library's per-query clocks of the hash-filter (base, warp) instances
// (QueryClock): out[3 q + 0..2] = start, end, hardware id of queries q < n (n <= 65536)
extern "C" int bs_query_clock_read(unsigned long long* out, uint64_t n) {
    if (n > QUERY_CLOCK_MAX) return 2;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(bs_query_clock), sizeof(unsigned long long) * 3 * n) == hipSuccess ? 0
                                                                                                             : 1;
}
#endif
hipError_t launch_search_hash(const SearchParams& p, int TR, int CR, int PB, dim3 g, dim3 b, size_t lds,
                              hipStream_t s, int* occ) {
    return launch_any(p, TR, CR, PB, g, b, lds, s, occ);
}
#elif BS_INST_MODE == 1
hipError_t launch_search_bloom(const SearchParams& p, int TR, int CR, int PB, dim3 g, dim3 b, size_t lds,
                              hipStream_t s, int* occ) {
    return launch_any(p, TR, CR, PB, g, b, lds, s, occ);
}
#elif BS_INST_MODE == 2
hipError_t launch_search_rabitq(const SearchParams& p, int TR, int CR, int PB, dim3 g, dim3 b, size_t lds,
                              hipStream_t s, int* occ) {
    return launch_any(p, TR, CR, PB, g, b, lds, s, occ);
}
#ifdef BS_PHASE_CLOCKS
// the instrumented library's per-query clocks of the narrow-code RaBitQ instances
// (QueryClock), as bs_query_clock_read gives them for the hash-filter ones
extern "C" int bs_query_clock_read_rabitq(unsigned long long* out, uint64_t n) {
    if (n > QUERY_CLOCK_MAX) return 2;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(bs_query_clock), sizeof(unsigned long long) * 3 * n) == hipSuccess ? 0
                                                                                                             : 1;
}
// the instrumented library's clock sums of the narrow-code RaBitQ instances (PhaseClock):
// out[0..16) as bs_phase_clock holds them; reset != 0 clears them afterwards
extern "C" int bs_phase_read(unsigned long long* out, int reset) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(bs_phase_clock), sizeof(unsigned long long) * 16) != hipSuccess) return 1;
    if (reset) {
        const unsigned long long z[16] = {};
        if (hipMemcpyToSymbol(HIP_SYMBOL(bs_phase_clock), z, sizeof(z)) != hipSuccess) return 2;
    }
    return 0;
}
#endif
#else
hipError_t launch_search_rabitq_wide(const SearchParams& p, int TR, int CR, int PB, dim3 g, dim3 b, size_t lds,
                              hipStream_t s, int* occ) {
    return launch_any(p, TR, CR, PB, g, b, lds, s, occ);
}
#endif

}  // namespace bsd
