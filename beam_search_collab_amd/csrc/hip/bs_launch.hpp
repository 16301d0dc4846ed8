// Launchers of the search kernel instances (one translation unit per mode).
#pragma once
#include <hip/hip_runtime.h>
#include "bs_search.hpp"

namespace bsd {
// TR in {1,2,4,8,16} (and 12 for the rabitq modes), CR in {1,2}, PB (L2 passes in flight)
// in {2,4,8}.  occ != null: no launch, *occ = the instance's resident wavefronts per CU.
hipError_t launch_search_hash(const SearchParams& p, int TR, int CR, int PB, dim3 grid, dim3 block,
                              size_t lds, hipStream_t s, int* occ = nullptr);
hipError_t launch_search_bloom(const SearchParams& p, int TR, int CR, int PB, dim3 grid, dim3 block,
                               size_t lds, hipStream_t s, int* occ = nullptr);
hipError_t launch_search_rabitq(const SearchParams& p, int TR, int CR, int PB, dim3 grid, dim3 block,
                                size_t lds, hipStream_t s, int* occ = nullptr);
hipError_t launch_search_rabitq_wide(const SearchParams& p, int TR, int CR, int PB, dim3 grid, dim3 block,
                                     size_t lds, hipStream_t s, int* occ = nullptr);
}  // namespace bsd
