// Query scheduling for cache locality (bs_order.hip): labels, bucket sort, launch map.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bso {

constexpr uint32_t ORDER_P = 256;    // pivots (unused slots: zero rows with a huge norm)
constexpr uint32_t ORDER_MAX_X = 32; // XCDs supported by the launch map

struct OrderParams {
    const float* queries;  // nq * dim
    uint64_t nq;
    uint32_t dim;
    const float* pivT;     // roundup(dim, 16) * ORDER_P, pivot j's coordinate k at [k * ORDER_P + j]
    const float* pnorm;    // ORDER_P squared norms
    uint32_t* key;         // nq labels
    uint32_t* hist;        // ORDER_P counts, zero between launches
    uint32_t* cursor;      // ORDER_P bucket cursors
    uint32_t* qmap;        // nq: launch position -> query
    uint32_t g;            // queries per workgroup of the search launch
    uint32_t X;            // XCDs, 1..ORDER_MAX_X
    uint32_t start[ORDER_MAX_X];  // first label-order rank of each XCD's run
};

// order_key, order_scan, order_place on stream s (nq >= 1)
hipError_t launch_order(const OrderParams& o, hipStream_t s);

// Launch map by predicted cost, longest first (nq >= 1): on entry key[q] holds query q's
// cost signal as a float (larger = longer), on return its bucket; o.X and o.start are
// ignored (one run).  Up to 65536 queries one workgroup does it all (cost_order_one);
// above, cost_range, cost_key, order_scan and order_place, with cursor[0..1] as scratch.
hipError_t launch_cost_order(const OrderParams& o, hipStream_t s);

}  // namespace bso
