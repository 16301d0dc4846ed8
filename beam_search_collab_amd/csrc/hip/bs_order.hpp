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
    const float* lcost;    // ORDER_P expected costs per label, or null (see order_one_cost)
    uint32_t g;            // queries per workgroup of the search launch
    uint32_t X;            // XCDs, 1..ORDER_MAX_X
    uint32_t start[ORDER_MAX_X];  // first label-order rank of each XCD's run
};

// o.start for a launch of m >= 1 queries in workgroups of o.g on o.X XCDs: XCD x runs
// workgroups x, x + X, ...; all are full but the launch's last one
inline void order_starts(OrderParams& o, uint64_t m) {
    const uint64_t g = o.g, X = o.X, B = (m + g - 1) / g;
    uint64_t acc = 0;
    for (uint32_t x = 0; x < X; ++x) {
        o.start[x] = static_cast<uint32_t>(acc);
        uint64_t cnt = (B > x ? (B - 1 - x) / X + 1 : 0) * g;
        if ((B - 1) % X == x) cnt -= B * g - m;
        acc += cnt;
    }
}

// the placement of launch_order alone (key[q] already holds query q's label, nq <= 65536)
hipError_t launch_place(const OrderParams& o, hipStream_t s);

// order_key, order_scan, order_place on stream s (nq >= 1); up to 65536 queries the counts,
// scan and placement run in one workgroup, and with lcost the labels of each XCD's run go by
// descending expected cost
hipError_t launch_order(const OrderParams& o, hipStream_t s);

// order_key alone: key[q] = query q's label (nq <= 65536: hist untouched)
hipError_t launch_labels(const OrderParams& o, hipStream_t s);

// Expected cost per label from a calibration search: labels[n] (order_key's), per_query[n*5]
// (iterations first) -> lcost[ORDER_P] (mean iterations of the label's queries; labels without
// a query get the mean of all).  One workgroup.
hipError_t launch_label_cost(const uint32_t* labels, const uint32_t* per_query, uint32_t n, float* lcost,
                             hipStream_t s);

// rows i * n / m (i < m) of vecs (row stride dstride floats) packed into out[m * dim]
hipError_t launch_gather_rows(const float* vecs, uint32_t dstride, uint32_t dim, uint64_t n, uint32_t m, float* out,
                              hipStream_t s);

// Launch map by predicted cost, longest first (nq >= 1): on entry key[q] holds query q's
// cost signal as a float (larger = longer), on return its bucket; o.X and o.start are
// ignored (one run).  Up to 65536 queries one workgroup does it all (cost_order_one);
// above, cost_range, cost_key, order_scan and order_place, with cursor[0..1] as scratch.
hipError_t launch_cost_order(const OrderParams& o, hipStream_t s);

}  // namespace bso
