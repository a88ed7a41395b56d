// Grid planning of the cooperative step launch, shared by the host runtime
// and its CPU unit check (tests/launch_plan_check.cpp).
//
// A launch over `lanes` lanes uses P workgroups per lane. With P > 1 the lanes
// are padded to a multiple of the XCD count and workgroup b serves lane
// b % padded, so the grid is padded * P; with P = 1 the grid is the lane count
// itself. Every workgroup of a cooperative launch must be resident at once:
// the grid may not exceed cus * blocks_per_cu.
#ifndef LEO_LAUNCH_PLAN_H
#define LEO_LAUNCH_PLAN_H

#include <stdint.h>

namespace leo {

struct LanePlan {
    uint32_t padded;  // lanes padded to the XCD count
    uint32_t P;       // workgroups per lane
    uint32_t stride;  // workgroup b serves lane b % stride
    uint32_t grid;    // workgroups of the launch
};

// Workgroups one cooperative launch may hold.
inline uint64_t cooperative_capacity(uint32_t cus, uint32_t blocks_per_cu) {
    return static_cast<uint64_t>(cus) * blocks_per_cu;
}

// Lanes one cooperative launch can serve (one workgroup each at the least),
// rounded down to the XCD count so that padding never pushes a full group
// past the capacity; at least one.
inline uint32_t cooperative_lane_limit(uint32_t cus, uint32_t blocks_per_cu, uint32_t xcds = 8) {
    const uint64_t cap = cooperative_capacity(cus, blocks_per_cu);
    const uint64_t rounded = cap / xcds * xcds;
    const uint64_t limit = rounded > 0 ? rounded : (cap > 0 ? cap : 1);
    return static_cast<uint32_t>(limit > 0xffffffffu ? 0xffffffffu : limit);
}

// The launch shape for `lanes` lanes when `want` workgroups per lane are
// wanted, capped by the capacity and by `max_per_lane`.
inline LanePlan plan_lanes(uint32_t lanes, uint32_t want, uint32_t cus, uint32_t blocks_per_cu,
                           uint32_t max_per_lane, uint32_t xcds = 8) {
    LanePlan p{};
    const uint64_t cap = cooperative_capacity(cus, blocks_per_cu);
    p.padded = (lanes + xcds - 1) / xcds * xcds;
    uint64_t limit = p.padded ? cap / p.padded : 1;
    if (limit > max_per_lane) limit = max_per_lane;
    if (limit < 1) limit = 1;
    uint64_t P = want < 1 ? 1 : want;
    if (P > limit) P = limit;
    p.P = static_cast<uint32_t>(P);
    p.stride = p.P > 1 ? p.padded : lanes;
    p.grid = p.stride * p.P;
    return p;
}

}  // namespace leo

#endif
