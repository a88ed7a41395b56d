// Checks the cooperative launch planning of leo_amd/csrc/launch_plan.h: for
// every lane count up to the lane limit the runtime allows, the planned grid
// fits the resident capacity, every lane gets at least one workgroup, and
// with several workgroups per lane the stride is a multiple of the XCD count
// (so a lane's workgroups share one XCD). Exits non-zero on the first failure.
#include <cstdint>
#include <cstdio>

#include "launch_plan.h"

int main() {
    uint64_t checked = 0;
    const uint32_t cus_list[] = {1, 8, 32, 80, 256, 304};
    const uint32_t per_cu_list[] = {1, 2, 3, 4, 8};
    const uint32_t want_list[] = {1, 2, 17, 32, 64, 1000};
    for (uint32_t cus : cus_list) {
        for (uint32_t per_cu : per_cu_list) {
            const uint64_t cap = leo::cooperative_capacity(cus, per_cu);
            const uint32_t limit = leo::cooperative_lane_limit(cus, per_cu, 8);
            if (limit < 1 || (cap >= 8 && limit > cap) || (cap >= 8 && limit % 8 != 0)) {
                std::printf("bad lane limit %u for capacity %llu\n", limit, static_cast<unsigned long long>(cap));
                return 1;
            }
            for (uint32_t lanes = 1; lanes <= limit; ++lanes) {
                for (uint32_t want : want_list) {
                    const leo::LanePlan p = leo::plan_lanes(lanes, want, cus, per_cu, 256, 8);
                    const bool fits = p.grid <= cap || cap < lanes;
                    const bool covers = p.stride >= lanes && p.P >= 1;
                    const bool local = p.P == 1 || p.stride % 8 == 0;
                    if (!fits || !covers || !local || p.P > want) {
                        std::printf("bad plan: cus %u per_cu %u lanes %u want %u -> P %u stride %u grid %u\n", cus,
                                    per_cu, lanes, want, p.P, p.stride, p.grid);
                        return 1;
                    }
                    ++checked;
                }
            }
        }
    }
    std::printf("checked %llu plans\n", static_cast<unsigned long long>(checked));
    return 0;
}
