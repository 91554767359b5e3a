// lane_weave.h — the internal half of the LaneWeave scheduler used by the
// session's decode waves.
#pragma once
#include <functional>

#include "../../include/glacier_hip.h"

namespace gh {

// One decode wave with the scheduler locked from planning to commit: plan
// the next quanta of distinct lanes (only quanta whose serve_one commits),
// run `device_step` over the planned slots, then serve them in plan order.
// A failing device step commits nothing; a serve that no longer matches the
// committed device step poisons the scheduler.
int lane_weave_run_wave(glacier_hip_lane_weave *lw, uint32_t max_count,
                        const std::function<int(const uint32_t *slots, uint32_t n)> &device_step,
                        uint32_t *slots_out, glacier_hip_lane_event_t *events_out,
                        uint32_t *count_out);

}  // namespace gh
