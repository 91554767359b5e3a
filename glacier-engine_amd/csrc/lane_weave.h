// lane_weave.h — the internal half of the LaneWeave scheduler used by the
// session's decode waves.
#pragma once
#include <functional>

#include "../../include/glacier_hip.h"

namespace gh {

// One decode wave with the scheduler locked from planning to the last
// commit. plan: the next quanta of distinct lanes (only quanta whose service
// commits). run: the device step over the planned slots, privately (nothing
// published; a failure leaves the scheduler unchanged). sink (optional): the
// caller's acknowledgement of the wave's stages before anything is
// published; a rejection aborts every private row and leaves the scheduler
// unchanged. Then for each planned quantum in order, the reference's service
// transaction (lane_weave_qos.zig prepareService :1127 -> publish ->
// commitService :1272): a permit is prepared, its selection must be the
// planned slot, the lane's token is published, the permit committed. A
// permit that does not select the planned slot, or a publication that fails,
// aborts the permit (abortService :1438) and the unpublished quanta and
// poisons the scheduler (the quanta before it are already published).
struct WaveOps {
  std::function<int(const uint32_t *slots, uint32_t n)> run;
  std::function<int()> sink;
  std::function<int(uint32_t i)> publish;
  std::function<void(uint32_t from)> abort;
};
int lane_weave_run_wave(glacier_hip_lane_weave *lw, uint32_t max_count, const WaveOps &ops,
                        uint32_t *slots_out, glacier_hip_lane_event_t *events_out,
                        uint32_t *count_out);

}  // namespace gh
