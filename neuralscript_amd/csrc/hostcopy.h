// Host <-> device copies of the host-pointer entry points (ns_eval_infer,
// ns_runtime_train_step, ns_model_get_weights) through pinned staging.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>

namespace nship {

// Pinned slots and the events that guard their reuse; allocated on the
// first staged copy, owned by one model (one call at a time per model).
constexpr int kStageSlots = 3;
struct HostStage {
  char* slot[kStageSlots] = {};
  hipEvent_t ev[kStageSlots] = {};
};

// dev[0, bytes) = host[0, bytes), enqueued on s.  Returns once `host` may be
// reused (its bytes are in pinned memory or on the device); the DMA of the
// last chunks may still be running, ordered before later work on s.
int stage_h2d(HostStage& st, void* dev, const void* host, size_t bytes, hipStream_t s);
// host[0, bytes) = dev[0, bytes) after the work already enqueued on s;
// returns with the bytes in host memory.
int stage_d2h(HostStage& st, void* host, const void* dev, size_t bytes, hipStream_t s);
void stage_free(HostStage& st);

}  // namespace nship
