// launch.h -- how the library launches its kernels: hipLaunchKernelGGL, or, while
// mmoe_forward_profile runs on this host thread, hipExtLaunchKernelGGL with a start and a stop
// event per launch. Those events take the dispatch's own timestamps (no event marker packet in
// front of the kernel), so each reads the kernel's duration inside the whole layer call, as a
// kernel trace does.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mmoe {

struct LaunchTimer {
  hipEvent_t const* events;  // 2 per launch: start, stop
  int32_t* stages;           // the stage of each launch (MMOE_STAGE_*), or null
  int capacity;              // launches that get events
  int count;                 // launches so far (those past capacity run without events)
  int stage;                 // the stage the next launches belong to
};

// This host thread's timer: null except inside mmoe_forward_profile.
LaunchTimer*& launch_timer();

template <typename... KArgs, typename... Args>
hipError_t launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t smem,
                         hipStream_t stream, Args... args) {
  LaunchTimer* t = launch_timer();
  if (t != nullptr && t->count < t->capacity) {
    const int i = t->count++;
    if (t->stages != nullptr) t->stages[i] = t->stage;
    hipExtLaunchKernelGGL(kernel, grid, block, smem, stream, t->events[2 * i], t->events[2 * i + 1], 0,
                          static_cast<KArgs>(args)...);
  } else {
    if (t != nullptr) ++t->count;
    hipLaunchKernelGGL(kernel, grid, block, smem, stream, static_cast<KArgs>(args)...);
  }
  return hipGetLastError();
}

}  // namespace mmoe
