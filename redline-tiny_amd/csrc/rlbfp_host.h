// Host-side helpers shared by the C-ABI entry points: error reporting and the device check.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlbfp.h"

namespace rl {

// Records a formatted message for rl_last_error() on the calling thread and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's message and returns RL_OK.
int ok();
// RL_OK if the current device is a gfx950; caches the answer per device.
int check_device();
// Compute units of the current device (after check_device; 256 if unknown).
int device_cus();
// Converts a launch's HIP status into an RL status.
int launch_status(const char* what);

}  // namespace rl
