// Host-side helpers shared by the kernel dispatchers and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mlpmk.h"

namespace mlpmk {

// Records a formatted message as the calling thread's last error; returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps a HIP error to MLPMK_ERR_NO_DEVICE / MLPMK_ERR_HIP with a message.
int hip_fail(hipError_t e, const char* what);

// Compute units of the current device, verifying that it is a gfx950 part.
// Cached per device after the first call.  Returns an mlpmk_status.
int current_device_cus(int* cus);

// Occupancy (workgroups per CU) of `kernel` at `threads` per workgroup on the
// current device; the caller caches it.
int kernel_occupancy(const void* kernel, int threads, int* wgs_per_cu);

// The launch a forward dispatcher makes.  Passed non-null, the dispatcher
// fills it in and returns without launching (mlpmk_fwd_launch_info).
struct LaunchInfo {
  int kernel;          // MLPMK_KERNEL_PERSISTENT or MLPMK_KERNEL_FEATURE_SPLIT
  int rows_per_block;  // rows of x per MFMA batch block
  int waves;           // 64-lane waves per workgroup
  int grid;            // workgroups
  int wgs_per_cu;      // resident workgroups per CU (occupancy)
};

}  // namespace mlpmk
