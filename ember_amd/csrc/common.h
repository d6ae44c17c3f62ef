// common.h -- internal helpers shared by the HIP translation units of
// libember_amd.so (not part of the public ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/ember_amd.h"

namespace ember {

// Records `status` in this thread's sticky error slot (first error wins) and
// prints `what` with the HIP error text when `err` is a HIP failure.
int record_error(int status, const char *what, hipError_t err = hipSuccess);

// Checks a HIP call; on failure records EMBER_ERR_DEVICE and returns false.
bool hip_ok(hipError_t err, const char *what);

// Checks for a launch-configuration error right after a kernel launch
// (asynchronous faults surface at the next synchronising call, as in the
// reference's CUDA_POST_LAUNCH, src/tensor/operators_gpu.cu:12-15).
bool launch_ok(const char *kernel);

// Library-owned device scratch, grown on demand and cached per device for
// the life of the process.  Slot ids keep independent users apart.
void *scratch(int slot, size_t bytes);

enum ScratchSlot {
    kScratchAttnDelta = 0,
    kScratchSum = 1,
    kScratchLayerNorm = 2,
    kScratchColSum = 3,
    kScratchGemmSplit = 4,
    kScratchAttnOrder = 5,
    kScratchSlots = 6
};

// The library-wide switch set by ember_set_deterministic.
bool deterministic();

// Compute units of the current device (cached per device), or 0 if the HIP
// runtime cannot say; records no error.
int device_cu_count();

}  // namespace ember
