// Host interface of the fixed per-device scratch array (scratch.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rfxq_scratch {

// 128 MiB: the activation layouts and split-K partials of an M = 512 GEMM up
// to in_features 16384 and the widest split of the 8B shapes (q_proj 4096 x
// 4096: 8 splits x 512 x 4096 x 4 B = 64 MiB of partials)
constexpr uint64_t kScratchBytes = 128ull << 20;

// Resolve the array's address on `device`, which must be current; once per
// device, later calls return the kept address.
hipError_t setup(int device, void** out);

// The address setup() resolved on `device`, or NULL before that.
void* address(int device);

}  // namespace rfxq_scratch
