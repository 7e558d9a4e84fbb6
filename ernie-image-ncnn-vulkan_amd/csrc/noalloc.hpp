// SPDX-License-Identifier: MIT
// Host interface of the fixed device scratch (noalloc.hip).
#pragma once
#include <stddef.h>

namespace ehip {

// 24 MiB: 16 MiB of GEMM split-K partials plus up to 8 MiB of text-block activations.
constexpr size_t kScratchSplitBytes = size_t(16) << 20;
constexpr size_t kScratchBytes = kScratchSplitBytes + (size_t(8) << 20);

// Looks up the scratch array's device address for `device`, which must be the current
// device, once; 0 or a negative status (-1 bad device, -hipError from the lookup).
int scratch_init(int device);
// The address scratch_init found for `device`, or nullptr before it succeeded. This,
// never the array's name, is what host code passes to kernels and copies.
void* scratch_address(int device);

}  // namespace ehip
