// SPDX-License-Identifier: MIT
// Fixed device scratch for the entry point that allocates nothing
// (ernie_hip_text_block_forward_noalloc). The array lives in the code object, one copy
// per GPU the library runs on, held until the process ends; its device address is
// looked up once per device with that device current and kept.
#include "noalloc.hpp"

#include <hip/hip_runtime.h>

#include <mutex>

namespace ehip {
namespace {

__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices] = {};

}  // namespace

int scratch_init(int device)
{
    if (device < 0 || device >= kMaxDevices) return -1;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_ptr[device]) return 0;
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess || current != device) return -1;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        return -int(e ? e : hipErrorInvalidSymbol);
    }
    scratch_ptr[device] = ptr;
    return 0;
}

void* scratch_address(int device)
{
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(scratch_mu);
    return scratch_ptr[device];
}

}  // namespace ehip
