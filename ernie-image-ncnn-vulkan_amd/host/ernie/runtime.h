// SPDX-License-Identifier: MIT
// Host-side types of the ernie C++ facade: the device context, device tensor
// views (the role ncnn::VkMat plays in the reference) and the error mapping.
#pragma once
#include <cstddef>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "ernie_hip.h"

namespace ernie {

// Allocation failures surface as this type, as in the reference
// (src/vulkan_memory.h:14-21), so denoise_with_recovery-style callers can
// classify them; every other device failure is a std::runtime_error.
struct GpuAllocationError : std::runtime_error {
    explicit GpuAllocationError(const std::string& what) : std::runtime_error(what) {}
};

// Throws for a non-zero ernie_hip status (-100 -> GpuAllocationError).
void check_status(int status, const ernie_hip_ctx* ctx, const char* action);

// Device context: plays the role of the VulkanDevice + session allocators. The
// ernie_hip context is shared with every DeviceMat allocated on it, so it is destroyed
// when the Device and the last of those tensors are gone, in whichever order.
class Device {
public:
    explicit Device(int index = 0);
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;
    ernie_hip_ctx* ctx() const { return ctx_.get(); }
    const std::shared_ptr<ernie_hip_ctx>& shared_ctx() const { return ctx_; }
    void synchronize() const;

private:
    std::shared_ptr<ernie_hip_ctx> ctx_;
};

// Refcounted FP32 device tensor with ncnn's w/h/c dimension naming (w fastest).
// `valid_prefix` is an optional hint carried by attention masks built by
// dit_constants: keys at or beyond it hold -1e30.
struct DeviceMat {
    std::shared_ptr<void> holder;
    float* data = nullptr;
    int dims = 0, w = 0, h = 1, c = 1;
    int valid_prefix = 0;
    // Set by upload_text_constants on its causal mask: applied by position, not read.
    bool causal = false;
    size_t total() const { return size_t(w) * h * c; }
    bool empty() const { return data == nullptr || total() == 0; }
    // Allocate on the device.
    static DeviceMat create(const Device& device, int w, int h = 1, int c = 1, int dims = 0);
    // A view that shares ownership with its parent.
    DeviceMat view(size_t offset, int w, int h = 1, int c = 1, int dims = 0) const;
    void upload(const Device& device, const float* host, size_t count) const;
    std::vector<float> download(const Device& device) const;
};

// Attention mask argument for the device: a mask built by dit_constants is
// canonical (0 below valid_prefix, -1e30 from it), so the key count alone
// carries it and the kernel skips the additive mask entirely.
inline const float* mask_arg(const DeviceMat& mask)
{
    return (mask.empty() || mask.valid_prefix > 0) ? nullptr : mask.data;
}

// Mirrors the ncnn::Option fields the block path reads (probes/block_runner.cpp:102-109):
// storage precision, FP32 arithmetic, and the device standing in for the Vulkan device.
struct Option {
    bool use_fp16_storage = false;
    bool use_bf16_storage = false;
    bool use_fp16_arithmetic = false;  // must stay false: arithmetic is FP32
    int num_threads = 4;               // host threads (unused by the device path)
    const Device* device = nullptr;
    int dtype() const;
};

}  // namespace ernie
