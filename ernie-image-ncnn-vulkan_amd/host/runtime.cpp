// SPDX-License-Identifier: MIT
#include "ernie/runtime.h"

#include <string>

namespace ernie {

void check_status(int status, const ernie_hip_ctx* ctx, const char* action)
{
    if (status == ERNIE_OK) return;
    const std::string msg = std::string(action) + ": " + ernie_hip_last_error(ctx);
    if (status == ERNIE_ALLOCATION_FAILED) throw GpuAllocationError(msg);
    throw std::runtime_error(msg);
}

Device::Device(int index)
{
    ernie_hip_ctx* ctx = nullptr;
    const int rc = ernie_hip_create(index, &ctx);
    if (rc == ERNIE_ALLOCATION_FAILED) throw GpuAllocationError("Create device context");
    if (rc != ERNIE_OK || !ctx) throw std::runtime_error("No HIP device " + std::to_string(index));
    ctx_ = std::shared_ptr<ernie_hip_ctx>(ctx, ernie_hip_destroy);
}

void Device::synchronize() const { check_status(ernie_hip_synchronize(ctx()), ctx(), "synchronize"); }

DeviceMat DeviceMat::create(const Device& device, int w, int h, int c, int dims)
{
    if (w < 1 || h < 1 || c < 1) throw std::invalid_argument("Device tensor dimensions must be positive");
    void* p = nullptr;
    ernie_hip_ctx* ctx = device.ctx();
    check_status(ernie_hip_malloc(ctx, size_t(w) * h * c * sizeof(float), &p), ctx, "Allocate device tensor");
    DeviceMat m;
    // The deleter keeps the context alive: a tensor may outlive its Device.
    std::shared_ptr<ernie_hip_ctx> owner = device.shared_ctx();
    m.holder = std::shared_ptr<void>(p, [owner](void* q) { ernie_hip_free(owner.get(), q); });
    m.data = static_cast<float*>(p);
    m.w = w;
    m.h = h;
    m.c = c;
    m.dims = dims ? dims : (c > 1 ? 3 : (h > 1 ? 2 : 1));
    return m;
}

DeviceMat DeviceMat::view(size_t offset, int w_, int h_, int c_, int dims_) const
{
    if (offset + size_t(w_) * h_ * c_ > total()) throw std::out_of_range("Device tensor view exceeds its parent");
    DeviceMat m = *this;
    m.data = data + offset;
    m.w = w_;
    m.h = h_;
    m.c = c_;
    m.dims = dims_ ? dims_ : (c_ > 1 ? 3 : (h_ > 1 ? 2 : 1));
    m.valid_prefix = 0;
    return m;
}

void DeviceMat::upload(const Device& device, const float* host, size_t count) const
{
    if (count > total()) throw std::out_of_range("Upload exceeds device tensor");
    check_status(ernie_hip_memcpy_h2d(device.ctx(), data, host, count * sizeof(float)), device.ctx(), "Upload");
}

std::vector<float> DeviceMat::download(const Device& device) const
{
    std::vector<float> out(total());
    check_status(ernie_hip_memcpy_d2h(device.ctx(), out.data(), data, out.size() * sizeof(float)), device.ctx(),
                 "Download");
    return out;
}

int Option::dtype() const
{
    if (use_fp16_arithmetic) throw std::invalid_argument("FP16 arithmetic is not supported; arithmetic is FP32");
    if (use_fp16_storage && use_bf16_storage) throw std::invalid_argument("Select one storage precision");
    return use_bf16_storage ? ERNIE_DTYPE_BF16 : (use_fp16_storage ? ERNIE_DTYPE_FP16 : ERNIE_DTYPE_FP32);
}

}  // namespace ernie
