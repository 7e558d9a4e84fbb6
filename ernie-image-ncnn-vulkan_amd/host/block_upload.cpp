// SPDX-License-Identifier: MIT
// Upload of an on-disk DiT block into a resident device slot (the device half of
// load_component, src/component_files.cpp:10-60). Parsing and checks live in
// block_files.cpp, which has no device dependency.
#include <stdexcept>

#include "ernie/block_files.h"
#include "ernie/runtime.h"

namespace ernie {

BlockFile load_block_files(const Device& device, int index, const std::string& param_path,
                           const std::string& bin_path, int storage_dtype, bool allow_unreviewed,
                           const std::string& expected_bin_sha256)
{
    if (storage_dtype != ERNIE_DTYPE_FP32 && storage_dtype != ERNIE_DTYPE_FP16 && storage_dtype != ERNIE_DTYPE_BF16)
        throw std::invalid_argument("invalid storage dtype");
    if (bin_path.empty()) throw std::invalid_argument("a weight file is required to load a block");
    const MappedFile bin(bin_path);
    BlockFile f = inspect_block_bytes(param_path, bin.data(), bin.size(), allow_unreviewed, expected_bin_sha256);
    ernie_host_tensor t[11];
    for (int i = 0; i < 11; ++i) t[i] = {bin.data() + f.sections[i].data, f.sections[i].dtype};
    // Section order is the field order of ernie_block_host_tensors.
    const ernie_block_host_tensors w = {t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8], t[9], t[10]};
    check_status(ernie_hip_block_upload_tensors(device.ctx(), index, &w, f.graph.dim, f.graph.ffn, storage_dtype),
                 device.ctx(), "block upload");
    return f;
}

}  // namespace ernie
