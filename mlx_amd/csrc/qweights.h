// qweights.h -- quantized linear layers in safetensors files (host code).
// The format and the layer layout are documented beside
// lux_quant_linear_info in lux_gpu_quant_backend.h.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "../../include/lux_gpu_quant_backend.h"

namespace lxq {

// a read-only memory map of a whole file
struct MappedFile {
    const uint8_t* data = nullptr;
    size_t size = 0;
    MappedFile() = default;
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    ~MappedFile();
    bool open(const char* path);  // false: missing, unreadable, or empty
};

// parse the header of `path` and describe layer `prefix`; group_size / bits
// 0 = take them from the file's string entries
LuxBackendError linear_describe(const char* path, const char* prefix, int group_size, int bits,
                                lux_quant_linear_info* out);

}  // namespace lxq
