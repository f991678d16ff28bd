// ModelLoader: the reference's model.bin reader (include/model_loader.h,
// src/model_loader.cu:14-53 of the reference), same API and messages.
//
// model.bin format (all little-endian, offsets absolute from file start):
//   u32 count
//   count x { u32 name_len; name_len bytes of name; u32 ndim; ndim x u32 dim;
//             u64 offset; u64 bytes }
//   tensor data: fp32, row-major, `bytes` bytes at `offset`
// The index is parsed once; load(name) reads one tensor into a Tensor and
// uploads it to the device (weights stay resident, as in the reference).
//
// Errors (std::runtime_error, the reference's messages): "cannot open model:
// <path>", "truncated model.bin", "missing tensor: <name>", "tensor is not
// float32: <name>", "cannot reopen model: <path>", "truncated tensor: <name>".
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "tensor.h"

class ModelLoader {
public:
    explicit ModelLoader(const std::string& path);
    Tensor load(const std::string& name) const;
    bool has(const std::string& name) const { return entries_.count(name) != 0; }

private:
    struct Entry {
        std::vector<std::size_t> shape;
        std::uint64_t offset = 0;
        std::uint64_t bytes = 0;
    };
    std::string path_;
    std::unordered_map<std::string, Entry> entries_;
};
