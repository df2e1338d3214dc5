// weights_dir.h -- reader for the SSLA weight directory (weights.npz +
// meta.json) in the schema written by tools/make_ssla_stub.py:29-149.
//
// Host code only.  Replaces vendor/src/weights_loader.cpp (load_meta
// :162-252, load_weights_npz :255-350) for the keys this path needs.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace ssla {

struct NpzTensor {
    std::vector<int64_t> shape;
    std::vector<float>   data;
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

struct ModelMeta {
    int schema_version = 0;
    std::string model;
    int height = 0;
    int width = 0;
    int num_classes = 0;
    int ssla_tdrop_window = 0;
};

// Both throw std::runtime_error with a message naming the file and field.
ModelMeta read_meta(const std::string& dir);
std::map<std::string, NpzTensor> read_npz(const std::string& dir);

}  // namespace ssla
