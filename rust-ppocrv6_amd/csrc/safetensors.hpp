// Read-only view of a safetensors model file (the format load_safetensors_model reads,
// src/engine/loader.rs:34-92): an 8-byte little-endian header length, a JSON header
// mapping tensor names to {"dtype", "shape", "data_offsets"} (plus "__metadata__"), then
// the tensor bytes.  The file is memory-mapped; a tensor is a pointer into the map.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <utility>
#include <vector>

namespace ppocr {

struct StTensor {
    std::string name;
    std::string dtype;           // "F32", "I64", ...
    std::vector<int64_t> shape;  // row-major
    const uint8_t* data = nullptr;
    size_t bytes = 0;
};

class StFile {
public:
    StFile() = default;
    StFile(const StFile&) = delete;
    StFile& operator=(const StFile&) = delete;
    ~StFile();
    // Maps and parses the file.  Returns PPOCR_OK or an error (message set).
    int open(const char* path);
    // Looks a tensor up by name; null when absent.
    const StTensor* find(const char* name) const;
    const std::vector<StTensor>& tensors() const { return tensors_; }
    // A "__metadata__" entry by key; null when absent.
    const std::string* metadata(const char* key) const {
        for (const auto& kv : metadata_)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }

private:
    void* map_ = nullptr;
    size_t size_ = 0;
    std::vector<StTensor> tensors_;
    std::vector<std::pair<std::string, std::string>> metadata_;
};

// Bytes per element of a safetensors dtype (0 for an unknown one).
size_t st_dtype_size(const std::string& dtype);

}  // namespace ppocr
