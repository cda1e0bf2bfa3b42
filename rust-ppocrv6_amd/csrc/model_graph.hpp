// The recognition head inside a model file's graph (see model_graph.cpp).
#pragma once
#include <stdint.h>

#include <string>

#include "safetensors.hpp"

namespace ppocr {

struct RecHeadNames {
    std::string weight;   // F32 [k][n] MatMul weight
    std::string bias;     // F32 [n] bias folded from the Add, "" when none
    std::string softmax;  // the Softmax node
    int64_t n = 0, k = 0;
};

// Finds the first MatMul -> [Add bias] -> Softmax(last axis) -> graph output segment.
// Returns PPOCR_OK, or PPOCR_ERR_MODEL with the message set.
int find_rec_head(const StFile& f, RecHeadNames* out);

}  // namespace ppocr
