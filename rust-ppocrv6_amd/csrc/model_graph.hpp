// The recognition head inside a model file's graph (see model_graph.cpp).
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

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

// The SVTR mixing tail before the head (neck.hip): weight names and constants.
struct RecNeckBlockNames {
    std::string ln1_w, ln1_b, qkv_w, qkv_b, proj_w, proj_b, ln2_w, ln2_b, fc1_w, fc1_b, fc2_w, fc2_b;
    float ln1_eps = 0.0f, ln2_eps = 0.0f;
};
struct RecNeckNames {
    std::vector<RecNeckBlockNames> blocks;
    std::string lnf_w, lnf_b;
    float lnf_eps = 0.0f;
    int64_t dim = 0, heads = 0, hidden = 0;
    float scale = 0.0f;
    std::string input, shortcut;  // the tail's activations: the flatten before Transpose.0, the shortcut
};

// Finds, between the first LayerNorm sub-graph and the head's MatMul, the transformer
// blocks, the final LayerNorm and the shortcut Add.  PPOCR_OK, or PPOCR_ERR_MODEL.
int find_rec_neck(const StFile& f, RecNeckNames* out);

}  // namespace ppocr
