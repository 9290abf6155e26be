// r97/params.h -- named f32 tensors: the trainable parameters and, under the same names, a step's
// gradients (the reference's include/r97/params.h contract).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace r97 {

struct Param {
    std::string name;            // e.g. "model.layers.3.mlp.down_proj.lora_A"
    std::vector<int64_t> shape;  // row-major
    std::vector<float> value;    // product(shape) elements
};

using ParamSet = std::vector<Param>;

}  // namespace r97
