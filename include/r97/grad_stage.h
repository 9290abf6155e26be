// r97/grad_stage.h -- where a step's trainable gradients wait on the card: the reference's
// src/adjoint/device/grad_stage.h:1-45 contract, restated.
//
// A device row adds its call's factor gradient into the step's f32 accumulator for the leaf
// (grad_stage_slot, by the leaf's name and shape: allocated and zeroed on the step's first ask,
// the same buffer on every later ask of the step). The walk ends the step with grad_stage_flush,
// which rounds each accumulator once from its f32 total to bf16 and adds it into the ParamSet leaf
// of that name (made when the step has not made it yet), then frees the staging; or with
// grad_stage_discard, which only frees it.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "r97/params.h"

namespace r97 {
namespace device {

// The step's f32 accumulator (device memory) for the leaf `name` of `shape`; nullptr when the card
// refuses it (no memory, an empty shape, or the name asked for before with another shape).
float* grad_stage_slot(const std::string& name, const std::vector<int64_t>& shape);
// The bytes of the step's staged f32 accumulators (0 once the step is flushed or discarded).
int64_t grad_stage_bytes();
// Each accumulator, rounded once to bf16, added into `grads`; the staging freed. False when a copy
// failed or a leaf of that name has another shape (the staging is freed either way).
bool grad_stage_flush(ParamSet* grads);
// The staging freed, nothing copied out.
void grad_stage_discard();

}  // namespace device
}  // namespace r97
