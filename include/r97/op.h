// r97/op.h -- one record of the op tape: the drop-in restatement of the reference's record type
// (include/r97/op.h of Code000-211/R9700Training), field for field, so a row written against the
// reference's contract compiles against this one unchanged.
//
// A record names its operands in schema order; `Operand::buffer` carries the schema name a row
// looks an operand up by ("a", "b", "lora_a", "t", ...).
#pragma once

#include <cstdint>
#include <string>
#include <utility>
#include <variant>
#include <vector>

namespace r97 {

struct Operand {
    std::string buffer;          // the operand's name on the tape (its schema name)
    std::string dtype;           // element type as the op reads it ("bf16", "f32", "invalid", ...)
    std::vector<int64_t> shape;  // full logical shape, row-major
    int64_t row_lo = 0;          // first row the op touches
    int64_t rows = 0;            // rows the op touches; 0 = the whole operand
    bool written = false;        // written (true) or read (false)
    bool in_place = false;       // a write that also reads the value it replaces
    std::vector<int64_t> view_shape;   // the tensor the kernel saw, when not the declared one
    std::vector<int64_t> view_stride;  // ... in elements of the declared layout
    int64_t view_off = 0;              // ... and its first element's offset
    const void* enc = nullptr;   // a stored weight's encoding, when its bytes are not one span
};

struct OpRecord {
    std::string op;  // the op's schema name
    std::vector<std::pair<std::string, std::variant<int64_t, std::string>>> params;
    std::vector<Operand> operands;  // schema order
    int64_t block = -1;             // transformer block, -1 outside one
    int64_t position = 0;           // append order within the step
    int64_t n = 0;                  // the ranged count the issue resolved to
};

}  // namespace r97
