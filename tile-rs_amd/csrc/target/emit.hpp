// The hip target's pure emit function (MLIR text -> HIP source).
#pragma once

#include <string>
#include <vector>

namespace th {
namespace target {

// Pure and deterministic.  On success fills `out` and the emitted kernel names;
// on failure returns false with a message in `err`.
bool convert_mlir_to_hip(const std::string& mlir_text, std::string* out,
                         std::vector<std::string>* kernel_names, std::string* err);

}  // namespace target
}  // namespace th
