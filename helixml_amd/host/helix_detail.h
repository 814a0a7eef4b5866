// helix_detail.h — error helpers shared by the host-layer sources (not part of the public API).
// Messages follow the reference's TensorError Display strings
// (crates/tensor-core/src/error.rs:7-37).
#pragma once

#include <string>
#include <vector>

#include "helix/helix.hpp"

namespace helix {
namespace detail {

inline std::string fmt_dims(const std::vector<size_t>& v) {
    std::string s = "[";
    for (size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + std::to_string(v[i]);
    return s + "]";
}

// "Shape mismatch: expected {expected:?}, got {actual:?}"
[[noreturn]] inline void shape_mismatch(const std::vector<size_t>& expected,
                                        const std::vector<size_t>& actual) {
    throw TensorError(ErrorKind::ShapeMismatch,
                      "Shape mismatch: expected " + fmt_dims(expected) + ", got " + fmt_dims(actual));
}

// "Invalid dimension: {dim} is out of bounds for shape {shape:?}"
[[noreturn]] inline void invalid_dimension(size_t dim, const std::vector<size_t>& shape) {
    throw TensorError(ErrorKind::InvalidDimension, "Invalid dimension: " + std::to_string(dim) +
                                                       " is out of bounds for shape " + fmt_dims(shape));
}

// "Operation not supported: {op}"
[[noreturn]] inline void unsupported(const std::string& op) {
    throw TensorError(ErrorKind::UnsupportedOperation, "Operation not supported: " + op);
}

// "Invalid input: {message}"
[[noreturn]] inline void invalid_input(const std::string& msg) {
    throw TensorError(ErrorKind::InvalidInput, "Invalid input: " + msg);
}

}  // namespace detail
}  // namespace helix
