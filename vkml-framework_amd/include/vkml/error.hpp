#pragma once

#include <stdexcept>

namespace vkml {

// Thrown for every failure vkml reports: no suitable GPU, a failed HIP call,
// invalid arguments. The message says what was being attempted.
// (Reference: include/vkml/error.hpp:7-12.)
class Error : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

}  // namespace vkml
