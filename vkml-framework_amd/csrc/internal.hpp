// internal.hpp -- host-side state shared by the C ABI's translation units:
// the stream, error reporting, and the profiled launch wrapper.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/vkml_hip.h"

namespace vkml::abi {

// The last error on this thread; returns code.
int fail(int code, const std::string& message);
int hip_fail(hipError_t e, const char* what);

bool initialized();
hipStream_t stream();
int device_index();
uint32_t compute_units();

// Profiling: begin() records a start event when profiling is on (not while
// capturing a graph); end(label) records the stop and queues the pair.
struct ProfileScope {
    explicit ProfileScope(const char* label);
    ~ProfileScope();
    const char* label;
    void* start = nullptr;
};

// Checks the launch that just happened.
int check_launch(const char* what);

// Polls a workgroup waiting for another of its launch makes before giving
// up (vkml_set_wait_limit; default 1 << 20).
uint32_t wait_limit();
void set_wait_limit(uint32_t polls);

// The device address of vkml_attend_step_noalloc's scratch on the current
// device (k_attend.hip); vkml_init calls it once per device.
int attend_scratch_setup(int device);

}  // namespace vkml::abi

#define VKML_REQUIRE_INIT()                                                              \
    do {                                                                                 \
        if (!::vkml::abi::initialized())                                                 \
            return ::vkml::abi::fail(VKML_ERROR_STATE, "vkml: vkml_init has not been called"); \
    } while (0)

#define VKML_CHECK_ARG(cond, msg)                                                 \
    do {                                                                          \
        if (!(cond)) return ::vkml::abi::fail(VKML_ERROR_INVALID_ARGUMENT, (msg)); \
    } while (0)
