#pragma once

#include <array>
#include <cstdint>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

#include "vkml/error.hpp"

namespace vkml {

namespace detail {
class Runtime;
}  // namespace detail

enum class DeviceType : std::uint8_t { Other, IntegratedGpu, DiscreteGpu, VirtualGpu, Cpu };

std::string_view to_string(DeviceType type) noexcept;

// The selected GPU (reference: include/vkml/context.hpp:28-70), filled from
// HIP's device properties. Vulkan-only fields keep their meaning where HIP
// has one (a "workgroup" is a HIP block, "subgroup" a wave64).
struct DeviceInfo {
    struct Version {
        std::uint32_t major = 0, minor = 0, patch = 0;
    };

    std::string name;
    std::string vendor;
    std::string driver;
    std::string arch;  // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
    DeviceType type = DeviceType::Other;
    Version api_version;

    bool unified_memory = false;
    std::uint64_t device_local_bytes = 0;

    std::uint32_t compute_units = 0;
    std::uint32_t subgroup_size = 0;
    std::uint32_t max_workgroup_invocations = 0;
    std::array<std::uint32_t, 3> max_workgroup_size{};
    std::array<std::uint32_t, 3> max_workgroup_count{};
    std::uint32_t max_shared_memory_bytes = 0;
    std::uint32_t max_push_constant_bytes = 0;

    std::uint64_t max_storage_buffer_range = 0;
    std::uint64_t min_storage_buffer_offset_alignment = 0;
    std::uint64_t non_coherent_atom_size = 0;

    bool validation_enabled = false;

    bool timestamps = false;
    double timestamp_period_ns = 0.0;

    // int8 dot products (v_dot4_i32_i8): always available on gfx950.
    bool integer_dot_product = false;
};

// GPU time of one kernel label (or "copy"), from Context::profile.
struct KernelTime {
    std::string name;
    std::uint64_t calls = 0;
    double milliseconds = 0.0;
};

struct ContextOptions {
    // Case-insensitive substring of the device name (or arch) to use; when
    // empty, the VKML_DEVICE environment variable, then device 0.
    std::string device_name;

    // Kept for source compatibility: HIP has no validation layers. Launch
    // errors are always checked and thrown.
    bool enable_validation = false;

    // Use int8 dot products for matrix-vector products with quantized
    // weights (the activations are quantized to Q8_0 on the fly); off,
    // quantized weights multiply f32 activations as they are.
    bool integer_dot_product = true;
};

// Owns the HIP device, its stream and the memory pool. Create one and keep it
// alive while any tensor is in use. One Context per process at a time, as
// in the reference (a second throws vkml::Error).
class Context {
public:
    explicit Context(ContextOptions options = {});
    ~Context();

    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    Context(Context&&) noexcept;
    Context& operator=(Context&&) noexcept;

    const DeviceInfo& device_info() const noexcept;
    const ContextOptions& options() const noexcept;

    // Always 0: there are no validation layers (reference: context.hpp:110).
    std::uint32_t validation_error_count() const noexcept { return 0; }

    // Profiling brackets every kernel with HIP events and totals them per
    // label; graphs are not replayed while it is on, so every kernel shows.
    // profile() covers finished work, slowest first.
    void set_profiling(bool enabled);
    bool profiling() const noexcept;
    std::vector<KernelTime> profile() const;
    void reset_profile();

    // Waits for all work submitted so far.
    void synchronize();

    detail::Runtime& runtime() noexcept { return *runtime_; }

private:
    std::unique_ptr<detail::Runtime> runtime_;
};

}  // namespace vkml
