// runtime.cpp -- Context, the memory pool and Tensor storage over the C ABI
// (the reference's src/core/context.cpp, runtime.cpp and tensor.cpp).
#include "runtime.hpp"

#include <algorithm>
#include <cstring>

namespace vkml {

namespace detail {

void check(int status, const char* what) {
    if (status == VKML_OK) return;
    std::string msg = vkml_last_error();
    if (what) msg = std::string(what) + ": " + msg;
    throw Error(msg);
}

std::int64_t numel_of(const Shape& shape) {
    std::int64_t n = 1;
    for (std::int64_t d : shape) {
        if (d < 0) throw Error("Tensor: negative dimension in " + to_string(shape));
        n *= d;
    }
    return n;
}

std::uint32_t type_code(DType dtype) {
    switch (dtype) {
        case DType::F32: return VKML_F32;
        case DType::F16: return VKML_F16;
        case DType::BF16: return VKML_BF16;
        case DType::I32: return VKML_I32;
    }
    return VKML_F32;
}

namespace {
// 4 KiB rounding below 1 MiB (the reference's pool, runtime.cpp:47-62),
// 1 MiB above, so large weights do not waste much.
std::uint64_t round_size(std::uint64_t bytes) {
    const std::uint64_t unit = bytes < (1u << 20) ? 4096 : (1u << 20);
    return std::max<std::uint64_t>(unit, (bytes + unit - 1) / unit * unit);
}
}  // namespace

Runtime::Runtime(const ContextOptions& options) : options_(options) {
    // A process that already drives the C ABI directly keeps its device; the
    // Context then shares it and leaves its shutdown to that owner.
    owns_device_ = vkml_is_initialized() == 0;
    if (owns_device_) check(vkml_init(options.device_name.c_str()), "Context");
    vkml_device_info d{};
    check(vkml_get_device_info(&d), "Context");
    info_.name = d.name;
    info_.vendor = "AMD";
    info_.driver = d.driver;
    info_.arch = d.arch;
    info_.type = DeviceType::DiscreteGpu;
    info_.device_local_bytes = d.global_memory_bytes;
    info_.compute_units = d.compute_units;
    info_.subgroup_size = d.wave_size;
    info_.max_workgroup_invocations = d.max_threads_per_block;
    for (int i = 0; i < 3; ++i) {
        info_.max_workgroup_size[i] = d.max_block_dims[i];
        info_.max_workgroup_count[i] = d.max_grid_dims[i];
    }
    info_.max_shared_memory_bytes = d.lds_bytes_per_block;
    info_.max_storage_buffer_range = d.global_memory_bytes;
    info_.min_storage_buffer_offset_alignment = 256;
    info_.timestamps = d.timestamps != 0;
    info_.timestamp_period_ns = d.timestamp_period_ns;
    info_.integer_dot_product = d.integer_dot_product != 0;
}

Runtime::~Runtime() {
    (void)vkml_synchronize();
    for (auto& [size, ptr] : free_) (void)vkml_free(ptr);
    free_.clear();
    if (owns_device_) (void)vkml_shutdown();
}

void* Runtime::acquire(std::uint64_t bytes, std::uint64_t& rounded) {
    rounded = round_size(bytes);
    auto it = free_.find(rounded);
    if (it != free_.end()) {
        void* p = it->second;
        free_.erase(it);
        pooled_bytes_ -= rounded;
        return p;
    }
    void* p = nullptr;
    int status = vkml_malloc(rounded, &p);
    if (status == VKML_ERROR_OUT_OF_MEMORY && !free_.empty()) {
        // Give the pool back and try once more.
        (void)vkml_synchronize();
        for (auto& [size, ptr] : free_) (void)vkml_free(ptr);
        free_.clear();
        pooled_bytes_ = 0;
        status = vkml_malloc(rounded, &p);
    }
    check(status, ("allocating " + std::to_string(bytes) + " bytes").c_str());
    return p;
}

void Runtime::release(void* ptr, std::uint64_t rounded) noexcept {
    if (!ptr) return;
    free_.emplace(rounded, ptr);
    pooled_bytes_ += rounded;
}

void Runtime::synchronize() { check(vkml_synchronize(), "synchronize"); }

Storage::~Storage() {
    if (runtime) runtime->release(ptr, bytes);
}

Runtime& TensorAccess::runtime(const Tensor& t) {
    if (!t.storage_ || !t.storage_->runtime) throw Error("Tensor: no storage");
    return *t.storage_->runtime;
}

}  // namespace detail

// ---------------------------------------------------------------- Context

std::string_view to_string(DeviceType type) noexcept {
    switch (type) {
        case DeviceType::IntegratedGpu: return "integrated GPU";
        case DeviceType::DiscreteGpu: return "discrete GPU";
        case DeviceType::VirtualGpu: return "virtual GPU";
        case DeviceType::Cpu: return "CPU";
        case DeviceType::Other: break;
    }
    return "other";
}

std::string_view to_string(DType dtype) noexcept {
    switch (dtype) {
        case DType::F32: return "f32";
        case DType::F16: return "f16";
        case DType::BF16: return "bf16";
        case DType::I32: return "i32";
    }
    return "?";
}

std::string to_string(const Shape& shape) {
    std::string s = "[";
    for (std::size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

Context::Context(ContextOptions options) : runtime_(std::make_unique<detail::Runtime>(options)) {}
Context::~Context() = default;
Context::Context(Context&&) noexcept = default;
Context& Context::operator=(Context&&) noexcept = default;

const DeviceInfo& Context::device_info() const noexcept { return runtime_->info(); }
const ContextOptions& Context::options() const noexcept { return runtime_->options(); }

void Context::set_profiling(bool enabled) { detail::check(vkml_set_profiling(enabled ? 1 : 0), "set_profiling"); }
bool Context::profiling() const noexcept { return vkml_get_profiling() != 0; }

std::vector<KernelTime> Context::profile() const {
    std::uint32_t count = 0;
    detail::check(vkml_profile(nullptr, 0, &count), "profile");
    std::vector<vkml_kernel_time> rows(count);
    detail::check(vkml_profile(rows.data(), count, &count), "profile");
    std::vector<KernelTime> out;
    for (std::uint32_t i = 0; i < count && i < rows.size(); ++i) out.push_back({rows[i].name, rows[i].calls, rows[i].milliseconds});
    return out;
}

void Context::reset_profile() { detail::check(vkml_reset_profile(), "reset_profile"); }
void Context::synchronize() { runtime_->synchronize(); }

// ---------------------------------------------------------------- Tensor

Tensor::Tensor(std::shared_ptr<detail::Storage> storage, Shape shape, DType dtype, std::int64_t numel)
    : storage_(std::move(storage)), shape_(std::move(shape)), dtype_(dtype), numel_(numel) {}

Tensor Tensor::empty(detail::Runtime& runtime, Shape shape, DType dtype) {
    const std::int64_t n = detail::numel_of(shape);
    auto storage = std::make_shared<detail::Storage>();
    storage->runtime = &runtime;
    const std::uint64_t bytes = static_cast<std::uint64_t>(n) * element_size(dtype);
    if (bytes > 0) storage->ptr = runtime.acquire(bytes, storage->bytes);
    return Tensor(std::move(storage), std::move(shape), dtype, n);
}

Tensor Tensor::empty(Context& context, Shape shape, DType dtype) { return empty(context.runtime(), std::move(shape), dtype); }

Tensor Tensor::zeros(Context& context, Shape shape, DType dtype) {
    Tensor t = empty(context, std::move(shape), dtype);
    if (t.nbytes() > 0) detail::check(vkml_fill_u32(t.data(), 0u, (t.nbytes() + 3) / 4), "Tensor::zeros");
    return t;
}

Tensor Tensor::from_bytes(Context& context, std::span<const std::byte> bytes, Shape shape, DType dtype) {
    const std::int64_t n = detail::numel_of(shape);
    if (bytes.size() != static_cast<std::size_t>(n) * element_size(dtype)) {
        throw Error("Tensor::from_bytes: " + std::to_string(bytes.size()) + " bytes for " + to_string(shape) + " " +
                    std::string(to_string(dtype)) + ", which needs " + std::to_string(n * element_size(dtype)));
    }
    Tensor t = empty(context, std::move(shape), dtype);
    if (!bytes.empty()) detail::check(vkml_memcpy_h2d(t.data(), bytes.data(), bytes.size()), "Tensor::from_bytes");
    return t;
}

std::vector<std::byte> Tensor::to_bytes() const {
    std::vector<std::byte> out(nbytes());
    if (!out.empty()) detail::check(vkml_memcpy_d2h(out.data(), data(), out.size()), "Tensor::to_bytes");
    return out;
}

void* Tensor::data() const noexcept { return storage_ ? storage_->ptr : nullptr; }

Tensor Tensor::reshape(Shape shape) const {
    int infer = -1;
    std::int64_t known = 1;
    for (std::size_t i = 0; i < shape.size(); ++i) {
        if (shape[i] == -1) {
            if (infer >= 0) throw Error("Tensor::reshape: more than one -1 in " + to_string(shape));
            infer = static_cast<int>(i);
        } else if (shape[i] < 0) {
            throw Error("Tensor::reshape: negative dimension in " + to_string(shape));
        } else {
            known *= shape[i];
        }
    }
    if (infer >= 0) {
        if (known == 0 || numel_ % known != 0) {
            throw Error("Tensor::reshape: cannot reshape " + to_string(shape_) + " to " + to_string(shape));
        }
        shape[static_cast<std::size_t>(infer)] = numel_ / known;
        known = numel_;
    }
    if (known != numel_) throw Error("Tensor::reshape: cannot reshape " + to_string(shape_) + " to " + to_string(shape));
    return Tensor(storage_, std::move(shape), dtype_, numel_);
}

}  // namespace vkml
