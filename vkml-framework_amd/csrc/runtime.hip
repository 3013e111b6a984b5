// runtime.hip -- device lifecycle, memory, stream timeline, profiling and
// graphs of the C ABI (include/vkml_hip.h). Replaces the reference's Vulkan
// HAL (src/hal/device.cpp, buffer.cpp, stream.cpp) with one HIP device and
// one in-order HIP stream at default priority.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "internal.hpp"

namespace vkml::abi {
namespace {

thread_local std::string g_error;

struct Pending {
    std::string label;
    hipEvent_t start, stop;
};

struct Fence {
    uint64_t value;
    hipEvent_t event;
};

struct State {
    bool ready = false;
    int device = -1;
    hipStream_t stream = nullptr;
    vkml_device_info info{};
    bool profiling = false;
    bool capturing = false;
    std::string tag;
    std::vector<Pending> pending;
    std::map<std::string, std::pair<uint64_t, double>> totals;  // label -> (calls, ms)
    std::deque<Fence> fences;
    uint64_t next_fence = 0, done_fence = 0;
    std::unordered_map<uint64_t, hipGraphExec_t> graphs;
    std::unordered_map<uint64_t, hipGraph_t> graph_sources;
    uint64_t next_graph = 1;
};

State g;

std::string lower(std::string s) {
    for (char& c : s) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
    return s;
}

// Folds finished profiled launches into the totals (Stream::wait's
// timestamp collection, src/hal/stream.cpp:258-306).
void collect_profile(bool all) {
    std::vector<Pending> keep;
    for (Pending& p : g.pending) {
        if (!all && hipEventQuery(p.stop) != hipSuccess) {
            keep.push_back(p);
            continue;
        }
        float ms = 0.0f;
        if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            auto& t = g.totals[p.label];
            t.first += 1;
            t.second += ms;
        }
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    g.pending.swap(keep);
}

void release_fences_upto(uint64_t value) {
    while (!g.fences.empty() && g.fences.front().value <= value) {
        (void)hipEventDestroy(g.fences.front().event);
        g.fences.pop_front();
    }
    g.done_fence = std::max(g.done_fence, value);
}

__global__ void k_fill_u32(uint32_t* dst, uint32_t value, uint64_t words) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride) dst[i] = value;
}

}  // namespace

int fail(int code, const std::string& message) {
    g_error = message;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(e == hipErrorOutOfMemory ? VKML_ERROR_OUT_OF_MEMORY : VKML_ERROR_DEVICE,
                std::string(what) + ": " + hipGetErrorString(e));
}

bool initialized() { return g.ready; }
hipStream_t stream() { return g.stream; }
int device_index() { return g.device; }
uint32_t compute_units() { return g.info.compute_units; }

ProfileScope::ProfileScope(const char* l) : label(l) {
    if (g.profiling && !g.capturing) {
        hipEvent_t e;
        if (hipEventCreate(&e) == hipSuccess) {
            (void)hipEventRecord(e, g.stream);
            start = e;
        }
    }
}

ProfileScope::~ProfileScope() {
    if (!start) return;
    hipEvent_t stop;
    if (hipEventCreate(&stop) == hipSuccess) {
        (void)hipEventRecord(stop, g.stream);
        g.pending.push_back({g.tag.empty() ? std::string(label) : std::string(label) + ":" + g.tag,
                             static_cast<hipEvent_t>(start), stop});
    } else {
        (void)hipEventDestroy(static_cast<hipEvent_t>(start));
    }
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    return VKML_OK;
}

namespace {
uint32_t g_wait_limit = 1u << 20;
}  // namespace

uint32_t wait_limit() { return g_wait_limit; }
void set_wait_limit(uint32_t polls) { g_wait_limit = polls; }

}  // namespace vkml::abi

using namespace vkml::abi;

extern "C" {

const char* vkml_last_error(void) { return g_error.c_str(); }
int vkml_abi_version(void) { return VKML_ABI_VERSION; }
int vkml_is_initialized(void) { return g.ready ? 1 : 0; }

int vkml_init(const char* device_name) {
    if (g.ready) return fail(VKML_ERROR_STATE, "vkml_init: a context is already alive in this process");
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return fail(VKML_ERROR_NO_DEVICE, "vkml_init: no HIP device is visible");
    std::string want = device_name ? device_name : "";
    if (want.empty()) {
        if (const char* env = std::getenv("VKML_DEVICE")) want = env;
    }
    want = lower(want);
    int chosen = -1;
    std::string names;
    for (int i = 0; i < count; ++i) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) != hipSuccess) continue;
        const std::string name = lower(prop.name), arch = lower(prop.gcnArchName);
        names += (names.empty() ? "" : ", ") + std::string(prop.name);
        if (want.empty() || name.find(want) != std::string::npos || arch.find(want) != std::string::npos ||
            want == std::to_string(i)) {
            chosen = i;
            break;
        }
    }
    if (chosen < 0) return fail(VKML_ERROR_NO_DEVICE, "vkml_init: no device matches \"" + want + "\" (have " + names + ")");
    if ((e = hipSetDevice(chosen)) != hipSuccess) return hip_fail(e, "vkml_init: hipSetDevice");
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, chosen)) != hipSuccess) return hip_fail(e, "vkml_init: properties");
    if ((e = hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking)) != hipSuccess) return hip_fail(e, "vkml_init: stream");
    vkml_device_info& info = g.info;
    std::memset(&info, 0, sizeof info);
    std::snprintf(info.name, sizeof info.name, "%s", prop.name);
    std::snprintf(info.arch, sizeof info.arch, "%s", prop.gcnArchName);
    int runtime = 0;
    (void)hipRuntimeGetVersion(&runtime);
    std::snprintf(info.driver, sizeof info.driver, "HIP %d.%d.%d", runtime / 10000000, runtime / 100000 % 100, runtime % 100000);
    info.global_memory_bytes = prop.totalGlobalMem;
    info.compute_units = static_cast<uint32_t>(prop.multiProcessorCount);
    info.wave_size = static_cast<uint32_t>(prop.warpSize);
    info.max_threads_per_block = static_cast<uint32_t>(prop.maxThreadsPerBlock);
    for (int i = 0; i < 3; ++i) {
        info.max_block_dims[i] = static_cast<uint32_t>(prop.maxThreadsDim[i]);
        info.max_grid_dims[i] = static_cast<uint32_t>(prop.maxGridSize[i]);
    }
    info.lds_bytes_per_block = static_cast<uint32_t>(prop.sharedMemPerBlock);
    info.l2_bytes = static_cast<uint32_t>(prop.l2CacheSize);
    info.clock_khz = static_cast<uint32_t>(prop.clockRate);
    info.memory_clock_khz = static_cast<uint32_t>(prop.memoryClockRate);
    info.memory_bus_bits = static_cast<uint32_t>(prop.memoryBusWidth);
    info.integer_dot_product = 1;
    info.timestamps = 1;
    info.timestamp_period_ns = 1.0;
    if (int r = attend_scratch_setup(chosen)) {
        (void)hipStreamDestroy(g.stream);
        g.stream = nullptr;
        return r;
    }
    g.device = chosen;
    g.ready = true;
    return VKML_OK;
}

int vkml_shutdown(void) {
    if (!g.ready) return VKML_OK;
    (void)hipStreamSynchronize(g.stream);
    collect_profile(true);
    release_fences_upto(UINT64_MAX);
    for (auto& [id, exec] : g.graphs) (void)hipGraphExecDestroy(exec);
    for (auto& [id, graph] : g.graph_sources) (void)hipGraphDestroy(graph);
    g.graphs.clear();
    g.graph_sources.clear();
    (void)hipStreamDestroy(g.stream);
    g = State{};
    return VKML_OK;
}

int vkml_get_device_info(vkml_device_info* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(out, "vkml_get_device_info: null output");
    *out = g.info;
    return VKML_OK;
}

int vkml_malloc(uint64_t bytes, void** out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(out, "vkml_malloc: null output");
    *out = nullptr;
    if (bytes == 0) return VKML_OK;
    const hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(e, ("vkml_malloc of " + std::to_string(bytes) + " bytes").c_str());
    }
    return VKML_OK;
}

int vkml_free(void* ptr) {
    VKML_REQUIRE_INIT();
    if (!ptr) return VKML_OK;
    const hipError_t e = hipFree(ptr);
    return e == hipSuccess ? VKML_OK : hip_fail(e, "vkml_free");
}

int vkml_host_malloc(uint64_t bytes, void** out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(out, "vkml_host_malloc: null output");
    *out = nullptr;
    if (bytes == 0) return VKML_OK;
    const hipError_t e = hipHostMalloc(out, bytes, hipHostMallocDefault);
    return e == hipSuccess ? VKML_OK : hip_fail(e, "vkml_host_malloc");
}

int vkml_host_free(void* ptr) {
    VKML_REQUIRE_INIT();
    if (!ptr) return VKML_OK;
    const hipError_t e = hipHostFree(ptr);
    return e == hipSuccess ? VKML_OK : hip_fail(e, "vkml_host_free");
}

static int copy(void* dst, const void* src, uint64_t bytes, hipMemcpyKind kind, const char* what) {
    VKML_REQUIRE_INIT();
    if (bytes == 0) return VKML_OK;
    VKML_CHECK_ARG(dst && src, std::string(what) + ": null pointer");
    ProfileScope prof("copy");
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, g.stream);
    return e == hipSuccess ? VKML_OK : hip_fail(e, what);
}

int vkml_memcpy_h2d(void* d, const void* h, uint64_t bytes) { return copy(d, h, bytes, hipMemcpyHostToDevice, "vkml_memcpy_h2d"); }
int vkml_memcpy_d2d(void* d, const void* s, uint64_t bytes) { return copy(d, s, bytes, hipMemcpyDeviceToDevice, "vkml_memcpy_d2d"); }

int vkml_memcpy_d2h(void* h, const void* d, uint64_t bytes) {
    const int r = copy(h, d, bytes, hipMemcpyDeviceToHost, "vkml_memcpy_d2h");
    if (r != VKML_OK) return r;
    // The host reads the data right away: wait for it (Tensor::to_bytes).
    const hipError_t e = hipStreamSynchronize(g.stream);
    if (e != hipSuccess) return hip_fail(e, "vkml_memcpy_d2h: synchronize");
    collect_profile(false);
    return VKML_OK;
}

int vkml_fill_u32(void* dst, uint32_t value, uint64_t words) {
    VKML_REQUIRE_INIT();
    if (words == 0) return VKML_OK;
    VKML_CHECK_ARG(dst, "vkml_fill_u32: null pointer");
    ProfileScope prof("fill");
    const uint64_t blocks = std::min<uint64_t>((words + 255) / 256, 4096);
    hipLaunchKernelGGL(k_fill_u32, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, g.stream,
                       static_cast<uint32_t*>(dst), value, words);
    return check_launch("vkml_fill_u32");
}

int vkml_submit(uint64_t* fence_out) {
    VKML_REQUIRE_INIT();
    hipEvent_t e;
    hipError_t err = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (err != hipSuccess) return hip_fail(err, "vkml_submit");
    if ((err = hipEventRecord(e, g.stream)) != hipSuccess) {
        (void)hipEventDestroy(e);
        return hip_fail(err, "vkml_submit: record");
    }
    g.fences.push_back({++g.next_fence, e});
    if (fence_out) *fence_out = g.next_fence;
    return VKML_OK;
}

int vkml_wait(uint64_t fence) {
    VKML_REQUIRE_INIT();
    if (fence <= g.done_fence) return VKML_OK;
    VKML_CHECK_ARG(fence <= g.next_fence, "vkml_wait: fence " + std::to_string(fence) + " was never submitted");
    for (const Fence& f : g.fences) {
        if (f.value >= fence) {
            const hipError_t e = hipEventSynchronize(f.event);
            if (e != hipSuccess) return hip_fail(e, "vkml_wait");
            break;
        }
    }
    release_fences_upto(fence);
    collect_profile(false);
    return VKML_OK;
}

int vkml_completed(uint64_t* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(out, "vkml_completed: null output");
    uint64_t done = g.done_fence;
    for (const Fence& f : g.fences) {
        if (hipEventQuery(f.event) != hipSuccess) break;
        done = f.value;
    }
    release_fences_upto(done);
    *out = done;
    return VKML_OK;
}

int vkml_synchronize(void) {
    VKML_REQUIRE_INIT();
    const hipError_t e = hipStreamSynchronize(g.stream);
    if (e != hipSuccess) return hip_fail(e, "vkml_synchronize");
    release_fences_upto(g.next_fence);
    collect_profile(true);
    return VKML_OK;
}

void* vkml_stream(void) { return g.ready ? static_cast<void*>(g.stream) : nullptr; }

int vkml_set_profiling(int enabled) {
    VKML_REQUIRE_INIT();
    g.profiling = enabled != 0;
    return VKML_OK;
}

int vkml_get_profiling(void) { return g.profiling ? 1 : 0; }

int vkml_set_wait_limit(uint32_t polls) {
    vkml::abi::set_wait_limit(polls == 0 ? (1u << 20) : polls);
    return VKML_OK;
}

int vkml_set_profile_tag(const char* tag) {
    g.tag = tag ? tag : "";
    return VKML_OK;
}

int vkml_profile(vkml_kernel_time* out, uint32_t capacity, uint32_t* count) {
    VKML_REQUIRE_INIT();
    collect_profile(false);
    std::vector<vkml_kernel_time> rows;
    for (const auto& [label, t] : g.totals) {
        vkml_kernel_time k{};
        std::snprintf(k.name, sizeof k.name, "%s", label.c_str());
        k.calls = t.first;
        k.milliseconds = t.second;
        rows.push_back(k);
    }
    std::sort(rows.begin(), rows.end(), [](const auto& a, const auto& b) { return a.milliseconds > b.milliseconds; });
    if (count) *count = static_cast<uint32_t>(rows.size());
    for (uint32_t i = 0; out && i < capacity && i < rows.size(); ++i) out[i] = rows[i];
    return VKML_OK;
}

int vkml_reset_profile(void) {
    VKML_REQUIRE_INIT();
    collect_profile(true);
    g.totals.clear();
    return VKML_OK;
}

int vkml_graph_begin(void) {
    VKML_REQUIRE_INIT();
    if (g.capturing) return fail(VKML_ERROR_STATE, "vkml_graph_begin: already capturing");
    const hipError_t e = hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(e, "vkml_graph_begin");
    g.capturing = true;
    return VKML_OK;
}

int vkml_graph_end(uint64_t* out) {
    VKML_REQUIRE_INIT();
    if (!g.capturing) return fail(VKML_ERROR_STATE, "vkml_graph_end: not capturing");
    g.capturing = false;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(g.stream, &graph);
    if (e != hipSuccess) return hip_fail(e, "vkml_graph_end: capture");
    hipGraphExec_t exec = nullptr;
    if ((e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(e, "vkml_graph_end: instantiate");
    }
    const uint64_t id = g.next_graph++;
    g.graphs[id] = exec;
    g.graph_sources[id] = graph;
    if (out) *out = id;
    return VKML_OK;
}

int vkml_graph_launch(uint64_t id) {
    VKML_REQUIRE_INIT();
    auto it = g.graphs.find(id);
    if (it == g.graphs.end()) return fail(VKML_ERROR_INVALID_ARGUMENT, "vkml_graph_launch: unknown graph");
    ProfileScope prof("graph");
    const hipError_t e = hipGraphLaunch(it->second, g.stream);
    return e == hipSuccess ? VKML_OK : hip_fail(e, "vkml_graph_launch");
}

int vkml_graph_destroy(uint64_t id) {
    VKML_REQUIRE_INIT();
    auto it = g.graphs.find(id);
    if (it == g.graphs.end()) return VKML_OK;
    (void)hipStreamSynchronize(g.stream);
    (void)hipGraphExecDestroy(it->second);
    g.graphs.erase(it);
    auto src = g.graph_sources.find(id);
    if (src != g.graph_sources.end()) {
        (void)hipGraphDestroy(src->second);
        g.graph_sources.erase(src);
    }
    return VKML_OK;
}

}  // extern "C"
