// runtime.hpp -- the C++ side of the backend seam (the reference's
// src/core/runtime.hpp and storage.hpp), over the C ABI of libvkml_hip.so.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "vkml/context.hpp"
#include "vkml/error.hpp"
#include "vkml/tensor.hpp"
#include "vkml_hip.h"

namespace vkml::detail {

// Throws vkml::Error with the library's message unless status is VKML_OK.
void check(int status, const char* what = nullptr);

// Device memory pool: freed buffers are kept by rounded size and handed out
// again. All work runs in order on one stream, so a buffer released while
// kernels that use it are queued is safe to reuse for later work on the
// same stream (the reference's retire-until-the-timeline-passes,
// src/core/runtime.cpp:30-62, is what stream order gives here).
class Runtime {
public:
    explicit Runtime(const ContextOptions& options);
    ~Runtime();

    void* acquire(std::uint64_t bytes, std::uint64_t& rounded);
    void release(void* ptr, std::uint64_t rounded) noexcept;

    const DeviceInfo& info() const noexcept { return info_; }
    const ContextOptions& options() const noexcept { return options_; }
    bool integer_dot() const noexcept { return options_.integer_dot_product && info_.integer_dot_product; }

    void synchronize();

private:
    ContextOptions options_;
    DeviceInfo info_;
    std::multimap<std::uint64_t, void*> free_;
    std::uint64_t pooled_bytes_ = 0;
    bool owns_device_ = true;
};

struct Storage {
    Runtime* runtime = nullptr;
    void* ptr = nullptr;
    std::uint64_t bytes = 0;  // as rounded by the pool
    ~Storage();
};

struct TensorAccess {
    static Runtime& runtime(const Tensor& t);
    static void* ptr(const Tensor& t) { return t.data(); }
    static Tensor empty(Runtime& runtime, Shape shape, DType dtype) { return Tensor::empty(runtime, std::move(shape), dtype); }
};

std::int64_t numel_of(const Shape& shape);

// The vkml_type code of a dtype.
std::uint32_t type_code(DType dtype);

// ops.cpp's internals the model shares (the reference's src/ops/internal.hpp).

// Attention's budget for one call's scores (ops/internal.hpp:92).
inline constexpr std::int64_t kMaxScoreBytes = std::int64_t{64} << 20;

// a [..., M, K] times b [K, N] (or [N, K] transposed); with b_group > 1, a's
// batch z against b's z / b_group; b_rows >= 0 uses b's first rows only.
// causal_offset >= 0: row r of each batch sees keys 0 .. r + causal_offset
// only (vkml_matmul's causal skip; no effect on up to 8 rows).
Tensor matmul(const char* name, const Tensor& a, const Tensor& b, bool transposed, std::int64_t b_group = 1, std::int64_t b_rows = -1,
              std::int64_t causal_offset = -1);

// Queries q [heads, q_len, hd] against keys 0..kv_len of caches [kv_heads,
// capacity, hd], query i at key position kv_len - q_len + i, in the
// reference's query chunks (attention.cpp:205-226).
// piece_bytes: this build's budget for one piece of the queries (results
// do not depend on it).
Tensor attention_prompt(const Tensor& q, const Tensor& k_cache, const Tensor& v_cache, std::int64_t kv_len, bool causal,
                        std::int64_t window, float softcap, std::int64_t max_score_bytes,
                        std::int64_t piece_bytes = std::int64_t{1} << 30);

// Sliding-window attention over rings [kv_heads, ring, hd] that hold key
// position p in row p % ring (attention.cpp:229-294), in pieces:
// sliding_rows gives how many of t queries from q0 (positions start + q0..)
// the next piece takes, so that the keys it appends overwrite no row a
// query of the piece still sees; ring_attention runs such a piece once its
// keys are in the rings.
// Rows start.. of every batch of src [B, *, width] into rows at.. of dst.
void copy_rows(const Tensor& src, std::int64_t start, const Tensor& dst, std::int64_t at, std::int64_t rows);

std::int64_t sliding_rows(std::int64_t heads, std::int64_t t, std::int64_t q0, std::int64_t start, std::int64_t ring, std::int64_t window,
                          std::int64_t max_score_bytes);
Tensor ring_attention(const Tensor& q, const Tensor& k_ring, const Tensor& v_ring, std::int64_t first, std::int64_t window, float softcap);
// The whole of it: q [heads, t, hd] at positions start.., their keys and
// values k, v [kv_heads, t, hd] appended to the rings piece by piece.
Tensor sliding_attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& k_ring, const Tensor& v_ring, std::int64_t start,
                         std::int64_t window, std::int64_t max_score_bytes, float softcap);

}  // namespace vkml::detail
