// Runs every op of the C++ API (include/vkml/ops.hpp) on the inputs a test
// wrote into a directory and writes each result beside them, for
// tests/test_gpu_ops.py to check against the CPU oracle. Links libvkml.so.
//
// Inputs and results are raw little-endian arrays <dir>/<name>.bin; every
// result is listed on stdout as "out <name> <dtype> <d0> <d1> ...". Then the
// error cases: "error <case> <message>" for each call that must throw.
#include <cstdio>
#include <fstream>
#include <functional>
#include <iterator>
#include <string>
#include <vector>

#include "vkml/context.hpp"
#include "vkml/error.hpp"
#include "vkml/ops.hpp"
#include "vkml/tensor.hpp"

namespace {

using vkml::DType;
using vkml::Shape;
using vkml::Tensor;

std::string g_dir;

std::vector<std::byte> read_bytes(const std::string& name) {
    std::ifstream in(g_dir + "/" + name + ".bin", std::ios::binary);
    if (!in) throw std::runtime_error("ops_dump: no input " + name);
    std::vector<char> raw((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    std::vector<std::byte> out(raw.size());
    for (std::size_t i = 0; i < raw.size(); ++i) out[i] = std::byte(static_cast<unsigned char>(raw[i]));
    return out;
}

Tensor load(vkml::Context& ctx, const std::string& name, Shape shape, DType dtype = DType::F32) {
    return Tensor::from_bytes(ctx, read_bytes(name), std::move(shape), dtype);
}

void save(const std::string& name, const Tensor& t) {
    const std::vector<std::byte> bytes = t.to_bytes();
    std::ofstream out(g_dir + "/" + name + ".bin", std::ios::binary);
    out.write(reinterpret_cast<const char*>(bytes.data()), static_cast<std::streamsize>(bytes.size()));
    std::printf("out %s %s", name.c_str(), std::string(vkml::to_string(t.dtype())).c_str());
    for (const auto d : t.shape()) std::printf(" %lld", static_cast<long long>(d));
    std::printf("\n");
}

void save_matrix(const std::string& name, const vkml::QuantizedMatrix& m, const Tensor& ids, const Tensor& one, const Tensor& many) {
    save(name + "_values", m.values);
    save(name + "_scales", m.scales);
    save(name + "_dequantized", vkml::dequantize(m));
    save(name + "_embedding", vkml::embedding(m, ids));
    save(name + "_times_one", vkml::matmul_transposed(one, m));
    save(name + "_times_many", vkml::matmul_transposed(many, m));
}

void expect_error(const char* name, const std::function<void()>& call) {
    try {
        call();
        std::printf("error %s (none)\n", name);
    } catch (const vkml::Error& e) {
        std::printf("error %s %s\n", name, e.what());
    }
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: ops_dump <dir>\n");
        return 2;
    }
    g_dir = argv[1];
    vkml::Context ctx;

    const Tensor a = load(ctx, "a", {3, 5, 64}), b = load(ctx, "b", {5, 64});
    save("add", vkml::add(a, b));
    save("sub", vkml::sub(a, b));
    save("mul", vkml::mul(a, b));
    save("div", vkml::div(a, b));

    const Tensor x = load(ctx, "x", {4, 300});
    save("silu", vkml::silu(x));
    save("gelu", vkml::gelu(x));
    save("softcap", vkml::softcap(x, 3.0f));
    save("softmax", vkml::softmax(x));
    save("argmax", vkml::argmax(x));
    save("cast_f16", vkml::cast(x, DType::F16));
    save("cast_bf16", vkml::cast(x, DType::BF16));
    save("cast_f32", vkml::cast(load(ctx, "h", {4, 300}, DType::F16), DType::F32));

    save("rms_norm", vkml::rms_norm(load(ctx, "xr", {4, 4096}), load(ctx, "w", {4096}), 1e-5f));

    const Tensor p = load(ctx, "p", {2, 3, 4, 5});
    save("permute", vkml::permute(p, {2, 0, 3, 1}));
    save("transpose", vkml::transpose(p, 1, 3));

    const Tensor ids = load(ctx, "ids", {7}, DType::I32);
    save("embedding", vkml::embedding(load(ctx, "table", {100, 64}), ids));

    const Tensor table = vkml::rope_table(ctx, 64, 128, 10000.0f);
    save("rope_table", table);
    const Tensor rx = load(ctx, "rx", {5, 4, 128});
    save("rope_interleaved", vkml::rope(rx, table, 3, vkml::RopeStyle::Interleaved));
    save("rope_rotate_half", vkml::rope(rx, table, 3, vkml::RopeStyle::RotateHalf));

    const Tensor ma = load(ctx, "ma", {2, 9, 96});
    save("matmul", vkml::matmul(ma, load(ctx, "mb", {96, 40})));
    const Tensor mbt = load(ctx, "mbt", {40, 96});
    save("matmul_transposed", vkml::matmul_transposed(ma, mbt));
    save("matmul_transposed_few", vkml::matmul_transposed(load(ctx, "ma3", {3, 96}), mbt));
    save("matmul_transposed_f16", vkml::matmul_transposed(ma, load(ctx, "mbt16", {40, 96}, DType::F16)));

    const Tensor qw = load(ctx, "qw", {64, 256});
    const Tensor qids = load(ctx, "qids", {5}, DType::I32);
    const Tensor one = load(ctx, "qa1", {1, 256}), many = load(ctx, "qa12", {12, 256});
    save_matrix("q8_0", vkml::quantize_q8(qw), qids, one, many);
    save_matrix("q4_0", vkml::quantize_q4(qw), qids, one, many);
    save_matrix("q4_1", vkml::quantize_q4_1(qw), qids, one, many);

    const Tensor dq = load(ctx, "dq", {8, 1, 64});
    save("attention_decode", vkml::attention(dq, load(ctx, "dk", {2, 50, 64}), load(ctx, "dv", {2, 50, 64}), true));
    save("attention_decode_f16",
         vkml::attention(dq, load(ctx, "dk16", {2, 50, 64}, DType::F16), load(ctx, "dv16", {2, 50, 64}, DType::F16), true));
    const Tensor pq = load(ctx, "pq", {8, 20, 64}), pk = load(ctx, "pk", {2, 20, 64}), pv = load(ctx, "pv", {2, 20, 64});
    save("attention_prompt", vkml::attention(pq, pk, pv, true));
    save("attention_window", vkml::attention(pq, pk, pv, true, 8, 30.0f));
    save("attention_full", vkml::attention(pq, pk, pv, false));

    // The reference's shape checks (tests/test_attention.cpp:212-229).
    const auto zeros = [&](Shape s) { return Tensor::zeros(ctx, std::move(s), DType::F32); };
    expect_error("heads", [&] { (void)vkml::attention(zeros({4, 2, 8}), zeros({3, 5, 8}), zeros({3, 5, 8}), false); });
    expect_error("v_shape", [&] { (void)vkml::attention(zeros({4, 2, 8}), zeros({4, 5, 8}), zeros({4, 6, 8}), false); });
    expect_error("head_dim", [&] { (void)vkml::attention(zeros({4, 2, 8}), zeros({4, 5, 4}), zeros({4, 5, 4}), false); });
    expect_error("rank", [&] { (void)vkml::attention(zeros({2, 8}), zeros({2, 8}), zeros({2, 8}), false); });
    expect_error("causal", [&] { (void)vkml::attention(zeros({4, 6, 8}), zeros({4, 5, 8}), zeros({4, 5, 8}), true); });
    expect_error("broadcast", [&] { (void)vkml::add(zeros({3, 5}), zeros({4})); });
    expect_error("quantize_width", [&] { (void)vkml::quantize_q8(zeros({4, 48})); });
    ctx.synchronize();
    return 0;
}
