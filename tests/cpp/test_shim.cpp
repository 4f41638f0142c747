// Tests of the C++ host interface (include/tts_qlinear.hpp).
//   test_shim host      : metadata and validation paths (no device needed)
//   test_shim gpu DIR   : end to end on the GPU: reads DIR/{x,w}.bf16 and
//                         DIR/shape.txt (M N K mode), quantizes W with
//                         launch_row_quantize (load-time path), runs
//                         ops::linear and writes DIR/y.bf16 plus the
//                         quantized weights DIR/{wq.u8,sw.f32}.
//                         DIR/dense.txt (ACTIVATION RESIDUAL) selects a dense
//                         output with an epilogue that is no prepared finish
//                         (bias.bf16, residual.bf16).
//   test_shim producers DIR : ops::quantized_norm (residual update, RMSNorm)
//                         on DIR/{x,u,w}.bf16 and ops::quantized_gated (SiLU)
//                         on DIR/g.bf16 (shape.txt: M WIDTH GROUP), writing
//                         DIR/{res.bf16,nq.u8,ns.f32,gq.u8,gs.f32}.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <string>
#include <vector>

#include "../../include/tts_qlinear.hpp"

using namespace tts;

static int failures = 0;
#define EXPECT(cond)                                                        \
    do {                                                                    \
        if (!(cond)) {                                                      \
            std::fprintf(stderr, "FAIL %s:%d %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                     \
        }                                                                   \
    } while (0)

// The projection calls of the reference's layers/linear.cpp, written as it
// writes them (its members weight_ / bias_, layers/linear.h:12-14), so this
// file compiles only where the header is a drop-in for those call sites.
struct LayerCalls {
    ops::LinearOperand weight_;
    TensorView bias_;
    // layers/linear.cpp:132-148 (prepare_range)
    void prepare_range(TensorView matrix, int capacity, int output_channels, int input_channels,
                       Type activation_type_, ops::Activation activation,
                       QuantizationGroups layout) const {
        ops::Epilogue finish;
        finish.bias = bias_;
        finish.activation = activation;
        ops::prepare_quantized(matrix, capacity, output_channels, input_channels,
                               activation_type_, finish, layout);
    }
    // layers/linear.cpp:179 (project with a quantized input)
    void project(RowScaledView input, TensorView output) const {
        ops::linear(input, weight_, {}, output);
    }
    // layers/linear.cpp:195
    bool normalized_forward(TensorView input, TensorView normalized, TensorView output,
                            TensorView norm_weight, TensorView norm_bias, float epsilon,
                            const ops::NormFusion &fusion, ops::Epilogue epilogue,
                            const QkvProjectionOutput *writeback) const {
        return ops::normalized_linear(input, weight_, bias_, normalized, output, norm_weight,
                                      norm_bias, epsilon, fusion, epilogue, writeback);
    }
    // layers/linear.cpp:207
    bool normalized_quantized(TensorView input, TensorView normalized, TensorView output,
                              TensorView norm_weight, TensorView norm_bias, float epsilon,
                              const ops::NormFusion &fusion, ops::Epilogue epilogue,
                              RowScaledView quantized_output) const {
        return ops::normalized_linear(input, weight_, bias_, normalized, output, norm_weight,
                                      norm_bias, epsilon, fusion, epilogue, nullptr,
                                      quantized_output);
    }
    // layers/linear.cpp:212
    void normalized_project(RowScaledView normalized_input, TensorView output,
                            ops::Epilogue epilogue, RowScaledView quantized_output) const {
        ops::linear(normalized_input, weight_, bias_, output, epilogue, {}, quantized_output);
    }
    // layers/linear.cpp:246 (apply)
    void apply(TensorView input, TensorView output, TensorView bias, ops::Epilogue epilogue,
               RowScaledView scratch, RowScaledView quantized_output = {}) const {
        ops::linear(input, weight_, bias, output, epilogue, scratch, quantized_output);
    }
};

template <class E> static bool throws(const std::function<void()> &f) {
    try {
        f();
    } catch (const E &) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

static int host_tests() {
    // quantization names (include/tts/quantization.h)
    EXPECT(quantization_from_string("group_int8") == Quantization::GroupINT8);
    EXPECT(std::string(quantization_name(Quantization::FP8)) == "fp8");
    EXPECT(throws<std::invalid_argument>([] { quantization_from_string("int4"); }));
    EXPECT(quantized_type(Quantization::GroupFP8) == Type::FP8);
    EXPECT(quantization_groups(Quantization::GroupINT8).rotation == 128);
    EXPECT(quantization_groups(Quantization::INT8).activation == 0);
    // row capacity classes (core/row_capacity.h)
    EXPECT(row_capacity(1) == 1 && row_capacity(17) == 18 && row_capacity(32) == 32);
    EXPECT(row_capacity(4096) == 4096 && row_capacity(4097) == 4608);
    EXPECT(throws<std::invalid_argument>([] { row_capacity(0); }));
    // RowScaledView::validate
    char dummy[64];
    RowScaledView ok{TensorView(dummy, 4, 256, Type::I8), TensorView(dummy, 4, 1, Type::F32), 0, 0};
    ok.validate();
    RowScaledView grouped{TensorView(dummy, 4, 256, Type::I8), TensorView(dummy, 2, 4, Type::F32),
                          128, 128};
    grouped.validate();
    RowScaledView bad = grouped;
    bad.scales = TensorView(dummy, 4, 2, Type::F32);
    EXPECT(throws<std::invalid_argument>([&] { bad.validate(); }));
    bad = ok;
    bad.values.type = Type::BF16;
    EXPECT(throws<std::invalid_argument>([&] { bad.validate(); }));
    bad = grouped;
    bad.rotation_size = 64;
    EXPECT(throws<std::invalid_argument>([&] { bad.validate(); }));
    // QuantizedGemm planning: prepare, seal, lookup by capacity class
    QuantizedGemm gemm(nullptr, nullptr, 0, Type::I8);
    gemm.prepare(30, 4096, 2048);
    EXPECT(gemm.planned(29, 4096, 2048).kind == LinearKind::Skinny);  // same class as 30
    gemm.prepare(4096, 4096, 2048);
    EXPECT(gemm.planned(4096, 4096, 2048).kind == LinearKind::Tiled);
    EXPECT(throws<std::logic_error>([&] { gemm.planned(7, 4096, 2048); }));
    EXPECT(throws<std::invalid_argument>([&] { gemm.prepare(8, 4096, 2040); }));  // K % 16
    EXPECT(throws<std::invalid_argument>([&] { gemm.prepare(8, 4096, 131072); }));
    gemm.seal();
    EXPECT(throws<std::logic_error>([&] { gemm.prepare(8, 512, 512); }));
    gemm.prepare(30, 4096, 2048);  // already prepared: allowed after seal
    EXPECT(gemm.cache_stats().prepared_plans == 2);
    // check_linear: mismatched shapes throw before any launch
    RowScaledView x{TensorView(dummy, 30, 2048, Type::I8), TensorView(dummy, 30, 1, Type::F32), 0,
                    0};
    RowScaledView w{TensorView(dummy, 4096, 2048, Type::I8),
                    TensorView(dummy, 4096, 1, Type::F32), 0, 0};
    EXPECT(throws<std::invalid_argument>(
        [&] { gemm.linear(x, w, TensorView(dummy, 30, 4000, Type::BF16)); }));
    RowScaledView xf = x;
    xf.values.type = Type::FP8;
    EXPECT(throws<std::invalid_argument>(
        [&] { gemm.linear(xf, w, TensorView(dummy, 30, 4096, Type::BF16)); }));
    // launcher status -> exception mapping
    EXPECT(throws<std::invalid_argument>([&] {
        launch_row_quantize(TensorView(dummy, 2, 64, Type::F32), ok, nullptr);
    }));
    EXPECT(throws<std::invalid_argument>([&] {
        launch_quant_linear({}, {16, 40, 256}, dummy, nullptr, dummy, nullptr, dummy, nullptr, 0,
                            nullptr, Type::I8, Type::BF16);
    }));
    // fused producers: the reference's shape checks throw before any launch
    RowScaledView nq{TensorView(dummy, 4, 2048, Type::I8), TensorView(dummy, 4, 1, Type::F32), 0, 0};
    EXPECT(throws<std::invalid_argument>([&] {  // weight length != cols
        launch_quantized_norm(TensorView(dummy, 4, 2048), {}, TensorView(dummy, 1, 1024), nq, 1e-6f,
                              false, {}, nullptr);
    }));
    RowScaledView wide{TensorView(dummy, 4, 4096, Type::I8), TensorView(dummy, 4, 1, Type::F32), 0, 0};
    EXPECT(throws<std::invalid_argument>([&] {  // cols > 2048
        launch_quantized_norm(TensorView(dummy, 4, 4096), {}, TensorView(dummy, 1, 4096), wide,
                              1e-6f, false, {}, nullptr);
    }));
    EXPECT(throws<std::invalid_argument>([&] {  // input is not [rows, 2*width]
        launch_quantized_gated(TensorView(dummy, 4, 4000), nq, 0, nullptr);
    }));
    EXPECT(throws<std::invalid_argument>([&] {  // kind
        launch_quantized_gated(TensorView(dummy, 4, 4096), nq, 2, nullptr);
    }));
    EXPECT(!quant_gated_supports_clusters(0));
    // normalized_linear declines what its kernel does not cover (no launch)
    {
        QuantizedGemm g8(nullptr, nullptr, 0, Type::I8);
        RowScaledView wsmall{TensorView(dummy, 64, 512, Type::I8), TensorView(dummy, 64, 1, Type::F32), 0, 0};
        RowScaledView wbig{TensorView(dummy, 64, 1024, Type::I8), TensorView(dummy, 64, 1, Type::F32), 0, 0};
        ops::NormFusion gated;
        int source_rows[2] = {0, 1};
        gated.source_rows = source_rows;
        EXPECT(!g8.normalized_linear(TensorView(dummy, 2, 1024), {}, {}, {}, 1e-5f, {}, wbig,
                                     TensorView(dummy, 2, 64)));  // k > 512
        EXPECT(!g8.normalized_linear(TensorView(dummy, 2, 512), {}, {}, {}, 1e-5f, gated, wsmall,
                                     TensorView(dummy, 2, 64)));  // source-row gather
        ops::Epilogue gelu;
        gelu.activation = ops::Activation::GeluTanh;
        EXPECT(!g8.normalized_linear(TensorView(dummy, 2, 512), {}, {}, {}, 1e-5f, {}, wsmall,
                                     TensorView(dummy, 2, 64), gelu));
    }
    // ops without a bound context
    EXPECT(throws<std::logic_error>([&] { ops::matmul(x, w, TensorView(dummy, 30, 4096)); }));
    // finishes are prepared on a prepared projection only
    {
        QuantizedGemm g(nullptr, nullptr, 0, Type::I8);
        ops::Epilogue relu;
        relu.activation = ops::Activation::Relu;
        EXPECT(throws<std::logic_error>([&] { g.prepare_finish(30, 4096, 2048, Type::BF16, relu); }));
        g.prepare(30, 4096, 2048);
        g.prepare_finish(30, 4096, 2048, Type::BF16, relu);
        ops::Epilogue silu;  // not a GEMM finish: ignored
        silu.activation = ops::Activation::Silu;
        g.prepare_finish(30, 4096, 2048, Type::BF16, silu);
        EXPECT(g.cache_stats().prepared_plans == 2);
    }
    // ops::linear / ops::normalized_linear over LinearOperand
    {
        LayerCalls dense{TensorView(dummy, 64, 512), {}};
        EXPECT(throws<std::invalid_argument>([&] {  // dense weights: not in this library
            dense.apply(TensorView(dummy, 2, 512), TensorView(dummy, 2, 64), {}, {}, {});
        }));
        EXPECT(!dense.normalized_forward(TensorView(dummy, 2, 512), {}, TensorView(dummy, 2, 64),
                                         {}, {}, 1e-5f, {}, {}, nullptr));
        RowScaledView wq{TensorView(dummy, 64, 512, Type::I8), TensorView(dummy, 64, 1, Type::F32), 0, 0};
        LayerCalls quantized{wq, {}};
        QkvProjectionOutput writeback;
        EXPECT(!quantized.normalized_forward(TensorView(dummy, 2, 512), {}, TensorView(dummy, 2, 64),
                                             {}, {}, 1e-5f, {}, {}, &writeback));
        ops::Epilogue owned;
        owned.bias = TensorView(dummy, 1, 64);
        EXPECT(throws<std::invalid_argument>([&] {  // ops::linear owns the bias
            quantized.apply(TensorView(dummy, 2, 512), TensorView(dummy, 2, 64), {}, owned, {});
        }));
        EXPECT(throws<std::invalid_argument>([&] {  // bias aliases the output
            quantized.apply(TensorView(dummy, 2, 512), TensorView(dummy, 2, 64),
                            TensorView(dummy + 8, 1, 64), {}, {});
        }));
    }
    std::printf("host tests: %s\n", failures ? "FAILED" : "ok");
    return failures ? 1 : 0;
}

template <class T> static std::vector<T> read_file(const std::string &path, size_t count) {
    std::vector<T> v(count);
    std::ifstream f(path, std::ios::binary);
    f.read(reinterpret_cast<char *>(v.data()), count * sizeof(T));
    if (!f) throw std::runtime_error("cannot read " + path);
    return v;
}
template <class T> static void write_file(const std::string &path, const std::vector<T> &v) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char *>(v.data()), v.size() * sizeof(T));
}
#define HIP(x)                                                               \
    do {                                                                     \
        if ((x) != hipSuccess) throw std::runtime_error("HIP error: " #x);  \
    } while (0)

static int gpu_test(const std::string &dir) {
    int M, N, K;
    std::string mode;
    std::ifstream(dir + "/shape.txt") >> M >> N >> K >> mode;
    const Quantization q = quantization_from_string(mode);
    const Type fmt = quantized_type(q);
    const QuantizationGroups groups = quantization_groups(q);
    auto x = read_file<uint16_t>(dir + "/x.bf16", size_t(M) * K);
    auto w = read_file<uint16_t>(dir + "/w.bf16", size_t(N) * K);
    void *dx, *dw, *dwq, *dsw, *dy;
    const int wgroups = groups.weight ? (K + groups.weight - 1) / groups.weight : 1;
    HIP(hipMalloc(&dx, x.size() * 2));
    HIP(hipMalloc(&dw, w.size() * 2));
    HIP(hipMalloc(&dwq, size_t(N) * K));
    HIP(hipMalloc(&dsw, size_t(N) * wgroups * 4));
    HIP(hipMalloc(&dy, size_t(M) * N * 2));
    HIP(hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(dw, w.data(), w.size() * 2, hipMemcpyHostToDevice));
    hipStream_t stream;
    HIP(hipStreamCreate(&stream));
    {
        // The execution context as the reference's runtime builds it
        // (runtime/cuda_context.cpp:61,72): an 8 MiB GEMM workspace Buffer.
        Buffer gemm_workspace(8 << 20);
        QuantizedGemm gemm(reinterpret_cast<qlin_stream_t>(stream), nullptr, gemm_workspace, fmt);
        ops::bind(0, &gemm);
        // Load time: weight quantization with the activation quantizer
        // (io/weights.cpp:80-87), plan preparation with the layer's finish
        // (layers/linear.cpp:132-148), seal.
        RowScaledView wq{TensorView(dwq, N, K, fmt, 0, 0),
                         groups.weight ? TensorView(dsw, wgroups, N, Type::F32, 0, 0)
                                       : TensorView(dsw, N, 1, Type::F32, 0, 0),
                         groups.weight, groups.rotation};
        ops::quantize_rows(TensorView(dw, N, K, Type::BF16, 0, 0), wq);
        std::ifstream act_file(dir + "/finish.txt"), epi_file(dir + "/epilogue.txt"),
            mode_file(dir + "/calls.txt");
        std::ifstream dense_file(dir + "/dense.txt");
        int act = 0, activation = 0, use_residual = 0, dense_act = 0, dense_residual = 0;
        std::string calls;
        const bool quantized_out = bool(epi_file >> activation >> use_residual);
        const bool finish = !quantized_out && (act_file >> act) && act;
        const bool dense_epilogue = bool(dense_file >> dense_act >> dense_residual);
        mode_file >> calls;
        void *db = nullptr;
        if (quantized_out || finish || dense_epilogue) {
            auto b = read_file<uint16_t>(dir + "/bias.bf16", size_t(N));
            HIP(hipMalloc(&db, b.size() * 2));
            HIP(hipMemcpy(db, b.data(), b.size() * 2, hipMemcpyHostToDevice));
        }
        LayerCalls layer{wq, db ? TensorView(db, 1, N) : TensorView()};
        const ops::Activation prepared = quantized_out ? static_cast<ops::Activation>(activation)
                                         : finish ? (act == 1 ? ops::Activation::Relu
                                                              : ops::Activation::GeluTanh)
                                                  : ops::Activation::Identity;
        layer.prepare_range(TensorView(dwq, N, K, fmt, 0, 0), row_capacity(M), N, K, Type::BF16,
                            prepared, groups);
        gemm.seal();
        // Serving: dense bf16 activations through ops::linear.
        QuantizationWorkspace workspace(M, QuantizationWorkspace::Capacity::matrix(K, groups.activation));
        RowScaledView scratch = workspace.view(M, K, fmt, groups);
        scratch.values.device = scratch.scales.device = 0;
        if (quantized_out) {
            // ops::linear with a quantized output for the next layer
            // (ops/linear.cpp:35-78): bias + activation (+ residual), then codes.
            auto r = read_file<uint16_t>(dir + "/residual.bf16", size_t(M) * N);
            void *dr, *dq, *dqs;
            HIP(hipMalloc(&dr, r.size() * 2));
            HIP(hipMalloc(&dq, size_t(M) * N));
            HIP(hipMalloc(&dqs, size_t(M) * 4));
            HIP(hipMemcpy(dr, r.data(), r.size() * 2, hipMemcpyHostToDevice));
            ops::Epilogue e;
            e.activation = static_cast<ops::Activation>(activation);
            if (use_residual) e.residual = TensorView(dr, M, N, Type::BF16, 0, 0);
            RowScaledView next{TensorView(dq, M, N, fmt, 0, 0), TensorView(dqs, M, 1, Type::F32, 0, 0)};
            layer.apply(TensorView(dx, M, K, Type::BF16, 0, 0), TensorView(dy, M, N, Type::BF16, 0, 0),
                        layer.bias_, e, scratch, next);
            HIP(hipStreamSynchronize(stream));
            std::vector<uint8_t> qh(size_t(M) * N);
            std::vector<float> qsh(M);
            HIP(hipMemcpy(qh.data(), dq, qh.size(), hipMemcpyDeviceToHost));
            HIP(hipMemcpy(qsh.data(), dqs, qsh.size() * 4, hipMemcpyDeviceToHost));
            write_file(dir + "/next.u8", qh);
            write_file(dir + "/next_scales.f32", qsh);
            for (void *p : {dr, dq, dqs}) (void)hipFree(p);
        } else if (dense_epilogue) {
            // ops::linear with a dense output and an epilogue that is no
            // prepared finish (none was prepared): the GEMM, then
            // pointwise(output, output, e) (ops/linear.cpp:68-82).
            auto r = read_file<uint16_t>(dir + "/residual.bf16", size_t(M) * N);
            void *dr;
            HIP(hipMalloc(&dr, r.size() * 2));
            HIP(hipMemcpy(dr, r.data(), r.size() * 2, hipMemcpyHostToDevice));
            ops::Epilogue e;
            e.activation = static_cast<ops::Activation>(dense_act);
            if (dense_residual) e.residual = TensorView(dr, M, N, Type::BF16, 0, 0);
            layer.apply(TensorView(dx, M, K, Type::BF16, 0, 0), TensorView(dy, M, N, Type::BF16, 0, 0),
                        layer.bias_, e, scratch);
            HIP(hipStreamSynchronize(stream));
            (void)hipFree(dr);
        } else if (finish) {
            // ops::linear with a bias + activation epilogue (fused finish)
            ops::Epilogue e;
            e.activation = prepared;
            layer.apply(TensorView(dx, M, K, Type::BF16, 0, 0), TensorView(dy, M, N, Type::BF16, 0, 0),
                        layer.bias_, e, scratch);
        } else if (calls == "rowscaled") {
            // A quantized input (layers/linear.cpp:179): quantize_rows, then
            // ops::linear(input, weight_, {}, output).
            ops::quantize_rows(TensorView(dx, M, K, Type::BF16, 0, 0), scratch);
            layer.project(scratch, TensorView(dy, M, N, Type::BF16, 0, 0));
        } else {
            layer.apply(TensorView(dx, M, K, Type::BF16, 0, 0), TensorView(dy, M, N, Type::BF16, 0, 0),
                        {}, {}, scratch);
        }
        if (db) (void)hipFree(db);
        HIP(hipStreamSynchronize(stream));
        std::vector<uint16_t> y(size_t(M) * N);
        std::vector<uint8_t> wqh(size_t(N) * K);
        std::vector<float> swh(size_t(N) * wgroups);
        HIP(hipMemcpy(y.data(), dy, y.size() * 2, hipMemcpyDeviceToHost));
        HIP(hipMemcpy(wqh.data(), dwq, wqh.size(), hipMemcpyDeviceToHost));
        HIP(hipMemcpy(swh.data(), dsw, swh.size() * 4, hipMemcpyDeviceToHost));
        write_file(dir + "/y.bf16", y);
        write_file(dir + "/wq.u8", wqh);
        write_file(dir + "/sw.f32", swh);
        ops::bind(0, nullptr);
    }
    for (void *p : {dx, dw, dwq, dsw, dy}) (void)hipFree(p);
    (void)hipStreamDestroy(stream);
    std::printf("gpu test %s M=%d N=%d K=%d: done\n", mode.c_str(), M, N, K);
    return 0;
}

static int producers_test(const std::string &dir) {
    int M, width, group;
    std::ifstream(dir + "/shape.txt") >> M >> width >> group;
    const int H = 2048, rot = group ? 128 : 0;
    auto x = read_file<uint16_t>(dir + "/x.bf16", size_t(M) * H);
    auto u = read_file<uint16_t>(dir + "/u.bf16", size_t(M) * H);
    auto w = read_file<uint16_t>(dir + "/w.bf16", size_t(H));
    auto g = read_file<uint16_t>(dir + "/g.bf16", size_t(M) * 2 * width);
    const int ng = group ? H / group : 1, gg = group ? (width + group - 1) / group : 1;
    void *dx, *du, *dw, *dg, *dnq, *dns, *dgq, *dgs, *dws;
    HIP(hipMalloc(&dx, x.size() * 2));
    HIP(hipMalloc(&du, u.size() * 2));
    HIP(hipMalloc(&dw, w.size() * 2));
    HIP(hipMalloc(&dg, g.size() * 2));
    HIP(hipMalloc(&dnq, size_t(M) * H));
    HIP(hipMalloc(&dns, size_t(M) * ng * 4));
    HIP(hipMalloc(&dgq, size_t(M) * width));
    HIP(hipMalloc(&dgs, size_t(M) * gg * 4));
    HIP(hipMalloc(&dws, 1 << 20));
    HIP(hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(du, u.data(), u.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(dw, w.data(), w.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(dg, g.data(), g.size() * 2, hipMemcpyHostToDevice));
    hipStream_t stream;
    HIP(hipStreamCreate(&stream));
    {
        QuantizedGemm gemm(reinterpret_cast<qlin_stream_t>(stream), dws, 1 << 20, Type::I8);
        ops::bind(0, &gemm);
        RowScaledView nq{TensorView(dnq, M, H, Type::I8, 0, 0),
                         group ? TensorView(dns, ng, M, Type::F32, 0, 0)
                               : TensorView(dns, M, 1, Type::F32, 0, 0),
                         group, rot};
        ops::quantized_norm(TensorView(dx, M, H, Type::BF16, 0, 0),
                            TensorView(du, M, H, Type::BF16, 0, 0), TensorView(dw, 1, H), nq, 1e-6f);
        RowScaledView gq{TensorView(dgq, M, width, Type::I8, 0, 0),
                         group ? TensorView(dgs, gg, M, Type::F32, 0, 0)
                               : TensorView(dgs, M, 1, Type::F32, 0, 0),
                         group, rot};
        ops::quantized_gated(TensorView(dg, M, 2 * width, Type::BF16, 0, 0), gq, 0);
        HIP(hipStreamSynchronize(stream));
        std::vector<uint16_t> res(x.size());
        std::vector<uint8_t> nqh(size_t(M) * H), gqh(size_t(M) * width);
        std::vector<float> nsh(size_t(M) * ng), gsh(size_t(M) * gg);
        HIP(hipMemcpy(res.data(), dx, res.size() * 2, hipMemcpyDeviceToHost));
        HIP(hipMemcpy(nqh.data(), dnq, nqh.size(), hipMemcpyDeviceToHost));
        HIP(hipMemcpy(nsh.data(), dns, nsh.size() * 4, hipMemcpyDeviceToHost));
        HIP(hipMemcpy(gqh.data(), dgq, gqh.size(), hipMemcpyDeviceToHost));
        HIP(hipMemcpy(gsh.data(), dgs, gsh.size() * 4, hipMemcpyDeviceToHost));
        write_file(dir + "/res.bf16", res);
        write_file(dir + "/nq.u8", nqh);
        write_file(dir + "/ns.f32", nsh);
        write_file(dir + "/gq.u8", gqh);
        write_file(dir + "/gs.f32", gsh);
        ops::bind(0, nullptr);
    }
    for (void *p : {dx, du, dw, dg, dnq, dns, dgq, dgs, dws}) (void)hipFree(p);
    (void)hipStreamDestroy(stream);
    std::printf("producers test M=%d width=%d group=%d: done\n", M, width, group);
    return 0;
}

// ops::layer_norm_quantize (hidden 2048, K128 groups + rotation) feeding
// ops::linear with a quantized input (layers/linear.cpp:212 form), and
// ops::normalized_linear (LayerNorm + residual -> INT8 GEMV, k 512; the
// layers/linear.cpp:195 and :207 forms) through the C++ interface.
static int sequence_test(const std::string &dir) {
    int M;
    std::ifstream(dir + "/shape.txt") >> M;
    const int H = 2048, k = 512, n = 384, n2 = 256;
    auto x = read_file<uint16_t>(dir + "/x.bf16", size_t(M) * H);
    auto w2 = read_file<uint16_t>(dir + "/w2.bf16", size_t(n2) * H);
    auto lw = read_file<uint16_t>(dir + "/lw.bf16", size_t(H));
    auto xs = read_file<uint16_t>(dir + "/xs.bf16", size_t(M) * k);
    auto rs = read_file<uint16_t>(dir + "/rs.bf16", size_t(M) * k);
    auto ws = read_file<uint16_t>(dir + "/ws.bf16", size_t(n) * k);
    void *dx, *dlw, *dq, *dqs, *dxs, *drs, *dws, *dwq, *dsw, *dy, *dnorm, *dgemm;
    HIP(hipMalloc(&dx, x.size() * 2));
    HIP(hipMalloc(&dlw, lw.size() * 2));
    HIP(hipMalloc(&dq, size_t(M) * H));
    HIP(hipMalloc(&dqs, size_t(H / 128) * M * 4));
    HIP(hipMalloc(&dxs, xs.size() * 2));
    HIP(hipMalloc(&drs, rs.size() * 2));
    HIP(hipMalloc(&dws, ws.size() * 2));
    HIP(hipMalloc(&dwq, size_t(n) * k));
    HIP(hipMalloc(&dsw, size_t(n) * 4));
    HIP(hipMalloc(&dy, size_t(M) * n * 2));
    HIP(hipMalloc(&dnorm, size_t(M) * k * 2));
    HIP(hipMalloc(&dgemm, 1 << 20));
    void *dw2, *dw2q, *dsw2, *dy2, *dnq, *dnqs;
    HIP(hipMalloc(&dw2, w2.size() * 2));
    HIP(hipMalloc(&dw2q, size_t(n2) * H));
    HIP(hipMalloc(&dsw2, size_t(H / 128) * n2 * 4));
    HIP(hipMalloc(&dy2, size_t(M) * n2 * 2));
    HIP(hipMalloc(&dnq, size_t(M) * n));
    HIP(hipMalloc(&dnqs, size_t(M) * 4));
    HIP(hipMemcpy(dw2, w2.data(), w2.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(dlw, lw.data(), lw.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(dxs, xs.data(), xs.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(drs, rs.data(), rs.size() * 2, hipMemcpyHostToDevice));
    HIP(hipMemcpy(dws, ws.data(), ws.size() * 2, hipMemcpyHostToDevice));
    hipStream_t stream;
    HIP(hipStreamCreate(&stream));
    {
        QuantizedGemm gemm(reinterpret_cast<qlin_stream_t>(stream), dgemm, 1 << 20, Type::I8);
        ops::bind(0, &gemm);
        RowScaledView q{TensorView(dq, M, H, Type::I8, 0, 0), TensorView(dqs, H / 128, M, Type::F32, 0, 0),
                        128, 128};
        ops::layer_norm_quantize(TensorView(dx, M, H, Type::BF16, 0, 0), q,
                                 TensorView(dlw, 1, H, Type::BF16, 0, 0), TensorView(), 1e-5f);
        // The K128 / H128 input feeds a projection with weights of the same
        // layout (group_int8), ops::linear with a quantized input.
        RowScaledView w2q{TensorView(dw2q, n2, H, Type::I8, 0, 0),
                          TensorView(dsw2, H / 128, n2, Type::F32, 0, 0), 128, 128};
        ops::quantize_rows(TensorView(dw2, n2, H, Type::BF16, 0, 0), w2q);
        LayerCalls grouped{w2q, {}};
        grouped.prepare_range(w2q.values, row_capacity(M), n2, H, Type::BF16,
                              ops::Activation::Identity, {128, 128, 128});
        grouped.normalized_project(q, TensorView(dy2, M, n2, Type::BF16, 0, 0), {}, {});
        RowScaledView wq{TensorView(dwq, n, k, Type::I8, 0, 0), TensorView(dsw, n, 1, Type::F32, 0, 0)};
        ops::quantize_rows(TensorView(dws, n, k, Type::BF16, 0, 0), wq);
        ops::NormFusion fusion;
        fusion.residual = TensorView(drs, M, k, Type::BF16, 0, 0);
        LayerCalls small{wq, {}};
        const bool fused = small.normalized_forward(
            TensorView(dxs, M, k, Type::BF16, 0, 0), TensorView(dnorm, M, k, Type::BF16, 0, 0),
            TensorView(dy, M, n, Type::BF16, 0, 0), TensorView(), TensorView(), 1e-5f, fusion, {},
            nullptr);
        EXPECT(fused);
        // Again with the next layer's quantized input (same output y).
        RowScaledView next{TensorView(dnq, M, n, Type::I8, 0, 0), TensorView(dnqs, M, 1, Type::F32, 0, 0)};
        const bool fused_next = small.normalized_quantized(
            TensorView(dxs, M, k, Type::BF16, 0, 0), TensorView(dnorm, M, k, Type::BF16, 0, 0),
            TensorView(dy, M, n, Type::BF16, 0, 0), TensorView(), TensorView(), 1e-5f, fusion, {},
            next);
        EXPECT(fused_next);
        HIP(hipStreamSynchronize(stream));
        std::vector<uint16_t> y2h(size_t(M) * n2);
        std::vector<uint8_t> nqh(size_t(M) * n);
        std::vector<float> nqsh(M);
        HIP(hipMemcpy(y2h.data(), dy2, y2h.size() * 2, hipMemcpyDeviceToHost));
        HIP(hipMemcpy(nqh.data(), dnq, nqh.size(), hipMemcpyDeviceToHost));
        HIP(hipMemcpy(nqsh.data(), dnqs, nqsh.size() * 4, hipMemcpyDeviceToHost));
        write_file(dir + "/y2.bf16", y2h);
        write_file(dir + "/next.u8", nqh);
        write_file(dir + "/next.f32", nqsh);
        std::vector<uint8_t> qh(size_t(M) * H), wqh(size_t(n) * k);
        std::vector<float> qsh(size_t(H / 128) * M), swh(n);
        std::vector<uint16_t> yh(size_t(M) * n), nh(size_t(M) * k);
        HIP(hipMemcpy(qh.data(), dq, qh.size(), hipMemcpyDeviceToHost));
        HIP(hipMemcpy(qsh.data(), dqs, qsh.size() * 4, hipMemcpyDeviceToHost));
        HIP(hipMemcpy(wqh.data(), dwq, wqh.size(), hipMemcpyDeviceToHost));
        HIP(hipMemcpy(swh.data(), dsw, swh.size() * 4, hipMemcpyDeviceToHost));
        HIP(hipMemcpy(yh.data(), dy, yh.size() * 2, hipMemcpyDeviceToHost));
        HIP(hipMemcpy(nh.data(), dnorm, nh.size() * 2, hipMemcpyDeviceToHost));
        write_file(dir + "/lq.u8", qh);
        write_file(dir + "/lqs.f32", qsh);
        write_file(dir + "/wq.u8", wqh);
        write_file(dir + "/sw.f32", swh);
        write_file(dir + "/y.bf16", yh);
        write_file(dir + "/norm.bf16", nh);
        ops::bind(0, nullptr);
    }
    for (void *p : {dx, dlw, dq, dqs, dxs, drs, dws, dwq, dsw, dy, dnorm, dgemm, dw2, dw2q, dsw2,
                    dy2, dnq, dnqs})
        (void)hipFree(p);
    (void)hipStreamDestroy(stream);
    std::printf("sequence test M=%d: %s\n", M, failures ? "FAILED" : "done");
    return failures ? 1 : 0;
}

int main(int argc, char **argv) {
    if (argc >= 2 && std::string(argv[1]) == "host") return host_tests();
    if (argc >= 3 && std::string(argv[1]) == "gpu") return gpu_test(argv[2]);
    if (argc >= 3 && std::string(argv[1]) == "producers") return producers_test(argv[2]);
    if (argc >= 3 && std::string(argv[1]) == "sequence") return sequence_test(argv[2]);
    std::fprintf(stderr, "usage: test_shim host | gpu DIR | producers DIR\n");
    return 2;
}
