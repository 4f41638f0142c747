// tts_qlinear.hpp — C++ host interface of the quantized linear path, with the
// names, argument meaning and error behaviour of TTS.cpp's layers/ops API, on
// top of the C ABI in qlinear.h (libqlinear.so). Callers written against the
// reference's src/ops and src/layers link against this unchanged:
//
//   tts::Type, TensorView                    <- core/tensor.h:8-114 (subset)
//   tts::Quantization, quantization_*        <- include/tts/quantization.h:6-29,
//                                               core/quantization.h:6-27
//   tts::RowScaledView                       <- core/quantization.h:33-49
//   tts::KernelProblem                       <- core/kernel_problem.h:4-7
//   tts::row_capacity                        <- core/row_capacity.h:10-19
//   tts::LinearPath                          <- ops/kernels/quant/kernel_config.h:5-9
//   tts::launch_row_quantize                 <- ops/kernels/quant/row_quantize.h:6
//   tts::launch_quant_linear                 <- ops/kernels/quant/quant_dispatch.h:11-15
//   tts::grouped_quant_gemm                  <- ops/kernels/quant/quant_dispatch.h:7-10
//   tts::launch_quantized_norm               <- ops/kernels/quant/quant_norm.h:5-7
//   tts::launch_quantized_gated,
//     quant_gated_supports_clusters          <- ops/kernels/quant/quant_gated.h:5-8
//   tts::Buffer                              <- core/buffer.h:4 (Tensor::Storage, device subset)
//   tts::QkvProjectionOutput                 <- core/qkv_projection.h:6-10 (fields only)
//   tts::QuantizedGemm                       <- ops/cuda/quantization.h:15-42
//     (normalized_linear                     <- ops/kernels/sequence/norm_projection.h:15)
//   tts::QuantizationWorkspace               <- layers/quantization.h:9-49
//   tts::ops::LinearOperand, linear,
//     normalized_linear                      <- ops/linear.h:8-18 (quantized weights)
//   tts::ops::quantize_rows / matmul /
//     prepare_quantized                      <- ops/storage.h:12, ops/basic.h:11,25-26
//   tts::ops::quantized_norm / quantized_gated <- ops/basic.h:33-35
//
// Errors: std::invalid_argument for shape/type/alignment/workspace problems,
// std::runtime_error for device errors and missing kernel variants,
// std::logic_error for unprepared shapes — as the reference throws.
// Device pointers only; nothing here allocates device memory except Buffer
// and QuantizationWorkspace, which own their memory like the reference's.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <set>
#include <string>
#include <tuple>
#include <variant>

#include "qlinear.h"

namespace tts {

// ---------------------------------------------------------------- tensors
enum class Type { BF16, F32, I32, FP8, I8, F16, I16, I64, F64 };

inline size_t bytes(Type type) {
    if (type == Type::I64 || type == Type::F64) return 8;
    return (type == Type::FP8 || type == Type::I8)                                   ? 1
           : (type == Type::BF16 || type == Type::F16 || type == Type::I16) ? 2
                                                                                      : 4;
}

struct TensorView {
    void *data = nullptr;
    int rows = 0, cols = 0;
    Type type = Type::BF16;
    int stride = 0;  // row stride in elements; zero means dense
    int device = -1;
    TensorView() = default;
    TensorView(void *pointer, int row_count, int column_count, Type data_type = Type::BF16,
               int leading_dimension = 0, int ordinal = -1)
        : data(pointer), rows(row_count), cols(column_count), type(data_type),
          stride(leading_dimension), device(ordinal) {
        if (rows < 0 || cols < 0) throw std::invalid_argument("negative tensor dimension");
        if (stride < 0 || (stride && stride < cols))
            throw std::invalid_argument("invalid tensor stride");
        if (size_t(rows) * size_t(cols) && !pointer)
            throw std::invalid_argument("invalid tensor pointer/stride");
    }
    int ld() const { return stride ? stride : cols; }
    bool dense() const { return rows <= 1 || ld() == cols; }
    // Whether the byte ranges the two views span intersect.
    bool overlaps(const TensorView &other) const {
        if (!data || !other.data || !numel() || !other.numel()) return false;
        const auto begin = reinterpret_cast<uintptr_t>(data);
        const auto other_begin = reinterpret_cast<uintptr_t>(other.data);
        const uintptr_t end = begin + (size_t(rows - 1) * ld() + cols) * bytes(type);
        const uintptr_t other_end =
            other_begin + (size_t(other.rows - 1) * other.ld() + other.cols) * bytes(other.type);
        return begin < other_end && other_begin < end;
    }
    size_t numel() const { return size_t(rows) * size_t(cols); }
    size_t size() const { return numel() * bytes(type); }
    template <typename T> T *ptr() const { return static_cast<T *>(data); }
};

// Owned device memory (the reference's Buffer = Tensor::Storage, core/buffer.h,
// core/tensor_storage.h:13-37, device subset): hipMalloc'ed on the current
// device, released on destruction; views borrow it.
class Buffer {
  public:
    Buffer() = default;
    explicit Buffer(size_t bytes);
    ~Buffer();
    Buffer(const Buffer &) = delete;
    Buffer &operator=(const Buffer &) = delete;
    Buffer(Buffer &&other) noexcept;
    Buffer &operator=(Buffer &&other) noexcept;
    void *data() const { return data_; }
    size_t size() const { return size_; }
    int device() const { return device_; }
    template <class Value> Value *ptr() const { return static_cast<Value *>(data_); }
    TensorView view(int rows, int columns, Type dtype = Type::BF16, size_t offset = 0,
                    int stride = 0) const;

  private:
    void *data_ = nullptr;
    size_t size_ = 0;
    int device_ = -1;
};

// ---------------------------------------------------------------- quantization metadata
enum class Quantization { None, FP8, INT8, GroupINT8, GroupFP8 };

const char *quantization_name(Quantization quantization);
Quantization quantization_from_string(const std::string &name);
Type quantized_type(Quantization quantization);

struct QuantizationGroups {
    int activation = 0, weight = 0, rotation = 0;
};
QuantizationGroups quantization_groups(Quantization quantization);

// Values row-major; scales [rows] (group 0) or [ceil(cols/group), rows].
struct RowScaledView {
    TensorView values, scales;
    int group_size = 0, rotation_size = 0;
    int groups() const { return group_size ? (values.cols + group_size - 1) / group_size : 1; }
    void validate() const;
};

struct KernelProblem {
    int rows, channels, reduction;
    int input_group = 0, weight_group = 0;
};

int row_capacity(int rows, unsigned bins_per_octave = 8);

// ---------------------------------------------------------------- kernel launchers
enum class LinearKind { Auto = QLIN_KIND_AUTO, Skinny = QLIN_KIND_SKINNY, Tiled = QLIN_KIND_TILED };
struct LinearPath {
    LinearKind kind = LinearKind::Auto;
    int tokens = 0, channels = 0, splits = 1, waves = 1, staged = 0;
};

void launch_row_quantize(TensorView source, RowScaledView destination, qlin_stream_t stream);
void launch_quant_linear(LinearPath config, KernelProblem shape, const void *input,
                         const float *input_scales, const void *weights,
                         const float *weight_scales, void *output, void *workspace,
                         size_t workspace_bytes, qlin_stream_t stream, Type format = Type::FP8,
                         Type output_type = Type::BF16);
void grouped_quant_gemm(KernelProblem, const void *input, const float *input_scales,
                        const void *weights, const float *weight_scales, void *output,
                        qlin_stream_t, Type format, Type output_type, int tokens = 16,
                        int splits = 1, void *workspace = nullptr, size_t workspace_bytes = 0);

// Fused quantizing producers. `residual` is updated in place when `update` is
// given; `update_scale` may be empty. The gated input is [rows, 2*width]
// (gate | up); kind 0 = SiLU, 1 = tanh-GeLU. Workgroup clusters do not exist
// on gfx950: `multiprocessors` and `clusters` are accepted and unused, and
// quant_gated_supports_clusters() is false.
void launch_quantized_norm(TensorView residual, TensorView update, TensorView weight,
                           RowScaledView output, float epsilon, bool gemma,
                           TensorView update_scale, qlin_stream_t stream);
bool quant_gated_supports_clusters(int device);
void launch_quantized_gated(TensorView input, RowScaledView output, int kind,
                            qlin_stream_t stream, int multiprocessors = 0, bool clusters = false);

// ---------------------------------------------------------------- finish epilogue
namespace ops {
// Activation kinds (reference ops/activation.h:4); the quantized finish
// supports Relu and GeluTanh (ops/cuda/quantization.cpp:75-82).
enum class Activation { Identity, Relu, LeakyRelu, Silu, Gelu, GeluTanh, Mish, Tanh, Sigmoid };
// The reference's ops::Epilogue (ops/sequence.h:8-27) without the packed /
// indirect addressing (packed, condition_sources, output_rows), which only
// its non-quantized pointwise consumers use. The quantized GEMM's fused
// finish covers bias + ReLU / tanh-GeLU; pointwise and pointwise_quantize
// cover all of it.
struct Epilogue {
    TensorView bias, residual;
    float value_scale = 1;
    float output_scale = 1;
    float residual_scale = 1;
    Activation activation = Activation::Identity;
    float alpha = .1f;
    TensorView raw;
    TensorView gate;
    TensorView condition;
    int rows_per_sequence = 1;
    int valid_rows_per_sequence = 0;  // zero disables sequence-tail masking
    int input_repeat = 1;
    const int *residual_rows = nullptr;  // index into residual rows; negative = none
};
// Fusions of a normalization's input (reference ops/sequence.h:55-59). The
// fused normalized projection declines source_rows (normalized_linear
// returns false), as the reference's does.
struct NormFusion {
    TensorView residual, projection_bias, raw, gate, shift, scale;
    int rows_per_sequence = 1;
    const int *source_rows = nullptr;
};
}  // namespace ops

// The fused QKV-projection cache writeback target (reference
// core/qkv_projection.h:6-10). The writeback kernel belongs to the attention
// path, which this library does not include: the normalized projections
// return false when given one, and the caller takes its unfused path.
struct QkvProjectionOutput {
    TensorView query, keys, values, bias;
    const int *positions = nullptr;
    int key_value_channels = 0, capacity = 0;
};

// ---------------------------------------------------------------- QuantizedGemm
struct SelectionStats {
    size_t entries = 0, hits = 0, searches = 0;
};
struct QuantCacheStats {
    SelectionStats selection;
    size_t prepared_plans = 0;
};

// Plans are prepared per row-capacity class at initialization and sealed;
// linear() only looks them up. `workspace` is caller-owned device memory
// (split-K partials), as the reference's CudaContext::gemm_workspace.
class QuantizedGemm {
  public:
    // The reference's constructor (ops/cuda/quantization.h:20-21): the BLAS
    // handle is accepted and unused (every GEMM is this library's own);
    // `workspace` receives the split-K partials and must outlive the object.
    QuantizedGemm(qlin_stream_t stream, void *blas_handle, Buffer &workspace,
                  Type format = Type::FP8);
    QuantizedGemm(qlin_stream_t stream, void *workspace, size_t workspace_bytes,
                  Type format = Type::FP8);
    QuantizedGemm(const QuantizedGemm &) = delete;
    void seal();
    QuantCacheStats cache_stats() const;
    void prepare(int rows, int output_channels, int input_channels, Type output_type = Type::BF16,
                 QuantizationGroups groups = {});
    // Registers the fused finish of a prepared projection (reference
    // ops/cuda/quantization.cpp:395-455): a bias / ReLU / tanh-GeLU finish
    // that linear_finish may then run in the GEMM's epilogue; any other
    // epilogue is ignored. logic_error when the projection itself was not
    // prepared.
    void prepare_finish(int rows, int output_channels, int input_channels, Type output_type,
                        const ops::Epilogue &finish, QuantizationGroups groups = {});
    void linear(RowScaledView input, RowScaledView weight, TensorView output);
    // ops::linear's quantize_rows + linear as one call (no reference
    // counterpart; qlin_linear): `scratch` receives the quantized input as
    // quantize_rows would fill it, then `linear(scratch, weight, output)`,
    // in one launch on decode paths that quantize inside the GEMM.
    void quantize_linear(TensorView input, RowScaledView scratch, RowScaledView weight,
                         TensorView output);
    // Fused bias + ReLU / tanh-GeLU finish (reference linear_finish,
    // ops/cuda/quantization.cpp:465-478), also bias-only: false when the
    // epilogue is none of those or its finish was not prepared (the caller
    // then finishes separately).
    bool linear_finish(RowScaledView input, RowScaledView weight, TensorView output,
                       const ops::Epilogue &finish);
    // LayerNorm -> quantize -> GEMV in one launch for hidden sizes <= 512
    // (reference QuantizedGemm::normalized_linear, ops/cuda/quantization.cpp:
    // 479-494): false when the request is outside that kernel (the caller
    // then normalizes and projects separately, as the reference does).
    bool normalized_linear(TensorView input, TensorView normalized, TensorView norm_weight,
                           TensorView norm_bias, float epsilon, const ops::NormFusion &fusion,
                           RowScaledView weight, TensorView output,
                           const ops::Epilogue &epilogue = {}, RowScaledView encoded = {},
                           const QkvProjectionOutput *writeback = nullptr);
    LinearPath planned(int rows, int output_channels, int input_channels,
                       Type output_type = Type::BF16, QuantizationGroups groups = {}) const;
    Type format() const { return format_; }
    qlin_stream_t stream() const { return stream_; }

  private:
    using Key = std::tuple<int, int, int, Type, int, int>;
    using FinishKey = std::tuple<Key, ops::Activation, bool>;  // + bias present
    qlin_stream_t stream_;
    void *workspace_;
    size_t workspace_bytes_;
    Type format_;
    bool sealed_ = false;
    std::map<Key, LinearPath> plans_;
    std::set<FinishKey> finishes_;
    SelectionStats stats_;
};

// ---------------------------------------------------------------- activation workspace
// Reusable activation storage (reference layers/quantization.h:9-49); owns
// device buffers allocated with hipMalloc.
class QuantizationWorkspace {
  public:
    struct Capacity {
        int columns = 0, scales_per_row = 0;
        static Capacity matrix(int columns, int group_size) {
            return {columns, group_size ? (columns + group_size - 1) / group_size : 1};
        }
    };
    QuantizationWorkspace() = default;
    QuantizationWorkspace(int rows, Capacity capacity);
    ~QuantizationWorkspace();
    QuantizationWorkspace(const QuantizationWorkspace &) = delete;
    QuantizationWorkspace &operator=(const QuantizationWorkspace &) = delete;
    RowScaledView view(int rows, int columns, Type format, QuantizationGroups layout) const;

  private:
    void *values_ = nullptr, *scales_ = nullptr;
    int rows_ = 0;
    Capacity capacity_;
};

// ---------------------------------------------------------------- semantic ops
namespace ops {
// The execution context the reference resolves per device
// (execution_context(device)); here bound once per device by the host.
void bind(int device, QuantizedGemm *gemm);
QuantizedGemm &context(int device);

void quantize_rows(TensorView input, RowScaledView output);
// Operand of a projection (reference ops/linear.h:8): a dense 16-bit matrix,
// or quantized values with row scales.
using LinearOperand = std::variant<TensorView, RowScaledView>;
// Pointwise epilogue -> row quantization (reference ops/sequence.h:38-42,
// sequence_pointwise.cu:307-357); `multiprocessors` is accepted and unused.
void pointwise_quantize(TensorView x, RowScaledView quantized, const Epilogue &e = {},
                        TensorView retained = {}, int multiprocessors = 0);
// Dense pointwise epilogue (reference ops/sequence.h:34,
// sequence_pointwise.cu:281-287): y = e(x) in x's 16-bit type; y may be x.
void pointwise(TensorView x, TensorView y, const Epilogue &e = {});
// LayerNorm -> row quantization (reference ops/sequence.h:63-65,
// sequence_norm.cu:412-440).
void layer_norm_quantize(TensorView x, RowScaledView quantized, TensorView weight, TensorView bias,
                         float eps, const NormFusion &fusion = {}, TensorView retained = {});
void matmul(RowScaledView input, RowScaledView weight, TensorView output);
// prepare + prepare_finish of the bound context (reference ops/basic.h:25-26,
// ops/basic.cpp:48-53).
void prepare_quantized(TensorView weight, int rows, int output_channels, int input_channels,
                       Type type, const Epilogue &epilogue = {}, QuantizationGroups groups = {});
void quantized_norm(TensorView input, TensorView update, TensorView weight, RowScaledView output,
                    float epsilon, bool gemma = false, TensorView scale = {});
void quantized_gated(TensorView input, RowScaledView output, int kind);
// The reference's ops::linear (ops/linear.h:11-13, ops/linear.cpp:26-93) for
// quantized weights. A dense `input` is quantized into `scratch` (one launch
// with the GEMM on decode paths without an epilogue); a RowScaledView input
// is used as is. A prepared bias + ReLU / tanh-GeLU finish runs in the
// GEMM's epilogue; with `quantized_output` the output is also quantized for
// the next layer, through the fused finish and quantize_rows, or the GEMM
// and pointwise_quantize for any other dense epilogue. Without
// `quantized_output`, an epilogue that is not a prepared fused finish runs
// as the GEMM followed by pointwise(output, output, e), as the reference
// does (ops/linear.cpp:79-82). A dense (TensorView) weight is rejected with
// invalid_argument: dense GEMMs are not part of this library.
void linear(const LinearOperand &input, const LinearOperand &weight, TensorView bias,
            TensorView output, Epilogue epilogue = {}, RowScaledView scratch = {},
            RowScaledView quantized_output = {});
// The reference's ops::normalized_linear (ops/linear.h:14-18,
// ops/linear.cpp:94-131) for quantized weights: LayerNorm -> quantize ->
// GEMV in one launch (QuantizedGemm::normalized_linear), optionally followed
// by the next layer's quantization. Returns false, leaving the caller's
// unfused path responsible, for requests outside that kernel: a dense
// weight, a QKV writeback, hidden sizes above 512, source-row gathers.
bool normalized_linear(TensorView input, const LinearOperand &weight, TensorView bias,
                       TensorView normalized, TensorView output, TensorView norm_weight,
                       TensorView norm_bias, float epsilon, const NormFusion &fusion,
                       Epilogue epilogue = {}, const QkvProjectionOutput *writeback = nullptr,
                       RowScaledView quantized_output = {});
}  // namespace ops

}  // namespace tts
