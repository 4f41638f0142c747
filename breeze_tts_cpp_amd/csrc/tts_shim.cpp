// C++ host interface (include/tts_qlinear.hpp) over the C ABI: the reference's
// layer/op names and exceptions, implemented by calls into qlin_* entry points.
#include "../../include/tts_qlinear.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <limits>
#include <mutex>

namespace tts {
namespace {

// Status -> exception of the reference's kind.
void check(int status, const char *what) {
    if (!status) return;
    std::string message = std::string(what) + ": " + qlin_last_error();
    switch (status) {
    case QLIN_ERR_INVALID:
    case QLIN_ERR_ALIGNMENT:
    case QLIN_ERR_WORKSPACE: throw std::invalid_argument(message);
    default: throw std::runtime_error(message);
    }
}

int code(Type type) { return static_cast<int>(type); }

}  // namespace

// ---------------------------------------------------------------- Buffer
Buffer::Buffer(size_t bytes) : size_(bytes) {
    if (hipGetDevice(&device_) != hipSuccess) throw std::runtime_error("no HIP device");
    if (bytes && hipMalloc(&data_, bytes) != hipSuccess)
        throw std::runtime_error("device buffer allocation failed");
}

Buffer::~Buffer() {
    if (data_) (void)hipFree(data_);
}

Buffer::Buffer(Buffer &&other) noexcept
    : data_(other.data_), size_(other.size_), device_(other.device_) {
    other.data_ = nullptr;
    other.size_ = 0;
}

Buffer &Buffer::operator=(Buffer &&other) noexcept {
    if (this != &other) {
        if (data_) (void)hipFree(data_);
        data_ = other.data_;
        size_ = other.size_;
        device_ = other.device_;
        other.data_ = nullptr;
        other.size_ = 0;
    }
    return *this;
}

// core/tensor_storage.h:35: a borrowed view at a byte offset, bounds-checked.
TensorView Buffer::view(int rows, int columns, Type dtype, size_t offset, int stride) const {
    const int ld = stride ? stride : columns;
    const size_t span = rows && columns ? (size_t(rows - 1) * ld + columns) * bytes(dtype) : 0;
    if (rows < 0 || columns < 0 || offset > size_ || span > size_ - offset)
        throw std::invalid_argument("buffer view out of range");
    return TensorView(static_cast<char *>(data_) + offset, rows, columns, dtype, stride, device_);
}

// ---------------------------------------------------------------- metadata
// include/tts/quantization.h:8-29
const char *quantization_name(Quantization quantization) {
    switch (quantization) {
    case Quantization::None: return "none";
    case Quantization::FP8: return "fp8";
    case Quantization::INT8: return "int8";
    case Quantization::GroupINT8: return "group_int8";
    case Quantization::GroupFP8: return "group_fp8";
    }
    throw std::invalid_argument("invalid quantization mode");
}

Quantization quantization_from_string(const std::string &name) {
    if (name.empty()) return Quantization::None;
    if (name == "fp8") return Quantization::FP8;
    if (name == "int8") return Quantization::INT8;
    if (name == "group_int8") return Quantization::GroupINT8;
    if (name == "group_fp8") return Quantization::GroupFP8;
    throw std::invalid_argument("quantization must be int8, fp8, group_int8 or group_fp8");
}

// core/quantization.h:6-23
Type quantized_type(Quantization quantization) {
    if (quantization == Quantization::FP8 || quantization == Quantization::GroupFP8)
        return Type::FP8;
    if (quantization == Quantization::INT8 || quantization == Quantization::GroupINT8)
        return Type::I8;
    throw std::invalid_argument("BF16 has no quantized storage type");
}

QuantizationGroups quantization_groups(Quantization quantization) {
    if (quantization == Quantization::GroupINT8 || quantization == Quantization::GroupFP8)
        return {128, 128, 128};
    return {};
}

// core/quantization.h:39-48
void RowScaledView::validate() const {
    const bool groups_ok =
        !group_size || group_size == 32 || group_size == 64 || group_size == 128;
    if ((values.type != Type::FP8 && values.type != Type::I8) || !values.dense() ||
        (rotation_size && (rotation_size != 128 || values.cols % 128)) || !groups_ok ||
        scales.type != Type::F32 || !scales.dense() ||
        scales.numel() != size_t(values.rows) * size_t(groups()) ||
        (group_size && (scales.rows != groups() || scales.cols != values.rows)) ||
        values.device != scales.device)
        throw std::invalid_argument("invalid row-scaled quantized tensor");
}

// core/row_capacity.h:10-19
int row_capacity(int rows, unsigned bins_per_octave) {
    if (rows < 1 || !bins_per_octave) throw std::invalid_argument("invalid row capacity class");
    int64_t upper = 1;
    while (upper < rows) upper *= 2;
    int64_t step = std::max<int64_t>(1, upper / (2ll * bins_per_octave));
    int64_t capacity = (int64_t(rows) + step - 1) / step * step;
    return int(std::min<int64_t>(capacity, std::numeric_limits<int>::max()));
}

// ---------------------------------------------------------------- launchers
void launch_row_quantize(TensorView source, RowScaledView destination, qlin_stream_t stream) {
    check(qlin_row_quantize(source.data, source.ld(), source.rows, source.cols, code(source.type),
                            destination.values.data, destination.scales.ptr<float>(),
                            code(destination.values.type), destination.group_size,
                            destination.rotation_size, stream),
          "row quantization");
}

// quant_norm.cu:166-188: the reference's shape/type checks, then the kernel.
void launch_quantized_norm(TensorView residual, TensorView update, TensorView weight,
                           RowScaledView output, float epsilon, bool gemma,
                           TensorView update_scale, qlin_stream_t stream) {
    output.validate();
    if ((residual.type != Type::BF16 && residual.type != Type::F16) || !residual.data ||
        !weight.data || !output.values.data || !output.scales.data || !residual.dense() ||
        residual.cols < 1 || residual.cols > 2048 || residual.rows < 1 ||
        residual.cols != output.values.cols || residual.rows != output.values.rows ||
        weight.type != residual.type || !weight.dense() ||
        weight.numel() != size_t(residual.cols) ||
        (update.data && (update.type != residual.type || update.rows != residual.rows ||
                         update.cols != residual.cols || !update.dense())) ||
        (update_scale.data && (update_scale.type != residual.type || !update_scale.dense() ||
                               update_scale.numel() != size_t(residual.cols))))
        throw std::invalid_argument("quantized RMS shape/type mismatch");
    check(qlin_quantized_norm(residual.data, update.data, update.data ? update_scale.data : nullptr,
                              weight.data, code(residual.type), residual.rows, residual.cols,
                              epsilon, gemma ? 1 : 0, output.values.data,
                              output.scales.ptr<float>(), code(output.values.type),
                              output.group_size, output.rotation_size, stream),
          "quantized norm");
}

bool quant_gated_supports_clusters(int) { return false; }

// quant_gated.cu:182-198: the reference's checks; one workgroup per row on gfx950.
void launch_quantized_gated(TensorView input, RowScaledView output, int kind,
                            qlin_stream_t stream, int, bool) {
    output.validate();
    const int width = output.values.cols;
    if ((input.type != Type::BF16 && input.type != Type::F16) || !input.data ||
        !output.values.data || !output.scales.data || !input.dense() ||
        input.rows != output.values.rows || input.cols != int64_t(2) * width || kind < 0 ||
        kind > 1 || width < 1 || width > 8192 || input.rows < 1)
        throw std::invalid_argument("quantized gated shape/type mismatch");
    check(qlin_quantized_gated(input.data, code(input.type), input.rows, width, kind,
                               output.values.data, output.scales.ptr<float>(),
                               code(output.values.type), output.group_size, output.rotation_size,
                               stream),
          "quantized gated");
}

void launch_quant_linear(LinearPath config, KernelProblem shape, const void *input,
                         const float *input_scales, const void *weights,
                         const float *weight_scales, void *output, void *workspace,
                         size_t workspace_bytes, qlin_stream_t stream, Type format,
                         Type output_type) {
    qlin_path path{static_cast<int>(config.kind), config.tokens, config.channels, config.splits,
                   config.waves, config.staged};
    check(qlin_gemm(&path, input, input_scales, weights, weight_scales, output, shape.rows,
                    shape.channels, shape.reduction, code(format), code(output_type),
                    shape.input_group, shape.weight_group, workspace, workspace_bytes, stream),
          "quantized GEMM");
}

// quant_grouped.cu:221-239: the token tile and split count select the variant;
// splits > 1 need a workspace of rows*channels*splits floats.
void grouped_quant_gemm(KernelProblem problem, const void *input, const float *input_scales,
                        const void *weights, const float *weight_scales, void *output,
                        qlin_stream_t stream, Type format, Type output_type, int tokens,
                        int splits, void *workspace, size_t workspace_bytes) {
    if (!problem.input_group && !problem.weight_group)
        throw std::invalid_argument("grouped GEMM requires K-group scales");
    qlin_path planned{};
    check(qlin_plan(problem.rows, problem.channels, problem.reduction, code(format),
                    problem.input_group, problem.weight_group, &planned),
          "grouped GEMM plan");
    LinearPath path{static_cast<LinearKind>(planned.kind), planned.tokens, planned.channels,
                    planned.splits, planned.waves, planned.staged};
    if (path.kind == LinearKind::Skinny) {
        path.tokens = std::max(16, std::min(64, tokens));
        if (splits > 1) path.splits = splits;
    }
    launch_quant_linear(path, problem, input, input_scales, weights, weight_scales, output,
                        workspace, workspace_bytes, stream, format, output_type);
}

// ---------------------------------------------------------------- QuantizedGemm
QuantizedGemm::QuantizedGemm(qlin_stream_t stream, void *, Buffer &workspace, Type format)
    : QuantizedGemm(stream, workspace.data(), workspace.size(), format) {}

QuantizedGemm::QuantizedGemm(qlin_stream_t stream, void *workspace, size_t workspace_bytes,
                             Type format)
    : stream_(stream), workspace_(workspace), workspace_bytes_(workspace_bytes), format_(format) {
    if (format != Type::FP8 && format != Type::I8)
        throw std::invalid_argument("unsupported quantized storage type");
}

void QuantizedGemm::seal() { sealed_ = true; }

QuantCacheStats QuantizedGemm::cache_stats() const {
    QuantCacheStats result{};
    result.selection = stats_;
    result.selection.entries = plans_.size();
    result.prepared_plans = plans_.size() + finishes_.size();
    return result;
}

LinearPath QuantizedGemm::planned(int rows, int channels, int reduction, Type output_type,
                                  QuantizationGroups groups) const {
    auto it = plans_.find(Key{row_capacity(rows), channels, reduction, output_type,
                              groups.activation, groups.weight});
    if (it == plans_.end())
        throw std::logic_error("quantized GEMM shape was not prepared before execution");
    return it->second;
}

// ops/cuda/quantization.cpp:366-393 and the shape rules of make_plan (:206-222).
void QuantizedGemm::prepare(int rows, int channels, int reduction, Type output_type,
                            QuantizationGroups groups) {
    if (output_type != Type::BF16 && output_type != Type::F16)
        throw std::invalid_argument("quantized GEMM output must be F16 or BF16");
    rows = row_capacity(rows);
    Key key{rows, channels, reduction, output_type, groups.activation, groups.weight};
    if (plans_.count(key)) {
        ++stats_.hits;
        return;
    }
    if (sealed_) throw std::logic_error("prepared resource missing after initialization");
    if (rows < 1 || channels < 1 || reduction < 1 || reduction % 16 || channels % 16)
        throw std::invalid_argument("quantized GEMM unsupported shape");
    if (format_ == Type::I8 && reduction > INT32_MAX / (128 * 128))
        throw std::invalid_argument("INT8 reduction can overflow INT32");
    qlin_path p{};
    check(qlin_plan(rows, channels, reduction, code(format_), groups.activation, groups.weight,
                    &p),
          "quantized GEMM plan");
    if (qlin_workspace_bytes(&p, rows, channels, reduction, code(format_), groups.activation,
                             groups.weight) > workspace_bytes_)
        throw std::invalid_argument("quantized GEMM workspace overflow");
    plans_.emplace(key, LinearPath{static_cast<LinearKind>(p.kind), p.tokens, p.channels,
                                   p.splits, p.waves, p.staged});
    ++stats_.searches;
}

// ops/cuda/quantization.cpp:94-102 (check_linear) and :455-464.
void QuantizedGemm::linear(RowScaledView input, RowScaledView weight, TensorView output) {
    input.validate();
    weight.validate();
    if (input.values.type != format_ || weight.values.type != format_ ||
        input.rotation_size != weight.rotation_size || input.values.cols != weight.values.cols ||
        input.values.rows != output.rows || weight.values.rows != output.cols ||
        (output.type != Type::BF16 && output.type != Type::F16) || !output.dense())
        throw std::invalid_argument("quantized linear dimensions/type mismatch");
    const QuantizationGroups groups{input.group_size, weight.group_size, input.rotation_size};
    LinearPath path = planned(output.rows, output.cols, input.values.cols, output.type, groups);
    launch_quant_linear(path,
                        {output.rows, output.cols, input.values.cols, input.group_size,
                         weight.group_size},
                        input.values.data, input.scales.ptr<float>(), weight.values.data,
                        weight.scales.ptr<float>(), output.data, workspace_, workspace_bytes_,
                        stream_, format_, output.type);
}

void QuantizedGemm::quantize_linear(TensorView input, RowScaledView scratch,
                                    RowScaledView weight, TensorView output) {
    // The checks of linear() on the scratch as its input, then qlin_linear.
    scratch.validate();
    weight.validate();
    if (scratch.values.type != format_ || weight.values.type != format_ ||
        scratch.rotation_size != weight.rotation_size || scratch.values.cols != weight.values.cols ||
        scratch.values.rows != output.rows || weight.values.rows != output.cols ||
        (output.type != Type::BF16 && output.type != Type::F16) || !output.dense())
        throw std::invalid_argument("quantized linear dimensions/type mismatch");
    const QuantizationGroups groups{scratch.group_size, weight.group_size, scratch.rotation_size};
    const LinearPath path = planned(output.rows, output.cols, scratch.values.cols, output.type,
                                    groups);
    qlin_path p{static_cast<int>(path.kind), path.tokens, path.channels, path.splits,
                path.waves, path.staged};
    check(qlin_linear(&p, input.data, input.ld(), code(input.type), scratch.values.data,
                      scratch.scales.ptr<float>(), weight.values.data, weight.scales.ptr<float>(),
                      output.data, int(output.rows), int(output.cols), int(scratch.values.cols),
                      code(format_), code(output.type), scratch.group_size, weight.group_size,
                      scratch.rotation_size, workspace_, workspace_bytes_, stream_),
          "quantized linear");
}

namespace {
// An epilogue with nothing beyond bias and activation.
bool finish_only(const ops::Epilogue &e) {
    return !e.residual.data && !e.raw.data && !e.gate.data && !e.condition.data &&
           !e.residual_rows && e.value_scale == 1 && e.output_scale == 1 &&
           !e.valid_rows_per_sequence && e.input_repeat == 1;
}

// The finish the GEMM epilogue runs: ReLU or tanh-GeLU (the reference's
// simple_finish, ops/cuda/quantization.cpp:75-82), or a bias alone; -1 for
// any other epilogue.
int finish_activation(const ops::Epilogue &e) {
    if (!finish_only(e)) return -1;
    if (e.activation == ops::Activation::Relu) return QLIN_FINISH_RELU;
    if (e.activation == ops::Activation::GeluTanh) return QLIN_FINISH_GELU_TANH;
    if (e.activation == ops::Activation::Identity && e.bias.data) return QLIN_FINISH_NONE;
    return -1;
}

// check_finish_bias (ops/cuda/quantization.cpp:83-87)
void check_finish_bias(const ops::Epilogue &e, int channels, Type output_type) {
    if (e.bias.data && (e.bias.type != output_type || !e.bias.dense() ||
                        e.bias.numel() != size_t(channels)))
        throw std::invalid_argument("quantized linear finish bias mismatch");
}
}  // namespace

void QuantizedGemm::prepare_finish(int rows, int channels, int reduction, Type output_type,
                                   const ops::Epilogue &finish, QuantizationGroups groups) {
    if (finish_activation(finish) < 0) return;
    check_finish_bias(finish, channels, output_type);
    const Key key{row_capacity(rows), channels, reduction, output_type, groups.activation,
                  groups.weight};
    if (!plans_.count(key))
        throw std::logic_error("quantized finish requires a prepared projection");
    const FinishKey fk{key, finish.activation, finish.bias.data != nullptr};
    if (finishes_.count(fk)) return;
    if (sealed_) throw std::logic_error("prepared resource missing after initialization");
    finishes_.insert(fk);
}

bool QuantizedGemm::linear_finish(RowScaledView input, RowScaledView weight, TensorView output,
                                  const ops::Epilogue &finish) {
    // The reference fuses ReLU / tanh-GeLU; a bias-only finish (identity
    // activation) is fused here as well. Only prepared finishes run.
    const int act = finish_activation(finish);
    if (act < 0) return false;
    const Key key{row_capacity(output.rows), output.cols, input.values.cols, output.type,
                  input.group_size, weight.group_size};
    if (!finishes_.count(FinishKey{key, finish.activation, finish.bias.data != nullptr}))
        return false;
    input.validate();
    weight.validate();
    if (input.values.type != format_ || weight.values.type != format_ ||
        input.rotation_size != weight.rotation_size || input.values.cols != weight.values.cols ||
        input.values.rows != output.rows || weight.values.rows != output.cols ||
        (output.type != Type::BF16 && output.type != Type::F16) || !output.dense())
        throw std::invalid_argument("quantized linear dimensions/type mismatch");
    check_finish_bias(finish, output.cols, output.type);
    const QuantizationGroups groups{input.group_size, weight.group_size, input.rotation_size};
    LinearPath path = planned(output.rows, output.cols, input.values.cols, output.type, groups);
    qlin_path c{static_cast<int>(path.kind), path.tokens, path.channels, path.splits, path.waves,
                path.staged};
    check(qlin_gemm_finish(&c, input.values.data, input.scales.ptr<float>(), weight.values.data,
                           weight.scales.ptr<float>(), finish.bias.data, act, output.data,
                           output.rows, output.cols, input.values.cols, code(format_),
                           code(output.type), input.group_size, weight.group_size, 0, workspace_,
                           workspace_bytes_, stream_),
          "quantized GEMM finish");
    return true;
}

bool QuantizedGemm::normalized_linear(TensorView input, TensorView normalized,
                                      TensorView norm_weight, TensorView norm_bias, float epsilon,
                                      const ops::NormFusion &fusion, RowScaledView weight,
                                      TensorView output, const ops::Epilogue &epilogue,
                                      RowScaledView encoded, const QkvProjectionOutput *writeback) {
    // The QKV cache writeback belongs to the attention path (not built here).
    if (writeback) return false;
    // The conditions of normalized_quantized_linear (sequence_norm.cu:522-545).
    if (weight.group_size || weight.rotation_size || encoded.group_size || encoded.rotation_size ||
        fusion.source_rows || weight.values.type != format_)
        return false;
    if ((epilogue.activation != ops::Activation::Identity &&
         epilogue.activation != ops::Activation::Relu) || !finish_only(epilogue))
        return false;
    const int n = weight.values.rows, k = weight.values.cols;
    if (!input.data || input.rows < 1 || input.rows > 65535 || k < 4 || k % 4 || k > 512 ||
        input.cols != k || (input.type != Type::BF16 && input.type != Type::F16) ||
        output.type != input.type || output.rows != input.rows || output.cols != n ||
        !input.dense() || !output.dense())
        return false;
    if (normalized.data && (normalized.rows != input.rows || normalized.cols != k ||
                            normalized.type != input.type))
        return false;
    for (const TensorView *v : std::initializer_list<const TensorView *>{&norm_weight, &norm_bias, &fusion.projection_bias})
        if (v->data && (v->type != input.type || v->numel() != size_t(k)))
            throw std::invalid_argument("normalization parameter mismatch");
    if (fusion.residual.data && (fusion.residual.type != input.type ||
                                 fusion.residual.rows != input.rows || fusion.residual.cols != k))
        throw std::invalid_argument("normalization residual mismatch");
    if (epilogue.bias.data && (epilogue.bias.type != output.type ||
                               epilogue.bias.numel() != size_t(n)))
        throw std::invalid_argument("quantized linear finish bias mismatch");
    if ((encoded.values.data || encoded.scales.data) &&
        (encoded.values.type != format_ || encoded.values.rows != input.rows ||
         encoded.values.cols != k))
        throw std::invalid_argument("normalized projection quantized output mismatch");
    if (!(epsilon > 0)) throw std::invalid_argument("invalid layer normalization");
    const int sequences = fusion.rows_per_sequence > 0 ? input.rows / fusion.rows_per_sequence : 0;
    for (const TensorView *v : std::initializer_list<const TensorView *>{&fusion.gate, &fusion.shift, &fusion.scale})
        if (v->data && (v->type != input.type || v->cols != k || (v->rows != 1 && v->rows != sequences)))
            throw std::invalid_argument("invalid normalization modulation");
    if (fusion.raw.data && (fusion.raw.type != input.type || fusion.raw.rows != input.rows ||
                            fusion.raw.cols != k))
        throw std::invalid_argument("sequence operation shape/type mismatch");
    qlin_norm_fusion f;
    qlin_norm_fusion_init(&f);
    f.residual = fusion.residual.data;
    f.projection_bias = fusion.projection_bias.data;
    f.gate = fusion.gate.data;
    f.gate_rows = fusion.gate.rows;
    f.shift = fusion.shift.data;
    f.shift_rows = fusion.shift.rows;
    f.scale = fusion.scale.data;
    f.scale_rows = fusion.scale.rows;
    f.raw = fusion.raw.data;
    f.rows_per_sequence = fusion.rows_per_sequence;
    check(qlin_norm_linear(input.data, &f, norm_weight.data, norm_bias.data, code(input.type), input.rows, k,
                           epsilon, weight.values.data, weight.scales.ptr<float>(), code(format_),
                           n, epilogue.bias.data,
                           epilogue.activation == ops::Activation::Relu ? QLIN_FINISH_RELU
                                                                        : QLIN_FINISH_NONE,
                           output.data, normalized.data, encoded.values.data,
                           encoded.scales.ptr<float>(), stream_),
          "normalized quantized linear");
    return true;
}

// ---------------------------------------------------------------- workspace
QuantizationWorkspace::QuantizationWorkspace(int rows, Capacity capacity)
    : rows_(rows), capacity_(capacity) {
    if (rows < 1 || capacity.columns < 0 || capacity.scales_per_row < 0 ||
        bool(capacity.columns) != bool(capacity.scales_per_row))
        throw std::invalid_argument("invalid quantization workspace capacity");
    const size_t values = size_t(rows) * size_t(std::max(1, capacity.columns));
    const size_t scales = size_t(rows) * size_t(std::max(1, capacity.scales_per_row)) * 4;
    if (hipMalloc(&values_, values) != hipSuccess || hipMalloc(&scales_, scales) != hipSuccess)
        throw std::runtime_error("quantization workspace allocation failed");
}

QuantizationWorkspace::~QuantizationWorkspace() {
    if (values_) (void)hipFree(values_);
    if (scales_) (void)hipFree(scales_);
}

// layers/quantization.h:39-48
RowScaledView QuantizationWorkspace::view(int rows, int columns, Type format,
                                          QuantizationGroups layout) const {
    const auto required = Capacity::matrix(columns, layout.activation);
    if (rows < 1 || rows > rows_ || columns < 1 || columns > capacity_.columns ||
        required.scales_per_row > capacity_.scales_per_row ||
        (format != Type::FP8 && format != Type::I8))
        throw std::invalid_argument("projection exceeds initialized quantization workspace");
    const int scale_rows = layout.activation ? required.scales_per_row : rows;
    const int scale_cols = layout.activation ? rows : 1;
    return {TensorView(values_, rows, columns, format), TensorView(scales_, scale_rows, scale_cols,
                                                                   Type::F32),
            layout.activation, layout.rotation};
}

// ---------------------------------------------------------------- ops
namespace ops {
namespace {
std::mutex g_mutex;
std::map<int, QuantizedGemm *> g_contexts;
}  // namespace

void bind(int device, QuantizedGemm *gemm) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (gemm) g_contexts[device] = gemm;
    else g_contexts.erase(device);
}

QuantizedGemm &context(int device) {
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_contexts.find(device);
    if (it == g_contexts.end()) throw std::logic_error("no execution context bound for device");
    return *it->second;
}

// ops/basic.cpp:69-78
void quantize_rows(TensorView input, RowScaledView output) {
    output.validate();
    if ((input.type != Type::BF16 && input.type != Type::F16) || input.rows < 1 ||
        input.cols < 1 || !input.data || !output.values.data || !output.scales.data ||
        input.rows != output.values.rows || input.cols != output.values.cols)
        throw std::invalid_argument("quantization source/destination shape/type mismatch");
    launch_row_quantize(input, output, context(input.device).stream());
}

// ops/basic.cpp:64-67
void matmul(RowScaledView input, RowScaledView weight, TensorView output) {
    context(output.device).linear(input, weight, output);
}

// ops/basic.cpp:48-53
void prepare_quantized(TensorView weight, int rows, int output_channels, int input_channels,
                       Type type, const Epilogue &epilogue, QuantizationGroups groups) {
    QuantizedGemm &gemm = context(weight.device);
    gemm.prepare(rows, output_channels, input_channels, type, groups);
    gemm.prepare_finish(rows, output_channels, input_channels, type, epilogue, groups);
}

namespace {
// check_linear_output (ops/linear.cpp:17-23)
void check_linear_output(TensorView output, TensorView bias, const Epilogue &e) {
    if (e.bias.data) throw std::invalid_argument("linear already owns its bias");
    for (const TensorView &source : {bias, e.residual, e.gate, e.condition})
        if (source.overlaps(output))
            throw std::invalid_argument("linear epilogue source aliases its projection output");
}

bool plain_epilogue(const Epilogue &e) {
    return e.activation == Activation::Identity && !e.bias.data && finish_only(e);
}
}  // namespace

// ops/linear.cpp:24-93 with a quantized weight: quantize a dense input into
// the scratch (one launch with the GEMM where the decode kernel quantizes its
// own token rows), then the GEMM with the prepared fused finish; with a
// quantized output, the fused finish + quantize_rows when the formats agree,
// else the GEMM + pointwise_quantize.
void linear(const LinearOperand &input, const LinearOperand &weight, TensorView bias,
            TensorView output, Epilogue epilogue, RowScaledView scratch,
            RowScaledView quantized_output) {
    check_linear_output(output, bias, epilogue);
    epilogue.bias = bias;
    const RowScaledView *matrix = std::get_if<RowScaledView>(&weight);
    if (!matrix)
        throw std::invalid_argument(
            "dense (unquantized) linear is not part of the quantized linear library");
    matrix->validate();
    QuantizedGemm &gemm = context(output.device);
    RowScaledView activation;
    if (const TensorView *dense = std::get_if<TensorView>(&input)) {
        if (!quantized_output.values.data && plain_epilogue(epilogue)) {
            scratch.validate();
            if ((dense->type != Type::BF16 && dense->type != Type::F16) || dense->rows < 1 ||
                dense->cols < 1 || !dense->data || !scratch.values.data ||
                !scratch.scales.data || dense->rows != scratch.values.rows ||
                dense->cols != scratch.values.cols)
                throw std::invalid_argument("quantization source/destination shape/type mismatch");
            if (scratch.values.cols != matrix->values.cols || output.rows != scratch.values.rows ||
                output.cols != matrix->values.rows || !output.dense())
                throw std::invalid_argument("quantized linear dimensions/layout mismatch");
            gemm.quantize_linear(*dense, scratch, *matrix, output);
            return;
        }
        quantize_rows(*dense, scratch);
        activation = scratch;
    } else {
        activation = std::get<RowScaledView>(input);
    }
    if (activation.values.cols != matrix->values.cols || output.rows != activation.values.rows ||
        output.cols != matrix->values.rows || !output.dense())
        throw std::invalid_argument("quantized linear dimensions/layout mismatch");
    if (quantized_output.values.data) {
        if (quantized_output.values.type == matrix->values.type &&
            gemm.linear_finish(activation, *matrix, output, epilogue)) {
            quantize_rows(output, quantized_output);
            return;
        }
        gemm.linear(activation, *matrix, output);
        pointwise_quantize(output, quantized_output, epilogue);
        return;
    }
    if (plain_epilogue(epilogue)) {
        gemm.linear(activation, *matrix, output);
        return;
    }
    if (gemm.linear_finish(activation, *matrix, output, epilogue)) return;
    // Not a prepared fused finish: the GEMM, then the dense epilogue in place
    // (ops/linear.cpp:68-82).
    gemm.linear(activation, *matrix, output);
    pointwise(output, output, epilogue);
}

// ops/linear.cpp:94-131 with a quantized weight.
bool normalized_linear(TensorView input, const LinearOperand &weight, TensorView bias,
                       TensorView normalized, TensorView output, TensorView norm_weight,
                       TensorView norm_bias, float epsilon, const NormFusion &fusion,
                       Epilogue e, const QkvProjectionOutput *writeback,
                       RowScaledView quantized_output) {
    check_linear_output(output, bias, e);
    if (writeback && writeback->bias.data != bias.data)
        throw std::invalid_argument("linear already owns its bias");
    const RowScaledView *quantized = std::get_if<RowScaledView>(&weight);
    if (!quantized || writeback) return false;
    QuantizedGemm &gemm = context(input.device);
    auto project = [&](const Epilogue &epilogue) {
        return gemm.normalized_linear(input, normalized, norm_weight, norm_bias, epsilon, fusion,
                                      *quantized, output, epilogue, {}, nullptr);
    };
    e.bias = bias;
    if (quantized_output.values.data) {
        if (quantized_output.values.type == quantized->values.type && project(e)) {
            quantize_rows(output, quantized_output);
        } else {
            if (!project({})) return false;
            pointwise_quantize(output, quantized_output, e);
        }
        return true;
    }
    return project(e);
}

namespace {
qlin_epilogue to_c(const Epilogue &e) {
    qlin_epilogue c;
    qlin_epilogue_init(&c);
    c.bias = e.bias.data;
    c.residual = e.residual.data;
    c.residual_rows = e.residual.rows;
    c.residual_index = e.residual_rows;
    c.value_scale = e.value_scale;
    c.output_scale = e.output_scale;
    c.residual_scale = e.residual_scale;
    c.activation = static_cast<int>(e.activation);
    c.alpha = e.alpha;
    c.raw = e.raw.data;
    c.gate = e.gate.data;
    c.gate_rows = e.gate.rows;
    c.condition = e.condition.data;
    c.condition_rows = e.condition.rows;
    c.rows_per_sequence = e.rows_per_sequence;
    c.valid_rows_per_sequence = e.valid_rows_per_sequence;
    c.input_repeat = e.input_repeat;
    return c;
}

// The reference's check_same for a vector ([cols]) or row-matching operand.
void check_operand(const TensorView &v, Type type, int cols, const char *what) {
    if (v.data && (v.type != type || v.cols != cols || !v.dense()))
        throw std::invalid_argument(what);
}
}  // namespace

void pointwise_quantize(TensorView x, RowScaledView q, const Epilogue &e, TensorView retained, int) {
    q.validate();
    if (!x.dense() || (retained.data && (retained.type != x.type || retained.rows != q.values.rows ||
                                         retained.cols != q.values.cols || !retained.dense())))
        throw std::invalid_argument("quantized sequence output requires dense F16/BF16 rows");
    if (e.bias.data && (e.bias.type != x.type || e.bias.numel() != size_t(q.values.cols)))
        throw std::invalid_argument("sequence operation shape/type mismatch");
    check_operand(e.residual, x.type, q.values.cols, "invalid indexed residual");
    check_operand(e.raw, x.type, q.values.cols, "sequence operation shape/type mismatch");
    check_operand(e.gate, x.type, q.values.cols, "invalid epilogue gate");
    check_operand(e.condition, x.type, q.values.cols, "invalid epilogue condition");
    if (e.raw.data && e.raw.rows != q.values.rows)
        throw std::invalid_argument("sequence operation shape/type mismatch");
    if (x.cols != q.values.cols)
        throw std::invalid_argument("invalid quantized pointwise input/repetition");
    const qlin_epilogue c = to_c(e);
    check(qlin_pointwise_quantize(x.data, x.rows, code(x.type), &c, retained.data, q.values.rows,
                                  q.values.cols, q.values.data, q.scales.ptr<float>(),
                                  code(q.values.type), q.group_size, q.rotation_size,
                                  context(x.device).stream()),
          "pointwise quantize");
}

void pointwise(TensorView x, TensorView y, const Epilogue &e) {
    // check_output / check_epilogue (sequence_pointwise.cu:283-287).
    if ((y.type != Type::BF16 && y.type != Type::F16) || !y.dense() || !x.dense())
        throw std::invalid_argument("sequence output requires dense F16/BF16 rows");
    if (!x.data || e.input_repeat < 1 || x.type != y.type || x.cols != y.cols ||
        int64_t(x.rows) * e.input_repeat != y.rows || (e.input_repeat > 1 && x.data == y.data))
        throw std::invalid_argument("invalid pointwise input/repetition");
    if (e.bias.data && (e.bias.type != y.type || e.bias.numel() != size_t(y.cols)))
        throw std::invalid_argument("sequence operation shape/type mismatch");
    check_operand(e.residual, y.type, y.cols, "invalid indexed residual");
    check_operand(e.raw, y.type, y.cols, "sequence operation shape/type mismatch");
    check_operand(e.gate, y.type, y.cols, "invalid epilogue gate");
    check_operand(e.condition, y.type, y.cols, "invalid epilogue condition");
    if (e.raw.data && e.raw.rows != y.rows)
        throw std::invalid_argument("sequence operation shape/type mismatch");
    const qlin_epilogue c = to_c(e);
    check(qlin_pointwise(x.data, x.rows, code(x.type), &c, y.data, y.rows, y.cols,
                         context(y.device).stream()),
          "pointwise");
}

void layer_norm_quantize(TensorView x, RowScaledView q, TensorView weight, TensorView bias,
                         float eps, const NormFusion &f, TensorView retained) {
    q.validate();
    const int cols = q.values.cols;
    if (!x.dense() || x.cols != cols ||
        (retained.data && (retained.type != x.type || retained.rows != q.values.rows ||
                           retained.cols != cols || !retained.dense())))
        throw std::invalid_argument("sequence operation shape/type mismatch");
    for (const TensorView *v : std::initializer_list<const TensorView *>{&weight, &bias, &f.projection_bias})
        if (v->data && (v->type != x.type || v->numel() != size_t(cols)))
            throw std::invalid_argument("sequence operation shape/type mismatch");
    for (const TensorView *v : std::initializer_list<const TensorView *>{&f.residual, &f.raw, &f.gate, &f.shift, &f.scale})
        check_operand(*v, x.type, cols, "sequence operation shape/type mismatch");
    if (f.residual.data && f.residual.rows != x.rows)
        throw std::invalid_argument("sequence operation shape/type mismatch");
    qlin_norm_fusion c;
    qlin_norm_fusion_init(&c);
    c.residual = f.residual.data;
    c.projection_bias = f.projection_bias.data;
    c.gate = f.gate.data;
    c.gate_rows = f.gate.rows;
    c.shift = f.shift.data;
    c.shift_rows = f.shift.rows;
    c.scale = f.scale.data;
    c.scale_rows = f.scale.rows;
    c.raw = f.raw.data;
    c.rows_per_sequence = f.rows_per_sequence;
    c.source_rows = f.source_rows;
    check(qlin_layer_norm_quantize(x.data, x.rows, code(x.type), weight.data, bias.data, eps, &c,
                                   retained.data, q.values.rows, cols, q.values.data,
                                   q.scales.ptr<float>(), code(q.values.type), q.group_size,
                                   q.rotation_size, context(x.device).stream()),
          "layer norm quantize");
}

// ops/basic.cpp:54-58
void quantized_norm(TensorView input, TensorView update, TensorView weight, RowScaledView output,
                    float epsilon, bool gemma, TensorView scale) {
    launch_quantized_norm(input, update, weight, output, epsilon, gemma, scale,
                          context(input.device).stream());
}

// ops/basic.cpp:59-63
void quantized_gated(TensorView input, RowScaledView output, int kind) {
    launch_quantized_gated(input, output, kind, context(input.device).stream());
}
}  // namespace ops

}  // namespace tts
