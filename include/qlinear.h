/*
 * qlinear.h — C ABI of the MI355X (gfx950) quantized linear library
 * (libqlinear.so). Plain pointers and sizes only; every entry point returns
 * an int status (0 = success, negative = error, message via
 * qlin_last_error()) and never throws.
 *
 * It replaces, one for one, the kernel-launcher layer of TTS.cpp's quantized
 * linear path (paths relative to the reference's src/):
 *   qlin_row_quantize   <- launch_row_quantize     ops/kernels/quant/row_quantize.h:6
 *                          (validation of ops::quantize_rows, ops/basic.cpp:69-78)
 *   qlin_gemm           <- launch_quant_linear     ops/kernels/quant/quant_dispatch.h:11-15
 *                          and grouped_quant_gemm  ops/kernels/quant/quant_dispatch.h:7-10
 *   qlin_plan           <- select_linear / KernelSelector
 *                          ops/cuda/quantization_policy.cpp:269-286, ops/cuda/quantization.cpp:27-64
 *   qlin_workspace_bytes   (the split-K bound checks of quant_gemm_sm80.cu:45-46,
 *                          quant_grouped.cu:232-233, made queryable)
 *   qlin_linear         <- the quantized branch of ops::linear  ops/linear.cpp:51-71
 *                          (quantize_rows into scratch, then QuantizedGemm::linear)
 *   qlin_quantized_norm <- launch_quantized_norm   ops/kernels/quant/quant_norm.h:5-7
 *                          (ops::quantized_norm, ops/basic.h:33-34, ops/basic.cpp:54-58)
 *   qlin_quantized_gated<- launch_quantized_gated  ops/kernels/quant/quant_gated.h:7-8
 *                          (ops::quantized_gated, ops/basic.h:35, ops/basic.cpp:59-63)
 *   qlin_norm_linear    <- normalized_quantized_linear ops/kernels/sequence/norm_projection.h:15
 *                          (QuantizedGemm::normalized_linear, ops/cuda/quantization.cpp:479-494)
 *   qlin_gemm_finish    <- QuantizedGemm::linear_finish  ops/cuda/quantization.cpp:465-478
 *                          (bias + ReLU / tanh-GeLU finish of ops::linear, ops/linear.cpp:71-93)
 *   qlin_pack_weights, qlin_packed_weight_bytes, qlin_gemm_packed, qlin_linear_packed
 *                       <- no launcher of the reference: the packed weight layout that
 *                          follows its load-time quantization (io/weights.cpp:80-87);
 *                          qlin_gemm / qlin_linear on that layout
 *   qlin_linear_noalloc, qlin_noalloc_scratch_bytes
 *                       <- no counterpart in the reference: qlin_linear with its
 *                          scratch in a fixed library-owned device array, for callers
 *                          that cannot allocate
 *
 * Operand layouts (reference core/quantization.h:24-49):
 *   x  int8/e4m3 [rows, K] dense          sx f32 [rows] or [ceil(K/ig), rows]
 *   w  int8/e4m3 [N, K]   dense (K fast)  sw f32 [N]    or [ceil(K/wg), N]
 *   y  bf16/f16  [rows, N] dense
 * All device pointers; the library never allocates, copies or repacks.
 * Launches are asynchronous on `stream` and graph-capturable.
 */
#ifndef QLINEAR_H
#define QLINEAR_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t; declared here so that bindings need no HIP headers. */
typedef struct ihipStream_t *qlin_stream_t;

/* Storage codes, numerically equal to tts::Type (reference core/tensor.h:8). */
enum {
    QLIN_BF16 = 0,
    QLIN_F32 = 1,
    QLIN_I32 = 2,
    QLIN_FP8 = 3, /* OCP e4m3fn */
    QLIN_I8 = 4,
    QLIN_F16 = 5
};

/* Status codes. */
enum {
    QLIN_OK = 0,
    QLIN_ERR_INVALID = -1,     /* shape/type/null pointer (reference: std::invalid_argument) */
    QLIN_ERR_ALIGNMENT = -2,   /* pointer alignment the kernels require */
    QLIN_ERR_WORKSPACE = -3,   /* workspace absent or too small */
    QLIN_ERR_UNSUPPORTED = -4, /* valid request without a kernel variant (e.g. path params) */
    QLIN_ERR_HIP = -5          /* HIP runtime error at launch */
};

/* Kernel families (qlin_path.kind). */
enum {
    QLIN_KIND_AUTO = 0,   /* qlin_gemm plans itself */
    QLIN_KIND_SKINNY = 1, /* decode regime: weight-streaming MFMA GEMM, tokens <= 64 per tile */
    QLIN_KIND_TILED = 2   /* prefill regime: LDS-tiled MFMA GEMM */
};

/* Execution path of one GEMM shape class; mirrors tts::LinearPath
 * (reference ops/kernels/quant/kernel_config.h:5-9). */
typedef struct qlin_path {
    int kind;     /* QLIN_KIND_* */
    int tokens;   /* token (M) tile */
    int channels; /* output-channel (N) tile */
    int splits;   /* grid-level K partitions (partials in workspace when > 1) */
    int waves;    /* skinny: 8 (wave64s splitting K inside a workgroup);
                     tiled: 1, 2, 4 or 8 (the macro tile's wave layout) */
    int staged;   /* skinny: 1 = each wave's weight slab staged global->LDS
                     in one shot, 0 = weights loaded straight to registers;
                     tiled: 0 */
} qlin_path;

/* Library version (major*10000 + minor*100 + patch). */
int qlin_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *qlin_last_error(void);

/* Quantize rows of a bf16/f16 matrix (row stride `ld` elements) into
 * int8/e4m3 values and f32 scales.
 *   group    0 (per-token scale, scales [rows]) or 32/64/128 (scales
 *            [ceil(cols/group), rows], rows contiguous)
 *   rotation 0 or 128 (normalized Walsh-Hadamard H128 with the reference's
 *            Rademacher signs; cols % 128 == 0)
 * Used for activations per call and for weights once at load. */
int qlin_row_quantize(const void *src, int ld, int rows, int cols, int src_type, void *values,
                      float *scales, int fmt, int group, int rotation, qlin_stream_t stream);

/* Choose a path for a shape (host only, no device calls). */
int qlin_plan(int rows, int N, int K, int fmt, int input_group, int weight_group,
              qlin_path *path);

/* Workspace bytes `path` needs for this shape (0 when none). */
size_t qlin_workspace_bytes(const qlin_path *path, int rows, int N, int K, int fmt,
                            int input_group, int weight_group);

/* y = D(dequant(x . w^T)). `path` may be NULL (planned internally, same as
 * qlin_plan). input_group / weight_group: 0 = per-row scales, 32 / 64 / 128 =
 * K-group scales (group_int8 / group_fp8 use 128); partials are taken per the
 * smaller of the two group sizes (reference quant_grouped.cu:185-202). Groups
 * of 32 / 64 run on the skinny path up to 64 rows and on eight-wave tiled
 * paths above (INT8 256x128 or 128x128, FP8 128x128); split-K and
 * packed-weight paths return QLIN_ERR_UNSUPPORTED for them. Shape rules of the reference make_plan
 * (ops/cuda/quantization.cpp:210-222): K % 16 == 0, N % 16 == 0, and for
 * INT8 K <= 131071. */
int qlin_gemm(const qlin_path *path, const void *x, const float *sx, const void *w,
              const float *sw, void *y, int rows, int N, int K, int fmt, int out_type,
              int input_group, int weight_group, void *workspace, size_t workspace_bytes,
              qlin_stream_t stream);

/* Quantized branch of the reference ops::linear (ops/linear.cpp:51-71): the
 * 16-bit activations x [rows, ld] are quantized with (fmt, input_group,
 * rotation) into the scratch activation (xq [rows, K], sx), as
 * qlin_row_quantize, then y = D(xq . w^T) as qlin_gemm with `path` (NULL =
 * planned). Two launches on `stream` (quantizer, GEMM), or one where the
 * path is an INT8 or FP8 decode path with 16-token tiles, per-wave weight slabs, one
 * 256-column block of K per wave (K <= 2048) and at most 256 workgroups, with
 * per-token scales or activation groups of 128 (weight groups of 128 or per
 * channel), no rotation and a 16-byte-aligned source with ld % 8 == 0, and
 * neither y nor (xq, sx) overlaps x: there the GEMM quantizes its own token
 * rows and fills (xq, sx) with the same bits. The first failing
 * check's status is returned. */
int qlin_linear(const qlin_path *path, const void *x, int ld, int src_type, void *xq, float *sx,
                const void *w, const float *sw, void *y, int rows, int N, int K, int fmt,
                int out_type, int input_group, int weight_group, int rotation, void *workspace,
                size_t workspace_bytes, qlin_stream_t stream);

/* Residual update + RMSNorm + row quantization in one pass (the reference's
 * quantized_norm producer, ops/kernels/quant/quant_norm.cu:14-123,166-188):
 *   if update:  residual[r,c] = s16(residual[r,c] + s16(update[r,c] * update_scale[c]))
 *               (update_scale optional), stored back into `residual`;
 *   n[r,c] = gemma ? s16((v*inv) * (weight[c] + 1)) : s16(s16(v*inv) * weight[c]),
 *               inv = 1/sqrt(mean_c(v^2) + eps);
 *   then n is quantized as qlin_row_quantize (fmt, group, rotation).
 * s16 = round to the 16-bit src_type. Dense rows, 1 <= cols <= 2048; residual,
 * update, update_scale and weight share src_type (BF16 or F16). */
int qlin_quantized_norm(void *residual, const void *update, const void *update_scale,
                        const void *weight, int src_type, int rows, int cols, float eps, int gemma,
                        void *values, float *scales, int fmt, int group, int rotation,
                        qlin_stream_t stream);

/* Gated activation + row quantization (the reference's quantized_gated
 * producer, ops/kernels/quant/quant_gated.cu:18-85,179-198): input is
 * [rows, 2*width] with the gate in columns [0, width) and up in [width, 2*width);
 *   a[r,c] = s16(s16(act(gate[r,c])) * up[r,c]),  act = SiLU (kind 0) or
 *   tanh-GeLU (kind 1), then a is quantized as qlin_row_quantize.
 * Dense rows, 1 <= width <= 8192. */
int qlin_quantized_gated(const void *input, int src_type, int rows, int width, int kind,
                         void *values, float *scales, int fmt, int group, int rotation,
                         qlin_stream_t stream);

/* Finish activations of the quantized GEMM (the ops::Activation subset of the
 * reference's quantized finish; qlin_norm_linear accepts NONE and RELU). */
enum { QLIN_FINISH_NONE = 0, QLIN_FINISH_RELU = 1, QLIN_FINISH_GELU_TANH = 2 };

/* qlin_gemm followed, in the same epilogue, by the reference's finish on the
 * stored result d: y = s16(act(s16(s16(d) + bias[n]))) (bias optional, in the
 * output type; act none / ReLU / tanh-GeLU; s16 = rounding to the output type).
 * `packed` = 1 when w is in the packed layout. */
int qlin_gemm_finish(const qlin_path *path, const void *x, const float *sx, const void *w,
                     const float *sw, const void *bias, int activation, void *y, int rows, int N,
                     int K, int fmt, int out_type, int input_group, int weight_group, int packed,
                     void *workspace, size_t workspace_bytes, qlin_stream_t stream);

/* Packed weight layout (for weights quantized once at load): tile (g, t) =
 * rows [16g, 16g+16) x K bytes [64t, 64t+64) is 1 KB at offset
 * (g*ceil(K/64) + t)*1024; inside it, 16-byte chunk 16q + r holds row 16g+r,
 * K bytes [64t + 16q, +16). Bytes past K are zero. N % 16 == 0.
 * qlin_packed_weight_bytes returns N * ceil(K/64)*64 (0 for an invalid shape). */
size_t qlin_packed_weight_bytes(int N, int K);
int qlin_pack_weights(const void *w, int N, int K, void *packed, qlin_stream_t stream);

/* qlin_gemm / qlin_linear with w in the packed layout (same scales, same
 * results bit for bit). Decode paths stream the packed tiles straight into
 * MFMA registers (no LDS staging; path.staged and path.splits > 1 are not
 * supported); prefill paths stage them through LDS like row-major weights. */
int qlin_gemm_packed(const qlin_path *path, const void *x, const float *sx, const void *w,
                     const float *sw, void *y, int rows, int N, int K, int fmt, int out_type,
                     int input_group, int weight_group, void *workspace, size_t workspace_bytes,
                     qlin_stream_t stream);
int qlin_linear_packed(const qlin_path *path, const void *x, int ld, int src_type, void *xq,
                       float *sx, const void *w, const float *sw, void *y, int rows, int N, int K,
                       int fmt, int out_type, int input_group, int weight_group, int rotation,
                       void *workspace, size_t workspace_bytes, qlin_stream_t stream);

/* Input fusions of a LayerNorm (the reference's ops::NormFusion,
 * src/ops/sequence.h:55-59; arithmetic of NormRow, sequence_norm.cu:40-53).
 * All tensors are dense, in the input's 16-bit type:
 *   v = s16(s16(s16(x + projection_bias) * gate) + residual)   (each optional)
 *   u = s16(s16(s16((v - mean) * inv * weight + bias) * s16(1 + scale)) + shift)
 * with (v - mean) * inv and * weight rounded separately to fp32.
 *   residual        [x_rows, cols]; projection_bias [cols]
 *   gate/shift/scale [1 or rows / rows_per_sequence, cols] (1 = broadcast),
 *                   indexed by the source row's sequence
 *   raw             [rows, cols] receives v, or NULL
 *   source_rows     output row r normalizes input row source_rows[r]; a
 *                   source outside [0, x_rows) gives NaN outputs and unit
 *                   scales (qlin_layer_norm_quantize only; excludes gate,
 *                   shift and scale) */
typedef struct qlin_norm_fusion {
    const void *residual;
    const void *projection_bias;
    const void *gate;
    const void *shift;
    const void *scale;
    int gate_rows, shift_rows, scale_rows;
    void *raw;
    int rows_per_sequence;
    const int *source_rows;
} qlin_norm_fusion;

/* Activations of the reference's ops::Activation (src/ops/activation.h:4),
 * same numbering. */
enum {
    QLIN_ACT_IDENTITY = 0,
    QLIN_ACT_RELU = 1,
    QLIN_ACT_LEAKY_RELU = 2,
    QLIN_ACT_SILU = 3,
    QLIN_ACT_GELU = 4,
    QLIN_ACT_GELU_TANH = 5,
    QLIN_ACT_MISH = 6,
    QLIN_ACT_TANH = 7,
    QLIN_ACT_SIGMOID = 8
};

/* The reference's dense pointwise epilogue (ops::Epilogue, src/ops/sequence.h:
 * 8-27, without the packed/indirect addressing; arithmetic of Finish::apply,
 * ops/kernels/sequence/sequence_internal.cuh:52-74). Per element of output
 * row r, sequence b = r / rows_per_sequence:
 *   masked (valid_rows_per_sequence > 0 and r % rows_per_sequence >=
 *   valid_rows_per_sequence): raw = 0, result 0; otherwise
 *   v = s16(x + bias);  v = s16(v * gate[b])              (gate optional)
 *   v = s16(fma(value_scale, v, residual_scale * skip))    skip = residual row
 *       residual_index[r] (or r), 0 when absent or negative, NaN past the end
 *   v = s16(v + condition[b]);  raw = v;                   (both optional)
 *   result = s16(act(s16(v * output_scale), alpha)).
 * x row r reads input row r / input_repeat (row 0 when x_rows == 1). gate and
 * condition have 1 (broadcast) or rows / rows_per_sequence rows. All 16-bit
 * tensors are dense, in the input's type. */
typedef struct qlin_epilogue {
    const void *bias;
    const void *residual;
    int residual_rows;
    const int *residual_index;
    float value_scale, output_scale, residual_scale;
    int activation;
    float alpha;
    void *raw;
    const void *gate;
    int gate_rows;
    const void *condition;
    int condition_rows;
    int rows_per_sequence, valid_rows_per_sequence, input_repeat;
} qlin_epilogue;

/* The reference's defaults: no tensors, scales 1, identity, alpha 0.1,
 * rows_per_sequence 1, input_repeat 1. */
void qlin_norm_fusion_init(qlin_norm_fusion *fusion);
void qlin_epilogue_init(qlin_epilogue *epilogue);

/* LayerNorm -> per-token quantization -> quantized GEMV in one launch, for
 * hidden sizes k <= 512 (the reference's normalized_quantized_linear,
 * ops/kernels/sequence/sequence_norm.cu:216-390,518-575, chosen by
 * QuantizedGemm::normalized_linear, ops/cuda/quantization.cpp:479-494):
 *   u = LayerNorm of the fused input (qlin_norm_fusion; fusion may be NULL;
 *       source_rows is not accepted)
 *   u quantized per token (fmt); optionally written to `normalized` (16-bit)
 *   and `encoded` / `encoded_scales` (codes and per-token scales);
 *   y[r, c] = s16(act(s16(s16((acc * sw[c]) * sx[r]) + bias[c]))), act none or ReLU.
 * w: int8/e4m3 [n, k] with per-channel scales sw; k % 4 == 0. */
int qlin_norm_linear(const void *x, const qlin_norm_fusion *fusion, const void *norm_weight,
                     const void *norm_bias, int src_type, int rows, int k, float eps,
                     const void *w, const float *sw, int fmt, int n, const void *bias,
                     int activation, void *y, void *normalized, void *encoded,
                     float *encoded_scales, qlin_stream_t stream);

/* LayerNorm -> row quantization (the reference's layer_norm_quantize,
 * ops/kernels/sequence/sequence_norm.cu:65-200,412-440): u as above for each
 * of `rows` output rows (x has x_rows rows; x_rows == rows unless
 * fusion->source_rows is given), optionally stored to `retained` [rows, cols],
 * then quantized as qlin_row_quantize (per token, or K groups with optional
 * H128 rotation; rotation requires a group). cols >= 1; rows longer than
 * 16384 columns are streamed (re-read per pass) instead of held on chip. */
int qlin_layer_norm_quantize(const void *x, int x_rows, int src_type, const void *norm_weight,
                             const void *norm_bias, float eps, const qlin_norm_fusion *fusion,
                             void *retained, int rows, int cols, void *values, float *scales,
                             int fmt, int group, int rotation, qlin_stream_t stream);

/* Pointwise epilogue -> row quantization (the reference's pointwise_quantize,
 * ops/kernels/sequence/sequence_pointwise.cu:149-260,325-357, used by
 * ops::linear to emit the next layer's quantized input, ops/linear.cpp:71-78):
 * the qlin_epilogue result of each element of x (x_rows * input_repeat ==
 * rows), optionally stored to `retained` [rows, cols], quantized as
 * qlin_row_quantize (rotation requires a group). epilogue may be NULL
 * (identity). cols >= 1; rows longer than 16384 columns are streamed. */
int qlin_pointwise_quantize(const void *x, int x_rows, int src_type,
                            const qlin_epilogue *epilogue, void *retained, int rows, int cols,
                            void *values, float *scales, int fmt, int group, int rotation,
                            qlin_stream_t stream);

/* Dense pointwise epilogue (the reference's ops::pointwise,
 * ops/kernels/sequence/sequence_pointwise.cu:281-287, ops/sequence.h:34),
 * which ops::linear applies to a dense output after the GEMM when the
 * epilogue is not a fused finish (ops/linear.cpp:79-82): y[r, :] = the
 * qlin_epilogue result of x's rows, as the rows qlin_pointwise_quantize
 * retains. y may be x (input_repeat 1). */
int qlin_pointwise(const void *x, int x_rows, int src_type, const qlin_epilogue *epilogue,
                   void *y, int rows, int cols, qlin_stream_t stream);

/* Allocation-free quantized linear. No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments and results
 * as qlin_linear (bit for bit), minus the scratch arguments: the activation
 * codes, scales and split-K partials live in a fixed device array of
 * QLIN_NOALLOC_SCRATCH_BYTES per GPU, held by the library until the process
 * ends. Needs rows*K + 4*rows*ceil(K/input_group or K) + partials (each
 * rounded up to 256 bytes) within that size, else QLIN_ERR_WORKSPACE. Calls no
 * hipMalloc/hipFree; its first call on a device looks up the array's device
 * address once. All calls on one device share the array: calls that overlap
 * in time on one device (two streams or threads) race. */
#define QLIN_NOALLOC_SCRATCH_BYTES (32 * 1024 * 1024)
size_t qlin_noalloc_scratch_bytes(void);
int qlin_linear_noalloc(const qlin_path *path, const void *x, int ld, int src_type,
                        const void *w, const float *sw, void *y, int rows, int N, int K, int fmt,
                        int out_type, int input_group, int weight_group, int rotation,
                        qlin_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QLINEAR_H */
