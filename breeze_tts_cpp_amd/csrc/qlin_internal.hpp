// Host-side contracts between the C-ABI layer (capi.cpp) and the kernel
// launchers (*.hip). Launchers assume arguments were validated by the caller.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/qlinear.h"

namespace qlin {

struct RowQuantizeArgs {
    const void *src;  // bf16/f16 [rows, ld]
    int src_type, ld, rows, cols;
    void *values;     // int8/e4m3 [rows, cols]
    float *scales;    // [rows] or [ceil(cols/group), rows]
    int fmt, group, rotation;
};
void launch_row_quantize(const RowQuantizeArgs &, hipStream_t);

// Fused producers (fused_quantize.hip). Dense rows; 16-bit tensors share src_type.
struct NormQuantizeArgs {
    void *residual;              // [rows, cols], updated in place when update != null
    const void *update;          // [rows, cols] or null
    const void *update_scale;    // [cols] or null
    const void *weight;          // [cols]
    int src_type, rows, cols;    // cols <= 2048
    void *values;                // int8/e4m3 [rows, cols]
    float *scales;
    int fmt, group, rotation, gemma;
    float eps;
};
void launch_quantized_norm(const NormQuantizeArgs &, hipStream_t);
struct GatedQuantizeArgs {
    const void *input;           // [rows, 2*width]: gate | up
    int src_type, rows, width;   // width <= 8192
    void *values;                // int8/e4m3 [rows, width]
    float *scales;
    int fmt, group, rotation, kind;  // kind 0 = SiLU, 1 = tanh-GeLU
};
void launch_quantized_gated(const GatedQuantizeArgs &, hipStream_t);
// Sequence-fusion producers; the fusion structs are the C ABI's, validated by
// the caller (dense rows, shapes and row counts checked).
struct NormLinearArgs {
    const void *x;                      // 16-bit [rows, k]
    qlin_norm_fusion f;                 // source_rows null
    const void *norm_weight, *norm_bias;
    int src_type, rows, k;              // k <= 512
    float eps;
    const void *w;      // int8/e4m3 [n, k]
    const float *sw;    // [n]
    int fmt, n;
    const void *bias;   // [n] or null
    int act;            // FINISH_NONE / FINISH_RELU
    void *y;            // [rows, n]
    void *normalized;   // [rows, k] or null
    void *encoded;      // [rows, k] or null
    float *encoded_scales;  // [rows] or null
};
struct LayerNormQuantizeArgs {
    const void *x;
    int x_rows, src_type;
    const void *norm_weight, *norm_bias;
    float eps;
    qlin_norm_fusion f;
    void *retained;     // [rows, cols] or null
    int rows, cols;
    void *values;
    float *scales;
    int fmt, group, rotation;
};
struct PointwiseQuantizeArgs {
    const void *x;
    int x_rows, src_type;
    qlin_epilogue e;
    void *retained;     // [rows, cols] or null
    int rows, cols;
    void *values;
    float *scales;
    int fmt, group, rotation;
};
void launch_norm_linear(const NormLinearArgs &, hipStream_t);
void launch_layer_norm_quantize(const LayerNormQuantizeArgs &, hipStream_t);
void launch_pointwise_quantize(const PointwiseQuantizeArgs &, hipStream_t);
// Per-format parts of the two row quantizers (vec: 16-byte row access).
void launch_layer_norm_quantize_i8(const LayerNormQuantizeArgs &, bool vec, hipStream_t);
void launch_layer_norm_quantize_fp8(const LayerNormQuantizeArgs &, bool vec, hipStream_t);
void launch_pointwise_quantize_i8(const PointwiseQuantizeArgs &, bool vec, hipStream_t);
void launch_pointwise_quantize_fp8(const PointwiseQuantizeArgs &, bool vec, hipStream_t);

// Kernel families; numbering is part of the C ABI (qlin_path.kind).
enum Kind : int { KIND_AUTO = 0, KIND_SKINNY = 1, KIND_TILED = 2 };

// Fused quantization of the 16-bit activation inside the decode GEMM
// (qlin_linear): the GEMM reads src [M, ld] instead of x, encodes it as the
// per-token or the 128-group (unrotated) quantizer does, and stores
// the codes and scales to xq [M, K] / sx.
struct FusedSource {
    const uint16_t *src = nullptr;
    int ld = 0, f16 = 0;
    uint8_t *xq = nullptr;
    float *sx = nullptr;  // [M], or [K/128, M] for K groups of 128
};

struct GemmArgs {
    const uint8_t *x;  // [M, K]
    const float *sx;   // [M] or [K/ig, M]
    const uint8_t *w;  // [N, K]
    const float *sw;   // [N] or [K/wg, N]
    void *y;           // [M, N] bf16/f16
    int M, N, K, fmt, out_type, input_group, weight_group;
    void *workspace;
    size_t workspace_bytes;
    int packed = 0;    // w in the packed fragment-tile layout (weight_pack.hip)
    const uint16_t *bias = nullptr;  // finish: [N] in the output type, or null
    int act = 0;                     // finish: qlin::Finish (0 = none)
    FusedSource fq{};                // src set: fused activation quantization
};
struct GemmPath {
    int kind, tokens, channels, splits, waves, staged;
};
// Skinny (decode) family: returns 0, or a negative status if the path's
// parameters are not an instantiated variant.
int launch_skinny(const GemmArgs &, const GemmPath &, hipStream_t);
// Fused-quantization decode GEMM (a.fq.src set, per-token scales, no finish):
// true when a variant exists for the path (staged per-wave slabs, 8 waves,
// no split, K a multiple of 2048, activation blocks held in registers).
bool skinny_fused_supported(const GemmArgs &, const GemmPath &);
int launch_skinny_fused(const GemmArgs &, const GemmPath &, hipStream_t);
size_t skinny_workspace_bytes(const GemmArgs &, const GemmPath &);
// LDS of a skinny launch (weight slab + cross-wave reduction buffer); a path
// above kLdsBytes must not be launched.
size_t skinny_lds_bytes(const GemmArgs &, const GemmPath &);
// K bytes per wave range of a skinny launch: ceil(ceil(K/256) / (splits*8))
// blocks of 256 (eight waves per workgroup; trailing ranges may be empty).
int skinny_span(int K, int splits);
constexpr size_t kLdsBytes = 160 * 1024;  // per workgroup on gfx950
int launch_tiled(const GemmArgs &, const GemmPath &, hipStream_t);
// Packed weight layout (weight_pack.hip): N % 16 == 0, bytes = N * ceil(K/64)*64.
size_t packed_weight_bytes(int N, int K);
void launch_pack_weights(const void *w, int N, int K, void *packed, hipStream_t);
size_t tiled_workspace_bytes(const GemmArgs &, const GemmPath &);
// Records `message` as qlin_last_error() of this thread; returns status.
int set_error(int status, const char *message);

}  // namespace qlin
