// Sequence-fusion producers of the quantized linear path for gfx950: the
// kernels that turn a 16-bit activation into the next projection's quantized
// input (or, for small hidden sizes, straight into the projection output):
//
//   layer_norm_quantize: NormFusion input (projection bias, gate, residual)
//     -> LayerNorm (weight, bias, scale, shift) -> row quantization
//     (reference layer_norm_quantize, ops/kernels/sequence/sequence_norm.cu:
//     65-200,412-440).
//   pointwise_quantize: the dense pointwise epilogue (bias, gate, scaled or
//     indexed residual, condition, sequence-tail mask, output scale,
//     activation) -> row quantization (reference pointwise_quantize,
//     sequence_pointwise.cu:149-260,325-357).
//   norm_project: LayerNorm -> per-token quantization -> GEMV in one launch,
//     k <= 512 (reference normalized_quantized_linear, sequence_norm.cu:
//     216-390,518-575).
//
// One 256-thread workgroup per row. The row quantizers hold the row in
// registers in the row encoder's layout (lane t owns columns
// (it * 256 + t) * 8 .. +8) and share its encoders (per token, H128-rotated
// K groups, K groups), so their codes and scales are those of the row
// quantizer applied to the 16-bit result.
//
// Arithmetic contract (this TU builds with -ffp-contract=off; the reference's
// sequence TUs are compiled with FMA contraction, so the two places where the
// reference's source has a contractible a*b+c use an explicit fma):
//  - LayerNorm statistics in the reference's order: thread t sums the columns
//    t, t + 256, t + 512, ... in order (values staged in LDS for that), then
//    the 256 partials reduce in cub::BlockReduce order (32-lane trees with
//    strides 1..16, then the 8 group totals in order); mean = sum / cols; the
//    variance partial accumulates fma(d, d, sum); inv = the correctly rounded
//    1/sqrt(var / cols + eps) (the reference's rsqrtf is within 2 ulp).
//  - The normalization (v - mean) * inv and * weight are separate roundings
//    (__fmul_rn in the reference), then the 16-bit rounding points of NormRow.
//  - The epilogue forms value_scale * v + residual_scale * skip as
//    fma(value_scale, v, residual_scale * skip).
//  - SiLU, sigmoid, tanh and tanh-GeLU use this library's fp32 qexp / qtanh;
//    GeLU's erf and Mish's exp / log1p / tanh are evaluated in fp64 and
//    rounded once to fp32 (the reference's expf, erff, log1pf, tanhf and
//    cutlass::fast_tanh approximate the same values); tanh-GeLU's inner term
//    is fma((0.044715x)x, x, x) as the contracting TUs compile it.
#include <algorithm>

#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "row_encode.hpp"

namespace qlin {
namespace {

// cub::BlockReduce<float, 256>::Sum with the warp-reductions algorithm
// (CUDA 13 CUB): each 32-lane group adds lane i + s into lane i for s = 1,
// 2, 4, 8, 16 (when i + s < 32), then the eight group totals are added in
// group order. Every thread returns the same total. The lane exchange is
// lane ^ s (DPP and row swaps, no LDS round trip): every lane whose value
// reaches the group's lane 0 is a multiple of 2s at step s, whose partner
// i ^ s is i + s, so lane 0 adds the same operands in the same order.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
    const int l32 = threadIdx.x & 31;
    v += lane_xor<1>(v);
    v += lane_xor<2>(v);
    v += lane_xor<4>(v);
    v += lane_xor<8>(v);
    v += lane_xor<16>(v);
    if (l32 == 0) red[threadIdx.x >> 5] = v;
    __syncthreads();
    float total = red[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) total += red[w];
    __syncthreads();
    return total;
}

__device__ __forceinline__ float block_max_256(float v, float *red) {
    v = group_max<64>(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}

// A 32-lane group's shuffle-down tree (lane i adds lane i + d for d = 16,
// 8, 4, 2, 1), exact in lane 0 of the group: the lanes whose values reach
// it are below d at step d, where the partner i ^ d is i + d, so the lane
// exchange needs no LDS round trip. Other lanes hold other sums.
__device__ __forceinline__ float sum32_down(float v) {
    v += lane_xor<16>(v);
    v += lane_xor<8>(v);
    v += lane_xor<4>(v);
    v += lane_xor<2>(v);
    v += lane_xor<1>(v);
    return v;
}
__device__ __forceinline__ int sum32_down(int v) {
    v += __float_as_int(lane_xor<16>(__int_as_float(v)));
    v += __float_as_int(lane_xor<8>(__int_as_float(v)));
    v += __float_as_int(lane_xor<4>(__int_as_float(v)));
    v += __float_as_int(lane_xor<2>(__int_as_float(v)));
    v += __float_as_int(lane_xor<1>(__int_as_float(v)));
    return v;
}

// Exact e4m3fn decode (OCP; 0x7f / 0xff NaN).
__device__ __forceinline__ float decode_fp8(uint32_t c) {
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float v;
    if ((c & 0x7fu) == 0x7fu) v = __builtin_nanf("");
    else if (e == 0) v = float(m) * 0x1p-9f;
    else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
    return (c & 0x80u) ? -v : v;
}

// GeLU (erf) and Mish (ops/kernels/common/activation.cuh:13-14,17-18) in
// fp64, rounded once to fp32 at the reference's rounding points; out of line
// so the row loops keep their registers.
__device__ __noinline__ float activate_fp64(float x, int kind) {
    if (kind == QLIN_ACT_GELU)
        return (0.5f * x) * (1.f + float(erf(double(x * 0.7071067811865475f))));
    const float softplus = x > 20.f ? x : float(log1p(double(float(exp(double(x))))));
    return x * float(tanh(double(softplus)));
}

// ops::activate on 8 values; the kind is uniform, so the switch sits outside
// the element loops. SiLU, sigmoid, tanh and tanh-GeLU use qexp / qtanh.
__device__ __forceinline__ void activate8(float (&v)[8], int kind, float alpha) {
    switch (kind) {
    case QLIN_ACT_IDENTITY: break;
    case QLIN_ACT_RELU:
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = fmaxf(v[i], 0.f);
        break;
    case QLIN_ACT_LEAKY_RELU:
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = v[i] >= 0.f ? v[i] : v[i] * alpha;
        break;
    case QLIN_ACT_SILU:
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = v[i] / (1.f + qexp(-v[i]));
        break;
    case QLIN_ACT_GELU_TANH:
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = gelu_tanh<true>(v[i]);
        break;
    case QLIN_ACT_TANH:
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = qtanh(v[i]);
        break;
    case QLIN_ACT_SIGMOID:
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 1.f / (1.f + qexp(-v[i]));
        break;
    default:
        for (int i = 0; i < 8; ++i) v[i] = activate_fp64(v[i], kind);
        break;
    }
}

// Row `r` of a [rows, cols] 16-bit tensor, row 0 when it has one row
// (the reference View's broadcast), or null.
__device__ __forceinline__ const uint16_t *row_of(const void *p, int rows, int r, int cols) {
    return p ? static_cast<const uint16_t *>(p) + size_t(rows == 1 ? 0 : r) * cols : nullptr;
}

template <class T, bool Vec>
__device__ __forceinline__ void load8_or(const uint16_t *row, int column, int cols, float (&v)[8],
                                         float absent) {
    if (row) load8<T, Vec>(row, column, cols, v);
    else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = absent;
    }
}

// ---------------------------------------------------------------- LayerNorm -> quant
// The operands of one LayerNorm row (NormRow, sequence_norm.cu:29-57) and its
// two 8-column steps: the fused input (projection bias, gate, residual) and
// the normalized output (weight, bias, scale, shift), each with the
// reference's 16-bit rounding points. Columns past `cols` come out as 0.
template <class T, bool Vec> struct LayerNormRow {
    const uint16_t *xr, *pb, *gate, *res, *nw, *nb, *scale, *shift;
    uint16_t *raw;
    int cols;

    __device__ LayerNormRow(const uint16_t *x, int x_rows, const uint16_t *norm_weight,
                            const uint16_t *norm_bias, const qlin_norm_fusion &f, int row,
                            int out_row, int cols_)
        : nw(norm_weight), nb(norm_bias), cols(cols_) {
        const int sequence = row / f.rows_per_sequence;
        xr = x + size_t(row) * cols;
        pb = row_of(f.projection_bias, 1, 0, cols);
        gate = row_of(f.gate, f.gate_rows, sequence, cols);
        res = row_of(f.residual, x_rows, row, cols);
        scale = row_of(f.scale, f.scale_rows, sequence, cols);
        shift = row_of(f.shift, f.shift_rows, sequence, cols);
        raw = f.raw ? static_cast<uint16_t *>(f.raw) + size_t(out_row) * cols : nullptr;
    }

    // An absent operand adds 0 (exact; -0 becomes +0 as the reference's).
    __device__ __forceinline__ void input8(int column, float (&v)[8]) const {
        float a[8], b[8];
        load8<T, Vec>(xr, column, cols, a);
        if (pb) {
            load8<T, Vec>(pb, column, cols, b);
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = round16<T>(a[i] + b[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] += 0.f;
        }
        if (gate) {
            load8<T, Vec>(gate, column, cols, b);
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = round16<T>(a[i] * b[i]);
        }
        if (res) {
            load8<T, Vec>(res, column, cols, b);
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = round16<T>(a[i] + b[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] += 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = Vec || column + i < cols ? a[i] : 0.f;
    }

    __device__ __forceinline__ void output8(int column, float (&v)[8], float mean, float inv) const {
        float w[8], b[8];
        load8_or<T, Vec>(nw, column, cols, w, 1.f);
        load8_or<T, Vec>(nb, column, cols, b, 0.f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float u = (v[i] - mean) * inv;
            if (nw) u = u * w[i];
            v[i] = round16<T>(u + b[i]);
        }
        if (scale) {
            load8<T, Vec>(scale, column, cols, w);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = round16<T>(v[i] * round16<T>(1.f + w[i]));
        }
        if (shift) {
            load8<T, Vec>(shift, column, cols, b);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = round16<T>(v[i] + b[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] += 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = Vec || column + i < cols ? v[i] : 0.f;
    }
};

// An out-of-range source row: NaN outputs, unit scales, codes of NaN
// (norm_kernel's first branch, sequence_norm.cu:73-81).
template <int Fmt, class T, bool Vec>
__device__ void nan_row(uint16_t *retained, uint8_t *q, float *scales, int out_row, int rows,
                        int cols, int group) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_nanf("");
    for (int column = threadIdx.x * 8; column < cols; column += kChunk) {
        if (retained) store16x8<T, Vec>(retained + size_t(out_row) * cols, column, cols, v);
        store8<Fmt, Vec>(q + size_t(out_row) * cols, column, cols, v, 1.f);
    }
    const int groups = group ? (cols + group - 1) / group : 1;
    for (int g = threadIdx.x; g < groups; g += kThreads) scales[size_t(g) * rows + out_row] = 1.f;
}

// Rows of up to Items * 2048 columns, held in registers (and in LDS for the
// statistics' column order).
template <int Fmt, class T, int Items, bool Vec>
__global__ __launch_bounds__(kThreads) void layer_norm_quantize(
    const uint16_t *__restrict__ x, int x_rows, const uint16_t *__restrict__ nw,
    const uint16_t *__restrict__ nb, float eps, qlin_norm_fusion f, uint16_t *__restrict__ retained,
    int rows, int cols, uint8_t *__restrict__ q, float *__restrict__ scales, int group, int rot) {
    __shared__ float cache[Items * kChunk];
    __shared__ float red[8];
    const int out_row = blockIdx.x, t = threadIdx.x;
    const int row = f.source_rows ? f.source_rows[out_row] : out_row;
    if (row < 0 || row >= x_rows) {
        nan_row<Fmt, T, Vec>(retained, q, scales, out_row, rows, cols, group);
        return;
    }
    const LayerNormRow<T, Vec> r(x, x_rows, nw, nb, f, row, out_row, cols);
    float v[Items][8];
#pragma unroll
    for (int it = 0; it < Items; ++it) {
        const int column = (it * kThreads + t) * 8;
        if (column >= cols) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[it][i] = 0.f;
            continue;
        }
        r.input8(column, v[it]);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (Vec || column + i < cols) cache[column + i] = v[it][i];
        if (r.raw) store16x8<T, Vec>(r.raw, column, cols, v[it]);
    }
    __syncthreads();
    // Thread t's columns t, t + 256, ... in order (the reference's per-thread
    // partial), all LDS reads issued together.
    float stat[Items * 8];
#pragma unroll
    for (int j = 0; j < Items * 8; ++j) stat[j] = t + j * kThreads < cols ? cache[t + j * kThreads] : 0.f;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < Items * 8; ++j)
        if (t + j * kThreads < cols) sum += stat[j];
    const float mean = block_sum_256(sum, red) / float(cols);
    sum = 0.f;
#pragma unroll
    for (int j = 0; j < Items * 8; ++j)
        if (t + j * kThreads < cols) {
            const float d = stat[j] - mean;
            sum = __builtin_fmaf(d, d, sum);
        }
    const float inv = rsqrt_rn(block_sum_256(sum, red) / float(cols) + eps);
#pragma unroll
    for (int it = 0; it < Items; ++it) {
        const int column = (it * kThreads + t) * 8;
        if (column >= cols) continue;
        r.output8(column, v[it], mean, inv);
        if (retained) store16x8<T, Vec>(retained + size_t(out_row) * cols, column, cols, v[it]);
    }
    encode_row<Fmt, Items, Vec>(v, q, scales, out_row, rows, cols, group, rot);
}

// Rows of any length, streamed in 2048-column chunks that are re-read from
// global memory for each pass, as the reference's uncached norm_kernel loops
// re-run NormRow::load (sequence_norm.cu:93-99,113-118,156-188): the sum, the
// squared deviations, then the output; per-token scales take one more pass
// for the amax before the codes. Every pass computes the same values, in the
// same per-thread column order as the register-resident kernel. The 16-bit
// raw and retained rows are written only by the last pass, so that they may
// alias the inputs.
template <int Fmt, class T, bool Vec>
__global__ __launch_bounds__(kThreads) void layer_norm_quantize_long(
    const uint16_t *__restrict__ x, int x_rows, const uint16_t *__restrict__ nw,
    const uint16_t *__restrict__ nb, float eps, qlin_norm_fusion f, uint16_t *retained, int rows,
    int cols, uint8_t *__restrict__ q, float *__restrict__ scales, int group, int rot) {
    __shared__ float cache[kChunk];
    __shared__ float red[8];
    const int out_row = blockIdx.x, t = threadIdx.x;
    const int row = f.source_rows ? f.source_rows[out_row] : out_row;
    if (row < 0 || row >= x_rows) {
        nan_row<Fmt, T, Vec>(retained, q, scales, out_row, rows, cols, group);
        return;
    }
    const LayerNormRow<T, Vec> r(x, x_rows, nw, nb, f, row, out_row, cols);
    uint16_t *kept = retained ? retained + size_t(out_row) * cols : nullptr;
    uint8_t *dst = q + size_t(out_row) * cols;
    const int chunks = (cols + kChunk - 1) / kChunk;
    // Passes 1 and 2: the statistics, each chunk staged through LDS so that
    // thread t adds the chunk's columns t, t + 256, ... in order.
    float mean = 0.f, sum = 0.f;
    for (int pass = 0; pass < 2; ++pass) {
        sum = 0.f;
        for (int ch = 0; ch < chunks; ++ch) {
            const int column = (ch * kThreads + t) * 8;
            float v[8];
            r.input8(column, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) cache[t * 8 + i] = v[i];
            __syncthreads();
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (ch * kChunk + t + j * kThreads < cols) {
                    const float value = cache[t + j * kThreads];
                    if (pass == 0) sum += value;
                    else {
                        const float d = value - mean;
                        sum = __builtin_fmaf(d, d, sum);
                    }
                }
            }
            __syncthreads();
        }
        if (pass == 0) mean = block_sum_256(sum, red) / float(cols);
    }
    const float inv = rsqrt_rn(block_sum_256(sum, red) / float(cols) + eps);
    float inverse = 0.f;
    if (!group) {
        float amax = 0.f;
        for (int ch = 0; ch < chunks; ++ch) {
            const int column = (ch * kThreads + t) * 8;
            float v[8];
            r.input8(column, v);
            r.output8(column, v, mean, inv);
            if (rot) rotate8(v, column);
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        }
        const float step = quant_scale<Fmt>(block_max_256(amax, red));
        if (t == 0) scales[out_row] = step;
        inverse = 1.f / step;
    }
    for (int ch = 0; ch < chunks; ++ch) {
        const int column = (ch * kThreads + t) * 8;
        float v[8];
        r.input8(column, v);
        if (r.raw) store16x8<T, Vec>(r.raw, column, cols, v);
        r.output8(column, v, mean, inv);
        if (kept) store16x8<T, Vec>(kept, column, cols, v);
        if (rot) rotate8(v, column);
        if (group) encode_group8<Fmt, Vec>(v, dst, scales, out_row, rows, cols, column, group);
        else store8<Fmt, Vec>(dst, column, cols, v, inverse);
    }
}

// ---------------------------------------------------------------- pointwise -> quant
// The operands of one pointwise-epilogue row and its 8-column step
// (sequence_pointwise.cu:149-260): bias, gate, the scaled or indexed
// residual, condition, then (after the optional raw store) the output scale
// and activation, with the reference's 16-bit rounding points. Columns past
// `cols` come out as 0; a masked row is all 0.
template <class T, bool Vec> struct PointwiseRow {
    const uint16_t *xr, *bias, *gate, *cond, *res;
    uint16_t *raw;
    int cols, activation;
    float value_scale, residual_scale, output_scale, alpha;
    bool masked, skip_nan, scaled_residual, scaled_output, rounded_act;

    __device__ PointwiseRow(const uint16_t *x, int x_rows, const qlin_epilogue &e, int row,
                            int cols_)
        : cols(cols_), activation(e.activation), value_scale(e.value_scale),
          residual_scale(e.residual_scale), output_scale(e.output_scale), alpha(e.alpha) {
        masked = e.valid_rows_per_sequence && row % e.rows_per_sequence >= e.valid_rows_per_sequence;
        const int sequence = row / e.rows_per_sequence;
        xr = row_of(x, x_rows, row / e.input_repeat, cols);
        bias = row_of(e.bias, 1, 0, cols);
        gate = row_of(e.gate, e.gate_rows, sequence, cols);
        cond = row_of(e.condition, e.condition_rows, sequence, cols);
        const int r = e.residual_index ? e.residual_index[row] : row;
        skip_nan = e.residual && r >= e.residual_rows;
        res = e.residual && r >= 0 && !skip_nan ? row_of(e.residual, e.residual_rows, r, cols)
                                                : nullptr;
        raw = e.raw ? static_cast<uint16_t *>(e.raw) + size_t(row) * cols : nullptr;
        // Steps that leave a 16-bit value unchanged skip their rounding:
        // without a residual, value_scale 1 and a positive finite
        // residual_scale the residual step is v + 0 (exact; it turns -0 into
        // +0 as the reference's does); output_scale 1 multiplies exactly;
        // identity and ReLU return a 16-bit value.
        scaled_residual = res || skip_nan || e.value_scale != 1.f ||
                          !(e.residual_scale > 0.f && e.residual_scale <= 3.4e38f);
        scaled_output = e.output_scale != 1.f;
        rounded_act = e.activation != QLIN_ACT_IDENTITY && e.activation != QLIN_ACT_RELU;
    }

    // The row's 8 values at `column`; the raw row is stored when `store_raw`.
    __device__ __forceinline__ void value8(int column, float (&v)[8], bool store_raw) const {
        if (masked) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.f;
            if (store_raw && raw) store16x8<T, Vec>(raw, column, cols, v);
            return;
        }
        float a[8], b[8];
        load8<T, Vec>(xr, column, cols, a);
        if (bias) {
            load8<T, Vec>(bias, column, cols, b);
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = round16<T>(a[i] + b[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] += 0.f;
        }
        if (gate) {
            load8<T, Vec>(gate, column, cols, b);
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = round16<T>(a[i] * b[i]);
        }
        if (scaled_residual) {
            load8_or<T, Vec>(res, column, cols, b, skip_nan ? __builtin_nanf("") : 0.f);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                a[i] = round16<T>(__builtin_fmaf(value_scale, a[i], residual_scale * b[i]));
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] += 0.f;
        }
        if (cond) {
            load8<T, Vec>(cond, column, cols, b);
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = round16<T>(a[i] + b[i]);
        }
        if (store_raw && raw) store16x8<T, Vec>(raw, column, cols, a);
        if (scaled_output) {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = round16<T>(a[i] * output_scale);
        }
        activate8(a, activation, alpha);
        if (rounded_act) {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = round16<T>(a[i]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = Vec || column + i < cols ? a[i] : 0.f;
    }
};

template <int Fmt, class T, int Items, bool Vec>
__global__ __launch_bounds__(kThreads) void pointwise_quantize(
    const uint16_t *__restrict__ x, int x_rows, qlin_epilogue e, uint16_t *__restrict__ retained,
    int rows, int cols, uint8_t *__restrict__ q, float *__restrict__ scales, int group, int rot) {
    const int row = blockIdx.x, t = threadIdx.x;
    const PointwiseRow<T, Vec> r(x, x_rows, e, row, cols);
    float v[Items][8];
#pragma unroll
    for (int it = 0; it < Items; ++it) {
        const int column = (it * kThreads + t) * 8;
        if (column >= cols) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[it][i] = 0.f;
            continue;
        }
        r.value8(column, v[it], true);
        if (retained) store16x8<T, Vec>(retained + size_t(row) * cols, column, cols, v[it]);
    }
    // q == nullptr: the dense pointwise (rows only, no codes).
    if (q) encode_row<Fmt, Items, Vec>(v, q, scales, row, rows, cols, group, rot);
}

// Rows of any length in 2048-column chunks: per-token scales take an amax
// pass before the pass that writes codes, raw and retained rows (so that
// those may alias the inputs); K-group scales need the one pass only.
template <int Fmt, class T, bool Vec>
__global__ __launch_bounds__(kThreads) void pointwise_quantize_long(
    const uint16_t *__restrict__ x, int x_rows, qlin_epilogue e, uint16_t *retained, int rows,
    int cols, uint8_t *__restrict__ q, float *__restrict__ scales, int group, int rot) {
    __shared__ float red[8];
    const int row = blockIdx.x, t = threadIdx.x;
    const PointwiseRow<T, Vec> r(x, x_rows, e, row, cols);
    uint16_t *kept = retained ? retained + size_t(row) * cols : nullptr;
    const int chunks = (cols + kChunk - 1) / kChunk;
    if (!q) {
        // The dense pointwise: one pass writing the rows.
        for (int ch = 0; ch < chunks; ++ch) {
            const int column = (ch * kThreads + t) * 8;
            float v[8];
            r.value8(column, v, true);
            if (kept) store16x8<T, Vec>(kept, column, cols, v);
        }
        return;
    }
    uint8_t *dst = q + size_t(row) * cols;
    float inverse = 0.f;
    if (!group) {
        float amax = 0.f;
        for (int ch = 0; ch < chunks; ++ch) {
            const int column = (ch * kThreads + t) * 8;
            float v[8];
            r.value8(column, v, false);
            if (rot) rotate8(v, column);
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        }
        const float step = quant_scale<Fmt>(block_max_256(amax, red));
        if (t == 0) scales[row] = step;
        inverse = 1.f / step;
    }
    for (int ch = 0; ch < chunks; ++ch) {
        const int column = (ch * kThreads + t) * 8;
        float v[8];
        r.value8(column, v, true);
        if (kept) store16x8<T, Vec>(kept, column, cols, v);
        if (rot) rotate8(v, column);
        if (group) encode_group8<Fmt, Vec>(v, dst, scales, row, rows, cols, column, group);
        else store8<Fmt, Vec>(dst, column, cols, v, inverse);
    }
}

// ---------------------------------------------------------------- LayerNorm -> GEMV
// One workgroup per (token row, 8 output channels); thread t holds columns t
// and t + 256. The row is LayerNormed and quantized per token into LDS
// (INT8 codes, or FP8 codes decoded to the 16-bit type as the reference
// stages them), then each 32-lane group computes one channel: INT8 by exact
// 4-way dot products, FP8 by fp32 fma in the lane's ascending columns, then
// a 32-lane shuffle-down tree, (acc * sw) * scale, bias and ReLU.
template <int Fmt, class T>
__global__ __launch_bounds__(256) void norm_project(
    const uint16_t *__restrict__ x, qlin_norm_fusion f, const uint16_t *__restrict__ nw,
    const uint16_t *__restrict__ nb, int k, float eps, const uint8_t *__restrict__ w,
    const float *__restrict__ sw, int n, int reps, const uint16_t *__restrict__ bias, int act,
    uint16_t *__restrict__ y, uint16_t *__restrict__ normalized, uint8_t *__restrict__ encoded,
    float *__restrict__ encoded_scales) {
    __shared__ float red[8];
    __shared__ __attribute__((aligned(16))) uint16_t act16[512];  // FP8: decoded T values
    __shared__ __attribute__((aligned(16))) uint8_t act8[512];    // INT8: codes
    const int row = blockIdx.y, t = threadIdx.x;
    const bool first = blockIdx.x == 0;
    const int sequence = row / f.rows_per_sequence;
    const uint16_t *pb = row_of(f.projection_bias, 1, 0, k);
    const uint16_t *gate = row_of(f.gate, f.gate_rows, sequence, k);
    const uint16_t *res = row_of(f.residual, gridDim.y, row, k);
    const uint16_t *scale = row_of(f.scale, f.scale_rows, sequence, k);
    const uint16_t *shift = row_of(f.shift, f.shift_rows, sequence, k);
    uint16_t *raw = f.raw ? static_cast<uint16_t *>(f.raw) + size_t(row) * k : nullptr;
    float v[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = t + i * 256;
        float a = 0.f;
        if (c < k) {
            a = to_float(x[size_t(row) * k + c], T{});
            a = round16<T>(a + (pb ? to_float(pb[c], T{}) : 0.f));
            if (gate) a = round16<T>(a * to_float(gate[c], T{}));
            a = round16<T>(a + (res ? to_float(res[c], T{}) : 0.f));
            if (first && raw) raw[c] = from_float(a, T{});
        }
        v[i] = a;
    }
    float sum = 0.f;
    sum += v[0];
    sum += v[1];
    const float mean = block_sum_256(sum, red) / float(k);
    sum = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (t + i * 256 < k) {
            const float d = v[i] - mean;
            sum = __builtin_fmaf(d, d, sum);
        }
    const float inv = rsqrt_rn(block_sum_256(sum, red) / float(k) + eps);
    float r[2] = {0.f, 0.f}, amax = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = t + i * 256;
        if (c < k) {
            float val = (v[i] - mean) * inv;
            if (nw) val = val * to_float(nw[c], T{});
            val = round16<T>(val + (nb ? to_float(nb[c], T{}) : 0.f));
            if (scale) val = round16<T>(val * round16<T>(1.f + to_float(scale[c], T{})));
            val = round16<T>(val + (shift ? to_float(shift[c], T{}) : 0.f));
            r[i] = val;
            amax = fmaxf(amax, fabsf(val));
            if (first && normalized) normalized[size_t(row) * k + c] = from_float(val, T{});
        }
    }
    const float step = quant_scale<Fmt>(block_max_256(amax, red));
    const float recip = 1.f / step;
    if (first && t == 0 && encoded_scales) encoded_scales[row] = step;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = t + i * 256;
        if (c < k) {
            const uint32_t code = encode<Fmt>(r[i] * recip);
            if constexpr (Fmt == I8) act8[c] = uint8_t(code);
            else act16[c] = from_float(decode_fp8(code), T{});
            if (first && encoded) encoded[size_t(row) * k + c] = uint8_t(code);
        }
    }
    __syncthreads();
    // Channels blockIdx.x * 8 * reps + 8r + g for r < reps, one per 32-lane
    // group g at a time: lane l covers words c = 4l + 128j.
    const int l32 = t & 31;
    for (int r = 0; r < reps; ++r) {
    const int channel = (blockIdx.x * reps + r) * 8 + (t >> 5);
    if (channel >= n) return;
    const uint8_t *wr = w + size_t(channel) * k;
    float result;
    if constexpr (Fmt == I8) {
        int acc = 0;
        for (int c = l32 * 4; c < k; c += 128)
            acc = __builtin_amdgcn_sdot4(*reinterpret_cast<const int *>(act8 + c),
                                         *reinterpret_cast<const int *>(wr + c), acc, false);
        acc = sum32_down(acc);
        result = (float(acc) * sw[channel]) * step;
    } else {
        float acc = 0.f;
        for (int c = l32 * 4; c < k; c += 128) {
            const uint32_t wq = *reinterpret_cast<const uint32_t *>(wr + c);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = __builtin_fmaf(to_float(act16[c + e], T{}), decode_fp8((wq >> (8 * e)) & 0xffu),
                                     acc);
        }
        acc = sum32_down(acc);
        result = (acc * sw[channel]) * step;
    }
    if (l32 == 0) {
        float o = round16<T>(result);
        o = round16<T>(o + (bias ? to_float(bias[channel], T{}) : 0.f));
        if (act == FINISH_RELU) o = fmaxf(o, 0.f);
        y[size_t(row) * n + channel] = from_float(o, T{});
    }
    }
}

// ---------------------------------------------------------------- launchers
// The row-quantizer variants (format x 16-bit type x items per lane x
// vector access) compile in four parallel parts, one
// per (family, format): QLIN_SEQ_PART names the part's launcher,
// QLIN_SEQ_FAMILY is 0 (LayerNorm) or 1 (pointwise), QLIN_SEQ_FMT the format.
// The build without QLIN_SEQ_PART holds the dispatchers and norm_project.
#ifdef QLIN_SEQ_PART
template <int Fmt, class T, int Items, bool Vec>
void launch_one(const LayerNormQuantizeArgs &a, hipStream_t s) {
    const int rot = a.rotation ? 1 : 0;
    auto *x = static_cast<const uint16_t *>(a.x);
    auto *nw = static_cast<const uint16_t *>(a.norm_weight);
    auto *nb = static_cast<const uint16_t *>(a.norm_bias);
    auto *kept = static_cast<uint16_t *>(a.retained);
    auto *q = static_cast<uint8_t *>(a.values);
    if constexpr (Items == 0)
        hipLaunchKernelGGL((layer_norm_quantize_long<Fmt, T, Vec>), dim3(a.rows), dim3(kThreads),
                           0, s, x, a.x_rows, nw, nb, a.eps, a.f, kept, a.rows, a.cols, q,
                           a.scales, a.group, rot);
    else
        hipLaunchKernelGGL((layer_norm_quantize<Fmt, T, Items, Vec>), dim3(a.rows), dim3(kThreads),
                           0, s, x, a.x_rows, nw, nb, a.eps, a.f, kept, a.rows, a.cols, q,
                           a.scales, a.group, rot);
}

template <int Fmt, class T, int Items, bool Vec>
void launch_one(const PointwiseQuantizeArgs &a, hipStream_t s) {
    const int rot = a.rotation ? 1 : 0;
    auto *x = static_cast<const uint16_t *>(a.x);
    auto *kept = static_cast<uint16_t *>(a.retained);
    auto *q = static_cast<uint8_t *>(a.values);
    if constexpr (Items == 0)
        hipLaunchKernelGGL((pointwise_quantize_long<Fmt, T, Vec>), dim3(a.rows), dim3(kThreads), 0,
                           s, x, a.x_rows, a.e, kept, a.rows, a.cols, q, a.scales, a.group, rot);
    else
        hipLaunchKernelGGL((pointwise_quantize<Fmt, T, Items, Vec>), dim3(a.rows), dim3(kThreads),
                           0, s, x, a.x_rows, a.e, kept, a.rows, a.cols, q, a.scales, a.group, rot);
}

template <int Fmt, class T, bool Vec, class Args>
void by_items(const Args &a, hipStream_t s) {
    // Items: 1, 2 or 8 register-resident chunks of 2048 columns, or (0) the
    // streaming kernel for rows longer than 16384 columns.
    if (a.cols > 8 * kChunk) launch_one<Fmt, T, 0, Vec>(a, s);
    else if (a.cols > 2 * kChunk) launch_one<Fmt, T, 8, Vec>(a, s);
    else if (a.cols > kChunk) launch_one<Fmt, T, 2, Vec>(a, s);
    else launch_one<Fmt, T, 1, Vec>(a, s);
}
#endif

bool aligned16(const void *p) { return !p || reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

#ifdef QLIN_SEQ_PART
#if QLIN_SEQ_FAMILY == 0
using SeqArgs = LayerNormQuantizeArgs;
#else
using SeqArgs = PointwiseQuantizeArgs;
#endif
void QLIN_SEQ_PART(const SeqArgs &a, bool vec, hipStream_t s) {
    if (a.src_type == F16) {
        if (vec) by_items<QLIN_SEQ_FMT, f16_t, true>(a, s);
        else by_items<QLIN_SEQ_FMT, f16_t, false>(a, s);
    } else {
        if (vec) by_items<QLIN_SEQ_FMT, bf16_t, true>(a, s);
        else by_items<QLIN_SEQ_FMT, bf16_t, false>(a, s);
    }
}
#else
void launch_layer_norm_quantize(const LayerNormQuantizeArgs &a, hipStream_t stream) {
    const qlin_norm_fusion &f = a.f;
    const bool vec = a.cols % 8 == 0 && aligned16(a.x) && aligned16(a.norm_weight) &&
                     aligned16(a.norm_bias) && aligned16(f.residual) &&
                     aligned16(f.projection_bias) && aligned16(f.gate) && aligned16(f.shift) &&
                     aligned16(f.scale) && aligned16(f.raw) && aligned16(a.retained) &&
                     reinterpret_cast<uintptr_t>(a.values) % 8 == 0;
    if (a.fmt == I8) launch_layer_norm_quantize_i8(a, vec, stream);
    else launch_layer_norm_quantize_fp8(a, vec, stream);
}

void launch_pointwise_quantize(const PointwiseQuantizeArgs &a, hipStream_t stream) {
    const qlin_epilogue &e = a.e;
    const bool vec = a.cols % 8 == 0 && aligned16(a.x) && aligned16(e.bias) &&
                     aligned16(e.residual) && aligned16(e.gate) && aligned16(e.condition) &&
                     aligned16(e.raw) && aligned16(a.retained) &&
                     reinterpret_cast<uintptr_t>(a.values) % 8 == 0;
    if (a.fmt == I8) launch_pointwise_quantize_i8(a, vec, stream);
    else launch_pointwise_quantize_fp8(a, vec, stream);
}

// About 2048 workgroups (8 per CU): fewer, with more channels each, are
// slower (rows 32, k 512, n 2048: 10.4 us at 2048, 16.4 at 512, 28 at 256),
// because a 32-lane group's channels run one after another.
constexpr int kTargetBlocks = 2048, kMaxReps = 16;
void launch_norm_linear(const NormLinearArgs &a, hipStream_t stream) {
    // Each workgroup repeats the row's LayerNorm; give it 8 * reps channels so
    // that about kTargetBlocks workgroups cover the output.
    const int blocks8 = (a.n + 7) / 8;
    const int reps = std::max(1, std::min(kMaxReps, int((size_t(blocks8) * a.rows + kTargetBlocks - 1) / kTargetBlocks)));
    dim3 grid(unsigned((blocks8 + reps - 1) / reps), unsigned(a.rows)), block(256);
#define QLIN_NL(F, T)                                                                           \
    hipLaunchKernelGGL((norm_project<F, T>), grid, block, 0, stream,                           \
                       static_cast<const uint16_t *>(a.x), a.f,                                \
                       static_cast<const uint16_t *>(a.norm_weight),                           \
                       static_cast<const uint16_t *>(a.norm_bias), a.k, a.eps,                 \
                       static_cast<const uint8_t *>(a.w), a.sw, a.n, reps,                     \
                       static_cast<const uint16_t *>(a.bias), a.act,                           \
                       static_cast<uint16_t *>(a.y), static_cast<uint16_t *>(a.normalized),   \
                       static_cast<uint8_t *>(a.encoded), a.encoded_scales)
    if (a.fmt == I8) { if (a.src_type == F16) QLIN_NL(I8, f16_t); else QLIN_NL(I8, bf16_t); }
    else { if (a.src_type == F16) QLIN_NL(FP8, f16_t); else QLIN_NL(FP8, bf16_t); }
#undef QLIN_NL
}
#endif  // QLIN_SEQ_PART

}  // namespace qlin
