// Fused quantizing producers for gfx950: the kernels that write the quantized
// activation of the next projection directly, without a 16-bit round trip
// through HBM.
//
//   residual_rms_quantize: optional residual update x += u (* s), RMSNorm
//     (plain or Gemma weight+1) in 16-bit storage precision, then row
//     quantization (reference launch_quantized_norm,
//     ops/kernels/quant/quant_norm.cu:14-123,166-188; cols <= 2048).
//   gated_quantize: act(gate) * up of a [rows, 2*width] gate|up matrix,
//     act = SiLU (kind 0) or tanh-GeLU (kind 1), then row quantization
//     (reference launch_quantized_gated, quant_gated.cu:18-85,179-198;
//     width <= 8192).
//
// Both hand the normalized / activated 16-bit row, held in registers, to the
// same row encoder as the row quantizer (per token, H128-rotated, K groups).
//
// Arithmetic contract (every TU builds with -ffp-contract=off):
//  - 16-bit pair arithmetic (the reference's __hadd2 / __hmul2 and packing)
//    is the fp32 result rounded to the storage type, to nearest even; for
//    bf16/f16 operands that equals the singly rounded 16-bit operation.
//  - The squared sum follows the reference's order: lane t of 256 sums its 8
//    columns as sum += x0*x0 + x1*x1 pairwise, a 32-lane shuffle-down tree
//    (strides 16..1) reduces each 32-lane group, and the 8 group partials are
//    added in order. The mean is total / cols (IEEE).
//  - 1/sqrt(mean + eps) is the correctly rounded fp32 value (evaluated in
//    fp64); the reference's rsqrtf is an approximation within 2 ulp of it.
//  - SiLU is (x*2^-16) / ((1 + e^-x) * 2^-16) and tanh-GeLU is
//    (0.5x)(1 + tanh(0.7978845608028654 (x + ((0.044715x)x)x))) in fp32, with
//    e^-x and tanh by this library's fp32 qexp / qtanh (within 1 and 2 ulp;
//    the reference's __expf / __fdividef / tanhf approximate the same
//    values).
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "row_encode.hpp"

namespace qlin {
namespace {

// One 256-thread workgroup per row; lane t holds columns [8t, 8t+8).
// update_scale (optional) and gemma are uniform run-time choices.
template <int Fmt, class T, bool Add, bool Vec>
__global__ __launch_bounds__(kThreads) void residual_rms_quantize(
    uint16_t *__restrict__ x, const uint16_t *__restrict__ update,
    const uint16_t *__restrict__ update_scale, const uint16_t *__restrict__ weight,
    uint8_t *__restrict__ q, float *__restrict__ scales, int rows, int cols, float eps,
    int gemma, int group, int rot) {
    const int row = blockIdx.x, column = threadIdx.x * 8;
    uint16_t *xr = x + size_t(row) * cols;
    float v[1][8], w[8];
    load8<T, Vec>(xr, column, cols, v[0]);
    load8<T, Vec>(weight, column, cols, w);
    if constexpr (Add) {
        float u[8];
        load8<T, Vec>(update + size_t(row) * cols, column, cols, u);
        if (update_scale) {
            float s[8];
            load8<T, Vec>(update_scale, column, cols, s);
#pragma unroll
            for (int i = 0; i < 8; ++i) u[i] = round16<T>(u[i] * s[i]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[0][i] = round16<T>(v[0][i] + u[i]);
        store16x8<T, Vec>(xr, column, cols, v[0]);
    }
    float sum = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) sum += v[0][2 * p] * v[0][2 * p] + v[0][2 * p + 1] * v[0][2 * p + 1];
    // The 32-lane shuffle-down tree (lane i adds lane i + d, d = 16 .. 1),
    // exact in lane 0 of each group, where it is read: the lanes whose values
    // reach it are below d at step d, so their partner i ^ d is i + d and the
    // exchange runs on DPP and row swaps instead of LDS.
    sum += lane_xor<16>(sum);
    sum += lane_xor<8>(sum);
    sum += lane_xor<4>(sum);
    sum += lane_xor<2>(sum);
    sum += lane_xor<1>(sum);
    __shared__ float partial[kThreads / 32];
    if ((threadIdx.x & 31) == 0) partial[threadIdx.x / 32] = sum;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int p = 0; p < kThreads / 32; ++p) total += partial[p];
    const float inv_norm = rsqrt_rn(total / float(cols) + eps);
    if (gemma) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[0][i] = round16<T>((v[0][i] * inv_norm) * (w[i] + 1.f));
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[0][i] = round16<T>(round16<T>(v[0][i] * inv_norm) * w[i]);
    }
    encode_row<Fmt, 1, Vec>(v, q, scales, row, rows, cols, group, rot);
}

template <int Kind> __device__ __forceinline__ float activate(float x) {
    if constexpr (Kind == 0) {
        const float e = qexp(-x);
        return (x * 0x1p-16f) / ((1.f + e) * 0x1p-16f);
    } else {
        return gelu_tanh<false>(x);
    }
}

// One NT-thread workgroup per row; chunk `it` of lane t covers output
// columns (it*NT + t)*8 .. +8 (gate at that column, up at width + column).
// Few rows (decode) use NT = 256 * chunks and one chunk per lane, so the
// activation chains of a row run on more SIMDs at once.
// The activation kind is a uniform run-time choice.
template <int Fmt, class T, int Items, bool Vec, int NT = kThreads>
__global__ __launch_bounds__(NT) void gated_quantize(const uint16_t *__restrict__ input,
                                                     uint8_t *__restrict__ q,
                                                     float *__restrict__ scales, int rows,
                                                     int width, int kind, int group, int rot) {
    const int row = blockIdx.x;
    const uint16_t *gate = input + size_t(row) * width * 2, *up = gate + width;
    float v[Items][8];
#pragma unroll
    for (int it = 0; it < Items; ++it) {
        const int column = (it * NT + threadIdx.x) * 8;
        float g[8], u[8];
        load8<T, Vec>(gate, column, width, g);
        load8<T, Vec>(up, column, width, u);
        if (kind) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[it][i] = round16<T>(round16<T>(activate<1>(g[i])) * u[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[it][i] = round16<T>(round16<T>(activate<0>(g[i])) * u[i]);
        }
    }
    encode_row<Fmt, Items, Vec, NT>(v, q, scales, row, rows, width, group, rot);
}

// ---------------------------------------------------------------- launchers
template <int Fmt, class T, bool Add, bool Vec>
void launch_norm_enc(const NormQuantizeArgs &a, hipStream_t s) {
    auto *x = static_cast<uint16_t *>(a.residual);
    auto *u = static_cast<const uint16_t *>(a.update);
    auto *us = static_cast<const uint16_t *>(a.update_scale);
    auto *w = static_cast<const uint16_t *>(a.weight);
    auto *q = static_cast<uint8_t *>(a.values);
hipLaunchKernelGGL((residual_rms_quantize<Fmt, T, Add, Vec>), dim3(a.rows), dim3(kThreads), 0, s,
                       x, u, Add ? us : nullptr, w, q, a.scales, a.rows, a.cols, a.eps, a.gemma,
                       a.group, a.rotation ? 1 : 0);
}

template <int Fmt, class T, bool Vec>
void launch_norm_t(const NormQuantizeArgs &a, hipStream_t s) {
    if (a.update) launch_norm_enc<Fmt, T, true, Vec>(a, s);
    else launch_norm_enc<Fmt, T, false, Vec>(a, s);
}

template <int Fmt, class T, int Items, bool Vec, int NT = kThreads>
void launch_gated_enc(const GatedQuantizeArgs &a, hipStream_t s) {
    auto *in = static_cast<const uint16_t *>(a.input);
    auto *q = static_cast<uint8_t *>(a.values);
hipLaunchKernelGGL((gated_quantize<Fmt, T, Items, Vec, NT>), dim3(a.rows), dim3(NT), 0, s, in,
                       q, a.scales, a.rows, a.width, a.kind, a.group, a.rotation ? 1 : 0);
}

// Rows at or below this count run one 2048-column chunk per lane (NT = 256 *
// chunks): at M = 32, width 6144 that is 4.4 us against 5.3 us for three
// chunks per lane; at M = 4096 it is 3% slower.
constexpr int kSpreadRows = 512;

template <int Fmt, class T, bool Vec>
void launch_gated_items(const GatedQuantizeArgs &a, hipStream_t s) {
    const int chunks = (a.width + kChunk - 1) / kChunk;
    if (a.rows <= kSpreadRows && chunks > 1) {
        if (chunks == 2) launch_gated_enc<Fmt, T, 1, Vec, 2 * kThreads>(a, s);
        else if (chunks == 3) launch_gated_enc<Fmt, T, 1, Vec, 3 * kThreads>(a, s);
        else launch_gated_enc<Fmt, T, 1, Vec, 4 * kThreads>(a, s);
        return;
    }
    switch (chunks) {
    case 1: launch_gated_enc<Fmt, T, 1, Vec>(a, s); break;
    case 2: launch_gated_enc<Fmt, T, 2, Vec>(a, s); break;
    case 3: launch_gated_enc<Fmt, T, 3, Vec>(a, s); break;
    default: launch_gated_enc<Fmt, T, 4, Vec>(a, s); break;
    }
}

template <int Fmt, bool Vec>
void launch_norm_f(const NormQuantizeArgs &a, hipStream_t s) {
    if (a.src_type == F16) launch_norm_t<Fmt, f16_t, Vec>(a, s);
    else launch_norm_t<Fmt, bf16_t, Vec>(a, s);
}

template <int Fmt, bool Vec>
void launch_gated_f(const GatedQuantizeArgs &a, hipStream_t s) {
    if (a.src_type == F16) launch_gated_items<Fmt, f16_t, Vec>(a, s);
    else launch_gated_items<Fmt, bf16_t, Vec>(a, s);
}

bool aligned_to(const void *p, uintptr_t bytes) {
    return !p || reinterpret_cast<uintptr_t>(p) % bytes == 0;
}

}  // namespace

void launch_quantized_norm(const NormQuantizeArgs &a, hipStream_t stream) {
    // 16-byte row loads/stores and 8-byte code stores need 8-column rows.
    const bool vec = a.cols % 8 == 0 && aligned_to(a.residual, 16) && aligned_to(a.update, 16) &&
                     aligned_to(a.update_scale, 16) && aligned_to(a.weight, 16) &&
                     aligned_to(a.values, 8);
    if (a.fmt == I8) {
        if (vec) launch_norm_f<I8, true>(a, stream);
        else launch_norm_f<I8, false>(a, stream);
    } else {
        if (vec) launch_norm_f<FP8, true>(a, stream);
        else launch_norm_f<FP8, false>(a, stream);
    }
}

void launch_quantized_gated(const GatedQuantizeArgs &a, hipStream_t stream) {
    const bool vec = a.width % 8 == 0 && aligned_to(a.input, 16) && aligned_to(a.values, 8);
    if (a.fmt == I8) {
        if (vec) launch_gated_f<I8, true>(a, stream);
        else launch_gated_f<I8, false>(a, stream);
    } else {
        if (vec) launch_gated_f<FP8, true>(a, stream);
        else launch_gated_f<FP8, false>(a, stream);
    }
}

}  // namespace qlin
