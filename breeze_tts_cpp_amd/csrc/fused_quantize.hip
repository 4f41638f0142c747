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
//    e^-x and tanh evaluated in fp64 and rounded to fp32 (the reference's
//    __expf / __fdividef / tanhf are approximations of the same values).
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "row_encode.hpp"

namespace qlin {
namespace {

template <class T, bool Vec>
__device__ __forceinline__ void store16x8(uint16_t *row, int column, int cols, const float (&v)[8]) {
    if constexpr (Vec) {
        if (column < cols) {
            uint4 packed;
            packed.x = pack2(v[0], v[1], T{});
            packed.y = pack2(v[2], v[3], T{});
            packed.z = pack2(v[4], v[5], T{});
            packed.w = pack2(v[6], v[7], T{});
            *reinterpret_cast<uint4 *>(row + column) = packed;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (column + i < cols) row[column + i] = from_float(v[i], T{});
    }
}

// Correctly rounded 1/sqrt(a) in fp32.
__device__ __forceinline__ float rsqrt_rn(float a) {
    return float(1.0 / sqrt(double(a)));
}

// One 256-thread workgroup per row; lane t holds columns [8t, 8t+8).
template <int Fmt, class T, bool Add, bool Scaled, bool Gemma, bool Rot, int G, bool Vec>
__global__ __launch_bounds__(kThreads) void residual_rms_quantize(
    uint16_t *__restrict__ x, const uint16_t *__restrict__ update,
    const uint16_t *__restrict__ update_scale, const uint16_t *__restrict__ weight,
    uint8_t *__restrict__ q, float *__restrict__ scales, int rows, int cols, float eps) {
    const int row = blockIdx.x, column = threadIdx.x * 8;
    uint16_t *xr = x + size_t(row) * cols;
    float v[1][8], w[8];
    load8<T, Vec>(xr, column, cols, v[0]);
    load8<T, Vec>(weight, column, cols, w);
    if constexpr (Add) {
        float u[8];
        load8<T, Vec>(update + size_t(row) * cols, column, cols, u);
        if constexpr (Scaled) {
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
#pragma unroll
    for (int d = 16; d; d /= 2) sum += __shfl_down(sum, d, 32);
    __shared__ float partial[kThreads / 32];
    if ((threadIdx.x & 31) == 0) partial[threadIdx.x / 32] = sum;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int p = 0; p < kThreads / 32; ++p) total += partial[p];
    const float inv_norm = rsqrt_rn(total / float(cols) + eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if constexpr (Gemma) v[0][i] = round16<T>((v[0][i] * inv_norm) * (w[i] + 1.f));
        else v[0][i] = round16<T>(round16<T>(v[0][i] * inv_norm) * w[i]);
    }
    encode_row<Fmt, 1, Rot, G, Vec>(v, q, scales, row, rows, cols);
}

template <int Kind> __device__ __forceinline__ float activate(float x) {
    if constexpr (Kind == 0) {
        const float e = float(exp(-double(x)));
        return (x * 0x1p-16f) / ((1.f + e) * 0x1p-16f);
    } else {
        return gelu_tanh(x);
    }
}

// One 256-thread workgroup per row; chunk `it` of lane t covers output
// columns (it*256 + t)*8 .. +8 (gate at that column, up at width + column).
template <int Fmt, class T, int Kind, int Items, bool Rot, int G, bool Vec>
__global__ __launch_bounds__(kThreads) void gated_quantize(const uint16_t *__restrict__ input,
                                                           uint8_t *__restrict__ q,
                                                           float *__restrict__ scales, int rows,
                                                           int width) {
    const int row = blockIdx.x;
    const uint16_t *gate = input + size_t(row) * width * 2, *up = gate + width;
    float v[Items][8];
#pragma unroll
    for (int it = 0; it < Items; ++it) {
        const int column = (it * kThreads + threadIdx.x) * 8;
        float g[8], u[8];
        load8<T, Vec>(gate, column, width, g);
        load8<T, Vec>(up, column, width, u);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[it][i] = round16<T>(round16<T>(activate<Kind>(g[i])) * u[i]);
    }
    encode_row<Fmt, Items, Rot, G, Vec>(v, q, scales, row, rows, width);
}

// ---------------------------------------------------------------- launchers
template <int Fmt, class T, bool Add, bool Scaled, bool Gemma, bool Vec>
void launch_norm_enc(const NormQuantizeArgs &a, hipStream_t s) {
    auto *x = static_cast<uint16_t *>(a.residual);
    auto *u = static_cast<const uint16_t *>(a.update);
    auto *us = static_cast<const uint16_t *>(a.update_scale);
    auto *w = static_cast<const uint16_t *>(a.weight);
    auto *q = static_cast<uint8_t *>(a.values);
#define QLIN_NORM(R, G)                                                                        \
    hipLaunchKernelGGL((residual_rms_quantize<Fmt, T, Add, Scaled, Gemma, R, G, Vec>),         \
                       dim3(a.rows), dim3(kThreads), 0, s, x, u, us, w, q, a.scales, a.rows,  \
                       a.cols, a.eps)
    if (a.group == 32) { if (a.rotation) QLIN_NORM(true, 32); else QLIN_NORM(false, 32); }
    else if (a.group == 64) { if (a.rotation) QLIN_NORM(true, 64); else QLIN_NORM(false, 64); }
    else if (a.group == 128) { if (a.rotation) QLIN_NORM(true, 128); else QLIN_NORM(false, 128); }
    else if (a.rotation) QLIN_NORM(true, 0);
    else QLIN_NORM(false, 0);
#undef QLIN_NORM
}

template <int Fmt, class T, bool Vec>
void launch_norm_t(const NormQuantizeArgs &a, hipStream_t s) {
    if (!a.update) {
        if (a.gemma) launch_norm_enc<Fmt, T, false, false, true, Vec>(a, s);
        else launch_norm_enc<Fmt, T, false, false, false, Vec>(a, s);
    } else if (!a.update_scale) {
        if (a.gemma) launch_norm_enc<Fmt, T, true, false, true, Vec>(a, s);
        else launch_norm_enc<Fmt, T, true, false, false, Vec>(a, s);
    } else {
        if (a.gemma) launch_norm_enc<Fmt, T, true, true, true, Vec>(a, s);
        else launch_norm_enc<Fmt, T, true, true, false, Vec>(a, s);
    }
}

template <int Fmt, class T, int Kind, int Items, bool Vec>
void launch_gated_enc(const GatedQuantizeArgs &a, hipStream_t s) {
    auto *in = static_cast<const uint16_t *>(a.input);
    auto *q = static_cast<uint8_t *>(a.values);
#define QLIN_GATED(R, G)                                                                       \
    hipLaunchKernelGGL((gated_quantize<Fmt, T, Kind, Items, R, G, Vec>), dim3(a.rows),         \
                       dim3(kThreads), 0, s, in, q, a.scales, a.rows, a.width)
    if (a.group == 32) { if (a.rotation) QLIN_GATED(true, 32); else QLIN_GATED(false, 32); }
    else if (a.group == 64) { if (a.rotation) QLIN_GATED(true, 64); else QLIN_GATED(false, 64); }
    else if (a.group == 128) { if (a.rotation) QLIN_GATED(true, 128); else QLIN_GATED(false, 128); }
    else if (a.rotation) QLIN_GATED(true, 0);
    else QLIN_GATED(false, 0);
#undef QLIN_GATED
}

template <int Fmt, class T, int Kind, bool Vec>
void launch_gated_items(const GatedQuantizeArgs &a, hipStream_t s) {
    switch ((a.width + kChunk - 1) / kChunk) {
    case 1: launch_gated_enc<Fmt, T, Kind, 1, Vec>(a, s); break;
    case 2: launch_gated_enc<Fmt, T, Kind, 2, Vec>(a, s); break;
    case 3: launch_gated_enc<Fmt, T, Kind, 3, Vec>(a, s); break;
    default: launch_gated_enc<Fmt, T, Kind, 4, Vec>(a, s); break;
    }
}

template <int Fmt, class T, bool Vec>
void launch_gated_t(const GatedQuantizeArgs &a, hipStream_t s) {
    if (a.kind == 0) launch_gated_items<Fmt, T, 0, Vec>(a, s);
    else launch_gated_items<Fmt, T, 1, Vec>(a, s);
}

template <int Fmt, bool Vec>
void launch_norm_f(const NormQuantizeArgs &a, hipStream_t s) {
    if (a.src_type == F16) launch_norm_t<Fmt, f16_t, Vec>(a, s);
    else launch_norm_t<Fmt, bf16_t, Vec>(a, s);
}

template <int Fmt, bool Vec>
void launch_gated_f(const GatedQuantizeArgs &a, hipStream_t s) {
    if (a.src_type == F16) launch_gated_t<Fmt, f16_t, Vec>(a, s);
    else launch_gated_t<Fmt, bf16_t, Vec>(a, s);
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


// ---------------------------------------------------------------- LayerNorm -> quantized GEMV
// The reference's normalized_quantized_linear (ops/kernels/sequence/
// sequence_norm.cu:260-390, 518-575; chosen by QuantizedGemm::normalized_linear,
// ops/cuda/quantization.cpp:479-494): for small hidden sizes (k <= 512) one
// workgroup of 256 threads per (token row, 8 output channels) loads the row
// (x + projection bias, + residual, 16-bit rounding points), LayerNorms it
// (mean, variance, (v - mean) * inv, * weight, + bias), quantizes it per token
// into LDS and computes 8 channels, one per 32-lane half-wave (the reference's
// warp per channel). Thread t holds columns t and t + 256.
namespace {

// cub::BlockReduce<float, 256>::Sum with the warp-reductions algorithm
// (CUDA 13 CUB): each 32-lane group adds lane i + s into lane i for s = 1,
// 2, 4, 8, 16 (when i + s < 32), then the eight group totals are added in
// group order. Every thread returns the same total.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
    const int l32 = threadIdx.x & 31;
#pragma unroll
    for (int s = 1; s < 32; s *= 2) {
        const float o = __shfl_down(v, s, 32);
        if (l32 + s < 32) v += o;
    }
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

// Exact e4m3fn decode (OCP; 0x7f / 0xff NaN).
__device__ __forceinline__ float decode_fp8(uint32_t c) {
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float v;
    if ((c & 0x7fu) == 0x7fu) v = __builtin_nanf("");
    else if (e == 0) v = float(m) * 0x1p-9f;
    else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
    return (c & 0x80u) ? -v : v;
}

template <int Fmt, class T>
__global__ __launch_bounds__(256) void norm_project(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ residual,
    const uint16_t *__restrict__ pbias, const uint16_t *__restrict__ nw,
    const uint16_t *__restrict__ nb, int k, float eps, const uint8_t *__restrict__ w,
    const float *__restrict__ sw, int n, const uint16_t *__restrict__ bias, int act,
    uint16_t *__restrict__ y, uint16_t *__restrict__ normalized, uint8_t *__restrict__ encoded,
    float *__restrict__ encoded_scales) {
    __shared__ float red[8];
    __shared__ __attribute__((aligned(16))) uint16_t act16[512];  // FP8: decoded T values
    __shared__ __attribute__((aligned(16))) uint8_t act8[512];    // INT8: codes
    const int row = blockIdx.y, t = threadIdx.x;
    const bool first = blockIdx.x == 0;
    float v[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = t + i * 256;
        float a = 0.f;
        if (c < k) {
            a = to_float(x[size_t(row) * k + c], T{});
            a = round16<T>(a + (pbias ? to_float(pbias[c], T{}) : 0.f));
            a = round16<T>(a + (residual ? to_float(residual[size_t(row) * k + c], T{}) : 0.f));
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
            sum += d * d;
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
            r[i] = val;
            amax = fmaxf(amax, fabsf(val));
            if (first && normalized) normalized[size_t(row) * k + c] = from_float(val, T{});
        }
    }
    const float scale = quant_scale<Fmt>(block_max_256(amax, red));
    const float recip = 1.f / scale;
    if (first && t == 0 && encoded_scales) encoded_scales[row] = scale;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = t + i * 256;
        if (c < k) {
            const uint32_t q = encode<Fmt>(r[i] * recip);
            if constexpr (Fmt == I8) act8[c] = uint8_t(q);
            else act16[c] = from_float(decode_fp8(q), T{});
            if (first && encoded) encoded[size_t(row) * k + c] = uint8_t(q);
        }
    }
    __syncthreads();
    // One channel per 32-lane group: lane l covers words c = 4l + 128j.
    const int l32 = t & 31, channel = blockIdx.x * 8 + (t >> 5);
    if (channel >= n) return;
    const uint8_t *wr = w + size_t(channel) * k;
    float result;
    if constexpr (Fmt == I8) {
        int acc = 0;
        for (int c = l32 * 4; c < k; c += 128)
            acc = __builtin_amdgcn_sdot4(*reinterpret_cast<const int *>(act8 + c),
                                         *reinterpret_cast<const int *>(wr + c), acc, false);
#pragma unroll
        for (int d = 16; d; d /= 2) acc += __shfl_down(acc, d, 32);
        result = (float(acc) * sw[channel]) * scale;
    } else {
        float acc = 0.f;
        for (int c = l32 * 4; c < k; c += 128) {
            const uint32_t wq = *reinterpret_cast<const uint32_t *>(wr + c);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = __builtin_fmaf(to_float(act16[c + e], T{}), decode_fp8((wq >> (8 * e)) & 0xffu),
                                     acc);
        }
#pragma unroll
        for (int d = 16; d; d /= 2) acc += __shfl_down(acc, d, 32);
        result = (acc * sw[channel]) * scale;
    }
    if (l32 == 0) {
        float o = round16<T>(result);
        if (bias) o = round16<T>(o + to_float(bias[channel], T{}));
        if (act == FINISH_RELU) o = fmaxf(o, 0.f);
        y[size_t(row) * n + channel] = from_float(o, T{});
    }
}

}  // namespace

void launch_norm_linear(const NormLinearArgs &a, hipStream_t stream) {
    dim3 grid(unsigned((a.n + 7) / 8), unsigned(a.rows)), block(256);
#define QLIN_NL(F, T)                                                                           \
    hipLaunchKernelGGL((norm_project<F, T>), grid, block, 0, stream,                           \
                       static_cast<const uint16_t *>(a.x), static_cast<const uint16_t *>(a.residual), \
                       static_cast<const uint16_t *>(a.projection_bias),                       \
                       static_cast<const uint16_t *>(a.norm_weight),                           \
                       static_cast<const uint16_t *>(a.norm_bias), a.k, a.eps,                 \
                       static_cast<const uint8_t *>(a.w), a.sw, a.n,                           \
                       static_cast<const uint16_t *>(a.bias), a.act,                           \
                       static_cast<uint16_t *>(a.y), static_cast<uint16_t *>(a.normalized),   \
                       static_cast<uint8_t *>(a.encoded), a.encoded_scales)
    if (a.fmt == I8) { if (a.src_type == F16) QLIN_NL(I8, f16_t); else QLIN_NL(I8, bf16_t); }
    else { if (a.src_type == F16) QLIN_NL(FP8, f16_t); else QLIN_NL(FP8, bf16_t); }
#undef QLIN_NL
}

}  // namespace qlin
