// Row encoders shared by the row quantizer and the fused quantizing producers
// (residual + RMSNorm, gated activation, LayerNorm and pointwise epilogue ->
// quant), with their 8-column load/store helpers: a 256-thread
// workgroup holds a row in registers, lane t owning the 8 columns
// (it * 256 + t) * 8 .. +8 of each 2048-column chunk `it`, and encodes it per
// token, per token after the H128 rotation, or per K group (optionally
// rotated) exactly as the reference quant_device helpers do
// (ops/kernels/quant/quant_device.cuh:63-195).
#pragma once
#include "qlin_device.hpp"

#include <type_traits>

namespace qlin {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = kThreads * 8;  // columns covered by one pass of the block

template <class Tin, bool Vec>
__device__ __forceinline__ void load8(const uint16_t *row, int column, int cols, float (&v)[8]) {
    if constexpr (Vec) {
        if (column < cols) {
            uint4 raw = *reinterpret_cast<const uint4 *>(row + column);
            uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = to_float(uint16_t(words[i] & 0xffffu), Tin{});
                v[2 * i + 1] = to_float(uint16_t(words[i] >> 16), Tin{});
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = column + i < cols ? to_float(row[column + i], Tin{}) : 0.f;
    }
}

template <int Fmt, bool Vec>
__device__ __forceinline__ void store8(uint8_t *row, int column, int cols, const float (&v)[8],
                                       float inverse) {
    uint32_t code[8];
    if constexpr (Fmt == FP8 && Vec) {
        const uint32_t lo = encode_fp8x4(v[0] * inverse, v[1] * inverse, v[2] * inverse,
                                         v[3] * inverse);
        const uint32_t hi = encode_fp8x4(v[4] * inverse, v[5] * inverse, v[6] * inverse,
                                         v[7] * inverse);
        if (column < cols) *reinterpret_cast<uint2 *>(row + column) = uint2{lo, hi};
        return;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) code[i] = encode<Fmt>(v[i] * inverse);
    }
    if constexpr (Vec) {
        if (column < cols) {
            uint2 packed;
            packed.x = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
            packed.y = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
            *reinterpret_cast<uint2 *>(row + column) = packed;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (column + i < cols) row[column + i] = uint8_t(code[i]);
    }
}

// 16-bit values of 8 columns [column, column+8) stored (rounded to T).
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

// H128 rotation of the 8 columns [column, column+8) held by this lane; the 16
// lanes sharing (lane >> 4) hold one aligned 128-column block.
__device__ __forceinline__ void rotate8(float (&v)[8], int column) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * rotation_sign(column + i);
#pragma unroll
    for (int span = 1; span < 8; span *= 2) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (!(i & span)) {
                float a = v[i], b = v[i | span];
                v[i] = a + b;
                v[i | span] = a - b;
            }
    }
    const int lane = threadIdx.x & 63;
    auto stage = [&](auto span_, auto xchg) {
        constexpr int span = decltype(span_)::value;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float other = xchg(v[i]);
            v[i] = (lane & span) ? other - v[i] : v[i] + other;
        }
    };
    stage(std::integral_constant<int, 1>{}, [](float x) { return lane_xor<1>(x); });
    stage(std::integral_constant<int, 2>{}, [](float x) { return lane_xor<2>(x); });
    stage(std::integral_constant<int, 4>{}, [](float x) { return lane_xor<4>(x); });
    stage(std::integral_constant<int, 8>{}, [](float x) { return lane_xor<8>(x); });
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] *= 0.08838834764831845f;
}

// Max over the NT threads of the workgroup.
template <int NT = kThreads> __device__ __forceinline__ float block_max(float v) {
    __shared__ float partial[NT / 64];
    v = group_max<64>(v);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = partial[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) r = fmaxf(r, partial[w]);
    return r;
}

// One lane's 8 columns [column, column+8) of a K-group encoding (group 32,
// 64 or 128, so the group spans group/8 adjacent lanes): the group's amax by
// lane shuffles, its scale written by the group's first lane, the codes.
template <int Fmt, bool Vec>
__device__ __forceinline__ void encode_group8(const float (&v)[8], uint8_t *__restrict__ dst,
                                              float *__restrict__ scales, int row, int rows,
                                              int cols, int column, int group) {
    const int lanes = group / 8;
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    if (lanes > 1) amax = fmaxf(amax, lane_xor<1>(amax));
    if (lanes > 2) amax = fmaxf(amax, lane_xor<2>(amax));
    if (lanes > 4) amax = fmaxf(amax, lane_xor<4>(amax));
    if (lanes > 8) amax = fmaxf(amax, lane_xor<8>(amax));
    const float step = quant_scale<Fmt>(amax);
    if (column < cols && (column % group) == 0) scales[size_t(column / group) * rows + row] = step;
    store8<Fmt, Vec>(dst, column, cols, v, 1.f / step);
}

// Encode a row held in registers by NT threads (v[it][i] = column
// (it*NT + t)*8 + i; columns past `cols` hold 0): optional H128 rotation
// (`rot`), then per-(row, group) scales ([ceil(cols/group), rows]) for group
// 32, 64 or 128, else (group 0) one per-token scale ([rows]). The reference's
// rotated_quantize / encode_group / token paths (quant_device.cuh:63-88,
// 145-195, row_quantize.cu:24-165). Groups and rotation blocks stay inside one
// wave for any NT (multiples of 64). `group` and `rot` are uniform across the
// workgroup, so their branches never diverge.
template <int Fmt, int Items, bool Vec, int NT = kThreads>
__device__ __forceinline__ void encode_row(float (&v)[Items][8], uint8_t *__restrict__ q,
                                           float *__restrict__ scales, int row, int rows,
                                           int cols, int group, int rot) {
    uint8_t *dst = q + size_t(row) * cols;
    if (rot) {
#pragma unroll
        for (int it = 0; it < Items; ++it) rotate8(v[it], (it * NT + threadIdx.x) * 8);
    }
    if (group) {
#pragma unroll
        for (int it = 0; it < Items; ++it)
            encode_group8<Fmt, Vec>(v[it], dst, scales, row, rows, cols,
                                    (it * NT + threadIdx.x) * 8, group);
    } else {
        float amax = 0.f;
#pragma unroll
        for (int it = 0; it < Items; ++it)
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[it][i]));
        const float step = quant_scale<Fmt>(block_max<NT>(amax));
        const float inverse = 1.f / step;
        if (threadIdx.x == 0) scales[row] = step;
#pragma unroll
        for (int it = 0; it < Items; ++it)
            store8<Fmt, Vec>(dst, (it * NT + threadIdx.x) * 8, cols, v[it], inverse);
    }
}

}  // namespace
}  // namespace qlin
