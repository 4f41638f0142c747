// Dynamic row quantization for gfx950: per-token, H128-rotated per-token and
// K-group (optionally rotated) INT8 / OCP-FP8 encoders.
//
// Semantics follow the reference dispatch launch_row_quantize
// (ops/kernels/quant/row_quantize.cu:167-193):
//   group == 0, rotation == 0 : per-token scale      (row_quantize.cu:24-87)
//   group == 0, rotation ==128: rotated per-token    (row_quantize.cu:90-115)
//   group  > 0                : per-(row, K group)   (row_quantize.cu:145-165,
//                               quant_device.cuh:63-88), rotation optional.
// The same kernels quantize weights at load time (io/weights.cpp:80-87).
//
// Mapping: one 256-thread workgroup (four wave64s) per row for the per-token
// modes, each lane holding 8 consecutive columns per 2048-column chunk in
// registers (16-byte loads, 8-byte stores); one workgroup per (row, 2048
// columns) for the group modes. A 128-column rotation block is 16 adjacent
// lanes: three in-register butterfly stages (stride 1,2,4) then four xor
// shuffles (stride 8..64), the ascending-stride order the reference uses.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "row_encode.hpp"

namespace qlin {
namespace {

// Per-token (optionally rotated) quantization. Items > 0 keeps the row in
// registers (cols <= Items * 2048); Items == 0 streams the row twice.
template <int Fmt, class Tin, bool Rot, int Items, bool Vec>
__global__ __launch_bounds__(kThreads) void token_quantize(const uint16_t *__restrict__ x,
                                                           uint8_t *__restrict__ q,
                                                           float *__restrict__ scales, int cols,
                                                           int ld) {
    const int row = blockIdx.x;
    const uint16_t *src = x + size_t(row) * ld;
    uint8_t *dst = q + size_t(row) * cols;
    float amax = 0.f;
    if constexpr (Items > 0) {
        float v[Items][8];
#pragma unroll
        for (int it = 0; it < Items; ++it) {
            int column = (it * kThreads + threadIdx.x) * 8;
            load8<Tin, Vec>(src, column, cols, v[it]);
            if constexpr (Rot) rotate8(v[it], column);
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[it][i]));
        }
        float step = quant_scale<Fmt>(block_max(amax));
        float inverse = 1.f / step;
        if (threadIdx.x == 0) scales[row] = step;
#pragma unroll
        for (int it = 0; it < Items; ++it)
            store8<Fmt, Vec>(dst, (it * kThreads + threadIdx.x) * 8, cols, v[it], inverse);
    } else {
        const int span = (cols + kChunk - 1) / kChunk * kChunk;
        for (int column = threadIdx.x * 8; column < span; column += kChunk) {
            float v[8];
            load8<Tin, Vec>(src, column, cols, v);
            if constexpr (Rot) rotate8(v, column);
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        }
        float step = quant_scale<Fmt>(block_max(amax));
        float inverse = 1.f / step;
        if (threadIdx.x == 0) scales[row] = step;
        for (int column = threadIdx.x * 8; column < span; column += kChunk) {
            float v[8];
            load8<Tin, Vec>(src, column, cols, v);
            if constexpr (Rot) rotate8(v, column);
            store8<Fmt, Vec>(dst, column, cols, v, inverse);
        }
    }
}

// Per-token (optionally rotated) quantization of rows up to 8192 columns by
// NT threads (NT / 64 waves, NT * 8 >= cols), one 8-column piece per lane:
// the row's loads are spread over as many waves as it has 512-column pieces,
// which shortens the load latency a decode row waits for. Same arithmetic as
// token_quantize (block absmax, order-free).
template <int Fmt, class Tin, bool Rot, bool Vec, int NT>
__global__ __launch_bounds__(NT) void token_quantize_wide(const uint16_t *__restrict__ x,
                                                          uint8_t *__restrict__ q,
                                                          float *__restrict__ scales, int cols,
                                                          int ld) {
    const int row = blockIdx.x;
    const int column = threadIdx.x * 8;
    float v[8];
    load8<Tin, Vec>(x + size_t(row) * ld, column, cols, v);
    if constexpr (Rot) rotate8(v, column);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    const float step = quant_scale<Fmt>(block_max<NT>(amax));
    if (threadIdx.x == 0) scales[row] = step;
    store8<Fmt, Vec>(q + size_t(row) * cols, column, cols, v, 1.f / step);
}

// Per-(row, K group) quantization, scales stored [ceil(cols/G), rows].
template <int Fmt, class Tin, bool Rot, int G, bool Vec>
__global__ __launch_bounds__(kThreads) void group_quantize(const uint16_t *__restrict__ x,
                                                           uint8_t *__restrict__ q,
                                                           float *__restrict__ scales, int rows,
                                                           int cols, int ld, int tiles) {
    const int row = blockIdx.x / tiles, tile = blockIdx.x % tiles;
    const int column = (tile * kThreads + threadIdx.x) * 8;
    float v[8];
    load8<Tin, Vec>(x + size_t(row) * ld, column, cols, v);
    if constexpr (Rot) rotate8(v, column);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = group_max<G / 8>(amax);
    float step = quant_scale<Fmt>(amax);
    if (column < cols && (column % G) == 0) scales[size_t(column / G) * rows + row] = step;
    store8<Fmt, Vec>(q + size_t(row) * cols, column, cols, v, 1.f / step);
}

template <int Fmt, class Tin, bool Vec>
void launch_group(const RowQuantizeArgs &a, hipStream_t stream) {
    const int tiles = (a.cols + kChunk - 1) / kChunk;
    dim3 grid(unsigned(size_t(a.rows) * tiles));
    auto *x = static_cast<const uint16_t *>(a.src);
    auto *q = static_cast<uint8_t *>(a.values);
#define QLIN_GROUP(R, G)                                                                       \
    hipLaunchKernelGGL((group_quantize<Fmt, Tin, R, G, Vec>), grid, dim3(kThreads), 0, stream, \
                       x, q, a.scales, a.rows, a.cols, a.ld, tiles)
    if (a.rotation) {
        if (a.group == 32) QLIN_GROUP(true, 32);
        else if (a.group == 64) QLIN_GROUP(true, 64);
        else QLIN_GROUP(true, 128);
    } else {
        if (a.group == 32) QLIN_GROUP(false, 32);
        else if (a.group == 64) QLIN_GROUP(false, 64);
        else QLIN_GROUP(false, 128);
    }
#undef QLIN_GROUP
}

template <int Fmt, class Tin, bool Rot, bool Vec>
void launch_token(const RowQuantizeArgs &a, hipStream_t stream) {
    const int items = (a.cols + kChunk - 1) / kChunk;
    auto *x = static_cast<const uint16_t *>(a.src);
    auto *q = static_cast<uint8_t *>(a.values);
    // Decode-sized row counts of 2049..8192 columns: one 8-column piece per
    // lane, 512..1024 threads (M = 32, K = 6144: 2.37 us against 2.69 us
    // with 256 threads of three pieces). Many rows keep the 256-thread form,
    // whose workgroups pack more rows per CU (M = 4096, K = 6144: 15.7 us
    // against 17.7 us).
    const int pieces = (a.cols + 511) / 512;  // 512-column pieces = waves
    if (pieces > 4 && pieces <= 16 && a.rows <= 512) {
#define QLIN_TOKEN_WIDE(NT)                                                                  \
    hipLaunchKernelGGL((token_quantize_wide<Fmt, Tin, Rot, Vec, NT>), dim3(a.rows), dim3(NT), 0, \
                       stream, x, q, a.scales, a.cols, a.ld)
        if (pieces <= 8) QLIN_TOKEN_WIDE(512);
        else if (pieces <= 12) QLIN_TOKEN_WIDE(768);
        else QLIN_TOKEN_WIDE(1024);
#undef QLIN_TOKEN_WIDE
        return;
    }
#define QLIN_TOKEN(I)                                                                          \
    hipLaunchKernelGGL((token_quantize<Fmt, Tin, Rot, I, Vec>), dim3(a.rows), dim3(kThreads), \
                       0, stream, x, q, a.scales, a.cols, a.ld)
    switch (items) {
    case 1: QLIN_TOKEN(1); break;
    case 2: QLIN_TOKEN(2); break;
    case 3: QLIN_TOKEN(3); break;
    case 4: QLIN_TOKEN(4); break;
    case 5: case 6: QLIN_TOKEN(6); break;
    case 7: case 8: QLIN_TOKEN(8); break;
    default: QLIN_TOKEN(0); break;
    }
#undef QLIN_TOKEN
}

template <int Fmt, class Tin, bool Vec>
void launch_fmt_in(const RowQuantizeArgs &a, hipStream_t stream) {
    if (a.group) launch_group<Fmt, Tin, Vec>(a, stream);
    else if (a.rotation) launch_token<Fmt, Tin, true, Vec>(a, stream);
    else launch_token<Fmt, Tin, false, Vec>(a, stream);
}

template <int Fmt>
void launch_fmt(const RowQuantizeArgs &a, bool vec, hipStream_t stream) {
    if (a.src_type == F16) {
        if (vec) launch_fmt_in<Fmt, f16_t, true>(a, stream);
        else launch_fmt_in<Fmt, f16_t, false>(a, stream);
    } else {
        if (vec) launch_fmt_in<Fmt, bf16_t, true>(a, stream);
        else launch_fmt_in<Fmt, bf16_t, false>(a, stream);
    }
}

}  // namespace

void launch_row_quantize(const RowQuantizeArgs &a, hipStream_t stream) {
    // 16-byte source loads and 8-byte code stores need 8-column alignment of
    // every row start; anything else takes the element-wise variant.
    bool vec = a.cols % 8 == 0 && a.ld % 8 == 0 &&
               reinterpret_cast<uintptr_t>(a.src) % 16 == 0 &&
               reinterpret_cast<uintptr_t>(a.values) % 8 == 0;
    if (a.fmt == I8) launch_fmt<I8>(a, vec, stream);
    else launch_fmt<FP8>(a, vec, stream);
}

}  // namespace qlin
