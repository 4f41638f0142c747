// Device helpers shared by the gfx950 quantized-linear kernels: 16-bit float
// conversions, INT8 / OCP e4m3fn encoders, the H128 rotation sign and wave64
// reductions. Every TU is compiled with -ffp-contract=off, so each a*b+c below
// is two roundings unless written as __builtin_fmaf.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qlin {

// Storage codes follow tts::Type (reference core/tensor.h:8).
enum Type : int { BF16 = 0, F32 = 1, I32 = 2, FP8 = 3, I8 = 4, F16 = 5 };

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- 16-bit floats
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float to_float(uint16_t h, bf16_t) {
    return __uint_as_float(uint32_t(h) << 16);
}
__device__ __forceinline__ float to_float(uint16_t h, f16_t) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return float(v);  // exact widening
}
// Round-to-nearest-even fp32 -> bf16 with quiet NaN.
__device__ __forceinline__ uint16_t from_float(float f, bf16_t) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}
// The empty asm keeps `f` a materialized fp32 value: without it the compiler
// may fold the fp32 operation producing `f` and this conversion into one
// mixed-precision instruction (v_mad_mixlo_f16) that rounds the exact result
// once, where the reference rounds to fp32 first and then to f16.
__device__ __forceinline__ uint16_t from_float(float f, f16_t) {
    asm volatile("" : "+v"(f));
    _Float16 v = (_Float16)f;  // v_cvt_f16_f32, round-to-nearest-even
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// Two values rounded to nearest even and packed low|high<<16. bf16 uses
// gfx950's v_cvt_pk_bf16_f32 (IEEE round-to-nearest-even, subnormals kept,
// NaN stays NaN): the bits of the integer rounding above for every non-NaN
// input, in one instruction per pair (the compiler emulates the conversion
// with integer operations).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
    uint32_t u;
    asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(u) : "v"(lo), "v"(hi));
    return u;
}
__device__ __forceinline__ uint32_t pack2(float lo, float hi, bf16_t) { return cvt_pk_bf16(lo, hi); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi, f16_t) {
    return uint32_t(from_float(lo, f16_t{})) | (uint32_t(from_float(hi, f16_t{})) << 16);
}

// ---------------------------------------------------------------- 8-bit encoders
// INT8: clamp to +-127, then round half to even (reference
// ops/kernels/quant/quant_format.cuh:37-47).
__device__ __forceinline__ uint32_t encode_i8(float x) {
    x = fminf(127.f, fmaxf(-127.f, x));
    return uint32_t(int(__builtin_rintf(x))) & 0xffu;
}

// Four INT8 codes, packed low to high, equal to encode_i8 of each value.
// After the same clamp, adding 1.5 * 2^23 rounds to an integer with the
// current round-to-nearest-even mode (the value rintf gives for |x| <= 127)
// and leaves that integer, two's complement, in the low mantissa byte of the
// sum; three byte permutes gather the four low bytes.
__device__ __forceinline__ uint32_t encode_i8x4(float a, float b, float c, float d) {
    constexpr float kMagic = 12582912.f;  // 1.5 * 2^23
    const uint32_t qa = __float_as_uint(fminf(127.f, fmaxf(-127.f, a)) + kMagic);
    const uint32_t qb = __float_as_uint(fminf(127.f, fmaxf(-127.f, b)) + kMagic);
    const uint32_t qc = __float_as_uint(fminf(127.f, fmaxf(-127.f, c)) + kMagic);
    const uint32_t qd = __float_as_uint(fminf(127.f, fmaxf(-127.f, d)) + kMagic);
    const uint32_t lo = __builtin_amdgcn_perm(qb, qa, 0x0c0c0400u);  // [a, b, 0, 0]
    const uint32_t hi = __builtin_amdgcn_perm(qd, qc, 0x0c0c0400u);  // [c, d, 0, 0]
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);               // [a, b, c, d]
}

// OCP e4m3fn, round-to-nearest-even, saturating to +-448 (the satfinite
// conversion of reference quant_format.cuh:12-17). Integer rounding on the
// fp32 bit pattern: exponent range [-6, 8] normal, 2^-9 subnormal step.
__device__ __forceinline__ uint32_t encode_fp8(float x) {
    uint32_t u = __float_as_uint(x);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7fu;            // NaN
    if (a >= 0x43e00000u) return sign | 0x7eu;    // >= 448 (incl. inf): max finite
    if (a < 0x3c800000u) {                        // < 2^-6: subnormal, step 2^-9
        float q = __builtin_rintf(__uint_as_float(a) * 512.f);  // exact scaling
        return sign | uint32_t(q);
    }
    uint32_t exponent = (a >> 23) - 127u + 7u;    // biased e4m3 exponent, 1..15
    uint32_t mantissa = a & 0x7fffffu;
    uint32_t kept = mantissa >> 20, rest = mantissa & 0xfffffu;
    uint32_t up = rest > 0x80000u || (rest == 0x80000u && (kept & 1u));
    return sign | ((exponent << 3) + kept + up);  // carry moves into the exponent
}

template <int Fmt> __device__ __forceinline__ uint32_t encode(float x) {
    if constexpr (Fmt == I8) return encode_i8(x);
    else return encode_fp8(x);
}

// Four e4m3 codes, packed low to high, of values of magnitude below 464:
// the hardware conversion (see encode_fp8x4).
__device__ __forceinline__ uint32_t encode_fp8x4_inrange(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}

// Four e4m3 codes, packed low to high, equal to encode_fp8 of each value.
// gfx950's v_cvt_pk_fp8_f32 (OCP e4m3fn, round to nearest even) gives
// encode_fp8's code for every fp32 of magnitude below 464, checked
// exhaustively against it (both signs, every bit pattern); at 464 and
// beyond (and for NaN) it gives NaN where encode_fp8 saturates, so those
// values take the integer encoder.
__device__ __forceinline__ uint32_t encode_fp8x4(float a, float b, float c, float d) {
    const int in = int(fabsf(a) < 464.f) & int(fabsf(b) < 464.f) & int(fabsf(c) < 464.f) &
                   int(fabsf(d) < 464.f);
    if (in) return encode_fp8x4_inrange(a, b, c, d);
    return encode_fp8(a) | (encode_fp8(b) << 8) | (encode_fp8(c) << 16) | (encode_fp8(d) << 24);
}

// quant_device::scale (reference quant_format.cuh:62-64). Division is IEEE
// correctly rounded (HIP default for fp32 '/').
template <int Fmt> __device__ __forceinline__ float quant_scale(float amax) {
    constexpr float range = Fmt == I8 ? 127.f : 448.f;
    return amax == 0 ? 1.f : fmaxf(amax / range, 1.17549435e-38f);
}

// Rademacher sign of the H128 rotation for an absolute column (reference
// quant_device.cuh:166-168).
__device__ __forceinline__ float rotation_sign(int column) {
    uint32_t h = uint32_t(column) * 0x45d9f3bu;
    h = (h ^ (h >> 16)) * 0x45d9f3bu;
    return ((h ^ (h >> 16)) & 1u) ? 1.f : -1.f;
}

// Value rounded to the 16-bit storage type and widened back (exact).
template <class T> __device__ __forceinline__ float round16(float x) {
    return to_float(from_float(x, T{}), T{});
}
// bf16: gfx950's conversion instruction (IEEE round-to-nearest-even,
// subnormals kept; a NaN stays a NaN) and a widening shift: the value of the
// integer rounding above in two instructions.
template <> __device__ __forceinline__ float round16<bf16_t>(float x) {
    return __uint_as_float(cvt_pk_bf16(x, 0.f) << 16);
}

// ---------------------------------------------------------------- fp32 exp / tanh
// This library's exponential (the reference's expf / __expf approximate the
// same function): Cody-Waite reduction x = k ln2 + r with ln2 split into a
// 16-bit head (0x1.62e4p-1, so k * head is exact) and a tail, |r| <= 0.347;
// e^r by its Taylor polynomial to degree 8 (next term < 2^-32 relative), in
// Horner form with fma; the result scaled by 2^k in two exact power-of-two
// factors so that only the final product rounds (subnormal results included).
// inf above 89, 0 below -104, NaN kept.
__device__ __forceinline__ float qexp(float x) {
    if (x != x) return x;
    x = fminf(fmaxf(x, -104.f), 89.f);
    const float k = rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-k, 0x1.62e4p-1f, x);
    r = __builtin_fmaf(-k, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-16f;
    p = __builtin_fmaf(p, r, 0x1.a01a02p-13f);
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.f);
    p = __builtin_fmaf(p, r, 1.f);
    const int ki = int(k), k1 = ki / 2, k2 = ki - k1;
    return (p * __uint_as_float(uint32_t(k1 + 127) << 23)) *
           __uint_as_float(uint32_t(k2 + 127) << 23);
}

// This library's tanh: the odd Taylor series to degree 15 for |y| < 0.5
// (next term < 2^-27 relative), else 1 - 2 / (e^{2|y|} + 1) with qexp, with
// the sign of y; 1 beyond |y| = 9.1 (where tanh rounds to 1 in fp32).
__device__ __forceinline__ float qtanh(float y) {
    if (y != y) return y;
    const float a = fabsf(y);
    float t;
    if (a < 0.5f) {
        const float s = a * a;
        float p = -0x1.7da364p-10f;
        p = __builtin_fmaf(p, s, 0x1.d6d3d0p-9f);
        p = __builtin_fmaf(p, s, -0x1.226e36p-7f);
        p = __builtin_fmaf(p, s, 0x1.664f48p-6f);
        p = __builtin_fmaf(p, s, -0x1.ba1ba2p-5f);
        p = __builtin_fmaf(p, s, 0x1.111112p-3f);
        p = __builtin_fmaf(p, s, -0x1.555556p-2f);
        t = __builtin_fmaf(a * s, p, a);
    } else if (a < 9.1f) {
        t = 1.f - 2.f / (qexp(2.f * a) + 1.f);
    } else {
        t = 1.f;
    }
    return __builtin_copysignf(t, y);
}

// tanh-GeLU of the reference: (0.5x)(1 + tanh(0.7978845608028654 * inner))
// in fp32 with qtanh. The reference's TUs differ in contraction:
// quant_gated.cu (built with --fmad=false, quant_gated.cu:14-15) forms
// inner = x + ((0.044715x)x)x with separate roundings; activation.cuh:15 as
// compiled into the GEMM epilogue and the pointwise finish (FMA contraction
// on) forms inner = fma((0.044715x)x, x, x).
template <bool Contracted>
__device__ __forceinline__ float gelu_tanh(float x) {
    const float cubic = (0.044715f * x) * x;
    const float inner = Contracted ? __builtin_fmaf(cubic, x, x) : x + cubic * x;
    return (0.5f * x) * (1.f + qtanh(0.7978845608028654f * inner));
}

// Finish of a quantized linear on its stored result d (the reference's
// pointwise finish, ops/kernels/sequence/sequence_internal.cuh:59-73, with
// value/output scale 1): s16(act(s16(s16(d) + bias[n]))); act 1 = ReLU,
// 2 = tanh-GeLU, 0 = none. The caller's store performs the final rounding.
enum Finish : int { FINISH_NONE = 0, FINISH_RELU = 1, FINISH_GELU_TANH = 2 };
// Out of line: the GEMM epilogues call it only when a finish is requested,
// so the tanh does not enlarge the register allocation of their loops.
template <class Out>
__device__ __noinline__ void finish4(float (&v)[4], const uint16_t *bias, int n, int n_last,
                                     int act) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float x = round16<Out>(v[r]);
        // The reference adds the bias read as 0 when absent (-0 becomes +0).
        x = round16<Out>(x + (bias ? to_float(bias[min(n + r, n_last)], Out{}) : 0.f));
        if (act == FINISH_RELU) x = fmaxf(x, 0.f);
        else if (act == FINISH_GELU_TANH) x = gelu_tanh<true>(x);
        v[r] = x;
    }
}

// ---------------------------------------------------------------- wave64 reductions
// The value held by lane (lane ^ S), S a power of two up to 32, without an
// LDS round trip: S = 1, 2 by a DPP quad permutation, 4 by two row rotations
// and a select, 8 by a row rotation, 16 / 32 by gfx950's row swaps
// (v_permlane16_swap / v_permlane32_swap, which with both operands x leave
// the partner's value in the first result for lanes with bit S set and in
// the second for the others).
template <int S> __device__ __forceinline__ float lane_xor(float v) {
    const int u = __float_as_int(v);
    if constexpr (S == 1) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
    } else if constexpr (S == 2) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
    } else if constexpr (S == 4) {
        // row_ror:n moves data n lanes up a 16-lane row: lane l reads l - n
        const int from_below = __builtin_amdgcn_update_dpp(0, u, 0x124, 0xF, 0xF, false);  // l - 4
        const int from_above = __builtin_amdgcn_update_dpp(0, u, 0x12C, 0xF, 0xF, false);  // l + 4
        return __int_as_float((threadIdx.x & 4) ? from_below : from_above);
    } else if constexpr (S == 8) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x128, 0xF, 0xF, false));  // row_ror:8
    } else {
        static_assert(S == 16 || S == 32, "lane distance");
        const auto r = S == 32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                               : __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __int_as_float(int((threadIdx.x & S) ? r[0] : r[1]));
    }
}

// Max over a power-of-two lane group of width W (aligned).
template <int W> __device__ __forceinline__ float group_max(float v) {
    if constexpr (W > 1) v = fmaxf(v, lane_xor<1>(v));
    if constexpr (W > 2) v = fmaxf(v, lane_xor<2>(v));
    if constexpr (W > 4) v = fmaxf(v, lane_xor<4>(v));
    if constexpr (W > 8) v = fmaxf(v, lane_xor<8>(v));
    if constexpr (W > 16) v = fmaxf(v, lane_xor<16>(v));
    if constexpr (W > 32) v = fmaxf(v, lane_xor<32>(v));
    return v;
}

}  // namespace qlin
