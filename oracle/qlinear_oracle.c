/*
 * qlinear_oracle.c — CPU restatement of TTS.cpp's quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP
 * library in breeze_tts_cpp_amd/. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product path never does.
 *
 * Every function names the reference file:line whose arithmetic it restates
 * (paths relative to the reference's src/). Build flags (oracle/Makefile):
 * -O3 -ffp-contract=off -fno-fast-math, so that every a*b+c here is two
 * IEEE fp32 roundings, matching the reference's `--fmad=false` translation
 * units (CMakeLists.txt:93-104). Where the reference leaves fusion to nvcc
 * (quant_grouped.cu:144) the contraction is written explicitly with fmaf().
 *
 * Pinning (tests/test_oracle.py): FP8 codec exhaustively against its closed
 * form and torch.float8_e4m3fn; INT8 quant against the closed form and
 * special cases; rotation against an explicit Sylvester-matrix product and
 * orthogonality; GEMMs against brute force, linearity and fp64 products.
 * NaN propagation through the quantizers is "parity unpinned": the reference
 * mixes fmaxf (NaN-dropping) with integer max over float bits, and no test of
 * the reference fixes which one a NaN meets first.
 */
#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Storage codes follow tts::Type (core/tensor.h:8). */
enum { T_BF16 = 0, T_F32 = 1, T_I32 = 2, T_FP8 = 3, T_I8 = 4, T_F16 = 5 };

/* ---------------------------------------------------------------- 16-bit floats */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Round-to-nearest-even fp32 -> bf16 (__float2bfloat16_rn semantics). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
    if (exp == 0) { /* subnormal: man * 2^-24, exact in fp32 */
        float v = (float)man * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    return u2f(sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13));
}

/* Round-to-nearest-even fp32 -> IEEE half (__float2half_rn semantics). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    float a = fabsf(f);
    if (a != a) return (uint16_t)(sign | 0x7e00u);
    if (a >= 65520.f) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (a < 6.103515625e-05f) { /* half subnormal range: step 2^-24 */
        float q = nearbyintf(a * 16777216.f);           /* exact scale, RNE */
        return (uint16_t)(sign | (uint16_t)q);           /* q == 1024 is min normal */
    }
    int e;
    float m = frexpf(a, &e); /* a = m * 2^e, m in [0.5,1) */
    float q = nearbyintf(m * 2048.f); /* 11 significant bits, RNE */
    if (q >= 2048.f) { q = 1024.f; ++e; }
    int biased = e - 1 + 15;
    if (biased >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)(biased << 10) | (uint16_t)((int)q - 1024));
}

static inline float load_src(const void *p, int type, size_t i) {
    const uint16_t *h = (const uint16_t *)p;
    return type == T_F16 ? orc_f16_to_f32(h[i]) : orc_bf16_to_f32(h[i]);
}
static inline uint16_t store_out(float v, int type) {
    return type == T_F16 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
}

/* ---------------------------------------------------------------- 8-bit codecs */
/* Format<FP8>::decode (ops/kernels/quant/quant_format.cuh:18-22): OCP e4m3fn,
 * bias 7, 3 mantissa bits, 0x7f/0xff NaN, max finite 448. */
float orc_fp8_decode(uint8_t c) {
    int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7) return s ? -NAN : NAN;
    if (e == 0) v = (float)m * 0.001953125f; /* m * 2^-9 */
    else v = ldexpf(1.f + (float)m / 8.f, e - 7);
    return s ? -v : v;
}

/* Format<FP8>::encode (quant_format.cuh:12-14): __nv_fp8_e4m3(x), i.e.
 * round-to-nearest-even with saturation to +-448 (satfinite). */
uint8_t orc_fp8_encode(float x) {
    uint8_t sign = (f2u(x) >> 31) ? 0x80 : 0;
    float a = fabsf(x);
    if (a != a) return 0x7f;
    if (a >= 448.f) return sign | 0x7e; /* satfinite: 448 and above -> max finite */
    if (a < 0.015625f) {                /* below 2^-6: subnormal step 2^-9 */
        float q = nearbyintf(a * 512.f); /* q in [0, 8]; 8 encodes 2^-6 (0x08) */
        return sign | (uint8_t)q;
    }
    int e;
    float m = frexpf(a, &e);            /* a = m * 2^e, m in [0.5, 1) */
    float q = nearbyintf(m * 16.f);     /* 4 significant bits, RNE, q in [8, 16] */
    if (q >= 16.f) { q = 8.f; ++e; }
    int biased = e - 1 + 7;             /* >= 1 here; a < 448 keeps it <= 15 */
    return sign | (uint8_t)(biased << 3) | (uint8_t)((int)q - 8);
}

/* Format<I8>::rounded (quant_format.cuh:37-44): clamp to +-127, then RNE. */
int orc_i8_round(float x) {
    x = fminf(127.f, fmaxf(-127.f, x));
    return (int)nearbyintf(x);
}

static inline uint8_t encode(float x, int fmt) {
    return fmt == T_I8 ? (uint8_t)(int8_t)orc_i8_round(x) : orc_fp8_encode(x);
}

/* quant_device::scale (quant_format.cuh:62-64). */
float orc_scale(float amax, int fmt) {
    float range = fmt == T_I8 ? 127.f : 448.f;
    return amax == 0 ? 1.f : fmaxf(amax / range, FLT_MIN);
}

/* ---------------------------------------------------------------- H128 rotation */
/* Rademacher sign of rotate_pack (quant_device.cuh:162-169), absolute column. */
float orc_rotation_sign(int column) {
    uint32_t h = (uint32_t)column * 0x45d9f3bu;
    h = (h ^ (h >> 16)) * 0x45d9f3bu;
    return ((h ^ (h >> 16)) & 1u) ? 1.f : -1.f;
}

/* rotate_pack (quant_device.cuh:161-190) over one 128-column block starting at
 * absolute column c0: sign, Sylvester butterflies with ascending stride
 * (lower index gets a+b, upper gets a-b), then a separate multiply by
 * 0.08838834764831845f. */
void orc_rotate128(float *v, int c0) {
    for (int i = 0; i < 128; ++i) v[i] = v[i] * orc_rotation_sign(c0 + i);
    for (int span = 1; span < 128; span *= 2)
        for (int i = 0; i < 128; ++i)
            if (!(i & span)) {
                float a = v[i], b = v[i | span];
                v[i] = a + b;
                v[i | span] = a - b;
            }
    for (int i = 0; i < 128; ++i) v[i] *= 0.08838834764831845f;
}

/* ---------------------------------------------------------------- row quantizer */
/* launch_row_quantize (ops/kernels/quant/row_quantize.cu:167-193) and its
 * kernels: dynamic/cached_token_quantize (:24-87, same arithmetic),
 * rotated_token_quantize (:90-115), group_token_quantize + encode_group
 * (:145-165, quant_device.cuh:63-88). Scales: [rows] for per-token,
 * [ceil(K/group), rows] group-major otherwise (core/quantization.h:24-32).
 * Returns 0, or -1 on an unsupported layout. */
int orc_quantize_rows(const void *src, int src_type, int ld, int rows, int cols, int fmt,
                      int group, int rotation, uint8_t *q, float *scales) {
    if (rotation && (rotation != 128 || cols % 128)) return -1;
    if (group && group != 32 && group != 64 && group != 128) return -1;
    float *row = (float *)malloc(sizeof(float) * (size_t)cols);
    if (!row) return -1;
    int groups = group ? (cols + group - 1) / group : 1;
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < cols; ++c) row[c] = load_src(src, src_type, (size_t)r * ld + c);
        if (rotation)
            for (int c0 = 0; c0 < cols; c0 += 128) orc_rotate128(row + c0, c0);
        if (group) {
            for (int g = 0; g < groups; ++g) {
                int c0 = g * group, c1 = c0 + group < cols ? c0 + group : cols;
                float amax = 0;
                for (int c = c0; c < c1; ++c) amax = fmaxf(amax, fabsf(row[c]));
                float step = orc_scale(amax, fmt), inverse = 1.f / step;
                scales[(size_t)g * rows + r] = step;
                for (int c = c0; c < c1; ++c) q[(size_t)r * cols + c] = encode(row[c] * inverse, fmt);
            }
        } else {
            float amax = 0;
            for (int c = 0; c < cols; ++c) amax = fmaxf(amax, fabsf(row[c]));
            float step = orc_scale(amax, fmt), inverse = 1.f / step;
            scales[r] = step;
            for (int c = 0; c < cols; ++c) q[(size_t)r * cols + c] = encode(row[c] * inverse, fmt);
        }
    }
    free(row);
    return 0;
}

/* ---------------------------------------------------------------- fused producers */
/* 1/sqrt(a) rounded once to fp32 (via fp64). The reference's rsqrtf
 * (quant_norm.cu:75) is an approximation within 2 ulp of this value, so the
 * normalized rows agree with the reference except where that error crosses a
 * 16-bit rounding boundary ("parity bounded" for this step). */
float orc_rsqrt_rn(float a) { return (float)(1.0 / sqrt((double)a)); }

/* Squared-sum reduction of residual_rms_quantize (quant_norm.cu:30-73) over
 * one row of 16-bit-rounded values v[0..cols): 256 threads, thread t owning
 * columns [8t, 8t+8) (cols <= 2048), sum += x0*x0 + x1*x1 per pair; per
 * 32-thread warp a __shfl_down_sync tree with strides 16..1 (a lane whose
 * source is out of range adds its own value); warp partials summed in order. */
float orc_norm_sumsq(const float *v, int cols) {
    float warp[32], next[32], total = 0.f;
    for (int w = 0; w < 8; ++w) {
        for (int i = 0; i < 32; ++i) {
            int t = w * 32 + i;
            float sum = 0.f;
            for (int p = 0; p < 4; ++p) {
                int c = 8 * t + 2 * p;
                float a = c < cols ? v[c] : 0.f, b = c + 1 < cols ? v[c + 1] : 0.f;
                sum += a * a + b * b;
            }
            warp[i] = sum;
        }
        for (int d = 16; d; d /= 2) {
            for (int i = 0; i < 32; ++i) next[i] = warp[i] + (i + d < 32 ? warp[i + d] : warp[i]);
            memcpy(warp, next, sizeof(warp));
        }
        total += warp[0];
    }
    return total;
}

/* launch_quantized_norm / residual_rms_quantize (quant_norm.cu:14-123,
 * 166-188): optional residual update (stored back), RMSNorm with 16-bit
 * rounding points (__hadd2/__hmul2/pack), then the row quantizer on the
 * normalized 16-bit row (its transformed branch calls the same encode_group /
 * rotated_quantize as launch_row_quantize). `normalized` (optional) receives
 * the normalized 16-bit rows. Returns 0, or -1 on bad layout. */
int orc_quantized_norm(uint16_t *residual, const uint16_t *update, const uint16_t *update_scale,
                       const uint16_t *weight, int src_type, int rows, int cols, float eps,
                       int gemma, int fmt, int group, int rotation, uint8_t *q, float *scales,
                       uint16_t *normalized) {
    if (cols < 1 || cols > 2048) return -1;
    float *v = (float *)malloc(sizeof(float) * 2048);
    uint16_t *n = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)rows * cols);
    if (!v || !n) { free(v); free(n); return -1; }
    for (int r = 0; r < rows; ++r) {
        uint16_t *x = residual + (size_t)r * cols;
        for (int c = 0; c < cols; ++c) {
            float a = load_src(x, src_type, c);
            if (update) {
                float b = load_src(update, src_type, (size_t)r * cols + c);
                if (update_scale)
                    b = load_src(&(uint16_t){store_out(b * load_src(update_scale, src_type, c),
                                                       src_type)}, src_type, 0);
                uint16_t sum = store_out(a + b, src_type);
                x[c] = sum;
                a = load_src(&sum, src_type, 0);
            }
            v[c] = a;
        }
        float inv = orc_rsqrt_rn(orc_norm_sumsq(v, cols) / (float)cols + eps);
        for (int c = 0; c < cols; ++c) {
            float w = load_src(weight, src_type, c);
            if (gemma) {
                n[(size_t)r * cols + c] = store_out((v[c] * inv) * (w + 1.f), src_type);
            } else {
                uint16_t h = store_out(v[c] * inv, src_type);
                n[(size_t)r * cols + c] = store_out(load_src(&h, src_type, 0) * w, src_type);
            }
        }
    }
    int status = orc_quantize_rows(n, src_type, cols, rows, cols, fmt, group, rotation, q, scales);
    if (normalized) memcpy(normalized, n, sizeof(uint16_t) * (size_t)rows * cols);
    free(v);
    free(n);
    return status;
}

/* The library's fp32 exponential (the reference's expf / __expf approximate
 * the same function): Cody-Waite reduction x = k ln2 + r with ln2 split into
 * a 16-bit head 0x1.62e4p-1 (k * head exact) and a tail, e^r by its Taylor
 * polynomial to degree 8 in Horner form with fmaf, scaled by 2^k as two
 * exact power-of-two factors (one final rounding). inf above 89, 0 below
 * -104, NaN kept. */
float orc_qexp(float x) {
    if (x != x) return x;
    x = fminf(fmaxf(x, -104.f), 89.f);
    float k = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-k, 0x1.62e4p-1f, x);
    r = fmaf(-k, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-16f;
    p = fmaf(p, r, 0x1.a01a02p-13f);
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.f);
    p = fmaf(p, r, 1.f);
    int ki = (int)k, k1 = ki / 2, k2 = ki - k1;
    return (p * u2f((uint32_t)(k1 + 127) << 23)) * u2f((uint32_t)(k2 + 127) << 23);
}

/* The library's fp32 tanh: odd Taylor series to degree 15 for |y| < 0.5,
 * else 1 - 2/(e^{2|y|} + 1) with orc_qexp; 1 beyond 9.1; sign of y. */
float orc_qtanh(float y) {
    if (y != y) return y;
    float a = fabsf(y), t;
    if (a < 0.5f) {
        float s = a * a;
        float p = -0x1.7da364p-10f;
        p = fmaf(p, s, 0x1.d6d3d0p-9f);
        p = fmaf(p, s, -0x1.226e36p-7f);
        p = fmaf(p, s, 0x1.664f48p-6f);
        p = fmaf(p, s, -0x1.ba1ba2p-5f);
        p = fmaf(p, s, 0x1.111112p-3f);
        p = fmaf(p, s, -0x1.555556p-2f);
        t = fmaf(a * s, p, a);
    } else if (a < 9.1f) {
        t = 1.f - 2.f / (orc_qexp(2.f * a) + 1.f);
    } else {
        t = 1.f;
    }
    return copysignf(t, y);
}

/* activate<Kind> (quant_gated.cu:9-16): SiLU (kind 0) as
 * (x*2^-16) / ((1 + e^-x) * 2^-16), tanh-GeLU (kind 1) as
 * (0.5x)(1 + tanh(0.7978845608028654f * (x + ((0.044715f*x)*x)*x))), fp32
 * arithmetic with e^-x and tanh from orc_qexp / orc_qtanh (the reference's
 * __expf, __fdividef and tanhf approximate the same functions). */
float orc_activate(float x, int kind) {
    if (kind == 0) {
        float e = orc_qexp(-x);
        return (x * 0x1p-16f) / ((1.f + e) * 0x1p-16f);
    }
    float inner = x + ((0.044715f * x) * x) * x;
    return (0.5f * x) * (1.f + orc_qtanh(0.7978845608028654f * inner));
}

/* launch_quantized_gated / vector_gated_quantize (quant_gated.cu:18-85,
 * 179-198): a = s16(s16(act(gate)) * up) over input [rows, 2*width]
 * (gate | up), then the row quantizer. `activated` (optional) receives the
 * 16-bit activated rows. Returns 0, or -1 on bad layout. */
int orc_quantized_gated(const uint16_t *input, int src_type, int rows, int width, int kind,
                        int fmt, int group, int rotation, uint8_t *q, float *scales,
                        uint16_t *activated) {
    if (width < 1 || width > 8192 || kind < 0 || kind > 1) return -1;
    uint16_t *a = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)rows * width);
    if (!a) return -1;
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < width; ++c) {
            float g = load_src(input, src_type, (size_t)r * 2 * width + c);
            float u = load_src(input, src_type, (size_t)r * 2 * width + width + c);
            uint16_t h = store_out(orc_activate(g, kind), src_type);
            a[(size_t)r * width + c] = store_out(load_src(&h, src_type, 0) * u, src_type);
        }
    int status = orc_quantize_rows(a, src_type, width, rows, width, fmt, group, rotation, q, scales);
    if (activated) memcpy(activated, a, sizeof(uint16_t) * (size_t)rows * width);
    free(a);
    return status;
}

/* tanh-GeLU as the reference's activation.cuh:15 compiles with FMA
 * contraction (the GEMM epilogue and the pointwise finish TUs): inner =
 * fma((0.044715x)x, x, x); tanh by orc_qtanh (the reference uses
 * cutlass::fast_tanh). */
float orc_gelu_tanh_contracted(float x) {
    float inner = fmaf((0.044715f * x) * x, x, x);
    return (0.5f * x) * (1.f + orc_qtanh(0.7978845608028654f * inner));
}

/* ---------------------------------------------------------------- finish */
/* The finish of a quantized linear on its stored 16-bit result y (the
 * reference's pointwise Finish::apply, ops/kernels/sequence/sequence_internal.cuh:61-73
 * with value/output scale 1, activations of ops/kernels/common/activation.cuh:7,14):
 * y' = s16(act(s16(y + bias[n]))), act 0 none, 1 ReLU, 2 tanh-GeLU (the
 * contracted form above). An absent bias adds 0 as the reference's View::get
 * does. In place. */
void orc_finish(uint16_t *y, const uint16_t *bias, int M, int N, int act, int type) {
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float v = load_src(y, type, (size_t)m * N + n);
            uint16_t h = store_out(v + (bias ? load_src(bias, type, n) : 0.f), type);
            v = load_src(&h, type, 0);
            if (act == 1) v = fmaxf(v, 0.f);
            else if (act == 2) v = orc_gelu_tanh_contracted(v);
            y[(size_t)m * N + n] = store_out(v, type);
        }
}

/* ---------------------------------------------------------------- LayerNorm -> GEMV */
/* cub::BlockReduce<float, 256>::Sum, warp-reductions algorithm (CUDA 13 CUB,
 * the NormReduce of ops/kernels/sequence/sequence_internal.cuh:135-136):
 * per 32-thread warp, lane i adds lane i+s for s = 1, 2, 4, 8, 16 (when
 * i+s < 32; all lanes update simultaneously), warp totals added in order. */
float orc_cub_sum256(const float *v) {
    float warp[32], next[32], total = 0.f;
    for (int w = 0; w < 8; ++w) {
        memcpy(warp, v + 32 * w, sizeof(warp));
        for (int s = 1; s < 32; s *= 2) {
            for (int i = 0; i < 32; ++i) next[i] = i + s < 32 ? warp[i] + warp[i + s] : warp[i];
            memcpy(warp, next, sizeof(warp));
        }
        total = w ? total + warp[0] : warp[0];
    }
    return total;
}

/* NormFusion / Epilogue layouts (the library's qlin_norm_fusion and
 * qlin_epilogue, restating ops::NormFusion, ops/sequence.h:55-59, and the
 * dense part of ops::Epilogue, ops/sequence.h:8-27). */
typedef struct {
    const uint16_t *residual, *projection_bias, *gate, *shift, *scale;
    int gate_rows, shift_rows, scale_rows;
    uint16_t *raw;
    int rows_per_sequence;
    const int *source_rows;
} orc_norm_fusion;

typedef struct {
    const uint16_t *bias, *residual;
    int residual_rows;
    const int *residual_index;
    float value_scale, output_scale, residual_scale;
    int activation;
    float alpha;
    uint16_t *raw;
    const uint16_t *gate;
    int gate_rows;
    const uint16_t *condition;
    int condition_rows;
    int rows_per_sequence, valid_rows_per_sequence, input_repeat;
} orc_epilogue;

static inline float r16(float v, int type) { uint16_t h = store_out(v, type); return load_src(&h, type, 0); }
/* View::get of a [rows, cols] tensor (row 0 when it has one row), 0 when absent
 * (ops/kernels/sequence/sequence_internal.cuh:21-25, sequence_norm.cu:18-27). */
static inline float view_get(const uint16_t *p, int rows, int r, int cols, int c, int type) {
    return p ? load_src(p, type, (size_t)(rows == 1 ? 0 : r) * cols + c) : 0.f;
}

/* LayerNorm rows with NormFusion (NormRow::load / transform,
 * sequence_norm.cu:40-53, statistics of norm_kernel :84-117 and
 * norm_project_kernel :272-292): thread t of 256 sums columns t, t+256, ...
 * in order; the partials reduce in cub::BlockReduce order; mean = sum/cols;
 * the variance partial is fma(d, d, sum) (the TU contracts sum += d*d);
 * inv = 1/sqrt(var/cols + eps) rounded once. u [rows, cols] receives the
 * normalized 16-bit rows; an out-of-range source row gives NaN. raw (from
 * f->raw) receives v. Returns 0. */
int orc_norm_rows(const uint16_t *x, int x_rows, int type, int rows, int cols,
                  const uint16_t *nw, const uint16_t *nb, float eps, const orc_norm_fusion *f,
                  uint16_t *u) {
    float *v = (float *)malloc(sizeof(float) * (size_t)cols);
    if (!v) return -1;
    float part[256];
    for (int out = 0; out < rows; ++out) {
        int row = f->source_rows ? f->source_rows[out] : out;
        if (row < 0 || row >= x_rows) {
            for (int c = 0; c < cols; ++c) u[(size_t)out * cols + c] = store_out(NAN, type);
            continue;
        }
        int seq = row / f->rows_per_sequence;
        for (int c = 0; c < cols; ++c) {
            float a = r16(load_src(x, type, (size_t)row * cols + c) +
                          view_get(f->projection_bias, 1, 0, cols, c, type), type);
            if (f->gate) a = r16(a * view_get(f->gate, f->gate_rows, seq, cols, c, type), type);
            a = r16(a + view_get(f->residual, x_rows, row, cols, c, type), type);
            v[c] = a;
            if (f->raw) f->raw[(size_t)out * cols + c] = store_out(a, type);
        }
        for (int t = 0; t < 256; ++t) {
            float sum = 0.f;
            for (int c = t; c < cols; c += 256) sum += v[c];
            part[t] = sum;
        }
        float mean = orc_cub_sum256(part) / (float)cols;
        for (int t = 0; t < 256; ++t) {
            float sum = 0.f;
            for (int c = t; c < cols; c += 256) { float d = v[c] - mean; sum = fmaf(d, d, sum); }
            part[t] = sum;
        }
        float inv = orc_rsqrt_rn(orc_cub_sum256(part) / (float)cols + eps);
        for (int c = 0; c < cols; ++c) {
            float val = (v[c] - mean) * inv;
            if (nw) val = val * load_src(nw, type, c);
            val = r16(val + (nb ? load_src(nb, type, c) : 0.f), type);
            if (f->scale)
                val = r16(val * r16(1.f + view_get(f->scale, f->scale_rows, seq, cols, c, type), type), type);
            val = r16(val + view_get(f->shift, f->shift_rows, seq, cols, c, type), type);
            u[(size_t)out * cols + c] = store_out(val, type);
        }
    }
    free(v);
    return 0;
}

/* layer_norm_quantize (sequence_norm.cu:65-200,412-440): the LayerNorm rows
 * above, optionally retained, quantized by the row quantizer (RowOutput
 * store/store_group, ops/kernels/quant/quant_output.cuh). A NaN row (bad
 * source) gets scales 1 and the codes of NaN, as the row quantizer gives. */
int orc_layer_norm_quantize(const uint16_t *x, int x_rows, int type, const uint16_t *nw,
                            const uint16_t *nb, float eps, const orc_norm_fusion *f,
                            uint16_t *retained, int rows, int cols, uint8_t *q, float *scales,
                            int fmt, int group, int rotation) {
    if (rotation && !group) return -1;
    uint16_t *u = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)rows * cols);
    if (!u) return -1;
    orc_norm_rows(x, x_rows, type, rows, cols, nw, nb, eps, f, u);
    int status = orc_quantize_rows(u, type, cols, rows, cols, fmt, group, rotation, q, scales);
    if (retained) memcpy(retained, u, sizeof(uint16_t) * (size_t)rows * cols);
    free(u);
    return status;
}

/* ops::activate (ops/kernels/common/activation.cuh:5-26), Activation
 * numbering of ops/activation.h:4. SiLU, sigmoid, tanh and tanh-GeLU use
 * orc_qexp / orc_qtanh; GeLU's erf and Mish's exp / log1p / tanh are
 * evaluated in fp64 and rounded once to fp32 at the points the reference
 * rounds its fp32 library calls (expf, erff, log1pf and tanhf approximate
 * them); tanh-GeLU's inner term is contracted as the pointwise TU compiles
 * it. */
float orc_act(float x, int kind, float alpha) {
    switch (kind) {
    case 1: return fmaxf(x, 0.f);
    case 2: return x >= 0.f ? x : x * alpha;
    case 3: return x / (1.f + orc_qexp(-x));
    case 4: return (0.5f * x) * (1.f + (float)erf((double)(x * 0.7071067811865475f)));
    case 5: return orc_gelu_tanh_contracted(x);
    case 6: {
        float sp = x > 20.f ? x : (float)log1p((double)(float)exp((double)x));
        return x * (float)tanh((double)sp);
    }
    case 7: return orc_qtanh(x);
    case 8: return 1.f / (1.f + orc_qexp(-x));
    default: return x;
    }
}

/* pointwise_quantize (sequence_pointwise.cu:149-260,325-357) with the dense
 * Finish::apply (ops/kernels/sequence/sequence_internal.cuh:52-74), per
 * element of output row r (x row r / input_repeat, row 0 when x_rows == 1):
 * masked rows give raw 0 and 0; else v = s16(x + bias); v = s16(v * gate[b]);
 * v = s16(fma(value_scale, v, residual_scale * skip)) (the TU contracts
 * value_scale*v + scale*skip on its first product); v = s16(v + condition[b]);
 * raw = v; out = s16(act(s16(v * output_scale))). Then the row quantizer. */
int orc_pointwise_quantize(const uint16_t *x, int x_rows, int type, const orc_epilogue *e,
                           uint16_t *retained, int rows, int cols, uint8_t *q, float *scales,
                           int fmt, int group, int rotation) {
    if (rotation && !group) return -1;
    uint16_t *o = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)rows * cols);
    if (!o) return -1;
    for (int r = 0; r < rows; ++r) {
        int masked = e->valid_rows_per_sequence &&
                     r % e->rows_per_sequence >= e->valid_rows_per_sequence;
        int seq = r / e->rows_per_sequence, xr = x_rows == 1 ? 0 : r / e->input_repeat;
        int rr = e->residual_index ? e->residual_index[r] : r;
        for (int c = 0; c < cols; ++c) {
            float value = 0.f;
            if (!masked) {
                value = r16(load_src(x, type, (size_t)xr * cols + c) + view_get(e->bias, 1, 0, cols, c, type), type);
                if (e->gate) value = r16(value * view_get(e->gate, e->gate_rows, seq, cols, c, type), type);
                float skip = 0.f;
                if (e->residual && rr >= 0)
                    skip = rr < e->residual_rows ? view_get(e->residual, e->residual_rows, rr, cols, c, type) : NAN;
                value = r16(fmaf(e->value_scale, value, e->residual_scale * skip), type);
                if (e->condition) value = r16(value + view_get(e->condition, e->condition_rows, seq, cols, c, type), type);
            }
            if (e->raw) e->raw[(size_t)r * cols + c] = store_out(value, type);
            if (!masked) value = r16(orc_act(r16(value * e->output_scale, type), e->activation, e->alpha), type);
            o[(size_t)r * cols + c] = store_out(value, type);
        }
    }
    int status = orc_quantize_rows(o, type, cols, rows, cols, fmt, group, rotation, q, scales);
    if (retained) memcpy(retained, o, sizeof(uint16_t) * (size_t)rows * cols);
    free(o);
    return status;
}

/* normalized_quantized_linear / norm_project_kernel<T, QuantProjection>
 * (ops/kernels/sequence/sequence_norm.cu:216-390, host :518-575): the
 * LayerNorm rows above (no source_rows), quantized per token; the Finish
 * with bias and ReLU/identity. INT8 dot products are exact; FP8 ones follow
 * the reference order: lane l of a warp sums words c = 4l + 128j with fmaf
 * over the 4 decoded bytes, then a shfl-down tree 16..1.
 * Outputs: y [rows, n]; normalized [rows, k] and encoded/escales optional. */
int orc_norm_linear(const uint16_t *x, const orc_norm_fusion *f, const uint16_t *nw,
                    const uint16_t *nb, int type, int rows, int k, float eps, const uint8_t *w,
                    const float *sw, int fmt, int n, const uint16_t *bias, int act, uint16_t *y,
                    uint16_t *normalized, uint8_t *encoded, float *escales) {
    if (k < 4 || k % 4 || k > 512 || f->source_rows) return -1;
    uint16_t *u = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)rows * k);
    if (!u) return -1;
    orc_norm_rows(x, rows, type, rows, k, nw, nb, eps, f, u);
    float r[512], a[512];
    for (int row = 0; row < rows; ++row) {
        float amax = 0.f;
        for (int c = 0; c < k; ++c) {
            r[c] = load_src(u, type, (size_t)row * k + c);
            amax = fmaxf(amax, fabsf(r[c]));
        }
        float scale = orc_scale(amax, fmt), recip = 1.f / scale;
        if (escales) escales[row] = scale;
        for (int c = 0; c < k; ++c) {
            uint8_t q = encode(r[c] * recip, fmt);
            a[c] = fmt == T_I8 ? (float)(int8_t)q : orc_fp8_decode(q);
            if (encoded) encoded[(size_t)row * k + c] = q;
        }
        for (int ch = 0; ch < n; ++ch) {
            const uint8_t *wr = w + (size_t)ch * k;
            float result;
            if (fmt == T_I8) {
                int64_t acc = 0;
                for (int c = 0; c < k; ++c) acc += (int64_t)(int)a[c] * (int8_t)wr[c];
                result = ((float)acc * sw[ch]) * scale;
            } else {
                float lane[32], next[32];
                for (int l = 0; l < 32; ++l) {
                    float acc = 0.f;
                    for (int c = 4 * l; c < k; c += 128)
                        for (int e = 0; e < 4; ++e) acc = fmaf(a[c + e], orc_fp8_decode(wr[c + e]), acc);
                    lane[l] = acc;
                }
                for (int d = 16; d; d /= 2) {
                    for (int l = 0; l < 32; ++l) next[l] = l + d < 32 ? lane[l] + lane[l + d] : lane[l];
                    memcpy(lane, next, sizeof(lane));
                }
                result = (lane[0] * sw[ch]) * scale;
            }
            float o = r16(r16(result, type) + (bias ? load_src(bias, type, ch) : 0.f), type);
            if (act == 1) o = fmaxf(o, 0.f);
            y[(size_t)row * n + ch] = store_out(o, type);
        }
    }
    if (normalized) memcpy(normalized, u, sizeof(uint16_t) * (size_t)rows * k);
    free(u);
    return 0;
}

/* ---------------------------------------------------------------- packed weights */
/* The packed layout of load-time-quantized weights (no reference counterpart;
 * follows io/weights.cpp:80-87): tile (g, t) = rows [16g, 16g+16) x K bytes
 * [64t, 64t+64) at (g*ceil(K/64) + t)*1024, chunk 16q + r of a tile = row
 * 16g + r, K bytes [64t + 16q, +16); zero past K. Returns 0, -1 if N % 16. */
int orc_pack_weights(const uint8_t *w, int N, int K, uint8_t *packed) {
    if (N % 16) return -1;
    int tk = (K + 63) / 64;
    for (int g = 0; g < N / 16; ++g)
        for (int t = 0; t < tk; ++t)
            for (int q = 0; q < 4; ++q)
                for (int r = 0; r < 16; ++r)
                    for (int b = 0; b < 16; ++b) {
                        int k = t * 64 + q * 16 + b;
                        packed[((size_t)g * tk + t) * 1024 + (size_t)(q * 16 + r) * 16 + b] =
                            k < K ? w[(size_t)(g * 16 + r) * K + k] : 0;
                    }
    return 0;
}

/* ---------------------------------------------------------------- GEMMs */
/* Exact INT8 GEMM: acc[m][n] = sum_k x[m][k]*w[n][k] in int32. Any tiling or
 * split of the reference (quant_dispatch.cu:58-61 dp4a, quant_gemm_sm80.cu
 * mma.16x8x32, split-K partials) produces exactly this value. */
void orc_gemm_i8_acc(const int8_t *x, const int8_t *w, int M, int N, int K, int32_t *acc) {
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            int32_t s = 0;
            const int8_t *a = x + (size_t)m * K, *b = w + (size_t)n * K;
            for (int k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)b[k];
            acc[(size_t)m * N + n] = s;
        }
}

/* INT8 per-channel epilogue. order 0: D((acc*sx)*sw) — the CUTLASS EVT tree of
 * quant_gemm_sm80.cu:24-29 (and sm90 :131-132); order 1: D((acc*sw)*sx) — the
 * GEMV store of quant_dispatch.cu:125. */
void orc_epilogue_i8(const int32_t *acc, const float *sx, const float *sw, int M, int N,
                     int order, int out_type, uint16_t *y) {
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float a = (float)acc[(size_t)m * N + n], v;
            if (order == 0) { v = a * sx[m]; v = v * sw[n]; }
            else { v = a * sw[n]; v = v * sx[m]; }
            y[(size_t)m * N + n] = store_out(v, out_type);
        }
}

/* FP8 per-channel ideal: exact products of e4m3 pairs summed in fp64, scaled
 * by sx*sw in fp64. The reference accumulates in fp32 in a hardware order
 * (sm90 WGMMA promotion, cuBLASLt) that no CPU can restate; FP8 parity is
 * therefore a tolerance against this value (rel-L2). */
void orc_gemm_fp8_ideal(const uint8_t *x, const float *sx, const uint8_t *w, const float *sw,
                        int M, int N, int K, float *y) {
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = orc_fp8_decode((uint8_t)i);
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double s = 0;
            const uint8_t *a = x + (size_t)m * K, *b = w + (size_t)n * K;
            for (int k = 0; k < K; ++k) s += (double)lut[a[k]] * (double)lut[b[k]];
            y[(size_t)m * N + n] = (float)(s * (double)sx[m] * (double)sw[n]);
        }
}

/* K-group GEMM of grouped_gemm (quant_grouped.cu:79-166) and its split-K
 * reduction (quant_grouped.cu:221-239, quant_reduce.cuh:9-19).
 * K is cut into splits*waves ranges of `span` columns (range r = s*waves+w
 * covers [r*span, min(K, (r+1)*span))). Inside a range, groups ascending:
 *   p_g   = sum_{k in g} x*w              (int32 exact for INT8;
 *                                           fp64-then-fp32 for FP8)
 *   scale = sxg * swg                      (quant_grouped.cu:135)
 *   r     = fmaf(p_g, scale, r)            (quant_grouped.cu:144, FMA-contracted)
 * A split's ranges are summed R_s = 0 + r_0 + r_1 + ..., then R_s *= the
 * outer scale of a side without groups (quant_grouped.cu:161-163), and
 * y = D(0 + R_0 + R_1 + ...) (quant_reduce.cuh:14-17). With splits = waves =
 * 1 and span >= K this is the reference's single-partition kernel (up to the
 * sign of an exact zero). The loop group is the smaller nonzero group
 * (quant_grouped.cu:185-187). Returns -1 on an unsupported layout. */
int orc_gemm_grouped(const uint8_t *x, const float *sx, const uint8_t *w, const float *sw,
                     int M, int N, int K, int fmt, int input_group, int weight_group, int splits,
                     int waves, int span, int out_type, uint16_t *y, float *y_f32) {
    int g = input_group ? input_group : weight_group;
    if (weight_group && weight_group < g) g = weight_group;
    if (!g || splits < 1 || waves < 1 || span < 1 || span % g) return -1;
    if ((long long)splits * waves * span < K) return -1;
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = orc_fp8_decode((uint8_t)i);
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float total = 0;
            for (int s = 0; s < splits; ++s) {
                float R = 0;
                for (int wv = 0; wv < waves; ++wv) {
                    int r0 = (s * waves + wv) * span;
                    int r1 = r0 + span < K ? r0 + span : K;
                    float r = 0;
                    for (int k0 = r0; k0 < r1; k0 += g) {
                        int k1 = k0 + g < K ? k0 + g : K;
                        float p;
                        if (fmt == T_I8) {
                            int32_t acc = 0;
                            for (int k = k0; k < k1; ++k)
                                acc += (int32_t)(int8_t)x[(size_t)m * K + k] *
                                       (int32_t)(int8_t)w[(size_t)n * K + k];
                            p = (float)acc;
                        } else {
                            double acc = 0;
                            for (int k = k0; k < k1; ++k)
                                acc += (double)lut[x[(size_t)m * K + k]] *
                                       (double)lut[w[(size_t)n * K + k]];
                            p = (float)acc;
                        }
                        float sa = input_group ? sx[(size_t)(k0 / input_group) * M + m] : 1.f;
                        float sb = weight_group ? sw[(size_t)(k0 / weight_group) * N + n] : 1.f;
                        r = fmaf(p, sa * sb, r);
                    }
                    R = R + r;
                }
                float outer = input_group ? 1.f : sx[m];
                if (!weight_group) outer *= sw[n];
                R = R * outer;
                total = total + R;
            }
            if (y) y[(size_t)m * N + n] = store_out(total, out_type);
            if (y_f32) y_f32[(size_t)m * N + n] = total;
        }
    return 0;
}

/* fp64 ideal of the grouped GEMM for tolerance checks: sum_g p_g*sxg*swg. */
void orc_gemm_grouped_ideal(const uint8_t *x, const float *sx, const uint8_t *w, const float *sw,
                            int M, int N, int K, int fmt, int input_group, int weight_group,
                            float *y) {
    float lut[256];
    for (int i = 0; i < 256; ++i)
        lut[i] = fmt == T_I8 ? (float)(int8_t)i : orc_fp8_decode((uint8_t)i);
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double s = 0;
            for (int k = 0; k < K; ++k) {
                double a = lut[x[(size_t)m * K + k]], b = lut[w[(size_t)n * K + k]];
                a *= input_group ? sx[(size_t)(k / input_group) * M + m] : sx[m];
                b *= weight_group ? sw[(size_t)(k / weight_group) * N + n] : sw[n];
                s += a * b;
            }
            y[(size_t)m * N + n] = (float)s;
        }
}

/* ---------------------------------------------------------------- CPU baseline */
/* Multithreaded quant -> GEMM -> dequant of the whole path (the same work the
 * GPU does per call), used as the reported CPU baseline. INT8 per-channel:
 * int32 dot products vectorised by the compiler; epilogue order 0. FP8:
 * 256-entry decode table, fp32 accumulation. Grouped modes: per-K-group
 * partials as orc_gemm_grouped with one split. */
typedef struct {
    const uint8_t *xq, *wq;
    const float *sx, *sw;
    uint16_t *y;
    int M, N, K, fmt, group, n0, n1, out_type;
    const float *lut;
} job_t;

static void *gemm_job(void *arg) {
    job_t *j = (job_t *)arg;
    int M = j->M, N = j->N, K = j->K, G = j->group;
    /* Blocks of 32 token rows stay cache-resident while the thread's weight
     * rows stream past them; every output is still one dot product in K
     * order. */
    for (int mb = 0; mb < M; mb += 32)
    for (int n = j->n0; n < j->n1; ++n) {
        const uint8_t *b = j->wq + (size_t)n * K;
        for (int m = mb; m < M && m < mb + 32; ++m) {
            const uint8_t *a = j->xq + (size_t)m * K;
            float v;
            if (j->fmt == T_I8 && !G) {
                const int8_t *ai = (const int8_t *)a, *bi = (const int8_t *)b;
                int32_t s = 0;
                for (int k = 0; k < K; ++k) s += (int32_t)ai[k] * (int32_t)bi[k];
                v = (float)s * j->sx[m];
                v = v * j->sw[n];
            } else if (!G) {
                float s = 0;
                for (int k = 0; k < K; ++k) s += j->lut[a[k]] * j->lut[b[k]];
                v = s * j->sx[m];
                v = v * j->sw[n];
            } else {
                float r = 0;
                for (int k0 = 0; k0 < K; k0 += G) {
                    float p;
                    if (j->fmt == T_I8) {
                        const int8_t *ai = (const int8_t *)a, *bi = (const int8_t *)b;
                        int32_t s = 0;
                        for (int k = k0; k < k0 + G; ++k) s += (int32_t)ai[k] * (int32_t)bi[k];
                        p = (float)s;
                    } else {
                        float s = 0;
                        for (int k = k0; k < k0 + G; ++k) s += j->lut[a[k]] * j->lut[b[k]];
                        p = s;
                    }
                    r = fmaf(p, j->sx[(size_t)(k0 / G) * M + m] * j->sw[(size_t)(k0 / G) * N + n], r);
                }
                v = r;
            }
            j->y[(size_t)m * N + n] = store_out(v, j->out_type);
        }
    }
    return NULL;
}

typedef struct {
    const void *src;
    int src_type, ld, r0, r1, rows, cols, fmt, group, rotation;
    uint8_t *q;
    float *scales;
} qjob_t;

static void *quant_job(void *arg) {
    qjob_t *j = (qjob_t *)arg;
    int n = j->r1 - j->r0;
    if (n <= 0) return NULL;
    /* quantize a row slice into a private scale buffer, then scatter */
    int groups = j->group ? (j->cols + j->group - 1) / j->group : 1;
    float *sc = (float *)malloc(sizeof(float) * (size_t)n * groups);
    const uint16_t *s = (const uint16_t *)j->src + (size_t)j->r0 * j->ld;
    orc_quantize_rows(s, j->src_type, j->ld, n, j->cols, j->fmt, j->group, j->rotation,
                      j->q + (size_t)j->r0 * j->cols, sc);
    for (int g = 0; g < groups; ++g)
        for (int r = 0; r < n; ++r)
            j->scales[(size_t)g * (j->group ? j->rows : 0) + j->r0 + r] = sc[(size_t)g * n + r];
    free(sc);
    return NULL;
}

/* One quantized linear call on the CPU: quantize X (bf16 [M,K]) with the
 * mode's activation layout, then GEMM against pre-quantized weights and
 * store bf16/f16. Weight quantization happens at load time in the reference
 * (io/weights.cpp:80-87) and is not part of a call. */
int orc_cpu_qlinear(const void *x, int x_type, int M, int N, int K, const uint8_t *wq,
                    const float *sw, int fmt, int group, int rotation, int out_type,
                    uint16_t *y, uint8_t *xq_scratch, float *sx_scratch, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    qjob_t qj[256];
    int rows_per = (M + threads - 1) / threads;
    int qt = 0;
    for (int t = 0; t < threads; ++t) {
        int r0 = t * rows_per, r1 = r0 + rows_per < M ? r0 + rows_per : M;
        if (r0 >= r1) break;
        qj[t] = (qjob_t){x, x_type, K, r0, r1, M, K, fmt, group, rotation, xq_scratch, sx_scratch};
        pthread_create(&tid[t], NULL, quant_job, &qj[t]);
        ++qt;
    }
    for (int t = 0; t < qt; ++t) pthread_join(tid[t], NULL);
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = orc_fp8_decode((uint8_t)i);
    job_t jobs[256];
    int per = (N + threads - 1) / threads, started = 0;
    for (int t = 0; t < threads; ++t) {
        int n0 = t * per, n1 = n0 + per < N ? n0 + per : N;
        if (n0 >= n1) break;
        jobs[t] = (job_t){xq_scratch, wq, sx_scratch, sw, y, M, N, K, fmt, group, n0, n1, out_type, lut};
        pthread_create(&tid[t], NULL, gemm_job, &jobs[t]);
        ++started;
    }
    for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
    return 0;
}
