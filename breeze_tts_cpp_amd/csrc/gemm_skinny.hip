// Decode-regime quantized GEMM (M <= 64 tokens) for gfx950.
//
// y[M,N] = D(epilogue(x[M,K] . w[N,K]^T)), the work of the reference's small-M
// path quant_gemv (ops/kernels/quant/quant_dispatch.cu:12-130), its split-K
// reduction (quant_reduce.cuh:9-19) and, for K-group scales, grouped_gemm
// (quant_grouped.cu:16-169).
//
// At these shapes the weight matrix is the only large operand: the kernel is
// bound by streaming w from HBM exactly once. Each wave64 owns 16*NF weight
// rows over a K range and issues 16-byte loads (64 lanes = 16 rows x 64
// contiguous bytes per load) straight into MFMA A-fragment registers; the
// tokens are the MFMA B side (zero-padded to 16*MT). INT8 uses
// v_mfma_i32_16x16x64_i8 (exact int32), FP8 e4m3 uses
// v_mfma_f32_16x16x128_f8f6f4 (zero scale operands to the f8f6f4 builtin,
// for which the compiler emits the unscaled instruction). The waves of a
// workgroup split K and reduce through LDS; optionally the grid splits K
// further into workspace partials that a second kernel reduces in split order.
//
// Epilogues (all fp32, no contraction):
//   per-channel : D((acc * sx[m]) * sw[n])      (quant_gemm_sm80.cu:24-29)
//   K-group     : r = fmaf(p_g, sx_g*sw_g, r) per group, groups ascending
//                 (quant_grouped.cu:135-144); ranges summed 0 + r_0 + r_1 ...
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

#include <type_traits>

// Each kernel-variant translation unit is built with or without the fused
// finish (bias + activation epilogue, see finish4); the plain build carries
// no finish code at all.
#ifndef QLIN_FIN
#define QLIN_FIN 0
#endif

namespace qlin {
namespace {

constexpr bool kFin = QLIN_FIN;
constexpr int kBlockK = 256;  // K handled per main-loop iteration (4 pieces of 64)

// f(std::integral_constant<int, I>{}) for I = B .. E-1, each I a constant
// expression in f (for per-step s_waitcnt immediates).
// s_waitcnt vmcnt(n) leaving expcnt / lgkmcnt unconstrained (gfx9 encoding).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int B, int E, class F> __device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

template <int Fmt> struct Mfma;
template <> struct Mfma<I8> {
    using Acc = i32x4;
    using Scalar = int;
    // Two 64-K pieces -> two MFMAs.
    __device__ static void run(Acc &c, const i32x4 &a0, const i32x4 &a1, const i32x4 &b0,
                               const i32x4 &b1) {
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, c, 0, 0, 0);
    }
};
template <> struct Mfma<FP8> {
    using Acc = f32x4;
    using Scalar = float;
    // Two 64-K pieces -> one 128-K MFMA (format 0 = e4m3 for A and B; zero
    // scale operands select the unscaled instruction).
    __device__ static void run(Acc &c, const i32x4 &a0, const i32x4 &a1, const i32x4 &b0,
                               const i32x4 &b1) {
        i32x8 a = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        i32x8 b = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};

__device__ __forceinline__ i32x4 load16(const uint8_t *p) {
    return *reinterpret_cast<const i32x4 *>(p);
}
// Packed-layout weight pieces (read once per step) are loaded non-temporally:
// M = 32 INT8 packed GEMMs measured 4-7% faster (gate_up 9.52 -> 8.81 us).
// The unstaged row-major register path keeps plain loads (gate_up 11.86 ->
// 12.81 us with non-temporal ones).
__device__ __forceinline__ i32x4 load16_packed(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(p));
}

// Four 16-byte LDS reads by explicit ds_read_b128 instructions and their
// wait, in one statement. The compiler's wait insertion treats any LDS read
// as possibly reading what an outstanding global->LDS copy writes and then
// waits for every outstanding vector load; reads of a region whose copy the
// caller has already waited for (counted vmcnt) go through this path so that
// later copies, still in flight, are not waited for. The wait is inside the
// statement because the compiler does not know these reads are pending: no
// instruction may consume the results before it.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) {
    typedef __attribute__((address_space(3))) const uint8_t *lds_cptr_t;
    return uint32_t(reinterpret_cast<uintptr_t>((lds_cptr_t)p));
}
__device__ __forceinline__ void lds_read16x4(const uint8_t *p0, const uint8_t *p1,
                                             const uint8_t *p2, const uint8_t *p3, i32x4 &v0,
                                             i32x4 &v1, i32x4 &v2, i32x4 &v3) {
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\t"
        "ds_read_b128 %3, %7\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
        : "v"(lds_addr(p0)), "v"(lds_addr(p1)), "v"(lds_addr(p2)), "v"(lds_addr(p3)));
}

// Cache policy of the weight slab DMA: non-temporal (the buffer
// instruction's nt bit). Decode weights are read once per step, so keeping
// them out of the caches' retained lines measured 4-6% faster per decode GEMM
// (gate_up INT8 M = 32: 7.50 -> 7.09 us) than the default policy; sc0 alone
// changed nothing. (Non-temporal output stores measured slower: o_proj
// 3.36 -> 3.57 us.)
constexpr int kWeightAux = 2;

template <class Out>
__device__ __forceinline__ void store4(void *y, size_t index, const float (&v)[4]) {
    uint2 packed;
    packed.x = pack2(v[0], v[1], Out{});
    packed.y = pack2(v[2], v[3], Out{});
    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + index) = packed;
}

// Four consecutive outputs of one row: the finish (finish TUs only), then the
// store in the output type, chosen at run time (a uniform branch at the end
// of the kernel, so one kernel serves bf16 and f16 outputs).
__device__ __forceinline__ void store_out(void *y, size_t index, float (&v)[4],
                                          const uint16_t *bias, int n, int n_last, int act,
                                          int out_f16) {
    if (out_f16) {
        if constexpr (kFin) finish4<f16_t>(v, bias, n, n_last, act);
        store4<f16_t>(y, index, v);
    } else {
        if constexpr (kFin) finish4<bf16_t>(v, bias, n, n_last, act);
        store4<bf16_t>(y, index, v);
    }
}

// One workgroup = WK waves over K, sharing 16*NF weight rows; tokens
// [m0, m0 + 16*MT). Split: store raw (per-channel) or outer-scaled (grouped)
// partials to workspace[blockIdx.y] instead of the output.
// NB > 0: each wave's weight slab (16*NF rows x NB*256 bytes of K) is first
// copied global -> LDS with buffer_load ... lds in one shot. Each load
// instruction moves 1 KB of consecutive (row, 16-byte granule) positions of
// the slab, so every instruction reads whole 256-byte (or longer) runs of a
// weight row instead of 64-byte pieces of 16 rows. Granule g of slab row r
// is stored at slot g ^ (r & 15) (the lane's global source is permuted, the
// LDS write stays linear), which keeps the MFMA fragment reads (16 rows, one
// granule) on distinct banks. Each wave reads back only what it loaded, so
// no workgroup barrier is needed. NB == 0: weights load straight to registers.
//
// Packed: w is the packed fragment-tile layout (weight_pack.hip); each wave
// loads all NB blocks of its K range straight into registers up front, one
// contiguous 1 KB piece per (16-row fragment, 64-K step).
template <int Fmt, int MT, int NF, int WK, bool Grouped, bool Split, int NB = 0,
          bool Packed = false, int FQ = 0, int GS = 128, bool XL = false>
__global__ __launch_bounds__(64 * WK) void skinny_gemm(
    const uint8_t *__restrict__ x, const float *__restrict__ sx, const uint8_t *__restrict__ w,
    const float *__restrict__ sw, void *__restrict__ y, void *__restrict__ partial, int M, int N,
    int K, int span, int input_group, int weight_group, const uint16_t *__restrict__ bias,
    int act, int out_f16, FusedSource fq) {
    using M_ = Mfma<Fmt>;
    using Acc = typename M_::Acc;
    using Scalar = typename M_::Scalar;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row16 = lane & 15, quad = lane >> 4;
    const int n0 = blockIdx.x * 16 * NF;
    const int m0 = blockIdx.z * 16 * MT;
    const int range = blockIdx.y * WK + wave;
    const int k_begin = range * span;
    const int k_end = min(K, k_begin + span);

    const uint8_t *wrow[NF];
    bool wvalid[NF];
    const int tiles_k = (K + 63) / 64;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        int n = n0 + f * 16 + row16;
        wvalid[f] = n < N;
        if constexpr (Packed)
            wrow[f] = w + size_t(wvalid[f] ? n0 / 16 + f : 0) * tiles_k * 1024 + lane * 16;
        else
            wrow[f] = w + size_t(wvalid[f] ? n : 0) * K + quad * 16;
    }
    const uint8_t *xrow[MT];
    bool xvalid[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        int m = m0 + t * 16 + row16;
        xvalid[t] = m < M;
        xrow[t] = x + size_t(xvalid[t] ? m : 0) * K + quad * 16;
    }

    // Epilogue scales, loaded before anything else so that their latency hides
    // under the weight stream instead of following the reduction. Thread
    // unit u = threadIdx.x + k*64*WK covers (token tile, fragment, lane) with
    // four output channels; the factors are the ones the epilogue applies
    // (K-group scales enter per group instead, leaving a factor of 1).
    constexpr int kUnits = MT * NF * 64;  // (token tile, fragment, lane), 4 values each
    constexpr int kMaxU = (kUnits + 64 * WK - 1) / (64 * WK);
    float pre_x[kMaxU];
    f32x4 pre_w[kMaxU];
#pragma unroll
    for (int k = 0; k < kMaxU; ++k) {
        const int u = threadIdx.x + k * 64 * WK;
        const int tf = u >> 6, l = u & 63;
        const int m = m0 + (tf / NF) * 16 + (l & 15);
        const int n = n0 + (tf % NF) * 16 + (l >> 4) * 4;
        const bool live = u < kUnits && m < M && n < N;
        // FQ: sx is produced by this kernel; the factor comes from LDS below.
        pre_x[k] = (live && !(Grouped && input_group) && !FQ) ? sx[m] : 1.f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            pre_w[k][r] = (live && !(Grouped && weight_group)) ? sw[n + r] : 1.f;
    }

    // K groups of 128 on a staged slab: every group scale of this wave's K
    // range (two groups per 256-column block) is requested here, ahead of the
    // slab, instead of when its block's MFMAs run after the slab has landed.
    constexpr bool kPreScale = Grouped && GS == 128 && NB > 0 && NB * MT <= 6 && !Packed;
    float pre_sw[kPreScale ? NB : 1][2][NF][4];
    float pre_sx[kPreScale ? NB : 1][2][MT];
    if constexpr (kPreScale) {
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int k = k_begin + blk * kBlockK + h * 128;
                const bool kin = k < k_end;
                const int g = k / 128;
#pragma unroll
                for (int f = 0; f < NF; ++f)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = n0 + f * 16 + quad * 4 + r;
                        pre_sw[blk][h][f][r] =
                            (kin && weight_group && n < N) ? sw[size_t(g) * N + n] : 1.f;
                    }
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const int m = m0 + t * 16 + row16;
                    // (FQ: computed from the 16-bit rows below)
                    pre_sx[blk][h][t] = (kin && input_group && m < M && !FQ) ? sx[size_t(g) * M + m] : 1.f;
                }
            }
    }

    // FQ: the 16-bit activation fragments of every block of this wave's K
    // range, requested before the weight slab so that they land first. Lane
    // (row16, quad) of token tile t holds K columns [kb + 64p + 16q, +16) of
    // row m0 + 16t + row16: exactly the codes its MFMA B fragments need.
    static_assert(!FQ || (NB > 0 && !Packed && !Split && NB * MT <= 3 &&
                          (!Grouped || (GS == 128 && NB == 1))),
                  "fused quantization: per-wave slab, activation blocks in registers");
    uint4 xraw[FQ ? NB : 1][MT][4][2];
    if constexpr (FQ && !XL) {
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int k = k_begin + blk * kBlockK + p * 64 + quad * 16;
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const int m = m0 + t * 16 + row16;
                    if (k < k_end && xvalid[t]) {
                        const uint4 *src = reinterpret_cast<const uint4 *>(
                            fq.src + size_t(m) * fq.ld + k);
                        xraw[blk][t][p][0] = src[0];
                        xraw[blk][t][p][1] = src[1];
                    } else {
                        xraw[blk][t][p][0] = xraw[blk][t][p][1] = uint4{0, 0, 0, 0};
                    }
                }
            }
    }

    // Activation fragments of block kb: lane quad q holds K bytes [kb + 64p + 16q, +16).
    auto load_x = [&](int kb, i32x4 (&b)[MT][4]) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int k = kb + p * 64;
            const bool in = k + quad * 16 < k_end;
#pragma unroll
            for (int t = 0; t < MT; ++t)
                b[t][p] = (in && xvalid[t]) ? load16(xrow[t] + k) : i32x4{0, 0, 0, 0};
        }
    };
    // With a staged slab of NB blocks, all of the wave's activation blocks are
    // requested up front (when they fit in registers), ahead of the slab
    // DMA, so no block waits for its own L2 round trip inside the loop.
    constexpr bool kPreX = NB > 0 && NB * MT <= 6 && !Packed;
    i32x4 wpre[1][NF][4];  // unused unless packed
    i32x4 xpre[kPreX && (FQ || !XL) ? NB : 1][MT][4];
    // Staged slabs are consumed chunk by chunk as they arrive (counted
    // waits): the activation is then in LDS (XL), encoded from the 16-bit
    // rows (FQ), or loaded into registers ahead of the slab (kPipeAct).
    constexpr bool kPipeAct = NB > 0 && !Packed && !XL && !FQ && kPreX;
    constexpr bool kPipe = NB > 0 && !Packed && (XL || FQ || kPipeAct);

    // Dynamic LDS: the waves' weight slabs, then (XL) their activation
    // tiles, then (FQ) the row absmax / scale exchange.
    extern __shared__ __attribute__((aligned(1024))) uint8_t wlds[];
    constexpr int SNB = Packed ? 0 : NB;                        // staged slab blocks
    constexpr int kSlabBytes = 16 * NF * SNB * kBlockK;         // per wave
    constexpr int kRowBytes = SNB * kBlockK;
    // XL: the wave's activation rows (16*MT tokens x its K range; 16-bit
    // source rows for FQ) are staged through LDS like the weights.
    static_assert(!XL || (SNB > 0 && !Split), "activation staging needs the weight slab");
    constexpr int kXElem = FQ ? 2 : 1;
    constexpr int kActRowBytes = kRowBytes * kXElem;
    constexpr int kActBytes = XL ? 16 * MT * kActRowBytes : 0;  // per wave
    uint8_t *slab = wlds + wave * kSlabBytes;
    uint8_t *xtile = wlds + WK * kSlabBytes + wave * kActBytes;
    float *fq_amax = reinterpret_cast<float *>(wlds + WK * (kSlabBytes + kActBytes));
    float *fq_scale = fq_amax + WK * MT * 16;
    const int slab_k0 = k_begin;
    if constexpr (SNB > 0) {
        typedef __attribute__((address_space(3))) void *lds_ptr_t;
        if constexpr (XL) {
            // Activation rows first (L2-resident, they land before the
            // weights): each instruction moves 1 KB of consecutive (row,
            // granule) positions, granule g of row r at slot g ^ (r & 15), as
            // the weight slab. Bytes past the range read as zero (offset out
            // of the buffer).
            const int xrows = max(0, min(16 * MT, M - m0));
            const uint8_t *xbase = FQ ? reinterpret_cast<const uint8_t *>(fq.src + size_t(m0) * fq.ld)
                                      : x + size_t(m0) * K;
            const uint32_t xstride = FQ ? uint32_t(fq.ld) * 2u : uint32_t(K);
            const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint8_t *>(xbase), 0, xrows * xstride, 0x00020000);
            constexpr int kActGranules = kActRowBytes / 16;
#pragma unroll
            for (int i = 0; i < kActBytes / 1024; ++i) {
                const int q = i * 64 + lane;
                const int r = q / kActGranules, slot = q % kActGranules;
                const int g = slot ^ (r & 15);
                const int kb = k_begin * kXElem + g * 16;  // byte column
                const uint32_t off = kb < k_end * kXElem ? uint32_t(r) * xstride + uint32_t(kb)
                                                         : 0x80000000u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr_t)(xtile + i * 1024), 16,
                                                         off, 0, 0, 0);
            }
            // Keep the weight DMA behind it (FQ counts the slab's loads).
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
        const int rows_valid = max(0, min(16 * NF, N - n0));
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(w + size_t(n0) * K), 0, rows_valid * K, 0x00020000);
        const int k_stop = k_end;
        // Chunk-major slab: chunk c = blk * NF + f holds weight rows
        // [16f, 16f + 16) x K bytes [256 blk, +256) of the wave's range, 4 KB
        // in 4 instructions of 4 whole 256-byte row runs; granule g of chunk
        // row r sits at slot g ^ r. The MFMAs consume the chunks in
        // instruction order while later ones are still arriving.
        if constexpr (kPipeAct) {
            // The activation blocks in registers, requested before the slab
            // so that the chunk waits below count only slab instructions.
#pragma unroll
            for (int blk = 0; blk < NB; ++blk) load_x(k_begin + blk * kBlockK, xpre[blk]);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int i = 0; i < kSlabBytes / 1024; ++i) {
            const int c = i / 4, blk = c / NF, f = c % NF;
            const int r = (i % 4) * 4 + lane / 16, slot = lane % 16;
            const int g = slot ^ r;
            const int k = slab_k0 + blk * kBlockK + g * 16;
            const uint32_t off = k < k_stop ? uint32_t(f * 16 + r) * uint32_t(K) + uint32_t(k)
                                            : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsrc, (lds_ptr_t)(slab + i * 1024), 16, off,
                0, 0, kWeightAux);
        }
    }

    // Cross-wave reduction: each wave stores its partial sums of unit (tf, l)
    // as four consecutive values, and the epilogue adds the slots in ascending
    // wave (= K) order. With a staged slab the slots reuse it: a slot is
    // MT*NF KB, never more than a wave's slab (16*NF*NB*256 bytes, MT <= 4 <=
    // 4*NB); with no slab they live in a static buffer.
    using Red = std::conditional_t<Grouped, float, Scalar>;
    typedef Red Red4 __attribute__((ext_vector_type(4)));
    constexpr int kSlotVals = MT * NF * 64 * 4;
    constexpr int kSlotStride = SNB > 0 ? kSlabBytes / int(sizeof(Red)) : kSlotVals;
    static_assert(SNB == 0 || kSlotVals * int(sizeof(Red)) <= kSlabBytes, "slot fits the slab");
    Red *red;
    if constexpr (SNB > 0) {
        red = reinterpret_cast<Red *>(wlds);
    } else {
        __shared__ Red4 red_static[WK == 1 ? 1 : WK * kSlotVals / 4];
        red = reinterpret_cast<Red *>(red_static);
    }

    // INT8 K groups of 128 on a staged slab accumulate in the reference's
    // order (quant_grouped.cu:112-146, one K range): r = fmaf(p_g, sx_g *
    // sw_g, r) over every group of K in ascending order, starting from 0.
    // Each wave keeps the exact int32 partial p_g of each of its groups in
    // registers (gp); after the main loop the partials and the group scales
    // go through LDS and the epilogue runs the whole chain per output.
    constexpr bool kRO = Grouped && Fmt == I8 && GS == 128 && kPreScale && WK > 1 && !Split;
    Acc gp[kRO ? NB : 1][2][kRO ? MT : 1][kRO ? NF : 1];
    if constexpr (kRO) {
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int f = 0; f < NF; ++f) gp[blk][h][t][f] = Acc{0, 0, 0, 0};
    }

    // Grouped: fp32 running sums; per-channel: the raw accumulator.
    Acc acc[MT][NF];
    float facc[MT][NF][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            acc[t][f] = Acc{0, 0, 0, 0};
#pragma unroll
            for (int r = 0; r < 4; ++r) facc[t][f][r] = 0.f;
        }

    // XL: the activation fragments of block kb from the staged tile.
    auto xfrag = [&](int kb, i32x4 (&b)[MT][4]) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint8_t *row = xtile + (t * 16 + row16) * kActRowBytes;
            const int g0 = (kb - slab_k0) / 16 + quad;
            lds_read16x4(row + ((g0 ^ row16) << 4), row + (((g0 + 4) ^ row16) << 4),
                         row + (((g0 + 8) ^ row16) << 4), row + (((g0 + 12) ^ row16) << 4),
                         b[t][0], b[t][1], b[t][2], b[t][3]);
        }
    };
    float fq_group_scale[MT][2];  // FQ, K groups: this wave's two group scales per token tile
    if constexpr (FQ) {
        // The per-token quantizer's arithmetic (row_quantize.hip
        // token_quantize; reference row_quantize.cu:24-87): row absmax over
        // all K (this wave's range, its four lane quads, then the WK waves
        // through LDS), scale = quant_scale(amax), codes = encode(v * (1 /
        // scale)). Max is order-free, so the codes and scales are the
        // quantizer's bit for bit.
        // Wait until at most the slab DMA's instructions are outstanding, so
        // the activation rows are in while the slab is still in flight.
        // Without XL this is a scheduling hint only (the compiler may order
        // the loads differently; correctness rests on its own waits before
        // xraw is used and on the vmcnt(0) before the slab is read). With XL
        // it is the wait for the activation DMA, which was issued, in
        // program order and unconditionally, before the slab's ns
        // instructions, with no vector memory access after them.
        constexpr int ns = kSlabBytes / 1024;
        __builtin_amdgcn_s_waitcnt((ns & 15) | ((ns >> 4) << 14) | (7 << 4) | (15 << 8));
        if constexpr (XL) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int p = 0; p < 4; p += 2) {
                        // granules of pieces p and p + 1, halves 0 and 1
                        const uint8_t *row = xtile + (t * 16 + row16) * kActRowBytes;
                        const int g = blk * 32 + p * 8 + quad * 2;
                        i32x4 r[4];
                        lds_read16x4(row + ((g ^ row16) << 4), row + (((g + 1) ^ row16) << 4),
                                     row + (((g + 8) ^ row16) << 4), row + (((g + 9) ^ row16) << 4),
                                     r[0], r[1], r[2], r[3]);
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            xraw[blk][t][p + q / 2][q % 2] =
                                uint4{uint32_t(r[q][0]), uint32_t(r[q][1]), uint32_t(r[q][2]),
                                      uint32_t(r[q][3])};
                    }
        }
        // FQ 1: bf16 source, 2: f16 source.
        using Tin = std::conditional_t<FQ == 2, f16_t, bf16_t>;
        auto widen = [](uint32_t h) { return to_float(uint16_t(h), Tin{}); };
        if constexpr (Grouped) {
            // K groups of 128, not rotated (reference group_token_quantize,
            // row_quantize.cu:145-165, with encode_group,
            // quant_device.cuh:63-88): a wave's 256-column block is two whole
            // groups, so no other wave is involved. Lane (row16, quad) holds,
            // per group g, columns 64p' + 16 quad + 8h + i (pieces p = 2g +
            // p', halves h, elements i): the group amax (fmaxf, order-free)
            // over the lane's 32 values and lanes xor 16, 32, scale =
            // quant_scale(amax), codes = encode(v * (1 / scale)), bit for bit
            // the group quantizer's. (With the H128 rotation, re-encoding in
            // every workgroup costs more than the separate quantizer: qkv at
            // M = 32 took 11.9 us in one launch against 8.5 us in two.)
            static_assert(NB == 1, "two 128-groups per wave");
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                float v[4][2][8];
#pragma unroll
                for (int p = 0; p < 4; ++p)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t wd[4] = {xraw[0][t][p][h].x, xraw[0][t][p][h].y,
                                                xraw[0][t][p][h].z, xraw[0][t][p][h].w};
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            v[p][h][2 * i] = widen(wd[i] & 0xffffu);
                            v[p][h][2 * i + 1] = widen(wd[i] >> 16);
                        }
                    }
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    float a = 0.f;
#pragma unroll
                    for (int p = 2 * g; p < 2 * g + 2; ++p)
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(v[p][h][i]));
                    a = fmaxf(a, lane_xor<16>(a));
                    a = fmaxf(a, lane_xor<32>(a));
                    const float step = quant_scale<Fmt>(a);
                    const float inverse = 1.f / step;
                    fq_group_scale[t][g] = step;
#pragma unroll
                    for (int p = 2 * g; p < 2 * g + 2; ++p) {
                        i32x4 codes;
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int j = 0; j < 2; ++j) {
                                const float *e = &v[p][h][4 * j];
                                if constexpr (Fmt == I8)
                                    codes[2 * h + j] = int(encode_i8x4(e[0] * inverse, e[1] * inverse,
                                                                       e[2] * inverse, e[3] * inverse));
                                else
                                    codes[2 * h + j] = int(encode_fp8x4(e[0] * inverse, e[1] * inverse,
                                                                        e[2] * inverse, e[3] * inverse));
                            }
                        const int k = k_begin + p * 64 + quad * 16;
                        const bool in = k < k_end && xvalid[t];
                        xpre[0][t][p] = in ? codes : i32x4{0, 0, 0, 0};
                    }
                    if constexpr (kPreScale) pre_sx[0][g][t] = step;
                }
            }
        } else {
            // |v| of a 16-bit float orders as its sign-cleared bits, so the
            // absmax is a packed unsigned 16-bit max of the bits; a NaN (bits
            // above the infinity pattern) makes the lane redo its values with
            // fmaxf, which ignores NaN as the quantizer's reduction does.
            constexpr uint32_t kInfBits = FQ == 2 ? 0x7c00u : 0x7f80u;
            typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
            float amax[MT];
            // FP8: per token tile, this lane's values are all finite. Then every
            // v * inverse is below 464 in magnitude, where the hardware
            // conversion equals encode_fp8 (encode_fp8x4): with the row's absmax
            // a finite, scale = max(a / 448, FLT_MIN) and inverse = 1 / scale
            // (both rounded to nearest) keep |v * inverse| <= 448 * (1 + 2^-24)^3
            // for |v| <= a (or |v| * 2^126 < 448 exactly); with a = Inf the
            // inverse is 0.
            bool finite[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                u16x2 top = {0, 0};
#pragma unroll
                for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                    for (int p = 0; p < 4; ++p)
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const uint32_t wd[4] = {xraw[blk][t][p][h].x, xraw[blk][t][p][h].y,
                                                    xraw[blk][t][p][h].z, xraw[blk][t][p][h].w};
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                top = __builtin_elementwise_max(
                                    top, __builtin_bit_cast(u16x2, wd[i] & 0x7fff7fffu));
                        }
                const uint32_t bits = top.x > top.y ? top.x : top.y;
                finite[t] = bits < kInfBits;
                if (bits <= kInfBits) {
                    amax[t] = widen(bits);
                } else {
                    amax[t] = 0.f;
#pragma unroll
                    for (int blk = 0; blk < NB; ++blk)
                        for (int p = 0; p < 4; ++p)
                            for (int h = 0; h < 2; ++h) {
                                const uint32_t wd[4] = {xraw[blk][t][p][h].x, xraw[blk][t][p][h].y,
                                                        xraw[blk][t][p][h].z, xraw[blk][t][p][h].w};
                                for (int i = 0; i < 4; ++i) {
                                    amax[t] = fmaxf(amax[t], fabsf(widen(wd[i] & 0xffffu)));
                                    amax[t] = fmaxf(amax[t], fabsf(widen(wd[i] >> 16)));
                                }
                            }
                }
                amax[t] = fmaxf(amax[t], lane_xor<16>(amax[t]));
                amax[t] = fmaxf(amax[t], lane_xor<32>(amax[t]));
                if (quad == 0) fq_amax[wave * MT * 16 + t * 16 + row16] = amax[t];
            }
            // A workgroup barrier that waits for LDS only: __syncthreads' fence
            // would also wait for the weight slab DMA still in flight.
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                float a = fq_amax[t * 16 + row16];
#pragma unroll
                for (int q = 1; q < WK; ++q) a = fmaxf(a, fq_amax[q * MT * 16 + t * 16 + row16]);
                const float step = quant_scale<Fmt>(a);
                const float inverse = 1.f / step;
                if (wave == 0 && quad == 0) fq_scale[t * 16 + row16] = step;
#pragma unroll
                for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        i32x4 codes;
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const uint32_t wd[4] = {xraw[blk][t][p][h].x, xraw[blk][t][p][h].y,
                                                    xraw[blk][t][p][h].z, xraw[blk][t][p][h].w};
#pragma unroll
                            for (int j = 0; j < 2; ++j) {
                                if constexpr (Fmt == I8) {
                                    codes[2 * h + j] = int(encode_i8x4(
                                        widen(wd[2 * j] & 0xffffu) * inverse,
                                        widen(wd[2 * j] >> 16) * inverse,
                                        widen(wd[2 * j + 1] & 0xffffu) * inverse,
                                        widen(wd[2 * j + 1] >> 16) * inverse));
                                    continue;
                                }
                                const float v0 = widen(wd[2 * j] & 0xffffu) * inverse;
                                const float v1 = widen(wd[2 * j] >> 16) * inverse;
                                const float v2 = widen(wd[2 * j + 1] & 0xffffu) * inverse;
                                const float v3 = widen(wd[2 * j + 1] >> 16) * inverse;
                                codes[2 * h + j] = int(finite[t] ? encode_fp8x4_inrange(v0, v1, v2, v3)
                                                                 : encode_fp8x4(v0, v1, v2, v3));
                            }
                        }
                        // Columns past the range (or rows past M) encode zeros,
                        // as the zero-filled plain activation loads.
                        const int k = k_begin + blk * kBlockK + p * 64 + quad * 16;
                        const bool in = k < k_end && xvalid[t];
                        xpre[blk][t][p] = in ? codes : i32x4{0, 0, 0, 0};
                    }
            }
        }
    }

    // MFMAs of block kb for fragment fsel (all fragments when fsel < 0;
    // fsel is a constant at every call, so the guards fold away).
    auto block = [&](int kb, const i32x4 (&b)[MT][4], const i32x4 (&wp)[NF][4], int fsel) {
        i32x4 a[NF][4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int k = kb + p * 64;
            const bool in = k + quad * 16 < k_end;
            (void)in;
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                if (fsel >= 0 && f != fsel) continue;
                if constexpr (Packed) {
                    a[f][p] = wp[f][p];
                } else if constexpr (NB > 0) {
                    const int chunk = ((kb - slab_k0) / kBlockK) * NF + f;
                    const int g = p * 4 + quad;
                    a[f][p] = *reinterpret_cast<const i32x4 *>(slab + chunk * 4096 + row16 * 256 +
                                                               ((g ^ row16) << 4));
                } else {
                    a[f][p] = (in && wvalid[f]) ? load16(wrow[f] + k) : i32x4{0, 0, 0, 0};
                }
            }
        }
        if constexpr (!Grouped) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int f = 0; f < NF; ++f)
                        if (fsel < 0 || f == fsel)
                            M_::run(acc[t][f], a[f][2 * h], a[f][2 * h + 1], b[t][2 * h],
                                    b[t][2 * h + 1]);
        } else if constexpr (GS == 128) {
            // Two 128-K groups per block, each reduced natively then scaled.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int k = kb + h * 128;
                if (k >= k_end) break;
                const int g_in = input_group ? k / input_group : 0;
                const int g_w = weight_group ? k / weight_group : 0;
                // with kPreScale, blk is a constant once the block loop is unrolled
                const int blk = kPreScale ? (kb - k_begin) / kBlockK : 0;
                float swg[NF][4];
#pragma unroll
                for (int f = 0; f < NF; ++f)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (fsel >= 0 && f != fsel) continue;
                        int n = n0 + f * 16 + quad * 4 + r;
                        if constexpr (kPreScale) swg[f][r] = pre_sw[blk][h][f][r];
                        else swg[f][r] = (weight_group && n < N) ? sw[size_t(g_w) * N + n] : 1.f;
                    }
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    int m = m0 + t * 16 + row16;
                    float sxg;
                    if constexpr (kPreScale) sxg = pre_sx[blk][h][t];
                    else sxg = (input_group && m < M) ? sx[size_t(g_in) * M + m] : 1.f;
#pragma unroll
                    for (int f = 0; f < NF; ++f) {
                        if (fsel >= 0 && f != fsel) continue;
                        Acc p = Acc{0, 0, 0, 0};
                        M_::run(p, a[f][2 * h], a[f][2 * h + 1], b[t][2 * h], b[t][2 * h + 1]);
                        if constexpr (kRO) {
                            gp[blk][h][t][f] = p;
                            continue;
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            facc[t][f][r] =
                                __builtin_fmaf(float(p[r]), sxg * swg[f][r], facc[t][f][r]);
                    }
                }
            }
        } else {
            // K groups of GS = 64 or 32 (the smaller of the two group sizes,
            // as the reference's grouped_gemm dispatch, quant_grouped.cu:
            // 185-202): each group reduced natively, then
            // r = fmaf(p_g, sx_g * sw_g, r), groups ascending. A 64-K piece
            // holds K bytes [16q, 16q + 16) in lane quad q of both operands,
            // so a 32-K group is the piece with the other half's activation
            // quads zeroed; a 64-K group of FP8 is the 128-K MFMA with the
            // second piece zeroed.
            const i32x4 zero = {0, 0, 0, 0};
            // One group starting at K = k: scales, then per (token tile,
            // fragment) the native partial from `part` and the fma.
            auto group = [&](int k, auto part) {
                const int g_in = input_group ? k / input_group : 0;
                const int g_w = weight_group ? k / weight_group : 0;
                float swg[NF][4];
#pragma unroll
                for (int f = 0; f < NF; ++f)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (fsel >= 0 && f != fsel) continue;
                        int n = n0 + f * 16 + quad * 4 + r;
                        swg[f][r] = (weight_group && n < N) ? sw[size_t(g_w) * N + n] : 1.f;
                    }
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    int m = m0 + t * 16 + row16;
                    float sxg = (input_group && m < M) ? sx[size_t(g_in) * M + m] : 1.f;
#pragma unroll
                    for (int f = 0; f < NF; ++f) {
                        if (fsel >= 0 && f != fsel) continue;
                        const Acc p = part(t, f);
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            facc[t][f][r] =
                                __builtin_fmaf(float(p[r]), sxg * swg[f][r], facc[t][f][r]);
                    }
                }
            };
            // Partial over one 64-K piece of the activation fragment bq.
            auto piece = [&](const i32x4 &aq, const i32x4 &bq) {
                Acc p = Acc{0, 0, 0, 0};
                if constexpr (Fmt == I8) p = __builtin_amdgcn_mfma_i32_16x16x64_i8(aq, bq, p, 0, 0, 0);
                else M_::run(p, aq, zero, bq, zero);
                return p;
            };
            if constexpr (GS == 64) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int k = kb + q * 64;
                    if (k >= k_end) break;
                    group(k, [&](int t, int f) { return piece(a[f][q], b[t][q]); });
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int half = 0; half < 2; ++half) {
                        const int k = kb + q * 64 + half * 32;
                        if (k >= k_end) break;
                        const bool mine = (quad >> 1) == half;
                        group(k, [&](int t, int f) {
                            return piece(a[f][q], mine ? b[t][q] : zero);
                        });
                    }
            }
        }
    };
    if constexpr (Packed) {
        // Chunks of NB blocks: every weight fragment and activation block of
        // a chunk is requested before its first MFMA.
        for (int kc = k_begin; kc < k_end; kc += NB * kBlockK) {
            i32x4 wc[NB][NF][4], xc[NB][MT][4];
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int k = kc + blk * kBlockK + p * 64;
#pragma unroll
                    for (int f = 0; f < NF; ++f)
                        wc[blk][f][p] = (k < k_end && wvalid[f])
                                            ? load16_packed(wrow[f] + size_t(k / 64) * 1024)
                                            : i32x4{0, 0, 0, 0};
                }
#pragma unroll
            for (int blk = 0; blk < NB; ++blk) load_x(kc + blk * kBlockK, xc[blk]);
#pragma unroll
            for (int blk = 0; blk < NB; ++blk) {
                const int kb = kc + blk * kBlockK;
                if (kb < k_end) block(kb, xc[blk], wc[blk], -1);
            }
        }
    } else if constexpr (kPreX) {
        // Chunk c = blk * NF + f of the slab is complete once at most the
        // 4 * (NB * NF - c - 1) slab instructions after it are outstanding:
        // every vector memory operation older than the slab (scales,
        // activation DMA or loads) completes first, and any issued later
        // (K-group scales) only makes the count stricter.
        static_assert(kPipe, "staged register-resident activations are consumed per chunk");
        // K groups of 32 / 64 consume whole blocks (their group scales are
        // loaded per block; per fragment they would be loaded NF times);
        // 128-group scales are prefetched, so those kernels go chunk by
        // chunk like the per-channel ones.
        constexpr bool kWhole = Grouped && !kPreScale;
        constexpr int kStep = kWhole ? NF : 1;
        i32x4 xb[MT][4];
        static_for<0, NB * NF / kStep>([&](auto c_) {
            constexpr int c = decltype(c_)::value * kStep;
            constexpr int blk = c / NF, f = kWhole ? -1 : c % NF;
            wait_vmcnt<4 * (NB * NF - c - kStep)>();
            const int kb = k_begin + blk * kBlockK;
            if (kb < k_end) {
                if constexpr (XL && !FQ) {
                    if constexpr (f <= 0) xfrag(kb, xb);
                    block(kb, xb, wpre[0], f);
                } else {
                    block(kb, xpre[blk], wpre[0], f);
                }
            }
        });
        if constexpr (FQ) {
            // The scratch activation is filled after the MFMAs, so that the
            // stores do not delay the slab waits, and spread over column
            // tiles so that no workgroup carries all of it: wave w's K range
            // of this token tile is written by column tile w % (column
            // tiles), the scales by column tile 0.
            if (int(blockIdx.x) == wave % int(gridDim.x)) {
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const int m = m0 + t * 16 + row16;
                    if (!xvalid[t]) continue;
                    if constexpr (Grouped) {
                        // scales [K/128, M]: this wave's two groups
                        if (quad == 0)
                            for (int g = 0; g < 2; ++g)
                                if (k_begin + g * 128 < k_end)
                                    fq.sx[size_t(k_begin / 128 + g) * M + m] = fq_group_scale[t][g];
                    } else {
                        if (blockIdx.x == 0 && wave == 0 && quad == 0) fq.sx[m] = fq_scale[t * 16 + row16];
                    }
#pragma unroll
                    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                        for (int p = 0; p < 4; ++p) {
                            const int k = k_begin + blk * kBlockK + p * 64 + quad * 16;
                            if (k < k_end)
                                *reinterpret_cast<i32x4 *>(fq.xq + size_t(m) * K + k) = xpre[blk][t][p];
                        }
                }
            }
        }
    } else {
        for (int kb = k_begin; kb < k_end; kb += kBlockK) {
            i32x4 b[MT][4];
            if constexpr (!XL) load_x(kb, b);
            if constexpr (NB > 0) {
                // The slab is in LDS once no load is outstanding.
                if (kb == k_begin) {
                    __builtin_amdgcn_s_waitcnt((0) | (7 << 4) | (15 << 8));
                }
            }
            if constexpr (XL) xfrag(kb, b);
            block(kb, b, wpre[0], -1);
        }
    }


    if constexpr (kRO) {
        // The reference-order chain. Per pass of kTP token tiles, the waves
        // put their groups' terms in LDS (the slab and activation tiles are
        // no longer read): PS[group][unit][r] = (float(p_g), sx_g * sw_g)
        // for unit = (tile, fragment, lane) of the MFMA layout, the scale
        // product computed as the reference does (activation scale times
        // weight scale, quant_grouped.cu:133) and the int32 partial
        // converted exactly (|p| < 2^22). Group g of the workgroup is wave
        // g / (2 NB), block (g / 2) % NB, half g % 2: ascending K. Then one
        // thread per output runs r = fmaf(p_g, s_g, r) over every group.
        constexpr int kGL = WK * 2 * NB;
        constexpr int kAvail = WK * (kSlabBytes + kActBytes);
        constexpr int kTP = kGL * MT * NF * 2048 <= kAvail ? MT
                            : (MT % 2 == 0 && kGL * (MT / 2) * NF * 2048 <= kAvail) ? MT / 2
                                                                                   : 1;
        static_assert(kGL * kTP * NF * 2048 <= kAvail, "chain terms fit the slab");
        constexpr int kUP = kTP * NF * 64;
        constexpr int kPasses = MT / kTP, kIters = (kUP * 4 + 64 * WK - 1) / (64 * WK);
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        f32x2 *PS = reinterpret_cast<f32x2 *>(wlds);
        // LDS-only barrier (builtins, so that the compiler's wait insertion
        // does not also wait for outstanding global memory operations).
        auto lds_barrier = [] {
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
        };
        float res[kPasses][kIters];
#pragma unroll
        for (int pass = 0; pass < kPasses; ++pass) {
            const int t0 = pass * kTP;
            // Every wave is done with the slab (first pass) or with the
            // previous pass's terms.
            lds_barrier();
#pragma unroll
            for (int blk = 0; blk < NB; ++blk)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int g = wave * 2 * NB + blk * 2 + h;
#pragma unroll
                    for (int tl = 0; tl < kTP; ++tl)
#pragma unroll
                        for (int f = 0; f < NF; ++f) {
                            f32x2 *dst = PS + (g * kUP + (tl * NF + f) * 64 + lane) * 4;
                            const Acc &p = gp[blk][h][t0 + tl][f];
                            const float sxg = pre_sx[blk][h][t0 + tl];
                            f32x4 lo = {float(p[0]), sxg * pre_sw[blk][h][f][0], float(p[1]),
                                        sxg * pre_sw[blk][h][f][1]};
                            f32x4 hi = {float(p[2]), sxg * pre_sw[blk][h][f][2], float(p[3]),
                                        sxg * pre_sw[blk][h][f][3]};
                            reinterpret_cast<f32x4 *>(dst)[0] = lo;
                            reinterpret_cast<f32x4 *>(dst)[1] = hi;
                        }
                }
            lds_barrier();
            // One output per thread and iteration; the four lanes of a unit
            // are adjacent. The results stay in registers until every pass
            // is done, so no store is waited for between passes.
#pragma unroll
            for (int it = 0; it < kIters; ++it) {
                const int o = threadIdx.x + it * 64 * WK;
                float sum = 0.f;
                if (o < kUP * 4) {
#pragma unroll
                    for (int g = 0; g < kGL; ++g) {
                        const f32x2 ps = PS[g * kUP * 4 + o];
                        sum = __builtin_fmaf(ps[0], ps[1], sum);
                    }
                }
                res[pass][it] = sum;
            }
        }
#pragma unroll
        for (int pass = 0; pass < kPasses; ++pass)
#pragma unroll
            for (int it = 0; it < kIters; ++it) {
                const int o = threadIdx.x + it * 64 * WK;
                if (kUP * 4 % (64 * WK) != 0 && o >= kUP * 4) break;  // whole waves
                const int unit = o >> 2, r = o & 3;
                const int tl = unit >> 6, l = unit & 63;
                const int t = pass * kTP + tl / NF, f = tl % NF;
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = __shfl(res[pass][it], (lane & ~3) | q);
                const int m = m0 + t * 16 + (l & 15), n = n0 + f * 16 + (l >> 4) * 4;
                if (r == 0 && m < M && n < N) {
                    // Outer scales of an operand without groups
                    // (quant_grouped.cu:161-165; 1 * 1 is exact), loaded
                    // only then: a load here would also wait for the
                    // previous iteration's store.
                    if (!input_group || !weight_group) {
                        const float ox = input_group ? 1.f : sx[m];
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            v[q] = v[q] * (ox * (weight_group ? 1.f : sw[n + q]));
                    }
                    store_out(y, size_t(m) * N + n, v, bias, n, N - 1, act, out_f16);
                }
            }
        return;
    }

    if constexpr (WK > 1) {
        Red *slot = red + wave * kSlotStride;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                Red4 v;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (Grouped) v[r] = facc[t][f][r];
                    else v[r] = acc[t][f][r];
                }
                *reinterpret_cast<Red4 *>(slot + ((t * NF + f) * 64 + lane) * 4) = v;
            }
        __syncthreads();
    }
    // Sum over the waves of the four values of unit (tf, l): ascending wave order.
    auto total = [&](int tf, int l, int t, int f, Red (&v)[4]) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = 0;
        if constexpr (WK > 1) {
#pragma unroll
            for (int q = 0; q < WK; ++q) {
                const Red4 s4 = *reinterpret_cast<const Red4 *>(red + q * kSlotStride + (tf * 64 + l) * 4);
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] += s4[r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (Grouped) v[r] += facc[t][f][r];
                else v[r] += acc[t][f][r];
            }
        }
    };
#pragma unroll
    for (int k = 0; k < kMaxU; ++k) {
        const int u = threadIdx.x + k * 64 * WK;
        if (u >= kUnits) break;
        const int tf = u >> 6, l = u & 63;
        const int t = tf / NF, f = tf % NF;
        const int m = m0 + t * 16 + (l & 15);
        const int n = n0 + f * 16 + (l >> 4) * 4;
        if (m >= M || n >= N) continue;
        if constexpr (FQ && !Grouped) pre_x[k] = fq_scale[t * 16 + (l & 15)];
        Red sum[4];
        total(tf, l, t, f, sum);
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = float(sum[r]);
        if constexpr (Split) {
            // Grouped partials carry their outer scales (quant_grouped.cu:161-165);
            // per-channel partials stay raw for the reduce kernel.
            if constexpr (Grouped) {
                // (sx or 1) * (sw or 1): a unit factor is exact.
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = v[r] * (pre_x[k] * pre_w[k][r]);
                float4 out = {v[0], v[1], v[2], v[3]};
                *reinterpret_cast<float4 *>(static_cast<float *>(partial) +
                                            (size_t(blockIdx.y) * M + m) * N + n) = out;
            } else {
                Scalar raw[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) raw[r] = Scalar(sum[r]);
                *reinterpret_cast<uint4 *>(static_cast<Scalar *>(partial) +
                                           (size_t(blockIdx.y) * M + m) * N + n) =
                    *reinterpret_cast<uint4 *>(raw);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (Grouped) {
                    v[r] = v[r] * (pre_x[k] * pre_w[k][r]);
                } else {
                    float s = v[r] * pre_x[k];
                    v[r] = s * pre_w[k][r];
                }
            }
            store_out(y, size_t(m) * N + n, v, bias, n, N - 1, act, out_f16);
        }
    }
}

// y = D((sum_s p_s) * sx * sw) or D(0 + sum_s p_s) for pre-scaled grouped
// partials; splits summed in ascending order (reference quant_reduce.cuh:9-19).
template <class Scalar, bool Scaled>
__global__ __launch_bounds__(256) void split_reduce(const Scalar *__restrict__ partial,
                                                    const float *__restrict__ sx,
                                                    const float *__restrict__ sw,
                                                    void *__restrict__ y, int M, int N,
                                                    int splits, const uint16_t *__restrict__ bias,
                                                    int act, int out_f16) {
    const size_t i4 = (size_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    const size_t total = size_t(M) * N;
    if (i4 >= total) return;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        Scalar s = 0;
        for (int q = 0; q < splits; ++q) s += partial[size_t(q) * total + i4 + r];
        if constexpr (Scaled) {
            const size_t i = i4 + r;
            float a = float(s) * sx[i / N];
            v[r] = a * sw[i % N];
        } else {
            v[r] = float(s);
        }
    }
    // N % 4 == 0: the four values share a row.
    store_out(y, i4, v, bias, int(i4 % N), N - 1, act, out_f16);
}

// Every launch uses eight wave64s per workgroup splitting K; K ranges are
// ceil(ceil(K/256) / (splits*8)) blocks, so trailing ranges may be short or
// empty (an empty range contributes zeros).
constexpr int kWaves = 8;

int span_of(int K, int splits) {
    const int blocks_k = (K + kBlockK - 1) / kBlockK;
    return (blocks_k + splits * kWaves - 1) / (splits * kWaves) * kBlockK;
}

#define QLIN_SKINNY_ARGS                                                                   \
    a.x, a.sx, a.w, a.sw, a.y, nullptr, a.M, a.N, a.K, span, a.input_group, a.weight_group, \
        a.bias, a.act, int(a.out_type == F16), a.fq

template <int Fmt, int MT, int NF, bool Grouped, int NB, int GS = 128>
int launch_slab(const GemmArgs &a, dim3 grid, int span, int staged, hipStream_t stream) {
    const size_t lds = size_t(kWaves) * 16 * (NF + (staged == 2 ? MT : 0)) * NB * kBlockK;
    if (staged == 2)
        hipLaunchKernelGGL((skinny_gemm<Fmt, MT, NF, kWaves, Grouped, false, NB, false, 0, GS, true>),
                           grid, dim3(64 * kWaves), lds, stream, QLIN_SKINNY_ARGS);
    else
        hipLaunchKernelGGL((skinny_gemm<Fmt, MT, NF, kWaves, Grouped, false, NB, false, 0, GS>),
                           grid, dim3(64 * kWaves), lds, stream, QLIN_SKINNY_ARGS);
    return 0;
}

template <int Fmt, int MT, int NF, bool Grouped, int NB, int GS = 128>
int launch_packed(const GemmArgs &a, dim3 grid, int span, hipStream_t stream) {
    hipLaunchKernelGGL((skinny_gemm<Fmt, MT, NF, kWaves, Grouped, false, NB, true, 0, GS>), grid,
                       dim3(64 * kWaves), 0, stream, QLIN_SKINNY_ARGS);
    return 0;
}

// GS: K-group size of the grouped partials (128, or 64 / 32 on the
// row-major, unsplit paths only).
template <int Fmt, int MT, int NF, bool Grouped, int GS = 128>
int launch_variant(const GemmArgs &a, const GemmPath &p, hipStream_t stream) {
    if (p.waves != kWaves) return -4;
    const int span = span_of(a.K, p.splits);
    if (a.packed) {
        // Packed weights: the waves split K (no grid split-K); each wave
        // streams its range in chunks of up to kMaxNB blocks held in
        // registers (weights and activations of a chunk: NB*(NF+MT) 64-byte
        // fragments per lane-quad, at most 10).
        if (p.splits != 1 || p.staged) return -4;
        dim3 grid((a.N + 16 * NF - 1) / (16 * NF), 1, (a.M + 16 * MT - 1) / (16 * MT));
        constexpr int kMaxNB = 10 / (NF + MT) > 4 ? 4 : (10 / (NF + MT) < 1 ? 1 : 10 / (NF + MT));
        const int nb = span / kBlockK < kMaxNB ? span / kBlockK : kMaxNB;
        switch (nb) {
        case 1: return launch_packed<Fmt, MT, NF, Grouped, 1, GS>(a, grid, span, stream);
        case 2: if constexpr (kMaxNB >= 2) return launch_packed<Fmt, MT, NF, Grouped, 2, GS>(a, grid, span, stream); break;
        case 3: if constexpr (kMaxNB >= 3) return launch_packed<Fmt, MT, NF, Grouped, 3, GS>(a, grid, span, stream); break;
        case 4: if constexpr (kMaxNB >= 4) return launch_packed<Fmt, MT, NF, Grouped, 4, GS>(a, grid, span, stream); break;
        default: break;
        }
        return -4;
    }
    if (skinny_lds_bytes(a, p) > kLdsBytes) return -4;  // would not launch
    dim3 grid((a.N + 16 * NF - 1) / (16 * NF), p.splits, (a.M + 16 * MT - 1) / (16 * MT));
    dim3 block(64 * kWaves);
    if (p.splits == 1) {
        // LDS-staged weight slabs: one-shot streaming of whole weight rows;
        // slab LDS per workgroup = 8 * 16*NF * span bytes.
        if (p.staged == 1 || p.staged == 2) {
            switch (span / kBlockK) {
            case 1: return launch_slab<Fmt, MT, NF, Grouped, 1, GS>(a, grid, span, p.staged, stream);
            case 2: return launch_slab<Fmt, MT, NF, Grouped, 2, GS>(a, grid, span, p.staged, stream);
            case 3: return launch_slab<Fmt, MT, NF, Grouped, 3, GS>(a, grid, span, p.staged, stream);
            default: return -4;
            }
        }
        if (p.staged) return -4;
        hipLaunchKernelGGL((skinny_gemm<Fmt, MT, NF, kWaves, Grouped, false, 0, false, 0, GS>), grid,
                           block, 0, stream, QLIN_SKINNY_ARGS);
        return 0;
    }
    if (p.staged) return -4;
    hipLaunchKernelGGL((skinny_gemm<Fmt, MT, NF, kWaves, Grouped, true, 0, false, 0, GS>), grid,
                       block, 0, stream,
                       a.x, a.sx, a.w, a.sw, a.y, a.workspace, a.M, a.N, a.K, span,
                       a.input_group, a.weight_group, a.bias, a.act, int(a.out_type == F16), a.fq);
    const size_t quads = (size_t(a.M) * a.N) / 4;
    dim3 rgrid(unsigned((quads + 255) / 256));
    using Scalar = typename Mfma<Fmt>::Scalar;
    if constexpr (Grouped)
        hipLaunchKernelGGL((split_reduce<float, false>), rgrid, dim3(256), 0, stream,
                           static_cast<const float *>(a.workspace), a.sx, a.sw, a.y, a.M, a.N,
                           p.splits, a.bias, a.act, int(a.out_type == F16));
    else
        hipLaunchKernelGGL((split_reduce<Scalar, true>), rgrid, dim3(256), 0, stream,
                           static_cast<const Scalar *>(a.workspace), a.sx, a.sw, a.y, a.M, a.N,
                           p.splits, a.bias, a.act, int(a.out_type == F16));
    return 0;
}

template <int Fmt, int MT, bool Grouped, int GS>
int dispatch_nf(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    if (p.channels == 16) return launch_variant<Fmt, MT, 1, Grouped, GS>(a, p, s);
    if (p.channels == 32) return launch_variant<Fmt, MT, 2, Grouped, GS>(a, p, s);
    if (p.channels == 48) return launch_variant<Fmt, MT, 3, Grouped, GS>(a, p, s);
    return -4;
}

// Fused activation quantization (FQ): eight waves, per-wave slabs of NB
// blocks, per-channel scales, no split.
template <int Fmt, int MT, int NF, int NB, bool XL, bool G>
int launch_fused_nb(const GemmArgs &a, hipStream_t stream) {
    // Every workgroup quantizes its token rows again (the activation is
    // re-encoded once per column tile). That ALU work overlaps the weight
    // slab's DMA: the encoding waits only for the 16-bit activation loads,
    // issued ahead of the slab. G: K groups of 128 (activation groups of 128;
    // weight groups of 128 or per-channel weight scales).
    const int span = NB * kBlockK;
    dim3 grid((a.N + 16 * NF - 1) / (16 * NF), 1, (a.M + 16 * MT - 1) / (16 * MT));
    // slabs, (XL) 16-bit activation tiles, the absmax / scale exchange
    const size_t lds = size_t(kWaves) * 16 * (NF + (XL ? 2 * MT : 0)) * NB * kBlockK +
                       size_t(kWaves + 1) * MT * 16 * 4;
    const int ig = G ? 128 : 0, wg = G ? a.weight_group : 0;
    if (a.fq.f16)
        hipLaunchKernelGGL((skinny_gemm<Fmt, MT, NF, kWaves, G, false, NB, false, 2, 128, XL>),
                           grid, dim3(64 * kWaves), lds, stream, nullptr, nullptr, a.w, a.sw,
                           a.y, nullptr, a.M, a.N, a.K, span, ig, wg, nullptr, 0,
                           int(a.out_type == F16), a.fq);
    else
        hipLaunchKernelGGL((skinny_gemm<Fmt, MT, NF, kWaves, G, false, NB, false, 1, 128, XL>),
                           grid, dim3(64 * kWaves), lds, stream, nullptr, nullptr, a.w, a.sw,
                           a.y, nullptr, a.M, a.N, a.K, span, ig, wg, nullptr, 0,
                           int(a.out_type == F16), a.fq);
    return 0;
}
template <int Fmt, int MT, int NB, bool XL, bool G>
int launch_fused_nf(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    switch (p.channels) {
    case 16: return launch_fused_nb<Fmt, MT, 1, NB, XL, G>(a, s);
    case 32: return launch_fused_nb<Fmt, MT, 2, NB, XL, G>(a, s);
    case 48: return launch_fused_nb<Fmt, MT, 3, NB, XL, G>(a, s);
    default: return -4;
    }
}
// Variants (skinny_fused_supported lists them): INT8 and FP8, 16-token
// tiles, one 256-column block of K per wave (staged 2: the 16-bit activation
// rows through LDS; staged 1: in registers). Measured on MI355X (graphs of
// launches over distinct weights, bf16 source, M = 32) against quantizer +
// GEMM: INT8 qkv 6.1 us against 6.7, o_proj 5.4 against 5.9; FP8 (hardware
// e4m3 conversion) qkv 6.1 against 7.3, o_proj 5.5 against 6.7. The kernel
// also takes 32-token tiles and two or three blocks per wave, but every
// workgroup re-encodes its rows, and there the encoding no longer hides
// under the weight stream: gate_up at M = 32 (32-token tile) 11.4 us against
// 10.2, down (three blocks) 13.9 against 10.2.
template <int Fmt>
int launch_fused(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    if (p.tokens != 16 || span_of(a.K, 1) != kBlockK) return -4;
    if (a.input_group) {
        if (p.staged == 2) return launch_fused_nf<Fmt, 1, 1, true, true>(a, p, s);
        return launch_fused_nf<Fmt, 1, 1, false, true>(a, p, s);
    }
    if (p.staged == 2) return launch_fused_nf<Fmt, 1, 1, true, false>(a, p, s);
    return launch_fused_nf<Fmt, 1, 1, false, false>(a, p, s);
}

template <int Fmt, bool Grouped, int GS = 128>
int dispatch_mt(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    switch (p.tokens) {
    case 16: return dispatch_nf<Fmt, 1, Grouped, GS>(a, p, s);
    case 32: return dispatch_nf<Fmt, 2, Grouped, GS>(a, p, s);
    case 64: return dispatch_nf<Fmt, 4, Grouped, GS>(a, p, s);
    default: return -4;
    }
}

template <int Fmt>
int dispatch_grouped(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    if (a.input_group || a.weight_group) {
        // Partials per the smaller group size (quant_grouped.cu:185-187).
        const int g = a.input_group && (!a.weight_group || a.input_group <= a.weight_group)
                          ? a.input_group : a.weight_group;
        if (g == 64) return dispatch_mt<Fmt, true, 64>(a, p, s);
        if (g == 32) return dispatch_mt<Fmt, true, 32>(a, p, s);
        if (g != 128) return -4;
        return dispatch_mt<Fmt, true>(a, p, s);
    }
    return dispatch_mt<Fmt, false>(a, p, s);
}

}  // namespace

#ifndef QLIN_SKINNY_PART
size_t skinny_lds_bytes(const GemmArgs &a, const GemmPath &p) {
    const int mt = p.tokens / 16, nf = p.channels / 16;
    const int nb = span_of(a.K, p.splits < 1 ? 1 : p.splits) / kBlockK;
    const size_t slab = p.staged ? size_t(kWaves) * 16 * nf * nb * kBlockK : 0;
    // staged 2: the activation tiles too (16-bit source rows when the GEMM
    // quantizes its own input)
    const size_t act = p.staged == 2 ? size_t(kWaves) * 16 * mt * nb * kBlockK * (a.fq.src ? 2 : 1) : 0;
    // Reduction slots reuse a staged slab; otherwise one static slot per wave.
    const size_t red = p.staged ? 0 : size_t(kWaves) * mt * nf * 64 * 4 * 4;
    // the fused quantization's absmax / scale exchange
    const size_t fq = a.fq.src ? size_t(kWaves + 1) * mt * 16 * 4 : 0;
    return red + slab + act + fq;
}

int skinny_span(int K, int splits) { return span_of(K, splits); }

size_t skinny_workspace_bytes(const GemmArgs &a, const GemmPath &p) {
    return p.splits > 1 ? size_t(p.splits) * a.M * a.N * 4 : 0;
}

bool skinny_fused_supported(const GemmArgs &a, const GemmPath &p) {
    // per-token scales, or activation groups of 128 with weight groups of 128
    // or per-channel weight scales (the caller takes unrotated sources only)
    const bool per_token = !a.input_group && !a.weight_group;
    const bool grouped = a.input_group == 128 && (a.weight_group == 0 || a.weight_group == 128);
    if (!a.fq.src || a.packed || a.bias || a.act || !(per_token || grouped) ||
        p.kind != KIND_SKINNY || p.splits != 1 || p.waves != kWaves ||
        (p.staged != 1 && p.staged != 2) || p.tokens != 16 ||
        (p.channels != 16 && p.channels != 32 && p.channels != 48) ||
        span_of(a.K, 1) != kBlockK)
        return false;
    // One round of workgroups (256 CUs, one workgroup each): over two rounds
    // the re-encoding no longer hides under the weight stream (qkv at M = 64,
    // 512 workgroups: 10.1 us against 9.0 us for quantizer + GEMM).
    if (long((a.N + p.channels - 1) / p.channels) * ((a.M + 15) / 16) > 256) return false;
    // slabs, (staged 2) the 16-bit activation tiles, the absmax exchange
    const size_t lds = size_t(kWaves) * p.channels * kBlockK +
                       (p.staged == 2 ? size_t(kWaves) * 16 * 2 * kBlockK : 0) +
                       size_t(kWaves + 1) * p.tokens * 4;
    return lds <= size_t(kLdsBytes);
}

#endif

// The kernel variants are compiled in four translation units (format, with
// and without the finish; see the Makefile) that each define one entry below.
#ifdef QLIN_SKINNY_PART
int QLIN_SKINNY_PART(const GemmArgs &a, const GemmPath &p, hipStream_t stream) {
    return dispatch_grouped<QLIN_SKINNY_FMT>(a, p, stream);
}
#if !QLIN_FIN
#define QLIN_CAT_(a, b) a##b
#define QLIN_CAT(a, b) QLIN_CAT_(a, b)
int QLIN_CAT(QLIN_SKINNY_PART, _fused)(const GemmArgs &a, const GemmPath &p, hipStream_t stream) {
    return launch_fused<QLIN_SKINNY_FMT>(a, p, stream);
}
#endif
#else
#define QLIN_PART_DECL(name)                                                  \
    int name(const GemmArgs &, const GemmPath &, hipStream_t);              \
    int name##_fin(const GemmArgs &, const GemmPath &, hipStream_t);        \
    int name##_fused(const GemmArgs &, const GemmPath &, hipStream_t);
QLIN_PART_DECL(launch_skinny_i8)
QLIN_PART_DECL(launch_skinny_fp8)
#undef QLIN_PART_DECL

int launch_skinny(const GemmArgs &a, const GemmPath &p, hipStream_t stream) {
    const bool fin = a.bias || a.act;
    if (a.fmt == I8) return fin ? launch_skinny_i8_fin(a, p, stream) : launch_skinny_i8(a, p, stream);
    return fin ? launch_skinny_fp8_fin(a, p, stream) : launch_skinny_fp8(a, p, stream);
}

int launch_skinny_fused(const GemmArgs &a, const GemmPath &p, hipStream_t stream) {
    if (!skinny_fused_supported(a, p)) return -4;
    return a.fmt == I8 ? launch_skinny_i8_fused(a, p, stream) : launch_skinny_fp8_fused(a, p, stream);
}
#endif

}  // namespace qlin
