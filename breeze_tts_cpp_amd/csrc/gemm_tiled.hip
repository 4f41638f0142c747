// Prefill-regime quantized GEMM (hundreds to thousands of tokens) for gfx950.
//
// Same contract as the skinny kernel (y = D(dequant(x . w^T))), replacing the
// reference's tensor-core paths: CUTLASS SM80 INT8 with the EVT epilogue
// D((acc*sx)*sw) (ops/kernels/quant/quant_gemm_sm80.cu:14-82), the SM90 INT8 /
// FP8 WGMMA kernels (quant_gemm_sm90.cu:16-283) and the K-group GEMM
// (quant_grouped.cu:16-169, quant_gemm_sm90.cu:289-372).
//
// Work decomposition: one workgroup per macro tile of BN weight rows x BM
// tokens; WN x WM wave64s, each owning a (16*WTN) x (16*WTM) sub-tile of
// 16x16 MFMA tiles (INT8: v_mfma_i32_16x16x64_i8, exact int32; FP8:
// v_mfma_f32_16x16x128_f8f6f4, the plain e4m3 product with fp32
// accumulation: the f8f6f4 builtins get zero scale operands, for which the
// compiler emits the unscaled instruction. With unit E8M0 scales (0x7f) it
// keeps the scaled form, whose scale operand occupies a VGPR: FP8 prefill
// measured 7% slower that way, and its 256x256 double-buffered tile spilled).
//
// Operand staging: K advances in BK-byte stages through a STAGES-deep LDS
// ring filled by buffer_load ... lds (global -> LDS without registers), so
// STAGES-1 stages are in flight while one feeds the MFMAs. Each wave's load
// instruction writes 1 KB of LDS contiguously in lane order; the swizzle is
// applied by choosing each lane's global source chunk, so that 16-byte chunk
// c of stage row r sits at chunk c ^ ((r >> 1) & (CPR - 1)). With it the MFMA
// fragment reads (16 rows, same logical chunk) measured free of LDS bank
// conflicts on gfx950 (SQ_LDS_BANK_CONFLICT = 0), where the unswizzled
// layout takes 12 conflict cycles per ds_read_b128. Buffer descriptors cover exactly the tile's valid rows, so rows
// past the matrix edge and chunks past K read as zero (out-of-range offset).
// The weight tile is the MFMA A operand: a lane's accumulator holds four
// consecutive output channels of one token -> 8-byte output stores.
// Tiles are numbered XCD-major (consecutive tiles on one XCD share its L2).
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

#include <algorithm>
#include <type_traits>

// Built twice: without (launch_tiled_plain) and with (launch_tiled_fin) the
// fused finish epilogue; the plain build carries no finish code.
#ifndef QLIN_FIN
#define QLIN_FIN 0
#endif

namespace qlin {
namespace {

constexpr bool kFin = QLIN_FIN;

template <int Fmt> struct TileMma;
template <> struct TileMma<I8> {
    using Acc = i32x4;
    __device__ static void run(Acc &c, const i32x4 &a, const i32x4 &b) {
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
    }
    // A 128-byte stage: K [0, 64) in registers 0-3, [64, 128) in 4-7.
    __device__ static void run(Acc &c, const i32x8 &a, const i32x8 &b) {
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(i32x4{a[0], a[1], a[2], a[3]},
                                                  i32x4{b[0], b[1], b[2], b[3]}, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(i32x4{a[4], a[5], a[6], a[7]},
                                                  i32x4{b[4], b[5], b[6], b[7]}, c, 0, 0, 0);
    }
};
template <> struct TileMma<FP8> {
    using Acc = f32x4;
    // Zero scale operands: the unscaled v_mfma_f32_16x16x128_f8f6f4.
    __device__ static void run(Acc &c, const i32x8 &a, const i32x8 &b) {
        c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};

// Physical 16-byte chunk of logical chunk c in stage row r is c ^ swizzle(r).
template <int BK> __device__ __forceinline__ int swizzle(int r) {
    if constexpr (BK == 128) return (r >> 1) & 7;
    else return (r >> 1) & 3;
}

// s_waitcnt vmcnt(n) leaving expcnt / lgkmcnt unconstrained (gfx9 encoding).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier for the LDS ring: this wave's LDS reads are complete
// (lgkmcnt(0)) before any wave passes, so a buffer read before the barrier
// may be refilled after it. No memory fence: the global->LDS loads are waited
// for explicitly with wait_vmcnt.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
}

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// Unit scales: the stage-slot scale DMA of an operand without K groups copies
// these, so the group rescale reads its slot unconditionally (1 * s and s * 1
// are exact).
#define QLIN_ONES4 1.f, 1.f, 1.f, 1.f
#define QLIN_ONES16 QLIN_ONES4, QLIN_ONES4, QLIN_ONES4, QLIN_ONES4
#define QLIN_ONES64 QLIN_ONES16, QLIN_ONES16, QLIN_ONES16, QLIN_ONES16
__device__ const float kUnitScales[256] = {QLIN_ONES64, QLIN_ONES64, QLIN_ONES64, QLIN_ONES64};
#undef QLIN_ONES64
#undef QLIN_ONES16
#undef QLIN_ONES4

// One 16-byte piece of a bf16/f16 output row, stored non-temporally: a
// prefill GEMM writes its whole output at the end of each tile (all CUs at
// once in one-round grids), and streaming it past the caches measured 5-8%
// faster over the four M = 4096 projections than plain stores. (The
// operand DMA keeps the default policy: non-temporal loads of the weight
// tiles, which other tiles re-read through L2, measured 10-20% slower.)
__device__ __forceinline__ void store_out16(uint16_t *dst, const uint4 &val) {
    __builtin_nontemporal_store(i32x4{int(val.x), int(val.y), int(val.z), int(val.w)},
                                reinterpret_cast<i32x4 *>(dst));
}

template <int Fmt, int WN, int WM, int WTN, int WTM, int BK, int STAGES, bool Grouped, bool KFull,
          class Out, bool PackedW = false, int GS = 128>
__global__ __launch_bounds__(64 * WN * WM) void tiled_gemm(
    const uint8_t *__restrict__ x, const float *__restrict__ sx, const uint8_t *__restrict__ w,
    const float *__restrict__ sw, void *__restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n, int input_group, int weight_group, const uint16_t *__restrict__ bias, int act) {
    constexpr int NW = WN * WM;
    constexpr int BN = 16 * WTN * WN, BM = 16 * WTM * WM;
    constexpr int CPR = BK / 16;          // 16-byte chunks per stage row
    constexpr int RPI = 64 / CPR;         // stage rows written by one wave instruction
    constexpr int ROWS = BN + BM;
    constexpr int INSTS = ROWS / (RPI * NW);
    constexpr int W_INSTS = BN / (RPI * NW);
    // K-group kernels: each stage slot also holds the stage's group scales
    // (weight [BN] floats in its first KB, token [BM] floats in the second),
    // copied by one extra DMA instruction per wave: wave 0 the weight scales,
    // wave 1 the token scales, the other waves nothing (out-of-range offsets
    // into a third, unused KB), so that the issue has no branch. Each gets a
    // whole KB: a lane past the tile still writes (zeros) at its position.
    // Groups of GS = 32 / 64 (the smaller of the two operands' group sizes)
    // read their scales from global memory instead.
    constexpr bool kScaleDma = Grouped && GS == 128;
    constexpr int SCALE_BYTES = kScaleDma ? 3072 : 0;
    constexpr int STAGE_BYTES = ROWS * BK + SCALE_BYTES;
    static_assert(ROWS % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "stage rows per instruction");
    static_assert(!kScaleDma || (BN * 4 <= 1024 && BM * 4 <= 1024 && NW >= 2),
                  "one scale instruction per operand");
    static_assert(GS == 128 || (Grouped && BK == 128 && (GS == 32 || GS == 64)),
                  "K groups of 32 / 64 use 128-byte stages");
    // FP8 per-channel on 64-byte stages uses v_mfma_f32_32x32x64_f8f6f4 (32-byte
    // fragments cover 32 rows x 64 K, half the registers of 16x16x128 per K).
    constexpr bool kMF32 = Fmt == FP8 && !Grouped && BK == 64;
    constexpr bool kAcc32 = kMF32;
    // K bytes per stage: the INT8 16x16x64 and FP8 32x32x64 pipelines consume
    // exactly 64, the FP8 16x16x128 pipeline 128; K groups are 128 wide (two
    // INT8 stages or one FP8 stage).
    static_assert(BK == 64 || BK == 128, "K bytes per stage");
    static_assert(!Grouped || Fmt == I8 || BK == 128, "FP8 K groups use 128-byte stages");
    constexpr int kGroupK = 128;
    constexpr int SPG = kGroupK / BK;  // stages per K group
    using MMA = TileMma<Fmt>;
    using Acc = typename MMA::Acc;

    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

    // XCD-major tile numbering: hardware places workgroup b on XCD b % 8.
    const int tiles = tiles_m * tiles_n;
    int b = blockIdx.x;
    if (tiles % 8 == 0) b = (b % 8) * (tiles / 8) + b / 8;
    // Column groups of kGroupN weight tiles: consecutive tiles (one XCD's
    // share) cover a kGroupN x (tiles/8/kGroupN) block, not one tall column.
    // 256x256 tiles take groups of 8 (qkv at M = 4096: INT8 35.1 -> 34.3 us,
    // FP8 33.6 -> 32.5 us, gate_up 0.5% faster); the other tiles groups of 4
    // (8 measured 1% slower on o_proj and down).
    constexpr int kGroupN = BN == 256 && BM == 256 ? 8 : 4;
    const int group = b / (kGroupN * tiles_m), in_group = b % (kGroupN * tiles_m);
    const int group_w = min(kGroupN, tiles_n - group * kGroupN);
    const int tn = group * kGroupN + in_group % group_w, tm = in_group / group_w;
    const int n_base = tn * BN, m_base = tm * BM;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave_n = wave % WN, wave_m = wave / WN;
    const int row16 = lane & 15, quad = lane >> 4;

    // Packed weights: the tile's row groups are (n_base/16 ..) x tiles_k 1 KB tiles.
    const int tiles_k = (K + 63) / 64;
    const __amdgpu_buffer_rsrc_t rsrc_w =
        PackedW ? __builtin_amdgcn_make_buffer_rsrc(
                      const_cast<uint8_t *>(w + size_t(n_base / 16) * tiles_k * 1024), 0,
                      min(BN, N - n_base) / 16 * tiles_k * 1024, 0x00020000)
                : __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w + size_t(n_base) * K),
                                                    0, min(BN, N - n_base) * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc_x = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(x + size_t(m_base) * K), 0, min(BM, M - m_base) * K, 0x00020000);
    // K-group scales [ceil(K/g), N] and [ceil(K/g), M] (the host checks that
    // both arrays stay below 2^31 bytes).
    const int kgroups = (K + kGroupK - 1) / kGroupK;
    // An operand without groups reads the 1 KB of unit scales instead, at
    // every group.
    const bool w_groups = Grouped && weight_group, x_groups = Grouped && input_group;
    const __amdgpu_buffer_rsrc_t rsrc_sw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(w_groups ? sw : kUnitScales), 0, w_groups ? kgroups * N * 4 : 1024,
        0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc_sx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(x_groups ? sx : kUnitScales), 0, x_groups ? kgroups * M * 4 : 1024,
        0x00020000);

    // Load instruction i of this wave fills stage rows [(i*NW + wave)*RPI, +RPI),
    // 1 KB of LDS in lane order: lane -> row += lane / CPR, physical chunk
    // lane % CPR. Every instruction's first row is a multiple of RPI, so the
    // swizzle (row bits 1..) and thus the lane's source column are the same
    // for all i: a per-lane voffset plus a wave-uniform soffset per i.
    const int lane_row = lane / CPR;
    const int lane_chunk = (lane % CPR) ^ swizzle<BK>(wave * RPI + lane_row);
    const uint32_t lane_voff = uint32_t(lane_row) * uint32_t(K) + uint32_t(lane_chunk * 16);
    // Packed weights: logical chunk c of a stage row lies in 64-K tile c/4,
    // fragment chunk (c%4)*16 + row%16; the stage's first tile and the row
    // group go in the uniform offset.
    const uint32_t lane_voff_p =
        uint32_t((lane_chunk / 4) * 1024 + (lane_chunk % 4) * 256 + lane_row * 16);
    // The scale DMA's per-lane offset (host-checked: both scale arrays stay
    // below 2^31 bytes): group g's row starts at g * scale_stride.
    const bool scale_wv = wave == 0, scale_xv = wave == 1;
    const bool scale_groups = scale_wv ? w_groups : x_groups;
    const bool scale_live = Grouped && (scale_wv || scale_xv) && lane * 4 < (scale_wv ? BN : BM);
    const uint32_t scale_stride = scale_groups ? uint32_t((scale_wv ? N : M) * 4) : 0u;
    const uint32_t scale_lane =
        uint32_t((scale_groups ? (scale_wv ? n_base : m_base) * 4 : 0) + lane * 16);
    auto issue = [&](int stage, int k0) {
        uint8_t *base = lds + (stage % STAGES) * STAGE_BYTES;
        const bool kin = KFull || k0 + lane_chunk * 16 < K;
        const uint32_t voff = kin ? lane_voff + uint32_t(k0) : 0x80000000u;
        const uint32_t voff_p = kin ? lane_voff_p : 0x80000000u;
#pragma unroll
        for (int i = 0; i < INSTS; ++i) {
            const int row = (i * NW + wave) * RPI;
            lds_ptr_t dst = (lds_ptr_t)(base + (i * NW + wave) * 1024);
            if (PackedW && i < W_INSTS) {
                const uint32_t soff = uint32_t((row / 16) * tiles_k * 1024 + (row % 16) * 16 +
                                               (k0 / 64) * 1024);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_w, dst, 16, voff_p, soff, 0, 0);
            } else {
                const uint32_t soff = uint32_t(i < W_INSTS ? row : row - BN) * uint32_t(K);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(i < W_INSTS ? rsrc_w : rsrc_x, dst, 16,
                                                         voff, soff, 0, 0);
            }
        }
        if constexpr (kScaleDma) {
            // The stage's group scales: sw[g][n_base ..) by wave 0, sx[g][m_base ..)
            // by wave 1 (unit scales for an operand without groups; lanes past
            // the tile read zero through an out-of-range offset); waves 2..
            // write zeros into the slot's third KB.
            const uint32_t g = uint32_t(k0 / kGroupK);
            const uint32_t off = scale_live ? g * scale_stride + scale_lane : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                scale_wv ? rsrc_sw : rsrc_sx,
                (lds_ptr_t)(base + ROWS * BK + (scale_wv ? 0 : scale_xv ? 1024 : 2048)), 16, off, 0,
                0, 0);
        }
    };
    // "Stage s+1 has landed" waits: the waves of a K-group kernel issue one
    // more instruction per stage.
    auto wait_ring = [&](auto outstanding_stages) {
        constexpr int S = decltype(outstanding_stages)::value;
        wait_vmcnt<(INSTS + (kScaleDma ? 1 : 0)) * S>();
    };

    Acc acc[(Grouped || kAcc32) ? 1 : WTN][(Grouped || kAcc32) ? 1 : WTM];
    f32x16 acc32[kAcc32 ? WTN / 2 : 1][kAcc32 ? WTM / 2 : 1];
    if constexpr (kAcc32) {
#pragma unroll
        for (int i = 0; i < WTN / 2; ++i)
#pragma unroll
            for (int j = 0; j < WTM / 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc32[i][j][e] = 0.f;
    }
    float facc[Grouped ? WTN : 1][Grouped ? WTM : 1][4];
    if constexpr (!Grouped && !kAcc32) {
#pragma unroll
        for (int i = 0; i < WTN; ++i)
#pragma unroll
            for (int j = 0; j < WTM; ++j) acc[i][j] = Acc{0, 0, 0, 0};
    } else if constexpr (Grouped) {
#pragma unroll
        for (int i = 0; i < WTN; ++i)
#pragma unroll
            for (int j = 0; j < WTM; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) facc[i][j][r] = 0.f;
    }

    // Fragment of stage row `row`, 64-K sub-step h: lane quad q holds K bytes
    // [64h + 16q, +16). Rows row0 + 16i share row bits 1..3, hence the chunk.
    auto frag16 = [&](const uint8_t *base, int row, int h) {
        const int chunk = (h * 4 + quad) ^ swizzle<BK>(row);
        return *reinterpret_cast<const i32x4 *>(base + row * BK + chunk * 16);
    };
    auto frag32 = [&](const uint8_t *base, int row) {
        const i32x4 lo = frag16(base, row, 0), hi = frag16(base, row, 1);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    // Per-channel and per-token scales of the tile go to LDS past the ring
    // (weight scales [BN], then token scales [BM]; 1.0 where the scales are
    // per K group): the loads are issued ahead of the stage prologue and the
    // epilogue reads them from LDS instead of waiting on global loads.
    constexpr int kRingBytes = STAGES * STAGE_BYTES > BN * BM * 2 ? STAGES * STAGE_BYTES : BN * BM * 2;
    float *scl = reinterpret_cast<float *>(lds + kRingBytes);
    constexpr int kScaleLoads = (BN + BM + 64 * NW - 1) / (64 * NW);
    float scale_v[kScaleLoads];
#pragma unroll
    for (int l = 0; l < kScaleLoads; ++l) {
        const int i = tid + l * 64 * NW;
        float v = 1.f;
        if (i < BN) {
            if (!Grouped || !weight_group) v = sw[min(n_base + i, N - 1)];
        } else if (i < BN + BM) {
            if (!Grouped || !input_group) v = sx[min(m_base + i - BN, M - 1)];
        }
        scale_v[l] = v;
    }
    const int stages = (K + BK - 1) / BK;
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < stages) issue(s, s * BK);
#pragma unroll
    for (int l = 0; l < kScaleLoads; ++l)
        if (tid + l * 64 * NW < BN + BM) scl[tid + l * 64 * NW] = scale_v[l];

    const int a_row0 = wave_n * 16 * WTN + row16;
    const int b_row0 = BN + wave_m * 16 * WTM + row16;

    if constexpr (kMF32) {
        // Same pipeline as below with 32x32x64 FP8 tiles: lane l holds row
        // l % 32 of a fragment and K bytes [32*(l/32), +32) of the stage.
        const int r32 = lane & 31, g32 = lane >> 5;
        const int a_r0 = wave_n * 16 * WTN + r32, b_r0 = BN + wave_m * 16 * WTM + r32;
        const int a_c0 = ((2 * g32) ^ swizzle<BK>(a_r0)) * 16, a_c1 = ((2 * g32 + 1) ^ swizzle<BK>(a_r0)) * 16;
        const int b_c0 = ((2 * g32) ^ swizzle<BK>(b_r0)) * 16, b_c1 = ((2 * g32 + 1) ^ swizzle<BK>(b_r0)) * 16;
        const int a_off = a_r0 * BK, b_off = b_r0 * BK;
        constexpr int NA = WTN / 2, NBF = WTM / 2;
        auto read = [&](int st, i32x8 (&a)[NA], i32x8 (&bb)[NBF]) {
            const uint8_t *cur = lds + (st % STAGES) * STAGE_BYTES;
            const uint8_t *pa = cur + a_off, *pb = cur + b_off;
#pragma unroll
            for (int j = 0; j < NBF; ++j) {
                const i32x4 lo = *reinterpret_cast<const i32x4 *>(pb + j * 32 * BK + b_c0);
                const i32x4 hi = *reinterpret_cast<const i32x4 *>(pb + j * 32 * BK + b_c1);
                bb[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                const i32x4 lo = *reinterpret_cast<const i32x4 *>(pa + i * 32 * BK + a_c0);
                const i32x4 hi = *reinterpret_cast<const i32x4 *>(pa + i * 32 * BK + a_c1);
                a[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
        };
        auto mma = [&](const i32x8 (&a)[NA], const i32x8 (&bb)[NBF], int i0, int i1) {
#pragma unroll
            for (int i = i0; i < i1; ++i)
#pragma unroll
                for (int j = 0; j < NBF; ++j)
                    acc32[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        a[i], bb[j], acc32[i][j], 0, 0, 0, 0, 0, 0);
        };
        constexpr int kEarly = NA / 4 > 0 ? NA / 4 : 1;
        auto step = [&](int s, const i32x8 (&a)[NA], const i32x8 (&bb)[NBF], i32x8 (&na)[NA],
                        i32x8 (&nb)[NBF]) {
            if (s + STAGES - 1 < stages) issue(s + STAGES - 1, (s + STAGES - 1) * BK);
            mma(a, bb, 0, kEarly);
            if (s + STAGES - 1 < stages) wait_vmcnt<INSTS * (STAGES - 2)>();
            else if (s + 1 < stages) wait_vmcnt<0>();
            lds_barrier();
            // Unconditional: see the 16x16 pipeline below.
            read(s + 1, na, nb);
            mma(a, bb, kEarly, NA);
        };
        i32x8 a0[NA], b0[NBF], a1[NA], b1[NBF];
        if (stages >= STAGES - 1) wait_vmcnt<INSTS * (STAGES - 2)>();
        else wait_vmcnt<0>();
        lds_barrier();
        read(0, a0, b0);
        int s = 0;
        for (; s + 1 < stages; s += 2) {
            step(s, a0, b0, a1, b1);
            step(s + 1, a1, b1, a0, b0);
        }
        if (s < stages) step(s, a0, b0, a1, b1);
    } else if constexpr (!Grouped && STAGES == 2) {
        // Two 128-byte stages, double-buffered (a 256x256 tile's 64 KB stages
        // fit the LDS twice). The DMA of stage s+1 is issued once every wave
        // has read stage s-1, and has the MFMAs of a whole stage to land. A
        // step reads its weight fragments one 16-row block ahead of that
        // block's MFMAs, so a wave holds the token fragments of two stages but
        // only two weight fragments: i32x8 fragments (FP8: one 16x16x128 MFMA
        // per tile and stage, INT8: two 16x16x64) at two waves per SIMD.
        static_assert(BK == 128, "double-buffered 128-byte stages");
        const int a_off = a_row0 * BK, b_off = b_row0 * BK;
        const int a_c0 = (quad ^ swizzle<BK>(a_row0)) * 16;
        const int a_c1 = ((4 + quad) ^ swizzle<BK>(a_row0)) * 16;
        const int b_c0 = (quad ^ swizzle<BK>(b_row0)) * 16;
        const int b_c1 = ((4 + quad) ^ swizzle<BK>(b_row0)) * 16;
        auto rd = [&](const uint8_t *p, int c0, int c1) {
            const i32x4 lo = *reinterpret_cast<const i32x4 *>(p + c0);
            const i32x4 hi = *reinterpret_cast<const i32x4 *>(p + c1);
            return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        };
        auto read_b = [&](int st, i32x8 (&bb)[WTM]) {
            const uint8_t *pb = lds + (st % 2) * STAGE_BYTES + b_off;
#pragma unroll
            for (int j = 0; j < WTM; ++j) bb[j] = rd(pb + j * 16 * BK, b_c0, b_c1);
        };
        auto read_a = [&](int st, int i) {
            return rd(lds + (st % 2) * STAGE_BYTES + a_off + i * 16 * BK, a_c0, a_c1);
        };
        auto row = [&](int i, const i32x8 &a, const i32x8 (&bb)[WTM]) {
#pragma unroll
            for (int j = 0; j < WTM; ++j) MMA::run(acc[i][j], a, bb[j]);
        };
        // Step s: weight blocks 0..WTN-2 (each reading the next block first);
        // wait for stage s+1 and barrier (every wave's reads of stage s are
        // complete: its slot takes stage s+2); read stage s+1's token
        // fragments and first weight block (unconditional: after the last
        // stage they read a slot whose values go unused); the last block.
        auto step = [&](int s, const i32x8 (&bb)[WTM], i32x8 a, i32x8 (&nb)[WTM], i32x8 &na) {
#pragma unroll
            for (int i = 0; i + 1 < WTN; ++i) {
                const i32x8 an = read_a(s, i + 1);
                row(i, a, bb);
                a = an;
                // Keeps the next block's reads from being hoisted (all of a
                // stage's weight fragments at once do not fit the registers).
                __builtin_amdgcn_sched_barrier(0);
            }
            wait_vmcnt<0>();
            lds_barrier();
            if (s + 2 < stages) issue(s + 2, (s + 2) * BK);
            read_b(s + 1, nb);
            na = read_a(s + 1, 0);
            row(WTN - 1, a, bb);
        };
        i32x8 b0[WTM], b1[WTM], a0;
        wait_vmcnt<0>();
        lds_barrier();
        if (1 < stages) issue(1, BK);
        read_b(0, b0);
        a0 = read_a(0, 0);
        int s = 0;
        for (; s + 1 < stages; s += 2) {
            step(s, b0, a0, b1, a0);
            step(s + 1, b1, a0, b0, a0);
        }
        if (s < stages) step(s, b0, a0, b1, a0);
    } else if constexpr (!Grouped) {
        // Software pipeline, one stage per step (INT8: BK = 64, one 64-K
        // MFMA per tile, or BK = 128, two; FP8: BK = 128, one 128-K MFMA).
        // Iteration s: issue the global loads of stage
        // s+STAGES-1; run the first MFMA rows of stage s; wait for stage s+1
        // and barrier; read stage s+1 fragments into the other register set
        // while the remaining MFMAs of stage s run. The barrier also retires
        // every wave's reads of buffer s % STAGES, which iteration s+1 refills.
        static_assert(BK == 64 ? Fmt == I8 : BK == 128, "per-channel stage size");
        using Frag = std::conditional_t<BK == 64, i32x4, i32x8>;
        const int a_off = a_row0 * BK, b_off = b_row0 * BK;
        const int a_c0 = (quad ^ swizzle<BK>(a_row0)) * 16, b_c0 = (quad ^ swizzle<BK>(b_row0)) * 16;
        const int a_c1 = ((4 + quad) ^ swizzle<BK>(a_row0)) * 16;
        const int b_c1 = ((4 + quad) ^ swizzle<BK>(b_row0)) * 16;
        auto read = [&](int st, Frag (&a)[WTN], Frag (&bb)[WTM]) {
            const uint8_t *cur = lds + (st % STAGES) * STAGE_BYTES;
            const uint8_t *pa = cur + a_off, *pb = cur + b_off;
#pragma unroll
            for (int j = 0; j < WTM; ++j) {
                const i32x4 lo = *reinterpret_cast<const i32x4 *>(pb + j * 16 * BK + b_c0);
                if constexpr (BK == 64) {
                    bb[j] = lo;
                } else {
                    const i32x4 hi = *reinterpret_cast<const i32x4 *>(pb + j * 16 * BK + b_c1);
                    bb[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
            }
#pragma unroll
            for (int i = 0; i < WTN; ++i) {
                const i32x4 lo = *reinterpret_cast<const i32x4 *>(pa + i * 16 * BK + a_c0);
                if constexpr (BK == 64) {
                    a[i] = lo;
                } else {
                    const i32x4 hi = *reinterpret_cast<const i32x4 *>(pa + i * 16 * BK + a_c1);
                    a[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
            }
        };
        auto mma = [&](const Frag (&a)[WTN], const Frag (&bb)[WTM], int i0, int i1) {
#pragma unroll
            for (int i = i0; i < i1; ++i)
#pragma unroll
                for (int j = 0; j < WTM; ++j) MMA::run(acc[i][j], a[i], bb[j]);
        };
        constexpr int kEarly = WTN / 4;  // MFMA rows issued before the barrier
        // The barrier (and its lgkmcnt(0)) runs on every step, also the last:
        // with no control-flow path around it, the compiler's LDS wait
        // counting never makes a stage's MFMAs wait on the next stage's reads.
        auto step = [&](int s, const Frag (&a)[WTN], const Frag (&bb)[WTM], Frag (&na)[WTN],
                        Frag (&nb)[WTM]) {
            if (s + STAGES - 1 < stages) issue(s + STAGES - 1, (s + STAGES - 1) * BK);
            mma(a, bb, 0, kEarly);
            if (s + STAGES - 1 < stages) wait_vmcnt<INSTS * (STAGES - 2)>();
            else if (s + 1 < stages) wait_vmcnt<0>();
            lds_barrier();
            // i32x8 fragments (128-byte stages) are read unconditionally
            // (after the last stage, a ring slot whose fragments go unused):
            // a conditional read makes the compiler copy every one of them at
            // each stage.
            if (BK == 128 || s + 1 < stages) read(s + 1, na, nb);
            mma(a, bb, kEarly, WTN);
        };
        Frag a0[WTN], b0[WTM], a1[WTN], b1[WTM];
        if (stages >= STAGES - 1) wait_vmcnt<INSTS * (STAGES - 2)>();
        else wait_vmcnt<0>();
        lds_barrier();
        read(0, a0, b0);
        int s = 0;
        for (; s + 1 < stages; s += 2) {
            step(s, a0, b0, a1, b1);
            step(s + 1, a1, b1, a0, b0);
        }
        if (s < stages) step(s, a0, b0, a1, b1);
    } else if constexpr (GS < kGroupK) {
        // K groups of GS = 32 / 64 (the reference grouped_gemm's GroupSize,
        // the smaller of the two operands' group sizes), stage-synchronous
        // over 128-byte stages. Sub-group g of a stage covers K bytes
        // [g*GS, (g+1)*GS) of it: its MFMAs accumulate natively from zero and
        // are applied as facc = fmaf(p, sx * sw, facc), sub-groups ascending.
        // The 16-byte fragment chunk c of a lane covers K [16c, 16c+16)
        // (INT8: chunk 4h + quad of 64-K sub-step h; FP8: chunks quad and
        // 4 + quad in registers 0-3 and 4-7); the sub-group's MFMAs run on B
        // fragments with the chunks of other sub-groups zeroed. The scales
        // are read from global memory (L2): sx[k / input_group][m],
        // sw[k / weight_group][n] at the sub-group's first K.
        constexpr int SUB = BK / GS;
        for (int s = 0; s < stages; ++s) {
            if (s + STAGES - 2 < stages) wait_ring(std::integral_constant<int, STAGES - 2>{});
            else wait_vmcnt<0>();
            __syncthreads();
            if (s + STAGES - 1 < stages) issue(s + STAGES - 1, (s + STAGES - 1) * BK);
            const uint8_t *cur = lds + (s % STAGES) * STAGE_BYTES;
            // Not unrolled: unrolled sub-groups hoist every scale load and spill.
#pragma unroll 1
            for (int g = 0; g < SUB; ++g) {
                const int k = s * BK + g * GS;
                if (!KFull && k >= K) break;
                float sxg[WTM];
#pragma unroll
                for (int j = 0; j < WTM; ++j) {
                    const int m = min(m_base + wave_m * 16 * WTM + j * 16 + row16, M - 1);
                    sxg[j] = input_group ? sx[size_t(k / input_group) * M + m] : 1.f;
                }
                const float *swr = sw + size_t(weight_group ? k / weight_group : 0) * N;
                // Chunk c belongs to sub-group c * 16 / GS.
                auto keep = [&](int c) { return c * 16 / GS == g; };
#pragma unroll
                for (int i = 0; i < WTN; ++i) {
                    Acc part[WTM];
#pragma unroll
                    for (int j = 0; j < WTM; ++j) part[j] = Acc{0, 0, 0, 0};
                    if constexpr (Fmt == I8) {
                        const int hs = g * GS / 64;  // the 64-K sub-step holding g
                        const i32x4 af = frag16(cur, a_row0 + i * 16, hs);
#pragma unroll
                        for (int j = 0; j < WTM; ++j) {
                            i32x4 bf = frag16(cur, b_row0 + j * 16, hs);
                            if (!keep(hs * 4 + quad)) bf = i32x4{0, 0, 0, 0};
                            MMA::run(part[j], af, bf);
                        }
                    } else {
                        const i32x8 af = frag32(cur, a_row0 + i * 16);
                        const bool k0 = keep(quad), k1 = keep(4 + quad);
#pragma unroll
                        for (int j = 0; j < WTM; ++j) {
                            i32x8 bf = frag32(cur, b_row0 + j * 16);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                bf[e] = k0 ? bf[e] : 0;
                                bf[4 + e] = k1 ? bf[4 + e] : 0;
                            }
                            MMA::run(part[j], af, bf);
                        }
                    }
                    float swg[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = min(n_base + wave_n * 16 * WTN + i * 16 + quad * 4 + r, N - 1);
                        swg[r] = weight_group ? swr[n] : 1.f;
                    }
#pragma unroll
                    for (int j = 0; j < WTM; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            facc[i][j][r] = __builtin_fmaf(float(part[j][r]), sxg[j] * swg[r],
                                                           facc[i][j][r]);
                }
            }
        }
    } else if constexpr (Fmt == FP8 && WTN * WTM > 8) {
        // FP8 K groups on wave tiles of more than 8 MFMA tiles (the 256x128
        // tile's 64x64 waves): one 128-K group per stage, stage-synchronous
        // (the software-pipelined form below needs a second set of i32x8
        // fragments that these waves have no registers for: it spilled and
        // ran slower; so did a double-buffered form reading weight fragments
        // a block ahead, 42-45 VGPRs). Stages wait for themselves; the group
        // scales are the stage slot's scale rows.
        for (int s = 0; s < stages; ++s) {
            // Stage s has landed once at most the newer stages are outstanding.
            if (s + STAGES - 2 < stages) wait_ring(std::integral_constant<int, STAGES - 2>{});
            else wait_vmcnt<0>();
            __syncthreads();
            if (s + STAGES - 1 < stages) issue(s + STAGES - 1, (s + STAGES - 1) * BK);
            const uint8_t *cur = lds + (s % STAGES) * STAGE_BYTES;
            const float *slot = reinterpret_cast<const float *>(cur + ROWS * BK);
            // One 128-wide K group per stage: r = fmaf(p, sxg*swg, r).
            float sxg[WTM];
#pragma unroll
            for (int j = 0; j < WTM; ++j)
                sxg[j] = slot[256 + wave_m * 16 * WTM + j * 16 + row16];
#pragma unroll
            for (int i = 0; i < WTN; ++i) {
                Acc part[WTM];
#pragma unroll
                for (int j = 0; j < WTM; ++j) part[j] = Acc{0, 0, 0, 0};
                if constexpr (Fmt == I8) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const i32x4 af = frag16(cur, a_row0 + i * 16, h);
#pragma unroll
                        for (int j = 0; j < WTM; ++j)
                            MMA::run(part[j], af, frag16(cur, b_row0 + j * 16, h));
                    }
                } else {
                    const i32x8 af = frag32(cur, a_row0 + i * 16);
#pragma unroll
                    for (int j = 0; j < WTM; ++j)
                        MMA::run(part[j], af, frag32(cur, b_row0 + j * 16));
                }
                float swg[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    swg[r] = slot[wave_n * 16 * WTN + i * 16 + quad * 4 + r];
#pragma unroll
                for (int j = 0; j < WTM; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        facc[i][j][r] =
                            __builtin_fmaf(float(part[j][r]), sxg[j] * swg[r], facc[i][j][r]);
            }
        }
    } else {
        // K groups of 128: the per-channel software pipeline (fragments of
        // stage s+1 read while stage s's MFMAs run). Each group's MFMAs
        // accumulate natively (exact int32 for INT8; fp32 from zero for FP8)
        // and the group is applied as facc = fmaf(p, sx_g * sw_g, facc),
        // groups ascending. The group's scales come with its last stage (the
        // stage slot's scale rows). INT8 on 64-byte stages (two per group) or
        // 128-byte stages (one group per stage, two MFMAs per tile); FP8 on
        // 128-byte stages with wave tiles of at most 8 MFMA tiles.
        static_assert(Fmt == I8 || BK == 128, "FP8 K groups use 128-byte stages");
        using Frag = std::conditional_t<BK == 64, i32x4, i32x8>;
        const int a_off = a_row0 * BK, b_off = b_row0 * BK;
        const int a_c0 = (quad ^ swizzle<BK>(a_row0)) * 16, b_c0 = (quad ^ swizzle<BK>(b_row0)) * 16;
        const int a_c1 = ((4 + quad) ^ swizzle<BK>(a_row0)) * 16;
        const int b_c1 = ((4 + quad) ^ swizzle<BK>(b_row0)) * 16;
        auto frag = [&](const uint8_t *p, int c0, int c1) {
            const i32x4 lo = *reinterpret_cast<const i32x4 *>(p + c0);
            if constexpr (BK == 64) {
                return lo;
            } else {
                const i32x4 hi = *reinterpret_cast<const i32x4 *>(p + c1);
                return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
        };
        auto read = [&](int st, Frag (&a)[WTN], Frag (&bb)[WTM]) {
            const uint8_t *cur = lds + (st % STAGES) * STAGE_BYTES;
            const uint8_t *pa = cur + a_off, *pb = cur + b_off;
#pragma unroll
            for (int j = 0; j < WTM; ++j) bb[j] = frag(pb + j * 16 * BK, b_c0, b_c1);
#pragma unroll
            for (int i = 0; i < WTN; ++i) a[i] = frag(pa + i * 16 * BK, a_c0, a_c1);
        };
      // Two banks of partials (tiles of at most 8 MFMA tiles per wave, i.e.
      // 128x128 with eight 64x32 waves): group g accumulates in bank g % 2,
      // and its conversion and fma are spread over group g+1's first stage,
      // one MFMA of the other bank between every 12 of them (gfx950 overlaps
      // VALU and MFMA work only a little, so this gains 5-13%, not the whole
      // rescale). Larger wave tiles have no registers for the second bank
      // (it spilled on 256x128) and apply each group at its last stage.
      constexpr bool kTwoBanks = WTN * WTM <= 8 && SPG == 2;
      static_assert(STAGES >= 3, "the K-group software pipeline keeps a stage in flight");
      if constexpr (kTwoBanks) {
        Acc pp[2][WTN][WTM];
        float xg[WTM];
        f32x4 wg[WTN];
        // Scales of group g from its last stage's slot (read before that
        // step's barrier: the next step's DMA refills the slot).
        auto load_scales = [&](int st) {
            const float *slot = reinterpret_cast<const float *>(lds + (st % STAGES) * STAGE_BYTES +
                                                                ROWS * BK);
#pragma unroll
            for (int j = 0; j < WTM; ++j)
                xg[j] = slot[256 + wave_m * 16 * WTM + j * 16 + row16];
#pragma unroll
            for (int i = 0; i < WTN; ++i)
                wg[i] = *reinterpret_cast<const f32x4 *>(slot + wave_n * 16 * WTN + i * 16 +
                                                         quad * 4);
        };
        auto apply = [&](auto bank_) {
            constexpr int B = decltype(bank_)::value;
#pragma unroll
            for (int i = 0; i < WTN; ++i)
#pragma unroll
                for (int j = 0; j < WTM; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        facc[i][j][r] = __builtin_fmaf(float(pp[B][i][j][r]), xg[j] * wg[i][r],
                                                       facc[i][j][r]);
        };
        // One stage into bank B. In the main loop every flag is a compile-time
        // constant and every stage-bound check is known to pass (Check =
        // false), so the step has no branches and the compiler interleaves
        // the previous group's conversion and fma with this stage's MFMAs;
        // the first group and the last stages run with run-time checks.
        auto step = [&](int s, auto bank_, auto first_, auto last_, auto apply_, auto check_,
                        const Frag (&a)[WTN], const Frag (&bb)[WTM], Frag (&na)[WTN],
                        Frag (&nb)[WTM]) {
            constexpr int B = decltype(bank_)::value;
            constexpr bool Check = decltype(check_)::value;
            const bool first = Check ? s % SPG == 0 : decltype(first_)::value;
            const bool last = Check ? (s % SPG == SPG - 1 || s + 1 == stages) : decltype(last_)::value;
            const bool apply_prev = Check ? (first && s > 0) : decltype(apply_)::value;
            // Without checks and with the previous group to apply, each MFMA
            // of this bank is followed by the 12 VALU operations (convert,
            // scale product, fma for 4 elements) of the other bank's same
            // tile, in that order.
            constexpr bool kInterleave = !Check && decltype(apply_)::value;
#pragma unroll
            for (int i = 0; i < WTN; ++i)
#pragma unroll
                for (int j = 0; j < WTM; ++j) {
                    if (first) pp[B][i][j] = Acc{0, 0, 0, 0};
                    MMA::run(pp[B][i][j], a[i], bb[j]);
                    if constexpr (kInterleave) {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            facc[i][j][r] = __builtin_fmaf(float(pp[1 - B][i][j][r]),
                                                           xg[j] * wg[i][r], facc[i][j][r]);
                    }
                }
            if constexpr (kInterleave) {
#pragma unroll
                for (int k = 0; k < WTN * WTM; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);  // twelve VALU
                }
                // Keep the updated accumulators in this step (not moved to a
                // loop boundary, away from the MFMAs they interleave with).
#pragma unroll
                for (int i = 0; i < WTN; ++i)
#pragma unroll
                    for (int j = 0; j < WTM; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(facc[i][j][r]));
            } else if (apply_prev) {
                apply(std::integral_constant<int, 1 - B>{});
            }
            // The next DMA after this stage's MFMAs: its control flow would
            // otherwise split the MFMA / VALU region.
            if (!Check || s + STAGES - 1 < stages) issue(s + STAGES - 1, (s + STAGES - 1) * BK);
            if (last) load_scales(s);
            if (!Check || s + STAGES - 1 < stages) wait_ring(std::integral_constant<int, STAGES - 2>{});
            else if (s + 1 < stages) wait_vmcnt<0>();
            lds_barrier();
            if (!Check || s + 1 < stages) read(s + 1, na, nb);
        };
        using B0 = std::integral_constant<int, 0>;
        using B1 = std::integral_constant<int, 1>;
        using T = std::true_type;
        using F = std::false_type;
        Frag a0[WTN], b0[WTM], a1[WTN], b1[WTM];
        if (stages >= STAGES - 1) wait_ring(std::integral_constant<int, STAGES - 2>{});
        else wait_vmcnt<0>();
        lds_barrier();
        read(0, a0, b0);
        // Group 0 (bank 0), checked.
        step(0, B0{}, F{}, F{}, F{}, T{}, a0, b0, a1, b1);
        if (1 < stages) step(1, B0{}, F{}, F{}, F{}, T{}, a1, b1, a0, b0);
        // Groups 1, 2, ... in pairs (banks 1, 0) while all four stages and
        // their DMAs lie inside K.
        int s = 2;
        for (; s + 3 + STAGES - 1 < stages; s += 4) {
            step(s, B1{}, T{}, F{}, T{}, F{}, a0, b0, a1, b1);
            step(s + 1, B1{}, F{}, T{}, F{}, F{}, a1, b1, a0, b0);
            step(s + 2, B0{}, T{}, F{}, T{}, F{}, a0, b0, a1, b1);
            step(s + 3, B0{}, F{}, T{}, F{}, F{}, a1, b1, a0, b0);
        }
        // The remaining stages (at most STAGES + 2), checked; s is even here,
        // so stage s opens a group of bank 1.
        for (; s < stages; s += 4) {
            step(s, B1{}, F{}, F{}, F{}, T{}, a0, b0, a1, b1);
            if (s + 1 < stages) step(s + 1, B1{}, F{}, F{}, F{}, T{}, a1, b1, a0, b0);
            if (s + 2 < stages) step(s + 2, B0{}, F{}, F{}, F{}, T{}, a0, b0, a1, b1);
            if (s + 3 < stages) step(s + 3, B0{}, F{}, F{}, F{}, T{}, a1, b1, a0, b0);
        }
        if (((stages - 1) / SPG) % 2 == 0) apply(B0{});
        else apply(B1{});
      } else {
        // One set of partials: group g's MFMAs accumulate natively (exact
        // int32 for INT8) and the group is applied at its last stage.
        // With two waves per SIMD the other wave's MFMAs run while one wave
        // waits for its last MFMA result.
        Acc part[WTN][WTM];
        auto apply = [&](int st) {
            const float *slot = reinterpret_cast<const float *>(lds + (st % STAGES) * STAGE_BYTES +
                                                                ROWS * BK);
            float xg[WTM];
#pragma unroll
            for (int j = 0; j < WTM; ++j)
                xg[j] = slot[256 + wave_m * 16 * WTM + j * 16 + row16];
#pragma unroll
            for (int i = 0; i < WTN; ++i) {
                const f32x4 wg =
                    *reinterpret_cast<const f32x4 *>(slot + wave_n * 16 * WTN + i * 16 + quad * 4);
#pragma unroll
                for (int j = 0; j < WTM; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        facc[i][j][r] =
                            __builtin_fmaf(float(part[i][j][r]), xg[j] * wg[r], facc[i][j][r]);
            }
        };
        // One stage: MFMAs into part (from zero on the group's first stage),
        // the group applied on its last stage from the scale rows of this
        // stage's slot (read before the barrier: the next step's DMA refills
        // the slot); then the ring wait, barrier and the next stage's
        // fragment reads.
        // first_ / last_: 1 or 0 when the caller knows whether stage s opens
        // or closes its group (the main loop), 2 to decide at run time. A
        // known first stage starts its MFMAs from an inline zero accumulator
        // instead of zeroing the partials with moves.
        auto step = [&](int s, auto first_, auto last_, const Frag (&a)[WTN],
                        const Frag (&bb)[WTM], Frag (&na)[WTN], Frag (&nb)[WTM]) {
            constexpr int FC = decltype(first_)::value, LC = decltype(last_)::value;
            const bool first = FC == 2 ? s % SPG == 0 : FC == 1;
            const bool last = LC == 2 ? (s % SPG == SPG - 1 || s + 1 == stages) : LC == 1;
            if (s + STAGES - 1 < stages) issue(s + STAGES - 1, (s + STAGES - 1) * BK);
#pragma unroll
            for (int i = 0; i < WTN; ++i)
#pragma unroll
                for (int j = 0; j < WTM; ++j) {
                    if (first) part[i][j] = Acc{0, 0, 0, 0};
                    MMA::run(part[i][j], a[i], bb[j]);
                }
            if (last) apply(s);
            if (s + STAGES - 1 < stages) wait_ring(std::integral_constant<int, STAGES - 2>{});
            else if (s + 1 < stages) wait_vmcnt<0>();
            lds_barrier();
            // i32x8 fragments: unconditional, as in the per-channel pipeline.
            if (BK == 128 || s + 1 < stages) read(s + 1, na, nb);
        };
        using C0 = std::integral_constant<int, 0>;
        using C1 = std::integral_constant<int, 1>;
        using C2 = std::integral_constant<int, 2>;
        // In the loop s is even: with two stages per group, stage s opens
        // and stage s+1 closes a group; with one, every stage does both.
        using F0 = C1;
        using L0 = std::conditional_t<SPG == 1, C1, C0>;
        using F1 = std::conditional_t<SPG == 1, C1, C0>;
        using L1 = C1;
        static_assert(SPG == 1 || SPG == 2, "stages per K group");
        Frag a0[WTN], b0[WTM], a1[WTN], b1[WTM];
        if (stages >= STAGES - 1) wait_ring(std::integral_constant<int, STAGES - 2>{});
        else wait_vmcnt<0>();
        lds_barrier();
        read(0, a0, b0);
        int s = 0;
        for (; s + 1 < stages; s += 2) {
            step(s, F0{}, L0{}, a0, b0, a1, b1);
            step(s + 1, F1{}, L1{}, a1, b1, a0, b0);
        }
        if (s < stages) step(s, C2{}, C2{}, a0, b0, a1, b1);
      }
    }

    // Epilogue. A lane holds C[n = 4*quad + r][m = row16] of each 16x16 tile:
    // scale, round to 16-bit, and transpose through LDS (the stage ring is
    // free now) so that each token row of the wave's sub-tile leaves as
    // contiguous 16-byte stores. Row m_l of the wave's [16*WTM][16*WTN]
    // buffer keeps 16-byte chunk c at c ^ (m_l % CH): conflict-free both for
    // the 8-byte column writes and the row reads.
    constexpr int TM = 16 * WTM, TN = 16 * WTN, ROWB = TN * 2, CH = ROWB / 16;
    lds_barrier();
    uint8_t *wbuf = lds + wave * TM * ROWB;
    auto emit = [&](int m_l, int n_l, const float (&v)[4]) {
        uint2 packed;
        packed.x = pack2(v[0], v[1], Out{});
        packed.y = pack2(v[2], v[3], Out{});
        const int byte = n_l * 2;
        *reinterpret_cast<uint2 *>(wbuf + m_l * ROWB + (((byte >> 4) ^ (m_l % CH)) << 4) +
                                   (byte & 15)) = packed;
    };
    if constexpr (kAcc32) {
        // 32x32 tile: lane l, register 4b+e holds C[n = 8b + 4*(l/32) + e][m = l % 32].
#pragma unroll
        for (int j = 0; j < WTM / 2; ++j) {
            const int m_l = j * 32 + (lane & 31);
            const float sxm = scl[BN + wave_m * TM + m_l];
#pragma unroll
            for (int i = 0; i < WTN / 2; ++i)
#pragma unroll
                for (int blk = 0; blk < 4; ++blk) {
                    const int n_l = i * 32 + blk * 8 + (lane >> 5) * 4;
                    const f32x4 swv = *reinterpret_cast<const f32x4 *>(scl + wave_n * TN + n_l);
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float t = acc32[i][j][blk * 4 + e] * sxm;
                        v[e] = t * swv[e];
                    }
                    if constexpr (kFin) finish4<Out>(v, bias, n_base + wave_n * TN + n_l, N - 1, act);
                    emit(m_l, n_l, v);
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < WTM; ++j) {
            const int m_l = j * 16 + row16;
            const float sxm = scl[BN + wave_m * TM + m_l];
#pragma unroll
            for (int i = 0; i < WTN; ++i) {
                const f32x4 swv =
                    *reinterpret_cast<const f32x4 *>(scl + wave_n * TN + i * 16 + quad * 4);
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (Grouped) {
                        // Unit scales stand in for per-K-group ones: 1*s and
                        // s*1 are exact, so this is (sx or 1) * (sw or 1).
                        const float outer = sxm * swv[r];
                        v[r] = (0.f + facc[i][j][r]) * outer;
                    } else {
                        float t = float(acc[i][j][r]) * sxm;
                        v[r] = t * swv[r];
                    }
                }
                if constexpr (kFin)
                    finish4<Out>(v, bias, n_base + wave_n * TN + i * 16 + quad * 4, N - 1, act);
                emit(m_l, i * 16 + quad * 4, v);
            }
        }
    }
    const bool vec16 = (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
    for (int r0 = 0; r0 < TM; r0 += 64 / CH) {
        const int m_l = r0 + lane / CH, c = lane % CH;
        const uint4 val =
            *reinterpret_cast<const uint4 *>(wbuf + m_l * ROWB + ((c ^ (m_l % CH)) << 4));
        const int m = m_base + wave_m * TM + m_l, n = n_base + wave_n * TN + c * 8;
        if (m >= M || n >= N) continue;
        uint16_t *dst = static_cast<uint16_t *>(y) + size_t(m) * N + n;
        if (vec16) {
            store_out16(dst, val);
        } else {
            reinterpret_cast<uint2 *>(dst)[0] = make_uint2(val.x, val.y);
            reinterpret_cast<uint2 *>(dst)[1] = make_uint2(val.z, val.w);
        }
    }
}

// Per-channel GEMM on 32x32 MFMA tiles with 128x128 wave tiles
// (INT8: v_mfma_i32_32x32x32_i8; FP8: v_mfma_f32_32x32x64_f8f6f4),
// WN x WM wave64s, one wave per SIMD. LDS traffic per MFMA op is what bounds
// the 128x64-wave kernel above on gfx950 (~128 B/clk per CU for ds_read_b128
// plus the global->LDS writes): a 128x128 wave tile reads (128+128)*64 bytes
// of fragments per 128*128*64 MACs, 2/3 of the 128x64 tile's bytes per MAC.
// The K ring is the same: 64-byte stages filled by buffer_load ... lds, 16-byte
// chunk c of stage row r at c ^ ((r >> 2) & 3) (conflict-free for 32-row
// fragment reads, where lanes l and l+32 read chunks 2h and 2h+1).
template <int Fmt, int WN, int WM, int STAGES, bool KFull, class Out, bool PackedW = false>
__global__ __launch_bounds__(64 * WN * WM, 1) void wide_gemm(
    const uint8_t *__restrict__ x, const float *__restrict__ sx, const uint8_t *__restrict__ w,
    const float *__restrict__ sw, void *__restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n, const uint16_t *__restrict__ bias, int act) {
    constexpr int NW = WN * WM, BN = 128 * WN, BM = 128 * WM, BK = 64, RPI = 16;
    constexpr int ROWS = BN + BM, INSTS = ROWS / (RPI * NW), W_INSTS = BN / (RPI * NW);
    constexpr int STAGE_BYTES = ROWS * BK;
    static_assert(ROWS % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "stage rows per instruction");
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

    const int tiles = tiles_m * tiles_n;
    int b = blockIdx.x;
    if (tiles % 8 == 0) b = (b % 8) * (tiles / 8) + b / 8;
    constexpr int kGroupN = 4;
    const int group = b / (kGroupN * tiles_m), in_group = b % (kGroupN * tiles_m);
    const int group_w = min(kGroupN, tiles_n - group * kGroupN);
    const int tn = group * kGroupN + in_group % group_w, tm = in_group / group_w;
    const int n_base = tn * BN, m_base = tm * BM;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave_n = wave % WN, wave_m = wave / WN;

    // Packed weights: the tile's row groups are (n_base/16 ..) x tiles_k 1 KB tiles.
    const int tiles_k = (K + 63) / 64;
    const __amdgpu_buffer_rsrc_t rsrc_w =
        PackedW ? __builtin_amdgcn_make_buffer_rsrc(
                      const_cast<uint8_t *>(w + size_t(n_base / 16) * tiles_k * 1024), 0,
                      min(BN, N - n_base) / 16 * tiles_k * 1024, 0x00020000)
                : __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w + size_t(n_base) * K),
                                                    0, min(BN, N - n_base) * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc_x = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(x + size_t(m_base) * K), 0, min(BM, M - m_base) * K, 0x00020000);

    // Load instruction i of this wave writes stage rows [(i*NW + wave)*16, +16)
    // in lane order (row += lane / 4, physical chunk lane % 4); the first row
    // is a multiple of 16, so the lane's logical source chunk is fixed.
    const int lane_row = lane >> 2;
    const int lane_chunk = (lane & 3) ^ ((lane >> 4) & 3);
    const uint32_t lane_voff = uint32_t(lane_row) * uint32_t(K) + uint32_t(lane_chunk * 16);
    // Packed weights: 16-row x 64-K tiles, chunk (c * 16 + row % 16).
    const uint32_t lane_voff_p = uint32_t(lane_chunk * 256 + lane_row * 16);
    constexpr int kRingBytes = STAGES * STAGE_BYTES > NW * 128 * 256 ? STAGES * STAGE_BYTES
                                                                      : NW * 128 * 256;
    float *scl = reinterpret_cast<float *>(lds + kRingBytes);
    const int stages = (K + BK - 1) / BK;
    auto issue = [&](int stage, int k0) {
        uint8_t *base = lds + (stage % STAGES) * STAGE_BYTES;
        const bool kin = KFull || k0 + lane_chunk * 16 < K;
        const uint32_t voff = kin ? lane_voff + uint32_t(k0) : 0x80000000u;
        const uint32_t voff_p = kin ? lane_voff_p : 0x80000000u;
#pragma unroll
        for (int i = 0; i < INSTS; ++i) {
            const int row = (i * NW + wave) * RPI;
            lds_ptr_t dst = (lds_ptr_t)(base + (i * NW + wave) * 1024);
            if (PackedW && i < W_INSTS) {
                const uint32_t soff = uint32_t((row / 16) * tiles_k * 1024 + (k0 / 64) * 1024);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_w, dst, 16, voff_p, soff, 0, 0);
            } else {
                const uint32_t soff = uint32_t(i < W_INSTS ? row : row - BN) * uint32_t(K);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(i < W_INSTS ? rsrc_w : rsrc_x, dst, 16,
                                                         voff, soff, 0, 0);
            }
        }
    };

    // Tile scales to LDS past the ring (read by the epilogue).
    constexpr int kScaleLoads = (BN + BM + 64 * NW - 1) / (64 * NW);
    float scale_v[kScaleLoads];
#pragma unroll
    for (int l = 0; l < kScaleLoads; ++l) {
        const int i = tid + l * 64 * NW;
        float v = 1.f;
        if (i < BN) v = sw[min(n_base + i, N - 1)];
        else if (i < BN + BM) v = sx[min(m_base + i - BN, M - 1)];
        scale_v[l] = v;
    }
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
        if (s < stages) issue(s, s * BK);
#pragma unroll
    for (int l = 0; l < kScaleLoads; ++l)
        if (tid + l * 64 * NW < BN + BM) scl[tid + l * 64 * NW] = scale_v[l];

    // Fragment reads: lane l covers row l % 32 of a 32-row tile; tiles t of
    // the wave's A (weights) and B (tokens) rows are 32*64 bytes apart.
    const int swz = (lane >> 2) & 3, g = lane >> 5;
    const int a_off = (wave_n * 128 + (lane & 31)) * BK;
    const int b_off = (BN + wave_m * 128 + (lane & 31)) * BK;
    const int c0 = ((2 * 0 + g) ^ swz) * 16, c1 = ((2 * 1 + g) ^ swz) * 16;  // INT8 sub-steps
    const int f0 = ((2 * g) ^ swz) * 16, f1 = ((2 * g + 1) ^ swz) * 16;      // FP8 halves

    using Acc = std::conditional_t<Fmt == I8, i32x16, f32x16>;
    Acc acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    if constexpr (Fmt == I8) {
        // Iteration s: read sub-step 1 of stage s while sub-step 0's MFMAs
        // run; barrier (stage s fully read by every wave, stage s+1 landed);
        // refill stage s's buffer with stage s+STAGES; read sub-step 0 of
        // stage s+1 while sub-step 1's MFMAs run.
        auto read = [&](int st, int h, i32x4 (&fa)[4], i32x4 (&fb)[4]) {
            const uint8_t *cur = lds + (st % STAGES) * STAGE_BYTES;
            const int c = h ? c1 : c0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                fa[t] = *reinterpret_cast<const i32x4 *>(cur + a_off + t * 32 * BK + c);
                fb[t] = *reinterpret_cast<const i32x4 *>(cur + b_off + t * 32 * BK + c);
            }
        };
        auto mma = [&](const i32x4 (&fa)[4], const i32x4 (&fb)[4]) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        };
        i32x4 a0[4], b0[4], a1[4], b1[4];
        if (stages >= STAGES) wait_vmcnt<INSTS * (STAGES - 1)>();
        else wait_vmcnt<0>();
        lds_barrier();
        read(0, 0, a0, b0);
        for (int s = 0; s < stages; ++s) {
            read(s, 1, a1, b1);
            mma(a0, b0);
            if (s + STAGES - 1 < stages) wait_vmcnt<INSTS * (STAGES - 2)>();
            else wait_vmcnt<0>();
            lds_barrier();
            if (s + STAGES < stages) issue(s + STAGES, (s + STAGES) * BK);
            if (s + 1 < stages) read(s + 1, 0, a0, b0);
            mma(a1, b1);
        }
    } else {
        // FP8: one 32x32x64 MFMA per tile pair per stage. Sub-step 0 = A
        // fragments + token tiles 0-1, sub-step 1 = token tiles 2-3.
        auto frag = [&](const uint8_t *p) {
            const i32x4 lo = *reinterpret_cast<const i32x4 *>(p + f0);
            const i32x4 hi = *reinterpret_cast<const i32x4 *>(p + f1);
            return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        };
        auto read0 = [&](int st, i32x8 (&fa)[4], i32x8 (&fb)[2]) {
            const uint8_t *cur = lds + (st % STAGES) * STAGE_BYTES;
#pragma unroll
            for (int t = 0; t < 4; ++t) fa[t] = frag(cur + a_off + t * 32 * BK);
#pragma unroll
            for (int t = 0; t < 2; ++t) fb[t] = frag(cur + b_off + t * 32 * BK);
        };
        auto read1 = [&](int st, i32x8 (&fb)[2]) {
            const uint8_t *cur = lds + (st % STAGES) * STAGE_BYTES;
#pragma unroll
            for (int t = 0; t < 2; ++t) fb[t] = frag(cur + b_off + (t + 2) * 32 * BK);
        };
        auto mma = [&](const i32x8 (&fa)[4], const i32x8 (&fb)[2], int j0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j0 + j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fa[i], fb[j], acc[i][j0 + j], 0, 0, 0, 0, 0, 0);
        };
        // Stage s uses A fragments fa (read during stage s-1); the next
        // stage's go to the other set, so that the loop, unrolled by two,
        // carries no fragment copies between iterations.
        i32x8 fa0[4], fa1[4], fb0[2], fb1[2];
        auto step = [&](int s, const i32x8 (&fa)[4], i32x8 (&na)[4]) {
            read1(s, fb1);
            mma(fa, fb0, 0);
            if (s + STAGES - 1 < stages) wait_vmcnt<INSTS * (STAGES - 2)>();
            else wait_vmcnt<0>();
            lds_barrier();
            if (s + STAGES < stages) issue(s + STAGES, (s + STAGES) * BK);
            mma(fa, fb1, 2);
            // Unconditional (after the last stage it reads a ring slot whose
            // fragments go unused): a conditional read here makes the
            // compiler copy every fragment register at each stage.
            read0(s + 1, na, fb0);
        };
        if (stages >= STAGES) wait_vmcnt<INSTS * (STAGES - 1)>();
        else wait_vmcnt<0>();
        lds_barrier();
        read0(0, fa0, fb0);
        int s = 0;
        for (; s + 1 < stages; s += 2) {
            step(s, fa0, fa1);
            step(s + 1, fa1, fa0);
        }
        if (s < stages) step(s, fa0, fa1);
    }

    // Epilogue: scale, round, transpose through LDS (the ring is free after
    // the barrier), 16-byte row stores. Lane l, register 4b+e of tile (i, j)
    // holds C[n = 32i + 8b + 4*(l/32) + e][m = 32j + l % 32].
    constexpr int TM = 128, TN = 128, ROWB = TN * 2, CH = ROWB / 16;
    lds_barrier();
    uint8_t *wbuf = lds + wave * TM * ROWB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m_l = j * 32 + (lane & 31);
        const float sxm = scl[BN + wave_m * TM + m_l];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int blk = 0; blk < 4; ++blk) {
                const int n_l = i * 32 + blk * 8 + g * 4;
                const f32x4 swv = *reinterpret_cast<const f32x4 *>(scl + wave_n * TN + n_l);
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float t = float(acc[i][j][blk * 4 + e]) * sxm;
                    v[e] = t * swv[e];
                }
                if constexpr (kFin) finish4<Out>(v, bias, n_base + wave_n * TN + n_l, N - 1, act);
                uint2 packed;
                packed.x = pack2(v[0], v[1], Out{});
                packed.y = pack2(v[2], v[3], Out{});
                const int byte = n_l * 2;
                *reinterpret_cast<uint2 *>(wbuf + m_l * ROWB + (((byte >> 4) ^ (m_l % CH)) << 4) +
                                           (byte & 15)) = packed;
            }
    }
    const bool vec16 = (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll 4
    for (int r0 = 0; r0 < TM; r0 += 64 / CH) {
        const int m_l = r0 + lane / CH, c = lane % CH;
        const uint4 val =
            *reinterpret_cast<const uint4 *>(wbuf + m_l * ROWB + ((c ^ (m_l % CH)) << 4));
        const int m = m_base + wave_m * TM + m_l, n = n_base + wave_n * TN + c * 8;
        if (m >= M || n >= N) continue;
        uint16_t *dst = static_cast<uint16_t *>(y) + size_t(m) * N + n;
        if (vec16) {
            store_out16(dst, val);
        } else {
            reinterpret_cast<uint2 *>(dst)[0] = make_uint2(val.x, val.y);
            reinterpret_cast<uint2 *>(dst)[1] = make_uint2(val.z, val.w);
        }
    }
}

template <int Fmt, int WN, int WM, int STAGES, class Out>
int launch_wide(const GemmArgs &a, hipStream_t stream) {
    constexpr int BN = 128 * WN, BM = 128 * WM;
    const int tiles_n = (a.N + BN - 1) / BN, tiles_m = (a.M + BM - 1) / BM;
    const size_t lds = std::max(size_t(STAGES) * (BN + BM) * 64, size_t(WN * WM) * 128 * 256) +
                       size_t(BN + BM) * 4;
    dim3 grid(unsigned(tiles_n * tiles_m)), block(64 * WN * WM);
#define QLIN_WIDE(KF, PW)                                                                      \
    hipLaunchKernelGGL((wide_gemm<Fmt, WN, WM, STAGES, KF, Out, PW>), grid, block, lds, stream, \
                       a.x, a.sx, a.w, a.sw, a.y, a.M, a.N, a.K, tiles_m, tiles_n, a.bias, a.act)
    if (a.K % 64 == 0) { if (a.packed) QLIN_WIDE(true, true); else QLIN_WIDE(true, false); }
    else { if (a.packed) QLIN_WIDE(false, true); else QLIN_WIDE(false, false); }
#undef QLIN_WIDE
    return 0;
}

template <int Fmt, int WN, int WM, int WTN, int WTM, int BK, int STAGES, bool Grouped, class Out,
          int GS = 128>
int launch_shape(const GemmArgs &a, hipStream_t stream) {
    constexpr int BN = 16 * WTN * WN, BM = 16 * WTM * WM;
    const int tiles_n = (a.N + BN - 1) / BN, tiles_m = (a.M + BM - 1) / BM;
    const size_t stage = size_t(BN + BM) * BK + (Grouped && GS == 128 ? 3072 : 0);
    const size_t lds = std::max(size_t(STAGES) * stage, size_t(BN) * BM * 2) + size_t(BN + BM) * 4;
    dim3 grid(unsigned(tiles_n * tiles_m)), block(64 * WN * WM);
#define QLIN_TILED(KF, PW)                                                                      \
    hipLaunchKernelGGL((tiled_gemm<Fmt, WN, WM, WTN, WTM, BK, STAGES, Grouped, KF, Out, PW, GS>), \
                       grid, block, lds, stream, a.x, a.sx, a.w, a.sw, a.y, a.M, a.N, a.K,      \
                       tiles_m, tiles_n, a.input_group, a.weight_group, a.bias, a.act)
    if (a.K % BK == 0) { if (a.packed) QLIN_TILED(true, true); else QLIN_TILED(true, false); }
    else { if (a.packed) QLIN_TILED(false, true); else QLIN_TILED(false, false); }
#undef QLIN_TILED
    return 0;
}

// K groups of 32 / 64 (GS, the smaller of the two operands' sizes) on
// 128-byte stages, eight waves: 256x128 (128x32 waves, INT8 only: the FP8
// tile spills) or 128x128 (64x32).
template <int Fmt, class Out, int GS>
int dispatch_small_groups(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    if constexpr (Fmt == I8)
        if (p.channels == 256 && p.tokens == 128 && p.waves == 8)
            return launch_shape<Fmt, 2, 4, 8, 2, 128, 3, true, Out, GS>(a, s);
    if (p.channels == 128 && p.tokens == 128 && p.waves == 8)
        return launch_shape<Fmt, 2, 4, 4, 2, 128, 4, true, Out, GS>(a, s);
    return -4;
}

// Macro tiles (weight rows x tokens) and waves per path: 256x256 with eight
// waves of 128x64 (waves 8) or four of 128x128 on 32x32 MFMAs (wide_gemm,
// waves 4); 256x128 with eight waves of 128x32 (8), one workgroup of four
// 128x64 waves (1) or two 128x128 waves (2); 128x128 with eight waves of
// 64x32 (8) or four of 64x64 (1).
template <int Fmt, bool Grouped, class Out>
int dispatch_shape(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    if constexpr (Grouped) {
        // No 256x256: the fp32 group accumulators would double the 128x128
        // register tile per wave and spill. FP8 in 128-byte stages; INT8 in
        // 128-byte stages on the 8-wave 128x128 and 128x64 tiles, 64-byte
        // stages (two per group) elsewhere: its 256x128 tile spilled on
        // 128-byte stages, and the 4-wave 128x64 tile runs two accumulator
        // banks.
        constexpr int GBK = Fmt == I8 ? 64 : 128;
        // 256x128, eight 64x64 waves: FP8 on two 128-byte stages in the
        // stage-synchronous loop (group_fp8 at 4096 1.44 against 1.41 PFLOPS
        // on three); INT8
        // on four 64-byte stages (on 128-byte stages it spills). 64x64 waves
        // read fewer fragment bytes than 128x32 waves: gate_up at 4096
        // INT8 161 us against 165 us, FP8 134 us against 138 us.
        if (p.channels == 256 && p.tokens == 128 && p.waves == 8) {
            if constexpr (Fmt == FP8)
                return launch_shape<Fmt, 4, 2, 4, 4, 128, 2, true, Out>(a, s);
            else
                return launch_shape<Fmt, 4, 2, 4, 4, 64, 4, true, Out>(a, s);
        }
        // 128x128 with eight 64x32 waves, one group per 128-byte stage (qkv
        // at 1024 23.7 us against 25.0 us for INT8's two-bank 64-byte-stage
        // pipeline, which the four-wave 128x64 tile keeps).
        if (p.channels == 128 && p.tokens == 128 && p.waves == 8)
            return launch_shape<Fmt, 2, 4, 4, 2, 128, 4, true, Out>(a, s);
        if (p.channels == 128 && p.tokens == 128)
            return launch_shape<Fmt, 2, 2, 4, 4, GBK, 4, true, Out>(a, s);
        if (p.channels == 128 && p.tokens == 64 && p.waves == 4)
            return launch_shape<Fmt, 2, 2, 4, 2, GBK, 4, true, Out>(a, s);
        // 128x64 with eight 32x32 waves, one group per 128-byte stage.
        if (p.channels == 128 && p.tokens == 64 && p.waves == 8)
            return launch_shape<Fmt, 4, 2, 2, 2, 128, 4, true, Out>(a, s);
        return -4;
    } else if constexpr (Fmt == I8) {
        // 256x128 with eight waves of 64x64 over 128-byte K stages (two
        // MFMAs per tile and stage, half the barriers of 64-byte stages:
        // down at 4096 54 us against 59 us, o_proj 28 against 29). A 64x64
        // wave reads 16 KB of fragments per stage where a 128x32 wave reads
        // 20 KB: down at 4096 46.8 us against 47.8 us.
        if (p.channels == 256 && p.tokens == 128 && p.waves == 8)
            return launch_shape<Fmt, 4, 2, 4, 4, 128, 3, false, Out>(a, s);
        if (p.channels == 256 && p.tokens == 256 && p.waves == 4)
            return launch_wide<Fmt, 2, 2, 4, Out>(a, s);
        if (p.channels == 256 && p.tokens == 128 && p.waves == 2)
            return launch_wide<Fmt, 2, 1, 3, Out>(a, s);
        // 256x256: eight 128x64 waves on two double-buffered 128-byte K
        // stages (gate_up at 4096 87 us against 95 us on four 64-byte stages).
        if (p.channels == 256 && p.tokens == 256 && p.waves == 8)
            return launch_shape<Fmt, 2, 4, 8, 4, 128, 2, false, Out>(a, s);
        if (p.channels == 256 && p.tokens == 128)
            return launch_shape<Fmt, 2, 2, 8, 4, 64, 4, false, Out>(a, s);
        // 128x128: eight waves of 64x32 (waves 8) or four of 64x64 (waves 1).
        // The eight-wave form runs two double-buffered 128-byte stages in
        // 65 KB of LDS, two workgroups per CU (qkv at 1024 12.1 us against
        // 13.0 us on four 64-byte stages).
        if (p.channels == 128 && p.tokens == 128 && p.waves == 8)
            return launch_shape<Fmt, 2, 4, 4, 2, 128, 2, false, Out>(a, s);
        if (p.channels == 128 && p.tokens == 128)
            return launch_shape<Fmt, 2, 2, 4, 4, 64, 4, false, Out>(a, s);
        // 128x64: four waves of 64x32, or eight of 32x32 over 128-byte K
        // stages (down at 1024 25 us against 32 us; 32x32 waves read 8 KB of
        // fragments per stage where 64x16 waves read 10 KB: 18.2 us against
        // 18.7 us).
        if (p.channels == 128 && p.tokens == 64 && p.waves == 4)
            return launch_shape<Fmt, 2, 2, 4, 2, 64, 4, false, Out>(a, s);
        if (p.channels == 128 && p.tokens == 64 && p.waves == 8)
            return launch_shape<Fmt, 4, 2, 2, 2, 128, 4, false, Out>(a, s);
        return -4;
    } else {
        // 256x128 with eight waves of 64x64 on two double-buffered 128-byte
        // K stages (down at 4096 45.5 us against 48.0 us on three stages, and
        // 60 us for one workgroup of four 128x64 waves; 64x64 waves against
        // 128x32: o_proj 18.9 us against 19.2 us).
        if (p.channels == 256 && p.tokens == 128 && p.waves == 8)
            return launch_shape<Fmt, 4, 2, 4, 4, 128, 2, false, Out>(a, s);
        if (p.channels == 256 && p.tokens == 256 && p.waves == 4)
            return launch_wide<Fmt, 2, 2, 4, Out>(a, s);
        if (p.channels == 256 && p.tokens == 128 && p.waves == 2)
            return launch_wide<Fmt, 2, 1, 3, Out>(a, s);
        // 256x256: eight 128x64 waves on two double-buffered 128-byte K stages
        // (gate_up at 4096 90 us against 103 us on four 64-byte stages of
        // 32x32x64 MFMAs).
        if (p.channels == 256 && p.tokens == 256 && p.waves == 8)
            return launch_shape<Fmt, 2, 4, 8, 4, 128, 2, false, Out>(a, s);
        if (p.channels == 256 && p.tokens == 128)
            return launch_shape<Fmt, 2, 2, 8, 4, 64, 4, false, Out>(a, s);
        // 128x128: eight waves of 64x32 on the 16x16x128 FP8 MFMA over
        // 128-byte K stages (waves 8), or four 64x64 waves of 32x32x64 (1).
        // Up to K = 2048 two double-buffered stages, two workgroups per CU
        // (o_proj at 4096 17.8 us against 18.3 us on 256x128, qkv at 1024
        // 11.7 us against 12.0 us on four stages); beyond, four stages (down
        // at 1024 on 128x128: 23.5 us, against 32.5 us double-buffered).
        if (p.channels == 128 && p.tokens == 128 && p.waves == 8) {
            if (a.K <= 2048) return launch_shape<Fmt, 2, 4, 4, 2, 128, 2, false, Out>(a, s);
            return launch_shape<Fmt, 2, 4, 4, 2, 128, 4, false, Out>(a, s);
        }
        if (p.channels == 128 && p.tokens == 128)
            return launch_shape<Fmt, 2, 2, 4, 4, 64, 4, false, Out>(a, s);
        // 128x64: four waves of 64x32 (32x32x64 MFMA) or eight of 32x32
        // (16x16x128 MFMA over 128-byte K stages).
        if (p.channels == 128 && p.tokens == 64 && p.waves == 4)
            return launch_shape<Fmt, 2, 2, 4, 2, 64, 4, false, Out>(a, s);
        if (p.channels == 128 && p.tokens == 64 && p.waves == 8)
            return launch_shape<Fmt, 4, 2, 2, 2, 128, 4, false, Out>(a, s);
        return -4;
    }
}

template <int Fmt, class Out>
int dispatch_grouped(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    const int g = a.input_group && a.weight_group ? std::min(a.input_group, a.weight_group)
                                                  : a.input_group + a.weight_group;
    if (g == 32) return dispatch_small_groups<Fmt, Out, 32>(a, p, s);
    if (g == 64) return dispatch_small_groups<Fmt, Out, 64>(a, p, s);
    if (g) return dispatch_shape<Fmt, true, Out>(a, p, s);
    return dispatch_shape<Fmt, false, Out>(a, p, s);
}

}  // namespace

#ifdef QLIN_TILED_PART
int QLIN_TILED_PART(const GemmArgs &a, const GemmPath &p, hipStream_t stream) {
    if (a.out_type == F16) {
        if (a.fmt == I8) return dispatch_grouped<I8, f16_t>(a, p, stream);
        return dispatch_grouped<FP8, f16_t>(a, p, stream);
    }
    if (a.fmt == I8) return dispatch_grouped<I8, bf16_t>(a, p, stream);
    return dispatch_grouped<FP8, bf16_t>(a, p, stream);
}
#else
size_t tiled_workspace_bytes(const GemmArgs &, const GemmPath &) { return 0; }

int launch_tiled_plain(const GemmArgs &, const GemmPath &, hipStream_t);
int launch_tiled_fin(const GemmArgs &, const GemmPath &, hipStream_t);
int launch_tiled(const GemmArgs &a, const GemmPath &p, hipStream_t stream) {
    return (a.bias || a.act) ? launch_tiled_fin(a, p, stream) : launch_tiled_plain(a, p, stream);
}
#endif

}  // namespace qlin
