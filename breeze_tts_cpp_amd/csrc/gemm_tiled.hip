// Prefill-regime quantized GEMM (hundreds to thousands of tokens) for gfx950.
//
// Same contract as the skinny kernel (y = D(dequant(x . w^T))), replacing the
// reference's tensor-core paths: CUTLASS SM80 INT8 with the EVT epilogue
// D((acc*sx)*sw) (ops/kernels/quant/quant_gemm_sm80.cu:14-82), the SM90 INT8 /
// FP8 WGMMA kernels (quant_gemm_sm90.cu:16-283) and the K-group GEMM
// (quant_grouped.cu:16-169, quant_gemm_sm90.cu:289-372).
//
// Work decomposition: one workgroup per (BN weight rows) x (BM token rows)
// macro tile; 64*WN*WM threads; each wave64 owns a 128 (weight rows) x 64
// (tokens) sub-tile = 8 x 4 MFMA 16x16 tiles, 128 accumulator registers.
// K advances in 128-byte stages through a double-buffered LDS ring: global
// loads for stage s+1 are in flight while stage s feeds the MFMAs. LDS rows
// are 128 bytes; the 16-byte chunk c of row r lives at chunk c ^ ((r>>1)&7),
// which makes both the 16-byte stores and the MFMA fragment reads
// bank-conflict free (16 lanes of a phase hit 16 distinct 16-byte slots).
// The weight tile is the MFMA A operand, so each lane's accumulator holds
// four consecutive output channels of one token: 8-byte output stores.
// Tiles are numbered XCD-major (consecutive tiles on one XCD share its L2).
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

namespace qlin {
namespace {

constexpr int kBK = 128;          // bytes of K per stage (= one K group of 128)
constexpr int kWaveN = 128;       // weight rows per wave
constexpr int kWaveM = 64;        // tokens per wave

// A 128-byte K slice of one MFMA operand row group: 32 bytes per lane, the two
// 16-byte halves covering K [0,64) and [64,128) of the stage.
template <int Fmt> struct TileMma;
template <> struct TileMma<I8> {
    using Acc = i32x4;
    // 128 K = two v_mfma_i32_16x16x64_i8.
    __device__ static void run(Acc &c, const i32x8 &a, const i32x8 &b) {
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(a, a, 0, 1, 2, 3),
                                                  __builtin_shufflevector(b, b, 0, 1, 2, 3), c, 0,
                                                  0, 0);
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_shufflevector(a, a, 4, 5, 6, 7),
                                                  __builtin_shufflevector(b, b, 4, 5, 6, 7), c, 0,
                                                  0, 0);
    }
};
template <> struct TileMma<FP8> {
    using Acc = f32x4;
    // 128 K = one v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3 x e4m3, unit scales).
    __device__ static void run(Acc &c, const i32x8 &a, const i32x8 &b) {
        c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0x7f7f7f7f, 0,
                                                             0x7f7f7f7f);
    }
};

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

template <class Out>
__device__ __forceinline__ void store4(void *y, size_t index, const float (&v)[4]) {
    uint2 packed;
    packed.x = uint32_t(from_float(v[0], Out{})) | (uint32_t(from_float(v[1], Out{})) << 16);
    packed.y = uint32_t(from_float(v[2], Out{})) | (uint32_t(from_float(v[3], Out{})) << 16);
    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + index) = packed;
}

template <int Fmt, int WN, int WM, bool Grouped, bool KFull, class Out>
__global__ __launch_bounds__(64 * WN * WM) void tiled_gemm(
    const uint8_t *__restrict__ x, const float *__restrict__ sx, const uint8_t *__restrict__ w,
    const float *__restrict__ sw, void *__restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n, int input_group, int weight_group) {
    constexpr int BN = kWaveN * WN, BM = kWaveM * WM, T = 64 * WN * WM;
    constexpr int kChunks = (BN + BM) * (kBK / 16);    // 16-byte chunks per stage
    constexpr int kPerThread = kChunks / T;
    static_assert(kChunks % T == 0, "stage chunks must divide evenly");
    using MMA = TileMma<Fmt>;
    using Acc = typename MMA::Acc;

    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int kStageBytes = (BN + BM) * kBK;

    // XCD-major tile numbering: hardware places workgroup b on XCD b % 8.
    const int tiles = tiles_m * tiles_n;
    int b = blockIdx.x;
    if (tiles % 8 == 0) b = (b % 8) * (tiles / 8) + b / 8;
    const int tn = b / tiles_m, tm = b % tiles_m;
    const int n_base = tn * BN, m_base = tm * BM;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wave_n = wave % WN, wave_m = wave / WN;
    const int row16 = lane & 15, quad = lane >> 4;

    // Chunk i of this thread: stage row row0 + i*(T/8), 16-byte column tid&7.
    // Rows [0, BN) are weight rows, [BN, BN+BM) token rows; rows past the
    // matrix edge are clamped to a valid row (their outputs are not stored).
    constexpr int kRowStep = T / 8;
    constexpr int kWeightChunks = BN / kRowStep;
    const int row0 = tid >> 3, chunk0 = tid & 7;
    uint32_t src_off[kPerThread];
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int row = row0 + i * kRowStep;
        if (i < kWeightChunks)
            src_off[i] = uint32_t(min(n_base + row, N - 1)) * uint32_t(K) + chunk0 * 16;
        else
            src_off[i] = uint32_t(min(m_base + row - BN, M - 1)) * uint32_t(K) + chunk0 * 16;
    }
    const int lds_off0 = row0 * kBK + swz(row0, chunk0) * 16;

    Acc acc[Grouped ? 1 : 8][4];
    float facc[Grouped ? 8 : 1][Grouped ? 4 : 1][4];
    if constexpr (!Grouped) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = Acc{0, 0, 0, 0};
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) facc[i][j][r] = 0.f;
    }

    i32x4 staged[kPerThread];
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const uint8_t *base = i < kWeightChunks ? w : x;
            if (KFull || k0 + chunk0 * 16 < K)
                staged[i] = *reinterpret_cast<const i32x4 *>(base + src_off[i] + uint32_t(k0));
            else
                staged[i] = i32x4{0, 0, 0, 0};
        }
    };
    auto store_stage = [&](uint8_t *base) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i)
            *reinterpret_cast<i32x4 *>(base + lds_off0 + i * kRowStep * kBK) = staged[i];
    };
    // 32-byte operand fragment of stage row `row`: K [16*quad, +16) and
    // [64 + 16*quad, +16).
    auto fragment = [&](const uint8_t *base, int row) {
        i32x4 lo = *reinterpret_cast<const i32x4 *>(base + row * kBK + swz(row, quad) * 16);
        i32x4 hi = *reinterpret_cast<const i32x4 *>(base + row * kBK + swz(row, 4 + quad) * 16);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    const int stages = (K + kBK - 1) / kBK;
    load_stage(0);
    store_stage(lds);
    __syncthreads();

    // Fragment rows within the stage: weight rows for A, token rows for B.
    const int a_row0 = wave_n * kWaveN + row16;
    const int b_row0 = BN + wave_m * kWaveM + row16;

    for (int s = 0; s < stages; ++s) {
        const uint8_t *cur = lds + (s & 1) * kStageBytes;
        if (s + 1 < stages) load_stage((s + 1) * kBK);

        i32x8 bf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[j] = fragment(cur, b_row0 + j * 16);
        if constexpr (!Grouped) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const i32x8 af = fragment(cur, a_row0 + i * 16);
#pragma unroll
                for (int j = 0; j < 4; ++j) MMA::run(acc[i][j], af, bf[j]);
            }
        } else {
            // One 128-wide K group per stage: r = fmaf(p, sxg*swg, r).
            const int k = s * kBK;
            const int g_in = input_group ? k / input_group : 0;
            const int g_w = weight_group ? k / weight_group : 0;
            float sxg[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int m = min(m_base + wave_m * kWaveM + j * 16 + row16, M - 1);
                sxg[j] = input_group ? sx[size_t(g_in) * M + m] : 1.f;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const i32x8 af = fragment(cur, a_row0 + i * 16);
                Acc part[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    part[j] = Acc{0, 0, 0, 0};
                    MMA::run(part[j], af, bf[j]);
                }
                float swg[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int n = min(n_base + wave_n * kWaveN + i * 16 + quad * 4 + r, N - 1);
                    swg[r] = weight_group ? sw[size_t(g_w) * N + n] : 1.f;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        facc[i][j][r] =
                            __builtin_fmaf(float(part[j][r]), sxg[j] * swg[r], facc[i][j][r]);
            }
        }
        if (s + 1 < stages) store_stage(lds + ((s + 1) & 1) * kStageBytes);
        __syncthreads();
    }

    // Epilogue: lane holds C[n = 4*quad + r][m = row16] of each 16x16 tile.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = m_base + wave_m * kWaveM + j * 16 + row16;
        if (m >= M) continue;
        const float sxm = sx[m];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int n = n_base + wave_n * kWaveN + i * 16 + quad * 4;
            if (n >= N) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (Grouped) {
                    float outer = input_group ? 1.f : sxm;
                    if (!weight_group) outer *= sw[n + r];
                    v[r] = (0.f + facc[i][j][r]) * outer;
                } else {
                    float t = float(acc[i][j][r]) * sxm;
                    v[r] = t * sw[n + r];
                }
            }
            store4<Out>(y, size_t(m) * N + n, v);
        }
    }
}

template <int Fmt, int WN, int WM, bool Grouped, class Out>
int launch_shape(const GemmArgs &a, hipStream_t stream) {
    constexpr int BN = kWaveN * WN, BM = kWaveM * WM;
    const int tiles_n = (a.N + BN - 1) / BN, tiles_m = (a.M + BM - 1) / BM;
    const size_t lds = size_t(2) * (BN + BM) * kBK;
    dim3 grid(unsigned(tiles_n * tiles_m)), block(64 * WN * WM);
    if (a.K % kBK == 0)
        hipLaunchKernelGGL((tiled_gemm<Fmt, WN, WM, Grouped, true, Out>), grid, block, lds, stream,
                           a.x, a.sx, a.w, a.sw, a.y, a.M, a.N, a.K, tiles_m, tiles_n,
                           a.input_group, a.weight_group);
    else
        hipLaunchKernelGGL((tiled_gemm<Fmt, WN, WM, Grouped, false, Out>), grid, block, lds,
                           stream, a.x, a.sx, a.w, a.sw, a.y, a.M, a.N, a.K, tiles_m, tiles_n,
                           a.input_group, a.weight_group);
    return 0;
}

template <int Fmt, bool Grouped, class Out>
int dispatch_shape(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    // channels x tokens macro tile
    if (p.channels == 256 && p.tokens == 256) return launch_shape<Fmt, 2, 4, Grouped, Out>(a, s);
    if (p.channels == 256 && p.tokens == 128) return launch_shape<Fmt, 2, 2, Grouped, Out>(a, s);
    if (p.channels == 128 && p.tokens == 256) return launch_shape<Fmt, 1, 4, Grouped, Out>(a, s);
    if (p.channels == 128 && p.tokens == 128) return launch_shape<Fmt, 1, 2, Grouped, Out>(a, s);
    return -4;
}

template <int Fmt, class Out>
int dispatch_grouped(const GemmArgs &a, const GemmPath &p, hipStream_t s) {
    if (a.input_group || a.weight_group) return dispatch_shape<Fmt, true, Out>(a, p, s);
    return dispatch_shape<Fmt, false, Out>(a, p, s);
}

}  // namespace

size_t tiled_workspace_bytes(const GemmArgs &, const GemmPath &) { return 0; }

int launch_tiled(const GemmArgs &a, const GemmPath &p, hipStream_t stream) {
    if (a.out_type == F16) {
        if (a.fmt == I8) return dispatch_grouped<I8, f16_t>(a, p, stream);
        return dispatch_grouped<FP8, f16_t>(a, p, stream);
    }
    if (a.fmt == I8) return dispatch_grouped<I8, bf16_t>(a, p, stream);
    return dispatch_grouped<FP8, bf16_t>(a, p, stream);
}

}  // namespace qlin
