// C ABI of libqlinear.so: argument validation, path planning and dispatch to
// the gfx950 kernel launchers. No exceptions cross this boundary.
#include "../../include/qlinear.h"

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <utility>

#include "qlin_internal.hpp"

namespace {

thread_local char g_error[512] = "";

int fail(int status, const char *fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, args);
    va_end(args);
    return status;
}

int ok() {
    g_error[0] = '\0';
    return QLIN_OK;
}

bool aligned(const void *p, size_t bytes) {
    return reinterpret_cast<uintptr_t>(p) % bytes == 0;
}

bool valid_group(int g) { return g == 0 || g == 32 || g == 64 || g == 128; }

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(QLIN_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

qlin::GemmPath to_internal(const qlin_path &p) {
    return {p.kind, p.tokens, p.channels, p.splits, p.waves, p.staged};
}

// The skinny path's staging for a tiling (tokens, channels, waves = 8): 1
// when each wave's weight slab (at most three 256-byte K blocks) is copied
// global->LDS in one shot, 2 when its activation rows fit beside it, else 0.
int skinny_staging(int rows, int N, int K, int fmt, int input_group, int weight_group,
                   qlin_path p) {
    p.waves = 8;
    const int nb = qlin::skinny_span(K, 1) / 256;
    p.staged = nb <= 3 && long(p.channels) * nb * 8 * 256 <= 160 * 1024 ? 1 : 0;
    qlin::GemmArgs a{};
    a.M = rows;
    a.N = N;
    a.K = K;
    a.fmt = fmt;
    a.input_group = input_group;
    a.weight_group = weight_group;
    if (p.staged && qlin::skinny_lds_bytes(a, to_internal(p)) > qlin::kLdsBytes) p.staged = 0;
    if (p.staged) {
        p.staged = 2;
        if (qlin::skinny_lds_bytes(a, to_internal(p)) > qlin::kLdsBytes) p.staged = 1;
    }
    return p.staged;
}

bool skinny_stages(int rows, int N, int K, int fmt, int input_group, int weight_group, int tokens,
                   int channels) {
    qlin_path p{};
    p.kind = QLIN_KIND_SKINNY;
    p.tokens = tokens;
    p.channels = channels;
    p.splits = 1;
    return skinny_staging(rows, N, K, fmt, input_group, weight_group, p) > 0;
}

// Path selection for gfx950 (256 CUs, 8 XCDs). Decode shapes stream the
// weights once through the skinny kernel; larger token counts use the
// LDS-tiled MFMA GEMM.
qlin_path choose(int rows, int N, int K, int fmt, int input_group, int weight_group) {
    qlin_path p{};
    if (rows <= 64) {
        // Decode: the weights are streamed once and each CU's share of them
        // bounds the time, so the grid is sized to about one workgroup per
        // CU (256 on MI355X). Rules measured on the BASELINE projections at
        // M = 1, 8, 16, 32, 64 (weights rotated through > 512 MB so they come
        // from HBM; variants interleaved, median of 5):
        //  - above 16 rows with weights under 16 MB (qkv, o_proj, down):
        //    16-token tiles and the fewest weight rows (16/32/48) that keep
        //    <= 256 workgroups, else 32: qkv at M = 32 4.9 us against 5.8 us
        //    with one 32-token tile;
        //  - otherwise the largest workgroup count up to 256, then wider token
        //    tiles (fewer activation re-reads), then fewer weight rows
        //    (gate_up keeps 32/64-token tiles).
        p.kind = QLIN_KIND_SKINNY;
        p.splits = 1;
        const int full_tokens = (rows + 15) / 16 * 16;
        if (rows > 64) {
            p.tokens = 64;
            p.channels = 32;
        } else if (rows > 16 && long(N) * K < (16L << 20)) {
            // 16-token tiles first, then 32; the first tiling with <= 256
            // workgroups whose weight slab can be staged in LDS, else the
            // first with <= 256 workgroups. Measured at M = 64 (INT8, weights
            // from HBM): qkv 32x32 4.62 us against 6.87 us on 16x32 (512
            // workgroups), down 32x16 (staged) 9.42 us against 11.24 us on
            // 16x32 (its 3-block slab does not fit).
            p.tokens = 16;
            p.channels = 32;
            bool found = false, found_staged = false;
            for (int tokens : {16, 32}) {
                if (found_staged) break;
                for (int channels : {16, 32, 48}) {
                    if (long((N + channels - 1) / channels) * ((rows + tokens - 1) / tokens) > 256)
                        continue;
                    const bool stages = skinny_stages(rows, N, K, fmt, input_group, weight_group,
                                                      tokens, channels);
                    if (!found || (stages && !found_staged)) {
                        p.tokens = tokens;
                        p.channels = channels;
                        found = true;
                        found_staged = stages;
                    }
                    if (found_staged) break;
                }
            }
        } else {
            // Token tiles of 16, 32 or 64 rows that divide the rows rounded
            // up to 16 (48 rows count as one padded 64-row tile).
            const int cap = full_tokens == 48 ? 64 : full_tokens;
            long best = -1;
            for (int channels : {16, 32, 48}) {
                for (int tokens : {64, 32, 16}) {
                    if (tokens > cap || (cap % tokens && tokens != 16)) continue;
                    const long wgs = long((N + channels - 1) / channels) * ((rows + tokens - 1) / tokens);
                    const long score = (wgs <= 256 ? wgs : 256 - (wgs - 256)) * 4096 + tokens * 64 - channels;
                    if (score > best) {
                        best = score;
                        p.tokens = tokens;
                        p.channels = channels;
                    }
                }
            }
        }
        // Eight wave64s split K inside a workgroup. Each wave's weight slab
        // is copied global->LDS in one shot when its range is at most three
        // 256-byte blocks and the slab fits (staged 1), and its activation
        // rows with it when those fit too (staged 2): the activation tile
        // then arrives as whole 256-byte row runs instead of 64-byte pieces
        // of 16 rows. Measured at M = 32 (weights from HBM): qkv 5.05 ->
        // 4.65 us, o_proj 4.24 -> 3.64 us.
        p.waves = 8;
        p.staged = skinny_staging(rows, N, K, fmt, input_group, weight_group, p);
        return p;
    }
    // Prefill: the macro tile by measured MI355X rules (BASELINE projections
    // at M = 1024 and 4096, per-channel and K128 groups, realistic data).
    // A grid is run in rounds of 256 workgroups (one per CU); `full` says its
    // last round is at least 90% occupied.
    //  - INT8 per-channel, all with eight waves: 256x256 (128x64 waves, two
    //    double-buffered 128-byte K stages) when
    //    it has >= 192 tiles (qkv/gate_up at 4096, gate_up at 1024); else
    //    256x128 (128x32 waves, 128-byte K stages) for >= 256 tiles in full
    //    rounds: down at 4096 54 us against 68 us on 128x128; else 128x128
    //    (64x32 waves): qkv
    //    at 1024 14.4 us against 19.1 us with four 64x64 waves.
    //  - FP8 per-channel: 256x256 with eight 128x64 waves (16x16x128 MFMA,
    //    two double-buffered 128-byte K stages) when it has >= 192 tiles
    //    (gate_up at 4096 90 us; 114 us with 64-byte stages against 116 us
    //    with four 128x128 waves; gate_up at 1024 29.3 us against 33.2 us on
    //    128x128); else 256x128 (eight 128x32 waves, the same
    //    pipeline) for >= 256 tiles in full
    //    rounds: o_proj at 4096 27.7 us against 30.2 us with four 128x64
    //    waves on 32x32x64 and 30.4 on 128x128; else 128x128 with eight 64x32 waves on
    //    the 16x16x128 MFMA over 128-byte K stages: down at 1024 35.5 us
    //    against 45.3 us with four 32x32x64 waves.
    //  (Variants timed interleaved after a warm-up, median of 5 rounds: the
    //  clock settles upward under sustained MFMA load.)
    //  - K groups (no wide-kernel variant), eight waves, both formats:
    //    256x128 (128x32 waves) for >= 256 tiles in full rounds (gate_up at
    //    4096: INT8 193 us against 222 us on 128x128, FP8 193 us against
    //    216 us), else 128x128 (64x32 waves): down at 1024 INT8 44 us
    //    against 80 us on 256x128. Groups of 32 / 64 follow the same rule
    //    for INT8 (qkv at 4096, G 32: 219 us against 267 us); FP8 takes
    //    128x128 (255 us against 428 us).
    p.kind = QLIN_KIND_TILED;
    p.splits = 1;
    p.waves = 1;
    const bool grouped = input_group || weight_group;
    const long tiles_256 = long((N + 255) / 256) * ((rows + 255) / 256);
    const long tiles_256x128 = long((N + 255) / 256) * ((rows + 127) / 128);
    const bool full = tiles_256x128 * 10 >= (tiles_256x128 + 255) / 256 * 256 * 9;
    p.channels = 128;
    p.tokens = 128;
    if (!grouped && fmt == QLIN_I8) {
        p.waves = 8;
        // 256x256 from 192 tiles. Below that, 256x128 only for long K: the
        // double-buffered 128x128 tile, two workgroups per CU, overlaps one
        // workgroup's prologue and epilogue with the other's MFMAs, which
        // pays while K is short (o_proj at M = 4096: 18.8 us against 19.7 us
        // on 256x128; down, K = 6144, keeps 256x128: 45.6 us against 48.3).
        if (tiles_256 >= 192) p.channels = p.tokens = 256;
        else if (tiles_256x128 >= 256 && full && K > 2048) p.channels = 256;
    } else if (!grouped) {
        if (tiles_256 >= 192) {
            p.channels = p.tokens = 256;
            p.waves = 8;
        } else if (tiles_256x128 >= 256 && full && K > 2048) {
            // as INT8: with K <= 2048 the double-buffered 128x128 tile (o_proj
            // at M = 4096: 17.8 us against 18.3 us on 256x128)
            p.channels = 256;
            p.waves = 8;
        } else {
            p.waves = 8;
        }
    } else {
        p.waves = 8;
        const bool small_group = (input_group && input_group < 128) || (weight_group && weight_group < 128);
        if (tiles_256x128 >= 256 && full && !(small_group && fmt == QLIN_FP8)) p.channels = 256;
    }
    // A 128x128 grid of at most 128 tiles fills half the GPU or less; 128x64
    // tiles (eight 64x16 waves over 128-byte K stages) double the
    // workgroups: o_proj / down at M = 1024 (128 tiles of 128x128), INT8
    // 18.2 / 36.9 us against 17.2 / 25.4 (four 64x32 waves: 16.9 / 32.2),
    // FP8 19.6 / 38.7 against 18.2 / 32.9, group_int8 22.0 / 46.4 against
    // 17.4 / 31.6 (four 64x32 waves: 20.0 / 38.8; random operands).
    const bool small_group = (input_group && input_group < 128) || (weight_group && weight_group < 128);
    const long tiles_128 = long((N + 127) / 128) * ((rows + 127) / 128);
    if (p.channels == 128 && p.tokens == 128 && tiles_128 <= 128 && !small_group) {
        p.tokens = 64;
        p.waves = 8;
    }
    return p;
}

int check_path(const qlin_path &p, int rows, int N, int K, int fmt, int input_group,
               int weight_group) {
    if (p.kind == QLIN_KIND_SKINNY) {
        if (p.tokens != 16 && p.tokens != 32 && p.tokens != 64)
            return fail(QLIN_ERR_UNSUPPORTED, "skinny path tokens must be 16/32/64 (got %d)",
                        p.tokens);
        if (p.channels != 16 && p.channels != 32 && p.channels != 48)
            return fail(QLIN_ERR_UNSUPPORTED,
                        "skinny path channels must be 16, 32 or 48 (got %d)", p.channels);
        if (p.waves != 8)
            return fail(QLIN_ERR_UNSUPPORTED, "skinny path waves must be 8 (got %d)", p.waves);
        const int blocks_k = (K + 255) / 256;
        if (p.splits < 1 || p.splits > blocks_k)
            return fail(QLIN_ERR_UNSUPPORTED,
                        "skinny path splits (%d) must be in 1..ceil(K/256) = %d", p.splits,
                        blocks_k);
        if (p.staged < 0 || p.staged > 2)
            return fail(QLIN_ERR_UNSUPPORTED, "skinny staged must be 0, 1 or 2");
        // Token tiles run along the grid's z dimension (at most 65535).
        if ((long(rows) + p.tokens - 1) / p.tokens > 65535)
            return fail(QLIN_ERR_UNSUPPORTED, "skinny path has more than 65535 token tiles");
        if (p.staged && (p.splits != 1 || qlin::skinny_span(K, 1) > 3 * 256))
            return fail(QLIN_ERR_UNSUPPORTED,
                        "staged skinny path needs no split and ceil(K/256) <= 24");
        qlin::GemmArgs a{};
        a.M = rows;
        a.N = N;
        a.K = K;
        a.fmt = fmt;
        a.input_group = input_group;
        a.weight_group = weight_group;
        const size_t lds = qlin::skinny_lds_bytes(a, to_internal(p));
        if (lds > qlin::kLdsBytes)
            return fail(QLIN_ERR_UNSUPPORTED,
                        "skinny path needs %zu bytes of LDS (slab + reduction), limit %zu", lds,
                        qlin::kLdsBytes);
        return ok();
    }
    if (p.kind == QLIN_KIND_TILED) {
        // No 512-channel tile: a register-streamed 512x128 INT8 kernel (four
        // 128x128 waves, weights global -> registers, tokens through LDS)
        // measured slower than the planned tiles and faulted the GPU under
        // graph replay with its cause unfound, so it is not built.
        if (p.channels == 512 || p.tokens == 512)
            return fail(QLIN_ERR_UNSUPPORTED,
                        "tiled 512-channel path is disabled (register-streamed kernel not built)");
        if (!((p.channels == 256 && (p.tokens == 256 || p.tokens == 128)) ||
              (p.channels == 128 && (p.tokens == 128 || p.tokens == 64))))
            return fail(QLIN_ERR_UNSUPPORTED,
                        "tiled path channels x tokens must be 256x256, 256x128, 128x128 or 128x64 (got %dx%d)",
                        p.channels, p.tokens);
        if (p.splits != 1)
            return fail(QLIN_ERR_UNSUPPORTED, "tiled path has no split-K variant");
        // Macro tiles run along the grid's x dimension (below 2^31).
        if (long((N + p.channels - 1) / p.channels) * ((long(rows) + p.tokens - 1) / p.tokens) >
            INT32_MAX)
            return fail(QLIN_ERR_UNSUPPORTED, "tiled path has more than 2^31 - 1 macro tiles");
        // 256x256: eight waves of 128x64 (16x16 MFMA) or four of 128x128
        // (32x32 MFMA); 256x128: one workgroup of 128x64 waves (1), two waves
        // of 128x128 (2) or eight of 128x32 (8); 128x128: four waves of 64x64
        // (1) or eight of 64x32 (8).
        const bool wave_ok = (p.channels == 256 && p.tokens == 256) ? (p.waves == 8 || p.waves == 4)
                             : (p.channels == 256 && p.tokens == 128) ? (p.waves == 1 || p.waves == 2 || p.waves == 8)
                             : p.tokens == 64 ? (p.waves == 4 || p.waves == 8)
                                              : (p.waves == 1 || p.waves == 8);
        if (!wave_ok)
            return fail(QLIN_ERR_UNSUPPORTED, "tiled %dx%d path has no %d-wave variant", p.channels,
                        p.tokens, p.waves);
        if (p.waves != 1 && p.waves != 8 && p.tokens != 256 && p.tokens != 64 &&
            (input_group || weight_group))
            return fail(QLIN_ERR_UNSUPPORTED, "K-group tiled path has no 32x32-tile variant");
        if ((input_group || weight_group) && p.tokens == 256)
            return fail(QLIN_ERR_UNSUPPORTED, "K-group tiled path has no 256-token tile");
        if ((input_group || weight_group) && p.channels == 256 && p.waves != 8)
            return fail(QLIN_ERR_UNSUPPORTED, "K-group 256x128 tiled path has eight waves only");
        // The K-group tiled kernel addresses its scale arrays through 32-bit
        // buffer ranges.
        if ((input_group || weight_group) &&
            ((long(K) + 127) / 128) * (long(N) > rows ? long(N) : long(rows)) * 4 > INT32_MAX)
            return fail(QLIN_ERR_UNSUPPORTED, "K-group scale arrays exceed 2 GiB");
        if (p.staged) return fail(QLIN_ERR_UNSUPPORTED, "tiled path staged must be 0");
        const bool small_group = (input_group && input_group < 128) || (weight_group && weight_group < 128);
        if (small_group && p.waves != 8)
            return fail(QLIN_ERR_UNSUPPORTED, "tiled K groups of 32/64 have eight-wave tiles only");
        if (small_group && fmt == QLIN_FP8 && p.channels != 128)
            return fail(QLIN_ERR_UNSUPPORTED, "FP8 tiled K groups of 32/64 have 128x128 tiles only");
        return ok();
    }
    return fail(QLIN_ERR_UNSUPPORTED, "unknown path kind %d", p.kind);
}

}  // namespace

namespace qlin {
int set_error(int status, const char *message) { return fail(status, "%s", message); }
}  // namespace qlin

extern "C" {

int qlin_version(void) { return 101; }

const char *qlin_last_error(void) { return g_error; }

int qlin_row_quantize(const void *src, int ld, int rows, int cols, int src_type, void *values,
                      float *scales, int fmt, int group, int rotation, qlin_stream_t stream) {
    // ops::quantize_rows (reference ops/basic.cpp:69-78) + RowScaledView::validate
    // (core/quantization.h:39-48).
    if (src_type != QLIN_BF16 && src_type != QLIN_F16)
        return fail(QLIN_ERR_INVALID, "quantization source must be BF16 or F16");
    if (fmt != QLIN_I8 && fmt != QLIN_FP8)
        return fail(QLIN_ERR_INVALID, "quantized storage must be I8 or FP8");
    if (rows < 1 || cols < 1 || ld < cols)
        return fail(QLIN_ERR_INVALID, "quantization shape rows=%d cols=%d ld=%d", rows, cols, ld);
    if (!src || !values || !scales)
        return fail(QLIN_ERR_INVALID, "quantization source/destination pointer is null");
    if (!valid_group(group))
        return fail(QLIN_ERR_INVALID, "quantization group must be 0, 32, 64 or 128 (got %d)",
                    group);
    if (rotation && (rotation != 128 || cols % 128))
        return fail(QLIN_ERR_INVALID, "rotation must be 128 with cols %% 128 == 0");
    if (!aligned(src, 2)) return fail(QLIN_ERR_ALIGNMENT, "16-bit source must be 2-byte aligned");
    if (!aligned(scales, 4)) return fail(QLIN_ERR_ALIGNMENT, "scales must be 4-byte aligned");
    if (group && uint64_t(rows) * ((uint64_t(cols) + 2047) / 2048) > INT32_MAX)
        return fail(QLIN_ERR_INVALID, "group quantization grid exceeds capacity");
    qlin::RowQuantizeArgs a{src, src_type, ld, rows, cols, values, scales, fmt, group, rotation};
    qlin::launch_row_quantize(a, reinterpret_cast<hipStream_t>(stream));
    return check_launch("row quantize launch");
}

int qlin_plan(int rows, int N, int K, int fmt, int input_group, int weight_group,
              qlin_path *path) {
    if (!path) return fail(QLIN_ERR_INVALID, "path is null");
    if (rows < 1 || N < 1 || K < 1)
        return fail(QLIN_ERR_INVALID, "invalid kernel problem rows=%d N=%d K=%d", rows, N, K);
    *path = choose(rows, N, K, fmt, input_group, weight_group);
    return ok();
}

size_t qlin_workspace_bytes(const qlin_path *path, int rows, int N, int K, int fmt,
                            int input_group, int weight_group) {
    qlin_path p = path && path->kind ? *path : choose(rows, N, K, fmt, input_group, weight_group);
    qlin::GemmArgs a{};
    a.M = rows;
    a.N = N;
    a.K = K;
    a.fmt = fmt;
    a.input_group = input_group;
    a.weight_group = weight_group;
    if (p.kind == QLIN_KIND_SKINNY) return qlin::skinny_workspace_bytes(a, to_internal(p));
    return 0;
}

}  // extern "C"

namespace {
constexpr int kNotFused = 1;  // gemm_impl with a fused source: no such variant, nothing launched
int gemm_impl(const qlin_path *path, const void *x, const float *sx, const void *w,
              const float *sw, void *y, int rows, int N, int K, int fmt, int out_type,
              int input_group, int weight_group, void *workspace, size_t workspace_bytes,
              qlin_stream_t stream, bool packed, const void *bias = nullptr, int act = 0,
              const qlin::FusedSource *fq = nullptr) {
    // check_linear + make_plan rules (reference ops/cuda/quantization.cpp:94-102,
    // 206-222) and launch_quant_linear's type checks (quant_dispatch.cu:194-233).
    if (fmt != QLIN_I8 && fmt != QLIN_FP8)
        return fail(QLIN_ERR_INVALID, "unsupported quantized storage type");
    if (out_type != QLIN_BF16 && out_type != QLIN_F16)
        return fail(QLIN_ERR_INVALID, "quantized GEMM output must be F16 or BF16");
    if (rows < 1 || N < 1 || K < 1 || K % 16 || N % 16)
        return fail(QLIN_ERR_INVALID, "quantized GEMM unsupported shape rows=%d N=%d K=%d", rows,
                    N, K);
    if (fmt == QLIN_I8 && K > INT32_MAX / (128 * 128))
        return fail(QLIN_ERR_INVALID, "INT8 reduction can overflow INT32");
    if (!valid_group(input_group) || !valid_group(weight_group))
        return fail(QLIN_ERR_INVALID, "group sizes must be 0, 32, 64 or 128");
    if (!x || !sx || !w || !sw || !y)
        return fail(QLIN_ERR_INVALID, "quantized GEMM operand pointer is null");
    if (!aligned(x, 16) || !aligned(w, 16))
        return fail(QLIN_ERR_ALIGNMENT, "quantized operands must be 16-byte aligned");
    if (!aligned(y, 8)) return fail(QLIN_ERR_ALIGNMENT, "output must be 8-byte aligned");
    if (!aligned(sx, 4) || !aligned(sw, 4))
        return fail(QLIN_ERR_ALIGNMENT, "scales must be 4-byte aligned");
    qlin_path p = path && path->kind ? *path : choose(rows, N, K, fmt, input_group, weight_group);
    // Packed weights stream straight into registers: no LDS slab staging.
    if (packed && !(path && path->kind)) p.staged = 0;
    int status = check_path(p, rows, N, K, fmt, input_group, weight_group);
    if (status) return status;
    qlin::GemmArgs a{static_cast<const uint8_t *>(x),
                     sx,
                     static_cast<const uint8_t *>(w),
                     sw,
                     y,
                     rows,
                     N,
                     K,
                     fmt,
                     out_type,
                     input_group,
                     weight_group,
                     workspace,
                     workspace_bytes,
                     packed ? 1 : 0,
                     static_cast<const uint16_t *>(bias),
                     act};
    const qlin::GemmPath ip = to_internal(p);
    if (fq) {
        // qlin_linear's one-launch form: taken only where a fused variant
        // exists, else the caller quantizes and launches the GEMM separately.
        a.fq = *fq;
        if (!qlin::skinny_fused_supported(a, ip)) return kNotFused;
        int r = qlin::launch_skinny_fused(a, ip, reinterpret_cast<hipStream_t>(stream));
        if (r) return fail(r, "no fused kernel variant for this path");
        return check_launch("fused quantize + GEMM launch");
    }
    size_t need = 0;
    if (p.kind == QLIN_KIND_SKINNY) need = qlin::skinny_workspace_bytes(a, ip);
    if (need && (!workspace || workspace_bytes < need))
        return fail(QLIN_ERR_WORKSPACE, "split-K partial workspace overflow: need %zu bytes, have %zu",
                    need, workspace ? workspace_bytes : size_t(0));
    if (need && !aligned(workspace, 16))
        return fail(QLIN_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    int r = p.kind == QLIN_KIND_SKINNY ? qlin::launch_skinny(a, ip, s) : qlin::launch_tiled(a, ip, s);
    if (r) return fail(r, "no kernel variant for this path");
    return check_launch("quantized GEMM launch");
}
}  // namespace

extern "C" {

int qlin_gemm(const qlin_path *path, const void *x, const float *sx, const void *w,
              const float *sw, void *y, int rows, int N, int K, int fmt, int out_type,
              int input_group, int weight_group, void *workspace, size_t workspace_bytes,
              qlin_stream_t stream) {
    return gemm_impl(path, x, sx, w, sw, y, rows, N, K, fmt, out_type, input_group, weight_group,
                     workspace, workspace_bytes, stream, false);
}

int qlin_gemm_finish(const qlin_path *path, const void *x, const float *sx, const void *w,
                     const float *sw, const void *bias, int activation, void *y, int rows, int N,
                     int K, int fmt, int out_type, int input_group, int weight_group, int packed,
                     void *workspace, size_t workspace_bytes, qlin_stream_t stream) {
    // QuantizedGemm::linear_finish + check_finish_bias (reference
    // ops/cuda/quantization.cpp:75-87,465-478): ReLU or tanh-GeLU (or none),
    // optional bias [N] in the output type.
    if (activation < QLIN_FINISH_NONE || activation > QLIN_FINISH_GELU_TANH)
        return fail(QLIN_ERR_INVALID, "finish activation must be 0 (none), 1 (ReLU) or 2 (tanh-GeLU)");
    if (bias && !aligned(bias, 2)) return fail(QLIN_ERR_ALIGNMENT, "bias must be 2-byte aligned");
    return gemm_impl(path, x, sx, w, sw, y, rows, N, K, fmt, out_type, input_group, weight_group,
                     workspace, workspace_bytes, stream, packed != 0, bias, activation);
}

size_t qlin_packed_weight_bytes(int N, int K) {
    if (N < 1 || K < 1 || N % 16) return 0;
    return qlin::packed_weight_bytes(N, K);
}

int qlin_pack_weights(const void *w, int N, int K, void *packed, qlin_stream_t stream) {
    if (N < 1 || K < 1 || N % 16 || K % 16)
        return fail(QLIN_ERR_INVALID, "packed weights need N %% 16 == 0 and K %% 16 == 0 (N=%d K=%d)",
                    N, K);
    if (!w || !packed) return fail(QLIN_ERR_INVALID, "weight pointer is null");
    if (!aligned(w, 16) || !aligned(packed, 16))
        return fail(QLIN_ERR_ALIGNMENT, "weights must be 16-byte aligned");
    qlin::launch_pack_weights(w, N, K, packed, reinterpret_cast<hipStream_t>(stream));
    return check_launch("weight packing launch");
}

int qlin_gemm_packed(const qlin_path *path, const void *x, const float *sx, const void *w,
                     const float *sw, void *y, int rows, int N, int K, int fmt, int out_type,
                     int input_group, int weight_group, void *workspace, size_t workspace_bytes,
                     qlin_stream_t stream) {
    return gemm_impl(path, x, sx, w, sw, y, rows, N, K, fmt, out_type, input_group, weight_group,
                     workspace, workspace_bytes, stream, true);
}

int qlin_linear_packed(const qlin_path *path, const void *x, int ld, int src_type, void *xq,
                       float *sx, const void *w, const float *sw, void *y, int rows, int N, int K,
                       int fmt, int out_type, int input_group, int weight_group, int rotation,
                       void *workspace, size_t workspace_bytes, qlin_stream_t stream) {
    if (!xq || !sx) return fail(QLIN_ERR_INVALID, "linear needs the scratch activation (xq, sx)");
    int status = qlin_row_quantize(x, ld, rows, K, src_type, xq, sx, fmt, input_group, rotation,
                                   stream);
    if (status) return status;
    return qlin_gemm_packed(path, xq, sx, w, sw, y, rows, N, K, fmt, out_type, input_group,
                            weight_group, workspace, workspace_bytes, stream);
}

int qlin_linear(const qlin_path *path, const void *x, int ld, int src_type, void *xq, float *sx,
                const void *w, const float *sw, void *y, int rows, int N, int K, int fmt,
                int out_type, int input_group, int weight_group, int rotation, void *workspace,
                size_t workspace_bytes, qlin_stream_t stream) {
    // ops::linear, quantized branch (reference ops/linear.cpp:51-71):
    // quantize_rows into the scratch activation, then the GEMM.
    if (!xq || !sx) return fail(QLIN_ERR_INVALID, "linear needs the scratch activation (xq, sx)");
    // Decode shapes with per-token scales or activation groups of 128 (no
    // rotation): one launch in which the GEMM quantizes its own token rows (and fills the scratch as the quantizer
    // would), when the planned path has a fused variant. In that launch some
    // workgroups still read x while others write y and the scratch, so an
    // output or scratch overlapping x takes the two-launch form, which
    // reads all of x before the GEMM writes.
    const auto span_of = [](const void *p, size_t bytes) {
        const uintptr_t b = reinterpret_cast<uintptr_t>(p);
        return std::pair<uintptr_t, uintptr_t>{b, b + bytes};
    };
    const auto overlaps = [](std::pair<uintptr_t, uintptr_t> a, std::pair<uintptr_t, uintptr_t> b) {
        return a.first < b.second && b.first < a.second;
    };
    const bool disjoint =
        rows >= 1 && N >= 1 && K >= 1 && ld >= 1 && x && y &&
        !overlaps(span_of(x, size_t(rows) * ld * 2), span_of(y, size_t(rows) * N * 2)) &&
        !overlaps(span_of(x, size_t(rows) * ld * 2), span_of(xq, size_t(rows) * K)) &&
        !overlaps(span_of(x, size_t(rows) * ld * 2),
                  span_of(sx, size_t(rows) * 4 *
                                  (input_group > 0 ? size_t(K + input_group - 1) / input_group : 1)));
    if ((!input_group || input_group == 128) && !rotation &&
        (src_type == QLIN_BF16 || src_type == QLIN_F16) && x &&
        aligned(x, 16) && ld % 8 == 0 && ld >= K && rows >= 1 && aligned(xq, 16) &&
        aligned(sx, 4) && disjoint) {
        const qlin::FusedSource fq{static_cast<const uint16_t *>(x), ld, src_type == QLIN_F16 ? 1 : 0,
                                   static_cast<uint8_t *>(xq), sx};
        int r = gemm_impl(path, xq, sx, w, sw, y, rows, N, K, fmt, out_type, input_group,
                          weight_group, workspace, workspace_bytes, stream, false, nullptr, 0, &fq);
        if (r != kNotFused) return r;
    }
    int status = qlin_row_quantize(x, ld, rows, K, src_type, xq, sx, fmt, input_group, rotation,
                                   stream);
    if (status) return status;
    return qlin_gemm(path, xq, sx, w, sw, y, rows, N, K, fmt, out_type, input_group, weight_group,
                     workspace, workspace_bytes, stream);
}

int qlin_quantized_norm(void *residual, const void *update, const void *update_scale,
                        const void *weight, int src_type, int rows, int cols, float eps, int gemma,
                        void *values, float *scales, int fmt, int group, int rotation,
                        qlin_stream_t stream) {
    // launch_quantized_norm's checks (reference quant_norm.cu:166-180) plus
    // RowScaledView::validate (core/quantization.h:39-48).
    if (src_type != QLIN_BF16 && src_type != QLIN_F16)
        return fail(QLIN_ERR_INVALID, "quantized RMS input must be BF16 or F16");
    if (fmt != QLIN_I8 && fmt != QLIN_FP8)
        return fail(QLIN_ERR_INVALID, "quantized storage must be I8 or FP8");
    if (rows < 1 || cols < 1 || cols > 2048)
        return fail(QLIN_ERR_INVALID, "quantized RMS shape rows=%d cols=%d (1 <= cols <= 2048)",
                    rows, cols);
    if (!residual || !weight || !values || !scales)
        return fail(QLIN_ERR_INVALID, "quantized RMS pointer is null");
    if (update_scale && !update)
        return fail(QLIN_ERR_INVALID, "update_scale without update");
    if (!valid_group(group))
        return fail(QLIN_ERR_INVALID, "quantization group must be 0, 32, 64 or 128 (got %d)", group);
    if (rotation && (rotation != 128 || cols % 128))
        return fail(QLIN_ERR_INVALID, "rotation must be 128 with cols %% 128 == 0");
    if (!aligned(residual, 2) || !aligned(weight, 2) || (update && !aligned(update, 2)) ||
        (update_scale && !aligned(update_scale, 2)))
        return fail(QLIN_ERR_ALIGNMENT, "16-bit tensors must be 2-byte aligned");
    if (!aligned(scales, 4)) return fail(QLIN_ERR_ALIGNMENT, "scales must be 4-byte aligned");
    qlin::NormQuantizeArgs a{residual, update, update_scale, weight, src_type, rows, cols,
                             values, scales, fmt, group, rotation, gemma ? 1 : 0, eps};
    qlin::launch_quantized_norm(a, reinterpret_cast<hipStream_t>(stream));
    return check_launch("quantized norm launch");
}

void qlin_norm_fusion_init(qlin_norm_fusion *f) {
    if (!f) return;
    *f = qlin_norm_fusion{};
    f->rows_per_sequence = 1;
}

void qlin_epilogue_init(qlin_epilogue *e) {
    if (!e) return;
    *e = qlin_epilogue{};
    e->value_scale = e->output_scale = e->residual_scale = 1.f;
    e->activation = QLIN_ACT_IDENTITY;
    e->alpha = .1f;
    e->rows_per_sequence = e->input_repeat = 1;
}

}  // extern "C"

namespace {

// A byte range of device memory (null = empty).
struct Span {
    const void *p;
    size_t bytes;
};
Span span16(const void *p, size_t rows, size_t cols) { return {p, p ? rows * cols * 2 : 0}; }
bool overlaps(Span a, Span b) {
    if (!a.p || !b.p || !a.bytes || !b.bytes) return false;
    const uintptr_t x = reinterpret_cast<uintptr_t>(a.p), y = reinterpret_cast<uintptr_t>(b.p);
    return x < y + b.bytes && y < x + a.bytes;
}

// Rows of a per-sequence modulation: 1 or the number of sequences.
bool modulation_rows(const void *p, int rows, int sequences) {
    return !p || rows == 1 || rows == sequences;
}

// The row quantizer output rules shared by the sequence producers
// (check_quantized_output, ops/kernels/sequence/sequence_internal.cuh:182-197).
int check_row_output(int src_type, int rows, int cols, const void *values, const float *scales,
                     int fmt, int group, int rotation, const char *what) {
    if (src_type != QLIN_BF16 && src_type != QLIN_F16)
        return fail(QLIN_ERR_INVALID, "%s input must be BF16 or F16", what);
    if (fmt != QLIN_I8 && fmt != QLIN_FP8)
        return fail(QLIN_ERR_INVALID, "quantized storage must be I8 or FP8");
    if (rows < 1 || cols < 1) return fail(QLIN_ERR_INVALID, "%s shape rows=%d cols=%d", what, rows, cols);
    if (!values || !scales) return fail(QLIN_ERR_INVALID, "%s output pointer is null", what);
    if (!valid_group(group))
        return fail(QLIN_ERR_INVALID, "quantization group must be 0, 32, 64 or 128 (got %d)", group);
    if (rotation && !group)
        return fail(QLIN_ERR_INVALID, "rotated sequence fusion requires group scales");
    if (rotation && (rotation != 128 || cols % 128))
        return fail(QLIN_ERR_INVALID, "rotation must be 128 with cols %% 128 == 0");
    if (!aligned(scales, 4)) return fail(QLIN_ERR_ALIGNMENT, "scales must be 4-byte aligned");
    const size_t groups = group ? size_t((cols + group - 1) / group) : 1;
    if (overlaps({values, size_t(rows) * cols}, {scales, groups * rows * 4}))
        return fail(QLIN_ERR_INVALID, "quantized values/scales overlap");
    return QLIN_OK;
}

int check_16bit_aligned(std::initializer_list<const void *> ptrs) {
    for (const void *p : ptrs)
        if (p && !aligned(p, 2)) return fail(QLIN_ERR_ALIGNMENT, "16-bit tensors must be 2-byte aligned");
    return QLIN_OK;
}

// check_norm_shape's NormFusion rules (sequence_norm.cu:371-397).
int check_fusion(const qlin_norm_fusion &f, int rows, float eps, bool allow_source_rows) {
    if (f.rows_per_sequence < 1 || rows % f.rows_per_sequence)
        return fail(QLIN_ERR_INVALID, "invalid normalization sequence length");
    const int sequences = rows / f.rows_per_sequence;
    if (!modulation_rows(f.gate, f.gate_rows, sequences) ||
        !modulation_rows(f.shift, f.shift_rows, sequences) ||
        !modulation_rows(f.scale, f.scale_rows, sequences))
        return fail(QLIN_ERR_INVALID, "invalid normalization modulation");
    if (f.source_rows && (!allow_source_rows || f.gate || f.shift || f.scale))
        return fail(QLIN_ERR_INVALID, "invalid indexed normalization");
    if (!(eps > 0) || eps != eps || eps > 3.4e38f)
        return fail(QLIN_ERR_INVALID, "invalid layer normalization");
    return check_16bit_aligned({f.residual, f.projection_bias, f.gate, f.shift, f.scale, f.raw});
}

}  // namespace

extern "C" {

int qlin_norm_linear(const void *x, const qlin_norm_fusion *fusion, const void *norm_weight,
                     const void *norm_bias, int src_type, int rows, int k, float eps,
                     const void *w, const float *sw, int fmt, int n, const void *bias,
                     int activation, void *y, void *normalized, void *encoded,
                     float *encoded_scales, qlin_stream_t stream) {
    // normalized_quantized_linear's conditions (reference
    // ops/kernels/sequence/sequence_norm.cu:518-558) and check_norm_shape.
    qlin_norm_fusion f;
    qlin_norm_fusion_init(&f);
    if (fusion) f = *fusion;
    if (src_type != QLIN_BF16 && src_type != QLIN_F16)
        return fail(QLIN_ERR_INVALID, "normalized linear input must be BF16 or F16");
    if (fmt != QLIN_I8 && fmt != QLIN_FP8)
        return fail(QLIN_ERR_INVALID, "quantized storage must be I8 or FP8");
    if (rows < 1 || rows > 65535 || n < 1 || k < 4 || k % 4 || k > 512)
        return fail(QLIN_ERR_INVALID,
                    "normalized linear shape rows=%d n=%d k=%d (k %% 4 == 0, 4 <= k <= 512)", rows,
                    n, k);
    if (activation != QLIN_FINISH_NONE && activation != QLIN_FINISH_RELU)
        return fail(QLIN_ERR_INVALID, "normalized linear activation must be none or ReLU");
    if (!x || !w || !sw || !y) return fail(QLIN_ERR_INVALID, "normalized linear pointer is null");
    if (bool(encoded) != bool(encoded_scales))
        return fail(QLIN_ERR_INVALID, "encoded output needs values and scales");
    if (int st = check_fusion(f, rows, eps, false)) return st;
    if (!aligned(w, 4)) return fail(QLIN_ERR_ALIGNMENT, "weights must be 4-byte aligned");
    if (int st = check_16bit_aligned({x, norm_weight, norm_bias, bias, y, normalized})) return st;
    if (!aligned(sw, 4) || (encoded_scales && !aligned(encoded_scales, 4)))
        return fail(QLIN_ERR_ALIGNMENT, "scales must be 4-byte aligned");
    // Outputs may not alias any operand (the reference declines the fusion).
    const Span outputs[] = {span16(y, rows, n), span16(normalized, rows, k), span16(f.raw, rows, k),
                            {encoded, encoded ? size_t(rows) * k : 0},
                            {encoded_scales, encoded_scales ? size_t(rows) * 4 : 0}};
    const Span sources[] = {span16(x, rows, k), span16(f.residual, rows, k),
                            span16(f.projection_bias, 1, k), span16(norm_weight, 1, k),
                            span16(norm_bias, 1, k), span16(bias, 1, n),
                            span16(f.gate, f.gate_rows, k), span16(f.shift, f.shift_rows, k),
                            span16(f.scale, f.scale_rows, k), {w, size_t(n) * k},
                            {sw, size_t(n) * 4}};
    for (size_t a = 0; a < 5; ++a) {
        for (const Span &b : sources)
            if (overlaps(outputs[a], b))
                return fail(QLIN_ERR_INVALID, "normalized linear output overlaps an operand");
        for (size_t b = a + 1; b < 5; ++b)
            if (overlaps(outputs[a], outputs[b]))
                return fail(QLIN_ERR_INVALID, "normalized linear outputs overlap");
    }
    qlin::NormLinearArgs a{x, f, norm_weight, norm_bias, src_type, rows, k, eps, w, sw, fmt, n,
                           bias, activation, y, normalized, encoded, encoded_scales};
    qlin::launch_norm_linear(a, reinterpret_cast<hipStream_t>(stream));
    return check_launch("normalized linear launch");
}

int qlin_layer_norm_quantize(const void *x, int x_rows, int src_type, const void *norm_weight,
                             const void *norm_bias, float eps, const qlin_norm_fusion *fusion,
                             void *retained, int rows, int cols, void *values, float *scales,
                             int fmt, int group, int rotation, qlin_stream_t stream) {
    // layer_norm_quantize's checks (reference sequence_norm.cu:412-425).
    qlin_norm_fusion f;
    qlin_norm_fusion_init(&f);
    if (fusion) f = *fusion;
    if (int st = check_row_output(src_type, rows, cols, values, scales, fmt, group, rotation,
                                  "layer norm quantize"))
        return st;
    if (!x || x_rows < 1) return fail(QLIN_ERR_INVALID, "layer norm quantize input is null");
    if (!f.source_rows && x_rows != rows)
        return fail(QLIN_ERR_INVALID, "layer norm input rows %d != output rows %d", x_rows, rows);
    if (int st = check_fusion(f, f.source_rows ? x_rows : rows, eps, true)) return st;
    if (int st = check_16bit_aligned({x, norm_weight, norm_bias, retained})) return st;
    const Span q_values{values, size_t(rows) * cols};
    const size_t groups = group ? size_t((cols + group - 1) / group) : 1;
    const Span q_scales{scales, groups * rows * 4};
    const Span sources[] = {span16(x, x_rows, cols), span16(retained, rows, cols),
                            span16(norm_weight, 1, cols), span16(norm_bias, 1, cols),
                            span16(f.residual, x_rows, cols), span16(f.projection_bias, 1, cols),
                            span16(f.raw, rows, cols), span16(f.gate, f.gate_rows, cols),
                            span16(f.shift, f.shift_rows, cols), span16(f.scale, f.scale_rows, cols)};
    for (const Span &b : sources)
        if (overlaps(q_values, b) || overlaps(q_scales, b))
            return fail(QLIN_ERR_INVALID, "quantized output overlaps sequence storage");
    // Row outputs (retained, raw) may replace x / residual only row for row.
    const Span row_outputs[] = {span16(retained, rows, cols), span16(f.raw, rows, cols)};
    if (overlaps(row_outputs[0], row_outputs[1]))
        return fail(QLIN_ERR_INVALID, "raw and retained sequence outputs overlap");
    for (const Span &o : row_outputs) {
        for (const Span &b : {span16(norm_weight, 1, cols), span16(norm_bias, 1, cols),
                              span16(f.projection_bias, 1, cols), span16(f.gate, f.gate_rows, cols),
                              span16(f.shift, f.shift_rows, cols), span16(f.scale, f.scale_rows, cols)})
            if (overlaps(o, b))
                return fail(QLIN_ERR_INVALID, "quantized sequence output has unsafe row alias");
        for (const void *src : {x, f.residual})
            if (overlaps(o, span16(src, x_rows, cols)) && (o.p != src || f.source_rows))
                return fail(QLIN_ERR_INVALID, "quantized sequence output has unsafe row alias");
    }
    qlin::LayerNormQuantizeArgs a{x, x_rows, src_type, norm_weight, norm_bias, eps, f, retained,
                                  rows, cols, values, scales, fmt, group, rotation};
    qlin::launch_layer_norm_quantize(a, reinterpret_cast<hipStream_t>(stream));
    return check_launch("layer norm quantize launch");
}

namespace {
// validate_pointwise_quantize (reference sequence_pointwise.cu:307-324) and
// check_epilogue (sequence_internal.cuh:154-178); with values == NULL (the
// dense pointwise, sequence_pointwise.cu:281-287) only the row outputs.
int check_pointwise(const void *x, int x_rows, const qlin_epilogue &e, const void *retained,
                    int rows, int cols, const void *values, const float *scales, int group) {
    if (!x || x_rows < 1 || e.input_repeat < 1 || int64_t(x_rows) * e.input_repeat != rows ||
        (e.input_repeat > 1 && retained && retained == x))
        return fail(QLIN_ERR_INVALID, "invalid quantized pointwise input/repetition");
    if (e.activation < QLIN_ACT_IDENTITY || e.activation > QLIN_ACT_SIGMOID)
        return fail(QLIN_ERR_INVALID, "unknown activation %d", e.activation);
    if (e.residual_index ? (!e.residual || e.residual_rows < 1)
                         : (e.residual && e.residual_rows != rows))
        return fail(QLIN_ERR_INVALID, "invalid indexed residual");
    if (e.rows_per_sequence < 1 || rows % e.rows_per_sequence || e.valid_rows_per_sequence < 0 ||
        e.valid_rows_per_sequence > e.rows_per_sequence)
        return fail(QLIN_ERR_INVALID, "invalid epilogue sequence length");
    const int sequences = rows / e.rows_per_sequence;
    if (!modulation_rows(e.gate, e.gate_rows, sequences))
        return fail(QLIN_ERR_INVALID, "invalid epilogue gate");
    if (!modulation_rows(e.condition, e.condition_rows, sequences))
        return fail(QLIN_ERR_INVALID, "invalid epilogue condition");
    if (int st = check_16bit_aligned({x, retained, e.bias, e.residual, e.raw, e.gate, e.condition}))
        return st;
    const Span q_values{values, size_t(rows) * cols};
    const size_t groups = group ? size_t((cols + group - 1) / group) : 1;
    const Span q_scales{scales, groups * rows * 4};
    const Span sources[] = {span16(x, x_rows, cols), span16(retained, rows, cols),
                            span16(e.bias, 1, cols), span16(e.residual, e.residual_rows, cols),
                            span16(e.raw, rows, cols), span16(e.gate, e.gate_rows, cols),
                            span16(e.condition, e.condition_rows, cols)};
    for (const Span &b : sources)
        if (overlaps(q_values, b) || overlaps(q_scales, b))
            return fail(QLIN_ERR_INVALID, "quantized output overlaps sequence storage");
    const Span row_outputs[] = {span16(retained, rows, cols), span16(e.raw, rows, cols)};
    if (overlaps(row_outputs[0], row_outputs[1]))
        return fail(QLIN_ERR_INVALID, "raw and retained sequence outputs overlap");
    for (const Span &o : row_outputs) {
        for (const Span &b : {span16(e.bias, 1, cols), span16(e.gate, e.gate_rows, cols),
                              span16(e.condition, e.condition_rows, cols)})
            if (overlaps(o, b))
                return fail(QLIN_ERR_INVALID, "quantized sequence output has unsafe row alias");
        if (overlaps(o, span16(x, x_rows, cols)) && (o.p != x || e.input_repeat != 1))
            return fail(QLIN_ERR_INVALID, "quantized sequence output has unsafe row alias");
        if (overlaps(o, span16(e.residual, e.residual_rows, cols)) &&
            (o.p != e.residual || e.residual_index))
            return fail(QLIN_ERR_INVALID, "quantized sequence output has unsafe row alias");
    }
    return QLIN_OK;
}
}  // namespace

int qlin_pointwise_quantize(const void *x, int x_rows, int src_type,
                            const qlin_epilogue *epilogue, void *retained, int rows, int cols,
                            void *values, float *scales, int fmt, int group, int rotation,
                            qlin_stream_t stream) {
    qlin_epilogue e;
    qlin_epilogue_init(&e);
    if (epilogue) e = *epilogue;
    if (int st = check_row_output(src_type, rows, cols, values, scales, fmt, group, rotation,
                                  "pointwise quantize"))
        return st;
    if (int st = check_pointwise(x, x_rows, e, retained, rows, cols, values, scales, group))
        return st;
    qlin::PointwiseQuantizeArgs a{x, x_rows, src_type, e, retained, rows, cols, values, scales,
                                  fmt, group, rotation};
    qlin::launch_pointwise_quantize(a, reinterpret_cast<hipStream_t>(stream));
    return check_launch("pointwise quantize launch");
}

int qlin_pointwise(const void *x, int x_rows, int src_type, const qlin_epilogue *epilogue,
                   void *y, int rows, int cols, qlin_stream_t stream) {
    qlin_epilogue e;
    qlin_epilogue_init(&e);
    if (epilogue) e = *epilogue;
    if (src_type != QLIN_BF16 && src_type != QLIN_F16)
        return fail(QLIN_ERR_INVALID, "pointwise input must be BF16 or F16");
    if (rows < 1 || cols < 1 || !y)
        return fail(QLIN_ERR_INVALID, "pointwise output rows=%d cols=%d", rows, cols);
    if (int st = check_pointwise(x, x_rows, e, y, rows, cols, nullptr, nullptr, 0)) return st;
    // The quantizing kernel with no codes: the epilogue's rows only.
    qlin::PointwiseQuantizeArgs a{x, x_rows, src_type, e, y, rows, cols, nullptr, nullptr,
                                  QLIN_I8, 0, 0};
    qlin::launch_pointwise_quantize(a, reinterpret_cast<hipStream_t>(stream));
    return check_launch("pointwise launch");
}

int qlin_quantized_gated(const void *input, int src_type, int rows, int width, int kind,
                         void *values, float *scales, int fmt, int group, int rotation,
                         qlin_stream_t stream) {
    // launch_quantized_gated's checks (reference quant_gated.cu:182-191).
    if (src_type != QLIN_BF16 && src_type != QLIN_F16)
        return fail(QLIN_ERR_INVALID, "quantized gated input must be BF16 or F16");
    if (fmt != QLIN_I8 && fmt != QLIN_FP8)
        return fail(QLIN_ERR_INVALID, "quantized storage must be I8 or FP8");
    if (rows < 1 || width < 1 || width > 8192 || kind < 0 || kind > 1)
        return fail(QLIN_ERR_INVALID, "quantized gated shape/kind rows=%d width=%d kind=%d", rows,
                    width, kind);
    if (!input || !values || !scales)
        return fail(QLIN_ERR_INVALID, "quantized gated pointer is null");
    if (!valid_group(group))
        return fail(QLIN_ERR_INVALID, "quantization group must be 0, 32, 64 or 128 (got %d)", group);
    if (rotation && (rotation != 128 || width % 128))
        return fail(QLIN_ERR_INVALID, "rotation must be 128 with width %% 128 == 0");
    if (!aligned(input, 2)) return fail(QLIN_ERR_ALIGNMENT, "16-bit input must be 2-byte aligned");
    if (!aligned(scales, 4)) return fail(QLIN_ERR_ALIGNMENT, "scales must be 4-byte aligned");
    qlin::GatedQuantizeArgs a{input, src_type, rows, width, values, scales, fmt, group, rotation,
                              kind};
    qlin::launch_quantized_gated(a, reinterpret_cast<hipStream_t>(stream));
    return check_launch("quantized gated launch");
}

}  // extern "C"
