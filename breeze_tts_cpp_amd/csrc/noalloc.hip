// qlin_linear_noalloc: the quantized linear (qlin_linear) with its scratch
// (activation codes, activation scales, split-K partials) in a fixed device
// array owned by the library, for callers that cannot allocate: code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
//
// The array `scratch` is a file-scope __device__ variable, so every GPU the
// library runs on holds its own copy (kScratchBytes) until the process ends.
// Host code never passes the array's name to a kernel (on the host it is only
// a stand-in symbol): its device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and that address is what the
// launches receive.
//
// Every call on a device shares that device's array and leaves its contents
// behind. Nothing in it needs to start at zero: each call writes every byte
// it reads (codes and scales by the quantizer or the fused GEMM, partials by
// the split-K GEMM before the reduction). Calls that overlap in time on one
// device (two streams, two threads) race on the array.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "qlin_internal.hpp"

namespace {

constexpr size_t kScratchBytes = size_t(QLIN_NOALLOC_SCRATCH_BYTES);
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mutex;
void *g_scratch[kMaxDevices] = {};

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Device address of `scratch` on `device` (looked up once, with the device
// current, then cached); nullptr with the error recorded on failure.
void *scratch_on(int device, int *status) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_scratch[device]) return g_scratch[device];
    int previous = -1;
    if (hipGetDevice(&previous) != hipSuccess) previous = -1;
    if (previous != device && hipSetDevice(device) != hipSuccess) {
        *status = qlin::set_error(QLIN_ERR_HIP, "qlin_linear_noalloc: cannot select the stream's device");
        return nullptr;
    }
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (previous >= 0 && previous != device) (void)hipSetDevice(previous);
    if (e != hipSuccess || !ptr) {
        char message[256];
        snprintf(message, sizeof(message), "qlin_linear_noalloc: hipGetSymbolAddress: %s",
                 hipGetErrorString(e));
        *status = qlin::set_error(QLIN_ERR_HIP, message);
        return nullptr;
    }
    g_scratch[device] = ptr;
    return ptr;
}

}  // namespace

extern "C" {

size_t qlin_noalloc_scratch_bytes(void) { return kScratchBytes; }

int qlin_linear_noalloc(const qlin_path *path, const void *x, int ld, int src_type,
                        const void *w, const float *sw, void *y, int rows, int N, int K, int fmt,
                        int out_type, int input_group, int weight_group, int rotation,
                        qlin_stream_t stream) {
    if (rows < 1 || N < 1 || K < 1)
        return qlin::set_error(QLIN_ERR_INVALID, "qlin_linear_noalloc: invalid shape");
    // The group sizes qlin_linear accepts, checked before they size the
    // scratch layout.
    auto valid_group = [](int g) { return g == 0 || g == 32 || g == 64 || g == 128; };
    if (!valid_group(input_group) || !valid_group(weight_group))
        return qlin::set_error(QLIN_ERR_INVALID,
                               "qlin_linear_noalloc: quantization group must be 0, 32, 64 or 128");
    // Layout: codes [rows, K] | scales [groups, rows] | split-K partials,
    // each 256-byte aligned.
    const size_t groups = input_group ? (size_t(K) + input_group - 1) / input_group : 1;
    const size_t codes = round_up(size_t(rows) * K, 256);
    const size_t scales = round_up(groups * rows * 4, 256);
    const size_t partials = qlin_workspace_bytes(path, rows, N, K, fmt, input_group, weight_group);
    const size_t need = codes + scales + round_up(partials, 256);
    if (need > kScratchBytes) {
        char message[256];
        snprintf(message, sizeof(message),
                 "qlin_linear_noalloc: scratch of %zu bytes exceeds the fixed %zu-byte array "
                 "(rows * K + scales + split-K partials)",
                 need, kScratchBytes);
        return qlin::set_error(QLIN_ERR_WORKSPACE, message);
    }
    int device = 0;
    if (hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &device) != hipSuccess ||
        device < 0 || device >= kMaxDevices)
        return qlin::set_error(QLIN_ERR_HIP, "qlin_linear_noalloc: cannot query the stream's device");
    int status = QLIN_ERR_HIP;
    unsigned char *base = static_cast<unsigned char *>(scratch_on(device, &status));
    if (!base) return status;
    return qlin_linear(path, x, ld, src_type, base, reinterpret_cast<float *>(base + codes), w, sw,
                       y, rows, N, K, fmt, out_type, input_group, weight_group, rotation,
                       partials ? base + codes + scales : nullptr, partials, stream);
}

}  // extern "C"
