// Load-time weight packing for gfx950: row-major int8/e4m3 weights [N, K]
// -> MFMA fragment tiles (the "pre-quantized, pre-shuffled packed weight
// layout" that follows the reference's load-time quantization,
// io/weights.cpp:80-87).
//
// Packed layout (Kp = K rounded up to 64, N a multiple of 16):
//   tile (g, t) = weight rows [16g, 16g+16) x K bytes [64t, 64t+64), 1 KB,
//   at byte offset (g * Kp/64 + t) * 1024; inside a tile, 16-byte chunk
//   l = 16*q + r holds row 16g + r, K bytes [64t + 16q, +16) — the A fragment
//   of lane l of a 16x16x64 MFMA. Bytes past K are zero.
// A decode wave thus loads each fragment of 16 rows x 64 K as one contiguous
// 1 KB piece (lane l -> chunk l), and the K range of a row group is one
// contiguous run.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

namespace qlin {
namespace {

__global__ __launch_bounds__(256) void pack_weights(const uint8_t *__restrict__ w,
                                                    uint8_t *__restrict__ packed, int N, int K,
                                                    int tiles_k, size_t chunks) {
    const size_t q = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (q >= chunks) return;
    const size_t tile = q / 64;
    const int lane = int(q % 64);
    const int g = int(tile / tiles_k), t = int(tile % tiles_k);
    const int row = g * 16 + (lane & 15), k = t * 64 + (lane >> 4) * 16;
    uint4 v = {0, 0, 0, 0};
    if (k < K) v = *reinterpret_cast<const uint4 *>(w + size_t(row) * K + k);
    *reinterpret_cast<uint4 *>(packed + q * 16) = v;
}

}  // namespace

size_t packed_weight_bytes(int N, int K) { return size_t(N) * size_t((K + 63) / 64 * 64); }

void launch_pack_weights(const void *w, int N, int K, void *packed, hipStream_t stream) {
    const int tiles_k = (K + 63) / 64;
    const size_t chunks = size_t(N / 16) * tiles_k * 64;
    hipLaunchKernelGGL(pack_weights, dim3(unsigned((chunks + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const uint8_t *>(w), static_cast<uint8_t *>(packed), N, K,
                       tiles_k, chunks);
}

}  // namespace qlin
