// Row-gather probe: the rate at which one MI355X gathers random 64-byte rows, the
// access that bounds the MSDA sample kernels (each bilinear corner of a bf16 head of
// 32 channels is one 64-byte row, fetched by 4 lanes x 16 bytes). bench.py runs it
// beside the MSDA calls and rates their corner gathers against it. Rows of 128
// bytes (8 lanes, one whole cache line) show whether the rate is set by bytes or by
// line requests.
//
// Every wave walks `iters` rounds of kUnroll loads; in each load its groups of
// row_bytes / 16 lanes fetch one pseudo-random row of a `rows`-row buffer (rows a
// power of two).
// With a buffer smaller than the 32 KB L1 of a CU the loads hit in L1; with one of a
// few MB they hit in each XCD's L2 after the first touch; a large one measures the
// memory behind the L2s. Lanes fold what they load into one word per lane, stored at
// the end, so no load is dead.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kWave = 64;
constexpr int kUnroll = 8;

typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));

// A 32-bit mixing function (Wellons' lowbias32), enough to spread rows over a buffer.
__device__ inline uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

template <int kPieces>  // 16-byte pieces per row
__global__ __launch_bounds__(256) void row_gather_kernel(const u32x4_v* __restrict__ buf, uint32_t row_mask,
                                                         int iters, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const uint32_t group = uint32_t(lane / kPieces), piece = uint32_t(lane % kPieces);
  uint32_t seed = mix(wave * 0x9e3779b9U + group);
  u32x4_v acc = {0u, 0u, 0u, 0u};
  for (int it = 0; it < iters; ++it) {
    u32x4_v v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      seed = mix(seed + uint32_t(u));
      v[u] = buf[size_t(seed & row_mask) * kPieces + piece];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
  }
  sink[blockIdx.x * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

}  // namespace

extern "C" {

// Launches the probe on `stream`: `blocks` workgroups of 256 threads, each wave
// gathering iters * 8 * (1024 / row_bytes) rows of row_bytes (64 or 128) bytes from
// `buffer` (rows * row_bytes bytes, rows a power of two). `sink` takes one uint32
// per thread. Returns 0, or 1 for bad arguments or a failed launch.
int msda_probe_row_gather(const void* buffer, int64_t rows, int row_bytes, int blocks, int iters, void* sink,
                          void* stream) {
  if (!buffer || !sink || rows <= 0 || (rows & (rows - 1)) != 0 || rows > (int64_t(1) << 31) || blocks <= 0 ||
      iters <= 0 || (row_bytes != 64 && row_bytes != 128))
    return 1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const auto* buf = static_cast<const u32x4_v*>(buffer);
  auto* out = static_cast<uint32_t*>(sink);
  if (row_bytes == 64)
    hipLaunchKernelGGL(row_gather_kernel<4>, dim3(unsigned(blocks)), dim3(256), 0, st, buf, uint32_t(rows - 1),
                       iters, out);
  else
    hipLaunchKernelGGL(row_gather_kernel<8>, dim3(unsigned(blocks)), dim3(256), 0, st, buf, uint32_t(rows - 1),
                       iters, out);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // extern "C"
