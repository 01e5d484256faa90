// Measurement kernels behind the benchmark's device ceilings (gfx950).
//
// calib_mfma_kernel: a register-only loop of v_mfma_i32_32x32x32_i8 on four
// independent accumulators, no memory traffic.  With constant operands the
// matrix cores run at the nominal clock; with random operands (eight
// fragments per operand, cycled) the datapath toggles as it does on real
// int8 data and the part settles at its power-limited clock -- the
// practical ceiling a W8A8 GEMM on random data can approach.
//
// calib_read_kernel: a grid-stride streaming read (16 bytes per lane,
// eight loads in flight, non-temporal) -- the practical HBM read ceiling
// for a given buffer size.
//
// Both write one int per thread to `sink` so that nothing is optimised
// away; the caller times the launches with events on the same stream.
#include "mw8_common.h"

namespace mw8 {
namespace {

constexpr int kCalibThreads = 1024;
constexpr int kCalibBlocks = 256;
constexpr int kReadThreads = 256;
constexpr int kReadBlocks = 2048;

__device__ __forceinline__ unsigned mix32(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

template <int RANDOM>
__global__ __launch_bounds__(kCalibThreads) void calib_mfma_kernel(int iters, int32_t* sink) {
  const int tid = threadIdx.x;
  const unsigned seed = mix32(blockIdx.x * kCalibThreads + tid + 1);
  v4i A[8], B[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      A[i][j] = RANDOM ? static_cast<int>(mix32(seed + 17 * i + j)) : 0x01010101;
      B[i][j] = RANDOM ? static_cast<int>(mix32(seed * 3 + 29 * i + j + 100)) : 0x01010101;
    }
  }
  v16i acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = v16i{0};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[(k + j) & 7], B[(k + 3 * j) & 7], acc[j], 0, 0, 0);
  }
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) s += acc[i][0] + acc[i][15];
  sink[blockIdx.x * kCalibThreads + tid] = s;
}

__global__ __launch_bounds__(kReadThreads) void calib_read_kernel(const v4i* __restrict__ p, int64_t n16,
                                                                  int32_t* sink) {
  constexpr int U = 8;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kReadThreads + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kReadThreads;
  v4i acc = v4i{0};
  int64_t i = tid;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    v4i v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= p[i];
  sink[tid] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

}  // namespace

int64_t calib_sink_len() {
  return static_cast<int64_t>(kCalibBlocks) * kCalibThreads > static_cast<int64_t>(kReadBlocks) * kReadThreads
             ? static_cast<int64_t>(kCalibBlocks) * kCalibThreads
             : static_cast<int64_t>(kReadBlocks) * kReadThreads;
}

int calib_mfma_i8(int random_operands, int iters, int32_t* sink, int64_t sink_len, hipStream_t st) {
  MW8_REQUIRE(sink != nullptr, kErrArg, "calib_mfma_i8: null sink");
  MW8_REQUIRE(sink_len >= calib_sink_len(), kErrShape, "calib_mfma_i8: sink needs %lld int32",
              (long long)calib_sink_len());
  MW8_REQUIRE(iters > 0, kErrShape, "calib_mfma_i8: iters must be positive");
  if (random_operands)
    hipLaunchKernelGGL(calib_mfma_kernel<1>, dim3(kCalibBlocks), dim3(kCalibThreads), 0, st, iters, sink);
  else
    hipLaunchKernelGGL(calib_mfma_kernel<0>, dim3(kCalibBlocks), dim3(kCalibThreads), 0, st, iters, sink);
  return check_launch("calib_mfma_i8");
}

int calib_read(const void* buf, int64_t bytes, int32_t* sink, int64_t sink_len, hipStream_t st) {
  MW8_REQUIRE(buf != nullptr && sink != nullptr, kErrArg, "calib_read: null pointer");
  MW8_REQUIRE(bytes > 0 && bytes % 16 == 0, kErrShape, "calib_read: bytes must be a positive multiple of 16");
  MW8_REQUIRE((reinterpret_cast<uintptr_t>(buf) & 15u) == 0, kErrAlign, "calib_read: 16-byte alignment");
  MW8_REQUIRE(sink_len >= calib_sink_len(), kErrShape, "calib_read: sink needs %lld int32",
              (long long)calib_sink_len());
  hipLaunchKernelGGL(calib_read_kernel, dim3(kReadBlocks), dim3(kReadThreads), 0, st,
                     static_cast<const v4i*>(buf), bytes / 16, sink);
  return check_launch("calib_read");
}

}  // namespace mw8
