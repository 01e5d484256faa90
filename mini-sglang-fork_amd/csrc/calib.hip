// Measurement kernels behind the benchmark's device ceilings (gfx950).
//
// calib_mfma_kernel: a register-only loop of v_mfma_i32_16x16x64_i8 (the
// instruction of the large-M tiles) on eight independent accumulators, no
// memory traffic.  With constant operands the matrix cores run at the
// nominal clock; with random operands (eight fragments per operand, cycled)
// the datapath toggles as it does on real int8 data and the part settles at
// its power-limited clock -- the practical ceiling a W8A8 GEMM on random
// data can approach.  (On MI355X: 4.98 POPS constant, 3.92-3.99 random; the
// same loop on v_mfma_i32_32x32x32_i8 reaches 3.35-3.41 random.)
//
// calib_read_kernel: a grid-stride streaming read (16 bytes per lane,
// eight loads in flight, non-temporal) -- the practical HBM read ceiling
// for a given buffer size.
//
// calib_stream_lds_kernel: the GEMM rings' operand path (16-byte
// buffer_load ... lds) streaming a region per block, shared by the 32
// blocks of an XCD or private to each block -- the L2-resident rate, the
// rate of lockstep streaming where every line is one miss and 31 merged
// requests (the pattern of a tile kernel's shared operand panels), and the
// plain HBM rate through this path.
//
// All write one int per thread to `sink` so that nothing is optimised
// away; the caller times the launches with events on the same stream.
//
// Built as its own library, libmw8_calib.so (C ABI in include/mw8_calib.h),
// so that the product library carries no measurement surface; its error
// state is its own (mw8_calib_last_error).
#include <cstdarg>
#include <cstdio>

#include "mw8_calib.h"
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
  v4i acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = v4i{0};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[(k + j) & 7], B[(k + 3 * j) & 7], acc[j], 0, 0, 0);
  }
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += acc[i][0] + acc[i][3];
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

// Streams a region from global memory into LDS with 16-byte buffer_load ...
// lds (the operand path of the GEMM rings): each of a block's 4 waves keeps
// 8-16 instructions (1 KB each) in flight through a 64 KB LDS ring.  Block
// b reads region b % 8 (shared) or region b (not shared), `passes` times.
constexpr int kStreamBlocks = 256;
__global__ __launch_bounds__(256) void calib_stream_lds_kernel(const char* buf, int64_t region, int passes,
                                                               int shared, int32_t* sink) {
  __shared__ __align__(16) unsigned char ring[65536];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t r = shared ? blockIdx.x % 8 : blockIdx.x;
  const uint64_t base = reinterpret_cast<uint64_t>(buf + r * region);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(base)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(base >> 32)));
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo), 0, 0x7fffffff, 0x00020000);
  const int64_t per_wave = region / 4096;  // 1 KB instructions per wave and pass (a multiple of 8)
  int slot = 0;
  for (int p = 0; p < passes; ++p) {
    for (int64_t i = 0; i < per_wave; i += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int off = static_cast<int>(((i + u) * 4 + wave) * 1024);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)(ring + ((slot + u) & 15) * 4096 + wave * 1024), 16,
            static_cast<uint32_t>(lane * 16), off, 0, 0);
      }
      slot += 8;
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  sink[blockIdx.x * 256 + threadIdx.x] = ring[threadIdx.x * 16];
}

thread_local char g_calib_error[512] = "";

int calib_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_calib_error, sizeof(g_calib_error), fmt, ap);
  va_end(ap);
  return code;
}

int calib_check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return calib_error(kErrLaunch, "%s: launch failed: %s", what, hipGetErrorString(e));
  return kOk;
}

#define CALIB_REQUIRE(cond, code, ...)                    \
  do {                                                    \
    if (!(cond)) return calib_error((code), __VA_ARGS__); \
  } while (0)

int64_t calib_sink_len() {
  return static_cast<int64_t>(kCalibBlocks) * kCalibThreads > static_cast<int64_t>(kReadBlocks) * kReadThreads
             ? static_cast<int64_t>(kCalibBlocks) * kCalibThreads
             : static_cast<int64_t>(kReadBlocks) * kReadThreads;
}

int calib_mfma_i8(int random_operands, int iters, int32_t* sink, int64_t sink_len, hipStream_t st) {
  CALIB_REQUIRE(sink != nullptr, kErrArg, "calib_mfma_i8: null sink");
  CALIB_REQUIRE(sink_len >= calib_sink_len(), kErrShape, "calib_mfma_i8: sink needs %lld int32",
              (long long)calib_sink_len());
  CALIB_REQUIRE(iters > 0, kErrShape, "calib_mfma_i8: iters must be positive");
  if (random_operands)
    hipLaunchKernelGGL(calib_mfma_kernel<1>, dim3(kCalibBlocks), dim3(kCalibThreads), 0, st, iters, sink);
  else
    hipLaunchKernelGGL(calib_mfma_kernel<0>, dim3(kCalibBlocks), dim3(kCalibThreads), 0, st, iters, sink);
  return calib_check_launch("calib_mfma_i8");
}

int calib_read(const void* buf, int64_t bytes, int32_t* sink, int64_t sink_len, hipStream_t st) {
  CALIB_REQUIRE(buf != nullptr && sink != nullptr, kErrArg, "calib_read: null pointer");
  CALIB_REQUIRE(bytes > 0 && bytes % 16 == 0, kErrShape, "calib_read: bytes must be a positive multiple of 16");
  CALIB_REQUIRE((reinterpret_cast<uintptr_t>(buf) & 15u) == 0, kErrAlign, "calib_read: 16-byte alignment");
  CALIB_REQUIRE(sink_len >= calib_sink_len(), kErrShape, "calib_read: sink needs %lld int32",
              (long long)calib_sink_len());
  hipLaunchKernelGGL(calib_read_kernel, dim3(kReadBlocks), dim3(kReadThreads), 0, st,
                     static_cast<const v4i*>(buf), bytes / 16, sink);
  return calib_check_launch("calib_read");
}

int calib_stream_lds(const void* buf, int64_t region_bytes, int passes, int shared, int32_t* sink,
                     int64_t sink_len, hipStream_t st) {
  CALIB_REQUIRE(buf != nullptr && sink != nullptr, kErrArg, "calib_stream_lds: null pointer");
  CALIB_REQUIRE(region_bytes >= 32768 && region_bytes % 32768 == 0 && region_bytes <= (int64_t{1} << 30), kErrShape,
              "calib_stream_lds: region_bytes must be a multiple of 32 KiB, at most 1 GiB");
  CALIB_REQUIRE(passes >= 1 && (shared == 0 || shared == 1), kErrArg, "calib_stream_lds: passes >= 1, shared 0 or 1");
  CALIB_REQUIRE((reinterpret_cast<uintptr_t>(buf) & 15u) == 0, kErrAlign, "calib_stream_lds: 16-byte alignment");
  CALIB_REQUIRE(sink_len >= static_cast<int64_t>(kStreamBlocks) * 256, kErrShape, "calib_stream_lds: sink too short");
  hipLaunchKernelGGL(calib_stream_lds_kernel, dim3(kStreamBlocks), dim3(256), 0, st, static_cast<const char*>(buf),
                     region_bytes, passes, shared, sink);
  return calib_check_launch("calib_stream_lds");
}

}  // namespace
}  // namespace mw8

extern "C" {

const char* mw8_calib_last_error(void) { return mw8::g_calib_error; }

int64_t mw8_calib_sink_len(void) { return mw8::calib_sink_len(); }

int mw8_calib_mfma_i8(int32_t random_operands, int32_t iters, int32_t* sink, int64_t sink_len,
                      mw8_stream_t st) {
  return mw8::calib_mfma_i8(random_operands, iters, sink, sink_len, static_cast<hipStream_t>(st));
}

int mw8_calib_read(const void* buf, int64_t bytes, int32_t* sink, int64_t sink_len, mw8_stream_t st) {
  return mw8::calib_read(buf, bytes, sink, sink_len, static_cast<hipStream_t>(st));
}

int mw8_calib_stream_lds(const void* buf, int64_t region_bytes, int32_t passes, int32_t shared, int32_t* sink,
                         int64_t sink_len, mw8_stream_t st) {
  return mw8::calib_stream_lds(buf, region_bytes, passes, shared, sink, sink_len, static_cast<hipStream_t>(st));
}

}  // extern "C"
