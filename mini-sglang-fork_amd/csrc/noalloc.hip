// The allocation-free dense GEMM entry (mw8_gemm_w8a8_bf16_noalloc): the K
// split's int32 partial tiles live in a file-scope device array instead of
// a caller's workspace.  The array sits in a code object of its own (no
// kernels here), so a device holds its kScratchBytes only once a process
// has called this entry there; the GEMM kernels it runs belong to gemm.hip.
#include <atomic>

#include "mw8_common.h"

namespace mw8 {

int gemm_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw, const void* bias, void* y,
                   int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes, hipStream_t st);

// kScratchBytes: 64 MiB, the workspace bound of a 256-CU MI355X (256 slots
// x one 256x256 int32 tile).  A split that would need more (a part with
// more CUs) is not taken: those tiles run whole, as with a short workspace.
// Host code never passes the array's name to a kernel (on the host it is
// only a stand-in for the symbol): the device address comes from
// hipGetSymbolAddress, taken once per device with that device current, and
// only that address is used.  Every call on a device shares its array; the
// partial tiles are fully written before they are read within one call, so
// nothing needs clearing, but calls that overlap on one device (concurrent
// streams) race.
namespace {
constexpr size_t kScratchBytes = size_t{64} << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
std::atomic<void*> g_scratch_ptr[64] = {};

int scratch_of_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(kErrLaunch, "hipGetDevice: %s", hipGetErrorString(e));
  MW8_REQUIRE(dev >= 0 && dev < 64, kErrArg, "gemm_noalloc: device %d out of range", dev);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(kErrLaunch, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return kOk;
}
}  // namespace

int gemm_w8a8_bf16_noalloc(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                           const void* bias, void* y, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  void* ws = nullptr;
  if (const int rc = scratch_of_current_device(&ws)) return rc;
  return gemm_w8a8_bf16(A, sa, W, sw, bias, y, M, N, K, ws, kScratchBytes, st);
}

}  // namespace mw8
