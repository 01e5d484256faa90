// C-ABI surface of libmw8.so (declared in include/mw8.h): argument
// forwarding, error codes and the thread-local last-error message.
#include <cstdarg>
#include <cstdio>

#include "mw8.h"
#include "mw8_common.h"

namespace mw8 {

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(kErrLaunch, "%s: launch failed: %s", what, hipGetErrorString(e));
  return kOk;
}

int quant_per_token_bf16(const void*, int64_t, int64_t, int64_t, int8_t*, int64_t, float*, hipStream_t);
int act_and_mul_quant_bf16(const void*, int64_t, int64_t, int, int8_t*, float*, void*, hipStream_t);
size_t gemm_workspace_bytes(int64_t, int64_t, int64_t);
int gemm_act_cfg(int64_t, int64_t, int64_t);
size_t gemm_act_workspace_bytes(int64_t, int64_t, int64_t);
int gemm_act_w8a8_bf16(const int8_t*, const float*, const int8_t*, const float*, int, void*, int64_t, int64_t,
                       int64_t, void*, size_t, hipStream_t);
size_t gemm_workspace_max_bytes();
void set_tuning(int, int, int);
int tuning_count(int);
const char* gemm_kernel_name(int64_t, int64_t, int64_t);
int gemm_w8a8_bf16(const int8_t*, const float*, const int8_t*, const float*, const void*, void*,
                   int64_t, int64_t, int64_t, void*, size_t, hipStream_t);
int gemm_w8a8_i32(const int8_t*, const int8_t*, int32_t*, int64_t, int64_t, int64_t, void*, size_t,
                  hipStream_t);
int gemm_w8a8_bf16_noalloc(const int8_t*, const float*, const int8_t*, const float*, const void*, void*,
                           int64_t, int64_t, int64_t, hipStream_t);
int topk_softmax(const void*, int, int64_t, int, int, int, float*, int32_t*, hipStream_t);
int64_t moe_align_max_padded(int64_t, int, int);
int moe_align_block_size(const int32_t*, int64_t, int, int, int32_t*, int32_t*, int32_t*, hipStream_t);
int moe_sum_reduce_bf16(const void*, int64_t, int, int64_t, void*, hipStream_t);
int moe_gemm_act_w8a8(const int8_t*, const float*, const int8_t*, const float*, const int32_t*,
                      const int32_t*, const int32_t*, int64_t, const float*, int, int64_t, int64_t,
                      int64_t, int, int, int, void*, hipStream_t);
int moe_route_quant(const void*, int, int64_t, int, int, int, const void*, int64_t, float*, int32_t*, int8_t*,
                    float*, hipStream_t);
int moe_prepare_small(const void*, int, int64_t, int, int, int, const void*, int64_t, float*, int32_t*,
                      int8_t*, float*, int, int, int32_t*, int32_t*, int32_t*, hipStream_t);
int moe_gemm_w8a8(const int8_t*, const float*, const int8_t*, const float*, const int32_t*,
                  const int32_t*, const int32_t*, int64_t, const float*, int, int64_t, int64_t,
                  int64_t, int, int, void*, int, hipStream_t);
int moe_gemm_sum_w8a8(const int8_t*, const float*, const int8_t*, const float*, const int32_t*,
                      const int32_t*, const int32_t*, int64_t, const float*, int, int64_t, int64_t,
                      int64_t, int, void*, hipStream_t);
int moe_gemm_sum_lds_bytes(int64_t, int64_t, int);
int moe_gemm_topk_w8a8(const int8_t*, const float*, const int8_t*, const float*, const int32_t*, const float*, int,
                       int64_t, int64_t, int64_t, int, void*, int, hipStream_t);
int moe_gemm_sum_topk_w8a8(const int8_t*, const float*, const int8_t*, const float*, const int32_t*, const float*,
                           int, int64_t, int64_t, int64_t, int, void*, hipStream_t);
int rmsnorm_quant_bf16(const void*, void*, const void*, float, int64_t, int64_t, int8_t*, float*, void*,
                       hipStream_t);
int rmsnorm_strided_bf16(const void*, int64_t, void*, int64_t, const void*, float, int64_t, int64_t, int64_t,
                         hipStream_t);
int linear_bf16_w8a8(const void*, int64_t, const int8_t*, const float*, const void*, void*, int64_t, int64_t,
                     int64_t, hipStream_t);
int linear_bf16_supported(int64_t, int64_t, int64_t);

}  // namespace mw8

#define MW8_ENTRY(expr)                                                   \
  do {                                                                    \
    try {                                                                 \
      return (expr);                                                      \
    } catch (...) {                                                       \
      return ::mw8::set_error(::mw8::kErrLaunch, "unexpected C++ exception"); \
    }                                                                     \
  } while (0)

static inline hipStream_t S(mw8_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

extern "C" {

const char* mw8_last_error(void) { return mw8::g_last_error; }

int mw8_version(void) { return 200; }

int mw8_device_info(int32_t device, int32_t* num_cu, int32_t* clock_khz, int64_t* l2_bytes) {
  MW8_REQUIRE(num_cu && clock_khz && l2_bytes, mw8::kErrArg, "device_info: null pointer");
  hipDeviceProp_t p;
  const hipError_t e = hipGetDeviceProperties(&p, device);
  MW8_REQUIRE(e == hipSuccess, mw8::kErrLaunch, "device_info: %s", hipGetErrorString(e));
  *num_cu = p.multiProcessorCount;
  *clock_khz = p.clockRate;
  *l2_bytes = p.l2CacheSize;
  return mw8::kOk;
}

int mw8_quant_per_token_bf16(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                             int64_t ldq, float* s, mw8_stream_t st) {
  MW8_ENTRY(mw8::quant_per_token_bf16(x, M, K, ldx, q, ldq, s, S(st)));
}

int mw8_act_and_mul_quant_bf16(const void* x, int64_t R, int64_t two_d, int32_t act, int8_t* q,
                               float* s, void* act_out, mw8_stream_t st) {
  MW8_ENTRY(mw8::act_and_mul_quant_bf16(x, R, two_d, act, q, s, act_out, S(st)));
}

void mw8_set_tuning(int32_t decode_cfg, int32_t tile_cfg, int32_t moe_cfg) {
  mw8::set_tuning(decode_cfg, tile_cfg, moe_cfg);
}

int mw8_linear_bf16_w8a8(const void* x, int64_t ldx, const int8_t* W, const float* sw, const void* bias, void* y,
                         int64_t M, int64_t N, int64_t K, mw8_stream_t st) {
  MW8_ENTRY(mw8::linear_bf16_w8a8(x, ldx, W, sw, bias, y, M, N, K, S(st)));
}

int32_t mw8_linear_bf16_supported(int64_t M, int64_t N, int64_t K) { return mw8::linear_bf16_supported(M, N, K); }

size_t mw8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return mw8::gemm_workspace_bytes(M, N, K);
}

size_t mw8_gemm_workspace_max_bytes(void) { return mw8::gemm_workspace_max_bytes(); }

int32_t mw8_tuning_count(int32_t kind) { return mw8::tuning_count(kind); }

const char* mw8_gemm_kernel_name(int64_t M, int64_t N, int64_t K) { return mw8::gemm_kernel_name(M, N, K); }

int mw8_gemm_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                       const void* bias, void* y, int64_t M, int64_t N, int64_t K, void* ws,
                       size_t ws_bytes, mw8_stream_t st) {
  MW8_ENTRY(mw8::gemm_w8a8_bf16(A, sa, W, sw, bias, y, M, N, K, ws, ws_bytes, S(st)));
}

int mw8_gemm_act_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw, int32_t act, void* y,
                           int64_t M, int64_t I, int64_t K, void* ws, size_t ws_bytes, mw8_stream_t st) {
  MW8_ENTRY(mw8::gemm_act_w8a8_bf16(A, sa, W, sw, act, y, M, I, K, ws, ws_bytes, S(st)));
}

int32_t mw8_gemm_act_supported(int64_t M, int64_t I, int64_t K) { return mw8::gemm_act_cfg(M, I, K) >= 0 ? 1 : 0; }

size_t mw8_gemm_act_workspace_bytes(int64_t M, int64_t I, int64_t K) {
  return mw8::gemm_act_workspace_bytes(M, I, K);
}

int mw8_gemm_w8a8_bf16_noalloc(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                               const void* bias, void* y, int64_t M, int64_t N, int64_t K, mw8_stream_t st) {
  MW8_ENTRY(mw8::gemm_w8a8_bf16_noalloc(A, sa, W, sw, bias, y, M, N, K, S(st)));
}

int mw8_gemm_w8a8_i32(const int8_t* A, const int8_t* W, int32_t* acc, int64_t M, int64_t N,
                      int64_t K, void* ws, size_t ws_bytes, mw8_stream_t st) {
  MW8_ENTRY(mw8::gemm_w8a8_i32(A, W, acc, M, N, K, ws, ws_bytes, S(st)));
}

int mw8_topk_softmax(const void* logits, int32_t is_bf16, int64_t M, int32_t E, int32_t topk,
                     int32_t renorm, float* tw, int32_t* ti, mw8_stream_t st) {
  MW8_ENTRY(mw8::topk_softmax(logits, is_bf16, M, E, topk, renorm, tw, ti, S(st)));
}

int64_t mw8_moe_align_max_padded(int64_t numel, int32_t slots, int32_t bsz) {
  return mw8::moe_align_max_padded(numel, slots, bsz);
}

int mw8_moe_align_block_size(const int32_t* ids, int64_t numel, int32_t slots, int32_t bsz,
                             int32_t* sorted_ids, int32_t* expert_ids, int32_t* npp,
                             mw8_stream_t st) {
  MW8_ENTRY(mw8::moe_align_block_size(ids, numel, slots, bsz, sorted_ids, expert_ids, npp, S(st)));
}

int mw8_moe_gemm_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                           const int32_t* sorted_ids, const int32_t* expert_ids,
                           const int32_t* npp, int64_t max_sorted, const float* topk_w,
                           int32_t top_k, int64_t num_valid, int64_t N, int64_t K, int32_t E,
                           int32_t bsz, void* out, mw8_stream_t st) {
  MW8_ENTRY(mw8::moe_gemm_w8a8(A, sa, W, sw, sorted_ids, expert_ids, npp, max_sorted, topk_w,
                               top_k, num_valid, N, K, E, bsz, out, 0 /* bf16 epilogue */, S(st)));
}

int mw8_moe_gemm_w8a8_i32(const int8_t* A, const int8_t* W, const int32_t* sorted_ids,
                          const int32_t* expert_ids, const int32_t* npp, int64_t max_sorted,
                          int32_t top_k, int64_t num_valid, int64_t N, int64_t K, int32_t E,
                          int32_t bsz, int32_t* out, mw8_stream_t st) {
  MW8_ENTRY(mw8::moe_gemm_w8a8(A, nullptr, W, nullptr, sorted_ids, expert_ids, npp, max_sorted,
                               nullptr, top_k, num_valid, N, K, E, bsz, out, 1 /* int32 out */, S(st)));
}

int mw8_moe_gemm_act_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                               const int32_t* sorted_ids, const int32_t* expert_ids,
                               const int32_t* num_post_pad, int64_t max_sorted, const float* topk_w,
                               int32_t top_k, int64_t num_valid, int64_t N, int64_t K, int32_t E,
                               int32_t block_size, int32_t act, void* out, mw8_stream_t stream) {
  MW8_ENTRY(mw8::moe_gemm_act_w8a8(A, sa, W, sw, sorted_ids, expert_ids, num_post_pad, max_sorted, topk_w,
                                   top_k, num_valid, N, K, E, block_size, act, out, S(stream)));
}

int mw8_moe_gemm_sum_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                               const int32_t* sorted_ids, const int32_t* expert_ids,
                               const int32_t* num_post_pad, int64_t max_sorted, const float* topk_w,
                               int32_t top_k, int64_t num_valid, int64_t N, int64_t K, int32_t E, void* out,
                               mw8_stream_t stream) {
  MW8_ENTRY(mw8::moe_gemm_sum_w8a8(A, sa, W, sw, sorted_ids, expert_ids, num_post_pad, max_sorted, topk_w,
                                   top_k, num_valid, N, K, E, out, S(stream)));
}

int mw8_moe_gemm_topk_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                                const int32_t* topk_ids, const float* topk_w, int32_t top_k, int64_t num_valid,
                                int64_t N, int64_t K, int32_t E, void* out, mw8_stream_t stream) {
  MW8_ENTRY(mw8::moe_gemm_topk_w8a8(A, sa, W, sw, topk_ids, topk_w, top_k, num_valid, N, K, E, out,
                                    0 /* bf16 epilogue */, S(stream)));
}

int mw8_moe_gemm_sum_topk_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                                    const int32_t* topk_ids, const float* topk_w, int32_t top_k,
                                    int64_t num_valid, int64_t N, int64_t K, int32_t E, void* out,
                                    mw8_stream_t stream) {
  MW8_ENTRY(mw8::moe_gemm_sum_topk_w8a8(A, sa, W, sw, topk_ids, topk_w, top_k, num_valid, N, K, E, out,
                                        S(stream)));
}

int32_t mw8_moe_gemm_sum_supported(int64_t max_sorted, int64_t num_valid, int32_t E) {
  return mw8::moe_gemm_sum_lds_bytes(max_sorted, num_valid, E) > 0 ? 1 : 0;
}

int mw8_moe_route_quant(const void* logits, int32_t is_bf16, int64_t M, int32_t E, int32_t topk,
                        int32_t renorm, const void* hidden, int64_t H, float* topk_w, int32_t* topk_ids,
                        int8_t* q, float* s, mw8_stream_t stream) {
  MW8_ENTRY(mw8::moe_route_quant(logits, is_bf16, M, E, topk, renorm, hidden, H, topk_w, topk_ids, q, s,
                                 S(stream)));
}

int mw8_moe_prepare_small(const void* logits, int32_t is_bf16, int64_t M, int32_t E, int32_t topk,
                          int32_t renorm, const void* hidden, int64_t H, float* topk_w,
                          int32_t* topk_ids, int8_t* q, float* s, int32_t slots, int32_t block_size,
                          int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_post_pad,
                          mw8_stream_t stream) {
  MW8_ENTRY(mw8::moe_prepare_small(logits, is_bf16, M, E, topk, renorm, hidden, H, topk_w, topk_ids, q, s,
                                   slots, block_size, sorted_ids, expert_ids, num_post_pad, S(stream)));
}

int mw8_moe_sum_reduce_bf16(const void* in, int64_t M, int32_t k, int64_t H, void* out,
                            mw8_stream_t st) {
  MW8_ENTRY(mw8::moe_sum_reduce_bf16(in, M, k, H, out, S(st)));
}

int mw8_rmsnorm_quant_bf16(const void* x, void* residual, const void* weight, float eps, int64_t M,
                           int64_t H, int8_t* q, float* s, void* y, mw8_stream_t st) {
  MW8_ENTRY(mw8::rmsnorm_quant_bf16(x, residual, weight, eps, M, H, q, s, y, S(st)));
}

int mw8_rmsnorm_strided_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, const void* weight, float eps,
                             int64_t G, int64_t inner, int64_t H, mw8_stream_t st) {
  MW8_ENTRY(mw8::rmsnorm_strided_bf16(x, ldx, y, ldy, weight, eps, G, inner, H, S(st)));
}

}  // extern "C"
