// Shared helpers for the W8A8 HIP library (gfx950 / CDNA4 only).
//
// Numerics contract (bit-exact against the CPU oracle):
//   * the per-token quantizer computes s = amax / 127 with one correctly
//     rounded fp32 division and q = clamp(rint(x / s), -127, 127) where x / s
//     is the correctly rounded fp32 quotient (obtained per element from the
//     row reciprocal plus one FMA correction, see quant_div_rne);
//   * the GEMM epilogue is ((float)acc * s_a) * s_w [+ bias] [* routed] with
//     every operation rounded separately (the library is compiled with
//     -ffp-contract=off), then round-to-nearest-even to bf16.
#pragma once

#include <stdint.h>

#ifndef MW8_HOST_ONLY
#include <hip/hip_runtime.h>
#define MW8_HD __host__ __device__ __forceinline__
#else
#define MW8_HD inline
#endif

namespace mw8 {

// ---------------------------------------------------------------- bf16 bits
MW8_HD float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even narrowing of a finite fp32 value to bf16.
MW8_HD uint16_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// ------------------------------------------------------------- quantization
// Rows whose absmax is below this bound take the plain IEEE-division path:
// there 1/s may overflow and the FMA residual may lose bits to underflow.
constexpr float kQuantFastMin = 0x1p-60f;

// Per-row constants of the quantizer.
struct RowScale {
  float s;    // amax / 127 (correctly rounded)
  float r;    // 1 / s      (correctly rounded), 0 if s == 0
  bool fast;  // Markstein path valid for this row
};

MW8_HD RowScale row_scale(float amax) {
  RowScale rs;
  rs.s = amax / 127.0f;
  rs.fast = amax >= kQuantFastMin;
  rs.r = rs.s > 0.0f ? 1.0f / rs.s : 0.0f;
  return rs;
}

// Clamp of an integral fp32 value to [-127, 127] (finite inputs): one
// v_med3_f32 on the device.
MW8_HD float clamp127(float t) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_fmed3f(t, -127.0f, 127.0f);
#else
  t = t < -127.0f ? -127.0f : t;
  return t > 127.0f ? 127.0f : t;
#endif
}

// rint(x / s) with x / s the correctly rounded fp32 quotient, clamped to
// [-127, 127].  Fast path: q0 = RN(x * r) is within one ulp of x / s when r
// is the correctly rounded reciprocal; e = x - q0 * s is exact (FMA) and
// RN(q0 + e * r) is then the correctly rounded quotient (Markstein, "IA-64
// and Elementary Functions", Theorem 8.10).  Exhaustively checked against
// IEEE division for every bf16 input on the CPU (tests/native).
// The FAST flag is per row: kernels branch once per row on rs.fast and
// instantiate both variants, so no element pays for the division path.
template <bool FAST>
MW8_HD float quant_div_rne_t(float x, const RowScale& rs) {
  float t;
  if (FAST) {
    float q0 = x * rs.r;
    float e = __builtin_fmaf(-q0, rs.s, x);
    t = __builtin_fmaf(e, rs.r, q0);
  } else {
    t = rs.s > 0.0f ? x / rs.s : 0.0f;
  }
  return clamp127(__builtin_rintf(t));
}

MW8_HD float quant_div_rne(float x, const RowScale& rs) {
  return rs.fast ? quant_div_rne_t<true>(x, rs) : quant_div_rne_t<false>(x, rs);
}

// ---------------------------------------------------------------- epilogue
MW8_HD float epi_scale(int32_t acc, float sa, float sw) {
  float t = static_cast<float>(acc);
  t = t * sa;
  t = t * sw;
  return t;
}

}  // namespace mw8

#ifndef MW8_HOST_ONLY
// ---------------------------------------------------------------- errors
namespace mw8 {
enum Status : int {
  kOk = 0,
  kErrArg = 1,        // null pointer / bad enum
  kErrShape = 2,      // unsupported or inconsistent sizes
  kErrAlign = 3,      // pointer or leading dimension not aligned
  kErrWorkspace = 4,  // workspace too small
  kErrLaunch = 5,     // HIP launch failure
};
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Gated activation of the MoE / MLP intermediate (shared by the activation
// kernel and the GEMM epilogue that fuses it): silu with the hardware
// reciprocal, or erf-gelu.
template <int ACT>
__device__ __forceinline__ float act_fn(float g) {
  if constexpr (ACT == 0) return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));  // silu
  else return 0.5f * g * (1.0f + erff(g * 0.70710678118654752440f));  // gelu (erf)
}

// Quantizer building blocks shared by the row quantizers and the fused
// decode GEMM.
// 8 bf16 values packed two per 32-bit register (element j in bits
// 16*(j&1) .. of word j/2), so a register-resident row costs 4 VGPRs per
// 16-byte vector.
struct alignas(16) U16x8 {
  uint32_t w[4];
  __device__ __forceinline__ uint32_t get(int j) const {
    return (j & 1) ? (w[j >> 1] >> 16) : (w[j >> 1] & 0xFFFFu);
  }
};

// bf16 element 2j / 2j+1 of a packed word as fp32 (one shift or one mask)
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }

// Four integral fp32 values in [-127, 127] -> four int8 bytes of a word.
__device__ __forceinline__ uint32_t pack4_i8(float a, float b, float c, float d) {
  const uint32_t lo = (static_cast<uint32_t>(static_cast<int>(a)) & 0xFFu) |
                      ((static_cast<uint32_t>(static_cast<int>(b)) & 0xFFu) << 8);
  const uint32_t hi = (static_cast<uint32_t>(static_cast<int>(c)) & 0xFFu) |
                      ((static_cast<uint32_t>(static_cast<int>(d)) & 0xFFu) << 8);
  return lo | (hi << 16);
}

template <bool FAST>
__device__ __forceinline__ uint2 quant8(const U16x8& v, const RowScale& rs) {
  float f[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = quant_div_rne_t<FAST>(bf16_lo(v.w[j]), rs);
    f[2 * j + 1] = quant_div_rne_t<FAST>(bf16_hi(v.w[j]), rs);
  }
  return make_uint2(pack4_i8(f[0], f[1], f[2], f[3]), pack4_i8(f[4], f[5], f[6], f[7]));
}

}  // namespace mw8

#define MW8_REQUIRE(cond, code, ...)                     \
  do {                                                   \
    if (!(cond)) return ::mw8::set_error((code), __VA_ARGS__); \
  } while (0)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
#endif
