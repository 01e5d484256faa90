// Host-side exhaustive check of the quantizer's per-element math
// (mw8::quant_div_rne in mini-sglang-fork_amd/csrc/mw8_common.h): the
// reciprocal + FMA-correction path must give the same integer as
// rint(x / s) with one IEEE division, for every bf16 input x with
// |x| <= amax and every bf16 mantissa of amax, over a spread of exponents.
// The fp32 quotient itself must also match whenever |x| >= 2^-100.
// Prints "mismatches=<n> checked=<m>" and exits nonzero on any mismatch.
#define MW8_HOST_ONLY 1
#include "mw8_common.h"

#include <cmath>
#include <cstdio>

int main() {
  long long checked = 0, bad = 0, bad_quot = 0;
  const int exps[] = {-59, -40, -10, -3, 0, 1, 4, 7, 20, 60, 126};
  for (int ei : exps) {
    for (int mant = 0; mant < 128; ++mant) {
      // amax = (1 + mant/128) * 2^ei, a positive normal bf16 value.
      uint16_t ab = static_cast<uint16_t>(((ei + 127) << 7) | mant);
      float amax = mw8::bf16_to_f32(ab);
      mw8::RowScale rs = mw8::row_scale(amax);
      if (!rs.fast) continue;
      for (uint32_t xb = 0; xb < 0x10000u; ++xb) {
        float x = mw8::bf16_to_f32(static_cast<uint16_t>(xb));
        if (!std::isfinite(x) || std::fabs(x) > amax) continue;
        float q0 = x * rs.r;
        float e = std::fma(-q0, rs.s, x);
        float q1 = std::fma(e, rs.r, q0);
        float ieee = x / rs.s;
        // For |x| < 2^-100 the residual x - q0*s can fall into the subnormal
        // range; with amax >= 2^-60 such quotients are below 2^-33 and round
        // to 0 whichever way they are rounded.
        if (q1 != ieee && std::fabs(x) >= 0x1p-100f) ++bad_quot;
        float ref = std::rint(ieee);
        ref = ref < -127.f ? -127.f : (ref > 127.f ? 127.f : ref);
        float got = mw8::quant_div_rne(x, rs);
        if (got != ref) ++bad;
        ++checked;
      }
    }
  }
  std::printf("mismatches=%lld quotient_mismatches=%lld checked=%lld\n", bad, bad_quot, checked);
  return (bad || bad_quot) ? 1 : 0;
}
