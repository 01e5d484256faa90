// Per-token dynamic int8 quantizer and fused activation + requant (gfx950).
//
// quant_rows:   x bf16 [M, K] -> q int8 [M, K], s fp32 [M]
//               s = amax/127, q = clamp(rint(x/s), -127, 127)   (bit-exact)
// act_rows:     x bf16 [R, 2d] (gate | up) -> a = bf16(act(g) * u) ->
//               quantized exactly as above; optionally also writes a.
//
// One row is owned by TPR threads (32 = half a wave, 64 = one wave, or 256 = four waves).
// Each thread keeps VPT 16-byte vectors (8 bf16) of the row in registers,
// so the row is read from HBM once: 16-byte coalesced loads, an integer
// max over the sign-cleared bf16 bit patterns (monotone for finite
// values), a wave/LDS max-reduction, then quantize-from-registers and
// 8-byte stores.  Rows whose length exceeds TPR*VPT*8 take the generic
// kernel, which re-reads the row (second read hits L2).
#include "mw8_common.h"

namespace mw8 {
namespace {

constexpr int kBlock = 256;


typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
// Row loads and stores of the streaming row kernels are non-temporal: every
// byte is touched once (config 2 quantizer on MI355X: 92.6 -> 80.3 us).
__device__ __forceinline__ U16x8 ld_row16(const U16x8* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  U16x8 r;
  r.w[0] = v[0]; r.w[1] = v[1]; r.w[2] = v[2]; r.w[3] = v[3];
  return r;
}
__device__ __forceinline__ void st_row16(U16x8* p, const U16x8& v) {
  __builtin_nontemporal_store(u32x4{v.w[0], v.w[1], v.w[2], v.w[3]}, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void st_row8(uint2* p, uint2 v) {
  __builtin_nontemporal_store(u32x2{v.x, v.y}, reinterpret_cast<u32x2*>(p));
}

// Max over aligned groups of W lanes (W = 32: each half of the wave).
template <int W = 64>
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = W / 2; off >= 1; off >>= 1) {
    uint32_t o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

// Max over the TPR threads owning one row.  TPR == 32 / 64: lanes of a
// half wave / the wave.  TPR == 256: one row per block, cross-wave through
// LDS.
template <int TPR>
__device__ __forceinline__ uint32_t row_max(uint32_t v, uint32_t* red) {
  if constexpr (TPR <= 64) {
    return wave_max_u32<TPR>(v);
  } else {
    v = wave_max_u32(v);
    const int wave = threadIdx.x >> 6, base = (threadIdx.x / TPR) * (TPR / 64);  // the row's first wave
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    uint32_t m = red[base];
#pragma unroll
    for (int w = 1; w < TPR / 64; ++w) m = red[base + w] > m ? red[base + w] : m;
    return m;
  }
}

__device__ __forceinline__ uint32_t absmax8(const U16x8& v, uint32_t m) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = v.w[j] & 0x7FFFu, hi = (v.w[j] >> 16) & 0x7FFFu;
    m = lo > m ? lo : m;
    m = hi > m ? hi : m;
  }
  return m;
}




// ------------------------------------------------------------ quantizer
template <int TPR, int VPT>
__global__ __launch_bounds__(kBlock) void quant_rows_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ s) {
  __shared__ uint32_t red[kBlock / 64];
  constexpr int kRowsPerBlock = kBlock / TPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / TPR;
  const int t = threadIdx.x % TPR;
  const bool live = row < M;  // uniform per TPR lanes; every lane reaches row_max
  const int64_t nvec = K >> 3;
  const U16x8* xr = reinterpret_cast<const U16x8*>(x + (live ? row : 0) * ldx);

  U16x8 v[VPT];
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t idx = t + static_cast<int64_t>(i) * TPR;
    if (live && idx < nvec) {
      v[i] = ld_row16(xr + idx);
      m = absmax8(v[i], m);
    }
  }
  m = row_max<TPR>(m, red);
  if (!live) return;
  const RowScale rs = row_scale(bf16_to_f32(static_cast<uint16_t>(m)));
  uint2* qr = reinterpret_cast<uint2*>(q + row * ldq);
  if (rs.fast) {  // row-uniform: one branch per row, not a select per element
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t idx = t + static_cast<int64_t>(i) * TPR;
      if (idx < nvec) st_row8(qr + idx, quant8<true>(v[i], rs));
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t idx = t + static_cast<int64_t>(i) * TPR;
      if (idx < nvec) st_row8(qr + idx, quant8<false>(v[i], rs));
    }
  }
  if (t == 0) s[row] = rs.s;
}

// Any K (no alignment beyond 2 bytes): one row per block, two passes.
__global__ __launch_bounds__(kBlock) void quant_rows_generic_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ s) {
  __shared__ uint32_t red[kBlock / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  uint32_t m = 0;
  for (int64_t k = threadIdx.x; k < K; k += kBlock) {
    uint32_t a = xr[k] & 0x7FFFu;
    m = a > m ? a : m;
  }
  m = row_max<kBlock>(m, red);
  const RowScale rs = row_scale(bf16_to_f32(static_cast<uint16_t>(m)));
  for (int64_t k = threadIdx.x; k < K; k += kBlock)
    q[row * ldq + k] = static_cast<int8_t>(static_cast<int>(quant_div_rne(bf16_to_f32(xr[k]), rs)));
  if (threadIdx.x == 0) s[row] = rs.s;
}

// --------------------------------------------------- activation + requant
// silu(g) = g * 1 / (1 + e^-g) with the hardware reciprocal (1 ulp) in place
// of an IEEE division: the activation is rounded to bf16 next and is held
// to a tolerance, while the requant that follows is exact on its bf16 value.

template <int TPR, int VPT, int ACT>
__global__ __launch_bounds__(kBlock) void act_rows_kernel(
    const uint16_t* __restrict__ x, int64_t R, int64_t d,
    int8_t* __restrict__ q, float* __restrict__ s, uint16_t* __restrict__ a_out) {
  __shared__ uint32_t red[kBlock / 64];
  constexpr int kRowsPerBlock = kBlock / TPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / TPR;
  const int t = threadIdx.x % TPR;
  const bool live = row < R;
  const int64_t nvec = d >> 3;
  const U16x8* gr = reinterpret_cast<const U16x8*>(x + (live ? row : 0) * 2 * d);
  const U16x8* ur = gr + nvec;

  U16x8 v[VPT];
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t idx = t + static_cast<int64_t>(i) * TPR;
    if (live && idx < nvec) {
      const U16x8 g = ld_row16(gr + idx);
      const U16x8 u = ld_row16(ur + idx);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a0 = act_fn<ACT>(bf16_to_f32(static_cast<uint16_t>(g.get(2 * j)))) *
                         bf16_to_f32(static_cast<uint16_t>(u.get(2 * j)));
        const float a1 = act_fn<ACT>(bf16_to_f32(static_cast<uint16_t>(g.get(2 * j + 1)))) *
                         bf16_to_f32(static_cast<uint16_t>(u.get(2 * j + 1)));
        v[i].w[j] = static_cast<uint32_t>(f32_to_bf16(a0)) |
                    (static_cast<uint32_t>(f32_to_bf16(a1)) << 16);
      }
      m = absmax8(v[i], m);
    }
  }
  m = row_max<TPR>(m, red);
  if (!live) return;
  U16x8* ar = a_out ? reinterpret_cast<U16x8*>(a_out + row * d) : nullptr;
  if (q == nullptr) {  // activation only (launch-uniform): no requant
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t idx = t + static_cast<int64_t>(i) * TPR;
      if (idx < nvec) st_row16(ar + idx, v[i]);
    }
    return;
  }
  const RowScale rs = row_scale(bf16_to_f32(static_cast<uint16_t>(m)));
  uint2* qr = reinterpret_cast<uint2*>(q + row * d);
  if (rs.fast) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t idx = t + static_cast<int64_t>(i) * TPR;
      if (idx < nvec) st_row8(qr + idx, quant8<true>(v[i], rs));
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t idx = t + static_cast<int64_t>(i) * TPR;
      if (idx < nvec) st_row8(qr + idx, quant8<false>(v[i], rs));
    }
  }
  if (ar) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t idx = t + static_cast<int64_t>(i) * TPR;
      if (idx < nvec) st_row16(ar + idx, v[i]);
    }
  }
  if (t == 0) s[row] = rs.s;
}

// ------------------------------------------------- RMSNorm + requant
// h = x (or bf16(x + residual), written back to residual), then
//   ss = sum_k h_k^2 in fp64 (every square of a bf16 value is exact),
//   r  = 1 / sqrt(fp32(ss / H) + eps)         (IEEE fp32 sqrt and division)
//   y  = bf16((h * r) * w)                    (each product rounded)
// and y is quantized per row exactly like quant_rows_kernel.  y is written
// only if y_out is given.  Replaces flashinfer rmsnorm / fused_add_rmsnorm
// (python/minisgl/layers/norm.py:8-38) followed by the quantizer of the
// next W8A8 linear.
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int TPR>
__device__ __forceinline__ double row_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
  if constexpr (TPR == 64) {
    return v;
  } else {
    const int wave = threadIdx.x >> 6, base = (threadIdx.x / TPR) * (TPR / 64);  // the row's first wave
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    double t = red[base];
#pragma unroll
    for (int w = 1; w < TPR / 64; ++w) t += red[base + w];
    return t;
  }
}

// Rows of x and y_out are addressed as [G, inner, H] with outer strides ldx
// / ldy (elements) and the inner rows contiguous at stride H: row r lives at
// (r / inner) * ld + (r % inner) * H.  inner = 1, ld = H is a plain [M, H]
// matrix; a per-head view q.view(M, heads, D) of a row of qkv is inner =
// heads, ld = qkv width.  residual, q and s are plain [M, H] / [M].
template <int TPR, int VPT, bool RES, bool QUANT>
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_kernel(
    const uint16_t* x, uint16_t* __restrict__ res, const uint16_t* __restrict__ w,
    float eps, int64_t M, int64_t H, int8_t* __restrict__ q, float* __restrict__ s,
    uint16_t* y_out, int64_t inner, int64_t ldx, int64_t ldy) {
  __shared__ double dred[kBlock / 64];
  __shared__ uint32_t red[kBlock / 64];
  constexpr int kRowsPerBlock = kBlock / TPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / TPR;
  const int t = threadIdx.x % TPR;
  const bool live = row < M;  // uniform per wave (TPR >= 64)
  const int64_t nvec = H >> 3;
  const int64_t lrow = live ? row : 0;
  const int64_t grp = inner == 1 ? lrow : lrow / inner, sub = lrow - grp * inner;
  const U16x8* xr = reinterpret_cast<const U16x8*>(x + grp * ldx + sub * H);
  U16x8* rr = RES ? reinterpret_cast<U16x8*>(res + (live ? row : 0) * H) : nullptr;
  const U16x8* wr = reinterpret_cast<const U16x8*>(w);

  U16x8 v[VPT];
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t idx = t + static_cast<int64_t>(i) * TPR;
    if (live && idx < nvec) {
      v[i] = ld_row16(xr + idx);
      if constexpr (RES) {
        const U16x8 r0 = ld_row16(rr + idx);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a0 = bf16_lo(v[i].w[j]) + bf16_lo(r0.w[j]);
          const float a1 = bf16_hi(v[i].w[j]) + bf16_hi(r0.w[j]);
          v[i].w[j] = static_cast<uint32_t>(f32_to_bf16(a0)) | (static_cast<uint32_t>(f32_to_bf16(a1)) << 16);
        }
        st_row16(rr + idx, v[i]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double lo = static_cast<double>(bf16_lo(v[i].w[j]));
        const double hi = static_cast<double>(bf16_hi(v[i].w[j]));
        ss = __builtin_fma(lo, lo, ss);
        ss = __builtin_fma(hi, hi, ss);
      }
    }
  }
  ss = row_sum_f64<TPR>(ss, dred);
  const float ms = static_cast<float>(ss / static_cast<double>(H));
  const float r = 1.0f / __builtin_sqrtf(ms + eps);
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t idx = t + static_cast<int64_t>(i) * TPR;
    if (live && idx < nvec) {
      const U16x8 wv = wr[idx];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float y0 = (bf16_lo(v[i].w[j]) * r) * bf16_lo(wv.w[j]);
        const float y1 = (bf16_hi(v[i].w[j]) * r) * bf16_hi(wv.w[j]);
        v[i].w[j] = static_cast<uint32_t>(f32_to_bf16(y0)) | (static_cast<uint32_t>(f32_to_bf16(y1)) << 16);
      }
      if constexpr (QUANT) m = absmax8(v[i], m);
    }
  }
  if constexpr (QUANT) m = row_max<TPR>(m, red);
  if (!live) return;
  if constexpr (QUANT) {
    const RowScale rs = row_scale(bf16_to_f32(static_cast<uint16_t>(m)));
    uint2* qr = reinterpret_cast<uint2*>(q + row * H);
    if (rs.fast) {
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const int64_t idx = t + static_cast<int64_t>(i) * TPR;
        if (idx < nvec) st_row8(qr + idx, quant8<true>(v[i], rs));
      }
    } else {
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const int64_t idx = t + static_cast<int64_t>(i) * TPR;
        if (idx < nvec) st_row8(qr + idx, quant8<false>(v[i], rs));
      }
    }
    if (t == 0) s[row] = rs.s;
  }
  if (y_out) {
    U16x8* yr = reinterpret_cast<U16x8*>(y_out + grp * ldy + sub * H);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int64_t idx = t + static_cast<int64_t>(i) * TPR;
      if (idx < nvec) st_row16(yr + idx, v[i]);
    }
  }
}

// Pick (TPR, VPT) for a row of nvec 16-byte vectors; false if none fits.
template <template <int, int> class Launch, typename... Args>
bool dispatch_rows(int64_t nvec, int64_t rows, hipStream_t st, Args... args) {
  auto go = [&](auto tpr_c, auto vpt_c) {
    constexpr int TPR = decltype(tpr_c)::value;
    constexpr int VPT = decltype(vpt_c)::value;
    const int64_t blocks = (rows + (kBlock / TPR) - 1) / (kBlock / TPR);
    Launch<TPR, VPT>::run(dim3(static_cast<unsigned>(blocks)), st, args...);
    return true;
  };
  using I32 = std::integral_constant<int, 32>;
  using I64 = std::integral_constant<int, 64>;
  using I256 = std::integral_constant<int, 256>;
  // two rows per wave where that keeps more lanes busy than one (short
  // rows: the MoE activation at I = 768 is 96 vectors, 75% of 64 x 2)
  if constexpr (Launch<32, 1>::kHalfWaveRows) {
    if (nvec <= 32) return go(I32{}, std::integral_constant<int, 1>{});
    if (nvec > 64 && nvec <= 96) return go(I32{}, std::integral_constant<int, 3>{});
  }
  // few lanes idle on the last vector (K = 5120: 640 of 768 slots, K =
  // 17408: 2176 of 2304).  Rows past 512 vectors use 256-thread rows: one
  // wave per 5120-wide row measured slower for the fused RMSNorm.
  if (nvec <= 64 * 1) return go(I64{}, std::integral_constant<int, 1>{});
  if (nvec <= 64 * 2) return go(I64{}, std::integral_constant<int, 2>{});
  if (nvec <= 64 * 3) return go(I64{}, std::integral_constant<int, 3>{});
  if (nvec <= 64 * 4) return go(I64{}, std::integral_constant<int, 4>{});
  if (nvec <= 64 * 6) return go(I64{}, std::integral_constant<int, 6>{});
  if (nvec <= 64 * 8) return go(I64{}, std::integral_constant<int, 8>{});
  if (nvec <= 256 * 3) return go(I256{}, std::integral_constant<int, 3>{});
  if (nvec <= 256 * 4) return go(I256{}, std::integral_constant<int, 4>{});
  if (nvec <= 256 * 6) return go(I256{}, std::integral_constant<int, 6>{});
  if (nvec <= 256 * 8) return go(I256{}, std::integral_constant<int, 8>{});
  if (nvec <= 256 * 9) return go(I256{}, std::integral_constant<int, 9>{});
  if (nvec <= 256 * 12) return go(I256{}, std::integral_constant<int, 12>{});
  if (nvec <= 256 * 16) return go(I256{}, std::integral_constant<int, 16>{});
  return false;
}

template <int TPR, int VPT>
struct QuantLaunch {
  static constexpr bool kHalfWaveRows = true;
  static void run(dim3 grid, hipStream_t st, const uint16_t* x, int64_t ldx, int64_t M,
                  int64_t K, int8_t* q, int64_t ldq, float* s) {
    hipLaunchKernelGGL((quant_rows_kernel<TPR, VPT>), grid, dim3(kBlock), 0, st, x, ldx, M, K,
                       q, ldq, s);
  }
};

template <int TPR, int VPT>
struct ActLaunch {
  static constexpr bool kHalfWaveRows = true;
  static void run(dim3 grid, hipStream_t st, const uint16_t* x, int64_t R, int64_t d, int act,
                  int8_t* q, float* s, uint16_t* a_out) {
    if (act == 0)
      hipLaunchKernelGGL((act_rows_kernel<TPR, VPT, 0>), grid, dim3(kBlock), 0, st, x, R, d, q, s,
                         a_out);
    else
      hipLaunchKernelGGL((act_rows_kernel<TPR, VPT, 1>), grid, dim3(kBlock), 0, st, x, R, d, q, s,
                         a_out);
  }
};

template <int TPR, int VPT>
struct NormLaunch {
  static constexpr bool kHalfWaveRows = false;
  static void run(dim3 grid, hipStream_t st, const uint16_t* x, uint16_t* res, const uint16_t* w,
                  float eps, int64_t M, int64_t H, int8_t* q, float* s, uint16_t* y, int64_t inner,
                  int64_t ldx, int64_t ldy) {
    if (res && q)
      hipLaunchKernelGGL((rmsnorm_rows_kernel<TPR, VPT, true, true>), grid, dim3(kBlock), 0, st, x, res,
                         w, eps, M, H, q, s, y, inner, ldx, ldy);
    else if (res)
      hipLaunchKernelGGL((rmsnorm_rows_kernel<TPR, VPT, true, false>), grid, dim3(kBlock), 0, st, x, res,
                         w, eps, M, H, q, s, y, inner, ldx, ldy);
    else if (q)
      hipLaunchKernelGGL((rmsnorm_rows_kernel<TPR, VPT, false, true>), grid, dim3(kBlock), 0, st, x, res,
                         w, eps, M, H, q, s, y, inner, ldx, ldy);
    else
      hipLaunchKernelGGL((rmsnorm_rows_kernel<TPR, VPT, false, false>), grid, dim3(kBlock), 0, st, x, res,
                         w, eps, M, H, q, s, y, inner, ldx, ldy);
  }
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

}  // namespace

int quant_per_token_bf16(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq,
                         float* s, hipStream_t st) {
  MW8_REQUIRE(x && q && s, kErrArg, "quant_per_token: null pointer");
  MW8_REQUIRE(M >= 0 && K > 0 && ldx >= K && ldq >= K, kErrShape,
              "quant_per_token: bad sizes M=%lld K=%lld ldx=%lld ldq=%lld", (long long)M,
              (long long)K, (long long)ldx, (long long)ldq);
  if (M == 0) return kOk;
  MW8_REQUIRE(M < (1ll << 31), kErrShape, "quant_per_token: M too large");
  const auto* xb = static_cast<const uint16_t*>(x);
  const bool vec_ok = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && aligned16(x) &&
                      aligned8(q);
  if (!(vec_ok && dispatch_rows<QuantLaunch>(K / 8, M, st, xb, ldx, M, K, q, ldq, s))) {
    hipLaunchKernelGGL(quant_rows_generic_kernel, dim3(static_cast<unsigned>(M)), dim3(kBlock), 0,
                       st, xb, ldx, M, K, q, ldq, s);
  }
  return check_launch("quant_per_token");
}

int act_and_mul_quant_bf16(const void* x, int64_t R, int64_t two_d, int act, int8_t* q, float* s,
                           void* a_out, hipStream_t st) {
  MW8_REQUIRE(x && ((q && s) || (!q && !s && a_out)), kErrArg,
              "act_and_mul_quant: null pointer (q and s both given, or both NULL with act_out)");
  MW8_REQUIRE(act == 0 || act == 1, kErrArg, "act_and_mul_quant: act must be 0 (silu) or 1 (gelu)");
  MW8_REQUIRE(R >= 0 && two_d > 0 && two_d % 16 == 0, kErrShape,
              "act_and_mul_quant: need 2d %% 16 == 0, got %lld", (long long)two_d);
  if (R == 0) return kOk;
  MW8_REQUIRE(R < (1ll << 31), kErrShape, "act_and_mul_quant: too many rows");
  MW8_REQUIRE(aligned16(x) && aligned8(q) && (!a_out || aligned16(a_out)), kErrAlign,
              "act_and_mul_quant: x/act_out need 16-byte and q 8-byte alignment");
  const int64_t d = two_d / 2;
  const bool ok = dispatch_rows<ActLaunch>(d / 8, R, st, static_cast<const uint16_t*>(x), R, d, act,
                                           q, s, static_cast<uint16_t*>(a_out));
  MW8_REQUIRE(ok, kErrShape, "act_and_mul_quant: d=%lld exceeds the register-resident limit 32768",
              (long long)d);
  return check_launch("act_and_mul_quant");
}

int rmsnorm_quant_bf16(const void* x, void* residual, const void* weight, float eps, int64_t M,
                       int64_t H, int8_t* q, float* s, void* y, hipStream_t st) {
  MW8_REQUIRE(x && weight, kErrArg, "rmsnorm_quant: null pointer");
  MW8_REQUIRE((q == nullptr) == (s == nullptr) && (q || y), kErrArg,
              "rmsnorm_quant: q and s both given or both NULL, and q or y given");
  MW8_REQUIRE(M >= 0 && H > 0 && H % 8 == 0, kErrShape, "rmsnorm_quant: need H %% 8 == 0 (H=%lld)",
              (long long)H);
  MW8_REQUIRE(eps >= 0.0f, kErrArg, "rmsnorm_quant: eps must be >= 0");
  if (M == 0) return kOk;
  MW8_REQUIRE(M < (1ll << 31), kErrShape, "rmsnorm_quant: too many rows");
  MW8_REQUIRE(aligned16(x) && aligned16(weight) && (!q || aligned8(q)) && (!residual || aligned16(residual)) &&
                  (!y || aligned16(y)),
              kErrAlign, "rmsnorm_quant: x/residual/weight/y need 16-byte and q 8-byte alignment");
  const bool ok = dispatch_rows<NormLaunch>(H / 8, M, st, static_cast<const uint16_t*>(x),
                                            static_cast<uint16_t*>(residual),
                                            static_cast<const uint16_t*>(weight), eps, M, H, q, s,
                                            static_cast<uint16_t*>(y), int64_t{1}, H, H);
  MW8_REQUIRE(ok, kErrShape, "rmsnorm_quant: H=%lld exceeds the register-resident limit 32768",
              (long long)H);
  return check_launch("rmsnorm_quant");
}

int rmsnorm_strided_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, const void* weight, float eps,
                         int64_t G, int64_t inner, int64_t H, hipStream_t st) {
  MW8_REQUIRE(x && y && weight, kErrArg, "rmsnorm_strided: null pointer");
  MW8_REQUIRE(G >= 0 && inner > 0 && H > 0 && H % 8 == 0, kErrShape,
              "rmsnorm_strided: need H %% 8 == 0 and inner > 0 (G=%lld inner=%lld H=%lld)", (long long)G,
              (long long)inner, (long long)H);
  MW8_REQUIRE(ldx >= inner * H && ldy >= inner * H && ldx % 8 == 0 && ldy % 8 == 0, kErrShape,
              "rmsnorm_strided: strides ldx=%lld ldy=%lld must be multiples of 8 and >= inner * H = %lld",
              (long long)ldx, (long long)ldy, (long long)(inner * H));
  MW8_REQUIRE(eps >= 0.0f, kErrArg, "rmsnorm_strided: eps must be >= 0");
  if (G == 0) return kOk;
  const int64_t M = G * inner;
  MW8_REQUIRE(M < (1ll << 31) && M / inner == G, kErrShape, "rmsnorm_strided: too many rows");
  MW8_REQUIRE(aligned16(x) && aligned16(y) && aligned16(weight), kErrAlign,
              "rmsnorm_strided: x, y and weight need 16-byte alignment");
  const bool ok = dispatch_rows<NormLaunch>(H / 8, M, st, static_cast<const uint16_t*>(x),
                                            static_cast<uint16_t*>(nullptr),
                                            static_cast<const uint16_t*>(weight), eps, M, H,
                                            static_cast<int8_t*>(nullptr), static_cast<float*>(nullptr),
                                            static_cast<uint16_t*>(y), inner, ldx, ldy);
  MW8_REQUIRE(ok, kErrShape, "rmsnorm_strided: H=%lld exceeds the register-resident limit 32768",
              (long long)H);
  return check_launch("rmsnorm_strided");
}

}  // namespace mw8
