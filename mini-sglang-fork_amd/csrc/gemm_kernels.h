// int8 x int8 -> int32 MFMA GEMM cores shared by the dense linear and the
// grouped (fused-MoE) GEMM.  gfx950 only.
//
// Layouts (row-major, K contiguous; "NT" like the reference's F.linear
// weight [N, K], python/minisgl/layers/linear.py:28):
//   A  int8 [rows, K]   activations (rows gathered through a RowMap)
//   W  int8 [N, K]      weights (per expert: base + e * N * K)
//   out[row, n]         bf16 (scaled epilogue) or int32 (raw accumulators)
//
// Two cores:
//   tile_core   -- large M (prefill): BM x BN x 128 block tile, 4 waves, each
//                  wave a (BM/WM) x (BN/WN) tile of v_mfma_i32_32x32x32_i8,
//                  A/W tiles double-buffered in LDS with an XOR swizzle of
//                  16-byte chunks (chunk ^ (row & 7)) so that the 32 rows
//                  read by one MFMA fragment load hit distinct banks.
//   stream_core -- small M (decode): weight streaming with
//                  v_mfma_i32_16x16x64_i8, weight rows as the MFMA "A"
//                  operand (read straight from HBM into registers, 64
//                  contiguous bytes per lane per 256-K step) and up to 64
//                  tokens as the "B" operand staged once per block in LDS.
//
// MFMA lane layouts (checked on gfx950 by an in-bounds probe):
//   32x32x32: lane l feeds A row l%32 / B col l%32 with 16 K-bytes of group
//             l/32; D reg v holds row 8*(v/4) + 4*(l/32) + v%4, col l%32.
//   16x16x64: lane l feeds A row l%16 / B col l%16 with 16 K-bytes of group
//             l/16; D reg v holds row 4*(l/16) + v, col l%16.
// Which K byte a (group, byte) pair stands for does not matter as long as A
// and B use the same mapping, which both cores do by construction.
#pragma once

#include "mw8_common.h"

namespace mw8 {

enum EpiKind : int { kEpiBf16 = 0, kEpiI32 = 1 };

// Everything a core needs to know about rows, experts and the epilogue.
struct GemmArgs {
  const int8_t* A;
  const float* sa;       // [rows of A]
  const int8_t* W;       // [E][N][K] (E = 1 for dense)
  const float* sw;       // [E][N]
  const uint16_t* bias;  // [N] bf16 or null (dense only)
  void* out;             // bf16 or int32 [out rows][ldo]
  int64_t M;             // dense: rows of A/out
  int64_t N, K;
  int64_t lda, ldo;
  // grouped GEMM only
  const int32_t* sorted_ids;   // [max_sorted]
  const int32_t* expert_ids;   // [max_sorted / BM]
  const int32_t* num_post_pad; // [1]
  const float* topk_w;         // routed weights [num_valid] or null
  int64_t num_valid;           // M * top_k
  int32_t top_k;
  int32_t num_experts;         // blocks owned by an id outside [0, E) are skipped
  // split-K (stream core, dense only)
  int32_t* partials;  // [splits][M][N]
  int32_t* counters;  // [n_tiles], zero between calls
  int32_t splits;
  int32_t kc;         // K per split (multiple of 256)
};

__device__ __forceinline__ uint16_t epi_bf16(int32_t acc, float sa, float sw, const uint16_t* bias,
                                             int64_t n, float routed, bool has_routed) {
  float t = epi_scale(acc, sa, sw);
  if (bias) t = t + bf16_to_f32(bias[n]);
  if (has_routed) t = t * routed;
  return f32_to_bf16(t);
}

// ------------------------------------------------------------------------
// Row maps: dense rows vs. expert-sorted rows (grouped GEMM).
// ------------------------------------------------------------------------
struct DenseRows {
  static constexpr bool kGrouped = false;
};
struct SortedRows {
  static constexpr bool kGrouped = true;
};

// ------------------------------------------------------------------------
// Large-M tile core
// ------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN>
struct TileShape {
  static constexpr int kBK = 128;                    // K bytes per stage
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
  static constexpr int kFM = kWaveM / 32, kFN = kWaveN / 32;
  static constexpr int kAChunks = BM * kBK / 16 / 256;  // 16-byte chunks per thread
  static constexpr int kBChunks = BN * kBK / 16 / 256;
  static constexpr int kLdsA = BM * kBK, kLdsB = BN * kBK;
  static constexpr int kLds = 2 * (kLdsA + kLdsB);
  static_assert(WM * WN == 4, "4 waves per block");
  static_assert(kFM >= 1 && kFN >= 1, "wave tile must hold one 32x32 MFMA");
  static_assert(kAChunks >= 1 && kBChunks >= 1, "tile too small");
};

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7)) << 4);
}

template <int BM, int BN, int WM, int WN, int EPI, class Rows>
__global__ __launch_bounds__(256) void tile_gemm_kernel(GemmArgs g) {
  using S = TileShape<BM, BN, WM, WN>;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- which tile: x = N tiles (fastest), y = M tiles / expert blocks
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;
  const int64_t mblk = blockIdx.y;
  const int8_t* W = g.W;
  const float* sw = g.sw;
  int64_t m0 = mblk * BM;
  if constexpr (Rows::kGrouped) {
    if (m0 >= static_cast<int64_t>(*g.num_post_pad)) return;
    const int e = g.expert_ids[mblk];
    if (e < 0 || e >= g.num_experts) return;
    W += static_cast<int64_t>(e) * g.N * g.K;
    sw += static_cast<int64_t>(e) * g.N;
  }

  // ---- per-thread global source rows for the A and W chunks it loads.
  // Chunk id = tid + 256 * i -> row id / 8, 16-byte column id % 8 (= tid % 8).
  const int cc = tid & 7;
  const int8_t* a_src[S::kAChunks];
  const int8_t* w_src[S::kBChunks];
  int a_lds[S::kAChunks], w_lds[S::kBChunks];
#pragma unroll
  for (int i = 0; i < S::kAChunks; ++i) {
    const int r = (tid + 256 * i) >> 3;
    int64_t arow;
    if constexpr (Rows::kGrouped) {
      const int32_t p = g.sorted_ids[m0 + r];
      arow = p < g.num_valid ? p / g.top_k : 0;
    } else {
      arow = m0 + r < g.M ? m0 + r : g.M - 1;
    }
    a_src[i] = g.A + arow * g.lda + 16 * cc;
    a_lds[i] = swz(r, cc);
  }
#pragma unroll
  for (int i = 0; i < S::kBChunks; ++i) {
    const int r = (tid + 256 * i) >> 3;
    const int64_t wrow = n0 + r < g.N ? n0 + r : g.N - 1;
    w_src[i] = W + wrow * g.K + 16 * cc;
    w_lds[i] = swz(r, cc);
  }

  v16i acc[S::kFM][S::kFN];
#pragma unroll
  for (int i = 0; i < S::kFM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFN; ++j) acc[i][j] = v16i{0};

  const int nk = static_cast<int>((g.K + S::kBK - 1) / S::kBK);
  v4i ra[S::kAChunks], rb[S::kBChunks];

  auto gload = [&](int kt) {
    const int64_t k0 = static_cast<int64_t>(kt) * S::kBK;
    const bool in = k0 + 16 * cc < g.K;  // K % 16 == 0: chunks are all-in or all-out
#pragma unroll
    for (int i = 0; i < S::kAChunks; ++i)
      ra[i] = in ? *reinterpret_cast<const v4i*>(a_src[i] + k0) : v4i{0};
#pragma unroll
    for (int i = 0; i < S::kBChunks; ++i)
      rb[i] = in ? *reinterpret_cast<const v4i*>(w_src[i] + k0) : v4i{0};
  };
  auto lstore = [&](int buf) {
    unsigned char* la = lds + buf * (S::kLdsA + S::kLdsB);
    unsigned char* lb = la + S::kLdsA;
#pragma unroll
    for (int i = 0; i < S::kAChunks; ++i) *reinterpret_cast<v4i*>(la + a_lds[i]) = ra[i];
#pragma unroll
    for (int i = 0; i < S::kBChunks; ++i) *reinterpret_cast<v4i*>(lb + w_lds[i]) = rb[i];
  };

  gload(0);
  lstore(0);
  __syncthreads();
  const int frow = lane & 31, fgrp = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const unsigned char* la = lds + buf * (S::kLdsA + S::kLdsB);
    const unsigned char* lb = la + S::kLdsA;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int ch = 2 * ks + fgrp;
      v4i fa[S::kFM], fb[S::kFN];
#pragma unroll
      for (int i = 0; i < S::kFM; ++i)
        fa[i] = *reinterpret_cast<const v4i*>(la + swz(wm * S::kWaveM + 32 * i + frow, ch));
#pragma unroll
      for (int j = 0; j < S::kFN; ++j)
        fb[j] = *reinterpret_cast<const v4i*>(lb + swz(wn * S::kWaveN + 32 * j + frow, ch));
#pragma unroll
      for (int i = 0; i < S::kFM; ++i)
#pragma unroll
        for (int j = 0; j < S::kFN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds column (lane & 31) of each 32x32 block
#pragma unroll
  for (int i = 0; i < S::kFM; ++i) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int r = wm * S::kWaveM + 32 * i + 8 * (v >> 2) + 4 * fgrp + (v & 3);
      int64_t orow, arow;
      bool rvalid;
      float routed = 1.0f;
      if constexpr (Rows::kGrouped) {
        const int32_t p = g.sorted_ids[m0 + r];
        rvalid = p < g.num_valid;
        orow = p;
        arow = rvalid ? p / g.top_k : 0;
        if (rvalid && g.topk_w) routed = g.topk_w[p];
      } else {
        orow = m0 + r;
        arow = orow;
        rvalid = orow < g.M;
      }
      if (!rvalid) continue;
      const float sa = EPI == kEpiBf16 ? g.sa[arow] : 0.0f;
#pragma unroll
      for (int j = 0; j < S::kFN; ++j) {
        const int64_t n = n0 + wn * S::kWaveN + 32 * j + frow;
        if (n >= g.N) continue;
        const int32_t a = acc[i][j][v];
        if constexpr (EPI == kEpiBf16) {
          static_cast<uint16_t*>(g.out)[orow * g.ldo + n] =
              epi_bf16(a, sa, sw[n], g.bias, n, routed, g.topk_w != nullptr);
        } else {
          static_cast<int32_t*>(g.out)[orow * g.ldo + n] = a;
        }
      }
    }
  }
}

// ------------------------------------------------------------------------
// Small-M weight-streaming core (dense decode and grouped small blocks)
// ------------------------------------------------------------------------
// Block = 4 waves = 64 weight rows; wave w owns rows n0 + 16w .. +16.
// MT groups of 16 tokens (MT <= 4) share every weight fragment.
// Dense: grid (N/64, splits); the K range [split*kc, +kc) is reduced across
// splits through int32 partials and a per-N-tile arrival counter; the last
// block to arrive applies the epilogue and re-arms the counter.
// Grouped: grid (N/64, expert blocks of 16 sorted rows); no split.
constexpr int kStreamRows = 64;
constexpr int kStreamStep = 256;  // K bytes per lane step (4 MFMAs)

template <int MT>
__host__ __device__ constexpr int stream_kc_max() {
  // keep the LDS token panel at or below 40 KB (4 blocks per CU)
  return (((40960 / (16 * MT)) - 16) / kStreamStep) * kStreamStep;
}

template <int MT, int EPI, class Rows>
__global__ __launch_bounds__(256) void stream_gemm_kernel(GemmArgs g) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kStreamRows;
  const int8_t* W = g.W;
  const float* sw = g.sw;
  int64_t k_begin = 0, k_end = g.K;
  int64_t m0 = 0;
  if constexpr (Rows::kGrouped) {
    m0 = static_cast<int64_t>(blockIdx.y) * 16;
    if (m0 >= static_cast<int64_t>(*g.num_post_pad)) return;
    const int e = g.expert_ids[blockIdx.y];
    if (e < 0 || e >= g.num_experts) return;
    W += static_cast<int64_t>(e) * g.N * g.K;
    sw += static_cast<int64_t>(e) * g.N;
  } else {
    k_begin = static_cast<int64_t>(blockIdx.y) * g.kc;
    k_end = k_begin + g.kc < g.K ? k_begin + g.kc : g.K;
  }
  const int kc = static_cast<int>(k_end - k_begin);
  const int kc_pad = ((kc + kStreamStep - 1) / kStreamStep) * kStreamStep;
  const int ldl = kc_pad + 16;  // padded LDS row: 16 token rows hit 16 bank groups

  // ---- stage the token panel [16*MT][kc] in LDS (zeros outside)
  {
    const int chunks_per_row = kc_pad / 16;
    for (int id = tid; id < 16 * MT * chunks_per_row; id += 256) {
      const int r = id / chunks_per_row, c = id % chunks_per_row;
      int64_t arow = -1;
      if constexpr (Rows::kGrouped) {
        const int32_t p = g.sorted_ids[m0 + r];
        if (p < g.num_valid) arow = p / g.top_k;
      } else {
        if (r < g.M) arow = r;
      }
      v4i v = v4i{0};
      if (arow >= 0 && 16 * c < kc) v = *reinterpret_cast<const v4i*>(g.A + arow * g.lda + k_begin + 16 * c);
      *reinterpret_cast<v4i*>(lds + r * ldl + 16 * c) = v;
    }
  }
  __syncthreads();

  // ---- stream the weights
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t wrow = n0 + 16 * wave + r16;
  const int8_t* wp = W + (wrow < g.N ? wrow : g.N - 1) * g.K + k_begin + 64 * grp;
  v4i acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = v4i{0};

  const int steps = kc_pad / kStreamStep;
  int s = 0;
  for (; s + 2 <= steps; s += 2) {
    v4i w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int kk = (j >> 2) * kStreamStep + 16 * (j & 3);
      const int koff = s * kStreamStep + kk;
      w[j] = (koff + 64 * grp < kc) ? *reinterpret_cast<const v4i*>(wp + koff) : v4i{0};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int kk = (s + (j >> 2)) * kStreamStep + 64 * grp + 16 * (j & 3);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const v4i b = *reinterpret_cast<const v4i*>(lds + (16 * t + r16) * ldl + kk);
        acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j], b, acc[t], 0, 0, 0);
      }
    }
  }
  for (; s < steps; ++s) {
    v4i w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int koff = s * kStreamStep + 16 * j;
      w[j] = (koff + 64 * grp < kc) ? *reinterpret_cast<const v4i*>(wp + koff) : v4i{0};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = s * kStreamStep + 64 * grp + 16 * j;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const v4i b = *reinterpret_cast<const v4i*>(lds + (16 * t + r16) * ldl + kk);
        acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j], b, acc[t], 0, 0, 0);
      }
    }
  }

  // D reg v of lane l: weight row n0 + 16*wave + 4*(l/16) + v, token 16*t + l%16
  const int64_t nb = n0 + 16 * wave + 4 * grp;
  if constexpr (Rows::kGrouped) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int32_t p = g.sorted_ids[m0 + 16 * t + r16];
      if (p >= g.num_valid) continue;
      const int64_t arow = p / g.top_k;
      const float sa = EPI == kEpiBf16 ? g.sa[arow] : 0.0f;
      const float routed = g.topk_w ? g.topk_w[p] : 1.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t n = nb + v;
        if (n >= g.N) continue;
        if constexpr (EPI == kEpiBf16)
          static_cast<uint16_t*>(g.out)[p * g.ldo + n] =
              epi_bf16(acc[t][v], sa, sw[n], nullptr, n, routed, g.topk_w != nullptr);
        else
          static_cast<int32_t*>(g.out)[p * g.ldo + n] = acc[t][v];
      }
    }
    return;
  } else {
    if (g.splits == 1) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int64_t m = 16 * t + r16;
        if (m >= g.M) continue;
        const float sa = EPI == kEpiBf16 ? g.sa[m] : 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t n = nb + v;
          if (n >= g.N) continue;
          if constexpr (EPI == kEpiBf16)
            static_cast<uint16_t*>(g.out)[m * g.ldo + n] =
                epi_bf16(acc[t][v], sa, sw[n], g.bias, n, 1.0f, false);
          else
            static_cast<int32_t*>(g.out)[m * g.ldo + n] = acc[t][v];
        }
      }
      return;
    }
    // ---- split-K: publish partials, last arriving block reduces
    int32_t* part = g.partials + static_cast<int64_t>(blockIdx.y) * g.M * g.N;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int64_t m = 16 * t + r16;
      if (m >= g.M) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (nb + v < g.N) part[m * g.N + nb + v] = acc[t][v];
    }
    __threadfence();
    __syncthreads();
    __shared__ int last;
    if (tid == 0) {
      const int old = atomicAdd(g.counters + blockIdx.x, 1);
      last = (old == g.splits - 1);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    const int64_t ncols = g.N - n0 < kStreamRows ? g.N - n0 : kStreamRows;
    for (int64_t id = tid; id < g.M * kStreamRows; id += 256) {
      const int64_t m = id / kStreamRows, n = n0 + id % kStreamRows;
      if (id % kStreamRows >= ncols) continue;
      int32_t a = 0;
      for (int sp = 0; sp < g.splits; ++sp)
        a += g.partials[(static_cast<int64_t>(sp) * g.M + m) * g.N + n];
      if constexpr (EPI == kEpiBf16)
        static_cast<uint16_t*>(g.out)[m * g.ldo + n] = epi_bf16(a, g.sa[m], sw[n], g.bias, n, 1.0f, false);
      else
        static_cast<int32_t*>(g.out)[m * g.ldo + n] = a;
    }
    if (tid == 0) g.counters[blockIdx.x] = 0;
  }
}

}  // namespace mw8
