// Dense W8A8 GEMM for 33 ... ~1024 rows: K split inside the block over a
// CU-balanced grid.  gfx950 only.
//
// Between the decode cores (weight streaming, M <= 32) and the large-M ring
// (256 x 256 tiles) a Qwen3-14B shape has too few output tiles to give
// every CU work at full MFMA efficiency: at M = 512, N = 7168 there are 56
// 256 x 256 tiles.  Cutting K across blocks fills the CUs but every split
// writes and re-reads a whole int32 partial tile through HBM (sp x M x N x
// 4 bytes: 59 MB at sp = 4, more than the 37 MB weight stream).  Here the K
// split happens inside a block instead:
//
//  * block = KG x WM x WN waves; wave (g, wm, wn) owns output rows
//    wm * BM/WM + [0, BM/WM) and columns wn * BN/WN + [0, BN/WN) of the
//    block tile and the K slice g of every stage;
//  * a stage is SK = KG * KS * 32 bytes of K for BM rows of A and BN rows
//    of W, moved global -> LDS with buffer_load ... lds (1 KB per wave
//    instruction, 16-byte chunks XOR-swizzled by row so the fragment reads
//    are bank-conflict-free), NSTAGE stages in flight, one barrier each;
//  * after the last stage the KG partial tiles are summed with LDS integer
//    atomics (exact, order-free) and the epilogue runs once per element;
//  * the grid is G_m x G_n blocks: G_m = ceil(M / BM) row tiles and G_n
//    column ranges whose boundaries are multiples of 16 and whose count
//    makes the grid a multiple of the CU count, so every CU streams the same
//    number of weight rows (no partial last wave); weight rows past a
//    block's range and A rows past M read zeros through the buffer range
//    check (no memory traffic).
//
// No workspace, no second kernel, no inter-block communication.
#pragma once

#include "gemm_kernels.h"

namespace mw8 {

// Chunk swizzle of an LDS row of SK bytes: chunk c of row r sits at
// r * SK + ((c ^ ks_swz<SK>(r)) << 4).  The 16 rows read by one 256-byte
// phase of a fragment load land in 16 distinct 16-byte bank groups.
template <int SK>
__device__ __forceinline__ int ks_swz(int row) {
  if constexpr (SK == 64 || SK == 128) return swz_f<SK>(row);
  else return row & 15;  // SK >= 256: one LDS row covers all 64 banks
}

// Column boundary of range j of G over N columns: a multiple of 16 (N's
// last range takes the remainder).
__device__ __forceinline__ int64_t ks_col0(int64_t N, int64_t j, int64_t G) {
  return j >= G ? N : 16 * ((N / 16) * j / G);
}

template <int BM, int BN, int KG, int WM, int WN, int KS, int NSTAGE>
struct KsplitShape {
  static constexpr int kWaves = KG * WM * WN, kThreads = 64 * kWaves;
  static constexpr int kSK = KG * KS * 32;            // K bytes per stage
  static constexpr int kC = kSK / 16;                 // 16-byte chunks per LDS row
  static constexpr int kRowsPerInst = 1024 / kSK;     // rows one DMA instruction fills
  static constexpr int kStageA = BM * kSK, kStage = (BM + BN) * kSK;
  static constexpr int kInstA = BM / kRowsPerInst, kInstB = BN / kRowsPerInst;
  // DMA instructions per wave and stage for A and for W; the last waves'
  // surplus instructions (if the counts do not divide) load zeros into a
  // scratch kilobyte past the ring
  static constexpr int kLA = (kInstA + kWaves - 1) / kWaves, kLB = (kInstB + kWaves - 1) / kWaves;
  static constexpr int kL = kLA + kLB;
  static constexpr bool kPad = kLA * kWaves != kInstA || kLB * kWaves != kInstB;
  static constexpr int kRedLd = BN + 8;               // reduction row stride (ints): rows r, r+4 on disjoint banks
  static constexpr int kRing = NSTAGE * kStage + (kPad ? 1024 : 0);
  static constexpr int kRed = BM * kRedLd * 4;
  static constexpr int kLds = kRing > kRed ? kRing : kRed;
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN, kFM = kWaveM / 32, kFN = kWaveN / 32;
  static constexpr int kSets = KS == 1 ? 1 : 2;       // fragment register sets
  static_assert(kSK == 64 || kSK == 128 || kSK == 256 || kSK == 512, "stage of 64 - 512 K bytes");
  static_assert(KS == 1 || KS % 2 == 0, "one k-step per stage, or an even count");
  static_assert(kInstA * kRowsPerInst == BM && kInstB * kRowsPerInst == BN, "whole rows per DMA instruction");
  static_assert(kFM >= 1 && kFN >= 1 && kFM * 32 * WM == BM && kFN * 32 * WN == BN, "32 x 32 MFMA tiles");
  static_assert(NSTAGE >= 2 && (NSTAGE - 2) * kL < 64, "stages in flight fit the vmcnt counter");
  static_assert(kLds <= 163840, "LDS budget");
};

template <int BM, int BN, int KG, int WM, int WN, int KS, int NSTAGE, int EPI>
__global__ __launch_bounds__(64 * KG * WM * WN) void ksplit_gemm_kernel(GemmArgs g) {
#if defined(__HIP_DEVICE_COMPILE__)
  using S = KsplitShape<BM, BN, KG, WM, WN, KS, NSTAGE>;
  constexpr int SK = S::kSK, kC = S::kC, kWaves = S::kWaves, kL = S::kL;
  static_assert(kC <= 64 && 64 % kC == 0, "a DMA instruction covers whole LDS rows");
  constexpr int kFM = S::kFM, kFN = S::kFN;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave / (WM * WN), wsub = wave % (WM * WN), wm = wsub / WN, wn = wsub % WN;

  // ---- block -> (row tile, column range); each XCD gets a contiguous range
  // of block indices, row tiles fastest, so the blocks sharing a weight
  // range run on one XCD and read it from its L2
  const int64_t G = gridDim.x, gm = (g.M + BM - 1) / BM, gn = G / gm;
  const int64_t t = xcd_tile_index(blockIdx.x, G);
  const int64_t im = t % gm, jn = t / gm;
  const int64_t m0 = im * BM;
  const int64_t n0 = ks_col0(g.N, jn, gn), nr = ks_col0(g.N, jn + 1, gn) - n0;
  const int64_t mr = g.M - m0 < BM ? g.M - m0 : BM;
  if (nr <= 0) return;  // block-uniform (host keeps every range non-empty)

  // buffer views: A rows [m0, m0 + mr), W rows [n0, n0 + nr); rows past them read zeros
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      scalar_ptr(const_cast<int8_t*>(g.A + m0 * g.lda)), 0, static_cast<int>(mr * g.lda), kBufferFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      scalar_ptr(const_cast<int8_t*>(g.W + n0 * g.K)), 0, static_cast<int>(nr * g.K), kBufferFlags);
  // A instruction j of this wave fills A rows of instruction i = j * kWaves
  // + wave, W instruction j those of W instruction i; an i past the count
  // loads zeros (offset past the buffer range) into the scratch kilobyte
  const int rl = lane / kC, pos = lane % kC;
  uint32_t aoff[S::kLA], woff[S::kLB];
  int alds[S::kLA], wlds[S::kLB];
#pragma unroll
  for (int j = 0; j < S::kLA; ++j) {
    const int i = j * kWaves + wave, row = i * S::kRowsPerInst + rl;
    const bool real = i < S::kInstA;
    aoff[j] = real ? static_cast<uint32_t>(row * g.lda + 16 * (pos ^ ks_swz<SK>(row))) : 0x80000000u;
    alds[j] = real ? i * 1024 : -1;
  }
#pragma unroll
  for (int j = 0; j < S::kLB; ++j) {
    const int i = j * kWaves + wave, row = i * S::kRowsPerInst + rl;
    const bool real = i < S::kInstB;
    woff[j] = real ? static_cast<uint32_t>(row * g.K + 16 * (pos ^ ks_swz<SK>(row))) : 0x80000000u;
    wlds[j] = real ? S::kStageA + i * 1024 : -1;
  }
  const int nk = static_cast<int>(g.K / SK);
  auto issue = [&](int kt) {
    const int base = (kt % NSTAGE) * S::kStage;
    const int k0 = kt * SK;
#pragma unroll
    for (int j = 0; j < S::kLA; ++j) {
      const int d = alds[j] < 0 ? NSTAGE * S::kStage : base + alds[j];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(lds + d), 16, aoff[j], k0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < S::kLB; ++j) {
      const int d = wlds[j] < 0 ? NSTAGE * S::kStage : base + wlds[j];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(lds + d), 16, woff[j], k0, 0, 0);
    }
  };

  // ---- fragments: lane -> row l % 32, 16 K bytes of chunk 2 * (grp * KS + ks) + l / 32
  const int frow = lane & 31, fgrp = lane >> 5;
  int a_row[kFM], b_row[kFN];
#pragma unroll
  for (int i = 0; i < kFM; ++i) a_row[i] = wm * S::kWaveM + 32 * i + frow;
#pragma unroll
  for (int j = 0; j < kFN; ++j) b_row[j] = wn * S::kWaveN + 32 * j + frow;
  constexpr int kSets = S::kSets;
  v4i fa[kSets][kFM], fb[kSets][kFN];
  auto read_frags = [&](int kt, int ks, int set) {
    const unsigned char* la = lds + (kt % NSTAGE) * S::kStage;
    const unsigned char* lb = la + S::kStageA;
    const int ch = 2 * (grp * KS + ks) + fgrp;
#pragma unroll
    for (int i = 0; i < kFM; ++i)
      fa[set][i] = *reinterpret_cast<const v4i*>(la + a_row[i] * SK + ((ch ^ ks_swz<SK>(a_row[i])) << 4));
#pragma unroll
    for (int j = 0; j < kFN; ++j)
      fb[set][j] = *reinterpret_cast<const v4i*>(lb + b_row[j] * SK + ((ch ^ ks_swz<SK>(b_row[j])) << 4));
  };
  v16i acc[kFM][kFN];
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j) acc[i][j] = v16i{0};
  auto mfmas = [&](int set) {
#pragma unroll
    for (int i = 0; i < kFM; ++i)
#pragma unroll
      for (int j = 0; j < kFN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
  };

  // ---- ring: NSTAGE - 1 stages in flight ahead of the one being consumed.
  // Iteration kt: wait for stage kt (this wave's loads, then the barrier
  // for everyone's, which also guarantees every wave has finished reading
  // stage kt - 1), refill stage kt - 1's slot with stage kt + NSTAGE - 1,
  // then the stage's KS k-steps, fragments read one step ahead (register
  // set ks & 1; one set when KS = 1).
#pragma unroll
  for (int s = 0; s < NSTAGE - 1; ++s)
    if (s < nk) issue(s);
  for (int kt = 0; kt < nk; ++kt) {
    const int later = nk - 1 - kt;
    wait_stages<kL, NSTAGE - 2>(later < NSTAGE - 2 ? later : NSTAGE - 2);
    raw_barrier();
    if (kt + NSTAGE - 1 < nk) issue(kt + NSTAGE - 1);
    read_frags(kt, 0, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) read_frags(kt, ks + 1, (ks + 1) % kSets);
      mfmas(ks % kSets);
    }
  }

  // ---- sum the KG partial tiles in LDS (integer atomics: exact, order-free)
  __syncthreads();  // every wave is past its last fragment read of the ring
  int32_t* red = reinterpret_cast<int32_t*>(lds);
  for (int e = tid; e < BM * S::kRedLd; e += S::kThreads) red[e] = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int r = wm * S::kWaveM + 32 * i + 8 * (v >> 2) + 4 * fgrp + (v & 3);
#pragma unroll
      for (int j = 0; j < kFN; ++j) atomicAdd(&red[r * S::kRedLd + wn * S::kWaveN + 32 * j + frow], acc[i][j][v]);
    }
  __syncthreads();

  // ---- epilogue: 8 consecutive columns of one row per thread and step
  constexpr int kC8 = BN / 8;
  for (int it = tid; it < BM * kC8; it += S::kThreads) {
    const int r = it / kC8, c = (it % kC8) * 8;
    if (r >= mr || c >= nr) continue;
    const int64_t m = m0 + r, n = n0 + c;
    const v4i x0 = *reinterpret_cast<const v4i*>(red + r * S::kRedLd + c);
    const v4i x1 = *reinterpret_cast<const v4i*>(red + r * S::kRedLd + c + 4);
    const int32_t a[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    const int cnt = nr - c < 8 ? static_cast<int>(nr - c) : 8;
    if constexpr (EPI == kEpiBf16) {
      const float sa = g.sa[m];
      uint16_t o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t nn = j < cnt ? n + j : n;
        o[j] = epi_bf16(a[j], sa, g.sw[nn], g.bias, nn, 1.0f, false);
      }
      uint16_t* dst = static_cast<uint16_t*>(g.out) + m * g.ldo + n;
      if (g.staged_out && cnt == 8) {  // N % 8 == 0 and 16-byte aligned rows: n is a multiple of 8
        v4i d;
#pragma unroll
        for (int j = 0; j < 4; ++j) d[j] = static_cast<int>(o[2 * j] | (static_cast<uint32_t>(o[2 * j + 1]) << 16));
        store_out16(dst, d);
      } else {
        for (int j = 0; j < cnt; ++j) dst[j] = o[j];
      }
    } else {
      int32_t* dst = static_cast<int32_t*>(g.out) + m * g.ldo + n;
      for (int j = 0; j < cnt; ++j) dst[j] = a[j];
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

}  // namespace mw8
