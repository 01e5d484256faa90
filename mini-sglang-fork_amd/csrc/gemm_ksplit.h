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
//  * after the last stage the KG partial tiles are summed through LDS:
//    each K group finalizes 1/KG of every lane's accumulators (exact int32
//    adds), applies the epilogue with scales fetched before the main loop,
//    and stages its bf16 values for 16-byte row stores;
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
  static constexpr int kRing = NSTAGE * kStage + (kPad ? 1024 : 0);
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN, kFM = kWaveM / 32, kFN = kWaveN / 32;
  static constexpr int kSets = KS == 1 ? 1 : 2;       // fragment register sets
  // Reduction of the KG partial tiles: each lane holds 16 * kF accumulators
  // (flat index f * 16 + v over its kF = kFM * kFN fragments); K group g
  // finalizes the kP of them in [g * kP, (g + 1) * kP) and receives the
  // other groups' values of that range through LDS exchange slots, one per
  // (owner, writer) pair: (KG - 1) * KG slots of WM * WN waves x kP / 4
  // chunks x 64 lanes x 16 bytes.  The bf16 tile is then staged row-major
  // (BN / 8 chunks of 16 bytes per row) behind the slots for 16-byte stores.
  static constexpr int kF = kFM * kFN;
  static constexpr int kP = 16 * kF / KG;
  static constexpr int kXchg = (KG - 1) * KG * WM * WN * 64 * kP * 4;
  static constexpr int kOC = BN / 8;
  static constexpr int kEpi = kXchg + BM * BN * 2;
  static constexpr int kLds = kRing > kEpi ? kRing : kEpi;
  static_assert(kP % 4 == 0 && kP * KG == 16 * kF, "each K group finalizes whole 4-row groups");
  static_assert(kOC == 4 || kOC == 8 || kOC == 16, "staged row of 4, 8 or 16 chunks");
  static_assert(kThreads >= BM && kThreads >= BN, "one scale-table entry per thread");
  static_assert(kSK == 64 || kSK == 128 || kSK == 256 || kSK == 512, "stage of 64 - 512 K bytes");
  static_assert(KS == 1 || KS % 2 == 0, "one k-step per stage, or an even count");
  static_assert(kInstA * kRowsPerInst == BM && kInstB * kRowsPerInst == BN, "whole rows per DMA instruction");
  static_assert(kFM >= 1 && kFN >= 1 && kFM * 32 * WM == BM && kFN * 32 * WN == BN, "32 x 32 MFMA tiles");
  static_assert(NSTAGE >= 2 && (NSTAGE - 2) * kL < 64, "stages in flight fit the vmcnt counter");
  static_assert(kLds + 4 * (BM + 2 * BN) <= 163840, "LDS budget (ring or exchange + staging, scale tables)");
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

  // epilogue operands (row scales, column scales, bias) are loaded here into
  // registers and kept in LDS tables from the prologue on, so the epilogue
  // has no dependent global loads
  constexpr bool kBf16 = epi_bf16_out(EPI);
  __shared__ float t_sa[kBf16 ? BM : 1], t_sw[kBf16 ? BN : 1], t_bias[kBf16 ? BN : 1];
  float v_sa = 0.0f, v_sw = 0.0f, v_bias = 0.0f;
  if constexpr (kBf16) {
    if (tid < mr) v_sa = g.sa[m0 + tid];
    if (tid < nr) {
      v_sw = g.sw[n0 + tid];
      if (g.bias) v_bias = bf16_to_f32(g.bias[n0 + tid]);
    }
  }

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
  if constexpr (kBf16) {  // read after the main loop's barriers
    if (tid < BM) t_sa[tid] = v_sa;
    if (tid < BN) {
      t_sw[tid] = v_sw;
      t_bias[tid] = v_bias;
    }
  }
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

  // ---- reduce the KG partial tiles (exact int32 adds).  Chunk q = (i * kFN
  // + j) * 4 + h of a lane is the 4 accumulators v = 4h .. 4h + 3 of
  // fragment (i, j): rows wm * kWaveM + 32 i + 8 h + 4 (lane / 32) + 0..3 of
  // column wn * kWaveN + 32 j + lane % 32.  K group g finalizes chunks
  // [g * kQo, (g + 1) * kQo); every other group writes its values of them
  // to the slot (g, writer), conflict-free (64 lanes x 16 bytes per chunk).
  constexpr int kQo = S::kP / 4;  // chunks each K group finalizes
  __syncthreads();  // every wave is past its last fragment read of the ring
  auto slot = [&](int owner, int writer, int c) -> v4i* {
    const int sl = owner * (KG - 1) + (writer < owner ? writer : writer - 1);
    return reinterpret_cast<v4i*>(lds + ((sl * (WM * WN) + wsub) * kQo + c) * 1024 + lane * 16);
  };
  if constexpr (KG > 1) {
#pragma unroll
    for (int i = 0; i < kFM; ++i)
#pragma unroll
      for (int j = 0; j < kFN; ++j)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int q = (i * kFN + j) * 4 + h;
          if (q / kQo != grp)
            *slot(q / kQo, grp, q % kQo) =
                v4i{acc[i][j][4 * h], acc[i][j][4 * h + 1], acc[i][j][4 * h + 2], acc[i][j][4 * h + 3]};
        }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kFM; ++i)
#pragma unroll
      for (int j = 0; j < kFN; ++j)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int q = (i * kFN + j) * 4 + h;
          if (q / kQo != grp) continue;
          for (int w = 0; w < KG; ++w) {
            if (w == grp) continue;
            const v4i d = *slot(grp, w, q % kQo);
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[i][j][4 * h + u] += d[u];
          }
        }
  }

  // ---- epilogue of the owned chunks
  if constexpr (kBf16) {
    if (g.staged_out) {
      // bf16 tile staged row-major behind the exchange slots, then written
      // with 16-byte row stores.  Lanes 2k / 2k+1 swap one value so that each
      // writes two adjacent columns of one row as a 32-bit word; chunk c of
      // row r sits at c ^ sf(r), which spreads the rows R, R+1, R+4, R+5 of
      // one write instruction over distinct banks.
      unsigned char* stg = lds + S::kXchg;
      constexpr int kRowB = BN * 2, kOC = S::kOC;
      auto sf = [](int r) -> int {
        if constexpr (kOC == 16) return 4 * ((r & 1) | (((r >> 2) & 1) << 1));
        else if constexpr (kOC == 8) return 4 * ((r >> 2) & 1);
        else return 0;
      };
      const bool odd = (lane & 1) != 0;
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      // Scales and bias of the owned chunks are read from the LDS tables
      // into registers before the first staging store: read between the
      // stores, each would wait on its own LDS round trip (the compiler
      // cannot prove the staging area and the tables disjoint).  The bias
      // choice is made outside the loop.
      float r_sa[kQo * 4], r_sw[kQo], r_bias[kQo];
#pragma unroll
      for (int i = 0; i < kFM; ++i)
#pragma unroll
        for (int j = 0; j < kFN; ++j)
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const int q = (i * kFN + j) * 4 + h;
            if (q / kQo != grp) continue;
            const int o = q % kQo;
            const int r0 = wm * S::kWaveM + 32 * i + 8 * h + 4 * fgrp, c = wn * S::kWaveN + 32 * j + frow;
            r_sw[o] = t_sw[c];
            r_bias[o] = t_bias[c];
#pragma unroll
            for (int u = 0; u < 4; ++u) r_sa[4 * o + u] = t_sa[r0 + u];
          }
      auto stage = [&](auto bias_tag) {
        constexpr bool kBias = decltype(bias_tag)::value;
#pragma unroll
        for (int i = 0; i < kFM; ++i)
#pragma unroll
          for (int j = 0; j < kFN; ++j)
#pragma unroll
            for (int h = 0; h < 4; ++h) {
              const int q = (i * kFN + j) * 4 + h;
              if (q / kQo != grp) continue;
              const int o = q % kQo;
              const int r0 = wm * S::kWaveM + 32 * i + 8 * h + 4 * fgrp, c = wn * S::kWaveN + 32 * j + frow;
              float tv[4];
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                tv[u] = epi_scale(acc[i][j][4 * h + u], r_sa[4 * o + u], r_sw[o]);
                if constexpr (kBias) tv[u] = tv[u] + r_bias[o];
              }
#pragma unroll
              for (int p = 0; p < 2; ++p) {
                const float t0 = tv[2 * p], t1 = tv[2 * p + 1];
                const float send = odd ? t0 : t1;
                const float got = __builtin_bit_cast(
                    float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, false));
                const bf16x2 pr = odd ? bf16x2{(__bf16)got, (__bf16)t1} : bf16x2{(__bf16)t0, (__bf16)got};
                const int rr = r0 + 2 * p + (odd ? 1 : 0), cc = odd ? c - 1 : c;
                *reinterpret_cast<bf16x2*>(stg + rr * kRowB + (((cc >> 3) ^ sf(rr)) << 4) + (cc & 7) * 2) = pr;
              }
            }
      };
      if (g.bias) stage(std::integral_constant<bool, true>{});
      else stage(std::integral_constant<bool, false>{});
      __syncthreads();
      // N % 8 == 0 (staged_out), so every column range is whole 8-column chunks
      for (int it = tid; it < BM * kOC; it += S::kThreads) {
        const int r = it / kOC, ch = it % kOC;
        if (r < mr && ch * 8 < nr) {
          const v4i d = *reinterpret_cast<const v4i*>(stg + r * kRowB + ((ch ^ sf(r)) << 4));
          store_out16(static_cast<uint16_t*>(g.out) + (m0 + r) * g.ldo + n0 + ch * 8, d);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < kFM; ++i)
#pragma unroll
        for (int j = 0; j < kFN; ++j)
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const int q = (i * kFN + j) * 4 + h;
            if (q / kQo != grp) continue;
            const int r0 = wm * S::kWaveM + 32 * i + 8 * h + 4 * fgrp, c = wn * S::kWaveN + 32 * j + frow;
            if (c >= nr) continue;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              if (r0 + u >= mr) continue;
              float tv = epi_scale(acc[i][j][4 * h + u], t_sa[r0 + u], t_sw[c]);
              if (g.bias) tv = tv + t_bias[c];
              static_cast<uint16_t*>(g.out)[(m0 + r0 + u) * g.ldo + n0 + c] = f32_to_bf16(tv);
            }
          }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kFM; ++i)
#pragma unroll
      for (int j = 0; j < kFN; ++j)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int q = (i * kFN + j) * 4 + h;
          if (q / kQo != grp) continue;
          const int r0 = wm * S::kWaveM + 32 * i + 8 * h + 4 * fgrp, c = wn * S::kWaveN + 32 * j + frow;
          if (c >= nr) continue;
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (r0 + u < mr) static_cast<int32_t*>(g.out)[(m0 + r0 + u) * g.ldo + n0 + c] = acc[i][j][4 * h + u];
        }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

}  // namespace mw8
