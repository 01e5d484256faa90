// Pipelined persistent ring GEMM ("stream" kernel), gfx950 only.
//
// One block per CU (8 waves of 64 x BN/2, v_mfma_i32_16x16x64_i8, a ring of
// two 128-byte K stages moved global -> LDS with buffer_load ... lds) walks
// a list of BM x BN output tiles: the tiles of a dense grid, or the
// (expert chunk, column tile) items of a grouped (fused-MoE) GEMM over
// expert runs.  Unlike one tile per block, the walk does not drain between
// tiles:
//
//  * the DMA ring runs on across items: the next item's first two stages
//    are issued during the current item's last two, so they land while the
//    current item finishes its MFMAs and writes its output;
//  * the epilogue writes through a small per-wave LDS slice (8 rows per
//    pass, no block barrier) with a fixed number of 16-byte buffer stores
//    per wave (a row or column outside the output gets an offset past the
//    buffer, which the hardware drops).  Vector memory operations retire in
//    issue order and vmcnt counts stores as well as loads, so the waits for
//    the next item's first stages count the stores exactly and do not wait
//    for them: the output write burst of item i overlaps item i+1's loads;
//  * the item metadata (sorted pair ids, row and column scales, routed
//    weights, bias) goes straight into double-buffered LDS tables by
//    buffer_load ... lds, a fixed count per wave issued in the first stage
//    of the previous (pair ids) or the same item behind that stage's refill
//    DMA; the next wait counts it, the one after drains it.  No loaded value
//    is held in registers across the K loop, and the walk never spills (a
//    scratch access would be a vector memory operation the waits do not
//    count; the build checks for it).
//
// An item needs at least 6 K stages (K >= 768); the host uses the one-tile
// kernels otherwise.  bf16 output only (the int32 parity hook stays on the
// one-tile kernels); no K split.
#pragma once

#include "gemm_kernels.h"

namespace mw8 {

// Offsets are 32-bit: the host keeps A, W, the output and every metadata
// array below 2^31 bytes.
struct StreamItem {
  int m0, n0;      // first (sorted) row; first output column (kAct: activation column)
  int e;           // expert (grouped), else 0
  int rows_valid;  // rows of the tile that hold rows of A (dense) or sorted positions of the chunk
  int ok;          // 0: no item
};

constexpr int kStreamBM = 256, kStreamBK = 128, kStreamMinStages = 6;

// Dynamic LDS of a stream launch: the ring plus eight 8-row staging slices.
template <int BN, int kAct>
constexpr int stream_lds_bytes() {
  return 2 * (kStreamBM + BN) * kStreamBK + 8 * 8 * (kAct >= 0 ? BN / 4 : BN / 2) * 2;
}

template <int BN, int EPI, bool kGrouped, int kAct = -1>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void stream_gemm_kernel(GemmArgs g) {
#if defined(__HIP_DEVICE_COMPILE__)
  static_assert(epi_bf16_out(EPI), "stream kernel: bf16 output");
  static_assert(kAct < 0 || kGrouped, "fused activation: grouped GEMM1");
  constexpr int BM = kStreamBM, BK = kStreamBK, WN = 2, kWaves = 8, MF = 16;
  using Mf = MfmaI8<MF>;
  using Acc = typename Mf::Acc;
  constexpr int kWaveM = 64, kWaveN = BN / WN, kFM = kWaveM / MF, kFN = kWaveN / MF;
  constexpr int kStageA = BM * BK, kStageB = BN * BK, kStage = kStageA + kStageB, kRing = 2 * kStage;
  constexpr int kLA = BM / (8 * kWaves), kLB = BN / (8 * kWaves), kL = kLA + kLB;
  // staging: 8 rows of the wave's output columns (kAct: its activation columns)
  constexpr int kOutCols = kAct >= 0 ? kWaveN / 2 : kWaveN;
  constexpr int kStgRow = kOutCols * 2, kStgChunks = kStgRow / 16, kStg = 8 * kStgRow;
  constexpr int kReadsPerPass = kStg / 1024;          // 16-byte reads (and stores) per lane and pass
  constexpr int kStores = kFM * 2 * kReadsPerPass;     // buffer stores per wave and item
  static_assert(kFN % 2 == 0 && (kAct < 0 || kFN == 8), "shape");
  static_assert(kStg % 1024 == 0 && (kStgChunks == 8 || kStgChunks == 16), "staging slice");
  static_assert(2 * kL + kStores + 8 < 64, "vmcnt range (two stages, the stores, the metadata loads)");
  static_assert(kRing + 8 * kStg == stream_lds_bytes<BN, kAct>(), "LDS layout");

  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ float t_sa[2][BM], t_rt[2][BM], t_sw[2][BN];
  __shared__ uint32_t t_bias[2][BN / 2];  // bf16 bias of columns 2 i, 2 i + 1
  __shared__ int32_t t_p[2][BM];
  constexpr int kSlots = kGrouped ? kPersistMaxSlots + 1 : 1;
  __shared__ int run_start[kSlots], act_base[kSlots], wave_tot[kWaves];
  static_assert(stream_lds_bytes<BN, kAct>() + 4 * (2 * 3 * BM + 2 * BN) + 4 * BN + 4 * (2 * kSlots + kWaves) <=
                    163840,
                "LDS budget");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int frow = lane & 15, fgrp = lane >> 4;
  // The lane id through an empty asm: per-lane values derived from it are
  // recomputed where they are used instead of being hoisted out of the walk
  // (the walk has no registers to keep them in, and a spill would be a
  // vector memory operation that the waits do not count).
  auto opaque_lane = [] {
    int l = static_cast<int>(threadIdx.x) & 63;
    asm volatile("" : "+v"(l));
    return l;
  };

  // ---------------------------------------------------------------- walk
  const int G = gridDim.x, xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
  const int per_xcd = G / kXcds + (xcd < G % kXcds ? 1 : 0);  // blocks on this XCD
  int tn = 0, total = 0, begin = 0, count = 0, rot = 0;
  uint32_t tm_d = 0;
  const int64_t half = g.N / 2;  // kAct: rows of each of the gate and up halves
  constexpr int kTileCols = kAct >= 0 ? BN / 2 : BN;
  if constexpr (kGrouped) {
    const int carry = build_run_tables<512, true>(g, BM / g.align_bsz, run_start, act_base, wave_tot);
    const int64_t out_cols = kAct >= 0 ? half : g.N;
    tn = static_cast<int>((out_cols + kTileCols - 1) / kTileCols);
    total = carry * tn;
  } else {
    tm_d = static_cast<uint32_t>((g.M + BM - 1) / BM);
    tn = static_cast<int>((g.N + BN - 1) / BN);
    total = static_cast<int>(tm_d) * tn;
  }
  {
    const int base = total / kXcds, rem = total % kXcds;
    begin = xcd * base + (xcd < rem ? xcd : rem);
    count = base + (xcd < rem ? 1 : 0);
    rot = kGrouped ? 0 : xcd * count / kXcds;  // dense: XCD x starts x/8 of the way into its range
  }
  auto item_of = [&](int j) -> StreamItem {
    StreamItem it{0, 0, 0, BM, 0};
    const int pos = local + j * per_xcd;
    if (pos >= count) return it;
    it.ok = 1;
    if constexpr (kGrouped) {
      const int item = begin + pos;
      int lo = 0, hi = g.num_experts - 1;  // the expert: last e with act_base[e] * tn <= item
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (act_base[mid] * tn <= item) lo = mid; else hi = mid - 1;
      }
      const int e = lo;
      const int b_first = run_start[e], nblocks = run_start[e + 1] - b_first;
      const int per_tile = BM / g.align_bsz;
      const int nch = (nblocks + per_tile - 1) / per_tile;
      const int off = item - act_base[e] * tn;
      const int n_tile = off / nch, c = off % nch;  // chunks of one column tile adjacent
      const int c0 = b_first + c * nblocks / nch, c1 = b_first + (c + 1) * nblocks / nch;
      it.m0 = c0 * g.align_bsz;
      it.n0 = n_tile * kTileCols;
      it.e = e;
      it.rows_valid = (c1 - c0) * g.align_bsz;
    } else {
      const uint32_t t = static_cast<uint32_t>(begin + (pos + rot) % count);
      int64_t pm, pn;
      tile_of_index(t, tm_d, static_cast<uint32_t>(tn), pm, pn);
      it.m0 = static_cast<int>(pm) * BM;
      it.n0 = static_cast<int>(pn) * BN;
      const int rv = static_cast<int>(g.M) - it.m0;
      it.rows_valid = rv < BM ? rv : BM;
    }
    it.m0 = __builtin_amdgcn_readfirstlane(it.m0);
    it.n0 = __builtin_amdgcn_readfirstlane(it.n0);
    it.e = __builtin_amdgcn_readfirstlane(it.e);
    it.rows_valid = __builtin_amdgcn_readfirstlane(it.rows_valid);
    return it;
  };

  // weight row of tile row r of item `it` (kAct: per wave half, 64 gate
  // rows then the 64 matching up rows, so that a lane holds the gate and up
  // values of its activation columns)
  const int N32 = static_cast<int>(g.N), half32 = static_cast<int>(half);
  const int K32 = static_cast<int>(g.K), lda32 = static_cast<int>(g.lda), ldo32 = static_cast<int>(g.ldo);
  const int M32 = static_cast<int>(g.M), nval32 = static_cast<int>(g.num_valid);
  auto w_row_of = [&](const StreamItem& it, int r) -> int {
    if constexpr (kAct >= 0) {
      const int rr = r % kWaveN;
      const int a = it.n0 + (r / kWaveN) * (kWaveN / 2) + (rr % (kWaveN / 2));
      const int ac = a < half32 ? a : half32 - 1;
      return rr < kWaveN / 2 ? ac : half32 + ac;
    } else {
      return it.n0 + r < N32 ? it.n0 + r : N32 - 1;
    }
  };

  // pair id of tile row r of an item whose ids sit in t_p[par] (-1: padding,
  // or a row past the chunk; the table holds the raw sorted ids)
  auto pair_of = [&](int par, int r, int rows_valid) -> int32_t {
    const int32_t p = t_p[par][r];
    return r < rows_valid && p >= 0 && p < nval32 ? p : -1;
  };

  // ------------------------------------------------- DMA of the issue item
  // The item whose stages the ring loads (the current item, from its
  // iteration nk-2 on the next one) and the parity of its pair-id table.
  // The per-lane source offsets are recomputed at every issue from these
  // scalars (a few dozen VALU operations per 128-byte stage) rather than
  // held in registers through the walk.
  StreamItem iss{0, 0, 0, BM, 0};
  int iss_par = 0;
  auto issue = [&](int slot, int kt) {
    unsigned char* base = lds + slot * kStage;
    const int k0 = kt * BK, ln = opaque_lane();
    const int64_t a_base_row = kGrouped ? 0 : iss.m0;
    const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        scalar_ptr(const_cast<int8_t*>(g.A + a_base_row * g.lda)), 0, 0x7fffffff, kBufferFlags);
    const int8_t* We = g.W + (kGrouped ? static_cast<int64_t>(iss.e) * g.N * g.K : 0);
    const int w_base_row = kAct >= 0 ? 0 : iss.n0;
    const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        scalar_ptr(const_cast<int8_t*>(We + static_cast<int64_t>(w_base_row) * g.K)), 0, 0x7fffffff, kBufferFlags);
#pragma unroll
    for (int j = 0; j < kLA; ++j) {
      const int unit = (j * kWaves + wave) * 64 + ln, row = unit / 8;
      const int c = (unit % 8) ^ swz_f<BK>(row);
      uint32_t off;
      if constexpr (kGrouped) {
        const int32_t p = pair_of(iss_par, row, iss.rows_valid);
        off = p >= 0 ? static_cast<uint32_t>((p / g.top_k) * lda32 + 16 * c) : 0x80000000u;
      } else {
        const int arow = iss.m0 + row < M32 ? row : M32 - 1 - iss.m0;
        off = static_cast<uint32_t>(arow * lda32 + 16 * c);
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(base + (j * kWaves + wave) * 1024), 16, off, k0, 0,
                                               0);
    }
#pragma unroll
    for (int j = 0; j < kLB; ++j) {
      const int unit = (j * kWaves + wave) * 64 + ln, row = unit / 8;
      const int c = (unit % 8) ^ swz_f<BK>(row);
      const uint32_t off = static_cast<uint32_t>((w_row_of(iss, row) - w_base_row) * K32 + 16 * c);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(base + kStageA + (j * kWaves + wave) * 1024), 16,
                                               off, k0, 0, 0);
    }
  };

  // ------------------------------------------------------------ metadata
  // buffer_load ... lds of 64 table entries each, kMetaLo per wave for waves
  // 0-3 and kMetaHi for waves 4-7 (unconditional: a fixed count):
  //   waves 0-3: row scales t_sa (rows 64 w ..) and weight scales t_sw
  //              (columns 64 w ..);
  //   waves 4-7: routed weights t_rt (grouped; rows 64 (w - 4) ..), or
  //              bias (dense; waves 4-5: columns 2 l, 2 l + 1 of t_bias entry
  //              l = 64 (w - 4) + lane, one dword each; waves 6-7 reload
  //              entries of waves 4-5), a dummy source when the pointer is
  //              null (the value is then unused);
  //   grouped:   the next item's raw pair ids into t_p[par ^ 1] (waves 0-3).
  // Row scales and routed weights are indexed by this item's pair ids
  // (t_p[par], loaded during the previous item).
  constexpr int kMetaLo = kGrouped ? 3 : 2, kMetaHi = 1;
  auto meta_dma = [&](const StreamItem& cur, const StreamItem& nxt, int par) {
    const int w4 = wave & 3, r = 64 * w4 + opaque_lane();
    auto rsrc = [](const void* p) {
      return __builtin_amdgcn_make_buffer_rsrc(scalar_ptr(const_cast<void*>(p)), 0, 0x7fffffff, kBufferFlags);
    };
    int pv = 0;
    if constexpr (kGrouped) {
      const int32_t p = pair_of(par, r, cur.rows_valid);
      pv = p >= 0 ? p : 0;
    } else {
      pv = cur.m0 + r < M32 ? cur.m0 + r : M32 - 1;
    }
    const int wr = w_row_of(cur, r);
    if (wave < 4) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc(g.sa), (lds_ptr_t)(&t_sa[par][64 * w4]), 4,
                                               static_cast<uint32_t>((kGrouped ? pv / g.top_k : pv) * 4), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc(g.sw), (lds_ptr_t)(&t_sw[par][64 * w4]), 4,
          static_cast<uint32_t>(((kGrouped ? cur.e * N32 : 0) + wr) * 4), 0, 0, 0);
      if constexpr (kGrouped) {
        const int idn = nxt.ok && r < nxt.rows_valid ? nxt.m0 + r : 0;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc(g.sorted_ids), (lds_ptr_t)(&t_p[par ^ 1][64 * w4]), 4,
                                                 static_cast<uint32_t>(idn * 4), 0, 0, 0);
      }
    } else {
      if constexpr (kGrouped) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc(g.topk_w ? static_cast<const void*>(g.topk_w) : g.sa),
                                                 (lds_ptr_t)(&t_rt[par][64 * w4]), 4,
                                                 static_cast<uint32_t>((g.topk_w ? pv : 0) * 4), 0, 0, 0);
      } else {
        const int e2 = 64 * (w4 & 1) + opaque_lane();          // t_bias entry: columns 2 e2, 2 e2 + 1
        const int c2 = cur.n0 + 2 * e2 < N32 ? cur.n0 + 2 * e2 : N32 - 2;  // N % 8 == 0 (staged output)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc(g.bias ? static_cast<const void*>(g.bias) : g.sw),
                                                 (lds_ptr_t)(&t_bias[par][64 * (w4 & 1)]), 4,
                                                 static_cast<uint32_t>((g.bias ? c2 : 0) * 2), 0, 0, 0);
      }
    }
  };

  // ----------------------------------------------------------- fragments
  // fragment rows wm*64 + 16 i + frow (A) and wn*kWaveN + 16 j + frow (B)
  // share their low 4 bits, and so the chunk swizzle: one lane offset per
  // operand and substep, the fragments 16 rows (2 KB) apart
  const int a_lane[2] = {swz_lds<BK>(wm * kWaveM + frow, 2 * fgrp), swz_lds<BK>(wm * kWaveM + frow, 2 * fgrp + 1)};
  const int b_lane[2] = {kStageA + swz_lds<BK>(wn * kWaveN + frow, 2 * fgrp),
                         kStageA + swz_lds<BK>(wn * kWaveN + frow, 2 * fgrp + 1)};
  v4i fa[2][kFM], fb[kFN];
  Acc acc[kFM][kFN];
  auto read_a = [&](int slot, int ks, int set) {
    const unsigned char* la = lds + slot * kStage + a_lane[ks];
#pragma unroll
    for (int i = 0; i < kFM; ++i) fa[set][i] = *reinterpret_cast<const v4i*>(la + MF * BK * i);
  };
  auto read_b = [&](int slot, int ks, int j) {
    fb[j] = *reinterpret_cast<const v4i*>(lds + slot * kStage + b_lane[ks] + MF * BK * j);
  };
  int live_w = kWaveM;  // rows of this wave's range holding real pairs (a prefix)
  auto col = [&](int set, int j) {
#pragma unroll
    for (int i = 0; i < kFM; ++i) {
      if (kGrouped && MF * i >= live_w) break;
      acc[i][j] = Mf::mma(fa[set][i], fb[j], acc[i][j]);
    }
  };

  // -------------------------------------------------------------- output
  const int64_t out_rows = kGrouped ? g.num_valid : g.M;
  const int out_cols32 = kAct >= 0 ? half32 : N32;
  const __amdgpu_buffer_rsrc_t o_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      scalar_ptr(g.out), 0, static_cast<int>(out_rows * g.ldo * 2), kBufferFlags);
  unsigned char* stg = lds + kRing + wave * kStg;
  auto sw_row = [](int srow) { return kStgChunks == 16 ? 2 * srow : 2 * (srow >> 1); };
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  // tag: bias (dense) or routed weight (grouped) present
  auto epilogue_tagged = [&](const StreamItem& it, int par, auto tag) {
    constexpr bool has_bias = !kGrouped && decltype(tag)::value;
    constexpr bool has_rt = kGrouped && decltype(tag)::value;
#pragma unroll
    for (int i = 0; i < kFM; ++i) {
#pragma unroll
      for (int vp = 0; vp < 2; ++vp) {
        const int lane = opaque_lane(), frow = lane & 15, fgrp = lane >> 4;
        const bool odd = (lane & 1) != 0;
        const int srow = 2 * fgrp + (odd ? 1 : 0);  // staged row of this lane's word
        const int v0 = 2 * vp;
        const int r0 = wm * kWaveM + MF * i + 4 * fgrp + v0;  // this lane's rows r0, r0 + 1
        const float sa0 = t_sa[par][r0], sa1 = t_sa[par][r0 + 1];
        float rt0 = 1.0f, rt1 = 1.0f;
        if constexpr (has_rt) {
          rt0 = t_rt[par][r0];
          rt1 = t_rt[par][r0 + 1];
        }
        auto val = [&](int j, int v) {
          const int c = wn * kWaveN + MF * j + frow;
          float t = epi_scale(acc[i][j][v], v == v0 ? sa0 : sa1, t_sw[par][c]);
          if constexpr (has_bias) t = t + bf16_to_f32(static_cast<uint16_t>(t_bias[par][c >> 1] >> (16 * (c & 1))));
          if constexpr (has_rt) t = t * (v == v0 ? rt0 : rt1);
          return t;
        };
        auto put = [&](int cl, float t0, float t1) {  // cl: this lane's column in the slice
          const float send = odd ? t0 : t1;
          const float got = __builtin_bit_cast(
              float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, false));
          const bf16x2 pr = odd ? bf16x2{(__bf16)got, (__bf16)t1} : bf16x2{(__bf16)t0, (__bf16)got};
          const int cc = odd ? cl - 1 : cl;
          *reinterpret_cast<bf16x2*>(stg + srow * kStgRow + (((cc >> 3) ^ sw_row(srow)) << 4) + (cc & 7) * 2) = pr;
        };
        if constexpr (kAct >= 0) {
#pragma unroll
          for (int j = 0; j < kFN / 2; ++j) {
            auto act = [&](int v) {
              const float gv = bf16_to_f32(f32_to_bf16(val(j, v)));
              const float uv = bf16_to_f32(f32_to_bf16(val(j + kFN / 2, v)));
              return act_fn<kAct>(gv) * uv;
            };
            put(MF * j + frow, act(v0), act(v0 + 1));
          }
        } else {
#pragma unroll
          for (int j = 0; j < kFN; ++j) put(MF * j + frow, val(j, v0), val(j, v0 + 1));
        }
        // the slice holds tile rows wm*64 + 16 i + 4 (s / 2) + v0 + (s & 1), s = 0..7;
        // each lane writes kReadsPerPass 16-byte chunks of it (the wave's own
        // LDS slice: its LDS operations execute in order, no barrier)
        asm volatile("" ::: "memory");
#pragma unroll
        for (int q = 0; q < kReadsPerPass; ++q) {
          const int u = q * 64 + lane, sr = u / kStgChunks, ch = u % kStgChunks;
          const v4i d = *reinterpret_cast<const v4i*>(stg + sr * kStgRow + ((ch ^ sw_row(sr)) << 4));
          const int r = wm * kWaveM + MF * i + 4 * (sr >> 1) + v0 + (sr & 1);
          int orow;
          if constexpr (kGrouped) orow = pair_of(par, r, it.rows_valid);
          else orow = r < it.rows_valid ? it.m0 + r : -1;
          const int ocol = it.n0 + wn * kOutCols + ch * 8;
          const uint32_t voff = orow >= 0 && ocol < out_cols32
                                    ? static_cast<uint32_t>(orow) * static_cast<uint32_t>(ldo32 * 2) +
                                          static_cast<uint32_t>(ocol * 2)
                                    : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b128(d, o_rsrc, voff, 0, kStreamAux);
        }
        asm volatile("" ::: "memory");
      }
    }
  };

  auto epilogue = [&](const StreamItem& it, int par) {
    if ((kGrouped ? static_cast<const void*>(g.topk_w) : static_cast<const void*>(g.bias)) != nullptr)
      epilogue_tagged(it, par, std::integral_constant<bool, true>{});
    else
      epilogue_tagged(it, par, std::integral_constant<bool, false>{});
  };

  // ---------------------------------------------------------------- main
  StreamItem cur = item_of(0);
  if (!cur.ok) return;  // block-uniform
  const int nk = static_cast<int>(g.K / BK);
  int par = 0, gbase = 0, jn = 1;
  // first item: its pair ids into t_p[0] (grouped) before any DMA
  if constexpr (kGrouped) {
    if (tid < BM) t_p[0][tid] = tid < cur.rows_valid ? g.sorted_ids[cur.m0 + tid] : -1;
    __syncthreads();
  }
  iss = cur;
  iss_par = 0;
  issue(0, 0);
  issue(1, 1);
  bool first = true;
  for (;;) {
    const StreamItem nxt = item_of(jn++);
    if constexpr (kGrouped) {  // this wave's real rows: a prefix of its 64 (pairs, then padding)
      live_w = __popcll(__ballot(pair_of(par, wm * kWaveM + lane, cur.rows_valid) >= 0));
      live_w = __builtin_amdgcn_readfirstlane(live_w);
    }
#pragma unroll
    for (int i = 0; i < kFM; ++i)
#pragma unroll
      for (int j = 0; j < kFN; ++j) acc[i][j] = Acc{0};
    auto slot = [&](int kt) { return (gbase + kt) & 1; };
    // stage 0 landed: after it were issued stage 1 and, past the first
    // item, the previous item's stores
    if (first) wait_vmcnt_lgkm0<kL>(); else wait_vmcnt_lgkm0<kL + kStores>();
    raw_barrier();
    read_a(slot(0), 0, 0);
#pragma unroll
    for (int j = 0; j < kFN; ++j) read_b(slot(0), 0, j);
    for (int kt = 0; kt + 1 < nk; ++kt) {
      read_a(slot(kt), 1, 1);
#pragma unroll
      for (int j = 0; j < kFN; ++j) {
        col(0, j);
        read_b(slot(kt), 1, j);
      }
      // stage kt+1 landed.  Issued after it: in iteration 0 the previous
      // item's stores (kStores per wave), in iteration 1 this item's
      // metadata DMA (kMetaLo / kMetaHi per wave), later nothing
      if (kt == 0) {
        if (first) wait_vmcnt_lgkm0<0>(); else wait_vmcnt_lgkm0<kStores>();
      } else if (kt == 1) {
        if (wave < 4) wait_vmcnt_lgkm0<kMetaLo>(); else wait_vmcnt_lgkm0<kMetaHi>();
      } else {
        wait_vmcnt_lgkm0<0>();
      }
      raw_barrier();  // from kt == 2 on, this item's metadata and the next item's pair ids are in the tables
      read_a(slot(kt + 1), 0, 0);
#pragma unroll
      for (int j = 0; j < kFN; ++j) {
        col(1, j);
        read_b(slot(kt + 1), 0, j);
      }
      if (kt + 2 < nk) {
        issue(slot(kt + 2), kt + 2);
      } else if (nxt.ok) {  // kt == nk - 2: the next item's stage 0
        iss = nxt;
        iss_par = par ^ 1;
        issue(slot(kt + 2), 0);
      }
      if (kt == 0) meta_dma(cur, nxt, par);
    }
    read_a(slot(nk - 1), 1, 1);
#pragma unroll
    for (int j = 0; j < kFN; ++j) {
      col(0, j);
      read_b(slot(nk - 1), 1, j);
    }
    // every wave is past its reads of stage nk-1: its slot takes the next item's stage 1
    wait_vmcnt_lgkm0<63>();
    raw_barrier();
    if (nxt.ok) issue(slot(nk + 1), 1);
#pragma unroll
    for (int j = 0; j < kFN; ++j) col(1, j);
    epilogue(cur, par);
    if (!nxt.ok) break;
    cur = nxt;
    par ^= 1;
    gbase += nk;
    first = false;
  }
#endif  // __HIP_DEVICE_COMPILE__
}

}  // namespace mw8
