// int8 x int8 -> int32 MFMA GEMM cores shared by the dense linear and the
// grouped (fused-MoE) GEMM.  gfx950 only.
//
// Layouts (row-major, K contiguous; "NT" like the reference's F.linear
// weight [N, K], python/minisgl/layers/linear.py:28):
//   A  int8 [rows, K]   activations (rows gathered through a RowMap)
//   W  int8 [N, K]      weights (per expert: base + e * N * K)
//   out[row, n]         bf16 (scaled epilogue) or int32 (raw accumulators)
//
// Cores:
//   tile_gemm_kernel  -- register-staged MFMA tile (any K % 16 == 0).
//   tile3_gemm_kernel -- the large-M ring: direct-to-LDS DMA of A and W
//                  tiles, NSTAGE-deep ring (optionally the W stages one
//                  stage further ahead in a ring of their own: kBLead),
//                  v_mfma_i32_16x16x64_i8 on 128-byte stages
//                  (v_mfma_i32_32x32x32_i8 on 64-byte ones), K split of
//                  the last partial wave of tiles (split_reduce_kernel).
//   grouped_persist_kernel -- the same ring walking (expert chunk, column
//                  tile) items of the fused-MoE GEMM.
//   (gemm_ksplit.h: in-block split-K tiles for 33-768 rows; gemm_stream.h:
//   the pipelined persistent walk over 256x256 tiles.)
//   decode_gemm_kernel / decode3_gemm_kernel -- dense small M (decode):
//                  weight streaming with v_mfma_i32_16x16x64_i8, weight rows
//                  as the MFMA "A" operand, up to 64 tokens as the "B"
//                  operand, K split across the waves of a block and reduced
//                  in LDS; decode3 streams through a per-wave LDS DMA ring
//                  and also serves 16/32-row fused-MoE alignment blocks.
//
// MFMA lane layouts (checked on gfx950 by an in-bounds probe):
//   32x32x32: lane l feeds A row l%32 / B col l%32 with 16 K-bytes of group
//             l/32; D reg v holds row 8*(v/4) + 4*(l/32) + v%4, col l%32.
//   16x16x64: lane l feeds A row l%16 / B col l%16 with 16 K-bytes of group
//             l/16; D reg v holds row 4*(l/16) + v, col l%16.
// Which K byte a (group, byte) pair stands for does not matter as long as A
// and B use the same mapping, which both cores do by construction.
#pragma once

#include <type_traits>

#include "mw8_common.h"

namespace mw8 {

enum EpiKind : int { kEpiBf16 = 0, kEpiI32 = 1 };
constexpr bool epi_bf16_out(int e) { return e == kEpiBf16; }

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
  // dense K split (ring tile core): blocks [0, full_tiles) own whole
  // tiles; block full_tiles + u owns K range u % tail_split of tile
  // full_tiles + u / tail_split and writes its int32 partial tile to
  // part[u][BM][BN] (summed in split order by split_reduce_kernel).
  // full_tiles = 0 splits every tile (grids with fewer tiles than CUs).
  int32_t* part;
  int64_t full_tiles;
  int32_t tail_split;          // <= 1: no split
  // bf16 output rows are 16-byte aligned with N % 8 == 0: the tile core may
  // assemble its output tile in LDS and store it with 16-byte row writes
  int32_t staged_out;
  // grouped GEMM over expert runs (SortedRunRows): rows of the alignment
  // blocks behind expert_ids / num_post_pad (the tile height BM is a
  // multiple of it)
  int32_t align_bsz;
  // router-id rows (TopkRows): 16-pair units per expert (ceil(tokens / 16))
  int32_t topk_units;
};

__device__ __forceinline__ uint16_t epi_bf16(int32_t acc, float sa, float sw, const uint16_t* bias,
                                             int64_t n, float routed, bool has_routed) {
  float t = epi_scale(acc, sa, sw);
  if (bias) t = t + bf16_to_f32(bias[n]);
  if (has_routed) t = t * routed;
  return f32_to_bf16(t);
}

// Output stores of a bf16 epilogue: 16-byte rows non-temporal (the output is
// written once; gate_up M=8192 1405 -> 1377 us on MI355X).
__device__ __forceinline__ void store_out16(uint16_t* dst, v4i d) {
  __builtin_nontemporal_store(d, reinterpret_cast<v4i*>(dst));
}

// ------------------------------------------------------------------------
// Row maps: dense rows vs. expert-sorted rows (grouped GEMM).
// ------------------------------------------------------------------------
struct DenseRows {
  static constexpr bool kGrouped = false;
  static constexpr bool kRuns = false;
};
// One tile per alignment block (BM == alignment block size).
struct SortedRows {
  static constexpr bool kGrouped = true;
  static constexpr bool kRuns = false;
};
// One tile per run of up to BM / align_bsz consecutive alignment blocks of
// one expert: the tile covers sorted rows [m0, m0 + rows_valid) and rows
// past the run are neither loaded, multiplied nor stored.  The grid has one
// block per alignment block; a block whose alignment block is not at a
// multiple of BM / align_bsz from the start of its expert's segment exits.
struct SortedRunRows {
  static constexpr bool kGrouped = true;
  static constexpr bool kRuns = true;
};
// An expert's rows taken straight from the router's ids (decode batches
// whose top-k experts are distinct per token, so an expert holds at most
// one pair per token): block y is unit y % U of expert y / U (U =
// GemmArgs::topk_units), its rows the pairs 16 u .. 16 u + 15 of the pairs
// p with topk_ids[p] == e in ascending order (GemmArgs::sorted_ids carries
// topk_ids).  No alignment pass.  Decode core only.
struct TopkRows {
  static constexpr bool kGrouped = true;
  static constexpr bool kRuns = false;
};

// ------------------------------------------------------------------------
// Large-M tile core
// ------------------------------------------------------------------------
template <int BM, int BN, int BK, int WM, int WN>
struct TileShape {
  static constexpr int kBK = BK;                     // K bytes per stage
  static constexpr int kChunksK = BK / 16;           // 16-byte chunks per tile row
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
  static constexpr int kFM = kWaveM / 32, kFN = kWaveN / 32;
  static constexpr int kAChunks = BM * BK / 16 / 256;  // 16-byte chunks per thread
  static constexpr int kBChunks = BN * BK / 16 / 256;
  static constexpr int kLdsA = BM * BK, kLdsB = BN * BK;
  static constexpr int kLds = 2 * (kLdsA + kLdsB);
  static_assert(BK == 64 || BK == 128, "BK is 64 or 128 bytes");
  static_assert(WM * WN == 4, "4 waves per block");
  static_assert(kFM >= 1 && kFN >= 1, "wave tile must hold one 32x32 MFMA");
  static_assert(kAChunks >= 1 && kBChunks >= 1, "tile too small");
};

// LDS byte offset of 16-byte chunk c of tile row r.  The chunk index is
// XOR-swizzled with low row bits so that the 8 rows read together by one
// phase of a ds_read_b128 fragment load land in 8 different bank groups.
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  if constexpr (BK == 128) return row * 128 + ((chunk ^ (row & 7)) << 4);
  else return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}

// Tile order for dense launches (1-D grid of tiles_m * tiles_n blocks).
// The hardware hands block b to XCD b % 8; each XCD is given a contiguous
// range of tile ids so that the tiles running together on one XCD share
// its L2.  Inside the range tiles follow a grouped raster: kGroupM tile
// rows advance together along N, so one wave of concurrent tiles reuses
// kGroupM A panels and a handful of W panels.
constexpr int kXcds = 8;
constexpr int kGroupM = 4;

// The tile arithmetic below is 32-bit: the host launches at most 2^31
// blocks and tiles, and a 64-bit division by a runtime value expands into
// a long scalar routine that every block would run before its first load.

// Tile index t of the grouped raster -> (pid_m, pid_n).
__device__ __forceinline__ void tile_of_index(uint32_t t, uint32_t tiles_m, uint32_t tiles_n,
                                              int64_t& pid_m, int64_t& pid_n) {
  const uint32_t per_group = kGroupM * tiles_n;
  const uint32_t group = t / per_group;
  const uint32_t first_m = group * kGroupM;
  const uint32_t gsize = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
  const uint32_t in_group = t - group * per_group;
  const uint32_t col = in_group / gsize;
  pid_m = first_m + (in_group - col * gsize);
  pid_n = col;
}

// Block b (b < count) -> tile index in [0, count): XCD b % 8 gets a
// contiguous range of tile indices.
__device__ __forceinline__ uint32_t xcd_tile_index(uint32_t b, uint32_t count) {
  const uint32_t xcd = b % kXcds, local = b / kXcds;
  const uint32_t base = count / kXcds, rem = count % kXcds;
  return xcd * base + (xcd < rem ? xcd : rem) + local;
}

// As xcd_tile_index, with XCD x walking its range from position x/8 of it
// (wrapping): the blocks resident at one time on different XCDs sit at
// different places of the grouped raster, so the eight L2s do not all miss
// on the same weight lines at once (a line requested by eight L2s together
// is fetched for one after the other).  The blocks concurrent on one XCD
// stay consecutive in the raster.  Measured on MI355X (graph-timed, weights
// from HBM): gate_up M=8192 1312-1324 -> 1259-1273 us, down M=8192 637 ->
// 628 us.
__device__ __forceinline__ uint32_t xcd_tile_index_rot(uint32_t b, uint32_t count) {
  const uint32_t xcd = b % kXcds, local = b / kXcds;
  const uint32_t base = count / kXcds, rem = count % kXcds;
  const uint32_t n_x = base + (xcd < rem ? 1 : 0);  // blocks b with b % 8 == xcd
  const uint32_t start = xcd * base + (xcd < rem ? xcd : rem);
  return start + (local + xcd * n_x / kXcds) % n_x;
}

__device__ __forceinline__ void tile_of_block(uint32_t b, uint32_t tiles_m, uint32_t tiles_n,
                                              int64_t& pid_m, int64_t& pid_n) {
  tile_of_index(xcd_tile_index_rot(b, tiles_m * tiles_n), tiles_m, tiles_n, pid_m, pid_n);
}

template <int BM, int BN, int BK, int WM, int WN, int EPI, class Rows>
__global__ __launch_bounds__(256) void tile_gemm_kernel(GemmArgs g) {
  using S = TileShape<BM, BN, BK, WM, WN>;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int8_t* W = g.W;
  const float* sw = g.sw;
  int64_t m0, n0, mblk = 0;
  if constexpr (Rows::kGrouped) {
    // 2-D grid: x = N tiles, y = expert blocks of BM sorted rows
    n0 = static_cast<int64_t>(blockIdx.x) * BN;
    mblk = blockIdx.y;
    m0 = mblk * BM;
    if (m0 >= static_cast<int64_t>(*g.num_post_pad)) return;
    const int e = g.expert_ids[mblk];
    if (e < 0 || e >= g.num_experts) return;
    W += static_cast<int64_t>(e) * g.N * g.K;
    sw += static_cast<int64_t>(e) * g.N;
  } else {
    int64_t pm, pn;
    tile_of_block(blockIdx.x, (g.M + BM - 1) / BM, (g.N + BN - 1) / BN, pm, pn);
    m0 = pm * BM;
    n0 = pn * BN;
  }

  // ---- per-thread global sources of the 16-byte chunks this thread stages:
  // chunk id = tid + 256 * i -> tile row id / kChunksK, column id % kChunksK.
  const int cc = tid % S::kChunksK;
  const int8_t* a_src[S::kAChunks];
  const int8_t* w_src[S::kBChunks];
  int a_lds[S::kAChunks], w_lds[S::kBChunks];
#pragma unroll
  for (int i = 0; i < S::kAChunks; ++i) {
    const int r = (tid + 256 * i) / S::kChunksK;
    int64_t arow;
    if constexpr (Rows::kGrouped) {
      const int32_t p = g.sorted_ids[m0 + r];
      arow = p < g.num_valid ? p / g.top_k : 0;
    } else {
      arow = m0 + r < g.M ? m0 + r : g.M - 1;
    }
    a_src[i] = g.A + arow * g.lda + 16 * cc;
    a_lds[i] = swz<BK>(r, cc);
  }
#pragma unroll
  for (int i = 0; i < S::kBChunks; ++i) {
    const int r = (tid + 256 * i) / S::kChunksK;
    const int64_t wrow = n0 + r < g.N ? n0 + r : g.N - 1;
    w_src[i] = W + wrow * g.K + 16 * cc;
    w_lds[i] = swz<BK>(r, cc);
  }

  v16i acc[S::kFM][S::kFN];
#pragma unroll
  for (int i = 0; i < S::kFM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFN; ++j) acc[i][j] = v16i{0};

  const int nk = static_cast<int>((g.K + BK - 1) / BK);
  v4i ra[S::kAChunks], rb[S::kBChunks];

  auto gload = [&](int kt) {
    const int64_t k0 = static_cast<int64_t>(kt) * BK;
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
    for (int ks = 0; ks < BK / 32; ++ks) {
      const int ch = 2 * ks + fgrp;
      v4i fa[S::kFM], fb[S::kFN];
#pragma unroll
      for (int i = 0; i < S::kFM; ++i)
        fa[i] = *reinterpret_cast<const v4i*>(la + swz<BK>(wm * S::kWaveM + 32 * i + frow, ch));
#pragma unroll
      for (int j = 0; j < S::kFN; ++j)
        fb[j] = *reinterpret_cast<const v4i*>(lb + swz<BK>(wn * S::kWaveN + 32 * j + frow, ch));
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
// Large-M tile core v3: direct-to-LDS loads, NSTAGE-deep ring
// ------------------------------------------------------------------------
// Every K step of BK bytes, each wave moves its share of the A and W tiles
// straight from global memory into LDS with global_load_lds_dwordx4 (one
// 1 KB contiguous LDS run per wave instruction; lane l fills 16-byte unit
// l of it, and is pointed at the global chunk that belongs there under the
// swizzle).  Stages are prefetched NSTAGE-1 K steps ahead and tracked with
// explicit vmcnt waits; one s_barrier per K step.  MFMA fragments are read
// from LDS one half-step ahead of the MFMAs that consume them (two register
// sets F0/F1), so LDS latency hides behind the MFMAs.  Requires K % BK == 0.
//
// LDS rows are BK bytes (4 or 8 chunks of 16 bytes).  Chunk c of row r sits
// at unit r*BK/16 + (c ^ f(r)), with f chosen so that the fragment reads of
// 8 waves per CU move 207-210 B/clk per CU through LDS on MI355X, the rate
// of a linear read (measured with an in-bounds ds_read_b128 probe):
//   BK = 64 : f(r) = (r ^ (r >> 2)) & 3        (32x32x32 fragments, chunks
//             2 s + g; ((r >> 1) ^ (r >> 3)) & 3 gave 130-139 B/clk here)
//   BK = 128: f(r) = (r & 7) ^ ((r >> 3) & 1)
// The 16x16x64 fragments of a 128-byte stage read chunk 2 g + s (lane group
// g = l / 16, substep s) rather than 4 s + g: with lane groups on chunks
// c..c+3 the reads of 8 waves per CU moved 136 B/clk per CU through LDS on
// MI355X, with groups on chunks 0,2,4,6 (or 1,3,5,7) 212-244 B/clk, as the
// 32x32x32 fragments do (an in-bounds ds_read_b128 probe; the MFMA sums
// over all of a stage's K bytes, so any chunk order serves A and B alike).
template <int BK>
__device__ __forceinline__ int swz_f(int row) {
  if constexpr (BK == 64) return (row ^ (row >> 2)) & 3;
  else return (row & 7) ^ ((row >> 3) & 1);
}
template <int BK>
__device__ __forceinline__ int swz_lds(int row, int chunk) {
  return row * BK + ((chunk ^ swz_f<BK>(row)) << 4);
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14,
// expcnt 6:4 left at its maximum, lgkmcnt 11:8 = 0).  Waiting for this
// wave's LDS reads as well makes the barrier that follows a point after
// which no wave still reads the stage buffer about to be refilled.
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
  asm volatile("" ::: "memory");
}
// Wait until a stage's DMA loads have landed while n (<= MAXS) later stage
// issues of L loads each may stay in flight.
template <int L, int MAXS>
__device__ __forceinline__ void wait_stages(int n) {
  if constexpr (MAXS >= 3) { if (n >= 3) { wait_vmcnt_lgkm0<3 * L>(); return; } }
  if constexpr (MAXS >= 2) { if (n == 2) { wait_vmcnt_lgkm0<2 * L>(); return; } }
  if constexpr (MAXS >= 1) { if (n == 1) { wait_vmcnt_lgkm0<L>(); return; } }
  wait_vmcnt_lgkm0<0>();
}

// Weight-lead rings: wait until a stage has landed while the loads issued
// after its A stage stay in flight: W stages for the next r stages and A
// stages for the next min(r, AMAX), L_A / L_B loads each (r <= MAXR <= 4).
template <int LA, int LB, int MAXR, int AMAX>
__device__ __forceinline__ void wait_lead(int r) {
  static_assert(MAXR <= 4 && (4 * LB + 4 * LA) < 64, "vmcnt range");
  constexpr auto cnt = [](int n) { return n * LB + (n < AMAX ? n : AMAX) * LA; };
  if constexpr (MAXR >= 4) { if (r >= 4) { wait_vmcnt_lgkm0<cnt(4)>(); return; } }
  if constexpr (MAXR >= 3) { if (r == 3) { wait_vmcnt_lgkm0<cnt(3)>(); return; } }
  if constexpr (MAXR >= 2) { if (r == 2) { wait_vmcnt_lgkm0<cnt(2)>(); return; } }
  if constexpr (MAXR >= 1) { if (r == 1) { wait_vmcnt_lgkm0<cnt(1)>(); return; } }
  wait_vmcnt_lgkm0<0>();
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// A pointer the compiler can prove wave-uniform (it lives in SGPRs).  A
// buffer descriptor built from a pointer it cannot prove uniform is kept in
// VGPRs, and every buffer load through it is then wrapped in a per-lane
// "waterfall" loop of readfirstlane/compare/exec-mask instructions.
template <class T>
__device__ __forceinline__ T* scalar_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
  return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

constexpr int kPersistMaxSlots = 512;  // expert slots of the persistent grouped walk (E < this)

// Buffer-resource word 3 for raw byte-addressed buffers on gfx9-family parts.
constexpr int kBufferFlags = 0x00020000;
// Cache policy of a streamed weight DMA: non-temporal (decode GEMM weights
// are read once).  Measured on MI355X against the default policy: gate_up
// M=1 32.5 -> 30.0 us, qkv / o_proj / down M=1 4-8% faster.
constexpr int kStreamAux = 2;

// Workgroup barrier without the release/acquire fence of __syncthreads()
// (which would force vmcnt(0) and drain the prefetch ring).  The empty asm
// statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The int8 MFMA a ring tile is built from (MF = output rows and columns of
// one instruction).  Both take 16 K-bytes per lane as A and B operands:
//   MF = 32: v_mfma_i32_32x32x32_i8, lane l feeds row / column l % 32 with
//            K group l / 32 (2 groups = 32 K bytes per instruction); D reg v
//            (16) holds row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32.
//   MF = 16: v_mfma_i32_16x16x64_i8, lane l feeds row / column l % 16 with
//            K group l / 16 (4 groups = 64 K bytes); D reg v (4) holds row
//            4 (l / 16) + v, column l % 16.
// On MI355X the two run at the same nominal rate (4.98 POPS with constant
// operands), but on random int8 data the part is power-limited and the
// 16x16x64 form sustains 3.92-3.99 POPS against 3.35-3.41 for 32x32x32
// (register-only loops, 4 waves per SIMD).
template <int MF>
struct MfmaI8;
template <>
struct MfmaI8<32> {
  using Acc = v16i;
  static constexpr int kK = 32, kV = 16, kGroups = 2;
  static __device__ __forceinline__ int row(int lane, int v) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }
  static __device__ __forceinline__ Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <>
struct MfmaI8<16> {
  using Acc = v4i;
  static constexpr int kK = 64, kV = 4, kGroups = 4;
  static __device__ __forceinline__ int row(int lane, int v) { return 4 * (lane >> 4) + v; }
  static __device__ __forceinline__ Acc mma(v4i a, v4i b, Acc c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
};

// One BM x BN output tile over K stages [kt_begin, kt_end) of the ring core.
struct TileJob {
  int64_t m0, n0;     // first (sorted) row and first output column
  const int8_t* W;    // weight rows of the tile's expert (dense: all of W)
  const float* sw;
  int kt_begin, kt_end;
  int rows_valid;     // rows of the tile that hold sorted positions (runs)
  int64_t split_unit; // >= 0: write the int32 partial tile part[split_unit]
};

// kAct >= 0 (bf16, staged epilogue; grouped or dense rows): the tile's B
// rows are the gate rows [n0, n0 + BN/2) and the up rows N/2 + [n0, n0 +
// BN/2) of a gate|up weight [N = 2I, K]; the epilogue writes act =
// bf16(act_fn(g) * u) for act columns [n0, n0 + BN/2) of an [rows, I]
// output (g.ldo = I), g and u the bf16-rounded GEMM outputs, as the separate
// activation kernel computes it.  A dense K-split unit writes its int32
// partial tile in the same column order (gate half, then up half).
// kWAux: cache policy of the weight DMA (0, or kStreamAux for weights that
// only one block reads: a dense grid with a single row tile).
template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI, class Rows, int kAct = -1, int kWAux = 0,
          int MF = 32, int kBLead = 0>
__device__ __forceinline__ void tile3_run(const GemmArgs& g, unsigned char* lds, const TileJob& job) {
#if defined(__HIP_DEVICE_COMPILE__)
  using Mf = MfmaI8<MF>;
  using Acc = typename Mf::Acc;
  constexpr int kWaves = WM * WN;
  constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
  constexpr int kFM = kWaveM / MF, kFN = kWaveN / MF;
  constexpr int kV = Mf::kV;  // accumulator registers per fragment and lane
  constexpr int kChunks = BK / 16;                 // 16-byte chunks per LDS row
  constexpr int kRowsPerInst = 1024 / BK;           // rows one 1 KB DMA instruction fills
  constexpr int kStageA = BM * BK, kStageB = BN * BK, kStage = kStageA + kStageB;
  constexpr int kLA = BM / (kRowsPerInst * kWaves), kLB = BN / (kRowsPerInst * kWaves);
  constexpr int kL = kLA + kLB;                     // DMA instructions per wave per stage
  static_assert(BK == 64 || BK == 128, "BK");
  static_assert((kWaves == 4 || kWaves == 8 || kWaves == 16) && kFM >= 1 && kFN >= 1, "shape");
  static_assert(BK / Mf::kK >= 2, "the fragment pipeline runs two k-substeps per stage");
  static_assert(kLA >= 1 && kLB >= 1 && kLA * kRowsPerInst * kWaves == BM &&
                kLB * kRowsPerInst * kWaves == BN, "DMA split");
  static_assert(NSTAGE >= 2 && NSTAGE <= 5 && (NSTAGE - 2) * kL < 64, "stages");
  // kBLead = 1: the weight stages run one stage ahead of the A stages, in a
  // ring of NSTAGE + 1 slots beside the A ring of NSTAGE (on a 256 x 256
  // tile the 2 + 3 slots of 32 KB fill the CU's 160 KB), so each weight
  // stage has one stage more of MFMA time to arrive from HBM.  The scale
  // tables then live in the ring, written after the main loop.  Issue
  // order: A0 W0, then W s A s for s < NSTAGE, then W NSTAGE; stage kt of
  // the main loop issues A kt+NSTAGE and W kt+NSTAGE+1.  Every W stage is
  // thus issued before its A stage, and the loads issued after A j are W
  // j+1, A j+1, W j+2, ... (wait_lead counts them).
  static_assert(kBLead == 0 || (kBLead == 1 && MF == 16 && NSTAGE <= 4 && !Rows::kGrouped), "weight lead");
  constexpr int kBSlots = NSTAGE + kBLead;
  constexpr int kRingBytes = NSTAGE * kStageA + kBSlots * kStageB;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int wm = wave / WN, wn = wave % WN;

  const int8_t* W = job.W;
  const float* sw = job.sw;
  const int64_t m0 = job.m0, n0 = job.n0, split_unit = job.split_unit;
  const int kt_begin = job.kt_begin, kt_end = job.kt_end, rows_valid = job.rows_valid;

  // ---- per-lane DMA sources: instruction j of this wave fills LDS units
  // (j*kWaves + wave)*64 .. +63 of the tile; lane -> (row, chunk)
  // DMA through buffer views (32-bit per-lane offsets, the K position in the
  // scalar offset): the A view starts at the tile's first row (row 0 for
  // gathered rows), the W view at the tile's first weight row.  The host
  // keeps every offset below 2^31 (gemm_common / moe_gemm_w8a8 checks).
  // Grouped bf16 epilogue: the tile's row metadata (pair index, activation
  // scale, routed weight) is fetched at the start and kept in LDS, so the
  // dependent loads overlap the main loop instead of stalling the epilogue.
  // The dense bf16 epilogue keeps its row scales in the same table, and
  // both keep the tile's column scales (and bias) in LDS.
  constexpr bool kMeta = Rows::kGrouped && epi_bf16_out(EPI);
  constexpr bool kMetaSa = epi_bf16_out(EPI);
  static_assert(!kMetaSa || (BM <= 64 * kWaves && BN <= 64 * kWaves), "one metadata row per thread");
  __shared__ int32_t meta_p[kMeta ? BM : 1];
  __shared__ float meta_rt[kMeta ? BM : 1];
  constexpr bool kTabInRing = kBLead > 0;  // the dense tables past the staged bf16 tile
  float *meta_sa, *meta_sw, *meta_bias;
  if constexpr (kTabInRing) {
    meta_sa = reinterpret_cast<float*>(lds + BM * BN * 2);
    meta_sw = meta_sa + BM;
    meta_bias = meta_sw + BN;
    static_assert(kRingBytes <= 163840 && BM * BN * 2 + 4 * (BM + 2 * BN) <= kRingBytes, "LDS budget");
  } else {
    __shared__ float t_sa[kMetaSa ? BM : 1], t_sw[kMetaSa ? BN : 1], t_bias[kMetaSa && !Rows::kGrouped ? BN : 1];
    meta_sa = t_sa;
    meta_sw = t_sw;
    meta_bias = t_bias;
    // ring + these tables + the persistent walk's run tables fit in the CU's 160 KB
    static_assert(kRingBytes + 4 * (3 * BM + 2 * BN) + 4 * (2 * kPersistMaxSlots + 2 + 16) <= 163840,
                  "LDS budget");
  }
  int32_t meta_pv = 0;
  float meta_sav = 0.0f, meta_rtv = 1.0f, meta_swv = 0.0f, meta_bv = 0.0f;
  if constexpr (kMeta) {
    if (tid < BM) meta_pv = tid < rows_valid ? g.sorted_ids[m0 + tid] : static_cast<int32_t>(g.num_valid);
  } else if constexpr (kMetaSa) {
    if (tid < BM) meta_sav = g.sa[m0 + tid < g.M ? m0 + tid : g.M - 1];
  }
  const int64_t a_base_row = Rows::kGrouped ? 0 : m0;
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      scalar_ptr(const_cast<int8_t*>(g.A + a_base_row * g.lda)), 0, 0x7fffffff, kBufferFlags);
  static_assert(kAct < 0 || epi_bf16_out(EPI),
                "fused activation: bf16 with the staged epilogue (the host sets staged_out)");
  constexpr int kHalfN = BN / 2;
  const int64_t half = g.N / 2;  // kAct: rows of each of the gate and up halves
  // weight row of tile row r (kAct: gate rows then the matching up rows)
  auto w_row_of = [&](int r) -> int64_t {
    if constexpr (kAct >= 0) {
      const int64_t a = n0 + (r < kHalfN ? r : r - kHalfN);
      const int64_t ac = a < half ? a : half - 1;
      return r < kHalfN ? ac : half + ac;
    } else {
      return n0 + r < g.N ? n0 + r : g.N - 1;
    }
  };
  const int64_t w_base_row = kAct >= 0 ? 0 : n0;
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      scalar_ptr(const_cast<int8_t*>(W + w_base_row * g.K)), 0, 0x7fffffff, kBufferFlags);
  uint32_t a_doff[kLA], w_doff[kLB];
#pragma unroll
  for (int j = 0; j < kLA; ++j) {
    const int unit = (j * kWaves + wave) * 64 + lane, row = unit / kChunks;
    const int c = (unit % kChunks) ^ swz_f<BK>(row);
    int64_t arow;
    bool a_live = true;  // false: the DMA reads past the buffer range (zeros, no traffic)
    if constexpr (Rows::kGrouped) {
      const int32_t p = row < rows_valid ? g.sorted_ids[m0 + row] : static_cast<int32_t>(g.num_valid);
      a_live = p < g.num_valid;
      arow = a_live ? p / g.top_k : 0;
    } else {
      arow = m0 + row < g.M ? m0 + row : g.M - 1;
    }
    a_doff[j] = a_live ? static_cast<uint32_t>((arow - a_base_row) * g.lda + 16 * c) : 0x80000000u;
  }
  if constexpr (kMeta) {
    if (tid < BM && meta_pv < g.num_valid) {
      meta_sav = g.sa[meta_pv / g.top_k];
      if (g.topk_w) meta_rtv = g.topk_w[meta_pv];
    }
  }
  if constexpr (kMetaSa) {
    if (tid < BN) {
      const int64_t nc = w_row_of(tid);
      meta_swv = sw[nc];
      if (!Rows::kGrouped && g.bias) meta_bv = bf16_to_f32(g.bias[nc]);
    }
  }
#pragma unroll
  for (int j = 0; j < kLB; ++j) {
    const int unit = (j * kWaves + wave) * 64 + lane, row = unit / kChunks;
    const int c = (unit % kChunks) ^ swz_f<BK>(row);
    const int64_t wrow = w_row_of(row);
    w_doff[j] = static_cast<uint32_t>((wrow - w_base_row) * g.K + 16 * c);
  }
  const int nk = kt_end - kt_begin;
  // LDS slots of stage kt: A and W side by side in one ring, or (kBLead)
  // the A ring followed by the W ring
  auto a_slot = [&](int kt) -> unsigned char* {
    return lds + (kBLead ? (kt % NSTAGE) * kStageA : (kt % NSTAGE) * kStage);
  };
  auto b_slot = [&](int kt) -> unsigned char* {
    if constexpr (kBLead > 0) return lds + NSTAGE * kStageA + (kt % kBSlots) * kStageB;
    else return lds + (kt % NSTAGE) * kStage + kStageA;
  };
  auto issue_a = [&](int kt) {
    unsigned char* base = a_slot(kt);
    const int k0 = (kt_begin + kt) * BK;
#pragma unroll
    for (int j = 0; j < kLA; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(base + (j * kWaves + wave) * 1024), 16,
                                               a_doff[j], k0, 0, 0);
  };
  auto issue_b = [&](int kt) {
    unsigned char* base = b_slot(kt);
    const int k0 = (kt_begin + kt) * BK;
#pragma unroll
    for (int j = 0; j < kLB; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(base + (j * kWaves + wave) * 1024), 16,
                                               w_doff[j], k0, 0, kWAux);
  };
  auto issue = [&](int kt) {
    issue_a(kt);
    issue_b(kt);
  };

  const int frow = lane & (MF - 1), fgrp = lane / MF;
  int a_off[kFM], b_off[kFN];  // tile rows of this lane's fragment rows
#pragma unroll
  for (int i = 0; i < kFM; ++i) a_off[i] = wm * kWaveM + MF * i + frow;
#pragma unroll
  for (int j = 0; j < kFN; ++j) b_off[j] = wn * kWaveN + MF * j + frow;
  v4i fa[2][kFM], fb[2][kFN];
  // fragments of k-substep ks (Mf::kK K bytes) of stage kt into register set ks & 1
  auto read_frags = [&](int kt, int ks) {
    const unsigned char* la = lds + (kt % NSTAGE) * kStage;
    const unsigned char* lb = la + kStageA;
    const int ch = Mf::kGroups * ks + fgrp;
#pragma unroll
    for (int i = 0; i < kFM; ++i) fa[ks & 1][i] = *reinterpret_cast<const v4i*>(la + swz_lds<BK>(a_off[i], ch));
#pragma unroll
    for (int j = 0; j < kFN; ++j) fb[ks & 1][j] = *reinterpret_cast<const v4i*>(lb + swz_lds<BK>(b_off[j], ch));
  };

  Acc acc[kFM][kFN];
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j) acc[i][j] = Acc{0};
  // Run tiles: the sorted positions of a run are real pairs up to the
  // expert's padding, which ends it, so the real rows of this wave's range
  // form a prefix of length live_w; 32-row fragments past it (padding or
  // past the run) have no MFMA work.  live_w is wave-uniform (ballot).
  int live_w = kWaveM;
  if constexpr (Rows::kRuns) {
    live_w = 0;
#pragma unroll
    for (int h = 0; h < kWaveM; h += 64) {
      const int r = wm * kWaveM + h + lane;
      const bool real = h + lane < kWaveM && r < rows_valid && g.sorted_ids[m0 + r] < g.num_valid;
      live_w += __popcll(__ballot(real));
    }
    live_w = __builtin_amdgcn_readfirstlane(live_w);
  }
  auto mfmas = [&](int set) {
#pragma unroll
    for (int i = 0; i < kFM; ++i) {
      if (Rows::kRuns && MF * i >= live_w) break;
#pragma unroll
      for (int j = 0; j < kFN; ++j) acc[i][j] = Mf::mma(fa[set][i], fb[set][j], acc[i][j]);
    }
  };
  constexpr int kSub = BK / Mf::kK;  // k-substeps per stage (2 or 4)

  // prologue: stages 0 .. NSTAGE-1 in flight (kBLead: A0 W0 W1 A1 W2), stage
  // 0 landed, its fragments read
  if constexpr (kBLead > 0) {
    issue(0);
#pragma unroll
    for (int s = 1; s < NSTAGE; ++s)
      if (s < nk) {
        issue_b(s);
        issue_a(s);
      }
    if (NSTAGE < nk) issue_b(NSTAGE);
  } else {
#pragma unroll
    for (int s = 0; s < NSTAGE; ++s)
      if (s < nk) issue(s);
  }
  if constexpr (kMeta) {
    if (tid < BM) {  // visible to every wave after the barriers of the main loop
      const bool ok = meta_pv < g.num_valid;
      meta_p[tid] = ok ? meta_pv : -1;
      meta_sa[tid] = ok ? meta_sav : 0.0f;
      meta_rt[tid] = ok ? meta_rtv : 0.0f;
    }
  } else if constexpr (kMetaSa && !kTabInRing) {
    if (tid < BM) meta_sa[tid] = meta_sav;
  }
  if constexpr (kMetaSa && !kTabInRing) {
    if (tid < BN) {
      meta_sw[tid] = meta_swv;
      if constexpr (!Rows::kGrouped) meta_bias[tid] = meta_bv;
    }
  }
  if constexpr (kBLead > 0) {
    // stage 0 (A0 W0) landed; W 1..NSTAGE and A 1..NSTAGE-1 may be in flight
    wait_lead<kLA, kLB, NSTAGE, NSTAGE - 1>(nk - 1 < NSTAGE ? nk - 1 : NSTAGE);
  } else {
    wait_stages<kL, NSTAGE - 1>(nk - 1 < NSTAGE - 1 ? nk - 1 : NSTAGE - 1);
  }
  raw_barrier();
  if constexpr (MF == 16) {
    // Two 64-byte substeps per stage.  The B fragments roll: fragment j of
    // the next substep is read as soon as the kFM MFMAs of column block j
    // have been issued.  The A fragments are double-buffered by substep
    // (2 kFM + kFN registers of 16 bytes instead of 2 (kFM + kFN)), or,
    // where that would not fit beside the accumulators (kASets == 1), held
    // once and re-read during the last column block, each right after its
    // last MFMA.  The next stage's fragments are read after the barrier
    // that follows its landing, in the middle of the stage's substep-1
    // MFMAs.
    static_assert(kSub == 2, "16x16x64 ring: 128-byte stages");
    constexpr int kASets = 4 * (2 * kFM + kFN) + 4 * kFM * kFN > 200 ? 1 : 2;
    auto read_a1 = [&](int kt, int ks, int set, int i) {
      const unsigned char* la = a_slot(kt);
      fa[set][i] = *reinterpret_cast<const v4i*>(la + swz_lds<BK>(a_off[i], 2 * fgrp + ks));
    };
    auto read_a = [&](int kt, int ks, int set) {
#pragma unroll
      for (int i = 0; i < kFM; ++i) read_a1(kt, ks, set, i);
    };
    auto read_b = [&](int kt, int ks, int j) {
      const unsigned char* lb = b_slot(kt);
      fb[0][j] = *reinterpret_cast<const v4i*>(lb + swz_lds<BK>(b_off[j], 2 * fgrp + ks));
    };
    // MFMAs of column block j on A set `set`; with one A set, the last
    // column block re-reads A fragment i of substep (nkt, nks) after its
    // MFMA (nkt < 0: no re-read)
    auto col = [&](int set, int j, int nkt, int nks) {
#pragma unroll
      for (int i = 0; i < kFM; ++i) {
        if (Rows::kRuns && MF * i >= live_w) break;
        acc[i][j] = Mf::mma(fa[kASets == 1 ? 0 : set][i], fb[0][j], acc[i][j]);
        if (kASets == 1 && j == kFN - 1 && nkt >= 0) read_a1(nkt, nks, 0, i);
      }
    };
    read_a(0, 0, 0);
#pragma unroll
    for (int j = 0; j < kFN; ++j) read_b(0, 0, j);
    for (int kt = 0; kt + 1 < nk; ++kt) {
      if constexpr (kASets == 2) read_a(kt, 1, 1);
#pragma unroll
      for (int j = 0; j < kFN; ++j) {
        col(0, j, kt, 1);
        read_b(kt, 1, j);
      }
      if constexpr (kBLead > 0) {
        // issued after stage kt+1's A: W kt+2 .. kt+NSTAGE, A kt+2 .. kt+NSTAGE-1
        const int r = nk - 2 - kt;
        wait_lead<kLA, kLB, NSTAGE - 1, NSTAGE - 2>(r < NSTAGE - 1 ? r : NSTAGE - 1);
      } else {
        const int later = nk - 2 - kt;  // stages after kt+1 already issued
        wait_stages<kL, NSTAGE - 2>(later < NSTAGE - 2 ? later : NSTAGE - 2);
      }
      raw_barrier();
      if constexpr (kASets == 2) read_a(kt + 1, 0, 0);
#pragma unroll
      for (int j = 0; j < kFN; ++j) {
        col(1, j, kt + 1, 0);
        read_b(kt + 1, 0, j);
      }
      if constexpr (kBLead > 0) {
        if (kt + NSTAGE < nk) issue_a(kt + NSTAGE);
        if (kt + NSTAGE + 1 < nk) issue_b(kt + NSTAGE + 1);
      } else {
        if (kt + NSTAGE < nk) issue(kt + NSTAGE);
      }
    }
    if constexpr (kASets == 2) read_a(nk - 1, 1, 1);
#pragma unroll
    for (int j = 0; j < kFN; ++j) {
      col(0, j, nk - 1, 1);
      read_b(nk - 1, 1, j);
    }
#pragma unroll
    for (int j = 0; j < kFN; ++j) col(1, j, -1, 0);
  } else {
  read_frags(0, 0);
  read_frags(0, 1);

  // Steady state for stage kt: the fragments of substeps 0 and 1 are in
  // registers on entry.  Substep s runs its MFMAs while the fragments of
  // substep s+2 load; the last substep pairs overlap the next stage's first
  // fragments, which need that stage landed (vmcnt) and, since its LDS
  // buffer is then recycled, every wave past its reads of stage kt.
  for (int kt = 0; kt + 1 < nk; ++kt) {
#pragma unroll
    for (int s = 0; s + 2 < kSub; ++s) {
      mfmas(s & 1);
      read_frags(kt, s + 2);
    }
    mfmas(kSub & 1);  // substep kSub-2
    const int later = nk - 2 - kt;  // stages after kt+1 already issued
    wait_stages<kL, NSTAGE - 2>(later < NSTAGE - 2 ? later : NSTAGE - 2);
    raw_barrier();
    // MFMAs first after the barrier: the refill DMA of the freed buffer is
    // issued behind them so that the matrix pipe restarts at once
    read_frags(kt + 1, 0);
    mfmas((kSub - 1) & 1);  // substep kSub-1
    if (kt + NSTAGE < nk) issue(kt + NSTAGE);
    read_frags(kt + 1, 1);
  }
#pragma unroll
  for (int s = 0; s + 2 < kSub; ++s) {
    mfmas(s & 1);
    read_frags(nk - 1, s + 2);
  }
  mfmas(kSub & 1);
  mfmas((kSub - 1) & 1);
  }  // MF == 32

  if constexpr (!Rows::kGrouped) {
    if (split_unit >= 0) {  // split-tail unit: raw int32 partial tile, rows/cols unmasked
      int32_t* pt = g.part + split_unit * (BM * BN);
#pragma unroll
      for (int i = 0; i < kFM; ++i)
#pragma unroll
        for (int v = 0; v < kV; ++v) {
          const int r = wm * kWaveM + MF * i + Mf::row(lane, v);
#pragma unroll
          for (int j = 0; j < kFN; ++j) pt[r * BN + wn * kWaveN + MF * j + frow] = acc[i][j][v];
        }
      return;
    }
  }

  // ---- staged bf16 epilogue: the tile is assembled in the (now idle) LDS
  // ring and written with 16-byte row stores.  Lanes 2k / 2k+1 swap one
  // value so that each writes two adjacent columns of one row as a 32-bit
  // word; the staging layout moves the 16-byte chunk c of row r to
  // spos(r, c) (an XOR with sf(r) when a row holds a multiple of 16 chunks,
  // else a rotation by it), which keeps both the word writes (rows R, R+1,
  // R+4, R+5 per instruction) and the 16-byte row reads on distinct LDS
  // banks.  A tile whose bf16 image exceeds the ring is staged in row
  // passes of whole wave rows (kStagePasses).
  constexpr int kRing = kRingBytes;
  constexpr int kStagePasses = (BM * BN * 2 + kRing - 1) / kRing;
  constexpr int kPassRows = BM / kStagePasses;
  constexpr bool kStaged = epi_bf16_out(EPI) && BN >= 128 && kStagePasses <= 2 &&
                           kPassRows * kStagePasses == BM && kPassRows % kWaveM == 0;
  static_assert(kAct < 0 || (kStaged && kStagePasses == 1), "fused activation: one staging pass");
  if constexpr (kStaged) {
    if (g.staged_out) {
      if constexpr (kTabInRing) {  // every wave past its last fragment read; then the tables
        __syncthreads();
        if (tid < BM) meta_sa[tid] = meta_sav;
        if (tid < BN) {
          meta_sw[tid] = meta_swv;
          meta_bias[tid] = meta_bv;
        }
        __syncthreads();
      }
      constexpr int kRowBytes = BN * 2;
      constexpr int kChunksRow = BN / 8;
      // MF = 32: one word-store instruction covers rows R, R+1, R+4, R+5 (64
      // bytes each); MF = 16: rows R, R+1, R+4, R+5, R+8, R+9, R+12, R+13
      // (32 bytes each).  sf spreads them over the 256 bytes of the banks.
      auto sf = [](int r) {
        if constexpr (MF == 32) return 4 * ((r & 1) | (((r >> 2) & 1) << 1));
        else return 2 * ((r & 1) | (((r >> 2) & 3) << 1));
      };
      auto spos = [&](int r, int c) {
        if constexpr (kChunksRow % 16 == 0) {
          return c ^ sf(r);
        } else {
          const int q = c + sf(r);
          return q >= kChunksRow ? q - kChunksRow : q;
        }
      };
      const bool odd = (lane & 1) != 0;
      constexpr int kThreads = 64 * kWaves;
      // The lane's column scales (and bias) are read from the LDS tables
      // into registers once, its row scales once per fragment row group:
      // read inside the staging loop, every table read would follow a
      // staging store to LDS that the compiler cannot prove disjoint from
      // the tables, and each output pair would wait on its own LDS round
      // trip.  The bias and routed-weight choices are made outside the loop.
      float r_sw[kFN], r_bias[kFN];
#pragma unroll
      for (int j = 0; j < kFN; ++j) {
        const int c = wn * kWaveN + MF * j + frow;
        r_sw[j] = meta_sw[c];
        r_bias[j] = 0.0f;
        if constexpr (!Rows::kGrouped) r_bias[j] = meta_bias[c];
      }
      auto stage_rows = [&](auto bias_tag, auto routed_tag, int prow0) {
        constexpr bool kBias = decltype(bias_tag)::value, kRouted = decltype(routed_tag)::value;
#pragma unroll
        for (int i = 0; i < kFM; ++i) {
          float r_sa[kV], r_rt[kV];
#pragma unroll
          for (int v = 0; v < kV; ++v) {
            const int r = wm * kWaveM + MF * i + Mf::row(lane, v);
            r_sa[v] = meta_sa[r];
            if constexpr (kRouted) r_rt[v] = meta_rt[r];
            else r_rt[v] = 1.0f;
          }
#pragma unroll
          for (int vp = 0; vp < kV / 2; ++vp) {
            const int v0 = 2 * vp;  // rows v0, v0 + 1 of this lane's kV (adjacent rows)
            const int r0 = wm * kWaveM + MF * i + Mf::row(lane, v0);
#pragma unroll
            for (int j = 0; j < kFN; ++j) {
              const int c = wn * kWaveN + MF * j + frow;
              float t0 = epi_scale(acc[i][j][v0], r_sa[v0], r_sw[j]);
              float t1 = epi_scale(acc[i][j][v0 + 1], r_sa[v0 + 1], r_sw[j]);
              if constexpr (kBias) {
                t0 = t0 + r_bias[j];
                t1 = t1 + r_bias[j];
              }
              if constexpr (kRouted) {
                t0 = t0 * r_rt[v0];
                t1 = t1 * r_rt[v0 + 1];
              }
              // even lane: row r0, columns (c, c+1); odd lane: row r0+1, columns (c-1, c)
              const float send = odd ? t0 : t1;
              const float got = __builtin_bit_cast(
                  float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, false));
              typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
              const bf16x2 pr = odd ? bf16x2{(__bf16)got, (__bf16)t1} : bf16x2{(__bf16)t0, (__bf16)got};
              const int rr = (odd ? r0 + 1 : r0) - prow0, cc = odd ? c - 1 : c;
              *reinterpret_cast<bf16x2*>(lds + rr * kRowBytes + (spos(rr, cc >> 3) << 4) + (cc & 7) * 2) = pr;
            }
          }
        }
      };
      using kYes = std::integral_constant<bool, true>;
      using kNo = std::integral_constant<bool, false>;
#pragma unroll
      for (int pass = 0; pass < kStagePasses; ++pass) {
        const int prow0 = pass * kPassRows;
        // every wave is past its last LDS fragment read (pass 0) or its
        // reads of the previous pass's rows
        __syncthreads();
        if (wm * kWaveM >= prow0 && wm * kWaveM < prow0 + kPassRows) {  // wave-uniform
          if constexpr (Rows::kGrouped) {
            if (g.topk_w) stage_rows(kNo{}, kYes{}, prow0);
            else stage_rows(kNo{}, kNo{}, prow0);
          } else {
            if (g.bias) stage_rows(kYes{}, kNo{}, prow0);
            else stage_rows(kNo{}, kNo{}, prow0);
          }
        }
        __syncthreads();
        if constexpr (kAct >= 0) {  // act chunk ch of row r: gate chunk ch, up chunk ch + BN/16
          constexpr int kActChunks = BN / 16;
#pragma unroll
          for (int q0 = 0; q0 < BM * kActChunks; q0 += kThreads) {
            const int q = q0 + tid, r = q / kActChunks, ch = q % kActChunks;
            int64_t orow;
            if constexpr (Rows::kGrouped) {
              orow = meta_p[r];
            } else {
              orow = m0 + r < g.M ? m0 + r : -1;
            }
            const int64_t n = n0 + ch * 8;
            if (orow >= 0 && n < half) {
              const v4i gv = *reinterpret_cast<const v4i*>(lds + r * kRowBytes + (spos(r, ch) << 4));
              const v4i uv = *reinterpret_cast<const v4i*>(lds + r * kRowBytes + (spos(r, ch + kActChunks) << 4));
              v4i o;
#pragma unroll
              for (int w = 0; w < 4; ++w) {
                const uint32_t gw = static_cast<uint32_t>(gv[w]), uw = static_cast<uint32_t>(uv[w]);
                const float a0 = act_fn<kAct>(bf16_to_f32(static_cast<uint16_t>(gw & 0xFFFFu))) *
                                 bf16_to_f32(static_cast<uint16_t>(uw & 0xFFFFu));
                const float a1 = act_fn<kAct>(bf16_to_f32(static_cast<uint16_t>(gw >> 16))) *
                                 bf16_to_f32(static_cast<uint16_t>(uw >> 16));
                o[w] = static_cast<int>(static_cast<uint32_t>(f32_to_bf16(a0)) |
                                        (static_cast<uint32_t>(f32_to_bf16(a1)) << 16));
              }
              __builtin_nontemporal_store(o, reinterpret_cast<v4i*>(static_cast<uint16_t*>(g.out) + orow * g.ldo + n));
            }
          }
          return;
        } else {
#pragma unroll
          for (int q0 = 0; q0 < kPassRows * kChunksRow; q0 += kThreads) {
            const int q = q0 + tid, r = q / kChunksRow, ch = q % kChunksRow;
            if (q < kPassRows * kChunksRow) {
              int64_t orow;
              if constexpr (Rows::kGrouped) {
                orow = meta_p[prow0 + r];
              } else {
                orow = m0 + prow0 + r < g.M ? m0 + prow0 + r : -1;
              }
              const int64_t n = n0 + ch * 8;
              if (orow >= 0 && n < g.N) {
                const v4i d = *reinterpret_cast<const v4i*>(lds + r * kRowBytes + (spos(r, ch) << 4));
                store_out16(static_cast<uint16_t*>(g.out) + orow * g.ldo + n, d);
              }
            }
          }
        }
      }
      return;
    }
  }

  // ---- epilogue: lane holds column frow of each MF x MF fragment
#pragma unroll
  for (int i = 0; i < kFM; ++i) {
#pragma unroll
    for (int v = 0; v < kV; ++v) {
      const int r = wm * kWaveM + MF * i + Mf::row(lane, v);
      int64_t orow, arow;
      bool rvalid;
      float routed = 1.0f;
      if constexpr (Rows::kGrouped) {
        const int32_t p = r < rows_valid ? g.sorted_ids[m0 + r] : static_cast<int32_t>(g.num_valid);
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
      const float sa = epi_bf16_out(EPI) ? g.sa[arow] : 0.0f;
#pragma unroll
      for (int j = 0; j < kFN; ++j) {
        const int64_t n = n0 + wn * kWaveN + MF * j + frow;
        if (n >= g.N) continue;
        const int32_t a = acc[i][j][v];
        if constexpr (epi_bf16_out(EPI)) {
          static_cast<uint16_t*>(g.out)[orow * g.ldo + n] =
              epi_bf16(a, sa, sw[n], g.bias, n, routed, g.topk_w != nullptr);
        } else {
          static_cast<int32_t*>(g.out)[orow * g.ldo + n] = a;
        }
      }
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// Work unit b of a dense ring grid: blocks [0, full_tiles) own whole tiles
// (XCD-contiguous), block full_tiles + u the K range u % tail_split of
// tail tile u / tail_split (an int32 partial tile); without a split, block
// b owns tile tile_of_block(b).
// kAct: a tile of BN weight rows covers BN / 2 output (activation) columns.
template <int BM, int BN, int BK, bool kAct = false>
__device__ __forceinline__ TileJob dense_tile_job(const GemmArgs& g, uint32_t b) {
  const uint32_t tm = static_cast<uint32_t>((g.M + BM - 1) / BM), tn = static_cast<uint32_t>((g.N + BN - 1) / BN);
  int64_t pm, pn, split_unit = -1;
  int kt_begin = 0, kt_end = static_cast<int>(g.K / BK);
  if (g.tail_split > 1) {
    const uint32_t full = static_cast<uint32_t>(g.full_tiles), ts = static_cast<uint32_t>(g.tail_split);
    if (b < full) {
      tile_of_index(xcd_tile_index_rot(b, full), tm, tn, pm, pn);
    } else {
      const uint32_t u = b - full, tile = u / ts, sp = u - tile * ts, nkt = static_cast<uint32_t>(g.K / BK);
      split_unit = u;
      tile_of_index(full + tile, tm, tn, pm, pn);
      kt_begin = static_cast<int>(nkt * sp / ts);
      kt_end = static_cast<int>(nkt * (sp + 1) / ts);
    }
  } else {
    tile_of_block(b, tm, tn, pm, pn);
  }
  return TileJob{pm * BM, pn * (kAct ? BN / 2 : BN), g.W, g.sw, kt_begin, kt_end, BM, split_unit};
}

template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI, class Rows, int kWAux = 0, int MF = 32,
          int kAct = -1, int kBLead = 0>
__global__ __launch_bounds__(64 * WM * WN) void tile3_gemm_kernel(GemmArgs g) {
  // The body uses device-only builtins (LDS DMA, raw waitcnt); the host
  // pass only needs the launch stub.
#if defined(__HIP_DEVICE_COMPILE__)
  extern __shared__ __align__(16) unsigned char lds[];
  static_assert(!Rows::kRuns, "run tiles are walked by grouped_persist_kernel");
  static_assert(kAct < 0 || !Rows::kGrouped, "grouped fused activation: grouped_persist_kernel");
  if constexpr (Rows::kGrouped) {
    // grouped grid: x = N tile, y = alignment block of BM sorted rows (an
    // XCD-contiguous walk of the (block, N tile) pairs measured slower at
    // 256 and 1024 tokens)
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN, m0 = static_cast<int64_t>(blockIdx.y) * BM;
    if (m0 >= static_cast<int64_t>(*g.num_post_pad)) return;
    const int e = g.expert_ids[blockIdx.y];
    if (e < 0 || e >= g.num_experts) return;
    const TileJob job{m0, n0, g.W + static_cast<int64_t>(e) * g.N * g.K, g.sw + static_cast<int64_t>(e) * g.N,
                      0, static_cast<int>(g.K / BK), BM, -1};
    tile3_run<BM, BN, BK, WM, WN, NSTAGE, EPI, Rows, -1, 0, MF>(g, lds, job);
  } else {
    tile3_run<BM, BN, BK, WM, WN, NSTAGE, EPI, Rows, kAct, kWAux, MF, kBLead>(
        g, lds, dense_tile_job<BM, BN, BK, (kAct >= 0)>(g, blockIdx.x));
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// ------------------------------------------------------------------------
// Persistent grouped GEMM (fused-MoE, 64/128-row alignment blocks).
// ------------------------------------------------------------------------
// An expert's alignment blocks form ceil(blocks / per_tile) chunks of
// near-equal size (per_tile = BM / align_bsz).  Work item = (expert with
// at least one block, BN-column tile), the block running all its chunks in
// turn (re-reading the weight tile it has just streamed), or, with
// kChunkItems, (expert, column tile, chunk), the chunks of one weight tile
// adjacent in the list and so running side by side on one XCD.
// Every block derives the item list from expert_ids on its own (no
// workspace, no extra launch): expert e's blocks are the run
// [run_start[e], run_start[e + 1]) (expert_ids is non-decreasing over the
// used blocks).  Items are numbered expert-major, and each XCD's blocks
// (block b runs on XCD b % 8) deal one contiguous range of them, so all
// column tiles of an expert share its gathered rows in one L2.  Each block
// walks its items with a static stride: no queue, no inter-block waiting.

__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}

// Run tables of a grouped walk, built by every block from expert_ids:
// run_start[e] = first alignment block of expert e (run_start[E] = blocks
// in use) and act_base[e] = units (experts with blocks, or chunks of up to
// per_tile blocks with kChunkItems) before e; returns the unit total.
// Ends with a __syncthreads: the tables are visible to the whole block.
template <int kThreads, bool kChunkItems>
__device__ __forceinline__ int build_run_tables(const GemmArgs& g, int per_tile, int* run_start, int* act_base,
                                                int* wave_tot) {
  constexpr int kWaves = kThreads / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = g.num_experts, ab = g.align_bsz;
  const int used = *g.num_post_pad / ab;  // alignment blocks in use
  // run starts: the block b where expert_ids steps from p to c starts the
  // runs of experts p+1 .. c (a virtual block `used` starts every later one)
  for (int b = tid; b <= used; b += kThreads) {
    const int prev = b == 0 ? -1 : g.expert_ids[b - 1];
    int cur = b == used ? E : g.expert_ids[b];
    if (cur > E) cur = E;
    for (int e = prev + 1; e <= cur; ++e) run_start[e] = b;
  }
  __syncthreads();
  // exclusive prefix over experts of their unit count: 1 if the expert has
  // blocks (expert items), or its chunk count (chunk items); two-level scan
  int carry = 0;
  for (int e0 = 0; e0 < E; e0 += kThreads) {
    const int e = e0 + tid;
    const int len = e < E ? run_start[e + 1] - run_start[e] : 0;
    const int act = kChunkItems ? (len + per_tile - 1) / per_tile : (len > 0 ? 1 : 0);
    const int incl = wave_incl_scan(act);
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int before = carry;
    for (int w = 0; w < wave; ++w) before += wave_tot[w];
    if (e < E) act_base[e] = before + incl - act;
    int tot = 0;
    for (int w = 0; w < kWaves; ++w) tot += wave_tot[w];
    carry += tot;
    __syncthreads();
  }
  if (tid == 0) act_base[E] = carry;
  __syncthreads();
  return carry;
}

template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI, bool kChunkItems, int kPerCu,
          int kAct = -1, int MF = 32>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(kPerCu * WM * WN / 4)))
void grouped_persist_kernel(GemmArgs g) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int kThreads = 64 * WM * WN, kWaves = WM * WN;
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int run_start[kPersistMaxSlots + 1];  // first alignment block of expert e
  __shared__ int act_base[kPersistMaxSlots + 1];   // units (experts or chunks) before e
  __shared__ int wave_tot[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = g.num_experts, ab = g.align_bsz, per_tile = BM / ab;
  const int carry = build_run_tables<kThreads, kChunkItems>(g, per_tile, run_start, act_base, wave_tot);
  // column tiles: BN output columns, or BN / 2 activation columns (kAct)
  constexpr int kTileCols = kAct >= 0 ? BN / 2 : BN;
  const int64_t out_cols = kAct >= 0 ? g.N / 2 : g.N;
  const int tn = static_cast<int>((out_cols + kTileCols - 1) / kTileCols);
  const int total = carry * tn;

  // this block's share: XCD x deals items [begin, begin + count)
  const int G = gridDim.x, xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds, per_xcd = G / kXcds;
  const int base = total / kXcds, rem = total % kXcds;
  const int begin = xcd * base + (xcd < rem ? xcd : rem), count = base + (xcd < rem ? 1 : 0);
  for (int j = local; j < count; j += per_xcd) {
    const int item = begin + j;
    const int a = item / tn;  // expert items: the active-expert index
    // the expert: last e with act_base[e] * tn <= item (act_base[e + 1] * tn > item)
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (act_base[mid] * tn <= item) lo = mid; else hi = mid - 1;
    }
    const int e = __builtin_amdgcn_readfirstlane(lo);
    const int b_first = __builtin_amdgcn_readfirstlane(run_start[e]);
    const int nblocks = __builtin_amdgcn_readfirstlane(run_start[e + 1]) - b_first;
    const int nch = (nblocks + per_tile - 1) / per_tile;
    int n_tile, c_lo, c_hi;
    if constexpr (kChunkItems) {  // item = (expert, column tile, chunk), chunk fastest
      const int off = item - act_base[e] * tn;
      n_tile = __builtin_amdgcn_readfirstlane(off / nch);
      c_lo = __builtin_amdgcn_readfirstlane(off % nch);
      c_hi = c_lo + 1;
    } else {  // item = (expert, column tile): all chunks in turn
      n_tile = __builtin_amdgcn_readfirstlane(item - a * tn);
      c_lo = 0;
      c_hi = nch;
    }
    for (int c = c_lo; c < c_hi; ++c) {
      const int c0 = b_first + c * nblocks / nch, c1 = b_first + (c + 1) * nblocks / nch;
      TileJob job{static_cast<int64_t>(c0) * ab,
                  static_cast<int64_t>(n_tile) * kTileCols,
                  g.W + static_cast<int64_t>(e) * g.N * g.K,
                  g.sw + static_cast<int64_t>(e) * g.N,
                  0,
                  static_cast<int>(g.K / BK),
                  (c1 - c0) * ab,
                  -1};
      __syncthreads();  // the previous tile's LDS staging has been read out
      tile3_run<BM, BN, BK, WM, WN, NSTAGE, EPI, SortedRunRows, kAct, 0, MF>(g, lds, job);
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// ------------------------------------------------------------------------
// Dense small-M core: weight streaming with in-block split-K
// ------------------------------------------------------------------------
// Block = WAVES waves over the same RG*16 weight rows; wave w accumulates
// the 64-byte K steps [w*S/WAVES, (w+1)*S/WAVES) of all of them, then the
// WAVES partial accumulators are summed with LDS integer atomics (exact and
// order-free) and the epilogue runs once.  No global atomics, fences or
// workspace.  Per 64-K step lane (r16, grp) loads 16 bytes of each of its
// RG weight rows and of each of its TG token rows (tokens read straight from
// L2: the int8 activation matrix is small), then issues RG*TG
// v_mfma_i32_16x16x64_i8 with the weight rows as the MFMA rows.  U steps
// of loads are issued before their MFMAs to keep bytes in flight.
template <int RG, int TG, int WAVES, int U, int EPI>
__global__ __launch_bounds__(64 * WAVES) void decode_gemm_kernel(GemmArgs g) {
  constexpr int kAcc = RG * TG * 4;  // int32 accumulators per lane
  __shared__ int32_t red[kAcc][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < kAcc * 64; e += 64 * WAVES) (&red[0][0])[e] = 0;
  __syncthreads();
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * RG);
  const int64_t steps = (g.K + 63) / 64;
  const int64_t s_begin = steps * wave / WAVES, s_end = steps * (wave + 1) / WAVES;

  const int8_t* wp[RG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const int64_t n = n0 + 16 * rg + r16;
    wp[rg] = g.W + (n < g.N ? n : g.N - 1) * g.K + 16 * grp;
  }
  const int8_t* xp[TG];
  bool xok[TG];
#pragma unroll
  for (int tg = 0; tg < TG; ++tg) {
    const int64_t m = 16 * tg + r16;
    xok[tg] = m < g.M;
    xp[tg] = g.A + (xok[tg] ? m : 0) * g.lda + 16 * grp;
  }
  v4i acc[RG][TG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg)
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) acc[rg][tg] = v4i{0};

  for (int64_t s0 = s_begin; s0 < s_end; s0 += U) {
    v4i wv[U][RG], xv[U][TG];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = (s0 + u) * 64 + 16 * grp;
      const bool in = (s0 + u < s_end) && (k < g.K);
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
        wv[u][rg] = in ? *reinterpret_cast<const v4i*>(wp[rg] + (s0 + u) * 64) : v4i{0};
#pragma unroll
      for (int tg = 0; tg < TG; ++tg)
        xv[u][tg] = (in && xok[tg]) ? *reinterpret_cast<const v4i*>(xp[tg] + (s0 + u) * 64) : v4i{0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int tg = 0; tg < TG; ++tg)
          acc[rg][tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[u][rg], xv[u][tg], acc[rg][tg], 0, 0, 0);
  }

#pragma unroll
  for (int rg = 0; rg < RG; ++rg)
#pragma unroll
    for (int tg = 0; tg < TG; ++tg)
#pragma unroll
      for (int v = 0; v < 4; ++v) atomicAdd(&red[(rg * TG + tg) * 4 + v][lane], acc[rg][tg][v]);
  __syncthreads();
  // every thread of the block finalises (accumulator index j, lane l) pairs
  for (int e = tid; e < kAcc * 64; e += 64 * WAVES) {
    const int j = e >> 6, l = e & 63;
    const int32_t a = red[j][l];
    const int rg = j / (TG * 4), tg = (j / 4) % TG, v = j & 3;
    const int64_t n = n0 + 16 * rg + 4 * (l >> 4) + v;
    const int64_t m = 16 * tg + (l & 15);
    if (n >= g.N || m >= g.M) continue;
    if constexpr (EPI == kEpiBf16)
      static_cast<uint16_t*>(g.out)[m * g.ldo + n] = epi_bf16(a, g.sa[m], g.sw[n], g.bias, n, 1.0f, false);
    else
      static_cast<int32_t*>(g.out)[m * g.ldo + n] = a;
  }
}

// A block of zeros the decode cores read in place of a token row past M (or
// of K bytes past a row end).  Never written: a global (not constant)
// object, so that a select between it and a kernel-argument pointer still
// yields a global-memory load.
__device__ __align__(16) int8_t kZeroChunk[16] = {0};

// ------------------------------------------------------------------------
// Dense small-M core, DMA ring: weights streamed to LDS in row-contiguous
// 256-byte segments
// ------------------------------------------------------------------------
// Block = WAVES waves over 16 weight rows; wave w owns K stages
// [s_begin, s_end) of 256 bytes each and streams them through a private
// ring of D LDS slots (16 rows x 256 B = 4 KB per slot) with
// buffer_load ... lds: one DMA instruction moves 4 rows x 256 contiguous
// bytes (1 KB), so every request covers whole 128-byte lines, and no VGPR
// holds data in flight.  The lane that fills LDS chunk c' of row r fetches
// global chunk c' ^ (r & 15): a fragment read (lane -> row l%16, chunk
// 4*kb + l/16) then touches 16 distinct 16-byte bank groups.  The token
// operand of each stage (16 bytes per lane per 64-byte K block, L1/L2
// resident) is loaded with plain loads into a register ring of the same
// depth, issued right after the stage's DMA, so one vmcnt wait covers both
// and the D-1 later stages stay in flight.  Token rows >= M and K bytes
// past the row end read a block of zeros; weight bytes past a row end read
// the next row (in bounds, multiplied by zero) and rows past N read as
// zeros through the buffer range check.  No barrier inside the loop; the
// waves' int32 partials are summed in LDS as in decode_gemm_kernel.
constexpr int kRingStage = 4096;  // 16 rows x 256 B

template <int TG, int WAVES, int D>
struct DecodeRing {
  static constexpr int kLds = WAVES * D * kRingStage;
};

// s_waitcnt vmcnt(n) (no lgkm wait), n < 64
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// Compile-time unrolled drain of a D-slot ring: slot d waits until at most
// (D-1-d) stages of OPS vector memory ops each remain in flight, then runs.
template <int D, int OPS, int d>
struct RingDrain {
  template <class F>
  __device__ __forceinline__ static void run(F& consume) {
    wait_vmcnt<(D - 1 - d) * OPS>();
    consume(d);
    RingDrain<D, OPS, d + 1>::run(consume);
  }
};
template <int D, int OPS>
struct RingDrain<D, OPS, D> {
  template <class F>
  __device__ __forceinline__ static void run(F&) {}
};

// Dense use: the N weight rows are cut into gridDim.x equal ranges
// (block b owns rows [N b / G, N (b+1) / G), at most 16 RG of them), so a
// grid of a multiple of 256 blocks gives every CU the same bytes to stream
// whatever N is; RG 16-row MFMA groups per block share the token fragments,
// and rows past the block's range read zeros through the buffer range check
// (no traffic) and are not stored.
// Grouped use (SortedRows, alignment blocks of 16 * TG rows): grid y is the
// alignment block; its expert's weights stream through the ring (16 RG rows
// per block), the token rows are gathered through sorted_ids (padding rows
// read zeros), and the epilogue scatters to pair rows with the routed
// weight.
// kXQ (dense, one token group, bf16 output): g.A holds the bf16 activation
// rows [M <= 16, lda elements], quantized inside the block -- the fused
// F.linear of a decode batch.  Each wave loads its K range of the M rows
// (16-element chunks spread over its lanes, all in flight at once) and
// then issues its first D-1 weight stages; it adds its partial row maxima
// into LDS and, after one barrier, quantizes its chunks with the
// quantizer's arithmetic into its last ring slot (the rows int8, row-major;
// M times the range fits one slot), loads its token fragments of every
// stage into registers (at most kXQMaxStages stages per wave) and issues
// the last weight stage into that slot.  Every block quantizes all M rows,
// so the fused form pays off while M K is small (MI355X, N = K = 5120, us,
// fused vs quantizer launch + GEMM: 5 tokens 10.6 vs 11.5, 6 tokens 11.7
// vs 11.5, 8 tokens 12.8 vs 11.9): the host takes it up to kXQMaxElems
// elements of x.  The epilogue takes the row scales from LDS.
constexpr int kXQMaxTokens = 16, kXQMaxStages = 6;
constexpr int64_t kXQMaxElems = 4 * 5120;  // M K
constexpr int kXQChunks = 6;               // 16-element chunks of x per lane, at most

template <int TG, int WAVES, int D, int EPI, class Rows = DenseRows, int RG = 1, bool kXQ = false>
__global__ __launch_bounds__(64 * WAVES) void decode3_gemm_kernel(GemmArgs g) {
#if defined(__HIP_DEVICE_COMPILE__)
  static_assert(!kXQ || (TG == 1 && !Rows::kGrouped && epi_bf16_out(EPI)), "fused quantization: dense bf16, <= 16 rows");
  constexpr int kAcc = RG * TG * 4;
  constexpr int kOps = 4 * RG + (kXQ ? 0 : 4 * TG);  // vector memory ops per stage (DMA + token loads)
  static_assert(D >= 2 && D <= 6 && (D - 1) * kOps < 64, "ring depth");
  static_assert(!Rows::kRuns, "grouped rows: one alignment block per block");
  extern __shared__ __align__(16) unsigned char ring[];
  __shared__ int32_t red[kAcc][64];
  constexpr bool kTopk = std::is_same<Rows, TopkRows>::value;
  static_assert(!kTopk || TG == 1, "router-id rows: one 16-row token group");
  __shared__ int32_t t_pair[kTopk ? 16 : 1];  // router-id rows: the block's pairs
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int8_t* W = g.W;
  const float* sw = g.sw;
  int64_t m0 = 0;  // grouped: first sorted position of the alignment block
  // grouped: pair of row r of token group tg (num_valid for a padding row)
  auto pair_of = [&](int tg, int r) -> int32_t {
    if constexpr (kTopk) return t_pair[r];
    else return g.sorted_ids[m0 + 16 * tg + r];
  };
  if constexpr (kTopk) {
    // wave 0 lists this unit's pairs of the block's expert, in ascending
    // order, by ballots over the router ids
    const int U = g.topk_units;
    const int e = static_cast<int>(blockIdx.y) / U, r0 = 16 * (static_cast<int>(blockIdx.y) % U);
    const int nv = static_cast<int>(g.num_valid);
    if (wave == 0) {
      int before = 0;
      for (int base = 0; base < nv; base += 64) {
        const int p = base + lane;
        const bool hit = p < nv && g.sorted_ids[p] == e;
        const uint64_t m = __ballot(hit);
        const int rank = before + static_cast<int>(__popcll(m & ((uint64_t{1} << lane) - 1))) - r0;
        if (hit && rank >= 0 && rank < 16) t_pair[rank] = p;
        before += static_cast<int>(__popcll(m));
      }
      if (lane < 16 && lane >= before - r0) t_pair[lane] = nv;
    }
    __syncthreads();
    if (t_pair[0] >= nv) return;  // no pair routed here (block-uniform)
    W += static_cast<int64_t>(e) * g.N * g.K;
    sw += static_cast<int64_t>(e) * g.N;
  } else if constexpr (Rows::kGrouped) {
    m0 = static_cast<int64_t>(blockIdx.y) * (16 * TG);
    if (m0 >= static_cast<int64_t>(*g.num_post_pad)) return;
    const int e = g.expert_ids[blockIdx.y];
    if (e < 0 || e >= g.num_experts) return;
    W += static_cast<int64_t>(e) * g.N * g.K;
    sw += static_cast<int64_t>(e) * g.N;
  }
  int64_t n0, rows;
  if constexpr (Rows::kGrouped) {
    n0 = static_cast<int64_t>(blockIdx.x) * (16 * RG);
    rows = g.N - n0 < 16 * RG ? g.N - n0 : 16 * RG;
  } else {
    n0 = g.N * blockIdx.x / gridDim.x;
    rows = g.N * (blockIdx.x + 1) / gridDim.x - n0;
    if (rows <= 0) return;  // more blocks than rows (uniform per block)
  }
  for (int e = tid; e < kAcc * 64; e += 64 * WAVES) (&red[0][0])[e] = 0;
  const int r16 = lane & 15, grp = lane >> 4;
  const int steps = static_cast<int>((g.K + 255) / 256);
  const int s_begin = steps * wave / WAVES, s_end = steps * (wave + 1) / WAVES;
  constexpr int kStage = RG * kRingStage;
  unsigned char* my_ring = ring + wave * (D * kStage);

  // weight DMA: instruction j of a stage fills LDS rows 4j .. 4j+3; lane l
  // fills row 4j + l/16, chunk l%16 from global chunk (l%16) ^ (row & 15)
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      scalar_ptr(const_cast<int8_t*>(W + n0 * g.K)), 0,
      static_cast<int>(rows * g.K), kBufferFlags);
  uint32_t w_off[4 * RG];
#pragma unroll
  for (int j = 0; j < 4 * RG; ++j) {
    const int row = 4 * j + (lane >> 4);
    w_off[j] = static_cast<uint32_t>(row * g.K + 16 * ((lane & 15) ^ (row & 15)));
  }
  // token operand: lane (token r16 of group tg, 16-byte group grp).  The
  // address is chosen by an integer select (no branch) and read through a
  // global-address-space pointer.
  typedef const v4i __attribute__((address_space(1)))* gv4i_ptr;
  const uint64_t zero_addr = reinterpret_cast<uint64_t>(kZeroChunk);
  uint64_t xrow[TG];
  bool mok[TG];
#pragma unroll
  for (int tg = 0; tg < TG; ++tg) {
    int64_t m;
    if constexpr (Rows::kGrouped) {
      const int32_t p = pair_of(tg, r16);
      mok[tg] = p < g.num_valid;
      m = p / g.top_k;
    } else {
      m = 16 * tg + r16;
      mok[tg] = m < g.M;
    }
    xrow[tg] = reinterpret_cast<uint64_t>(g.A + (mok[tg] ? m : 0) * g.lda);
  }
  v4i xr[D][4][TG];  // token chunks of the stages in flight, per ring slot

  // Dense one-wave blocks walk their stages from stage s_begin + n b / G on
  // (wrapping): blocks in lockstep at one K offset put a row stride of a
  // power of two on the same low address bits (MI355X, N 34816, K 8192 at
  // 2 / 3 tokens: 52.3 / 54.6 -> 44.4 / 47.4 us; K 5120 and the K-split
  // configurations, which already walk several offsets per block,
  // unchanged; the grouped walks measured level to 1% slower).
  const int n_w = s_end - s_begin;
  const int s_rot = kXQ || WAVES > 1 || Rows::kGrouped || n_w <= 0
                        ? 0
                        : static_cast<int>(static_cast<int64_t>(n_w) * blockIdx.x / gridDim.x);
  auto issue = [&](int d, int st) {
    unsigned char* slot = my_ring + d * kStage;
    int se = st;  // the K stage that slot d takes (a wave's own stages only)
    if (st < s_end) {
      se = st + s_rot;
      if (se >= s_end) se -= n_w;
    }
    // a padding stage (st >= s_end) reads past the buffer range: zeros, no traffic
    const int soff = st < s_end ? se * 256 : 0x7fff0000;
#pragma unroll
    for (int j = 0; j < 4 * RG; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(slot + j * 1024), 16, w_off[j], soff, 0,
                                               kStreamAux);
    if constexpr (!kXQ) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const int64_t k = static_cast<int64_t>(se) * 256 + 64 * kb + 16 * grp;
        const bool kin = k < g.K;
#pragma unroll
        for (int tg = 0; tg < TG; ++tg) {
          const uint64_t a = (mok[tg] & kin) ? xrow[tg] + static_cast<uint64_t>(k) : zero_addr;
          xr[d][kb][tg] = *reinterpret_cast<gv4i_ptr>(a);
        }
      }
    }
  };
  // epilogue operands of this thread's output elements, fetched before the
  // stream so that the loads (dependent ones for gathered rows) overlap it
  // (output row, or -1; activation scale; column scale; routed weight or
  // bias).  Gathered rows only: their loads depend on sorted_ids (measured on
  // MI355X: 16-token MoE layer 96.8 -> 93.9 us); for dense rows the extra
  // registers cost 1-2% at 8-32 tokens and the epilogue loads directly.
  constexpr bool kPre = Rows::kGrouped;
  constexpr int kEpiPerThread = (kAcc * 64 + 64 * WAVES - 1) / (64 * WAVES);
  int32_t e_orow[kPre ? kEpiPerThread : 1];
  float e_sa[kPre ? kEpiPerThread : 1], e_sw[kPre ? kEpiPerThread : 1], e_x[kPre ? kEpiPerThread : 1];
#pragma unroll
  for (int u = 0; u < (kPre ? kEpiPerThread : 0); ++u) {
    const int e = tid + u * 64 * WAVES;
    const int j = e >> 6, l = e & 63;
    const int tg = (j / 4) % TG, v = j & 3;
    const int nl = 16 * (j / (4 * TG)) + 4 * (l >> 4) + v;  // row within the block's range
    const int64_t n = n0 + nl;
    e_orow[u] = -1;
    e_sa[u] = 0.0f;
    e_sw[u] = 0.0f;
    e_x[u] = 0.0f;
    if (e >= kAcc * 64 || nl >= rows) continue;
    int32_t arow;
    if constexpr (Rows::kGrouped) {
      const int32_t p = pair_of(tg, l & 15);
      if (p >= g.num_valid) continue;
      e_orow[u] = p;
      arow = p / g.top_k;
      if (g.topk_w) e_x[u] = g.topk_w[p];
    } else {
      const int32_t m = 16 * tg + (l & 15);
      if (m >= g.M) continue;
      e_orow[u] = m;
      arow = m;
      if (g.bias) e_x[u] = bf16_to_f32(g.bias[n]);
    }
    if constexpr (epi_bf16_out(EPI)) {
      e_sa[u] = g.sa[arow];
      e_sw[u] = sw[n];
    }
  }

  // fused quantization (kXQ): the wave's K range of the rows loaded at once,
  // the rows' absmax over the block, the range quantized into the wave's
  // ring slots, its token fragments into registers
  __shared__ uint32_t xq_max[kXQ ? 16 : 1];
  __shared__ float xq_s[kXQ ? 16 : 1], xq_r[kXQ ? 16 : 1];
  __shared__ int xq_fast[kXQ ? 16 : 1];
  constexpr int kXS = kXQ ? kXQMaxStages : 1;
  v4i xq[kXS][4];
  if constexpr (kXQ) {
    static_assert(D * kOps < 64, "token loads complete before the weight stages");
    const int M = static_cast<int>(g.M);
    if (tid < 16) xq_max[tid] = 0;
    __syncthreads();  // nothing in flight yet
    // this wave's K range [256 s_begin, 256 s_end) of each row in 16-element
    // chunks, chunk c = m * cpr + j (row m, elements 256 s_begin + 16 j ..),
    // lane l holding chunks l, l + 64, ... through a buffer view of the M
    // rows; chunks past the rows' chunks or past K (K % 16 == 0: a chunk is
    // all in or all out) read zeros without traffic
    const int kw = 256 * (s_end - s_begin), cpr = kw / 16, nch = M * cpr;
    const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        scalar_ptr(const_cast<int8_t*>(g.A)), 0, static_cast<int>(g.M * g.lda * 2), kBufferFlags);
    v4i xc[kXQChunks][2];
#pragma unroll
    for (int u = 0; u < kXQChunks; ++u) {
      xc[u][0] = xc[u][1] = v4i{0};
      if (64 * u < nch) {  // wave-uniform: the wave's chunks only
        const int c = lane + 64 * u, m = c / cpr, j = c - m * cpr;
        const int64_t k = 256 * static_cast<int64_t>(s_begin) + 16 * j;
        const uint32_t off = c < nch && k < g.K ? static_cast<uint32_t>((m * g.lda + k) * 2) : 0x80000000u;
        xc[u][0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off, 0, 0));
        xc[u][1] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off + 16, 0, 0));
      }
    }
    // weight stages 0 .. D-2 behind the loads (stages past the wave's range
    // read zeros without traffic, so exactly D-1 stages of operations follow
    // the loads); the last slot stays free for the int8 rows
#pragma unroll
    for (int d = 0; d < D - 1; ++d) issue(d, s_begin + d);
    wait_vmcnt<(D - 1) * kOps>();  // the row loads are in
#pragma unroll
    for (int u = 0; u < kXQChunks; ++u) {
      const int c = lane + 64 * u;
      if (64 * u >= nch) break;  // wave-uniform
      uint32_t mx = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = static_cast<uint32_t>(xc[u][h][j]), lo = w & 0x7FFFu, hi = (w >> 16) & 0x7FFFu;
          mx = lo > mx ? lo : mx;
          mx = hi > mx ? hi : mx;
        }
      if (c < nch) atomicMax(&xq_max[c / cpr], mx);
    }
    // raw barriers (LDS waits only): the weight stages stay in flight
    __builtin_amdgcn_s_waitcnt(0xC07F);
    raw_barrier();
    if (tid < 16) {
      const RowScale rs = row_scale(bf16_to_f32(static_cast<uint16_t>(xq_max[tid])));
      xq_s[tid] = tid < M ? rs.s : 0.0f;
      xq_r[tid] = rs.r;
      xq_fast[tid] = rs.fast ? 1 : 0;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    raw_barrier();
    // this wave's range of each row, int8, row-major in its last ring slot
    unsigned char* xslot = my_ring + (D - 1) * kStage;
#pragma unroll
    for (int u = 0; u < kXQChunks; ++u) {
      const int c = lane + 64 * u;
      if (64 * u >= nch) break;  // wave-uniform
      if (c < nch) {
        const int m = c / cpr, j = c - m * cpr;
        RowScale rs;
        rs.s = xq_s[m];
        rs.r = xq_r[m];
        rs.fast = xq_fast[m] != 0;
        U16x8 a, b;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          a.w[t] = static_cast<uint32_t>(xc[u][0][t]);
          b.w[t] = static_cast<uint32_t>(xc[u][1][t]);
        }
        uint2 qa, qb;
        if (rs.fast) {
          qa = quant8<true>(a, rs);
          qb = quant8<true>(b, rs);
        } else {
          qa = quant8<false>(a, rs);
          qb = quant8<false>(b, rs);
        }
        *reinterpret_cast<v4i*>(xslot + m * kw + 16 * j) =
            v4i{static_cast<int>(qa.x), static_cast<int>(qa.y), static_cast<int>(qb.x), static_cast<int>(qb.y)};
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's ring writes done (one wave reads them)
#pragma unroll
    for (int i = 0; i < kXS; ++i)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        xq[i][kb] = r16 < M && i < s_end - s_begin
                        ? *reinterpret_cast<const v4i*>(xslot + r16 * kw + 256 * i + 64 * kb + 16 * grp)
                        : v4i{0};
    __builtin_amdgcn_s_waitcnt(0xC07F);  // fragments read before the weight DMA reuses the slot
    issue(D - 1, s_begin + D - 1);  // (past the wave's range: zeros, no traffic)
  }

  v4i acc[RG][TG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg)
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) acc[rg][tg] = v4i{0};
  auto consume = [&](int d) {
    const unsigned char* slot = my_ring + d * kStage;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const v4i w = *reinterpret_cast<const v4i*>(slot + (16 * rg + r16) * 256 + 16 * ((4 * kb + grp) ^ r16));
#pragma unroll
        for (int tg = 0; tg < TG; ++tg)
          acc[rg][tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, xr[d][kb][tg], acc[rg][tg], 0, 0, 0);
      }
    }
  };

  // The wave's stages, padded to a multiple of D with zero-weight stages,
  // run branch-free: D stages in flight, refill after each consume; the last
  // D stages drain with compile-time waits.
  const int n_st = s_end - s_begin;
  if constexpr (kXQ) {
    // fused quantization: every stage's token fragments are in xq (compile-
    // time indices), so the wave's stages run fully unrolled; the first D
    // stages went out in the prologue
#pragma unroll
    for (int i = 0; i < kXS; ++i) {
      if (i < n_st) {
        const int later = n_st - 1 - i < D - 1 ? n_st - 1 - i : D - 1;  // stages issued after stage i
        wait_stages<kOps, (D - 1 < 3 ? D - 1 : 3)>(later);
        const unsigned char* slot = my_ring + (i % D) * kStage;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
          for (int rg = 0; rg < RG; ++rg) {
            const v4i w = *reinterpret_cast<const v4i*>(slot + (16 * rg + r16) * 256 + 16 * ((4 * kb + grp) ^ r16));
            acc[rg][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, xq[i][kb], acc[rg][0], 0, 0, 0);
          }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): fragments read before the refill
        if (i + D < n_st) issue(i % D, s_begin + i + D);
      }
    }
  } else if (n_st > 0) {
    const int n_pad = ((n_st + D - 1) / D) * D;
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, s_begin + d);
    for (int st0 = s_begin; st0 < s_begin + n_pad - D; st0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        wait_vmcnt<(D - 1) * kOps>();
        consume(d);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): fragments read before the refill
        issue(d, st0 + d + D);
      }
    }
    // drain: stage d of the last group waits with D-1-d later stages in flight
    RingDrain<D, kOps, 0>::run(consume);
  }

  __syncthreads();  // red[] zeroed by every thread before any wave adds into it
#pragma unroll
  for (int rg = 0; rg < RG; ++rg)
#pragma unroll
    for (int tg = 0; tg < TG; ++tg)
#pragma unroll
      for (int v = 0; v < 4; ++v) atomicAdd(&red[(rg * TG + tg) * 4 + v][lane], acc[rg][tg][v]);
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kEpiPerThread; ++u) {
    const int e = tid + u * 64 * WAVES;
    if (e >= kAcc * 64) continue;
    const int j = e >> 6, l = e & 63;
    const int v = j & 3;
    const int nl = 16 * (j / (4 * TG)) + 4 * (l >> 4) + v;  // row within the block's range
    const int64_t n = n0 + nl;
    if constexpr (!kPre) {  // dense rows: operands loaded here
      const int32_t m = 16 * ((j / 4) % TG) + (l & 15);
      if (nl >= rows || m >= g.M) continue;
      e_orow[0] = m;
      if constexpr (epi_bf16_out(EPI)) {
        e_sa[0] = kXQ ? xq_s[m] : g.sa[m];
        e_sw[0] = sw[n];
        e_x[0] = g.bias ? bf16_to_f32(g.bias[n]) : 0.0f;
      }
    }
    const int ui = kPre ? u : 0;
    if (e_orow[ui] < 0) continue;
    const int32_t a = red[j][l];
    if constexpr (epi_bf16_out(EPI)) {
      float t = epi_scale(a, e_sa[ui], e_sw[ui]);
      if constexpr (Rows::kGrouped) {
        if (g.topk_w) t = t * e_x[ui];
      } else {
        if (g.bias) t = t + e_x[ui];
      }
      static_cast<uint16_t*>(g.out)[static_cast<int64_t>(e_orow[ui]) * g.ldo + n] = f32_to_bf16(t);
    } else {
      static_cast<int32_t*>(g.out)[static_cast<int64_t>(e_orow[ui]) * g.ldo + n] = a;
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// ------------------------------------------------------------------------
// Dense decode core with a shared token ring (up to 16 TG tokens, K % 256 == 0)
// ------------------------------------------------------------------------
// Wide N at a few dozen tokens: one-wave decode3 blocks (nine per CU at
// N = 34816) each read the whole token panel through the texture path,
// about half as many bytes again as their weight rows (gate_up at 8
// tokens: 94 MB of token reads beside 178 MB of weights), and from 33
// tokens the tile rings take over at a fraction of the weight stream's
// rate.  Here one block per CU (a grid of a multiple of the CU count) owns
// a range of at most 16 WAVES weight rows: wave w streams rows
// [n0 + 16 w, n0 + 16 w + 16) of the range through its own LDS ring of D
// stages of 256 K bytes (the decode3 DMA and swizzle), and the block's TG
// groups of 16 token rows come once per block into a shared ring of D
// stages.  Wave t < TG issues token group t of each stage, one stage
// later than its own weight stage of the same index and after the barrier
// that frees the slot, so its issue order is W(0) X(0) W(1) X(1) ...: at
// stage s it waits with D-1 weight and D-2 token stages still in flight,
// the other waves with D-1 weight stages.  One barrier per stage makes
// token stage s visible to every wave and frees the slot of stage s-1.
// Token rows past M and weight rows past the range read zeros through the
// buffer range check (no traffic); stages past K are issued past the range
// as well, so every stage issues the same number of operations.  Block b
// walks the K stages from stage b n_st / G on: with every block at the
// same K offset, a row stride of 8192 bytes put all the concurrent
// requests on the same low address bits (MI355X, N = 34816 at K = 8192
// and 8 tokens: 59.2 us in lockstep, 45.8 us staggered; K = 5120
// unchanged).
template <int TG, int WAVES, int D, int EPI>
__global__ __launch_bounds__(64 * WAVES) void decode_sx_gemm_kernel(GemmArgs g) {
#if defined(__HIP_DEVICE_COMPILE__)
  static_assert(TG >= 1 && TG <= 4 && WAVES >= TG && D >= 2 && D <= 4, "shape");
  constexpr int kOps = 4;  // 1 KB DMA instructions per weight stage and per token group stage
  static_assert((2 * D - 3) * kOps < 64, "vmcnt range");
  constexpr int kXStage = TG * kRingStage;  // TG groups of 16 rows x 256 bytes
  extern __shared__ __align__(16) unsigned char ring[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, grp = lane >> 4;
  unsigned char* wring = ring + wave * (D * kRingStage);
  unsigned char* xring = ring + WAVES * (D * kRingStage);
  const int64_t n0 = g.N * blockIdx.x / gridDim.x;
  const int64_t rows = g.N * (blockIdx.x + 1) / gridDim.x - n0;  // <= 16 WAVES (host)
  const int64_t left = rows - 16 * static_cast<int64_t>(wave);
  const int nrows = left <= 0 ? 0 : (left < 16 ? static_cast<int>(left) : 16);
  const int64_t wr0 = n0 + 16 * static_cast<int64_t>(wave);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      scalar_ptr(const_cast<int8_t*>(g.W + (nrows > 0 ? wr0 : 0) * g.K)), 0, static_cast<int>(nrows * g.K),
      kBufferFlags);
  const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      scalar_ptr(const_cast<int8_t*>(g.A)), 0, static_cast<int>(g.M * g.lda), kBufferFlags);
  const bool x_issuer = wave < TG;  // wave t issues token group t (wave-uniform)
  // instruction j of a stage fills LDS rows 4j .. 4j+3 of its 16-row slot:
  // lane l fills row 4j + l/16, chunk l%16, from global chunk (l%16) ^ (row & 15)
  uint32_t w_off[4], x_off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 4 * j + (lane >> 4), c = (lane & 15) ^ (row & 15);
    const int m = 16 * wave + row;  // token row of this wave's group (issuers only)
    w_off[j] = static_cast<uint32_t>(row * g.K + 16 * c);
    x_off[j] = x_issuer && m < g.M ? static_cast<uint32_t>(m * g.lda + 16 * c) : 0x80000000u;
  }
  const int n_st = static_cast<int>(g.K / 256);
  // block b walks the stages from b n_st / G on (wrapping)
  const int s0 = static_cast<int>(static_cast<int64_t>(n_st) * blockIdx.x / gridDim.x);
  auto soff = [&](int st) {
    const int t = st + s0;
    return st < n_st ? (t < n_st ? t : t - n_st) * 256 : 0x7fff0000;
  };
  auto issue_w = [&](int st) {
    unsigned char* slot = wring + (st % D) * kRingStage;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(slot + j * 1024), 16, w_off[j], soff(st), 0,
                                               kStreamAux);
  };
  auto issue_x = [&](int st) {  // waves < TG: token group `wave`
    unsigned char* slot = xring + (st % D) * kXStage + wave * kRingStage;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rsrc, (lds_ptr_t)(slot + j * 1024), 16, x_off[j], soff(st), 0, 0);
  };
  v4i acc[TG];
#pragma unroll
  for (int tg = 0; tg < TG; ++tg) acc[tg] = v4i{0};
  auto consume = [&](int st) {
    const unsigned char* ws = wring + (st % D) * kRingStage;
    const unsigned char* xs = xring + (st % D) * kXStage;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int off = r16 * 256 + 16 * ((4 * kb + grp) ^ r16);
      const v4i w = *reinterpret_cast<const v4i*>(ws + off);
#pragma unroll
      for (int tg = 0; tg < TG; ++tg) {
        const v4i x = *reinterpret_cast<const v4i*>(xs + tg * kRingStage + off);
        acc[tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, x, acc[tg], 0, 0, 0);
      }
    }
  };
  // prologue: W(0) X(0) ... W(D-2) X(D-2) W(D-1)
#pragma unroll
  for (int d = 0; d < D; ++d) {
    issue_w(d);
    if (x_issuer && d < D - 1) issue_x(d);
  }
  for (int s = 0; s < n_st; ++s) {
    if (x_issuer) wait_vmcnt<(2 * D - 3) * kOps>(); else wait_vmcnt<(D - 1) * kOps>();
    raw_barrier();  // token stage s visible to every wave; every wave past its reads of stage s-1
    if (x_issuer) issue_x(s + D - 1);
    consume(s);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the slots done before their refill
    issue_w(s + D);
  }
  wait_vmcnt<0>();  // the padding stages' DMA has landed before the wave ends

  // lane (r16, grp) holds weight rows wr0 + 4 grp + v of token 16 tg + r16
#pragma unroll
  for (int tg = 0; tg < TG; ++tg) {
    const int m = 16 * tg + r16;
    if (m >= g.M) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int nl = 4 * grp + v;
      if (nl >= nrows) continue;
      const int64_t n = wr0 + nl;
      if constexpr (epi_bf16_out(EPI)) {
        float t = epi_scale(acc[tg][v], g.sa[m], g.sw[n]);
        if (g.bias) t = t + bf16_to_f32(g.bias[n]);
        static_cast<uint16_t*>(g.out)[static_cast<int64_t>(m) * g.ldo + n] = f32_to_bf16(t);
      } else {
        static_cast<int32_t*>(g.out)[static_cast<int64_t>(m) * g.ldo + n] = acc[tg][v];
      }
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// ------------------------------------------------------------------------
// Decode down-projection with the top-k slot sum fused in
// ------------------------------------------------------------------------
// For 16-row alignment blocks (decode batches).  Block b owns output
// columns [n0, n0 + R) of every token (R <= 8: the N columns cut into
// gridDim.x equal ranges, as the dense decode grid cuts them) and walks
// every alignment block whose expert lies in [0, E).  The expert's R
// weight rows for those columns stream through the waves' private LDS
// rings (slots of 8 rows x 256 K bytes filled by buffer_load ... lds with
// the decode ring's chunk swizzle on row & 7; the MFMA's weight rows 8-15
// read rows 0-7 again and are dropped), the 16 gathered pair rows through
// the token register ring.  After an alignment block's last K stage its
// wave applies the GEMM2 epilogue (activation scale, column scale, routed
// weight: the operations of the grouped decode epilogue) and keeps the
// bf16 value of each (pair, column) in an LDS table.  A pair sits in one
// alignment block, so the waves write disjoint entries; after one barrier
// the block sums each token's top_k entries in slot order in fp32 and
// writes bf16 -- the operations of moe_sum_reduce_kernel.  A pair whose
// expert lies outside [0, E) contributes +0.  No workspace, no exchange
// between blocks.  The tables the loop reads (sorted ids, the list of
// alignment blocks with their experts, the pairs' activation scales and
// routed weights, every expert's column scales for this block's columns)
// are loaded into LDS once, before the weight stream.
struct MoeSumLds {
  int sid, exp, list, sa, rw, sw, out, total;
};
// Sizes one prologue pass of moe_gemm_sum_kernel loads (the host checks them).
constexpr int kMoeSumMaxSorted = 6144, kMoeSumMaxPairs = 2048, kMoeSumMaxExperts = 256;
__host__ __device__ inline int moe_sum_up16(int64_t bytes) { return static_cast<int>((bytes + 15) & ~int64_t{15}); }
__host__ __device__ inline MoeSumLds moe_sum_lds(int ring_bytes, int64_t max_sorted, int64_t num_valid, int E) {
  MoeSumLds l;
  l.sid = ring_bytes;
  l.exp = l.sid + moe_sum_up16(4 * max_sorted);
  l.list = l.exp + moe_sum_up16(4 * (max_sorted / 16));
  l.sa = l.list + moe_sum_up16(4 * (max_sorted / 16));
  l.rw = l.sa + moe_sum_up16(4 * num_valid);
  l.sw = l.rw + moe_sum_up16(4 * num_valid);
  l.out = l.sw + 32 * E;
  l.total = l.out + moe_sum_up16(16 * num_valid);
  return l;
}
constexpr int kMoeSumSlot = 2048;  // 8 weight rows x 256 K bytes

// kTopk: units of 16 pairs per expert (U = GemmArgs::topk_units of them,
// unit e * U + u), the pairs listed in the prologue from the router ids
// (GemmArgs::sorted_ids carries topk_ids; distinct experts per token, so an
// expert holds at most 16 U pairs); max_sorted is then 16 * E * U.  Pairs
// sit in the order of the LDS atomics that place them, which changes no
// result: each pair's row is its own dot products, and the slot sum reads
// the pairs by index.
template <int WAVES, int D, bool kTopk = false>
__global__ __launch_bounds__(64 * WAVES) void moe_gemm_sum_kernel(GemmArgs g, int64_t max_sorted) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int kOps = 2 + 4;  // vector memory ops per stage: 2 DMA + 4 token loads
  static_assert(D >= 2 && D <= 8 && (D - 1) * kOps < 64, "ring depth");
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int s_count;
  const int nv = static_cast<int>(g.num_valid), E = g.num_experts;
  const MoeSumLds L = moe_sum_lds(WAVES * D * kMoeSumSlot, max_sorted, nv, E);
  int32_t* t_sid = reinterpret_cast<int32_t*>(lds + L.sid);
  int32_t* t_exp = reinterpret_cast<int32_t*>(lds + L.exp);
  int32_t* t_list = reinterpret_cast<int32_t*>(lds + L.list);
  float* t_sa = reinterpret_cast<float*>(lds + L.sa);
  float* t_rw = reinterpret_cast<float*>(lds + L.rw);
  float* t_sw = reinterpret_cast<float*>(lds + L.sw);
  uint16_t* t_out = reinterpret_cast<uint16_t*>(lds + L.out);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = g.N * blockIdx.x / gridDim.x;
  const int R = static_cast<int>(g.N * (blockIdx.x + 1) / gridDim.x - n0);
  if (R <= 0) return;  // more blocks than columns (uniform per block)
  int n_sorted, nb;
  if constexpr (kTopk) {
    nb = E * g.topk_units;
    n_sorted = 16 * nb;
  } else {
    const int64_t npp = *g.num_post_pad;
    n_sorted = static_cast<int>(npp < max_sorted ? npp : max_sorted);
    nb = n_sorted / 16;
  }
  const bool routed = g.topk_w != nullptr;

  // ---- tables, every global load of the prologue issued before the first
  // LDS store (one round trip; the host bounds the sizes to one pass)
  constexpr int kT = 64 * WAVES;
  constexpr int kSidPer = (kMoeSumMaxSorted + kT - 1) / kT, kPairPer = (kMoeSumMaxPairs + kT - 1) / kT;
  static_assert(!kTopk || kMoeSumMaxSorted / 16 <= kT, "router-id units: one per thread");
  constexpr int kSwPer = (8 * kMoeSumMaxExperts + kT - 1) / kT, kExpPer = (kMoeSumMaxSorted / 16 + kT - 1) / kT;
  int32_t v_sid[kSidPer], v_exp[kExpPer];
  float v_sa[kPairPer], v_rw[kPairPer], v_sw[kSwPer];
  if constexpr (kTopk) {  // the router ids of the pairs, one per thread
#pragma unroll
    for (int u = 0; u < kSidPer; ++u) {
      const int i = u * kT + tid;
      v_sid[u] = i < nv ? g.sorted_ids[i] : -1;
    }
  } else {
#pragma unroll
    for (int u = 0; u < kSidPer; ++u) {
      const int i = u * kT + tid;
      v_sid[u] = i < n_sorted ? g.sorted_ids[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kExpPer; ++u) {
      const int i = u * kT + tid;
      v_exp[u] = i < nb ? g.expert_ids[i] : -1;
    }
  }
#pragma unroll
  for (int u = 0; u < kPairPer; ++u) {
    const int i = u * kT + tid;
    v_sa[u] = i < nv ? g.sa[i] : 0.0f;
    v_rw[u] = (routed && i < nv) ? g.topk_w[i] : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < kSwPer; ++u) {
    const int i = u * kT + tid, r = i & 7;
    v_sw[u] = (i < E * 8 && r < R) ? g.sw[static_cast<int64_t>(i >> 3) * g.N + n0 + r] : 0.0f;
  }
  if constexpr (kTopk) {
    // the pairs of expert e fill units e * U .. e * U + U - 1: per-expert
    // counts in t_exp[0, E), slots of t_sid claimed with LDS atomics, then
    // t_exp[unit] = e for the units that hold pairs (nb <= kT: one unit per
    // thread, its count read before any unit entry is written)
    const int U = g.topk_units;
    for (int i = tid; i < n_sorted; i += kT) t_sid[i] = nv;
    for (int i = tid; i < E; i += kT) t_exp[i] = 0;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kSidPer; ++u) {
      const int i = u * kT + tid, e = v_sid[u];
      if (i < nv && e >= 0 && e < E) {
        const int pos = atomicAdd(&t_exp[e], 1);
        if (pos < 16 * U) t_sid[(e * U + pos / 16) * 16 + pos % 16] = i;
      }
    }
    __syncthreads();
    const int cnt = tid < nb ? t_exp[tid / U] : 0;
    __syncthreads();
    if (tid < nb) t_exp[tid] = cnt > 16 * (tid % U) ? tid / U : -1;
  } else {
#pragma unroll
    for (int u = 0; u < kSidPer; ++u) {
      const int i = u * kT + tid;
      if (i < n_sorted) t_sid[i] = v_sid[u];
    }
#pragma unroll
    for (int u = 0; u < kExpPer; ++u) {
      const int i = u * kT + tid;
      if (i < nb) t_exp[i] = v_exp[u];
    }
  }
#pragma unroll
  for (int u = 0; u < kPairPer; ++u) {
    const int i = u * kT + tid;
    if (i < nv) {
      t_sa[i] = v_sa[u];
      t_rw[i] = v_rw[u];
    }
  }
#pragma unroll
  for (int u = 0; u < kSwPer; ++u) {
    const int i = u * kT + tid;
    if (i < E * 8) t_sw[i] = v_sw[u];
  }
  for (int i = tid; i < 4 * nv; i += kT) reinterpret_cast<uint32_t*>(t_out)[i] = 0u;
  __syncthreads();
  if (wave == 0) {  // alignment blocks of an expert in [0, E), packed (expert << 20) | block
    int cnt = 0;
    for (int base = 0; base < nb; base += 64) {
      const int a = base + lane;
      const int e = a < nb ? t_exp[a] : -1;
      const bool ok = e >= 0 && e < E;
      const uint64_t m = __ballot(ok);
      if (ok) t_list[cnt + __popcll(m & ((uint64_t{1} << lane) - 1))] = (e << 20) | a;
      cnt += __popcll(m);
    }
    if (lane == 0) s_count = cnt;
  }
  __syncthreads();
  const int nlist = s_count;

  // ---- the wave's alignment blocks i = wave, wave + WAVES, ...: S stages of 256 K bytes each
  const int S = static_cast<int>((g.K + 255) / 256);
  const int n_mine = nlist > wave ? (nlist - wave + WAVES - 1) / WAVES : 0;
  const int n_st = n_mine * S;
  unsigned char* my_ring = lds + wave * (D * kMoeSumSlot);
  const int r16 = lane & 15, grp = lane >> 4, r8 = lane & 7;
  // weight DMA: instruction j fills LDS rows 4j .. 4j+3; lane l fills row
  // 4j + l/16, chunk l%16 from global chunk (l%16) ^ row
  uint32_t w_off[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = 4 * j + (lane >> 4);
    w_off[j] = static_cast<uint32_t>(row * g.K + 16 * ((lane & 15) ^ row));
  }
  typedef const v4i __attribute__((address_space(1)))* gv4i_ptr;
  const uint64_t zero_addr = reinterpret_cast<uint64_t>(kZeroChunk);
  v4i xr[D][4];

  auto issue = [&](int d, int s) {
    unsigned char* slot = my_ring + d * kMoeSumSlot;
    int a = 0, e = 0, st = 0;
    const bool real = s < n_st;  // wave-uniform
    if (real) {
      const int i = s / S;
      st = s - i * S;
      const int ent = __builtin_amdgcn_readfirstlane(t_list[wave + WAVES * i]);
      a = ent & 0xFFFFF;
      e = ent >> 20;
    }
    // a padding stage reads past the buffer range: zeros, no traffic
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        scalar_ptr(const_cast<int8_t*>(g.W + (static_cast<int64_t>(e) * g.N + n0) * g.K)), 0,
        static_cast<int>(R * g.K), kBufferFlags);
    const int soff = real ? st * 256 : 0x7fff0000;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(slot + j * 1024), 16, w_off[j], soff, 0,
                                               kStreamAux);
    // the token address is selected bitwise and every load is unconditional:
    // a branch around a load makes its result a merge that the compiler
    // waits for with vmcnt(0), which would drain the whole ring each stage
    const int32_t p_raw = t_sid[a * 16 + r16];  // a = 0 on a padding stage (nlist > 0 there)
    const int32_t p = real ? p_raw : nv;
    const bool pok = p < nv;
    const uint64_t xrow = reinterpret_cast<uint64_t>(g.A) + static_cast<uint64_t>(pok ? p : 0) * g.lda;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int64_t k = static_cast<int64_t>(st) * 256 + 64 * kb + 16 * grp;
      const uint64_t m = (pok && k < g.K) ? ~uint64_t{0} : uint64_t{0};
      const uint64_t addr = ((xrow + static_cast<uint64_t>(k)) & m) | (zero_addr & ~m);
      xr[d][kb] = *reinterpret_cast<gv4i_ptr>(addr);
    }
  };

  v4i acc = v4i{0};
  auto consume = [&](int d, int s) {
    const unsigned char* slot = my_ring + d * kMoeSumSlot;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const v4i w = *reinterpret_cast<const v4i*>(slot + r8 * 256 + 16 * ((4 * kb + grp) ^ r8));
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, xr[d][kb], acc, 0, 0, 0);
    }
    if (s >= n_st) return;
    const int i = s / S;
    if (s - i * S != S - 1) return;  // not the alignment block's last stage (uniform)
    // epilogue: lane holds weight row 4 * grp + v (rows 0-7 in lanes 0-31)
    // of token column r16 of the alignment block
    const int ent = __builtin_amdgcn_readfirstlane(t_list[wave + WAVES * i]);
    const int a = ent & 0xFFFFF, e = ent >> 20;
    const int32_t p = t_sid[a * 16 + r16];
    if (grp < 2 && p < nv) {
      const float sa = t_sa[p], rw = t_rw[p];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 4 * grp + v;
        if (row >= R) continue;
        float t = epi_scale(acc[v], sa, t_sw[e * 8 + row]);
        if (routed) t = t * rw;
        t_out[p * 8 + row] = f32_to_bf16(t);
      }
    }
    acc = v4i{0};
  };

  if (n_st > 0) {
    const int n_pad = ((n_st + D - 1) / D) * D;
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);
    for (int s0 = 0; s0 < n_pad - D; s0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        wait_vmcnt<(D - 1) * kOps>();
        consume(d, s0 + d);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): fragments read before the refill
        issue(d, s0 + d + D);
      }
    }
    auto drain = [&](int d) { consume(d, n_pad - D + d); };
    RingDrain<D, kOps, 0>::run(drain);
  }
  __syncthreads();

  // ---- slot sum in slot order (fp32), one (token, column) per thread
  const int tk = g.top_k, T = nv / tk;
  uint16_t* out = static_cast<uint16_t*>(g.out);
  for (int idx = tid; idx < T * R; idx += 64 * WAVES) {
    const int t = idx / R, r = idx - t * R;
    float sum = 0.0f;
    for (int i = 0; i < tk; ++i) sum = sum + bf16_to_f32(t_out[(t * tk + i) * 8 + r]);
    out[static_cast<int64_t>(t) * g.ldo + n0 + r] = f32_to_bf16(sum);
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// ------------------------------------------------------------------------
// K-split reduction: out[tile rows, tile cols] = epilogue(sum_s part[u0 + s])
// with the partials summed in split order (exact int32).  One thread per 8
// consecutive columns of one tile row.
// ------------------------------------------------------------------------
// Sums over the ts K ranges of a split tile of kRows runs of 8 int32
// partial values each (run i at p + off[i], range s at + s * stride).  The
// loads go out in batches of kBatch ranges before any add, so a thread waits
// on memory once per batch rather than once per range (int32 sums wrap
// alike in any order: the result does not depend on the batching).
// Measured on MI355X (kernel trace): down M=512's 6-range reduction 15.0 ->
// 14.4 us, down M=64's 4.7 -> 4.2 us; the reduction then moves its 68 MB at
// 4.7 TB/s, so the partial tiles' stream bounds it.
template <int kRows, int kBatch>
__device__ __forceinline__ void split_sum8(const int32_t* p, const int (&off)[kRows], int ts, int64_t stride,
                                           int32_t (&a)[kRows][8]) {
#pragma unroll
  for (int i = 0; i < kRows; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) a[i][j] = 0;
  for (int s0 = 0; s0 < ts; s0 += kBatch) {
    v4i x[kBatch][kRows][2];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        if (s0 + u < ts) {
          const int32_t* q = p + static_cast<int64_t>(s0 + u) * stride + off[i];
          x[u][i][0] = *reinterpret_cast<const v4i*>(q);
          x[u][i][1] = *reinterpret_cast<const v4i*>(q + 4);
        } else {
          x[u][i][0] = v4i{0, 0, 0, 0};
          x[u][i][1] = v4i{0, 0, 0, 0};
        }
      }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
#pragma unroll
      for (int i = 0; i < kRows; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a[i][j] += x[u][i][0][j];
          a[i][4 + j] += x[u][i][1][j];
        }
  }
}

template <int EPI, int BM, int BN>
__global__ __launch_bounds__(256) void split_reduce_kernel(GemmArgs g) {
  constexpr int kC8 = BN / 8;
  const int64_t tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  const int64_t tail = tm * tn - g.full_tiles;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // (tile, row, col8)
  if (idx >= tail * BM * kC8) return;
  const int64_t tt = idx / (BM * kC8);
  const int r = static_cast<int>((idx / kC8) % BM), c8 = static_cast<int>(idx % kC8) * 8;
  int64_t pm, pn;
  tile_of_index(g.full_tiles + tt, tm, tn, pm, pn);
  const int64_t m = pm * BM + r;
  if (m >= g.M) return;
  const int32_t* p = g.part + (tt * g.tail_split) * (BM * BN) + r * BN + c8;
  int32_t sum[1][8];
  split_sum8<1, 8>(p, {0}, g.tail_split, BM * BN, sum);
  const int32_t(&a)[8] = sum[0];
  const int64_t n0 = pn * BN + c8;
  if constexpr (EPI == kEpiBf16) {
    const float sa = g.sa[m];
    uint16_t o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t n = n0 + j < g.N ? n0 + j : g.N - 1;
      o[j] = epi_bf16(a[j], sa, g.sw[n], g.bias, n, 1.0f, false);
    }
    uint16_t* dst = static_cast<uint16_t*>(g.out) + m * g.ldo + n0;
    if (g.staged_out && n0 + 8 <= g.N) {  // 16-byte aligned full chunk
      v4i v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = static_cast<int>(o[2 * j] | (static_cast<uint32_t>(o[2 * j + 1]) << 16));
      *reinterpret_cast<v4i*>(dst) = v;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (n0 + j < g.N) dst[j] = o[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t n = n0 + j;
      if (n < g.N) static_cast<int32_t*>(g.out)[m * g.ldo + n] = a[j];
    }
  }
}

// K-split reduction of fused-activation tiles (kAct): a partial tile holds
// the gate half of its columns, then the up half.  One thread per 8
// activation columns of one tile row sums both halves in split order,
// rounds g and u to bf16 as the tile epilogue does, and writes act =
// bf16(act_fn(g) * u) to out[rows, N / 2] (N / 2 % 8 == 0, 16-byte rows).
template <int BM, int BN, int kAct>
__global__ __launch_bounds__(256) void split_reduce_act_kernel(GemmArgs g) {
  constexpr int kH = BN / 2, kC8 = kH / 8;
  const int64_t half = g.N / 2;
  const int64_t tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  const int64_t tail = tm * tn - g.full_tiles;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // (tile, row, act col8)
  if (idx >= tail * BM * kC8) return;
  const int64_t tt = idx / (BM * kC8);
  const int r = static_cast<int>((idx / kC8) % BM), c8 = static_cast<int>(idx % kC8) * 8;
  int64_t pm, pn;
  tile_of_index(g.full_tiles + tt, tm, tn, pm, pn);
  const int64_t m = pm * BM + r, n0 = pn * kH + c8;
  if (m >= g.M || n0 >= half) return;
  const int32_t* p = g.part + (tt * g.tail_split) * (BM * BN) + r * BN + c8;
  int32_t sum[2][8];
  split_sum8<2, 4>(p, {0, kH}, g.tail_split, BM * BN, sum);
  const int32_t(&ga)[8] = sum[0];
  const int32_t(&ua)[8] = sum[1];
  const float sa = g.sa[m];
  v4i o;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t pk = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * w + h;
      const int64_t n = n0 + j;
      const float gv = bf16_to_f32(epi_bf16(ga[j], sa, g.sw[n], nullptr, n, 1.0f, false));
      const float uv = bf16_to_f32(epi_bf16(ua[j], sa, g.sw[half + n], nullptr, half + n, 1.0f, false));
      pk |= static_cast<uint32_t>(f32_to_bf16(act_fn<kAct>(gv) * uv)) << (16 * h);
    }
    o[w] = static_cast<int>(pk);
  }
  *reinterpret_cast<v4i*>(static_cast<uint16_t*>(g.out) + m * g.ldo + n0) = o;
}

}  // namespace mw8
