// Dense W8A8 GEMM: dispatch between the decode core (M <= 32, or up to 64
// when K % 128 != 0: weight streaming, in-block split-K) and the MFMA tile
// core, plus the grouped-tile launchers used by the fused-MoE GEMM.
#include <atomic>

#include "gemm_kernels.h"

namespace mw8 {
namespace {

constexpr int64_t kDecodeMaxM = 64;

// Tuning override (-1 = automatic); set through mw8_set_tuning.
std::atomic<int> g_decode_cfg{-1};
std::atomic<int> g_tile_cfg{-1};
std::atomic<int> g_moe_cfg{-1};

// ------------------------------------------------------------------ decode
// (rows of 16 per block, waves per block, K steps per load batch).
// 0-6: decode_gemm_kernel (U steps loaded, then their MFMAs);
// 7-12: decode2_gemm_kernel (batches double-buffered, branch-free loads).
struct DecodeCfg {
  int rg, waves, u;
};
constexpr DecodeCfg kDecodeCfgs[] = {
    {1, 4, 8}, {2, 4, 4}, {1, 8, 4}, {2, 8, 4}, {4, 4, 4}, {4, 8, 2}, {2, 8, 2},
    {1, 16, 4}, {1, 8, 4}, {2, 16, 2}, {1, 16, 2}, {2, 8, 4}, {4, 16, 1},
    // 13-21: decode3_gemm_kernel (16 rows, LDS DMA ring; u = ring depth)
    {1, 4, 4}, {1, 4, 3}, {1, 2, 4}, {1, 8, 2}, {1, 4, 2}, {1, 2, 3}, {1, 2, 2}, {1, 1, 4}, {1, 8, 3},
    // 22-31: decode3_gemm_kernel over a CU-balanced grid (a multiple of the
    // CU count, each block up to 16 rg rows)
    {1, 1, 4}, {1, 2, 2}, {1, 4, 3}, {1, 8, 2}, {2, 1, 4}, {2, 2, 3}, {2, 2, 4}, {2, 4, 2},
    {2, 4, 3}, {2, 8, 2},
};
constexpr int kNumDecodeCfgs = sizeof(kDecodeCfgs) / sizeof(kDecodeCfgs[0]);

template <int RG, int TG, int WAVES, int U, int EPI>
void launch_decode(const GemmArgs& g, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>((g.N + 16 * RG - 1) / (16 * RG));
  hipLaunchKernelGGL((decode_gemm_kernel<RG, TG, WAVES, U, EPI>), dim3(blocks), dim3(64 * WAVES), 0,
                     st, g);
}

template <int RG, int TG, int WAVES, int U, int EPI>
void launch_decode2(const GemmArgs& g, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>((g.N + 16 * RG - 1) / (16 * RG));
  hipLaunchKernelGGL((decode2_gemm_kernel<RG, TG, WAVES, U, EPI>), dim3(blocks), dim3(64 * WAVES), 0,
                     st, g);
}

// Compute units of the current device (cached per device).
int device_cus() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Ring depth is capped by the token-register ring (D x 4 x TG x 4 VGPRs).
// kBal: a grid of c x CUs blocks of at most 16 RG rows each (every CU
// streams the same bytes); otherwise one block per 16 rows.
template <int TG, int WAVES, int D, int EPI, int RG = 1, bool kBal = false>
void launch_decode3(const GemmArgs& g, hipStream_t st) {
  constexpr int kD = TG == 1 ? D : (TG == 2 ? (D < 3 ? D : 3) : 2);
  constexpr int kLds = RG * DecodeRing<TG, WAVES, kD>::kLds;
  auto kern = decode3_gemm_kernel<TG, WAVES, kD, EPI, DenseRows, RG>;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    attr_set = true;
  }
  int64_t blocks = (g.N + 15) / 16;
  if (kBal) {
    const int64_t cus = device_cus();
    blocks = cus * ((g.N + cus * 16 * RG - 1) / (cus * 16 * RG));
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(64 * WAVES), kLds, st, g);
}

template <int TG, int EPI>
void decode_by_cfg(int cfg, const GemmArgs& g, hipStream_t st) {
  switch (cfg) {
    case 0: launch_decode<1, TG, 4, 8, EPI>(g, st); break;
    case 1: launch_decode<2, TG, 4, 4, EPI>(g, st); break;
    case 2: launch_decode<1, TG, 8, 4, EPI>(g, st); break;
    case 3: launch_decode<2, TG, 8, 4, EPI>(g, st); break;
    case 4: launch_decode<4, TG, 4, 4, EPI>(g, st); break;
    case 5: launch_decode<4, TG, 8, 2, EPI>(g, st); break;
    case 6: launch_decode<2, TG, 8, 2, EPI>(g, st); break;
    case 7: launch_decode2<1, TG, 16, 4, EPI>(g, st); break;
    case 8: launch_decode2<1, TG, 8, 4, EPI>(g, st); break;
    case 9: launch_decode2<2, TG, 16, 2, EPI>(g, st); break;
    case 10: launch_decode2<1, TG, 16, 2, EPI>(g, st); break;
    case 11: launch_decode2<2, TG, 8, 4, EPI>(g, st); break;
    case 12: launch_decode2<4, TG, 16, 1, EPI>(g, st); break;
    case 13: launch_decode3<TG, 4, 4, EPI>(g, st); break;
    case 14: launch_decode3<TG, 4, 3, EPI>(g, st); break;
    case 15: launch_decode3<TG, 2, 4, EPI>(g, st); break;
    case 16: launch_decode3<TG, 8, 2, EPI>(g, st); break;
    case 17: launch_decode3<TG, 4, 2, EPI>(g, st); break;
    case 18: launch_decode3<TG, 2, 3, EPI>(g, st); break;
    case 19: launch_decode3<TG, 2, 2, EPI>(g, st); break;
    case 20: launch_decode3<TG, 1, 4, EPI>(g, st); break;
    case 21: launch_decode3<TG, 8, 3, EPI>(g, st); break;
    case 22: launch_decode3<TG, 1, 4, EPI, 1, true>(g, st); break;
    case 23: launch_decode3<TG, 2, 2, EPI, 1, true>(g, st); break;
    case 24: launch_decode3<TG, 4, 3, EPI, 1, true>(g, st); break;
    case 25: launch_decode3<TG, 8, 2, EPI, 1, true>(g, st); break;
    case 26: launch_decode3<TG, 1, 4, EPI, 2, true>(g, st); break;
    case 27: launch_decode3<TG, 2, 3, EPI, 2, true>(g, st); break;
    case 28: launch_decode3<TG, 2, 4, EPI, 2, true>(g, st); break;
    case 29: launch_decode3<TG, 4, 2, EPI, 2, true>(g, st); break;
    case 30: launch_decode3<TG, 4, 3, EPI, 2, true>(g, st); break;
    default: launch_decode3<TG, 8, 2, EPI, 2, true>(g, st); break;
  }
}

// Measured on MI355X at the Qwen3-14B shapes (K 5120 / 17408, N 5120 -
// 34816), weights streamed from HBM.  Up to 32 tokens the LDS DMA ring
// (decode3) over a CU-balanced grid streams fastest.  With one block per
// 16 rows, N = 5120 gives 320 blocks: a quarter of the CUs stream twice
// the bytes of the others (down at M = 1: 22.3 us, against 13.5 us for
// N = 4096).  The balanced grid (256 blocks of 20 rows, two MFMA row
// groups sharing the token fragments) takes 18.1 us, and 21.6 us instead
// of 28.8 us at 16 tokens.  Narrow N (<= 16384): 4 waves x 3 slots of 32
// rows at one token, 8 waves x 2 slots up to 8 and from 17 tokens, 4
// waves x 2 slots at 9-16.  Wide N (gate_up, 2176 row groups): 16-row
// blocks, 2 waves x 2 slots at one token (30.6 us, 5.8 TB/s), one wave x
// 4 slots up to 8, 32-row blocks of one wave x 4 slots at 17-32 tokens.
// From 33 tokens on the token operand, read per wave through the texture
// path, costs more than the weight stream: the register-streaming core
// with 32 rows over 8 waves (cfg 3) wins, or 64 rows per block for very
// wide N (cfg 4), which keeps fewer blocks re-reading the token panel.
int default_decode_cfg(int64_t M, int64_t N, int64_t K) {
  (void)K;
  const bool wide = N >= 16384;
  if (M == 1) return wide ? 23 : 30;
  if (M <= 8) return wide ? 22 : 31;
  if (M <= 16) return 29;
  if (M <= 32) return wide ? 26 : 31;
  if (M > 48 && wide) return 4;
  return 3;
}

template <int EPI>
void dispatch_decode(const GemmArgs& g, hipStream_t st) {
  const int tg = static_cast<int>((g.M + 15) / 16);
  int cfg = g_decode_cfg.load(std::memory_order_relaxed);
  if (cfg < 0 || cfg >= kNumDecodeCfgs) cfg = default_decode_cfg(g.M, g.N, g.K);
  switch (tg) {
    case 1: decode_by_cfg<1, EPI>(cfg, g, st); break;
    case 2: decode_by_cfg<2, EPI>(cfg, g, st); break;
    case 3: decode_by_cfg<3, EPI>(cfg, g, st); break;
    default: decode_by_cfg<4, EPI>(cfg, g, st); break;
  }
}

// -------------------------------------------------------------------- tile
template <int BM, int BN, int BK, int WM, int WN, int EPI, class Rows>
void launch_tile(const GemmArgs& g, dim3 grid, hipStream_t st) {
  using S = TileShape<BM, BN, BK, WM, WN>;
  auto kern = tile_gemm_kernel<BM, BN, BK, WM, WN, EPI, Rows>;
  static bool attr_set = false;  // per instantiation; idempotent, so a race is benign
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, S::kLds);
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, grid, dim3(256), S::kLds, st, g);
}

template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI, class Rows>
void launch_tile3(const GemmArgs& g, dim3 grid, hipStream_t st) {
  constexpr int kLds = NSTAGE * (BM + BN) * BK;
  auto kern = tile3_gemm_kernel<BM, BN, BK, WM, WN, NSTAGE, EPI, Rows>;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, grid, dim3(64 * WM * WN), kLds, st, g);
}

// Persistent form: min(units, CUs x per_cu) resident blocks walk the units.
template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI>
void launch_tile3_persist(const GemmArgs& g, unsigned units, int per_cu, hipStream_t st) {
  constexpr int kLds = NSTAGE * (BM + BN) * BK;
  auto kern = tile3_persist_kernel<BM, BN, BK, WM, WN, NSTAGE, EPI>;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    attr_set = true;
  }
  const int64_t slots = static_cast<int64_t>(device_cus()) * per_cu;
  const unsigned grid = static_cast<unsigned>(units < slots ? units : slots);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * WM * WN), kLds, st, g);
}

// 0-4: register-staged tile core (any K % 16 == 0); 5 and up: direct-to-LDS
// ring (K % bk == 0).  per_cu: resident blocks per CU (LDS-bound).
struct TileCfg {
  int bm, bn;
  bool dma;
  int bk, per_cu;
};
constexpr TileCfg kTileCfgs[] = {
    {256, 256, false, 128, 1}, {256, 256, false, 64, 1}, {128, 128, false, 128, 2},
    {256, 128, false, 128, 1}, {128, 256, false, 128, 1},
    {256, 256, true, 64, 1},   // 5: 4 waves, 4 stages
    {256, 256, true, 64, 1},   // 6: 4 waves, 3 stages
    {128, 128, true, 64, 2},   // 7: 4 waves, 4 stages
    {256, 128, true, 64, 1},   // 8: 4 waves, 4 stages
    {256, 256, true, 64, 1},   // 9: 8 waves (2x4), 3 stages
    {256, 256, true, 64, 1},   // 10: 8 waves (4x2), 3 stages
    {256, 256, true, 64, 1},   // 11: 8 waves (2x4), 4 stages
    {256, 128, true, 64, 2},   // 12: 8 waves (4x2), 3 stages
    {256, 256, true, 64, 1},   // 13: 16 waves (4x4), 3 stages
    {256, 256, true, 128, 1},  // 14: 8 waves (4x2), 2 stages
    {256, 128, true, 128, 1},  // 15: 8 waves (4x2), 2 stages
    {256, 256, true, 128, 1},  // 16: 16 waves (4x4), 2 stages
    {256, 128, true, 128, 1},  // 17: 8 waves (4x2), 3 stages
    {64, 256, true, 128, 1},   // 18: 4 waves (1x4), 3 stages
    {64, 128, true, 128, 2},   // 19: 4 waves (1x4), 3 stages
    {128, 256, true, 128, 1},  // 20: 8 waves (2x4), 2 stages
    {128, 128, true, 128, 2},  // 21: 4 waves (2x2), 2 stages
    {64, 256, true, 64, 2},    // 22: 4 waves (1x4), 3 stages
    {128, 256, true, 64, 2},   // 23: 8 waves (2x4), 3 stages
    {64, 256, true, 64, 1},    // 24: 4 waves (1x4), 4 stages
    {64, 128, true, 128, 1},   // 25: 4 waves (1x4), 4 stages
    {256, 256, true, 64, 1},   // 26: 8 waves (4x2), 4 stages
    {256, 256, true, 128, 1},  // 27: 14 as a persistent walk
};
constexpr int kNumTileCfgs = sizeof(kTileCfgs) / sizeof(kTileCfgs[0]);

// K split of a ring tiling.  With T tiles and S = 256 * per_cu resident
// slots: T >= S cuts the r = T mod S tiles of the last, partial wave into
// sp = min(S / r, K / bk, 16) K ranges; T < S cuts every tile into
// sp = min(S / T, K / bk, 16) ranges.  No split when sp < 2.
struct SplitPlan {
  int64_t full = 0, tail = 0;
  int sp = 1;
  size_t ws = 0;
};

SplitPlan plan_split(int64_t M, int64_t N, int64_t K, const TileCfg& c) {
  SplitPlan p;
  if (!c.dma || K % c.bk != 0) return p;
  const int64_t T = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
  const int64_t slots = 256 * static_cast<int64_t>(c.per_cu);
  const int64_t r = T >= slots ? T % slots : T;
  if (r == 0) return p;
  int64_t sp = slots / r;
  const int64_t nkt = K / c.bk;
  if (sp > nkt) sp = nkt;
  if (sp > 16) sp = 16;
  if (sp < 2) return p;
  p.full = T - r;
  p.tail = r;
  p.sp = static_cast<int>(sp);
  p.ws = static_cast<size_t>(r) * sp * c.bm * c.bn * sizeof(int32_t);
  return p;
}

// Only the 256 x 256 rings split automatically; the skinny rings (18-25)
// split whenever their plan does.
bool split_enabled(int cfg) {
  const TileCfg& c = kTileCfgs[cfg];
  return c.dma && ((c.bm == 256 && c.bn == 256) || cfg >= 18);
}

// Modelled time (us) of one ring configuration: waves of resident blocks,
// each wave costing c0 + b x (block ops) / (per-CU rate with b blocks
// resident on the busiest CU), plus the K split's partial tiles (written
// and read back at ~4 TB/s) and its reduction launch, floored by the
// weight stream (~3.6 TB/s for these tilings).  Rates (TOPS per CU) fitted
// to MI355X sweeps of the Qwen3-14B shapes at M = 40 - 8192.
struct ModelCfg {
  int cfg;
  double c0, r1, r2;  // us per wave; rate with one / two blocks per CU
};
constexpr ModelCfg kModelCfgs[] = {
    {14, 5.0, 9.2, 9.2},  // 256x256, 8 waves
    {21, 3.0, 3.7, 6.1},  // 128x128 BK 128, 2 stages, two per CU
    {7, 3.0, 4.6, 5.9},   // 128x128 BK 64, 4 stages, two per CU
    {25, 3.0, 3.36, 3.36},  // 64x128, 4 stages
    {17, 6.0, 8.0, 8.0},    // 256x128, 8 waves, 3 stages (no K split): grids of 129-256 tiles
};

double model_us(int64_t M, int64_t N, int64_t K, const ModelCfg& mc) {
  const TileCfg& t = kTileCfgs[mc.cfg];
  const int64_t T = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  const int64_t slots = 256 * static_cast<int64_t>(t.per_cu);
  const double blk_ops = 2.0 * t.bm * t.bn * static_cast<double>(K);
  auto wave_us = [&](int64_t units, double kfrac) {
    int64_t b = (units + 255) / 256;
    if (b > t.per_cu) b = t.per_cu;
    const double r = b >= 2 ? mc.r2 : mc.r1;
    return mc.c0 + static_cast<double>(b) * blk_ops * kfrac / (r * 1e6);
  };
  const SplitPlan sp = split_enabled(mc.cfg) ? plan_split(M, N, K, t) : SplitPlan{};
  const int64_t whole = sp.sp > 1 ? sp.full : T;
  double us = static_cast<double>(whole / slots) * wave_us(slots, 1.0);
  if (whole % slots) us += wave_us(whole % slots, 1.0);
  if (sp.sp > 1) {
    us += wave_us(sp.tail * sp.sp, 1.0 / sp.sp);
    us += 2.0 * static_cast<double>(sp.ws) / 4e6 + 3.0;
  }
  const double stream_us = static_cast<double>(N) * static_cast<double>(K) / 3.6e6;
  return us > stream_us ? us : stream_us;
}

int default_tile_cfg(int64_t M, int64_t N, int64_t K) {
  if (K % 64 != 0) return 2;
  int best = 7;
  double best_us = 1e300;
  for (const ModelCfg& mc : kModelCfgs) {
    if (K % kTileCfgs[mc.cfg].bk != 0) continue;
    const double us = model_us(M, N, K, mc);
    if (us < best_us) {
      best_us = us;
      best = mc.cfg;
    }
  }
  return best;
}

// The ring configuration a dense call at (M, N, K) runs (override first).
int select_tile_cfg(int64_t M, int64_t N, int64_t K) {
  const int cfg = g_tile_cfg.load(std::memory_order_relaxed);
  if (cfg < 0 || cfg >= kNumTileCfgs || (kTileCfgs[cfg].dma && K % kTileCfgs[cfg].bk != 0))
    return default_tile_cfg(M, N, K);
  return cfg;
}

template <int BM, int BN, int EPI>
void launch_split_reduce(const GemmArgs& g, const SplitPlan& sp, hipStream_t st) {
  const int64_t threads = sp.tail * BM * (BN / 8);
  hipLaunchKernelGGL((split_reduce_kernel<EPI, BM, BN>),
                     dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, st, g);
}

template <int EPI>
void dispatch_tile(GemmArgs g, void* ws, size_t ws_bytes, hipStream_t st) {
  const int cfg = select_tile_cfg(g.M, g.N, g.K);
  const TileCfg c = kTileCfgs[cfg];
  unsigned tiles =
      static_cast<unsigned>(((g.M + c.bm - 1) / c.bm) * ((g.N + c.bn - 1) / c.bn));
  // K split (ring configurations): needs the caller's workspace
  const SplitPlan sp = plan_split(g.M, g.N, g.K, c);
  const bool split = split_enabled(cfg) && sp.sp > 1 && ws != nullptr && ws_bytes >= sp.ws;
  g.tail_split = 1;
  if (split) {
    g.part = static_cast<int32_t*>(ws);
    g.full_tiles = sp.full;
    g.tail_split = sp.sp;
    tiles = static_cast<unsigned>(sp.full + sp.tail * sp.sp);
  }
  switch (cfg) {
    case 0: launch_tile<256, 256, 128, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 1: launch_tile<256, 256, 64, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 3: launch_tile<256, 128, 128, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 4: launch_tile<128, 256, 128, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 5: launch_tile3<256, 256, 64, 2, 2, 4, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 6: launch_tile3<256, 256, 64, 2, 2, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 7: launch_tile3<128, 128, 64, 2, 2, 4, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 8: launch_tile3<256, 128, 64, 2, 2, 4, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 9: launch_tile3<256, 256, 64, 2, 4, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 10: launch_tile3<256, 256, 64, 4, 2, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 11: launch_tile3<256, 256, 64, 2, 4, 4, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 12: launch_tile3<256, 128, 64, 4, 2, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 13: launch_tile3<256, 256, 64, 4, 4, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 14: launch_tile3<256, 256, 128, 4, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 15: launch_tile3<256, 128, 128, 4, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 16: launch_tile3<256, 256, 128, 4, 4, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 17: launch_tile3<256, 128, 128, 4, 2, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 18: launch_tile3<64, 256, 128, 1, 4, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 19: launch_tile3<64, 128, 128, 1, 4, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 20: launch_tile3<128, 256, 128, 2, 4, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 21: launch_tile3<128, 128, 128, 2, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 22: launch_tile3<64, 256, 64, 1, 4, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 23: launch_tile3<128, 256, 64, 2, 4, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 24: launch_tile3<64, 256, 64, 1, 4, 4, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 25: launch_tile3<64, 128, 128, 1, 4, 4, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 26: launch_tile3<256, 256, 64, 4, 2, 4, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 27: launch_tile3_persist<256, 256, 128, 4, 2, 2, EPI>(g, tiles, c.per_cu, st); break;
    default: launch_tile<128, 128, 128, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
  }
  if (split) {
    switch (c.bm * 1000 + c.bn) {
      case 64256: launch_split_reduce<64, 256, EPI>(g, sp, st); break;
      case 64128: launch_split_reduce<64, 128, EPI>(g, sp, st); break;
      case 128256: launch_split_reduce<128, 256, EPI>(g, sp, st); break;
      case 128128: launch_split_reduce<128, 128, EPI>(g, sp, st); break;
      default: launch_split_reduce<256, 256, EPI>(g, sp, st); break;
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Decode core up to 32 tokens, the tile core above 64.  In between the
// tile core when K % 128 == 0 (its 64-row rings stream 1.2-2x faster than
// the decode core at 33-64 tokens on MI355X), unless a decode
// configuration is forced; a forced tile configuration takes it for any K.
bool use_tile_path(int64_t M, int64_t K) {
  if (M > kDecodeMaxM) return true;
  if (M <= 32 || g_decode_cfg.load(std::memory_order_relaxed) >= 0) return false;
  return K % 128 == 0 || g_tile_cfg.load(std::memory_order_relaxed) >= 0;
}

int gemm_common(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                const void* bias, void* out, int64_t M, int64_t N, int64_t K, void* ws,
                size_t ws_bytes, hipStream_t st, int epi) {
  MW8_REQUIRE(A && W && out, kErrArg, "gemm: null A/W/out");
  MW8_REQUIRE(epi == kEpiI32 || (sa && sw), kErrArg, "gemm: null scales");
  MW8_REQUIRE(M >= 0 && N > 0 && K > 0, kErrShape, "gemm: bad sizes M=%lld N=%lld K=%lld",
              (long long)M, (long long)N, (long long)K);
  MW8_REQUIRE(K % 16 == 0, kErrShape, "gemm: K=%lld must be a multiple of 16", (long long)K);
  MW8_REQUIRE(K <= (1ll << 17), kErrShape, "gemm: K=%lld exceeds the int32-exact bound 131072",
              (long long)K);
  MW8_REQUIRE(aligned16(A) && aligned16(W), kErrAlign, "gemm: A and W need 16-byte alignment");
  if (M == 0) return kOk;
  MW8_REQUIRE(M < (1ll << 31) && N < (1ll << 31), kErrShape, "gemm: M or N too large");

  GemmArgs g{};
  g.A = A; g.sa = sa; g.W = W; g.sw = sw;
  g.bias = static_cast<const uint16_t*>(bias);
  g.out = out; g.M = M; g.N = N; g.K = K; g.lda = K; g.ldo = N;
  g.top_k = 1;
  g.staged_out = epi == kEpiBf16 && N % 8 == 0 && aligned16(out);
  if (!use_tile_path(M, K)) {
    if (epi == kEpiBf16) dispatch_decode<kEpiBf16>(g, st);
    else dispatch_decode<kEpiI32>(g, st);
  } else {
    MW8_REQUIRE(ws == nullptr || aligned16(ws), kErrAlign, "gemm: workspace needs 16-byte alignment");
    if (epi == kEpiBf16) dispatch_tile<kEpiBf16>(g, ws, ws_bytes, st);
    else dispatch_tile<kEpiI32>(g, ws, ws_bytes, st);
  }
  return check_launch("gemm");
}

}  // namespace

void set_tuning(int decode_cfg, int tile_cfg, int moe_cfg) {
  g_decode_cfg.store(decode_cfg, std::memory_order_relaxed);
  g_tile_cfg.store(tile_cfg, std::memory_order_relaxed);
  g_moe_cfg.store(moe_cfg, std::memory_order_relaxed);
}

size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || !use_tile_path(M, K)) return 0;
  const int cfg = select_tile_cfg(M, N, K);
  return split_enabled(cfg) ? plan_split(M, N, K, kTileCfgs[cfg]).ws : 0;
}

int gemm_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                   const void* bias, void* y, int64_t M, int64_t N, int64_t K, void* ws,
                   size_t ws_bytes, hipStream_t st) {
  return gemm_common(A, sa, W, sw, bias, y, M, N, K, ws, ws_bytes, st, kEpiBf16);
}

int gemm_w8a8_i32(const int8_t* A, const int8_t* W, int32_t* acc, int64_t M, int64_t N,
                  int64_t K, void* ws, size_t ws_bytes, hipStream_t st) {
  return gemm_common(A, nullptr, W, nullptr, nullptr, acc, M, N, K, ws, ws_bytes, st, kEpiI32);
}

// Grouped (fused-MoE) GEMM launchers over expert-sorted rows.  BM equals
// the alignment block size, so every block reads one expert's weights.
template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI>
void launch_grouped3(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((g.N + BN - 1) / BN), blocks);
  launch_tile3<BM, BN, BK, WM, WN, NSTAGE, EPI, SortedRows>(g, grid, st);
}

// Run tiles: one block per alignment block; a tile spans up to BM / bm
// consecutive alignment blocks of one expert (SortedRunRows).
template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI>
void launch_grouped_runs(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((g.N + BN - 1) / BN), blocks);
  launch_tile3<BM, BN, BK, WM, WN, NSTAGE, EPI, SortedRunRows>(g, grid, st);
}

// Persistent grouped GEMM: 256 x per_cu blocks walk the (expert chunk,
// column tile) items.
template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI, bool kChunkItems = false, int kPerCu = 1,
          int kAct = -1>
void launch_grouped_persist(const GemmArgs& g, hipStream_t st) {
  constexpr int kLds = NSTAGE * (BM + BN) * BK;
  auto kern = grouped_persist_kernel<BM, BN, BK, WM, WN, NSTAGE, EPI, kChunkItems, kPerCu, kAct>;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(256 * kPerCu)), dim3(64 * WM * WN), kLds, st, g);
}

// Grouped configurations (mw8_set_tuning moe_cfg): 0-6 one tile per
// alignment block (tile height = block size), 7 and 8 run tiles of 256 and
// 128 rows on the 8-wave 256-wide ring (K % 128 == 0), 9-12 the persistent
// item walk with 256x256, 128x256, 256x128 and 128x128 tiles (K % 128 == 0),
// 13 as 9 with chunk items, 14-17 4-wave 128x256 / 256x128 tiles on
// 64-byte K stages, two blocks per CU (expert items, chunk items), 18-19
// 4-wave 128x128 tiles with chunk items, three / four blocks per CU.
//
// Automatic choice, measured on MI355X at config 3 (E 128, top-8, H 2048,
// I 768; whole layer): with at least 32 pairs per expert on average the
// persistent chunk walk on 128x256 tiles, two blocks per CU (cfg 15):
// 1024 tokens 237 -> 215 us, 4096 tokens 536 -> 459 us against cfg 0; at
// 16 pairs per expert (256 tokens) cfg 0 (167 us against 177).  The
// 256-row run tiles (cfg 7/8) lose at every size: three of every four of
// their blocks only read routing metadata and exit.
int default_moe_cfg(const GemmArgs& g, int bm) {
  (void)bm;
  if (g.K % 64 == 0 && g.num_experts < kPersistMaxSlots &&
      g.num_valid >= 32 * static_cast<int64_t>(g.num_experts))
    return 15;
  return 0;
}

template <int EPI>
void launch_grouped_epi(const GemmArgs& g, unsigned blocks, int bm, hipStream_t st) {
  int cfg = g_moe_cfg.load(std::memory_order_relaxed);
  if (g.K % 64 != 0) {  // register-staged core
    const dim3 grid(static_cast<unsigned>((g.N + 127) / 128), blocks);
    if (bm == 64) launch_tile<64, 128, 128, 2, 2, EPI, SortedRows>(g, grid, st);
    else launch_tile<128, 128, 128, 2, 2, EPI, SortedRows>(g, grid, st);
    return;
  }
  const bool bk128 = g.K % 128 == 0;
  if (cfg < 0) cfg = default_moe_cfg(g, bm);
  if (!bk128 && cfg >= 3) cfg = 0;
  if (cfg >= 9 && (cfg >= 14 || bk128) && g.num_experts < kPersistMaxSlots) {  // persistent item walk
    switch (cfg) {
      case 9: launch_grouped_persist<256, 256, 128, 4, 2, 2, EPI>(g, st); break;
      case 10: launch_grouped_persist<128, 256, 128, 2, 4, 2, EPI>(g, st); break;
      case 11: launch_grouped_persist<256, 128, 128, 4, 2, 2, EPI>(g, st); break;
      case 12: launch_grouped_persist<128, 128, 128, 2, 2, 2, EPI, false, 2>(g, st); break;
      case 13: launch_grouped_persist<256, 256, 128, 4, 2, 2, EPI, true>(g, st); break;
      case 14: launch_grouped_persist<128, 256, 64, 2, 2, 3, EPI, false, 2>(g, st); break;
      case 15: launch_grouped_persist<128, 256, 64, 2, 2, 3, EPI, true, 2>(g, st); break;
      case 16: launch_grouped_persist<256, 128, 64, 2, 2, 3, EPI, false, 2>(g, st); break;
      case 17: launch_grouped_persist<256, 128, 64, 2, 2, 3, EPI, true, 2>(g, st); break;
      case 18: launch_grouped_persist<128, 128, 64, 2, 2, 3, EPI, true, 3>(g, st); break;
      default: launch_grouped_persist<128, 128, 64, 2, 2, 2, EPI, true, 4>(g, st); break;
    }
    return;
  }
  if (cfg >= 9) cfg = 0;
  if (cfg == 7 || (cfg == 8 && bm == 128)) {  // 256-row run tiles (bm 64 or 128)
    launch_grouped_runs<256, 256, 128, 4, 2, 2, EPI>(g, blocks, st);
    return;
  }
  if (cfg == 8) {  // 128-row run tiles over 64-row blocks
    launch_grouped_runs<128, 256, 128, 2, 4, 2, EPI>(g, blocks, st);
    return;
  }
  if (bm == 64) {
    switch (cfg) {
      case 1: launch_grouped3<64, 128, 64, 2, 2, 2, EPI>(g, blocks, st); break;
      case 2: launch_grouped3<64, 256, 64, 2, 2, 3, EPI>(g, blocks, st); break;
      case 3: launch_grouped3<64, 256, 128, 2, 4, 2, EPI>(g, blocks, st); break;
      case 4: launch_grouped3<64, 128, 128, 2, 2, 2, EPI>(g, blocks, st); break;
      case 5: launch_grouped3<64, 256, 128, 2, 2, 2, EPI>(g, blocks, st); break;
      case 6: launch_grouped3<64, 128, 128, 2, 4, 3, EPI>(g, blocks, st); break;
      default: launch_grouped3<64, 128, 64, 2, 2, 4, EPI>(g, blocks, st); break;
    }
  } else {
    switch (cfg) {
      case 1: launch_grouped3<128, 128, 64, 2, 2, 2, EPI>(g, blocks, st); break;
      case 2: launch_grouped3<128, 256, 64, 2, 4, 3, EPI>(g, blocks, st); break;
      case 3: launch_grouped3<128, 256, 128, 2, 4, 2, EPI>(g, blocks, st); break;
      case 4: launch_grouped3<128, 128, 128, 2, 2, 2, EPI>(g, blocks, st); break;
      case 5: launch_grouped3<128, 256, 128, 2, 2, 2, EPI>(g, blocks, st); break;
      case 6: launch_grouped3<128, 128, 128, 2, 4, 3, EPI>(g, blocks, st); break;
      default: launch_grouped3<128, 128, 64, 2, 2, 4, EPI>(g, blocks, st); break;
    }
  }
}

// Gate|up GEMM with the gated activation fused (persistent chunk walk, the
// cfg-15 tiling): out [rows, N/2] = act(gate) * up, bf16.
void launch_grouped_act(const GemmArgs& g, int act, hipStream_t st) {
  if (act == 0) launch_grouped_persist<128, 256, 64, 2, 2, 3, kEpiBf16, true, 2, 0>(g, st);
  else launch_grouped_persist<128, 256, 64, 2, 2, 3, kEpiBf16, true, 2, 1>(g, st);
}

void launch_grouped_tile(const GemmArgs& g, unsigned blocks, int bm, int epi, hipStream_t st) {
  if (epi == kEpiBf16) launch_grouped_epi<kEpiBf16>(g, blocks, bm, st);
  else launch_grouped_epi<kEpiI32>(g, blocks, bm, st);
}

void launch_grouped_stream(const GemmArgs& g, unsigned blocks, int epi, hipStream_t st);

// 16- or 32-row alignment blocks on the LDS DMA ring (decode3 core,
// gathered rows; TG token groups of 16).
template <int WAVES, int D, int EPI, int TG = 1, int RG = 1>
void launch_grouped_ring(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  constexpr int kLds = RG * DecodeRing<TG, WAVES, D>::kLds;
  auto kern = decode3_gemm_kernel<TG, WAVES, D, EPI, SortedRows, RG>;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>((g.N + 16 * RG - 1) / (16 * RG)), blocks), dim3(64 * WAVES),
                     kLds, st, g);
}

template <int EPI>
void launch_grouped_ring_cfg(int cfg, const GemmArgs& g, unsigned blocks, hipStream_t st) {
  switch (cfg) {
    case 1: launch_grouped_ring<1, 4, EPI>(g, blocks, st); break;
    case 2: launch_grouped_ring<1, 3, EPI>(g, blocks, st); break;
    case 3: launch_grouped_ring<2, 4, EPI>(g, blocks, st); break;
    case 4: launch_grouped_ring<2, 3, EPI>(g, blocks, st); break;
    case 5: launch_grouped_ring<4, 3, EPI>(g, blocks, st); break;
    case 6: launch_grouped_ring<1, 6, EPI>(g, blocks, st); break;
    case 7: launch_grouped_ring<1, 3, EPI, 1, 2>(g, blocks, st); break;
    default: launch_grouped_ring<2, 3, EPI, 1, 2>(g, blocks, st); break;
  }
}

// 16-row alignment blocks (decode MoE): moe_cfg 0 the register-streaming
// core with the block's tokens gathered in LDS (K <= 4080), 1-6 the LDS DMA
// ring with (waves, ring depth) = (1,4), (1,3), (2,4), (2,3), (4,3), (1,6),
// 7-8 the ring over 32 weight rows per block, (1,3) and (2,3) (16-token
// layer 102 and 111 us against 93 for cfg 2: fewer, larger blocks lose).
// Measured on MI355X at config 3 (whole layer): 16 tokens 120 us (cfg 0)
// -> 107 us (cfg 2), 64 tokens 156 -> 145 us; at 256 tokens the 64-row
// tiles win (167 us against 210 for cfg 2 over 16-row blocks).
int default_stream_cfg(const GemmArgs& g) {
  (void)g;
  return 2;
}

bool grouped_stream_fits(int64_t K) {
  const int64_t ldl = ((K + kStreamStep - 1) / kStreamStep) * kStreamStep + 16;
  return 16 * ldl <= 65536;
}

void launch_grouped_small(const GemmArgs& g, unsigned blocks, int epi, hipStream_t st) {
  if (g.align_bsz == 32) {  // two token groups per block (ring depth 3)
    if (epi == kEpiBf16) launch_grouped_ring<1, 3, kEpiBf16, 2>(g, blocks, st);
    else launch_grouped_ring<1, 3, kEpiI32, 2>(g, blocks, st);
    return;
  }
  int cfg = g_moe_cfg.load(std::memory_order_relaxed);
  if (cfg < 0 || cfg > 8) cfg = default_stream_cfg(g);
  if (cfg == 0 && grouped_stream_fits(g.K)) {
    launch_grouped_stream(g, blocks, epi, st);
    return;
  }
  if (cfg == 0) cfg = 1;
  if (epi == kEpiBf16) launch_grouped_ring_cfg<kEpiBf16>(cfg, g, blocks, st);
  else launch_grouped_ring_cfg<kEpiI32>(cfg, g, blocks, st);
}

// GEMM2 with the fused slot sum (kEpiBf16Sum): the automatic choice of the
// plain GEMM2 for the block size (the tuning override does not apply).
void launch_grouped_sum(const GemmArgs& g, unsigned blocks, int bm, hipStream_t st) {
  if (bm == 32) {
    launch_grouped_ring<1, 3, kEpiBf16Sum, 2>(g, blocks, st);
  } else if (bm == 16) {
    launch_grouped_ring<1, 3, kEpiBf16Sum>(g, blocks, st);
  } else if (default_moe_cfg(g, bm) == 15) {
    launch_grouped_persist<128, 256, 64, 2, 2, 3, kEpiBf16Sum, true, 2>(g, st);
  } else if (bm == 64) {
    launch_grouped3<64, 128, 64, 2, 2, 4, kEpiBf16Sum>(g, blocks, st);
  } else {
    launch_grouped3<128, 128, 64, 2, 2, 4, kEpiBf16Sum>(g, blocks, st);
  }
}

void launch_grouped_stream(const GemmArgs& g, unsigned blocks, int epi, hipStream_t st) {
  const int ldl = static_cast<int>(((g.K + kStreamStep - 1) / kStreamStep) * kStreamStep + 16);
  const size_t lds = static_cast<size_t>(16) * ldl;
  const dim3 grid(static_cast<unsigned>((g.N + kStreamRows - 1) / kStreamRows), blocks);
  if (epi == kEpiBf16)
    hipLaunchKernelGGL(grouped_stream_kernel<kEpiBf16>, grid, dim3(256), lds, st, g);
  else
    hipLaunchKernelGGL(grouped_stream_kernel<kEpiI32>, grid, dim3(256), lds, st, g);
}

}  // namespace mw8
