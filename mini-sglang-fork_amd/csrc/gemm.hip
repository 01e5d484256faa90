// Dense W8A8 GEMM: dispatch between the decode core (M <= 64: weight
// streaming, in-block split-K) and the MFMA tile core (M > 64), plus the
// grouped-tile launchers used by the fused-MoE GEMM.
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

// Ring depth is capped by the token-register ring (D x 4 x TG x 4 VGPRs).
template <int TG, int WAVES, int D, int EPI>
void launch_decode3(const GemmArgs& g, hipStream_t st) {
  constexpr int kD = TG == 1 ? D : (TG == 2 ? (D < 3 ? D : 3) : 2);
  constexpr int kLds = DecodeRing<TG, WAVES, kD>::kLds;
  auto kern = decode3_gemm_kernel<TG, WAVES, kD, EPI>;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    attr_set = true;
  }
  const unsigned blocks = static_cast<unsigned>((g.N + 15) / 16);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * WAVES), kLds, st, g);
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
    default: launch_decode3<TG, 8, 3, EPI>(g, st); break;
  }
}

// Measured on MI355X at the Qwen3-14B shapes (K 5120 / 17408, N 5120 -
// 34816).  Up to 32 tokens the LDS DMA ring (decode3) streams fastest:
// at M = 1, 4 waves x 3 slots per block for wide N (gate_up: 32.6 us,
// 5.5 TB/s) and 2 waves x 2 slots otherwise (o_proj: 7.9 us); for 2-32
// tokens one wave x 4 slots per block (more resident blocks per CU).
// From 33 tokens on the token operand, read per wave through the texture
// path, costs more than the weight stream: the register-streaming core
// with 32 rows over 8 waves (cfg 3) wins, or 64 rows per block for very
// wide N (cfg 4), which keeps fewer blocks re-reading the token panel.
int default_decode_cfg(int64_t M, int64_t N, int64_t K) {
  (void)K;
  if (M == 1) return N >= 16384 ? 14 : 19;
  if (M <= 32) return 20;
  if (M > 48 && N >= 16384) return 4;
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

// 0-4: register-staged tile core (any K % 16 == 0); 5 and up: direct-to-LDS
// ring (K % bk == 0).
struct TileCfg {
  int bm, bn;
  bool dma;
  int bk;
};
constexpr TileCfg kTileCfgs[] = {
    {256, 256, false, 128}, {256, 256, false, 64}, {128, 128, false, 128},
    {256, 128, false, 128}, {128, 256, false, 128},
    {256, 256, true, 64},   // 5: 4 waves, 4 stages
    {256, 256, true, 64},   // 6: 4 waves, 3 stages
    {128, 128, true, 64},   // 7: 4 waves, 4 stages
    {256, 128, true, 64},   // 8: 4 waves, 4 stages
    {256, 256, true, 64},   // 9: 8 waves (2x4), 3 stages
    {256, 256, true, 64},   // 10: 8 waves (4x2), 3 stages
    {256, 256, true, 64},   // 11: 8 waves (2x4), 4 stages
    {256, 128, true, 64},   // 12: 8 waves (4x2), 3 stages
    {256, 256, true, 64},   // 13: 16 waves (4x4), 3 stages
    {256, 256, true, 128},  // 14: 8 waves (4x2), 2 stages
    {256, 128, true, 128},  // 15: 8 waves (4x2), 2 stages
    {256, 256, true, 128},  // 16: 16 waves (4x4), 2 stages
    {256, 128, true, 128},  // 17: 8 waves (4x2), 3 stages
};
constexpr int kNumTileCfgs = sizeof(kTileCfgs) / sizeof(kTileCfgs[0]);

// Split of the last, partial wave of 256 x 256 tiles (one resident tile per
// CU): the r = T mod 256 tail tiles (all T tiles when T < 256) are cut into
// sp = min(256 / r, K / 128, 16) K ranges when that gives sp >= 2.
struct SplitPlan {
  int64_t full = 0, tail = 0;
  int sp = 1;
  size_t ws = 0;
};
constexpr int64_t kSlotsPerWave = 256;

SplitPlan plan_split(int64_t M, int64_t N, int64_t K) {
  SplitPlan p;
  if (M <= kDecodeMaxM || K % 128 != 0) return p;
  const int64_t T = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t r = T % kSlotsPerWave;
  if (r == 0) return p;
  int64_t sp = kSlotsPerWave / r;
  const int64_t nkt = K / 128;
  if (sp > nkt) sp = nkt;
  if (sp > 16) sp = 16;
  if (sp < 2) return p;
  p.full = T - r;
  p.tail = r;
  p.sp = static_cast<int>(sp);
  p.ws = static_cast<size_t>(r) * sp * 65536 * sizeof(int32_t);
  return p;
}

// Pick the configuration with the smallest modelled time: waves of
// resident tiles x per-wave tile area / relative efficiency.  The
// efficiencies are per-op throughputs measured on MI355X relative to the
// 128x128 ring (cfg 7, two blocks per CU): the 8-wave 256x256 BK=128 ring
// with 64x128 wave tiles (cfg 14, one block per CU) runs ~1.35x faster per
// op at K ~ 5K and ~1.37x at K ~ 17K (3-5% ahead of the 16-wave cfg 16);
// the 8-wave 256x128 ring (cfg 12, two blocks per CU) ~1.12x.  Shapes with
// K % 64 != 0 use the register-staged core.
int default_tile_cfg(int64_t M, int64_t N, int64_t K) {
  if (K % 64 != 0) return 2;
  struct Cand {
    int cfg, per_cu;
    double eff;
  };
  const Cand cands[] = {{14, 1, K > 8192 ? 1.37 : 1.35}, {12, 2, 1.12}, {7, 2, 1.0}};
  int best = 7;
  double best_cost = 1e300;
  const SplitPlan sp = plan_split(M, N, K);
  for (const Cand& c : cands) {
    const TileCfg t = kTileCfgs[c.cfg];
    if (K % t.bk != 0) continue;
    const int64_t tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
    const int64_t slots = 256 * static_cast<int64_t>(c.per_cu);
    double waves = static_cast<double>((tiles + slots - 1) / slots);
    // the 256 x 256 tail split: full waves plus one wave of 1/sp-length units
    // (and the partial-tile reduction, modelled as a tenth of a wave)
    if (t.bm == 256 && t.bn == 256 && sp.sp > 1)
      waves = static_cast<double>(sp.full / kSlotsPerWave) + 1.0 / sp.sp + 0.1;
    const double cost = waves * t.bm * t.bn * c.per_cu / c.eff;
    if (cost < best_cost) {
      best_cost = cost;
      best = c.cfg;
    }
  }
  return best;
}

template <int EPI>
void dispatch_tile(GemmArgs g, void* ws, size_t ws_bytes, hipStream_t st) {
  int cfg = g_tile_cfg.load(std::memory_order_relaxed);
  if (cfg < 0 || cfg >= kNumTileCfgs || (kTileCfgs[cfg].dma && g.K % kTileCfgs[cfg].bk != 0))
    cfg = default_tile_cfg(g.M, g.N, g.K);
  const TileCfg c = kTileCfgs[cfg];
  unsigned tiles =
      static_cast<unsigned>(((g.M + c.bm - 1) / c.bm) * ((g.N + c.bn - 1) / c.bn));
  // tail split (256 x 256 ring configurations): needs the caller's workspace
  const SplitPlan sp = plan_split(g.M, g.N, g.K);
  const bool split = c.dma && c.bm == 256 && c.bn == 256 && sp.sp > 1 && ws != nullptr &&
                     ws_bytes >= sp.ws && g.K % c.bk == 0;
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
    default: launch_tile<128, 128, 128, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
  }
  if (split) {
    const int64_t threads = sp.tail * 256 * 32;
    hipLaunchKernelGGL(split_reduce_kernel<EPI>, dim3(static_cast<unsigned>((threads + 255) / 256)),
                       dim3(256), 0, st, g);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }



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
  if (M <= kDecodeMaxM) {
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
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return plan_split(M, N, K).ws;
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

// Grouped configurations (mw8_set_tuning moe_cfg): 0-6 one tile per
// alignment block (tile height = block size), 7 and 8 run tiles of 256 and
// 128 rows on the 8-wave 256-wide ring (K % 128 == 0).  Automatic choice:
// cfg 0.  Measured on MI355X at config 3 (E 128, top-8, H 2048, I 768) the
// run tiles lose at 256, 1024 and 4096 tokens (226 / 308 / 614 us per layer
// against 169 / 238 / 548 us): three of every four run-tile blocks only
// read the routing metadata and exit, each holding the CU's LDS through a
// chain of dependent loads of arrays the alignment kernel has just written.
int default_moe_cfg(const GemmArgs& g, int bm) {
  (void)g;
  (void)bm;
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

void launch_grouped_tile(const GemmArgs& g, unsigned blocks, int bm, int epi, hipStream_t st) {
  if (epi == kEpiBf16) launch_grouped_epi<kEpiBf16>(g, blocks, bm, st);
  else launch_grouped_epi<kEpiI32>(g, blocks, bm, st);
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
