// Dense W8A8 GEMM: dispatch between the decode cores (M <= 32, or up to 64
// when K % 128 != 0: weight streaming, in-block split-K) and the MFMA tile
// ring, plus the grouped-tile launchers used by the fused-MoE GEMM.
#include <atomic>
#include <type_traits>

#include "gemm_kernels.h"
#include "gemm_ksplit.h"
#include "gemm_stream.h"

namespace mw8 {

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

// Raises the dynamic-LDS limit of kernel Kern to `bytes`, once per device
// (the attribute is set on the current device); returns kOk or an error.
template <auto Kern>
int set_lds_limit(int bytes) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(kErrLaunch, "hipGetDevice: %s", hipGetErrorString(e));
  const uint64_t bit = dev >= 0 && dev < 64 ? uint64_t{1} << dev : 0;
  if (bit != 0 && (done.load(std::memory_order_acquire) & bit) != 0) return kOk;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(Kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          bytes);
  if (e != hipSuccess)
    return set_error(kErrLaunch, "hipFuncSetAttribute(%d bytes of LDS): %s", bytes, hipGetErrorString(e));
  done.fetch_or(bit, std::memory_order_acq_rel);
  return kOk;
}

namespace {

constexpr int64_t kDecodeMaxM = 64;

// Tuning override (-1 = automatic), per calling thread: set through
// mw8_set_tuning, it changes the choice for the calls of the thread that set
// it and leaves every other thread on the automatic choice.
thread_local int g_decode_cfg = -1;
thread_local int g_tile_cfg = -1;
thread_local int g_moe_cfg = -1;

// ------------------------------------------------------------------ decode
// core 0: decode_gemm_kernel (RG 16-row groups per block, WAVES waves, D = U
// K steps per load batch); core 1: decode3_gemm_kernel over a CU-balanced
// grid (a multiple of the CU count, each block up to 16 RG rows, D = ring
// depth); core 2: decode_sx_gemm_kernel (up to 64 tokens, K % 256 == 0:
// one block per CU, a wave per 16 rows of its range, a shared token ring;
// waves from N, D = ring depth; other sizes take the automatic choice).
struct DecodeCfg {
  int core, rg, waves, d;
};
constexpr DecodeCfg kDecodeCfgs[] = {
    {0, 2, 8, 4},  // 0: 32 rows over 8 waves (33-64 tokens with K % 128 != 0)
    {0, 4, 4, 4},  // 1: 64 rows over 4 waves (very wide N at 49-64 tokens)
    {1, 1, 1, 4},  // 2
    {1, 1, 2, 2},  // 3
    {1, 2, 1, 4},  // 4
    {1, 2, 4, 2},  // 5
    {1, 2, 4, 3},  // 6
    {1, 2, 8, 2},  // 7
    {2, 1, 0, 3},  // 8: shared token ring, 3 stages
    {2, 1, 0, 4},  // 9: shared token ring, 4 stages for up to 16 tokens (else 3)
};
constexpr int kNumDecodeCfgs = sizeof(kDecodeCfgs) / sizeof(kDecodeCfgs[0]);

template <int RG, int TG, int WAVES, int U, int EPI>
int launch_decode(const GemmArgs& g, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>((g.N + 16 * RG - 1) / (16 * RG));
  hipLaunchKernelGGL((decode_gemm_kernel<RG, TG, WAVES, U, EPI>), dim3(blocks), dim3(64 * WAVES), 0, st, g);
  return kOk;
}

// Ring depth is capped by the token-register ring (D x 4 x TG x 4 VGPRs).
template <int TG, int WAVES, int D, int EPI, int RG>
int launch_decode3_bal(const GemmArgs& g, hipStream_t st) {
  constexpr int kD = TG == 1 ? D : (TG == 2 ? (D < 3 ? D : 3) : 2);
  constexpr int kLds = RG * DecodeRing<TG, WAVES, kD>::kLds;
  constexpr auto kern = decode3_gemm_kernel<TG, WAVES, kD, EPI, DenseRows, RG>;
  if (const int rc = set_lds_limit<kern>(kLds)) return rc;
  const int64_t cus = device_cus();
  const int64_t blocks = cus * ((g.N + cus * 16 * RG - 1) / (cus * 16 * RG));
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(64 * WAVES), kLds, st, g);
  return kOk;
}

// Fused quantization (bf16 activation rows, kXQ): the decode3
// configurations with one token group.
template <int WAVES, int D, int RG>
int launch_decode3_xq(const GemmArgs& g, hipStream_t st) {
  constexpr int kLds = RG * DecodeRing<1, WAVES, D>::kLds;
  constexpr auto kern = decode3_gemm_kernel<1, WAVES, D, kEpiBf16, DenseRows, RG, true>;
  if (const int rc = set_lds_limit<kern>(kLds)) return rc;
  const int64_t cus = device_cus();
  const int64_t blocks = cus * ((g.N + cus * 16 * RG - 1) / (cus * 16 * RG));
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(64 * WAVES), kLds, st, g);
  return kOk;
}

// core 2: one block per CU (a multiple of the CU count), a wave per 16 rows
// of the widest block's range, TG = ceil(M / 16) token groups; the LDS of
// (WAVES + TG) D stages of 4 KB bounds the waves: WAVES + TG <= 40 / D.
bool sx_fits(int64_t M, int64_t K) { return M >= 1 && M <= 64 && K % 256 == 0; }

constexpr int sx_max_waves(int tg, int d) { return 40 / d - tg; }

void sx_plan(int64_t N, int tg, int d, int& waves, int64_t& blocks) {
  const int64_t cus = device_cus();
  const int64_t per = cus * 16 * sx_max_waves(tg, d);
  blocks = cus * ((N + per - 1) / per);
  waves = static_cast<int>(((N + blocks - 1) / blocks + 15) / 16);
  if (waves < tg) waves = tg;  // wave t issues token group t
}

template <int TG, int WAVES, int D, int EPI>
int launch_decode_sx_w(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  constexpr int kLds = (WAVES + TG) * D * kRingStage;
  static_assert(kLds <= 163840, "LDS");
  constexpr auto kern = decode_sx_gemm_kernel<TG, WAVES, D, EPI>;
  if (const int rc = set_lds_limit<kern>(kLds)) return rc;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * WAVES), kLds, st, g);
  return kOk;
}

// the instance with `waves` waves among WAVES .. sx_max_waves(TG, D)
template <int TG, int D, int EPI, int WAVES = TG>
int launch_decode_sx_n(const GemmArgs& g, int waves, unsigned blocks, hipStream_t st) {
  if constexpr (WAVES < sx_max_waves(TG, D)) {
    if (waves > WAVES) return launch_decode_sx_n<TG, D, EPI, WAVES + 1>(g, waves, blocks, st);
  }
  return launch_decode_sx_w<TG, WAVES, D, EPI>(g, blocks, st);
}

template <int TG, int D, int EPI>
int launch_decode_sx_tg(const GemmArgs& g, hipStream_t st) {
  int waves = 0;
  int64_t blocks = 0;
  sx_plan(g.N, TG, D, waves, blocks);
  MW8_REQUIRE(blocks < (int64_t{1} << 31), kErrShape, "gemm: N=%lld too large", (long long)g.N);
  return launch_decode_sx_n<TG, D, EPI>(g, waves, static_cast<unsigned>(blocks), st);
}

// D = 4 stages for one token group (D = 3 otherwise: LDS)
template <int EPI>
int launch_decode_sx(const GemmArgs& g, int d, hipStream_t st) {
  switch ((g.M + 15) / 16) {
    case 1: return d == 4 ? launch_decode_sx_tg<1, 4, EPI>(g, st) : launch_decode_sx_tg<1, 3, EPI>(g, st);
    case 2: return launch_decode_sx_tg<2, 3, EPI>(g, st);
    case 3: return launch_decode_sx_tg<3, 3, EPI>(g, st);
    default: return launch_decode_sx_tg<4, 3, EPI>(g, st);
  }
}

template <int TG, int EPI>
int decode_by_cfg(int cfg, const GemmArgs& g, hipStream_t st) {
  switch (cfg) {
    case 0: return launch_decode<2, TG, 8, 4, EPI>(g, st);
    case 1: return launch_decode<4, TG, 4, 4, EPI>(g, st);
    case 2: return launch_decode3_bal<TG, 1, 4, EPI, 1>(g, st);
    case 3: return launch_decode3_bal<TG, 2, 2, EPI, 1>(g, st);
    case 4: return launch_decode3_bal<TG, 1, 4, EPI, 2>(g, st);
    case 5: return launch_decode3_bal<TG, 4, 2, EPI, 2>(g, st);
    case 6: return launch_decode3_bal<TG, 4, 3, EPI, 2>(g, st);
    default: return launch_decode3_bal<TG, 8, 2, EPI, 2>(g, st);
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
// rows at one token (and at 2-8 tokens for K > 8192: down M=2 / 8 17.0-17.2
// / 17.6-17.8 us against 17.4 / 17.9-18.2 for 8 waves x 2), 8 waves x 2
// slots up to 8 and from 17 tokens, 4 waves x 2 slots at 9-16.  Wide N
// (gate_up, 2176 row groups): 16-row blocks, 2 waves x 2 slots at one
// token (30.6 us, 5.8 TB/s), one wave x 4 slots up to 8, 32-row blocks of
// one wave x 4 slots at 17-32 tokens.
// Wide N at 4-64 tokens (K % 256 == 0, one block per CU covering the
// widest row range): the shared token ring (cfg 8).  The one-wave blocks
// re-read the token panel per 16 rows (gate_up at 8 tokens: 13% more L2
// read requests than the weights alone), and from 33 tokens the 64x128
// ring runs a K-split tail.  Same box, us, previous automatic choice ->
// cfg 8: N 34816, K 5120 at 4 / 8 / 12 / 16 / 24 / 32 / 48 / 64 tokens
// 31.7 / 34.2 / 37.5 / 40.6 / 43.4 / 51.1 / 46.1 / 48.0 -> 31.4 / 31.4 /
// 31.7 / 31.7 / 32.3 / 34.3 / 36.2 / 38.5; N 16384 at 8 tokens 17.5 ->
// 16.7; N 51200 at 8 / 16 tokens 47.9 / 56.0 -> 45.1 / 46.1 (at 64 tokens
// two blocks per CU: 63.0 against 61.9 for the tile ring, not taken); at
// 2-3 tokens decode3 stays (29.5 / 31.1 against 30.5 / 31.2).  With
// K = 8192 and the walk staggered per block, level with the K-split decode3
// (N 25600: 36.0 / 36.2; N 34816: 45.8 / 44.1) and ahead of the one-wave
// blocks (55.7).
// From 33 tokens on the token operand, read per wave through the texture
// path, costs more than the weight stream: the register-streaming core
// with 32 rows over 8 waves (cfg 0) wins, or 64 rows per block for very
// wide N (cfg 1), which keeps fewer blocks re-reading the token panel.
// Whether the shared token ring is the automatic choice at (M, N, K): wide
// N at 4-64 tokens, one block per CU holding the widest row range.
bool sx_default(int64_t M, int64_t N, int64_t K) {
  if (N < 16384 || M < 4 || !sx_fits(M, K)) return false;
  const int tg = static_cast<int>((M + 15) / 16);
  return (N + device_cus() - 1) / device_cus() <= 16 * sx_max_waves(tg, 3);
}

int default_decode_cfg(int64_t M, int64_t N, int64_t K) {
  const bool wide = N >= 16384;
  if (M == 1) return wide ? 3 : 6;
  if (sx_default(M, N, K)) return 8;
  if (M <= 8) return wide ? 2 : (K > 8192 ? 6 : 7);
  if (M <= 16) return 5;
  if (M <= 32) return wide ? 4 : 7;
  if (M > 48 && wide) return 1;
  return 0;
}

template <int EPI>
int dispatch_decode(const GemmArgs& g, hipStream_t st) {
  const int tg = static_cast<int>((g.M + 15) / 16);
  int cfg = g_decode_cfg;
  if (cfg < 0 || cfg >= kNumDecodeCfgs) cfg = default_decode_cfg(g.M, g.N, g.K);
  if (kDecodeCfgs[cfg].core == 2) {
    if (sx_fits(g.M, g.K)) return launch_decode_sx<EPI>(g, kDecodeCfgs[cfg].d, st);
    cfg = default_decode_cfg(g.M, g.N, g.K);
  }
  switch (tg) {
    case 1: return decode_by_cfg<1, EPI>(cfg, g, st);
    case 2: return decode_by_cfg<2, EPI>(cfg, g, st);
    case 3: return decode_by_cfg<3, EPI>(cfg, g, st);
    default: return decode_by_cfg<4, EPI>(cfg, g, st);
  }
}

// -------------------------------------------------------------------- tile
template <int BM, int BN, int BK, int WM, int WN, int EPI, class Rows>
int launch_tile(const GemmArgs& g, dim3 grid, hipStream_t st) {
  using S = TileShape<BM, BN, BK, WM, WN>;
  constexpr auto kern = tile_gemm_kernel<BM, BN, BK, WM, WN, EPI, Rows>;
  if (const int rc = set_lds_limit<kern>(S::kLds)) return rc;
  hipLaunchKernelGGL(kern, grid, dim3(256), S::kLds, st, g);
  return kOk;
}

// The dense 256 x 256 ring streams its weight stages one stage ahead of its
// A stages (2 A slots + 3 W slots of 32 KB, the whole LDS; the scale tables
// move into the ring after the main loop).  Measured on MI355X (graph-timed,
// rotating weights, us, lead 0 -> 1, bit-identical): gate_up M=8192
// 1182.1 -> 1153.8, M=4096 620.3 -> 607.8; 8192 x 5120 x 17408 600.1 ->
// 575.8; qkv M=8192 261.9 -> 259.3, M=4096 137.0 -> 132.5; 2080 x 10240 x
// 5120 130.2 -> 122.8.  The weights' first touch comes from HBM, and one
// stage of MFMA time does not cover it; the A panels mostly hit in L2.
// The 128 x 128 (two per CU) and 64 x 128 rings gain 1-3% from the same
// lead (256 x 5120 x 17408 49.6 -> 48.5, 256 x 7168 x 5120 33.4 -> 32.5;
// 64 x 5120 x 17408 26.3 -> 25.8, 64 x 34816 x 5120 47.5 -> 46.7); the
// 3-stage 256 x 128 ring, whose weights are already two stages ahead,
// loses 1-4% with it (2080 x 10240 x 5120 120.3 -> 123.3) and keeps none.
// With the lead the 256 x 256 tile runs its 8 waves as 2 x 4 of 128 x 64
// (one A fragment set, re-read during the last column block) rather than
// 4 x 2 of 64 x 128: 8 alternating rounds, us, 4x2 -> 2x4, bit-identical:
// gate_up M=8192 1153.7 -> 1142.4, M=4096 608.7 -> 604.2; 2080 x 10240 x
// 5120 125.9 -> 125.0; qkv M=8192 256.4 -> 256.2.  The 256 x 320 ring
// (no lead) gains more from 2 x 4 waves of 128 x 80, which spill 60 bytes
// per lane against 144 for 4 x 2 of 64 x 160 (6 alternating rounds, us):
// 8192 x 5120 x 17408 575.3 -> 534.3, 8192 x 5120 x 5120 193.8 -> 175.4,
// 4096 x 5120 x 17408 298.9 -> 276.8, 4096 x 5120 x 5120 103.5 -> 91.9,
// 512 x 34816 x 5120 104.7 -> 99.1.
constexpr int kLead256 = 1, kLeadSmall = 1;

// 128-byte K stages hold two 64-byte substeps of v_mfma_i32_16x16x64_i8
// (the int8 MFMA with the higher power-limited rate on MI355X); 64-byte
// stages run v_mfma_i32_32x32x32_i8 (two 32-byte substeps).
template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI, class Rows, int kWAux = 0, int kBLead = 0>
int launch_tile3(const GemmArgs& g, dim3 grid, hipStream_t st) {
  constexpr int kLds = NSTAGE * BM * BK + (NSTAGE + kBLead) * BN * BK;
  constexpr auto kern =
      tile3_gemm_kernel<BM, BN, BK, WM, WN, NSTAGE, EPI, Rows, kWAux, BK == 128 ? 16 : 32, -1, kBLead>;
  if (const int rc = set_lds_limit<kern>(kLds)) return rc;
  hipLaunchKernelGGL(kern, grid, dim3(64 * WM * WN), kLds, st, g);
  return kOk;
}

// 0: register-staged tile core (any K % 16 == 0); 1 and up: direct-to-LDS
// ring (K % bk == 0).  per_cu: resident blocks per CU (LDS-bound); split:
// the K split of the last partial wave applies.
struct TileCfg {
  int bm, bn;
  bool dma;
  int bk, per_cu;
  bool split;
  const char* name;  // kernel name with its leading template arguments, as a trace shows it
};
constexpr TileCfg kTileCfgs[] = {
    // 0: register-staged, 4 waves
    {128, 128, false, 128, 2, false, "tile_gemm_kernel<128, 128, 128, 2, 2>"},
    // 1: ring, 4 waves (2x2), 4 stages, two per CU
    {128, 128, true, 64, 2, false, "tile3_gemm_kernel<128, 128, 64, 2, 2, 4>"},
    // 2: ring, 8 waves (2x4 of 128 x 64), 2 stages (the weight stages a
    // stage further ahead, in a ring of 3: kLead256)
    {256, 256, true, 128, 1, true, "tile3_gemm_kernel<256, 256, 128, 2, 4, 2>"},
    // 3: ring, 8 waves (4x2), 3 stages: grids of 129-256 tiles
    {256, 128, true, 128, 1, false, "tile3_gemm_kernel<256, 128, 128, 4, 2, 3>"},
    // 4: ring, 4 waves (2x2), 2 stages (weight lead: kLeadSmall), two per CU
    {128, 128, true, 128, 2, true, "tile3_gemm_kernel<128, 128, 128, 2, 2, 2>"},
    // 5: ring, 4 waves (1x4), 4 stages (weight lead: kLeadSmall)
    {64, 128, true, 128, 1, true, "tile3_gemm_kernel<64, 128, 128, 1, 4, 4>"},
    // 6: ring, 8 waves (2x4 of 128 x 80), 2 stages, the bf16 tile staged in
    // two row passes: N = 5120 at 4096 / 8192 rows in whole waves of the CUs
    // (no LDS for a weight lead: 2 x 32 KB A + 3 x 40 KB W would be 184 KB)
    {256, 320, true, 128, 1, false, "tile3_gemm_kernel<256, 320, 128, 2, 4, 2>"},
    // 7: the pipelined persistent walk over 256x256 tiles (bf16 output, at
    // least 6 K stages and one tile per CU; else as cfg 2)
    {256, 256, true, 128, 1, false, "stream_gemm_kernel<256, 0, false, -1>"},
};
constexpr int kNumRingCfgs = sizeof(kTileCfgs) / sizeof(kTileCfgs[0]);

// In-block split-K configurations (ksplit_gemm_kernel), tile cfg
// kNumRingCfgs + i: block tile BM x BN, KG K groups of WM x WN waves, KS
// 32-byte k-steps per group and stage, NSTAGE stages.
struct KsplitCfg {
  int bm, bn, kg, wm, wn, ks, nstage;
  const char* name;
};
constexpr KsplitCfg kKsplitCfgs[] = {
    {64, 32, 8, 1, 1, 1, 4, "ksplit_gemm_kernel<64, 32, 8, 1, 1, 1, 4>"},      // 0: 256-byte stages, waves of 64 x 32
    {64, 32, 8, 1, 1, 2, 3, "ksplit_gemm_kernel<64, 32, 8, 1, 1, 2, 3>"},      // 1: 512-byte stages, waves of 64 x 32
    {64, 64, 8, 1, 1, 1, 4, "ksplit_gemm_kernel<64, 64, 8, 1, 1, 1, 4>"},      // 2: 256-byte stages, waves of 64 x 64
    {128, 64, 4, 2, 1, 2, 3, "ksplit_gemm_kernel<128, 64, 4, 2, 1, 2, 3>"},    // 3: 256-byte stages, 2 k-steps per stage
    {128, 128, 2, 2, 2, 2, 3, "ksplit_gemm_kernel<128, 128, 2, 2, 2, 2, 3>"},  // 4: 128-byte stages, 2 k-steps
};
constexpr int kNumKsplitCfgs = sizeof(kKsplitCfgs) / sizeof(kKsplitCfgs[0]);
constexpr int kNumTileCfgs = kNumRingCfgs + kNumKsplitCfgs;

constexpr int ksplit_sk(const KsplitCfg& c) { return c.kg * c.ks * 32; }

// Column ranges of a ksplit grid over N: the fewest whose boundaries are
// multiples of 16 and whose widest range fits BN, raised so that the grid
// of gm x gn blocks fills whole waves of the CUs.  0 if no range fits.
int64_t ksplit_ranges(int64_t M, int64_t N, const KsplitCfg& c, int64_t& gm) {
  gm = (M + c.bm - 1) / c.bm;
  const int64_t n16 = N / 16, tail = N % 16;
  const int64_t q = (c.bn - tail) / 16;  // 16-column groups a range may hold
  if (q < 1) return 0;
  int64_t gn = n16 == 0 ? 1 : (n16 + q - 1) / q;
  const int64_t cus = device_cus();
  const int64_t waves = (gm * gn + cus - 1) / cus;
  const int64_t fill = waves * cus / gm;
  const int64_t most = n16 > 0 ? n16 : 1;  // every range keeps at least 16 columns
  if (fill > gn) gn = fill < most ? fill : most;
  return gn;
}

// K split of a ring tiling.  With T tiles and S = CUs * per_cu resident
// slots: T >= S cuts the r = T mod S tiles of the last, partial wave into
// sp = min(S / r, K / bk, 16) K ranges; T < S cuts every tile into
// sp = min(S / T, K / bk, 16) ranges.  No split when sp < 2, nor for a tail
// of more than a third of a wave (sp < 3): a partial last wave costs about
// one tile time whatever its occupancy, while two K ranges add the partial
// tiles' round trip and the reduction launch (256x256 tiles on MI355X,
// with / without the split: gate_up M=4096 729 / 669 us, o_proj M=8192
// 220 / 206, qkv M=8192 296 / 278; with sp >= 4 the split wins: o_proj
// M=4096 124 / 126, gate_up M=1024 213 / 229).  r * sp <= S, so the
// workspace never exceeds S * bm * bn int32 values.
struct SplitPlan {
  int64_t full = 0, tail = 0;
  int sp = 1;
  size_t ws = 0;
};

SplitPlan plan_split(int64_t M, int64_t N, int64_t K, const TileCfg& c) {
  SplitPlan p;
  if (!c.dma || !c.split || K % c.bk != 0) return p;
  const int64_t T = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
  const int64_t slots = static_cast<int64_t>(device_cus()) * c.per_cu;
  const int64_t r = T >= slots ? T % slots : T;
  if (r == 0) return p;
  int64_t sp = slots / r;
  const int64_t nkt = K / c.bk;
  if (sp > nkt) sp = nkt;
  if (sp > 16) sp = 16;
  if (sp < 2 || (T >= slots && sp < 3)) return p;
  p.full = T - r;
  p.tail = r;
  p.sp = static_cast<int>(sp);
  p.ws = static_cast<size_t>(r) * sp * c.bm * c.bn * sizeof(int32_t);
  return p;
}

// Modelled time (us) of one ring configuration: waves of resident blocks,
// each wave costing c0 + b x (block ops) / (per-CU rate with b blocks
// resident on the busiest CU), plus the K split's partial tiles (written
// and read back at ~4 TB/s) and its reduction launch, floored by the
// weight stream (~3.6 TB/s for these tilings).  Rates (TOPS per CU) fitted
// to MI355X sweeps of the Qwen3-14B shapes at M = 40 - 8192.  The 256x256
// rate was raised with the weight lead (us, 256x256 vs 256x320, same box):
// 4096 x 34816 x 5120 632.1 vs 659.3, 8192 x 7168 x 5120 263.3 vs 276.1;
// the N = 5120 shapes keep 256x320's whole waves (8192 x 5120 x 17408 597.7
// vs 572.9, 4096 x 5120 x 5120 117.9 vs 101.7).  With 2 x 4 waves the
// 256x320 rate rose in turn (256x256 vs 256x320, us): qkv M=8192 255.8 vs
// 250.2 and 6144 x 10240 x 5120 263.9 vs 256.4 go to 256x320; 4096 x 51200
// x 5120 907.9 vs 941.7, 6144 x 34816 x 5120 868.0 vs 892.5, 2080 x 34816 x
// 5120 338.9 vs 350.4 and qkv M=4096 133.0 vs 158.9 stay on 256x256.  One
// rate cannot also give gate_up M=4096 to 256x320 (605.8 vs 600.4) without
// taking 4096 x 51200 from 256x256; the model keeps the smaller miss.
struct ModelCfg {
  int cfg;
  double c0, r1, r2;  // us per wave; rate with one / two blocks per CU
};
constexpr ModelCfg kModelCfgs[] = {
    {2, 5.0, 9.8, 9.8},     // 256x256, 8 waves, weight lead (gate_up M=4096 and qkv M=8192 over 256x320)
    {4, 3.0, 3.7, 6.1},     // 128x128 BK 128, 2 stages, two per CU
    {1, 3.0, 4.6, 5.9},     // 128x128 BK 64, 4 stages, two per CU
    {5, 3.0, 3.36, 3.36},   // 64x128, 4 stages
    {3, 6.0, 8.0, 8.0},     // 256x128, 8 waves, 3 stages (no K split): grids of 129-256 tiles
    {6, 5.0, 9.2, 9.2},     // 256x320, 8 waves 2x4 (near-ties go to 256x256)
};

double model_us(int64_t M, int64_t N, int64_t K, const ModelCfg& mc) {
  const TileCfg& t = kTileCfgs[mc.cfg];
  const int64_t cus = device_cus();
  const int64_t T = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  const int64_t slots = cus * t.per_cu;
  const double blk_ops = 2.0 * t.bm * t.bn * static_cast<double>(K);
  auto wave_us = [&](int64_t units, double kfrac) {
    int64_t b = (units + cus - 1) / cus;
    if (b > t.per_cu) b = t.per_cu;
    const double r = b >= 2 ? mc.r2 : mc.r1;
    return mc.c0 + static_cast<double>(b) * blk_ops * kfrac / (r * 1e6);
  };
  const SplitPlan sp = plan_split(M, N, K, t);
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

// In-block split-K choice, measured on MI355X (us per launch, weights
// streamed from HBM; auto = the best ring configuration):
//              M = 40     64    128    256    512   1024
//   qkv  ks     12.8   14.3   18.6   24.1   36.8   69.6
//        auto   16.5   16.8   23.6   27.0   38.7   42.9
//   o    ks     11.8   13.2   16.7   21.8   32.3   62.4
//        auto   15.9   16.5   19.3   26.1   37.4   40.5
// With K > 8192 (down, K = 17408) every block re-reads a long token panel
// and with N > 16384 (gate_up) the ring already fills the CUs: the ring
// wins there.  Above 64 rows the tile is the smallest of 64 x 64, 128 x 64
// and 128 x 128 whose fewest column ranges fit one wave of the CUs (a second
// wave costs nearly a whole launch), and the ring when none does; same box,
// chosen tile (runner-up in brackets):
//   qkv M=192  128x64 20.4 (64x64 30.2)    qkv M=384  128x128 31.2 (128x64 38.9)
//   o   M=192  64x64  17.6 (128x64 19.4)   qkv M=640  ring 256x128 40.9 (128x128 58.2)
//   o   M=768  128x128 34.7 (ring 39.1)    qkv M=768  ring 256x128 44.3 (128x128 61.0)
// Split-K stages: the 128 x 128 tile runs 3 stages of 32 KB (64 KB in
// flight); 4 stages measured 1-4% slower at M = 384-768 (the per-CU operand
// stream saturates near 48 GB/s, not on the bytes in flight).
int64_t ksplit_min_waves(int64_t M, int64_t N, const KsplitCfg& c) {
  const int64_t q = (c.bn - N % 16) / 16;
  if (q < 1) return INT64_MAX;
  const int64_t gn = N < 16 ? 1 : (N / 16 + q - 1) / q;
  const int64_t cus = device_cus();
  return ((M + c.bm - 1) / c.bm * gn + cus - 1) / cus;
}

int default_ksplit_cfg(int64_t M, int64_t N, int64_t K) {
  if (M > 768 || N > 16384 || K > 8192) return -1;
  if (M <= 64) return K % 512 == 0 ? 1 : (K % 256 == 0 ? 0 : -1);
  if (K % 256 != 0) return -1;
  for (const int c : {2, 3, 4})
    if (ksplit_min_waves(M, N, kKsplitCfgs[c]) <= 1) return c;
  return -1;
}

// The stream walk (cfg 7) replaces the one-tile 256 x 256 ring (cfg 2)
// where its tiles are short: fewer than 16 K stages of 128 bytes, at least
// one tile per CU.  Measured on MI355X (graph-timed, rotating weights, us,
// cfg 2 -> cfg 7, bit-identical): 32768 x 2048 x 768 71.9 -> 64.2, 32768 x
// 1536 x 2048 101.9 -> 100.1; with 40 or more stages the walk's static tile
// lists lose to the hardware's dynamic block dispatch (gate_up M=8192 1160
// -> 1228, down M=8192 591 -> 635, qkv M=8192 263 -> 283).
constexpr int64_t kStreamMaxStages = 15;

int default_tile_cfg(int64_t M, int64_t N, int64_t K) {
  if (K % 64 != 0) return 0;
  const int ks = default_ksplit_cfg(M, N, K);
  if (ks >= 0) return kNumRingCfgs + ks;
  int best = 1;
  double best_us = 1e300;
  for (const ModelCfg& mc : kModelCfgs) {
    if (K % kTileCfgs[mc.cfg].bk != 0) continue;
    const double us = model_us(M, N, K, mc);
    if (us < best_us) {
      best_us = us;
      best = mc.cfg;
    }
  }
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  if (best == 2 && K % kStreamBK == 0 && K / kStreamBK >= kStreamMinStages && K / kStreamBK <= kStreamMaxStages &&
      tiles >= device_cus() && plan_split(M, N, K, kTileCfgs[2]).sp <= 1)
    return 7;
  return best;
}

// The ring configuration a dense call at (M, N, K) runs (override first).
bool tile_cfg_fits(int cfg, int64_t M, int64_t N, int64_t K) {
  if (cfg < 0 || cfg >= kNumTileCfgs) return false;
  if (cfg < kNumRingCfgs) return !kTileCfgs[cfg].dma || K % kTileCfgs[cfg].bk == 0;
  const KsplitCfg& c = kKsplitCfgs[cfg - kNumRingCfgs];
  int64_t gm = 0;
  return K % ksplit_sk(c) == 0 && ksplit_ranges(M, N, c, gm) > 0;
}

int select_tile_cfg(int64_t M, int64_t N, int64_t K) {
  const int cfg = g_tile_cfg;
  if (!tile_cfg_fits(cfg, M, N, K)) return default_tile_cfg(M, N, K);
  return cfg;
}

template <int BM, int BN, int KG, int WM, int WN, int KS, int NSTAGE, int EPI>
int launch_ksplit(const GemmArgs& g, hipStream_t st) {
  using Sh = KsplitShape<BM, BN, KG, WM, WN, KS, NSTAGE>;
  constexpr auto kern = ksplit_gemm_kernel<BM, BN, KG, WM, WN, KS, NSTAGE, EPI>;
  if (const int rc = set_lds_limit<kern>(Sh::kLds)) return rc;
  int64_t gm = 0;
  const int64_t gn = ksplit_ranges(g.M, g.N, KsplitCfg{BM, BN, KG, WM, WN, KS, NSTAGE}, gm);
  MW8_REQUIRE(gn > 0 && gm * gn < (int64_t{1} << 31), kErrShape, "gemm: no ksplit grid for N=%lld", (long long)g.N);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(gm * gn)), dim3(Sh::kThreads), Sh::kLds, st, g);
  return kOk;
}

template <int EPI>
int dispatch_ksplit(int i, const GemmArgs& g, hipStream_t st) {
  switch (i) {
    case 0: return launch_ksplit<64, 32, 8, 1, 1, 1, 4, EPI>(g, st);
    case 1: return launch_ksplit<64, 32, 8, 1, 1, 2, 3, EPI>(g, st);
    case 2: return launch_ksplit<64, 64, 8, 1, 1, 1, 4, EPI>(g, st);
    case 3: return launch_ksplit<128, 64, 4, 2, 1, 2, 3, EPI>(g, st);
    default: return launch_ksplit<128, 128, 2, 2, 2, 2, 3, EPI>(g, st);
  }
}

template <int BM, int BN, int EPI>
int launch_split_reduce(const GemmArgs& g, const SplitPlan& sp, hipStream_t st) {
  const int64_t threads = sp.tail * BM * (BN / 8);
  hipLaunchKernelGGL((split_reduce_kernel<EPI, BM, BN>), dim3(static_cast<unsigned>((threads + 255) / 256)),
                     dim3(256), 0, st, g);
  return kOk;
}

// The stream walk (gemm_stream.h) over 256 x 256 tiles: one block per CU.
template <bool kGrouped, int kAct = -1>
int launch_stream(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  constexpr int kLds = stream_lds_bytes<256, kAct>();
  constexpr auto kern = stream_gemm_kernel<256, kEpiBf16, kGrouped, kAct>;
  if (const int rc = set_lds_limit<kern>(kLds)) return rc;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(512), kLds, st, g);
  return kOk;
}

// Whether the stream walk takes a bf16 GEMM: whole 128-byte K stages, at
// least kStreamMinStages of them, 16-byte output rows, and an output the
// 32-bit buffer offsets reach.
bool stream_fits(const GemmArgs& g, int64_t out_rows, int64_t out_cols) {
  return g.staged_out && g.K % kStreamBK == 0 && g.K / kStreamBK >= kStreamMinStages && out_cols % 8 == 0 &&
         out_rows * g.ldo * 2 < (int64_t{1} << 31);
}

template <int EPI>
int dispatch_tile(GemmArgs g, void* ws, size_t ws_bytes, hipStream_t st) {
  const int cfg = select_tile_cfg(g.M, g.N, g.K);
  if (cfg >= kNumRingCfgs) return dispatch_ksplit<EPI>(cfg - kNumRingCfgs, g, st);
  const TileCfg c = kTileCfgs[cfg];
  const int64_t tiles64 = ((g.M + c.bm - 1) / c.bm) * ((g.N + c.bn - 1) / c.bn);
  // the tile walk computes in 32 bits; a K split multiplies the blocks by at most 16
  MW8_REQUIRE(tiles64 <= (int64_t{1} << 26), kErrShape, "gemm: %lld output tiles exceed the tile walk's range",
              (long long)tiles64);
  unsigned tiles = static_cast<unsigned>(tiles64);
  // K split (ring configurations): needs the caller's workspace
  const SplitPlan sp = plan_split(g.M, g.N, g.K, c);
  const bool split = sp.sp > 1 && ws != nullptr && ws_bytes >= sp.ws;
  g.tail_split = 1;
  if (split) {
    g.part = static_cast<int32_t*>(ws);
    g.full_tiles = sp.full;
    g.tail_split = sp.sp;
    tiles = static_cast<unsigned>(sp.full + sp.tail * sp.sp);
  }
  // One row tile: every weight tile is read by one block only, so the
  // 128- and 64-row rings stream the weights with the non-temporal policy.
  // Measured on MI355X (graph-timed, rotating weight copies, us, default ->
  // streaming): 64x128 gate_up M=40 48.9 -> 46.0, M=64 48.9-51.3 ->
  // 46.8-49.7, down M=64 28.0 -> 27.6; 128x128 gate_up M=128 67.6 -> 66.4.
  // With more row tiles the weight tiles are re-read from L2 and the policy
  // loses (down M=256 on two 128-row tiles: 50.9 -> 58.3).
  const bool one_row = g.M <= c.bm;
  int rc;
  switch (cfg) {
    case 0: rc = launch_tile<128, 128, 128, 2, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 1: rc = launch_tile3<128, 128, 64, 2, 2, 4, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 2: rc = launch_tile3<256, 256, 128, 2, 4, 2, EPI, DenseRows, 0, kLead256>(g, dim3(tiles), st); break;
    case 3: rc = launch_tile3<256, 128, 128, 4, 2, 3, EPI, DenseRows>(g, dim3(tiles), st); break;
    case 4:
      rc = one_row ? launch_tile3<128, 128, 128, 2, 2, 2, EPI, DenseRows, kStreamAux, kLeadSmall>(g, dim3(tiles), st)
                   : launch_tile3<128, 128, 128, 2, 2, 2, EPI, DenseRows, 0, kLeadSmall>(g, dim3(tiles), st);
      break;
    case 5:
      rc = one_row ? launch_tile3<64, 128, 128, 1, 4, 4, EPI, DenseRows, kStreamAux, kLeadSmall>(g, dim3(tiles), st)
                   : launch_tile3<64, 128, 128, 1, 4, 4, EPI, DenseRows, 0, kLeadSmall>(g, dim3(tiles), st);
      break;
    case 6: rc = launch_tile3<256, 320, 128, 2, 4, 2, EPI, DenseRows>(g, dim3(tiles), st); break;
    default: {
      const int64_t cus = device_cus();
      if (EPI == kEpiBf16 && tiles >= cus && stream_fits(g, g.M, g.N))
        rc = launch_stream<false>(g, static_cast<unsigned>(cus), st);
      else
        rc = launch_tile3<256, 256, 128, 2, 4, 2, EPI, DenseRows, 0, kLead256>(g, dim3(tiles), st);
      break;
    }
  }
  if (rc != kOk || !split) return rc;
  switch (c.bm * 1000 + c.bn) {
    case 64128: return launch_split_reduce<64, 128, EPI>(g, sp, st);
    case 128128: return launch_split_reduce<128, 128, EPI>(g, sp, st);
    default: return launch_split_reduce<256, 256, EPI>(g, sp, st);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Whether decode configuration cfg takes a fused-quantization call: a
// decode3 configuration whose waves each stream at most kXQMaxStages K
// stages of 256 bytes, load their range of the M rows in at most
// kXQChunks 16-element chunks per lane and hold it as int8 in one ring
// slot.
bool xq_cfg_fits(int cfg, int64_t M, int64_t K) {
  const DecodeCfg& c = kDecodeCfgs[cfg];
  if (c.core != 1) return false;
  const int64_t per_wave = ((K + 255) / 256 + c.waves - 1) / c.waves;
  return per_wave <= kXQMaxStages && (M * 16 * per_wave + 63) / 64 <= kXQChunks &&
         M * 256 * per_wave <= int64_t{c.rg} * kRingStage;
}

// The decode configuration a fused-quantization call at (M, N, K) runs, or
// -1 if it does not take it: at most kXQMaxTokens rows and kXQMaxElems
// elements, the override or the default decode configuration.
int xq_decode_cfg(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > kXQMaxTokens || M * K > kXQMaxElems || N < 1 || K < 16 || K % 16 != 0) return -1;
  int cfg = g_decode_cfg;
  if (cfg < 0 || cfg >= kNumDecodeCfgs) {
    cfg = default_decode_cfg(M, N, K);
    // past 16 K stages the 8-wave blocks quantize their shorter ranges
    // sooner (MI355X, one token, us, 4 x 3 -> 8 x 2 slots: K 5120 N 5120
    // 9.56 -> 8.82, N 7168 11.23 -> 10.44; K 4096 N 4096 7.41 -> 7.68)
    if (cfg == 6 && (K + 255) / 256 > 16 && xq_cfg_fits(7, M, K)) cfg = 7;
  }
  return xq_cfg_fits(cfg, M, K) ? cfg : -1;
}


// Decode core up to 32 tokens, the tile core above 64.  In between the
// tile core when K % 128 == 0 (its 64-row rings stream 1.2-2x faster than
// the decode core at 33-64 tokens on MI355X), unless a decode
// configuration is forced; a forced tile configuration takes it for any K.
bool use_tile_path(int64_t M, int64_t N, int64_t K) {
  if (M > kDecodeMaxM) return true;
  if (M <= 32 || g_decode_cfg >= 0) return false;
  if (g_tile_cfg < 0 && sx_default(M, N, K)) return false;  // the shared token ring
  return K % 128 == 0 || g_tile_cfg >= 0;
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
  // the ring cores address A and W through 32-bit buffer offsets
  MW8_REQUIRE(M * K < (1ll << 31) && N * K < (1ll << 31), kErrShape,
              "gemm: A (%lld x %lld) or W (%lld x %lld) exceeds 2^31 bytes", (long long)M, (long long)K,
              (long long)N, (long long)K);

  GemmArgs g{};
  g.A = A; g.sa = sa; g.W = W; g.sw = sw;
  g.bias = static_cast<const uint16_t*>(bias);
  g.out = out; g.M = M; g.N = N; g.K = K; g.lda = K; g.ldo = N;
  g.top_k = 1;
  g.staged_out = epi == kEpiBf16 && N % 8 == 0 && aligned16(out);
  int rc;
  if (!use_tile_path(M, N, K)) {
    rc = epi == kEpiBf16 ? dispatch_decode<kEpiBf16>(g, st) : dispatch_decode<kEpiI32>(g, st);
  } else {
    MW8_REQUIRE(ws == nullptr || aligned16(ws), kErrAlign, "gemm: workspace needs 16-byte alignment");
    rc = epi == kEpiBf16 ? dispatch_tile<kEpiBf16>(g, ws, ws_bytes, st)
                         : dispatch_tile<kEpiI32>(g, ws, ws_bytes, st);
  }
  if (rc != kOk) return rc;
  return check_launch("gemm");
}

}  // namespace

int linear_bf16_supported(int64_t M, int64_t N, int64_t K) { return xq_decode_cfg(M, N, K) >= 0 ? 1 : 0; }

int linear_bf16_w8a8(const void* x, int64_t ldx, const int8_t* W, const float* sw, const void* bias, void* y,
                     int64_t M, int64_t N, int64_t K, hipStream_t st) {
  MW8_REQUIRE(x && W && sw && y, kErrArg, "linear_bf16: null x/W/scales/y");
  const int cfg = xq_decode_cfg(M, N, K);
  MW8_REQUIRE(cfg >= 0, kErrShape,
              "linear_bf16: M=%lld N=%lld K=%lld is not a fused decode shape (M <= %d, M K <= %lld, at most %d K "
              "stages of 256 bytes per wave, the rows' range within one ring slot)",
              (long long)M, (long long)N, (long long)K, kXQMaxTokens, (long long)kXQMaxElems, kXQMaxStages);
  MW8_REQUIRE(ldx >= K && ldx % 8 == 0 && aligned16(x) && aligned16(W), kErrAlign,
              "linear_bf16: x rows and W need 16-byte alignment (ldx=%lld)", (long long)ldx);
  MW8_REQUIRE(N < (1ll << 31) && N * K < (1ll << 31), kErrShape, "linear_bf16: W exceeds 2^31 bytes");
  MW8_REQUIRE(M * ldx * 2 < (1ll << 31), kErrShape, "linear_bf16: x (%lld rows of %lld) exceeds 2^31 bytes",
              (long long)M, (long long)ldx);
  GemmArgs g{};
  g.A = static_cast<const int8_t*>(x);  // bf16 rows, quantized in the kernel
  g.W = W; g.sw = sw;
  g.bias = static_cast<const uint16_t*>(bias);
  g.out = y; g.M = M; g.N = N; g.K = K; g.lda = ldx; g.ldo = N;
  g.top_k = 1;
  int rc;
  switch (cfg) {
    case 2: rc = launch_decode3_xq<1, 4, 1>(g, st); break;
    case 3: rc = launch_decode3_xq<2, 2, 1>(g, st); break;
    case 4: rc = launch_decode3_xq<1, 4, 2>(g, st); break;
    case 5: rc = launch_decode3_xq<4, 2, 2>(g, st); break;
    case 6: rc = launch_decode3_xq<4, 3, 2>(g, st); break;
    default: rc = launch_decode3_xq<8, 2, 2>(g, st); break;
  }
  if (rc != kOk) return rc;
  return check_launch("linear_bf16");
}

void set_tuning(int decode_cfg, int tile_cfg, int moe_cfg) {
  g_decode_cfg = decode_cfg;
  g_tile_cfg = tile_cfg;
  g_moe_cfg = moe_cfg;
}

int tuning_count(int kind);

size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || !use_tile_path(M, N, K)) return 0;
  const int cfg = select_tile_cfg(M, N, K);
  return cfg < kNumRingCfgs ? plan_split(M, N, K, kTileCfgs[cfg]).ws : 0;
}

size_t gemm_workspace_max_bytes() {
  size_t mx = 0;
  for (const TileCfg& c : kTileCfgs) {
    if (!c.dma || !c.split) continue;
    const size_t b = static_cast<size_t>(device_cus()) * c.per_cu * c.bm * c.bn * sizeof(int32_t);
    if (b > mx) mx = b;
  }
  return mx;
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

// ----------------------------------------- GEMM with the gated activation
// y [M, I] = act_fn(gate) * up of the W8A8 GEMM against a gate|up weight
// [2I, K] (gate rows first), each tile's B rows the gate rows and the
// matching up rows of BN/2 activation columns (tile3_run kAct): the
// [M, 2I] gate|up output never reaches memory.  The ring configurations
// with a one-pass staged epilogue take it; the plain GEMM's pick at
// (M, 2I, K) decides which, with the same K split of a short last wave
// (split_reduce_act_kernel applies the activation).
namespace {
int act_tile_cfg(int64_t M, int64_t N2, int64_t K) {
  const int cfg = select_tile_cfg(M, N2, K);
  if (cfg == 2 || cfg == 3 || cfg == 4 || cfg == 5) return cfg;
  if (cfg == 6 || cfg == 7) return 2;  // the 256x320 ring and the stream walk: 256x256
  return M > 128 ? 2 : 4;
}

template <int BM, int BN, int WM, int WN, int NSTAGE, int kAct, int kBLead = 0>
int launch_tile3_act(const GemmArgs& g, unsigned tiles, hipStream_t st) {
  constexpr int kLds = NSTAGE * BM * 128 + (NSTAGE + kBLead) * BN * 128;
  constexpr auto kern = tile3_gemm_kernel<BM, BN, 128, WM, WN, NSTAGE, kEpiBf16, DenseRows, 0, 16, kAct, kBLead>;
  if (const int rc = set_lds_limit<kern>(kLds)) return rc;
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * WM * WN), kLds, st, g);
  return kOk;
}

template <int BM, int BN, int kAct>
int launch_split_reduce_act(const GemmArgs& g, const SplitPlan& sp, hipStream_t st) {
  const int64_t threads = sp.tail * BM * (BN / 16);
  hipLaunchKernelGGL((split_reduce_act_kernel<BM, BN, kAct>), dim3(static_cast<unsigned>((threads + 255) / 256)),
                     dim3(256), 0, st, g);
  return kOk;
}

template <int kAct>
int dispatch_act(const GemmArgs& g, int cfg, unsigned tiles, bool split, const SplitPlan& sp, hipStream_t st) {
  int rc;
  switch (cfg) {
    case 3: rc = launch_tile3_act<256, 128, 4, 2, 3, kAct>(g, tiles, st); break;
    case 4: rc = launch_tile3_act<128, 128, 2, 2, 2, kAct, kLeadSmall>(g, tiles, st); break;
    case 5: rc = launch_tile3_act<64, 128, 1, 4, 4, kAct, kLeadSmall>(g, tiles, st); break;
    default: rc = launch_tile3_act<256, 256, 2, 4, 2, kAct, kLead256>(g, tiles, st); break;
  }
  if (rc != kOk || !split) return rc;
  switch (cfg) {
    case 4: return launch_split_reduce_act<128, 128, kAct>(g, sp, st);
    case 5: return launch_split_reduce_act<64, 128, kAct>(g, sp, st);
    default: return launch_split_reduce_act<256, 256, kAct>(g, sp, st);
  }
}
}  // namespace

// The ring configuration a fused-activation GEMM at (M, I, K) runs, or -1:
// I % 8 == 0 (16-byte output rows), K % 128 == 0, and a shape the plain
// GEMM at (M, 2I, K) runs on the ring cores (not the decode cores).
int gemm_act_cfg(int64_t M, int64_t I, int64_t K) {
  if (M < 1 || I < 8 || I % 8 != 0 || K < 128 || K % 128 != 0 || K > (1ll << 17)) return -1;
  if (!use_tile_path(M, 2 * I, K)) return -1;
  return act_tile_cfg(M, 2 * I, K);
}

size_t gemm_act_workspace_bytes(int64_t M, int64_t I, int64_t K) {
  const int cfg = gemm_act_cfg(M, I, K);
  return cfg < 0 ? 0 : plan_split(M, 2 * I, K, kTileCfgs[cfg]).ws;
}

int gemm_act_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw, int act, void* y,
                       int64_t M, int64_t I, int64_t K, void* ws, size_t ws_bytes, hipStream_t st) {
  MW8_REQUIRE(A && sa && W && sw && y, kErrArg, "gemm_act: null pointer");
  MW8_REQUIRE(act == 0 || act == 1, kErrArg, "gemm_act: act must be 0 (silu) or 1 (gelu)");
  if (M == 0) return kOk;
  const int cfg = gemm_act_cfg(M, I, K);
  MW8_REQUIRE(cfg >= 0, kErrShape,
              "gemm_act: M=%lld I=%lld K=%lld not taken (I %% 8 == 0, K %% 128 == 0, a ring-core shape)",
              (long long)M, (long long)I, (long long)K);
  MW8_REQUIRE(aligned16(A) && aligned16(W) && aligned16(y) && (ws == nullptr || aligned16(ws)), kErrAlign,
              "gemm_act: A, W, y and the workspace need 16-byte alignment");
  MW8_REQUIRE(M < (1ll << 31) && M * K < (1ll << 31) && 2 * I * K < (1ll << 31), kErrShape,
              "gemm_act: A (%lld x %lld) or W (%lld x %lld) exceeds 2^31 bytes", (long long)M, (long long)K,
              (long long)(2 * I), (long long)K);
  GemmArgs g{};
  g.A = A; g.sa = sa; g.W = W; g.sw = sw;
  g.out = y; g.M = M; g.N = 2 * I; g.K = K; g.lda = K; g.ldo = I;
  g.top_k = 1;
  g.staged_out = 1;
  const TileCfg c = kTileCfgs[cfg];
  const int64_t tiles64 = ((M + c.bm - 1) / c.bm) * ((2 * I + c.bn - 1) / c.bn);
  MW8_REQUIRE(tiles64 <= (int64_t{1} << 26), kErrShape, "gemm_act: %lld output tiles exceed the tile walk's range",
              (long long)tiles64);
  unsigned tiles = static_cast<unsigned>(tiles64);
  const SplitPlan sp = plan_split(M, 2 * I, K, c);
  const bool split = sp.sp > 1 && ws != nullptr && ws_bytes >= sp.ws;
  g.tail_split = 1;
  if (split) {
    g.part = static_cast<int32_t*>(ws);
    g.full_tiles = sp.full;
    g.tail_split = sp.sp;
    tiles = static_cast<unsigned>(sp.full + sp.tail * sp.sp);
  }
  const int rc = act == 0 ? dispatch_act<0>(g, cfg, tiles, split, sp, st) : dispatch_act<1>(g, cfg, tiles, split, sp, st);
  if (rc != kOk) return rc;
  return check_launch("gemm_act");
}

// ------------------------------------------------------------------ grouped
namespace {

// Grouped (fused-MoE) GEMM launchers over expert-sorted rows.  BM equals
// the alignment block size, so every block reads one expert's weights.
template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI>
int launch_grouped3(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((g.N + BN - 1) / BN), blocks);
  return launch_tile3<BM, BN, BK, WM, WN, NSTAGE, EPI, SortedRows>(g, grid, st);
}

// Persistent grouped GEMM: CUs x kPerCu blocks walk the (expert chunk,
// column tile) items.
template <int BM, int BN, int BK, int WM, int WN, int NSTAGE, int EPI, int kPerCu, int kAct = -1>
int launch_grouped_persist(const GemmArgs& g, hipStream_t st) {
  constexpr int kLds = NSTAGE * (BM + BN) * BK;
  constexpr auto kern =
      grouped_persist_kernel<BM, BN, BK, WM, WN, NSTAGE, EPI, true, kPerCu, kAct, BK == 128 ? 16 : 32>;
  if (const int rc = set_lds_limit<kern>(kLds)) return rc;
  const unsigned grid = static_cast<unsigned>(device_cus() * kPerCu);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * WM * WN), kLds, st, g);
  return kOk;
}

// Grouped configurations for 64/128-row alignment blocks (mw8_set_tuning
// moe_cfg): 0 one 128-wide ring tile per alignment block (tile height =
// block size), 1 the persistent walk over (expert, column tile, chunk)
// items with 128x256 tiles on 64-byte K stages, two blocks per CU.
//
// Automatic choice, measured on MI355X at config 3 (E 128, top-8, H 2048,
// I 768; whole layer): with at least 32 pairs per expert on average the
// persistent chunk walk (cfg 1): 1024 tokens 237 -> 215 us, 4096 tokens
// 536 -> 459 us against cfg 0; at 16 pairs per expert (256 tokens) cfg 0
// (167 us against 177).
constexpr int kNumMoeCfgs = 3;
int default_moe_cfg(const GemmArgs& g) {
  if (g.K % 64 == 0 && g.num_experts < kPersistMaxSlots &&
      g.num_valid >= 32 * static_cast<int64_t>(g.num_experts))
    return 1;
  return 0;
}

template <int EPI>
int launch_grouped_epi(const GemmArgs& g, unsigned blocks, int bm, hipStream_t st) {
  if (g.K % 64 != 0) {  // register-staged core
    const dim3 grid(static_cast<unsigned>((g.N + 127) / 128), blocks);
    if (bm == 64) return launch_tile<64, 128, 128, 2, 2, EPI, SortedRows>(g, grid, st);
    return launch_tile<128, 128, 128, 2, 2, EPI, SortedRows>(g, grid, st);
  }
  int cfg = g_moe_cfg;
  if (cfg < 0 || cfg >= kNumMoeCfgs) cfg = default_moe_cfg(g);
  if (cfg == 1 && g.num_experts < kPersistMaxSlots)
    return launch_grouped_persist<128, 256, 64, 2, 2, 3, EPI, 2>(g, st);
  if (cfg == 2 && EPI == kEpiBf16 && g.num_experts < kPersistMaxSlots && 256 % g.align_bsz == 0 &&
      stream_fits(g, g.num_valid, g.N))
    return launch_stream<true>(g, static_cast<unsigned>(device_cus()), st);
  if (bm == 64) return launch_grouped3<64, 128, 64, 2, 2, 4, EPI>(g, blocks, st);
  return launch_grouped3<128, 128, 64, 2, 2, 4, EPI>(g, blocks, st);
}

// 16- or 32-row alignment blocks on the LDS DMA ring (decode3 core,
// gathered rows; TG token groups of 16).
template <int WAVES, int D, int EPI, int TG = 1>
int launch_grouped_ring(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  constexpr int kLds = DecodeRing<TG, WAVES, D>::kLds;
  constexpr auto kern = decode3_gemm_kernel<TG, WAVES, D, EPI, SortedRows, 1>;
  if (const int rc = set_lds_limit<kern>(kLds)) return rc;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>((g.N + 15) / 16), blocks), dim3(64 * WAVES), kLds, st, g);
  return kOk;
}

// 16-row alignment blocks (decode MoE), moe_cfg 0-2: the LDS DMA ring with
// (waves, ring depth) = (1, 3), (2, 3), (1, 4).  Measured on MI355X at
// config 3 (whole layer): 16 tokens 107 us on (1, 3) against 120 us for a
// register-streaming core, 64 tokens 145 against 156; at 256 tokens the
// 64-row tiles win (167 us against 210 for (1, 3) over 16-row blocks).
// Fewer, larger blocks (32 weight rows per block) measured slower
// (16-token layer 102-111 us against 93).
constexpr int kNumSmallMoeCfgs = 3;

template <int EPI>
int launch_grouped_small_epi(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  if (g.align_bsz == 32) return launch_grouped_ring<1, 3, EPI, 2>(g, blocks, st);  // two token groups
  const int cfg = g_moe_cfg;
  switch (cfg) {
    case 1: return launch_grouped_ring<2, 3, EPI>(g, blocks, st);
    case 2: return launch_grouped_ring<1, 4, EPI>(g, blocks, st);
    default: return launch_grouped_ring<1, 3, EPI>(g, blocks, st);
  }
}

}  // namespace

// Name of the kernel family a dense GEMM at (M, N, K) runs (tuning and
// profiling aid: matches the kernel names of a trace).
const char* gemm_kernel_name(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 16 != 0) return "";
  if (!use_tile_path(M, N, K)) {
    int cfg = g_decode_cfg;
    if (cfg < 0 || cfg >= kNumDecodeCfgs) cfg = default_decode_cfg(M, N, K);
    if (kDecodeCfgs[cfg].core == 2) {
      if (sx_fits(M, K)) return "decode_sx_gemm_kernel";
      cfg = default_decode_cfg(M, N, K);
    }
    return kDecodeCfgs[cfg].core == 0 ? "decode_gemm_kernel" : "decode3_gemm_kernel";
  }
  const int cfg = select_tile_cfg(M, N, K);
  if (cfg >= kNumRingCfgs) return kKsplitCfgs[cfg - kNumRingCfgs].name;
  return kTileCfgs[cfg].name;
}

int tuning_count(int kind) {
  switch (kind) {
    case 0: return kNumDecodeCfgs;
    case 1: return kNumTileCfgs;
    case 2: return kNumMoeCfgs;
    case 3: return kNumSmallMoeCfgs;
    default: return 0;
  }
}

int launch_grouped_tile(const GemmArgs& g, unsigned blocks, int bm, int epi, hipStream_t st) {
  return epi == kEpiBf16 ? launch_grouped_epi<kEpiBf16>(g, blocks, bm, st)
                         : launch_grouped_epi<kEpiI32>(g, blocks, bm, st);
}

// Router-id rows (TopkRows): one block per (16 weight rows, expert), the
// 16-row ring configuration (1 wave, 3 slots).
int launch_grouped_topk(const GemmArgs& g, int epi, hipStream_t st) {
  constexpr int kLds = DecodeRing<1, 1, 3>::kLds;
  const dim3 grid(static_cast<unsigned>((g.N + 15) / 16), static_cast<unsigned>(g.num_experts * g.topk_units));
  if (epi == kEpiBf16) {
    constexpr auto kern = decode3_gemm_kernel<1, 1, 3, kEpiBf16, TopkRows, 1>;
    if (const int rc = set_lds_limit<kern>(kLds)) return rc;
    hipLaunchKernelGGL(kern, grid, dim3(64), kLds, st, g);
  } else {
    constexpr auto kern = decode3_gemm_kernel<1, 1, 3, kEpiI32, TopkRows, 1>;
    if (const int rc = set_lds_limit<kern>(kLds)) return rc;
    hipLaunchKernelGGL(kern, grid, dim3(64), kLds, st, g);
  }
  return kOk;
}

int launch_grouped_small(const GemmArgs& g, unsigned blocks, int epi, hipStream_t st) {
  return epi == kEpiBf16 ? launch_grouped_small_epi<kEpiBf16>(g, blocks, st)
                         : launch_grouped_small_epi<kEpiI32>(g, blocks, st);
}

// Decode down-projection with the slot sum fused in: 16 waves with 3-slot
// rings, one block per 8 output columns (a multiple of the CU count).
// Measured on MI355X, config 3 (kernel alone, us, 16 / 64 tokens): 16 x 3
// 26.8-27.3 / 37.6-38.0; 8 x 4 28.2-29.3 / 37.8-38.7; 8 x 6 28.8-29.7 /
// 38.5-39.3; 8 x 8 30.6-31.4 / 39.2-39.8 (GEMM2 26.5-27.4 + slot sum 3.2
// / 40.0-40.5 + 3.1 as two kernels).
constexpr int kMoeSumWaves = 16, kMoeSumDepth = 3;
constexpr int kMoeSumRing = kMoeSumWaves * kMoeSumDepth * kMoeSumSlot;
constexpr int kMoeSumMaxLds = 163840 - 256;  // beside the kernel's static LDS

int moe_gemm_sum_lds_bytes(int64_t max_sorted, int64_t num_valid, int E) {
  if (max_sorted < 0 || num_valid < 0 || E < 1 || E > kMoeSumMaxExperts || max_sorted > kMoeSumMaxSorted ||
      num_valid > kMoeSumMaxPairs)
    return -1;
  const int total = moe_sum_lds(kMoeSumRing, max_sorted, num_valid, E).total;
  return total <= kMoeSumMaxLds ? total : -1;
}

// topk: units are the experts, listed from the router ids (max_sorted = 16 E).
int launch_moe_gemm_sum(const GemmArgs& g, int64_t max_sorted, hipStream_t st, bool topk) {
  const int lds = moe_gemm_sum_lds_bytes(max_sorted, g.num_valid, g.num_experts);
  if (lds < 0)
    return set_error(kErrShape, "moe_gemm_sum: %lld pairs over %lld sorted rows and %d experts exceed the LDS tables",
                     (long long)g.num_valid, (long long)max_sorted, g.num_experts);
  const int64_t cus = device_cus();
  const dim3 grid(static_cast<unsigned>(cus * ((g.N + cus * 8 - 1) / (cus * 8))));
  if (topk) {
    constexpr auto kern = moe_gemm_sum_kernel<kMoeSumWaves, kMoeSumDepth, true>;
    if (const int rc = set_lds_limit<kern>(kMoeSumMaxLds)) return rc;
    hipLaunchKernelGGL(kern, grid, dim3(64 * kMoeSumWaves), lds, st, g, max_sorted);
  } else {
    constexpr auto kern = moe_gemm_sum_kernel<kMoeSumWaves, kMoeSumDepth, false>;
    if (const int rc = set_lds_limit<kern>(kMoeSumMaxLds)) return rc;
    hipLaunchKernelGGL(kern, grid, dim3(64 * kMoeSumWaves), lds, st, g, max_sorted);
  }
  return kOk;
}

// Gate|up GEMM with the gated activation fused (persistent chunk walk, the
// moe cfg 1 tiling): out [rows, N/2] = act(gate) * up, bf16.
int launch_grouped_act(const GemmArgs& g, int act, hipStream_t st) {
  const int cfg = g_moe_cfg;
  if (cfg == 2 && 256 % g.align_bsz == 0 && stream_fits(g, g.num_valid, g.N / 2)) {
    if (act == 0) return launch_stream<true, 0>(g, static_cast<unsigned>(device_cus()), st);
    return launch_stream<true, 1>(g, static_cast<unsigned>(device_cus()), st);
  }
  if (act == 0) return launch_grouped_persist<128, 256, 64, 2, 2, 3, kEpiBf16, 2, 0>(g, st);
  return launch_grouped_persist<128, 256, 64, 2, 2, 3, kEpiBf16, 2, 1>(g, st);
}

}  // namespace mw8
