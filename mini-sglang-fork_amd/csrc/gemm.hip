// Dense W8A8 GEMM: dispatch between the weight-streaming core (M <= 64) and
// the MFMA tile core (M > 64), plus the C-ABI entry points.
#include "gemm_kernels.h"

namespace mw8 {
namespace {

constexpr int64_t kStreamMaxM = 64;
constexpr int kStreamTargetBlocks = 1024;  // ~4 resident blocks per CU on 256 CUs

struct StreamPlan {
  int mt;        // 16-token groups
  int splits;    // K splits
  int kc;        // K bytes per split (multiple of 256)
  int64_t n_tiles;
  size_t ws_bytes;  // counters + partials (0 when splits == 1)
};

int kc_max_for(int mt) {
  switch (mt) {
    case 1: return stream_kc_max<1>();
    case 2: return stream_kc_max<2>();
    case 3: return stream_kc_max<3>();
    default: return stream_kc_max<4>();
  }
}

constexpr size_t kCounterBytes = 64 * 1024;  // room for 16384 N tiles

StreamPlan plan_stream(int64_t M, int64_t N, int64_t K) {
  StreamPlan p{};
  p.mt = static_cast<int>((M + 15) / 16);
  p.n_tiles = (N + kStreamRows - 1) / kStreamRows;
  const int64_t ksteps = (K + kStreamStep - 1) / kStreamStep;
  int64_t splits = (kStreamTargetBlocks + p.n_tiles - 1) / p.n_tiles;
  splits = splits < 1 ? 1 : (splits > ksteps ? ksteps : splits);
  int64_t kc = ((ksteps + splits - 1) / splits) * kStreamStep;
  const int kcm = kc_max_for(p.mt);
  if (kc > kcm) kc = kcm;
  p.kc = static_cast<int>(kc);
  p.splits = static_cast<int>((K + kc - 1) / kc);
  p.ws_bytes = p.splits > 1 ? kCounterBytes + static_cast<size_t>(p.splits) * M * N * 4 : 0;
  return p;
}

template <int MT, int EPI>
void launch_stream(const GemmArgs& g, const StreamPlan& p, hipStream_t st) {
  const int ldl = ((p.kc + kStreamStep - 1) / kStreamStep) * kStreamStep + 16;
  const size_t lds = static_cast<size_t>(16 * MT) * ldl;
  hipLaunchKernelGGL((stream_gemm_kernel<MT, EPI, DenseRows>),
                     dim3(static_cast<unsigned>(p.n_tiles), static_cast<unsigned>(p.splits)),
                     dim3(256), lds, st, g);
}

template <int EPI>
void dispatch_stream(const GemmArgs& g, const StreamPlan& p, hipStream_t st) {
  switch (p.mt) {
    case 1: launch_stream<1, EPI>(g, p, st); break;
    case 2: launch_stream<2, EPI>(g, p, st); break;
    case 3: launch_stream<3, EPI>(g, p, st); break;
    default: launch_stream<4, EPI>(g, p, st); break;
  }
}

template <int BM, int BN, int WM, int WN, int EPI, class Rows>
void launch_tile(const GemmArgs& g, unsigned grid_y, hipStream_t st) {
  using S = TileShape<BM, BN, WM, WN>;
  auto kern = tile_gemm_kernel<BM, BN, WM, WN, EPI, Rows>;
  static bool attr_set = false;  // per instantiation; benign race (idempotent)
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                        hipFuncAttributeMaxDynamicSharedMemorySize, S::kLds);
    attr_set = true;
  }
  const unsigned gx = static_cast<unsigned>((g.N + BN - 1) / BN);
  hipLaunchKernelGGL(kern, dim3(gx, grid_y), dim3(256), S::kLds, st, g);
}

template <int EPI>
void dispatch_tile(const GemmArgs& g, hipStream_t st) {
  const unsigned gy = static_cast<unsigned>((g.M + 127) / 128);
  launch_tile<128, 128, 2, 2, EPI, DenseRows>(g, gy, st);
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

  if (M <= kStreamMaxM) {
    const StreamPlan p = plan_stream(M, N, K);
    if (p.splits > 1) {
      MW8_REQUIRE(ws && ws_bytes >= p.ws_bytes, kErrWorkspace,
                  "gemm: workspace of %zu bytes needed (got %zu); zero-fill it once at allocation",
                  p.ws_bytes, ws_bytes);
      MW8_REQUIRE(p.n_tiles * 4 <= static_cast<int64_t>(kCounterBytes), kErrShape,
                  "gemm: N too large for the split-K counters");
      MW8_REQUIRE(aligned16(ws), kErrAlign, "gemm: workspace needs 16-byte alignment");
      g.counters = static_cast<int32_t*>(ws);
      g.partials = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + kCounterBytes);
    }
    g.splits = p.splits;
    g.kc = p.kc;
    if (epi == kEpiBf16) dispatch_stream<kEpiBf16>(g, p, st);
    else dispatch_stream<kEpiI32>(g, p, st);
  } else {
    if (epi == kEpiBf16) dispatch_tile<kEpiBf16>(g, st);
    else dispatch_tile<kEpiI32>(g, st);
  }
  return check_launch("gemm");
}

}  // namespace

size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || M > kStreamMaxM) return 0;
  return plan_stream(M, N, K).ws_bytes;
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

// Exposed for the grouped GEMM (moe.hip): tile core over expert-sorted rows.
void launch_grouped_tile_bf16(const GemmArgs& g, unsigned blocks, int bm, hipStream_t st);
void launch_grouped_tile_i32(const GemmArgs& g, unsigned blocks, int bm, hipStream_t st);

void launch_grouped_tile_bf16(const GemmArgs& g, unsigned blocks, int bm, hipStream_t st) {
  if (bm == 64) launch_tile<64, 128, 2, 2, kEpiBf16, SortedRows>(g, blocks, st);
  else launch_tile<128, 128, 2, 2, kEpiBf16, SortedRows>(g, blocks, st);
}
void launch_grouped_tile_i32(const GemmArgs& g, unsigned blocks, int bm, hipStream_t st) {
  if (bm == 64) launch_tile<64, 128, 2, 2, kEpiI32, SortedRows>(g, blocks, st);
  else launch_tile<128, 128, 2, 2, kEpiI32, SortedRows>(g, blocks, st);
}

}  // namespace mw8
