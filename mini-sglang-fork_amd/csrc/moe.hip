// Fused-MoE building blocks (gfx950): router top-k softmax, expert
// alignment (stable counting sort with block padding), grouped W8A8 GEMM
// over expert segments, and the top-k slot sum.
#include <type_traits>

#include "gemm_kernels.h"

namespace mw8 {

int launch_grouped_tile(const GemmArgs& g, unsigned blocks, int bm, int epi, hipStream_t st);
int launch_grouped_small(const GemmArgs& g, unsigned blocks, int epi, hipStream_t st);
int launch_grouped_act(const GemmArgs& g, int act, hipStream_t st);
int launch_moe_gemm_sum(const GemmArgs& g, int64_t max_sorted, hipStream_t st, bool topk);
int launch_grouped_topk(const GemmArgs& g, int epi, hipStream_t st);
int moe_gemm_sum_lds_bytes(int64_t max_sorted, int64_t num_valid, int E);

namespace {

// ------------------------------------------------------------------ top-k
// Full-wave reductions without LDS: DPP quad permutes and row mirrors
// combine within each 16-lane row, then the gfx950 permlane16/32 swaps
// combine rows; every lane ends with the result.
template <class Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t x, Op op) {
  x = op(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xF, 0xF, false)));  // quad [1,0,3,2]
  x = op(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xF, 0xF, false)));  // quad [2,3,0,1]
  x = op(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x141, 0xF, 0xF, false)));  // row half mirror
  x = op(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x140, 0xF, 0xF, false)));  // row mirror
  const auto r16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = op(r16[0], r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return op(r32[0], r32[1]);
}
__device__ __forceinline__ float wave_max_f32(float v) {
  return __builtin_bit_cast(float, wave_reduce_u32(__builtin_bit_cast(uint32_t, v), [](uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)));
  }));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
  return __builtin_bit_cast(float, wave_reduce_u32(__builtin_bit_cast(uint32_t, v), [](uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b));
  }));
}
__device__ __forceinline__ int wave_min_i32(int v) {
  return static_cast<int>(wave_reduce_u32(static_cast<uint32_t>(v), [](uint32_t a, uint32_t b) {
    return static_cast<int>(a) < static_cast<int>(b) ? a : b;
  }));
}

// One wave per token.  Softmax in fp32 over E logits (bf16 or fp32 input),
// then k rounds of a wave arg-max (larger value wins, lower expert index
// wins ties: a max over values, then a min over the indices holding it),
// then the two renormalisations of the reference
// (python/minisgl/moe/fused.py:22-24).
// Token t on the calling wave; the selected ids also go to ids_copy[t * topk
// + i] when ids_copy is given (the fused small-batch preparation).
template <int VPL>
__device__ __forceinline__ void topk_token(const void* logits, int is_bf16, int64_t t, int E,
                                           int topk, int renorm, float* __restrict__ tw,
                                           int32_t* __restrict__ tid_out, int32_t* ids_copy) {
  const int lane = threadIdx.x & 63;
  float v[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    if (e < E) {
      v[j] = is_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(logits)[t * E + e])
                     : static_cast<const float*>(logits)[t * E + e];
    } else {
      v[j] = -__builtin_huge_valf();
    }
  }
  float mx = v[0];
#pragma unroll
  for (int j = 1; j < VPL; ++j) mx = fmaxf(mx, v[j]);
  mx = wave_max_f32(mx);
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    v[j] = (lane + 64 * j < E) ? expf(v[j] - mx) : 0.0f;
    sum += v[j];
  }
  sum = wave_sum_f32(sum);
#pragma unroll
  for (int j = 0; j < VPL; ++j) v[j] = (lane + 64 * j < E) ? v[j] / sum : -1.0f;

  float w_sel = 0.0f;  // lane i keeps the i-th selected weight / id
  int id_sel = 0;
  for (int i = 0; i < topk; ++i) {
    float bv = v[0];
    int bi = lane;
#pragma unroll
    for (int j = 1; j < VPL; ++j)
      if (v[j] > bv) { bv = v[j]; bi = lane + 64 * j; }
    const float best = wave_max_f32(bv);
    const int sel = wave_min_i32(bv == best ? bi : 0x7fffffff);
    if (lane == i) { w_sel = best; id_sel = sel; }
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (lane + 64 * j == sel) v[j] = -1.0f;
  }
  if (renorm) {
    const float s1 = wave_sum_f32(lane < topk ? w_sel : 0.0f);
    w_sel = w_sel / s1;
    const float s2 = wave_sum_f32(lane < topk ? w_sel : 0.0f);
    w_sel = w_sel / (s2 + 1e-8f);
  }
  if (lane < topk) {
    tw[t * topk + lane] = w_sel;
    tid_out[t * topk + lane] = id_sel;
    if (ids_copy) ids_copy[t * topk + lane] = id_sel;
  }
}

template <int VPL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const void* logits, int is_bf16,
                                                           int64_t M, int E, int topk,
                                                           int renorm, float* __restrict__ tw,
                                                           int32_t* __restrict__ tid_out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= M) return;
  topk_token<VPL>(logits, is_bf16, t, E, topk, renorm, tw, tid_out, nullptr);
}

// ------------------------------------------------------------ alignment
// One launch, no scratch (the reference call passes none that survives the
// call), no communication between blocks.  Block b owns the flat range
// [b*R, (b+1)*R) with R = 1024*U pairs: wave w of the block owns the
// sub-range of 64*U pairs starting at b*R + w*64*U.  Every block histograms
// the whole id array (it is small and L2-resident) into three parts: pairs
// before its range, pairs after it, and per-wave counts inside it.  From
// these every block derives the same padded segment offsets (exclusive scan
// over slots), the start position of each of its waves inside each expert
// segment, and the post-padding total.  Waves then place their pairs in
// flat order: lanes holding the same expert are found with a bitwise ballot
// match and ranked by the popcount of lower matching lanes.  Segment order
// is therefore ascending flat index.  The sentinel fill (padding tails and
// everything past the total) and expert_ids are split over blocks by
// striding; fill and placement never write the same element.
constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kAlignMaxSlots = 512;

// Block `bid` of `nblk` (ids may live in global memory or in LDS).
__device__ __forceinline__ void align_body(
    const int32_t* __restrict__ ids, int64_t numel, int slots, int bsz, int unroll,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ npp, int64_t max_padded, int64_t max_blocks, int nbits, int bid, int nblk) {
  __shared__ int wpos[kAlignWaves][kAlignMaxSlots];  // counts, then start positions
  __shared__ int before[kAlignMaxSlots];
  __shared__ int after[kAlignMaxSlots];
  __shared__ int cnt[kAlignMaxSlots];
  __shared__ int off[kAlignMaxSlots];
  __shared__ int wave_tot[kAlignWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t wave_span = 64 * static_cast<int64_t>(unroll);
  const int64_t lo = static_cast<int64_t>(bid) * kAlignWaves * wave_span;
  const int64_t hi = lo + kAlignWaves * wave_span < numel ? lo + kAlignWaves * wave_span : numel;

  for (int j = tid; j < kAlignWaves * kAlignMaxSlots; j += kAlignThreads) (&wpos[0][0])[j] = 0;
  for (int j = tid; j < kAlignMaxSlots; j += kAlignThreads) { before[j] = 0; after[j] = 0; }
  __syncthreads();
  constexpr int kU = 8;
  for (int64_t c = 0; c < numel; c += kU * kAlignThreads) {
    int e[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = c + u * kAlignThreads + tid;
      e[u] = i < numel ? ids[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = c + u * kAlignThreads + tid;
      if (e[u] < 0 || e[u] >= slots) continue;
      int* slot = i < lo ? &before[e[u]]
                  : i >= hi ? &after[e[u]]
                            : &wpos[static_cast<int>(i - lo) / static_cast<int>(wave_span)][e[u]];
      atomicAdd(slot, 1);
    }
  }
  __syncthreads();

  // exclusive scan of padded counts over slots (slots <= 1024: one per thread)
  int total_e = 0, padded = 0;
  if (tid < slots) {
    total_e = before[tid] + after[tid];
    for (int w = 0; w < kAlignWaves; ++w) total_e += wpos[w][tid];
    padded = ((total_e + bsz - 1) / bsz) * bsz;
  }
  int x = padded;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  int base = 0, total = 0;
  for (int w = 0; w < kAlignWaves; ++w) {
    if (w < wave) base += wave_tot[w];
    total += wave_tot[w];
  }
  const int64_t gstride = static_cast<int64_t>(nblk) * kAlignThreads;
  const int64_t gtid = static_cast<int64_t>(bid) * kAlignThreads + tid;
  if (tid < slots) {
    const int start = base + x - padded;
    off[tid] = start;
    cnt[tid] = total_e;
    int p = start + before[tid];
    for (int w = 0; w < kAlignWaves; ++w) {
      const int c = wpos[w][tid];
      wpos[w][tid] = p;
      p += c;
    }
  }
  if (gtid == 0) *npp = total;
  for (int64_t i = total + gtid; i < max_padded; i += gstride) sorted_ids[i] = static_cast<int32_t>(numel);
  for (int64_t b = static_cast<int64_t>(total) / bsz + gtid; b < max_blocks; b += gstride) expert_ids[b] = -1;
  __syncthreads();
  // expert_ids of the padded segments and the sentinel in each padding tail
  for (int64_t j = gtid; j < static_cast<int64_t>(slots) * bsz; j += gstride) {  // < 2^21
    const int s = static_cast<int>(j) / bsz, r = static_cast<int>(j) - s * bsz;
    const int c = cnt[s];
    const int padded_s = ((c + bsz - 1) / bsz) * bsz;
    if (r < padded_s - c) sorted_ids[off[s] + c + r] = static_cast<int32_t>(numel);
    if (r == 0)
      for (int b = off[s] / bsz; b < (off[s] + padded_s) / bsz; ++b) expert_ids[b] = s;
  }

  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t wlo = lo + wave * wave_span;
  const int64_t whi = wlo + wave_span < hi ? wlo + wave_span : hi;
  for (int64_t c = wlo; c < whi; c += 64) {  // wave-uniform bounds
    const int64_t i = c + lane;
    const int ev = i < whi ? ids[i] : -1;
    const bool valid = ev >= 0 && ev < slots;
    uint64_t m = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (ev >> b) & 1;
      const uint64_t bb = __ballot(bit);
      m &= bit ? bb : ~bb;
    }
    const int rank = __popcll(m & below);
    const int pos = valid ? wpos[wave][ev] : 0;
    if (valid) sorted_ids[pos + rank] = static_cast<int32_t>(i);
    __builtin_amdgcn_wave_barrier();
    if (valid && rank == 0) wpos[wave][ev] = pos + __popcll(m);
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int slots, int bsz, int unroll,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ npp, int64_t max_padded, int64_t max_blocks, int nbits) {
  align_body(ids, numel, slots, bsz, unroll, sorted_ids, expert_ids, npp, max_padded, max_blocks, nbits,
             blockIdx.x, gridDim.x);
}

// ------------------------------------------------ small-batch preparation
// One block does the router, the per-token quantization of the hidden rows
// and the alignment (pairs <= 1024, one block of the alignment kernel's
// own code with the ids in LDS): three launches of the decode MoE layer in
// one.  Each part is the code of its own kernel, so the outputs are those
// of topk_softmax, quant_per_token and moe_align_block_size bit for bit.
constexpr int kPrepMaxPairs = kAlignThreads;

// Row r of the hidden states quantized by the calling wave (two passes over
// the L2-resident row: integer absmax of sign-cleared bf16 bits, then the
// quantizer's own closed form per element).
__device__ __forceinline__ void quant_row_wave(const uint16_t* __restrict__ x, int64_t K,
                                               int8_t* __restrict__ q, float* __restrict__ s) {
  const int lane = threadIdx.x & 63;
  const int64_t nvec = K >> 3;
  uint32_t m = 0;
  for (int64_t v = lane; v < nvec; v += 64) {
    const v4i w = *reinterpret_cast<const v4i*>(x + 8 * v);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = static_cast<uint32_t>(w[j]);
      const uint32_t lo = u & 0x7FFFu, hi = (u >> 16) & 0x7FFFu;
      m = lo > m ? lo : m;
      m = hi > m ? hi : m;
    }
  }
  m = wave_reduce_u32(m, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
  const RowScale rs = row_scale(bf16_to_f32(static_cast<uint16_t>(m)));
  for (int64_t v = lane; v < nvec; v += 64) {
    const v4i w = *reinterpret_cast<const v4i*>(x + 8 * v);
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = static_cast<uint32_t>(w[j]);
      const int a = static_cast<int>(quant_div_rne(bf16_to_f32(static_cast<uint16_t>(u & 0xFFFFu)), rs));
      const int b = static_cast<int>(quant_div_rne(bf16_to_f32(static_cast<uint16_t>(u >> 16)), rs));
      packed[j >> 1] |= ((static_cast<uint32_t>(a) & 0xFFu) | ((static_cast<uint32_t>(b) & 0xFFu) << 8)) << (16 * (j & 1));
    }
    *reinterpret_cast<uint2*>(q + 8 * v) = make_uint2(packed[0], packed[1]);
  }
  if (lane == 0) *s = rs.s;
}

template <int VPL>
__global__ __launch_bounds__(kAlignThreads) void moe_prepare_kernel(
    const void* logits, int is_bf16, int64_t M, int E, int topk, int renorm,
    const uint16_t* __restrict__ hidden, int64_t H, float* __restrict__ tw, int32_t* __restrict__ tid_out,
    int8_t* __restrict__ q, float* __restrict__ s, int slots, int bsz, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ npp, int64_t max_padded, int64_t max_blocks,
    int nbits) {
  __shared__ int32_t ids[kPrepMaxPairs];
  const int wave = threadIdx.x >> 6;
  for (int64_t t = wave; t < M; t += kAlignWaves)
    topk_token<VPL>(logits, is_bf16, t, E, topk, renorm, tw, tid_out, ids);
  for (int64_t r = wave; r < M; r += kAlignWaves) quant_row_wave(hidden + r * H, H, q + r * H, s + r);
  __syncthreads();  // the ids of every token are in LDS
  align_body(ids, M * topk, slots, bsz, 1, sorted_ids, expert_ids, npp, max_padded, max_blocks, nbits, 0, 1);
}

// Router and hidden-state quantizer of four tokens per block (both read
// only their own token): waves 0-3 route tokens 4b .. 4b+3 while waves 4-7
// quantize their rows, so the two latency chains overlap; the outputs of
// topk_softmax_kernel and quant_rows_kernel bit for bit, from one launch.
template <int VPL>
__global__ __launch_bounds__(512) void route_quant_kernel(const void* logits, int is_bf16, int64_t M, int E,
                                                          int topk, int renorm, const uint16_t* __restrict__ hidden,
                                                          int64_t H, float* __restrict__ tw,
                                                          int32_t* __restrict__ tid_out, int8_t* __restrict__ q,
                                                          float* __restrict__ s) {
  const int w = threadIdx.x >> 6;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (w & 3);
  if (t >= M) return;  // whole waves
  if (w < 4) topk_token<VPL>(logits, is_bf16, t, E, topk, renorm, tw, tid_out, nullptr);
  else quant_row_wave(hidden + t * H, H, q + t * H, s + t);
}

// ------------------------------------------------------------ slot sum
// out[t, h] = bf16(sum_i in[t, i, h]) in fp32, slot order i = 0..k-1
// (python/minisgl/kernel/triton/fused_moe.py:36-47); 8 columns per thread.
__global__ __launch_bounds__(256) void moe_sum_reduce_kernel(const uint16_t* __restrict__ in,
                                                             int64_t M, int k, int64_t H,
                                                             uint16_t* __restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t hv = H >> 3;
  if (idx >= M * hv) return;
  const int64_t t = idx / hv, h = (idx % hv) * 8;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
  for (int i = 0; i < k; ++i) {
    const v4i raw = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(in + (t * k + i) * H + h));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = static_cast<uint32_t>(raw[j]);
      acc[2 * j] = acc[2 * j] + bf16_to_f32(static_cast<uint16_t>(u & 0xFFFFu));
      acc[2 * j + 1] = acc[2 * j + 1] + bf16_to_f32(static_cast<uint16_t>(u >> 16));
    }
  }
  v4i o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = static_cast<int>(static_cast<uint32_t>(f32_to_bf16(acc[2 * j])) |
                            (static_cast<uint32_t>(f32_to_bf16(acc[2 * j + 1])) << 16));
  __builtin_nontemporal_store(o, reinterpret_cast<v4i*>(out + t * H + h));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int VPL>
void launch_topk(const void* lg, int is_bf16, int64_t M, int E, int k, int renorm, float* tw,
                 int32_t* ti, hipStream_t st) {
  hipLaunchKernelGGL((topk_softmax_kernel<VPL>), dim3(static_cast<unsigned>((M + 3) / 4)),
                     dim3(256), 0, st, lg, is_bf16, M, E, k, renorm, tw, ti);
}

}  // namespace

int topk_softmax(const void* logits, int is_bf16, int64_t M, int E, int topk, int renorm,
                 float* topk_w, int32_t* topk_ids, hipStream_t st) {
  MW8_REQUIRE(logits && topk_w && topk_ids, kErrArg, "topk_softmax: null pointer");
  MW8_REQUIRE(E > 0 && E <= 1024 && topk > 0 && topk <= E && topk <= 64, kErrShape,
              "topk_softmax: need 0 < topk <= min(E, 64), E <= 1024 (E=%d topk=%d)", E, topk);
  if (M <= 0) return kOk;
  MW8_REQUIRE(M < (1ll << 32), kErrShape, "topk_softmax: too many tokens");
  const int vpl = (E + 63) / 64;
  if (vpl <= 1) launch_topk<1>(logits, is_bf16, M, E, topk, renorm, topk_w, topk_ids, st);
  else if (vpl <= 2) launch_topk<2>(logits, is_bf16, M, E, topk, renorm, topk_w, topk_ids, st);
  else if (vpl <= 4) launch_topk<4>(logits, is_bf16, M, E, topk, renorm, topk_w, topk_ids, st);
  else if (vpl <= 8) launch_topk<8>(logits, is_bf16, M, E, topk, renorm, topk_w, topk_ids, st);
  else launch_topk<16>(logits, is_bf16, M, E, topk, renorm, topk_w, topk_ids, st);
  return check_launch("topk_softmax");
}

int moe_route_quant(const void* logits, int is_bf16, int64_t M, int E, int topk, int renorm, const void* hidden,
                    int64_t H, float* topk_w, int32_t* topk_ids, int8_t* q, float* s, hipStream_t st) {
  MW8_REQUIRE(logits && hidden && topk_w && topk_ids && q && s, kErrArg, "moe_route_quant: null pointer");
  MW8_REQUIRE(E > 0 && E <= 1024 && topk > 0 && topk <= E && topk <= 64, kErrShape,
              "moe_route_quant: need 0 < topk <= min(E, 64), E <= 1024 (E=%d topk=%d)", E, topk);
  MW8_REQUIRE(H > 0 && H % 8 == 0, kErrShape, "moe_route_quant: need H %% 8 == 0 (H=%lld)", (long long)H);
  MW8_REQUIRE(aligned16(hidden) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0, kErrAlign,
              "moe_route_quant: hidden needs 16-byte and q 8-byte alignment");
  if (M <= 0) return kOk;
  MW8_REQUIRE(M < (1ll << 32), kErrShape, "moe_route_quant: too many tokens");
  const int vpl = (E + 63) / 64;
  auto go = [&](auto vpl_c) {
    constexpr int V = decltype(vpl_c)::value;
    hipLaunchKernelGGL((route_quant_kernel<V>), dim3(static_cast<unsigned>((M + 3) / 4)), dim3(512), 0, st, logits,
                       is_bf16, M, E, topk, renorm, static_cast<const uint16_t*>(hidden), H, topk_w, topk_ids, q, s);
  };
  if (vpl <= 1) go(std::integral_constant<int, 1>{});
  else if (vpl <= 2) go(std::integral_constant<int, 2>{});
  else if (vpl <= 4) go(std::integral_constant<int, 4>{});
  else if (vpl <= 8) go(std::integral_constant<int, 8>{});
  else go(std::integral_constant<int, 16>{});
  return check_launch("moe_route_quant");
}

int64_t moe_align_max_padded(int64_t numel, int slots, int bsz) {
  return numel + static_cast<int64_t>(slots) * (bsz - 1);
}

int moe_align_block_size(const int32_t* topk_ids, int64_t numel, int slots, int bsz,
                         int32_t* sorted_ids, int32_t* expert_ids, int32_t* npp,
                         hipStream_t st) {
  MW8_REQUIRE(topk_ids && sorted_ids && expert_ids && npp, kErrArg, "moe_align: null pointer");
  MW8_REQUIRE(slots > 0 && slots <= kAlignMaxSlots && bsz > 0 && bsz <= 4096, kErrShape,
              "moe_align: need 0 < slots <= 512 and 0 < block <= 4096 (slots=%d block=%d)", slots,
              bsz);
  MW8_REQUIRE(numel >= 0 && numel < (1ll << 31) - static_cast<int64_t>(slots) * bsz, kErrShape,
              "moe_align: too many pairs");
  const int64_t max_padded = moe_align_max_padded(numel, slots, bsz);
  const int64_t max_blocks = (max_padded + bsz - 1) / bsz;
  int nbits = 1;
  while ((1 << nbits) < slots) ++nbits;
  // each block places R = 1024 * unroll pairs; at most 256 blocks
  const int64_t unroll64 = (numel + 256ll * kAlignThreads - 1) / (256ll * kAlignThreads);
  const int unroll = static_cast<int>(unroll64 < 1 ? 1 : unroll64);
  const int64_t per_block = static_cast<int64_t>(kAlignThreads) * unroll;
  const unsigned grid = static_cast<unsigned>(numel > 0 ? (numel + per_block - 1) / per_block : 1);
  hipLaunchKernelGGL(moe_align_kernel, dim3(grid), dim3(kAlignThreads), 0, st, topk_ids, numel,
                     slots, bsz, unroll, sorted_ids, expert_ids, npp, max_padded, max_blocks, nbits);
  return check_launch("moe_align");
}

int moe_prepare_small(const void* logits, int is_bf16, int64_t M, int E, int topk, int renorm,
                      const void* hidden, int64_t H, float* topk_w, int32_t* topk_ids, int8_t* q,
                      float* s, int slots, int bsz, int32_t* sorted_ids, int32_t* expert_ids,
                      int32_t* npp, hipStream_t st) {
  MW8_REQUIRE(logits && hidden && topk_w && topk_ids && q && s && sorted_ids && expert_ids && npp, kErrArg,
              "moe_prepare_small: null pointer");
  MW8_REQUIRE(M > 0 && E > 0 && E <= 1024 && topk > 0 && topk <= E && topk <= 64 &&
                  M * topk <= kPrepMaxPairs,
              kErrShape, "moe_prepare_small: need 0 < M * topk <= %d, topk <= min(E, 64), E <= 1024 "
              "(M=%lld E=%d topk=%d)", kPrepMaxPairs, (long long)M, E, topk);
  MW8_REQUIRE(slots >= E && slots <= kAlignMaxSlots && bsz > 0 && bsz <= 4096, kErrShape,
              "moe_prepare_small: need E <= slots <= 512 and 0 < block <= 4096 (slots=%d block=%d)",
              slots, bsz);
  MW8_REQUIRE(H > 0 && H % 8 == 0, kErrShape, "moe_prepare_small: need H %% 8 == 0 (H=%lld)", (long long)H);
  MW8_REQUIRE(aligned16(hidden) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0, kErrAlign,
              "moe_prepare_small: hidden needs 16-byte and q 8-byte alignment");
  const int64_t numel = M * topk;
  const int64_t max_padded = moe_align_max_padded(numel, slots, bsz);
  const int64_t max_blocks = (max_padded + bsz - 1) / bsz;
  int nbits = 1;
  while ((1 << nbits) < slots) ++nbits;
  const int vpl = (E + 63) / 64;
  auto go = [&](auto vpl_c) {
    constexpr int V = decltype(vpl_c)::value;
    hipLaunchKernelGGL((moe_prepare_kernel<V>), dim3(1), dim3(kAlignThreads), 0, st, logits, is_bf16, M, E,
                       topk, renorm, static_cast<const uint16_t*>(hidden), H, topk_w, topk_ids, q, s, slots,
                       bsz, sorted_ids, expert_ids, npp, max_padded, max_blocks, nbits);
  };
  if (vpl <= 1) go(std::integral_constant<int, 1>{});
  else if (vpl <= 2) go(std::integral_constant<int, 2>{});
  else if (vpl <= 4) go(std::integral_constant<int, 4>{});
  else if (vpl <= 8) go(std::integral_constant<int, 8>{});
  else go(std::integral_constant<int, 16>{});
  return check_launch("moe_prepare_small");
}

int moe_sum_reduce_bf16(const void* in, int64_t M, int k, int64_t H, void* out, hipStream_t st) {
  MW8_REQUIRE(in && out, kErrArg, "moe_sum_reduce: null pointer");
  MW8_REQUIRE(M >= 0 && k > 0 && H > 0 && H % 8 == 0, kErrShape,
              "moe_sum_reduce: need H %% 8 == 0 (H=%lld)", (long long)H);
  MW8_REQUIRE(aligned16(in) && aligned16(out), kErrAlign, "moe_sum_reduce: 16-byte alignment");
  if (M == 0) return kOk;
  const int64_t n = M * (H / 8);
  hipLaunchKernelGGL(moe_sum_reduce_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                     0, st, static_cast<const uint16_t*>(in), M, k, H, static_cast<uint16_t*>(out));
  return check_launch("moe_sum_reduce");
}

int moe_gemm_w8a8(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                  const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* npp,
                  int64_t max_sorted, const float* topk_w, int top_k, int64_t num_valid,
                  int64_t N, int64_t K, int E, int bsz, void* out, int epi, hipStream_t st) {
  MW8_REQUIRE(A && W && sorted_ids && expert_ids && npp && out, kErrArg, "moe_gemm: null pointer");
  MW8_REQUIRE(epi == kEpiI32 || (sa && sw), kErrArg, "moe_gemm: null scales");
  MW8_REQUIRE(N > 0 && K > 0 && K % 16 == 0 && K <= (1ll << 17), kErrShape,
              "moe_gemm: need K %% 16 == 0 and K <= 131072 (N=%lld K=%lld)", (long long)N,
              (long long)K);
  MW8_REQUIRE(bsz == 16 || bsz == 32 || bsz == 64 || bsz == 128, kErrShape,
              "moe_gemm: block size must be 16, 32, 64 or 128 (got %d)", bsz);
  MW8_REQUIRE(top_k >= 1 && E >= 1 && num_valid >= 0 && max_sorted >= 0, kErrShape,
              "moe_gemm: bad routing sizes");
  MW8_REQUIRE(aligned16(A) && aligned16(W), kErrAlign, "moe_gemm: A and W need 16-byte alignment");
  // the tile core addresses A rows through a 32-bit buffer offset
  MW8_REQUIRE((num_valid / top_k + 1) * K < (1ll << 31), kErrShape,
              "moe_gemm: token matrix of %lld x %lld bytes exceeds 2^31", (long long)(num_valid / top_k),
              (long long)K);
  const int64_t blocks = max_sorted / bsz;  // blocks past num_post_pad exit on device
  if (blocks == 0) return kOk;
  MW8_REQUIRE(blocks < 65536, kErrShape, "moe_gemm: too many expert blocks");
  GemmArgs g{};
  g.A = A; g.sa = sa; g.W = W; g.sw = sw; g.bias = nullptr; g.out = out;
  g.M = 0; g.N = N; g.K = K; g.lda = K; g.ldo = N;
  g.sorted_ids = sorted_ids; g.expert_ids = expert_ids; g.num_post_pad = npp;
  g.topk_w = topk_w; g.num_valid = num_valid; g.top_k = top_k; g.num_experts = E;
  g.staged_out = epi == kEpiBf16 && N % 8 == 0 && aligned16(out);
  g.align_bsz = bsz;
  const int rc = bsz <= 32 ? launch_grouped_small(g, static_cast<unsigned>(blocks), epi, st)
                           : launch_grouped_tile(g, static_cast<unsigned>(blocks), bsz, epi, st);
  if (rc != kOk) return rc;
  return check_launch("moe_gemm");
}

int moe_gemm_act_w8a8(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                      const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* npp,
                      int64_t max_sorted, const float* topk_w, int top_k, int64_t num_valid,
                      int64_t N, int64_t K, int E, int bsz, int act, void* out, hipStream_t st) {
  MW8_REQUIRE(A && sa && W && sw && sorted_ids && expert_ids && npp && out, kErrArg,
              "moe_gemm_act: null pointer");
  MW8_REQUIRE(act == 0 || act == 1, kErrArg, "moe_gemm_act: act must be 0 (silu) or 1 (gelu)");
  MW8_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 64 == 0 && K <= (1ll << 17), kErrShape,
              "moe_gemm_act: need N %% 16 == 0, K %% 64 == 0 and K <= 131072 (N=%lld K=%lld)",
              (long long)N, (long long)K);
  MW8_REQUIRE(bsz == 64 || bsz == 128, kErrShape, "moe_gemm_act: block size must be 64 or 128 (got %d)", bsz);
  MW8_REQUIRE(top_k >= 1 && E >= 1 && E < kPersistMaxSlots && num_valid >= 0 && max_sorted >= 0, kErrShape,
              "moe_gemm_act: bad routing sizes (E=%d)", E);
  MW8_REQUIRE(aligned16(A) && aligned16(W) && aligned16(out), kErrAlign,
              "moe_gemm_act: A, W and out need 16-byte alignment");
  MW8_REQUIRE((num_valid / top_k + 1) * K < (1ll << 31) && N * K < (1ll << 31), kErrShape,
              "moe_gemm_act: operands exceed 32-bit buffer offsets");
  if (max_sorted / bsz == 0) return kOk;
  GemmArgs g{};
  g.A = A; g.sa = sa; g.W = W; g.sw = sw; g.bias = nullptr; g.out = out;
  g.M = 0; g.N = N; g.K = K; g.lda = K; g.ldo = N / 2;
  g.sorted_ids = sorted_ids; g.expert_ids = expert_ids; g.num_post_pad = npp;
  g.topk_w = topk_w; g.num_valid = num_valid; g.top_k = top_k; g.num_experts = E;
  g.staged_out = 1;
  g.align_bsz = bsz;
  if (const int rc = launch_grouped_act(g, act, st)) return rc;
  return check_launch("moe_gemm_act");
}

int moe_gemm_sum_w8a8(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                      const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* npp,
                      int64_t max_sorted, const float* topk_w, int top_k, int64_t num_valid, int64_t N,
                      int64_t K, int E, void* out, hipStream_t st) {
  MW8_REQUIRE(A && sa && W && sw && sorted_ids && expert_ids && npp && out, kErrArg, "moe_gemm_sum: null pointer");
  MW8_REQUIRE(N > 0 && K > 0 && K % 16 == 0 && K <= (1ll << 17), kErrShape,
              "moe_gemm_sum: need K %% 16 == 0 and K <= 131072 (N=%lld K=%lld)", (long long)N, (long long)K);
  MW8_REQUIRE(top_k >= 1 && num_valid >= 0 && num_valid % top_k == 0 && max_sorted >= 0,
              kErrShape, "moe_gemm_sum: bad routing sizes (top_k=%d num_valid=%lld max_sorted=%lld)", top_k,
              (long long)num_valid, (long long)max_sorted);
  MW8_REQUIRE(moe_gemm_sum_lds_bytes(max_sorted, num_valid, E) > 0, kErrShape,
              "moe_gemm_sum: %lld pairs over %lld sorted rows and %d experts exceed the LDS tables "
              "(mw8_moe_gemm_sum_supported)",
              (long long)num_valid, (long long)max_sorted, E);
  MW8_REQUIRE(aligned16(A) && aligned16(W), kErrAlign, "moe_gemm_sum: A and W need 16-byte alignment");
  if (num_valid == 0) return kOk;
  GemmArgs g{};
  g.A = A; g.sa = sa; g.W = W; g.sw = sw; g.bias = nullptr; g.out = out;
  g.M = 0; g.N = N; g.K = K; g.lda = K; g.ldo = N;
  g.sorted_ids = sorted_ids; g.expert_ids = expert_ids; g.num_post_pad = npp;
  g.topk_w = topk_w; g.num_valid = num_valid; g.top_k = top_k; g.num_experts = E;
  g.align_bsz = 16;
  if (const int rc = launch_moe_gemm_sum(g, max_sorted, st, false)) return rc;
  return check_launch("moe_gemm_sum");
}

// ------------------------------------------- router-id rows (no alignment)
// Decode batches of at most kTopkMaxTokens tokens whose top-k experts are
// distinct per token (what topk_softmax produces): an expert then holds at
// most one pair per token, U = ceil(tokens / 16) units of 16, so the grouped
// GEMMs list each expert's pairs from topk_ids themselves and the
// alignment launch disappears.  Ids outside [0, E) are skipped, as the
// alignment does.
constexpr int64_t kTopkMaxTokens = 48;

int topk_units(int64_t num_valid, int top_k) {
  const int64_t tokens = num_valid / top_k;
  return static_cast<int>(tokens <= 16 ? 1 : (tokens + 15) / 16);
}

int moe_topk_check(const int8_t* A, const float* sa, const int8_t* W, const float* sw, const int32_t* topk_ids,
                   int top_k, int64_t num_valid, int64_t N, int64_t K, int E, const void* out, const char* what) {
  MW8_REQUIRE(A && W && topk_ids && out && (sa == nullptr) == (sw == nullptr), kErrArg, "%s: null pointer", what);
  MW8_REQUIRE(N > 0 && K > 0 && K % 16 == 0 && K <= (1ll << 17), kErrShape,
              "%s: need K %% 16 == 0 and K <= 131072 (N=%lld K=%lld)", what, (long long)N, (long long)K);
  MW8_REQUIRE(top_k >= 1 && E >= 1 && E <= 16384 && num_valid >= 0 && num_valid % top_k == 0 &&
                  num_valid / top_k <= kTopkMaxTokens,
              kErrShape, "%s: needs at most %lld tokens (top_k=%d num_valid=%lld E=%d)", what,
              (long long)kTopkMaxTokens, top_k, (long long)num_valid, E);
  MW8_REQUIRE(aligned16(A) && aligned16(W), kErrAlign, "%s: A and W need 16-byte alignment", what);
  MW8_REQUIRE((num_valid / top_k + 1) * K < (1ll << 31) && N * K < (1ll << 31), kErrShape,
              "%s: operands exceed 32-bit buffer offsets", what);
  return kOk;
}

int moe_gemm_topk_w8a8(const int8_t* A, const float* sa, const int8_t* W, const float* sw, const int32_t* topk_ids,
                       const float* topk_w, int top_k, int64_t num_valid, int64_t N, int64_t K, int E, void* out,
                       int epi, hipStream_t st) {
  MW8_REQUIRE(epi == kEpiI32 || (sa && sw), kErrArg, "moe_gemm_topk: null scales");
  if (const int rc = moe_topk_check(A, sa, W, sw, topk_ids, top_k, num_valid, N, K, E, out, "moe_gemm_topk")) return rc;
  if (num_valid == 0) return kOk;
  GemmArgs g{};
  g.A = A; g.sa = sa; g.W = W; g.sw = sw; g.bias = nullptr; g.out = out;
  g.M = 0; g.N = N; g.K = K; g.lda = K; g.ldo = N;
  g.sorted_ids = topk_ids; g.expert_ids = nullptr; g.num_post_pad = nullptr;
  g.topk_w = topk_w; g.num_valid = num_valid; g.top_k = top_k; g.num_experts = E;
  g.align_bsz = 16;
  g.topk_units = topk_units(num_valid, top_k);
  if (const int rc = launch_grouped_topk(g, epi, st)) return rc;
  return check_launch("moe_gemm_topk");
}

int moe_gemm_sum_topk_w8a8(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                           const int32_t* topk_ids, const float* topk_w, int top_k, int64_t num_valid, int64_t N,
                           int64_t K, int E, void* out, hipStream_t st) {
  MW8_REQUIRE(sa && sw, kErrArg, "moe_gemm_sum_topk: null scales");
  if (const int rc = moe_topk_check(A, sa, W, sw, topk_ids, top_k, num_valid, N, K, E, out, "moe_gemm_sum_topk"))
    return rc;
  const int U = topk_units(num_valid, top_k);
  MW8_REQUIRE(moe_gemm_sum_lds_bytes(16 * static_cast<int64_t>(E) * U, num_valid, E) > 0, kErrShape,
              "moe_gemm_sum_topk: %lld pairs over %d experts (%d units each) exceed the LDS tables",
              (long long)num_valid, E, U);
  if (num_valid == 0) return kOk;
  GemmArgs g{};
  g.A = A; g.sa = sa; g.W = W; g.sw = sw; g.bias = nullptr; g.out = out;
  g.M = 0; g.N = N; g.K = K; g.lda = K; g.ldo = N;
  g.sorted_ids = topk_ids; g.expert_ids = nullptr; g.num_post_pad = nullptr;
  g.topk_w = topk_w; g.num_valid = num_valid; g.top_k = top_k; g.num_experts = E;
  g.align_bsz = 16;
  g.topk_units = U;
  if (const int rc = launch_moe_gemm_sum(g, 16 * static_cast<int64_t>(E) * U, st, true)) return rc;
  return check_launch("moe_gemm_sum_topk");
}

}  // namespace mw8
