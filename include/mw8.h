/*
 * mw8.h -- C ABI of the MI355X-native W8A8 int8 linear + fused-MoE library
 * (libmw8.so, built for gfx950 with hipcc).
 *
 * Every entry point is asynchronous on the given HIP stream (pass
 * torch.cuda.current_stream().cuda_stream, or 0 for the null stream),
 * never synchronizes, never allocates device memory and is safe to capture
 * in a HIP graph.  The caller owns every buffer; pointers are device
 * pointers, tensors are row-major with the last dimension contiguous.
 *
 * Return value: 0 on success, a nonzero MW8_ERR_* code otherwise; the
 * message of the last failure on the calling thread is returned by
 * mw8_last_error().  No C++ exception crosses this boundary.
 *
 * Numerics (checked bit-exactly against the CPU oracle):
 *   quantizer   s[m] = amax_k|x[m,k]| / 127 (fp32 IEEE division),
 *               q[m,k] = clamp(rint(x[m,k] / s[m]), -127, 127), zero row -> s = 0, q = 0
 *   GEMM        acc[m,n] = sum_k A[m,k] * W[n,k]   (exact int32)
 *   epilogue    y[m,n] = bf16_rne(((float)acc * sa[m]) * sw[n] [+ bias[n]] [* routed])
 *               each operation rounded separately (no FMA contraction)
 */
#ifndef MW8_H_
#define MW8_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mw8_stream_t; /* hipStream_t */

enum {
  MW8_OK = 0,
  MW8_ERR_ARG = 1,       /* null pointer or bad enum */
  MW8_ERR_SHAPE = 2,     /* unsupported or inconsistent sizes */
  MW8_ERR_ALIGN = 3,     /* pointer / leading dimension misaligned */
  MW8_ERR_WORKSPACE = 4, /* workspace missing or too small */
  MW8_ERR_LAUNCH = 5     /* HIP launch failure */
};

/* Message of the last failure on this thread ("" if none). */
const char* mw8_last_error(void);

/* ABI version (major * 100 + minor). */
int mw8_version(void);

/*
 * Compute units, peak engine clock (kHz) and L2 bytes of a device; used to
 * derive the MFMA peak the benchmark reports against.  No reference
 * counterpart (measurement helper).
 */
int mw8_device_info(int32_t device, int32_t* num_cu, int32_t* clock_khz, int64_t* l2_bytes);

/*
 * Per-token dynamic int8 quantizer: x bf16 [M, K] (row stride ldx elements)
 * -> q int8 [M, K] (row stride ldq) and s fp32 [M].
 * No reference counterpart: it is inserted before the reference's
 * F.linear (python/minisgl/layers/linear.py:32) and before both grouped
 * GEMMs of fused_experts_impl (python/minisgl/moe/fused.py:192,208).
 */
int mw8_quant_per_token_bf16(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                             int64_t ldq, float* s, mw8_stream_t stream);

/*
 * Fused activation + requant: x bf16 [R, 2d] (gate | up) ->
 * a = bf16(act(gate) * up), then quantized like mw8_quant_per_token_bf16 into
 * q int8 [R, d], s fp32 [R].  act: 0 = silu, 1 = gelu (erf).  act_out
 * (bf16 [R, d]) is optional and receives a.  q and s may both be NULL when
 * act_out is given (activation only, no requant).  2d % 16 == 0.
 * Replaces silu_and_mul / gelu_and_mul (python/minisgl/layers/activation.py:9-18)
 * as called at python/minisgl/moe/fused.py:206-207 and
 * python/minisgl/models/utils.py:48, fused with the requant of the next GEMM.
 */
int mw8_act_and_mul_quant_bf16(const void* x, int64_t R, int64_t two_d, int32_t act, int8_t* q,
                               float* s, void* act_out, mw8_stream_t stream);

/*
 * Fused RMSNorm + per-token requant: x bf16 [M, H], weight bf16 [H].
 *   h = x, or h = bf16(x + residual) written back to residual (in place)
 *   ss = sum_k h_k^2 accumulated in fp64 (each square exact),
 *   r  = 1 / sqrt(fp32(ss / H) + eps)      (IEEE fp32),
 *   y  = bf16((h * r) * weight)            (each product rounded)
 * then y is quantized like mw8_quant_per_token_bf16 into q int8 [M, H] and
 * s fp32 [M]; y (bf16 [M, H], may alias x) is written only if non-NULL.
 * q and s may both be NULL (plain RMSNorm; y required).  H % 8 == 0,
 * H <= 32768.
 * Replaces flashinfer rmsnorm / fused_add_rmsnorm (RMSNorm / RMSNormFused,
 * python/minisgl/layers/norm.py:8-38, called at
 * python/minisgl/models/qwen3.py:37-40) together with the input quantizer
 * of the W8A8 linear that follows them.
 */
int mw8_rmsnorm_quant_bf16(const void* x, void* residual, const void* weight, float eps, int64_t M,
                           int64_t H, int8_t* q, float* s, void* y, mw8_stream_t stream);

/*
 * Plain RMSNorm over strided rows: rows are addressed as [G, inner, H] --
 * row (g, i) of x at x + g * ldx + i * H, of y at y + g * ldy + i * H
 * (elements; the inner rows contiguous) -- with the numerics of
 * mw8_rmsnorm_quant_bf16 (no residual, no quantization).  y may equal x
 * (in place).  H % 8 == 0, H <= 32768, ldx and ldy multiples of 8 and
 * >= inner * H, x, y and weight 16-byte aligned.
 * Replaces flashinfer rmsnorm on the per-head views of a qkv row
 * (RMSNorm.forward_inplace(q.view(-1, heads, head_dim)),
 * python/minisgl/layers/norm.py:18-19, called at
 * python/minisgl/layers/attention.py:49-53), which are not contiguous.
 */
int mw8_rmsnorm_strided_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, const void* weight,
                             float eps, int64_t G, int64_t inner, int64_t H, mw8_stream_t stream);

/*
 * Tile-configuration override of the calling thread (other threads keep
 * the automatic choice; a thread starts on it): decode_cfg indexes the dense
 * decode-core configurations (forcing one keeps M <= 64 on the decode
 * core), tile_cfg the dense tile-core ones (forcing one takes M > 32 to the
 * tile core), moe_cfg the grouped (fused-MoE) configurations (for block
 * sizes 64 and 128, and separately numbered for block size 16); -1
 * restores the automatic choice.  Results do not depend on the
 * configuration (exact integer accumulation).  Tuning hook; no reference
 * counterpart.
 */
void mw8_set_tuning(int32_t decode_cfg, int32_t tile_cfg, int32_t moe_cfg);

/*
 * Number of configurations mw8_set_tuning accepts: kind 0 decode, 1 tile,
 * 2 grouped (64/128-row blocks), 3 grouped (16-row blocks); 0 for other
 * kinds.  Tuning hook; no reference counterpart.
 */
int32_t mw8_tuning_count(int32_t kind);

/*
 * Name of the kernel mw8_gemm_w8a8_* runs for (M, N, K) under the current
 * tuning: "decode3_gemm_kernel" or "decode_gemm_kernel" for the decode
 * cores, else the tile kernel with its leading template arguments as a
 * kernel trace prints them (e.g. "tile3_gemm_kernel<256, 256, 128, 4, 2,
 * 2>", "ksplit_gemm_kernel<128, 128, 2, 2, 2, 2, 3>"); "" for invalid
 * sizes.  Profiling aid; no reference counterpart.
 */
const char* mw8_gemm_kernel_name(int64_t M, int64_t N, int64_t K);

/*
 * Bytes of workspace mw8_gemm_w8a8_* uses for (M, N, K): the int32 partial
 * tiles of the tile core's K split (for the tiling the call will choose,
 * including a mw8_set_tuning override: with T tiles and S = CUs x resident
 * blocks per CU, the r = T mod S tiles of the last partial wave, all T when
 * T < S, are cut into sp = min(S / r, K / BK, 16) K ranges when sp >= 2;
 * each range writes one BM x BN int32 tile, summed in range order by a
 * second kernel on the same stream).  0 when no split applies.  A NULL or
 * smaller workspace is not an error: the GEMM then runs every tile whole
 * (same result, slower).  The workspace holds no state between calls;
 * calls that share one must be ordered (one stream).  No reference
 * counterpart.
 */
size_t mw8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * Upper bound of mw8_gemm_workspace_bytes over every (M, N, K) and tuning
 * override on the current device (r x sp <= S, so S x the largest split
 * tile): a caller that reserves this once never has to grow the workspace,
 * e.g. between HIP graph captures.  No reference counterpart.
 */
size_t mw8_gemm_workspace_max_bytes(void);

/*
 * W8A8 linear: y bf16 [M, N] = epilogue(A int8 [M, K] . W int8 [N, K]^T,
 * sa fp32 [M], sw fp32 [N], bias bf16 [N] or NULL).  K % 16 == 0,
 * A and W 16-byte aligned.
 * Replaces _LinearTPImpl.forward -> F.linear(x, weight, bias)
 * (python/minisgl/layers/linear.py:31-32, also :103 and :124).
 */
int mw8_gemm_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                       const void* bias, void* y, int64_t M, int64_t N, int64_t K, void* workspace,
                       size_t workspace_bytes, mw8_stream_t stream);

/*
 * mw8_gemm_w8a8_bf16 without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The K split's partial tiles go to a static 64 MiB device
 * array of the library, in a code object of its own: a device holds it from
 * the first call of this entry there until the process ends (the other
 * entries never load it); a split that would need more
 * is not taken and those tiles run whole, as mw8_gemm_w8a8_bf16 does with a
 * short workspace (none needs more on a 256-CU MI355X: the bound is
 * mw8_gemm_workspace_max_bytes).
 * The array of the current device is used (make the device of the
 * operands current).  Calls on one device share that array: calls that
 * overlap on one device (concurrent streams) race.  Allocates nothing;
 * results equal mw8_gemm_w8a8_bf16's bit for bit.  (The Python wrappers
 * use mw8_gemm_w8a8_bf16 with a per-call workspace, which concurrent
 * streams do not share.)
 */
int mw8_gemm_w8a8_bf16_noalloc(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                               const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                               mw8_stream_t stream);

/*
 * F.linear of a decode batch in one launch: y bf16 [M, N] = the W8A8
 * linear of the bf16 activations x [M, K] (row stride ldx elements, a
 * multiple of 8; x 16-byte aligned): per-token quantization (the
 * mw8_quant_per_token_bf16 arithmetic), int8 GEMM and epilogue, bit for
 * bit what the two calls write.  Each block of the decode core quantizes
 * the few token rows itself, so there is no quantizer launch and no int8
 * copy of x.  Takes M <= 16 and M K <= 20480 where the decode core
 * streams at most 6 K stages of 256 bytes per wave and one ring slot holds
 * a wave's range of the int8 rows (mw8_linear_bf16_supported); returns
 * MW8_ERR_SHAPE otherwise, also when x spans 2^31 bytes or more.  Replaces _LinearTPImpl.forward -> F.linear
 * (python/minisgl/layers/linear.py:31-32) for an input with no quantizing
 * producer (the attention output into o_proj, python/minisgl/models/utils.py:123).
 */
int mw8_linear_bf16_w8a8(const void* x, int64_t ldx, const int8_t* W, const float* sw, const void* bias,
                         void* y, int64_t M, int64_t N, int64_t K, mw8_stream_t stream);
int32_t mw8_linear_bf16_supported(int64_t M, int64_t N, int64_t K);

/*
 * Same GEMM, raw int32 accumulators acc [M, N] (parity hook; no scales).
 * Test hook for the A4 int32 contract; no reference counterpart.
 */
int mw8_gemm_w8a8_i32(const int8_t* A, const int8_t* W, int32_t* acc, int64_t M, int64_t N,
                      int64_t K, void* workspace, size_t workspace_bytes, mw8_stream_t stream);

/*
 * The gate_up GEMM with the gated activation in its epilogue: y bf16
 * [M, I] = bf16(act(g) * u), g and u the bf16 W8A8 linear outputs of the
 * gate rows W[0:I] and the up rows W[I:2I] of a gate|up weight W int8
 * [2I, K] (scales sw fp32 [2I]), act 0 = silu, 1 = gelu (erf): bit for bit
 * mw8_gemm_w8a8_bf16 into [M, 2I] followed by the activation of
 * mw8_act_and_mul_quant_bf16 (its act_out), without the [M, 2I]
 * intermediate.  Replaces gate_up_proj -> act_fn of GatedMLP.forward
 * (python/minisgl/models/utils.py:44-50; silu_and_mul,
 * python/minisgl/layers/activation.py:9-12).  Takes I % 8 == 0,
 * K % 128 == 0 and shapes the plain GEMM runs on its ring cores (large
 * enough M; mw8_gemm_act_supported), else MW8_ERR_SHAPE.  Workspace as
 * mw8_gemm_w8a8_bf16, sized by mw8_gemm_act_workspace_bytes.
 */
int mw8_gemm_act_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw, int32_t act, void* y,
                           int64_t M, int64_t I, int64_t K, void* workspace, size_t workspace_bytes,
                           mw8_stream_t stream);
int32_t mw8_gemm_act_supported(int64_t M, int64_t I, int64_t K);
size_t mw8_gemm_act_workspace_bytes(int64_t M, int64_t I, int64_t K);

/*
 * Router: logits [M, E] (bf16 if logits_is_bf16 else fp32) -> fp32 softmax,
 * top-k, optional renormalisation (w / sum w, then w / (sum w + 1e-8)).
 * topk_w fp32 [M, topk], topk_ids int32 [M, topk].  E <= 1024, topk <= 64.
 * Replaces fused_topk -> sgl_kernel.topk_softmax (python/minisgl/moe/fused.py:9-28).
 */
int mw8_topk_softmax(const void* logits, int32_t logits_is_bf16, int64_t M, int32_t E,
                     int32_t topk, int32_t renormalize, float* topk_w, int32_t* topk_ids,
                     mw8_stream_t stream);

/* numel + slots * (block - 1): length of sorted_ids (python/minisgl/moe/fused.py:73). */
int64_t mw8_moe_align_max_padded(int64_t numel, int32_t slots, int32_t block_size);

/*
 * Expert alignment: topk_ids int32 [numel] -> sorted_ids int32
 * [mw8_moe_align_max_padded(...)] (pairs grouped by expert in ascending flat
 * order, each group padded to a multiple of block_size with the sentinel
 * numel), expert_ids int32 [ceil(max_padded / block_size)] (-1 past the
 * used blocks), num_post_pad int32 [1].  Ids outside [0, slots) are skipped.
 * slots <= 512.  The count stays on the device.
 * Replaces moe_align_block_size -> sgl_kernel.moe_align_block_size
 * (python/minisgl/moe/fused.py:31-89; the reference passes slots = E + 1, :81).
 */
int mw8_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int32_t slots,
                             int32_t block_size, int32_t* sorted_ids, int32_t* expert_ids,
                             int32_t* num_post_pad, mw8_stream_t stream);

/*
 * Grouped W8A8 GEMM over expert segments.  For every sorted position r
 * below *num_post_pad with p = sorted_ids[r] < num_valid:
 *   out[p, :] = epilogue(A[p / top_k] . W[e]^T, sa[p / top_k], sw[e], routed = topk_w[p])
 * where e = expert_ids[r / block_size]; topk_w may be NULL (no routed
 * multiply).  A int8 [*, K], W int8 [E, N, K], sw fp32 [E, N], out bf16
 * [num_valid, N].  block_size in {16, 32, 64, 128}.
 * Replaces fused_moe_kernel_triton / fused_moe_kernel
 * (python/minisgl/kernel/moe_impl.py:6-62, python/minisgl/kernel/triton/fused_moe.py:50-193).
 */
int mw8_moe_gemm_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                           const int32_t* sorted_ids, const int32_t* expert_ids,
                           const int32_t* num_post_pad, int64_t max_sorted, const float* topk_w,
                           int32_t top_k, int64_t num_valid, int64_t N, int64_t K, int32_t E,
                           int32_t block_size, void* out, mw8_stream_t stream);

/*
 * The MoE layer's down-projection GEMM with the top-k slot sum fused in, for
 * decode batches (16-row alignment blocks).  For every token t <
 * num_valid / top_k and column n < N:
 *   out[t, n] = bf16(sum over slots i = 0 .. top_k-1, in order, in fp32, of
 *               bf16(epilogue(A[p] . W[e_p][n], sa[p], sw[e_p][n], routed = topk_w[p])))
 * with p = t * top_k + i and e_p the expert of p's alignment block -- the
 * bits of mw8_moe_gemm_w8a8_bf16 (top_k = 1, block_size 16) followed by
 * mw8_moe_sum_reduce_bf16 over [num_valid / top_k, top_k, N].  topk_w null:
 * no routed weight (routed on GEMM1's input).  A pair whose expert lies
 * outside [0, E) contributes +0.  Each block owns 8 output columns of every
 * token and keeps its pairs' values in LDS, so no workspace and no second
 * launch.  A int8 [num_valid, K], sa fp32 [num_valid], W int8 [E, N, K], sw
 * fp32 [E, N], sorted_ids / expert_ids / num_post_pad from
 * mw8_moe_align_block_size with block_size 16 (max_sorted = length of
 * sorted_ids), out bf16 [num_valid / top_k, N]; K % 16 ==
 * 0, num_valid % top_k == 0, 16-byte aligned A and W, and
 * mw8_moe_gemm_sum_supported(max_sorted, num_valid, E) (E <= 256,
 * num_valid <= 2048, max_sorted <= 6144, and the LDS tables fit: every
 * decode batch of 128 experts x top-8, up to 1024 pairs at 256 experts).
 * Replaces fused_moe_kernel
 * (GEMM2, MUL_ROUTED_WEIGHT) + moe_sum_reduce
 * (python/minisgl/moe/fused.py:212-226, python/minisgl/kernel/moe_impl.py:65-98).
 */
int mw8_moe_gemm_sum_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                               const int32_t* sorted_ids, const int32_t* expert_ids,
                               const int32_t* num_post_pad, int64_t max_sorted, const float* topk_w,
                               int32_t top_k, int64_t num_valid, int64_t N, int64_t K, int32_t E, void* out,
                               mw8_stream_t stream);

/* 1 if mw8_moe_gemm_sum_w8a8_bf16 accepts these routing sizes (its LDS tables fit), else 0.  Host only. */
int32_t mw8_moe_gemm_sum_supported(int64_t max_sorted, int64_t num_valid, int32_t E);

/*
 * The two grouped GEMMs of a decode batch without the alignment pass: the
 * expert rows come straight from the router's topk_ids [num_valid] (blocks
 * list the pairs routed to their expert, in units of 16), for batches of at
 * most 48 tokens (num_valid / top_k <= 48) whose top_k experts per token
 * are distinct, as topk_softmax produces them -- every expert then holds at
 * most one pair per token, ceil(tokens / 16) units.  Ids outside [0, E) are
 * skipped, as the alignment skips them.  Results are bit-identical to the
 * aligned forms with 16-row blocks.
 *
 * mw8_moe_gemm_topk_w8a8_bf16: GEMM1 as mw8_moe_gemm_w8a8_bf16 (out bf16
 * [num_valid, N], pair rows; topk_w null or the routed weights).
 * mw8_moe_gemm_sum_topk_w8a8_bf16: GEMM2 + slot sum as
 * mw8_moe_gemm_sum_w8a8_bf16 (out bf16 [num_valid / top_k, N]; E <= 256 and
 * E * ceil(tokens / 16) <= 384).
 * Replace moe_align_block_size + fused_moe_kernel (GEMM1), and
 * fused_moe_kernel (GEMM2) + moe_sum_reduce, for decode batches
 * (python/minisgl/moe/fused.py:71-89, :192-226).
 */
int mw8_moe_gemm_topk_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                                const int32_t* topk_ids, const float* topk_w, int32_t top_k, int64_t num_valid,
                                int64_t N, int64_t K, int32_t E, void* out, mw8_stream_t stream);
int mw8_moe_gemm_sum_topk_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                                    const int32_t* topk_ids, const float* topk_w, int32_t top_k,
                                    int64_t num_valid, int64_t N, int64_t K, int32_t E, void* out,
                                    mw8_stream_t stream);

/*
 * Gate|up grouped GEMM with the gated activation fused into its epilogue:
 * W int8 [E, N = 2I, K] holds the gate rows then the up rows of each expert;
 * out bf16 [num_valid, I] receives act(g) * u with g, u the bf16 outputs the
 * grouped GEMM above would write for columns i and I + i (act 0: silu with
 * the hardware reciprocal, 1: erf-gelu), rounded to bf16 -- bit-identical to
 * mw8_moe_gemm_w8a8_bf16 followed by mw8_act_and_mul_quant_bf16's
 * activation output.  block_size 64 or 128, N % 16 == 0, K % 64 == 0,
 * E < 512, out 16-byte aligned.  Replaces fused_moe_kernel (GEMM1) +
 * silu_and_mul (python/minisgl/moe/fused.py:195-210,
 * python/minisgl/layers/activation.py:9-12) for prefill batches.
 */
int mw8_moe_gemm_act_w8a8_bf16(const int8_t* A, const float* sa, const int8_t* W, const float* sw,
                               const int32_t* sorted_ids, const int32_t* expert_ids,
                               const int32_t* num_post_pad, int64_t max_sorted, const float* topk_w,
                               int32_t top_k, int64_t num_valid, int64_t N, int64_t K, int32_t E,
                               int32_t block_size, int32_t act, void* out, mw8_stream_t stream);

/* Same, raw int32 accumulators out [num_valid, N] (parity hook; no reference counterpart). */
int mw8_moe_gemm_w8a8_i32(const int8_t* A, const int8_t* W, const int32_t* sorted_ids,
                          const int32_t* expert_ids, const int32_t* num_post_pad,
                          int64_t max_sorted, int32_t top_k, int64_t num_valid, int64_t N,
                          int64_t K, int32_t E, int32_t block_size, int32_t* out,
                          mw8_stream_t stream);

/*
 * Router and hidden-state quantizer in one launch (one wave per token):
 * topk_w / topk_ids as mw8_topk_softmax and q / s as
 * mw8_quant_per_token_bf16 on hidden bf16 [M, H] (row stride H), bit for
 * bit.  H % 8 == 0, hidden 16-byte and q 8-byte aligned; E and topk as
 * mw8_topk_softmax.  Replaces fused_topk (python/minisgl/moe/fused.py:9-28)
 * plus the quantization of hidden_states before GEMM1 (:192).
 */
int mw8_moe_route_quant(const void* logits, int32_t is_bf16, int64_t M, int32_t E, int32_t topk,
                        int32_t renorm, const void* hidden, int64_t H, float* topk_w, int32_t* topk_ids,
                        int8_t* q, float* s, mw8_stream_t stream);

/*
 * Small-batch MoE preparation in one launch: the router of
 * mw8_topk_softmax (logits [M, E] -> topk_w fp32 / topk_ids int32 [M, topk]),
 * the per-token quantization of the hidden rows of mw8_quant_per_token_bf16
 * (hidden bf16 [M, H] -> q int8 [M, H], s fp32 [M]) and the alignment of
 * mw8_moe_align_block_size over the selected ids (same outputs and buffer
 * sizes), each bit-identical to its own entry point.  M * topk <= 1024,
 * topk <= min(E, 64), E <= 1024, E <= slots <= 512, H % 8 == 0, hidden
 * 16-byte and q 8-byte aligned.  Replaces, for decode batches, the
 * sequence fused_topk (python/minisgl/moe/fused.py:9-28) ->
 * moe_align_block_size (:31-89) of fused_experts_impl (:157-227) plus the
 * activation quantization of the W8A8 grouped GEMM.
 */
int mw8_moe_prepare_small(const void* logits, int32_t is_bf16, int64_t M, int32_t E, int32_t topk,
                          int32_t renorm, const void* hidden, int64_t H, float* topk_w,
                          int32_t* topk_ids, int8_t* q, float* s, int32_t slots, int32_t block_size,
                          int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_post_pad,
                          mw8_stream_t stream);

/*
 * Slot sum: in bf16 [M, k, H] -> out bf16 [M, H], fp32 sum in slot order.
 * H % 8 == 0.  Replaces moe_sum_reduce_triton
 * (python/minisgl/kernel/moe_impl.py:65-98, python/minisgl/kernel/triton/fused_moe.py:5-47).
 */
int mw8_moe_sum_reduce_bf16(const void* in, int64_t M, int32_t k, int64_t H, void* out,
                            mw8_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MW8_H_ */
