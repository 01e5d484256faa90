/*
 * libmw8_calib.so -- measurement kernels behind the benchmark's device
 * ceilings (bench.py device.measured and --mode ceilings).  No reference
 * counterpart: the reference times only its own kernels
 * (python/minisgl/benchmark/perf.py:10-51).  They live in a library of
 * their own so that the product library (include/mw8.h) carries no
 * measurement surface; nothing on the model path calls them.
 *
 * Launch-only like every entry point of libmw8.so: the caller times them
 * with events on the same stream.  They return 0 or an MW8_ERR_* code
 * (include/mw8.h); mw8_calib_last_error() holds this library's last
 * message.  `sink` (device int32 [mw8_calib_sink_len()]) receives one value
 * per thread, so that nothing is optimised away.
 *
 * mw8_calib_mfma_i8: 256 x 1024 threads, each running iters x 64
 *   v_mfma_i32_16x16x64_i8 (the instruction of the large-M GEMM tiles) on
 *   registers only, 32768 int8 ops each: random_operands = 0 uses constant
 *   operands (the nominal-clock rate), 1 random ones (the power-limited
 *   rate int8 GEMMs on real data see).
 * mw8_calib_read: grid-stride streaming read of `bytes` (multiple of 16,
 *   16-byte aligned) -- the practical HBM read rate at that size.
 * mw8_calib_stream_lds: 256 blocks x 4 waves moving region_bytes (a
 *   multiple of 32 KiB, at most 1 GiB) per block, `passes` times, from
 *   global memory into LDS with 16-byte buffer_load ... lds, 8-16 KB in
 *   flight per wave.  shared = 1: block b reads region b % 8, so the 32
 *   blocks of an XCD share one region (L2-resident for a small region read
 *   several times; for a large one a lockstep stream in which each line is
 *   fetched once and requested 32 times together); shared = 0: block b
 *   reads region b.  buf holds region_bytes x (shared ? 8 : 256) bytes.
 */
#ifndef MW8_CALIB_H_
#define MW8_CALIB_H_

#include <stdint.h>

#include "mw8.h" /* mw8_stream_t, MW8_ERR_* */

#ifdef __cplusplus
extern "C" {
#endif

const char* mw8_calib_last_error(void);
int64_t mw8_calib_sink_len(void);
int mw8_calib_mfma_i8(int32_t random_operands, int32_t iters, int32_t* sink, int64_t sink_len,
                      mw8_stream_t stream);
int mw8_calib_read(const void* buf, int64_t bytes, int32_t* sink, int64_t sink_len,
                   mw8_stream_t stream);
int mw8_calib_stream_lds(const void* buf, int64_t region_bytes, int32_t passes, int32_t shared,
                         int32_t* sink, int64_t sink_len, mw8_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MW8_CALIB_H_ */
