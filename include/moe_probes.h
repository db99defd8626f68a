/*
 * moe_probes.h -- measurement probes in libmoe_probes.so (gfx950).
 *
 * Not part of the dispatch path and no counterpart in the reference: small
 * kernels that measure, on the GPU at hand, the ceilings the dispatch kernels'
 * roofline fractions are read against (bench.py --ceilings).  A library of
 * their own, kept out of libmoe_dispatch.so; it links libmoe_dispatch.so for
 * the status functions, so the conventions are those of moe_dispatch.h
 * (status codes, moe_last_error() of libmoe_dispatch.so, `void *stream`).
 */
#ifndef MOE_PROBES_H_
#define MOE_PROBES_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* `waves` wavefronts (a multiple of 4; 256 threads per workgroup) each issue
 * iters x 16 independent v_mfma_f32_16x16x32_bf16 on register operands:
 * waves * iters * 16 * 16384 FLOP.  sink: fp32 [waves * 64] (one value per
 * thread, keeps the work observable). */
int moe_probe_mfma(int64_t waves, int64_t iters, float *sink, void *stream);

/* Streams n_vec 16-byte vectors with `blocks` workgroups of 256 threads, each
 * over a contiguous segment: mode 0 copy src -> dst, 1 read src (dst receives
 * one vector per thread, at most blocks * 256), 2 write dst; mode + 4: the
 * same with non-temporal loads and stores.  16-byte aligned buffers. */
int moe_probe_stream(int mode, const void *src, void *dst, int64_t n_vec, int64_t blocks, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MOE_PROBES_H_ */
