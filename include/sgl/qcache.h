/* sgl/qcache.h — the device copies behind the host-pointer entry points.
 *
 * No counterpart in the reference, whose sgl_matmul_w8a16 / sgl_matmul_nt (reference
 * src/quant.c:44-89, src/ops.c:243-279) keep no state.  In this build those calls run on the GPU,
 * and the weight (W with its scales sw, or the f32 W) is uploaded once, on its first use, and
 * kept on the device, keyed by the host pointers, the shape and a fingerprint of sampled weight
 * bytes (and of every scale).  Callers that load a model once and multiply many times, as the
 * reference's proj_nt does (reference src/llama.c:876-884), pay the upload once.
 *
 * A caller that frees a weight buffer, or writes into it after it has been multiplied, releases
 * its device copy first: the fingerprint catches most, not all, such changes.  The total size of
 * the copies is bounded by the environment variable SGL_QCACHE_MB (default 16384); beyond it the
 * least recently used copies are dropped.  Thread-safe.
 */
#ifndef SGL_QCACHE_H
#define SGL_QCACHE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Drop every device copy made from the host buffer `weight` (the W argument of
 * sgl_matmul_w8a16 or sgl_matmul_nt); returns how many were dropped. */
int sgl_qcache_release(const void *weight);
/* Drop every device copy; returns how many were dropped. */
int sgl_qcache_clear(void);

#ifdef __cplusplus
}
#endif

#endif /* SGL_QCACHE_H */
