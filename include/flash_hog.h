/*
 * flash_hog.h - C ABI of the MI355X-native Flash-HOG attention kernels.
 *
 * Plain pointers and sizes only. Every entry point enqueues its kernels on the
 * given HIP stream and returns without synchronising; it allocates nothing,
 * frees nothing and keeps no pointer after it returns (all outputs and the
 * fp32 row-statistic workspace are caller owned, as the reference's XLA FFI
 * handler exposes its dD/B scratch as results). No entry point except
 * fhog_attention_bwdbwd_noalloc holds mutable global state, so concurrent
 * calls on different streams are safe.
 *
 * Layouts (identical to the reference's attention seam):
 *   q, o, dout, ddq, dq, dq2, ddo   : (batch, n_q, heads, head_dim) contiguous
 *   k, v, ddk, ddv, dk, dv, dk2, dv2: (batch, n_k, kv_heads, head_dim) contiguous
 *   lse, delta, ddelta, bstat       : (batch, heads, n_q) fp32 contiguous
 * lse is the natural-log logsumexp of the scaled, masked logits
 * (flash_hog/jax/_pallas_gpu_kernel.py:97).
 *
 * Grouped-query attention: heads must be a multiple of kv_heads; query head h
 * attends with key/value head h / (heads / kv_heads), and dk, dv, dk2, dv2 sum
 * over the heads of a group (_pallas_gpu_kernel.py:99, 106-107, 333-370).
 *
 * causal (enum fhog_causal): FHOG_CAUSAL_TOP_LEFT shows key j to query i iff
 * j <= i (_pallas_gpu_kernel.py:37-41, the reference kernel's mask);
 * FHOG_CAUSAL_BOTTOM_RIGHT iff j <= i + n_k - n_q
 * (flash_hog/_jax_refs/jax_impl.py:104-109); the two agree when n_q == n_k.
 * A query that sees no key (bottom-right with n_q > n_k) gets o = 0,
 * lse = +inf and zero gradients.
 * Tensor pointers must be 16-byte aligned, row-statistic pointers 4-byte aligned.
 *
 * Supported: dtype FHOG_DTYPE_{BF16,F16} with head_dim 64, 128 or 256,
 * FHOG_DTYPE_F32 with head_dim 64 or 128; any n_q, n_k >= 1 (ragged tails
 * are masked); any finite nonzero scale, negative included (scale 0 returns
 * FHOG_ERR_UNSUPPORTED).
 */
#ifndef FLASH_HOG_H_
#define FLASH_HOG_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as hipStream_t. */
typedef struct ihipStream_t* fhog_stream_t;

enum fhog_status {
  FHOG_OK = 0,
  FHOG_ERR_INVALID_ARGUMENT = 1, /* null/misaligned pointer, bad size, bad enum */
  FHOG_ERR_UNSUPPORTED = 2,      /* valid request the library has no kernel for */
  FHOG_ERR_LAUNCH = 3            /* the HIP runtime rejected a kernel launch */
};

enum fhog_dtype { FHOG_DTYPE_F32 = 0, FHOG_DTYPE_F16 = 1, FHOG_DTYPE_BF16 = 2 };

/* Values of the `causal` argument. */
enum fhog_causal { FHOG_CAUSAL_NONE = 0, FHOG_CAUSAL_TOP_LEFT = 1, FHOG_CAUSAL_BOTTOM_RIGHT = 2 };

/* Version of this ABI (major * 100 + minor). */
int fhog_abi_version(void);

/* Static description of a status code. */
const char* fhog_status_string(int status);

/* Message of the last failed call on this thread ("" if none). */
const char* fhog_last_error(void);

/*
 * Whether this library has kernels for the given problem, without launching
 * or allocating anything: FHOG_OK, or the status (with its fhog_last_error
 * message) that the entry points would return for these sizes, dtype, causal
 * and scale. device >= 0 also requires HIP device `device` to be a gfx950
 * GPU (else FHOG_ERR_UNSUPPORTED); device < 0 checks the arguments only.
 * Counterpart of the reference's supported() (flash_hog/jax/_tk_gpu.py:70-80),
 * which answers the same question for its ThunderKittens kernels before a
 * call, so that a caller can route unsupported shapes elsewhere.
 */
int fhog_attention_supported(int device, int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim,
                             int dtype, int causal, float scale);

/* Bytes of fp32 row-statistic workspace per (delta, ddelta, bstat) array:
 * batch * heads * n_q * 4. */
size_t fhog_row_stat_bytes(int batch, int heads, int n_q);

/*
 * Forward: o = softmax(scale q k^T [causal]) v and lse.
 * Replaces the cuDNN forward the reference reaches through
 * dot_product_attention_fwd / dot_product_attention_fwd_rule
 * (flash_hog/jax/_attention_impl.py:224-239), which returns (out, activation)
 * with activation = the (B, N, T) fp32 logsumexp.
 */
int fhog_attention_fwd(fhog_stream_t stream,
                       const void* q, const void* k, const void* v,
                       void* o, float* lse,
                       int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim,
                       int dtype, int causal, float scale);

/*
 * First backward: dq, dk, dv from (q, k, v, o, lse, dout).
 * Replaces the cuDNN backward the reference reaches through
 * dot_product_attention_bwd_rule (flash_hog/jax/_attention_impl.py:242-261).
 * delta (caller-owned, fhog_row_stat_bytes) receives D = rowsum(o * dout).
 */
int fhog_attention_bwd(fhog_stream_t stream,
                       const void* q, const void* k, const void* v,
                       const void* o, const void* dout, const float* lse,
                       void* dq, void* dk, void* dv, float* delta,
                       int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim,
                       int dtype, int causal, float scale);

/*
 * Double backward (Flash-HOG): given the residual (q, k, v, o, lse, dout) of
 * the first backward and the cotangents (ddq, ddk, ddv) of its outputs,
 * returns dq2, dk2, dv2 (cotangents of q, k, v) and ddo (cotangent of dout).
 * Replaces dot_product_attention_bwd_rule_bwd_rule
 * (flash_hog/jax/_attention_impl.py:278-303) -> flash_bwdbwd
 * (flash_hog/jax/_pallas_gpu.py:51-114) -> flash_bwdbwd0
 * (flash_hog/jax/_pallas_gpu_kernel.py:49-422), and the XLA FFI handler
 * TkBwdBwd (flash_hog/csrc/tk_bwdbwd/ffi.cu:26-98), whose inputs
 * (Q,K,V,dO,ddQ,ddK,ddV,L,D), attribute scale and results
 * (dQ2,ddO,dK2,dV2,dD,B) it mirrors, except that D is computed here from o
 * (as flash_bwdbwd0 does at _pallas_gpu_kernel.py:110) and written to delta.
 * delta, ddelta, bstat: caller-owned workspace, fhog_row_stat_bytes each;
 * on return they hold D, dD and B. Like TkBwdBwd's dD and B they are
 * scratch between the two passes (pass 4 uses B through c = D dD + B).
 * Accuracy: D, dD and B are fp32 sums of fp32 per-pair terms (2-byte types:
 * B = sum_j X_j - dD (sum_j P_j u_j + D), the per-pair form; fp32:
 * B = r1 - dD r2 - D dD + r3). Over a call each is within the dtype's
 * tolerance of its exact value relative to its own largest entry. Per row,
 * B = c - D dD is a difference that any formula for it must take, so a row
 * whose B is much smaller than its D dD holds B only to about 1e-7 |c|
 * (fp32 rounding of c), not to 1e-7 |B|.
 * Two kernels are enqueued on stream; the second reads the statistics the
 * first writes.
 */
int fhog_attention_bwdbwd(fhog_stream_t stream,
                          const void* q, const void* k, const void* v,
                          const void* o, const void* dout,
                          const void* ddq, const void* ddk, const void* ddv,
                          const float* lse,
                          void* dq2, void* dk2, void* dv2, void* ddo,
                          float* delta, float* ddelta, float* bstat,
                          int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim,
                          int dtype, int causal, float scale);

/*
 * One stage of fhog_attention_bwdbwd: stage 1 = passes 1-3 (tiled over
 * queries; computes D, dD, B into delta/ddelta/bstat and writes dq2, ddo),
 * stage 2 = pass 4 (tiled over keys; reads delta/ddelta/bstat, writes dk2,
 * dv2). Running stage 1 then stage 2 on one stream equals
 * fhog_attention_bwdbwd. The reference's handler always launches both
 * (ffi.cu:71-73); the split exists so that the stages can be timed, profiled
 * or ordered by the caller (stage 2 must see stage 1's statistics). Pointers
 * a stage does not touch may be null: stage 1 ignores dk2, dv2; stage 2
 * ignores o, dq2, ddo.
 */
int fhog_attention_bwdbwd_stage(fhog_stream_t stream, int stage,
                                const void* q, const void* k, const void* v,
                                const void* o, const void* dout,
                                const void* ddq, const void* ddk, const void* ddv,
                                const float* lse,
                                void* dq2, void* dk2, void* dv2, void* ddo,
                                float* delta, float* ddelta, float* bstat,
                                int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim,
                                int dtype, int causal, float scale);

/*
 * fhog_attention_bwdbwd without the row-statistic workspace arguments: D, dD
 * and B go to a static device array inside the library (12 MiB per device,
 * for batch * heads * n_q up to 1048576 rows; larger calls return
 * FHOG_ERR_UNSUPPORTED). Outputs are those of fhog_attention_bwdbwd, bit for
 * bit. It calls no allocating routine, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc); the first call on a device looks up the array's
 * address there once. It has no counterpart in the reference; it is for
 * callers that cannot allocate. Every call on a device shares
 * that device's array: calls that overlap on one device (concurrent streams)
 * race on it and must be serialised by the caller.
 */
int fhog_attention_bwdbwd_noalloc(fhog_stream_t stream,
                                  const void* q, const void* k, const void* v,
                                  const void* o, const void* dout,
                                  const void* ddq, const void* ddk, const void* ddv,
                                  const float* lse,
                                  void* dq2, void* dk2, void* dv2, void* ddo,
                                  int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim,
                                  int dtype, int causal, float scale);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_HOG_H_ */
