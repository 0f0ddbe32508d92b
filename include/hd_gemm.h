#ifndef HD_GEMM_HIP_H
#define HD_GEMM_HIP_H

/*
 * GEMM runtime of the MI355X engine: hand-written bf16 MFMA kernels for
 * gfx950 (v_mfma_f32_16x16x32_bf16, fp32 accumulation, multi-stage LDS
 * rings filled by direct global->LDS loads, fused epilogues).
 *
 * Replaces the reference's src/cuda/gemm.h (lines 35-68). Same symbols and
 * argument meaning. There is no vendor library behind hd_linear: the
 * "runtime" holds the tile-configuration choice per shape and a persistent
 * workspace for the caller, nothing else.
 */

#include <stddef.h>
#include <stdint.h>

#include "hidream_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hd_gemm_runtime hd_gemm_runtime;

/* gemm.h:35 - selects the device, allocates `workspace_bytes` of device
 * memory for the caller, becomes the active runtime. NULL on failure. */
hd_gemm_runtime *hd_gemm_runtime_init(int device_id, size_t workspace_bytes);
/* gemm.h:38 */
void hd_gemm_runtime_destroy(hd_gemm_runtime *rt);
/* gemm.h:41-42 */
void *hd_gemm_workspace(hd_gemm_runtime *rt);
size_t hd_gemm_workspace_bytes(hd_gemm_runtime *rt);

/* gemm.h:48 - simple one-output-per-thread fp32 kernel; correctness/debug
 * backend. y[M,N] = x[M,K] . w[N,K]^T (+bias), bf16 out. */
void hd_linear_reference(const void *x_dev, const void *w_dev,
                         const void *bias_dev, void *y_dev,
                         int M, int N, int K, int transpose_w);

/* gemm.h:57 - production linear on the MFMA kernels (reference backend when
 * hd_gemm_set_backend(0)). Only transpose_w == 1 ([out,in] weights). Bias is
 * added in the epilogue with the production reference's two roundings,
 * y = bf16(bf16(acc) + bias): the reference writes the bf16 GEMM result and
 * then adds the bias in a second kernel (gemm.cu:226-235, :317-320). */
void hd_linear(const void *x_dev, const void *w_dev, const void *bias_dev,
               void *y_dev, int M, int N, int K, int transpose_w);

/* gemm.h:61 - 1 = production (MFMA, default), 0 = reference kernel. */
void hd_gemm_set_backend(int use_production);
/* gemm.h:67 - accepted for source compatibility; there is one production
 * kernel family, so the value is ignored. */
void hd_gemm_set_prod_backend(int backend);

/* Extension: hd_linear (transpose_w = 1) writing rows of stride ldc >= N
 * (ldc % 8 == 0); columns [N, ldc) are left untouched. */
void hd_linear_ld(const void *x_dev, const void *w_dev, const void *bias_dev, void *y_dev, int M,
                  int N, int K, int ldc);

/* Extension: hd_linear / hd_linear_residual with a device workspace for the
 * tail split: when the tiles leave a last round of resident blocks at most
 * half full, those tiles run as 2-8 K chunks writing fp32 partial tiles into
 * ws and a merge kernel sums them (chunk order) and applies the epilogue.
 * Results agree with the unsplit GEMM to the fp32 reassociation of the K
 * sum (then one bf16 rounding). ws 16-byte aligned; ws == NULL or too small
 * runs the unsplit GEMM. Launches on one stream must not share ws
 * concurrently. */
void hd_linear_ws(const void *x_dev, const void *w_dev, const void *bias_dev, void *y_dev, int M,
                  int N, int K, void *ws, int64_t ws_bytes);
void hd_linear_residual_ws(const void *x_dev, const void *w_dev, const void *res_dev, void *y_dev,
                           int M, int N, int K, void *ws, int64_t ws_bytes);
/* Workspace bytes that let every tail split of the current device run. */
int64_t hd_gemm_ws_bytes(void);

/* hd_linear_noalloc: no counterpart in the reference. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): hd_linear_ws with the tail-split
 * workspace in a static device array of hd_linear_noalloc_scratch_bytes()
 * (80 MiB, one copy per GPU, held until the process ends) instead of a
 * workspace argument. Allocates nothing. Errors (hd_cuda_last_error) when
 * the current device's tail split needs more than the array holds. Calls
 * that overlap on one GPU share the array and race. */
void hd_linear_noalloc(const void *x_dev, const void *w_dev, const void *bias_dev, void *y_dev,
                       int M, int N, int K);
int64_t hd_linear_noalloc_scratch_bytes(void);

/* ---- fused-epilogue entry points (extension) --------------------------
 * y = bf16(res + bf16(x . W^T))      : residual epilogue (o_proj, down)   */
void hd_linear_residual(const void *x_dev, const void *w_dev,
                        const void *res_dev, void *y_dev, int M, int N, int K);

/* y[M,F] = bf16(bf16(silu(bf16(x.Wg^T))) * bf16(x.Wu^T)) : gate/up GEMM
 * with the SwiGLU epilogue; the gate and up products never reach HBM. */
void hd_linear_swiglu(const void *x_dev, const void *wg_dev,
                      const void *wu_dev, void *y_dev, int M, int F, int K);
/* Extension: hd_linear_swiglu with the tail-split workspace of
 * hd_linear_residual_ws. */
void hd_linear_swiglu_ws(const void *x_dev, const void *wg_dev, const void *wu_dev, void *y_dev,
                         int M, int F, int K, void *ws, int64_t ws_bytes);

/* y[M, N0+N1+N2] = x . [W0;W1;W2]^T with three separately stored weight
 * matrices (the q/k/v projections) computed as one GEMM; every Ni must be
 * a multiple of 256. w1/w2 may be NULL (then N1/N2 must be 0). */
void hd_linear_concat3(const void *x_dev, const void *w0, int N0,
                       const void *w1, int N1, const void *w2, int N2,
                       void *y_dev, int M, int K);

/* Extension (diagnostic, no counterpart in the reference): matrix-core
 * ceiling probe. `blocks` blocks of 8 waves each run 8 independent
 * v_mfma_f32_32x32x16_bf16 chains (shape 32) or 16 v_mfma_f32_16x16x32_bf16
 * chains (shape 16) for `iters` rounds of 32x32x16-equivalent work (a
 * multiple of 4) over bf16 operands read once from `ops` (n_ops elements,
 * >= 16400); `out` receives blocks * 512 checksums. Returns the FLOP count
 * of the launch (0 on bad arguments). */
double hd_mfma_probe(const void *ops, int n_ops, int blocks, int iters, int shape, float *out);

/* Name of the kernel configuration hd_linear* would launch for a shape
 * (diagnostics; static string). */
const char *hd_gemm_config_name(int M, int N, int K, int epilogue);

/* Extension: the block's QKV projection with the per-head q/k RMSNorm and
 * rotary (hd_qkv_epilogue semantics, bit-identical) fused into the GEMM
 * epilogue: x [batch*seq, hidden] against wq/wk/wv, writing q [B,H,S,128],
 * k [B,KV,S,128] and the flash V^T layout vt [B,KV,128,S]. cs: rotary table
 * [seq, 64] (cos, sin). Returns 0 when launched, 1 (nothing done) when the
 * shape is outside the fused path: seq % 64 != 0, head counts not even,
 * hidden > 8192 or not a multiple of 64, operands of 2 GiB or more, a
 * pointer (x, norm weights, cs, q, k, vt) not 16-byte aligned. */
int hd_linear_qkv_rope(const void *x, const void *wq, const void *wk, const void *wv,
                       const void *qn_w, const void *kn_w, const float *cs, void *q, void *k,
                       void *vt, int batch, int seq, int heads, int kv_heads, int hidden,
                       float eps);
/* Extension: hd_linear_qkv_rope with the tail-split workspace of
 * hd_linear_residual_ws (the tail tiles' epilogue runs in the merge). */
int hd_linear_qkv_rope_ws(const void *x, const void *wq, const void *wk, const void *wv,
                          const void *qn_w, const void *kn_w, const float *cs, void *q, void *k,
                          void *vt, int batch, int seq, int heads, int kv_heads, int hidden,
                          float eps, void *ws, int64_t ws_bytes);

#ifdef __cplusplus
}
#endif

#endif /* HD_GEMM_HIP_H */
