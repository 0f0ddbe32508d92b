#ifndef HD_SDPA_HIP_H
#define HD_SDPA_HIP_H

/*
 * Scaled-dot-product attention on a hand-written flash kernel for gfx950.
 *
 * Replaces the reference's cuDNN-frontend backend (include/hd_cudnn_sdpa.h
 * lines 37-94; src/cuda/hd_cudnn_sdpa.cu). Same plan object life cycle and
 * the same layout contract:
 *   q   [B, Hq,  S, D] bf16      k, v [B, Hkv, S, D] bf16
 *   out [B, Hq,  S, D] bf16      mask [1, 1, S, S] bf16 additive (optional)
 * GQA maps query head h to kv head h / (Hq / Hkv). Softmax is fp32, the
 * probabilities are rounded to bf16 before the P.V product (as the fused
 * cuDNN kernel does), the running max/sum are kept in fp32.
 *
 * A split plan (0 < ar_len < S) computes exactly what the reference's two
 * passes compute (hd_cudnn_sdpa.cu:307-441): rows < ar_len are causal over
 * keys [0, row], rows >= ar_len see every key; it does so in ONE launch
 * with no staging copies, and ignores the mask argument like the reference.
 *
 * Return values: 0 on success, non-zero with hd_cuda_last_error() set.
 */

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hd_sdpa_plan hd_sdpa_plan;

/* hd_cudnn_sdpa.h:42 */
int hd_sdpa_create(hd_sdpa_plan **out, int batch, int q_heads, int kv_heads,
                   int seq_q, int seq_kv, int head_dim, float scale);
/* hd_cudnn_sdpa.h:51. `stream` is a hipStream_t (NULL = library stream). */
int hd_sdpa_execute(hd_sdpa_plan *plan, const void *q, const void *k,
                    const void *v, const void *mask, void *out, void *stream);
/* hd_cudnn_sdpa.h:57 */
void hd_sdpa_destroy(hd_sdpa_plan *plan);
/* hd_cudnn_sdpa.h:71 */
int hd_sdpa_create_split(hd_sdpa_plan **out, int batch, int q_heads,
                         int kv_heads, int seq, int ar_len, int head_dim,
                         float scale);
/* hd_cudnn_sdpa.h:78 */
int hd_sdpa_execute_split(hd_sdpa_plan *plan, const void *q, const void *k,
                          const void *v, void *out, void *stream);
/* hd_cudnn_sdpa.h:83. which = 0: causal head rows [0, ar_len) only, into
 * the plan's staging buffer (`out` is left untouched, as the reference's
 * pass 0 writes only its staged head); which = 1: every row of `out` with
 * full (non-causal) attention. */
int hd_sdpa_execute_split_pass(hd_sdpa_plan *plan, int which, const void *q,
                               const void *k, const void *v, void *out,
                               void *stream);
/* Extension: the staging buffer pass 0 of a split plan writes, seq-major
 * [batch, ar_len, q_heads, head_dim] bf16 (NULL for a non-split plan). */
const void *hd_sdpa_plan_stage(const hd_sdpa_plan *plan);
/* hd_cudnn_sdpa.h:94 */
int hd_sdpa_create_prod(hd_sdpa_plan **out, int batch, int q_heads,
                        int kv_heads, int seq, int ar_len, int head_dim,
                        float scale);

/* ---- extension: the kernel entry the decoder block uses ----------------
 * q  [B,Hq,S,D] head-major, k [B,Hkv,S,D], vt [B,Hkv,D,S] (V transposed),
 * out written SEQ-major [B,S,Hq*D] so the o_proj GEMM reads it directly
 * (no head_merge). mask: optional [S,S] bf16 additive bias; ar_len as in a
 * split plan. D must be 128. */
int hd_flash_attention(const void *q, const void *k, const void *vt,
                       const void *mask, void *out, int batch, int q_heads,
                       int kv_heads, int seq, int head_dim, int ar_len,
                       float scale, int out_seq_major);

/* Causal prefix length of a plan (0 for a non-split plan or NULL). */
/* Extension: hd_flash_attention with a workspace for the tail split. When the
 * (batch x heads x 128-query tiles) units leave a last, partly filled round
 * of resident blocks, those units run as 2-8 key-range chunks writing fp32
 * partials (running max, sum, unnormalised O) into ws, and a merge kernel
 * combines them; full attention only (no mask, ar_len == 0), otherwise and
 * when ws_bytes < hd_flash_ws_bytes() it behaves as hd_flash_attention.
 * Results agree with the unsplit kernel to fp32 rounding of the merge. */
int hd_flash_attention_ws(const void *q, const void *k, const void *vt, const void *mask,
                          void *out, int batch, int q_heads, int kv_heads, int seq, int head_dim,
                          int ar_len, float scale, int out_seq_major, void *ws, int64_t ws_bytes);
/* Workspace bytes for the tail split on the current device (one round of
 * resident flash blocks x 128 rows x (128 + 2) floats). */
int64_t hd_flash_ws_bytes(void);

int hd_sdpa_plan_ar_len(const hd_sdpa_plan *plan);

/* Bytes of the flash kernel's V^T layout [B,Hkv,128,round_up(S,64)]. */
int64_t hd_flash_vt_bytes(int batch, int kv_heads, int seq);
/* Head-major V [bh, S, 128] -> V^T layout (key columns with bits 2 and 3
 * exchanged, zero padding). */
void hd_flash_make_vt(const void *v, void *vt, int bh, int seq);

#ifdef __cplusplus
}
#endif

#endif /* HD_SDPA_HIP_H */
