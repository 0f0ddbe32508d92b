#ifndef HD_FORWARD_HIP_H
#define HD_FORWARD_HIP_H

/*
 * The whole denoiser for one step: t-embedder, token embedding with the
 * timestep-token substitution, x_embedder, n_layers decoder blocks, final
 * RMSNorm and the output head.
 *
 * Replaces the reference's src/model/forward.h (lines 40-181): same
 * binding/workspace/diagnostics structs and entry points. Differences that
 * a caller can observe are only extensions: the stream argument is honoured
 * (the reference ignores it, forward.c:205), mask_dev may be NULL for full
 * attention, and hd_forward_batched runs B equal-length sequences.
 */

#include <stdint.h>

#include "hidream_hip.h"
#include "hd_sdpa.h"
#include "hd_weights.h"
#include "hd_block.h"

#ifdef __cplusplus
extern "C" {
#endif

/* forward.h:40-59 */
typedef struct {
    const void *embed_tokens;   /* [vocab, H]     */
    const void *te0_w;          /* [H, 256]       */
    const void *te0_b;          /* [H]            */
    const void *te2_w;          /* [H, H]         */
    const void *te2_b;          /* [H]            */
    const void *xe1_w;          /* [1024, 3072]   */
    const void *xe2_w;          /* [H, 1024]      */
    const void *xe2_b;          /* [H]            */
    const void *fl_w;           /* [3072, H]      */
    const void *fl_b;           /* [3072]         */
    const void *fnorm_w;        /* [H]            */
    int n_layers;
    hd_block_binding *blocks;   /* [n_layers], owned by the binding */
} hd_forward_binding;

/* forward.h:66-93. `hidden_a` is the base of one caller-allocated arena of
 * hd_forward_workspace_bytes(); the other pointers are informational. */
typedef struct {
    void *hidden_a;
    void *hidden_b;
    void *h_text;
    void *norm_out;
    void *head_out;
    void *t_emb;
    void *te_hidden;
    void *freq;
    void *freq_bf16;
    void *t_scaled;
    void *xe_stage;
    void *xe_out;
    void *xe_ref;         /* optional cached x_embedder rows of references */
    int n_ref;
    void *block_scratch;
    int64_t block_scratch_bytes;
    hd_sdpa_plan *sdpa;
} hd_forward_workspace;

/* forward.h:96-107 */
typedef struct {
    void *after_embedding;
    void *after_timestep_conditioning;
    void *after_target_embedding;
    void *after_block_0_input;
    void *after_block_0;
    void *after_block_mid;
    void *after_block_last;
    void *before_final_norm;
    void *after_final_norm;
    void *after_final_head;
} hd_forward_diagnostics;

/* forward.h:127-134: vision conditioning for hd_forward (batch 1). Device
 * pointers, bf16: image_embeds [v_tokens, hidden] replace the rows whose
 * visual_mask [S] byte is set, in order (text rows only); deepstack[i]
 * [v_tokens, hidden] is added to those rows of block i's output, i < 3
 * (a NULL deepstack[i] skips that layer). */
typedef struct {
    const void *image_embeds;
    const void *deepstack[3];
    const uint8_t *visual_mask;
    int v_tokens;
} hd_visual_cond;

/* forward.h:122 */
hd_status hd_forward_resolve(const hd_weight_store *wstore, int n_layers,
                             hd_forward_binding *out);
void hd_forward_binding_free(hd_forward_binding *b);

/* forward.h:131. Batch 1. */
int64_t hd_forward_workspace_bytes(int64_t seq, int img_tokens, int heads,
                                   int kv_heads, int hidden, int ff_hidden,
                                   int head_dim, int64_t *block_scratch_bytes);

/* forward.h:156. sec_dev: the MRoPE section, int64[3] in device memory, read
 * by the rotary-table kernel (NULL: the block config's section). */
hd_status hd_forward(const hd_forward_binding *bw, hd_forward_workspace *ws,
                     const int64_t *input_ids, int text_len,
                     const float *pos_f32, const void *mask_dev,
                     const void *vinputs, int img_tokens,
                     const hd_visual_cond *visual, const float *timestep,
                     const int64_t *sec_dev, int seq, int heads, int kv_heads,
                     int hidden, int ff_hidden, int head_dim, int tms_token_id,
                     hd_forward_diagnostics *diag, void *out_dev, void *stream);

/* forward.h:171 */
int hd_forward_num_layers(const hd_forward_binding *bw);

/* forward.h:179 - byte offset of a named region inside the workspace. */
int64_t hd_forward_ws_offset(const char *name, int64_t seq, int text_len,
                             int img_tokens, int heads, int kv_heads,
                             int hidden, int ff_hidden, int head_dim,
                             int64_t *block_scratch_bytes);

/* ---- extension: B sequences of equal length per launch chain ----------
 * input_ids [B, text_len] int64, vinputs [B, img_tokens, 3072] bf16,
 * timestep [B] fp32, pos_f32 [3, seq] shared by the batch, out
 * [B, seq, 3072] bf16. ar_len: causal text prefix (0 = full attention).
 * n_ref > 0 with ws->xe_ref set reuses cached x_embedder rows for the last
 * n_ref image tokens of every sequence (edit mode, forward.c:301-313). */
int64_t hd_forward_batched_workspace_bytes(int batch, int64_t seq,
                                           int img_tokens, int heads,
                                           int kv_heads, int hidden,
                                           int ff_hidden, int head_dim);
hd_status hd_forward_batched(const hd_forward_binding *bw,
                             hd_forward_workspace *ws, int batch,
                             const int64_t *input_ids, int text_len,
                             const float *pos_f32, int ar_len,
                             const void *vinputs, int img_tokens,
                             const float *timestep, int seq, int heads,
                             int kv_heads, int hidden, int ff_hidden,
                             int head_dim, int tms_token_id,
                             hd_forward_diagnostics *diag, void *out_dev,
                             void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HD_FORWARD_HIP_H */
