#ifndef HD_VISION_HIP_H
#define HD_VISION_HIP_H

/*
 * Qwen3-VL vision tower (reference image conditioning) on MI355X.
 *
 * Replaces src/model/vision.h:1-221 and src/cuda/vision_kernels.h of the
 * reference: same constants, binding/workspace structs (field for field) and
 * entry points, so a caller of the reference compiles unchanged.
 *
 *   pixel_values [n, 1536] bf16 (patchified, processor layout)
 *     -> patch embed GEMM + interpolated position embedding  [n, 1152]
 *     -> 27 blocks: LayerNorm, qkv, 2-D rotary, full attention (the flash
 *        kernel at head_dim 128 over zero-padded heads), proj, LayerNorm,
 *        fc1, GELU(tanh), fc2                                  [n, 1152]
 *     -> merger: LayerNorm(1152), 4-row view, fc1, GELU(erf), fc2 -> [m, 4096]
 *     -> deepstack mergers after blocks 8/16/24 (LayerNorm over 4608)
 *
 * Tokens are in the merge-block order (bh, bw, mh, mw), so the 2x2 spatial
 * merge is a view of 4 consecutive rows.
 */

#include <stdint.h>

#include "hd_sdpa.h"
#include "hd_weights.h"
#include "hidream_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define HD_VISION_DEPTH        27
#define HD_VISION_HIDDEN       1152
#define HD_VISION_HEADS        16
#define HD_VISION_HEAD_DIM     72
#define HD_VISION_INTERMEDIATE 4304
#define HD_VISION_OUT_HIDDEN   4096
#define HD_VISION_MERGE_SIZE   2
#define HD_VISION_PATCH_SIZE   16
#define HD_VISION_TEMPORAL_PATCH 2
#define HD_VISION_PATCH_DIM    1536
#define HD_VISION_NUM_POS      2304
#define HD_VISION_NUM_DS       3
#define HD_VISION_DS_LAYERS    {8, 16, 24}

/* vision.h:51-69: block-0 snapshot slots. This build captures HD_B0_INPUT,
 * HD_B0_NORM1, HD_B0_QKV, HD_B0_ATTN_MERGED, HD_B0_PROJ, HD_B0_ATTN_RESID,
 * HD_B0_NORM2, HD_B0_FC2 and HD_B0_OUTPUT; the head-major q/k/v slots hold
 * the zero-padded [16, n, 128] layout the flash kernel reads, and HD_B0_FC1
 * the GELU input at a 4352-column row stride. */
enum {
    HD_B0_INPUT = 0,
    HD_B0_NORM1,
    HD_B0_QKV,
    HD_B0_Q,
    HD_B0_K,
    HD_B0_V,
    HD_B0_Q_ROT,
    HD_B0_K_ROT,
    HD_B0_ATTN_HEADS,
    HD_B0_ATTN_MERGED,
    HD_B0_PROJ,
    HD_B0_ATTN_RESID,
    HD_B0_NORM2,
    HD_B0_FC1,
    HD_B0_FC2,
    HD_B0_OUTPUT,
    HD_B0_SNAP_COUNT
};

typedef struct {              /* vision.h:72-85 */
    const void *norm1_w, *norm1_b, *norm2_w, *norm2_b;
    const void *qkv_w, *qkv_b, *proj_w, *proj_b;
    const void *fc1_w, *fc1_b, *fc2_w, *fc2_b;
} hd_vision_block_binding;

typedef struct {              /* vision.h:88-95 */
    const void *norm_w, *norm_b, *fc1_w, *fc1_b, *fc2_w, *fc2_b;
} hd_vision_merger_binding;

typedef struct {              /* vision.h:98-105 */
    const void *patch_proj_w;  /* [1152, 1536] */
    const void *patch_proj_b;
    const void *pos_embed;     /* [2304, 1152] */
    hd_vision_block_binding blocks[HD_VISION_DEPTH];
    hd_vision_merger_binding merger;
    hd_vision_merger_binding deepstack[HD_VISION_NUM_DS];
} hd_vision_binding;

/* vision.h:112-176, same fields. The forward carves its buffers from
 * `patch_out` (the base of hd_vision_workspace_bytes(n) bytes); the other
 * buffer pointers are not read. `sdpa` is not used (attention runs on the
 * flash kernel directly). `tables` points at hd_vision_tables_bytes(n)
 * bytes, filled by hd_vision_prepare_tables. */
typedef struct {
    void *patch_out, *pos_emb, *rot, *cosf, *sinf, *h_a, *h_b, *ln1, *qkv, *q, *k, *v, *qr, *kr,
        *scores, *probs, *attn_out, *attn_resid, *ln2, *fc1, *fc2, *mlp_resid, *merged,
        *merge_norm, *merge_fc1, *merge_fc2, *ds_merged, *ds_fc1, *ds_fc2;
    void *pos_idx, *pos_wgt, *rot_coords, *rot_inv;
    void *tables;
    int tables_n;
    int tables_gh, tables_gw;
    int64_t bytes;
    hd_sdpa_plan *sdpa;
    void *block0_snap;
    void *block0_snaps[HD_B0_SNAP_COUNT];
    void *block_out_snaps[HD_VISION_DEPTH];
    void *merger_snaps[5];
    void *ds_merger_snaps[HD_VISION_NUM_DS][4];
} hd_vision_workspace;

/* vision.h:180-186, same fields. Offsets of this build's regions (bytes
 * from the workspace base); fields of buffers this build does not keep have
 * size zero:
 *   patch_out  [n,1152]  patch embedding, later the proj / fc2 outputs
 *   h_a        [n,1152]  residual stream (block input / output)
 *   attn_resid [n,1152]  residual after attention
 *   ln1        [n,1152]  LayerNorm output, later the merged attention rows
 *   qkv        [n,3456]  qkv projection, later the flash output [n,16*128]
 *   q, k, v    [16,n+128,128] zero-padded head-major operands
 *   scores     [16,128,round_up(n,64)] V^T for the flash kernel
 *   fc1        [n,4352]  fc1 / GELU rows (zero columns 4304..4351)
 *   fc2        [1152,4352] the current block's fc2 weight, zero-padded
 *   cosf, sinf [n,72]    fp32 rotary tables */
typedef struct {
    int64_t patch_out, pos_emb, rot, h_a, h_b, ln1, attn_resid, ln2, fc2, mlp_resid, q, k, v, qr,
        kr, qkv, scores, probs, mask, attn_out, fc1, cosf, sinf, merged, merge_norm, merge_fc1,
        merge_fc2, ds_merged, ds_fc1, ds_fc2, total_bytes;
} hd_vision_offsets;

void hd_vision_layout(int64_t n, int64_t m, hd_vision_offsets *o);              /* vision.h:182 */
hd_status hd_vision_resolve(const hd_weight_store *wstore, hd_vision_binding *out); /* :188 */
int64_t hd_vision_workspace_bytes(int64_t n);                                    /* :192 */
int64_t hd_vision_tables_bytes(int64_t n);                                       /* :200 */
/* vision.c:288-343: builds the position-interpolation taps and rotary
 * coordinates for (n, grid_h, grid_w) into ws->tables (host build, one
 * synchronous upload); a repeated shape returns at once. */
hd_status hd_vision_prepare_tables(hd_vision_workspace *ws, int n, int grid_h, int grid_w);
/* vision.h:216: batch 1, one image (grid_t = 1), n = grid_h * grid_w,
 * grid_h and grid_w even. image_embeds_out [n/4, 4096] bf16; deepstack_out
 * (may be NULL) three [n/4, 4096] bf16 buffers. Device-resident, no
 * allocation, no synchronisation; runs on the library stream. */
hd_status hd_vision_forward(const hd_vision_binding *bw, hd_vision_workspace *ws,
                            const void *pixel_values, int n, int grid_h, int grid_w,
                            void *image_embeds_out, void *deepstack_out[HD_VISION_NUM_DS]);

/* Extension: `images` reference images of the same grid in one call
 * (pixel_values [images*n, 1536], image_embeds_out [images*n/4, 4096] and
 * each deepstack_out [images*n/4, 4096], images in order: the row layout
 * hd_visual_cond takes for several references). GEMMs and elementwise
 * kernels run over all rows at once, attention per image; each image's
 * rows equal what hd_vision_forward computes for it alone. The workspace
 * is hd_vision_workspace_bytes_multi(images, n) bytes; the tables are the
 * single-image ones for (n, grid_h, grid_w). */
hd_status hd_vision_forward_multi(const hd_vision_binding *bw, hd_vision_workspace *ws,
                                  const void *pixel_values, int images, int n, int grid_h,
                                  int grid_w, void *image_embeds_out,
                                  void *deepstack_out[HD_VISION_NUM_DS]);
int64_t hd_vision_workspace_bytes_multi(int images, int64_t n);

/* ---- kernels (src/cuda/vision_kernels.h) ------------------------------ */
/* patch embed as GEMM + bias: y [n, out_dim] = x [n, in_dim] . w^T + b */
void hd_vision_patch(const void *x, const void *w, const void *bias, void *y, int n, int in_dim,
                     int out_dim);
/* LayerNorm over the last dim, fp32 statistics (mean, E[x^2] - mean^2) */
void hd_vision_layernorm(const void *x, const void *w, const void *b, void *y, int rows, int cols,
                         float eps);
void hd_vision_gelu(const void *x, void *y, size_t n);        /* tanh form */
void hd_vision_gelu_exact(const void *x, void *y, size_t n);  /* erf form */
void hd_vision_pos_interp(const void *pos_embed, const int *idx, const float *wgt, void *y, int n,
                          int hidden);
/* angles [n, 2*half] bf16: inv_freq[k] * row | inv_freq[k] * col */
void hd_vision_rot(const float *inv_freq, const int *coords, void *y, int n, int half);
/* cos / sin [n, 4*half] fp32 of the angles repeated twice */
void hd_vision_rot_cos_sin(const void *rot, float *cosd, float *sind, int n, int half);
/* [gh*gw, hidden] row-major grid -> [gh/2*gw/2, 4*hidden] 2x2 blocks */
void hd_vision_spatial_merge(const void *in, void *out, int gh, int gw, int hidden);
/* qkv [n, 3*heads*d] -> q, k, v [heads, n, d] */
void hd_vision_qkv_split(const void *qkv, void *q, void *k, void *v, int n, int heads, int d);
/* [heads, n, d] -> [n, heads*d] */
void hd_vision_attn_merge(const void *hm, void *sm, int heads, int n, int d);
/* out[row] = mask[row] ? src[#set rows before row] : dst[row], rows [0, rows) */
void hd_vision_masked_scatter(const void *dst, const uint8_t *mask, const void *src, void *out,
                              int rows, int cols);
/* out[row] = mask[row] ? bf16(in[row] + emb[#set rows before row]) : in[row] */
void hd_vision_deepstack_inject(const void *in, const uint8_t *mask, const void *emb, void *out,
                                int rows, int cols);

/* Extension: the two kernels above bounded by the number of embedding rows
 * (hd_visual_cond.v_tokens): set mask rows past `src_rows` are left as they
 * are instead of reading past the embeddings. Used by hd_forward. */
void hd_vision_masked_scatter_n(const void *dst, const uint8_t *mask, const void *src, void *out,
                                int rows, int cols, int src_rows);
void hd_vision_deepstack_inject_n(const void *in, const uint8_t *mask, const void *emb, void *out,
                                  int rows, int cols, int emb_rows);

#ifdef __cplusplus
}
#endif

#endif /* HD_VISION_HIP_H */
