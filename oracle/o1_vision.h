/*
 * CPU oracle of the Qwen3-VL vision tower (TEST INFRASTRUCTURE ONLY).
 * Restates src/model/vision.c and src/cuda/vision_kernels.cu of the
 * reference with generic dimensions; see o1_vision.c.
 */
#ifndef O1_VISION_H
#define O1_VISION_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif
typedef struct {
    const float *norm1_w, *norm1_b, *norm2_w, *norm2_b, *qkv_w, *qkv_b, *proj_w, *proj_b, *fc1_w,
        *fc1_b, *fc2_w, *fc2_b;
} o1o_vision_block;            /* vision.h hd_vision_block_binding */
typedef struct {
    const float *norm_w, *norm_b, *fc1_w, *fc1_b, *fc2_w, *fc2_b;
} o1o_vision_merger;           /* vision.h hd_vision_merger_binding */
typedef struct {
    const float *patch_w, *patch_b, *pos_embed;
    const o1o_vision_block *blocks;
    o1o_vision_merger merger;
    o1o_vision_merger deepstack[4];
} o1o_vision_weights;
typedef struct {
    int depth, hidden, heads, inter, out_hidden, patch_dim, nside, merge;
    int n_ds, ds_layers[4];
    int faithful;
} o1o_vision_cfg;
void o1o_layernorm(const float *x, const float *w, const float *b, float *y, int rows, int cols,
                   float eps, int round);
void o1o_gelu_tanh(const float *x, float *y, size_t n, int round);
void o1o_gelu_erf(const float *x, float *y, size_t n, int round);
void o1o_vision_tables(int grid_h, int grid_w, int nside, int merge, int *idx, float *wgt,
                       int *coords);
void o1o_vision_rotary(const int *coords, int n, int head_dim, int faithful, float *cosd,
                       float *sind);
int o1o_vision_forward(const o1o_vision_weights *w, const o1o_vision_cfg *c, const float *pixels,
                       int grid_h, int grid_w, float *embeds, float **deepstack,
                       float *after_blocks);
#ifdef __cplusplus
}
#endif
#endif
