/*
 * CPU oracle of the Qwen3-VL vision tower. TEST INFRASTRUCTURE ONLY (same
 * rules as o1_oracle.c: tests/, smoke() and the CPU baseline may call it;
 * the product library never does).
 *
 * fp32 restatement of src/model/vision.c:345-640 and the kernels of
 * src/cuda/vision_kernels.cu, with generic dimensions so that a tiny
 * configuration can be checked against transformers' Qwen3VLVisionModel
 * (the model vision.c:1-21 states it reproduces). `faithful` = 1 rounds to
 * bf16 where the reference holds bf16 buffers; 0 keeps fp32 throughout (and
 * the rotary angles unrounded), which is what the transformers pin uses.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "o1_oracle.h"
#include "o1_vision.h"

static inline float rnd(float v, int r) { return r ? o1o_bf16_round(v) : v; }

/* vision_kernels.cu:50-87: mean and E[x^2] - mean^2 in fp32, rsqrt(var + eps),
 * (x - mean) * inv * w + b. */
void o1o_layernorm(const float *x, const float *w, const float *b, float *y, int rows, int cols,
                   float eps, int round) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * cols;
        double s = 0.0, s2 = 0.0;
        for (int i = 0; i < cols; i++) {
            s += xr[i];
            s2 += (double)xr[i] * xr[i];
        }
        const float mean = (float)(s / cols);
        float var = (float)(s2 / cols) - mean * mean;
        if (var < 0.f) var = 0.f;
        const float inv = 1.0f / sqrtf(var + eps);
        float *yr = y + (size_t)r * cols;
        for (int i = 0; i < cols; i++)
            yr[i] = rnd((xr[i] - mean) * inv * w[i] + (b ? b[i] : 0.f), round);
    }
}

/* vision_kernels.cu:101-110 (gelu_pytorch_tanh) */
void o1o_gelu_tanh(const float *x, float *y, size_t n, int round) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        const float v = x[i];
        const float g = 0.7978845608028654f * (v + 0.044715f * v * v * v);
        y[i] = rnd(0.5f * v * (1.0f + tanhf(g)), round);
    }
}

/* vision_kernels.cu:125-133 (nn.GELU(), erf form) */
void o1o_gelu_erf(const float *x, float *y, size_t n, int round) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        const float v = x[i];
        y[i] = rnd(0.5f * v * (1.0f + erff(v * 0.7071067811865476f)), round);
    }
}

/* vision.c:215-285: four-corner bilinear taps of the position-embedding grid
 * (nside x nside) and the (row, col) rotary coordinates, both in the
 * block-major token order (bh, bw, mh, mw) of the merge. idx/wgt [4, n],
 * coords [2, n]; n = grid_h * grid_w. */
void o1o_vision_tables(int grid_h, int grid_w, int nside, int merge, int *idx, float *wgt,
                       int *coords) {
    const int n = grid_h * grid_w;
    int row = 0;
    for (int bh = 0; bh < grid_h / merge; bh++)
        for (int bw = 0; bw < grid_w / merge; bw++)
            for (int ih = 0; ih < merge; ih++)
                for (int iw = 0; iw < merge; iw++, row++) {
                    const int h = bh * merge + ih, w = bw * merge + iw;
                    const float hf = grid_h > 1 ? (float)h * (float)(nside - 1) / (float)(grid_h - 1) : 0.f;
                    const float wf = grid_w > 1 ? (float)w * (float)(nside - 1) / (float)(grid_w - 1) : 0.f;
                    const int h0 = (int)hf, w0 = (int)wf;
                    const int h1 = h0 + 1 < nside ? h0 + 1 : nside - 1;
                    const int w1 = w0 + 1 < nside ? w0 + 1 : nside - 1;
                    const float dh = hf - (float)h0, dw = wf - (float)w0;
                    idx[row] = h0 * nside + w0;
                    idx[n + row] = h0 * nside + w1;
                    idx[2 * n + row] = h1 * nside + w0;
                    idx[3 * n + row] = h1 * nside + w1;
                    wgt[row] = (1.f - dh) * (1.f - dw);
                    wgt[n + row] = (1.f - dh) * dw;
                    wgt[2 * n + row] = dh * (1.f - dw);
                    wgt[3 * n + row] = dh * dw;
                    coords[row] = h;
                    coords[n + row] = w;
                }
}

/* vision.c:415-420 + vision_kernels.cu:183-231: angle[k] = inv_freq[k] * row
 * (k < D/4) and inv_freq[k] * col, inv_freq[k] = 10000^(-2k/(D/2)); the
 * reference stores the angles as bf16 (faithful), cos/sin [n, D] repeat the
 * D/2 angles twice. */
void o1o_vision_rotary(const int *coords, int n, int head_dim, int faithful, float *cosd,
                       float *sind) {
    const int quarter = head_dim / 4, half = head_dim / 2;
    for (int s = 0; s < n; s++)
        for (int k = 0; k < half; k++) {
            const int j = k % quarter;
            const float inv = 1.0f / powf(10000.0f, (float)(2 * j) / (float)half);
            const float a = rnd(inv * (float)(k < quarter ? coords[s] : coords[n + s]), faithful);
            const float c = cosf(a), sn = sinf(a);
            cosd[(size_t)s * head_dim + k] = cosd[(size_t)s * head_dim + half + k] = c;
            sind[(size_t)s * head_dim + k] = sind[(size_t)s * head_dim + half + k] = sn;
        }
}

/* rope.cu:157-180: q*cos + rotate_half(q)*sin in fp32, one rounding;
 * x, y [heads, n, D] (not in place) */
static void rotary(const float *x, const float *cs, const float *sn, float *y, int heads, int n,
                   int D, int round) {
    const int half = D / 2;
#pragma omp parallel for schedule(static)
    for (long hs = 0; hs < (long)heads * n; hs++) {
        const int s = (int)(hs % n);
        const float *xr = x + (size_t)hs * D;
        float *yr = y + (size_t)hs * D;
        for (int d = 0; d < D; d++) {
            const float c = cs[(size_t)s * D + d], sv = sn[(size_t)s * D + d];
            const float v = d < half ? xr[d] * c - xr[d + half] * sv : xr[d] * c + xr[d - half] * sv;
            yr[d] = rnd(v, round);
        }
    }
}

/* Qwen3VLVisionPatchMerger as vision.c:558-580 (final, norm over hidden
 * before the 4-row view) and :493-527 (deepstack, norm over merge^2*hidden
 * after it): x [n, hidden] -> out [n / merge^2, out_hidden]. */
static void merger(const float *x, const o1o_vision_merger *mw, const o1o_vision_cfg *c,
                   int postshuffle, int n, float *out) {
    const int R = c->faithful, lm = c->faithful ? 2 : 0;
    const int U = c->merge * c->merge, m = n / U, W = c->hidden * U;
    float *nrm = (float *)malloc(sizeof(float) * (size_t)n * c->hidden);
    float *f1 = (float *)malloc(sizeof(float) * (size_t)m * W);
    if (postshuffle) o1o_layernorm(x, mw->norm_w, mw->norm_b, nrm, m, W, 1e-6f, R);
    else o1o_layernorm(x, mw->norm_w, mw->norm_b, nrm, n, c->hidden, 1e-6f, R);
    o1o_linear(nrm, mw->fc1_w, mw->fc1_b, f1, m, W, W, lm);
    o1o_gelu_erf(f1, f1, (size_t)m * W, R);
    o1o_linear(f1, mw->fc2_w, mw->fc2_b, out, m, c->out_hidden, W, lm);
    free(nrm);
    free(f1);
}

/* vision.c:345-640 for one image of grid_h x grid_w patches:
 * pixels [n, patch_dim] -> embeds [n/merge^2, out_hidden] and, when
 * deepstack != NULL, deepstack[j] [n/merge^2, out_hidden] after block
 * ds_layers[j]; after_blocks (optional) [depth][n, hidden] block outputs. */
int o1o_vision_forward(const o1o_vision_weights *w, const o1o_vision_cfg *c, const float *pixels,
                       int grid_h, int grid_w, float *embeds, float **deepstack,
                       float *after_blocks) {
    if (grid_h % c->merge || grid_w % c->merge || c->hidden % c->heads) return 1;
    const int n = grid_h * grid_w, H = c->hidden, NH = c->heads, D = H / NH, I = c->inter;
    const int R = c->faithful, lm = c->faithful ? 2 : 0;
    const size_t nH = (size_t)n * H;
    float *h = (float *)malloc(sizeof(float) * nH), *tmp = (float *)malloc(sizeof(float) * nH);
    float *ln = (float *)malloc(sizeof(float) * nH), *att = (float *)malloc(sizeof(float) * nH);
    float *qkv = (float *)malloc(sizeof(float) * nH * 3);
    float *q = (float *)malloc(sizeof(float) * nH), *k = (float *)malloc(sizeof(float) * nH);
    float *v = (float *)malloc(sizeof(float) * nH);
    float *qr = (float *)malloc(sizeof(float) * nH), *kr = (float *)malloc(sizeof(float) * nH);
    float *f1 = (float *)malloc(sizeof(float) * (size_t)n * I);
    float *cs = (float *)malloc(sizeof(float) * (size_t)n * D), *sn = (float *)malloc(sizeof(float) * (size_t)n * D);
    int *idx = (int *)malloc(sizeof(int) * 4 * (size_t)n), *co = (int *)malloc(sizeof(int) * 2 * (size_t)n);
    float *wg = (float *)malloc(sizeof(float) * 4 * (size_t)n);

    /* patch embed: fp32 accumulation + bias, one rounding (vision_kernels.cu:16-31) */
    o1o_linear(pixels, w->patch_w, w->patch_b, tmp, n, H, c->patch_dim, R ? 1 : 0);
    /* position embedding: bf16(sum of 4 weighted taps), then bf16(patch + pos) */
    o1o_vision_tables(grid_h, grid_w, c->nside, c->merge, idx, wg, co);
    for (int r = 0; r < n; r++)
        for (int j = 0; j < H; j++) {
            float acc = 0.f;
            for (int t = 0; t < 4; t++) acc += wg[(size_t)t * n + r] * w->pos_embed[(size_t)idx[(size_t)t * n + r] * H + j];
            h[(size_t)r * H + j] = rnd(tmp[(size_t)r * H + j] + rnd(acc, R), R);
        }
    o1o_vision_rotary(co, n, D, R, cs, sn);
    const float scale = (float)(1.0 / sqrt((double)D));

    int ds_j = 0;
    for (int L = 0; L < c->depth; L++) {
        const o1o_vision_block *b = &w->blocks[L];
        o1o_layernorm(h, b->norm1_w, b->norm1_b, ln, n, H, 1e-6f, R);
        o1o_linear(ln, b->qkv_w, b->qkv_b, qkv, n, 3 * H, H, lm);
        /* qkv [n, 3, NH, D] -> head-major q/k/v [NH, n, D] (vision_kernels.cu:283-302) */
        for (int s = 0; s < n; s++)
            for (int hh = 0; hh < NH; hh++) {
                memcpy(q + ((size_t)hh * n + s) * D, qkv + (size_t)s * 3 * H + (size_t)hh * D, sizeof(float) * D);
                memcpy(k + ((size_t)hh * n + s) * D, qkv + (size_t)s * 3 * H + H + (size_t)hh * D, sizeof(float) * D);
                memcpy(v + ((size_t)hh * n + s) * D, qkv + (size_t)s * 3 * H + 2 * H + (size_t)hh * D, sizeof(float) * D);
            }
        /* rotary in fp32, one rounding (rope.cu:157-180) */
        rotary(q, cs, sn, qr, NH, n, D, R);
        rotary(k, cs, sn, kr, NH, n, D, R);
        /* full (non-causal) attention, bf16 probabilities as the fused
         * kernel rounds them; out seq-major [n, NH*D] */
        o1o_attention(qr, kr, v, NULL, NH, NH, n, D, 0, scale, R ? 1 : 0, R, att);
        o1o_linear(att, b->proj_w, b->proj_b, tmp, n, H, H, lm);
        o1o_residual_add(h, tmp, tmp, nH, R);                         /* attn_resid */
        o1o_layernorm(tmp, b->norm2_w, b->norm2_b, ln, n, H, 1e-6f, R);
        o1o_linear(ln, b->fc1_w, b->fc1_b, f1, n, I, H, lm);
        o1o_gelu_tanh(f1, f1, (size_t)n * I, R);
        o1o_linear(f1, b->fc2_w, b->fc2_b, att, n, H, I, lm);
        o1o_residual_add(tmp, att, h, nH, R);                          /* mlp_resid */
        if (after_blocks) memcpy(after_blocks + (size_t)L * nH, h, sizeof(float) * nH);
        if (deepstack && ds_j < c->n_ds && c->ds_layers[ds_j] == L) {
            merger(h, &w->deepstack[ds_j], c, 1, n, deepstack[ds_j]);
            ds_j++;
        }
    }
    merger(h, &w->merger, c, 0, n, embeds);
    free(h); free(tmp); free(ln); free(att); free(qkv); free(q); free(k); free(v); free(qr); free(kr); free(f1);
    free(cs); free(sn); free(idx); free(co); free(wg);
    return 0;
}
