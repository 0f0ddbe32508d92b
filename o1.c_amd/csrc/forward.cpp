// Whole-denoiser forward (replaces the reference's src/model/forward.c).
//
// Steps (forward.c:253-397): t-embedder MLP, token embedding + timestep
// token substitution, x_embedder (2 GEMMs), concat, n_layers blocks, final
// RMSNorm, output head. Differences by design: the block updates the hidden
// state in place (no A/B ping-pong, no per-block D2D copy), the text rows
// and the projected image rows are written straight into the hidden state
// (no h_text/xe_out concat copies), the rotary table is built once per
// forward instead of once per block, and B sequences share each launch.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/hd_hip.h"
#include "../../include/hd_gemm.h"
#include "../../include/hd_sdpa.h"
#include "../../include/hd_block.h"
#include "../../include/hd_forward.h"
#include "../../include/hd_vision.h"

#define HD_PATCH_FEATS 3072   // forward.c:299-301 (3 x 32 x 32)
#define HD_XE_MID 1024        // x_embedder bottleneck
#define HD_TDIM 256           // timestep sinusoid width
#define HD_VOCAB 151936LL     // forward.c:274

static inline int64_t al256(int64_t x) { return (x + 255) & ~(int64_t)255; }

enum { R_HIDDEN, R_HTEXT, R_NORM, R_HEAD, R_TEMB, R_TEH, R_FREQ, R_FREQB, R_TS, R_XES, R_XEO,
       R_CS, R_BLOCK, R_COUNT };

static int64_t layout(int batch, int64_t seq, int text, int img, int heads, int kv, int hidden,
                      int ff, int hd, int64_t off[R_COUNT], int64_t *block_bytes) {
    const int64_t M = (int64_t)batch * seq;
    int64_t o = 0;
    auto take = [&](int idx, int64_t bytes) { off[idx] = o; o = al256(o + bytes); };
    take(R_HIDDEN, M * hidden * 2);
    take(R_HTEXT, (int64_t)batch * text * hidden * 2);
    take(R_NORM, M * hidden * 2);
    take(R_HEAD, M * HD_PATCH_FEATS * 2);
    take(R_TEMB, (int64_t)batch * hidden * 2);
    take(R_TEH, (int64_t)batch * hidden * 2);
    take(R_FREQ, (int64_t)batch * HD_TDIM * 4);
    take(R_FREQB, (int64_t)batch * HD_TDIM * 2);
    take(R_TS, (int64_t)batch * 4);
    take(R_XES, (int64_t)batch * img * HD_XE_MID * 2);
    take(R_XEO, (int64_t)batch * img * hidden * 2);
    take(R_CS, seq * (int64_t)hd * 4);
    int64_t bs = hd_decoder_block_batched_scratch_bytes(batch, seq, heads, kv, hidden, ff, hd);
    if (block_bytes) *block_bytes = bs;
    take(R_BLOCK, bs);
    return o;
}

extern "C" hd_status hd_forward_resolve(const hd_weight_store *ws, int n_layers,
                                        hd_forward_binding *out) {
    if (!ws || !out || n_layers <= 0) {
        hd_set_error("forward: null argument in resolve");
        return HD_ERR_MISSING;
    }
    hd_forward_binding b;
    memset(&b, 0, sizeof(b));
    // Tensor names of forward.c:72-82.
    b.embed_tokens = hd_weight_store_find(ws, "model.language_model.embed_tokens.weight");
    b.te0_w = hd_weight_store_find(ws, "model.t_embedder1.mlp.0.weight");
    b.te0_b = hd_weight_store_find(ws, "model.t_embedder1.mlp.0.bias");
    b.te2_w = hd_weight_store_find(ws, "model.t_embedder1.mlp.2.weight");
    b.te2_b = hd_weight_store_find(ws, "model.t_embedder1.mlp.2.bias");
    b.xe1_w = hd_weight_store_find(ws, "model.x_embedder.proj1.weight");
    b.xe2_w = hd_weight_store_find(ws, "model.x_embedder.proj2.weight");
    b.xe2_b = hd_weight_store_find(ws, "model.x_embedder.proj2.bias");
    b.fl_w = hd_weight_store_find(ws, "model.final_layer2.linear.weight");
    b.fl_b = hd_weight_store_find(ws, "model.final_layer2.linear.bias");
    b.fnorm_w = hd_weight_store_find(ws, "model.language_model.norm.weight");
    if (!b.embed_tokens || !b.te0_w || !b.te0_b || !b.te2_w || !b.te2_b || !b.xe1_w || !b.xe2_w ||
        !b.xe2_b || !b.fl_w || !b.fl_b || !b.fnorm_w) {
        hd_set_error("forward: missing global weight(s) in store");
        return HD_ERR_MISSING;
    }
    b.n_layers = n_layers;
    b.blocks = (hd_block_binding *)calloc((size_t)n_layers, sizeof(hd_block_binding));
    if (!b.blocks) {
        hd_set_error("forward: oom allocating block bindings");
        return HD_ERR_OOM;
    }
    for (int i = 0; i < n_layers; i++) {
        hd_status s = hd_block_resolve(ws, i, &b.blocks[i]);
        if (s != HD_OK) {
            hd_forward_binding_free(&b);
            return s;
        }
    }
    *out = b;
    return HD_OK;
}

extern "C" void hd_forward_binding_free(hd_forward_binding *b) {
    if (!b) return;
    free(b->blocks);
    b->blocks = nullptr;
    b->n_layers = 0;
}

extern "C" int hd_forward_num_layers(const hd_forward_binding *bw) { return bw ? bw->n_layers : 0; }

extern "C" int64_t hd_forward_workspace_bytes(int64_t seq, int img_tokens, int heads, int kv_heads,
                                              int hidden, int ff_hidden, int head_dim,
                                              int64_t *block_scratch_bytes) {
    int64_t off[R_COUNT];
    int text = (int)(seq - img_tokens);
    if (text < 0) text = 0;
    return layout(1, seq, text, img_tokens, heads, kv_heads, hidden, ff_hidden, head_dim, off,
                  block_scratch_bytes);
}

extern "C" int64_t hd_forward_batched_workspace_bytes(int batch, int64_t seq, int img_tokens,
                                                      int heads, int kv_heads, int hidden,
                                                      int ff_hidden, int head_dim) {
    int64_t off[R_COUNT];
    int text = (int)(seq - img_tokens);
    if (text < 0) text = 0;
    return layout(batch, seq, text, img_tokens, heads, kv_heads, hidden, ff_hidden, head_dim, off,
                  nullptr);
}

extern "C" int64_t hd_forward_ws_offset(const char *name, int64_t seq, int text_len, int img_tokens,
                                        int heads, int kv_heads, int hidden, int ff_hidden,
                                        int head_dim, int64_t *block_scratch_bytes) {
    if (!name) return -1;
    int64_t off[R_COUNT];
    layout(1, seq, text_len, img_tokens, heads, kv_heads, hidden, ff_hidden, head_dim, off,
           block_scratch_bytes);
    static const struct { const char *n; int i; } map[] = {
        {"hidden_a", R_HIDDEN}, {"hidden_b", R_HIDDEN}, {"h_text", R_HTEXT}, {"norm_out", R_NORM},
        {"head_out", R_HEAD}, {"t_emb", R_TEMB}, {"te_hidden", R_TEH}, {"freq", R_FREQ},
        {"freq_bf16", R_FREQB}, {"t_scaled", R_TS}, {"xe_stage", R_XES}, {"xe_out", R_XEO},
        {"rope_cs", R_CS}, {"block_scratch", R_BLOCK}};
    for (auto &m : map)
        if (strcmp(m.n, name) == 0) return off[m.i];
    return -1;
}

static hd_status fwd_err(const char *where) {
    const char *e = hd_cuda_last_error();
    if (e && e[0]) {
        hd_set_error("forward: %s: %s", where, e);
        return HD_ERR_RUNTIME;
    }
    return HD_OK;
}

static hd_status d2d(void *dst, const void *src, size_t bytes, hipStream_t st) {
    if (!dst || !bytes) return HD_OK;
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st) != hipSuccess) {
        hd_set_error("forward: device copy failed");
        return HD_ERR_IO;
    }
    return HD_OK;
}

// Shared body of hd_forward / hd_forward_batched.
static hd_status forward_core(const hd_forward_binding *bw, hd_forward_workspace *ws, int B,
                              const int64_t *ids, int T, const float *pos, const void *mask,
                              int ar_len, const void *vin, int I, const float *tstep, int S,
                              int H, int KV, int HID, int FF, int D, int tms,
                              hd_forward_diagnostics *dg, void *out,
                              const hd_visual_cond *vis = nullptr,
                              const int64_t *sec_dev = nullptr) {
    const hd_block_config *cfg;
    hd_block_config c;
    hd_block_get_config(&c);
    cfg = &c;
    uint8_t *base = (uint8_t *)ws->hidden_a;
    int64_t off[R_COUNT], bs;
    layout(B, S, T, I, H, KV, HID, FF, D, off, &bs);
    uint16_t *hidden = (uint16_t *)(base + off[R_HIDDEN]);
    void *norm_out = base + off[R_NORM];
    void *t_emb = base + off[R_TEMB];
    void *te_h = base + off[R_TEH];
    float *freq = (float *)(base + off[R_FREQ]);
    void *freq_b = base + off[R_FREQB];
    float *ts = (float *)(base + off[R_TS]);
    uint16_t *xe_s = (uint16_t *)(base + off[R_XES]);
    uint16_t *h_text = (uint16_t *)(base + off[R_HTEXT]);
    float *cs = (float *)(base + off[R_CS]);
    void *scratch = base + off[R_BLOCK];
    hipStream_t st = (hipStream_t)hd_hip_get_stream();
    const size_t row = (size_t)HID * 2;
    hd_status s;

    hd_cuda_clear_error();
    // t-embedder (forward.c:253-265): t*1000 -> sinusoid(256) -> bf16 ->
    // linear+bias -> SiLU -> linear+bias, one row per sequence.
    hd_scale_f32(tstep, ts, 1000.0f, B);
    hd_timestep_embed(ts, freq, B, HD_TDIM);
    hd_f32_convert_bf16(freq, freq_b, B * HD_TDIM);
    hd_linear(freq_b, bw->te0_w, bw->te0_b, te_h, B, HID, HD_TDIM, 1);
    hd_silu(te_h, t_emb, (size_t)B * HID);
    hd_linear(t_emb, bw->te2_w, bw->te2_b, te_h, B, HID, HID, 1);   // te_h = t_emb (final)
    if ((s = fwd_err("t-embedder")) != HD_OK) return s;

    // text rows: gather + timestep-token substitution into the hidden state
    for (int b = 0; b < B && T > 0; b++) {
        uint16_t *ht = h_text + (size_t)b * T * HID;
        hd_gather_rows(bw->embed_tokens, ids + (size_t)b * T, ht, T, HID, HD_VOCAB);
        if (dg && b == 0 && (s = d2d(dg->after_embedding, ht, (size_t)T * row, st)) != HD_OK) return s;
        // vision conditioning (forward.c:278-287): the image-pad rows take the
        // vision tower's embeddings in order, before the timestep substitution
        if (vis) hd_vision_masked_scatter_n(ht, vis->visual_mask, vis->image_embeds, ht, T, HID, vis->v_tokens);
        hd_apply_tms_condition(ids + (size_t)b * T, ht, (const uint16_t *)te_h + (size_t)b * HID,
                               hidden + (size_t)b * S * HID, T, HID, tms);
        if (dg && b == 0 &&
            (s = d2d(dg->after_timestep_conditioning, hidden, (size_t)T * row, st)) != HD_OK)
            return s;
    }
    // image rows: x_embedder proj1 over all sequences, proj2(+bias) straight
    // into each sequence's image rows (forward.c:301-324)
    const int n_ref = (ws->xe_ref && ws->n_ref > 0 && ws->n_ref < I) ? ws->n_ref : 0;
    const int I_t = I - n_ref;
    for (int b = 0; b < B; b++) {
        const uint16_t *vb = (const uint16_t *)vin + (size_t)b * I * HD_PATCH_FEATS;
        uint16_t *xs = xe_s + (size_t)b * I * HD_XE_MID;
        uint16_t *dst = hidden + ((size_t)b * S + T) * HID;
        hd_linear(vb, bw->xe1_w, nullptr, xs, I_t, HD_XE_MID, HD_PATCH_FEATS, 1);
        hd_linear(xs, bw->xe2_w, bw->xe2_b, dst, I_t, HID, HD_XE_MID, 1);
        if (n_ref && (s = d2d(dst + (size_t)I_t * HID, ws->xe_ref, (size_t)n_ref * row, st)) != HD_OK)
            return s;
    }
    if ((s = fwd_err("embedding")) != HD_OK) return s;
    if (dg) {
        if ((s = d2d(dg->after_target_embedding, hidden + (size_t)T * HID, (size_t)I * row, st)) != HD_OK) return s;
        if ((s = d2d(dg->after_block_0_input, hidden, (size_t)S * row, st)) != HD_OK) return s;
    }

    if (sec_dev)   // the caller's device section (forward.c passes sec_dev to every block)
        hd_rope_table_dev(pos, S, sec_dev, 3, D, cfg->rope_theta, cfg->attention_scaling,
                          cfg->interleaved, cs);
    else
        hd_rope_table(pos, S, cfg->section, 3, D, cfg->rope_theta, cfg->attention_scaling,
                      cfg->interleaved, cs);
    if ((s = fwd_err("rope table")) != HD_OK) return s;

    const int n = bw->n_layers;
    for (int i = 0; i < n; i++) {
        s = hd_decoder_block_batched(hidden, cs, mask, ar_len, &bw->blocks[i], scratch, bs, nullptr,
                                     hidden, B, S, H, KV, HID, FF, D);
        if (s != HD_OK) return s;
        if (dg) {
            void *dst = i == 0 ? dg->after_block_0
                               : (i == n / 2 ? dg->after_block_mid
                                             : (i == n - 1 ? dg->after_block_last : nullptr));
            if ((s = d2d(dst, hidden, (size_t)S * row, st)) != HD_OK) return s;
        }
        // DeepStack (forward.c:363-370): blocks 0..2 add the deepstack
        // embeddings to the image-pad rows of their output
        if (vis && i < 3 && vis->deepstack[i])
            hd_vision_deepstack_inject_n(hidden, vis->visual_mask, vis->deepstack[i], hidden, S, HID,
                                         vis->v_tokens);
    }
    if (dg && (s = d2d(dg->before_final_norm, hidden, (size_t)S * row, st)) != HD_OK) return s;
    hd_rmsnorm(hidden, bw->fnorm_w, norm_out, B * S, HID, cfg->eps);
    if (dg && (s = d2d(dg->after_final_norm, norm_out, (size_t)S * row, st)) != HD_OK) return s;
    hd_linear(norm_out, bw->fl_w, bw->fl_b, out, B * S, HD_PATCH_FEATS, HID, 1);
    if ((s = fwd_err("head")) != HD_OK) return s;
    if (dg && (s = d2d(dg->after_final_head, out, (size_t)S * HD_PATCH_FEATS * 2, st)) != HD_OK) return s;
    return HD_OK;
}

struct StreamScope {
    void *prev;
    explicit StreamScope(void *s) : prev(hd_hip_get_stream()) { if (s) hd_hip_set_stream(s); }
    ~StreamScope() { hd_hip_set_stream(prev); }
};

static hd_status common_checks(const hd_forward_binding *bw, hd_forward_workspace *ws, int T, int I,
                               int S, int H, int KV, int HID, int FF, int D) {
    if (!bw->blocks || bw->n_layers <= 0) {
        hd_set_error("forward: binding not resolved");
        return HD_ERR_MISSING;
    }
    if (!ws->hidden_a) {
        hd_set_error("forward: workspace buffer not allocated");
        return HD_ERR_MISSING;
    }
    if (T < 0 || I <= 0 || T + I != S) {
        hd_set_error("forward: text+img != seq");
        return HD_ERR_MISSING;
    }
    if (D != 128 || HID % 64 || FF % 64 || (H * D) % 256 || (KV * D) % 256 || H % KV) {
        hd_set_error("forward: unsupported model shape");
        return HD_ERR_UNSUPPORTED;
    }
    return HD_OK;
}

extern "C" hd_status hd_forward(const hd_forward_binding *bw, hd_forward_workspace *ws,
                                const int64_t *input_ids, int text_len, const float *pos_f32,
                                const void *mask_dev, const void *vinputs, int img_tokens,
                                const hd_visual_cond *visual, const float *timestep,
                                const int64_t *sec_dev, int seq, int heads, int kv_heads,
                                int hidden, int ff_hidden, int head_dim, int tms_token_id,
                                hd_forward_diagnostics *diag, void *out_dev, void *stream) {
    if (!bw || !ws || (!input_ids && text_len > 0) || !pos_f32 || !vinputs || !timestep || !out_dev) {
        hd_set_error("forward: null argument");
        return HD_ERR_MISSING;
    }
    if (visual && (!visual->image_embeds || !visual->visual_mask || visual->v_tokens < 0)) {
        hd_set_error("forward: visual conditioning without embeddings or mask");
        return HD_ERR_MISSING;
    }
    hd_status s = common_checks(bw, ws, text_len, img_tokens, seq, heads, kv_heads, hidden,
                                ff_hidden, head_dim);
    if (s != HD_OK) return s;
    StreamScope scope(stream);
    int ar_len = hd_sdpa_plan_ar_len(ws->sdpa);
    const void *mask = ar_len > 0 ? nullptr : mask_dev;
    return forward_core(bw, ws, 1, input_ids, text_len, pos_f32, mask, ar_len, vinputs, img_tokens,
                        timestep, seq, heads, kv_heads, hidden, ff_hidden, head_dim, tms_token_id,
                        diag, out_dev, visual, sec_dev);
}

extern "C" hd_status hd_forward_batched(const hd_forward_binding *bw, hd_forward_workspace *ws,
                                        int batch, const int64_t *input_ids, int text_len,
                                        const float *pos_f32, int ar_len, const void *vinputs,
                                        int img_tokens, const float *timestep, int seq, int heads,
                                        int kv_heads, int hidden, int ff_hidden, int head_dim,
                                        int tms_token_id, hd_forward_diagnostics *diag,
                                        void *out_dev, void *stream) {
    if (!bw || !ws || (!input_ids && text_len > 0) || !pos_f32 || !vinputs || !timestep ||
        !out_dev || batch < 1) {
        hd_set_error("forward: null argument");
        return HD_ERR_MISSING;
    }
    hd_status s = common_checks(bw, ws, text_len, img_tokens, seq, heads, kv_heads, hidden,
                                ff_hidden, head_dim);
    if (s != HD_OK) return s;
    if (ar_len < 0 || ar_len > seq) {
        hd_set_error("forward: invalid ar_len");
        return HD_ERR_MISMATCH;
    }
    StreamScope scope(stream);
    return forward_core(bw, ws, batch, input_ids, text_len, pos_f32, nullptr, ar_len, vinputs,
                        img_tokens, timestep, seq, heads, kv_heads, hidden, ff_hidden, head_dim,
                        tms_token_id, diag, out_dev);
}
