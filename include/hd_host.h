#ifndef HD_HOST_H
#define HD_HOST_H

/*
 * Host-side modules around the forward: the seeded initial noise (torch CPU
 * MT19937 randn), the sampler sigma schedules, position-id / mask tables and
 * the flow-match Euler + CFG denoising loop that drives hd_forward_batched.
 *
 * Replaces (same names, same struct layouts, same results):
 *   src/runtime/torch_rng.h:30-56     hd_torch_rng_*  / hd_torch_randn_f32
 *   src/model/scheduler.h             hd_scheduler_* (sigma derivations, Euler step,
 *                                     UniPC plan and CPU step)
 *   src/runtime/sequence.c:102-142    T2I position ids and causal-prefix mask
 *   src/runtime/generate.c:78-104     initial noise (seed + 1) and pixel_unshuffle
 */

#include <stddef.h>
#include <stdint.h>

#include "hidream_hip.h"
#include "hd_forward.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- torch CPU MT19937 (torch_rng.h:30-56) ---------------------------- */
typedef struct hd_torch_rng {
    uint64_t seed_;
    int left_;
    int seeded_;
    uint32_t next_;
    uint32_t state[624];
} hd_torch_rng;

void hd_torch_rng_seed(hd_torch_rng *rng, uint64_t seed);
uint32_t hd_torch_rng_u32(hd_torch_rng *rng);
float hd_torch_uniform_f32(hd_torch_rng *rng);
/* torch.randn(n) on a CPU generator: n >= 16 uses the 16-wide Box-Muller
 * fill (last 16 redrawn when n % 16 != 0); n < 16 the double-precision
 * serial path with a cached second sample. */
void hd_torch_randn_f32(hd_torch_rng *rng, float *out, int64_t n);

/* ---- scheduler (scheduler.h) ------------------------------------------ */
#define HD_SCHED_MAX_STEPS 64
typedef struct {
    float sigmas[HD_SCHED_MAX_STEPS];
    int num_steps;          /* sigmas written, including the trailing 0 */
    int step_index;
    float noise_clip_std;
} hd_scheduler;

hd_status hd_scheduler_init(hd_scheduler *s, const float *sigmas, int num_steps,
                            float noise_clip_std);
float hd_scheduler_sigma(const hd_scheduler *s);
/* Dev recipe: the 28 frozen timesteps / 1000 + 0 (scheduler.c:28-72). */
int hd_scheduler_derive_dev(hd_scheduler *s, float noise_clip_std);
/* flash / flow_match: ramp in timestep space, shift applied (fp64). */
int hd_scheduler_derive_flash(hd_scheduler *s, int steps, float shift, float noise_clip_std);
int hd_scheduler_derive_flow_match(hd_scheduler *s, int steps, float shift,
                                   float noise_clip_std);
/* default (UniPC recipe): linear in sigma space, shift applied (fp64). */
int hd_scheduler_derive_default(hd_scheduler *s, int steps, float shift, float noise_clip_std);
float hd_scheduler_noise_scale(const hd_scheduler *s, int step_index, float noise_scale_start,
                               float noise_scale_end);
/* Flash SDE step on the device (scheduler.c:74-102): upcast z, denoised =
 * z - mo*sigma, z' = (sigma'*noise)*s_noise + (1-sigma')*denoised -> bf16.
 * scratch: 3n floats of device memory. */
hd_status hd_scheduler_step(hd_scheduler *s, const void *z_bf16, const float *model_output,
                            const float *noise_post_clamp, float s_noise, void *z_next_bf16,
                            int n, float *scratch);

/* ---- FlowUniPC multistep, solver order 2, bh2, predict_x0 (scheduler.h:107-178)
 * Same struct layouts as the reference. The per-step coefficients are derived
 * on the host in fp64 (hd_scheduler_unipc_plan); the pointwise math runs on
 * the device (hd_unipc_convert / hd_unipc_correct / hd_unipc_predict). */
#define HD_UNIPC_ORDER 2
typedef struct {
    float *model_outputs[HD_UNIPC_ORDER]; /* ring, newest at index ORDER-1 */
    float *last_sample;                   /* pre-predictor sample */
    int has_last_sample;
    int this_order;
    int lower_order_nums;
    int step_index;
} hd_scheduler_unipc;

typedef struct {
    int corr_order;        /* corrector order (0: no corrector) */
    int pred_order;        /* predictor order (1 during warm-up, 2 after) */
    int next_this_order;   /* persist for the next step's corrector */
    int next_lower_order;  /* persist: warm-up counter */
    double c_sig_t, c_sig_s0, c_alpha_t;
    double c_h_phi_1, c_B_h;
    double c_rhos0, c_rhos1, c_inv_rks0;
    double p_sig_t, p_sig_s0, p_alpha_t;
    double p_h_phi_1, p_B_h;
    double p_rhos_p, p_inv_rks0;
} hd_unipc_plan;

/* scheduler.h:170: coefficients for step si given the persisted predictor
 * order (this_order, 0 on the first step) and warm-up counter. */
void hd_scheduler_unipc_plan(const hd_scheduler *s, int si, int this_order,
                             int lower_order_nums, hd_unipc_plan *plan);
/* scheduler.h:174: one whole UniPC step on host arrays (convert, optional
 * corrector, history shift, predictor), fp64 scalar math; scratch: n floats. */
hd_status hd_scheduler_unipc_step(const hd_scheduler *s, hd_scheduler_unipc *u,
                                  const float *model_output, const float *sample,
                                  float *prev_sample, int n, float *scratch);

/* Per-step SDE noise of the flash/dev samplers (generate.c:907-925): n draws
 * of hd_torch_randn_f32, then, when clip > 0, clamped to +-clip * std (std
 * unbiased, fp64 accumulation). */
void hd_step_noise(hd_torch_rng *rng, float *out, int64_t n, float clip);

/* ---- sequence tables (sequence.c:102-142) ------------------------------ */
/* T2I position ids, pos [3, S] fp32, S = text_len + grid_h*grid_w: text row i
 * = (i, i, i); image token (r, c) = fix_point + (0, r, c). */
hd_status hd_seq_t2i_positions(int text_len, int grid_h, int grid_w, int fix_point, float *pos);
/* [S, S] bf16 additive mask: -max_bf16 (0xFF7F) above the diagonal on rows
 * < text_len - 1, 0 elsewhere. */
hd_status hd_seq_t2i_mask(int text_len, int seq, uint16_t *mask);
/* Synthetic 2-D layout: n_text text rows at (base, base, base), then for each
 * image segment i a grid_h[i] x grid_w[i] grid at (base, base + row_off[i] + r,
 * base + col_off[i] + c). Returns the sequence length, or -1. */
int hd_seq_grid_positions(int n_text, int n_seg, const int *grid_h, const int *grid_w,
                          const int *row_off, const int *col_off, float base, float *pos);

/* ---- initial latent (generate.c:78-104) -------------------------------- */
/* randn(3*H*W) from seed + 1, laid out [3, H, W] fp32. */
void hd_initial_noise(uint64_t seed, int width, int height, float *out);
/* tok[r*gw + c][ch*p*p + i*p + j] = img[ch][r*p + i][c*p + j] (host). */
void hd_pixel_unshuffle(const float *img, int channels, int height, int width, int patch,
                        float *tok);
/* decode.c:5-27: (v+1)/2*255, round half away from zero, clamp, HWC u8. */
void hd_decode_to_rgb(const float *z_f32, int grid_h, int grid_w, int patch, int channels,
                      unsigned char *out);

/* ---- denoising loops (extension; generate.c:855-935 and :1314-1455) ----
 * The model is fed t = 1 - sigma_i, and sigma_i is floored at 1e-6 before the
 * velocity division, as the reference's step loops do.
 *
 * hd_denoise_euler_cfg: flow-match Euler with classifier-free guidance, batch
 * 2 in one forward (row 0 = cond ids, row 1 = uncond ids), all on the device:
 *   for i in [0, steps):
 *     x = hd_forward_batched(ids, z, 1 - sigma_i)     [2, S, 3072]
 *     mo_c = (z - x_c[img])/sigma_i, mo_u likewise    (hd_sched_vcond)
 *     mo = (1-g) mo_u + g mo_c                        (hd_sched_cfg_guided)
 *     z = bf16(z + (sigma_{i+1} - sigma_i) mo)        (hd_sched_flow_match_step)
 * z: [img_tokens, 3072] bf16, updated in place. sigmas: host, steps + 1.
 * `ws` must be sized by hd_forward_batched_workspace_bytes(2, ...) and
 * `scratch` by hd_denoise_scratch_bytes(). */
int64_t hd_denoise_scratch_bytes(int seq, int img_tokens, int steps);
hd_status hd_denoise_euler_cfg(const hd_forward_binding *bw, hd_forward_workspace *ws,
                               const int64_t *ids_dev, int text_len, const float *pos_dev,
                               int ar_len, void *z_dev, int img_tokens, const float *sigmas,
                               int steps, float guidance, int seq, int heads, int kv_heads,
                               int hidden, int ff_hidden, int head_dim, int tms_token_id,
                               void *scratch, int64_t scratch_bytes, void *stream);

/* Final-latent check of every denoise loop (generate.c:1474-1496): after the
 * last step the loop returns HD_ERR_MISSING (generate's failure status,
 * generate.c:1546) with hd_last_error() set when the latent holds a NaN/Inf
 * ("final latent contains NaN/Inf") or, in mode 2, a value outside [-2, 2]
 * ("final latent range [lo, hi] out of bounds"); z keeps the values the last
 * step wrote. mode 2 = the reference's check (default), 1 = NaN/Inf only
 * (random-weight runs leave the range), 0 = off. Process-wide; returns the
 * previous mode, or -1 for a mode outside 0..2. */
int hd_denoise_set_output_check(int mode);

/* hd_denoise: the reference's three samplers on the device.
 *   HD_SAMPLER_EULER  flow_match: z = bf16(z + (s_{i+1} - s_i) mo)
 *   HD_SAMPLER_FLASH  dev/flash SDE: per-step noise (hd_step_noise from
 *                     seed + 1, clip noise_clip_std), s_noise ramped from
 *                     s_noise_start to s_noise_end, hd_scheduler_step
 *   HD_SAMPLER_UNIPC  default: FlowUniPC order 2 (hd_scheduler_unipc_plan +
 *                     hd_unipc_*), z = bf16(predictor output)
 * batch 2 runs classifier-free guidance (row 0 cond, row 1 uncond, combined
 * with `guidance`) over two sequences of equal length sharing text_len and
 * positions (pad the unconditional prompt, or use hd_denoise_cfg for the
 * reference's shorter unconditional sequence); batch 1 runs the conditional
 * forward only. The sigma schedule comes from `sched` (steps + 1 values). Scratch:
 * hd_denoise_run_scratch_bytes(). The flash sampler's noise is drawn on the
 * host into pinned staging while the previous step's forward runs. */
enum { HD_SAMPLER_EULER = 0, HD_SAMPLER_FLASH = 1, HD_SAMPLER_UNIPC = 2 };
int64_t hd_denoise_run_scratch_bytes(int batch, int seq, int img_tokens, int steps);
hd_status hd_denoise(const hd_forward_binding *bw, hd_forward_workspace *ws, int sampler,
                     const hd_scheduler *sched, int steps, int batch, const int64_t *ids_dev,
                     int text_len, const float *pos_dev, int ar_len, void *z_dev, int img_tokens,
                     float guidance, uint64_t seed, float s_noise_start, float s_noise_end,
                     float noise_clip_std, int seq, int heads, int kv_heads, int hidden,
                     int ff_hidden, int head_dim, int tms_token_id, void *scratch,
                     int64_t scratch_bytes, void *stream);

/* hd_denoise_cfg (extension): guided generation with the unconditional
 * branch as a sequence of its own, as the reference runs it: its " "
 * caption gives it a shorter text (T_uncond), its own positions, causal
 * prefix and workspace (generate.c:1075, :1119-1120, :1341). Each step runs
 * the conditional forward over [text | image] (S = T + I rows) and the
 * unconditional one over [text_uncond | image] (S_uncond rows) on the same
 * latent z, combines the two velocities with `guidance` and applies the
 * sampler, as hd_denoise with batch 2 does for equal-length sequences.
 * ws_uncond must be a different workspace, sized for S_uncond
 * (hd_forward_batched_workspace_bytes with batch 1). Scratch:
 * hd_denoise_cfg_scratch_bytes(). */
int64_t hd_denoise_cfg_scratch_bytes(int seq, int seq_uncond, int img_tokens, int steps);
hd_status hd_denoise_cfg(const hd_forward_binding *bw, hd_forward_workspace *ws,
                         hd_forward_workspace *ws_uncond, int sampler, const hd_scheduler *sched,
                         int steps, const int64_t *ids_dev, int text_len, const float *pos_dev,
                         int ar_len, int seq, const int64_t *ids_uncond_dev, int text_len_uncond,
                         const float *pos_uncond_dev, int ar_len_uncond, int seq_uncond, void *z_dev,
                         int img_tokens, float guidance, uint64_t seed, float s_noise_start,
                         float s_noise_end, float noise_clip_std, int heads, int kv_heads,
                         int hidden, int ff_hidden, int head_dim, int tms_token_id, void *scratch,
                         int64_t scratch_bytes, void *stream);

/* hd_denoise_visual: the edit / personalize loop (generate.c:855-935), batch
 * 1 with vision conditioning. Each step runs hd_forward over
 * [text | target img_tokens | ref_tokens references] with `mask` (or the
 * workspace's SDPA plan) and `visual`, takes the velocity of the target rows
 * only and applies the sampler to z [img_tokens, 3072] in place. The
 * references are `ref_patches` [ref_tokens, 3072] bf16, copied once behind
 * the target rows, unless the workspace caches their x_embedder rows
 * (ws->xe_ref with ws->n_ref == ref_tokens, as generate.c:792-805 sets up):
 * then the cache is used and ref_patches may be NULL. The reference's edit loop runs the flash step for its default
 * schedule: pass HD_SAMPLER_FLASH with a hd_scheduler_derive_default
 * schedule for that. Scratch: hd_denoise_run_scratch_bytes(1, seq,
 * img_tokens + ref_tokens, steps). */
hd_status hd_denoise_visual(const hd_forward_binding *bw, hd_forward_workspace *ws, int sampler,
                            const hd_scheduler *sched, int steps, const int64_t *ids_dev,
                            int text_len, const float *pos_dev, const void *mask_dev,
                            const hd_visual_cond *visual, void *z_dev, int img_tokens,
                            const void *ref_patches, int ref_tokens, uint64_t seed,
                            float s_noise_start, float s_noise_end, float noise_clip_std, int seq,
                            int heads, int kv_heads, int hidden, int ff_hidden, int head_dim,
                            int tms_token_id, void *scratch, int64_t scratch_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HD_HOST_H */
