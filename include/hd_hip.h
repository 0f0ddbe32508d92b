#ifndef HD_HIP_H
#define HD_HIP_H

/*
 * C ABI of the MI355X (gfx950) transformer primitives.
 *
 * Replaces the reference's src/cuda/hd_cuda.h (lines 34-198) symbol for
 * symbol: same names, argument order and meaning, bf16 payloads passed as
 * `void *` (IEEE bfloat16, round-to-nearest-even), fp32 as `float *`.
 * Every pointer is a device pointer. Every primitive is asynchronous on the
 * library's launch stream (the null stream unless hd_hip_set_stream() chose
 * another one), performs no allocation and no synchronisation.
 *
 * Errors follow the reference convention (support.cu:12-17): a primitive
 * returns void; on bad arguments or a failed launch it writes a message into
 * the process-global buffer read by hd_cuda_last_error() and returns.
 *
 * Additions beyond the reference are marked "extension" and are never
 * required by reference-style callers.
 */

#include <stddef.h>
#include <stdint.h>

#include "hidream_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t hd_bf16;

/* ---- host bf16 helpers (hd_cuda.h:34-41) ------------------------------ */
float hd_bf16_to_f32(uint16_t b);
uint16_t hd_f32_to_bf16(float f);
void hd_bf16_buf_to_f32(const void *src, float *dst, size_t n);
void hd_f32_buf_to_bf16(const float *src, void *dst, size_t n);

/* ---- error buffer (hd_cuda.h:47-48) ----------------------------------- */
const char *hd_cuda_last_error(void);
void hd_cuda_clear_error(void);

/* ---- launch stream (extension) ----------------------------------------
 * The reference launches on the legacy default stream. These select the
 * hipStream_t (passed as void*) every later launch of this library uses;
 * NULL restores the null stream. */
void hd_hip_set_stream(void *stream);
void *hd_hip_get_stream(void);
/* Blocks until the launch stream drains; returns 0 or the hipError_t. */
int hd_hip_sync(void);

/* ---- primitives ------------------------------------------------------- */

/* y = w * x * rsqrt(mean(x^2) + eps) per row, fp32 inside (hd_cuda.h:59). */
void hd_rmsnorm(const void *x_dev, const void *w_dev, void *y_dev,
                int rows, int cols, float eps);

/* y = x * sigmoid(x) (hd_cuda.h:63). */
void hd_silu(const void *x_dev, void *y_dev, size_t n);

/* y = bf16(bf16(silu(gate)) * up) (hd_cuda.h:66). */
void hd_swiglu(const void *gate_dev, const void *up_dev, void *y_dev, size_t n);

/* y = bf16(x + a) (hd_cuda.h:69). */
void hd_residual_add(const void *x_dev, const void *a_dev, void *y_dev, size_t n);

/* y[M,N] = x[M,K] . W[N,K]^T (+bias[N]), fp32 accumulate (hd_cuda.h:77).
 * Declared in hd_gemm.h as well; only transpose_w == 1 is supported. */
void hd_linear(const void *x_dev, const void *w_dev, const void *bias_dev,
               void *y_dev, int M, int N, int K, int transpose_w);

/* Sinusoidal timestep table [N,dim] fp32: cos first half, sin second
 * (hd_cuda.h:84). */
void hd_timestep_embed(const float *t_dev, float *y_dev, int N, int dim);

/* MRoPE cos/sin [bs,seq,head_dim] fp32 from pos [3,bs,seq] (hd_cuda.h:91). */
void hd_mrope_cos_sin(const float *pos_dev, int bs, int seq,
                      const int64_t *section_dev, int n_section,
                      int head_dim, float theta, float attention_scaling,
                      int interleaved, float *cos_dev, float *sin_dev);

/* Rotate-half RoPE with bf16 per-op rounding on [heads,seq,dim]
 * (hd_cuda.h:100). */
void hd_apply_rotary(const void *x_dev, const float *cos_dev,
                     const float *sin_dev, void *y_dev,
                     int heads, int seq, int dim);

/* Same rotation in fp32, one final bf16 rounding (hd_cuda.h:110). */
void hd_apply_rotary_f32(const void *x_dev, const float *cos_dev,
                         const float *sin_dev, void *y_dev,
                         int heads, int seq, int dim);

/* Attention with an additive [seq,seq] bf16 mask, GQA head h -> h/(H/KV).
 * q [heads,seq,dim], k/v [kv_heads,seq,dim], out seq-major [seq,heads,dim].
 * scores/probs [heads,seq,seq] bf16 receive the pre-softmax scores and the
 * probabilities (hd_cuda.h:121). Meant for small validation shapes. */
void hd_attention_eager(const void *q_dev, const void *k_dev, const void *v_dev,
                        const void *mask_dev, void *scores_dev,
                        void *probs_dev, void *out_dev,
                        int heads, int kv_heads, int seq, int dim,
                        float scaling);

/* [seq,heads,dim] <-> [heads,seq,dim] byte permutations (hd_cuda.h:132). */
void hd_head_split(const void *in_dev, void *out_dev, int seq, int heads, int dim);
void hd_head_merge(const void *in_dev, void *out_dev, int seq, int heads, int dim);

/* out[m] = table[idx[m]] (row 0 when idx is out of range) (hd_cuda.h:140). */
void hd_gather_rows(const void *table_dev, const void *idx_dev, void *out_dev,
                    int M, int cols, int64_t nrows);

/* out[row] = idx[row]==tms_id ? t_emb : emb[row] (hd_cuda.h:148). */
void hd_apply_tms_condition(const void *idx_dev, const void *emb_dev,
                            const void *t_emb_dev, void *out_dev,
                            int M, int H, int64_t tms_id);

/* y = x * s (fp32) and fp32 -> bf16 conversion (hd_cuda.h:153-155). */
void hd_scale_f32(const float *in_dev, float *out_dev, float s, int n);
void hd_f32_convert_bf16(const float *in_dev, void *out_dev, int n);

/* ---- sampler pointwise kernels (hd_cuda.h:161-186) -------------------- */
void hd_sched_bf16_upcast(const void *in_dev, float *out_dev, int n);
void hd_sched_denoised(const float *z_dev, const float *mo_dev, float sigma,
                       float *denoised_dev, int n);
void hd_sched_z_next(const float *noise_dev, const float *denoised_dev,
                     float sigma_next, float s_noise, float *z_next_dev, int n);
void hd_sched_vcond(const void *z_dev, const void *xp_dev, float sigma,
                    float *mo_dev, int n);
void hd_sched_flow_match_step(const void *z_dev, const float *mo_dev,
                              float sigma, float sigma_next,
                              void *z_next_dev, int n);
void hd_sched_cfg_guided(const float *mo_cond, const float *mo_uncond, float g,
                         float *mo_guided, int n);

/* ---- FlowUniPC pointwise kernels (hd_cuda.h:183-198), fp32 -------------
 * convert: conv = sample - sigma_cur * mo
 * correct: x = (sig_t/sig_s0) last - alpha_t h_phi_1 mo0;
 *          corr = rhos_c1 (conv - mo0)                       (order 1)
 *               = rhos_c0 (mo_old - mo0) inv_rks0 + rhos_c1 (conv - mo0)   (2)
 *          out = x - alpha_t B_h corr
 * predict: x = (sig_t/sig_s0) sample - alpha_t h_phi_1 mo0;
 *          order 2: x -= alpha_t B_h (rhos_p (mo_old - mo0) inv_rks0)
 * The products a*b - c*d are evaluated as fma(a, b, -(c*d)) and x - a*b as
 * fma(-a, b, x); sig_t/sig_s0, alpha_t*h_phi_1 and alpha_t*B_h are fp32. */
void hd_unipc_convert(const float *sample_dev, const float *mo_dev, float sigma_cur,
                      float *conv_dev, int n);
void hd_unipc_correct(const float *last_dev, const float *mo0_dev, const float *mo_old_dev,
                      const float *conv_dev, float sig_t, float sig_s0, float alpha_t,
                      float h_phi_1, float B_h, float rhos_c0, float rhos_c1, float inv_rks0,
                      int order_c, float *out_dev, int n);
void hd_unipc_predict(const float *sample_dev, const float *mo0_dev, const float *mo_old_dev,
                      float sig_t, float sig_s0, float alpha_t, float h_phi_1, float B_h,
                      float rhos_p, float inv_rks0, int order_p, float *out_dev, int n);

/* ---- fused kernels (extension) ----------------------------------------
 * The block composes these instead of the one-op-per-launch reference
 * chain; each reproduces the reference's bf16 rounding points exactly. */

/* y = rmsnorm(bf16(x + a)) and s = bf16(x + a), one pass over the row. */
void hd_add_rmsnorm(const void *x_dev, const void *a_dev, const void *w_dev,
                    void *sum_dev, void *y_dev, int rows, int cols, float eps);

/* Rotary table in the compact form the fused kernels read: cs[s, f] =
 * (cos, sin) of frequency f < head_dim/2 for token s, fp32 pairs, from
 * pos [3, seq] with the interleaved-MRoPE section rule (rope.cu:28-71). */
void hd_rope_table(const float *pos_dev, int seq, const int64_t *section_host,
                   int n_section, int head_dim, float theta,
                   float attention_scaling, int interleaved, float *cs_dev);
/* The same table with the section in device memory (int64[n_section], as
 * the reference's sec_dev), read by the kernel. */
void hd_rope_table_dev(const float *pos_dev, int seq, const int64_t *section_dev,
                       int n_section, int head_dim, float theta,
                       float attention_scaling, int interleaved, float *cs_dev);

/* QKV epilogue: qkv [B*S, (H+2KV)*D] projection output ->
 *   q  [B,H,S,D]  = rope(rmsnorm_D(q_proj) * q_norm)
 *   k  [B,KV,S,D] = rope(rmsnorm_D(k_proj) * k_norm)
 *   vt [B,KV,D,S_pad] = v_proj transposed (the flash kernel's V layout:
 *       S_pad = round_up(S, 64), key s stored at column s with bits 2 and 3
 *       exchanged, padding columns zero)
 * with the reference's roundings: norm -> bf16, rope products and sum
 * -> bf16 (block.c:260-282). vt may be NULL, then v [B,KV,S,D] is written
 * to v_dev instead. */
void hd_qkv_epilogue(const void *qkv_dev, const void *qn_w, const void *kn_w,
                     const float *cs_dev, void *q_dev, void *k_dev,
                     void *v_dev, void *vt_dev, int batch, int seq, int heads,
                     int kv_heads, int head_dim, float eps);

/* [B,KV,S,D] -> [B,KV,D,S] bf16 transpose (V operand layout). */
void hd_transpose_sd(const void *in_dev, void *out_dev, int bh, int seq, int dim);

/* Patch (un)shuffle (generate.c:85-104): img [C, Hp*p, Wp*p] fp32 <->
 * tokens [Hp*Wp, C*p*p]; tok[r*Wp+c][ch*p*p + i*p + j] =
 * img[ch][r*p+i][c*p+j]. Pure index permutation, bit-exact. */
void hd_patchify_f32(const float *img_dev, float *tok_dev, int C, int Hp,
                     int Wp, int p);
void hd_unpatchify_f32(const float *tok_dev, float *img_dev, int C, int Hp,
                       int Wp, int p);
/* Same permutation reading fp32 pixels and writing bf16 tokens. */
void hd_patchify_bf16(const float *img_dev, void *tok_dev, int C, int Hp,
                      int Wp, int p);

#ifdef __cplusplus
}
#endif

#endif /* HD_HIP_H */
