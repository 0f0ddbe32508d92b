/*
 * CPU oracle of the o1 decoder-block hot path. TEST INFRASTRUCTURE ONLY:
 * it is imported by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py, as the checker; the product path (libo1hip)
 * never links or calls it.
 *
 * An fp32 C restatement of the reference's per-block forward and its
 * primitives. Every function cites the reference file:line it follows.
 * Tensors are fp32 arrays holding bf16-exact values where the reference
 * holds bf16. `faithful` = 1 rounds to bf16 (RNE) at exactly the points the
 * reference rounds (block.c:245-349 chain of bf16 buffers); 0 keeps every
 * intermediate in fp32 (the "fp32 CPU reference" of the parity bound).
 *
 * Parity pins (see tests/test_oracle.py): closed forms and known-answer
 * tests of tests/unit/test_primitives.c and test_gemm_smoke.c, brute force
 * on tiny shapes, invariants (rotation norm, uniform/one-hot attention),
 * and torch CPU for the bf16 rounding rule. Composite block/forward parity
 * with the upstream PyTorch model is unpinned (no weights/oracle offline).
 */
#ifndef O1_ORACLE_H
#define O1_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

float o1o_bf16_round(float f);                       /* support.cu:21-28 */
void o1o_round_buf(float *x, size_t n);
int o1o_num_threads(void);
void o1o_set_threads(int n);

/* y[M,N] = x[M,K] . w[N,K]^T (+bias). mode 0: fp32; 1: bf16(acc[+bias]);
 * 2: bf16(bf16(acc) + bias) (production reference, gemm.cu:226-235). */
void o1o_linear(const float *x, const float *w, const float *bias, float *y, int M, int N, int K,
                int mode);
/* norm.cu:12-48 */
void o1o_rmsnorm(const float *x, const float *w, float *y, int rows, int cols, float eps, int round);
/* act.cu:13-34 */
void o1o_silu(const float *x, float *y, size_t n, int round);
void o1o_swiglu(const float *g, const float *u, float *y, size_t n, int round);
/* residual.cu:14-23 */
void o1o_residual_add(const float *x, const float *a, float *y, size_t n, int round);
/* rope.cu:28-71: cos/sin [seq, dim] from pos [3, seq] */
void o1o_mrope_cos_sin(const float *pos, int seq, const int64_t *section, int n_section, int dim,
                       float theta, float scaling, int interleaved, float *cosd, float *sind);
/* rope.cu:97-134 (per_op = 1) and :157-180 (per_op = 0), x [heads,seq,dim] */
void o1o_apply_rotary(const float *x, const float *cosd, const float *sind, float *y, int heads,
                      int seq, int dim, int per_op);
/* attn.cu:22-127 + hd_cudnn_sdpa split semantics. q [Hq,S,D], k/v [Hkv,S,D]
 * head-major; out [S, Hq*D] seq-major. mask: optional [S,S] additive; rows
 * < ar_len causal. prob_mode 0: fp32 probabilities; 1: normalised probs
 * rounded to bf16 before P.V (eager reference). round: bf16 output. */
void o1o_attention(const float *q, const float *k, const float *v, const float *mask, int Hq,
                   int Hkv, int S, int D, int ar_len, float scale, int prob_mode, int round,
                   float *out);
/* gemm.cu:531-545 */
void o1o_timestep_embed(const float *t, float *y, int N, int dim);

typedef struct {
    const float *q_proj, *k_proj, *v_proj, *o_proj, *input_ln, *post_ln, *gate_proj, *up_proj,
        *down_proj, *q_norm, *k_norm;
} o1o_block_weights;

typedef struct {
    int heads, kv_heads, hidden, ff, head_dim;
    float eps, theta, attention_scaling;
    int64_t section[3];
    int interleaved;
    int ar_len;
    int faithful;     /* 1: bf16 at the reference's rounding points */
    int prob_mode;    /* attention probabilities, see o1o_attention */
} o1o_block_cfg;

/* block.c:137-386 for `batch` sequences of `seq` tokens:
 * x [batch*seq, hidden] -> out [batch*seq, hidden]; pos [3, seq]; mask
 * optional [seq,seq]. Optional internals (NULL to skip), each
 * [batch*seq, hidden]: ln0, attn_resid, post_ln, delta = out - x (fp32). */
int o1o_decoder_block(const float *x, const float *pos, const float *mask,
                      const o1o_block_weights *w, const o1o_block_cfg *cfg, int batch, int seq,
                      float *out, float *ln0, float *attn_resid, float *post_ln);

typedef struct {
    const float *embed_tokens; int64_t vocab;
    const float *te0_w, *te0_b, *te2_w, *te2_b;
    const float *xe1_w, *xe2_w, *xe2_b;
    const float *fl_w, *fl_b, *fnorm_w;
    int n_layers;
    const o1o_block_weights *blocks;
} o1o_forward_weights;

/* forward.c:190-404 for one sequence: ids [T], vin [I,3072], t scalar,
 * pos [3,S], out [S,3072]. Optional after_blocks [n_layers][S,hidden]. */
int o1o_forward(const o1o_forward_weights *w, const o1o_block_cfg *cfg, const int64_t *ids, int T,
                const float *vin, int I, float t, const float *pos, const float *mask,
                int64_t tms_id, float *out, float *after_blocks);

/* o1o_forward with vision conditioning (forward.c:278-287, :363-370):
 * vmask [S] bytes, image_embeds [V, hidden], deepstack[3] [V, hidden]. */
int o1o_forward_visual(const o1o_forward_weights *w, const o1o_block_cfg *cfg, const int64_t *ids,
                       int T, const float *vin, int I, float t, const float *pos, const float *mask,
                       int64_t tms_id, const float *image_embeds, const float *const *deepstack,
                       const uint8_t *vmask, float *out, float *after_blocks);
/* lora_merge.cu:26-104: W = bf16(W + scale * up[N,R] @ down[R,K]) */
void o1o_lora_merge(float *w, const float *up, const float *down, int N, int K, int R, float scale);

/* sched.cu:50-72, :137-145 */
void o1o_sched_vcond(const float *z, const float *xp, float sigma, float *mo, int n);
void o1o_sched_flow_match_step(const float *z, const float *mo, float sigma, float sigma_next,
                               float *zn, int n);
void o1o_sched_cfg_guided(const float *c, const float *u, float g, float *o, int n);
/* sched.cu:160-263 FlowUniPC pointwise steps, with the fma placement the
 * device kernels state (a*b - c*d = fma(a, b, -(c*d)); x - a*b = fma(-a, b, x)) */
void o1o_unipc_convert(const float *smp, const float *mo, float sigma, float *conv, int n);
void o1o_unipc_correct(const float *last, const float *mo0, const float *mo_old, const float *conv,
                       float sig_t, float sig_s0, float alpha_t, float h_phi_1, float B_h,
                       float rc0, float rc1, float inv_rk, int order, float *out, int n);
void o1o_unipc_predict(const float *smp, const float *mo0, const float *mo_old, float sig_t,
                       float sig_s0, float alpha_t, float h_phi_1, float B_h, float rp,
                       float inv_rk, int order, float *out, int n);

/* generate.c:85-104 / decode.c:5-27 */
void o1o_patchify(const float *img, float *tok, int C, int Hp, int Wp, int p);
void o1o_unpatchify(const float *tok, float *img, int C, int Hp, int Wp, int p);
void o1o_decode_to_rgb(const float *z, int grid_h, int grid_w, int patch, int channels,
                       uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
