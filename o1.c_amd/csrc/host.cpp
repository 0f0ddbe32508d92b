// Host modules around the forward: torch CPU MT19937 noise, sigma schedules,
// the UniPC plan and CPU step, sequence tables, initial latent, RGB decode,
// and the device-side denoising loops.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "../../include/hd_hip.h"
#include "../../include/hd_host.h"

extern "C" void hd_fill_f32(float *dst, float value, int n);

// ---------------------------------------------------------------------------
// MT19937 (Matsumoto & Nishimura 1998) with torch's seeding and draw rules.
// ---------------------------------------------------------------------------
static const int MT_N = 624, MT_M = 397;

static void mt_regenerate(hd_torch_rng *g) {
    uint32_t *s = g->state;
    for (int k = 0; k < MT_N; k++) {
        uint32_t y = (s[k] & 0x80000000u) | (s[(k + 1) % MT_N] & 0x7fffffffu);
        uint32_t v = s[(k + MT_M) % MT_N] ^ (y >> 1);
        if (s[(k + 1) % MT_N] & 1u) v ^= 0x9908b0dfu;
        s[k] = v;
    }
    g->left_ = MT_N;
    g->next_ = 0;
}

extern "C" void hd_torch_rng_seed(hd_torch_rng *g, uint64_t seed) {
    memset(g, 0, sizeof(*g));
    g->seed_ = seed;
    g->seeded_ = 1;
    g->state[0] = (uint32_t)seed;
    for (int j = 1; j < MT_N; j++)
        g->state[j] = 1812433253u * (g->state[j - 1] ^ (g->state[j - 1] >> 30)) + (uint32_t)j;
    g->left_ = 1;     // the first draw regenerates the state (torch's rule)
    g->next_ = 0;
}

extern "C" uint32_t hd_torch_rng_u32(hd_torch_rng *g) {
    if (--g->left_ == 0) mt_regenerate(g);
    uint32_t y = g->state[g->next_++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

// uniform_real_distribution<float>: low 24 bits scaled by 2^-24
extern "C" float hd_torch_uniform_f32(hd_torch_rng *g) {
    return (float)(hd_torch_rng_u32(g) & 0xFFFFFFu) * (1.0f / 16777216.0f);
}

// Box-Muller over 16 uniforms: pairs (j, j + 8), angle in double then float.
static void box_muller16(float *d) {
    for (int j = 0; j < 8; j++) {
        const float u1 = 1.0f - d[j];
        const float u2 = d[j + 8];
        const float radius = sqrtf(-2.0f * logf(u1));
        const float theta = (float)(2.0 * M_PI * (double)u2);
        d[j] = radius * cosf(theta);
        d[j + 8] = radius * sinf(theta);
    }
}

extern "C" void hd_torch_randn_f32(hd_torch_rng *g, float *out, int64_t n) {
    if (n >= 16) {
        for (int64_t i = 0; i < n; i++) out[i] = hd_torch_uniform_f32(g);
        for (int64_t i = 0; i + 16 <= n; i += 16) box_muller16(out + i);
        if (n % 16) {
            float *tail = out + (n - 16);
            for (int j = 0; j < 16; j++) tail[j] = hd_torch_uniform_f32(g);
            box_muller16(tail);
        }
        return;
    }
    // n < 16: normal_distribution<double>, 53-bit uniforms from two words,
    // the sine sample cached for the next element
    bool have = false;
    double cached = 0.0;
    for (int64_t i = 0; i < n; i++) {
        if (have) {
            out[i] = (float)cached;
            have = false;
            continue;
        }
        uint64_t a = ((uint64_t)hd_torch_rng_u32(g) << 32) | hd_torch_rng_u32(g);
        uint64_t b = ((uint64_t)hd_torch_rng_u32(g) << 32) | hd_torch_rng_u32(g);
        const double u1 = (double)(a & ((1ull << 53) - 1)) / 9007199254740992.0;
        const double u2 = (double)(b & ((1ull << 53) - 1)) / 9007199254740992.0;
        const double r = sqrt(-2.0 * log1p(-u2));
        const double th = 2.0 * M_PI * u1;
        cached = r * sin(th);
        have = true;
        out[i] = (float)(r * cos(th));
    }
}

// ---------------------------------------------------------------------------
// Sigma schedules (scheduler.c:28-195): fp64 arithmetic, fp32 storage.
// ---------------------------------------------------------------------------
static const int DEV_TIMESTEPS[28] = {999, 987, 974, 960, 945, 929, 913, 895, 877, 857,
                                      836, 814, 790, 764, 737, 707, 675, 640, 602, 560,
                                      515, 464, 409, 347, 278, 199, 110, 8};

extern "C" hd_status hd_scheduler_init(hd_scheduler *s, const float *sigmas, int num_steps,
                                       float noise_clip_std) {
    if (!s || !sigmas || num_steps <= 0 || num_steps > HD_SCHED_MAX_STEPS) {
        hd_set_error("scheduler: bad init args");
        return HD_ERR_MISSING;
    }
    memset(s, 0, sizeof(*s));
    memcpy(s->sigmas, sigmas, sizeof(float) * num_steps);
    s->num_steps = num_steps;
    s->noise_clip_std = noise_clip_std;
    return HD_OK;
}

extern "C" float hd_scheduler_sigma(const hd_scheduler *s) {
    if (!s || s->step_index < 0 || s->step_index >= s->num_steps) return 0.0f;
    return s->sigmas[s->step_index];
}

extern "C" int hd_scheduler_derive_dev(hd_scheduler *s, float noise_clip_std) {
    if (!s) return 0;
    memset(s, 0, sizeof(*s));
    for (int i = 0; i < 28; i++) s->sigmas[i] = (float)DEV_TIMESTEPS[i] / 1000.0f;
    s->sigmas[28] = 0.0f;
    s->num_steps = 29;
    s->noise_clip_std = noise_clip_std;
    return 29;
}

static double shift_sigma(double sig, double sh) { return sh * sig / (1.0 + (sh - 1.0) * sig); }

// ramp sigma_max*1000 -> sigma_min*1000 in timestep space, shift applied;
// sigma_min is the shifted fp32 value of 1/1000 (the scheduler's init grid)
static int derive_ramp(hd_scheduler *s, int steps, float shift, float clip) {
    if (!s || steps < 2 || steps > HD_SCHED_MAX_STEPS - 1) {
        hd_set_error("scheduler: derive: bad steps");
        return 0;
    }
    memset(s, 0, sizeof(*s));
    const double sh = shift;
    const double min_raw = (double)(float)(1.0 / 1000.0);
    const double t_hi = 1000.0, t_lo = 1000.0 * shift_sigma(min_raw, sh);
    const double dt = (t_lo - t_hi) / (double)(steps - 1);
    for (int i = 0; i < steps; i++) s->sigmas[i] = (float)shift_sigma((t_hi + dt * i) / 1000.0, sh);
    s->sigmas[steps] = 0.0f;
    s->num_steps = steps + 1;
    s->noise_clip_std = clip;
    return steps + 1;
}
extern "C" int hd_scheduler_derive_flash(hd_scheduler *s, int steps, float shift, float clip) {
    return derive_ramp(s, steps, shift, clip);
}
extern "C" int hd_scheduler_derive_flow_match(hd_scheduler *s, int steps, float shift, float clip) {
    return derive_ramp(s, steps, shift, clip);
}

// linear in sigma space from the UniPC init grid's sigma_max down to 0,
// shift applied. sigma_max = 0.9996663928031921 is the value the upstream
// schedule dump (tests/unit/oracle_dump.txt, recipe default_full50)
// reproduces bit for bit; scheduler.c:179 names it in its comment but its
// code uses 0.9996664524078369, one fp32 ulp off on 21 of the 50 sigmas.
extern "C" int hd_scheduler_derive_default(hd_scheduler *s, int steps, float shift, float clip) {
    if (!s || steps < 1 || steps > HD_SCHED_MAX_STEPS - 1) {
        hd_set_error("scheduler: derive_default: bad steps");
        return 0;
    }
    memset(s, 0, sizeof(*s));
    const double smax = 0.9996663928031921, smin = 0.0, sh = shift;
    const double d = (smin - smax) / (double)steps;
    for (int i = 0; i < steps; i++) s->sigmas[i] = (float)shift_sigma(smax + d * i, sh);
    s->sigmas[steps] = 0.0f;
    s->num_steps = steps + 1;
    s->noise_clip_std = clip;
    return steps + 1;
}

extern "C" float hd_scheduler_noise_scale(const hd_scheduler *s, int step_index, float start,
                                          float end) {
    int n = (s && s->num_steps > 1) ? s->num_steps - 1 : 1;
    if (n <= 1) return start;
    if (step_index < 0) step_index = 0;
    if (step_index >= n) step_index = n - 1;
    return start + (end - start) * (float)step_index / (float)(n - 1);
}

extern "C" hd_status hd_scheduler_step(hd_scheduler *s, const void *z, const float *mo,
                                       const float *noise, float s_noise, void *z_next, int n,
                                       float *scratch) {
    if (!s || !z || !mo || !noise || !z_next || !scratch || n <= 0) {
        hd_set_error("scheduler: null argument");
        return HD_ERR_MISSING;
    }
    if (s->step_index < 0 || s->step_index >= s->num_steps - 1) {
        hd_set_error("scheduler: step_index out of range");
        return HD_ERR_MISSING;
    }
    const float sg = s->sigmas[s->step_index], sn = s->sigmas[s->step_index + 1];
    float *zf = scratch, *den = scratch + n, *zn = scratch + 2 * (size_t)n;
    hd_cuda_clear_error();
    hd_sched_bf16_upcast(z, zf, n);
    hd_sched_denoised(zf, mo, sg, den, n);
    hd_sched_z_next(noise, den, sn, s_noise, zn, n);
    hd_f32_convert_bf16(zn, z_next, n);
    if (hd_cuda_last_error()[0]) {
        hd_set_error("scheduler: %s", hd_cuda_last_error());
        return HD_ERR_RUNTIME;
    }
    s->step_index++;
    return HD_OK;
}

// ---------------------------------------------------------------------------
// FlowUniPC (UniPC, Zhao et al. 2023; bh2 variant, data prediction, order 2)
// in the flow parametrisation alpha = 1 - sigma, lambda = log(alpha/sigma).
// The arithmetic order follows scheduler.c:215-330 so the fp64 scalars agree
// bit for bit; everything here runs on the host.
// ---------------------------------------------------------------------------
static double unipc_lambda(double sigma) { return log(1.0 - sigma) - log(sigma); }

// rho for the order-2 corrector: solve [[1, 1], [rk, 1]] x = [b0, b1]
// (scheduler.c:16-23, :264-274); the singular case keeps rho = (0, 0.5)
static void unipc_rhos_c(double hh, double phi, double B, double rk, double *r0, double *r1) {
    double k1 = phi / hh - 1.0;
    const double b0 = k1 * 1.0 / B;
    k1 = k1 / hh - 1.0 / 2.0;
    const double b1 = k1 * 2.0 / B;
    const double det = 1.0 * 1.0 - 1.0 * rk;
    if (det == 0.0) {
        *r0 = 0.0;
        *r1 = 0.5;
        return;
    }
    *r0 = (b0 * 1.0 - 1.0 * b1) / det;
    *r1 = (1.0 * b1 - b0 * rk) / det;
}

extern "C" void hd_scheduler_unipc_plan(const hd_scheduler *s, int si, int this_order,
                                        int lower_order_nums, hd_unipc_plan *plan) {
    if (!s || !plan) return;
    memset(plan, 0, sizeof(*plan));
    const int n_inf = s->num_steps - 1;
    if (si < 0 || si >= n_inf) return;
    if (si > 0 && this_order > 0) {
        // corrector: refines the sample of step si with the new model output
        const int co = this_order >= 2 ? 2 : 1;
        const double st = s->sigmas[si], s0 = s->sigmas[si - 1];
        const double h = unipc_lambda(st) - unipc_lambda(s0), hh = -h;
        const double phi = expm1(hh), B = expm1(hh);
        double rk = 1.0, r0 = 0.0, r1 = 0.5;
        if (co == 2) {
            const double sm = si - 2 >= 0 ? (double)s->sigmas[si - 2] : (double)s->sigmas[0];
            rk = (unipc_lambda(sm) - unipc_lambda(s0)) / h;
            unipc_rhos_c(hh, phi, B, rk, &r0, &r1);
        }
        plan->corr_order = co;
        plan->c_sig_t = st;
        plan->c_sig_s0 = s0;
        plan->c_alpha_t = 1.0 - st;
        plan->c_h_phi_1 = phi;
        plan->c_B_h = B;
        plan->c_rhos0 = r0;
        plan->c_rhos1 = r1;
        plan->c_inv_rks0 = rk == 0.0 ? 0.0 : 1.0 / rk;
    }
    // predictor: order min(2, steps left) during warm-up limited to
    // lower_order_nums + 1 (lower_order_final)
    int po = n_inf - si < 2 ? n_inf - si : 2;
    if (po > lower_order_nums + 1) po = lower_order_nums + 1;
    if (po < 1) po = 1;
    const double st = s->sigmas[si + 1], s0 = s->sigmas[si];
    const double h = unipc_lambda(st) - unipc_lambda(s0), hh = -h;
    const double phi = expm1(hh), B = expm1(hh);
    double rk = 1.0, rp = 0.0;
    if (po == 2) {
        const double sm = si - 1 >= 0 ? (double)s->sigmas[si - 1] : (double)s->sigmas[0];
        rk = (unipc_lambda(sm) - unipc_lambda(s0)) / h;
        if (rk != 0.0) rp = 0.5;
    }
    plan->pred_order = po;
    plan->p_sig_t = st;
    plan->p_sig_s0 = s0;
    plan->p_alpha_t = 1.0 - st;
    plan->p_h_phi_1 = phi;
    plan->p_B_h = B;
    plan->p_rhos_p = rp;
    plan->p_inv_rks0 = rk == 0.0 ? 0.0 : 1.0 / rk;
    plan->next_this_order = po;
    plan->next_lower_order = lower_order_nums < 2 ? lower_order_nums + 1 : lower_order_nums;
}

extern "C" hd_status hd_scheduler_unipc_step(const hd_scheduler *s, hd_scheduler_unipc *u,
                                             const float *mo, const float *sample, float *prev,
                                             int n, float *scratch) {
    if (!s || !u || !mo || !sample || !prev || !scratch || n <= 0) {
        hd_set_error("scheduler: unipc: null argument");
        return HD_ERR_MISSING;
    }
    const int si = u->step_index;
    if (si < 0 || si >= s->num_steps - 1) {
        hd_set_error("scheduler: unipc: step_index out of range");
        return HD_ERR_MISSING;
    }
    float *m_new = u->model_outputs[HD_UNIPC_ORDER - 1], *m_old = u->model_outputs[0];
    if (!m_new || !u->last_sample) {
        hd_set_error("scheduler: unipc: history not initialized");
        return HD_ERR_MISSING;
    }
    // converted model output (data prediction): x0 = sample - sigma * mo
    float *conv = scratch;
    const float sc = s->sigmas[si];
    for (int j = 0; j < n; j++) {
        const float p = sc * mo[j];
        conv[j] = sample[j] - p;
    }
    for (int j = 0; j < n; j++) prev[j] = sample[j];
    // The reference's CPU step keeps rk = 1 (its rks[0]) where the per-step
    // plan uses rk = (lambda_prev - lambda_s0) / h: the order-2 corrector's
    // 2x2 system is then singular and keeps rho = (0, 0.5), and the order-2
    // predictor's difference is not divided by rk (scheduler.c:305-380).
    // hd_denoise follows the plan, as generate.c's production loop does.
    const double rk_cpu = 1.0;
    if (si > 0 && u->has_last_sample && u->this_order > 0) {
        // UniC: the sample of this step from last_sample, using conv_{t-1}
        // (m_new, before the shift) and conv_{t-2} (m_old)
        const int order = u->this_order;
        const double st = s->sigmas[si], s0 = s->sigmas[si - 1];
        const double h = unipc_lambda(st) - unipc_lambda(s0), hh = -h;
        const double phi = expm1(hh), B = expm1(hh), at = 1.0 - st;
        double r0 = 0.0, r1 = 0.5;
        if (order == 2) unipc_rhos_c(hh, phi, B, rk_cpu, &r0, &r1);
        const double scale = st / s0, coef = at * phi;
        for (int j = 0; j < n; j++)
            prev[j] = (float)(scale * (double)u->last_sample[j] - coef * (double)m_new[j]);
        if (order == 2) {
            const double inv = 1.0 / rk_cpu, bc = at * B;
            for (int j = 0; j < n; j++) {
                const double d1 = ((double)m_old[j] - (double)m_new[j]) * inv;
                const double d1t = (double)conv[j] - (double)m_new[j];
                prev[j] = (float)((double)prev[j] - bc * (r0 * d1 + r1 * d1t));
            }
        } else {
            const double bc = at * B * 0.5;
            for (int j = 0; j < n; j++)
                prev[j] = (float)((double)prev[j] - bc * ((double)conv[j] - (double)m_new[j]));
        }
    }
    // history: oldest <- newest <- conv
    for (int i = 0; i < HD_UNIPC_ORDER - 1; i++)
        memcpy(u->model_outputs[i], u->model_outputs[i + 1], (size_t)n * sizeof(float));
    memcpy(m_new, conv, (size_t)n * sizeof(float));
    int order = s->num_steps - 1 - si < HD_UNIPC_ORDER ? s->num_steps - 1 - si : HD_UNIPC_ORDER;
    if (order > u->lower_order_nums + 1) order = u->lower_order_nums + 1;
    u->this_order = order;
    memcpy(u->last_sample, prev, (size_t)n * sizeof(float));
    u->has_last_sample = 1;
    {
        // UniP from the (corrected) sample in prev, in place
        const double st = s->sigmas[si + 1], s0 = s->sigmas[si];
        const double h = unipc_lambda(st) - unipc_lambda(s0), hh = -h;
        const double phi = expm1(hh), B = expm1(hh), at = 1.0 - st;
        const float *m0 = u->model_outputs[HD_UNIPC_ORDER - 1];
        const double scale = st / s0, coef = at * phi;
        for (int j = 0; j < n; j++)
            prev[j] = (float)(scale * (double)prev[j] - coef * (double)m0[j]);
        if (order == 2) {
            const float *m1 = u->model_outputs[HD_UNIPC_ORDER - 2];
            const double inv = 1.0 / rk_cpu, bc = at * B * 0.5;
            for (int j = 0; j < n; j++) {
                const double d1 = ((double)m1[j] - (double)m0[j]) * inv;
                prev[j] = (float)((double)prev[j] - bc * d1);
            }
        }
    }
    if (u->lower_order_nums < HD_UNIPC_ORDER) u->lower_order_nums++;
    u->step_index++;
    return HD_OK;
}

extern "C" void hd_step_noise(hd_torch_rng *rng, float *out, int64_t n, float clip) {
    if (!rng || !out || n <= 0) return;
    hd_torch_randn_f32(rng, out, n);
    if (clip <= 0.0f) return;
    double mean = 0.0, m2 = 0.0;
    for (int64_t k = 0; k < n; k++) mean += out[k];
    mean /= (double)n;
    for (int64_t k = 0; k < n; k++) {
        const double d = (double)out[k] - mean;
        m2 += d * d;
    }
    const double sd = sqrt(m2 / (double)(n - 1));
    const float cv = clip * (float)sd;
    for (int64_t k = 0; k < n; k++) {
        if (out[k] > cv) out[k] = cv;
        else if (out[k] < -cv) out[k] = -cv;
    }
}

// ---------------------------------------------------------------------------
// Sequence tables
// ---------------------------------------------------------------------------
extern "C" hd_status hd_seq_t2i_positions(int text_len, int gh, int gw, int fix_point, float *pos) {
    if (!pos || text_len < 0 || gh <= 0 || gw <= 0) {
        hd_set_error("sequence: bad args");
        return HD_ERR_MISSING;
    }
    const int S = text_len + gh * gw;
    for (int i = 0; i < text_len; i++) pos[i] = pos[S + i] = pos[2 * S + i] = (float)i;
    for (int r = 0; r < gh; r++)
        for (int c = 0; c < gw; c++) {
            int k = text_len + r * gw + c;
            pos[k] = (float)fix_point;
            pos[S + k] = (float)(fix_point + r);
            pos[2 * S + k] = (float)(fix_point + c);
        }
    return HD_OK;
}

extern "C" hd_status hd_seq_t2i_mask(int text_len, int S, uint16_t *mask) {
    if (!mask || text_len < 0 || S <= 0 || text_len > S) {
        hd_set_error("sequence: bad mask args");
        return HD_ERR_MISSING;
    }
    const int causal_rows = text_len > 0 ? text_len - 1 : 0;
    for (int r = 0; r < S; r++)
        for (int c = 0; c < S; c++)
            mask[(size_t)r * S + c] = (r < causal_rows && c > r) ? (uint16_t)0xFF7F : (uint16_t)0;
    return HD_OK;
}

extern "C" int hd_seq_grid_positions(int n_text, int n_seg, const int *gh, const int *gw,
                                     const int *row_off, const int *col_off, float base,
                                     float *pos) {
    if (!pos || n_text < 0 || n_seg < 0 || (n_seg && (!gh || !gw))) return -1;
    int S = n_text;
    for (int i = 0; i < n_seg; i++) S += gh[i] * gw[i];
    int k = 0;
    for (; k < n_text; k++) pos[k] = pos[S + k] = pos[2 * S + k] = base;
    for (int i = 0; i < n_seg; i++)
        for (int r = 0; r < gh[i]; r++)
            for (int c = 0; c < gw[i]; c++, k++) {
                pos[k] = base;
                pos[S + k] = base + (float)(r + (row_off ? row_off[i] : 0));
                pos[2 * S + k] = base + (float)(c + (col_off ? col_off[i] : 0));
            }
    return S;
}

// ---------------------------------------------------------------------------
// Initial latent and decode
// ---------------------------------------------------------------------------
extern "C" void hd_initial_noise(uint64_t seed, int width, int height, float *out) {
    hd_torch_rng g;
    hd_torch_rng_seed(&g, seed + 1);
    hd_torch_randn_f32(&g, out, (int64_t)3 * height * width);
}

extern "C" void hd_pixel_unshuffle(const float *img, int C, int H, int W, int p, float *tok) {
    const int gh = H / p, gw = W / p;
    const size_t F = (size_t)C * p * p;
    for (int r = 0; r < gh; r++)
        for (int c = 0; c < gw; c++)
            for (int ch = 0; ch < C; ch++)
                for (int i = 0; i < p; i++)
                    for (int j = 0; j < p; j++)
                        tok[((size_t)r * gw + c) * F + (size_t)ch * p * p + (size_t)i * p + j] =
                            img[((size_t)ch * H + (size_t)(r * p + i)) * W + (size_t)(c * p + j)];
}

extern "C" void hd_decode_to_rgb(const float *z, int gh, int gw, int p, int C, unsigned char *out) {
    const size_t F = (size_t)C * p * p, wpx = (size_t)gw * p;
    for (int t = 0; t < gh * gw; t++) {
        const int tr = t / gw, tc = t % gw;
        for (int ch = 0; ch < C; ch++)
            for (int i = 0; i < p; i++)
                for (int j = 0; j < p; j++) {
                    float v = (z[(size_t)t * F + (size_t)ch * p * p + (size_t)i * p + j] + 1.0f) / 2.0f;
                    float px = roundf(v * 255.0f);
                    px = px < 0.0f ? 0.0f : (px > 255.0f ? 255.0f : px);
                    out[((size_t)(tr * p + i) * wpx + (size_t)(tc * p + j)) * C + ch] = (unsigned char)px;
                }
    }
}

// ---------------------------------------------------------------------------
// Flow-match Euler + CFG denoising loop (device resident)
// ---------------------------------------------------------------------------
static inline int64_t al256(int64_t x) { return (x + 255) & ~(int64_t)255; }
static const float kTEps = 1e-6f;   // sigma floor of the velocity division (generate.c:64)

// ---------------------------------------------------------------------------
// Final-latent check. The reference's generate fails closed on the raw output
// latent (generate.c:1474-1496): any NaN/Inf, or a value outside [-2, 2],
// sets the error and returns its failure status (generate.c:1546). The
// loops below run the same check after their last step: mode 2 (default) is
// the reference's check, 1 keeps only the NaN/Inf test (random-weight runs
// leave the [-2, 2] range), 0 switches it off.
// ---------------------------------------------------------------------------
extern "C" void hd_latent_stats(const void *z, int64_t n, float *part, int blocks);
static constexpr int kLatentStatBlocks = 256;
static std::atomic<int> g_output_check{2};

extern "C" int hd_denoise_set_output_check(int mode) {
    if (mode < 0 || mode > 2) return -1;
    return g_output_check.exchange(mode);
}

static int64_t latent_check_bytes() { return al256((int64_t)kLatentStatBlocks * 3 * 4); }

// z: [n] bf16 on the device; part: device scratch of latent_check_bytes()
static hd_status check_final_latent(const void *z, int64_t n, float *part, hipStream_t st) {
    const int mode = g_output_check.load();
    if (mode == 0 || n <= 0) return HD_OK;
    const int64_t want = (n + 2047) / 2048;
    const int blocks = (int)(want < kLatentStatBlocks ? want : kLatentStatBlocks);
    hd_cuda_clear_error();
    hd_latent_stats(z, n, part, blocks);
    float h[kLatentStatBlocks * 3];
    if (hd_cuda_last_error()[0] ||
        hipMemcpyAsync(h, part, (size_t)blocks * 3 * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        hd_set_error("denoise: final latent check failed to run");
        return HD_ERR_RUNTIME;
    }
    float bad = 0.f, mn = INFINITY, mx = -INFINITY;
    for (int b = 0; b < blocks; b++) {
        bad += h[3 * b];
        mn = fminf(mn, h[3 * b + 1]);
        mx = fmaxf(mx, h[3 * b + 2]);
    }
    if (bad > 0.f) {
        hd_set_error("denoise: final latent contains NaN/Inf");
        return HD_ERR_MISSING;   // generate.c's failure status (generate.c:1546)
    }
    if (mode == 2 && (mn < -2.0f || mx > 2.0f)) {
        hd_set_error("denoise: final latent range [%.4f, %.4f] out of bounds", mn, mx);
        return HD_ERR_MISSING;
    }
    return HD_OK;
}

extern "C" int64_t hd_denoise_scratch_bytes(int seq, int img, int steps) {
    const int64_t n = (int64_t)img * 3072;
    return al256(2 * n * 2)                       // vin [2, I, 3072] bf16
           + al256((int64_t)2 * seq * 3072 * 2)   // x_pred [2, S, 3072] bf16
           + al256(3 * n * 4)                     // mo_c, mo_u, mo fp32
           + al256((int64_t)(steps + 1) * 2 * 4)  // t pairs
           + latent_check_bytes();                // final-latent check partials
}

extern "C" hd_status hd_denoise_euler_cfg(const hd_forward_binding *bw, hd_forward_workspace *ws,
                                          const int64_t *ids, int T, const float *pos, int ar_len,
                                          void *z, int I, const float *sigmas, int steps,
                                          float guidance, int S, int H, int KV, int HID, int FF,
                                          int D, int tms, void *scratch, int64_t scratch_bytes,
                                          void *stream) {
    if (!bw || !ws || !pos || !z || !sigmas || !scratch || steps < 1 || I <= 0) {
        hd_set_error("denoise: null argument");
        return HD_ERR_MISSING;
    }
    if (scratch_bytes < hd_denoise_scratch_bytes(S, I, steps)) {
        hd_set_error("denoise: scratch too small");
        return HD_ERR_OOM;
    }
    void *prev = hd_hip_get_stream();
    if (stream) hd_hip_set_stream(stream);
    hipStream_t st = (hipStream_t)hd_hip_get_stream();
    const int64_t n = (int64_t)I * 3072;
    char *p = (char *)scratch;
    uint16_t *vin = (uint16_t *)p; p += al256(2 * n * 2);
    uint16_t *xp = (uint16_t *)p; p += al256((int64_t)2 * S * 3072 * 2);
    float *mo_c = (float *)p, *mo_u = mo_c + n, *mo = mo_u + n; p += al256(3 * n * 4);
    float *tdev = (float *)p; p += al256((int64_t)(steps + 1) * 2 * 4);
    float *chk = (float *)p;
    hd_status status = HD_OK;
    if (steps > HD_SCHED_MAX_STEPS) {
        hd_set_error("denoise: too many steps");
        status = HD_ERR_UNSUPPORTED;
    }
    // per-step timestep pairs (t = 1 - sigma for both rows, generate.c:1315),
    // written by a fill kernel: the values travel as kernel arguments, no
    // host buffer outlives the call
    for (int i = 0; status == HD_OK && i < steps; i++) hd_fill_f32(tdev + 2 * i, 1.0f - sigmas[i], 2);
    for (int i = 0; status == HD_OK && i < steps; i++) {
        const float sg = sigmas[i] < kTEps ? kTEps : sigmas[i], sn = sigmas[i + 1];
        for (int b = 0; b < 2 && status == HD_OK; b++)
            if (hipMemcpyAsync(vin + b * n, z, n * 2, hipMemcpyDeviceToDevice, st) != hipSuccess) {
                hd_set_error("denoise: latent copy failed");
                status = HD_ERR_IO;
            }
        if (status != HD_OK) break;
        status = hd_forward_batched(bw, ws, 2, ids, T, pos, ar_len, vin, I, tdev + 2 * i, S, H, KV,
                                    HID, FF, D, tms, nullptr, xp, nullptr);
        if (status != HD_OK) break;
        hd_cuda_clear_error();
        hd_sched_vcond(z, xp + (size_t)T * 3072, sg, mo_c, (int)n);
        hd_sched_vcond(z, xp + ((size_t)S + T) * 3072, sg, mo_u, (int)n);
        hd_sched_cfg_guided(mo_c, mo_u, guidance, mo, (int)n);
        hd_sched_flow_match_step(z, mo, sigmas[i], sn, z, (int)n);
        if (hd_cuda_last_error()[0]) {
            hd_set_error("denoise: %s", hd_cuda_last_error());
            status = HD_ERR_RUNTIME;
        }
    }
    if (status == HD_OK) status = check_final_latent(z, n, chk, st);
    hd_hip_set_stream(prev);
    return status;
}

// ---------------------------------------------------------------------------
// hd_denoise: Euler / flash SDE / UniPC samplers, optional CFG (batch 2)
// ---------------------------------------------------------------------------
extern "C" int64_t hd_denoise_run_scratch_bytes(int B, int S, int I, int steps) {
    const int64_t n = (int64_t)I * 3072;
    return al256((int64_t)B * n * 2)                 // vin [B, I, 3072] bf16
           + al256((int64_t)B * S * 3072 * 2)        // x_pred [B, S, 3072] bf16
           + al256(3 * n * 4)                        // mo_c, mo_u, mo
           + al256(7 * n * 4)                        // sampler state (UniPC: z, 3 conv slots,
                                                     // last, corrected, predicted; flash: noise
                                                     // + the step's 3n scratch)
           + al256((int64_t)(steps + 1) * B * 4)     // timesteps
           + latent_check_bytes();                   // final-latent check partials
}

namespace {
struct PinnedNoise {
    float *buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    ~PinnedNoise() {
        for (int k = 0; k < 2; k++) {
            if (done[k]) {
                (void)hipEventSynchronize(done[k]);
                (void)hipEventDestroy(done[k]);
            }
            if (buf[k]) (void)hipHostFree(buf[k]);
        }
    }
};
}  // namespace

// The unconditional branch of a guided loop when it is its own sequence
// (generate.c:1075, :1119-1120, :1341: the " " caption gives it a shorter
// text and its own positions, mask and workspace).
struct UncondSeq {
    hd_forward_workspace *ws;
    const int64_t *ids;
    int T, ar_len, S;
    const float *pos;
};

// Shared loop of hd_denoise / hd_denoise_cfg / hd_denoise_visual. I_t target rows are
// denoised; with n_ref reference rows the forward sees I_t + n_ref image
// tokens (target first), the references either as patches copied once after
// the target rows (`ref`) or as cached x_embedder rows (ws->xe_ref).
static hd_status denoise_loop(const hd_forward_binding *bw, hd_forward_workspace *ws, int sampler,
                              const hd_scheduler *sched, int steps, int B, const int64_t *ids,
                              int T, const float *pos, int ar_len, const void *mask,
                              const hd_visual_cond *vis, void *z, int I_t, const void *ref,
                              int n_ref, float guidance, uint64_t seed, float sn_start,
                              float sn_end, float clip, int S, int H, int KV, int HID, int FF,
                              int D, int tms, void *scratch, int64_t scratch_bytes, void *stream,
                              const UncondSeq *u = nullptr) {
    const int I = I_t + n_ref;
    if (steps > sched->num_steps - 1) {
        hd_set_error("denoise: %d steps but the schedule has %d sigmas", steps, sched->num_steps);
        return HD_ERR_UNSUPPORTED;
    }
    // a separate unconditional sequence: x_pred rows for the longer of the two
    const int S_rows = u && u->S > S ? u->S : S;
    if (scratch_bytes < hd_denoise_run_scratch_bytes(B, S_rows, I, steps)) {
        hd_set_error("denoise: scratch too small");
        return HD_ERR_OOM;
    }
    const int64_t n = (int64_t)I_t * 3072;
    char *p = (char *)scratch;
    uint16_t *vin = (uint16_t *)p; p += al256((int64_t)B * I * 3072 * 2);
    uint16_t *xp = (uint16_t *)p; p += al256((int64_t)B * S_rows * 3072 * 2);
    uint16_t *xp_u = xp + (size_t)S_rows * 3072;
    float *mo_c = (float *)p, *mo_u = mo_c + n, *mo = mo_u + n; p += al256(3 * n * 4);
    float *st = (float *)p; p += al256(7 * n * 4);
    float *tdev = (float *)p; p += al256((int64_t)(steps + 1) * B * 4);
    float *chk = (float *)p;

    PinnedNoise pn;
    hd_torch_rng rng;
    if (sampler == HD_SAMPLER_FLASH) {
        for (int k = 0; k < 2; k++)
            if (hipHostMalloc((void **)&pn.buf[k], n * sizeof(float), hipHostMallocDefault) !=
                    hipSuccess ||
                hipEventCreateWithFlags(&pn.done[k], hipEventDisableTiming) != hipSuccess) {
                hd_set_error("denoise: pinned noise staging failed");
                return HD_ERR_OOM;
            }
        hd_torch_rng_seed(&rng, seed + 1);   // generate.c:1295-1296
    }

    void *prev_stream = hd_hip_get_stream();
    if (stream) hd_hip_set_stream(stream);
    hipStream_t hs = (hipStream_t)hd_hip_get_stream();
    hd_status status = HD_OK;
    for (int i = 0; i < steps; i++) hd_fill_f32(tdev + (size_t)B * i, 1.0f - sched->sigmas[i], B);
    // reference patches stay put behind the target rows for every step
    if (ref && hipMemcpyAsync(vin + n, ref, (size_t)n_ref * 3072 * 2, hipMemcpyDeviceToDevice, hs) !=
                   hipSuccess) {
        hd_set_error("denoise: reference copy failed");
        status = HD_ERR_IO;
    }

    // UniPC state: converted outputs rotate through three slots
    float *zf = st, *slot[3] = {st + n, st + 2 * n, st + 3 * n};
    float *last = st + 4 * n, *corr_buf = st + 5 * n, *pred = st + 6 * n;
    int this_order = 0, lower = 0, have_hist = 0;
    hd_scheduler fs = *sched;   // flash: step_index walks with i

    for (int i = 0; status == HD_OK && i < steps; i++) {
        const float sig = sched->sigmas[i];
        const float sg = sig < kTEps ? kTEps : sig;
        const void *vptr = z;
        if (ref) {
            if (hipMemcpyAsync(vin, z, n * 2, hipMemcpyDeviceToDevice, hs) != hipSuccess) {
                hd_set_error("denoise: latent copy failed");
                status = HD_ERR_IO;
            }
            vptr = vin;
        } else if (B == 2 && !u) {
            for (int b = 0; b < 2 && status == HD_OK; b++)
                if (hipMemcpyAsync(vin + b * n, z, n * 2, hipMemcpyDeviceToDevice, hs) != hipSuccess) {
                    hd_set_error("denoise: latent copy failed");
                    status = HD_ERR_IO;
                }
            vptr = vin;
        }
        if (status != HD_OK) break;
        if (B == 1 && (vis || mask || n_ref))
            status = hd_forward(bw, ws, ids, T, pos, mask, vptr, I, vis, tdev + i, nullptr, S, H, KV,
                                HID, FF, D, tms, nullptr, xp, nullptr);
        else if (u)   // cond and uncond as two sequences of their own lengths
            status = hd_forward_batched(bw, ws, 1, ids, T, pos, ar_len, z, I, tdev + (size_t)B * i,
                                        S, H, KV, HID, FF, D, tms, nullptr, xp, nullptr);
        else
            status = hd_forward_batched(bw, ws, B, ids, T, pos, ar_len, vptr, I,
                                        tdev + (size_t)B * i, S, H, KV, HID, FF, D, tms, nullptr, xp,
                                        nullptr);
        if (status == HD_OK && u)
            status = hd_forward_batched(bw, u->ws, 1, u->ids, u->T, u->pos, u->ar_len, z, I,
                                        tdev + (size_t)B * i + 1, u->S, H, KV, HID, FF, D, tms,
                                        nullptr, xp_u, nullptr);
        if (status != HD_OK) break;
        hd_cuda_clear_error();
        hd_sched_vcond(z, xp + (size_t)T * 3072, sg, mo_c, (int)n);
        const float *m = mo_c;
        if (B == 2) {
            const uint16_t *xu = u ? xp_u + (size_t)u->T * 3072 : xp + ((size_t)S + T) * 3072;
            hd_sched_vcond(z, xu, sg, mo_u, (int)n);
            hd_sched_cfg_guided(mo_c, mo_u, guidance, mo, (int)n);
            m = mo;
        }
        if (sampler == HD_SAMPLER_EULER) {
            hd_sched_flow_match_step(z, m, sig, sched->sigmas[i + 1], z, (int)n);
        } else if (sampler == HD_SAMPLER_FLASH) {
            // the host draws this step's noise while the forward runs; the
            // staging buffer is reused only after its previous copy is done
            const int k = i & 1;
            if (i >= 2) (void)hipEventSynchronize(pn.done[k]);
            hd_step_noise(&rng, pn.buf[k], n, clip);
            float *noise_dev = st;
            if (hipMemcpyAsync(noise_dev, pn.buf[k], n * sizeof(float), hipMemcpyHostToDevice, hs) !=
                    hipSuccess ||
                hipEventRecord(pn.done[k], hs) != hipSuccess) {
                hd_set_error("denoise: noise upload failed");
                status = HD_ERR_IO;
                break;
            }
            fs.step_index = i;
            const float s_noise = hd_scheduler_noise_scale(sched, i, sn_start, sn_end);
            status = hd_scheduler_step(&fs, z, m, noise_dev, s_noise, z, (int)n, st + n);
        } else {
            hd_unipc_plan pl;
            hd_scheduler_unipc_plan(sched, i, this_order, lower, &pl);
            hd_sched_bf16_upcast(z, zf, (int)n);
            float *cur = slot[0];
            hd_unipc_convert(zf, m, sig, cur, (int)n);
            const float *corr = zf;
            if (i > 0 && this_order > 0 && have_hist) {
                hd_unipc_correct(last, slot[1], slot[2], cur, (float)pl.c_sig_t, (float)pl.c_sig_s0,
                                 (float)pl.c_alpha_t, (float)pl.c_h_phi_1, (float)pl.c_B_h,
                                 (float)pl.c_rhos0, (float)pl.c_rhos1, (float)pl.c_inv_rks0,
                                 pl.corr_order, corr_buf, (int)n);
                corr = corr_buf;
            }
            if (hipMemcpyAsync(last, corr, n * sizeof(float), hipMemcpyDeviceToDevice, hs) !=
                hipSuccess) {
                hd_set_error("denoise: unipc state copy failed");
                status = HD_ERR_IO;
                break;
            }
            hd_unipc_predict(corr, cur, slot[1], (float)pl.p_sig_t, (float)pl.p_sig_s0,
                             (float)pl.p_alpha_t, (float)pl.p_h_phi_1, (float)pl.p_B_h,
                             (float)pl.p_rhos_p, (float)pl.p_inv_rks0, pl.pred_order, pred, (int)n);
            hd_f32_convert_bf16(pred, z, (int)n);
            // conv_t -> slot 1, conv_{t-1} -> slot 2, the oldest buffer is reused
            float *oldest = slot[2];
            slot[2] = slot[1];
            slot[1] = slot[0];
            slot[0] = oldest;
            this_order = pl.next_this_order;
            lower = pl.next_lower_order;
            have_hist = 1;
        }
        if (status == HD_OK && hd_cuda_last_error()[0]) {
            hd_set_error("denoise: %s", hd_cuda_last_error());
            status = HD_ERR_RUNTIME;
        }
    }
    if (status == HD_OK) status = check_final_latent(z, n, chk, hs);
    hd_hip_set_stream(prev_stream);
    return status;
}

extern "C" hd_status hd_denoise(const hd_forward_binding *bw, hd_forward_workspace *ws, int sampler,
                                const hd_scheduler *sched, int steps, int B, const int64_t *ids,
                                int T, const float *pos, int ar_len, void *z, int I,
                                float guidance, uint64_t seed, float sn_start, float sn_end,
                                float clip, int S, int H, int KV, int HID, int FF, int D, int tms,
                                void *scratch, int64_t scratch_bytes, void *stream) {
    if (!bw || !ws || !sched || !ids || !pos || !z || !scratch || I <= 0 || steps < 1) {
        hd_set_error("denoise: null argument");
        return HD_ERR_MISSING;
    }
    if ((B != 1 && B != 2) || sampler < HD_SAMPLER_EULER || sampler > HD_SAMPLER_UNIPC) {
        hd_set_error("denoise: batch must be 1 or 2 and sampler 0..2");
        return HD_ERR_UNSUPPORTED;
    }
    return denoise_loop(bw, ws, sampler, sched, steps, B, ids, T, pos, ar_len, nullptr, nullptr, z,
                        I, nullptr, 0, guidance, seed, sn_start, sn_end, clip, S, H, KV, HID, FF, D,
                        tms, scratch, scratch_bytes, stream);
}

extern "C" int64_t hd_denoise_cfg_scratch_bytes(int seq, int seq_uncond, int img_tokens,
                                                int steps) {
    return hd_denoise_run_scratch_bytes(2, seq > seq_uncond ? seq : seq_uncond, img_tokens, steps);
}

extern "C" hd_status hd_denoise_cfg(const hd_forward_binding *bw, hd_forward_workspace *ws,
                                    hd_forward_workspace *ws_uncond, int sampler,
                                    const hd_scheduler *sched, int steps, const int64_t *ids, int T,
                                    const float *pos, int ar_len, int S, const int64_t *ids_uncond,
                                    int T_uncond, const float *pos_uncond, int ar_len_uncond,
                                    int S_uncond, void *z, int I, float guidance, uint64_t seed,
                                    float sn_start, float sn_end, float clip, int H, int KV,
                                    int HID, int FF, int D, int tms, void *scratch,
                                    int64_t scratch_bytes, void *stream) {
    if (!bw || !ws || !ws_uncond || !sched || !ids || !pos || !ids_uncond || !pos_uncond || !z ||
        !scratch || I <= 0 || steps < 1) {
        hd_set_error("denoise_cfg: null argument");
        return HD_ERR_MISSING;
    }
    if (sampler < HD_SAMPLER_EULER || sampler > HD_SAMPLER_UNIPC) {
        hd_set_error("denoise_cfg: sampler must be 0..2");
        return HD_ERR_UNSUPPORTED;
    }
    if (T + I != S || T_uncond + I != S_uncond || T_uncond < 1) {
        hd_set_error("denoise_cfg: text + image tokens != seq (cond %d + %d vs %d, uncond %d + %d vs %d)",
                     T, I, S, T_uncond, I, S_uncond);
        return HD_ERR_MISMATCH;
    }
    if (ws_uncond == ws) {
        hd_set_error("denoise_cfg: the unconditional sequence needs its own workspace");
        return HD_ERR_MISMATCH;
    }
    const UncondSeq u{ws_uncond, ids_uncond, T_uncond, ar_len_uncond, S_uncond, pos_uncond};
    return denoise_loop(bw, ws, sampler, sched, steps, 2, ids, T, pos, ar_len, nullptr, nullptr, z,
                        I, nullptr, 0, guidance, seed, sn_start, sn_end, clip, S, H, KV, HID, FF, D,
                        tms, scratch, scratch_bytes, stream, &u);
}

extern "C" hd_status hd_denoise_visual(const hd_forward_binding *bw, hd_forward_workspace *ws,
                                       int sampler, const hd_scheduler *sched, int steps,
                                       const int64_t *ids, int T, const float *pos,
                                       const void *mask, const hd_visual_cond *visual, void *z,
                                       int img_tokens, const void *ref_patches, int ref_tokens,
                                       uint64_t seed, float sn_start, float sn_end, float clip,
                                       int S, int H, int KV, int HID, int FF, int D, int tms,
                                       void *scratch, int64_t scratch_bytes, void *stream) {
    if (!bw || !ws || !sched || (!ids && T > 0) || !pos || !z || !scratch || img_tokens <= 0 ||
        steps < 1 || ref_tokens < 0) {
        hd_set_error("denoise: null argument");
        return HD_ERR_MISSING;
    }
    if (sampler < HD_SAMPLER_EULER || sampler > HD_SAMPLER_UNIPC) {
        hd_set_error("denoise: sampler must be 0..2");
        return HD_ERR_UNSUPPORTED;
    }
    if (T + img_tokens + ref_tokens != S) {
        hd_set_error("denoise: text + target + reference tokens != seq");
        return HD_ERR_MISMATCH;
    }
    // a workspace x_embedder cache stands in for the references' patches
    // (forward.c:301-313), so it must describe exactly these references
    const bool cached = ws->xe_ref && ws->n_ref > 0;
    if (cached && ws->n_ref != ref_tokens) {
        hd_set_error("denoise: workspace caches %d reference rows, call has %d", ws->n_ref,
                     ref_tokens);
        return HD_ERR_MISMATCH;
    }
    if (ref_tokens > 0 && !ref_patches && !cached) {
        hd_set_error("denoise: %d reference tokens without patches or a cache", ref_tokens);
        return HD_ERR_MISSING;
    }
    return denoise_loop(bw, ws, sampler, sched, steps, 1, ids, T, pos, 0, mask, visual, z,
                        img_tokens, cached ? nullptr : ref_patches, ref_tokens, 0.0f, seed, sn_start, sn_end, clip,
                        S, H, KV, HID, FF, D, tms, scratch, scratch_bytes, stream);
}
