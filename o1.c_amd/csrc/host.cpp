// Host modules around the forward: torch CPU MT19937 noise, sigma schedules,
// sequence tables, initial latent, RGB decode, and the device-side
// flow-match Euler + CFG denoising loop.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

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

extern "C" int64_t hd_denoise_scratch_bytes(int seq, int img, int steps) {
    const int64_t n = (int64_t)img * 3072;
    return al256(2 * n * 2)                       // vin [2, I, 3072] bf16
           + al256((int64_t)2 * seq * 3072 * 2)   // x_pred [2, S, 3072] bf16
           + al256(3 * n * 4)                     // mo_c, mo_u, mo fp32
           + al256((int64_t)(steps + 1) * 2 * 4); // t pairs
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
    float *tdev = (float *)p;
    hd_status status = HD_OK;
    if (steps > HD_SCHED_MAX_STEPS) {
        hd_set_error("denoise: too many steps");
        status = HD_ERR_UNSUPPORTED;
    }
    // per-step timestep pairs (t = sigma for both rows), written by a fill
    // kernel: the values travel as kernel arguments, no host buffer outlives
    // the call
    for (int i = 0; status == HD_OK && i < steps; i++) hd_fill_f32(tdev + 2 * i, sigmas[i], 2);
    for (int i = 0; status == HD_OK && i < steps; i++) {
        const float sg = sigmas[i], sn = sigmas[i + 1];
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
        hd_sched_flow_match_step(z, mo, sg, sn, z, (int)n);
        if (hd_cuda_last_error()[0]) {
            hd_set_error("denoise: %s", hd_cuda_last_error());
            status = HD_ERR_RUNTIME;
        }
    }
    hd_hip_set_stream(prev);
    return status;
}
