/*
 * CPU oracle of the o1 decoder-block hot path (TEST INFRASTRUCTURE ONLY; see
 * o1_oracle.h). fp32, OpenMP, a packed-panel SGEMM with a 6 x 16 FMA
 * micro-kernel. Each function cites the reference code it restates.
 */
#include "o1_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif


int o1o_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
void o1o_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* support.cu:21-28: round-to-nearest-even on the bit pattern. */
float o1o_bf16_round(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}
void o1o_round_buf(float *x, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) x[i] = o1o_bf16_round(x[i]);
}
static inline float rnd(float v, int r) { return r ? o1o_bf16_round(v) : v; }

/* ------------------------------------------------------------------ */
/* SGEMM y = x . w^T (both K-contiguous), gemm.cu:35-70 math in fp32.  */
/* Packed-panel FMA kernel: 6 rows x 16 columns of C per call, B packed */
/* K-major in panels of 16 columns, K in blocks of 256. Per output the  */
/* products are accumulated in ascending k order.                      */
/* ------------------------------------------------------------------ */
#define GM 6
#define GN 16
#define GKC 256
#define GMC 96
#define GNC 128

/* acc[6][16] += Ap[kc][6] * Bp[kc][16] (both packed K-major). */
static void kern6x16(int kc, const float *Ap, const float *Bp, float acc[GM][GN]) {
    __m256 c[GM][2];
    for (int i = 0; i < GM; i++) {
        c[i][0] = _mm256_loadu_ps(acc[i]);
        c[i][1] = _mm256_loadu_ps(acc[i] + 8);
    }
    for (int k = 0; k < kc; k++) {
        const __m256 b0 = _mm256_loadu_ps(Bp + (size_t)k * GN);
        const __m256 b1 = _mm256_loadu_ps(Bp + (size_t)k * GN + 8);
        for (int i = 0; i < GM; i++) {
            const __m256 av = _mm256_broadcast_ss(Ap + (size_t)k * GM + i);
            c[i][0] = _mm256_fmadd_ps(av, b0, c[i][0]);
            c[i][1] = _mm256_fmadd_ps(av, b1, c[i][1]);
        }
    }
    for (int i = 0; i < GM; i++) {
        _mm256_storeu_ps(acc[i], c[i][0]);
        _mm256_storeu_ps(acc[i] + 8, c[i][1]);
    }
}

/* C[m][n] (ldc) = sum_k A[m][k] * B(k, n) for one M x N tile, where
 * B(k, n) = b[n * ldb + k] when bt (weights [N][K]) else b[k * ldb + n]
 * (values [K][N]). Bp: scratch of GNC * GKC floats. */
static void gemm_tile(const float *A, long lda, const float *b, long ldb, int bt, float *C, long ldc,
                      int M, int N, int K, float *Bp) {
    float Ap[GKC * GM];
    for (int m = 0; m < M; m++) memset(C + (size_t)m * ldc, 0, sizeof(float) * N);
    const int np = (N + GN - 1) / GN;
    for (int k0 = 0; k0 < K; k0 += GKC) {
        const int kc = K - k0 < GKC ? K - k0 : GKC;
        for (int p = 0; p < np; p++) {
            float *dst = Bp + (size_t)p * GKC * GN;
            for (int j = 0; j < GN; j++) {
                const int n = p * GN + j;
                if (n >= N)
                    for (int k = 0; k < kc; k++) dst[(size_t)k * GN + j] = 0.f;
                else if (bt)
                    for (int k = 0; k < kc; k++) dst[(size_t)k * GN + j] = b[(size_t)n * ldb + k0 + k];
                else
                    for (int k = 0; k < kc; k++) dst[(size_t)k * GN + j] = b[(size_t)(k0 + k) * ldb + n];
            }
        }
        for (int m = 0; m < M; m += GM) {
            const int mr = M - m < GM ? M - m : GM;
            for (int i = 0; i < GM; i++) {
                const float *ar = A + (size_t)(m + (i < mr ? i : 0)) * lda + k0;
                for (int k = 0; k < kc; k++) Ap[(size_t)k * GM + i] = ar[k];
            }
            for (int p = 0; p < np; p++) {
                const int nr = N - p * GN < GN ? N - p * GN : GN;
                float acc[GM][GN];
                for (int i = 0; i < GM; i++)
                    for (int j = 0; j < GN; j++)
                        acc[i][j] = (i < mr && j < nr) ? C[(size_t)(m + i) * ldc + p * GN + j] : 0.f;
                kern6x16(kc, Ap, Bp + (size_t)p * GKC * GN, acc);
                for (int i = 0; i < mr; i++)
                    for (int j = 0; j < nr; j++) C[(size_t)(m + i) * ldc + p * GN + j] = acc[i][j];
            }
        }
    }
}

void o1o_linear(const float *x, const float *w, const float *bias, float *y, int M, int N, int K,
                int mode) {
    const int tm = (M + GMC - 1) / GMC, tn = (N + GNC - 1) / GNC;
#pragma omp parallel
    {
        float *Bp = (float *)malloc(sizeof(float) * GNC * GKC);
        float *C = (float *)malloc(sizeof(float) * GMC * GNC);
#pragma omp for schedule(dynamic, 1)
        for (long t = 0; t < (long)tm * tn; t++) {
            const int m0 = (int)(t / tn) * GMC, n0 = (int)(t % tn) * GNC;
            const int mb = M - m0 < GMC ? M - m0 : GMC, nb = N - n0 < GNC ? N - n0 : GNC;
            gemm_tile(x + (size_t)m0 * K, K, w + (size_t)n0 * K, K, 1, C, GNC, mb, nb, K, Bp);
            for (int i = 0; i < mb; i++)
                for (int j = 0; j < nb; j++) {
                    float v = C[(size_t)i * GNC + j];
                    float bb = bias ? bias[n0 + j] : 0.f;
                    if (mode == 0) v = v + bb;
                    else if (mode == 1) v = o1o_bf16_round(v + bb);
                    else v = bias ? o1o_bf16_round(o1o_bf16_round(v) + bb) : o1o_bf16_round(v);
                    y[(size_t)(m0 + i) * N + n0 + j] = v;
                }
        }
        free(Bp);
        free(C);
    }
}

/* norm.cu:12-48: fp32 sum of squares, inv = 1/sqrt(mean + eps), (w*x)*inv. */
void o1o_rmsnorm(const float *x, const float *w, float *y, int rows, int cols, float eps, int round) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * cols;
        float *yr = y + (size_t)r * cols;
        double ss = 0.0;
        for (int c = 0; c < cols; c++) ss += (double)xr[c] * xr[c];
        float inv = 1.0f / sqrtf((float)(ss / cols) + eps);
        for (int c = 0; c < cols; c++) yr[c] = rnd(w[c] * xr[c] * inv, round);
    }
}

/* act.cu:13-34 */
void o1o_silu(const float *x, float *y, size_t n, int round) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) y[i] = rnd(x[i] / (1.0f + expf(-x[i])), round);
}
void o1o_swiglu(const float *g, const float *u, float *y, size_t n, int round) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        float s = rnd(g[i] / (1.0f + expf(-g[i])), round);
        y[i] = rnd(s * u[i], round);
    }
}
/* residual.cu:14-23 */
void o1o_residual_add(const float *x, const float *a, float *y, size_t n, int round) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) y[i] = rnd(x[i] + a[i], round);
}

/* rope.cu:28-71. Frequency f < dim/2 takes its position from row
 * interleaved: slot f%3 in {1,2} with f/3 < section[slot] -> H/W, else T;
 * chunked: the section f falls in. angle = pos * theta^(-2f/dim). */
static int rope_row(int f, const int64_t *sec, int n_section, int interleaved) {
    if (interleaved) {
        int slot = f % 3, chunk = f / 3;
        if ((slot == 1 || slot == 2) && slot <= n_section - 1 && chunk < sec[slot]) return slot;
        return 0;
    }
    int acc = 0;
    for (int t = 0; t < n_section && t < 3; t++) {
        if (f < acc + sec[t]) return t;
        acc += (int)sec[t];
    }
    return 0;
}
void o1o_mrope_cos_sin(const float *pos, int seq, const int64_t *section, int n_section, int dim,
                       float theta, float scaling, int interleaved, float *cosd, float *sind) {
    int half = dim / 2;
    for (int s = 0; s < seq; s++)
        for (int f = 0; f < half; f++) {
            int row = rope_row(f, section, n_section, interleaved);
            float p = pos[(size_t)row * seq + s];
            float base = expf(-logf(theta) * (2.0f * (float)f) / (float)dim);
            float ang = base * p;
            float c = cosf(ang) * scaling, sn = sinf(ang) * scaling;
            cosd[(size_t)s * dim + f] = cosd[(size_t)s * dim + f + half] = c;
            sind[(size_t)s * dim + f] = sind[(size_t)s * dim + f + half] = sn;
        }
}
/* rope.cu:97-134 (bf16 per op) / :157-180 (fp32): rotate-half pairs. */
void o1o_apply_rotary(const float *x, const float *cosd, const float *sind, float *y, int heads,
                      int seq, int dim, int per_op) {
    int half = dim / 2;
#pragma omp parallel for schedule(static)
    for (long hs = 0; hs < (long)heads * seq; hs++) {
        int s = (int)(hs % seq);
        const float *xr = x + (size_t)hs * dim;
        float *yr = y + (size_t)hs * dim;
        for (int d = 0; d < dim; d++) {
            int dp = d < half ? d + half : d - half;
            float c = cosd[(size_t)s * dim + d], sn = sind[(size_t)s * dim + d];
            float a = rnd(xr[d] * c, per_op), b = rnd(xr[dp] * sn, per_op);
            float v = d < half ? a - b : a + b;
            yr[d] = o1o_bf16_round(v);   /* bf16 output in both variants */
        }
    }
}

/* attn.cu:22-127 (GQA kv head = h / (Hq/Hkv), fp32 softmax) with the
 * split-plan row structure of hd_cudnn_sdpa.cu:307-441. Blocked by 16
 * query rows: scores through the SGEMM micro-kernel, P.V as row axpys. */
void o1o_attention(const float *q, const float *k, const float *v, const float *mask, int Hq,
                   int Hkv, int S, int D, int ar_len, float scale, int prob_mode, int round,
                   float *out) {
    const int QB = 48;
    const int nqb = (S + QB - 1) / QB;
    const int grp = Hq / Hkv;
#pragma omp parallel
    {
        float *sc = (float *)malloc(sizeof(float) * QB * (size_t)S);
        float *acc = (float *)malloc(sizeof(float) * QB * (size_t)D);
        float *Bp = (float *)malloc(sizeof(float) * GKC * (size_t)((D + GN - 1) / GN * GN > GNC
                                                                       ? (D + GN - 1) / GN * GN : GNC));
#pragma omp for schedule(dynamic, 1)
        for (long job = 0; job < (long)Hq * nqb; job++) {
            const int h = (int)(job / nqb), qb = (int)(job % nqb);
            const int kh = h / grp;
            const int s0 = qb * QB, s1 = s0 + QB < S ? s0 + QB : S, nq = s1 - s0;
            const float *qh = q + ((size_t)h * S + s0) * D;
            const float *kk = k + (size_t)kh * S * D;
            const float *vv = v + (size_t)kh * S * D;
            /* raw scores Q K^T, key columns in chunks of GNC */
            for (int t0 = 0; t0 < S; t0 += GNC) {
                const int nt = S - t0 < GNC ? S - t0 : GNC;
                gemm_tile(qh, D, kk + (size_t)t0 * D, D, 1, sc + t0, S, nq, nt, D, Bp);
            }
            for (int i = 0; i < nq; i++) {
                const int s = s0 + i;
                float *row = sc + (size_t)i * S;
                const int lim = s < ar_len ? s + 1 : S;
                float mx = -INFINITY;
                for (int t = 0; t < lim; t++) {
                    float val = row[t] * scale;
                    if (mask) val += mask[(size_t)s * S + t];
                    row[t] = val;
                    if (val > mx) mx = val;
                }
                double sum = 0.0;
                for (int t = 0; t < lim; t++) {
                    float e = expf(row[t] - mx);
                    row[t] = e;
                    sum += e;
                }
                const float inv = (float)(1.0 / sum);
                for (int t = 0; t < lim; t++) {
                    float p = row[t] * inv;
                    if (prob_mode == 1) p = o1o_bf16_round(p);
                    row[t] = p;
                }
                for (int t = lim; t < S; t++) row[t] = 0.f;   /* masked keys */
            }
            /* P V: V [S][D] is already K-major */
            gemm_tile(sc, S, vv, D, 0, acc, D, nq, D, S, Bp);
            for (int i = 0; i < nq; i++) {
                float *dst = out + ((size_t)(s0 + i) * Hq + h) * D;
                const float *ar = acc + (size_t)i * D;
                for (int d = 0; d < D; d++) dst[d] = rnd(ar[d], round);
            }
        }
        free(sc);
        free(acc);
        free(Bp);
    }
}

/* gemm.cu:531-545 */
void o1o_timestep_embed(const float *t, float *y, int N, int dim) {
    int half = dim / 2;
    for (int n = 0; n < N; n++)
        for (int d = 0; d < dim; d++) {
            float v = 0.f;
            if (!(dim % 2 && d == dim - 1)) {
                int p = d < half ? d : d - half;
                float freq = expf(-logf(10000.0f) * (float)p / (float)half);
                float arg = t[n] * freq;
                v = d < half ? cosf(arg) : sinf(arg);
            }
            y[(size_t)n * dim + d] = v;
        }
}

/* ------------------------------------------------------------------ */
/* Decoder block, block.c:245-349 op for op.                           */
/* ------------------------------------------------------------------ */
int o1o_decoder_block(const float *x, const float *pos, const float *mask,
                      const o1o_block_weights *w, const o1o_block_cfg *c, int batch, int seq,
                      float *out, float *ln0, float *attn_resid, float *post_ln) {
    const int H = c->heads, KV = c->kv_heads, HID = c->hidden, FF = c->ff, D = c->head_dim;
    const int R = c->faithful;
    const size_t S = (size_t)seq;
    const size_t M = (size_t)batch * S;
    float *ln = malloc(sizeof(float) * M * HID);
    float *qp = malloc(sizeof(float) * M * H * D);
    float *kp = malloc(sizeof(float) * M * KV * D);
    float *vp = malloc(sizeof(float) * M * KV * D);
    float *qh = malloc(sizeof(float) * S * H * D);
    float *kh = malloc(sizeof(float) * S * KV * D);
    float *vh = malloc(sizeof(float) * S * KV * D);
    float *tmp = malloc(sizeof(float) * S * H * D);
    float *att = malloc(sizeof(float) * M * H * D);
    float *ar = malloc(sizeof(float) * M * HID);
    float *g = malloc(sizeof(float) * M * FF);
    float *u = malloc(sizeof(float) * M * FF);
    float *cs = malloc(sizeof(float) * S * D);
    float *sn = malloc(sizeof(float) * S * D);
    if (!ln || !qp || !kp || !vp || !qh || !kh || !vh || !tmp || !att || !ar || !g || !u || !cs || !sn) {
        free(ln); free(qp); free(kp); free(vp); free(qh); free(kh); free(vh); free(tmp);
        free(att); free(ar); free(g); free(u); free(cs); free(sn);
        return -1;
    }
    const float scale = (float)(1.0 / sqrt((double)D));
    const int lmode = R ? 1 : 0;

    o1o_rmsnorm(x, w->input_ln, ln, (int)M, HID, c->eps, R);                       /* :248 */
    if (ln0) memcpy(ln0, ln, sizeof(float) * M * HID);
    o1o_linear(ln, w->q_proj, NULL, qp, (int)M, H * D, HID, lmode);                  /* :253 */
    o1o_linear(ln, w->k_proj, NULL, kp, (int)M, KV * D, HID, lmode);                 /* :254 */
    o1o_linear(ln, w->v_proj, NULL, vp, (int)M, KV * D, HID, lmode);                 /* :255 */
    o1o_mrope_cos_sin(pos, seq, c->section, 3, D, c->theta, c->attention_scaling,
                      c->interleaved, cs, sn);                                         /* :275 */
    for (int b = 0; b < batch; b++) {
        /* head split (:260-262) + q/k norm over D (:267-268) + rope (:281-282) */
        const float *qb = qp + (size_t)b * S * H * D, *kb = kp + (size_t)b * S * KV * D;
        const float *vb = vp + (size_t)b * S * KV * D;
        for (size_t s = 0; s < S; s++) {
            for (int hh = 0; hh < H; hh++) memcpy(tmp + ((size_t)hh * S + s) * D, qb + (s * H + hh) * D, sizeof(float) * D);
            for (int hh = 0; hh < KV; hh++) {
                memcpy(vh + ((size_t)hh * S + s) * D, vb + (s * KV + hh) * D, sizeof(float) * D);
                memcpy(kh + ((size_t)hh * S + s) * D, kb + (s * KV + hh) * D, sizeof(float) * D);
            }
        }
        o1o_rmsnorm(tmp, w->q_norm, tmp, (int)(S * H), D, c->eps, R);
        if (R) o1o_apply_rotary(tmp, cs, sn, qh, H, seq, D, 1);
        else {
            /* fp32 rotation, no rounding */
            int half = D / 2;
            for (size_t hs = 0; hs < S * H; hs++) {
                size_t s = hs % S;
                for (int d = 0; d < D; d++) {
                    int dp = d < half ? d + half : d - half;
                    float cc = cs[s * D + d], ss = sn[s * D + d];
                    float xv = tmp[hs * D + d], xr = tmp[hs * D + dp];
                    qh[hs * D + d] = d < half ? xv * cc - xr * ss : xv * cc + xr * ss;
                }
            }
        }
        o1o_rmsnorm(kh, w->k_norm, kh, (int)(S * KV), D, c->eps, R);
        memcpy(tmp, kh, sizeof(float) * S * KV * D);
        if (R) o1o_apply_rotary(tmp, cs, sn, kh, KV, seq, D, 1);
        else {
            int half = D / 2;
            for (size_t hs = 0; hs < S * KV; hs++) {
                size_t s = hs % S;
                for (int d = 0; d < D; d++) {
                    int dp = d < half ? d + half : d - half;
                    float cc = cs[s * D + d], ss = sn[s * D + d];
                    float xv = tmp[hs * D + d], xr = tmp[hs * D + dp];
                    kh[hs * D + d] = d < half ? xv * cc - xr * ss : xv * cc + xr * ss;
                }
            }
        }
        o1o_attention(qh, kh, vh, mask, H, KV, seq, D, c->ar_len, scale, c->prob_mode, R,
                      att + (size_t)b * S * H * D);                                    /* :296 */
    }
    o1o_linear(att, w->o_proj, NULL, ar, (int)M, HID, H * D, lmode); /* :321 */
    o1o_residual_add(x, ar, ar, M * HID, R);                                          /* :326 */
    if (attn_resid) memcpy(attn_resid, ar, sizeof(float) * M * HID);
    o1o_rmsnorm(ar, w->post_ln, ln, (int)M, HID, c->eps, R);                          /* :331 */
    if (post_ln) memcpy(post_ln, ln, sizeof(float) * M * HID);
    o1o_linear(ln, w->gate_proj, NULL, g, (int)M, FF, HID, lmode);                    /* :336 */
    o1o_linear(ln, w->up_proj, NULL, u, (int)M, FF, HID, lmode);                      /* :337 */
    o1o_swiglu(g, u, g, M * FF, R);                                                   /* :340 */
    o1o_linear(g, w->down_proj, NULL, out, (int)M, HID, FF, lmode);                   /* :343 */
    o1o_residual_add(ar, out, out, M * HID, R);                                       /* :348 */
    free(ln); free(qp); free(kp); free(vp); free(qh); free(kh); free(vh); free(tmp);
    free(att); free(ar); free(g); free(u); free(cs); free(sn);
    return 0;
}

/* forward.c:253-397 for one sequence. */
/* forward.c:278-287 + :363-370 when vmask != NULL: text rows whose vmask
 * byte is set take image_embeds rows in order (before the timestep-token
 * substitution); after block l < 3, deepstack[l] (if non-NULL) is added to
 * the set rows of the block output with one bf16 rounding. */
int o1o_forward_visual(const o1o_forward_weights *w, const o1o_block_cfg *c, const int64_t *ids,
                       int T, const float *vin, int I, float t, const float *pos, const float *mask,
                       int64_t tms_id, const float *image_embeds, const float *const *deepstack,
                       const uint8_t *vmask, float *out, float *after_blocks) {
    const int HID = c->hidden, S = T + I, R = c->faithful;
    const int lmode = R ? 2 : 0;
    float *h = malloc(sizeof(float) * (size_t)S * HID);
    float *h2 = malloc(sizeof(float) * (size_t)S * HID);
    float *xs = malloc(sizeof(float) * (size_t)(I > 0 ? I : 1) * 1024);
    float freq[256], te[4096 * 2];
    if (!h || !h2 || !xs || HID > 4096) { free(h); free(h2); free(xs); return -1; }
    float *th = malloc(sizeof(float) * HID), *temb = malloc(sizeof(float) * HID);
    float ts = t * 1000.0f;                                        /* :253 */
    o1o_timestep_embed(&ts, freq, 1, 256);                         /* :254 */
    if (R) o1o_round_buf(freq, 256);                               /* :255 */
    o1o_linear(freq, w->te0_w, w->te0_b, th, 1, HID, 256, lmode);  /* :257 */
    o1o_silu(th, temb, HID, R);                                    /* :258 */
    o1o_linear(temb, w->te2_w, w->te2_b, th, 1, HID, HID, lmode);  /* :264 */
    (void)te;
    for (int i = 0; i < T; i++) {                                  /* :272-291 */
        int64_t id = ids[i];
        const float *src;
        if (id == tms_id) src = th;
        else {
            if (id < 0 || id >= w->vocab) id = 0;
            src = w->embed_tokens + (size_t)id * HID;
        }
        if (vmask && vmask[i] && id != tms_id) {
            int r = 0;
            for (int j = 0; j < i; j++) r += vmask[j] != 0;
            src = image_embeds + (size_t)r * HID;
        }
        memcpy(h + (size_t)i * HID, src, sizeof(float) * HID);
    }
    if (I > 0) {                                                   /* :301-313 */
        o1o_linear(vin, w->xe1_w, NULL, xs, I, 1024, 3072, lmode);
        o1o_linear(xs, w->xe2_w, w->xe2_b, h + (size_t)T * HID, I, HID, 1024, lmode);
    }
    for (int l = 0; l < w->n_layers; l++) {                        /* :341-375 */
        if (o1o_decoder_block(h, pos, mask, &w->blocks[l], c, 1, S, h2, NULL, NULL, NULL)) {
            free(h); free(h2); free(xs); free(th); free(temb);
            return -1;
        }
        float *sw = h; h = h2; h2 = sw;
        if (vmask && l < 3 && deepstack && deepstack[l]) {
            int r = 0;
            for (int i = 0; i < S; i++) {
                if (!vmask[i]) continue;
                for (int j = 0; j < HID; j++)
                    h[(size_t)i * HID + j] = rnd(h[(size_t)i * HID + j] + deepstack[l][(size_t)r * HID + j], R);
                r++;
            }
        }
        if (after_blocks) memcpy(after_blocks + (size_t)l * S * HID, h, sizeof(float) * (size_t)S * HID);
    }
    o1o_rmsnorm(h, w->fnorm_w, h2, S, HID, c->eps, R);             /* :388 */
    o1o_linear(h2, w->fl_w, w->fl_b, out, S, 3072, HID, lmode);    /* :396 */
    free(h); free(h2); free(xs); free(th); free(temb);
    return 0;
}

int o1o_forward(const o1o_forward_weights *w, const o1o_block_cfg *c, const int64_t *ids, int T,
                const float *vin, int I, float t, const float *pos, const float *mask,
                int64_t tms_id, float *out, float *after_blocks) {
    return o1o_forward_visual(w, c, ids, T, vin, I, t, pos, mask, tms_id, NULL, NULL, NULL, out,
                              after_blocks);
}

/* lora_merge.cu:26-104 */
void o1o_lora_merge(float *w, const float *up, const float *down, int N, int K, int R, float scale) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++) {
            float d = 0.f;
            for (int r = 0; r < R; r++) d += up[(size_t)n * R + r] * down[(size_t)r * K + k];
            w[(size_t)n * K + k] = o1o_bf16_round(w[(size_t)n * K + k] + scale * d);
        }
}

/* sched.cu:50-72, :137-145 (fp32, reference operand order) */
/* The reference's CUDA build contracts a*b + c into one fma (nvcc default);
 * the fused forms are written out so the result is defined, and the HIP
 * kernels use the same explicit fmaf. */
void o1o_sched_vcond(const float *z, const float *xp, float sigma, float *mo, int n) {
    for (int i = 0; i < n; i++) mo[i] = (z[i] - xp[i]) / sigma;
}
void o1o_sched_flow_match_step(const float *z, const float *mo, float sigma, float sigma_next,
                               float *zn, int n) {
    float dt = sigma_next - sigma;
    for (int i = 0; i < n; i++) zn[i] = o1o_bf16_round(fmaf(dt, mo[i], z[i]));
}
void o1o_sched_cfg_guided(const float *c, const float *u, float g, float *o, int n) {
    for (int i = 0; i < n; i++) o[i] = fmaf(g, c[i], (1.0f - g) * u[i]);
}

/* sched.cu:162-170 */
void o1o_unipc_convert(const float *smp, const float *mo, float sigma, float *conv, int n) {
    for (int i = 0; i < n; i++) conv[i] = fmaf(-sigma, mo[i], smp[i]);
}
/* sched.cu:172-201: x_t = (sig_t/sig_s0) last - alpha_t h_phi_1 m0;
 * out = x_t - alpha_t B_h corr */
void o1o_unipc_correct(const float *last, const float *mo0, const float *mo_old, const float *conv,
                       float sig_t, float sig_s0, float alpha_t, float h_phi_1, float B_h,
                       float rc0, float rc1, float inv_rk, int order, float *out, int n) {
    const float r = sig_t / sig_s0, ah = alpha_t * h_phi_1, ab = alpha_t * B_h;
    for (int i = 0; i < n; i++) {
        const float m0 = mo0[i];
        const float x = fmaf(r, last[i], -(ah * m0));
        const float d1t = conv[i] - m0;
        float corr;
        if (order == 2) {
            const float d1s = (mo_old[i] - m0) * inv_rk;
            corr = fmaf(rc0, d1s, rc1 * d1t);
        } else {
            corr = rc1 * d1t;
        }
        out[i] = fmaf(-ab, corr, x);
    }
}
/* sched.cu:203-228 */
void o1o_unipc_predict(const float *smp, const float *mo0, const float *mo_old, float sig_t,
                       float sig_s0, float alpha_t, float h_phi_1, float B_h, float rp,
                       float inv_rk, int order, float *out, int n) {
    const float r = sig_t / sig_s0, ah = alpha_t * h_phi_1, ab = alpha_t * B_h;
    for (int i = 0; i < n; i++) {
        const float m0 = mo0[i];
        float x = fmaf(r, smp[i], -(ah * m0));
        if (order == 2) {
            const float d1s = (mo_old[i] - m0) * inv_rk;
            x = fmaf(-ab, rp * d1s, x);
        }
        out[i] = x;
    }
}

/* generate.c:85-104: tok[r*Wp+c][ch*p*p + i*p + j] = img[ch][r*p+i][c*p+j] */
void o1o_patchify(const float *img, float *tok, int C, int Hp, int Wp, int p) {
    const size_t W = (size_t)Wp * p, Hh = (size_t)Hp * p, F = (size_t)C * p * p;
    for (int r = 0; r < Hp; r++)
        for (int c = 0; c < Wp; c++)
            for (int ch = 0; ch < C; ch++)
                for (int i = 0; i < p; i++)
                    for (int j = 0; j < p; j++)
                        tok[((size_t)r * Wp + c) * F + (size_t)ch * p * p + (size_t)i * p + j] =
                            img[((size_t)ch * Hh + (size_t)(r * p + i)) * W + (size_t)(c * p + j)];
}
void o1o_unpatchify(const float *tok, float *img, int C, int Hp, int Wp, int p) {
    const size_t W = (size_t)Wp * p, Hh = (size_t)Hp * p, F = (size_t)C * p * p;
    for (int r = 0; r < Hp; r++)
        for (int c = 0; c < Wp; c++)
            for (int ch = 0; ch < C; ch++)
                for (int i = 0; i < p; i++)
                    for (int j = 0; j < p; j++)
                        img[((size_t)ch * Hh + (size_t)(r * p + i)) * W + (size_t)(c * p + j)] =
                            tok[((size_t)r * Wp + c) * F + (size_t)ch * p * p + (size_t)i * p + j];
}
/* decode.c:5-27: (v+1)/2*255, round half away from zero, clamp, HWC */
void o1o_decode_to_rgb(const float *z, int grid_h, int grid_w, int patch, int channels,
                       uint8_t *out) {
    const int feats = channels * patch * patch, wpx = grid_w * patch;
    for (int tok = 0; tok < grid_h * grid_w; tok++) {
        int tr = tok / grid_w, tc = tok % grid_w;
        for (int c = 0; c < channels; c++)
            for (int p1 = 0; p1 < patch; p1++)
                for (int p2 = 0; p2 < patch; p2++) {
                    float v = (z[(size_t)tok * feats + (size_t)c * patch * patch + (size_t)p1 * patch + p2] + 1.0f) / 2.0f;
                    float px = roundf(v * 255.0f);
                    if (px < 0.0f) px = 0.0f;
                    if (px > 255.0f) px = 255.0f;
                    out[((size_t)(tr * patch + p1) * wpx + (size_t)(tc * patch + p2)) * channels + c] = (uint8_t)px;
                }
    }
}
