// Bandwidth-bound kernels of the block and the forward: RMSNorm, SiLU /
// SwiGLU, residual add, rotary tables and rotation, the fused QKV epilogue,
// head layout permutations, embedding gathers, timestep table, sampler
// pointwise ops and patch (un)shuffle.
//
// Rounding points follow the reference kernels cited on each entry point;
// the memory access pattern is MI355X-first: 64-lane waves own rows, loads
// are 16-byte vectors where the row length allows, reductions are wave
// shuffles (no LDS round trips).
#include <stdio.h>
#include <math.h>

#include "hd_common.hpp"
#include "../../include/hd_hip.h"

#define BAD(name) do { snprintf(hd_cuda_errbuf(), 512, name ": bad args"); return; } while (0)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ---------------------------------------------------------------------------
// RMSNorm: one wave per row (norm.cu:12-48 semantics: fp32 sum of squares,
// inv = 1/sqrt(mean + eps), y = bf16((w * x) * inv)).
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ a,
    const uint16_t *__restrict__ w, uint16_t *__restrict__ sum_out,
    uint16_t *__restrict__ y, int rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const size_t base = (size_t)row * cols;
    float ss = 0.f;
    if (VEC) {
        // cols % 8 == 0: 16-byte chunks; up to 8 chunks per lane in registers
        // (cols <= 4096), a second pass re-reads beyond that.
        const int nch = cols >> 3;
        u32x4_t buf[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            int c = lane + i * 64;
            if (c < nch) {
                u32x4_t v = *(const u32x4_t *)(x + base + (size_t)c * 8);
                if (a) {
                    u32x4_t r = *(const u32x4_t *)(a + base + (size_t)c * 8);
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        v[j] = pack_bf2(lo_bf(v[j]) + lo_bf(r[j]), hi_bf(v[j]) + hi_bf(r[j]));
                    if (sum_out) *(u32x4_t *)(sum_out + base + (size_t)c * 8) = v;
                }
                buf[i] = v;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float l = lo_bf(v[j]), h = hi_bf(v[j]);
                    ss += l * l + h * h;
                }
            }
        }
        for (int c = lane + 512; c < nch; c += 64) {   // very wide rows
            u32x4_t v = *(const u32x4_t *)(x + base + (size_t)c * 8);
            if (a) {
                u32x4_t r = *(const u32x4_t *)(a + base + (size_t)c * 8);
                for (int j = 0; j < 4; j++)
                    v[j] = pack_bf2(lo_bf(v[j]) + lo_bf(r[j]), hi_bf(v[j]) + hi_bf(r[j]));
                if (sum_out) *(u32x4_t *)(sum_out + base + (size_t)c * 8) = v;
            }
            for (int j = 0; j < 4; j++) {
                float l = lo_bf(v[j]), h = hi_bf(v[j]);
                ss += l * l + h * h;
            }
        }
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            int c = lane + i * 64;
            if (c < nch) {
                u32x4_t wv = *(const u32x4_t *)(w + (size_t)c * 8);
                u32x4_t v = buf[i], o;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    o[j] = pack_bf2(lo_bf(wv[j]) * lo_bf(v[j]) * inv, hi_bf(wv[j]) * hi_bf(v[j]) * inv);
                *(u32x4_t *)(y + base + (size_t)c * 8) = o;
            }
        }
        for (int c = lane + 512; c < nch; c += 64) {
            const uint16_t *src = a ? sum_out : x;   // summed row already written
            u32x4_t v = *(const u32x4_t *)(src + base + (size_t)c * 8);
            u32x4_t wv = *(const u32x4_t *)(w + (size_t)c * 8), o;
            for (int j = 0; j < 4; j++)
                o[j] = pack_bf2(lo_bf(wv[j]) * lo_bf(v[j]) * inv, hi_bf(wv[j]) * hi_bf(v[j]) * inv);
            *(u32x4_t *)(y + base + (size_t)c * 8) = o;
        }
    } else {
        for (int c = lane; c < cols; c += 64) {
            float v = bf2f(x[base + c]);
            if (a) {
                v = bfround(v + bf2f(a[base + c]));
                if (sum_out) sum_out[base + c] = f2bf(v);
            }
            ss += v * v;
        }
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
        for (int c = lane; c < cols; c += 64) {
            float v = bf2f(x[base + c]);
            if (a) v = bfround(v + bf2f(a[base + c]));
            y[base + c] = f2bf(bf2f(w[c]) * v * inv);
        }
    }
}

// The same row math for cols <= 4096 (cols % 8 == 0, 16-byte aligned rows)
// with two rows per wave: both rows' loads are in flight together and the
// weight chunks are read once for the pair. Halving the wave count puts a
// whole block-sized activation (8704 rows) in one round of resident waves.
__global__ __launch_bounds__(256) void rmsnorm2_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ a,
    const uint16_t *__restrict__ w, uint16_t *__restrict__ sum_out,
    uint16_t *__restrict__ y, int rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
    if (row0 >= rows) return;
    const bool two = row0 + 1 < rows;
    const int nch = cols >> 3;
    u32x4_t buf[2][8];
    float ss[2] = {0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 2; q++) {
        if (q == 1 && !two) break;
        const size_t base = (size_t)(row0 + q) * cols;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = lane + i * 64;
            if (c < nch) buf[q][i] = *(const u32x4_t *)(x + base + (size_t)c * 8);
        }
    }
    if (a) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            if (q == 1 && !two) break;
            const size_t base = (size_t)(row0 + q) * cols;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int c = lane + i * 64;
                if (c < nch) {
                    const u32x4_t r = *(const u32x4_t *)(a + base + (size_t)c * 8);
                    u32x4_t v = buf[q][i];
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        v[j] = pack_bf2(lo_bf(v[j]) + lo_bf(r[j]), hi_bf(v[j]) + hi_bf(r[j]));
                    if (sum_out) *(u32x4_t *)(sum_out + base + (size_t)c * 8) = v;
                    buf[q][i] = v;
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 2; q++) {
        if (q == 1 && !two) break;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = lane + i * 64;
            if (c < nch) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float l = lo_bf(buf[q][i][j]), h = hi_bf(buf[q][i][j]);
                    ss[q] += l * l + h * h;
                }
            }
        }
    }
    const float inv0 = 1.0f / sqrtf(wave_sum(ss[0]) / (float)cols + eps);
    const float inv1 = 1.0f / sqrtf(wave_sum(ss[1]) / (float)cols + eps);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int c = lane + i * 64;
        if (c < nch) {
            const u32x4_t wv = *(const u32x4_t *)(w + (size_t)c * 8);
#pragma unroll
            for (int q = 0; q < 2; q++) {
                if (q == 1 && !two) break;
                const float inv = q ? inv1 : inv0;
                const u32x4_t v = buf[q][i];
                u32x4_t o;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    o[j] = pack_bf2(lo_bf(wv[j]) * lo_bf(v[j]) * inv, hi_bf(wv[j]) * hi_bf(v[j]) * inv);
                *(u32x4_t *)(y + (size_t)(row0 + q) * cols + (size_t)c * 8) = o;
            }
        }
    }
}

static void launch_rmsnorm(const void *x, const void *a, const void *w, void *s,
                           void *y, int rows, int cols, float eps) {
    bool vec = (cols % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) &&
               ((uintptr_t)w % 16 == 0) && (!a || (uintptr_t)a % 16 == 0) &&
               (!s || (uintptr_t)s % 16 == 0) && !(a && !s && cols > 4096);
    dim3 grid(hd_cdiv(rows, 4));
    if (vec && cols <= 4096 && rows >= 1024)
        rmsnorm2_kernel<<<dim3(hd_cdiv(rows, 8)), 256, 0, hd_stream()>>>(
            (const uint16_t *)x, (const uint16_t *)a, (const uint16_t *)w, (uint16_t *)s,
            (uint16_t *)y, rows, cols, eps);
    else if (vec)
        rmsnorm_kernel<true><<<grid, 256, 0, hd_stream()>>>(
            (const uint16_t *)x, (const uint16_t *)a, (const uint16_t *)w, (uint16_t *)s,
            (uint16_t *)y, rows, cols, eps);
    else
        rmsnorm_kernel<false><<<grid, 256, 0, hd_stream()>>>(
            (const uint16_t *)x, (const uint16_t *)a, (const uint16_t *)w, (uint16_t *)s,
            (uint16_t *)y, rows, cols, eps);
    hd_check_launch("rmsnorm");
}

extern "C" void hd_rmsnorm(const void *x_dev, const void *w_dev, void *y_dev,
                           int rows, int cols, float eps) {
    if (!x_dev || !w_dev || !y_dev || rows <= 0 || cols <= 0) BAD("rmsnorm");
    launch_rmsnorm(x_dev, nullptr, w_dev, nullptr, y_dev, rows, cols, eps);
}

extern "C" void hd_add_rmsnorm(const void *x_dev, const void *a_dev, const void *w_dev,
                               void *sum_dev, void *y_dev, int rows, int cols, float eps) {
    if (!x_dev || !a_dev || !w_dev || !sum_dev || !y_dev || rows <= 0 || cols <= 0)
        BAD("add_rmsnorm");
    launch_rmsnorm(x_dev, a_dev, w_dev, sum_dev, y_dev, rows, cols, eps);
}

// ---------------------------------------------------------------------------
// Pointwise bf16 kernels (act.cu:13-34, residual.cu:14-23). Grid-stride,
// 8 elements per thread per iteration when n % 8 == 0.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu_f(float g) { return g * (1.0f / (1.0f + expf(-g))); }

template <int OP>  // 0 silu(x), 1 swiglu(x=gate, b=up), 2 add(x, b)
__global__ __launch_bounds__(256) void pointwise_kernel(const uint16_t *__restrict__ x,
                                                        const uint16_t *__restrict__ b,
                                                        uint16_t *__restrict__ y, size_t n) {
    const size_t nv = n / 8;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
        u32x4_t xv = *(const u32x4_t *)(x + i * 8), bv = {0, 0, 0, 0}, o;
        if (OP != 0) bv = *(const u32x4_t *)(b + i * 8);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float x0 = lo_bf(xv[j]), x1 = hi_bf(xv[j]);
            float r0, r1;
            if (OP == 0) { r0 = silu_f(x0); r1 = silu_f(x1); }
            else if (OP == 1) { r0 = bfround(silu_f(x0)) * lo_bf(bv[j]); r1 = bfround(silu_f(x1)) * hi_bf(bv[j]); }
            else { r0 = x0 + lo_bf(bv[j]); r1 = x1 + hi_bf(bv[j]); }
            o[j] = pack_bf2(r0, r1);
        }
        *(u32x4_t *)(y + i * 8) = o;
    }
    // tail (n % 8)
    for (size_t i = nv * 8 + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float xv = bf2f(x[i]), r;
        if (OP == 0) r = silu_f(xv);
        else if (OP == 1) r = bfround(silu_f(xv)) * bf2f(b[i]);
        else r = xv + bf2f(b[i]);
        y[i] = f2bf(r);
    }
}

// Scalar fallback for unaligned pointers.
template <int OP>
__global__ void pointwise_scalar_kernel(const uint16_t *x, const uint16_t *b, uint16_t *y, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float xv = bf2f(x[i]), r;
    if (OP == 0) r = silu_f(xv);
    else if (OP == 1) r = bfround(silu_f(xv)) * bf2f(b[i]);
    else r = xv + bf2f(b[i]);
    y[i] = f2bf(r);
}

template <int OP>
static void run_pointwise(const void *x, const void *b, void *y, size_t n, const char *nm) {
    bool al = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) && (!b || (uintptr_t)b % 16 == 0);
    if (al) {
        unsigned blocks = hd_cdiv(n / 8 ? n / 8 : 1, 256);
        if (blocks > 8192) blocks = 8192;
        pointwise_kernel<OP><<<blocks, 256, 0, hd_stream()>>>((const uint16_t *)x, (const uint16_t *)b,
                                                             (uint16_t *)y, n);
    } else {
        pointwise_scalar_kernel<OP><<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(
            (const uint16_t *)x, (const uint16_t *)b, (uint16_t *)y, n);
    }
    hd_check_launch(nm);
}

extern "C" void hd_silu(const void *x_dev, void *y_dev, size_t n) {
    if (!x_dev || !y_dev) BAD("silu");
    if (n == 0) return;
    run_pointwise<0>(x_dev, nullptr, y_dev, n, "silu");
}
extern "C" void hd_swiglu(const void *g, const void *u, void *y, size_t n) {
    if (!g || !u || !y) BAD("swiglu");
    if (n == 0) return;
    run_pointwise<1>(g, u, y, n, "swiglu");
}
extern "C" void hd_residual_add(const void *x, const void *a, void *y, size_t n) {
    if (!x || !a || !y) BAD("residual_add");
    if (n == 0) return;
    run_pointwise<2>(x, a, y, n, "residual_add");
}

// ---------------------------------------------------------------------------
// Timestep table (gemm.cu:531-545): freq_p = exp(-ln(1e4) * p / half),
// first half cos(t*freq), second half sin(t*freq); odd dim pads a zero.
// ---------------------------------------------------------------------------
__global__ void timestep_kernel(const float *t, float *y, int N, int dim) {
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N * dim) return;
    int n = idx / dim, d = idx % dim, half = dim / 2;
    float v = 0.f;
    if (!(dim % 2 && d == dim - 1)) {
        int p = d < half ? d : d - half;
        float freq = expf(-logf(10000.0f) * (float)p / (float)half);
        float arg = t[n] * freq;
        v = d < half ? cosf(arg) : sinf(arg);
    }
    y[idx] = v;
}
extern "C" void hd_timestep_embed(const float *t_dev, float *y_dev, int N, int dim) {
    if (!t_dev || !y_dev || N <= 0 || dim <= 0) BAD("timestep_embed");
    timestep_kernel<<<hd_cdiv((size_t)N * dim, 256), 256, 0, hd_stream()>>>(t_dev, y_dev, N, dim);
    hd_check_launch("timestep_embed");
}

// ---------------------------------------------------------------------------
// Rotary tables. Frequency f in [0, dim/2) takes its position from row
//   interleaved: slot f%3 (1 = H, 2 = W) when f/3 < section[slot], else T;
//   chunked:     the section f falls into;
// angle = pos * theta^(-2f/dim) (rope.cu:28-71).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int rope_row(int f, const int64_t *sec, int n_section, int interleaved) {
    if (interleaved) {
        int slot = f % 3, chunk = f / 3;
        if ((slot == 1 || slot == 2) && slot <= n_section - 1 && chunk < (int)sec[slot]) return slot;
        return 0;
    }
    int acc = 0;
    for (int t = 0; t < n_section && t < 3; t++) {
        if (f < acc + (int)sec[t]) return t;
        acc += (int)sec[t];
    }
    return 0;
}

__global__ void mrope_kernel(const float *pos, const int64_t *sec, float *cosd, float *sind,
                             int bs, int seq, int dim, float theta, float scaling, int n_section,
                             int interleaved) {
    int s = blockIdx.x, b = blockIdx.y;
    int half = dim / 2;
    for (int k = threadIdx.x; k < dim; k += blockDim.x) {
        int f = k < half ? k : k - half;
        int row = rope_row(f, sec, n_section, interleaved);
        float p = pos[(size_t)row * bs * seq + (size_t)b * seq + s];
        float base = expf(-logf(theta) * (2.0f * (float)f) / (float)dim);
        float ang = base * p;
        size_t o = ((size_t)b * seq + s) * dim + k;
        cosd[o] = cosf(ang) * scaling;
        sind[o] = sinf(ang) * scaling;
    }
}
extern "C" void hd_mrope_cos_sin(const float *pos_dev, int bs, int seq, const int64_t *section_dev,
                                 int n_section, int head_dim, float theta, float attention_scaling,
                                 int interleaved, float *cos_dev, float *sin_dev) {
    if (!pos_dev || !section_dev || !cos_dev || !sin_dev || seq <= 0 || head_dim <= 0 || bs <= 0)
        BAD("mrope");
    mrope_kernel<<<dim3(seq, bs), 128, 0, hd_stream()>>>(pos_dev, section_dev, cos_dev, sin_dev, bs,
                                                         seq, head_dim, theta, attention_scaling,
                                                         n_section, interleaved);
    hd_check_launch("mrope");
}

struct RopeSec { int64_t s[3]; };
__global__ void rope_table_kernel(const float *pos, RopeSec sec, float2 *cs, int seq, int dim,
                                  float theta, float scaling, int n_section, int interleaved) {
    int half = dim / 2;
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= seq * half) return;
    int s = idx / half, f = idx % half;
    int row = rope_row(f, sec.s, n_section, interleaved);
    float p = pos[(size_t)row * seq + s];
    float base = expf(-logf(theta) * (2.0f * (float)f) / (float)dim);
    float ang = base * p;
    cs[idx] = make_float2(cosf(ang) * scaling, sinf(ang) * scaling);
}
extern "C" void hd_rope_table(const float *pos_dev, int seq, const int64_t *section_host,
                              int n_section, int head_dim, float theta, float attention_scaling,
                              int interleaved, float *cs_dev) {
    if (!pos_dev || !section_host || !cs_dev || seq <= 0 || head_dim <= 0 || head_dim % 2 ||
        n_section < 1 || n_section > 3)
        BAD("rope_table");
    RopeSec sec = {{0, 0, 0}};
    for (int i = 0; i < n_section; i++) sec.s[i] = section_host[i];
    rope_table_kernel<<<hd_cdiv((size_t)seq * head_dim / 2, 256), 256, 0, hd_stream()>>>(
        pos_dev, sec, (float2 *)cs_dev, seq, head_dim, theta, attention_scaling, n_section,
        interleaved);
    hd_check_launch("rope_table");
}

// The same table with the section read from device memory (the reference's
// int64[3] sec_dev, rope.cu:73-95), so a caller's per-call section is honoured
// without a host round trip.
__global__ void rope_table_dev_kernel(const float *pos, const int64_t *sec_dev, float2 *cs, int seq,
                                      int dim, float theta, float scaling, int n_section,
                                      int interleaved) {
    int half = dim / 2;
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= seq * half) return;
    int64_t sec[3] = {0, 0, 0};
    for (int i = 0; i < n_section; i++) sec[i] = sec_dev[i];
    int s = idx / half, f = idx % half;
    int row = rope_row(f, sec, n_section, interleaved);
    float p = pos[(size_t)row * seq + s];
    float base = expf(-logf(theta) * (2.0f * (float)f) / (float)dim);
    float ang = base * p;
    cs[idx] = make_float2(cosf(ang) * scaling, sinf(ang) * scaling);
}
extern "C" void hd_rope_table_dev(const float *pos_dev, int seq, const int64_t *section_dev,
                                  int n_section, int head_dim, float theta, float attention_scaling,
                                  int interleaved, float *cs_dev) {
    if (!pos_dev || !section_dev || !cs_dev || seq <= 0 || head_dim <= 0 || head_dim % 2 ||
        n_section < 1 || n_section > 3)
        BAD("rope_table_dev");
    rope_table_dev_kernel<<<hd_cdiv((size_t)seq * head_dim / 2, 256), 256, 0, hd_stream()>>>(
        pos_dev, section_dev, (float2 *)cs_dev, seq, head_dim, theta, attention_scaling, n_section,
        interleaved);
    hd_check_launch("rope_table_dev");
}

static bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Rotate-half rotation on [heads, seq, dim] (rope.cu:97-134 / :157-180).
template <bool PEROP>
__global__ void rotary_kernel(const uint16_t *x, const float *cosd, const float *sind, uint16_t *y,
                              int heads, int seq, int dim) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)heads * seq * dim;
    if (idx >= total) return;
    int d = idx % dim;
    size_t hs = idx / dim;
    int s = hs % seq;
    int half = dim / 2;
    int dp = d < half ? d + half : d - half;
    float x0 = bf2f(x[idx]), xh = bf2f(x[hs * dim + dp]);
    float c = cosd[(size_t)s * dim + d], sn = sind[(size_t)s * dim + d];
    float v;
    if (PEROP) {
        float a = bfround(x0 * c), b = bfround(xh * sn);
        v = d < half ? a - b : a + b;
    } else {
        v = d < half ? x0 * c - xh * sn : x0 * c + xh * sn;
    }
    y[idx] = f2bf(v);
}
// 16-byte variant (dim % 16 == 0, aligned operands): one thread rotates 8
// consecutive pairs (d, d + dim/2) of one row, the same arithmetic per
// element as rotary_kernel<true> (bf16 rounding of each product).
__global__ void rotary16_kernel(const uint16_t *x, const float *cosd, const float *sind, uint16_t *y,
                                int heads, int seq, int dim) {
    const int half = dim / 2, c8 = half / 8;
    const size_t total = (size_t)heads * seq * c8;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int d0 = (int)(idx % c8) * 8;
    const size_t hs = idx / c8;
    const int s = hs % seq;
    const uint16_t *xr = x + hs * dim;
    const float *cr = cosd + (size_t)s * dim, *sr = sind + (size_t)s * dim;
    const u32x4_t lo = *(const u32x4_t *)(xr + d0), hi = *(const u32x4_t *)(xr + half + d0);
    const f32x4_t cl0 = *(const f32x4_t *)(cr + d0), cl1 = *(const f32x4_t *)(cr + d0 + 4);
    const f32x4_t ch0 = *(const f32x4_t *)(cr + half + d0), ch1 = *(const f32x4_t *)(cr + half + d0 + 4);
    const f32x4_t sl0 = *(const f32x4_t *)(sr + d0), sl1 = *(const f32x4_t *)(sr + d0 + 4);
    const f32x4_t sh0 = *(const f32x4_t *)(sr + half + d0), sh1 = *(const f32x4_t *)(sr + half + d0 + 4);
    u32x4_t olo, ohi;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float r0[2], r1[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int k = 2 * e + t;
            const float a = t ? hi_bf(lo[e]) : lo_bf(lo[e]);   // x[d]
            const float b = t ? hi_bf(hi[e]) : lo_bf(hi[e]);   // x[d + half]
            const float cl = k < 4 ? cl0[k] : cl1[k - 4], ch = k < 4 ? ch0[k] : ch1[k - 4];
            const float sl = k < 4 ? sl0[k] : sl1[k - 4], sh = k < 4 ? sh0[k] : sh1[k - 4];
            r0[t] = bfround(a * cl) - bfround(b * sl);
            r1[t] = bfround(b * ch) + bfround(a * sh);
        }
        olo[e] = pack_bf2(r0[0], r0[1]);
        ohi[e] = pack_bf2(r1[0], r1[1]);
    }
    *(u32x4_t *)(y + hs * dim + d0) = olo;
    *(u32x4_t *)(y + hs * dim + half + d0) = ohi;
}
extern "C" void hd_apply_rotary(const void *x, const float *c, const float *s, void *y, int heads,
                                int seq, int dim) {
    if (!x || !c || !s || !y || heads <= 0 || seq <= 0 || dim <= 0) BAD("apply_rotary");
    if (dim % 16 == 0 && al16(x) && al16(c) && al16(s) && al16(y)) {
        rotary16_kernel<<<hd_cdiv((size_t)heads * seq * (dim / 16), 256), 256, 0, hd_stream()>>>(
            (const uint16_t *)x, c, s, (uint16_t *)y, heads, seq, dim);
    } else {
        rotary_kernel<true><<<hd_cdiv((size_t)heads * seq * dim, 256), 256, 0, hd_stream()>>>(
            (const uint16_t *)x, c, s, (uint16_t *)y, heads, seq, dim);
    }
    hd_check_launch("apply_rotary");
}
extern "C" void hd_apply_rotary_f32(const void *x, const float *c, const float *s, void *y,
                                    int heads, int seq, int dim) {
    if (!x || !c || !s || !y || heads <= 0 || seq <= 0 || dim <= 0) BAD("apply_rotary_f32");
    rotary_kernel<false><<<hd_cdiv((size_t)heads * seq * dim, 256), 256, 0, hd_stream()>>>(
        (const uint16_t *)x, c, s, (uint16_t *)y, heads, seq, dim);
    hd_check_launch("apply_rotary_f32");
}

// ---------------------------------------------------------------------------
// Fused QKV epilogue. One wave per (token, head) for q and k: lane l owns
// the rotate-half pair (l, l+64) of the 128-wide head, so the norm is a wave
// sum and the rotation needs no shuffle. Roundings: norm -> bf16
// (norm.cu:44-46), products and sum -> bf16 (rope.cu:121-132).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const uint16_t *__restrict__ qkv, const uint16_t *__restrict__ qn_w,
    const uint16_t *__restrict__ kn_w, const float2 *__restrict__ cs,
    uint16_t *__restrict__ q, uint16_t *__restrict__ k, int seq, int heads, int kv_heads,
    float eps) {
    const int D = 128;
    const int lane = threadIdx.x & 63;
    const int hslot = blockIdx.y * 4 + (threadIdx.x >> 6);   // 0 .. heads+kv_heads-1
    const int m = blockIdx.x;                                // token row b*seq + s
    if (hslot >= heads + kv_heads) return;
    const int ncol = (heads + 2 * kv_heads) * D;
    const uint16_t *src = qkv + (size_t)m * ncol + (size_t)hslot * D;
    float x0 = bf2f(src[lane]), x1 = bf2f(src[lane + 64]);
    // the q/k norm's summation tree: partners 4, 2, 1, then 32, 16, 8 apart
    float ss = fmaf(x0, x0, x1 * x1);
    ss += __shfl_xor(ss, 4, 64);
    ss += __shfl_xor(ss, 2, 64);
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 32, 64);
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 8, 64);
    float inv = 1.0f / sqrtf(ss / (float)D + eps);
    const uint16_t *w = hslot < heads ? qn_w : kn_w;
    float y0 = bfround(bf2f(w[lane]) * x0 * inv);
    float y1 = bfround(bf2f(w[lane + 64]) * x1 * inv);
    const int b = m / seq, s = m % seq;
    float2 r = cs[(size_t)s * (D / 2) + lane];
    float o0 = bfround(y0 * r.x) - bfround(y1 * r.y);
    float o1 = bfround(y1 * r.x) + bfround(y0 * r.y);
    uint16_t *dst;
    if (hslot < heads) dst = q + (((size_t)b * heads + hslot) * seq + s) * D;
    else dst = k + (((size_t)b * kv_heads + (hslot - heads)) * seq + s) * D;
    dst[lane] = f2bf(o0);
    dst[lane + 64] = f2bf(o1);
}

// V columns of the projection -> the flash kernel's V^T layout
// [B,KV,128,S_pad] (S_pad = round_up(S,64), key s at column s with bits 2
// and 3 exchanged, zero padding) or plain [B,KV,S,D]. Block: 64 tokens x one
// kv head through LDS, so reads (256 B per token) and the transposed writes
// (128 B per d row) both coalesce.
__device__ __forceinline__ int perm16_ew(int s) { return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1); }

__global__ __launch_bounds__(256) void v_layout_kernel(const uint16_t *__restrict__ qkv,
                                                       uint16_t *__restrict__ v,
                                                       uint16_t *__restrict__ vt, int seq,
                                                       int heads, int kv_heads) {
    const int D = 128;
    __shared__ uint16_t tile[64][D + 2];
    const int s0 = blockIdx.x * 64;
    const int hk = blockIdx.y % kv_heads, b = blockIdx.y / kv_heads;
    const int ncol = (heads + 2 * kv_heads) * D;
    const int col0 = (heads + kv_heads + hk) * D;
    const int s_pad = (seq + 63) / 64 * 64;
    for (int i = threadIdx.x; i < 64 * D / 2; i += 256) {
        int t = i / (D / 2), d2 = (i % (D / 2)) * 2;
        int s = s0 + t;
        uint32_t val = 0;
        if (s < seq) val = *(const uint32_t *)(qkv + ((size_t)b * seq + s) * ncol + col0 + d2);
        if (vt) { tile[t][d2] = val & 0xFFFF; tile[t][d2 + 1] = val >> 16; }
        else if (s < seq) *(uint32_t *)(v + (((size_t)b * kv_heads + hk) * seq + s) * D + d2) = val;
    }
    if (!vt) return;
    __syncthreads();
    uint16_t *dst = vt + ((size_t)b * kv_heads + hk) * D * (size_t)s_pad + s0;
    for (int i = threadIdx.x; i < 64 * D; i += 256) {
        int d = i / 64, p = i % 64;
        dst[(size_t)d * s_pad + p] = tile[perm16_ew(p)][d];
    }
}

// 16-byte variant of qk_norm_rope_kernel: 8 lanes per (row, head); lane j
// holds elements 8j..8j+7 and their rotate-half partners 64+8j..64+8j+7
// (two 16-byte loads), so x_l^2 + x_{l+64}^2 and the rotation stay inside the
// lane. The sum of squares follows the same tree as qk_norm_rope_kernel
// (pairs 4, 2, 1 apart inside the lane, then 32, 16, 8 apart = lanes 4, 2,
// 1 apart), so results are bit-identical. For 16-byte aligned operands.
__global__ __launch_bounds__(256) void qk_norm_rope16_kernel(
    const uint16_t *__restrict__ qkv, const uint16_t *__restrict__ qn_w,
    const uint16_t *__restrict__ kn_w, const float2 *__restrict__ cs,
    uint16_t *__restrict__ q, uint16_t *__restrict__ k, int rows, int seq, int heads,
    int kv_heads, float eps) {
    const int D = 128;
    const int j = threadIdx.x & 7;
    const int nh = heads + kv_heads;
    const size_t hr = (size_t)blockIdx.x * 32 + (threadIdx.x >> 3);   // (row, head slot)
    const bool live = hr < (size_t)rows * nh;
    const int m = live ? (int)(hr / nh) : 0, hslot = live ? (int)(hr % nh) : 0;
    const int ncol = (heads + 2 * kv_heads) * D;
    const int d0 = j * 8;
    const uint16_t *src = qkv + (size_t)m * ncol + (size_t)hslot * D;
    u32x4_t xa = {0u, 0u, 0u, 0u}, xb = {0u, 0u, 0u, 0u};
    if (live) {
        xa = *(const u32x4_t *)(src + d0);
        xb = *(const u32x4_t *)(src + 64 + d0);
    }
    float a[8], b[8];   // x_l, x_{l+64}
#pragma unroll
    for (int e = 0; e < 4; e++) {
        a[2 * e] = lo_bf(xa[e]); a[2 * e + 1] = hi_bf(xa[e]);
        b[2 * e] = lo_bf(xb[e]); b[2 * e + 1] = hi_bf(xb[e]);
    }
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = fmaf(a[e], a[e], b[e] * b[e]);
    // pairs 4 apart, then 2, then 1 (inside the lane)
    const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    float ss = (s0 + s2) + (s1 + s3);
    ss += __shfl_xor(ss, 4, 64);
    ss += __shfl_xor(ss, 2, 64);
    ss += __shfl_xor(ss, 1, 64);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    const uint16_t *w = hslot < heads ? qn_w : kn_w;
    const u32x4_t wa = *(const u32x4_t *)(w + d0), wb = *(const u32x4_t *)(w + 64 + d0);
    const int bi = m / seq, s = m % seq;
    const float2 *cr = cs + (size_t)s * (D / 2) + d0;
    float o0[8], o1[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float w0 = (e & 1) ? hi_bf(wa[e / 2]) : lo_bf(wa[e / 2]);
        const float w1 = (e & 1) ? hi_bf(wb[e / 2]) : lo_bf(wb[e / 2]);
        const float y0 = bfround(w0 * a[e] * inv), y1 = bfround(w1 * b[e] * inv);
        const float2 r = cr[e];
        o0[e] = bfround(y0 * r.x) - bfround(y1 * r.y);
        o1[e] = bfround(y1 * r.x) + bfround(y0 * r.y);
    }
    if (!live) return;
    uint16_t *dst;
    if (hslot < heads) dst = q + (((size_t)bi * heads + hslot) * seq + s) * D;
    else dst = k + (((size_t)bi * kv_heads + (hslot - heads)) * seq + s) * D;
    *(u32x4_t *)(dst + d0) = {pack_bf2(o0[0], o0[1]), pack_bf2(o0[2], o0[3]), pack_bf2(o0[4], o0[5]),
                              pack_bf2(o0[6], o0[7])};
    *(u32x4_t *)(dst + 64 + d0) = {pack_bf2(o1[0], o1[1]), pack_bf2(o1[2], o1[3]), pack_bf2(o1[4], o1[5]),
                                   pack_bf2(o1[6], o1[7])};
}

// 16-byte variant of v_layout_kernel (16-byte aligned operands): 16-byte
// reads of the V columns and 16-byte writes of 8 consecutive V^T columns.
__global__ __launch_bounds__(256) void v_layout16_kernel(const uint16_t *__restrict__ qkv,
                                                         uint16_t *__restrict__ v,
                                                         uint16_t *__restrict__ vt, int seq,
                                                         int heads, int kv_heads) {
    const int D = 128;
    __shared__ uint32_t tile[64][D / 2 + 1];   // bf16 pairs, one pad word per token row
    const int s0 = blockIdx.x * 64;
    const int hk = blockIdx.y % kv_heads, b = blockIdx.y / kv_heads;
    const int ncol = (heads + 2 * kv_heads) * D;
    const int col0 = (heads + kv_heads + hk) * D;
    const int s_pad = (seq + 63) / 64 * 64;
    for (int i = threadIdx.x; i < 64 * D / 8; i += 256) {
        const int t = i / (D / 8), d8 = (i % (D / 8)) * 8;
        const int s = s0 + t;
        u32x4_t val = {0u, 0u, 0u, 0u};
        if (s < seq) val = *(const u32x4_t *)(qkv + ((size_t)b * seq + s) * ncol + col0 + d8);
        if (vt) {
#pragma unroll
            for (int e = 0; e < 4; e++) tile[t][d8 / 2 + e] = val[e];
        } else if (s < seq) {
            *(u32x4_t *)(v + (((size_t)b * kv_heads + hk) * seq + s) * D + d8) = val;
        }
    }
    if (!vt) return;
    __syncthreads();
    uint16_t *dst = vt + ((size_t)b * kv_heads + hk) * D * (size_t)s_pad + s0;
    for (int i = threadIdx.x; i < D * 8; i += 256) {
        const int d = i / 8, p0 = (i % 8) * 8;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t a = tile[perm16_ew(p0 + 2 * e)][d / 2], c = tile[perm16_ew(p0 + 2 * e + 1)][d / 2];
            const uint32_t lo = (d & 1) ? a >> 16 : a & 0xFFFFu, hi = (d & 1) ? c >> 16 : c & 0xFFFFu;
            w[e] = lo | (hi << 16);
        }
        *(u32x4_t *)(dst + (size_t)d * s_pad + p0) = {w[0], w[1], w[2], w[3]};
    }
}

extern "C" void hd_qkv_epilogue(const void *qkv_dev, const void *qn_w, const void *kn_w,
                                const float *cs_dev, void *q_dev, void *k_dev, void *v_dev,
                                void *vt_dev, int batch, int seq, int heads, int kv_heads,
                                int head_dim, float eps) {
    if (!qkv_dev || !qn_w || !kn_w || !cs_dev || !q_dev || !k_dev || (!v_dev && !vt_dev) ||
        batch <= 0 || seq <= 0 || heads <= 0 || kv_heads <= 0 || head_dim != 128)
        BAD("qkv_epilogue");
    if (al16(qkv_dev) && al16(qn_w) && al16(kn_w) && al16(cs_dev) && al16(q_dev) && al16(k_dev)) {
        const size_t nhr = (size_t)batch * seq * (heads + kv_heads);
        qk_norm_rope16_kernel<<<hd_cdiv(nhr, 32), 256, 0, hd_stream()>>>(
            (const uint16_t *)qkv_dev, (const uint16_t *)qn_w, (const uint16_t *)kn_w,
            (const float2 *)cs_dev, (uint16_t *)q_dev, (uint16_t *)k_dev, batch * seq, seq, heads,
            kv_heads, eps);
    } else {
        dim3 g1(batch * seq, hd_cdiv(heads + kv_heads, 4));
        qk_norm_rope_kernel<<<g1, 256, 0, hd_stream()>>>(
            (const uint16_t *)qkv_dev, (const uint16_t *)qn_w, (const uint16_t *)kn_w,
            (const float2 *)cs_dev, (uint16_t *)q_dev, (uint16_t *)k_dev, seq, heads, kv_heads, eps);
    }
    hd_check_launch("qkv_epilogue(qk)");
    dim3 g2(hd_cdiv(seq, 64), batch * kv_heads);
    if (al16(qkv_dev) && (vt_dev ? al16(vt_dev) && ((seq + 63) / 64 * 64) % 8 == 0 : al16(v_dev)))
        v_layout16_kernel<<<g2, 256, 0, hd_stream()>>>((const uint16_t *)qkv_dev, (uint16_t *)v_dev,
                                                       (uint16_t *)vt_dev, seq, heads, kv_heads);
    else
        v_layout_kernel<<<g2, 256, 0, hd_stream()>>>((const uint16_t *)qkv_dev, (uint16_t *)v_dev,
                                                     (uint16_t *)vt_dev, seq, heads, kv_heads);
    hd_check_launch("qkv_epilogue(v)");
}

// [BH, S, D] -> [BH, D, S]
__global__ __launch_bounds__(256) void transpose_sd_kernel(const uint16_t *in, uint16_t *out,
                                                           int seq, int dim) {
    __shared__ uint16_t tile[64][65];
    const int bh = blockIdx.z;
    const int s0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
    const uint16_t *src = in + (size_t)bh * seq * dim;
    uint16_t *dst = out + (size_t)bh * seq * dim;
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        int t = i / 64, d = i % 64;
        if (s0 + t < seq && d0 + d < dim) tile[t][d] = src[(size_t)(s0 + t) * dim + d0 + d];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        int d = i / 64, t = i % 64;
        if (s0 + t < seq && d0 + d < dim) dst[(size_t)(d0 + d) * seq + s0 + t] = tile[t][d];
    }
}
extern "C" void hd_transpose_sd(const void *in_dev, void *out_dev, int bh, int seq, int dim) {
    if (!in_dev || !out_dev || bh <= 0 || seq <= 0 || dim <= 0) BAD("transpose_sd");
    dim3 g(hd_cdiv(seq, 64), hd_cdiv(dim, 64), bh);
    transpose_sd_kernel<<<g, 256, 0, hd_stream()>>>((const uint16_t *)in_dev, (uint16_t *)out_dev,
                                                    seq, dim);
    hd_check_launch("transpose_sd");
}

// ---------------------------------------------------------------------------
// Head permutations (attn.cu:180-218): [S,H,D] <-> [H,S,D], 4-byte moves.
// ---------------------------------------------------------------------------
template <bool SPLIT>
__global__ void head_perm_kernel(const uint16_t *in, uint16_t *out, int seq, int heads, int d) {
    size_t total = (size_t)seq * heads * d;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    int dd = idx % d;
    size_t r = idx / d;
    // idx enumerates the OUTPUT layout so writes coalesce
    if (SPLIT) {  // out [H,S,D]
        int s = r % seq, h = r / seq;
        out[idx] = in[((size_t)s * heads + h) * d + dd];
    } else {      // out [S,H,D]
        int h = r % heads, s = r / heads;
        out[idx] = in[((size_t)h * seq + s) * d + dd];
    }
}
// 16-byte variant (dim % 8 == 0, 16-byte aligned operands): one thread
// moves 8 consecutive elements of a row; the same permutation.
template <bool SPLIT>
__global__ void head_perm16_kernel(const u32x4_t *in, u32x4_t *out, int seq, int heads, int d8) {
    const size_t total = (size_t)seq * heads * d8;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int dd = idx % d8;
    const size_t r = idx / d8;
    if (SPLIT) {
        const int s = r % seq, h = r / seq;
        out[idx] = in[((size_t)s * heads + h) * d8 + dd];
    } else {
        const int h = r % heads, s = r / heads;
        out[idx] = in[((size_t)h * seq + s) * d8 + dd];
    }
}
template <bool SPLIT>
static void launch_head_perm(const void *in, void *out, int seq, int heads, int dim) {
    if (dim % 8 == 0 && al16(in) && al16(out)) {
        head_perm16_kernel<SPLIT><<<hd_cdiv((size_t)seq * heads * (dim / 8), 256), 256, 0, hd_stream()>>>(
            (const u32x4_t *)in, (u32x4_t *)out, seq, heads, dim / 8);
    } else {
        head_perm_kernel<SPLIT><<<hd_cdiv((size_t)seq * heads * dim, 256), 256, 0, hd_stream()>>>(
            (const uint16_t *)in, (uint16_t *)out, seq, heads, dim);
    }
}
extern "C" void hd_head_split(const void *in, void *out, int seq, int heads, int dim) {
    if (!in || !out || seq <= 0 || heads <= 0 || dim <= 0) BAD("head_split");
    launch_head_perm<true>(in, out, seq, heads, dim);
    hd_check_launch("head_split");
}
extern "C" void hd_head_merge(const void *in, void *out, int seq, int heads, int dim) {
    if (!in || !out || seq <= 0 || heads <= 0 || dim <= 0) BAD("head_merge");
    launch_head_perm<false>(in, out, seq, heads, dim);
    hd_check_launch("head_merge");
}

// ---------------------------------------------------------------------------
// Embedding gather and timestep-token substitution (embed.cu:15-70).
// One block per output row, 4-byte moves (cols is even for every model dim;
// an odd cols falls back to 2-byte moves).
// ---------------------------------------------------------------------------
__global__ void gather_rows_kernel(const uint16_t *table, const int64_t *idx, uint16_t *out,
                                   int cols, int64_t nrows) {
    int row = blockIdx.x;
    int64_t id = idx[row];
    if (id < 0 || id >= nrows) id = 0;
    const uint16_t *src = table + (size_t)id * cols;
    uint16_t *dst = out + (size_t)row * cols;
    for (int c = threadIdx.x; c < cols; c += blockDim.x) dst[c] = src[c];
}
extern "C" void hd_gather_rows(const void *table, const void *idx, void *out, int M, int cols,
                               int64_t nrows) {
    if (!table || !idx || !out || M <= 0 || cols <= 0) BAD("gather_rows");
    gather_rows_kernel<<<M, 256, 0, hd_stream()>>>((const uint16_t *)table, (const int64_t *)idx,
                                                   (uint16_t *)out, cols, nrows);
    hd_check_launch("gather_rows");
}
__global__ void tms_kernel(const int64_t *idx, const uint16_t *emb, const uint16_t *temb,
                           uint16_t *out, int H, int64_t tms) {
    int row = blockIdx.x;
    const uint16_t *src = idx[row] == tms ? temb : emb + (size_t)row * H;
    uint16_t *dst = out + (size_t)row * H;
    for (int c = threadIdx.x; c < H; c += blockDim.x) dst[c] = src[c];
}
extern "C" void hd_apply_tms_condition(const void *idx, const void *emb, const void *temb,
                                       void *out, int M, int H, int64_t tms_id) {
    if (!idx || !emb || !temb || !out || M <= 0 || H <= 0) BAD("tms_condition");
    tms_kernel<<<M, 256, 0, hd_stream()>>>((const int64_t *)idx, (const uint16_t *)emb,
                                           (const uint16_t *)temb, (uint16_t *)out, H, tms_id);
    hd_check_launch("tms_condition");
}

__global__ void scale_kernel(const float *in, float *out, float s, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = in[i] * s;
}
extern "C" void hd_scale_f32(const float *in, float *out, float s, int n) {
    if (!in || !out || n <= 0) BAD("scale_f32");
    scale_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(in, out, s, n);
    hd_check_launch("scale_f32");
}
__global__ void fill_kernel(float *dst, float v, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = v;
}
// Internal (host.cpp): device fill whose value travels as a kernel argument.
extern "C" void hd_fill_f32(float *dst, float value, int n) {
    if (!dst || n <= 0) BAD("fill_f32");
    fill_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(dst, value, n);
    hd_check_launch("fill_f32");
}
__global__ void cvt_kernel(const float *in, uint16_t *out, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2bf(in[i]);
}
extern "C" void hd_f32_convert_bf16(const float *in, void *out, int n) {
    if (!in || !out || n <= 0) BAD("f32_convert_bf16");
    cvt_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(in, (uint16_t *)out, n);
    hd_check_launch("f32_convert_bf16");
}

// ---------------------------------------------------------------------------
// Sampler pointwise kernels (sched.cu:21-72, :137-145), fp32, same operand
// order as the reference. Where the reference's CUDA build contracts
// a*b + c into an fma (nvcc's default), the fma is written out explicitly so
// the rounding does not depend on the compiler's contraction choice.
// ---------------------------------------------------------------------------
__global__ void upcast_kernel(const uint16_t *in, float *out, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = bf2f(in[i]);
}
__global__ void denoised_kernel(const float *z, const float *mo, float sigma, float *o, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = fmaf(-mo[i], sigma, z[i]);
}
__global__ void znext_kernel(const float *noise, const float *den, float sn, float s_noise, float *o,
                             int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = fmaf(1.0f - sn, den[i], (sn * noise[i]) * s_noise);
}
__global__ void vcond_kernel(const uint16_t *z, const uint16_t *xp, float sigma, float *mo, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) mo[i] = (bf2f(z[i]) - bf2f(xp[i])) / sigma;
}
__global__ void fm_step_kernel(const uint16_t *z, const float *mo, float dt, uint16_t *zn, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) zn[i] = f2bf(fmaf(dt, mo[i], bf2f(z[i])));
}
__global__ void cfg_kernel(const float *c, const float *u, float g, float *o, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = fmaf(g, c[i], (1.0f - g) * u[i]);
}
// 4-wide variants of the sampler kernels: one thread per 4 consecutive
// elements (16-byte fp32 / 8-byte bf16 accesses), the same per-element
// arithmetic as the scalar kernels above (each functor's `one` is that
// arithmetic; `vec` applies it to 4 loaded elements). The last thread does
// its partial group element by element. Taken when every operand is 16-byte
// aligned; otherwise the scalar kernels run.
__device__ __forceinline__ void ld4b(const uint16_t *p, size_t i, float v[4]) {
    const u32x2_t w = *(const u32x2_t *)(p + i);
    v[0] = lo_bf(w[0]); v[1] = hi_bf(w[0]); v[2] = lo_bf(w[1]); v[3] = hi_bf(w[1]);
}
struct PwUpcast {
    const uint16_t *in; float *out;
    __device__ void one(size_t i) const { out[i] = bf2f(in[i]); }
    __device__ void vec(size_t i) const {
        float v[4];
        ld4b(in, i, v);
        *(f32x4_t *)(out + i) = {v[0], v[1], v[2], v[3]};
    }
};
struct PwDenoised {
    const float *z, *mo; float sigma; float *o;
    __device__ float f(float zv, float m) const { return fmaf(-m, sigma, zv); }
    __device__ void one(size_t i) const { o[i] = f(z[i], mo[i]); }
    __device__ void vec(size_t i) const {
        const f32x4_t a = *(const f32x4_t *)(z + i), b = *(const f32x4_t *)(mo + i);
        *(f32x4_t *)(o + i) = {f(a[0], b[0]), f(a[1], b[1]), f(a[2], b[2]), f(a[3], b[3])};
    }
};
struct PwZnext {
    const float *noise, *den; float sn, s_noise; float *o;
    __device__ float f(float nz, float d) const { return fmaf(1.0f - sn, d, (sn * nz) * s_noise); }
    __device__ void one(size_t i) const { o[i] = f(noise[i], den[i]); }
    __device__ void vec(size_t i) const {
        const f32x4_t a = *(const f32x4_t *)(noise + i), b = *(const f32x4_t *)(den + i);
        *(f32x4_t *)(o + i) = {f(a[0], b[0]), f(a[1], b[1]), f(a[2], b[2]), f(a[3], b[3])};
    }
};
struct PwVcond {
    const uint16_t *z, *xp; float sigma; float *mo;
    __device__ void one(size_t i) const { mo[i] = (bf2f(z[i]) - bf2f(xp[i])) / sigma; }
    __device__ void vec(size_t i) const {
        float a[4], b[4];
        ld4b(z, i, a);
        ld4b(xp, i, b);
        *(f32x4_t *)(mo + i) = {(a[0] - b[0]) / sigma, (a[1] - b[1]) / sigma, (a[2] - b[2]) / sigma,
                                (a[3] - b[3]) / sigma};
    }
};
struct PwFmStep {
    const uint16_t *z; const float *mo; float dt; uint16_t *zn;
    __device__ void one(size_t i) const { zn[i] = f2bf(fmaf(dt, mo[i], bf2f(z[i]))); }
    __device__ void vec(size_t i) const {
        float a[4];
        ld4b(z, i, a);
        const f32x4_t m = *(const f32x4_t *)(mo + i);
        *(u32x2_t *)(zn + i) = {pack_bf2(fmaf(dt, m[0], a[0]), fmaf(dt, m[1], a[1])),
                                pack_bf2(fmaf(dt, m[2], a[2]), fmaf(dt, m[3], a[3]))};
    }
};
struct PwCfg {
    const float *c, *u; float g; float *o;
    __device__ float f(float cv, float uv) const { return fmaf(g, cv, (1.0f - g) * uv); }
    __device__ void one(size_t i) const { o[i] = f(c[i], u[i]); }
    __device__ void vec(size_t i) const {
        const f32x4_t a = *(const f32x4_t *)(c + i), b = *(const f32x4_t *)(u + i);
        *(f32x4_t *)(o + i) = {f(a[0], b[0]), f(a[1], b[1]), f(a[2], b[2]), f(a[3], b[3])};
    }
};
template <class F>
__global__ void pw4_kernel(F f, int n) {
    const size_t i0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i0 + 4 <= (size_t)n) {
        f.vec(i0);
    } else {
        for (size_t i = i0; i < (size_t)n; i++) f.one(i);
    }
}
template <class F>
static void launch_pw4(const F &f, int n) {
    pw4_kernel<F><<<hd_cdiv(hd_cdiv(n, 4), 256), 256, 0, hd_stream()>>>(f, n);
}

extern "C" void hd_sched_bf16_upcast(const void *in, float *out, int n) {
    if (!in || !out || n <= 0) BAD("sched_bf16_upcast");
    if (al16(in) && al16(out)) launch_pw4(PwUpcast{(const uint16_t *)in, out}, n);
    else upcast_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>((const uint16_t *)in, out, n);
    hd_check_launch("sched_bf16_upcast");
}
extern "C" void hd_sched_denoised(const float *z, const float *mo, float sigma, float *o, int n) {
    if (!z || !mo || !o || n <= 0) BAD("sched_denoised");
    if (al16(z) && al16(mo) && al16(o)) launch_pw4(PwDenoised{z, mo, sigma, o}, n);
    else denoised_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(z, mo, sigma, o, n);
    hd_check_launch("sched_denoised");
}
extern "C" void hd_sched_z_next(const float *noise, const float *den, float sn, float s_noise,
                                float *o, int n) {
    if (!noise || !den || !o || n <= 0) BAD("sched_z_next");
    if (al16(noise) && al16(den) && al16(o)) launch_pw4(PwZnext{noise, den, sn, s_noise, o}, n);
    else znext_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(noise, den, sn, s_noise, o, n);
    hd_check_launch("sched_z_next");
}
extern "C" void hd_sched_vcond(const void *z, const void *xp, float sigma, float *mo, int n) {
    if (!z || !xp || !mo || n <= 0) BAD("sched_vcond");
    if (al16(z) && al16(xp) && al16(mo))
        launch_pw4(PwVcond{(const uint16_t *)z, (const uint16_t *)xp, sigma, mo}, n);
    else
        vcond_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>((const uint16_t *)z, (const uint16_t *)xp,
                                                               sigma, mo, n);
    hd_check_launch("sched_vcond");
}
extern "C" void hd_sched_flow_match_step(const void *z, const float *mo, float sigma,
                                         float sigma_next, void *zn, int n) {
    if (!z || !mo || !zn || n <= 0) BAD("sched_flow_match_step");
    if (al16(z) && al16(mo) && al16(zn))
        launch_pw4(PwFmStep{(const uint16_t *)z, mo, sigma_next - sigma, (uint16_t *)zn}, n);
    else
        fm_step_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>((const uint16_t *)z, mo,
                                                                 sigma_next - sigma, (uint16_t *)zn, n);
    hd_check_launch("sched_flow_match_step");
}
extern "C" void hd_sched_cfg_guided(const float *c, const float *u, float g, float *o, int n) {
    if (!c || !u || !o || n <= 0) BAD("sched_cfg_guided");
    if (al16(c) && al16(u) && al16(o)) launch_pw4(PwCfg{c, u, g, o}, n);
    else cfg_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(c, u, g, o, n);
    hd_check_launch("sched_cfg_guided");
}

// FlowUniPC pointwise steps (sched.cu:160-263). The per-step scalars
// r = sig_t/sig_s0, ah = alpha_t*h_phi_1 and ab = alpha_t*B_h are formed once
// in fp32 on the host (correctly rounded, as the per-element device
// expressions would be); a*b - c*d is fma(a, b, -(c*d)), x - a*b is fma(-a, b, x).
__global__ void unipc_convert_kernel(const float *smp, const float *mo, float sigma, float *conv,
                                     int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) conv[i] = fmaf(-sigma, mo[i], smp[i]);
}
__global__ void unipc_correct_kernel(const float *last, const float *mo0, const float *mo_old,
                                     const float *conv, float r, float ah, float ab, float rc0,
                                     float rc1, float inv_rk, int order, float *out, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float m0 = mo0[i];
    const float x = fmaf(r, last[i], -(ah * m0));
    const float d1t = conv[i] - m0;
    const float corr = order == 2 ? fmaf(rc0, (mo_old[i] - m0) * inv_rk, rc1 * d1t) : rc1 * d1t;
    out[i] = fmaf(-ab, corr, x);
}
__global__ void unipc_predict_kernel(const float *smp, const float *mo0, const float *mo_old,
                                     float r, float ah, float ab, float rp, float inv_rk, int order,
                                     float *out, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float m0 = mo0[i];
    float x = fmaf(r, smp[i], -(ah * m0));
    if (order == 2) x = fmaf(-ab, rp * ((mo_old[i] - m0) * inv_rk), x);
    out[i] = x;
}
extern "C" void hd_unipc_convert(const float *smp, const float *mo, float sigma, float *conv, int n) {
    if (!smp || !mo || !conv || n <= 0) BAD("unipc_convert");
    unipc_convert_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(smp, mo, sigma, conv, n);
    hd_check_launch("unipc_convert");
}
extern "C" void hd_unipc_correct(const float *last, const float *mo0, const float *mo_old,
                                 const float *conv, float sig_t, float sig_s0, float alpha_t,
                                 float h_phi_1, float B_h, float rc0, float rc1, float inv_rk,
                                 int order, float *out, int n) {
    if (!last || !mo0 || !conv || !out || n <= 0 || (order == 2 && !mo_old)) BAD("unipc_correct");
    unipc_correct_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(
        last, mo0, mo_old, conv, sig_t / sig_s0, alpha_t * h_phi_1, alpha_t * B_h, rc0, rc1, inv_rk,
        order, out, n);
    hd_check_launch("unipc_correct");
}
extern "C" void hd_unipc_predict(const float *smp, const float *mo0, const float *mo_old,
                                 float sig_t, float sig_s0, float alpha_t, float h_phi_1,
                                 float B_h, float rp, float inv_rk, int order, float *out, int n) {
    if (!smp || !mo0 || !out || n <= 0 || (order == 2 && !mo_old)) BAD("unipc_predict");
    unipc_predict_kernel<<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>(
        smp, mo0, mo_old, sig_t / sig_s0, alpha_t * h_phi_1, alpha_t * B_h, rp, inv_rk, order, out,
        n);
    hd_check_launch("unipc_predict");
}

// ---------------------------------------------------------------------------
// Patch (un)shuffle (generate.c:85-104, decode.c:10-27 index rule).
// Enumerates the token-major layout so the token side is coalesced.
// ---------------------------------------------------------------------------
template <int DIR, typename TO>  // DIR 0: img -> tok, 1: tok -> img
__global__ void patch_kernel(const float *src, TO *dst, int C, int Hp, int Wp, int p) {
    size_t feats = (size_t)C * p * p;
    size_t total = (size_t)Hp * Wp * feats;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    size_t tok = idx / feats;
    int f = idx % feats;
    int ch = f / (p * p), i = (f / p) % p, j = f % p;
    int r = tok / Wp, c = tok % Wp;
    size_t pix = ((size_t)ch * Hp * p + (size_t)(r * p + i)) * ((size_t)Wp * p) + (size_t)(c * p + j);
    if (DIR == 0) {
        float v = src[pix];
        if constexpr (sizeof(TO) == 2) dst[idx] = f2bf(v); else dst[idx] = v;
    } else {
        dst[pix] = src[idx];
    }
}
// 4-wide variant (p % 4 == 0, aligned operands): one thread moves 4
// consecutive pixels of a patch row (16-byte image accesses), the same index
// rule and conversion per element.
template <int DIR, typename TO>
__global__ void patch4_kernel(const float *src, TO *dst, int C, int Hp, int Wp, int p) {
    const size_t feats = (size_t)C * p * p;
    const size_t total = (size_t)Hp * Wp * feats / 4;
    const size_t idx4 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx4 >= total) return;
    const size_t idx = idx4 * 4;
    const size_t tok = idx / feats;
    const int f = idx % feats;
    const int ch = f / (p * p), i = (f / p) % p, j = f % p;
    const int r = tok / Wp, c = tok % Wp;
    const size_t pix = ((size_t)ch * Hp * p + (size_t)(r * p + i)) * ((size_t)Wp * p) + (size_t)(c * p + j);
    if (DIR == 0) {
        const f32x4_t v = *(const f32x4_t *)(src + pix);
        if constexpr (sizeof(TO) == 2)
            *(u32x2_t *)((uint16_t *)dst + idx) = {pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
        else
            *(f32x4_t *)((float *)dst + idx) = v;
    } else {
        *(f32x4_t *)((float *)dst + pix) = *(const f32x4_t *)(src + idx);
    }
}
template <int DIR, typename TO>
static void launch_patch(const float *src, TO *dst, int C, int Hp, int Wp, int p) {
    const size_t total = (size_t)C * Hp * Wp * p * p;
    if (p % 4 == 0 && al16(src) && al16(dst))
        patch4_kernel<DIR, TO><<<hd_cdiv(total / 4, 256), 256, 0, hd_stream()>>>(src, dst, C, Hp, Wp, p);
    else
        patch_kernel<DIR, TO><<<hd_cdiv(total, 256), 256, 0, hd_stream()>>>(src, dst, C, Hp, Wp, p);
}
extern "C" void hd_patchify_f32(const float *img, float *tok, int C, int Hp, int Wp, int p) {
    if (!img || !tok || C <= 0 || Hp <= 0 || Wp <= 0 || p <= 0) BAD("patchify");
    launch_patch<0, float>(img, tok, C, Hp, Wp, p);
    hd_check_launch("patchify");
}
extern "C" void hd_unpatchify_f32(const float *tok, float *img, int C, int Hp, int Wp, int p) {
    if (!img || !tok || C <= 0 || Hp <= 0 || Wp <= 0 || p <= 0) BAD("unpatchify");
    launch_patch<1, float>(tok, img, C, Hp, Wp, p);
    hd_check_launch("unpatchify");
}
extern "C" void hd_patchify_bf16(const float *img, void *tok, int C, int Hp, int Wp, int p) {
    if (!img || !tok || C <= 0 || Hp <= 0 || Wp <= 0 || p <= 0) BAD("patchify_bf16");
    launch_patch<0, uint16_t>(img, (uint16_t *)tok, C, Hp, Wp, p);
    hd_check_launch("patchify_bf16");
}

// ---------------------------------------------------------------------------
// Final-latent check (generate.c:1474-1496 fails closed on the raw output):
// per block, the count of NaN/Inf values and the min / max of the finite ones
// over a bf16 latent. Block b writes part[3b .. 3b+2]; the host folds the
// `blocks` triples. Grid-stride over 16-byte chunks (8 values per lane) with
// a scalar tail, so any n and alignment of 2 bytes is accepted.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void latent_stats_kernel(const uint16_t *__restrict__ z, int64_t n,
                                                           float *__restrict__ part) {
    float bad = 0.f, mn = INFINITY, mx = -INFINITY;
    auto one = [&](uint32_t bits16) {
        const float v = __uint_as_float(bits16 << 16);
        if ((bits16 & 0x7F80u) == 0x7F80u) {
            bad += 1.f;
        } else {
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
    };
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nthr = (int64_t)gridDim.x * blockDim.x;
    int64_t done = 0;
    if (((uintptr_t)z & 15) == 0) {
        const int64_t nch = n / 8;
        for (int64_t c = tid; c < nch; c += nthr) {
            const u32x4_t v = *(const u32x4_t *)(z + c * 8);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                one(v[e] & 0xFFFFu);
                one(v[e] >> 16);
            }
        }
        done = nch * 8;
    }
    for (int64_t i = done + tid; i < n; i += nthr) one(z[i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        bad += __shfl_xor(bad, o, 64);
        mn = fminf(mn, __shfl_xor(mn, o, 64));
        mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    }
    __shared__ float red[4][3];
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[w][0] = bad;
        red[w][1] = mn;
        red[w][2] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = red[0][0], lo = red[0][1], hi = red[0][2];
        for (int k = 1; k < (int)(blockDim.x >> 6); k++) {
            b += red[k][0];
            lo = fminf(lo, red[k][1]);
            hi = fmaxf(hi, red[k][2]);
        }
        part[3 * blockIdx.x] = b;
        part[3 * blockIdx.x + 1] = lo;
        part[3 * blockIdx.x + 2] = hi;
    }
}
// Internal (host.cpp): `blocks` <= HD_LATENT_STAT_BLOCKS partial triples.
extern "C" void hd_latent_stats(const void *z, int64_t n, float *part, int blocks) {
    if (!z || !part || n <= 0 || blocks <= 0) BAD("latent_stats");
    latent_stats_kernel<<<blocks, 256, 0, hd_stream()>>>((const uint16_t *)z, n, part);
    hd_check_launch("latent_stats");
}
