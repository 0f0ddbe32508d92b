// Qwen3-VL vision tower for gfx950: LayerNorm / GELU / embedding / rotary /
// head-layout kernels and the 27-block forward over the library's GEMM and
// flash-attention kernels. Follows src/model/vision.c:345-640 and
// src/cuda/vision_kernels.cu of the reference (bf16 buffers at the same
// points; fp32 statistics and accumulation).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "hd_common.hpp"
#include "../../include/hd_gemm.h"
#include "../../include/hd_hip.h"
#include "../../include/hd_sdpa.h"
#include "../../include/hd_vision.h"

namespace {

constexpr int kH = HD_VISION_HIDDEN, kNH = HD_VISION_HEADS, kD = HD_VISION_HEAD_DIM;
constexpr int kI = HD_VISION_INTERMEDIATE, kIP = 4352;   // fc1 width padded to 64
constexpr int kO = HD_VISION_OUT_HIDDEN, kU = HD_VISION_MERGE_SIZE * HD_VISION_MERGE_SIZE;
constexpr int kDP = 128;                                  // head_dim of the flash kernel
constexpr int kQKV = 3 * kH;
constexpr int kNSide = 48;                                // sqrt(HD_VISION_NUM_POS)
constexpr int kDsLayers[HD_VISION_NUM_DS] = HD_VISION_DS_LAYERS;

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// One wave per row. x = bf16(a + b) when b is given (written to sum_out if
// non-null), then y = bf16((x - mean) * rsqrt(var + eps) * w + bias) with
// mean and var = E[x^2] - mean^2 in fp32 (vision_kernels.cu:50-87).
__global__ void __launch_bounds__(256) v_layernorm_kernel(const uint16_t *__restrict__ a,
                                                          const uint16_t *__restrict__ b,
                                                          uint16_t *__restrict__ sum_out,
                                                          const uint16_t *__restrict__ w,
                                                          const uint16_t *__restrict__ bias,
                                                          uint16_t *__restrict__ y, int rows,
                                                          int cols, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const size_t base = (size_t)row * cols;
    const int nch = cols >> 3;
    float s = 0.f, s2 = 0.f;
    for (int c = lane; c < nch; c += 64) {
        u32x4_t va = *(const u32x4_t *)(a + base + c * 8), vb = {0, 0, 0, 0};
        if (b) vb = *(const u32x4_t *)(b + base + c * 8);
        u32x4_t vs;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float x0 = lo_bf(va[j]), x1 = hi_bf(va[j]);
            if (b) {
                x0 = bfround(x0 + lo_bf(vb[j]));
                x1 = bfround(x1 + hi_bf(vb[j]));
                vs[j] = pack_bf2(x0, x1);
            }
            s += x0 + x1;
            s2 += x0 * x0 + x1 * x1;
        }
        if (b && sum_out) *(u32x4_t *)(sum_out + base + c * 8) = vs;
    }
    s = wsum(s);
    s2 = wsum(s2);
    const float mean = s / (float)cols;
    const float var = s2 / (float)cols - mean * mean;
    const float inv = rsqrtf(var + eps);
    for (int c = lane; c < nch; c += 64) {
        u32x4_t va = *(const u32x4_t *)(a + base + c * 8), vb = {0, 0, 0, 0};
        if (b) vb = *(const u32x4_t *)(b + base + c * 8);
        u32x4_t gw = *(const u32x4_t *)(w + c * 8), gb = {0, 0, 0, 0};
        if (bias) gb = *(const u32x4_t *)(bias + c * 8);
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float x0 = lo_bf(va[j]), x1 = hi_bf(va[j]);
            if (b) {
                x0 = bfround(x0 + lo_bf(vb[j]));
                x1 = bfround(x1 + hi_bf(vb[j]));
            }
            o[j] = pack_bf2((x0 - mean) * inv * lo_bf(gw[j]) + lo_bf(gb[j]),
                            (x1 - mean) * inv * hi_bf(gw[j]) + hi_bf(gb[j]));
        }
        *(u32x4_t *)(y + base + c * 8) = o;
    }
}

__device__ __forceinline__ float gelu_tanh_f(float v) {
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}
__device__ __forceinline__ float gelu_erf_f(float v) {
    return 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
}

// In place over [rows, ld] with `cols` live columns; columns [cols, ld)
// are set to zero (the padded K of the following GEMM). ld, cols % 8 == 0.
template <bool TANH>
__global__ void v_gelu_kernel(uint16_t *__restrict__ x, int rows, int cols, int ld) {
    const int cpr = ld >> 3;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * cpr) return;
    const int c = (int)(i % cpr) * 8;
    u32x4_t *p = (u32x4_t *)(x + (i / cpr) * ld + c);
    if (c >= cols) {
        *p = u32x4_t{0, 0, 0, 0};
        return;
    }
    u32x4_t v = *p;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float a = lo_bf(v[j]), b = hi_bf(v[j]);
        v[j] = TANH ? pack_bf2(gelu_tanh_f(a), gelu_tanh_f(b)) : pack_bf2(gelu_erf_f(a), gelu_erf_f(b));
    }
    *p = v;
}

template <bool TANH>
__global__ void v_gelu_flat_kernel(const uint16_t *__restrict__ x, uint16_t *__restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = bf2f(x[i]);
    y[i] = f2bf(TANH ? gelu_tanh_f(v) : gelu_erf_f(v));
}

// h[row] = bf16(patch[row] + bf16(sum_t wgt[t][row] * pe[idx[t][row]]))
// (vision.c:409-412: interpolated position embedding, then the residual add).
// pos_out (optional) receives the rounded interpolation; h == nullptr skips
// the sum (patch is then not read).
__global__ void v_embed_kernel(const uint16_t *__restrict__ patch, const uint16_t *__restrict__ pe,
                               const int *__restrict__ idx, const float *__restrict__ wgt,
                               uint16_t *__restrict__ pos_out, uint16_t *__restrict__ h, int rows,
                               int n, int hidden) {
    const int cpr = hidden >> 3;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * cpr) return;
    const int grow = (int)(i / cpr), c = (int)(i % cpr) * 8;
    const int row = grow % n;                  // tables are per image of n patches
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const float wt = wgt[(size_t)t * n + row];
        const u32x4_t v = *(const u32x4_t *)(pe + (size_t)idx[(size_t)t * n + row] * hidden + c);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc[2 * j] += wt * lo_bf(v[j]);
            acc[2 * j + 1] += wt * hi_bf(v[j]);
        }
    }
    u32x4_t pv = {0, 0, 0, 0};
    if (h) pv = *(const u32x4_t *)(patch + (size_t)grow * hidden + c);
    u32x4_t o, po;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float p0 = bfround(acc[2 * j]), p1 = bfround(acc[2 * j + 1]);
        po[j] = pack_bf2(p0, p1);
        o[j] = pack_bf2(lo_bf(pv[j]) + p0, hi_bf(pv[j]) + p1);
    }
    if (pos_out) *(u32x4_t *)(pos_out + (size_t)grow * hidden + c) = po;
    if (h) *(u32x4_t *)(h + (size_t)grow * hidden + c) = o;
}

// Rotary tables (vision.c:415-420, vision_kernels.cu:183-231): angle
// a = bf16(inv_freq[j] * coord) with coord the row for j < half/2 and the
// column otherwise; cos / sin [n, 2*half] fp32 repeat the half angles twice.
__global__ void v_rot_kernel(const float *__restrict__ inv, const int *__restrict__ coords,
                             uint16_t *__restrict__ rot, float *__restrict__ cosd,
                             float *__restrict__ sind, int n, int quarter) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int half = 2 * quarter;
    if (i >= n * half) return;
    const int s = i / half, k = i % half;
    const int j = k < quarter ? k : k - quarter;
    const float a = bfround(inv[j] * (float)(k < quarter ? coords[s] : coords[n + s]));
    if (rot) rot[(size_t)s * half + k] = f2bf(a);
    if (cosd) {
        const float c = cosf(a), sn = sinf(a);
        cosd[(size_t)s * 2 * half + k] = c;
        cosd[(size_t)s * 2 * half + half + k] = c;
        sind[(size_t)s * 2 * half + k] = sn;
        sind[(size_t)s * 2 * half + half + k] = sn;
    }
}

__global__ void v_cos_sin_kernel(const uint16_t *__restrict__ rot, float *__restrict__ cosd,
                                 float *__restrict__ sind, int n, int half) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * half) return;
    const int s = i / half, k = i % half;
    const float a = bf2f(rot[i]), c = cosf(a), sn = sinf(a);
    cosd[(size_t)s * 2 * half + k] = cosd[(size_t)s * 2 * half + half + k] = c;
    sind[(size_t)s * 2 * half + k] = sind[(size_t)s * 2 * half + half + k] = sn;
}

// qkv [R*n, 3, heads, D] (R images of n rows) -> q, k (rotary applied in
// fp32, one rounding, rope.cu:157-180), head-major [R, heads, n, DP] with
// columns [D, DP) zero (the flash kernel's head_dim-128 operands), and v
// written straight into the flash kernel's V^T operand [R*heads, DP, S_pad]
// (64-key tiles whose storage column p holds key p with bits 2 and 3
// exchanged; rows d >= D and keys >= n zero). One block per (64-row tile,
// image, head) stages the tile's q, k and v slices in LDS; 16-byte loads and
// stores. v itself (head-major like q) is written only when v_out is not
// null (the block-0 snapshots). D = 72, DP = 128 (D % 8 == 0, and the
// 144-byte head slices keep 16-byte alignment).
__global__ __launch_bounds__(256) void v_qkv_rope_vt_kernel(
    const uint16_t *__restrict__ qkv, const float *__restrict__ cosd, const float *__restrict__ sind,
    uint16_t *__restrict__ q, uint16_t *__restrict__ k, uint16_t *__restrict__ vt,
    uint16_t *__restrict__ v_out, int n, int s_pad) {
    constexpr int D = kD, DP = kDP, CH = D / 8, LD = D + 8;
    static_assert(D % 8 == 0 && D <= DP && DP % 8 == 0, "16-byte head slices");
    __shared__ __attribute__((aligned(16))) uint16_t t[3][64][LD];
    const int s0 = blockIdx.x * 64, h = blockIdx.y % kNH, img = blockIdx.y / kNH;
    const int bh = blockIdx.y;
    for (int i = threadIdx.x; i < 3 * 64 * CH; i += 256) {
        const int part = i / (64 * CH), r = (i / CH) % 64, c = (i % CH) * 8;
        u32x4_t val = {0, 0, 0, 0};
        if (s0 + r < n)
            val = *(const u32x4_t *)(qkv + ((size_t)img * n + s0 + r) * 3 * kNH * D +
                                     (size_t)(part * kNH + h) * D + c);
        *(u32x4_t *)&t[part][r][c] = val;
    }
    __syncthreads();
    const int half = D / 2;
    // q, k: rows [s0, s0 + 64) x 16 chunks of 8 columns (chunks >= CH zero)
    for (int i = threadIdx.x; i < 64 * (DP / 8); i += 256) {
        const int r = i / (DP / 8), c = (i % (DP / 8)) * 8, srow = s0 + r;
        if (srow >= n) continue;
        const size_t o = ((size_t)bh * n + srow) * DP + c;
        u32x4_t oq = {0, 0, 0, 0}, ok = {0, 0, 0, 0};
        if (c < D) {
            uint16_t rq[8], rk[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int d = c + e, dp = d < half ? d + half : d - half;
                const float cc = cosd[(size_t)srow * D + d], sn = sind[(size_t)srow * D + d];
                const float q0 = bf2f(t[0][r][d]), qh = bf2f(t[0][r][dp]);
                const float k0 = bf2f(t[1][r][d]), kh = bf2f(t[1][r][dp]);
                rq[e] = f2bf(d < half ? q0 * cc - qh * sn : q0 * cc + qh * sn);
                rk[e] = f2bf(d < half ? k0 * cc - kh * sn : k0 * cc + kh * sn);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                oq[e] = (uint32_t)rq[2 * e] | ((uint32_t)rq[2 * e + 1] << 16);
                ok[e] = (uint32_t)rk[2 * e] | ((uint32_t)rk[2 * e + 1] << 16);
            }
        }
        *(u32x4_t *)(q + o) = oq;
        *(u32x4_t *)(k + o) = ok;
        if (v_out) {
            u32x4_t ov = {0, 0, 0, 0};
            if (c < D) ov = *(const u32x4_t *)&t[2][r][c];
            *(u32x4_t *)(v_out + o) = ov;
        }
    }
    // V^T: rows d < DP, 8 chunks of 8 storage columns of this 64-key tile
    for (int i = threadIdx.x; i < DP * 8; i += 256) {
        const int d = i / 8, p0 = (i % 8) * 8;
        u32x4_t ov = {0, 0, 0, 0};
        if (d < D) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int pa = p0 + 2 * e, pb = pa + 1;
                const int ka = (pa & ~12) | ((pa & 4) << 1) | ((pa & 8) >> 1);
                const int kb = (pb & ~12) | ((pb & 4) << 1) | ((pb & 8) >> 1);
                ov[e] = (uint32_t)t[2][ka][d] | ((uint32_t)t[2][kb][d] << 16);
            }
        }
        *(u32x4_t *)(vt + ((size_t)bh * DP + d) * s_pad + s0 + p0) = ov;
    }
}

// flash output [n, heads*DP] (seq-major) -> [n, heads*D]; one thread per
// 8 consecutive columns (D % 8 == 0)
__global__ void v_unpad_heads_kernel(const uint16_t *__restrict__ in, uint16_t *__restrict__ out,
                                     int n, int heads, int D, int DP) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int cpr = D / 8;
    if (i >= (size_t)n * heads * cpr) return;
    const int c = (int)(i % cpr) * 8, h = (int)((i / cpr) % heads);
    const size_t s = i / ((size_t)cpr * heads);
    *(u32x4_t *)(out + (s * heads + h) * D + c) = *(const u32x4_t *)(in + (s * heads + h) * DP + c);
}

// rows x cols -> rows x ld, columns [cols, ld) zero (cols, ld % 8 == 0)
__global__ void v_pad_rows_kernel(const uint16_t *__restrict__ in, uint16_t *__restrict__ out,
                                  int rows, int cols, int ld) {
    const int cpr = ld >> 3;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * cpr) return;
    const size_t r = i / cpr;
    const int c = (int)(i % cpr) * 8;
    u32x4_t v = {0, 0, 0, 0};
    if (c < cols) v = *(const u32x4_t *)(in + r * cols + c);
    *(u32x4_t *)(out + r * ld + c) = v;
}

// Generic element kernels of vision_kernels.cu (the forward does not use
// them; kept for callers of the reference's kernel API).
__global__ void v_spatial_merge_kernel(const uint16_t *__restrict__ in, uint16_t *__restrict__ out,
                                       int gh, int gw, int hidden) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int mw = gw / 2;
    const size_t total = (size_t)(gh / 2) * mw * 4 * hidden;
    if (i >= total) return;
    const int c = (int)(i % hidden), slot = (int)((i / hidden) % 4);
    const size_t orow = i / ((size_t)4 * hidden);
    const int oh = (int)(orow / mw), ow = (int)(orow % mw);
    const int in_row = (2 * oh + slot / 2) * gw + 2 * ow + slot % 2;
    out[i] = in[(size_t)in_row * hidden + c];
}

__global__ void v_qkv_split_kernel(const uint16_t *__restrict__ qkv, uint16_t *__restrict__ q,
                                   uint16_t *__restrict__ k, uint16_t *__restrict__ v, int n,
                                   int heads, int d) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n * heads * d) return;
    const int dd = (int)(i % d), s = (int)((i / d) % n), h = (int)(i / ((size_t)d * n));
    const size_t src = (size_t)s * 3 * heads * d + (size_t)h * d + dd;
    q[i] = qkv[src];
    k[i] = qkv[src + (size_t)heads * d];
    v[i] = qkv[src + (size_t)2 * heads * d];
}

__global__ void v_attn_merge_kernel(const uint16_t *__restrict__ hm, uint16_t *__restrict__ sm,
                                    int heads, int n, int d) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n * heads * d) return;
    const int dd = (int)(i % d), h = (int)((i / d) % heads);
    const size_t s = i / ((size_t)d * heads);
    sm[i] = hm[((size_t)h * n + s) * d + dd];
}

// Rank of `row` among the set rows of mask: a block-wide count over
// mask[0, row) (256 threads, one value per block).
__device__ int mask_rank(const uint8_t *__restrict__ mask, int row) {
    __shared__ int part[4];
    int cnt = 0;
    for (int r = threadIdx.x; r < row; r += blockDim.x) cnt += mask[r] != 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = cnt;
    __syncthreads();
    return part[0] + part[1] + part[2] + part[3];
}

// forward.c:278-283 / vision_kernels.cu:343-364: one block per row.
__global__ void __launch_bounds__(256) v_masked_scatter_kernel(
    const uint16_t *__restrict__ dst, const uint8_t *__restrict__ mask,
    const uint16_t *__restrict__ src, uint16_t *__restrict__ out, int cols, int src_rows) {
    const int row = blockIdx.x;
    const uint16_t *from = dst + (size_t)row * cols;
    if (mask[row]) {
        const int r = mask_rank(mask, row);
        if (src_rows >= 0 && r >= src_rows) return;   // more set rows than embeddings
        from = src + (size_t)r * cols;
    }
    uint16_t *to = out + (size_t)row * cols;
    if (from == to) return;
    for (int c = threadIdx.x; c < cols; c += blockDim.x) to[c] = from[c];
}

// forward.c:363-370 / vision_kernels.cu:368-399: one block per row.
__global__ void __launch_bounds__(256) v_deepstack_kernel(
    const uint16_t *__restrict__ in, const uint8_t *__restrict__ mask,
    const uint16_t *__restrict__ emb, uint16_t *__restrict__ out, int cols, int emb_rows) {
    const int row = blockIdx.x;
    const uint16_t *ir = in + (size_t)row * cols;
    uint16_t *orow = out + (size_t)row * cols;
    if (mask[row]) {
        const int r = mask_rank(mask, row);
        if (emb_rows < 0 || r < emb_rows) {
            const uint16_t *er = emb + (size_t)r * cols;
            for (int c = threadIdx.x; c < cols; c += blockDim.x) orow[c] = f2bf(bf2f(ir[c]) + bf2f(er[c]));
            return;
        }
    }
    if (ir == orow) return;
    for (int c = threadIdx.x; c < cols; c += blockDim.x) orow[c] = ir[c];
}

bool bad(const char *what) {
    snprintf(hd_cuda_errbuf(), 512, "%s: bad args", what);
    return true;
}

void layernorm(const void *a, const void *b, void *sum_out, const void *w, const void *bias, void *y,
               int rows, int cols, float eps) {
    v_layernorm_kernel<<<hd_cdiv(rows, 4), 256, 0, hd_stream()>>>(
        (const uint16_t *)a, (const uint16_t *)b, (uint16_t *)sum_out, (const uint16_t *)w,
        (const uint16_t *)bias, (uint16_t *)y, rows, cols, eps);
}

template <bool TANH>
void gelu_padded(void *x, int rows, int cols, int ld) {
    v_gelu_kernel<TANH><<<hd_cdiv((size_t)rows * (ld / 8), 256), 256, 0, hd_stream()>>>(
        (uint16_t *)x, rows, cols, ld);
}

// ---- workspace layout ----
struct Layout {
    int64_t h, ar, ln, tmp, qkv, q, k, v, vt, f1, w2, cs, sn, gws, total;
};

int64_t al(int64_t b) { return (b + 255) & ~(int64_t)255; }

// R images of n patches each
Layout layout_of(int64_t R, int64_t n) {
    Layout L;
    int64_t b = 0;
    const int64_t N = R * n;
    // head-major operands [R, 16, n, 128] plus one 128-row tile of slack:
    // the flash kernel reads whole 128-row query / key tiles
    const int64_t hm = (R * kNH * n + 128) * kDP * 2;
    L.tmp = b; b += al(N * kH * 2);
    L.h = b; b += al(N * kH * 2);
    L.ar = b; b += al(N * kH * 2);
    L.ln = b; b += al(N * kH * 2);
    L.qkv = b; b += al(N * (kQKV > kNH * kDP ? kQKV : kNH * kDP) * 2);
    L.q = b; b += al(hm);
    L.k = b; b += al(hm);
    L.v = b; b += al(hm);
    L.vt = b; b += al(hd_flash_vt_bytes((int)R, kNH, (int)n));
    L.f1 = b; b += al(N * kIP * 2);
    L.w2 = b; b += al((int64_t)kH * kIP * 2);
    L.cs = b; b += al(n * kD * 4);
    L.sn = b; b += al(n * kD * 4);
    L.gws = b; b += al(hd_gemm_ws_bytes());   // split-K partials of the small GEMMs
    L.total = b;
    return L;
}

void snap(void *dst, const void *src, size_t bytes) {
    if (dst) (void)hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, hd_stream());
}

hd_status launch_err(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        hd_set_error("vision: %s: %s", what, hipGetErrorString(e));
        return HD_ERR_RUNTIME;
    }
    const char *ce = hd_cuda_last_error();
    if (ce && *ce) {
        hd_set_error("vision: %s: %s", what, ce);
        return HD_ERR_RUNTIME;
    }
    return HD_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Kernel API of vision_kernels.h
// ---------------------------------------------------------------------------
extern "C" void hd_vision_patch(const void *x, const void *w, const void *bias, void *y, int n,
                                int in_dim, int out_dim) {
    if (!x || !w || !y || n <= 0 || in_dim <= 0 || out_dim <= 0) {
        bad("vision_patch");
        return;
    }
    hd_linear(x, w, bias, y, n, out_dim, in_dim, 1);
}

extern "C" void hd_vision_layernorm(const void *x, const void *w, const void *b, void *y, int rows,
                                    int cols, float eps) {
    if (!x || !w || !y || rows <= 0 || cols <= 0 || cols % 8) {
        bad("vision_layernorm");
        return;
    }
    layernorm(x, nullptr, nullptr, w, b, y, rows, cols, eps);
    hd_check_launch("vision_layernorm");
}

extern "C" void hd_vision_gelu(const void *x, void *y, size_t n) {
    if (!x || !y || n == 0) {
        bad("vision_gelu");
        return;
    }
    v_gelu_flat_kernel<true><<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>((const uint16_t *)x,
                                                                        (uint16_t *)y, n);
    hd_check_launch("vision_gelu");
}

extern "C" void hd_vision_gelu_exact(const void *x, void *y, size_t n) {
    if (!x || !y || n == 0) {
        bad("vision_gelu_exact");
        return;
    }
    v_gelu_flat_kernel<false><<<hd_cdiv(n, 256), 256, 0, hd_stream()>>>((const uint16_t *)x,
                                                                         (uint16_t *)y, n);
    hd_check_launch("vision_gelu_exact");
}

extern "C" void hd_vision_pos_interp(const void *pos_embed, const int *idx, const float *wgt, void *y,
                                     int n, int hidden) {
    if (!pos_embed || !idx || !wgt || !y || n <= 0 || hidden <= 0 || hidden % 8) {
        bad("vision_pos_interp");
        return;
    }
    v_embed_kernel<<<hd_cdiv((size_t)n * (hidden / 8), 256), 256, 0, hd_stream()>>>(
        nullptr, (const uint16_t *)pos_embed, idx, wgt, (uint16_t *)y, nullptr, n, n, hidden);
    hd_check_launch("vision_pos_interp");
}

extern "C" void hd_vision_rot(const float *inv_freq, const int *coords, void *y, int n, int half) {
    if (!inv_freq || !coords || !y || n <= 0 || half <= 0 || half % 2) {
        bad("vision_rot");
        return;
    }
    v_rot_kernel<<<hd_cdiv((size_t)n * 2 * half, 256), 256, 0, hd_stream()>>>(
        inv_freq, coords, (uint16_t *)y, nullptr, nullptr, n, half);
    hd_check_launch("vision_rot");
}

extern "C" void hd_vision_rot_cos_sin(const void *rot, float *cosd, float *sind, int n, int half) {
    if (!rot || !cosd || !sind || n <= 0 || half <= 0) {
        bad("vision_rot_cos_sin");
        return;
    }
    v_cos_sin_kernel<<<hd_cdiv((size_t)n * 2 * half, 256), 256, 0, hd_stream()>>>(
        (const uint16_t *)rot, cosd, sind, n, 2 * half);
    hd_check_launch("vision_rot_cos_sin");
}

extern "C" void hd_vision_spatial_merge(const void *in, void *out, int gh, int gw, int hidden) {
    if (!in || !out || gh <= 0 || gw <= 0 || hidden <= 0 || gh % 2 || gw % 2) {
        bad("vision_spatial_merge");
        return;
    }
    const size_t total = (size_t)gh * gw * hidden;
    v_spatial_merge_kernel<<<hd_cdiv(total, 256), 256, 0, hd_stream()>>>(
        (const uint16_t *)in, (uint16_t *)out, gh, gw, hidden);
    hd_check_launch("vision_spatial_merge");
}

extern "C" void hd_vision_qkv_split(const void *qkv, void *q, void *k, void *v, int n, int heads,
                                    int d) {
    if (!qkv || !q || !k || !v || n <= 0 || heads <= 0 || d <= 0) {
        bad("vision_qkv_split");
        return;
    }
    v_qkv_split_kernel<<<hd_cdiv((size_t)n * heads * d, 256), 256, 0, hd_stream()>>>(
        (const uint16_t *)qkv, (uint16_t *)q, (uint16_t *)k, (uint16_t *)v, n, heads, d);
    hd_check_launch("vision_qkv_split");
}

extern "C" void hd_vision_attn_merge(const void *hm, void *sm, int heads, int n, int d) {
    if (!hm || !sm || heads <= 0 || n <= 0 || d <= 0) {
        bad("vision_attn_merge");
        return;
    }
    v_attn_merge_kernel<<<hd_cdiv((size_t)n * heads * d, 256), 256, 0, hd_stream()>>>(
        (const uint16_t *)hm, (uint16_t *)sm, heads, n, d);
    hd_check_launch("vision_attn_merge");
}

extern "C" void hd_vision_masked_scatter(const void *dst, const uint8_t *mask, const void *src,
                                         void *out, int rows, int cols) {
    if (!dst || !mask || !src || !out || rows <= 0 || cols <= 0) {
        bad("vision_masked_scatter");
        return;
    }
    v_masked_scatter_kernel<<<rows, 256, 0, hd_stream()>>>((const uint16_t *)dst, mask,
                                                           (const uint16_t *)src, (uint16_t *)out,
                                                           cols, -1);
    hd_check_launch("vision_masked_scatter");
}

extern "C" void hd_vision_deepstack_inject(const void *in, const uint8_t *mask, const void *emb,
                                           void *out, int rows, int cols) {
    if (!in || !mask || !emb || !out || rows <= 0 || cols <= 0) {
        bad("vision_deepstack_inject");
        return;
    }
    v_deepstack_kernel<<<rows, 256, 0, hd_stream()>>>((const uint16_t *)in, mask,
                                                      (const uint16_t *)emb, (uint16_t *)out, cols, -1);
    hd_check_launch("vision_deepstack_inject");
}

// Bounded variants for the forward (rows past `src_rows` set rows are left alone).
extern "C" void hd_vision_masked_scatter_n(const void *dst, const uint8_t *mask, const void *src,
                                           void *out, int rows, int cols, int src_rows) {
    v_masked_scatter_kernel<<<rows, 256, 0, hd_stream()>>>((const uint16_t *)dst, mask,
                                                           (const uint16_t *)src, (uint16_t *)out,
                                                           cols, src_rows);
}
extern "C" void hd_vision_deepstack_inject_n(const void *in, const uint8_t *mask, const void *emb,
                                             void *out, int rows, int cols, int emb_rows) {
    v_deepstack_kernel<<<rows, 256, 0, hd_stream()>>>((const uint16_t *)in, mask,
                                                      (const uint16_t *)emb, (uint16_t *)out, cols,
                                                      emb_rows);
}

// ---------------------------------------------------------------------------
// Tower API of vision.h
// ---------------------------------------------------------------------------
extern "C" void hd_vision_layout(int64_t n, int64_t m, hd_vision_offsets *o) {
    (void)m;
    if (!o) return;
    const Layout L = layout_of(1, n);
    for (int64_t *p = &o->patch_out; p <= &o->total_bytes; p++) *p = L.total;   // absent: empty
    o->patch_out = L.tmp;
    o->h_a = L.h;
    o->attn_resid = L.ar;
    o->ln1 = L.ln;
    o->qkv = L.qkv;
    o->q = L.q;
    o->k = L.k;
    o->v = L.v;
    o->scores = L.vt;
    o->fc1 = L.f1;
    o->fc2 = L.w2;
    o->cosf = L.cs;
    o->sinf = L.sn;
    o->total_bytes = L.total;
}

extern "C" int64_t hd_vision_workspace_bytes(int64_t n) {
    if (n <= 0) return 0;
    return layout_of(1, n).total;
}

extern "C" int64_t hd_vision_workspace_bytes_multi(int images, int64_t n) {
    if (n <= 0 || images <= 0) return 0;
    return layout_of(images, n).total;
}

extern "C" int64_t hd_vision_tables_bytes(int64_t n) {
    if (n <= 0) return 0;
    return n * 4 * 4 + n * 4 * 4 + n * 2 * 4 + 18 * 4;
}

extern "C" hd_status hd_vision_resolve(const hd_weight_store *wstore, hd_vision_binding *out) {
    if (!wstore || !out) {
        hd_set_error("vision: null argument in resolve");
        return HD_ERR_MISSING;
    }
    memset(out, 0, sizeof(*out));
    char name[256];
    auto find = [&](const void **dst, const char *nm) -> bool {
        *dst = hd_weight_store_find(wstore, nm);
        if (!*dst) hd_set_error("vision: missing %s", nm);
        return *dst != nullptr;
    };
    if (!find(&out->patch_proj_w, "model.visual.patch_embed.proj.weight") ||
        !find(&out->patch_proj_b, "model.visual.patch_embed.proj.bias") ||
        !find(&out->pos_embed, "model.visual.pos_embed.weight"))
        return HD_ERR_MISSING;
    static const char *bsuf[12] = {"norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias",
                                   "attn.qkv.weight", "attn.qkv.bias", "attn.proj.weight",
                                   "attn.proj.bias", "mlp.linear_fc1.weight", "mlp.linear_fc1.bias",
                                   "mlp.linear_fc2.weight", "mlp.linear_fc2.bias"};
    for (int i = 0; i < HD_VISION_DEPTH; i++) {
        const void **dst = &out->blocks[i].norm1_w;
        for (int k = 0; k < 12; k++) {
            snprintf(name, sizeof(name), "model.visual.blocks.%d.%s", i, bsuf[k]);
            if (!find(dst + k, name)) return HD_ERR_MISSING;
        }
    }
    static const char *msuf[6] = {"norm.weight", "norm.bias", "linear_fc1.weight",
                                  "linear_fc1.bias", "linear_fc2.weight", "linear_fc2.bias"};
    for (int j = -1; j < HD_VISION_NUM_DS; j++) {
        const void **dst = j < 0 ? &out->merger.norm_w : &out->deepstack[j].norm_w;
        for (int k = 0; k < 6; k++) {
            if (j < 0) snprintf(name, sizeof(name), "model.visual.merger.%s", msuf[k]);
            else snprintf(name, sizeof(name), "model.visual.deepstack_merger_list.%d.%s", j, msuf[k]);
            if (!find(dst + k, name)) return HD_ERR_MISSING;
        }
    }
    return HD_OK;
}

extern "C" hd_status hd_vision_prepare_tables(hd_vision_workspace *ws, int n, int grid_h, int grid_w) {
    if (!ws || n <= 0 || grid_h <= 0 || grid_w <= 0 || grid_h % 2 || grid_w % 2 ||
        n != grid_h * grid_w) {
        hd_set_error("vision: bad prepare_tables args");
        return HD_ERR_MISSING;
    }
    if (!ws->tables) {
        hd_set_error("vision: table region not bound");
        return HD_ERR_MISSING;
    }
    if (ws->tables_n == n && ws->tables_gh == grid_h && ws->tables_gw == grid_w && ws->pos_idx)
        return HD_OK;
    // vision.c:215-285: bilinear taps (align-corners) of the 48x48 position
    // grid and the (row, col) coordinates, rows in merge-block order
    std::vector<int> idx(4 * (size_t)n), co(2 * (size_t)n);
    std::vector<float> wgt(4 * (size_t)n);
    const int M = HD_VISION_MERGE_SIZE;
    int row = 0;
    for (int bh = 0; bh < grid_h / M; bh++)
        for (int bw = 0; bw < grid_w / M; bw++)
            for (int ih = 0; ih < M; ih++)
                for (int iw = 0; iw < M; iw++, row++) {
                    const int h = bh * M + ih, w = bw * M + iw;
                    const float hf = grid_h > 1 ? (float)h * (float)(kNSide - 1) / (float)(grid_h - 1) : 0.f;
                    const float wf = grid_w > 1 ? (float)w * (float)(kNSide - 1) / (float)(grid_w - 1) : 0.f;
                    const int h0 = (int)hf, w0 = (int)wf;
                    const int h1 = h0 + 1 < kNSide ? h0 + 1 : kNSide - 1;
                    const int w1 = w0 + 1 < kNSide ? w0 + 1 : kNSide - 1;
                    const float dh = hf - (float)h0, dw = wf - (float)w0;
                    idx[row] = h0 * kNSide + w0;
                    idx[n + row] = h0 * kNSide + w1;
                    idx[2 * n + row] = h1 * kNSide + w0;
                    idx[3 * n + row] = h1 * kNSide + w1;
                    wgt[row] = (1.f - dh) * (1.f - dw);
                    wgt[n + row] = (1.f - dh) * dw;
                    wgt[2 * n + row] = dh * (1.f - dw);
                    wgt[3 * n + row] = dh * dw;
                    co[row] = h;
                    co[n + row] = w;
                }
    float inv[18];
    for (int k = 0; k < 18; k++) inv[k] = 1.0f / powf(10000.0f, (float)(2 * k) / 36.0f);
    uint8_t *t = (uint8_t *)ws->tables;
    int *d_idx = (int *)t;
    float *d_wgt = (float *)(t + (size_t)n * 16);
    int *d_co = (int *)(t + (size_t)n * 32);
    float *d_inv = (float *)(t + (size_t)n * 40);
    hipStream_t st = hd_stream();
    if (hipMemcpyAsync(d_idx, idx.data(), idx.size() * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(d_wgt, wgt.data(), wgt.size() * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(d_co, co.data(), co.size() * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(d_inv, inv, sizeof(inv), hipMemcpyHostToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        hd_set_error("vision: table upload failed");
        return HD_ERR_IO;
    }
    ws->pos_idx = d_idx;
    ws->pos_wgt = d_wgt;
    ws->rot_coords = d_co;
    ws->rot_inv = d_inv;
    ws->tables_n = n;
    ws->tables_gh = grid_h;
    ws->tables_gw = grid_w;
    return HD_OK;
}

// R images of the same grid_h x grid_w: every GEMM, LayerNorm and
// elementwise kernel runs over the R*n rows at once, attention per image
// (the flash kernel's batch dimension).
static hd_status forward_impl(const hd_vision_binding *bw, hd_vision_workspace *ws,
                              const void *pixel_values, int R, int n, int grid_h, int grid_w,
                              void *image_embeds_out, void *const *deepstack_out) {
    if (!bw || !ws || !pixel_values || R <= 0 || n <= 0 || grid_h <= 0 || grid_w <= 0 ||
        !image_embeds_out || !ws->patch_out) {
        hd_set_error("vision: null argument");
        return HD_ERR_MISSING;
    }
    if (grid_h % 2 || grid_w % 2 || n != grid_h * grid_w) {
        hd_set_error("vision: grid %dx%d (n=%d) not divisible by merge size 2", grid_h, grid_w, n);
        return HD_ERR_MISSING;
    }
    if (!ws->pos_idx || ws->tables_n != n || ws->tables_gh != grid_h || ws->tables_gw != grid_w) {
        hd_set_error("vision: persistent tables not prepared for this grid");
        return HD_ERR_MISSING;
    }
    hd_cuda_clear_error();
    const int m = R * (n / kU), N = R * n;
    const float eps = 1e-6f, scale = (float)(1.0 / sqrt((double)kD));
    const Layout L = layout_of(R, n);
    uint8_t *base = (uint8_t *)ws->patch_out;
    uint16_t *tmp = (uint16_t *)(base + L.tmp), *h = (uint16_t *)(base + L.h);
    uint16_t *ar = (uint16_t *)(base + L.ar), *ln = (uint16_t *)(base + L.ln);
    uint16_t *qkv = (uint16_t *)(base + L.qkv), *q = (uint16_t *)(base + L.q);
    uint16_t *k = (uint16_t *)(base + L.k), *v = (uint16_t *)(base + L.v);
    uint16_t *vt = (uint16_t *)(base + L.vt), *f1 = (uint16_t *)(base + L.f1);
    uint16_t *w2 = (uint16_t *)(base + L.w2);
    float *cs = (float *)(base + L.cs), *sn = (float *)(base + L.sn);
    void *gws = base + L.gws;
    const int64_t gwsb = hd_gemm_ws_bytes();
    hipStream_t st = hd_stream();
    const size_t nH = (size_t)N * kH * 2;
    hd_status s;

    // patch embed + position embedding, rotary tables
    hd_linear_ws(pixel_values, bw->patch_proj_w, bw->patch_proj_b, tmp, N, kH, HD_VISION_PATCH_DIM, gws, gwsb);
    v_embed_kernel<<<hd_cdiv((size_t)N * (kH / 8), 256), 256, 0, st>>>(
        tmp, (const uint16_t *)bw->pos_embed, (const int *)ws->pos_idx, (const float *)ws->pos_wgt,
        nullptr, h, N, n, kH);
    v_rot_kernel<<<hd_cdiv((size_t)n * (kD / 2), 256), 256, 0, st>>>(
        (const float *)ws->rot_inv, (const int *)ws->rot_coords, nullptr, cs, sn, n, kD / 4);
    if ((s = launch_err("embedding")) != HD_OK) return s;

    layernorm(h, nullptr, nullptr, bw->blocks[0].norm1_w, bw->blocks[0].norm1_b, ln, N, kH, eps);
    int ds_j = 0;
    for (int i = 0; i < HD_VISION_DEPTH; i++) {
        const hd_vision_block_binding *b = &bw->blocks[i];
        void **s0 = i == 0 ? ws->block0_snaps : nullptr;
        if (s0) {
            snap(s0[HD_B0_INPUT], h, nH);
            snap(s0[HD_B0_NORM1], ln, nH);
        }
        hd_linear_ws(ln, b->qkv_w, b->qkv_b, qkv, N, kQKV, kH, gws, gwsb);
        if (s0) snap(s0[HD_B0_QKV], qkv, (size_t)N * kQKV * 2);
        v_qkv_rope_vt_kernel<<<dim3((unsigned)((n + 63) / 64), (unsigned)(R * kNH)), 256, 0, st>>>(
            qkv, cs, sn, q, k, vt, s0 ? v : nullptr, n, (int)((n + 63) / 64 * 64));
        if (s0) {
            snap(s0[HD_B0_Q], q, (size_t)R * kNH * n * kDP * 2);
            snap(s0[HD_B0_K], k, (size_t)R * kNH * n * kDP * 2);
            snap(s0[HD_B0_V], v, (size_t)R * kNH * n * kDP * 2);
        }
        // full attention per image over the zero-padded heads; output
        // [R*n, 16*128] (seq-major) into qkv
        if (hd_flash_attention(q, k, vt, nullptr, qkv, R, kNH, kNH, n, kDP, 0, scale, 1)) {
            hd_set_error("vision: attention failed: %s", hd_cuda_last_error());
            return HD_ERR_RUNTIME;
        }
        v_unpad_heads_kernel<<<hd_cdiv((size_t)N * kH / 8, 256), 256, 0, st>>>(qkv, ln, N, kNH, kD, kDP);
        if (s0) snap(s0[HD_B0_ATTN_MERGED], ln, nH);
        hd_linear_ws(ln, b->proj_w, b->proj_b, tmp, N, kH, kH, gws, gwsb);
        if (s0) snap(s0[HD_B0_PROJ], tmp, nH);
        // attn_resid = bf16(h + proj); ln = LayerNorm2(attn_resid)
        layernorm(h, tmp, ar, b->norm2_w, b->norm2_b, ln, N, kH, eps);
        if (s0) {
            snap(s0[HD_B0_ATTN_RESID], ar, nH);
            snap(s0[HD_B0_NORM2], ln, nH);
        }
        hd_linear_ld(ln, b->fc1_w, b->fc1_b, f1, N, kI, kH, kIP);
        gelu_padded<true>(f1, N, kI, kIP);
        if (s0) snap(s0[HD_B0_FC1], f1, (size_t)N * kIP * 2);
        v_pad_rows_kernel<<<hd_cdiv((size_t)kH * (kIP / 8), 256), 256, 0, st>>>(
            (const uint16_t *)b->fc2_w, w2, kH, kI, kIP);
        hd_linear_ws(f1, w2, b->fc2_b, tmp, N, kH, kIP, gws, gwsb);
        if (s0) snap(s0[HD_B0_FC2], tmp, nH);
        // h = bf16(attn_resid + fc2), then the next LayerNorm (next block's
        // norm1, or the final merger's norm over 1152)
        const bool last = i + 1 == HD_VISION_DEPTH;
        const void *nw = last ? bw->merger.norm_w : bw->blocks[i + 1].norm1_w;
        const void *nb = last ? bw->merger.norm_b : bw->blocks[i + 1].norm1_b;
        layernorm(ar, tmp, h, nw, nb, ln, N, kH, eps);
        if (s0) snap(s0[HD_B0_OUTPUT], h, nH);
        if (i == 0) snap(ws->block0_snap, h, nH);
        snap(ws->block_out_snaps[i], h, nH);
        if ((s = launch_err("block")) != HD_OK) return s;

        const bool ds_here = ds_j < HD_VISION_NUM_DS && kDsLayers[ds_j] == i;
        if (ds_here && deepstack_out) {
            // deepstack merger: LayerNorm over 4 rows viewed as one 4608 row
            const hd_vision_merger_binding *d = &bw->deepstack[ds_j];
            void **sd = ws->ds_merger_snaps[ds_j];
            uint16_t *dn = ar;                 // [m, 4608] == [N, 1152]; attn_resid is dead here
            layernorm(h, nullptr, nullptr, d->norm_w, d->norm_b, dn, m, kU * kH, eps);
            snap(sd[0], dn, nH);
            hd_linear_ws(dn, d->fc1_w, d->fc1_b, f1, m, kU * kH, kU * kH, gws, gwsb);
            snap(sd[1], f1, (size_t)m * kU * kH * 2);
            gelu_padded<false>(f1, m, kU * kH, kU * kH);
            snap(sd[2], f1, (size_t)m * kU * kH * 2);
            if (deepstack_out[ds_j])
                hd_linear_ws(f1, d->fc2_w, d->fc2_b, deepstack_out[ds_j], m, kO, kU * kH, gws, gwsb);
            if (deepstack_out[ds_j]) snap(sd[3], deepstack_out[ds_j], (size_t)m * kO * 2);
            if ((s = launch_err("deepstack merger")) != HD_OK) return s;
        }
        if (ds_here) ds_j++;
    }
    // final merger: ln holds LayerNorm(h) over 1152; view as [m, 4608]
    void **sm = ws->merger_snaps;
    snap(sm[0], ln, nH);
    snap(sm[1], ln, nH);
    hd_linear_ws(ln, bw->merger.fc1_w, bw->merger.fc1_b, f1, m, kU * kH, kU * kH, gws, gwsb);
    snap(sm[2], f1, (size_t)m * kU * kH * 2);
    gelu_padded<false>(f1, m, kU * kH, kU * kH);
    snap(sm[3], f1, (size_t)m * kU * kH * 2);
    hd_linear_ws(f1, bw->merger.fc2_w, bw->merger.fc2_b, image_embeds_out, m, kO, kU * kH, gws, gwsb);
    snap(sm[4], image_embeds_out, (size_t)m * kO * 2);
    return launch_err("merger");
}

extern "C" hd_status hd_vision_forward(const hd_vision_binding *bw, hd_vision_workspace *ws,
                                       const void *pixel_values, int n, int grid_h, int grid_w,
                                       void *image_embeds_out, void *deepstack_out[HD_VISION_NUM_DS]) {
    return forward_impl(bw, ws, pixel_values, 1, n, grid_h, grid_w, image_embeds_out, deepstack_out);
}

extern "C" hd_status hd_vision_forward_multi(const hd_vision_binding *bw, hd_vision_workspace *ws,
                                             const void *pixel_values, int images, int n, int grid_h,
                                             int grid_w, void *image_embeds_out,
                                             void *deepstack_out[HD_VISION_NUM_DS]) {
    return forward_impl(bw, ws, pixel_values, images, n, grid_h, grid_w, image_embeds_out,
                        deepstack_out);
}
