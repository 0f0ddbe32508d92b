// GPU LoRA merge-on-load: W = bf16(float(W) + s * (up @ down)), fp32 delta.
// Replaces hd_lora_merge_gpu (lora_merge.cu:35-104). One kernel per target:
// a block owns a tile of W, stages the matching slice of `up` and of `down`
// in LDS (r in chunks of 64), forms the fp32 delta in registers and does the
// single read-modify-write of W. The delta never reaches HBM; nothing is
// allocated.
#include <stdio.h>

#include "hd_common.hpp"
#include "../../include/hd_hip.h"
#include "../../include/hd_lora.h"

// A block owns a 128 x 128 tile of W (two blocks per CU); the rank
// product runs on v_mfma_f32_32x32x2_f32 (fp32 products, fp32 accumulation,
// as an SGEMM does). Wave w computes rows [32w, 32w+32) x all 128 columns
// (4 accumulators); MFMA A = up (row = output row), B = down (column = output
// column), so a lane holds 16 rows of one column and the read-modify-write of
// W is coalesced along the row.
#define LM_T 128
#define LM_RC 64
#define LM_SU (LM_T * (LM_RC + 1))          // up slice [row][r], +1: conflict-free column reads
#define LM_SD (LM_RC * (LM_T + 32))         // down slice [r][col], +32: the half-waves read
                                            // consecutive r rows in opposite bank halves
#define LM_ST (LM_T * (LM_T + 8))           // fp32 delta tile [row][col] for the W update
template <int OCC, bool UNROLL = true>
__global__ __launch_bounds__(256, OCC) void lora_merge_mfma_kernel(uint16_t *__restrict__ w,
                                                              const float *__restrict__ up,
                                                              const float *__restrict__ down, int N,
                                                              int K, int R, float scale) {
    __shared__ __attribute__((aligned(16))) float lds[LM_SU + LM_SD > LM_ST ? LM_SU + LM_SD : LM_ST];
    float *su = lds, *sd = lds + LM_SU;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.y * LM_T, k0 = blockIdx.x * LM_T;
    const int l32 = lane & 31, lh = lane >> 5;
    const bool full = n0 + LM_T <= N && k0 + LM_T <= K && R % 4 == 0 && K % 8 == 0;
    // W update chunks of this thread: 8 x 8 consecutive weights, loaded
    // before the rank product so their latency hides under it
    u32x4_t wch[8];
    if (full) {
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int c = threadIdx.x + t * 256, row = c / 16, col = (c % 16) * 8;
            wch[t] = *(const u32x4_t *)(w + (size_t)(n0 + row) * K + k0 + col);
        }
    }
    f32x16_t acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[j][e] = 0.f;
    for (int r0 = 0; r0 < R; r0 += LM_RC) {
        const int rc = min(LM_RC, R - r0);
        if (full && rc == LM_RC) {
            // all 16 loads in flight before the first LDS store
            float4 ua[8], da[8];
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int i = threadIdx.x + t * 256;
                ua[t] = *(const float4 *)(up + (size_t)(n0 + i / (LM_RC / 4)) * R + r0 + (i % (LM_RC / 4)) * 4);
                da[t] = *(const float4 *)(down + (size_t)(r0 + i / (LM_T / 4)) * K + k0 + (i % (LM_T / 4)) * 4);
            }
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int i = threadIdx.x + t * 256;
                float *u = su + (i / (LM_RC / 4)) * (LM_RC + 1) + (i % (LM_RC / 4)) * 4;
                u[0] = ua[t].x; u[1] = ua[t].y; u[2] = ua[t].z; u[3] = ua[t].w;
                *(float4 *)(sd + (i / (LM_T / 4)) * (LM_T + 32) + (i % (LM_T / 4)) * 4) = da[t];
            }
        } else {
            for (int i = threadIdx.x; i < LM_T * LM_RC; i += 256) {
                const int row = i / LM_RC, r = i % LM_RC;
                su[row * (LM_RC + 1) + r] =
                    (r < rc && n0 + row < N) ? up[(size_t)(n0 + row) * R + r0 + r] : 0.f;
            }
            for (int i = threadIdx.x; i < LM_RC * LM_T; i += 256) {
                const int r = i / LM_T, c = i % LM_T;
                sd[r * (LM_T + 32) + c] = (r < rc && k0 + c < K) ? down[(size_t)(r0 + r) * K + k0 + c] : 0.f;
            }
        }
        __syncthreads();
        auto step = [&](int r) {
            const float a = su[(wave * 32 + l32) * (LM_RC + 1) + r + lh];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float b = sd[(r + lh) * (LM_T + 32) + j * 32 + l32];
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0, 0, 0);
            }
        };
        if (UNROLL && rc == LM_RC) {
            // unrolled: the operand reads of later steps issue ahead of the
            // MFMAs instead of one LDS round trip per step
#pragma unroll
            for (int r = 0; r < LM_RC; r += 2) step(r);
        } else {
            for (int r = 0; r < rc; r += 2) step(r);
        }
        __syncthreads();
    }
    // delta tile to LDS, row-major (acc[j][e]: row (e/4)*8 + lh*4 + e%4 of the
    // wave's 32, column j*32 + l32); row stride 136 floats keeps the two
    // half-waves' rows (4 apart) in opposite bank halves
    float *st = lds;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int e = 0; e < 16; e++)
            st[(wave * 32 + (e >> 2) * 8 + lh * 4 + (e & 3)) * (LM_T + 8) + j * 32 + l32] = acc[j][e];
    __syncthreads();
    if (full) {
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int c = threadIdx.x + t * 256, row = c / 16, col = (c % 16) * 8;
            const float4 d0 = *(const float4 *)(st + row * (LM_T + 8) + col);
            const float4 d1 = *(const float4 *)(st + row * (LM_T + 8) + col + 4);
            const float dv[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
            u32x4_t o;
#pragma unroll
            for (int e = 0; e < 4; e++)
                o[e] = pack_bf2(fmaf(scale, dv[2 * e], lo_bf(wch[t][e])),
                                fmaf(scale, dv[2 * e + 1], hi_bf(wch[t][e])));
            *(u32x4_t *)(w + (size_t)(n0 + row) * K + k0 + col) = o;
        }
    } else {
        for (int c = threadIdx.x; c < LM_T * LM_T; c += 256) {
            const int row = c / LM_T, col = c % LM_T, n = n0 + row, k = k0 + col;
            if (n < N && k < K) {
                const size_t o = (size_t)n * K + k;
                w[o] = f2bf(fmaf(scale, st[row * (LM_T + 8) + col], bf2f(w[o])));
            }
        }
    }
}

// hd_lora_set_family: 0 = the unrolled rank loop (default), 1 = the rolled
// loop (same-process comparisons; identical results)
static int g_lora_family = 0;
extern "C" int hd_lora_set_family(int family) {
    const int prev = g_lora_family;
    g_lora_family = family == 1 ? 1 : 0;
    return prev;
}

extern "C" hd_status hd_lora_merge_gpu(hd_lora_entry *entries, size_t count, void *stream) {
    if (count == 0) return HD_OK;
    if (!entries) {
        hd_set_error("lora: null entries");
        return HD_ERR_MISSING;
    }
    hipStream_t st = stream ? (hipStream_t)stream : hd_stream();
    for (size_t i = 0; i < count; i++) {
        hd_lora_entry *e = &entries[i];
        if (!e->base_dev || !e->up_dev || !e->down_dev || e->rank == 0 || e->in_dim == 0 ||
            e->out_dim == 0) {
            hd_set_error("lora: entry %zu has a null pointer or zero dim", i);
            return HD_ERR_MISSING;
        }
        if (e->rank > 256) {
            hd_set_error("lora: entry %zu rank %u > 256", i, e->rank);
            return HD_ERR_UNSUPPORTED;
        }
        const int N = (int)e->out_dim, K = (int)e->in_dim, R = (int)e->rank;
        const float scale = e->multiplier * e->alpha / (float)e->rank;   // lora_merge.cu:54
        dim3 grid(hd_cdiv(K, LM_T), hd_cdiv(N, LM_T));
        if (g_lora_family == 1)
            lora_merge_mfma_kernel<2, false><<<grid, 256, 0, st>>>((uint16_t *)e->base_dev, (const float *)e->up_dev,
                                                            (const float *)e->down_dev, N, K, R, scale);
        else
            lora_merge_mfma_kernel<2><<<grid, 256, 0, st>>>((uint16_t *)e->base_dev, (const float *)e->up_dev,
                                                            (const float *)e->down_dev, N, K, R, scale);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) {
            hd_set_error("lora: merge launch failed: %s", hipGetErrorString(err));
            return HD_ERR_RUNTIME;
        }
    }
    return HD_OK;
}
