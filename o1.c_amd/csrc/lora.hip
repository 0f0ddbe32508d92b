// GPU LoRA merge-on-load: W = bf16(float(W) + s * (up @ down)), fp32 delta.
// Replaces hd_lora_merge_gpu (lora_merge.cu:35-104). One kernel per target:
// a block owns a 64 x 128 tile of W, stages the matching 64 x r slice of
// `up` and r x 128 slice of `down` in LDS (r in chunks of 64), forms the
// fp32 delta in registers (4 x 8 outputs per thread) and does the single
// read-modify-write of W. The delta never reaches HBM; nothing is allocated.
#include <stdio.h>

#include "hd_common.hpp"
#include "../../include/hd_hip.h"
#include "../../include/hd_lora.h"

#define LR_TM 64
#define LR_TN 128
#define LR_RC 64

__global__ __launch_bounds__(256) void lora_merge_kernel(uint16_t *__restrict__ w,
                                                         const float *__restrict__ up,
                                                         const float *__restrict__ down, int N,
                                                         int K, int R, float scale) {
    __shared__ float su[LR_RC][LR_TM + 1];   // up^T slice: [r][row]
    __shared__ float sd[LR_RC][LR_TN];       // down slice: [r][col]
    const int n0 = blockIdx.y * LR_TM, k0 = blockIdx.x * LR_TN;
    const int tr = threadIdx.x / 16, tc = threadIdx.x % 16;   // 16 x 16 threads
    float acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = 0.f;
    for (int r0 = 0; r0 < R; r0 += LR_RC) {
        const int rc = min(LR_RC, R - r0);
        for (int i = threadIdx.x; i < LR_TM * LR_RC; i += 256) {
            int row = i / LR_RC, r = i % LR_RC;
            su[r][row] = (r < rc && n0 + row < N) ? up[(size_t)(n0 + row) * R + r0 + r] : 0.f;
        }
        for (int i = threadIdx.x; i < LR_RC * LR_TN; i += 256) {
            int r = i / LR_TN, c = i % LR_TN;
            sd[r][c] = (r < rc && k0 + c < K) ? down[(size_t)(r0 + r) * K + k0 + c] : 0.f;
        }
        __syncthreads();
        for (int r = 0; r < rc; r++) {
            float a[4], b[8];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = su[r][tr + 16 * i];
#pragma unroll
            for (int j = 0; j < 8; j++) b[j] = sd[r][tc + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 8; j++) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int n = n0 + tr + 16 * i;
        if (n >= N) continue;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int k = k0 + tc + 16 * j;
            if (k < K) {
                size_t o = (size_t)n * K + k;
                w[o] = f2bf(bf2f(w[o]) + scale * acc[i][j]);
            }
        }
    }
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
        dim3 grid(hd_cdiv(K, LR_TN), hd_cdiv(N, LR_TM));
        lora_merge_kernel<<<grid, 256, 0, st>>>((uint16_t *)e->base_dev, (const float *)e->up_dev,
                                                (const float *)e->down_dev, N, K, R, scale);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) {
            hd_set_error("lora: merge launch failed: %s", hipGetErrorString(err));
            return HD_ERR_RUNTIME;
        }
    }
    return HD_OK;
}
