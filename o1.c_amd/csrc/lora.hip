// GPU LoRA merge-on-load: W = bf16(float(W) + s * (up @ down)), fp32 delta.
// Replaces hd_lora_merge_gpu (lora_merge.cu:35-104). One launch per target;
// the delta never reaches HBM. Two kernels:
//  - lora_merge_stream_kernel (R <= 64, R % 4 == 0): persistent blocks
//    stream W through an LDS ring, rank product on the bf16 matrix cores
//    with fp32 operands split in three bf16 parts;
//  - lora_merge_mfma_kernel (any other R): a block per 128 x 128 tile, rank
//    product on the fp32 matrix cores (v_mfma_f32_32x32x2_f32).
#include <stdio.h>

#include <map>
#include <vector>

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
template <int OCC>
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
        if (rc == LM_RC) {
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

// Split-operand variant on the bf16 matrix cores. Each fp32 operand x is
// held as three bf16 parts x = x0 + x1 + x2 (x0 = bf16(x), x1 =
// bf16(x - x0), x2 = bf16(x - x0 - x1); both differences are exact in fp32),
// and the rank product keeps the six part products down to 2^-16 of the
// leading one: a0b0 + a0b1 + a1b0 + a0b2 + a1b1 + a2b0 (summed smallest
// first). What is dropped is below 2^-24 of |ab|, fp32's own rounding level,
// so the delta matches an fp32 SGEMM up to summation order. Six
// v_mfma_f32_32x32x16_bf16 per 16 ranks replace eight v_mfma_f32_32x32x2_f32,
// about 2.7x less matrix-core time: the merge becomes bound by the
// read-modify-write of W in HBM. Ranks are staged 32 at a time: the six part
// planes of the up slice and of the transposed down slice are staged in LDS.
__device__ __forceinline__ void split3(float x, uint16_t &h0, uint16_t &h1, uint16_t &h2) {
    h0 = f2bf(x);
    const float r1 = x - bf2f(h0);
    h1 = f2bf(r1);
    h2 = f2bf(r1 - bf2f(h1));
}

// Streaming merge for R <= 64 (R % 4 == 0, K % 8 == 0): a persistent block of
// 8 waves per CU walks a contiguous run of 128 x 64 tiles of W (row strips
// first), so the whole launch is one stream of W reads and writes:
//  - W tiles go global -> LDS with buffer loads straight to LDS, two tiles
//    ahead, into a ring of three 16 KB slots; the update reads W from LDS in
//    the accumulator layout, writes the bf16 result back in place, and the
//    tile leaves with coalesced 16-byte buffer stores;
//  - the rank product uses the three-part split above (six bf16 part
//    products per fp32 product, in three accumulators); the up strip's part
//    planes are staged once per row strip and each wave keeps its B
//    fragments of them in registers for the whole strip; the down slice's
//    planes are staged once per tile, into one of two plane buffers, from
//    registers loaded a tile ahead, while the tile's MFMAs run (all twelve A
//    fragments of a tile are requested before its first MFMA);
//  - MFMA A = down^T (rows: W columns k), B = up (columns: W rows n), so a
//    lane holds four consecutive k of one W row per accumulator group.
// Every vector memory instruction in the loop is issued unconditionally
// (offsets past the data read as zero or are dropped), so the counts behind
// the hand-placed vmcnt waits for the ring hold on every path; register
// loads go through the compiler, which places their waits.
#define LT_N 128
#define LT_K 64
#define LT_LD 72   // plane row stride (bf16): 144-byte rows, conflict-free 16-byte reads
__device__ __forceinline__ __amdgpu_buffer_rsrc_t lt_rsrc(const void *base, uint32_t nbytes) {
    const uint64_t b = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((uint64_t)hi << 32) | lo), 0,
                                             __builtin_amdgcn_readfirstlane(nbytes), 0x00020000);
}
// One launch merges every target of a batch that shares (N, K, R): the
// tiles of all of them form one index space (target-major, then row strip,
// then column tile) that the persistent blocks split evenly, so small
// targets (the 1024-row k / v projections) no longer pay a launch and a
// pipeline fill each.
struct LmTarget {
    uint16_t *w;
    const float *up;
    const float *down;
    float scale;
};
__global__ __launch_bounds__(512, 1) void lora_merge_stream_kernel(const LmTarget *__restrict__ tg, int N,
                                                                 int K, int R, int ntk, int nstrip,
                                                                 int total) {
    __shared__ __attribute__((aligned(1024))) uint16_t wring[3][LT_N * LT_K];
    __shared__ __attribute__((aligned(16))) uint16_t upl[3][LT_N * LT_LD];
    __shared__ __attribute__((aligned(16))) uint16_t dpl[2][3][LT_K * LT_LD];
#if defined(__HIP_DEVICE_COMPILE__)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, lh = lane >> 5;
    const int tb = (int)((int64_t)blockIdx.x * total / gridDim.x);
    const int te = (int)((int64_t)(blockIdx.x + 1) * total / gridDim.x);
    if (tb >= te) return;
    const uint32_t OOB = 0x80000000u;
    const uint32_t w_bytes = (uint32_t)((size_t)N * K * 2), u_bytes = (uint32_t)((size_t)N * R * 4),
                   d_bytes = (uint32_t)((size_t)R * K * 4);
    const int tpt = nstrip * ntk;   // tiles per target
    // Each wave owns the 32 x 32 sub-tile of W its accumulator covers (rows
    // nblk*32.., columns kblk*32..) and alone loads, updates and stores it,
    // so W needs no barrier. Its 2 KB in a ring slot: instruction i, lane L
    // -> sub-tile row r = 16 i + L / 4, 16-byte position p = L % 4 of the
    // 64-byte row, holding column chunk c = p ^ ((r >> 2) & 3) (the XOR
    // spreads the update's 8-byte reads of 32 rows over the banks).
    const int kblk = wave & 1, nblk = wave >> 1;
    int wn[2], wc[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = i * 16 + (lane >> 2);
        wn[i] = nblk * 32 + r;
        wc[i] = kblk * 32 + ((lane & 3) ^ ((r >> 2) & 3)) * 8;
    }
    // tile coordinates (row strip, column tile) and ring slots advance
    // incrementally: a division by the runtime ntk costs tens of scalar
    // instructions, and every wave needs them for three tiles per step
    struct TC {
        int g, tn, tk;   // target, row strip, column tile
        bool ok;         // the tile exists (t < te)
        uint16_t *w;     // the target's tensors and scale (wave-uniform)
        const float *up, *down;
        float scale;
    };
    auto tc_load = [&](TC &c) {
        const int gg = c.g < total / tpt ? c.g : 0;   // past the last target: any valid entry
        c.w = tg[gg].w;
        c.up = tg[gg].up;
        c.down = tg[gg].down;
        c.scale = tg[gg].scale;
    };
    auto tc_next = [&](TC c, int t_next) {
        c.tk++;
        if (c.tk == ntk) {
            c.tk = 0;
            c.tn++;
            if (c.tn == nstrip) {
                c.tn = 0;
                c.g++;
                tc_load(c);
            }
        }
        c.ok = t_next < te;
        return c;
    };
    auto w_off = [&](const TC &c, int i) -> uint32_t {
        const int gn = c.tn * LT_N + wn[i], gk = c.tk * LT_K + wc[i];
        return c.ok && gn < N && gk < K ? (uint32_t)(gn * K + gk) * 2u : OOB;
    };
    auto issue_w = [&](const TC &c, int sl) {
        uint16_t *sub = wring[sl] + wave * 1024;
        const __amdgpu_buffer_rsrc_t rw = lt_rsrc(c.w, w_bytes);
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (HD_LDS void *)(sub + i * 512), 16, w_off(c, i), 0, 0,
                                                     0);
    };
    // down slice of a tile: ranks rr, rr + 1, columns kc .. kc + 3
    const int kc = (tid % 16) * 4, rr = (tid / 16) * 2;
    f32x4_t DA[2], DB[2];
    auto load_down = [&](const TC &c, f32x4_t (&d)[2]) {
        const __amdgpu_buffer_rsrc_t rd = lt_rsrc(c.down, d_bytes);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int r = rr + j, gk = c.tk * LT_K + kc;
            const uint32_t o = c.ok && r < R && gk < K ? (uint32_t)(r * K + gk) * 4u : OOB;
            d[j] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rd, o, 0, 0));
        }
    };
    // down registers -> part planes [k][r] of buffer b
    auto put_down = [&](const f32x4_t (&d)[2], int b) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint16_t h0[3], h1[3];
            split3(d[0][e], h0[0], h0[1], h0[2]);
            split3(d[1][e], h1[0], h1[1], h1[2]);
#pragma unroll
            for (int pl = 0; pl < 3; pl++)
                *(uint32_t *)(dpl[b][pl] + (kc + e) * LT_LD + rr) = (uint32_t)h0[pl] | ((uint32_t)h1[pl] << 16);
        }
    };
    auto stage_up = [&](const TC &c) {   // the up strip's part planes; drains the queue
        const __amdgpu_buffer_rsrc_t ru = lt_rsrc(c.up, u_bytes);
        const int row = tid / 4, r16 = (tid % 4) * 16, gn = c.tn * LT_N + row;
        float uv[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = r16 + 4 * j;
            const uint32_t o = gn < N && r < R ? (uint32_t)(gn * R + r) * 4u : OOB;
            const f32x4_t v = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ru, o, 0, 0));
            uv[4 * j] = v[0]; uv[4 * j + 1] = v[1]; uv[4 * j + 2] = v[2]; uv[4 * j + 3] = v[3];
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint16_t h[3][16];
#pragma unroll
        for (int e = 0; e < 16; e++) split3(uv[e], h[0][e], h[1][e], h[2][e]);
#pragma unroll
        for (int pl = 0; pl < 3; pl++)
#pragma unroll
            for (int q = 0; q < 2; q++) {
                u32x4_t v;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    v[e] = (uint32_t)h[pl][q * 8 + 2 * e] | ((uint32_t)h[pl][q * 8 + 2 * e + 1] << 16);
                *(u32x4_t *)(upl[pl] + row * LT_LD + r16 + q * 8) = v;
            }
    };
    // prologue: W(tb), down(tb), W(tb+1), down(tb+1); the planes of tile tb
    TC c0;                                // tile t
    c0.g = tb / tpt;
    c0.tn = (tb % tpt) / ntk;
    c0.tk = tb % ntk;
    c0.ok = true;
    tc_load(c0);
    TC c1 = tc_next(c0, tb + 1);          // tile t + 1
    TC c2 = tc_next(c1, tb + 2);          // tile t + 2
    int sl = 0;                           // ring slot of tile t
    issue_w(c0, 0);
    load_down(c0, DA);
    issue_w(c1, 1);
    load_down(c1, DB);
    int staged = c0.g * nstrip + c0.tn;   // target and row strip of the staged up planes
    stage_up(c0);          // vmcnt(0): down(tb) landed as well
    put_down(DA, tb & 1);
    // this wave's up fragments (B operands) stay in registers for the whole
    // row strip: read from the staged planes after each staging barrier
    bf16x8_t fb[4][3];
    auto read_up = [&]() {
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
#pragma unroll
            for (int p = 0; p < 3; p++)
                fb[ks][p] = *(const bf16x8_t *)(upl[p] + (nblk * 32 + l32) * LT_LD + ks * 16 + lh * 8);
    };
    bool need_up = true;
    // tile t splits down(t+1) (registers dsplit) for the next tile and loads
    // down(t+2) into the registers down(t) used (dload); the loop runs two
    // tiles per trip with the two register sets swapped, so no register
    // holding a load in flight is ever copied
    auto step = [&](int t, const f32x4_t (&dsplit)[2], f32x4_t (&dload)[2]) {
        // the planes of tile t are written; every wave is past the previous
        // tile's MFMAs (the other plane buffer is free)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (c0.g * nstrip + c0.tn != staged) {
            stage_up(c0);
            staged = c0.g * nstrip + c0.tn;
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            need_up = true;
        }
        if (need_up) {
            read_up();
            need_up = false;
        }
        // the MFMAs of tile t; the next tile's down slice is split into the
        // other plane buffer in between (independent VALU and LDS work)
        const int b = t & 1;
        // three accumulators by part-product order (2^-16: a2b0 a1b1 a0b2;
        // 2^-8: a1b0 a0b1; leading: a0b0), summed smallest first at the end:
        // three dependent MFMA chains of at most 12 instead of one of 24
        f32x16_t acc_s, acc_m, acc_l;
#pragma unroll
        for (int e = 0; e < 16; e++) acc_s[e] = acc_m[e] = acc_l[e] = 0.f;
        // every fragment of the tile is requested before the first MFMA
        bf16x8_t fa[4][3];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int rc = ks * 16 + lh * 8;
#pragma unroll
            for (int p = 0; p < 3; p++)
                fa[ks][p] = *(const bf16x8_t *)(dpl[b][p] + (kblk * 32 + l32) * LT_LD + rc);
        }
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const bf16x8_t *a = fa[ks], *bb = fb[ks];
            acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], bb[0], acc_s, 0, 0, 0);
            acc_m = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], bb[0], acc_m, 0, 0, 0);
            acc_l = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], bb[0], acc_l, 0, 0, 0);
            acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], bb[1], acc_s, 0, 0, 0);
            acc_m = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], bb[1], acc_m, 0, 0, 0);
            acc_s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], bb[2], acc_s, 0, 0, 0);
        }
        // the next tile's down slice into the other plane buffer (its reads
        // above are issued; the MFMAs run meanwhile)
        put_down(dsplit, b ^ 1);
        f32x16_t acc;
#pragma unroll
        for (int e = 0; e < 16; e++) acc[e] = acc_l[e] + (acc_m[e] + acc_s[e]);
        // loads for two tiles ahead, issued after down(t+1)'s registers are
        // consumed so that waiting for those never waits for these
        const int sl2 = sl == 0 ? 2 : sl - 1;   // tile t+2 takes the slot tile t-1 used
        issue_w(c2, sl2);
        load_down(c2, dload);
        // W update in LDS, in this wave's own sub-tile: row l32, columns
        // 8q + 4lh .. +3 (chunk q at position q ^ ((l32 >> 2) & 3)). W(t) of
        // this wave landed: newer than it are the loads down(t), W(t+1),
        // down(t+1), W(t+2) and down(t+2) (10) and the stores of t-2 and t-1
        // (4). The count allows only the 10 newer loads in flight, so it
        // holds even if the stores complete before older loads return (on
        // the first tiles a full drain came since). The ring is touched
        // through assembly only: the compiler would otherwise wait for every
        // buffer->LDS load in flight (vmcnt(0)) before each access.
        const uint16_t *sub = wring[sl] + wave * 1024;
        {
            uint32_t ad[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
                ad[q] = (uint32_t)(size_t)(HD_LDS void *)(sub + (l32 * 4 + (q ^ ((l32 >> 2) & 3))) * 8 + lh * 4);
            u32x2_t wv[4];
            asm volatile(
                "s_waitcnt vmcnt(10)\n\t"
                "ds_read_b64 %0, %4\n\tds_read_b64 %1, %5\n\tds_read_b64 %2, %6\n\tds_read_b64 %3, %7\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=v"(wv[0]), "=v"(wv[1]), "=v"(wv[2]), "=v"(wv[3])
                : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3])
                : "memory");
            u32x2_t o[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
                o[q] = (u32x2_t){pack_bf2(fmaf(c0.scale, acc[4 * q], lo_bf(wv[q][0])),
                                          fmaf(c0.scale, acc[4 * q + 1], hi_bf(wv[q][0]))),
                                 pack_bf2(fmaf(c0.scale, acc[4 * q + 2], lo_bf(wv[q][1])),
                                          fmaf(c0.scale, acc[4 * q + 3], hi_bf(wv[q][1])))};
            asm volatile(
                "ds_write_b64 %0, %1\n\tds_write_b64 %2, %3\n\tds_write_b64 %4, %5\n\tds_write_b64 %6, %7"
                :
                : "v"(ad[0]), "v"(o[0]), "v"(ad[1]), "v"(o[1]), "v"(ad[2]), "v"(o[2]), "v"(ad[3]), "v"(o[3])
                : "memory");
        }
        // the sub-tile leaves as it arrived (same lanes, same offsets)
        const __amdgpu_buffer_rsrc_t rw = lt_rsrc(c0.w, w_bytes);
        {
            // LDS operations of one wave complete in order, so these reads
            // see the update's writes above
            const uint32_t sa0 = (uint32_t)(size_t)(HD_LDS void *)(sub + lane * 8);
            const uint32_t sa1 = (uint32_t)(size_t)(HD_LDS void *)(sub + (64 + lane) * 8);
            u32x4_t v0, v1;
            asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                         : "=v"(v0), "=v"(v1) : "v"(sa0), "v"(sa1) : "memory");
            __builtin_amdgcn_raw_buffer_store_b128(v0, rw, w_off(c0, 0), 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(v1, rw, w_off(c0, 1), 0, 0);
        }
        c0 = c1;
        c1 = c2;
        c2 = tc_next(c2, t + 3);
        sl = sl == 2 ? 0 : sl + 1;
    };
    for (int t = tb; t < te; t += 2) {
        step(t, DB, DA);
        if (t + 1 < te) step(t + 1, DA, DB);
    }
    // no LDS-bound load may land after the block ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
}

extern "C" hd_status hd_lora_merge_gpu(hd_lora_entry *entries, size_t count, void *stream) {
    if (count == 0) return HD_OK;
    if (!entries) {
        hd_set_error("lora: null entries");
        return HD_ERR_MISSING;
    }
    hipStream_t st = stream ? (hipStream_t)stream : hd_stream();
    // every entry is checked before the GPU is touched
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
    }
    // Batches. An entry's level is one past the level of the last earlier
    // entry on the same weight (two adapters on one target merge in entry
    // order, as the reference's loop does); levels launch in order. Within a
    // level, the entries the streaming kernel takes (R <= 64, R % 4 == 0,
    // K % 8 == 0, W under 2 GiB) go into one launch per (N, K, R); the others
    // run the fp32 matrix-core kernel, one launch each.
    struct Key {
        int level, N, K, R;
        bool operator<(const Key &o) const {
            return level != o.level ? level < o.level
                                    : (N != o.N ? N < o.N : (K != o.K ? K < o.K : R < o.R));
        }
    };
    std::map<const void *, int> last;
    std::map<Key, std::vector<LmTarget>> stream_batches;
    std::vector<std::pair<int, size_t>> mfma_entries;   // (level, entry)
    int nlevels = 0;
    for (size_t i = 0; i < count; i++) {
        hd_lora_entry *e = &entries[i];
        auto it = last.find(e->base_dev);
        const int level = it == last.end() ? 0 : it->second + 1;
        last[e->base_dev] = level;
        nlevels = level + 1 > nlevels ? level + 1 : nlevels;
        const int N = (int)e->out_dim, K = (int)e->in_dim, R = (int)e->rank;
        const float scale = e->multiplier * e->alpha / (float)e->rank;   // lora_merge.cu:54
        const bool stream_ok = R <= 64 && R % 4 == 0 && K % 8 == 0 && (size_t)N * K * 2 < ((size_t)1 << 31);
        if (stream_ok)
            stream_batches[Key{level, N, K, R}].push_back(
                LmTarget{(uint16_t *)e->base_dev, (const float *)e->up_dev, (const float *)e->down_dev, scale});
        else
            mfma_entries.push_back({level, i});
    }
    // the batches' target lists in one small device buffer (freed after the
    // stream has run the launches, as the reference frees its delta scratch)
    size_t ntg = 0;
    for (auto &b : stream_batches) ntg += b.second.size();
    std::vector<LmTarget> host_tg;
    host_tg.reserve(ntg);
    for (auto &b : stream_batches) host_tg.insert(host_tg.end(), b.second.begin(), b.second.end());
    LmTarget *dev_tg = nullptr;
    if (ntg) {
        if (hipMalloc((void **)&dev_tg, ntg * sizeof(LmTarget)) != hipSuccess) {
            hd_set_error("lora: target list allocation failed");
            return HD_ERR_OOM;
        }
        if (hipMemcpyAsync(dev_tg, host_tg.data(), ntg * sizeof(LmTarget), hipMemcpyHostToDevice, st) !=
            hipSuccess) {
            (void)hipFree(dev_tg);
            hd_set_error("lora: target list upload failed");
            return HD_ERR_IO;
        }
    }
    int cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    hd_status status = HD_OK;
    size_t off = 0;
    auto sb = stream_batches.begin();
    for (int level = 0; level < nlevels && status == HD_OK; level++) {
        for (; sb != stream_batches.end() && sb->first.level == level; ++sb) {
            const int N = sb->first.N, K = sb->first.K, R = sb->first.R;
            const int ntk = hd_cdiv(K, LT_K), nstrip = hd_cdiv(N, LT_N);
            const long tot = (long)nstrip * ntk * (long)sb->second.size();
            if (tot >= ((long)1 << 31)) {
                hd_set_error("lora: batch of %zu targets has too many tiles", sb->second.size());
                status = HD_ERR_UNSUPPORTED;
                break;
            }
            lora_merge_stream_kernel<<<tot < cus ? (unsigned)tot : (unsigned)cus, 512, 0, st>>>(
                dev_tg + off, N, K, R, ntk, nstrip, (int)tot);
            off += sb->second.size();
        }
        for (auto &m : mfma_entries) {
            if (m.first != level || status != HD_OK) continue;
            hd_lora_entry *e = &entries[m.second];
            const int N = (int)e->out_dim, K = (int)e->in_dim, R = (int)e->rank;
            const float scale = e->multiplier * e->alpha / (float)e->rank;
            dim3 grid(hd_cdiv(K, LM_T), hd_cdiv(N, LM_T));
            lora_merge_mfma_kernel<2><<<grid, 256, 0, st>>>((uint16_t *)e->base_dev, (const float *)e->up_dev,
                                                            (const float *)e->down_dev, N, K, R, scale);
        }
        hipError_t err = hipGetLastError();
        if (status == HD_OK && err != hipSuccess) {
            hd_set_error("lora: merge launch failed: %s", hipGetErrorString(err));
            status = HD_ERR_RUNTIME;
        }
    }
    if (dev_tg) {
        (void)hipStreamSynchronize(st);
        (void)hipFree(dev_tg);
    }
    return status;
}
