// Flash attention for gfx950 (head_dim 128, GQA, fp32 online softmax) and
// the hd_sdpa_* plan API that replaces the reference's cuDNN-frontend SDPA
// (src/cuda/hd_cudnn_sdpa.cu), plus the small eager attention used for
// validation (attn.cu:22-173 semantics).
//
// Kernel layout (one wave = 32 query rows of one head, 4 waves per block):
//  * S^T = K . Q^T with v_mfma_f32_32x32x16_bf16: the MFMA output puts one
//    query per lane (lane % 32) and 16 key positions per lane, so the row
//    max / row sum need a single xor-32 exchange;
//  * O^T = V^T . P^T: the output accumulator also keeps one query per lane,
//    so the online-softmax rescale is a per-lane scalar;
//  * P^T feeds the second MFMA straight from the S^T registers. The key
//    order inside each 16-key group that this implies (lane half h holds keys
//    h*4..h*4+3 and 8+h*4..8+h*4+3) is matched by storing V^T with bits 2
//    and 3 of the key index swapped ("vt" layout below), so every operand
//    fetch is one 16-byte LDS read;
//  * K and V^T tiles go global -> LDS with buffer_load_dwordx4 ... lds into two
//    buffers (64 keys per tile), XOR-swizzled by row.
// The 8-wave blocks run flash_pp16_kernel: the same online softmax on
// v_mfma_f32_16x16x32_bf16 tiles, split into alternating MFMA and softmax
// phases with the two waves of each SIMD one phase apart (four LDS tile
// buffers, loads two tiles ahead).
//
// vt layout: [B, Hkv, 128, S_pad] bf16, S_pad = round_up(S, 64), key s
// stored at column perm16(s) = s with bits 2 and 3 exchanged, padding zero.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

#include "hd_common.hpp"
#include "../../include/hd_hip.h"
#include "../../include/hd_sdpa.h"

#define FA_D 128
#define FA_BQ 128      // queries per block (4 waves x 32)
#define FA_BK 64       // keys per tile
#define FA_TAU 8.0f    // lazy-rescale threshold (log2 units)
#ifndef FA_PF
#define FA_PF 8        // LDS fragment reads in flight ahead of the MFMAs (ping-pong kernel)
#endif

__host__ __device__ __forceinline__ int perm16(int s) {
    return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1);
}
static inline int64_t fa_spad(int64_t s) { return (s + FA_BK - 1) / FA_BK * FA_BK; }

struct FaArgs {
    const uint16_t *q;     // [B,Hq,S,D]
    const uint16_t *k;     // [B,Hkv,S,D]
    const uint16_t *vt;    // [B,Hkv,D,S_pad] (perm16 columns)
    const uint16_t *mask;  // optional [S,S] additive bf16
    uint16_t *out;         // seq-major [B,S,Hq*D] or head-major [B,Hq,S,D]
    int S, S_pad, Hq, Hkv;
    int ar_len;            // rows < ar_len: causal
    int q_row_begin;       // first query row of the launch (its q tiles start here)
    int q_row_end;         // only rows < q_row_end are computed/written
    float scale_log2;      // scale * log2(e)
    float inv_scale;       // 1 / scale (mask values are added to raw scores)
    int out_seq_major;
    int out_rows;          // rows per sequence in `out` (S, or fewer for a staging buffer)
    // tail split: blocks [0, n_whole) each run one (b, head, q tile) unit over
    // all keys; the units from n_whole on run as `split` chunks of the key
    // tiles each, writing unnormalised partials to `part` (merged afterwards)
    int n_whole, split;
    float *part;           // [n_tail * split][FA_BQ][FA_D] O, then [..][FA_BQ] (m, l)
};

// 16-byte buffer load straight to LDS against a wave-uniform descriptor
// (base, nbytes); the descriptor type exists in the device pass only
__device__ __forceinline__ void fa_buf_load16(const void *base, int nbytes, uint32_t voff, uint32_t soff,
                                              HD_LDS void *dst) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint64_t b = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(((uint64_t)hi << 32) | lo), 0, __builtin_amdgcn_readfirstlane(nbytes), 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
#endif
}

__device__ __forceinline__ void fa_wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// max / sum with the lane 32 positions away (v_permlane32_swap exchanges
// the two 32-lane halves; max/sum of the pair is the same in both lanes)
__device__ __forceinline__ float xor32_max(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Blocks are dispatched to the 8 XCDs round-robin (block b to XCD b % 8):
// give each XCD a contiguous range of linear ids instead, so the blocks one
// XCD runs at a time share their kv heads' K / V^T in that XCD's L2.
__device__ __forceinline__ int fa_xcd_remap(int b, int nb) {
    const int per = nb / 8, rem = nb % 8;
    const int xcd = b % 8, idx = b / 8;
    return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// NWV waves per block (4: two blocks per CU; 8: one block of 256 queries
// per CU sharing one copy of the K / V^T tiles); 32 queries per wave either way.
template <bool MASKED, int NWV>
__global__ __launch_bounds__(NWV * 64, 8 / NWV) void flash_fwd_kernel(FaArgs a) {
    constexpr int BQ = NWV * 32, LPW = 16 / NWV;   // queries per block, loads per wave per tile
    __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * (FA_BK * FA_D + FA_D * FA_BK)];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, h = lane >> 5;

    // block -> (b, head, q tile). Query heads sharing one kv head get
    // consecutive linear ids so they run close together in time.
    const int nqt = (a.q_row_end - a.q_row_begin + BQ - 1) / BQ;
    const int group = a.Hq / a.Hkv;
    int lin = blockIdx.x, chunk = -1, item = 0;
    if (lin >= a.n_whole) {
        item = lin - a.n_whole;
        chunk = item % a.split;
        lin = a.n_whole + item / a.split;
    } else {
        lin = fa_xcd_remap(lin, a.n_whole);
    }
    const int g = lin % group; lin /= group;
    const int qt = lin % nqt; lin /= nqt;
    const int hk = lin % a.Hkv;
    const int b = lin / a.Hkv;
    const int hq = hk * group + g;

    const int qb = a.q_row_begin + qt * BQ;          // the block's first query row
    const int q0 = qb + wave * 32;
    const int my_q = q0 + l32;                       // this lane's query row
    const bool causal_block = qb < a.ar_len;
    // keys needed by this block
    int kv_end = a.S;
    if (causal_block) {
        int last_row = min(qb + BQ, a.q_row_end) - 1;
        if (last_row < a.ar_len) kv_end = last_row + 1;
    }
    int t_begin = 0, t_end = (kv_end + FA_BK - 1) / FA_BK;
    if (chunk >= 0) {
        const int nt = t_end;
        t_begin = chunk * nt / a.split;
        t_end = (chunk + 1) * nt / a.split;
    }

    // ---- Q fragments (B operand of S^T), held for the whole loop ---------
    const uint16_t *qrow = a.q + (((size_t)b * a.Hq + hq) * a.S + min(my_q, a.S - 1)) * FA_D;
    bf16x8_t qf[8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) qf[ks] = *(const bf16x8_t *)(qrow + ks * 16 + h * 8);

    // ---- loader addressing ------------------------------------------------
    const uint16_t *kbase = a.k + ((size_t)b * a.Hkv + hk) * (size_t)a.S * FA_D;
    const uint16_t *vbase = a.vt + ((size_t)b * a.Hkv + hk) * (size_t)FA_D * a.S_pad;
    // K tile: 64 rows x 16 chunks; wave instr i covers rows 4*(wave*4+i) ..+4
    // V^T tile: 128 rows x 8 chunks; wave instr i covers rows 8*(wave*4+i) ..+8
    // LDS slots are XOR-swizzled so the 16 rows one ds_read_b128 phase
    // touches land in 16 distinct 16-byte bank groups: chunk ^ (row & 15)
    // for the 256-byte K rows, chunk ^ ((row >> 1) & 7) for the 128-byte V^T
    // rows (two rows per 64-bank line)
    uint16_t *Ks0 = smem, *Vs0 = smem + 2 * FA_BK * FA_D;
    // buffer loads straight to LDS: per-lane byte offsets fixed for the
    // block, the tile advance goes in the scalar offset; K rows past S read
    // as zero (their scores are masked: S % 64 != 0 selects the masked
    // kernel), V^T columns are zero-padded to S_pad
    const int kbytes = a.S * FA_D * 2, vbytes = FA_D * a.S_pad * 2;
    uint32_t k_vo[LPW], v_vo[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int krow = (wave * LPW + i) * 4 + (lane >> 4);
        k_vo[i] = (uint32_t)(krow * FA_D + (((lane & 15) ^ (krow & 15)) * 8)) * 2;
        const int vrow = (wave * LPW + i) * 8 + (lane >> 3);
        v_vo[i] = (uint32_t)(vrow * a.S_pad + (((lane & 7) ^ ((vrow >> 1) & 7)) * 8)) * 2;
    }
    auto issue = [&](int t, int buf) {
        uint16_t *Ks = Ks0 + buf * FA_BK * FA_D, *Vs = Vs0 + buf * FA_D * FA_BK;
#pragma unroll
        for (int i = 0; i < LPW; i++)
            fa_buf_load16(kbase, kbytes, k_vo[i], (uint32_t)t * FA_BK * FA_D * 2,
                          (HD_LDS void *)(Ks + (wave * LPW + i) * 512));
#pragma unroll
        for (int i = 0; i < LPW; i++)
            fa_buf_load16(vbase, vbytes, v_vo[i], (uint32_t)t * FA_BK * 2,
                          (HD_LDS void *)(Vs + (wave * LPW + i) * 512));
    };

    f32x16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.f;
    float m_run = -1e30f, l_run = 0.f;

    issue(t_begin, t_begin & 1);
    fa_wait_vm0();
    __syncthreads();
    for (int t = t_begin; t < t_end; t++) {
        const int buf = t & 1;
        if (t + 1 < t_end) issue(t + 1, buf ^ 1);
        const uint16_t *Ks = Ks0 + buf * FA_BK * FA_D, *Vs = Vs0 + buf * FA_D * FA_BK;

        // S^T for 64 keys: two 32-key tiles
        f32x16_t s[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) s[j][r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int row = j * 32 + l32;
                const int c = ((ks * 2 + h) ^ (row & 15)) * 8;
                bf16x8_t kf = *(const bf16x8_t *)(Ks + row * FA_D + c);
                s[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[j], 0, 0, 0);
            }
        }

        // tile max on raw scores (the positive scale commutes with max)
        const int kv0 = t * FA_BK;
        // masking is decided per tile and wave: keys past S, causal rows
        // whose diagonal falls in the tile, or a dense mask
        const bool need_mask = MASKED && (a.mask != nullptr || kv0 + FA_BK > a.S ||
                                          (q0 < a.ar_len && kv0 + FA_BK - 1 > q0));
        float mt = -INFINITY;
        // the wave-uniform test is taken once per tile, so tiles without
        // masked keys run exactly the unmasked kernel's max loop
        if (need_mask) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float v = s[j][r];
                    const int kv = kv0 + j * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                    bool dead = kv >= a.S || (my_q < a.ar_len && kv > my_q);
                    if (a.mask && !dead && my_q < a.S)
                        v += bf2f(a.mask[(size_t)my_q * a.S + kv]) * a.inv_scale;
                    if (dead) v = -INFINITY;
                    s[j][r] = v;
                    mt = fmaxf(mt, v);
                }
        } else {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) mt = fmaxf(mt, s[j][r]);
        }
        mt = xor32_max(mt);
        // Lazy rescale: the running max only moves when some row's tile max
        // exceeds it by more than 2^FA_TAU in probability terms, so the O
        // rescale is rare after the first tiles; p stays <= 2^FA_TAU.
        if (__builtin_amdgcn_ballot_w64((mt - m_run) * a.scale_log2 > FA_TAU)) {
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * a.scale_log2);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[i][r] *= alpha;
        }
        const float mc = -m_run * a.scale_log2;
        bf16x8_t pf[4];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                bf16x8_t pv;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float p = __builtin_amdgcn_exp2f(fmaf(s[j][hh * 8 + e], a.scale_log2, mc));
                    l_run += p;
                    pv[e] = (__bf16)p;
                }
                pf[j * 2 + hh] = pv;
            }
        // O^T += V^T . P^T over 4 steps of 16 keys
#pragma unroll
        for (int st = 0; st < 4; st++) {
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const int row = dt * 32 + l32;
                const int c = ((st * 2 + h) ^ ((row >> 1) & 7)) * 8;
                bf16x8_t vf = *(const bf16x8_t *)(Vs + row * FA_BK + c);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[st], o[dt], 0, 0, 0);
            }
        }
        fa_wait_vm0();
        __syncthreads();
    }

    // ---- normalise and store ----------------------------------------------
    const float l_tot = xor32_sum(l_run);
    if (chunk >= 0) {
        // partial: O relative to this chunk's running max, with (m, l)
        float *po = a.part + ((size_t)item * BQ + wave * 32 + l32) * FA_D;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int gq = 0; gq < 4; gq++) {
                const int d = dt * 32 + gq * 8 + h * 4;
                *(f32x4_t *)(po + d) = {o[dt][gq * 4], o[dt][gq * 4 + 1], o[dt][gq * 4 + 2],
                                        o[dt][gq * 4 + 3]};
            }
        if (h == 0) {
            float2 *pml = (float2 *)(a.part + (size_t)(gridDim.x - a.n_whole) * BQ * FA_D);
            pml[(size_t)item * BQ + wave * 32 + l32] = make_float2(m_run, l_tot);
        }
        return;
    }
    const float inv = 1.0f / l_tot;
    if (my_q >= a.q_row_end) return;
    uint16_t *dst;
    if (a.out_seq_major)
        dst = a.out + (((size_t)b * a.out_rows + my_q) * a.Hq + hq) * FA_D;
    else
        dst = a.out + (((size_t)b * a.Hq + hq) * a.out_rows + my_q) * FA_D;
    // Lanes l and l + 32 hold the low and high 4 columns of each 8-column
    // chunk of row l. For each pair of chunks (g0, g1) one swap across the
    // half-waves gives lane l all of chunk g0 and lane l + 32 all of g1, so
    // each lane writes 16-byte chunks (8 stores of 16 bytes, not 16 of 8).
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int gp = 0; gp < 2; gp++) {
            const int g0 = 2 * gp, g1 = g0 + 1;
            const u32x2_t p0 = {pack_bf2(o[dt][g0 * 4] * inv, o[dt][g0 * 4 + 1] * inv),
                                pack_bf2(o[dt][g0 * 4 + 2] * inv, o[dt][g0 * 4 + 3] * inv)};
            const u32x2_t p1 = {pack_bf2(o[dt][g1 * 4] * inv, o[dt][g1 * 4 + 1] * inv),
                                pack_bf2(o[dt][g1 * 4 + 2] * inv, o[dt][g1 * 4 + 3] * inv)};
            // the half this lane gives away: chunk g1's low half (lane l) or
            // chunk g0's high half (lane l + 32)
            const uint32_t z0 = h ? p0[0] : p1[0], z1 = h ? p0[1] : p1[1];
            const auto s0 = __builtin_amdgcn_permlane32_swap(z0, z0, false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(z1, z1, false, false);
            const uint32_t r0 = h ? s0[0] : s0[1], r1 = h ? s1[0] : s1[1];
            const u32x4_t v = h ? (u32x4_t){r0, r1, p1[0], p1[1]} : (u32x4_t){p0[0], p0[1], r0, r1};
            *(u32x4_t *)(dst + dt * 32 + (h ? g1 : g0) * 8) = v;
        }
}

// Ping-pong form of the 8-wave kernel. Each wave alternates an MFMA phase
// (O += P(t-1) V(t-1) and S(t) = K(t) Q^T) with a softmax phase
// (max, lazy rescale, exp2, P(t): VALU only). Waves w and w + 4 share a SIMD;
// waves 4..7 run one phase behind waves 0..3, so on every SIMD one wave's
// softmax issues while the other wave's MFMAs run. A block barrier closes
// every phase. K / V^T tiles go through four LDS buffers, loaded two tiles
// ahead: the buffer tile t + 2 goes to was last read in phase M(t-1), which
// both wave groups have finished when the first group starts M(t).
// (the scheduling fences keep register-only work, e.g. the exp2 of a softmax
// phase, from being moved across the barrier into the neighbouring phase)
__device__ __forceinline__ void fa_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// The ping-pong kernel (the automatic 8-wave choice) on 16x16x32 tiles: the
// phases, barriers, LDS buffers and loads above; each wave's 32 queries are
// two 16-query blocks, and every product runs on
// v_mfma_f32_16x16x32_bf16 (under the power limit the matrix cores sustain
// more FLOP/s with it on random operands than with 32x32x16):
//  * S^T = K Q^T: 4 MFMAs of 16 keys per tile and query block, each summing
//    4 steps of 32 head dimensions. The K rows feeding output row i of
//    MFMA u are key(u, i) = (u/2)*32 + (i/8)*16 + (u%2)*8 + ((i/4)%2)*4 + i%4,
//    so a lane (query lane % 16, row group lane / 16) ends with exactly the
//    8 keys that the V^T layout stores, for each 32-key step, in its 8 P^T
//    operand slots (perm16 columns g*8 .. g*8+7); P feeds the second MFMA
//    straight from the S registers, as in the 32x32 kernels;
//  * O^T = V^T P^T: 8 MFMAs of 16 head dimensions per query block, the V^T
//    rows of MFMA pair (w, v) ordered so that a lane holds 8 consecutive
//    dimensions w*32 + g*8 .. +7 (one 16-byte output store);
//  * a query's 64 scores of a tile sit in the 4 lanes lane % 16 + 16 r: the
//    row max / sum take an xor-16 and an xor-32 lane exchange;
//  * K rows are swizzled by key bits 0-2 and 4, V^T rows by dimension bits
//    1, 3 and 4, so every 16-lane fragment read hits 16 distinct banks.
__device__ __forceinline__ int fa16_kswz(int row) { return (row & 7) | (((row >> 4) & 1) << 3); }
__device__ __forceinline__ int fa16_vswz(int row) { return ((row >> 1) & 1) | (((row >> 3) & 3) << 1); }
__device__ __forceinline__ int fa16_key(int u, int i) {
    return (u >> 1) * 32 + (i >> 3) * 16 + (u & 1) * 8 + ((i >> 2) & 1) * 4 + (i & 3);
}
// max / sum over the 4 lanes lane % 16 + 16 r (v_permlane16_swap exchanges
// rows 0 <-> 1 and 2 <-> 3 of 16 lanes, v_permlane32_swap the two halves)
__device__ __forceinline__ float xor16_32_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return xor32_max(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float xor16_32_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return xor32_sum(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

template <bool MASKED>
__global__ __launch_bounds__(512, 1) void flash_pp16_kernel(FaArgs a) {
    constexpr int PF16 = FA_PF;   // 4 and 12 measured equal or slower
    constexpr int BQ = 256, LPW = 2, NB = 4;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[NB * (FA_BK * FA_D + FA_D * FA_BK)];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave >> 2;
    const int l16 = lane & 15, g = lane >> 4;

    const int nqt = (a.q_row_end - a.q_row_begin + BQ - 1) / BQ;
    const int group = a.Hq / a.Hkv;
    int lin = blockIdx.x, chunk = -1, item = 0;
    if (lin >= a.n_whole) {
        item = lin - a.n_whole;
        chunk = item % a.split;
        lin = a.n_whole + item / a.split;
    } else {
        lin = fa_xcd_remap(lin, a.n_whole);
    }
    const int gq = lin % group; lin /= group;
    const int qt = lin % nqt; lin /= nqt;
    const int hk = lin % a.Hkv;
    const int b = lin / a.Hkv;
    const int hq = hk * group + gq;

    const int qbase = a.q_row_begin + qt * BQ;
    const int q0 = qbase + wave * 32;
    int my_q[2];
    my_q[0] = q0 + l16;
    my_q[1] = q0 + 16 + l16;
    const bool causal_block = qbase < a.ar_len;
    int kv_end = a.S;
    if (causal_block) {
        int last_row = min(qbase + BQ, a.q_row_end) - 1;
        if (last_row < a.ar_len) kv_end = last_row + 1;
    }
    int t_begin = 0, t_end = (kv_end + FA_BK - 1) / FA_BK;
    if (chunk >= 0) {
        const int nt = t_end;
        t_begin = chunk * nt / a.split;
        t_end = (chunk + 1) * nt / a.split;
    }

    // Q^T operand: query block qq, head dimensions ks*32 + g*8 .. +7
    bf16x8_t qf[2][4];
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {
        const uint16_t *qrow = a.q + (((size_t)b * a.Hq + hq) * a.S + min(my_q[qq], a.S - 1)) * FA_D;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) qf[qq][ks] = *(const bf16x8_t *)(qrow + ks * 32 + g * 8);
    }

    const uint16_t *kbase = a.k + ((size_t)b * a.Hkv + hk) * (size_t)a.S * FA_D;
    const uint16_t *vbase = a.vt + ((size_t)b * a.Hkv + hk) * (size_t)FA_D * a.S_pad;
    uint16_t *Ks0 = smem, *Vs0 = smem + NB * FA_BK * FA_D;
    const int kbytes = a.S * FA_D * 2, vbytes = FA_D * a.S_pad * 2;
    uint32_t k_vo[LPW], v_vo[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int krow = (wave * LPW + i) * 4 + (lane >> 4);
        k_vo[i] = (uint32_t)(krow * FA_D + (((lane & 15) ^ fa16_kswz(krow)) * 8)) * 2;
        const int vrow = (wave * LPW + i) * 8 + (lane >> 3);
        v_vo[i] = (uint32_t)(vrow * a.S_pad + (((lane & 7) ^ fa16_vswz(vrow)) * 8)) * 2;
    }
    auto issue = [&](int t) {
        const int buf = t & (NB - 1);
        uint16_t *Ks = Ks0 + buf * FA_BK * FA_D, *Vs = Vs0 + buf * FA_D * FA_BK;
#pragma unroll
        for (int i = 0; i < LPW; i++)
            fa_buf_load16(kbase, kbytes, k_vo[i], (uint32_t)t * FA_BK * FA_D * 2,
                          (HD_LDS void *)(Ks + (wave * LPW + i) * 512));
#pragma unroll
        for (int i = 0; i < LPW; i++)
            fa_buf_load16(vbase, vbytes, v_vo[i], (uint32_t)t * FA_BK * 2,
                          (HD_LDS void *)(Vs + (wave * LPW + i) * 512));
    };

    // this lane's fragment rows: K row of S-MFMA u, V^T row of O-MFMA (w, v)
    int krow_u[4];
#pragma unroll
    for (int u = 0; u < 4; u++) krow_u[u] = fa16_key(u, l16);
    const int vrow0 = (l16 >> 2) * 8 + (l16 & 3);   // + w*32 + v*4

    f32x4_t o[2][8];
#pragma unroll
    for (int qq = 0; qq < 2; qq++)
#pragma unroll
        for (int i = 0; i < 8; i++) o[qq][i] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-1e30f, -1e30f}, l_run[2] = {0.f, 0.f};
    f32x4_t s[2][4];
    bf16x8_t pf[2][2];

    auto kfrag = [&](const uint16_t *Ks, int u, int ks) {
        const int row = krow_u[u];
        const int c = ((ks * 4 + g) ^ fa16_kswz(row)) * 8;
        return *(const bf16x8_t *)(Ks + row * FA_D + c);
    };
    auto vfrag = [&](const uint16_t *Vs, int w, int v, int st) {
        const int row = w * 32 + v * 4 + vrow0;
        const int c = ((st * 4 + g) ^ fa16_vswz(row)) * 8;
        return *(const bf16x8_t *)(Vs + row * FA_BK + c);
    };
    // S(t) = K(t) Q^T
    auto qk = [&](int t) {
        const uint16_t *Ks = Ks0 + (t & (NB - 1)) * FA_BK * FA_D;
#pragma unroll
        for (int qq = 0; qq < 2; qq++)
#pragma unroll
            for (int u = 0; u < 4; u++) s[qq][u] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const bf16x8_t kf = kfrag(Ks, u, ks);
#pragma unroll
                for (int qq = 0; qq < 2; qq++)
                    s[qq][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[qq][ks], s[qq][u], 0, 0, 0);
            }
    };
    // O += V^T(t) P(t)^T
    auto pv = [&](int t) {
        const uint16_t *Vs = Vs0 + (t & (NB - 1)) * FA_D * FA_BK;
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
            for (int x = 0; x < 8; x++) {
                const bf16x8_t vf = vfrag(Vs, x >> 1, x & 1, st);
#pragma unroll
                for (int qq = 0; qq < 2; qq++)
                    o[qq][x] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[qq][st], o[qq][x], 0, 0, 0);
            }
    };
    // both products of one MFMA phase, interleaved (independent chains)
    auto pv_qk = [&](int t) {
        const uint16_t *Vs = Vs0 + ((t - 1) & (NB - 1)) * FA_D * FA_BK;
        const uint16_t *Ks = Ks0 + (t & (NB - 1)) * FA_BK * FA_D;
#pragma unroll
        for (int qq = 0; qq < 2; qq++)
#pragma unroll
            for (int u = 0; u < 4; u++) s[qq][u] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int y = 0; y < 16; y++) {
            const int st = y >> 3, x = y & 7;
            const bf16x8_t vf = vfrag(Vs, x >> 1, x & 1, st);
#pragma unroll
            for (int qq = 0; qq < 2; qq++)
                o[qq][x] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[qq][st], o[qq][x], 0, 0, 0);
            const int ks = y >> 2, u = y & 3;
            const bf16x8_t kf = kfrag(Ks, u, ks);
#pragma unroll
            for (int qq = 0; qq < 2; qq++)
                s[qq][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[qq][ks], s[qq][u], 0, 0, 0);
        }
        // fragment reads run PF16 reads ahead of the MFMAs (two MFMAs per read)
        __builtin_amdgcn_sched_group_barrier(0x100, PF16, 0);
#pragma unroll
        for (int i = 0; i < 32 - PF16; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * PF16, 0);
    };
    // softmax of S(t) into P(t), with the lazy O rescale
    auto softmax = [&](int t) {
        const int kv0 = t * FA_BK;
        const bool need_mask = MASKED && (a.mask != nullptr || kv0 + FA_BK > a.S ||
                                          (q0 < a.ar_len && kv0 + FA_BK - 1 > q0));
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            float mt = -INFINITY;
            if (need_mask) {
                const int mq = my_q[qq];
#pragma unroll
                for (int u = 0; u < 4; u++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        float v = s[qq][u][e];
                        const int kv = kv0 + fa16_key(u, g * 4 + e);
                        const bool dead = kv >= a.S || (mq < a.ar_len && kv > mq);
                        if (a.mask && !dead && mq < a.S) v += bf2f(a.mask[(size_t)mq * a.S + kv]) * a.inv_scale;
                        if (dead) v = -INFINITY;
                        s[qq][u][e] = v;
                        mt = fmaxf(mt, v);
                    }
            } else {
#pragma unroll
                for (int u = 0; u < 4; u++)
#pragma unroll
                    for (int e = 0; e < 4; e++) mt = fmaxf(mt, s[qq][u][e]);
            }
            mt = xor16_32_max(mt);
            if (__builtin_amdgcn_ballot_w64((mt - m_run[qq]) * a.scale_log2 > FA_TAU)) {
                const float m_new = fmaxf(m_run[qq], mt);
                const float alpha = __builtin_amdgcn_exp2f((m_run[qq] - m_new) * a.scale_log2);
                m_run[qq] = m_new;
                l_run[qq] *= alpha;
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) o[qq][i][e] *= alpha;
            }
            const float mc = -m_run[qq] * a.scale_log2;
#pragma unroll
            for (int st = 0; st < 2; st++) {
                bf16x8_t p8;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[qq][st * 2 + (e >> 2)][e & 3], a.scale_log2, mc));
                    l_run[qq] += p;
                    p8[e] = (__bf16)p;
                }
                pf[qq][st] = p8;
            }
        }
    };
    auto pin_softmax = [&]() {
        asm volatile("" ::"v"(pf[0][0]), "v"(pf[0][1]), "v"(pf[1][0]), "v"(pf[1][1]), "v"(l_run[0]),
                     "v"(l_run[1]));
    };
    auto wait_next = [&](bool issued) {
        if (issued) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else fa_wait_vm0();
    };
    {
        float *part = a.part;
        uint16_t *outp = a.out;
        asm volatile("" ::"s"(part), "s"(outp));
    }
    // the barrier sequence of the phases above (2T + 3 barriers per wave)
    issue(t_begin);
    if (t_begin + 1 < t_end) {
        issue(t_begin + 1);
        wait_next(true);
    } else {
        fa_wait_vm0();
    }
    fa_barrier();
    if (grp) fa_barrier();
    {
        const bool ld = t_begin + 2 < t_end;
        if (ld) issue(t_begin + 2);
        qk(t_begin);
        wait_next(ld);
        fa_barrier();
    }
    for (int t = t_begin + 1; t < t_end; t++) {
        softmax(t - 1);
        pin_softmax();
        fa_barrier();
        const bool ld = t + 2 < t_end;
        if (ld) issue(t + 2);
        pv_qk(t);
        wait_next(ld);
        fa_barrier();
    }
    softmax(t_end - 1);
    pin_softmax();
    fa_barrier();
    pv(t_end - 1);
    fa_barrier();

    // ---- normalise and store: a lane holds dimensions w*32 + g*8 .. +7 -----
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {
        const float l_tot = xor16_32_sum(l_run[qq]);
        const int row = wave * 32 + qq * 16 + l16;
        if (chunk >= 0) {
            float *po = a.part + ((size_t)item * BQ + row) * FA_D;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                *(f32x4_t *)(po + w * 32 + g * 8) = o[qq][w * 2];
                *(f32x4_t *)(po + w * 32 + g * 8 + 4) = o[qq][w * 2 + 1];
            }
            if (g == 0) {
                float2 *pml = (float2 *)(a.part + (size_t)(gridDim.x - a.n_whole) * BQ * FA_D);
                pml[(size_t)item * BQ + row] = make_float2(m_run[qq], l_tot);
            }
        } else if (my_q[qq] < a.q_row_end) {
            const float inv = 1.0f / l_tot;
            uint16_t *dst;
            if (a.out_seq_major)
                dst = a.out + (((size_t)b * a.out_rows + my_q[qq]) * a.Hq + hq) * FA_D;
            else
                dst = a.out + (((size_t)b * a.Hq + hq) * a.out_rows + my_q[qq]) * FA_D;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const f32x4_t x0 = o[qq][w * 2], x1 = o[qq][w * 2 + 1];
                const u32x4_t v = {pack_bf2(x0[0] * inv, x0[1] * inv), pack_bf2(x0[2] * inv, x0[3] * inv),
                                   pack_bf2(x1[0] * inv, x1[1] * inv), pack_bf2(x1[2] * inv, x1[3] * inv)};
                *(u32x4_t *)(dst + w * 32 + g * 8) = v;
            }
        }
    }
    if (!grp) fa_barrier();
}

// V [BH, S, D] -> vt [BH, D, S_pad] with perm16 columns and zero padding.
__global__ __launch_bounds__(256) void fa_vt_kernel(const uint16_t *v, uint16_t *vt, int S,
                                                    int S_pad) {
    __shared__ uint16_t tile[64][FA_D + 2];
    const int bh = blockIdx.y, s0 = blockIdx.x * 64;
    const uint16_t *src = v + (size_t)bh * S * FA_D;
    for (int i = threadIdx.x; i < 64 * FA_D; i += 256) {
        int t = i / FA_D, d = i % FA_D;
        tile[t][d] = (s0 + t < S) ? src[(size_t)(s0 + t) * FA_D + d] : (uint16_t)0;
    }
    __syncthreads();
    uint16_t *dst = vt + (size_t)bh * FA_D * S_pad;
    for (int i = threadIdx.x; i < 64 * FA_D; i += 256) {
        int d = i / 64, p = i % 64;   // p: storage column within the tile
        dst[(size_t)d * S_pad + s0 + p] = tile[perm16(p)][d];
    }
}

// Merges the tail units' key-chunk partials: O = sum_i w_i O_i / sum_i w_i l_i
// with w_i = 2^((m_i - max_j m_j) * scale_log2). One thread per (row, 8
// consecutive d): two 16-byte partial loads per chunk, one 16-byte store.
template <int BQ>
__global__ __launch_bounds__(256) void fa_merge_kernel(FaArgs a, int n_tail) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    const int d0 = (idx % (FA_D / 8)) * 8, row = (idx / (FA_D / 8)) % BQ, tu = idx / (FA_D / 8 * BQ);
    if (tu >= n_tail) return;
    const int P = a.split, n_items = n_tail * P;
    const float2 *pml = (const float2 *)(a.part + (size_t)n_items * BQ * FA_D);
    float m = -INFINITY;
    for (int i = 0; i < P; i++) m = fmaxf(m, pml[(size_t)(tu * P + i) * BQ + row].x);
    float L = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < P; i++) {
        const float2 ml = pml[(size_t)(tu * P + i) * BQ + row];
        const float w = __builtin_amdgcn_exp2f((ml.x - m) * a.scale_log2);
        L = fmaf(w, ml.y, L);
        const float4 *src = (const float4 *)(a.part + ((size_t)(tu * P + i) * BQ + row) * FA_D + d0);
        const float4 p0 = src[0], p1 = src[1];
        const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = fmaf(w, pv[e], acc[e]);
    }
    const int nqt = (a.q_row_end - a.q_row_begin + BQ - 1) / BQ, group = a.Hq / a.Hkv;
    int lin = a.n_whole + tu;
    const int g = lin % group; lin /= group;
    const int qt = lin % nqt; lin /= nqt;
    const int hk = lin % a.Hkv, b = lin / a.Hkv, hq = hk * group + g;
    const int my_q = a.q_row_begin + qt * BQ + row;
    if (my_q >= a.q_row_end) return;
    const size_t o = a.out_seq_major ? (((size_t)b * a.out_rows + my_q) * a.Hq + hq) * FA_D + d0
                                     : (((size_t)b * a.Hq + hq) * a.out_rows + my_q) * FA_D + d0;
    const float inv = 1.0f / L;
    u32x4_t v;
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = pack_bf2(acc[2 * e] * inv, acc[2 * e + 1] * inv);
    *(u32x4_t *)(a.out + o) = v;
}

// Resident flash blocks on the current device (occupancy x CUs), cached.
static int fa_slots(int nwv = 4) {
    static int dev_cached = -1, slots4 = 0, slots8 = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (dev != dev_cached) {
        int per4 = 0, per8 = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per4, flash_fwd_kernel<false, 4>, 256, 0) !=
                hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per8, flash_pp16_kernel<false>, 512, 0) !=
                hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        slots4 = per4 * cus;
        slots8 = per8 * cus;
        dev_cached = dev;
    }
    return nwv == 8 ? slots8 : slots4;
}

// Workspace for the tail split: at most one round of partial blocks.
extern "C" int64_t hd_flash_ws_bytes(void) {
    // one round of partial blocks of either family (slots x rows per block)
    const int64_t r4 = (int64_t)fa_slots(4) * 128, r8 = (int64_t)fa_slots(8) * 256;
    const int64_t rows = r4 > r8 ? r4 : r8;
    return (rows > 0 ? rows : 1024 * 128) * (FA_D + 2) * 4;
}

extern "C" int64_t hd_flash_vt_bytes(int batch, int kv_heads, int seq) {
    return (int64_t)batch * kv_heads * FA_D * fa_spad(seq) * 2;
}

// Writes the flash V^T layout from a head-major V (used by the plan API; the
// decoder block's QKV epilogue writes it directly).
extern "C" void hd_flash_make_vt(const void *v, void *vt, int bh, int seq) {
    if (!v || !vt || bh <= 0 || seq <= 0) {
        snprintf(hd_cuda_errbuf(), 512, "flash_make_vt: bad args");
        return;
    }
    dim3 g(hd_cdiv(fa_spad(seq), 64), bh);
    fa_vt_kernel<<<g, 256, 0, hd_stream()>>>((const uint16_t *)v, (uint16_t *)vt, seq,
                                             (int)fa_spad(seq));
    hd_check_launch("flash_make_vt");
}

static int fa_launch(const void *q, const void *k, const void *vt, const void *mask, void *out,
                     int batch, int hq, int hkv, int seq, int ar_len, int q_row_end, float scale,
                     int out_seq_major, hipStream_t st, void *ws = nullptr, int64_t ws_bytes = 0,
                     int out_rows = 0, int q_row_begin = 0) {
    // A causal text prefix (rows < ar_len see keys <= row) over full
    // attention below it: the prefix rows run as a masked launch of their
    // own, whose blocks all end at their diagonal, and rows ar_len.. are plain
    // full attention in the unmasked kernel with the tail split. One masked
    // launch over all rows costs 7-12 % more: its block holding row ar_len
    // runs every key with most of its waves masked, and it has no split.
    if (ar_len > 0 && !mask && ws && q_row_begin == 0 && (seq % FA_BK) == 0 && ar_len < q_row_end) {
        const int rc = fa_launch(q, k, vt, nullptr, out, batch, hq, hkv, seq, ar_len, ar_len, scale,
                                 out_seq_major, st, nullptr, 0, out_rows, 0);
        if (rc) return rc;
        return fa_launch(q, k, vt, nullptr, out, batch, hq, hkv, seq, 0, q_row_end, scale, out_seq_major, st,
                         ws, ws_bytes, out_rows, ar_len);
    }
    FaArgs a;
    a.q = (const uint16_t *)q;
    a.k = (const uint16_t *)k;
    a.vt = (const uint16_t *)vt;
    a.mask = (const uint16_t *)mask;
    a.out = (uint16_t *)out;
    a.S = seq;
    a.S_pad = (int)fa_spad(seq);
    a.Hq = hq;
    a.Hkv = hkv;
    a.ar_len = ar_len;
    a.q_row_begin = q_row_begin;
    a.q_row_end = q_row_end;
    a.scale_log2 = scale * 1.44269504088896341f;
    a.inv_scale = 1.0f / scale;
    a.out_seq_major = out_seq_major;
    a.out_rows = out_rows > 0 ? out_rows : seq;
    // 8-wave blocks (one copy of each K / V^T tile for 256 queries) when the
    // tail split can fill the last round and the sequence is long enough to
    // amortise the larger block: +3 % at S = 16640 / 16896, equal at 4352;
    // 4-wave blocks otherwise (without the split their finer grain wins)
    const bool split_ok = ws && !mask && ar_len == 0;
    const int nwv = split_ok && seq >= 1024 ? 8 : 4;
    const int BQ = nwv * 32;
    const int nqt = (q_row_end - q_row_begin + BQ - 1) / BQ;
    const int units = batch * hq * nqt;
    bool masked = mask || ar_len > 0 || (seq % FA_BK) != 0;
    // Tail split (full attention only): the units of the last partial round
    // of resident blocks run as P key chunks each, launched last, so that
    // round is filled instead of running a few blocks for a whole round.
    a.n_whole = units;
    a.split = 1;
    a.part = (float *)ws;
    int n_tail = 0;
    const int slots = ws ? fa_slots(nwv) : 0;
    if (slots > 0 && !mask && ar_len == 0 && units >= slots) {
        const int rem = units % slots, ntile = (seq + FA_BK - 1) / FA_BK;
        int P = rem ? slots / rem : 1;
        if (P > 8) P = 8;
        if (P > ntile) P = ntile;
        if (rem && P >= 2 && (int64_t)rem * P * BQ * (FA_D + 2) * 4 <= ws_bytes) {
            n_tail = rem;
            a.n_whole = units - rem;
            a.split = P;
        }
    }
    dim3 grid((unsigned)(a.n_whole + n_tail * a.split));
    if (nwv == 8) {
        // the ping-pong form: +2.5-4.7 % at S = 4352-16640 over 8-wave
        // blocks in lockstep
        if (masked) flash_pp16_kernel<true><<<grid, 512, 0, st>>>(a);
        else flash_pp16_kernel<false><<<grid, 512, 0, st>>>(a);
    } else {
        if (masked) flash_fwd_kernel<true, 4><<<grid, 256, 0, st>>>(a);
        else flash_fwd_kernel<false, 4><<<grid, 256, 0, st>>>(a);
    }
    if (n_tail) {
        dim3 gm((unsigned)hd_cdiv((int64_t)n_tail * BQ * (FA_D / 8), 256));
        if (nwv == 8) fa_merge_kernel<256><<<gm, 256, 0, st>>>(a, n_tail);
        else fa_merge_kernel<128><<<gm, 256, 0, st>>>(a, n_tail);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(hd_cuda_errbuf(), 512, "hd_sdpa: flash launch failed: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

extern "C" int hd_flash_attention(const void *q, const void *k, const void *vt, const void *mask,
                                  void *out, int batch, int q_heads, int kv_heads, int seq,
                                  int head_dim, int ar_len, float scale, int out_seq_major) {
    if (!q || !k || !vt || !out || batch <= 0 || q_heads <= 0 || kv_heads <= 0 ||
        q_heads % kv_heads || seq <= 0 || head_dim != FA_D || ar_len < 0 || ar_len > seq) {
        snprintf(hd_cuda_errbuf(), 512, "hd_sdpa: flash bad args");
        return 1;
    }
    return fa_launch(q, k, vt, mask, out, batch, q_heads, kv_heads, seq, ar_len, seq, scale,
                     out_seq_major, hd_stream());
}

extern "C" int hd_flash_attention_ws(const void *q, const void *k, const void *vt, const void *mask,
                                     void *out, int batch, int q_heads, int kv_heads, int seq,
                                     int head_dim, int ar_len, float scale, int out_seq_major,
                                     void *ws, int64_t ws_bytes) {
    if (!q || !k || !vt || !out || batch <= 0 || q_heads <= 0 || kv_heads <= 0 ||
        q_heads % kv_heads || seq <= 0 || head_dim != FA_D || ar_len < 0 || ar_len > seq) {
        snprintf(hd_cuda_errbuf(), 512, "hd_sdpa: flash bad args");
        return 1;
    }
    return fa_launch(q, k, vt, mask, out, batch, q_heads, kv_heads, seq, ar_len, seq, scale,
                     out_seq_major, hd_stream(), ws, ws_bytes);
}

// ---------------------------------------------------------------------------
// Plan API (hd_cudnn_sdpa.h). A plan is shape + split point + a V^T staging
// buffer allocated once at create time (the reference allocates its cuDNN
// workspace and causal staging there too, hd_cudnn_sdpa.cu:233-247, :354-368).
// ---------------------------------------------------------------------------
struct hd_sdpa_plan {
    int B, Hq, Hkv, Sq, Skv, D;
    int ar_len;
    float scale;
    void *vt;
    size_t vt_bytes;
    void *ws = nullptr;      // tail-split partials (hd_flash_ws_bytes)
    int64_t ws_bytes = 0;
    void *o_stage = nullptr; // split plans: causal-prefix rows of pass 0, [B, ar_len, Hq, D]
};

static int sdpa_err(const char *m) {
    snprintf(hd_cuda_errbuf(), 512, "hd_sdpa: %s", m);
    return 1;
}

static int plan_new(hd_sdpa_plan **out, int batch, int hq, int hkv, int sq, int skv, int d,
                    int ar_len, float scale) {
    if (!out) return sdpa_err("null out");
    *out = nullptr;
    if (batch < 1) return sdpa_err("invalid batch");
    if (hq < 1 || hkv < 1 || hq % hkv) return sdpa_err("invalid head counts (q_heads % kv_heads != 0)");
    if (sq < 1 || skv < 1 || d < 1) return sdpa_err("invalid dims");
    if (d != FA_D) return sdpa_err("head_dim must be 128");
    if (sq != skv) return sdpa_err("seq_q must equal seq_kv");
    hd_sdpa_plan *p = new hd_sdpa_plan();
    p->B = batch; p->Hq = hq; p->Hkv = hkv; p->Sq = sq; p->Skv = skv; p->D = d;
    p->ar_len = ar_len;
    p->scale = scale;
    p->vt_bytes = (size_t)hd_flash_vt_bytes(batch, hkv, skv);
    if (hipMalloc(&p->vt, p->vt_bytes) != hipSuccess) {
        delete p;
        return sdpa_err("hipMalloc V^T staging failed");
    }
    p->ws_bytes = hd_flash_ws_bytes();
    if (hipMalloc(&p->ws, (size_t)p->ws_bytes) != hipSuccess) {
        (void)hipFree(p->vt);
        delete p;
        return sdpa_err("hipMalloc flash workspace failed");
    }
    if (ar_len > 0 &&
        hipMalloc(&p->o_stage, (size_t)batch * ar_len * hq * d * 2) != hipSuccess) {
        (void)hipFree(p->vt);
        (void)hipFree(p->ws);
        delete p;
        return sdpa_err("hipMalloc causal-prefix staging failed");
    }
    *out = p;
    return 0;
}

extern "C" int hd_sdpa_create(hd_sdpa_plan **out, int batch, int q_heads, int kv_heads, int seq_q,
                              int seq_kv, int head_dim, float scale) {
    return plan_new(out, batch, q_heads, kv_heads, seq_q, seq_kv, head_dim, 0, scale);
}

extern "C" int hd_sdpa_create_split(hd_sdpa_plan **out, int batch, int q_heads, int kv_heads,
                                    int seq, int ar_len, int head_dim, float scale) {
    if (out) *out = nullptr;
    if (ar_len < 0 || ar_len >= seq) return sdpa_err("invalid ar_len (must be 0 < ar_len < seq)");
    return plan_new(out, batch, q_heads, kv_heads, seq, seq, head_dim, ar_len, scale);
}

extern "C" int hd_sdpa_create_prod(hd_sdpa_plan **out, int batch, int q_heads, int kv_heads,
                                   int seq, int ar_len, int head_dim, float scale) {
    if (!out) return sdpa_err("null out");
    *out = nullptr;
    if (ar_len > 0 && ar_len < seq)
        return hd_sdpa_create_split(out, batch, q_heads, kv_heads, seq, ar_len, head_dim, scale);
    return hd_sdpa_create(out, batch, q_heads, kv_heads, seq, seq, head_dim, scale);
}

extern "C" void hd_sdpa_destroy(hd_sdpa_plan *p) {
    if (!p) return;
    if (p->vt) (void)hipFree(p->vt);
    if (p->ws) (void)hipFree(p->ws);
    if (p->o_stage) (void)hipFree(p->o_stage);
    delete p;
}

static int plan_run(hd_sdpa_plan *p, const void *q, const void *k, const void *v, const void *mask,
                    void *out, void *stream, int ar_len, int q_row_end, bool to_stage = false) {
    hipStream_t st = stream ? (hipStream_t)stream : hd_stream();
    dim3 g(hd_cdiv(fa_spad(p->Skv), 64), p->B * p->Hkv);
    fa_vt_kernel<<<g, 256, 0, st>>>((const uint16_t *)v, (uint16_t *)p->vt, p->Skv,
                                    (int)fa_spad(p->Skv));
    if (hipGetLastError() != hipSuccess) return sdpa_err("V^T staging launch failed");
    if (to_stage)   // pass 0: the causal rows into the plan's staging, seq-major
        return fa_launch(q, k, p->vt, mask, p->o_stage, p->B, p->Hq, p->Hkv, p->Sq, ar_len, q_row_end,
                         p->scale, 1, st, p->ws, p->ws_bytes, p->ar_len);
    return fa_launch(q, k, p->vt, mask, out, p->B, p->Hq, p->Hkv, p->Sq, ar_len, q_row_end,
                     p->scale, 0, st, p->ws, p->ws_bytes);
}

extern "C" int hd_sdpa_execute(hd_sdpa_plan *p, const void *q, const void *k, const void *v,
                               const void *mask, void *out, void *stream) {
    if (!p || !q || !k || !v || !out) return sdpa_err("null arg in execute");
    if (p->ar_len > 0) return hd_sdpa_execute_split(p, q, k, v, out, stream);
    return plan_run(p, q, k, v, mask, out, stream, 0, p->Sq);
}

extern "C" int hd_sdpa_execute_split(hd_sdpa_plan *p, const void *q, const void *k, const void *v,
                                     void *out, void *stream) {
    if (!p || !q || !k || !v || !out) return sdpa_err("null arg in execute");
    if (p->ar_len <= 0) return sdpa_err("execute_split on a non-split plan");
    return plan_run(p, q, k, v, nullptr, out, stream, p->ar_len, p->Sq);
}

extern "C" const void *hd_sdpa_plan_stage(const hd_sdpa_plan *p) { return p ? p->o_stage : nullptr; }

extern "C" int hd_sdpa_execute_split_pass(hd_sdpa_plan *p, int which, const void *q, const void *k,
                                          const void *v, void *out, void *stream) {
    if (!p || !q || !k || !v || !out) return sdpa_err("null arg in execute");
    if (p->ar_len <= 0) return sdpa_err("execute_split_pass on a non-split plan");
    // pass 0 leaves `out` untouched: its rows go to the plan's staging, as
    // the reference's causal pass writes only its staged head
    // (hd_cudnn_sdpa.cu:455-468)
    if (which == 0) return plan_run(p, q, k, v, nullptr, out, stream, p->ar_len, p->ar_len, true);
    return plan_run(p, q, k, v, nullptr, out, stream, 0, p->Sq);
}

// ---------------------------------------------------------------------------
// Eager attention (attn.cu:22-173 semantics) for small validation shapes:
// fp32 scores, fp32 softmax, bf16 probs, fp32 P.V over bf16 probs,
// seq-major output. Scores are recomputed instead of kept in an fp32
// scratch, so nothing is allocated.
// ---------------------------------------------------------------------------
__global__ void eager_probs_kernel(const uint16_t *q, const uint16_t *k, const uint16_t *mask,
                                   uint16_t *scores, uint16_t *probs, int H, int KV, int S, int D,
                                   float scaling) {
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= H * S) return;
    int s = idx % S, hh = idx / S, kh = hh / (H / KV);
    const uint16_t *qr = q + ((size_t)hh * S + s) * D;
    auto score = [&](int t) {
        const uint16_t *kr = k + ((size_t)kh * S + t) * D;
        float acc = 0.f;
        for (int d = 0; d < D; d++) acc += bf2f(qr[d]) * bf2f(kr[d]);
        acc *= scaling;
        return acc + bf2f(mask[(size_t)s * S + t]);
    };
    float mx = -INFINITY;
    for (int t = 0; t < S; t++) mx = fmaxf(mx, score(t));
    float sum = 0.f;
    for (int t = 0; t < S; t++) sum += expf(score(t) - mx);
    float inv = 1.0f / sum;
    for (int t = 0; t < S; t++) {
        float sc = score(t);
        scores[((size_t)hh * S + s) * S + t] = f2bf(sc);
        probs[((size_t)hh * S + s) * S + t] = f2bf(expf(sc - mx) * inv);
    }
}
__global__ void eager_out_kernel(const uint16_t *probs, const uint16_t *v, uint16_t *out, int H,
                                 int KV, int S, int D) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)H * S * D) return;
    int d = idx % D;
    size_t r = idx / D;
    int hh = r % H, s = r / H, kh = hh / (H / KV);   // idx enumerates [S,H,D]
    const uint16_t *pr = probs + ((size_t)hh * S + s) * S;
    float acc = 0.f;
    for (int t = 0; t < S; t++) acc += bf2f(pr[t]) * bf2f(v[((size_t)kh * S + t) * D + d]);
    out[idx] = f2bf(acc);
}
extern "C" void hd_attention_eager(const void *q, const void *k, const void *v, const void *mask,
                                   void *scores, void *probs, void *out, int heads, int kv_heads,
                                   int seq, int dim, float scaling) {
    if (!q || !k || !v || !mask || !scores || !probs || !out || heads <= 0 || kv_heads <= 0 ||
        seq <= 0 || dim <= 0 || heads % kv_heads) {
        snprintf(hd_cuda_errbuf(), 512, "attention_eager: bad args");
        return;
    }
    eager_probs_kernel<<<hd_cdiv((size_t)heads * seq, 128), 128, 0, hd_stream()>>>(
        (const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)mask, (uint16_t *)scores,
        (uint16_t *)probs, heads, kv_heads, seq, dim, scaling);
    eager_out_kernel<<<hd_cdiv((size_t)heads * seq * dim, 256), 256, 0, hd_stream()>>>(
        (const uint16_t *)probs, (const uint16_t *)v, (uint16_t *)out, heads, kv_heads, seq, dim);
    hd_check_launch("attention_eager");
}

extern "C" int hd_sdpa_plan_ar_len(const hd_sdpa_plan *p) { return p ? p->ar_len : 0; }
