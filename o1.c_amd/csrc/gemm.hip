// bf16 GEMM for gfx950: C[M,N] = A[M,K] . B[N,K]^T, fp32 accumulation.
//
// Both operands are K-contiguous (activations [M,K], weights [out,in]).
// Design (MI355X-first, not a translation of the reference's cuBLASLt use):
//  * block tile BM x BN x 64, WGM x WGN waves, each wave a (BM/WGM) x
//    (BN/WGN) sub-tile of 32x32 MFMA tiles (v_mfma_f32_32x32x16_bf16);
//  * global -> LDS with global_load_lds_dwordx4 (no register staging), two
//    LDS buffers, one barrier per K tile; 16-byte chunks XOR-swizzled by row
//    so the ds_read_b128 fragment loads spread over the banks;
//  * the MFMA is issued as weights x activations, so each lane ends with 4
//    consecutive output columns of one output row per register group; the
//    epilogue stages bf16 results through LDS and writes 16-byte coalesced
//    rows, applying bias / residual there;
//  * SwiGLU: a block's B tile holds gate rows and up rows of the same output
//    columns, so gate and up land in the same lane and the epilogue forms
//    bf16(bf16(silu(g)) * u) without either product reaching HBM;
//  * blockIdx -> tile mapping is XCD-aware (the 8 XCDs get contiguous
//    ranges of the grouped raster, so neighbouring tiles share an L2).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <atomic>
#include <type_traits>

#include "hd_common.hpp"
#include "../../include/hd_hip.h"
#include "../../include/hd_gemm.h"

enum { EPI_NONE = 0, EPI_BIAS = 1, EPI_RES = 2, EPI_SWIGLU = 3, EPI_QKV = 4 };

struct GemmArgs {
    const uint16_t *A;       // [M, K]
    const uint16_t *B[3];    // weight segments, each [rows, K]
    int seg_end[3];          // exclusive end (in B-row space) of each segment
    uint16_t *C;             // [M, ldc]
    const uint16_t *bias;    // [N]
    const uint16_t *res;     // [M, ldc]
    int M, N, K;             // N = output columns
    int ldc;
    int ntm, ntn;            // tile grid
    // EPI_QKV: per-head q/k RMSNorm + rotary into head-major q, k and the
    // flash V^T layout (columns: q heads, k heads, v heads of 128)
    const uint16_t *qn_w, *kn_w;   // [128] norm gains
    const float2 *cs;              // [seq, 64] (cos, sin)
    uint16_t *q_out, *k_out, *vt_out;
    int seq, heads, kv_heads;
    float eps;
    // tail split (gemm_ms_kernel): the first gridDim.x - n_whole blocks run
    // the K chunks (split per tile) of the last n_tail tiles and write fp32
    // partial tiles [BM][BN] to `part`; the n_whole blocks after them run
    // whole tiles
    int n_whole, split;
    float *part;
};

// SiLU for the SwiGLU epilogues: g * 1/(1 + e^-g) with the hardware exp and
// reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each) instead of an IEEE
// division. The result is rounded to bf16 right after, so it differs from
// the correctly rounded form only when the exact value lies within a few
// fp32 ulps of a bf16 rounding boundary. The full-precision division was
// ~10 VALU instructions per output and most of the per-tile epilogue time.
__device__ __forceinline__ float silu_rcp(float g) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

__device__ __forceinline__ void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ int xcd_remap(int b, int nb) {
    const int per = nb / 8, rem = nb % 8;
    const int xcd = b % 8, idx = b / 8;
    return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// ---------------------------------------------------------------------------
// Multi-stage variant: an NS-deep LDS ring of BK-wide K tiles. Tile kt+NS-1
// is requested while tile kt is consumed, and the wait before each barrier
// only drains the oldest outstanding tile (s_waitcnt vmcnt(N)), so NS-1
// tiles of global->LDS traffic stay in flight behind the MFMAs.
// ---------------------------------------------------------------------------
template <int N> __device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until at most N of this wave's global->LDS loads are outstanding,
// then joins the workgroup barrier. Written as one asm statement: the
// compiler's __syncthreads() lowering adds a full vmcnt(0) drain, which
// would empty the prefetch ring at every K step. The memory clobber keeps
// LDS reads from moving across the barrier.
template <int N> __device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// 16-byte buffer load straight to LDS (buffer_load_dwordx4 ... lds): base and
// nbytes form the scalar descriptor (reads at or past nbytes return zero).
// The descriptor type exists in the device pass only.
__device__ __forceinline__ void buf_load_lds16(const void *base, int nbytes, uint32_t voff, uint32_t soff,
                                               HD_LDS void *dst) {
#if defined(__HIP_DEVICE_COMPILE__)
    // the descriptor must live in SGPRs: base and size are wave-uniform
    const uint64_t b = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(((uint64_t)hi << 32) | lo), 0, __builtin_amdgcn_readfirstlane(nbytes), 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
#endif
}

// as above, and the wave's own LDS reads have completed (the barrier then
// also means no wave still reads the stage about to be refilled)
template <int N> __device__ __forceinline__ void wait_lgk_vm_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <int BM, int BN, int BK, int NS, int WGM, int WGN, int EPI, int MF = 32, int XA = 0, int XB = 0>
struct MsCfg {
    static constexpr int NW = WGM * WGN, NT = NW * 64;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / MF, TN = WTN / MF;
    static constexpr int WTN_OUT = EPI == EPI_SWIGLU ? WTN / 2 : WTN;
    static constexpr int BN_OUT = EPI == EPI_SWIGLU ? BN / 2 : BN;
    static constexpr int CPR = BK / 8;            // 16-byte chunks per tile row
    static constexpr int RPI = 64 / CPR;          // rows per wave load instruction
    static constexpr int AI = BM / RPI / NW, BI = BN / RPI / NW;   // load instrs per wave
    static constexpr int LPT = AI + BI;           // per tile per wave
    static constexpr int STAGE = (BM + BN) * BK;  // elements per stage
    static constexpr int EPAD = 8;
    // XA / XB extra A / B stages (schedules 4, 5): rings NS + XA and NS + XB deep
    static constexpr int MAIN_BYTES = ((NS + XA) * BM + (NS + XB) * BN) * BK * 2;
    static constexpr int EPI_BYTES = NW * WTM * (WTN_OUT + EPAD) * 2;
    static constexpr int LDS_BYTES = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
    static_assert(BK == 32 || BK == 64, "BK");
    static_assert(BM % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "loader split");
    static_assert((NS - 2) * LPT < 64, "vmcnt");
};

// chunk swizzle: 16 consecutive rows of a tile map to 16 distinct 16-byte
// bank groups (64 banks x 4 bytes)
template <int CPR> __device__ __forceinline__ int ms_swz(int r) {
    return CPR == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3);
}

// EPI_QKV epilogue for one wave: its WTM rows x 128 columns (one head) are
// staged in LDS as the bf16 projection output (the reference's rounding
// point). q/k heads: RMSNorm with 8 lanes per row (the sum of squares uses
// the pairing and summation tree of the standalone kernels, x_l^2 +
// x_{l+64}^2 then pairs 4, 2, 1 and 32, 16, 8 apart, so results are
// bit-identical) and rotate-half rotary with bf16 rounding of every
// product, stored straight to [B,H,S,128].
// v heads: transposed stores into [B,KV,128,S] with key bits 2 and 3
// exchanged (the flash kernel's V^T layout; S % 64 == 0 so no padding).
template <int WTM, int LDW>
__device__ __forceinline__ void qkv_epilogue(const GemmArgs &g, uint16_t *stg, int gm0, int hslot,
                                             int lane) {
    const int H = g.heads, KV = g.kv_heads, S = g.seq;
    if (hslot < H + KV) {
        // 8 lanes per row, 8 rows per pass: lane j of a row holds columns
        // 8j .. 8j+7 and their rotary partners 64 + 8j .. 64 + 8j+7, so the
        // pair sums x_l^2 + x_{l+64}^2 of one lane are one group of 8 of the
        // summation tree (pairs 4, 2, 1 apart in registers) and the group
        // sums 32, 16, 8 apart are lanes 4, 2, 1 apart. The rotary table and
        // the output rows are read and written as 512- and 256-byte runs.
        const uint16_t *w = hslot < H ? g.qn_w : g.kn_w;
        const int j = lane & 7;
        const u32x4_t wlo = *(const u32x4_t *)(w + j * 8), whi = *(const u32x4_t *)(w + 64 + j * 8);
        const int hx = hslot < H ? hslot : hslot - H, nh = hslot < H ? H : KV;
        uint16_t *base = hslot < H ? g.q_out : g.k_out;
        // two passes at a time: their staged rows and rotary rows are
        // requested before any of them is used
        constexpr int NP8 = WTM / 8;
        constexpr int NPASS = NP8 % 2 == 0 ? 2 : 1;
        static_assert(WTM % (8 * NPASS) == 0, "q/k epilogue passes");
        for (int rb = 0; rb < WTM; rb += 8 * NPASS) {
            u32x4_t lo[NPASS], hi[NPASS];
            float4 csv[NPASS][4];
#pragma unroll
            for (int p = 0; p < NPASS; p++) {
                const int r = rb + p * 8 + (lane >> 3);
                const uint16_t *row = stg + r * LDW;
                lo[p] = *(const u32x4_t *)(row + j * 8);
                hi[p] = *(const u32x4_t *)(row + 64 + j * 8);
                const int s = (gm0 + r) % S;
                const float4 *cs4 = (const float4 *)(g.cs + (size_t)s * 64 + j * 8);
#pragma unroll
                for (int c = 0; c < 4; c++) csv[p][c] = cs4[c];
            }
#pragma unroll
            for (int p = 0; p < NPASS; p++) {
                const int m = gm0 + rb + p * 8 + (lane >> 3);
                float v[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float a0 = lo_bf(lo[p][e]), a1 = hi_bf(lo[p][e]);
                    const float b0 = lo_bf(hi[p][e]), b1 = hi_bf(hi[p][e]);
                    v[2 * e] = fmaf(a0, a0, b0 * b0);
                    v[2 * e + 1] = fmaf(a1, a1, b1 * b1);
                }
#pragma unroll
                for (int o = 4; o > 0; o >>= 1)
#pragma unroll
                    for (int k = 0; k < o; k++) v[k] = v[k] + v[k + o];
                float ss = v[0];
                ss = ss + __shfl_xor(ss, 4, 64);
                ss = ss + __shfl_xor(ss, 2, 64);
                ss = ss + __shfl_xor(ss, 1, 64);
                if (m >= g.M) continue;
                const float inv = 1.0f / sqrtf(ss / 128.0f + g.eps);
                const int b = m / S, s = m % S;
                u32x4_t olo, ohi;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float o0[2], o1[2];
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const float x0 = t ? hi_bf(lo[p][e]) : lo_bf(lo[p][e]);
                        const float x1 = t ? hi_bf(hi[p][e]) : lo_bf(hi[p][e]);
                        const float w0 = t ? hi_bf(wlo[e]) : lo_bf(wlo[e]);
                        const float w1 = t ? hi_bf(whi[e]) : lo_bf(whi[e]);
                        const float y0 = bfround(w0 * x0 * inv);
                        const float y1 = bfround(w1 * x1 * inv);
                        const float4 c4 = csv[p][e];
                        const float cr = t ? c4.z : c4.x, sr = t ? c4.w : c4.y;
                        o0[t] = bfround(y0 * cr) - bfround(y1 * sr);
                        o1[t] = bfround(y1 * cr) + bfround(y0 * sr);
                    }
                    olo[e] = pack_bf2(o0[0], o0[1]);
                    ohi[e] = pack_bf2(o1[0], o1[1]);
                }
                uint16_t *orow = base + (((size_t)b * nh + hx) * S + s) * 128;
                *(u32x4_t *)(orow + j * 8) = olo;
                *(u32x4_t *)(orow + 64 + j * 8) = ohi;
            }
        }
    } else {
        const int hk = hslot - H - KV;
        // 8 keys x 8 dimensions per lane and item: 8 16-byte row reads (the
        // item's keys, dimensions 8*lane%16 .. +7), a register transpose, 8
        // 16-byte stores (one per dimension: the 8 storage columns of one
        // half of a 16-key group). Items: (16-key group, half), 4 per pass.
        const int dblk = lane & 15;
        constexpr int NITEM = WTM / 8;
        for (int it = lane >> 4; it < NITEM; it += 4) {
            const int grp = it >> 1, half = it & 1;
            const int m = gm0 + grp * 16;
            u32x4_t rw[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int p = half * 8 + e;                                   // storage column in the group
                const int src = (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1);  // key at that column
                rw[e] = *(const u32x4_t *)(stg + (grp * 16 + src) * LDW + dblk * 8);
            }
            if (m >= g.M) continue;
            const int b = m / S, s = m % S;
            uint16_t *dst = g.vt_out + (((size_t)b * KV + hk) * 128 + dblk * 8) * S + s + half * 8;
#pragma unroll
            for (int dd = 0; dd < 8; dd++) {
                const uint32_t sel = dd & 1 ? 0x07060302u : 0x05040100u;
                u32x4_t pk;
#pragma unroll
                for (int w = 0; w < 4; w++)
                    pk[w] = __builtin_amdgcn_perm(rw[2 * w + 1][dd >> 1], rw[2 * w][dd >> 1], sel);
                *(u32x4_t *)(dst + (size_t)dd * S) = pk;
            }
        }
    }
}

// Production GEMM kernel. Template arguments: block tile BM x BN x BK, NS
// LDS stages, WGM x WGN waves, epilogue EPI, schedule SGB, blocks per CU OCC,
// loader LDR, MFMA shape MF (16: v_mfma_f32_16x16x32_bf16).
//   SGB 8, LDR 5: split operand rings (A three stages, B two; 160 KB for
//     256 x 256 tiles) filled by buffer loads straight to LDS (operands under
//     2 GiB: 32-bit byte offsets), the next k-step's fragment reads and a
//     tile's refill loads placed between every other MFMA;
//   SGB 3, LDR 0: equal-depth rings filled by global_load_lds (64-bit
//     addresses), for operands of 2 GiB or more.
// Both keep one fragment ring across the whole K loop: the fragments of
// k-step ks+1 load under the MFMAs of ks, and at the last k-step of a tile
// the barrier, the refill of the freed stage and the first fragments of the
// next tile all go under that k-step's MFMAs.
template <int BM, int BN, int BK, int NS, int WGM, int WGN, int EPI, int SGB = 8, int OCC = 1,
          int LDR = 5, int MF = 16>
__global__ __launch_bounds__(WGM * WGN * 64, OCC) void gemm_ms_kernel(GemmArgs g) {
    static_assert(MF == 16 && BK == 64 && NS == 2, "16x16x32 MFMA tiles, 64-deep K tiles, 2+ stages");
    static_assert((SGB == 8 && LDR == 5) || (SGB == 3 && LDR == 0), "schedule / loader pair");
    constexpr bool SPLITR = SGB == 8;
    using C = MsCfg<BM, BN, BK, NS, WGM, WGN, EPI, MF, SPLITR ? 1 : 0, 0>;
    using AccT = f32x4_t;
    constexpr int WTM = C::WTM, WTN = C::WTN, TM = C::TM, TN = C::TN, CPR = C::CPR;
    constexpr int AI = C::AI, BI = C::BI, GROUP_M = 8;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[C::LDS_BYTES / 2];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    // the K chunks of the tail tiles (lin >= n_whole, `split` consecutive
    // blocks per tile) first, then the whole tiles (XCD-contiguous over
    // them). The CUs that start with a chunk run their whole tiles offset
    // from the others, so a round's epilogues (output stores, residual
    // reads) do not all reach HBM at once: +2-3 % for the residual GEMMs
    // at 4-6 rounds, equal elsewhere.
    int lin, chunk = -1, item = 0;
    const int n_chunks = (int)gridDim.x - g.n_whole;
    if ((int)blockIdx.x >= n_chunks) {
        lin = xcd_remap(blockIdx.x - n_chunks, g.n_whole);
    } else {
        item = blockIdx.x;
        chunk = item % g.split;
        lin = g.n_whole + item / g.split;
    }
    const int in_group = GROUP_M * g.ntn;
    const int first_m = (lin / in_group) * GROUP_M;
    const int gm = min(g.ntm - first_m, GROUP_M);
    const int tm = first_m + (lin % in_group) % gm;
    const int tn = (lin % in_group) / gm;
    const int m0 = tm * BM;
    // K tiles of this block: all, or chunk `chunk` of `split`
    int kbase = 0, nk = g.K / BK;
    if (chunk >= 0) {
        const int k0 = chunk * nk / g.split, k1 = (chunk + 1) * nk / g.split;
        kbase = k0;
        nk = k1 - k0;
    }

    const int sub = lane / CPR, cl = lane % CPR;
    // segment of this column tile (QKV: a 256-aligned column tile lies in one
    // of the q/k/v weights) or the gate and up matrices (SwiGLU)
    const int bt0 = tn * BN;
    const int bsg = EPI == EPI_SWIGLU ? 0 : (bt0 < g.seg_end[0] ? 0 : (bt0 < g.seg_end[1] ? 1 : 2));
    const int bbase = bsg == 0 ? 0 : (bsg == 1 ? g.seg_end[0] : g.seg_end[1]);
    const int brows = EPI == EPI_SWIGLU ? g.N
                                        : (bsg == 0 ? g.seg_end[0] : (bsg == 1 ? g.seg_end[1] : g.seg_end[2])) - bbase;
    const void *bp_a = g.A, *bp_b0 = bsg == 0 ? g.B[0] : (bsg == 1 ? g.B[1] : g.B[2]), *bp_b1 = g.B[1];
    // B row r of the tile -> weight row n (SwiGLU: each wave's WTN rows are
    // WTN/2 gate rows then the up rows of the same output columns), and
    // which matrix it comes from
    auto b_row = [&](int r, int &rs) {
        if (EPI == EPI_SWIGLU) {
            const int grp = r / WTN, j = r % WTN;
            rs = j < WTN / 2 ? 0 : 1;
            return tn * C::BN_OUT + grp * (WTN / 2) + (j % (WTN / 2));
        }
        rs = 0;
        return bt0 + r - bbase;
    };
    // LDR 0: 64-bit source pointers per loader row (global_load_lds)
    const uint16_t *a_src[AI];
    const uint16_t *b_src[BI];
    // LDR 5: 32-bit per-lane byte offsets against a scalar descriptor; the K
    // advance is the scalar offset; rows past the matrix read as zero
    // through the record limit
    const int nb_a = (int)((size_t)g.M * g.K * 2), nb_b = (int)((size_t)brows * g.K * 2);
    uint32_t a_vo[AI], b_vo[BI];
    int b_rs[BI];
#pragma unroll
    for (int i = 0; i < AI; i++) {
        const int r = (wave * AI + i) * C::RPI + sub;
        if constexpr (LDR == 5) {
            a_vo[i] = ((uint32_t)(m0 + r) * (uint32_t)g.K + (uint32_t)(cl ^ ms_swz<CPR>(r)) * 8) * 2;
        } else {
            const int m = min(m0 + r, g.M - 1);
            a_src[i] = g.A + (size_t)m * g.K + (cl ^ ms_swz<CPR>(r)) * 8;
        }
    }
#pragma unroll
    for (int i = 0; i < BI; i++) {
        const int r = (wave * BI + i) * C::RPI + sub;
        int rs, rs0;
        const int n = b_row(r, rs);
        // the RPI rows of one load share a side of the gate/up split: take it
        // from the wave-uniform first row, so the descriptor stays scalar
        (void)b_row((wave * BI + i) * C::RPI, rs0);
        b_rs[i] = rs0;
        if constexpr (LDR == 5) {
            b_vo[i] = n >= brows ? 0x80000000u   // past the records (< 2^31): reads zero
                                 : ((uint32_t)n * (uint32_t)g.K + (uint32_t)(cl ^ ms_swz<CPR>(r)) * 8) * 2;
        } else {
            const int nn = min(n, brows - 1);
            b_src[i] = (const uint16_t *)(rs ? bp_b1 : bp_b0) + (size_t)nn * g.K + (cl ^ ms_swz<CPR>(r)) * 8;
        }
    }

    AccT acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = 0.f;

    // k-steps of 32 per 64-deep tile; a lane reads 8 consecutive k of row
    // lane % 16, chunk lane / 16 of the step
    constexpr int KS = BK / 32, CPS = 4, NR = TM + TN, NM = TM * TN;
    static_assert(KS % 2 == 0, "fragment slots");
    const int lr = lane % MF, lc = lane / MF, swr = ms_swz<CPR>(lr);
    bf16x8_t af[2][TM], bw[2][TN];
    auto mfmas = [&](int sl) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw[sl][j], af[sl][i], acc[i][j], 0, 0, 0);
    };
    if constexpr (SGB == 3) {
        constexpr int LPT = C::LPT;
        auto issue = [&](int kt, int st) {
            uint16_t *As = smem + st * C::STAGE, *Bs = As + BM * BK;
#pragma unroll
            for (int i = 0; i < AI; i++)
                __builtin_amdgcn_global_load_lds((const void *)(a_src[i] + (kbase + kt) * BK),
                                                 (HD_LDS void *)(As + (wave * AI + i) * 512), 16, 0, 0);
#pragma unroll
            for (int i = 0; i < BI; i++)
                __builtin_amdgcn_global_load_lds((const void *)(b_src[i] + (kbase + kt) * BK),
                                                 (HD_LDS void *)(Bs + (wave * BI + i) * 512), 16, 0, 0);
        };
        auto ld = [&](const uint16_t *As, int ks, int sl) {
            const uint16_t *Bs = As + BM * BK;
            const int c = ((ks * CPS + lc) ^ swr) * 8;
#pragma unroll
            for (int i = 0; i < TM; i++)
                af[sl][i] = *(const bf16x8_t *)(As + (wm * WTM + i * MF + lr) * BK + c);
#pragma unroll
            for (int j = 0; j < TN; j++)
                bw[sl][j] = *(const bf16x8_t *)(Bs + (wn * WTN + j * MF + lr) * BK + c);
        };
#pragma unroll
        for (int st = 0; st < NS; st++)
            if (st < nk) issue(st, st);
        if (nk >= NS) wait_vm_barrier<(NS - 1) * LPT>();
        else wait_vm_barrier<0>();
        ld(smem, 0, 0);
        // REFILL: tile kt+NS exists; NEXT: tile kt+1 exists. Compile-time
        // flags keep the steady-state body free of branches, so the MFMA /
        // load / read interleave below survives scheduling.
        auto tile = [&](int kt, auto refill, auto next) {
            constexpr bool REFILL = decltype(refill)::value, NEXT = decltype(next)::value;
            const uint16_t *As = smem + (kt % NS) * C::STAGE;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const bool last = ks + 1 == KS;
                if (!last) {
                    ld(As, ks + 1, (ks + 1) & 1);
                } else {
                    // tile kt+1 has landed and every wave is done reading
                    // stage kt % NS (its last fragments are in registers)
                    if (REFILL) wait_lgk_vm_barrier<(NS - 2) * LPT>();
                    else wait_lgk_vm_barrier<0>();
                    __builtin_amdgcn_sched_barrier(0);
                    if (REFILL) issue(kt + NS, kt % NS);
                    if (NEXT) ld(smem + ((kt + 1) % NS) * C::STAGE, 0, 0);
                }
                mfmas(ks & 1);
                const int nv = last && REFILL ? LPT : 0;
                const int nr = !last || NEXT ? NR : 0;
#pragma unroll
                for (int q = 0; q < NM; q++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (q < nv) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                    if (q < nr) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
            }
        };
        using T_ = std::true_type;
        using F_ = std::false_type;
        int kt = 0;
        for (; kt + NS < nk; kt++) tile(kt, T_{}, T_{});
        for (; kt + 1 < nk; kt++) tile(kt, F_{}, T_{});
        tile(kt, F_{}, F_{});
    } else {
        // Split operand rings in the 160 KB of LDS: A (the activation rows,
        // shared by fewer of an XCD's concurrent tiles than the weight rows,
        // so more of their slices miss L2) three stages deep, B two. Each
        // refill batch issues B's tile kt+2 before A's tile kt+3, so the wait
        // at the end of tile kt (both operands of tile kt+1 landed) may leave
        // the newest A loads in flight: A gets two tiles of latency, B one.
        constexpr int NSA = NS + 1, NSB = NS, ASTG = BM * BK, BSTG = BN * BK;
        uint16_t *const Abase = smem, *const Bbase = smem + NSA * ASTG;
        auto ld = [&](int kt, int ks, int sl) {
            const uint16_t *As = Abase + (kt % NSA) * ASTG, *Bs = Bbase + (kt % NSB) * BSTG;
            const int c = ((ks * CPS + lc) ^ swr) * 8;
#pragma unroll
            for (int i = 0; i < TM; i++)
                af[sl][i] = *(const bf16x8_t *)(As + (wm * WTM + i * MF + lr) * BK + c);
#pragma unroll
            for (int j = 0; j < TN; j++)
                bw[sl][j] = *(const bf16x8_t *)(Bs + (wn * WTN + j * MF + lr) * BK + c);
        };
        auto issue_a = [&](int kt) {
            uint16_t *As = Abase + (kt % NSA) * ASTG;
            const uint32_t so = (uint32_t)(kbase + kt) * BK * 2;
#pragma unroll
            for (int i = 0; i < AI; i++)
                buf_load_lds16(bp_a, nb_a, a_vo[i], so, (HD_LDS void *)(As + (wave * AI + i) * 512));
        };
        auto issue_b = [&](int kt) {
            uint16_t *Bs = Bbase + (kt % NSB) * BSTG;
            const uint32_t so = (uint32_t)(kbase + kt) * BK * 2;
#pragma unroll
            for (int i = 0; i < BI; i++)
                buf_load_lds16(b_rs[i] ? bp_b1 : bp_b0, nb_b, b_vo[i], so,
                               (HD_LDS void *)(Bs + (wave * BI + i) * 512));
        };
        // prologue: [B0 A0] [B1 A1] [A2]; tile 0 may leave the later ones in flight
        issue_b(0);
        issue_a(0);
        if (nk >= 2) {
            issue_b(1);
            issue_a(1);
        }
        if (nk >= 3) {
            issue_a(2);
            wait_vm_barrier<BI + 2 * AI>();
        } else if (nk == 2) {
            wait_vm_barrier<BI + AI>();
        } else {
            wait_vm_barrier<0>();
        }
        ld(0, 0, 0);
        // RD: A tile kt+3 exists, RS: B tile kt+2 exists, NX: tile kt+1 exists
        auto tile = [&](int kt, auto rd, auto rs, auto nx) {
            constexpr bool RD = decltype(rd)::value, RS = decltype(rs)::value, NX = decltype(nx)::value;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const bool last = ks + 1 == KS;
                if (!last) {
                    ld(kt, ks + 1, (ks + 1) & 1);
                } else {
                    // both operands of tile kt+1 have landed (A's tile kt+2,
                    // issued after them, may still fly) and every wave is
                    // done reading the stages of tile kt
                    if (RS) wait_lgk_vm_barrier<AI>();
                    else wait_lgk_vm_barrier<0>();
                    __builtin_amdgcn_sched_barrier(0);
                    if (RS) issue_b(kt + 2);
                    if (RD) issue_a(kt + 3);
                    if (NX) ld(kt + 1, 0, 0);
                }
                mfmas(ks & 1);
                // fragment reads and refill loads between every other MFMA
                const int nv = last ? (RD ? AI : 0) + (RS ? BI : 0) : 0;
                const int nr = !last || NX ? NR : 0;
#pragma unroll
                for (int q = 0; q < NM; q++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (q % 2 == 0 && q / 2 < nv) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                    if (q % 2 == 1 && q / 2 < nr) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
            }
        };
        using T_ = std::true_type;
        using F_ = std::false_type;
        int kt = 0;
        for (; kt + 3 < nk; kt++) tile(kt, T_{}, T_{}, T_{});
        if (kt + 2 < nk) tile(kt++, F_{}, T_{}, T_{});
        if (kt + 1 < nk) tile(kt++, F_{}, F_{}, T_{});
        tile(kt, F_{}, F_{}, F_{});
    }
    if (chunk >= 0) {
        // K chunk of a tail tile: the raw fp32 accumulators, tile-local
        // [BM][BN] (a lane holds rows i*16 + lane%16, columns j*16 +
        // (lane/16)*4 .. +3, B-row column order); the merge kernel sums the
        // chunks and applies the epilogue
        float *pt = g.part + (size_t)item * BM * BN;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int row = wm * WTM + i * 16 + (lane & 15);
                const int col = wn * WTN + j * 16 + (lane >> 4) * 4;
                *(f32x4_t *)(pt + (size_t)row * BN + col) = acc[i][j];
            }
        return;
    }
    // residual epilogue: this lane's residual chunks are requested before
    // the staging, so their latency hides under it (the write-out below
    // then finds them in registers instead of waiting on each row group)
    constexpr int RES_N = EPI == EPI_RES ? WTM / (64 / (C::WTN_OUT / 8)) : 1;
    u32x4_t resv[RES_N];
    if constexpr (EPI == EPI_RES) {
        constexpr int CPRO_ = C::WTN_OUT / 8, RPIO_ = 64 / CPRO_;
        const int gm0_ = m0 + wm * WTM, gn0_ = tn * C::BN_OUT + wn * C::WTN_OUT;
#pragma unroll
        for (int t = 0; t < RES_N; t++) {
            const int m = gm0_ + t * RPIO_ + lane / CPRO_, n = gn0_ + (lane % CPRO_) * 8;
            if (m < g.M && n < g.N) resv[t] = *(const u32x4_t *)(g.res + (size_t)m * g.ldc + n);
        }
    }
    __syncthreads();   // every wave is done with the ring before staging reuses it

    // QKV with 64-wide wave tiles (8 waves): the two waves of one 128-wide
    // head stage into one [WTM][128 + pad] area, side by side
    constexpr bool QHALF = EPI == EPI_QKV && WTN == 64;
    static_assert(EPI != EPI_QKV || WTN == 128 || WTN == 64, "QKV epilogue: 64- or 128-wide wave tiles");
    constexpr int WO = C::WTN_OUT, LDW = QHALF ? 128 + C::EPAD : WO + C::EPAD;
    uint16_t *const hstg = smem + (wm * (WGN / 2) + wn / 2) * WTM * LDW;   // QHALF: the head's area
    uint16_t *stg = QHALF ? hstg + (wn % 2) * 64 : smem + wave * WTM * LDW;
    // a lane holds, per accumulator, 4 consecutive output columns
    // (lane / 16)*4 .. +3 of row lane % 16
    constexpr int NQ = 1;
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int row = i * MF + (lane & 15);
#pragma unroll
        for (int j = 0; j < (EPI == EPI_SWIGLU ? TN / 2 : TN); j++) {
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float x = acc[i][j][q * 4 + e];
                    if (EPI == EPI_SWIGLU) {
                        float gt = bfround(x);
                        float up = bfround(acc[i][j + TN / 2][q * 4 + e]);
                        float sg = bfround(silu_rcp(gt));
                        x = sg * up;
                    }
                    v[e] = x;
                }
                const int col = j * 16 + (lane >> 4) * 4;
                u32x2_t pk = {pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
                *(u32x2_t *)(stg + row * LDW + col) = pk;
            }
        }
    }
    __syncthreads();
    constexpr int CPRO = WO / 8, RPIO = 64 / CPRO;
    const int gm0 = m0 + wm * WTM;
    const int gn0 = tn * C::BN_OUT + wn * WO;
    if constexpr (QHALF) {
        // each of the head's two waves finishes half of its rows
        const int hr = (wn % 2) * (WTM / 2);
        qkv_epilogue<WTM / 2, LDW>(g, hstg + hr * LDW, gm0 + hr, gn0 / 128, lane);
        return;
    } else if constexpr (EPI == EPI_QKV) {
        qkv_epilogue<WTM, LDW>(g, stg, gm0, gn0 / 128, lane);
        return;
    }
#pragma unroll(EPI == EPI_RES ? WTM / RPIO : 4)
    for (int r0 = 0; r0 < WTM; r0 += RPIO) {
        const int r = r0 + lane / CPRO, cc = (lane % CPRO) * 8;
        const int m = gm0 + r, n = gn0 + cc;
        if (m < g.M && n < g.N) {
            u32x4_t v = *(const u32x4_t *)(stg + r * LDW + cc);
            if (EPI == EPI_BIAS || EPI == EPI_RES) {
                u32x4_t o = EPI == EPI_BIAS ? *(const u32x4_t *)(g.bias + n) : resv[EPI == EPI_RES ? r0 / RPIO : 0];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    v[e] = pack_bf2(lo_bf(v[e]) + lo_bf(o[e]), hi_bf(v[e]) + hi_bf(o[e]));
            }
            *(u32x4_t *)(g.C + (size_t)m * g.ldc + n) = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Reference kernel (gemm.cu:35-70 role): one fp32 dot product per output,
// y = bf16(acc + bias). Correctness/debug backend and the fallback for
// shapes the MFMA kernels do not take (K % 64, N % 8, misaligned).
// ---------------------------------------------------------------------------
__global__ void gemm_ref_kernel(const uint16_t *x, const uint16_t *w, const uint16_t *bias,
                                uint16_t *y, int M, int N, int K) {
    int n = blockIdx.x * 16 + (threadIdx.x & 15);
    int m = blockIdx.y * 16 + (threadIdx.x >> 4);
    if (m >= M || n >= N) return;
    float acc = 0.f;
    for (int k = 0; k < K; k++) acc += bf2f(x[(size_t)m * K + k]) * bf2f(w[(size_t)n * K + k]);
    if (bias) acc += bf2f(bias[n]);
    y[(size_t)m * N + n] = f2bf(acc);
}

__global__ void bias_add_kernel(const uint16_t *bias, uint16_t *y, int M, int N) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)M * N) return;
    y[idx] = f2bf(bf2f(y[idx]) + bf2f(bias[idx % N]));
}

// ---------------------------------------------------------------------------
// Runtime + dispatch
// ---------------------------------------------------------------------------
struct hd_gemm_runtime {
    int device_id;
    void *workspace;
    size_t workspace_bytes;
};
static hd_gemm_runtime *g_rt = nullptr;
static int g_use_production = 1;   // hd_gemm_set_backend

extern "C" hd_gemm_runtime *hd_gemm_runtime_init(int device_id, size_t workspace_bytes) {
    if (hipSetDevice(device_id) != hipSuccess) {
        snprintf(hd_cuda_errbuf(), 512, "gemm rt: hipSetDevice(%d) failed", device_id);
        return nullptr;
    }
    hd_gemm_runtime *rt = (hd_gemm_runtime *)calloc(1, sizeof(hd_gemm_runtime));
    if (!rt) { snprintf(hd_cuda_errbuf(), 512, "gemm rt oom"); return nullptr; }
    rt->device_id = device_id;
    if (workspace_bytes) {
        if (hipMalloc(&rt->workspace, workspace_bytes) != hipSuccess) {
            snprintf(hd_cuda_errbuf(), 512, "gemm rt: workspace hipMalloc failed");
            free(rt);
            return nullptr;
        }
        rt->workspace_bytes = workspace_bytes;
    }
    g_rt = rt;
    return rt;
}
extern "C" void hd_gemm_runtime_destroy(hd_gemm_runtime *rt) {
    if (!rt) return;
    if (rt->workspace) (void)hipFree(rt->workspace);
    if (g_rt == rt) g_rt = nullptr;
    free(rt);
}
extern "C" void *hd_gemm_workspace(hd_gemm_runtime *rt) { return rt ? rt->workspace : nullptr; }
extern "C" size_t hd_gemm_workspace_bytes(hd_gemm_runtime *rt) { return rt ? rt->workspace_bytes : 0; }
extern "C" void hd_gemm_set_backend(int p) { g_use_production = p; }
extern "C" void hd_gemm_set_prod_backend(int) {}   // one production family

// Sums the K chunks of each tail tile (fp32, chunk order) and applies the
// epilogue exactly as gemm_ms_kernel does on its accumulators: four output
// columns per thread.
template <int BM, int BN, int WGN, int EPI>
__global__ void gemm_tail_merge_kernel(GemmArgs g, int n_tail) {
    constexpr int BN_OUT = EPI == EPI_SWIGLU ? BN / 2 : BN, WTN = BN / WGN, WO = EPI == EPI_SWIGLU ? WTN / 2 : WTN;
    constexpr int GROUP_M = 8;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n_tail * BM * (BN_OUT / 4)) return;
    const int c = (int)(i % (BN_OUT / 4)) * 4, r = (int)((i / (BN_OUT / 4)) % BM);
    const int t = (int)(i / ((size_t)BM * (BN_OUT / 4)));
    const int lin = g.n_whole + t;
    const int in_group = GROUP_M * g.ntn;
    const int first_m = (lin / in_group) * GROUP_M;
    const int gm = min(g.ntm - first_m, GROUP_M);
    const int tm = first_m + (lin % in_group) % gm, tn = (lin % in_group) / gm;
    const int m = tm * BM + r, n = tn * BN_OUT + c;
    if (m >= g.M || n >= g.N) return;
    const int ca = EPI == EPI_SWIGLU ? (c / WO) * WTN + c % WO : c;   // accumulator column
    static_assert(EPI != EPI_QKV, "QKV tails: gemm_tail_qkv_fused_kernel");
    f32x4_t a = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < g.split; p++) {
        const float *pt = g.part + ((size_t)(t * g.split + p) * BM + r) * BN;
        a += *(const f32x4_t *)(pt + ca);
        if (EPI == EPI_SWIGLU) u += *(const f32x4_t *)(pt + ca + WTN / 2);
    }
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float x = a[e];
        if (EPI == EPI_SWIGLU) {
            const float gt = bfround(x), up = bfround(u[e]);
            const float sg = bfround(silu_rcp(gt));
            x = sg * up;
        }
        v[e] = x;
    }
    u32x2_t pk = {pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
    if (EPI == EPI_BIAS || EPI == EPI_RES) {
        const uint16_t *o = EPI == EPI_BIAS ? g.bias + n : g.res + (size_t)m * g.ldc + n;
        const u32x2_t ov = *(const u32x2_t *)o;
#pragma unroll
        for (int e = 0; e < 2; e++) pk[e] = pack_bf2(lo_bf(pk[e]) + lo_bf(ov[e]), hi_bf(pk[e]) + hi_bf(ov[e]));
    }
    *(u32x2_t *)(g.C + (size_t)m * g.ldc + n) = pk;
}

// Rows per wave of the fused QKV tail (32: 22.6 vs 23.6 us with 64 for a
// 1152-token block's all-split grid, equal at 8704 rows).
constexpr int QKV_TAIL_RS = 32;

// EPI_QKV tail tiles in one pass: one wave per (tile, RS-row slice, head)
// sums the K chunks' fp32 partials of its rows (in chunk order, as
// gemm_tail_merge_kernel does), stages the bf16 projection in LDS exactly as
// gemm_ms_kernel stages it and runs the same qkv_epilogue; no bf16 staging
// round trip through memory and one launch instead of two.
template <int BM, int BN, int RS>
__global__ __launch_bounds__(64) void gemm_tail_qkv_fused_kernel(GemmArgs g, int n_tail) {
    constexpr int LDW = 128 + 8, GROUP_M = 8, NSL = BM / RS, NH = BN / 128;
    __shared__ __attribute__((aligned(16))) uint16_t stg[RS * LDW];
    const int lane = threadIdx.x;
    const int b = blockIdx.x;
    const int hc = b % NH, sl = (b / NH) % NSL, t = b / (NH * NSL);
    const int lin = g.n_whole + t;
    const int in_group = GROUP_M * g.ntn;
    const int first_m = (lin / in_group) * GROUP_M;
    const int gm = min(g.ntm - first_m, GROUP_M);
    const int tm = first_m + (lin % in_group) % gm, tn = (lin % in_group) / gm;
    // lane: 4 consecutive columns c4 .. c4+3 of rows 2i + rh (i < 32); the
    // partials of 4 rows x every chunk (split <= 8) are loaded before any
    // is summed, so up to 32 loads per lane are in flight
    const int c4 = (lane % 32) * 4, rh = lane / 32;
    const float *pbase = g.part + ((size_t)t * g.split * BM + sl * RS + rh) * BN + hc * 128 + c4;
    for (int i0 = 0; i0 < RS / 2; i0 += 4) {
        f32x4_t pv[8][4];
#pragma unroll
        for (int p = 0; p < 8; p++)
            if (p < g.split)
#pragma unroll
                for (int k = 0; k < 4; k++)
                    pv[p][k] = *(const f32x4_t *)(pbase + ((size_t)p * BM + 2 * (i0 + k)) * BN);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < 8; p++)
                if (p < g.split) a += pv[p][k];
            const int r = 2 * (i0 + k) + rh;
            *(u32x2_t *)(stg + r * LDW + c4) = (u32x2_t){pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    qkv_epilogue<RS, LDW>(g, stg, tm * BM + sl * RS, (tn * BN) / 128 + hc, lane);
}

// Resident blocks of one round (one GEMM block per CU).
static int gemm_slots() {
    static int dev_cached = -1, cus = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (dev != dev_cached) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        dev_cached = dev;
    }
    return cus;
}

// Tail split plan for `units` tiles of nk K tiles on `occ` blocks per CU:
// the tiles of the last, partly filled round (all tiles when there are
// fewer than half a round) run as P K chunks (2..8) when that round is at
// most half full and the partial tiles fit in ws_bytes. Returns P (1: no
// split).
static int tail_split_of(long units, int nk, size_t tile_bytes, int64_t ws_bytes,
                         size_t stage_bytes = 0, int occ = 1) {
    const int slots = gemm_slots() * occ;
    if (slots <= 0 || ws_bytes <= 0) return 1;
    const long rem = units % slots;
    if (rem == 0 || rem > slots / 2) return 1;
    int P = (int)(slots / rem);
    if (P > 8) P = 8;
    if (P > nk / 4) P = nk / 4;   // chunks of at least 4 K tiles
    if (P < 2 || (int64_t)rem * (P * (int64_t)tile_bytes + (int64_t)stage_bytes) > ws_bytes) return 1;
    return P;
}

template <int BM, int BN, int BK, int NS, int WGM, int WGN, int EPI, int SGB = 0, int OCC = 1,
          int LDR = 0, int MF = 32>
static void launch_ms(GemmArgs &g, void *ws = nullptr, int64_t ws_bytes = 0) {
    using Cfg = MsCfg<BM, BN, BK, NS, WGM, WGN, EPI, MF>;
    g.ntm = (g.M + BM - 1) / BM;
    g.ntn = (g.N + Cfg::BN_OUT - 1) / Cfg::BN_OUT;
    const long units = (long)g.ntm * g.ntn;
    int P = 1;
    if (ws)
        P = tail_split_of(units, g.K / BK, (size_t)BM * BN * 4, ws_bytes,
                          EPI == EPI_QKV ? (size_t)BM * BN * 2 : 0, OCC);
    const long n_tail = P > 1 ? units % ((long)gemm_slots() * OCC) : 0;
    g.n_whole = (int)(units - n_tail);
    g.split = P;
    g.part = (float *)ws;
    gemm_ms_kernel<BM, BN, BK, NS, WGM, WGN, EPI, SGB, OCC, LDR, MF>
        <<<(unsigned)(g.n_whole + n_tail * P), Cfg::NT, 0, hd_stream()>>>(g);
    if (n_tail) {
        if constexpr (EPI == EPI_QKV) {
            static_assert(BM % QKV_TAIL_RS == 0, "QKV tail slices");
            gemm_tail_qkv_fused_kernel<BM, BN, QKV_TAIL_RS>
                <<<(unsigned)(n_tail * (BM / QKV_TAIL_RS) * (BN / 128)), 64, 0, hd_stream()>>>(g, (int)n_tail);
        } else {
            gemm_tail_merge_kernel<BM, BN, WGN, EPI>
                <<<hd_cdiv((size_t)n_tail * BM * (Cfg::BN_OUT / 4), 256), 256, 0, hd_stream()>>>(
                    g, (int)n_tail);
        }
    }
}

// Tile configuration per shape. The 8-wave 256-wide kernels are the main
// path; a 192-row tile is taken when it quantises the grid onto the 256 CUs
// better (M = 8704 without a workspace: 34 -> 46 row tiles), and 128x128
// tiles for grids too small to fill the chip with 256x256 tiles.
static double quant_eff(long tiles) {
    long rounds = (tiles + 255) / 256;
    return (double)tiles / (double)(rounds * 256);
}

// Estimated time (s) of a tile family: rounds of resident blocks, each the
// time of `occ` tiles on a CU (2*BM*BNA*K flops at ~half the per-CU peak x
// the family's relative per-flop efficiency: 192-row tiles 8-18 % slower
// per flop than 256-row ones, 128x128 tiles at two per CU ~20 %); with the
// tail split the last round is one chunk plus the merge (the fp32 partials
// written and read once at HBM rate, and a launch).
static double tile_cost(long units, int occ, int BM, int BNA, int K, double eff, int P) {
    const long slots = (long)(gemm_slots() > 0 ? gemm_slots() : 256) * occ;
    const double rate = 2.5e15 / 256 * 0.5 * eff;
    const double t_round = occ * 2.0 * BM * BNA * (double)K / rate;
    const long full = units / slots, rem = units % slots;
    double t = full * t_round;
    if (rem) {
        if (P > 1)
            t += t_round / P + (double)rem * P * BM * BNA * 8.0 / 8e12 + 4e-6;
        else
            t += t_round;
    }
    return t;
}

template <int EPI>
static const char *pick_and_launch(GemmArgs &g, bool launch, void *ws = nullptr, int64_t ws_bytes = 0) {
    const int bn_out = EPI == EPI_SWIGLU ? 128 : 256;
    const long tn = (g.N + bn_out - 1) / bn_out;
    const long t256 = (long)((g.M + 255) / 256) * tn;
    const long t192 = (long)((g.M + 191) / 192) * tn;
    const long t128 = (long)((g.M + 127) / 128) * ((g.N + bn_out / 2 - 1) / (bn_out / 2));
    const int nk = g.K / 64;
    // tail split plans (P = 1: none) of the three tile families
    const int p256 = ws ? tail_split_of(t256, nk, (size_t)256 * 256 * 4, ws_bytes) : 1;
    const int p192 = ws ? tail_split_of(t192, nk, (size_t)192 * 256 * 4, ws_bytes) : 1;
    const int p128 = ws ? tail_split_of(t128, nk, (size_t)128 * 128 * 4, ws_bytes, 0, 2) : 1;
    const double c256 = tile_cost(t256, 1, 256, 256, g.K, 1.0, p256);
    const double c192 = tile_cost(t192, 1, 192, 256, g.K, 0.9, p192);
    const double c128 = tile_cost(t128, 2, 128, 128, g.K, 0.8, p128);
    // buffer loads address with 32-bit byte offsets: both operands under 2 GiB
    const bool fits = (size_t)(g.M + 256) * g.K * 2 < ((size_t)1 << 31) &&
                      (size_t)g.N * g.K * 2 < ((size_t)1 << 31);
    const bool use192 = c192 < c256;
    const bool split256 = p256 > 1;
    if (!fits) {
        // operands of 2 GiB or more: equal-depth rings filled by
        // global_load_lds (64-bit addresses), the same MFMA tiles and K order
        if (use192) {
            if (launch) launch_ms<192, 256, 64, 2, 2, 4, EPI, 3, 1, 0, 16>(g, ws, ws_bytes);
            return "bf16_192x256x64_w2x4_m16_ring";
        }
        if (launch) launch_ms<256, 256, 64, 2, 2, 4, EPI, 3, 1, 0, 16>(g, ws, ws_bytes);
        return split256 ? "bf16_256x256x64_w2x4_m16_ring_tailsplit" : "bf16_256x256x64_w2x4_m16_ring";
    }
    // Small grids (the 256 x 256 tiles fill at most one round, K <= 4096, no
    // SwiGLU): 128 x 128 tiles, two blocks per CU, no K split. The vision
    // tower's M = 1728 GEMMs (K = 1152): 11.5-20 us against 22-27 us with a
    // 4-chunk K split; a 1152-token block's o_proj: equal at block level.
    // Longer K (the 12288-deep down projection) and the SwiGLU epilogue stay
    // on the 256-row tiles (120 vs 139-150 us; 192-212 vs 208-223 us).
    const int slots1 = gemm_slots() > 0 ? gemm_slots() : 256;
    if (EPI != EPI_SWIGLU && t256 <= slots1 && g.K <= 4096) {
        if (launch) launch_ms<128, 128, 64, 2, 2, 2, EPI, 8, 2, 5, 16>(g);
        return "bf16_128x128x64_w2x2_occ2_m16";
    }
    if (c128 < c256 && c128 < c192) {
        if (launch) launch_ms<128, 128, 64, 2, 2, 2, EPI, 8, 2, 5, 16>(g, ws, ws_bytes);
        return p128 > 1 ? "bf16_128x128x64_w2x2_occ2_m16_split" : "bf16_128x128x64_w2x2_occ2_m16";
    }
    // 8 waves (2 x 4) of 128x64 (96x64) on v_mfma_f32_16x16x32_bf16 (8 x 4
    // accumulator tiles per wave) with one fragment ring across the K loop
    // and buffer loads straight to LDS, the A operand's LDS ring one stage
    // deeper than B's, and the next k-step's fragment reads and the refill
    // loads placed between every other MFMA; two waves per SIMD cover each
    // other's barrier and load-issue stalls. On N(0,1) data the matrix cores
    // sustain ~14 % more FLOP/s with 16x16x32 than with 32x32x16
    // instructions under the power limit.
    if (use192) {
        if (launch) launch_ms<192, 256, 64, 2, 2, 4, EPI, 8, 1, 5, 16>(g, ws, ws_bytes);
        return "bf16_192x256x64_w2x4_m16_ring_buf";
    }
    if (launch) launch_ms<256, 256, 64, 2, 2, 4, EPI, 8, 1, 5, 16>(g, ws, ws_bytes);
    return split256 ? "bf16_256x256x64_w2x4_m16_ring_buf_tailsplit" : "bf16_256x256x64_w2x4_m16_ring_buf";
}

static bool mfma_ok(const void *x, const void *y, int N, int K) {
    return K % 64 == 0 && N % 8 == 0 && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0);
}

static void gemm_launch(int epi, GemmArgs &g, void *ws = nullptr, int64_t ws_bytes = 0) {
    switch (epi) {
    case EPI_NONE: pick_and_launch<EPI_NONE>(g, true, ws, ws_bytes); break;
    case EPI_BIAS: pick_and_launch<EPI_BIAS>(g, true, ws, ws_bytes); break;
    case EPI_RES: pick_and_launch<EPI_RES>(g, true, ws, ws_bytes); break;
    case EPI_SWIGLU: pick_and_launch<EPI_SWIGLU>(g, true, ws, ws_bytes); break;
    }
}

// QKV projection with the q/k RMSNorm + rotary and the V^T layout fused into
// the GEMM epilogue (EPI_QKV). Returns 1 without launching when the shape is
// outside the fused path (the caller then runs hd_linear_concat3 +
// hd_qkv_epilogue, which compute the same values).
extern "C" int hd_linear_qkv_rope_ws(const void *x, const void *wq, const void *wk, const void *wv,
                                     const void *qn_w, const void *kn_w, const float *cs, void *q,
                                     void *k, void *vt, int batch, int seq, int heads, int kv_heads,
                                     int hidden, float eps, void *ws, int64_t ws_bytes) {
    if (!x || !wq || !wk || !wv || !qn_w || !kn_w || !cs || !q || !k || !vt || batch <= 0 ||
        seq <= 0 || heads <= 0 || kv_heads <= 0 || hidden <= 0)
        return 1;
    const int M = batch * seq, N = (heads + 2 * kv_heads) * 128;
    const bool ok = seq % 64 == 0 && (heads * 128) % 256 == 0 &&
                    (kv_heads * 128) % 256 == 0 && hidden % 64 == 0 && hidden <= 8192 &&
                    (size_t)(M + 256) * hidden * 2 < ((size_t)1 << 31) &&
                    (size_t)heads * 128 * hidden * 2 < ((size_t)1 << 31) &&
                    ((((uintptr_t)x | (uintptr_t)vt | (uintptr_t)q | (uintptr_t)k | (uintptr_t)qn_w |
                       (uintptr_t)kn_w | (uintptr_t)cs) & 15) == 0);
    if (!ok) return 1;
    GemmArgs g = {};
    g.A = (const uint16_t *)x;
    g.B[0] = (const uint16_t *)wq;
    g.B[1] = (const uint16_t *)wk;
    g.B[2] = (const uint16_t *)wv;
    g.seg_end[0] = heads * 128;
    g.seg_end[1] = (heads + kv_heads) * 128;
    g.seg_end[2] = N;
    g.M = M; g.N = N; g.K = hidden; g.ldc = N;
    g.qn_w = (const uint16_t *)qn_w;
    g.kn_w = (const uint16_t *)kn_w;
    g.cs = (const float2 *)cs;
    g.q_out = (uint16_t *)q;
    g.k_out = (uint16_t *)k;
    g.vt_out = (uint16_t *)vt;
    g.seq = seq; g.heads = heads; g.kv_heads = kv_heads; g.eps = eps;
    const long tn = N / 256;
    const long t256 = (long)((M + 255) / 256) * tn, t192 = (long)((M + 191) / 192) * tn;
    if (ws && (uintptr_t)ws % 16) ws = nullptr;
    const bool split256 =
        ws && tail_split_of(t256, hidden / 64, (size_t)256 * 256 * 4, ws_bytes, (size_t)256 * 256 * 2) > 1;
    const bool use192 = !split256 && quant_eff(t192) > quant_eff(t256) * 1.12;
    // 8 waves: two 64-wide wave tiles per head, 16x16x32 MFMA tiles
    if (use192) launch_ms<192, 256, 64, 2, 2, 4, EPI_QKV, 8, 1, 5, 16>(g, ws, ws ? ws_bytes : 0);
    else launch_ms<256, 256, 64, 2, 2, 4, EPI_QKV, 8, 1, 5, 16>(g, ws, ws ? ws_bytes : 0);
    hd_check_launch("linear_qkv_rope");
    return 0;
}

extern "C" int hd_linear_qkv_rope(const void *x, const void *wq, const void *wk, const void *wv,
                                  const void *qn_w, const void *kn_w, const float *cs, void *q,
                                  void *k, void *vt, int batch, int seq, int heads, int kv_heads,
                                  int hidden, float eps) {
    return hd_linear_qkv_rope_ws(x, wq, wk, wv, qn_w, kn_w, cs, q, k, vt, batch, seq, heads,
                                 kv_heads, hidden, eps, nullptr, 0);
}

// Matrix-core ceiling probe (diagnostic): every wave runs 8 independent
// v_mfma_f32_32x32x16_bf16 accumulator chains (MF 32), or 16 chains of
// v_mfma_f32_16x16x32_bf16 (MF 16: the same FLOP per round), over operands
// held in registers (4 A and 4 B fragments loaded once from `ops`, rotated so
// that consecutive MFMAs see different data), no memory traffic in the loop.
// One block of 8 waves per CU. Random operands give the rate the chip
// sustains under its power limit with GEMM-like data; constant operands, the
// issue ceiling.
template <int MF>
__global__ __launch_bounds__(512) void mfma_probe_kernel(const uint16_t *__restrict__ ops, int n_ops,
                                                         int iters, float *__restrict__ out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    bf16x8_t a[4], b[4];
#pragma unroll
    for (int f = 0; f < 4; f++) {
        const long fi = ((long)(blockIdx.x * 8 + wave) * 8 + f) * 64 + lane, nf = n_ops / 8;
        a[f] = *(const bf16x8_t *)(ops + (fi % nf) * 8);
        b[f] = *(const bf16x8_t *)(ops + ((fi + 4 * 64) % nf) * 8);
    }
    float t = 0.f;
    if constexpr (MF == 32) {
        f32x16_t acc[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[j][e] = 0.f;
        for (int it = 0; it < iters; it += 4) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < 8; j++)
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(j + r) & 3], b[((j >> 2) + r) & 3],
                                                                     acc[j], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) t += acc[j][e];
    } else {
        // 16x16x32: half the FLOP per instruction, twice the instructions
        f32x4_t acc[16];
#pragma unroll
        for (int j = 0; j < 16; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[j][e] = 0.f;
        for (int it = 0; it < iters; it += 4) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < 16; j++)
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[(j + r) & 3], b[((j >> 2) + r) & 3],
                                                                     acc[j], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 16; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) t += acc[j][e];
    }
    out[(size_t)blockIdx.x * 512 + threadIdx.x] = t;
}

// Runs the probe on `blocks` blocks (one per CU: the CU count) with `iters`
// (a multiple of 4) rounds of 32x32x16-equivalent work per chain, on MFMA
// shape 32 or 16; returns the FLOP it performs.
extern "C" double hd_mfma_probe(const void *ops, int n_ops, int blocks, int iters, int shape, float *out) {
    const bool m16 = shape == 16;   // 16 chains of half-size instructions: the same FLOP per round
    if (!ops || !out || n_ops < 4 * 4096 + 16 || blocks <= 0 || iters <= 0 || iters % 4 ||
        (shape != 16 && shape != 32)) {
        snprintf(hd_cuda_errbuf(), 512, "mfma_probe: bad args");
        return 0.0;
    }
    if (m16) mfma_probe_kernel<16><<<blocks, 512, 0, hd_stream()>>>((const uint16_t *)ops, n_ops, iters, out);
    else mfma_probe_kernel<32><<<blocks, 512, 0, hd_stream()>>>((const uint16_t *)ops, n_ops, iters, out);
    hd_check_launch("mfma_probe");
    return (double)blocks * 8 * 8 * (double)iters * 32.0 * 32.0 * 16.0 * 2.0;
}

extern "C" const char *hd_gemm_config_name(int M, int N, int K, int epi) {
    GemmArgs g = {};
    g.M = M; g.N = N; g.K = K;
    if (K % 64 || N % 8) return "reference";
    switch (epi) {
    case EPI_BIAS: return pick_and_launch<EPI_BIAS>(g, false);
    case EPI_RES: return pick_and_launch<EPI_RES>(g, false);
    case EPI_SWIGLU: return pick_and_launch<EPI_SWIGLU>(g, false);
    default: return pick_and_launch<EPI_NONE>(g, false);
    }
}

extern "C" void hd_linear_reference(const void *x, const void *w, const void *bias, void *y,
                                    int M, int N, int K, int transpose_w) {
    if (!x || !w || !y || M <= 0 || N <= 0 || K <= 0) {
        snprintf(hd_cuda_errbuf(), 512, "linear: bad args");
        return;
    }
    if (!transpose_w) {
        snprintf(hd_cuda_errbuf(), 512, "linear: transpose_w=0 unsupported");
        return;
    }
    dim3 grid(hd_cdiv(N, 16), hd_cdiv(M, 16));
    gemm_ref_kernel<<<grid, 256, 0, hd_stream()>>>((const uint16_t *)x, (const uint16_t *)w,
                                                   (const uint16_t *)bias, (uint16_t *)y, M, N, K);
    hd_check_launch("linear_reference");
}

extern "C" void hd_linear(const void *x, const void *w, const void *bias, void *y, int M, int N,
                          int K, int transpose_w) {
    if (!x || !w || !y || M <= 0 || N <= 0 || K <= 0) {
        snprintf(hd_cuda_errbuf(), 512, "linear: bad args");
        return;
    }
    if (!transpose_w) {
        snprintf(hd_cuda_errbuf(), 512, "linear: transpose_w=0 unsupported");
        return;
    }
    if (!g_use_production || !mfma_ok(x, y, N, K) || (bias && (uintptr_t)bias % 16)) {
        // reference backend: fp32 result + bias rounded once; production
        // rounding (two roundings) is kept by adding the bias separately.
        hd_linear_reference(x, w, nullptr, y, M, N, K, 1);
        if (bias) {
            bias_add_kernel<<<hd_cdiv((size_t)M * N, 256), 256, 0, hd_stream()>>>(
                (const uint16_t *)bias, (uint16_t *)y, M, N);
            hd_check_launch("linear bias");
        }
        return;
    }
    GemmArgs g = {};
    g.A = (const uint16_t *)x;
    g.B[0] = g.B[1] = g.B[2] = (const uint16_t *)w;
    g.seg_end[0] = g.seg_end[1] = g.seg_end[2] = N;
    g.C = (uint16_t *)y;
    g.bias = (const uint16_t *)bias;
    g.M = M; g.N = N; g.K = K; g.ldc = N;
    gemm_launch(bias ? EPI_BIAS : EPI_NONE, g);
    hd_check_launch("linear");
}

extern "C" void hd_linear_ws(const void *x, const void *w, const void *bias, void *y, int M, int N,
                             int K, void *ws, int64_t ws_bytes) {
    if (!x || !w || !y || M <= 0 || N <= 0 || K <= 0 || !mfma_ok(x, y, N, K) ||
        (bias && (uintptr_t)bias % 16) || (ws && (uintptr_t)ws % 16) || !g_use_production) {
        hd_linear(x, w, bias, y, M, N, K, 1);
        return;
    }
    GemmArgs g = {};
    g.A = (const uint16_t *)x;
    g.B[0] = g.B[1] = g.B[2] = (const uint16_t *)w;
    g.seg_end[0] = g.seg_end[1] = g.seg_end[2] = N;
    g.C = (uint16_t *)y;
    g.bias = (const uint16_t *)bias;
    g.M = M; g.N = N; g.K = K; g.ldc = N;
    gemm_launch(bias ? EPI_BIAS : EPI_NONE, g, ws, ws ? ws_bytes : 0);
    hd_check_launch("linear");
}

// ---- hd_linear_noalloc: hd_linear_ws with the tail-split workspace in a
// file-scope device array, for callers that cannot allocate (code under
// graph capture, serving loops, harnesses that forbid hipMalloc). 80 MiB:
// the workspace hd_gemm_ws_bytes() asks for on a 256-CU device (256 fp32
// 256x256 partial tiles + 128 bf16 staging tiles). Each GPU the library runs
// on holds its own copy until the process ends. Every call on a device
// shares that device's array: calls that overlap on one GPU (two streams,
// two threads) race. The split partials are written in full before the
// merge reads them, so nothing in the array has to start at zero.
static constexpr int64_t kNoAllocScratchBytes = (int64_t)256 * 256 * 256 * 4 + 128 * 256 * 256 * 2;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
static constexpr int kMaxDevices = 64;
// the array's device address, per device; atomic slots, since two host
// threads may look the address up at once (both store the same value)
static std::atomic<void *> g_scratch_dev[kMaxDevices];

extern "C" int64_t hd_linear_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" void hd_linear_noalloc(const void *x, const void *w, const void *bias, void *y, int M,
                                  int N, int K) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        snprintf(hd_cuda_errbuf(), 512, "linear_noalloc: no current device (or device id >= %d)",
                 kMaxDevices);
        return;
    }
    void *sp = g_scratch_dev[dev].load(std::memory_order_acquire);
    if (!sp) {
        // once per device, with that device current: the host-side name of
        // the array is not its device address
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            snprintf(hd_cuda_errbuf(), 512, "linear_noalloc: hipGetSymbolAddress(scratch): %s",
                     hipGetErrorString(e));
            return;
        }
        g_scratch_dev[dev].store(p, std::memory_order_release);
        sp = p;
    }
    const int64_t need = hd_gemm_ws_bytes();
    if (need > kNoAllocScratchBytes) {
        snprintf(hd_cuda_errbuf(), 512,
                 "linear_noalloc: this device's tail split needs %lld workspace bytes, the static "
                 "scratch holds %lld",
                 (long long)need, (long long)kNoAllocScratchBytes);
        return;
    }
    hd_linear_ws(x, w, bias, y, M, N, K, sp, kNoAllocScratchBytes);
}

// hd_linear writing rows of stride ldc (>= N, ldc % 8 == 0): the vision
// tower's fc1 lands in a row padded to the next GEMM's K.
extern "C" void hd_linear_ld(const void *x, const void *w, const void *bias, void *y, int M, int N,
                             int K, int ldc) {
    if (!x || !w || !y || M <= 0 || N <= 0 || K <= 0 || ldc < N || ldc % 8 || !mfma_ok(x, y, N, K) ||
        (bias && (uintptr_t)bias % 16)) {
        snprintf(hd_cuda_errbuf(), 512, "linear_ld: bad args");
        return;
    }
    GemmArgs g = {};
    g.A = (const uint16_t *)x;
    g.B[0] = g.B[1] = g.B[2] = (const uint16_t *)w;
    g.seg_end[0] = g.seg_end[1] = g.seg_end[2] = N;
    g.C = (uint16_t *)y;
    g.bias = (const uint16_t *)bias;
    g.M = M; g.N = N; g.K = K; g.ldc = ldc;
    gemm_launch(bias ? EPI_BIAS : EPI_NONE, g);
    hd_check_launch("linear_ld");
}

extern "C" void hd_linear_residual_ws(const void *x, const void *w, const void *res, void *y, int M,
                                      int N, int K, void *ws, int64_t ws_bytes) {
    if (!x || !w || !res || !y || M <= 0 || N <= 0 || K <= 0 || !mfma_ok(x, y, N, K) ||
        (uintptr_t)res % 16 || (ws && (uintptr_t)ws % 16)) {
        snprintf(hd_cuda_errbuf(), 512, "linear_residual: bad args");
        return;
    }
    GemmArgs g = {};
    g.A = (const uint16_t *)x;
    g.B[0] = g.B[1] = g.B[2] = (const uint16_t *)w;
    g.seg_end[0] = g.seg_end[1] = g.seg_end[2] = N;
    g.C = (uint16_t *)y;
    g.res = (const uint16_t *)res;
    g.M = M; g.N = N; g.K = K; g.ldc = N;
    gemm_launch(EPI_RES, g, ws, ws ? ws_bytes : 0);
    hd_check_launch("linear_residual");
}

extern "C" void hd_linear_residual(const void *x, const void *w, const void *res, void *y, int M,
                                   int N, int K) {
    hd_linear_residual_ws(x, w, res, y, M, N, K, nullptr, 0);
}

// Workspace for the tail split of one GEMM on the current device: one round
// of 256x256 fp32 partial tiles (at most half a round of tiles, split up to
// 8 ways, at most one round of chunks) plus bf16 staging of half a round of
// tiles (the QKV epilogue pass).
extern "C" int64_t hd_gemm_ws_bytes(void) {
    const int64_t slots = gemm_slots() > 0 ? gemm_slots() : 256;
    return slots * 256 * 256 * 4 + (slots / 2) * 256 * 256 * 2;
}

extern "C" void hd_linear_swiglu_ws(const void *x, const void *wg, const void *wu, void *y, int M,
                                    int F, int K, void *ws, int64_t ws_bytes) {
    if (!x || !wg || !wu || !y || M <= 0 || F <= 0 || K <= 0 || !mfma_ok(x, y, F, K) ||
        F % 64 || (ws && (uintptr_t)ws % 16)) {
        snprintf(hd_cuda_errbuf(), 512, "linear_swiglu: bad args");
        return;
    }
    GemmArgs g = {};
    g.A = (const uint16_t *)x;
    g.B[0] = (const uint16_t *)wg;
    g.B[1] = (const uint16_t *)wu;
    g.B[2] = nullptr;
    g.seg_end[0] = g.seg_end[1] = g.seg_end[2] = F;
    g.C = (uint16_t *)y;
    g.M = M; g.N = F; g.K = K; g.ldc = F;
    gemm_launch(EPI_SWIGLU, g, ws, ws ? ws_bytes : 0);
    hd_check_launch("linear_swiglu");
}

extern "C" void hd_linear_swiglu(const void *x, const void *wg, const void *wu, void *y, int M,
                                 int F, int K) {
    hd_linear_swiglu_ws(x, wg, wu, y, M, F, K, nullptr, 0);
}

extern "C" void hd_linear_concat3(const void *x, const void *w0, int N0, const void *w1, int N1,
                                  const void *w2, int N2, void *y, int M, int K) {
    int N = N0 + N1 + N2;
    if (!x || !w0 || !y || M <= 0 || N0 <= 0 || K <= 0 || N0 % 256 || N1 % 256 || N2 % 256 ||
        (N1 && !w1) || (N2 && !w2) || !mfma_ok(x, y, N, K)) {
        snprintf(hd_cuda_errbuf(), 512, "linear_concat3: bad args");
        return;
    }
    GemmArgs g = {};
    g.A = (const uint16_t *)x;
    g.B[0] = (const uint16_t *)w0;
    g.B[1] = (const uint16_t *)(w1 ? w1 : w0);
    g.B[2] = (const uint16_t *)(w2 ? w2 : w0);
    g.seg_end[0] = N0;
    g.seg_end[1] = N0 + N1;
    g.seg_end[2] = N;
    g.C = (uint16_t *)y;
    g.M = M; g.N = N; g.K = K; g.ldc = N;
    gemm_launch(EPI_NONE, g);
    hd_check_launch("linear_concat3");
}
