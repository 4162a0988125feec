// Single-column GEMV (batch-1 decode): y[n] = sum_k W[n][k] x[k] for one activation column, on MFMA.
//
// Replaces, for one column, F.linear in Qwen2Engine.forward (seedplane/qwen_engine.py:121,136,138-139,143) and the
// Vulkan gemv.comp / swiglu.comp kernels (native/vulkan_decode/shaders/gemv.comp:1-51, swiglu.comp:1-44).
//
// A one-column GEMV streams its matrix once and is bound by how many bytes the chip keeps in flight, so this kernel
// is built for memory-level parallelism at low register cost:
//   * every wave issues the weight (and scale) loads of ALL its k-tiles first, unconditionally (tiles past the slice
//     re-read the slice's last tile and contribute zero), so the code is straight-line and each tile is consumed as
//     soon as its own loads land (progressive vmcnt waits) instead of after a whole batch;
//   * the activation column lives in LDS (staged once per block, or built there by the RMSNorm / attention-combine
//     prologue), not in registers: an MFMA A operand is read just before use, so a wave holds only its weight
//     tiles and the block's waves all fit on the CU at once;
//   * Q8 / Q4 codes enter the MFMA offset by a constant (1152 / 1024: one perm or mask per pair, no subtraction) and
//     each quant block's result is corrected by (offset + zero) * sum(x) in fp32, one FMA per output row;
//   * the A operand's row 0 is the column in fp16 and row 1 its fp16 remainders (split_f16: the norm prologue's, or
//     a.xlo), rows 2..15 zero, so output components 0 + 1 are the product with fp32-class activations at no extra
//     MFMA; the per-block scale work is one FMA per row group and quant block.
// Work decomposition: one block per (16-row unit, k-slice); unit = 16 rows, or 16 gate + 16 up rows for the SwiGLU
// pair (RG = 2); wave w of NW takes k-tiles w, w + NW, ... of the slice (T per wave); waves are reduced through LDS
// in wave order (deterministic).  Epilogues: store (+bias), residual add, SwiGLU to fp16, or a raw k-slice partial
// that the consuming kernel adds (no atomics, no fences).
#pragma once
#include "sp_gemv.h"

// The block's LDS: the slice's activations (fp16) and 16 bytes of zeros read by the lanes of MFMA rows 2..15
// (g1_x_halves halves), then the same span for their remainders (MFMA row 1), the cross-wave reduction, the prologue's
// scratch.
__host__ __device__ inline size_t g1_x_halves(int kslice, int KT) { return ((size_t)kslice * KT + 7) / 8 * 8 + 8; }
__host__ __device__ inline size_t g1_smem_bytes(int kslice, int KT, int nw, int rg, int pro_floats) {
    return g1_x_halves(kslice, KT) * 2 * 2 + (size_t)nw * rg * 16 * 4 + (size_t)pro_floats * 4;
}

template <int FMT, int RG, int T, int PRO>
__global__ void __launch_bounds__(1024) k_gemv1(GemvArgs a, ProArgs p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    constexpr int KT = TileGeom<FMT>::KT, ST = TileGeom<FMT>::STEPS;
    const int NW = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, r = lane & 15, g = lane >> 4;
    const int unit = blockIdx.x;
    const int k0 = blockIdx.y * a.kslice;
    const int k1 = min(a.nkt, k0 + a.kslice);
    const int klen = max(k1 - k0, 0) * KT;
    f16 *xs_lds = (f16 *)smem_raw;
    const size_t xh = g1_x_halves(a.kslice, KT);
    f16 *xl_lds = xs_lds + xh;                      // remainders
    float *red = (float *)(smem_raw + xh * 2 * 2);
    float *scr = red + NW * RG * 16;
    const bool has_lo = PRO == PRO_NORM || (PRO == PRO_NONE && a.xlo != nullptr);

    // ---- 0. the activation side's own global loads first: loads complete in issue order, so the activation work
    // below then waits only for them and runs while the weight tiles are still streaming in
    const int nx = klen / 8;                         // 16-byte pieces of the slice's activations
    uint4 xpre, xpre_lo;
    NormOps npre;
    if constexpr (PRO == PRO_NONE) {
        // from a clamped base and index (an empty last slice reads the final piece and stores nothing)
        const size_t base = (size_t)min(k0, a.nkt - 1) * KT;
        const int pc = min((int)threadIdx.x, max(nx - 1, 0));
        xpre = ((const uint4 *)(a.x + base))[pc];
        xpre_lo = has_lo ? ((const uint4 *)(a.xlo + base))[pc] : ((const uint4 *)g_zero_line)[0];
    } else if constexpr (PRO == PRO_NORM) {
        pro_norm_load(p, k0 * KT, npre);
    }
    __builtin_amdgcn_sched_barrier(0);               // keep these loads ahead of the weight loads

    // ---- 1. every weight / scale load of the wave's tiles, in tile order
    const uint8_t *wb[RG];
    const f16 *sb[RG];
#pragma unroll
    for (int i = 0; i < RG; ++i) {
        const size_t grp = (size_t)unit * RG + i;
        wb[i] = a.w + grp * a.nkt * TILE_BYTES;
        sb[i] = a.sz + grp * a.nkt * (FMT == 2 ? 32 : 128);
    }
    u32x4 wt[T][RG];
    uint32_t sq8[T][RG];
    u32x4 sq4[T][RG];
    bool valid[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int kt = k0 + wv + NW * t;
        valid[t] = kt < k1;
        const int kc = valid[t] ? kt : max(k1 - 1, 0);
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            wt[t][i] = __builtin_nontemporal_load((const u32x4 *)(wb[i] + (size_t)kc * TILE_BYTES) + lane);
            if constexpr (FMT == 2) sq8[t][i] = *((const uint32_t *)(sb[i] + (size_t)kc * 32) + r);
            if constexpr (FMT == 3) sq4[t][i] = *((const u32x4 *)(sb[i] + (size_t)kc * 128) + r);
        }
    }

    // ---- 2. the activation column of the slice in LDS (+ the zero line)
    if constexpr (PRO == PRO_NONE) {
        const uint4 *src = (const uint4 *)(a.x + (size_t)k0 * KT);
        uint4 *dst = (uint4 *)xs_lds, *dstl = (uint4 *)xl_lds;
        // unconditional stores (threads past the slice write the first pieces of the reduction area, which is only
        // written again after the barrier below), so the loads above are not moved behind the weight loads
        dst[(int)threadIdx.x < nx ? (int)threadIdx.x : (int)(xh / 4)] = xpre;          // red[0..3]
        dstl[(int)threadIdx.x < nx ? (int)threadIdx.x : (int)(xh / 8) + 1] = xpre_lo;  // red[4..7]
        for (int i = threadIdx.x + blockDim.x; i < nx; i += blockDim.x) dst[i] = src[i];
        if (has_lo) {
            const uint4 *srcl = (const uint4 *)(a.xlo + (size_t)k0 * KT);
            for (int i = threadIdx.x + blockDim.x; i < nx; i += blockDim.x) dstl[i] = srcl[i];
        }
    } else if constexpr (PRO == PRO_NORM) {
        pro_norm_finish(p, npre, xs_lds, xl_lds, k0 * KT, klen, scr);
    } else {
        pro_comb(p, xs_lds, k0 * KT, klen, scr);
    }
    if (threadIdx.x < 8) xs_lds[xh - 8 + threadIdx.x] = (f16)0.f;
    __syncthreads();

    // ---- 3. MFMA per tile and quant block; lanes of row 1 read the remainders, rows 2..15 the zero line
    const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};
    float acc[RG];
    f32x4 acc4[RG];
#pragma unroll
    for (int i = 0; i < RG; ++i) { acc[i] = 0.f; acc4[i] = (f32x4){0.f, 0.f, 0.f, 0.f}; }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int kt = k0 + wv + NW * t;
#pragma unroll
        for (int s = 0; s < ST; ++s) {
            const int xo = (kt - k0) * KT + s * 32 + 8 * g;
            const int off = !valid[t] ? (int)xh - 8 : r == 0 ? xo : (r == 1 && has_lo ? (int)xh + xo : (int)xh - 8);
            const f16x8 xa = *(const f16x8 *)(xs_lds + off);
            if constexpr (FMT == 1) {
#pragma unroll
                for (int i = 0; i < RG; ++i) acc4[i] = mfma16(xa, __builtin_bit_cast(f16x8, wt[t][i]), acc4[i]);
            } else {
                const f32x4 sx = mfma16(xa, ones8, (f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int i = 0; i < RG; ++i) {
                    const f32x4 dd = mfma16(xa, biased_step<FMT>(wt[t][i], s), (f32x4){0.f, 0.f, 0.f, 0.f});
                    float scale, offs;
                    if constexpr (FMT == 2) {
                        const uint32_t d = sq8[t][i];
                        scale = (float)__builtin_bit_cast(f16, (uint16_t)(s == 0 ? (d & 0xffffu) : (d >> 16)));
                        offs = QBias<FMT>::V;
                    } else {
                        uint32_t d;
                        if (s == 0) d = sq4[t][i].x; else if (s == 1) d = sq4[t][i].y; else if (s == 2) d = sq4[t][i].z; else d = sq4[t][i].w;
                        scale = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                        offs = QBias<FMT>::V + (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
                    }
                    acc[i] = fmaf(scale, fmaf(-offs, sx[0], dd[0]) + fmaf(-offs, sx[1], dd[1]), acc[i]);
                }
            }
        }
    }

    // ---- 4. waves reduced in wave order; lanes 0..15 of wave 0 finish row unit * 16 + r
    if (g == 0) {
#pragma unroll
        for (int i = 0; i < RG; ++i) red[(wv * RG + i) * 16 + r] = FMT == 1 ? acc4[i][0] + acc4[i][1] : acc[i];
    }
    __syncthreads();
    if (threadIdx.x >= 16) return;
    const int n = unit * 16 + r;
    if (n >= a.n_real) return;
    float v[RG];
#pragma unroll
    for (int i = 0; i < RG; ++i) {
        float t = red[i * 16 + r];
        for (int w2 = 1; w2 < NW; ++w2) t += red[(w2 * RG + i) * 16 + r];
        v[i] = t;
    }
    if constexpr (RG == 2) {
        f16 hi, lo;
        split_f16(silu_f(v[0]) * v[1], hi, lo);
        a.out_f16[n] = hi;
        if (a.out_lo) a.out_lo[n] = lo;
    } else if (a.epi == EPI_STORE) {
        a.out_f32[n] = v[0] + (a.bias ? a.bias[n] : 0.f);
    } else if (a.epi == EPI_RESID) {
        a.out_f32[n] += v[0];
    } else {
        a.out_f32[(size_t)blockIdx.y * a.pstride + n] = v[0];
    }
}
