// Block-dequant GEMV / small GEMM on MFMA: y[m][n] = sum_k x[m][k] * W[n][k] for m < M columns (M <= 64).
//
// Replaces F.linear in Qwen2Engine.forward (seedplane/qwen_engine.py:121,136,138-139,143) and the Vulkan gemv.comp /
// swiglu.comp / gemm_b.comp kernels (native/vulkan_decode/shaders/gemv.comp:1-51, swiglu.comp:1-44).
//
// Work decomposition
//   unit   = 16 output rows (32 for the SwiGLU epilogue: the packer interleaves the 16 gate rows i..i+15 with the 16
//            up rows of the same i, so one wave holds gate and up of the same output in the same lanes);
//   block  = R consecutive units x one k-slice (gridDim.y slices of kslice k-tiles); the NW waves of the block take
//            the slice's k-tiles w, w + NW, ... in batches of TB whose weight AND activation loads are all issued
//            before any is consumed.  Each activation fragment feeds the R * RG weight tiles of its k-tile (row-group
//            reuse: the L2 -> CU activation traffic per weight byte falls by R * RG).
//   reduce = the NW waves through LDS in a fixed order; with one slice the block finishes the outputs itself
//            (store / bias / residual add / SwiGLU); with S slices it writes its raw partial sums to slice s of a
//            partial buffer (EPI_PART) and the consuming kernel (RMSNorm, RoPE) adds the S slices in slice order.
//            No atomics and no device-scope fences (on gfx950 each agent-scope fence writes back / invalidates the
//            XCD's whole L2, which costs microseconds), and results are bit-identical from run to run.
// Per k-tile and wave: one 1 KiB dwordx4 load of codes per row group (fully coalesced), the per-row scales, the
// activation fragments (A operand, fp16, L2-resident), exact code->fp16 unpack and one 16x16x32 MFMA per quant block
// (K = 32 = one block): block scales are applied to the fp32 MFMA result, so the codes enter the matrix cores
// exactly and only the activations are rounded (to fp16).
#pragma once
#include "sp_device.h"

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_PART = 3 };

struct GemvArgs {
    const uint8_t *w;      // packed tiles
    const f16 *sz;         // per-tile scales (Q8) / scale+zero pairs (Q4); unused for F16
    int nkt;               // k-tiles per row group
    int units;             // R * gridDim.x
    int n_real;            // real output rows (EPI_SILU: intermediate size)
    const f16 *x;          // activations [m][ldx] fp16
    int ldx;
    int m;                 // columns (<= 16 * MT)
    float *out_f32;        // EPI_STORE / EPI_RESID output [m][ldo]; EPI_PART: slice s at out_f32 + s * pstride
    f16 *out_f16;          // EPI_SILU output [m][ldo]
    int ldo;
    const float *bias;     // EPI_STORE optional bias [n]
    int epi;
    int kslice;            // k-tiles per slice
    size_t pstride;        // EPI_PART: floats between slices
};
template <int FMT>
__device__ __forceinline__ f16x8 unpack_step(const u32x4 &t, int s) {
    if constexpr (FMT == 1) {              // F16: the lane's 16 bytes are 8 fp16 weights
        return __builtin_bit_cast(f16x8, t);
    } else if constexpr (FMT == 2) {       // Q8: bytes 0-7 block 0, bytes 8-15 block 1
        return s == 0 ? q8_unpack8(t[0], t[1]) : q8_unpack8(t[2], t[3]);
    } else {                               // Q4: dword s = group s
        return q4_unpack8(t[s]);
    }
}

// Threads per block: single-column-tile variants use up to 4 waves, wider ones up to 8 (each wave may then hold up to
// 256 VGPRs: the weight tiles and activation fragments of a whole batch stay in registers without spilling).
// TB = k-tiles per wave whose loads are in flight together.
template <int MT> struct GemvLimits { static constexpr int MAX_THREADS = MT == 1 ? 256 : 512; };
template <int FMT, int MT> struct GemvBatch { static constexpr int TB = MT == 1 ? (FMT == 3 ? 2 : 4) : 2; };

// Lane holds D[m = mt*16 + 4g + j][n = unit*16 + r], j < 4.  Operands the epilogue reads (bias, the residual) are
// loaded from clamped addresses before any store, so their loads are in flight together.
template <int RG>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, int unit, int mt, const f32x4 &v0, const f32x4 &v1) {
    const int r = threadIdx.x & 15, g = (threadIdx.x >> 4) & 3;
    const int n = unit * 16 + r;
    if (n >= a.n_real) return;
    int mrow[4];
    bool live[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = mt * 16 + 4 * g + j;
        live[j] = m < a.m;
        mrow[j] = live[j] ? m : a.m - 1;
    }
    if constexpr (RG == 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (live[j]) a.out_f16[(size_t)mrow[j] * a.ldo + n] = (f16)(silu_f(v0[j]) * v1[j]);
    } else if (a.epi == EPI_STORE) {
        const float bn = a.bias ? a.bias[n] : 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (live[j]) a.out_f32[(size_t)mrow[j] * a.ldo + n] = v0[j] + bn;
    } else if (a.epi == EPI_RESID) {
        float prev[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) prev[j] = a.out_f32[(size_t)mrow[j] * a.ldo + n];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (live[j]) a.out_f32[(size_t)mrow[j] * a.ldo + n] = prev[j] + v0[j];
    } else {
        float *dst = a.out_f32 + (size_t)blockIdx.y * a.pstride;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (live[j]) dst[(size_t)mrow[j] * a.ldo + n] = v0[j];
    }
}

template <int FMT, int MT, int RG, int R>
__global__ void __launch_bounds__(GemvLimits<MT>::MAX_THREADS) k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    constexpr int KT = TileGeom<FMT>::KT, ST = TileGeom<FMT>::STEPS;
    constexpr int TB = GemvBatch<FMT, MT>::TB;
    constexpr int NR = R * RG;                 // row groups per wave
    const int NW = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int u0 = blockIdx.x * R;
    const int k0 = blockIdx.y * a.kslice;
    const int k1 = min(a.nkt, k0 + a.kslice);

    f32x4 acc[NR][MT];
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[i][mt] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const f16x8 zero8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};
    const uint8_t *wbase[NR];
    const f16 *sbase[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const size_t grp = (size_t)u0 * RG + i;            // row group i of the block = unit u0 + i / RG, half i % RG
        wbase[i] = a.w + grp * a.nkt * TILE_BYTES;
        sbase[i] = a.sz + grp * a.nkt * (FMT == 2 ? 32 : 128);
    }
    const f16 *xrow[MT];
    bool xon[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        xon[mt] = m < a.m;
        xrow[mt] = a.x + (size_t)(xon[mt] ? m : 0) * a.ldx + 8 * g;
    }

    for (int kb = k0 + wv; kb < k1; kb += NW * TB) {
        // ---- issue the weight and activation loads of TB k-tiles before anything is consumed
        u32x4 wt[TB][NR];
        uint32_t sq8[TB][NR];
        u32x4 sq4[TB][NR];
        f16x8 xa[TB][MT][ST];
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int kt = kb + t * NW;
            if (kt >= k1) break;
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                wt[t][i] = __builtin_nontemporal_load((const u32x4 *)(wbase[i] + (size_t)kt * TILE_BYTES) + lane);
                if constexpr (FMT == 2) sq8[t][i] = *((const uint32_t *)(sbase[i] + (size_t)kt * 32) + r);
                if constexpr (FMT == 3) sq4[t][i] = *((const u32x4 *)(sbase[i] + (size_t)kt * 128) + r);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int s = 0; s < ST; ++s)
                    xa[t][mt][s] = xon[mt] ? *(const f16x8 *)(xrow[mt] + kt * KT + s * 32) : zero8;
        }
        // ---- MFMA per quant block
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int kt = kb + t * NW;
            if (kt >= k1) break;
#pragma unroll
            for (int s = 0; s < ST; ++s) {
                f32x4 xs[MT];
                if constexpr (FMT == 3) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) xs[mt] = mfma16(xa[t][mt][s], ones8, (f32x4){0.f, 0.f, 0.f, 0.f});
                }
#pragma unroll
                for (int i = 0; i < NR; ++i) {
                    const f16x8 b = unpack_step<FMT>(wt[t][i], s);
                    if constexpr (FMT == 1) {
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) acc[i][mt] = mfma16(xa[t][mt][s], b, acc[i][mt]);
                    } else if constexpr (FMT == 2) {
                        const uint32_t d = sq8[t][i];
                        const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(s == 0 ? (d & 0xffffu) : (d >> 16)));
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            acc[i][mt] += scale * mfma16(xa[t][mt][s], b, (f32x4){0.f, 0.f, 0.f, 0.f});
                    } else {
                        uint32_t d;
                        if (s == 0) d = sq4[t][i].x; else if (s == 1) d = sq4[t][i].y; else if (s == 2) d = sq4[t][i].z; else d = sq4[t][i].w;
                        const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                        const float zero = (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            const f32x4 dd = mfma16(xa[t][mt][s], b, (f32x4){0.f, 0.f, 0.f, 0.f});
                            acc[i][mt] += scale * (dd - zero * xs[mt]);
                        }
                    }
                }
            }
        }
    }

    // ---- one wave: finish in registers; several: reduce through LDS in wave order, wave w finishing the (unit,
    // column tile) outputs w, w + NW, ...   Lane holds D[m = mt*16 + 4g + j][n = unit*16 + r].
    if (NW == 1) {
#pragma unroll
        for (int rr = 0; rr < R; ++rr)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) gemv_epilogue<RG>(a, u0 + rr, mt, acc[rr * RG][mt], acc[rr * RG + RG - 1][mt]);
        return;
    }
    f32x4 *red = (f32x4 *)smem_raw;   // [NW][NR*MT][64]
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[(wv * NR * MT + i * MT + mt) * 64 + lane] = acc[i][mt];
    __syncthreads();
    for (int o = wv; o < R * MT; o += NW) {
        const int rr = o / MT, mt = o - rr * MT;
        f32x4 v[RG];
#pragma unroll
        for (int h = 0; h < RG; ++h) {
            const int idx = (rr * RG + h) * MT + mt;
            f32x4 t = red[idx * 64 + lane];
            for (int w2 = 1; w2 < NW; ++w2) t += red[(w2 * NR * MT + idx) * 64 + lane];
            v[h] = t;
        }
        gemv_epilogue<RG>(a, u0 + rr, mt, v[0], v[RG - 1]);
    }
}
