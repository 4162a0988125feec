// Block-dequant GEMV / small GEMM on MFMA: y[m][n] = sum_k x[m][k] * W[n][k] for m < M columns (M <= 64).
//
// Replaces F.linear in Qwen2Engine.forward (seedplane/qwen_engine.py:121,136,138-139,143) and the Vulkan gemv.comp /
// swiglu.comp / gemm_b.comp kernels (native/vulkan_decode/shaders/gemv.comp:1-51, swiglu.comp:1-44).
//
// Work decomposition
//   unit   = 16 output rows (32 for the SwiGLU epilogue: the packer interleaves the 16 gate rows i..i+15 with the 16
//            up rows of the same i, so one wave holds gate and up of the same output in the same lanes);
//   grid   = units x ksplit; a block of NW waves covers one unit over k-tiles [kt0, kt1), wave w taking
//            kt0 + w, kt0 + w + NW, ...  Waves are reduced through LDS in a fixed order; split-K partials are
//            reduced by the last-arriving block of a unit (arrival counter), also in fixed split order, so results
//            are bit-identical from run to run.
// Per k-tile and wave: one 1 KiB dwordx4 load of codes (fully coalesced), the per-row scales, the activation
// fragments (A operand, fp16, from the L2-resident activation buffer), exact code->fp16 unpack and one
// 16x16x32 MFMA per quant block (K = 32 = one block): block scales are applied to the fp32 MFMA result, so the
// codes enter the matrix cores exactly and only the activations are rounded (to fp16).
#pragma once
#include "sp_device.h"

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2 };

struct GemvArgs {
    const uint8_t *w;      // packed tiles
    const f16 *sz;         // per-tile scales (Q8) / scale+zero pairs (Q4); unused for F16
    int nkt;               // k-tiles per row group
    int units;             // grid.x
    int n_real;            // real output rows (EPI_SILU: intermediate size)
    const f16 *x;          // activations [m][ldx] fp16
    int ldx;
    int m;                 // columns (<= 16 * MT)
    float *out_f32;        // EPI_STORE / EPI_RESID output [m][ldo]
    f16 *out_f16;          // EPI_SILU output [m][ldo]
    int ldo;
    const float *bias;     // EPI_STORE optional bias [n]
    float *partial;        // split-K partials [ksplit][units][RG*MT][64] float4
    uint32_t *counters;    // [units], zero between launches
    int ksplit;
    int epi;
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

template <int FMT, int MT, int RG>
__global__ void __launch_bounds__(512) k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    constexpr int KT = TileGeom<FMT>::KT, ST = TileGeom<FMT>::STEPS;
    const int NW = blockDim.x >> 6;
    const int unit = blockIdx.x, split = blockIdx.y;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int kt0 = (int)((long)split * a.nkt / a.ksplit), kt1 = (int)((long)(split + 1) * a.nkt / a.ksplit);

    f32x4 acc[RG][MT];
#pragma unroll
    for (int i = 0; i < RG; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[i][mt] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const f16x8 zero8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};

    for (int kt = kt0 + wv; kt < kt1; kt += NW) {
        // ---- loads: codes (1 KiB per row group), per-step scale (and zero), activation fragments
        u32x4 wt[RG];
        float scale[RG][ST], zero[RG][ST];
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const size_t tile = (size_t)(unit * RG + rg) * a.nkt + kt;
            wt[rg] = __builtin_nontemporal_load((const u32x4 *)(a.w + tile * TILE_BYTES) + lane);
            if constexpr (FMT == 2) {
                const uint32_t d = *((const uint32_t *)(a.sz + tile * 32) + r);
                scale[rg][0] = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                scale[rg][1] = (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
            }
            if constexpr (FMT == 3) {
                const uint32_t *p = (const uint32_t *)(a.sz + tile * 128) + 4 * r;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const uint32_t d = p[s];
                    scale[rg][s] = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                    zero[rg][s] = (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
                }
            }
        }
        f16x8 xa[MT][ST];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + r;
#pragma unroll
            for (int s = 0; s < ST; ++s)
                xa[mt][s] = m < a.m ? *(const f16x8 *)(a.x + (size_t)m * a.ldx + kt * KT + s * 32 + 8 * g) : zero8;
        }
        // ---- MFMA per quant block
#pragma unroll
        for (int s = 0; s < ST; ++s) {
            f32x4 xs[MT];
            if constexpr (FMT == 3) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) xs[mt] = mfma16(xa[mt][s], ones8, (f32x4){0.f, 0.f, 0.f, 0.f});
            }
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                const f16x8 b = unpack_step<FMT>(wt[rg], s);
                if constexpr (FMT == 1) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[rg][mt] = mfma16(xa[mt][s], b, acc[rg][mt]);
                } else if constexpr (FMT == 2) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const f32x4 d = mfma16(xa[mt][s], b, (f32x4){0.f, 0.f, 0.f, 0.f});
                        acc[rg][mt] += scale[rg][s] * d;
                    }
                } else {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const f32x4 d = mfma16(xa[mt][s], b, (f32x4){0.f, 0.f, 0.f, 0.f});
                        acc[rg][mt] += scale[rg][s] * (d - zero[rg][s] * xs[mt]);
                    }
                }
            }
        }
    }

    // ---- reduce the NW waves (fixed order)
    f32x4 *red = (f32x4 *)smem_raw;   // [NW][RG*MT][64]
    if (NW > 1) {
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) red[(wv * RG * MT + rg * MT + mt) * 64 + lane] = acc[rg][mt];
        __syncthreads();
        if (wv != 0) return;
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 t = red[(rg * MT + mt) * 64 + lane];
                for (int w2 = 1; w2 < NW; ++w2) t += red[(w2 * RG * MT + rg * MT + mt) * 64 + lane];
                acc[rg][mt] = t;
            }
    }

    // ---- split-K: publish the partial; the last block of this unit sums all partials in split order
    if (a.ksplit > 1) {
        f32x4 *part = (f32x4 *)a.partial;
        const size_t stride = (size_t)RG * MT * 64;
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) part[((size_t)split * a.units + unit) * stride + (rg * MT + mt) * 64 + lane] = acc[rg][mt];
        __threadfence();
        uint32_t prev = 0;
        if (lane == 0) prev = atomicAdd(&a.counters[unit], 1u);
        prev = __shfl(prev, 0, SP_WAVE);
        if (prev != (uint32_t)(a.ksplit - 1)) return;
        __threadfence();
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 t = (f32x4){0.f, 0.f, 0.f, 0.f};
                for (int s2 = 0; s2 < a.ksplit; ++s2)
                    t += __builtin_nontemporal_load(&part[((size_t)s2 * a.units + unit) * stride + (rg * MT + mt) * 64 + lane]);
                acc[rg][mt] = t;
            }
        if (lane == 0) a.counters[unit] = 0u;
    }

    // ---- epilogue: lane holds D[m = mt*16 + 4g + j][n = unit*16 + r]
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = mt * 16 + 4 * g + j;
            const int n = unit * 16 + r;
            if (m >= a.m || n >= a.n_real) continue;
            if (a.epi == EPI_STORE) {
                float v = acc[0][mt][j];
                if (a.bias) v += a.bias[n];
                a.out_f32[(size_t)m * a.ldo + n] = v;
            } else if (a.epi == EPI_RESID) {
                a.out_f32[(size_t)m * a.ldo + n] += acc[0][mt][j];
            } else if constexpr (RG == 2) {
                const float gt = acc[0][mt][j], up = acc[RG - 1][mt][j];
                a.out_f16[(size_t)m * a.ldo + n] = (f16)(silu_f(gt) * up);
            }
        }
}
