// Block-dequant GEMV / small GEMM on MFMA: y[m][n] = sum_k x[m][k] * W[n][k] for m < M columns (M <= 64).
//
// Replaces F.linear in Qwen2Engine.forward (seedplane/qwen_engine.py:121,136,138-139,143) and the Vulkan gemv.comp /
// swiglu.comp / gemm_b.comp kernels (native/vulkan_decode/shaders/gemv.comp:1-51, swiglu.comp:1-44).
//
// Work decomposition
//   unit   = 16 output rows (32 for the SwiGLU epilogue: the packer interleaves the 16 gate rows i..i+15 with the 16
//            up rows of the same i, so one wave holds gate and up of the same output in the same lanes);
//   grid   = units; a block of NW waves (4..16) covers one unit over all of K, wave w taking k-tiles w, w + NW,
//            ... in batches of TB whose loads are all issued before any is consumed.  Waves are reduced through LDS
//            in a fixed order, so results are bit-identical from run to run.  There is no cross-block reduction:
//            no atomics and no device-scope fences (on gfx950 each agent-scope fence writes back / invalidates the
//            XCD's whole L2, which costs microseconds).
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

// Threads per block: single-column-tile variants use up to 16 waves (128 VGPRs each); wider variants up to 8 waves
// (256 VGPRs) so the activation fragments of several column tiles stay in registers without spilling.
template <int MT> struct GemvLimits { static constexpr int MAX_THREADS = MT == 1 ? 1024 : 512; };

template <int FMT, int MT, int RG>
__global__ void __launch_bounds__(GemvLimits<MT>::MAX_THREADS) k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    constexpr int KT = TileGeom<FMT>::KT, ST = TileGeom<FMT>::STEPS;
    // k-tiles whose loads are in flight together per wave, sized to the register budget
    constexpr int TB = FMT == 3 ? 2 : 4;
    const int NW = blockDim.x >> 6;
    const int unit = blockIdx.x;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;

    f32x4 acc[RG][MT];
#pragma unroll
    for (int i = 0; i < RG; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[i][mt] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const f16x8 zero8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};
    const uint8_t *wbase[RG];
    const f16 *sbase[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        wbase[rg] = a.w + (size_t)(unit * RG + rg) * a.nkt * TILE_BYTES;
        sbase[rg] = a.sz + (size_t)(unit * RG + rg) * a.nkt * (FMT == 2 ? 32 : 128);
    }

    for (int kb = wv; kb < a.nkt; kb += NW * TB) {
        // ---- issue the weight loads of TB tiles (HBM latency) before anything is consumed; with one column tile
        // the activation fragments are issued with them, wider variants fetch theirs (L2 hits) per tile below
        u32x4 wt[TB][RG];
        uint32_t sq8[TB][RG];
        u32x4 sq4[TB][RG];
        constexpr int XB = MT == 1 ? TB : 1;       // tiles whose activation fragments are held at once
        f16x8 xa[XB][MT][ST];
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int kt = kb + t * NW;
            if (kt >= a.nkt) break;
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                wt[t][rg] = __builtin_nontemporal_load((const u32x4 *)(wbase[rg] + (size_t)kt * TILE_BYTES) + lane);
                if constexpr (FMT == 2) sq8[t][rg] = *((const uint32_t *)(sbase[rg] + (size_t)kt * 32) + r);
                if constexpr (FMT == 3) sq4[t][rg] = *((const u32x4 *)(sbase[rg] + (size_t)kt * 128) + r);
            }
            if constexpr (MT == 1) {
#pragma unroll
                for (int s = 0; s < ST; ++s)
                    xa[t][0][s] = r < a.m ? *(const f16x8 *)(a.x + (size_t)r * a.ldx + kt * KT + s * 32 + 8 * g) : zero8;
            }
        }
        // ---- MFMA per quant block
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int kt = kb + t * NW;
            if (kt >= a.nkt) break;
            const int xt = MT == 1 ? t : 0;
            if constexpr (MT > 1) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int m = mt * 16 + r;
#pragma unroll
                    for (int s = 0; s < ST; ++s)
                        xa[0][mt][s] = m < a.m ? *(const f16x8 *)(a.x + (size_t)m * a.ldx + kt * KT + s * 32 + 8 * g) : zero8;
                }
            }
#pragma unroll
            for (int s = 0; s < ST; ++s) {
                f32x4 xs[MT];
                if constexpr (FMT == 3) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) xs[mt] = mfma16(xa[xt][mt][s], ones8, (f32x4){0.f, 0.f, 0.f, 0.f});
                }
#pragma unroll
                for (int rg = 0; rg < RG; ++rg) {
                    const f16x8 b = unpack_step<FMT>(wt[t][rg], s);
                    if constexpr (FMT == 1) {
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) acc[rg][mt] = mfma16(xa[xt][mt][s], b, acc[rg][mt]);
                    } else if constexpr (FMT == 2) {
                        const uint32_t d = sq8[t][rg];
                        const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(s == 0 ? (d & 0xffffu) : (d >> 16)));
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            acc[rg][mt] += scale * mfma16(xa[xt][mt][s], b, (f32x4){0.f, 0.f, 0.f, 0.f});
                    } else {
                        uint32_t d;
                        if (s == 0) d = sq4[t][rg].x; else if (s == 1) d = sq4[t][rg].y; else if (s == 2) d = sq4[t][rg].z; else d = sq4[t][rg].w;
                        const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                        const float zero = (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            const f32x4 dd = mfma16(xa[xt][mt][s], b, (f32x4){0.f, 0.f, 0.f, 0.f});
                            acc[rg][mt] += scale * (dd - zero * xs[mt]);
                        }
                    }
                }
            }
        }
    }

    // ---- reduce the NW waves through LDS (fixed order -> deterministic)
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

    // ---- epilogue: lane holds D[m = mt*16 + 4g + j][n = unit*16 + r]
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = mt * 16 + 4 * g + j;
            const int n = unit * 16 + r;
            if (m >= a.m || n >= a.n_real) continue;
            if constexpr (RG == 2) {
                const float gt = acc[0][mt][j], up = acc[RG - 1][mt][j];
                a.out_f16[(size_t)m * a.ldo + n] = (f16)(silu_f(gt) * up);
            } else {
                if (a.epi == EPI_STORE) {
                    float v = acc[0][mt][j];
                    if (a.bias) v += a.bias[n];
                    a.out_f32[(size_t)m * a.ldo + n] = v;
                } else {
                    a.out_f32[(size_t)m * a.ldo + n] += acc[0][mt][j];
                }
            }
        }
}
