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
#include "sp_attn.h"

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_PART = 3 };

// 16 zero bytes, never written: the activation load address of lanes whose column does not exist
static __device__ __align__(16) f16 g_zero_line[8];

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
    int nwk;               // prologue kernels: waves that take k-tiles (the others only help with the prologue)
    int xmtp;              // x layout: 0 row-major [m][ldx], else fragment-major with xmtp column tiles (act_off)
    int omtp;              // EPI_SILU output layout, the same way
    const f16 *xlo;        // optional: the fp16 remainders of x (split_f16), same layout; NULL = x is exact in fp16
    f16 *out_lo;           // optional EPI_SILU output: the fp16 remainders of the SwiGLU values
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
// The codes of step s offset by QBIAS<FMT> (exact fp16; Q8 and Q4 only).
template <int FMT> struct QBias { static constexpr float V = FMT == 2 ? 1152.f : 1024.f; };
template <int FMT>
__device__ __forceinline__ f16x8 biased_step(const u32x4 &t, int s) {
    if constexpr (FMT == 2) return s == 0 ? q8_biased8(t[0], t[1]) : q8_biased8(t[2], t[3]);
    else return q4_biased8(t[s]);
}

// Threads per block: single-column-tile variants with one unit per block use up to 16 waves (128 VGPRs each), those
// with two units up to 4, wider ones up to 8 (each wave may then hold up to 256 VGPRs: the weight tiles and
// activation fragments of a whole batch stay in registers).
// TB = k-tiles per wave whose loads are in flight together.  The SwiGLU pair at one column tile (2-16 columns) by
// format, from a sweep of batch depth x waves x units per wave at 8 and 16 columns: int8 2 (Qwen2-1.5B gate_up
// 10.3 -> 9.7 us at 16 columns; deeper batches hold more registers than the loads they overlap pay for), fp16 8
// with two units per wave (Qwen2-0.5B 6.75 -> 6.34 us), int4 2.  Several column tiles of int4 codes: 1 (the
// Qwen2-7B matrices at 32 columns, 71.4 -> 67.8 us per layer over qkv, o, gate_up and down).
template <int MT, int RG, int R> struct GemvLimits {
    static constexpr int MAX_THREADS = MT == 1 ? (R == 1 ? 1024 : 256) : 512;
};
// SHALLOW (several column tiles): one k-tile per batch.  Fewer registers (e.g. 132 -> 98 VGPRs for the int8 gate_up
// pair at 3 column tiles) and so more resident waves, which the int8 matrices with short per-wave k-ranges prefer.
template <int FMT, int MT, int RG, bool SHALLOW = false> struct GemvBatch {
    static constexpr int TB = MT == 1 ? (FMT == 3 ? 2 : (RG == 2 ? (FMT == 1 ? 8 : 2) : 4)) : (SHALLOW || FMT == 3 ? 1 : 2);
};

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
        for (int j = 0; j < 4; ++j) {
            f16 hi, lo;
            split_f16(silu_f(v0[j]) * v1[j], hi, lo);
            if (live[j]) a.out_f16[act_off(mrow[j], n, a.ldo, a.omtp)] = hi;
            if (live[j] && a.out_lo) a.out_lo[act_off(mrow[j], n, a.ldo, a.omtp)] = lo;
        }
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

// ---------------------------------------------------------------------------------------------------------------
// Activation prologues (one column).  The block builds the fp16 activations of its own k-range in LDS, so the kernel
// that would have produced them (the RMSNorm before qkv / gate_up, the attention combine before o_proj) does not run
// on its own; the block's first batch of weight loads is issued before the prologue and streams in meanwhile.  Both
// prologues repeat the arithmetic of the kernel they stand in for operation by operation (same element sums, same
// reduction trees), so a step gives bit-identical results with and without them.  Prologue kernels run pro_threads()
// threads (the norm prologue needs 8 waves for the qkv plan; the combine prologue is fastest with 4); the first
// a.nwk waves take the k-tiles, exactly as a plain launch with a.nwk waves would.
enum { PRO_NONE = 0, PRO_NORM = 1, PRO_COMB = 2 };
__host__ __device__ constexpr int pro_threads(int pro) { return pro == PRO_NORM ? 512 : 256; }
constexpr int PRO_NORM_HMAX = 2048;         // hidden sizes the norm prologue takes (PRO_NORM_HMAX / 512 per thread)
constexpr int PRO_MAX_SLICES = 8;           // pending residual slices
struct ProArgs {
    // PRO_NORM: v = res + part[0] + ... + part[np - 1] (slice order); act, act_lo = split_f16((v * rs) * w) with
    // rs = 1 / sqrt(mean(v^2) + eps) (k_rmsnorm); block (0, 0) writes v to res_out, a buffer the blocks do not read
    const float *res;
    float *res_out;
    const float *part;
    size_t pstride;
    int np;
    const float *w;
    float eps;
    int H;
    // PRO_COMB: act = the attention partials [NH][nchunk][part_floats(HD)] of column 0 merged as k_attn_combine merges them
    const float *apart;
    const int *colnc;
    int NH, HD, nchunk;
};
// LDS floats a prologue needs beyond the activations
__host__ __device__ inline int pro_scratch_floats(int pro, int H, int HD) {
    if (pro == PRO_NORM) return H + 16;
    if (pro == PRO_COMB) return (pro_threads(PRO_COMB) / HD) * (2 * ATT_MAX_CHUNKS + 16);
    return 0;
}

// The norm prologue's operands (the residual, every slice, the norm weights of this block's k-range), loaded from
// clamped addresses with no branch: a slice index past the pending ones re-reads the last pending slice (slice 0
// when none is pending), whose values the sum skips.
constexpr int PRO_NORM_QMAX = PRO_NORM_HMAX / pro_threads(PRO_NORM);
struct NormOps { float xv[PRO_NORM_QMAX], wk[PRO_NORM_QMAX], pv[PRO_MAX_SLICES][PRO_NORM_QMAX]; };
__device__ __forceinline__ void pro_norm_load(const ProArgs &p, int klo, NormOps &o) {
    constexpr int PRO_THREADS = pro_threads(PRO_NORM);
    const int tid = threadIdx.x, H = p.H;
#pragma unroll
    for (int q = 0; q < PRO_NORM_QMAX; ++q) {
        o.xv[q] = p.res[min(tid + PRO_THREADS * q, H - 1)];
        o.wk[q] = p.w[min(klo + tid + PRO_THREADS * q, H - 1)];
    }
#pragma unroll
    for (int s = 0; s < PRO_MAX_SLICES; ++s) {
        const size_t so = (size_t)min(s, max(p.np - 1, 0)) * p.pstride;
#pragma unroll
        for (int q = 0; q < PRO_NORM_QMAX; ++q) o.pv[s][q] = p.part[so + min(tid + PRO_THREADS * q, H - 1)];
    }
}
__device__ __forceinline__ void pro_norm_finish(const ProArgs &p, const NormOps &o, f16 *act, f16 *act_lo, int klo,
                                                int klen, float *scr) {
    constexpr int PRO_THREADS = pro_threads(PRO_NORM), PRO_QMAX = PRO_NORM_QMAX;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, H = p.H;
    float *v_s = scr, *red = scr + H;
    const float *xv = o.xv, *wk = o.wk;
    const auto &pv = o.pv;
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
    for (int q = 0; q < PRO_QMAX; ++q) {
        const int k = tid + PRO_THREADS * q;
        float v = xv[q];
#pragma unroll
        for (int s = 0; s < PRO_MAX_SLICES; ++s)
            if (s < p.np) v += pv[s][q];
        if (k < H) {
            v_s[k] = v;
            if (writer) p.res_out[k] = v;
        }
    }
    __syncthreads();
    // k_rmsnorm's reduction: virtual thread t < NORM_THREADS squares and sums elements t + NORM_THREADS * i (zeros
    // past H); real wave w plays virtual waves w, w + PRO_THREADS / 64, ...; the 16 DPP wave sums are then added in
    // order
#pragma unroll
    for (int j = 0; j < NORM_THREADS / PRO_THREADS; ++j) {
        const int vt = tid + PRO_THREADS * j;
        float ss = 0.f;
        {
#pragma clang fp contract(off)      // k_rmsnorm's rounding order: each square rounded, added in element order
#pragma unroll
            for (int i = 0; i < NORM_PER_THREAD; ++i) {
                const int k = vt + NORM_THREADS * i;
                const float v = k < H ? v_s[k] : 0.f;
                ss += v * v;
            }
        }
        ss = wave_sum_dpp(ss);
        if (lane == 0) red[wv + (PRO_THREADS / 64) * j] = ss;
    }
    __syncthreads();
    float tot = 0.f;
    for (int j = 0; j < NORM_THREADS / 64; ++j) tot += red[j];
    const float rs = 1.0f / sqrtf(tot / (float)H + p.eps);
#pragma unroll
    for (int q = 0; q < PRO_QMAX; ++q) {
        const int e = tid + PRO_THREADS * q;
        if (e < klen) {
            f16 hi, lo;
            split_f16((v_s[klo + e] * rs) * wk[q], hi, lo);
            act[e] = hi;
            act_lo[e] = lo;
        }
    }
    __syncthreads();
}
__device__ __forceinline__ void pro_norm(const ProArgs &p, f16 *act, f16 *act_lo, int klo, int klen, float *scr) {
    NormOps o;
    pro_norm_load(p, klo, o);
    pro_norm_finish(p, o, act, act_lo, klo, klen, scr);
}

// Heads overlapping the k-range, pro_threads(PRO_COMB) / HD at a time: thread group g of HD threads plays
// k_attn_combine's block for head h0 + g.
__device__ __forceinline__ void pro_comb(const ProArgs &p, f16 *act, int klo, int klen, float *scr) {
    constexpr int PRO_THREADS = pro_threads(PRO_COMB);
    const int HD = p.HD, tid = threadIdx.x, lane = tid & 63;
    const int ngrp = PRO_THREADS / HD, grp = tid / HD, gt = tid - grp * HD, gw = gt >> 6, gnw = HD / 64;
    float *w_s = scr + grp * 2 * ATT_MAX_CHUNKS, *l_s = w_s + ATT_MAX_CHUNKS;
    float *red = scr + ngrp * 2 * ATT_MAX_CHUNKS + grp * 16;
    const int h_lo = klo / HD, h_hi = (klo + klen - 1) / HD;
    const int nc = p.colnc[0], last = max(nc - 1, 0);
    for (int h0 = h_lo; h0 <= h_hi; h0 += ngrp) {
        const bool live = h0 + grp <= h_hi;
        const int h = min(h0 + grp, h_hi);
        const int rec = part_floats(HD);
        const float *pp = p.apart + (size_t)h * p.nchunk * rec;
        float v[CMB_BATCH];
#pragma unroll
        for (int i = 0; i < CMB_BATCH; ++i) v[i] = (float)((const f16 *)(pp + (size_t)min(i, last) * rec + 2))[gt];
        float mloc = -INFINITY;
        for (int c = gt; c < nc; c += HD) {
            const float mc = pp[(size_t)c * rec], lc = pp[(size_t)c * rec + 1];
            w_s[c] = lc > 0.f ? mc : -INFINITY;
            l_s[c] = lc;
            mloc = fmaxf(mloc, w_s[c]);
        }
        mloc = wave_max_dpp(mloc);
        if (lane == 0) red[gw] = mloc;
        __syncthreads();
        float M = red[0];
        for (int i = 1; i < gnw; ++i) M = fmaxf(M, red[i]);
        float lsum = 0.f;
        for (int c = gt; c < nc; c += HD) {
            const float wc = w_s[c] == -INFINITY ? 0.f : expf(w_s[c] - M) * l_s[c];
            w_s[c] = wc;
            lsum += wc;
        }
        __syncthreads();
        lsum = wave_sum_dpp(lsum);
        __syncthreads();
        if (lane == 0) red[8 + gw] = lsum;
        __syncthreads();
        float L = 0.f;
        for (int j = 0; j < gnw; ++j) L += red[8 + j];
        float acc = 0.f;
        for (int c0 = 0; c0 < nc; c0 += CMB_BATCH) {
            if (c0 > 0) {
#pragma unroll
                for (int i = 0; i < CMB_BATCH; ++i) v[i] = (float)((const f16 *)(pp + (size_t)min(c0 + i, last) * rec + 2))[gt];
            }
#pragma unroll
            for (int i = 0; i < CMB_BATCH; ++i)
                if (c0 + i < nc) acc += w_s[c0 + i] * v[i];
        }
        const int k = h * HD + gt;
        if (live && k >= klo && k < klo + klen) act[k - klo] = (f16)(acc / L);
        __syncthreads();                               // w_s / red are reused by the next heads
    }
}

// MT == 1 (up to 16 columns) with Q8 / Q4 codes: the MFMA takes the codes offset by QBias (no per-weight subtraction)
// and each quant block's result is corrected by QBias (+ the Q4 zero) times the block's activation sums, one fp32 FMA
// per output; ONE (a single column) keeps only output components 0 and 1: row 0 of the MFMA A operand is the column,
// row 1 its fp16 remainders (a.xlo, or the norm prologue's; a zero line without them), rows 2..15 zero, so the
// remainders cost no extra MFMA.  LO (several columns): a second MFMA per fragment takes the remainders a.xlo.
// Every column gets the same operations in either case, so one column and a batch give the same bits.
template <int FMT, int MT, int RG, int R, int PRO, bool ONE = false, bool SHALLOW = false, bool LO = false>
__device__ __forceinline__ void gemv_run(const GemvArgs &a, const ProArgs &p, unsigned char *smem_raw) {
    constexpr int KT = TileGeom<FMT>::KT, ST = TileGeom<FMT>::STEPS;
    constexpr int TB = PRO == PRO_NONE ? GemvBatch<FMT, MT, RG, SHALLOW>::TB : GemvBatch<FMT, MT, 1>::TB;
    constexpr int NR = R * RG;                 // row groups per wave
    const int NW = PRO == PRO_NONE ? (int)(blockDim.x >> 6) : a.nwk;   // waves taking k-tiles
    // the wave index as a wave-uniform value: the per-wave k-tile bounds below become scalar branches
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool worker = PRO == PRO_NONE || wv < NW;
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
    size_t xrow[MT];          // row-major offset of the lane's column (column 0 for lanes past m)
    bool xon[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        xon[mt] = m < a.m;
        xrow[mt] = (size_t)(xon[mt] ? m : 0) * a.ldx + 8 * g;
    }
    // ONE: the lanes of MFMA row 1 hold column 0's remainders (row-major input)
    const bool lrow = ONE && r == 1 && a.xlo != nullptr && a.xmtp == 0;
    // LDS: [cross-wave reduction: NW x NR x MT x 1 KiB][prologue: activations of the k-range, scratch]
    f32x4 *red = (f32x4 *)smem_raw;
    f16 *act = (f16 *)(smem_raw + (size_t)NW * NR * MT * 1024);
    const int klen = (k1 - k0) * KT;

    u32x4 wt[TB][NR];
    uint32_t sq8[TB][NR];
    u32x4 sq4[TB][NR];
    auto load_weights = [&](int kb) {
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
        }
    };
    f16 *act_lo = act + ((klen + 7) & ~7);      // the norm prologue's remainders
    if constexpr (PRO != PRO_NONE) {
        if (worker && k0 + wv < k1) load_weights(k0 + wv);
        float *scr = (float *)(act_lo + ((klen + 7) & ~7));
        if constexpr (PRO == PRO_NORM) pro_norm(p, act, act_lo, k0 * KT, klen, scr);
        else pro_comb(p, act, k0 * KT, klen, scr);
    }

    if (worker) {
    for (int kb = k0 + wv; kb < k1; kb += NW * TB) {
        // ---- issue the weight and activation loads of TB k-tiles before anything is consumed
        if (PRO == PRO_NONE || kb != k0 + wv) load_weights(kb);
        f16x8 xa[TB][MT][ST];
        f16x8 xal[LO ? TB : 1][MT][ST];
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int kt = kb + t * NW;
            if (kt >= k1) break;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int s = 0; s < ST; ++s) {
                    if constexpr (PRO == PRO_NONE) {
                        // lanes of columns past m load the zero line (one L1-resident line: a partly used column
                        // tile, e.g. column 32 of 33, reads only its live columns from L2), the others their
                        // fragment (fragment-major, xmtp == MT) or row slice (row-major).  One unconditional load
                        // from a selected address: no branch and no select on the value, so the loads of a batch
                        // stay in flight together.
                        const size_t off = a.xmtp ? ((size_t)(kt * ST + s) * MT + mt) * 512 + lane * 8
                                                  : xrow[mt] + kt * KT + s * 32;
                        const f16 *src = xon[mt] ? a.x + off : (mt == 0 && lrow ? a.xlo + off : g_zero_line);
                        xa[t][mt][s] = *(const f16x8 *)src;
                        if constexpr (LO) xal[t][mt][s] = *(const f16x8 *)(xon[mt] ? a.xlo + off : g_zero_line);
                    } else {
                        const int e = (kt - k0) * KT + s * 32 + 8 * g;
                        xa[t][mt][s] = xon[mt] ? *(const f16x8 *)(act + e)
                                               : (PRO == PRO_NORM && mt == 0 && r == 1 ? *(const f16x8 *)(act_lo + e) : zero8);
                    }
                }
        }
        // ---- MFMA per quant block
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const int kt = kb + t * NW;
            if (kt >= k1) break;
#pragma unroll
            for (int s = 0; s < ST; ++s) {
                f32x4 xs[MT];
                if constexpr (FMT == 3 || (FMT == 2 && MT == 1)) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        xs[mt] = mfma16(xa[t][mt][s], ones8, (f32x4){0.f, 0.f, 0.f, 0.f});
                        if constexpr (LO) xs[mt] = mfma16(xal[t][mt][s], ones8, xs[mt]);
                    }
                }
                if constexpr (FMT != 1 && MT == 1) {
                    // biased codes: acc_j += scale * (mfma(x, code + bias)_j - (bias + zero) * sum(x)_j)
                    constexpr int NJ = ONE ? 1 : 4;
                    // the products of every row group first, then their corrections: no FMA waits on the MFMA it
                    // follows
                    f32x4 ddv[NR];
#pragma unroll
                    for (int i = 0; i < NR; ++i) {
                        const f16x8 bq = biased_step<FMT>(wt[t][i], s);
                        ddv[i] = mfma16(xa[t][0][s], bq, (f32x4){0.f, 0.f, 0.f, 0.f});
                        if constexpr (LO) ddv[i] = mfma16(xal[t][0][s], bq, ddv[i]);
                    }
#pragma unroll
                    for (int i = 0; i < NR; ++i) {
                        const f32x4 dd = ddv[i];
                        float scale, off;
                        if constexpr (FMT == 2) {
                            const uint32_t d = sq8[t][i];
                            scale = (float)__builtin_bit_cast(f16, (uint16_t)(s == 0 ? (d & 0xffffu) : (d >> 16)));
                            off = QBias<FMT>::V;
                        } else {
                            uint32_t d;
                            if (s == 0) d = sq4[t][i].x; else if (s == 1) d = sq4[t][i].y; else if (s == 2) d = sq4[t][i].z; else d = sq4[t][i].w;
                            scale = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                            off = QBias<FMT>::V + (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
                        }
                        if constexpr (ONE) {     // column 0 = row 0 (fp16 part) + row 1 (remainders)
                            acc[i][0][0] = fmaf(scale, fmaf(-off, xs[0][0], dd[0]) + fmaf(-off, xs[0][1], dd[1]), acc[i][0][0]);
                        } else {
#pragma unroll
                            for (int j = 0; j < NJ; ++j) acc[i][0][j] = fmaf(scale, fmaf(-off, xs[0][j], dd[j]), acc[i][0][j]);
                        }
                    }
                    continue;
                }
#pragma unroll
                for (int i = 0; i < NR; ++i) {
                    const f16x8 b = unpack_step<FMT>(wt[t][i], s);
                    if constexpr (FMT == 1) {
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            acc[i][mt] = mfma16(xa[t][mt][s], b, acc[i][mt]);
                            if constexpr (LO) acc[i][mt] = mfma16(xal[t][mt][s], b, acc[i][mt]);
                        }
                    } else if constexpr (FMT == 2) {
                        const uint32_t d = sq8[t][i];
                        const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(s == 0 ? (d & 0xffffu) : (d >> 16)));
                        f32x4 dd[MT];                  // every column tile's product first, then the scaling
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            dd[mt] = mfma16(xa[t][mt][s], b, (f32x4){0.f, 0.f, 0.f, 0.f});
                            if constexpr (LO) dd[mt] = mfma16(xal[t][mt][s], b, dd[mt]);
                        }
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) acc[i][mt] += scale * dd[mt];
                    } else {
                        uint32_t d;
                        if (s == 0) d = sq4[t][i].x; else if (s == 1) d = sq4[t][i].y; else if (s == 2) d = sq4[t][i].z; else d = sq4[t][i].w;
                        const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                        const float zero = (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
                        f32x4 dd[MT];
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            dd[mt] = mfma16(xa[t][mt][s], b, (f32x4){0.f, 0.f, 0.f, 0.f});
                            if constexpr (LO) dd[mt] = mfma16(xal[t][mt][s], b, dd[mt]);
                        }
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) acc[i][mt] += scale * (dd[mt] - zero * xs[mt]);
                    }
                }
            }
        }
    }
    }

    // ONE with fp16 weights: rows 0 and 1 accumulated the column's two parts separately
    if constexpr (ONE && FMT == 1) {
#pragma unroll
        for (int i = 0; i < NR; ++i) acc[i][0][0] += acc[i][0][1];
    }
    // ---- one wave: finish in registers; several: reduce through LDS in wave order, wave w finishing the (unit,
    // column tile) outputs w, w + NW, ...   Lane holds D[m = mt*16 + 4g + j][n = unit*16 + r].
    if (NW == 1) {
        if (wv != 0) return;
#pragma unroll
        for (int rr = 0; rr < R; ++rr)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) gemv_epilogue<RG>(a, u0 + rr, mt, acc[rr * RG][mt], acc[rr * RG + RG - 1][mt]);
        return;
    }
    if (worker) {
#pragma unroll
        for (int i = 0; i < NR; ++i)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) red[(wv * NR * MT + i * MT + mt) * 64 + lane] = acc[i][mt];
    }
    __syncthreads();
    if (!worker) return;
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

template <int FMT, int MT, int RG, int R, bool ONE = false, bool SHALLOW = false, bool LO = false>
__global__ void __launch_bounds__((GemvLimits<MT, RG, R>::MAX_THREADS)) k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    gemv_run<FMT, MT, RG, R, PRO_NONE, ONE, SHALLOW, LO>(a, ProArgs{}, smem_raw);
}

// One column with an activation prologue (PRO_NORM before qkv / gate_up, PRO_COMB before o_proj).
template <int FMT, int RG, int PRO>
__global__ void __launch_bounds__(pro_threads(PRO)) k_gemv_pro(GemvArgs a, ProArgs p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    gemv_run<FMT, 1, RG, 1, PRO, true>(a, p, smem_raw);
}
