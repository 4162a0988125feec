// libseedplane_hip: C ABI (include/seedplane_hip.h) over the gfx950 decode / verify kernels.
//
// The engine owns every device buffer: packed weights, the fp16 KV ring of every layer, the activation buffers
// for up to max_tokens columns, split-K / attention / argmax scratch.  One forward call = one stream-ordered
// sequence of kernels (optionally captured once into a hipGraph per (columns, flags) and replayed).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <algorithm>
#include <atomic>
#include <cstring>
#include <functional>
#include <map>
#include <set>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <string>
#include <utility>
#include <vector>

#include "../../include/seedplane_hip.h"
#include "sp_attn.h"
#include "sp_decode1.h"
#include "sp_gemv.h"
#include "sp_gemv1.h"
#include "sp_pack.h"
#include "sp_sample.h"

namespace {

thread_local std::string g_err;

struct Fail {
    int code;
    std::string msg;
};

#define HIPCHK(expr)                                                                                     \
    do {                                                                                                 \
        hipError_t _e = (expr);                                                                          \
        if (_e != hipSuccess)                                                                            \
            throw Fail{SP_EHIP, std::string(#expr) + ": " + hipGetErrorString(_e)};                      \
    } while (0)

inline void require(bool ok, int code, const std::string &msg) {
    if (!ok) throw Fail{code, msg};
}
// A literal message builds its string only on failure (per-column checks run on every call).
inline void require(bool ok, int code, const char *msg) {
    if (!ok) throw Fail{code, msg};
}

template <class T>
T *dev_alloc(size_t count, uint64_t *acct = nullptr) {
    void *p = nullptr;
    if (count == 0) count = 1;
    hipError_t e = hipMalloc(&p, count * sizeof(T));
    if (e != hipSuccess) throw Fail{SP_ENOMEM, "hipMalloc of " + std::to_string(count * sizeof(T)) + " bytes failed: " + hipGetErrorString(e)};
    if (acct) *acct += count * sizeof(T);
    return (T *)p;
}
inline void dev_free(void *p) {
    if (p) (void)hipFree(p);
}

// ------------------------------------------------------------------------------------------- packed matrix on HBM
struct DevMat {
    int fmt = 0, rows = 0, cols = 0, rows_pad = 0, nkt = 0;
    bool paired = false;
    uint8_t *w = nullptr;
    f16 *sz = nullptr;
    uint64_t bytes = 0;
    void release() { dev_free(w); dev_free(sz); w = nullptr; sz = nullptr; bytes = 0; }
};

DevMat upload_matrix(int fmt, int rows, int cols, const void *data, const void *scales, const void *zeros, bool paired) {
    sp::Packed p;
    try {
        p = sp::pack_matrix(fmt, rows, cols, data, scales, zeros, paired);
    } catch (const std::invalid_argument &ex) {
        throw Fail{SP_EINVAL, ex.what()};
    }
    DevMat m;
    m.fmt = fmt; m.rows = rows; m.cols = cols; m.rows_pad = p.rows_pad; m.nkt = p.nkt; m.paired = paired;
    m.w = dev_alloc<uint8_t>(p.codes.size());
    HIPCHK(hipMemcpy(m.w, p.codes.data(), p.codes.size(), hipMemcpyHostToDevice));
    m.bytes = p.codes.size();
    if (!p.sz.empty()) {
        m.sz = dev_alloc<f16>(p.sz.size());
        HIPCHK(hipMemcpy(m.sz, p.sz.data(), p.sz.size() * 2, hipMemcpyHostToDevice));
        m.bytes += p.sz.size() * 2;
    }
    return m;
}

// ------------------------------------------------------------------------------------------- GEMV planning/launch
constexpr int GEMV_MAX_MT = 4;
constexpr int GEMV_MAX_SLICES = 8;
constexpr int GEMV_MAX_LDS = 64 * 1024;

struct GemvPlan {
    int units, nw, rg, r, s, kslice;
    bool shallow;      // several column tiles: one k-tile per load batch (k_gemv<..., SHALLOW>)
};


// Launch shape of one GEMV, from launch-shape sweeps (row groups per wave x waves x slices) of the Qwen2-0.5B fp16,
// 1.5B int8 and 7B int4 matrices at 1, 16 and 32-33 columns.  Small-batch GEMVs are latency-bound: what counts is
// the number of waves with loads in flight and a grid that the chip (256 CUs) holds at once.  Matrices with few row
// groups (qkv, o, down) are split along K into slices that the consuming kernel adds up; the LM head and the wider
// column tiles give each wave two row groups (R = 2: twice the loads in flight per wave, half the activation reads
// per weight byte).
// `slices` / `waves` (> 0) replace the slice count and wave count of the heuristic (single-column steps, whose
// residual must reach the next norm in few slices).
GemvPlan plan_gemv(const DevMat &m, int mt, bool split_ok, int slices = 0, int waves = 0) {
    GemvPlan p;
    p.rg = m.paired ? 2 : 1;
    p.units = m.rows_pad / 16 / p.rg;
    // one column tile: two units per wave for the LM head and for the fp16 SwiGLU pair (whose 8-k-tile batches they
    // share; see GemvBatch)
    if (mt == 1) p.r = (p.units >= 2048 || (m.paired && m.fmt == 1)) && p.units % 2 == 0 ? 2 : 1;
    // the head at 2-3 column tiles: 4 units per wave (each activation fragment feeds 4 weight tiles); the int4 and
    // 4-tile variants would spill registers
    else if (!split_ok && !m.paired && p.units % 4 == 0 && mt <= 3 && m.fmt != 3) p.r = 4;
    else p.r = p.units % 2 == 0 && !m.paired ? 2 : 1;
    int s = 1;
    if (split_ok && !m.paired) {
        s = std::max(1, 2048 / (p.units / p.r));
        s = std::min(s, std::max(1, m.nkt / 2));
        // several int4 column tiles: up to 8 slices of 4 waves (7B shape at 32 columns: qkv 10.7 -> 7.4 us, o 7.7 ->
        // 6.9, down 21.3 -> 19.8 against 4 slices of 8 waves)
        s = std::min(s, mt == 1 || m.fmt == 3 ? GEMV_MAX_SLICES : 4);
        if (slices > 0) s = std::min(slices, std::max(1, m.nkt / 2));
    }
    p.s = s;
    p.kslice = (m.nkt + s - 1) / s;
    // several column tiles: 8 waves for the split layer matrices and long k-ranges, 4 for the gate_up pair and the
    // unsplit head (A/B runs of the whole tree-verify step at 33 columns: gate_up with 4 waves -100 us per pass)
    // One column tile of a split matrix whose slices hold >= 16 k-tiles (the down projection at 2-16 columns): 8
    // waves as well (sweep of single launches, 8 and 16 columns: 1.5B int8 down 6.04 -> 5.60 and 6.59 -> 6.10 us,
    // 0.5B fp16 down 4.42 -> 4.20 and 4.65 -> 4.42; int4 not swept, so it keeps 4).
    // The int4 SwiGLU pair at several column tiles: 8 waves (7B at 32 columns, one k-tile per batch: 34.3 -> 32.2 us).
    const bool wide = mt > 1 ? (m.fmt != 3 && (p.kslice >= 32 || s > 1)) || (m.fmt == 3 && m.paired)
                             : m.fmt != 3 && s > 1 && p.kslice >= 16;
    int nw = std::min(p.kslice, wide ? 8 : 4);
    if (waves > 0) nw = std::min(p.kslice, std::min(waves, mt == 1 ? 16 : 8));
    // int8 codes at 3 column tiles (33-48 columns, a tree pass): one k-tile per batch (98 instead of 132 VGPRs for
    // the gate_up pair, so more resident waves) unless a split matrix gives each wave a long k-range (the down
    // projection); the LM head then runs 2 waves of 4 units.  Launch sweeps at 33 columns: gate_up 13.2 -> 12.5 us,
    // head 69.7 -> 59.4, qkv and o -0.15, down 7.8 -> 8.6 (so it keeps 2 k-tiles); at 2 and 4 column tiles and
    // with int4 codes shallow batches are slower (head at 32 columns 58 -> 64 us, int4 matrices 10-35 %).
    p.shallow = mt == 3 && m.fmt == 2 && !(s > 1 && p.kslice >= 32);
    if (p.shallow && p.r == 4 && waves == 0) nw = std::min(nw, 2);
    if (mt == 1 && p.r > 1) nw = std::min(nw, 4);
    while (nw > 1 && (size_t)nw * p.r * p.rg * mt * 1024 > GEMV_MAX_LDS) --nw;
    p.nw = std::max(1, nw);
    return p;
}

// LO: several columns whose inputs come with fp16 remainders (a.xlo): a second MFMA per fragment.  One column takes
// its remainders in MFMA row 1 of the ONE variant instead.
template <int FMT, int RG, int R, bool LO>
void launch_gemv_r_lo(int mt, bool shallow, dim3 grid, dim3 block, size_t smem, hipStream_t st, const GemvArgs &a) {
    if (mt == 1) {
        if constexpr (R == 4) {
            throw Fail{SP_EINVAL, "gemv plan: 4 units per wave need several column tiles"};
        } else {
            if (a.m == 1) hipLaunchKernelGGL((k_gemv<FMT, 1, RG, R, true>), grid, block, smem, st, a);
            else hipLaunchKernelGGL((k_gemv<FMT, 1, RG, R, false, false, LO>), grid, block, smem, st, a);
        }
        return;
    }
    if constexpr (FMT == 2) {
        if (shallow) {
            require(mt == 3, SP_EINVAL, "gemv plan: shallow batches are built for 3 column tiles");
            hipLaunchKernelGGL((k_gemv<FMT, 3, RG, R, false, true, LO>), grid, block, smem, st, a);
            return;
        }
    }
    switch (mt) {
        case 2: hipLaunchKernelGGL((k_gemv<FMT, 2, RG, R, false, false, LO>), grid, block, smem, st, a); break;
        case 3: hipLaunchKernelGGL((k_gemv<FMT, 3, RG, R, false, false, LO>), grid, block, smem, st, a); break;
        default: hipLaunchKernelGGL((k_gemv<FMT, 4, RG, R, false, false, LO>), grid, block, smem, st, a); break;
    }
}
template <int FMT, int RG, int R>
void launch_gemv_r(int mt, bool shallow, dim3 grid, dim3 block, size_t smem, hipStream_t st, const GemvArgs &a) {
    if (a.xlo && a.m > 1) launch_gemv_r_lo<FMT, RG, R, true>(mt, shallow, grid, block, smem, st, a);
    else launch_gemv_r_lo<FMT, RG, R, false>(mt, shallow, grid, block, smem, st, a);
}
template <int FMT>
void launch_gemv_fmt(int mt, bool paired, int r, bool shallow, dim3 grid, dim3 block, size_t smem, hipStream_t st,
                     const GemvArgs &a) {
    if (paired) {
        if (r == 2) launch_gemv_r<FMT, 2, 2>(mt, shallow, grid, block, smem, st, a);
        else launch_gemv_r<FMT, 2, 1>(mt, shallow, grid, block, smem, st, a);
    } else if (r == 4) {
        launch_gemv_r<FMT, 1, 4>(mt, shallow, grid, block, smem, st, a);
    } else {
        if (r == 2) launch_gemv_r<FMT, 1, 2>(mt, shallow, grid, block, smem, st, a);
        else launch_gemv_r<FMT, 1, 1>(mt, shallow, grid, block, smem, st, a);
    }
}

template <int FMT>
void launch_gemv_pro_fmt(bool paired, int pro, dim3 grid, size_t smem, hipStream_t st, const GemvArgs &a,
                         const ProArgs &pa) {
    const dim3 block(pro_threads(pro));
    if (pro == PRO_NORM) {
        if (paired) hipLaunchKernelGGL((k_gemv_pro<FMT, 2, PRO_NORM>), grid, block, smem, st, a, pa);
        else hipLaunchKernelGGL((k_gemv_pro<FMT, 1, PRO_NORM>), grid, block, smem, st, a, pa);
    } else {
        if (paired) hipLaunchKernelGGL((k_gemv_pro<FMT, 2, PRO_COMB>), grid, block, smem, st, a, pa);
        else hipLaunchKernelGGL((k_gemv_pro<FMT, 1, PRO_COMB>), grid, block, smem, st, a, pa);
    }
}

static_assert(GEMV_MAX_SLICES <= PRO_MAX_SLICES, "a norm prologue adds at most PRO_MAX_SLICES pending slices");
// A prologue GEMV takes one column, one row unit per block and (norm) a hidden size up to PRO_NORM_HMAX.
// (The packer makes K an exact multiple of the k-tile, so a block's k-range never passes H or NH * HD.)
bool gemv_pro_ok(const DevMat &m, int pro, int H, int HD, int slices = 0, int waves = 0) {
    if (pro == PRO_NONE) return true;
    const GemvPlan p = plan_gemv(m, 1, true, slices, waves);
    const int nt = pro_threads(pro);
    if (p.r != 1 || p.nw > nt / 64) return false;
    if (pro == PRO_NORM && (H > PRO_NORM_HMAX || H < 1)) return false;
    if (pro == PRO_COMB && (HD < 64 || HD > nt || nt % HD != 0 || HD % 64 != 0)) return false;
    return true;
}

// One column through k_gemv1: T = the wave's k-tile count (template), NW waves, the prologue if any.
template <int FMT, int RG, int PRO>
bool launch_gemv1_t(int T, dim3 grid, dim3 block, size_t smem, hipStream_t st, const GemvArgs &a, const ProArgs &pa) {
    switch (T) {
        case 1: hipLaunchKernelGGL((k_gemv1<FMT, RG, 1, PRO>), grid, block, smem, st, a, pa); return true;
        case 2: hipLaunchKernelGGL((k_gemv1<FMT, RG, 2, PRO>), grid, block, smem, st, a, pa); return true;
        case 3: hipLaunchKernelGGL((k_gemv1<FMT, RG, 3, PRO>), grid, block, smem, st, a, pa); return true;
        case 4: hipLaunchKernelGGL((k_gemv1<FMT, RG, 4, PRO>), grid, block, smem, st, a, pa); return true;
        default: break;
    }
    if constexpr (PRO == PRO_NONE) {
        switch (T) {
            case 5: hipLaunchKernelGGL((k_gemv1<FMT, RG, 5, PRO>), grid, block, smem, st, a, pa); return true;
            case 6: hipLaunchKernelGGL((k_gemv1<FMT, RG, 6, PRO>), grid, block, smem, st, a, pa); return true;
            case 7: case 8: hipLaunchKernelGGL((k_gemv1<FMT, RG, 8, PRO>), grid, block, smem, st, a, pa); return true;
            default: break;
        }
    }
    return false;
}
template <int FMT>
bool launch_gemv1_fmt(bool paired, int pro, int T, dim3 grid, dim3 block, size_t smem, hipStream_t st, const GemvArgs &a,
                      const ProArgs &pa) {
    if (paired) return pro == PRO_NONE && launch_gemv1_t<FMT, 2, PRO_NONE>(T, grid, block, smem, st, a, pa);
    if (pro == PRO_NORM) return launch_gemv1_t<FMT, 1, PRO_NORM>(T, grid, block, smem, st, a, pa);
    if (pro == PRO_COMB) return launch_gemv1_t<FMT, 1, PRO_COMB>(T, grid, block, smem, st, a, pa);
    return launch_gemv1_t<FMT, 1, PRO_NONE>(T, grid, block, smem, st, a, pa);
}

// Launches y = W x for mcols columns.  With `part` given (and a matrix that is not the SwiGLU pair) the plan may
// split K: the kernel then writes raw slices to part[s][m][ldo] and the return value is the slice count that the
// consumer must add (plus the bias, for EPI_STORE); otherwise the epilogue is applied and 0 is returned.  With a
// prologue (pro != PRO_NONE, one column) the activations come from *pa instead of x.
// `xlo` (optional): the fp16 remainders of x in x's layout; `out_lo` (optional, the SwiGLU pair): where the remainders
// of the SwiGLU output go.
int launch_gemv(const DevMat &m, int epi, const f16 *x, int ldx, int mcols, float *out_f32, f16 *out_f16, int ldo,
                const float *bias, hipStream_t st, float *part = nullptr, size_t pstride = 0, int pro = PRO_NONE,
                const ProArgs *pa = nullptr, int slices = 0, int waves = 0, int xmtp = 0, int omtp = 0,
                const f16 *xlo = nullptr, f16 *out_lo = nullptr) {
    require(mcols >= 1 && mcols <= 16 * GEMV_MAX_MT, SP_EINVAL, "gemv columns out of range");
    require((epi == EPI_SILU) == m.paired, SP_EINVAL, "gemv epilogue does not match the matrix packing");
    require(pro == PRO_NONE || (mcols == 1 && pa), SP_EINVAL, "gemv prologue needs one column and its arguments");
    const int mt = (mcols + 15) / 16;
    const GemvPlan p = plan_gemv(m, mt, part != nullptr, slices, waves);
    require(p.units % p.r == 0 && p.s >= 1 && p.s <= GEMV_MAX_SLICES, SP_EINVAL, "gemv plan out of range");
    GemvArgs a;
    a.w = m.w; a.sz = m.sz; a.nkt = m.nkt; a.units = p.units;
    a.n_real = m.paired ? m.rows / 2 : m.rows;
    a.x = x; a.ldx = ldx; a.m = mcols;
    a.out_f32 = out_f32; a.out_f16 = out_f16; a.ldo = ldo; a.bias = bias; a.epi = epi;
    a.kslice = p.kslice; a.pstride = pstride; a.nwk = p.nw;
    require(xmtp == 0 || xmtp == mt, SP_EINVAL, "gemv input layout does not match the column count");
    a.xmtp = xmtp; a.omtp = omtp;
    require(pro == PRO_NONE || xlo == nullptr, SP_EINVAL, "a prologue GEMV builds its own activations");
    a.xlo = xlo; a.out_lo = m.paired ? out_lo : nullptr;
    if (p.s > 1) { a.epi = EPI_PART; a.out_f32 = part; a.bias = nullptr; }
    // one column of a layer matrix: k_gemv1 (row groups one per block; the prologues need their fixed block sizes)
    if (mcols == 1 && xmtp == 0 && p.units < 2048 && m.rows_pad / 16 / p.rg == p.units) {
        int nw = pro == PRO_NONE ? p.nw : pro_threads(pro) / 64;
        // the SwiGLU pair: 8 waves of <= 3 k-tiles each keep the most loads in flight (launch-shape sweep)
        if (m.paired && waves == 0) {
            nw = std::min(p.kslice, 8);
        }
        const int T = (p.kslice + nw - 1) / nw;
        const int kt = m.fmt == 1 ? 32 : (m.fmt == 2 ? 64 : 128);
        const int prof = pro == PRO_NONE ? 0 : pro_scratch_floats(pro, pa->H, pa->HD);
        const size_t smem = g1_smem_bytes(p.kslice, kt, nw, p.rg, prof);
        const dim3 grid1(p.units, p.s), block1(64 * nw);
        const ProArgs pz = pro == PRO_NONE ? ProArgs{} : *pa;
        if (smem <= GEMV_MAX_LDS) {
            bool ok = false;
            switch (m.fmt) {
                case 1: ok = launch_gemv1_fmt<1>(m.paired, pro, T, grid1, block1, smem, st, a, pz); break;
                case 2: ok = launch_gemv1_fmt<2>(m.paired, pro, T, grid1, block1, smem, st, a, pz); break;
                default: ok = launch_gemv1_fmt<3>(m.paired, pro, T, grid1, block1, smem, st, a, pz); break;
            }
            if (ok) return p.s > 1 ? p.s : 0;
        }
    }
    dim3 grid(p.units / p.r, p.s), block(64 * p.nw);
    if (pro != PRO_NONE) {
        require(p.r == 1 && p.nw <= pro_threads(pro) / 64, SP_EINVAL, "gemv prologue plan out of range");
        const int kt = m.fmt == 1 ? 32 : (m.fmt == 2 ? 64 : 128);
        const size_t klen = ((size_t)p.kslice * kt + 7) & ~(size_t)7;
        // activations and their remainders, then the prologue's scratch
        const size_t smem = (size_t)p.nw * p.rg * 1024 + klen * 2 * 2 + (size_t)pro_scratch_floats(pro, pa->H, pa->HD) * 4;
        require(smem <= GEMV_MAX_LDS, SP_EINVAL, "gemv prologue LDS out of range");
        switch (m.fmt) {
            case 1: launch_gemv_pro_fmt<1>(m.paired, pro, grid, smem, st, a, *pa); break;
            case 2: launch_gemv_pro_fmt<2>(m.paired, pro, grid, smem, st, a, *pa); break;
            default: launch_gemv_pro_fmt<3>(m.paired, pro, grid, smem, st, a, *pa); break;
        }
        return p.s > 1 ? p.s : 0;
    }
    const size_t smem = p.nw > 1 ? (size_t)p.nw * p.r * p.rg * mt * 64 * 16 : 0;
    switch (m.fmt) {
        case 1: launch_gemv_fmt<1>(mt, m.paired, p.r, p.shallow, grid, block, smem, st, a); break;
        case 2: launch_gemv_fmt<2>(mt, m.paired, p.r, p.shallow, grid, block, smem, st, a); break;
        default: launch_gemv_fmt<3>(mt, m.paired, p.r, p.shallow, grid, block, smem, st, a); break;
    }
    return p.s > 1 ? p.s : 0;
}

// ------------------------------------------------------------------------------------------- attention dispatch
template <int HD>
void launch_attn_hd(int G, dim3 grid, hipStream_t st, const AttnArgs &a) {
    switch (G) {
        case 1: hipLaunchKernelGGL((k_attn_part<HD, 1>), grid, dim3(64 * 1), 0, st, a); break;
        case 2: hipLaunchKernelGGL((k_attn_part<HD, 2>), grid, dim3(64 * 2), 0, st, a); break;
        case 3: hipLaunchKernelGGL((k_attn_part<HD, 3>), grid, dim3(64 * 3), 0, st, a); break;
        case 4: hipLaunchKernelGGL((k_attn_part<HD, 4>), grid, dim3(64 * 4), 0, st, a); break;
        case 5: hipLaunchKernelGGL((k_attn_part<HD, 5>), grid, dim3(64 * 5), 0, st, a); break;
        case 6: hipLaunchKernelGGL((k_attn_part<HD, 6>), grid, dim3(64 * 6), 0, st, a); break;
        case 7: hipLaunchKernelGGL((k_attn_part<HD, 7>), grid, dim3(64 * 7), 0, st, a); break;
        default: hipLaunchKernelGGL((k_attn_part<HD, 8>), grid, dim3(64 * 8), 0, st, a); break;
    }
}

template <int HD>
void launch_attn_rope_hd(int G, dim3 grid, hipStream_t st, const AttnArgs &a, const RopeArgs &r, int np) {
    switch (G) {
        case 1: hipLaunchKernelGGL((k_attn_part_rope<HD, 1>), grid, dim3(64 * 1), 0, st, a, r, np); break;
        case 2: hipLaunchKernelGGL((k_attn_part_rope<HD, 2>), grid, dim3(64 * 2), 0, st, a, r, np); break;
        case 3: hipLaunchKernelGGL((k_attn_part_rope<HD, 3>), grid, dim3(64 * 3), 0, st, a, r, np); break;
        case 4: hipLaunchKernelGGL((k_attn_part_rope<HD, 4>), grid, dim3(64 * 4), 0, st, a, r, np); break;
        case 5: hipLaunchKernelGGL((k_attn_part_rope<HD, 5>), grid, dim3(64 * 5), 0, st, a, r, np); break;
        case 6: hipLaunchKernelGGL((k_attn_part_rope<HD, 6>), grid, dim3(64 * 6), 0, st, a, r, np); break;
        case 7: hipLaunchKernelGGL((k_attn_part_rope<HD, 7>), grid, dim3(64 * 7), 0, st, a, r, np); break;
        default: hipLaunchKernelGGL((k_attn_part_rope<HD, 8>), grid, dim3(64 * 8), 0, st, a, r, np); break;
    }
}

// Keys per multi-query block (one partial record per block and row): 128 for tree groups (verify pass: 33 x 12
// query rows, fewer and larger blocks, half the records to merge; -1 % per pass), 64 otherwise (the plain batches
// and prefill chunks got slower with 128: bs16 +16 %, prefill +3 %).
template <int HD, int CH>
void launch_attn_mq_ch(int G, dim3 grid, hipStream_t st, const AttnMqArgs &a) {
    switch (G) {
        case 1: hipLaunchKernelGGL((k_attn_mq<HD, 1, CH>), grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((k_attn_mq<HD, 2, CH>), grid, dim3(256), 0, st, a); break;
        case 3: hipLaunchKernelGGL((k_attn_mq<HD, 3, CH>), grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((k_attn_mq<HD, 4, CH>), grid, dim3(256), 0, st, a); break;
        case 5: hipLaunchKernelGGL((k_attn_mq<HD, 5, CH>), grid, dim3(256), 0, st, a); break;
        case 6: hipLaunchKernelGGL((k_attn_mq<HD, 6, CH>), grid, dim3(256), 0, st, a); break;
        case 7: hipLaunchKernelGGL((k_attn_mq<HD, 7, CH>), grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL((k_attn_mq<HD, 8, CH>), grid, dim3(256), 0, st, a); break;
    }
}
template <int HD>
void launch_attn_mq_hd(int G, int ch, dim3 grid, hipStream_t st, const AttnMqArgs &a) {
    if (ch == 128) launch_attn_mq_ch<HD, 128>(G, grid, st, a);
    else launch_attn_mq_ch<HD, 64>(G, grid, st, a);
}

template <class F>
void by_slices(int np, F &&f) {
    switch (np) {
        case 0: f(std::integral_constant<int, 0>()); break;
        case 1: f(std::integral_constant<int, 1>()); break;
        case 2: f(std::integral_constant<int, 2>()); break;
        case 3: f(std::integral_constant<int, 3>()); break;
        case 4: f(std::integral_constant<int, 4>()); break;
        case 5: f(std::integral_constant<int, 5>()); break;
        case 6: f(std::integral_constant<int, 6>()); break;
        case 7: f(std::integral_constant<int, 7>()); break;
        default: f(std::integral_constant<int, 8>()); break;
    }
}

// RMSNorm of n columns of x, first adding np pending split-K residual slices; the fp16 output and its remainders
void launch_rmsnorm(int n, float *x, int H, const float *part, int np, size_t ps, const float *w, float eps, f16 *out,
                    f16 *out_lo, hipStream_t st, int mtp) {
    by_slices(np, [&](auto c) {
        hipLaunchKernelGGL((k_rmsnorm<decltype(c)::value>), dim3(n), dim3(NORM_THREADS), 0, st, x, H, part, ps, w, H, eps,
                           out, out_lo, H, mtp);
    });
}

void launch_rope(int n, const RopeArgs &ra, int np, hipStream_t st) {
    by_slices(np, [&](auto c) { hipLaunchKernelGGL((k_rope_kv<decltype(c)::value>), dim3(n, 2), dim3(ROPE_THREADS), 0, st, ra); });
}

// decode attention split: waves per block x 32-key sub-chunks per wave
struct DecShape { int nwv, sub; };
// Keys per decode-attention block: 1024 (2 waves streaming 16 sub-chunks of 32 keys, two sub-chunks of loads in
// flight per wave) when the ranges give the chip at least two such blocks per CU, else 256 (4 waves x 2 sub-chunks).
// 32 columns of 8260 keys, 4 kv heads: 126 -> 111 us per launch.
DecShape dec_shape(int kpb) {
    return kpb >= 1024 ? DecShape{2, 16} : DecShape{4, 2};
}
int dec_keys(const DecShape &d) { return d.nwv * d.sub * DEC_KC; }
// The routing between the attention kernels (plan_attention) counts work in splits of this many keys (the sweeps
// that set its thresholds used 256-key blocks); the decode kernel's own grid uses its shape's key count.
constexpr int DEC_ROUTE_KEYS = 256;

template <int HD>
void launch_attn_dec_hd(int kpb, dim3 grid, hipStream_t st, const AttnArgs &aa, f16 *out, int ldo, int direct, int mtp) {
    const DecShape d = dec_shape(kpb);
    if (d.nwv == 2 && d.sub == 16) hipLaunchKernelGGL((k_attn_dec<HD, 2, 16>), grid, dim3(128), 0, st, aa, out, ldo, direct, mtp);
    else hipLaunchKernelGGL((k_attn_dec<HD, 4, 2>), grid, dim3(256), 0, st, aa, out, ldo, direct, mtp);
}
void launch_attn_dec(int HD, int kpb, dim3 grid, hipStream_t st, const AttnArgs &aa, f16 *out, int ldo, int direct,
                     int mtp) {
    if (HD == 64) launch_attn_dec_hd<64>(kpb, grid, st, aa, out, ldo, direct, mtp);
    else launch_attn_dec_hd<128>(kpb, grid, st, aa, out, ldo, direct, mtp);
}

// SP_F_DEVCOLS: the uploaded column records take their tokens (clamped to the vocabulary, as a fed token is) and,
// when given, their tree masks from device arrays, on the stream ahead of the step.
__global__ void k_patch_columns(sp_token *t, int n, const int32_t *tokens, const uint64_t *masks, int vocab) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    t[i].token = min(max(tokens[i], 0), vocab - 1);
    if (masks) t[i].tree_mask = masks[i];
}

template <int FMT>
void launch_embed(const DevMat &m, const sp_token *toks, int n, int H, float *x, hipStream_t st, const int *feed,
                  int vocab, const float *inv_freq, int half, float2 *rtab) {
    hipLaunchKernelGGL((k_embed<FMT>), dim3(n), dim3(256), 0, st, m.w, m.sz, m.nkt, toks, H, x, H, feed, vocab,
                       inv_freq, half, rtab);
}

// Instantiations of the persistent one-column step: (format, head_dim, k-tiles per wave for K = hidden, k-tiles per
// wave of a down item).  Shapes without one run the chain.
struct D1Kernel {
    int fmt, hd, th, t5;
    const void *fn;
};
const D1Kernel D1_KERNELS[] = {
    {2, 128, 3, 9, (const void *)d1::k_decode1<2, 128, 3, 9>},     // Qwen2-1.5B int8
    {3, 128, 2, 5, (const void *)d1::k_decode1<3, 128, 2, 5>},     // Qwen2-1.5B int4
    {1, 64, 4, 10, (const void *)d1::k_decode1<1, 64, 4, 10>},     // Qwen2-0.5B fp16
    {2, 64, 2, 5, (const void *)d1::k_decode1<2, 64, 2, 5>},       // Qwen2-0.5B int8
    {1, 64, 1, 1, (const void *)d1::k_decode1<1, 64, 1, 1>},       // small test shapes
    {2, 64, 1, 1, (const void *)d1::k_decode1<2, 64, 1, 1>},
    {3, 64, 1, 1, (const void *)d1::k_decode1<3, 64, 1, 1>},
};
const D1Kernel *find_d1_kernel(const d1::Geom &g) {
    const int th = std::max(d1::cdiv(g.nkt_h, d1::NW), d1::cdiv(g.nkt_a, d1::NW)), t5 = d1::cdiv(g.nk5, d1::NW);
    for (const D1Kernel &k : D1_KERNELS)
        if (k.fmt == g.fmt && k.hd == g.HD && k.th == th && k.t5 == t5) return &k;
    return nullptr;
}

}  // namespace

// ============================================================================================== engine
struct sp_engine {
    sp_model_desc d{};
    std::string err;
    hipStream_t stream = nullptr;
    hipStream_t capture_stream = nullptr;   // private: graphs are recorded here and launched on `stream`
    bool own_stream = false;
    int device = 0;

    struct Layer {
        DevMat qkv, o, gate_up, down;
        float *qkv_b = nullptr, *in_norm = nullptr, *post_norm = nullptr;
    };
    std::vector<Layer> layers;
    DevMat embed, head;
    float *final_norm = nullptr, *inv_freq = nullptr;
    uint64_t weight_bytes = 0, kv_bytes = 0;

    // activations
    int Nqkv = 0, maxT = 0, max_nchunk = 0;
    float *x = nullptr, *qkv = nullptr, *q = nullptr, *logits = nullptr, *attn_part = nullptr;
    float2 *rtab = nullptr;      // the step's RoPE (cos, sin) per column and frequency, written by the embedding kernel
    float *gpart = nullptr;      // split-K GEMV slices [GEMV_MAX_SLICES][maxT][max(H, Nqkv)]
    size_t gpart_stride = 0;
    // single-column steps with the norms / combine folded into the GEMVs: the residual alternates between x (layer
    // boundaries) and x2 (after the input norm), and the qkv slices go to gpart2 while the down slices in gpart are
    // still being read
    float *x2 = nullptr, *gpart2 = nullptr;
    f16 *xn = nullptr, *attn = nullptr, *act = nullptr;
    // the fp16 remainders (split_f16) of the normalised GEMV inputs (qkv always; gate_up in one-column steps) and of
    // the SwiGLU activation of one-column steps
    f16 *xn_lo = nullptr, *act_lo = nullptr;
    float *am_v = nullptr;
    int *am_i = nullptr, *am_out = nullptr;
    int argmax_cols = 0;         // columns whose argmax ids am_out holds (the last SP_F_ARGMAX call)
    // column descriptors of a call: tokens, attention groups, chunk counts, uploaded together from a pinned staging
    // buffer (one copy per call); `upload_done` marks the copy so the staging buffer is not rewritten before it ran
    sp_token *dtoks = nullptr;
    AttnGroup *dgroups = nullptr;
    int *dcolnc = nullptr;
    char *d_upload = nullptr, *h_upload = nullptr;
    size_t upload_bytes = 0;
    hipEvent_t upload_done = nullptr;
    int *h_ids = nullptr;        // pinned landing buffer of the greedy ids a call returns to the host
    // SP_F_DEVCOLS: device arrays the columns' tokens and tree masks are read from (sp_engine_set_device_columns)
    const int32_t *dev_tokens = nullptr;
    const uint64_t *dev_masks = nullptr;

    // KV ring
    int n_seq = 0, n_slots = 0;
    std::vector<f16 *> kc, vc;
    f16 **d_kl = nullptr, **d_vl = nullptr;
    int *d_move = nullptr;

    std::map<std::tuple<int, int, int>, hipGraphExec_t> graphs;
    std::map<std::tuple<int, int, int>, int> graph_kernels;     // kernel nodes of each recorded step part
    int last_dispatches = -1;                                   // kernels of the last graph replay (-1: eager call)
    void drop_graphs() {
        for (auto &kv : graphs) (void)hipGraphExecDestroy(kv.second);
        graphs.clear();
        graph_kernels.clear();
    }

    int last_path = -1;

    // persistent one-column step (sp_decode1.h): geometry for the current pool, tagged words, the error word
    int d1_state = 0;            // 0: to be prepared, 1: ready, -1: does not apply (d1_why says why)
    std::string d1_why;
    d1::Geom d1g{};
    const D1Kernel *d1k = nullptr;
    unsigned long long *d1_ll = nullptr;
    unsigned *d1_err = nullptr, *h_d1err = nullptr;
    d1::LayerPtr *d1_layers = nullptr;
    d1::Static *d1_static = nullptr;
    unsigned d1_seq = 0;
    bool d1_plain = false;       // the runtime refused a cooperative launch once: plain launches from then on
    bool prepare_d1();
    bool launch_d1(const sp_token &t, int flags);     // the persistent kernel alone
    bool run_d1(const sp_token &t, int flags);        // + the error word copy, the head GEMV and the argmax
    void check_d1_error();

    // attention plan of one forward call: same-sequence column groups (multi-query kernel) or one block row per column
    struct AttnPlan {
        bool mq = false;
        bool dec = false;        // every column a plain ring range (no tree block): k_attn_dec over key splits
        bool dec_direct = false; // ... and every column fits one split: no combine
        bool rope_fused = false; // chunk kernel with RoPE / KV write folded in (plain columns of distinct sequences)
        int mq_ch = ATT_CH;      // keys per multi-query block
        int dec_kpb = 256;       // keys per decode-attention block
        int ngroups = 0, nchunk = 1, splits = 1;
        std::vector<AttnGroup> groups;
        std::vector<int> colnc;
    };
    AttnPlan plan_attention(int n, const sp_token *t, bool graph) const;

    void free_all();
    void alloc_activations();
    void step(int n, int flags, const AttnPlan &ap, int l0, int l1);
    void launch_attention(int l, int n, const AttnPlan &ap, int mtp, hipStream_t st);
    void check_columns(int n, const sp_token *toks, bool feed) const;
    void upload(int n, const sp_token *toks, const AttnPlan &ap);
};

void sp_engine::free_all() {
    drop_graphs();
    dev_free(d1_ll); dev_free(d1_err); dev_free(d1_layers); dev_free(d1_static);
    if (h_d1err) (void)hipHostFree(h_d1err);
    d1_ll = nullptr; d1_err = nullptr; d1_layers = nullptr; d1_static = nullptr; h_d1err = nullptr; d1_state = 0;
    for (auto &l : layers) {
        l.qkv.release(); l.o.release(); l.gate_up.release(); l.down.release();
        dev_free(l.qkv_b); dev_free(l.in_norm); dev_free(l.post_norm);
    }
    layers.clear();
    embed.release(); head.release();
    dev_free(final_norm); dev_free(inv_freq);
    for (void *p : {(void *)x, (void *)x2, (void *)qkv, (void *)q, (void *)rtab, (void *)logits, (void *)attn_part, (void *)gpart,
                    (void *)gpart2, (void *)xn, (void *)attn, (void *)xn_lo, (void *)act_lo,
                    (void *)act, (void *)am_v, (void *)am_i, (void *)am_out,
                    (void *)d_upload, (void *)d_kl, (void *)d_vl, (void *)d_move})
        dev_free(p);
    for (auto p : kc) dev_free(p);
    for (auto p : vc) dev_free(p);
    kc.clear(); vc.clear();
    if (h_upload) (void)hipHostFree(h_upload);
    if (h_ids) (void)hipHostFree(h_ids);
    if (upload_done) (void)hipEventDestroy(upload_done);
    h_upload = nullptr; h_ids = nullptr; upload_done = nullptr; d_upload = nullptr;
    dtoks = nullptr; dgroups = nullptr; dcolnc = nullptr;
    if (own_stream && stream) (void)hipStreamDestroy(stream);
    if (capture_stream) (void)hipStreamDestroy(capture_stream);
    stream = nullptr;
    capture_stream = nullptr;
}

void sp_engine::alloc_activations() {
    const int H = d.hidden, I = d.intermediate, V = d.vocab;
    Nqkv = (d.n_heads + 2 * d.n_kv_heads) * d.head_dim;
    maxT = d.max_tokens;
    const int kmax = std::max(std::max(H, I), d.n_heads * d.head_dim);
    const size_t tpad = (size_t)(maxT + 15) / 16 * 16;       // fragment-major inputs hold whole 16-column tiles
    x = dev_alloc<float>((size_t)maxT * H);
    xn = dev_alloc<f16>(tpad * kmax);
    xn_lo = dev_alloc<f16>(tpad * kmax);
    act_lo = dev_alloc<f16>(I);
    qkv = dev_alloc<float>((size_t)maxT * Nqkv);
    gpart_stride = (size_t)maxT * std::max(H, Nqkv);
    gpart = dev_alloc<float>(GEMV_MAX_SLICES * gpart_stride);
    gpart2 = dev_alloc<float>(GEMV_MAX_SLICES * gpart_stride);
    x2 = dev_alloc<float>((size_t)maxT * H);
    q = dev_alloc<float>((size_t)maxT * d.n_heads * d.head_dim);
    rtab = dev_alloc<float2>((size_t)maxT * (d.head_dim / 2));
    HIPCHK(hipMemset(rtab, 0, (size_t)maxT * (d.head_dim / 2) * sizeof(float2)));
    attn = dev_alloc<f16>(tpad * d.n_heads * d.head_dim);
    act = dev_alloc<f16>(tpad * I);
    logits = dev_alloc<float>((size_t)maxT * V);
    am_v = dev_alloc<float>((size_t)maxT * ARGMAX_BLOCKS);
    am_i = dev_alloc<int>((size_t)maxT * ARGMAX_BLOCKS);
    am_out = dev_alloc<int>(maxT);
    HIPCHK(hipMemset(am_out, 0, maxT * sizeof(int)));
    argmax_cols = 0;
    // [tokens][groups][chunk counts], each part 16-byte aligned
    const size_t tb = ((size_t)maxT * sizeof(sp_token) + 15) & ~(size_t)15;
    const size_t gb = ((size_t)maxT * sizeof(AttnGroup) + 15) & ~(size_t)15;
    upload_bytes = tb + gb + (size_t)maxT * sizeof(int);
    d_upload = dev_alloc<char>(upload_bytes);
    dtoks = (sp_token *)d_upload;
    dgroups = (AttnGroup *)(d_upload + tb);
    dcolnc = (int *)(d_upload + tb + gb);
    HIPCHK(hipHostMalloc((void **)&h_upload, upload_bytes, hipHostMallocDefault));
    HIPCHK(hipHostMalloc((void **)&h_ids, (size_t)maxT * sizeof(int), hipHostMallocDefault));
    HIPCHK(hipEventCreateWithFlags(&upload_done, hipEventDisableTiming));
    d_move = dev_alloc<int>(2 * 64);
    HIPCHK(hipMemset(xn, 0, tpad * kmax * sizeof(f16)));
    HIPCHK(hipMemset(xn_lo, 0, tpad * kmax * sizeof(f16)));
    HIPCHK(hipMemset(act_lo, 0, I * sizeof(f16)));
    HIPCHK(hipMemset(attn, 0, tpad * d.n_heads * d.head_dim * sizeof(f16)));
    HIPCHK(hipMemset(act, 0, tpad * I * sizeof(f16)));
}

sp_engine::AttnPlan sp_engine::plan_attention(int n, const sp_token *t, bool graph) const {
    AttnPlan p;
    auto nlin_of = [](const sp_token &x) { return x.ctx_hi >= x.ctx_lo ? x.ctx_hi - x.ctx_lo + 1 : 0; };
    // maximal runs of columns with the same sequence and tree block whose union ring range fits the slots
    int i = 0;
    while (i < n) {
        AttnGroup g{};
        g.first_col = i; g.seq = t[i].seq; g.tree_base = t[i].tree_base; g.tree_count = t[i].tree_count;
        int lo = INT32_MAX, hi = -1;
        int j = i;
        for (; j < n; ++j) {
            if (t[j].seq != g.seq || t[j].tree_count != g.tree_count || (g.tree_count && t[j].tree_base != g.tree_base)) break;
            int l2 = lo, h2 = hi;
            if (nlin_of(t[j]) > 0) { l2 = std::min(lo, t[j].ctx_lo); h2 = std::max(hi, t[j].ctx_hi); }
            if (h2 >= l2 && h2 - l2 + 1 > n_slots) break;
            lo = l2; hi = h2;
        }
        g.ncols = j - i;
        g.lo = hi >= lo ? lo : 0;
        g.nlin = hi >= lo ? hi - lo + 1 : 0;
        p.groups.push_back(g);
        i = j;
    }
    p.ngroups = (int)p.groups.size();
    int maxcols = 1;
    for (auto &g : p.groups) { p.mq = p.mq || g.ncols > 1; maxcols = std::max(maxcols, g.ncols); }
    const int G = d.n_heads / d.n_kv_heads;
    // blocks per kv head and column: decode key splits of DEC_ROUTE_KEYS keys, chunk-kernel blocks of ATT_CH
    long dec_work = 0, chunk_work = 0;
    bool dec_cols = G <= 8;
    for (int c = 0; c < n; ++c) {
        dec_cols = dec_cols && t[c].tree_count == 0 && nlin_of(t[c]) >= 1;
        dec_work += (long)(nlin_of(t[c]) + DEC_ROUTE_KEYS - 1) / DEC_ROUTE_KEYS * d.n_kv_heads;
        chunk_work += (long)(nlin_of(t[c]) + ATT_CH - 1) / ATT_CH * d.n_kv_heads;
    }
    // several plain columns whose 64-key chunks fill the chip but whose decode splits would not give each CU a few
    // blocks: the multi-query kernel (MFMA scores for all query heads of a kv head) is the fastest there.  Measured per
    // step: 16 x 1024 keys, 2 kv heads (512 chunks, 128 splits) multi-query 2.3% faster than the chunk kernel;
    // 32 x 8192 keys, 4 kv heads (4096 splits) the decode kernel 2.8% faster; 16 ragged prompts of 16-128 keys
    // (about 64 chunks) the chunk kernel with the rotation fused 7% faster.
    if (n > 1 && dec_cols && chunk_work >= 256 && dec_work < 1024) p.mq = true;
    p.splits = (maxcols * G + 63) / 64;
    p.colnc.assign(n, 0);
    int mx = 1;
    if (p.mq) {
        // 128-key blocks for tree groups of many query rows (the 33-node target pass: 198 rows); a drafter level's
        // 8 columns (56 rows, 4 row tiles) fill more CUs with 64-key blocks (speculative step -1.2 %)
        bool trees = true;
        int rows = 0;
        for (auto &g : p.groups) {
            trees = trees && g.tree_count > 0;
            rows = std::max(rows, g.ncols * G);
        }
        p.mq_ch = trees && rows >= 128 ? 128 : ATT_CH;
        for (auto &g : p.groups) {
            const int nc = (g.nlin + g.tree_count + p.mq_ch - 1) / p.mq_ch;
            for (int c = 0; c < g.ncols; ++c) p.colnc[g.first_col + c] = nc;
            mx = std::max(mx, nc);
        }
    } else {
        for (int c = 0; c < n; ++c) {
            p.colnc[c] = (nlin_of(t[c]) + t[c].tree_count + ATT_CH - 1) / ATT_CH;
            mx = std::max(mx, p.colnc[c]);
        }
    }
    // a recorded graph serves every later length: its grid covers the longest visible list the slots allow
    p.nchunk = graph ? (p.mq ? (max_nchunk * ATT_CH + p.mq_ch - 1) / p.mq_ch : max_nchunk) : mx;
    if (!p.mq && dec_cols) {
        // the MFMA decode kernel pays off once its key splits fill the chip (long contexts, large batches); short
        // ranges stay on the 64-key chunk kernel, which spreads them over more CUs
        p.dec = dec_work >= 256;
    }
    if (!p.mq && !p.dec) {
        // every column a plain ring range of its own sequence: no column sees another column's new key, so each
        // attention block may rotate and store the key of the position it holds
        bool plain = true;
        std::vector<int> seqs;
        for (int c = 0; c < n; ++c) {
            plain = plain && t[c].tree_count == 0 && nlin_of(t[c]) >= 1 && t[c].slot == t[c].ctx_hi % n_slots;
            seqs.push_back(t[c].seq);
        }
        std::sort(seqs.begin(), seqs.end());
        p.rope_fused = plain && std::adjacent_find(seqs.begin(), seqs.end()) == seqs.end();
    }
    if (p.dec) {
        long big = 0;                    // blocks of the 1024-key shape
        for (int c = 0; c < n; ++c) big += (long)(nlin_of(t[c]) + 1023) / 1024 * d.n_kv_heads;
        const int kpb = dec_keys(dec_shape(big >= 512 ? 1024 : 256));
        p.dec_kpb = kpb;
        // splits of kpb keys; a graph is sized for the longest range the ring allows
        int ms = 1;
        for (int c = 0; c < n; ++c) {
            p.colnc[c] = (nlin_of(t[c]) + kpb - 1) / kpb;
            ms = std::max(ms, p.colnc[c]);
        }
        p.nchunk = graph ? (n_slots + kpb - 1) / kpb : ms;
        p.dec_direct = p.nchunk == 1;
        if (p.nchunk > max_nchunk || p.nchunk > ATT_MAX_CHUNKS) {      // splits must fit the partial buffer
            p.dec = p.dec_direct = false;
            p.nchunk = graph ? max_nchunk : mx;
            for (int c = 0; c < n; ++c) p.colnc[c] = (nlin_of(t[c]) + t[c].tree_count + ATT_CH - 1) / ATT_CH;
        }
    }
    return p;
}

// Every column must name a token (unless fed from the last argmax), a reserved sequence and slot, and a visible range
// the ring holds; a tree block lies inside the ring.
void sp_engine::check_columns(int n, const sp_token *toks, bool feed) const {
    for (int i = 0; i < n; ++i) {
        const sp_token &t = toks[i];
        require(feed || (t.token >= 0 && t.token < d.vocab), SP_EINVAL, "token id out of range");
        require(t.seq >= 0 && t.seq < n_seq, SP_EINVAL, "sequence index out of range");
        require(t.slot >= 0 && t.slot < n_slots, SP_EINVAL, "slot out of range");
        require(t.pos >= 0, SP_EINVAL, "position must be non-negative");
        require(t.ctx_lo >= 0, SP_EINVAL, "ctx_lo must be non-negative");
        const int nlin = t.ctx_hi >= t.ctx_lo ? t.ctx_hi - t.ctx_lo + 1 : 0;
        require(nlin <= n_slots, SP_ECAPACITY, "visible range exceeds the KV slots");
        require(t.tree_count >= 0 && t.tree_count <= 64, SP_EINVAL, "tree_count must be in [0, 64]");
        require(t.tree_count == 0 || (t.tree_base >= 0 && t.tree_base < n_slots), SP_EINVAL, "tree_base out of range");
        require(nlin + t.tree_count >= 1, SP_EINVAL, "a column must see at least one key");
    }
}

// The call's column descriptors, attention groups and chunk counts go up in one copy from the pinned staging buffer.
void sp_engine::upload(int n, const sp_token *toks, const AttnPlan &ap) {
    HIPCHK(hipEventSynchronize(upload_done));       // the previous call's copy has read the staging buffer
    const size_t go = (char *)dgroups - d_upload, co = (char *)dcolnc - d_upload;
    std::memcpy(h_upload, toks, n * sizeof(sp_token));
    std::memcpy(h_upload + go, ap.groups.data(), ap.ngroups * sizeof(AttnGroup));
    std::memcpy(h_upload + co, ap.colnc.data(), n * sizeof(int));
    HIPCHK(hipMemcpyAsync(d_upload, h_upload, co + n * sizeof(int), hipMemcpyHostToDevice, stream));
    HIPCHK(hipEventRecord(upload_done, stream));
}

// The attention kernel of layer l for a plan without the fused RoPE: multi-query groups, MFMA decode splits (written
// straight to `attn` when one split covers every column) or 64-key chunks, reading q from the q buffer.
void sp_engine::launch_attention(int l, int n, const AttnPlan &ap, int mtp, hipStream_t st) {
    const int NH = d.n_heads, NKV = d.n_kv_heads, HD = d.head_dim, G = NH / NKV, nchunk = ap.nchunk;
    const float scale = 1.0f / std::sqrt((float)HD);
    if (ap.mq) {
        AttnMqArgs am{q, kc[l], vc[l], dtoks, dgroups, NH, NKV, HD, n_slots, nchunk, scale, attn_part, ap.splits};
        dim3 agrid(nchunk, NKV, ap.ngroups * ap.splits);
        if (HD == 64) launch_attn_mq_hd<64>(G, ap.mq_ch, agrid, st, am);
        else launch_attn_mq_hd<128>(G, ap.mq_ch, agrid, st, am);
    } else if (ap.dec) {
        AttnArgs aa{q, kc[l], vc[l], dtoks, NH, NKV, HD, n_slots, nchunk, scale, attn_part};
        launch_attn_dec(HD, ap.dec_kpb, dim3(NKV, n, nchunk), st, aa, attn, NH * HD, ap.dec_direct ? 1 : 0, mtp);
    } else {
        AttnArgs aa{q, kc[l], vc[l], dtoks, NH, NKV, HD, n_slots, nchunk, scale, attn_part};
        dim3 agrid(nchunk, NKV, n);
        if (HD == 64) launch_attn_hd<64>(G, agrid, st, aa);
        else launch_attn_hd<128>(G, agrid, st, aa);
    }
}

// Layers [l0, l1) of a forward call; the embedding when l0 == 0, the final norm / head / argmax when l1 == n_layers.
// A call may run as several such parts in order (each captured as a graph of its own): the state crossing a part
// boundary (which residual buffer holds the stream, how many split-K slices are pending) follows from the layer index.
void sp_engine::step(int n, int flags, const AttnPlan &ap, int l0, int l1) {
    const int nchunk = ap.nchunk;
    const int H = d.hidden, I = d.intermediate, NH = d.n_heads, NKV = d.n_kv_heads, HD = d.head_dim;
    hipStream_t st = stream;
    const int *feed = (flags & SP_F_FEED) ? am_out : nullptr;   // tokens = the previous step's argmax ids
    if (l0 == 0) {
        switch (embed.fmt) {
            case 1: launch_embed<1>(embed, dtoks, n, H, x, st, feed, d.vocab, inv_freq, HD / 2, rtab); break;
            case 2: launch_embed<2>(embed, dtoks, n, H, x, st, feed, d.vocab, inv_freq, HD / 2, rtab); break;
            default: launch_embed<3>(embed, dtoks, n, H, x, st, feed, d.vocab, inv_freq, HD / 2, rtab); break;
        }
    }
    const bool logits_on = flags & SP_F_LOGITS;
    const size_t ps = gpart_stride;
    // several columns: the fp16 GEMV inputs (xn, attn, act) are written fragment-major with mtp column tiles
    const int mtp = n > 1 ? (n + 15) / 16 : 0;
    int pend = 0;     // residual slices of a split-K o / down GEMV waiting in gpart (added by the next RMSNorm)
    // One column: the input RMSNorm runs as the prologue of the qkv GEMV and the attention combine as the prologue of
    // o_proj (two launches fewer per layer); qkv and the down projection run in the k-slices below, which the next
    // norm adds.  The prologue writes the updated residual to the other one of x / x2 (its blocks still read the first), so the
    // residual changes buffer at every layer; the qkv slices go to gpart2 while the blocks still read the down slices
    // in gpart.  SP_F_UNFUSED keeps the plans and runs the norm and the combine as kernels of their own.
    // launch-shape sweep of whole bs1 steps (1.5B int8): qkv in 2 slices of 8 waves, down in 8 slices of 8 waves
    int one_qs = 2, one_qw = 8, one_ds = 8, one_dw = 8;
    const bool one = n == 1 && !layers.empty() && gemv_pro_ok(layers[0].qkv, PRO_NORM, H, HD, one_qs, one_qw) &&
                     gemv_pro_ok(layers[0].o, PRO_COMB, H, HD);
    const bool fuse = one && !(flags & SP_F_UNFUSED);
    // batches of one column tile: qkv and o_proj in 2 k-slices (whole steps, 16 columns: Qwen2-1.5B int8 1.422 ->
    // 1.404 ms for qkv, then 1.406 -> 1.398 for o_proj, Qwen2-0.5B fp16 -0.8 %; the RoPE kernel and the norm then add
    // 2 slices instead of 8); int4 o_proj at several column tiles in 4 (Qwen2-7B at 32 columns: -0.3 %)
    const int qkv_s = one ? one_qs : (n > 1 && n <= 16 ? 2 : 0), qkv_w = one ? one_qw : 0;
    const int down_s = one ? one_ds : 0, down_w = one ? one_dw : 0;
    float *const qpart = fuse ? gpart2 : gpart;
    float *res = x;                             // residual at the start of the layer
    if (l0 > 0) {
        // fused one-column steps alternate x / x2 every layer; the down GEMV of layer l0 - 1 left its slices pending
        res = fuse && (l0 & 1) ? x2 : x;
        const GemvPlan dp = plan_gemv(layers[l0 - 1].down, (n + 15) / 16, true, down_s, down_w);
        pend = dp.s > 1 ? dp.s : 0;
    }
    for (int l = l0; l < l1; ++l) {
        Layer &ly = layers[l];
        float *rmid = res;                      // residual after the input norm
        int sq;
        if (fuse) {
            rmid = res == x ? x2 : x;
            ProArgs pn{};
            pn.res = res; pn.res_out = rmid; pn.part = gpart; pn.pstride = ps; pn.np = pend; pn.w = ly.in_norm;
            pn.eps = d.rms_eps; pn.H = H;
            sq = launch_gemv(ly.qkv, EPI_STORE, nullptr, H, n, qkv, nullptr, Nqkv, ly.qkv_b, st, qpart, ps, PRO_NORM, &pn,
                             qkv_s, qkv_w);
        } else {
            launch_rmsnorm(n, res, H, gpart, pend, ps, ly.in_norm, d.rms_eps, xn, xn_lo, st, mtp);
            sq = launch_gemv(ly.qkv, EPI_STORE, xn, H, n, qkv, nullptr, Nqkv, ly.qkv_b, st, qpart, ps, PRO_NONE, nullptr,
                             qkv_s, qkv_w, mtp, 0, xn_lo);
        }
        RopeArgs ra{qkv, Nqkv, NH, NKV, HD, rtab, dtoks, q, kc[l], vc[l], n_slots, qpart, ps, ly.qkv_b};
        const bool fused = ap.rope_fused && logits_on;
        if (!fused) launch_rope(n, ra, sq, st);
        if (l + 1 == d.n_layers && !logits_on) break;   // K/V-only: the last layer only needs its K/V
        const int G = NH / NKV;
        if (fused) {
            AttnArgs aa{q, kc[l], vc[l], dtoks, NH, NKV, HD, n_slots, nchunk, 1.0f / std::sqrt((float)HD), attn_part};
            dim3 agrid(nchunk, NKV, n);
            if (HD == 64) launch_attn_rope_hd<64>(G, agrid, st, aa, ra, sq);
            else launch_attn_rope_hd<128>(G, agrid, st, aa, ra, sq);
        } else {
            launch_attention(l, n, ap, mtp, st);
        }
        if (fuse && !ap.dec_direct) {
            ProArgs pc{};
            pc.apart = attn_part; pc.colnc = dcolnc; pc.NH = NH; pc.HD = HD; pc.nchunk = nchunk;
            pend = launch_gemv(ly.o, EPI_RESID, nullptr, NH * HD, n, rmid, nullptr, H, nullptr, st, gpart, ps, PRO_COMB, &pc);
        } else {
            if (!ap.dec_direct)
                hipLaunchKernelGGL(k_attn_combine, dim3(NH, n), dim3(HD), 0, st, attn_part, dcolnc, NH, HD, nchunk, attn,
                                   NH * HD, mtp);
            const int o_s = n > 1 && n <= 16 ? 2 : (n > 16 && ly.o.fmt == 3 ? 4 : 0);
            pend = launch_gemv(ly.o, EPI_RESID, attn, NH * HD, n, rmid, nullptr, H, nullptr, st, gpart, ps, PRO_NONE,
                               nullptr, o_s, 0, mtp);
        }
        // Remainders where they cost nothing (one column: MFMA row 1) or where the logits need them (the qkv input,
        // above: its rounding reaches the attention scores).  Several columns would pay a second MFMA and twice the
        // activation reads per fragment for the gate_up, down and head inputs, whose fp16 rounding moves the logits
        // far less.
        f16 *xlo = n == 1 ? xn_lo : nullptr, *alo = n == 1 ? act_lo : nullptr;
        launch_rmsnorm(n, rmid, H, gpart, pend, ps, ly.post_norm, d.rms_eps, xn, xlo, st, mtp);
        launch_gemv(ly.gate_up, EPI_SILU, xn, H, n, nullptr, act, I, nullptr, st, nullptr, 0, PRO_NONE, nullptr, 0, 0, mtp,
                    mtp, xlo, alo);
        pend = launch_gemv(ly.down, EPI_RESID, act, I, n, rmid, nullptr, H, nullptr, st, gpart, ps, PRO_NONE, nullptr,
                           down_s, down_w, mtp, 0, alo);
        res = rmid;
    }
    if (logits_on && l1 == d.n_layers) {
        const DevMat &hm = d.tied_head ? embed : head;
        // the head takes its input in fp16 alone: its rounding moves the logits by about 2.5e-4 max-rel at the
        // 1.5B int8 workload (against 6.7e-2 for the qkv input), and its remainders would double the head's
        // activation reads
        launch_rmsnorm(n, res, H, gpart, pend, ps, final_norm, d.rms_eps, xn, nullptr, st, mtp);
        launch_gemv(hm, EPI_STORE, xn, H, n, logits, nullptr, d.vocab, nullptr, st, nullptr, 0, PRO_NONE, nullptr, 0, 0, mtp);
        if (flags & SP_F_ARGMAX) {
            hipLaunchKernelGGL(k_argmax_part, dim3(ARGMAX_BLOCKS, n), dim3(256), 0, st, logits, d.vocab, d.vocab, am_v, am_i);
            hipLaunchKernelGGL(k_argmax_final, dim3(n), dim3(64), 0, st, am_v, am_i, am_out);
        }
    }
    HIPCHK(hipGetLastError());
}

// The persistent step for the current weights and KV pool: geometry, bounds walk, instantiation, co-residency, the
// tagged-word area and the per-layer pointer table.  Returns false (d1_why set) when the step does not apply.
bool sp_engine::prepare_d1() {
    if (d1_state != 0) return d1_state > 0;
    d1_state = -1;
    int nb = 0;
    HIPCHK(hipDeviceGetAttribute(&nb, hipDeviceAttributeMultiprocessorCount, device));
    const char *why = "";
    if (n_slots < 1 || !d1::make_geom(d, n_slots, nb, d1g, &why)) { d1_why = why; return false; }
    d1k = find_d1_kernel(d1g);
    if (!d1k) { d1_why = "no instantiation for this shape"; return false; }
    if (!d1::check_geom(d1g, d1k->th, d1k->t5, &why)) { d1_why = why; return false; }
    for (auto &l : layers)
        if (l.qkv.fmt != d.weight_format || l.o.fmt != d.weight_format || l.gate_up.fmt != d.weight_format ||
            l.down.fmt != d.weight_format) { d1_why = "mixed weight formats"; return false; }
    if (embed.fmt != d.weight_format) { d1_why = "mixed weight formats"; return false; }
    int per_cu = 0;
    HIPCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, d1k->fn, d1::NT, d1::SMEM_BYTES));
    if (per_cu < 1) { d1_why = "the block does not fit a CU"; return false; }
    dev_free(d1_ll); dev_free(d1_layers); dev_free(d1_static);
    d1_ll = nullptr; d1_layers = nullptr; d1_static = nullptr;
    d1_ll = dev_alloc<unsigned long long>(d1g.words);
    HIPCHK(hipMemset(d1_ll, 0, d1g.words * sizeof(unsigned long long)));     // tag 0 is never current
    if (!d1_err) {
        d1_err = dev_alloc<unsigned>(1);
        HIPCHK(hipMemset(d1_err, 0, sizeof(unsigned)));
        HIPCHK(hipHostMalloc((void **)&h_d1err, sizeof(unsigned), hipHostMallocDefault));
        *h_d1err = 0;
    }
    std::vector<d1::LayerPtr> lp(d.n_layers);
    for (int l = 0; l < d.n_layers; ++l) {
        const Layer &ly = layers[l];
        const DevMat *m[4] = {&ly.qkv, &ly.o, &ly.gate_up, &ly.down};
        for (int i = 0; i < 4; ++i) { lp[l].w[i] = m[i]->w; lp[l].sz[i] = m[i]->sz; }
        lp[l].qkv_b = ly.qkv_b; lp[l].n_in = ly.in_norm; lp[l].n_post = ly.post_norm;
        lp[l].kc = kc[l]; lp[l].vc = vc[l];
    }
    d1_layers = dev_alloc<d1::LayerPtr>(d.n_layers);
    HIPCHK(hipMemcpy(d1_layers, lp.data(), lp.size() * sizeof(d1::LayerPtr), hipMemcpyHostToDevice));
    d1::Static sa{};
    sa.g = d1g;
    sa.layers = d1_layers;
    sa.emb_w = embed.w; sa.emb_sz = embed.sz;
    sa.final_norm = final_norm; sa.inv_freq = inv_freq;
    sa.eps = d.rms_eps; sa.scale = 1.0f / std::sqrt((float)d.head_dim);
    sa.ll = d1_ll;
    sa.err = d1_err;
    sa.xn = xn;
    d1_static = dev_alloc<d1::Static>(1);
    HIPCHK(hipMemcpy(d1_static, &sa, sizeof(sa), hipMemcpyHostToDevice));
    d1_state = 1;
    d1_why.clear();
    return true;
}

// One column through the persistent kernel, then the LM head GEMV and the argmax as in the chain.
// The kernel needs its blocks co-resident (one per CU; the LDS size allows no second one, checked in prepare_d1) but
// no grid barrier.  It is launched cooperatively; where the runtime refuses that (a second process on the device can
// find the cooperative-launch resources taken), as a plain launch of the same grid, which an otherwise idle device
// also places one block per CU.  Either way every wait in the kernel is bounded: a grid that is not all resident
// ends with the error word set, never a hang.  Returns false, with nothing enqueued, if both launches fail (the step
// is then marked as not applying and the caller runs the chain).
bool sp_engine::launch_d1(const sp_token &t, int flags) {
    d1::Step a{};
    a.tok = t;
    a.feed = (flags & SP_F_FEED) ? am_out : nullptr;
    d1_seq = (d1_seq + 1) & 0xFFFFFFu;
    if (d1_seq == 0) d1_seq = 1;
    a.seq = d1_seq;
    const d1::Static *sp = d1_static;
    void *args[] = {(void *)&sp, &a};
    hipError_t le = d1_plain ? hipErrorNotSupported
                             : hipLaunchCooperativeKernel(d1k->fn, dim3(d1g.nb), dim3(d1::NT), args, d1::SMEM_BYTES, stream);
    if (le != hipSuccess) {
        (void)hipGetLastError();
        d1_plain = true;
        le = hipLaunchKernel(d1k->fn, dim3(d1g.nb), dim3(d1::NT), args, d1::SMEM_BYTES, stream);
    }
    if (le != hipSuccess) {
        (void)hipGetLastError();
        d1_state = -1;
        d1_why = std::string("launch refused: ") + hipGetErrorString(le);
        return false;
    }
    return true;
}
bool sp_engine::run_d1(const sp_token &t, int flags) {
    if (!launch_d1(t, flags)) return false;
    const DevMat &hm = d.tied_head ? embed : head;
    launch_gemv(hm, EPI_STORE, xn, d.hidden, 1, logits, nullptr, d.vocab, nullptr, stream);
    if (flags & SP_F_ARGMAX) {
        hipLaunchKernelGGL(k_argmax_part, dim3(ARGMAX_BLOCKS, 1), dim3(256), 0, stream, logits, d.vocab, d.vocab, am_v, am_i);
        hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(64), 0, stream, am_v, am_i, am_out);
    }
    // the error word's read-back goes last: a copy between the kernel and the head would delay the head (the word
    // is checked only after a synchronisation)
    HIPCHK(hipMemcpyAsync(h_d1err, d1_err, sizeof(unsigned), hipMemcpyDeviceToHost, stream));
    HIPCHK(hipGetLastError());
    return true;
}

// After a synchronisation: a persistent step whose block gave up (a hand-off that never arrived) is reported once.
void sp_engine::check_d1_error() {
    if (!h_d1err || *(volatile unsigned *)h_d1err == 0) return;
    *(volatile unsigned *)h_d1err = 0;
    (void)hipMemsetAsync(d1_err, 0, sizeof(unsigned), stream);
    throw Fail{SP_EHIP, "persistent decode step: a block hand-off timed out (the step's results are invalid)"};
}

// ============================================================================================== C ABI
namespace {
int fail_engine(sp_engine *e, const Fail &f) {
    if (e) e->err = f.msg;
    g_err = f.msg;
    return f.code;
}
template <class F>
int guarded(sp_engine *e, F &&fn) {
    try {
        fn();
        return SP_OK;
    } catch (const Fail &f) {
        return fail_engine(e, f);
    } catch (const std::exception &ex) {
        return fail_engine(e, Fail{SP_EHIP, ex.what()});
    }
}
}  // namespace

extern "C" {

const char *sp_last_error(void) { return g_err.c_str(); }
const char *sp_engine_last_error(const sp_engine *e) { return e ? e->err.c_str() : g_err.c_str(); }

int sp_engine_create(const sp_model_desc *desc, sp_engine **out) {
    if (!out) { g_err = "out is NULL"; return SP_EINVAL; }
    *out = nullptr;
    sp_engine *e = new sp_engine();
    int rc = guarded(nullptr, [&] {
        require(desc != nullptr, SP_EINVAL, "desc is NULL");
        const sp_model_desc &d = *desc;
        require(d.n_layers > 0 && d.hidden > 0 && d.n_heads > 0 && d.n_kv_heads > 0 && d.vocab > 0 && d.intermediate > 0,
                SP_EINVAL, "model dimensions must be positive");
        require(d.n_heads % d.n_kv_heads == 0 && d.n_heads / d.n_kv_heads <= 8, SP_EINVAL,
                "n_heads must be a multiple of n_kv_heads with at most 8 query heads per kv head");
        require(d.head_dim == 64 || d.head_dim == 128, SP_EINVAL, "head_dim must be 64 or 128");
        require(d.weight_format == SP_FMT_F16 || d.weight_format == SP_FMT_Q8 || d.weight_format == SP_FMT_Q4, SP_EINVAL,
                "weight_format must be SP_FMT_F16, SP_FMT_Q8 or SP_FMT_Q4");
        require(d.max_tokens >= 1 && d.max_tokens <= 16 * GEMV_MAX_MT, SP_EINVAL, "max_tokens must be in [1, 64]");
        require(d.hidden % 128 == 0 && d.intermediate % 128 == 0 && (d.n_heads * d.head_dim) % 128 == 0, SP_EINVAL,
                "hidden, intermediate and heads*head_dim must be multiples of 128");
        require(d.inv_freq != nullptr, SP_EINVAL, "inv_freq is NULL");
        require(d.hidden <= NORM_PER_THREAD * NORM_THREADS, SP_EINVAL, "hidden must be <= 4096");
        e->d = d;
        e->d.inv_freq = nullptr;
        HIPCHK(hipGetDevice(&e->device));
        HIPCHK(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
        HIPCHK(hipStreamCreateWithFlags(&e->capture_stream, hipStreamNonBlocking));
        e->own_stream = true;
        e->layers.resize(d.n_layers);
        e->inv_freq = dev_alloc<float>(d.head_dim / 2);
        HIPCHK(hipMemcpy(e->inv_freq, d.inv_freq, d.head_dim / 2 * sizeof(float), hipMemcpyHostToDevice));
        e->alloc_activations();
    });
    if (rc != SP_OK) { e->free_all(); delete e; return rc; }
    *out = e;
    return SP_OK;
}

void sp_engine_destroy(sp_engine *e) {
    if (!e) return;
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    e->free_all();
    delete e;
}

int sp_engine_set_stream(sp_engine *e, void *s) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        HIPCHK(hipStreamSynchronize(e->stream));
        if (e->own_stream) HIPCHK(hipStreamDestroy(e->stream));
        e->drop_graphs();
        e->stream = (hipStream_t)s;
        e->own_stream = false;
    });
}

int sp_engine_load(sp_engine *e, int32_t kind, int32_t layer, int32_t fmt, int32_t rows, int32_t cols, const void *data,
                   const void *scales, const void *zeros) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        const sp_model_desc &d = e->d;
        const int Nqkv = (d.n_heads + 2 * d.n_kv_heads) * d.head_dim;
        auto vec = [&](float *&dst, int n) {
            require(fmt == SP_FMT_F32 && rows == 1 && cols == n, SP_EINVAL, "vector tensor must be fp32 [1][n] with the model's width");
            require(data != nullptr, SP_EINVAL, "data is NULL");
            dev_free(dst);
            dst = dev_alloc<float>(n, &e->weight_bytes);
            HIPCHK(hipMemcpy(dst, data, n * sizeof(float), hipMemcpyHostToDevice));
        };
        auto mat = [&](DevMat &dst, int want_rows, int want_cols, bool paired) {
            require(fmt == d.weight_format, SP_EINVAL, "matrix format differs from the model's weight_format");
            require(rows == want_rows && cols == want_cols, SP_EINVAL, "matrix shape does not match the model description");
            e->weight_bytes -= dst.bytes;
            dst.release();
            dst = upload_matrix(fmt, rows, cols, data, scales, zeros, paired);
            e->weight_bytes += dst.bytes;
        };
        const bool per_layer = kind >= SP_T_IN_NORM;
        if (per_layer) require(layer >= 0 && layer < d.n_layers, SP_EINVAL, "layer out of range");
        switch (kind) {
            case SP_T_EMBED: mat(e->embed, d.vocab, d.hidden, false); break;
            case SP_T_HEAD: require(!d.tied_head, SP_EINVAL, "the model has a tied head"); mat(e->head, d.vocab, d.hidden, false); break;
            case SP_T_FINAL_NORM: vec(e->final_norm, d.hidden); break;
            case SP_T_IN_NORM: vec(e->layers[layer].in_norm, d.hidden); break;
            case SP_T_POST_NORM: vec(e->layers[layer].post_norm, d.hidden); break;
            case SP_T_QKV: mat(e->layers[layer].qkv, Nqkv, d.hidden, false); break;
            case SP_T_QKV_BIAS: vec(e->layers[layer].qkv_b, Nqkv); break;
            case SP_T_O: mat(e->layers[layer].o, d.hidden, d.n_heads * d.head_dim, false); break;
            case SP_T_GATE_UP: mat(e->layers[layer].gate_up, 2 * d.intermediate, d.hidden, true); break;
            case SP_T_DOWN: mat(e->layers[layer].down, d.hidden, d.intermediate, false); break;
            default: throw Fail{SP_EINVAL, "unknown tensor kind"};
        }
        e->drop_graphs();
        e->d1_state = 0;
    });
}

namespace {
// A zeroed K/V pool for n_seq x n_slots in every layer (nothing of the engine's state changes; on failure the new
// allocations are released and the exception propagates).
void alloc_pool(const sp_engine *e, int n_seq, int n_slots, std::vector<f16 *> &k, std::vector<f16 *> &v, uint64_t &bytes) {
    k.assign(e->d.n_layers, nullptr);
    v.assign(e->d.n_layers, nullptr);
    bytes = 0;
    const size_t per = (size_t)n_seq * e->d.n_kv_heads * n_slots * e->d.head_dim;
    try {
        for (int l = 0; l < e->d.n_layers; ++l) {
            k[l] = dev_alloc<f16>(per, &bytes);
            v[l] = dev_alloc<f16>(per, &bytes);
            HIPCHK(hipMemsetAsync(k[l], 0, per * sizeof(f16), e->stream));
            HIPCHK(hipMemsetAsync(v[l], 0, per * sizeof(f16), e->stream));
        }
    } catch (...) {
        for (auto p : k) dev_free(p);
        for (auto p : v) dev_free(p);
        k.clear(); v.clear();
        throw;
    }
}

// Makes (k, v) the engine's pool: frees the old one, sizes the attention partials for n_slots and drops the recorded
// graphs (they hold the old addresses).  The stream must be idle.
void install_pool(sp_engine *e, int n_seq, int n_slots, std::vector<f16 *> &k, std::vector<f16 *> &v, uint64_t bytes) {
    for (auto p : e->kc) dev_free(p);
    for (auto p : e->vc) dev_free(p);
    e->kc.swap(k);
    e->vc.swap(v);
    k.clear(); v.clear();
    e->kv_bytes = bytes;
    dev_free(e->attn_part); e->attn_part = nullptr;
    e->n_seq = 0; e->n_slots = 0;
    if (!e->d_kl) e->d_kl = dev_alloc<f16 *>(e->d.n_layers);
    if (!e->d_vl) e->d_vl = dev_alloc<f16 *>(e->d.n_layers);
    HIPCHK(hipMemcpy(e->d_kl, e->kc.data(), e->d.n_layers * sizeof(f16 *), hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(e->d_vl, e->vc.data(), e->d.n_layers * sizeof(f16 *), hipMemcpyHostToDevice));
    e->max_nchunk = (n_slots + 64 + ATT_CH - 1) / ATT_CH;
    e->attn_part = dev_alloc<float>((size_t)e->maxT * e->d.n_heads * e->max_nchunk * part_floats(e->d.head_dim));
    e->n_seq = n_seq; e->n_slots = n_slots;
    e->drop_graphs();
    e->d1_state = 0;
}
}  // namespace

int sp_engine_kv_reserve(sp_engine *e, int32_t n_seq, int32_t n_slots) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        require(n_seq >= 1 && n_slots >= 1, SP_EINVAL, "n_seq and n_slots must be positive");
        require((n_slots + 64 + ATT_CH - 1) / ATT_CH <= ATT_MAX_CHUNKS, SP_EINVAL, "n_slots too large for the attention combine");
        HIPCHK(hipStreamSynchronize(e->stream));
        // the old pool goes first, so a re-reservation never needs both at once
        for (auto p : e->kc) dev_free(p);
        for (auto p : e->vc) dev_free(p);
        e->kc.clear(); e->vc.clear();
        e->kv_bytes = 0;
        e->n_seq = 0; e->n_slots = 0;
        std::vector<f16 *> k, v;
        uint64_t bytes = 0;
        alloc_pool(e, n_seq, n_slots, k, v, bytes);
        install_pool(e, n_seq, n_slots, k, v, bytes);
        HIPCHK(hipStreamSynchronize(e->stream));
    });
}

int sp_engine_kv_layer(sp_engine *e, int32_t layer, void **k_dev, void **v_dev) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        require(k_dev && v_dev, SP_EINVAL, "NULL pointer");
        require(e->n_seq > 0, SP_ESTATE, "KV cache not reserved");
        require(layer >= 0 && layer < (int)e->kc.size(), SP_EINVAL, "layer out of range");
        *k_dev = e->kc[layer];
        *v_dev = e->vc[layer];
    });
}

int sp_engine_kv_grow(sp_engine *e, int32_t n_seq, int32_t n_slots, int32_t n_keep, const int32_t *keep_seq,
                      const int32_t *keep_len) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        require(e->n_seq > 0, SP_ESTATE, "KV cache not reserved");
        require(n_seq >= e->n_seq && n_slots >= e->n_slots, SP_EINVAL, "a grown pool must not be smaller in either dimension");
        require((n_slots + 64 + ATT_CH - 1) / ATT_CH <= ATT_MAX_CHUNKS, SP_EINVAL, "n_slots too large for the attention combine");
        require(n_keep >= 0 && n_keep <= e->n_seq, SP_EINVAL, "n_keep must be in [0, n_seq of the current pool]");
        require(n_keep == 0 || (keep_seq && keep_len), SP_EINVAL, "keep arrays are NULL");
        std::vector<int> keep(3 * (size_t)std::max(n_keep, 1));
        std::vector<char> seen(e->n_seq, 0);
        int most = 0;
        for (int i = 0; i < n_keep; ++i) {
            require(keep_seq[i] >= 0 && keep_seq[i] < e->n_seq && !seen[keep_seq[i]], SP_EINVAL,
                    "kept sequences must be distinct indices of the current pool");
            require(keep_len[i] >= 0, SP_EINVAL, "kept lengths must be non-negative");
            seen[keep_seq[i]] = 1;
            const int np = std::min(keep_len[i], e->n_slots);     // the ring holds the last n_slots positions
            keep[3 * i] = keep_seq[i];
            keep[3 * i + 1] = keep_len[i] - np;
            keep[3 * i + 2] = np;
            most = std::max(most, np);
        }
        HIPCHK(hipStreamSynchronize(e->stream));
        std::vector<f16 *> k, v;
        uint64_t bytes = 0;
        alloc_pool(e, n_seq, n_slots, k, v, bytes);
        int *dkeep = nullptr;
        try {
            if (n_keep > 0 && most > 0) {
                dkeep = dev_alloc<int>(keep.size());
                HIPCHK(hipMemcpyAsync(dkeep, keep.data(), keep.size() * sizeof(int), hipMemcpyHostToDevice, e->stream));
                const int per = most * (e->d.head_dim / 8);
                const dim3 grid((per + 255) / 256 < 512 ? (per + 255) / 256 : 512, n_keep * e->d.n_kv_heads);
                for (int l = 0; l < e->d.n_layers; ++l)
                    hipLaunchKernelGGL(k_kv_regrid, grid, dim3(256), 0, e->stream, e->kc[l], e->vc[l], k[l], v[l], dkeep,
                                       e->d.n_kv_heads, e->d.head_dim, e->n_slots, n_slots);
                HIPCHK(hipGetLastError());
            }
            HIPCHK(hipStreamSynchronize(e->stream));
        } catch (...) {
            dev_free(dkeep);
            for (auto p : k) dev_free(p);
            for (auto p : v) dev_free(p);
            throw;
        }
        dev_free(dkeep);
        install_pool(e, n_seq, n_slots, k, v, bytes);
    });
}

int sp_engine_forward(sp_engine *e, int32_t n, const sp_token *toks, int32_t flags, float *logits_dev, int32_t *argmax_host) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        const sp_model_desc &d = e->d;
        require(n >= 1 && n <= e->maxT, SP_ECAPACITY, "column count must be in [1, max_tokens]");
        require(toks != nullptr, SP_EINVAL, "toks is NULL");
        require(e->n_seq > 0, SP_ESTATE, "KV cache not reserved");
        require(e->embed.w && e->final_norm && (d.tied_head || e->head.w), SP_ESTATE, "embedding / head / final norm not loaded");
        for (auto &l : e->layers)
            require(l.qkv.w && l.o.w && l.gate_up.w && l.down.w && l.qkv_b && l.in_norm && l.post_norm, SP_ESTATE,
                    "a layer's weights are not loaded");
        require(!(argmax_host && !(flags & SP_F_ARGMAX)), SP_EINVAL, "argmax_host needs SP_F_ARGMAX");
        require(!((flags & SP_F_ARGMAX) && !(flags & SP_F_LOGITS)), SP_EINVAL, "SP_F_ARGMAX needs SP_F_LOGITS");
        const bool feed = flags & SP_F_FEED, devcols = flags & SP_F_DEVCOLS;
        require(!(devcols && feed), SP_EINVAL, "SP_F_DEVCOLS and SP_F_FEED both name the tokens");
        require(!devcols || e->dev_tokens, SP_ESTATE, "SP_F_DEVCOLS needs sp_engine_set_device_columns");
        require(!feed || n <= e->argmax_cols, SP_ESTATE,
                "SP_F_FEED needs a previous SP_F_ARGMAX call over at least as many columns");
        e->check_columns(n, toks, feed || devcols);
        e->check_d1_error();
        const bool use_graph = flags & SP_F_GRAPH;
        const int sflags = flags & (SP_F_LOGITS | SP_F_ARGMAX | SP_F_UNFUSED | SP_F_FEED);
        // one plain decode column: the persistent step, where the shape and the pool allow it
        const sp_token &t0 = toks[0];
        if (n == 1 && (flags & SP_F_LOGITS) && !(flags & (SP_F_UNFUSED | SP_F_CHAIN | SP_F_DEVCOLS)) && t0.tree_count == 0 &&
            t0.ctx_hi >= t0.ctx_lo && t0.slot == t0.ctx_hi % e->n_slots && e->prepare_d1() && e->run_d1(t0, sflags)) {
            e->last_path = 1;
            e->last_dispatches = (sflags & SP_F_ARGMAX) ? 4 : 2;
            if (sflags & SP_F_ARGMAX) e->argmax_cols = 1;
            if (logits_dev)
                HIPCHK(hipMemcpyAsync(logits_dev, e->logits, (size_t)d.vocab * sizeof(float), hipMemcpyDeviceToDevice, e->stream));
            if (argmax_host) {
                HIPCHK(hipMemcpyAsync(e->h_ids, e->am_out, sizeof(int32_t), hipMemcpyDeviceToHost, e->stream));
                HIPCHK(hipStreamSynchronize(e->stream));
                e->check_d1_error();
                std::memcpy(argmax_host, e->h_ids, sizeof(int32_t));
            }
            return;
        }
        e->last_path = 0;
        const sp_engine::AttnPlan ap = e->plan_attention(n, toks, use_graph);
        e->upload(n, toks, ap);
        if (devcols) {
            hipLaunchKernelGGL(k_patch_columns, dim3((n + 63) / 64), dim3(64), 0, e->stream, e->dtoks, n, e->dev_tokens,
                               e->dev_masks, d.vocab);
            HIPCHK(hipGetLastError());
        }
        if (use_graph) {
            // The step's three parts (the embedding and layer 0, layers 1-4, the rest) are recorded as graphs once per
            // (columns, flags, attention plan); their kernel nodes are the reported dispatch count.  The first part
            // always runs as plain launches (the GPU starts after the first of them, not after a graph launch's
            // set-up).  The others run as plain launches too when the host runs ahead of the GPU -- a fed greedy loop,
            // or several columns, whose kernels each take longer than their launch -- because a replayed graph costs
            // the GPU more per kernel than in-order launches (A/B of whole steps: fed bs1 0.974 -> 0.968 ms/token, tree
            // pass 1.499 -> 1.490 ms, 16-request 0.5B burst 18.0k -> 18.2k tok/s, bs16 1.442 -> 1.430 ms); a single
            // column whose caller waits for every token replays them (plain launches there leave the GPU waiting for
            // the host: 0.995 -> 1.02-1.05 ms per token).
            const bool plain = (sflags & SP_F_FEED) || n > 1;
            const int L = d.n_layers;
            const int cuts[4] = {0, std::min(1, L), std::min(5, L), L};
            const int plan_code = ap.mq ? (ap.mq_ch == 128 ? 1 << 20 : 0) + ap.ngroups * 1024 + ap.splits
                                        : (ap.dec ? (ap.dec_direct ? -3 : -2) - 8 * ap.dec_kpb : (ap.rope_fused ? -4 : -1));
            int total = 0;
            for (int part = 0; part < 3; ++part) {
                if (cuts[part] >= cuts[part + 1]) continue;      // empty (short models); the head ran in its part
                auto key = std::make_tuple(n, sflags | (part << 8), plan_code);
                const bool replay = part > 0 && !plain;
                if (!e->graph_kernels.count(key) || (replay && !e->graphs.count(key))) {
                    // record on the private stream (the caller's may be the null stream, which cannot capture)
                    hipGraph_t g;
                    hipStream_t run_stream = e->stream;
                    e->stream = e->capture_stream;
                    HIPCHK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
                    try {
                        e->step(n, sflags, ap, cuts[part], cuts[part + 1]);
                    } catch (...) {
                        hipGraph_t dummy;
                        (void)hipStreamEndCapture(e->stream, &dummy);
                        e->stream = run_stream;
                        throw;
                    }
                    hipError_t ce = hipStreamEndCapture(e->stream, &g);
                    e->stream = run_stream;
                    HIPCHK(ce);
                    size_t nn = 0;
                    HIPCHK(hipGraphGetNodes(g, nullptr, &nn));
                    std::vector<hipGraphNode_t> nodes(nn);
                    if (nn) HIPCHK(hipGraphGetNodes(g, nodes.data(), &nn));
                    int kernels = 0;
                    for (auto nd : nodes) {
                        hipGraphNodeType ty;
                        HIPCHK(hipGraphNodeGetType(nd, &ty));
                        kernels += ty == hipGraphNodeTypeKernel;
                    }
                    if (replay) {               // instantiated only for the parts that are replayed
                        hipGraphExec_t ge;
                        hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
                        (void)hipGraphDestroy(g);
                        HIPCHK(ie);
                        e->graphs[key] = ge;
                    } else {
                        (void)hipGraphDestroy(g);
                    }
                    e->graph_kernels[key] = kernels;
                }
                if (replay) HIPCHK(hipGraphLaunch(e->graphs[key], e->stream));
                else e->step(n, sflags, ap, cuts[part], cuts[part + 1]);
                total += e->graph_kernels[key];
            }
            e->last_dispatches = total;
        } else {
            e->step(n, sflags, ap, 0, d.n_layers);
            e->last_dispatches = -1;
        }
        if (sflags & SP_F_ARGMAX) e->argmax_cols = n;
        if (logits_dev && (flags & SP_F_LOGITS))
            HIPCHK(hipMemcpyAsync(logits_dev, e->logits, (size_t)n * d.vocab * sizeof(float), hipMemcpyDeviceToDevice, e->stream));
        if (argmax_host) {
            // through pinned memory: a device-to-host copy into pageable memory is staged by the runtime
            HIPCHK(hipMemcpyAsync(e->h_ids, e->am_out, n * sizeof(int32_t), hipMemcpyDeviceToHost, e->stream));
            HIPCHK(hipStreamSynchronize(e->stream));
            std::memcpy(argmax_host, e->h_ids, n * sizeof(int32_t));
        }
    });
}

int sp_engine_last_path(const sp_engine *e) { return e ? e->last_path : -1; }

int sp_engine_set_device_columns(sp_engine *e, const int32_t *tokens_dev, const uint64_t *masks_dev) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        require(tokens_dev || !masks_dev, SP_EINVAL, "masks need tokens");
        e->dev_tokens = tokens_dev;
        e->dev_masks = masks_dev;
    });
}

int sp_engine_last_dispatches(const sp_engine *e) { return e ? e->last_dispatches : -1; }


int sp_engine_logits(sp_engine *e, float **logits_dev) {
    if (!e || !logits_dev) { g_err = "NULL argument"; return SP_EINVAL; }
    *logits_dev = e->logits;
    return SP_OK;
}

int sp_engine_kv_move(sp_engine *e, int32_t seq, int32_t n, const int32_t *src, const int32_t *dst) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        require(e->n_seq > 0, SP_ESTATE, "KV cache not reserved");
        require(seq >= 0 && seq < e->n_seq, SP_EINVAL, "sequence index out of range");
        require(n >= 0 && n <= 64, SP_EINVAL, "at most 64 slot moves per call");
        if (n == 0) return;
        require(src && dst, SP_EINVAL, "slot arrays are NULL");
        std::vector<int> buf(2 * n);
        for (int i = 0; i < n; ++i) {
            require(src[i] >= 0 && src[i] < e->n_slots && dst[i] >= 0 && dst[i] < e->n_slots, SP_EINVAL, "slot out of range");
            buf[i] = src[i]; buf[n + i] = dst[i];
        }
        HIPCHK(hipMemcpyAsync(e->d_move, buf.data(), 2 * n * sizeof(int), hipMemcpyHostToDevice, e->stream));
        hipLaunchKernelGGL(k_kv_move, dim3(e->d.n_layers * e->d.n_kv_heads), dim3(128), 0, e->stream, e->d_kl, e->d_vl, seq,
                           e->d.n_kv_heads, e->n_slots, e->d.head_dim, e->d_move, e->d_move + n, n);
        HIPCHK(hipGetLastError());
        HIPCHK(hipStreamSynchronize(e->stream));
    });
}

int sp_engine_copy_ids(sp_engine *e, int32_t n, int32_t *host) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        require(host != nullptr, SP_EINVAL, "host is NULL");
        require(n >= 1 && n <= e->argmax_cols, SP_EINVAL, "n must be in [1, columns of the last SP_F_ARGMAX call]");
        HIPCHK(hipMemcpyAsync(host, e->am_out, n * sizeof(int32_t), hipMemcpyDeviceToHost, e->stream));
    });
}

int sp_engine_sync(sp_engine *e) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        HIPCHK(hipStreamSynchronize(e->stream));
        e->check_d1_error();
    });
}

int sp_persistent_geometry(const sp_model_desc *desc, int32_t n_slots, int32_t n_blocks, int32_t *info) {
    if (!desc || !info) { g_err = "NULL argument"; return SP_EINVAL; }
    d1::Geom g;
    const char *why = "";
    if (!d1::make_geom(*desc, n_slots, n_blocks, g, &why)) { g_err = why; return SP_EINVAL; }
    const D1Kernel *k = find_d1_kernel(g);
    if (!k) { g_err = "no instantiation for this shape"; return SP_EINVAL; }
    if (!d1::check_geom(g, k->th, k->t5, &why)) { g_err = why; return SP_EINVAL; }
    const int32_t v[12] = {g.NQ, g.NKV * g.CM, g.NH, g.NO, g.NU, g.ND, g.nu_max, g.B2, g.B3, g.B5,
                           (int32_t)g.words, (int32_t)d1::SMEM_BYTES};
    std::memcpy(info, v, sizeof(v));
    return SP_OK;
}

int sp_engine_persistent_status(sp_engine *e, char *why, int32_t why_len) {
    if (!e) { g_err = "engine is NULL"; return -1; }
    int ok = 0;
    int rc = guarded(e, [&] { ok = e->n_seq > 0 && e->prepare_d1() ? 1 : 0; });
    if (rc != SP_OK) return -1;
    if (why && why_len > 0) {
        std::strncpy(why, e->d1_why.c_str(), (size_t)why_len - 1);
        why[why_len - 1] = 0;
    }
    return ok;
}

int sp_engine_time_gemv(sp_engine *e, int32_t kind, int32_t layer, int32_t n_cols, int32_t iters, float *avg_us,
                        uint64_t *bytes) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        const sp_model_desc &d = e->d;
        require(avg_us && bytes, SP_EINVAL, "NULL output");
        require(n_cols >= 1 && n_cols <= e->maxT && iters >= 1, SP_EINVAL, "n_cols must be in [1, max_tokens], iters >= 1");
        const bool per_layer = kind == SP_T_QKV || kind == SP_T_O || kind == SP_T_GATE_UP || kind == SP_T_DOWN;
        require(!per_layer || (layer >= -1 && layer < d.n_layers), SP_EINVAL, "layer out of range");
        const int H = d.hidden, I = d.intermediate, NHD = d.n_heads * d.head_dim;
        hipStream_t st = e->stream;
        // layer -1: launch i uses layer i mod n_layers, so the matrices stream from HBM as in a decode step
        // instead of staying cached between launches
        int cur = layer < 0 ? 0 : layer;
        auto next_layer = [&] { if (layer < 0) cur = (cur + 1) % d.n_layers; };
        const int tm = n_cols > 1 ? (n_cols + 15) / 16 : 0;     // activation layout of a step with n_cols columns
        std::function<void()> launch;
        const DevMat *m = nullptr;
        switch (kind) {
            case SP_T_QKV: m = &e->layers[cur].qkv;
                launch = [&] { launch_gemv(e->layers[cur].qkv, EPI_STORE, e->xn, H, n_cols, e->qkv, nullptr, e->Nqkv,
                                           e->layers[cur].qkv_b, st, e->gpart, e->gpart_stride, PRO_NONE, nullptr, 0, 0,
                                           tm, 0, e->xn_lo); next_layer(); };
                break;
            case SP_T_O: m = &e->layers[cur].o;
                launch = [&] { launch_gemv(e->layers[cur].o, EPI_RESID, e->attn, NHD, n_cols, e->x, nullptr, H, nullptr,
                                           st, e->gpart, e->gpart_stride, PRO_NONE, nullptr, 0, 0, tm); next_layer(); };
                break;
            case SP_T_GATE_UP: m = &e->layers[cur].gate_up;
                launch = [&] { launch_gemv(e->layers[cur].gate_up, EPI_SILU, e->xn, H, n_cols, nullptr, e->act, I,
                                           nullptr, st, nullptr, 0, PRO_NONE, nullptr, 0, 0, tm, tm,
                                           n_cols == 1 ? e->xn_lo : nullptr, n_cols == 1 ? e->act_lo : nullptr);
                               next_layer(); };
                break;
            case SP_T_DOWN: m = &e->layers[cur].down;
                launch = [&] { launch_gemv(e->layers[cur].down, EPI_RESID, e->act, I, n_cols, e->x, nullptr, H, nullptr,
                                           st, e->gpart, e->gpart_stride, PRO_NONE, nullptr, 0, 0, tm, 0,
                                           n_cols == 1 ? e->act_lo : nullptr); next_layer(); };
                break;
            case SP_T_HEAD: case SP_T_EMBED: m = d.tied_head || kind == SP_T_EMBED ? &e->embed : &e->head;
                launch = [&] { launch_gemv(*m, EPI_STORE, e->xn, H, n_cols, e->logits, nullptr, d.vocab, nullptr, st,
                                           nullptr, 0, PRO_NONE, nullptr, 0, 0, tm); };
                break;
            default: throw Fail{SP_EINVAL, "kind must name a matrix"};
        }
        // back-to-back launches between one event pair: the command processor overlaps each dispatch with the
        // previous kernel's tail, so the average is the launch duration seen in a stream of GEMVs
        hipEvent_t a, b;
        HIPCHK(hipEventCreate(&a));
        HIPCHK(hipEventCreate(&b));
        launch();                       // warm-up
        HIPCHK(hipEventRecord(a, st));
        for (int i = 0; i < iters; ++i) launch();
        HIPCHK(hipEventRecord(b, st));
        HIPCHK(hipEventSynchronize(b));
        float ms = 0.f;
        HIPCHK(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        HIPCHK(hipGetLastError());
        *avg_us = ms * 1000.f / iters;
        *bytes = m->bytes;
    });
}

int sp_engine_time_persistent(sp_engine *e, const sp_token *tok, int32_t iters, float *avg_us, uint64_t *bytes) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        const sp_model_desc &d = e->d;
        require(avg_us && bytes && tok, SP_EINVAL, "NULL argument");
        require(iters >= 1, SP_EINVAL, "iters must be >= 1");
        require(e->n_seq > 0, SP_ESTATE, "KV cache not reserved");
        e->check_columns(1, tok, false);
        const sp_token &t = *tok;
        require(t.tree_count == 0 && t.ctx_hi >= t.ctx_lo && t.slot == t.ctx_hi % e->n_slots, SP_EINVAL,
                "not a plain decode column");
        require(e->prepare_d1(), SP_ESTATE, "the persistent step does not apply: " + e->d1_why);
        hipEvent_t a, b;
        HIPCHK(hipEventCreate(&a));
        HIPCHK(hipEventCreate(&b));
        require(e->launch_d1(t, 0), SP_ESTATE, "persistent launch refused: " + e->d1_why);      // warm-up
        HIPCHK(hipEventRecord(a, e->stream));
        for (int i = 0; i < iters; ++i) require(e->launch_d1(t, 0), SP_ESTATE, "persistent launch refused: " + e->d1_why);
        HIPCHK(hipEventRecord(b, e->stream));
        HIPCHK(hipEventSynchronize(b));
        float ms = 0.f;
        HIPCHK(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        HIPCHK(hipMemcpy(e->h_d1err, e->d1_err, sizeof(unsigned), hipMemcpyDeviceToHost));
        e->check_d1_error();
        *avg_us = ms * 1000.f / iters;
        // algorithmic bytes: every layer's packed weights (codes + scales), norms and qkv bias, the visible K / V
        // of each kv head (the new key and value are written, the others read), and the embedding row
        uint64_t nb = 0;
        const int vis = t.ctx_hi - t.ctx_lo + 1;
        for (const auto &ly : e->layers) {
            nb += ly.qkv.bytes + ly.o.bytes + ly.gate_up.bytes + ly.down.bytes;
            nb += (uint64_t)(2 * d.hidden + e->Nqkv) * sizeof(float);
            nb += (uint64_t)2 * d.n_kv_heads * vis * d.head_dim * sizeof(f16);
        }
        nb += (uint64_t)d.hidden * (e->embed.bytes / ((uint64_t)d.vocab * d.hidden) + 1);
        *bytes = nb;
    });
}

int sp_engine_time_attention(sp_engine *e, int32_t n, const sp_token *toks, int32_t iters, float *avg_us,
                             uint64_t *bytes) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        const sp_model_desc &d = e->d;
        require(avg_us && bytes && toks, SP_EINVAL, "NULL argument");
        require(n >= 1 && n <= e->maxT && iters >= 1, SP_EINVAL, "n must be in [1, max_tokens], iters >= 1");
        require(e->n_seq > 0, SP_ESTATE, "KV cache not reserved");
        e->check_columns(n, toks, true);
        sp_engine::AttnPlan ap = e->plan_attention(n, toks, false);
        ap.rope_fused = false;
        e->upload(n, toks, ap);
        HIPCHK(hipMemsetAsync(e->q, 0, (size_t)e->maxT * d.n_heads * d.head_dim * sizeof(float), e->stream));
        const int mtp = n > 1 ? (n + 15) / 16 : 0;
        int cur = 0;
        auto launch = [&] { e->launch_attention(cur, n, ap, mtp, e->stream); cur = (cur + 1) % d.n_layers; };
        hipEvent_t a, b;
        HIPCHK(hipEventCreate(&a));
        HIPCHK(hipEventCreate(&b));
        launch();
        HIPCHK(hipEventRecord(a, e->stream));
        for (int i = 0; i < iters; ++i) launch();
        HIPCHK(hipEventRecord(b, e->stream));
        HIPCHK(hipEventSynchronize(b));
        float ms = 0.f;
        HIPCHK(hipEventElapsedTime(&ms, a, b));
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        HIPCHK(hipGetLastError());
        uint64_t keys = 0;
        for (int i = 0; i < n; ++i)
            keys += (uint64_t)(toks[i].ctx_hi >= toks[i].ctx_lo ? toks[i].ctx_hi - toks[i].ctx_lo + 1 : 0) + toks[i].tree_count;
        // every visible key's K and V (fp16) of its kv head; a multi-query group reads its shared keys once
        if (ap.mq) {
            keys = 0;
            for (const AttnGroup &g : ap.groups) keys += (uint64_t)g.nlin + g.tree_count;
        }
        *avg_us = ms * 1000.f / iters;
        *bytes = keys * d.n_kv_heads * d.head_dim * 2 * 2;
    });
}

int sp_engine_kv_fill(sp_engine *e, int32_t seq, int32_t first_slot, int32_t n, uint64_t seed, float scale) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    return guarded(e, [&] {
        require(e->n_seq > 0, SP_ESTATE, "KV cache not reserved");
        require(seq >= 0 && seq < e->n_seq, SP_EINVAL, "sequence index out of range");
        require(first_slot >= 0 && n >= 0 && first_slot + n <= e->n_slots, SP_EINVAL, "slot range out of bounds");
        if (n == 0) return;
        hipLaunchKernelGGL(k_kv_fill, dim3(1024, e->d.n_layers), dim3(256), 0, e->stream, e->d_kl, e->d_vl, seq,
                           e->d.n_kv_heads, e->n_slots, e->d.head_dim, first_slot, n, (uint64_t)seed, scale);
        HIPCHK(hipGetLastError());
        HIPCHK(hipStreamSynchronize(e->stream));
    });
}

int sp_engine_bytes(const sp_engine *e, uint64_t *wb, uint64_t *kb) {
    if (!e) { g_err = "engine is NULL"; return SP_EINVAL; }
    if (wb) *wb = e->weight_bytes;
    if (kb) *kb = e->kv_bytes;
    return SP_OK;
}

int sp_tree_columns(int32_t n, const int32_t *token, const int32_t *depth, const uint64_t *mask, int32_t seq,
                    int64_t length, int32_t n_slots, int32_t window, sp_token *out) {
    if (n < 1 || n > 64) { g_err = "a tree pass has 1 to 64 nodes"; return SP_EINVAL; }
    if (!token || !depth || !mask || !out) { g_err = "tree column arrays are NULL"; return SP_EINVAL; }
    if (n_slots < 1 || window < 0 || seq < 0 || length < 0 || length + 64 + 64 > INT32_MAX) {
        g_err = "bad slot count, window, sequence or cache length";
        return SP_EINVAL;
    }
    const int32_t P = (int32_t)length, base = (int32_t)(length % n_slots);
    for (int i = 0; i < n; ++i) {
        if (depth[i] < 0 || depth[i] >= 64) { g_err = "tree depth out of range"; return SP_EINVAL; }
        sp_token &c = out[i];
        c.token = token[i];
        c.seq = seq;
        c.pos = P + depth[i];
        c.slot = (int32_t)((base + i) % n_slots);
        c.ctx_lo = window > 0 ? std::max(0, c.pos - window + 1) : 0;
        c.ctx_hi = P - 1;
        c.tree_base = base;
        c.tree_count = n;
        c.tree_mask = mask[i];
    }
    return SP_OK;
}

// ---------------------------------------------------------------------------------------------- standalone ops
size_t sp_op_argmax_workspace(int32_t rows, int32_t cols) {
    (void)cols;
    return rows <= 0 ? 0 : (size_t)rows * ARGMAX_BLOCKS * (sizeof(float) + sizeof(int));
}

}  // extern "C"

namespace {
// Both argmax entry points: ARGMAX_BLOCKS partial (value, index) pairs per row in `ws` (fp32 values of every row,
// then int32 indices), then one wave per row merges them.  Every partial is written before it is read, so `ws` needs
// no clearing.
void launch_argmax(const float *logits, int rows, int cols, int *out, void *ws, hipStream_t st) {
    float *pv = (float *)ws;
    int *pi = (int *)(pv + (size_t)rows * ARGMAX_BLOCKS);
    hipLaunchKernelGGL(k_argmax_part, dim3(ARGMAX_BLOCKS, rows), dim3(256), 0, st, logits, cols, cols, pv, pi);
    hipLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(64), 0, st, pv, pi, out);
    HIPCHK(hipGetLastError());
}

// The partials of sp_op_argmax_noalloc live in this array of the library's own, so that entry point allocates
// nothing.  In host code `scratch` names a host-side stand-in, not device memory: kernels get the device address that
// hipGetSymbolAddress returns, looked up once per device with that device current (each GPU holds its own copy at
// its own address until the process ends).
constexpr int NOALLOC_ARGMAX_MAX_ROWS = 512;
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)NOALLOC_ARGMAX_MAX_ROWS * ARGMAX_BLOCKS * (sizeof(float) + sizeof(int));
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
std::map<int, void *> g_scratch_of;      // device ordinal -> device address of `scratch` there

void *scratch_on_current_device() {
    int dev = 0;
    HIPCHK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch_of.find(dev);
    if (it != g_scratch_of.end()) return it->second;
    void *ptr = nullptr;
    HIPCHK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    require(ptr != nullptr, SP_EHIP, "hipGetSymbolAddress returned no address for the argmax scratch array");
    g_scratch_of.emplace(dev, ptr);
    return ptr;
}
}  // namespace

extern "C" {

int sp_op_argmax(const float *logits_dev, int32_t rows, int32_t cols, int32_t *out_dev, void *ws, void *stream) {
    return guarded(nullptr, [&] {
        require(logits_dev && out_dev && ws, SP_EINVAL, "NULL pointer");
        require(rows >= 1 && rows <= 65535 && cols >= 1, SP_EINVAL, "rows must be in [1, 65535] and cols positive");
        launch_argmax(logits_dev, rows, cols, out_dev, ws, (hipStream_t)stream);
    });
}

int sp_op_argmax_noalloc(const float *logits_dev, int32_t rows, int32_t cols, int32_t *out_dev, void *stream) {
    return guarded(nullptr, [&] {
        require(logits_dev && out_dev, SP_EINVAL, "NULL pointer");
        require(cols >= 1, SP_EINVAL, "cols must be positive");
        require(rows >= 1 && rows <= NOALLOC_ARGMAX_MAX_ROWS, SP_EINVAL,
                "rows must be in [1, 512]: the allocation-free argmax keeps the partials of at most 512 rows");
        launch_argmax(logits_dev, rows, cols, out_dev, scratch_on_current_device(), (hipStream_t)stream);
    });
}

}  // extern "C"

struct sp_weight {
    DevMat m;
};

extern "C" {

int sp_weight_create(int32_t fmt, int32_t rows, int32_t cols, const void *data, const void *scales, const void *zeros,
                     sp_weight **out) {
    if (!out) { g_err = "out is NULL"; return SP_EINVAL; }
    *out = nullptr;
    sp_weight *w = new sp_weight();
    int rc = guarded(nullptr, [&] {
        require(fmt == SP_FMT_F16 || fmt == SP_FMT_Q8 || fmt == SP_FMT_Q4, SP_EINVAL, "fmt must be F16, Q8 or Q4");
        w->m = upload_matrix(fmt, rows, cols, data, scales, zeros, false);
    });
    if (rc != SP_OK) { delete w; return rc; }
    *out = w;
    return SP_OK;
}

void sp_weight_destroy(sp_weight *w) {
    if (!w) return;
    w->m.release();
    delete w;
}

uint64_t sp_weight_bytes(const sp_weight *w) { return w ? w->m.bytes : 0; }

int sp_pack_matrix(int32_t fmt, int32_t rows, int32_t cols, const void *data, const void *scales, const void *zeros,
                   int32_t pair_halves, void *out_codes, uint64_t *codes_bytes, void *out_side, uint64_t *side_bytes) {
    return guarded(nullptr, [&] {
        require(codes_bytes && side_bytes, SP_EINVAL, "size outputs are NULL");
        sp::Packed p;
        try {
            p = sp::pack_matrix(fmt, rows, cols, data, scales, zeros, pair_halves != 0);
        } catch (const std::invalid_argument &ex) {
            throw Fail{SP_EINVAL, ex.what()};
        }
        *codes_bytes = p.codes.size();
        *side_bytes = p.sz.size() * 2;
        if (out_codes) std::memcpy(out_codes, p.codes.data(), p.codes.size());
        if (out_side && !p.sz.empty()) std::memcpy(out_side, p.sz.data(), p.sz.size() * 2);
    });
}

size_t sp_op_gemv_workspace(const sp_weight *w, int32_t m_cols) {
    (void)w; (void)m_cols;
    return 0;
}

int sp_op_gemv(const sp_weight *w, const void *x_dev, int32_t m_cols, float *y_dev, void *ws, void *stream) {
    (void)ws;
    return guarded(nullptr, [&] {
        require(w && x_dev && y_dev, SP_EINVAL, "NULL pointer");
        require(m_cols >= 1 && m_cols <= 16 * GEMV_MAX_MT, SP_EINVAL, "m_cols must be in [1, 64]");
        launch_gemv(w->m, EPI_STORE, (const f16 *)x_dev, w->m.cols, m_cols, y_dev, nullptr, w->m.rows, nullptr,
                    (hipStream_t)stream);
        HIPCHK(hipGetLastError());
    });
}

}  // extern "C"

// Per-device scratch of the sampling and acceptance entry points: created on a device's first call, kept until
// sp_library_release (or the process end); each map is guarded by its mutex.
namespace lib_scratch {
struct Smp { float *pmax; double *csum; };
struct Fm { FmHist *hist; FmState *st; };
struct Acc { unsigned long long *xbuf; unsigned *err; int32_t *host; };
struct Stage { unsigned char *buf = nullptr; size_t cap = 0; hipEvent_t done = nullptr; bool used = false; };
std::map<int, Smp> smp;
std::map<int, Fm> fm;
std::map<int, Acc> acc;
std::map<int, Stage> stage;
std::mutex smp_mu, fm_mu, acc_mu, stage_mu;
}  // namespace lib_scratch

extern "C" {

int sp_op_sample(const float *logits_dev, int32_t vocab, int32_t ld, const int32_t *row_dev, const double *u_dev,
                 int32_t n, double temperature, int32_t *out_dev, void *stream) {
    return guarded(nullptr, [&] {
        require(logits_dev && row_dev && u_dev && out_dev, SP_EINVAL, "NULL pointer");
        require(vocab >= 1 && ld >= vocab && n >= 1 && n <= 65535, SP_EINVAL, "bad sizes");
        require(temperature > 0.0, SP_EINVAL, "temperature must be positive");
        hipStream_t st = (hipStream_t)stream;
        // partial maxima and chunk sums of SMP_BATCH draws, one set per device (calls on one device must not overlap)
        constexpr int SMP_BATCH = 512;
        int dev = 0;
        HIPCHK(hipGetDevice(&dev));
        lib_scratch::Smp sc;
        {
            std::lock_guard<std::mutex> lock(lib_scratch::smp_mu);
            auto it = lib_scratch::smp.find(dev);
            if (it == lib_scratch::smp.end())
                it = lib_scratch::smp.emplace(dev, lib_scratch::Smp{dev_alloc<float>((size_t)SMP_BATCH * SMX_BLOCKS),
                                                                    dev_alloc<double>((size_t)SMP_BATCH * SMP_THREADS)})
                         .first;
            sc = it->second;
        }
        const double invT = 1.0 / temperature;
        for (int r0 = 0; r0 < n; r0 += SMP_BATCH) {
            const int nr = std::min(SMP_BATCH, n - r0);
            hipLaunchKernelGGL(k_smp_max, dim3(SMX_BLOCKS, nr), dim3(SMS_T), 0, st, logits_dev, vocab, ld, row_dev + r0,
                               sc.pmax);
            hipLaunchKernelGGL(k_smp_sum, dim3(SMP_THREADS / SMS_CPB, nr), dim3(SMS_T), 0, st, logits_dev, vocab, ld,
                               row_dev + r0, invT, (const float *)sc.pmax, sc.csum);
            hipLaunchKernelGGL(k_smp_draw, dim3(nr), dim3(SMS_T), 0, st, logits_dev, vocab, ld, row_dev + r0, u_dev + r0,
                               invT, (const float *)sc.pmax, (const double *)sc.csum, out_dev + r0);
            HIPCHK(hipGetLastError());
        }
    });
}

int sp_op_sample_filtered(const float *logits_dev, int32_t vocab, int32_t ld, const int32_t *row_dev,
                          const double *u_dev, int32_t n, double temperature, int32_t top_k, double top_p,
                          int32_t *out_dev, void *stream) {
    return guarded(nullptr, [&] {
        require(logits_dev && row_dev && u_dev && out_dev, SP_EINVAL, "NULL pointer");
        require(vocab >= 1 && ld >= vocab && n >= 1 && n <= 65535, SP_EINVAL, "bad sizes");
        require(temperature > 0.0, SP_EINVAL, "temperature must be positive");
        require(top_p > 0.0, SP_EINVAL, "top_p must be positive");
        hipStream_t st = (hipStream_t)stream;
        // histograms and per-row state for FM_ROWS draws, one set per device (calls on one device must not overlap)
        int dev = 0;
        HIPCHK(hipGetDevice(&dev));
        lib_scratch::Fm sc;
        {
            std::lock_guard<std::mutex> lock(lib_scratch::fm_mu);
            auto it = lib_scratch::fm.find(dev);
            if (it == lib_scratch::fm.end())
                it = lib_scratch::fm.emplace(dev, lib_scratch::Fm{dev_alloc<FmHist>((size_t)FM_ROWS * FM_NLEV),
                                                                  dev_alloc<FmState>(FM_ROWS)}).first;
            sc = it->second;
        }
        const int nb = (vocab + FM_SPAN - 1) / FM_SPAN;
        const bool topk = top_k > 0 && top_k < vocab;
        for (int r0 = 0; r0 < n; r0 += FM_ROWS) {
            const int nr = std::min(FM_ROWS, n - r0);
            const FmArgs a{logits_dev, vocab, ld, row_dev, u_dev, (float)temperature, top_k, top_p, out_dev, sc.hist,
                           sc.st, r0};
            const dim3 grid(nb, nr), block(FS_THREADS);
            hipLaunchKernelGGL(k_fm_init, dim3(nr), dim3(256), 0, st, a);
            hipLaunchKernelGGL(k_fm_max, grid, block, 0, st, a);
            if (topk)
                for (int j = 0; j < 4; ++j) hipLaunchKernelGGL(k_fm_topk, grid, block, 0, st, a, j);
            hipLaunchKernelGGL(k_fm_h1, grid, block, 0, st, a);
            if (top_p < 1.0)
                for (int j = 0; j < 3; ++j) hipLaunchKernelGGL(k_fm_select<false>, grid, block, 0, st, a, j);
            for (int j = 0; j < 3; ++j) hipLaunchKernelGGL(k_fm_select<true>, grid, block, 0, st, a, j);
            hipLaunchKernelGGL(k_fm_finish, dim3(nr), block, 0, st, a);
            HIPCHK(hipGetLastError());
        }
    });
}

}  // extern "C"

// The acceptance walk over device-readable tree arrays (device memory, or the library's pinned staging for the
// host-array entry point).  `staged` (may be NULL): an event recorded after the launch, which the host-array entry
// waits on before it refills its staging.
static void accept_tree_run(const float *p_logits_dev, const float *q_logits_dev, int32_t vocab, int32_t ld,
                            int32_t n_nodes, const int32_t *token, const int32_t *trial_start, const int32_t *n_trials,
                            const int32_t *trials, int32_t n_trials_total, const double *u, int32_t n_u,
                            double temperature, int32_t max_depth, int32_t *out_dev, hipStream_t st, int32_t *out_host,
                            hipEvent_t staged, const int32_t *q_row = nullptr, int32_t n_q_rows = 0) {
    {
        require(p_logits_dev && q_logits_dev && token && trial_start && n_trials && trials && u && out_dev, SP_EINVAL,
                "NULL pointer");
        require(n_trials_total >= 0 && n_trials_total <= ACC_MAX_TRIALS, SP_EINVAL, "n_trials_total must be in [0, 1024]");
        require(vocab >= 1 && vocab <= ACC_NB * ACC_T * ACC_PER && ld >= vocab, SP_EINVAL, "bad vocab / ld");
        require(n_nodes >= 1 && n_nodes <= ACC_MAX_NODES, SP_EINVAL, "n_nodes must be in [1, 64]");
        require(max_depth >= 1 && max_depth <= 63, SP_EINVAL, "max_depth must be in [1, 63]");
        require(n_u >= 1, SP_EINVAL, "need at least one uniform");
        require(temperature > 0.0, SP_EINVAL, "temperature must be positive");
        // the kernel checks every node / trial / token index it follows before using it (err = 2 if one is bad)
        // exchange words and the error word in device memory, and a pinned host block the kernel writes its result
        // and completion tags into, one set per device; tags never repeat within 2^20 launches, so nothing needs
        // clearing between launches (the kernel writes every entry of out_dev itself).  The host polls the tags
        // (block 0's, then the drawing block's) instead of synchronising the stream; a poll that runs out (about
        // 1 s) falls back to the synchronisation, which reports any error of the kernel.
        static unsigned launches = 0;   // guarded by acc_mu like the map (shared by every host thread)
        int dev = 0;
        HIPCHK(hipGetDevice(&dev));
        std::unique_lock<std::mutex> lock(lib_scratch::acc_mu);
        auto it = lib_scratch::acc.find(dev);
        if (it == lib_scratch::acc.end()) {
            unsigned long long *xb = dev_alloc<unsigned long long>(4 * ACC_NB * ACC_XW);
            unsigned *err = dev_alloc<unsigned>(1);
            HIPCHK(hipMemset(xb, 0, 4 * ACC_NB * ACC_XW * sizeof(unsigned long long)));
            HIPCHK(hipMemset(err, 0, sizeof(unsigned)));
            int32_t *host = nullptr;
            HIPCHK(hipHostMalloc((void **)&host, (ACC_HOST_OUT + 64 + 4) * sizeof(int32_t), hipHostMallocCoherent));
            std::memset(host, 0, (ACC_HOST_OUT + 64 + 4) * sizeof(int32_t));
            it = lib_scratch::acc.emplace(dev, lib_scratch::Acc{xb, err, host}).first;
        }
        const lib_scratch::Acc sc = it->second;
        launches = launches % 0xFFFFFu + 1;
        const unsigned tag = launches << 12;
        lock.unlock();
        AcceptArgs a{p_logits_dev, q_logits_dev, vocab, ld, token, trial_start, n_trials, trials, u,
                     n_u, 1.0 / temperature, sc.xbuf, sc.err, tag, n_nodes, n_trials_total, out_dev, max_depth, sc.host,
                     q_row, n_q_rows};
        volatile int32_t *hb = sc.host;
        // entries per thread as a compile-time count (151936 entries: 10)
        const int C = (vocab + ACC_NB * ACC_T - 1) / (ACC_NB * ACC_T);
        if (C <= 2) hipLaunchKernelGGL(k_accept_tree<2>, dim3(ACC_NB), dim3(ACC_T), 0, st, a);
        else if (C <= 4) hipLaunchKernelGGL(k_accept_tree<4>, dim3(ACC_NB), dim3(ACC_T), 0, st, a);
        else if (C <= 8) hipLaunchKernelGGL(k_accept_tree<8>, dim3(ACC_NB), dim3(ACC_T), 0, st, a);
        else if (C <= 10) hipLaunchKernelGGL(k_accept_tree<10>, dim3(ACC_NB), dim3(ACC_T), 0, st, a);
        else hipLaunchKernelGGL(k_accept_tree<ACC_PER>, dim3(ACC_NB), dim3(ACC_T), 0, st, a);
        HIPCHK(hipGetLastError());
        if (staged) HIPCHK(hipEventRecord(staged, st));
        auto wait_tag = [&](int i) {
            for (long spin = 0; spin < (1l << 26); ++spin)
                if (hb[i] == (int32_t)tag) return true;
            return false;
        };
        auto failed = [&] { const unsigned e = (unsigned)hb[0]; return (e & ~0xfffu) == tag && (e & 0xfffu) != 0; };
        if (!(wait_tag(1) && (failed() || wait_tag(2)))) HIPCHK(hipStreamSynchronize(st));
        std::atomic_thread_fence(std::memory_order_acquire);
        require(hb[1] == (int32_t)tag, SP_EHIP, "acceptance walk did not report completion");
        const unsigned err = (unsigned)hb[0];
        if (out_host)
            for (int i = 0; i < max_depth + 4; ++i) out_host[i] = hb[ACC_HOST_OUT + i];
        const unsigned code = (err & ~0xfffu) == tag ? err & 0xfffu : 0u;
        require(code != 2, SP_EINVAL, "malformed tree: node, trial or token index out of range");
        require(code == 0, SP_EHIP, "acceptance exchange timed out");
    }
}

extern "C" {

int sp_op_accept_tree(const float *p_logits_dev, const float *q_logits_dev, int32_t vocab, int32_t ld, int32_t n_nodes,
                      const int32_t *token_dev, const int32_t *trial_start_dev, const int32_t *n_trials_dev,
                      const int32_t *trials_dev, int32_t n_trials_total, const double *u_dev, int32_t n_u,
                      double temperature, int32_t max_depth, double *resid_dev, int32_t *out_dev, void *stream,
                      int32_t *out_host) {
    (void)resid_dev;
    return guarded(nullptr, [&] {
        accept_tree_run(p_logits_dev, q_logits_dev, vocab, ld, n_nodes, token_dev, trial_start_dev, n_trials_dev,
                        trials_dev, n_trials_total, u_dev, n_u, temperature, max_depth, out_dev, (hipStream_t)stream,
                        out_host, nullptr);
    });
}

}  // extern "C"

static void accept_tree_host(const float *p_logits_dev, const float *q_logits_dev, int32_t vocab, int32_t ld,
                             int32_t n_nodes, const int32_t *token, const int32_t *trial_start, const int32_t *n_trials,
                             const int32_t *trials, int32_t n_trials_total, const int32_t *q_row, int32_t n_q_rows,
                             const double *u, int32_t n_u, double temperature, int32_t max_depth, int32_t *out_dev,
                             void *stream, int32_t *out_host) {
    {
        require(token && trial_start && n_trials && trials && u, SP_EINVAL, "NULL pointer");
        require(!q_row || n_q_rows >= 1, SP_EINVAL, "n_q_rows must be positive");
        require(n_nodes >= 1 && n_nodes <= ACC_MAX_NODES, SP_EINVAL, "n_nodes must be in [1, 64]");
        require(n_trials_total >= 0 && n_trials_total <= ACC_MAX_TRIALS, SP_EINVAL, "n_trials_total must be in [0, 1024]");
        require(n_u >= 1 && n_u <= (1 << 20), SP_EINVAL, "n_u must be in [1, 2^20]");
        // per device: a pinned staging block the kernel reads the tree and the uniforms from (no copy on the stream),
        // and an event after the last walk that read it (waited on before the block is refilled)
        int dev = 0;
        HIPCHK(hipGetDevice(&dev));
        lib_scratch::Stage *sgp;
        {
            // guards the map; calls that overlap on one device race as documented
            std::lock_guard<std::mutex> lock(lib_scratch::stage_mu);
            sgp = &lib_scratch::stage[dev];    // std::map references stay valid across inserts
        }
        lib_scratch::Stage &sg = *sgp;
        const size_t ints = (size_t)4 * n_nodes + std::max(n_trials_total, 1);
        const size_t need = (size_t)n_u * sizeof(double) + ints * sizeof(int32_t);
        if (!sg.done) HIPCHK(hipEventCreateWithFlags(&sg.done, hipEventDisableTiming));
        if (sg.used) HIPCHK(hipEventSynchronize(sg.done));
        if (sg.cap < need) {
            if (sg.buf) HIPCHK(hipHostFree(sg.buf));
            sg.buf = nullptr;
            sg.cap = 0;
            const size_t cap = std::max<size_t>(need, 64 * 1024);
            HIPCHK(hipHostMalloc((void **)&sg.buf, cap, hipHostMallocCoherent));
            sg.cap = cap;
        }
        double *su = (double *)sg.buf;
        int32_t *si = (int32_t *)(sg.buf + (size_t)n_u * sizeof(double));
        std::memcpy(su, u, (size_t)n_u * sizeof(double));
        std::memcpy(si, token, (size_t)n_nodes * sizeof(int32_t));
        std::memcpy(si + n_nodes, trial_start, (size_t)n_nodes * sizeof(int32_t));
        std::memcpy(si + 2 * n_nodes, n_trials, (size_t)n_nodes * sizeof(int32_t));
        if (q_row) std::memcpy(si + 3 * n_nodes, q_row, (size_t)n_nodes * sizeof(int32_t));
        int32_t *st = si + 4 * n_nodes;
        if (n_trials_total > 0) std::memcpy(st, trials, (size_t)n_trials_total * sizeof(int32_t));
        else st[0] = 0;
        sg.used = true;
        accept_tree_run(p_logits_dev, q_logits_dev, vocab, ld, n_nodes, si, si + n_nodes, si + 2 * n_nodes, st,
                        n_trials_total, su, n_u, temperature, max_depth, out_dev, (hipStream_t)stream, out_host, sg.done,
                        q_row ? si + 3 * n_nodes : nullptr, n_q_rows);
    }
}

extern "C" {

int sp_op_accept_tree_host(const float *p_logits_dev, const float *q_logits_dev, int32_t vocab, int32_t ld,
                           int32_t n_nodes, const int32_t *token, const int32_t *trial_start, const int32_t *n_trials,
                           const int32_t *trials, int32_t n_trials_total, const double *u, int32_t n_u,
                           double temperature, int32_t max_depth, int32_t *out_dev, void *stream, int32_t *out_host) {
    return guarded(nullptr, [&] {
        accept_tree_host(p_logits_dev, q_logits_dev, vocab, ld, n_nodes, token, trial_start, n_trials, trials,
                         n_trials_total, nullptr, 0, u, n_u, temperature, max_depth, out_dev, stream, out_host);
    });
}

int sp_op_accept_tree_rows(const float *p_logits_dev, const float *q_logits_dev, int32_t n_q_rows, int32_t vocab,
                           int32_t ld, int32_t n_nodes, const int32_t *token, const int32_t *trial_start,
                           const int32_t *n_trials, const int32_t *trials, int32_t n_trials_total,
                           const int32_t *q_row, const double *u, int32_t n_u, double temperature, int32_t max_depth,
                           int32_t *out_dev, void *stream, int32_t *out_host) {
    return guarded(nullptr, [&] {
        require(q_row != nullptr, SP_EINVAL, "NULL pointer");
        accept_tree_host(p_logits_dev, q_logits_dev, vocab, ld, n_nodes, token, trial_start, n_trials, trials,
                         n_trials_total, q_row, n_q_rows, u, n_u, temperature, max_depth, out_dev, stream, out_host);
    });
}

int sp_library_release(void) {
    return guarded(nullptr, [&] {
        std::lock_guard<std::mutex> a(lib_scratch::smp_mu), b(lib_scratch::fm_mu), c(lib_scratch::acc_mu),
            d(lib_scratch::stage_mu);
        if (lib_scratch::smp.empty() && lib_scratch::fm.empty() && lib_scratch::acc.empty() &&
            lib_scratch::stage.empty())
            return;                  // nothing held: no HIP call (a process that never used a GPU stays so)
        int cur = 0;
        HIPCHK(hipGetDevice(&cur));
        // every device that holds scratch: wait for its work (a kernel may still read the scratch), then free it
        std::set<int> devs;
        {
            for (auto &kv : lib_scratch::smp) devs.insert(kv.first);
            for (auto &kv : lib_scratch::fm) devs.insert(kv.first);
            for (auto &kv : lib_scratch::acc) devs.insert(kv.first);
            for (auto &kv : lib_scratch::stage) devs.insert(kv.first);
            for (int dev : devs) {
                HIPCHK(hipSetDevice(dev));
                HIPCHK(hipDeviceSynchronize());
            }
            for (auto &kv : lib_scratch::smp) { HIPCHK(hipSetDevice(kv.first)); dev_free(kv.second.pmax); dev_free(kv.second.csum); }
            for (auto &kv : lib_scratch::fm) { HIPCHK(hipSetDevice(kv.first)); dev_free(kv.second.hist); dev_free(kv.second.st); }
            for (auto &kv : lib_scratch::acc) {
                HIPCHK(hipSetDevice(kv.first));
                dev_free(kv.second.xbuf);
                dev_free(kv.second.err);
                if (kv.second.host) HIPCHK(hipHostFree(kv.second.host));
            }
            for (auto &kv : lib_scratch::stage) {
                HIPCHK(hipSetDevice(kv.first));
                if (kv.second.buf) HIPCHK(hipHostFree(kv.second.buf));
                if (kv.second.done) HIPCHK(hipEventDestroy(kv.second.done));
            }
            lib_scratch::smp.clear();
            lib_scratch::fm.clear();
            lib_scratch::acc.clear();
            lib_scratch::stage.clear();
        }
        HIPCHK(hipSetDevice(cur));
    });
}

int sp_op_draft_link(const int32_t *tokens_dev, int32_t n_branches, int32_t level, int32_t *canon_dev,
                     uint64_t *masks_dev, int32_t *rows_dev, void *stream) {
    return guarded(nullptr, [&] {
        require(tokens_dev && canon_dev && masks_dev && rows_dev, SP_EINVAL, "NULL pointer");
        require(n_branches >= 1 && n_branches <= 64 && level >= 0 && n_branches * (level + 1) <= 64, SP_EINVAL,
                "the drafted nodes (branches x levels) must fit one 64-bit tree mask");
        hipLaunchKernelGGL(k_draft_link, dim3(1), dim3(64), 0, (hipStream_t)stream, tokens_dev, n_branches, level,
                           canon_dev, (unsigned long long *)masks_dev, rows_dev);
        HIPCHK(hipGetLastError());
    });
}

}  // extern "C"
