// Decode-side kernels around the GEMVs: embedding gather, RMSNorm, RoPE + KV-cache write, split-K GQA attention
// (windowed ring slots + tree ancestor mask), split-K combine, two-pass argmax, KV slot moves.
#pragma once
#include "sp_device.h"
#include "../../include/seedplane_hip.h"

// ---------------------------------------------------------------------------------------------------------------
// Element (row, k) of a packed matrix (layout written by sp_pack.h), dequantised in fp32 exactly as the canonical
// definition: Q8 code*scale, Q4 (code - zero)*scale, F16 the value itself.
template <int FMT>
__device__ __forceinline__ float packed_elem(const uint8_t *w, const f16 *sz, int nkt, int row, int k) {
    const int rg = row >> 4, r = row & 15;
    if constexpr (FMT == 1) {
        const int kt = k >> 5, lk = k & 31, g = lk >> 3, i = lk & 7;
        const f16 *t = (const f16 *)(w + ((size_t)rg * nkt + kt) * TILE_BYTES);
        return (float)t[(g * 16 + r) * 8 + i];
    } else if constexpr (FMT == 2) {
        const int kt = k >> 6, lk = k & 63, blk = lk >> 5, kk = lk & 31, g = kk >> 3, i = kk & 7;
        const size_t tile = (size_t)rg * nkt + kt;
        const int8_t c = (int8_t)w[tile * TILE_BYTES + (g * 16 + r) * 16 + blk * 8 + i];
        return (float)c * (float)sz[tile * 32 + r * 2 + blk];
    } else {
        const int kt = k >> 7, lk = k & 127, s = lk >> 5, kk = lk & 31, g = kk >> 3, i = kk & 7;
        const size_t tile = (size_t)rg * nkt + kt;
        const uint32_t d = *(const uint32_t *)(w + tile * TILE_BYTES + (g * 16 + r) * 16 + s * 4);
        const int pos = (i >> 1) + 4 * (i & 1);
        const float code = (float)((d >> (4 * pos)) & 15u);
        const float scale = (float)sz[tile * 128 + (r * 4 + s) * 2], zero = (float)sz[tile * 128 + (r * 4 + s) * 2 + 1];
        return __fmul_rn(code - zero, scale);
    }
}

// x[b][k] = E[token_b][k] (fp32).  Replaces F.embedding (qwen_engine.py:117) / embed.comp.  With `feed` the token
// of column b is feed[b] (the previous step's argmax of that column, kept on the device), clamped to the vocabulary.
template <int FMT>
__global__ void __launch_bounds__(256) k_embed(const uint8_t *w, const f16 *sz, int nkt, const sp_token *toks,
                                               int H, float *x, int ldx, const int *feed, int vocab,
                                               const float *inv_freq, int half, float2 *rtab) {
    const int b = blockIdx.x, tok = feed ? min(max(feed[b], 0), vocab - 1) : toks[b].token;
    for (int k = threadIdx.x; k < H; k += blockDim.x) x[(size_t)b * ldx + k] = packed_elem<FMT>(w, sz, nkt, tok, k);
    // the step's rotation table: (cos, sin) of phase = float(pos) * inv_freq[j] for every column, computed once here
    // and read by the RoPE steps of every layer (the same values they would compute themselves)
    const float fpos = (float)toks[b].pos;
    for (int j = threadIdx.x; j < half; j += blockDim.x) {
        const float ph = fpos * inv_freq[j];
        rtab[(size_t)b * half + j] = make_float2(cosf(ph), sinf(ph));
    }
}

// out[b][k] = fp16(x * rsqrt(mean(x^2) + eps) * w), and with out_lo the fp16 remainder of that fp32 value (split_f16).
// Replaces Qwen2Engine._norm (qwen_engine.py:90-92): the weight multiply happens in fp32 before the cast.  One block
// of 1024 threads per column; every load (x, the weight and
// the NP split-K slices) is issued before the first use.  With NP > 0 the residual update of a split-K GEMV is
// completed first: x[b] += part[0][b] + ... + part[NP-1][b] (in slice order) and written back to x.
constexpr int NORM_THREADS = 1024, NORM_PER_THREAD = 4;
// NG = the element groups of NORM_THREADS that H needs (<= NORM_PER_THREAD; the missing groups are zeros, which add
// nothing to the sum of squares): the body is straight-line code whose loads are all unconditional, from clamped
// indices (elements past H re-read element H - 1 and become zeros after loading), so they are in flight together.
template <int NP, int NG>
__device__ __forceinline__ void rmsnorm_body(float *x, int ldx, const float *part, size_t pstride, const float *w, int H,
                                             float eps, f16 *out, f16 *out_lo, int ldo, int mtp) {
    __shared__ float red[16];
    const int b = blockIdx.x;
    float *xr = x + (size_t)b * ldx;
    float v[NORM_PER_THREAD], wk[NORM_PER_THREAD], pv[NP > 0 ? NP : 1][NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int kc = min((int)threadIdx.x + i * NORM_THREADS, H - 1);
        v[i] = xr[kc];
        wk[i] = w[kc];
#pragma unroll
        for (int s = 0; s < NP; ++s) pv[s][i] = part[(size_t)s * pstride + (size_t)b * ldx + kc];
    }
#pragma unroll
    for (int i = NG; i < NORM_PER_THREAD; ++i) { v[i] = 0.f; wk[i] = 0.f; }
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const bool in = (int)threadIdx.x + i * NORM_THREADS < H;
        v[i] = in ? v[i] : 0.f;
#pragma unroll
        for (int s = 0; s < NP; ++s) pv[s][i] = in ? pv[s][i] : 0.f;
    }
    if constexpr (NP > 0) {
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            const int k = threadIdx.x + i * NORM_THREADS;
#pragma unroll
            for (int s = 0; s < NP; ++s) v[i] += pv[s][i];
            if (k < H) xr[k] = v[i];
        }
    }
    // the sum of squares in one fixed rounding order (no contraction: each square rounded, then added in element
    // order), which the GEMV norm prologue repeats bit for bit
    float ss = 0.f;
    {
#pragma clang fp contract(off)
#pragma unroll
        for (int i = 0; i < NORM_PER_THREAD; ++i) ss += v[i] * v[i];
    }
    ss = block_sum_dpp(ss, red);
    const float rs = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int k = threadIdx.x + i * NORM_THREADS;
        f16 hi, lo;
        split_f16((v[i] * rs) * wk[i], hi, lo);
        if (k < H) out[act_off(b, k, ldo, mtp)] = hi;
        if (k < H && out_lo) out_lo[act_off(b, k, ldo, mtp)] = lo;
    }
}
template <int NP>
__global__ void __launch_bounds__(NORM_THREADS) k_rmsnorm(float *x, int ldx, const float *part, size_t pstride,
                                                          const float *w, int H, float eps, f16 *out, f16 *out_lo,
                                                          int ldo, int mtp) {
    if (H <= NORM_THREADS) rmsnorm_body<NP, 1>(x, ldx, part, pstride, w, H, eps, out, out_lo, ldo, mtp);
    else if (H <= 2 * NORM_THREADS) rmsnorm_body<NP, 2>(x, ldx, part, pstride, w, H, eps, out, out_lo, ldo, mtp);
    else rmsnorm_body<NP, NORM_PER_THREAD>(x, ldx, part, pstride, w, H, eps, out, out_lo, ldo, mtp);
}

// ---------------------------------------------------------------------------------------------------------------
// One RoPE rotation pair as the reference rounds it: o1 = x1 c - x2 s, o2 = x2 c + x1 s, each product rounded to fp32,
// then the sum (qwen_engine.py:94-103: q * cos + rotate_half(q) * sin).  Contraction into fused multiply-adds is off
// here (hipcc contracts a * b + c by default, and __fmul_rn / __fadd_rn are plain operators in HIP), so every kernel
// that rotates produces the same bits.
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float &o1, float &o2) {
#pragma clang fp contract(off)
    o1 = x1 * c - x2 * s;
    o2 = x2 * c + x1 * s;
}

struct RopeArgs {
    const float *qkv;       // [n][Nqkv] fp32 (bias already added) when nparts == 0
    int Nqkv, NH, NKV, HD;
    const float2 *rtab;     // [n][HD/2] (cos, sin) of float(pos) * inv_freq, from the step's embedding kernel
    const sp_token *toks;
    float *q;               // [n][NH*HD] fp32, rotated
    f16 *kc, *vc;           // this layer's K/V: [seq][kvh][slot][HD]
    int n_slots;
    const float *part;      // NP > 0: the projection is part[0] + ... + part[NP-1] + bias (slices [n][Nqkv])
    size_t pstride;
    const float *bias;
};

template <int NP>
__device__ __forceinline__ float qkv_value(const RopeArgs &a, int b, int idx) {
    if constexpr (NP == 0) {
        return a.qkv[(size_t)b * a.Nqkv + idx];
    } else {
        const float *p = a.part + (size_t)b * a.Nqkv + idx;
        float t[NP];
#pragma unroll
        for (int s = 0; s < NP; ++s) t[s] = p[(size_t)s * a.pstride];
        float v = t[0];
#pragma unroll
        for (int s = 1; s < NP; ++s) v += t[s];
        return v + a.bias[idx];
    }
}
// Non-interleaved half rotation x*cos + rotate_half(x)*sin with phase = float(pos) * inv_freq (qwen_engine.py:94-103,
// rope_kv.comp:1-32); K and V of every column are written to their slot.  Two blocks of ROPE_THREADS per column:
// block y = 0 rotates the queries and the key, block y = 1 copies the value (each in one memory round trip; one block
// doing both would issue the value loads only after the rotation's stores).
constexpr int ROPE_THREADS = 1024;
template <int NP>
__global__ void __launch_bounds__(ROPE_THREADS) k_rope_kv(RopeArgs a) {
    const int b = blockIdx.x;
    const sp_token t = a.toks[b];
    const int half = a.HD >> 1;
    if (blockIdx.y == 1) {
        const int v0 = (a.NH + a.NKV) * a.HD;
        for (int idx = threadIdx.x; idx < a.NKV * a.HD; idx += blockDim.x) {
            const int kvh = idx / a.HD, d = idx - kvh * a.HD;
            a.vc[(((size_t)t.seq * a.NKV + kvh) * a.n_slots + t.slot) * a.HD + d] = (f16)qkv_value<NP>(a, b, v0 + idx);
        }
        return;
    }
    for (int idx = threadIdx.x; idx < (a.NH + a.NKV) * half; idx += blockDim.x) {
        const int head = idx / half, i = idx - head * half;
        const float2 cs = a.rtab[(size_t)b * half + i];
        const float c = cs.x, s = cs.y;
        const float x1 = qkv_value<NP>(a, b, head * a.HD + i), x2 = qkv_value<NP>(a, b, head * a.HD + i + half);
        float o1, o2;
        rope_pair(x1, x2, c, s, o1, o2);
        if (head < a.NH) {
            float *q = a.q + (size_t)b * a.NH * a.HD + head * a.HD;
            q[i] = o1; q[i + half] = o2;
        } else {
            const int kvh = head - a.NH;
            f16 *k = a.kc + (((size_t)t.seq * a.NKV + kvh) * a.n_slots + t.slot) * a.HD;
            k[i] = (f16)o1; k[i + half] = (f16)o2;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Split-K GQA attention.  One block per (chunk of CH visible keys, kv head, column); the G query heads of the kv
// head share the K/V chunk staged in LDS.  Visible keys of a column: ring positions [ctx_lo, ctx_hi] then the tree
// block (slots tree_base + j, bit j of tree_mask).  Each block records {m, l, o[HD]} per query head (o = acc / l, the
// chunk's own normalised output); k_attn_combine merges them with l exp(m - M) weights.  Replaces the SDPA call with its causal/slot mask (qwen_engine.py:126-135)
// and attn_part.comp / attn_combine.comp.
constexpr int ATT_CH = 64;
// One partial record per (column, head, chunk): m and l as fp32, then o[HD] = acc / l as fp16 (half the bytes of an
// fp32 record; o is a convex combination of the chunk's fp16 values, so it never exceeds the fp16 range, which the
// unnormalised acc (up to l x max |v|) could; the rounding is below the fp16 rounding of the merged output).  Length
// in floats:
__host__ __device__ constexpr int part_floats(int HD) { return 2 + HD / 2; }
struct AttnArgs {
    const float *q;        // [n][NH*HD]
    const f16 *kc, *vc;    // this layer
    const sp_token *toks;
    int NH, NKV, HD, n_slots, nchunk;   // nchunk = grid.x (max over columns)
    float scale;
    float *part;           // [n][NH][nchunk][HD + 2]
};

__device__ __forceinline__ int att_visible(const sp_token &t, int &nlin) {
    nlin = t.ctx_hi >= t.ctx_lo ? t.ctx_hi - t.ctx_lo + 1 : 0;
    return nlin + t.tree_count;
}

constexpr int ATT_MAX_CHUNKS = 512;

// One block per (chunk of ATT_CH visible keys, kv head, column); wave h handles query head kvh*G + h: lane j scores
// key j of the chunk, the wave takes max / exp / sum over its 64 lanes, then lanes own output dims for P.V.
template <int HD, int G>
__global__ void __launch_bounds__(64 * G) k_attn_part(AttnArgs a) {
    constexpr int KP = HD + 8;                       // padded K row (halves) to spread LDS banks
    __shared__ float q_s[G][HD];
    __shared__ __align__(16) f16 k_s[ATT_CH][KP];
    __shared__ __align__(16) f16 v_s[ATT_CH][HD];
    __shared__ float e_s[G][ATT_CH];
    __shared__ int ok_s[ATT_CH];

    const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const sp_token t = a.toks[b];
    int nlin;
    const int nvis = att_visible(t, nlin);
    const int v0 = c * ATT_CH;
    if (v0 >= nvis) return;
    const int cnt = min(ATT_CH, nvis - v0);
    const int tid = threadIdx.x, lane = tid & 63, h = tid >> 6;
    constexpr int NT = 64 * G;

    for (int i = tid; i < G * HD; i += NT)
        q_s[i / HD][i % HD] = a.q[(size_t)b * a.NH * HD + (kvh * G) * HD + i] * a.scale;
    const size_t head_base = ((size_t)t.seq * a.NKV + kvh) * a.n_slots;
    constexpr int CPR = HD / 8;                     // 16-byte chunks per row
    for (int i = tid; i < cnt * CPR; i += NT) {
        const int j = i / CPR, ch = i - j * CPR;
        const int vis = v0 + j;
        int slot, ok = 1;
        if (vis < nlin) {
            slot = (t.ctx_lo + vis) % a.n_slots;
        } else {
            const int tj = vis - nlin;
            slot = (t.tree_base + tj) % a.n_slots;
            ok = (int)((t.tree_mask >> tj) & 1ull);
        }
        if (ch == 0) ok_s[j] = ok;
        const size_t off = (head_base + slot) * HD + ch * 8;
        *(f16x8 *)&k_s[j][ch * 8] = *(const f16x8 *)(a.kc + off);
        *(f16x8 *)&v_s[j][ch * 8] = *(const f16x8 *)(a.vc + off);
    }
    __syncthreads();

    float sc = -INFINITY;
    if (lane < cnt && ok_s[lane]) {
        float acc = 0.f;
#pragma unroll 4
        for (int d = 0; d < HD; d += 8) {
            const f16x8 kv = *(const f16x8 *)&k_s[lane][d];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += q_s[h][d + e] * (float)kv[e];
        }
        sc = acc;
    }
    const float m = wave_max_dpp(sc);
    const float ex = (sc == -INFINITY) ? 0.f : expf(sc - m);
    const float l = wave_sum_dpp(ex);
    e_s[h][lane] = ex;
    __syncthreads();

    float *out = a.part + (((size_t)b * a.NH + kvh * G + h) * a.nchunk + c) * part_floats(HD);
    constexpr int DPL = HD / 64;                    // output dims per lane
    float o[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[i] = 0.f;
    for (int j = 0; j < cnt; ++j) {
        const float p = e_s[h][j];
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[i] += p * (float)v_s[j][lane + 64 * i];
    }
    const float il = l > 0.f ? 1.f / l : 0.f;         // acc / l: bounded by max |v|, so fp16 holds it
#pragma unroll
    for (int i = 0; i < DPL; ++i) ((f16 *)(out + 2))[lane + 64 * i] = (f16)(o[i] * il);
    if (lane == 0) { out[0] = m; out[1] = l; }
}

// k_attn_part with the RoPE / KV-write step folded in, for plain decode columns (no tree block): each block rotates
// the queries of its kv head from the projection (split-K slices + bias, in slice order, exactly as k_rope_kv), and
// the block whose chunk holds the column's newest position (ctx_hi) also rotates its key, writes key and value to
// their cache slot and uses them for that row.  Same arithmetic and summation order as k_rope_kv + k_attn_part, so
// the results are bit-identical; one launch (and one dependent step) fewer per layer.
template <int HD, int G>
__global__ void __launch_bounds__(64 * G) k_attn_part_rope(AttnArgs a, RopeArgs r, int np) {
    constexpr int KP = HD + 8, HALF = HD / 2;
    __shared__ float q_s[G][HD];
    __shared__ __align__(16) f16 k_s[ATT_CH][KP];
    __shared__ __align__(16) f16 v_s[ATT_CH][HD];
    __shared__ float e_s[G][ATT_CH];

    const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const sp_token t = a.toks[b];
    const int nlin = t.ctx_hi >= t.ctx_lo ? t.ctx_hi - t.ctx_lo + 1 : 0;
    const int v0 = c * ATT_CH;
    if (v0 >= nlin) return;
    const int cnt = min(ATT_CH, nlin - v0);
    const int jn = nlin - 1 - v0;                   // row of the newest position in this chunk (< cnt: owned here)
    const bool own = jn < cnt;
    const int tid = threadIdx.x, lane = tid & 63, h = tid >> 6;
    constexpr int NT = 64 * G;
    const size_t head_base = ((size_t)t.seq * a.NKV + kvh) * a.n_slots;

    // the chunk's cached K/V rows into registers first, so their loads overlap the projection loads below
    constexpr int CPR = HD / 8;                     // 16-byte chunks per row
    constexpr int PER = (ATT_CH * CPR + NT - 1) / NT;
    f16x8 kr[PER], vr[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        // unconditional loads (rows past the chunk re-read row 0) so that all of them are in flight together
        const int i = tid + k * NT, j = i < cnt * CPR ? i / CPR : 0, ch = i % CPR;
        const size_t off = (head_base + (t.ctx_lo + v0 + j) % a.n_slots) * HD + ch * 8;
        kr[k] = *(const f16x8 *)(a.kc + off);
        vr[k] = *(const f16x8 *)(a.vc + off);
    }
    // queries of the group (then the key of the newest position, in the owning block) are rotated; the owning block
    // also stores the new value.  Every projection load of the thread (all slices and the bias of its rotation pairs
    // and of its value dim) is issued in one batch from clamped indices before the first add, so the owning block
    // pays one memory round trip like the others.
    const int nrot = (own ? G + 1 : G) * HALF;
    constexpr int RI = ((G + 1) * HALF + NT - 1) / NT;    // rotation items per thread
    const int nsl = np == 0 ? 1 : np;                    // slices to load (np == 0: the finished row)
    const float *prow = np == 0 ? r.qkv + (size_t)b * r.Nqkv : r.part + (size_t)b * r.Nqkv;
    const size_t pstr = np == 0 ? 0 : r.pstride;
    float t1[RI][8], t2[RI][8], bb1[RI], bb2[RI], tv[8], bv = 0.f;
    float2 tw[RI];
    int id1[RI];
#pragma unroll
    for (int ri = 0; ri < RI; ++ri) {
        const int i = min(tid + ri * NT, nrot - 1);
        const int hh = i / HALF, j = i - hh * HALF;
        const int head = hh < G ? kvh * G + hh : a.NH + kvh;
        id1[ri] = head * HD + j;
#pragma unroll
        for (int sl = 0; sl < 8; ++sl) {
            if (sl < nsl) {
                t1[ri][sl] = prow[(size_t)sl * pstr + id1[ri]];
                t2[ri][sl] = prow[(size_t)sl * pstr + id1[ri] + HALF];
            }
        }
        bb1[ri] = np == 0 ? 0.f : r.bias[id1[ri]];
        bb2[ri] = np == 0 ? 0.f : r.bias[id1[ri] + HALF];
        tw[ri] = r.rtab[(size_t)b * HALF + j];
    }
    const int vidx = (a.NH + a.NKV + kvh) * HD + min(tid, HD - 1);
#pragma unroll
    for (int sl = 0; sl < 8; ++sl)
        if (sl < nsl) tv[sl] = prow[(size_t)sl * pstr + vidx];
    if (np != 0) bv = r.bias[vidx];
    // the projection value: the finished row, or the slices in slice order plus the bias (as k_rope_kv)
    auto sum_of = [&](const float *tt, float bias) {
        float v = tt[0];
#pragma unroll
        for (int sl = 1; sl < 8; ++sl) if (sl < np) v += tt[sl];
        return np == 0 ? v : v + bias;
    };
#pragma unroll
    for (int ri = 0; ri < RI; ++ri) {
        const int i = tid + ri * NT;
        if (i >= nrot) break;
        const int hh = i / HALF, j = i - hh * HALF;
        const float cs = tw[ri].x, sn = tw[ri].y;
        const float x1 = sum_of(t1[ri], bb1[ri]), x2 = sum_of(t2[ri], bb2[ri]);
        float o1, o2;
        rope_pair(x1, x2, cs, sn, o1, o2);
        if (hh < G) {
            q_s[hh][j] = o1 * a.scale;
            q_s[hh][j + HALF] = o2 * a.scale;
        } else {
            const f16 k1 = (f16)o1, k2 = (f16)o2;
            k_s[jn][j] = k1; k_s[jn][j + HALF] = k2;
            f16 *kd = r.kc + (head_base + t.slot) * HD;
            kd[j] = k1; kd[j + HALF] = k2;
        }
    }
    if (own && tid < HD) {
        const f16 v = (f16)sum_of(tv, bv);
        v_s[jn][tid] = v;
        r.vc[(head_base + t.slot) * HD + tid] = v;
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = tid + k * NT, j = i / CPR, ch = i - j * CPR;
        if (i < cnt * CPR && !(own && j == jn)) {   // the newest row came from the projection
            *(f16x8 *)&k_s[j][ch * 8] = kr[k];
            *(f16x8 *)&v_s[j][ch * 8] = vr[k];
        }
    }
    __syncthreads();

    float sc = -INFINITY;
    if (lane < cnt) {
        float acc = 0.f;
#pragma unroll 4
        for (int d = 0; d < HD; d += 8) {
            const f16x8 kv = *(const f16x8 *)&k_s[lane][d];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += q_s[h][d + e] * (float)kv[e];
        }
        sc = acc;
    }
    const float m = wave_max_dpp(sc);
    const float ex = (sc == -INFINITY) ? 0.f : expf(sc - m);
    const float l = wave_sum_dpp(ex);
    e_s[h][lane] = ex;
    __syncthreads();

    float *out = a.part + (((size_t)b * a.NH + kvh * G + h) * a.nchunk + c) * part_floats(HD);
    constexpr int DPL = HD / 64;                    // output dims per lane
    float o[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[i] = 0.f;
    for (int j = 0; j < cnt; ++j) {
        const float p = e_s[h][j];
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[i] += p * (float)v_s[j][lane + 64 * i];
    }
    const float il = l > 0.f ? 1.f / l : 0.f;         // acc / l: bounded by max |v|, so fp16 holds it
#pragma unroll
    for (int i = 0; i < DPL; ++i) ((f16 *)(out + 2))[lane + 64 * i] = (f16)(o[i] * il);
    if (lane == 0) { out[0] = m; out[1] = l; }
}

// Decode attention on MFMA for columns whose keys are one ring range (no tree block).  One block per (kv head, column,
// split of NWV * SUB * DEC_KC keys); wave w owns SUB * DEC_KC consecutive keys of the split and streams them with two
// sub-chunks of K / V loads in flight while it computes.  Per sub-chunk of DEC_KC keys: S = Q K^T on
// MFMA (rows = the G query heads of the kv head, K fragments straight from the cache), online softmax per row, P and
// V^T staged in the wave's own LDS region, O += P V on MFMA.  The wave states are merged in wave order; a column
// whose keys fit one split gets its fp16 attention row directly, otherwise each split writes {m, l, acc / l} in
// k_attn_part's layout and k_attn_combine merges the splits.
constexpr int DEC_KC = 32;
template <int HD, int NWV, int SUB>
__global__ void __launch_bounds__(64 * NWV) k_attn_dec(AttnArgs a, f16 *out, int ldo, int direct, int mtp) {
    constexpr int DEC_WAVES = NWV, DEC_SUB = SUB, DEC_KW = DEC_KC * SUB, DEC_KB = NWV * DEC_KW;
    constexpr int ST = HD / 32, NDT = HD / 16, KP = DEC_KC + 8;
    constexpr int VPL = HD / 2 / 8;                          // 16-byte V pieces per lane per sub-chunk
    __shared__ __align__(16) f16 vt[DEC_WAVES][HD][KP];      // V^T of the wave's current sub-chunk
    __shared__ __align__(16) f16 ps[DEC_WAVES][16][KP];      // P of the wave's current sub-chunk
    __shared__ float wm[DEC_WAVES][16], wl[DEC_WAVES][16];
    __shared__ float wo[DEC_WAVES][8][HD];                   // wave outputs of the (at most 8) query heads
    const int kvh = blockIdx.x, b = blockIdx.y, split = blockIdx.z;
    const sp_token t = a.toks[b];
    const int G = a.NH / a.NKV;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r16 = lane & 15, g4 = lane >> 4;
    const int nlin = t.ctx_hi - t.ctx_lo + 1;
    const int b_lo = split * DEC_KB;
    if (b_lo >= nlin) return;
    const int v_lo = b_lo + w * DEC_KW, v_hi = min(nlin, v_lo + DEC_KW);
    const size_t head_base = ((size_t)t.seq * a.NKV + kvh) * a.n_slots;
    const f16x8 zero8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    // ---- the wave's K / V stream: sub-chunk sc's loads (K fragments -- lane: key r16 of a 16-key tile, dims g4 * 8 ..
    // -- and V rows -- lane: key lane / 2, dims (lane & 1) * HD/2 .., the layout whose transposed LDS stores are
    // conflict-free) land in register slot sc % 2; the loads of
    // sub-chunk sc + 2 are issued as soon as sub-chunk sc has been consumed, so two sub-chunks are always in flight
    // while the wave computes (loads complete in order, so each use waits only for its own sub-chunk).  Keys past the
    // range load the first key of the range instead (unconditional loads: a per-lane condition would split them into
    // branches and the waits at their joins would also wait for the prefetched sub-chunks); their scores are masked
    // (P = 0) and the values they load are finite cache entries, so they contribute nothing.
    f16x8 kf[2][2][ST], vf[2][VPL];
    auto load_sub = [&](int sc, int slot) {
        const int v0 = v_lo + sc * DEC_KC;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const int key = v0 + kt * 16 + r16;
            const size_t off = (head_base + (size_t)((t.ctx_lo + (key < v_hi ? key : 0)) % a.n_slots)) * HD + g4 * 8;
#pragma unroll
            for (int st = 0; st < ST; ++st) kf[slot][kt][st] = *(const f16x8 *)(a.kc + off + st * 32);
        }
        const int key = v0 + (lane >> 1);
        const size_t off =
            (head_base + (size_t)((t.ctx_lo + (key < v_hi ? key : 0)) % a.n_slots)) * HD + (lane & 1) * (HD / 2);
#pragma unroll
        for (int i = 0; i < VPL; ++i) vf[slot][i] = *(const f16x8 *)(a.vc + off + i * 8);
    };
    load_sub(0, 0);
    if (DEC_SUB > 1) load_sub(1, 1);
    // Q fragments (rows = query heads of this kv head, scaled, fp16 with their fp16 remainders: the scores take two
    // MFMAs per step, so Q enters them at fp32-class precision -- the scores at long contexts are large, and a query
    // rounded to fp16 alone moves the softmax weights by more than the fp16 logits bar): unconditional vector loads
    // from a clamped row (a load under a per-lane condition is issued and waited for one at a time)
    f16x8 qa[ST], ql[ST];
    {
        const float *qrow = a.q + (size_t)b * a.NH * HD + (size_t)(kvh * G + min(r16, G - 1)) * HD + g4 * 8;
        f32x4 qv[ST][2];
#pragma unroll
        for (int st = 0; st < ST; ++st) {
            qv[st][0] = *(const f32x4 *)(qrow + st * 32);
            qv[st][1] = *(const f32x4 *)(qrow + st * 32 + 4);
        }
        const float qs = r16 < G ? a.scale : 0.f;
#pragma unroll
        for (int st = 0; st < ST; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                f16 hi, lo;
                split_f16(qv[st][e >> 2][e & 3] * qs, hi, lo);
                qa[st][e] = hi;
                ql[st][e] = lo;
            }
    }
    float mrow[4], lrow[4];
    f32x4 o[NDT];
#pragma unroll
    for (int j = 0; j < 4; ++j) { mrow[j] = -INFINITY; lrow[j] = 0.f; }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sc = 0; sc < DEC_SUB; ++sc) {
        const int v0 = v_lo + sc * DEC_KC;
        if (v0 >= v_hi) break;                               // wave-uniform
        const int slot = sc & 1;
#pragma unroll
        for (int i = 0; i < VPL; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) vt[w][(lane & 1) * (HD / 2) + i * 8 + e][lane >> 1] = vf[slot][i][e];
        f32x4 sc2[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            sc2[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < ST; ++st) {
                sc2[kt] = mfma16(qa[st], kf[slot][kt][st], sc2[kt]);
                sc2[kt] = mfma16(ql[st], kf[slot][kt][st], sc2[kt]);
            }
        }
        if (sc + 2 < DEC_SUB) load_sub(sc + 2, slot);      // the slot's registers are consumed: refill them
        // online softmax: lane holds rows 4 g4 + j, keys v0 + kt * 16 + r16
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float mx = mrow[j];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) if (v0 + kt * 16 + r16 < v_hi) mx = fmaxf(mx, sc2[kt][j]);
            mx = row16_max(mx);
            const float corr = mrow[j] == -INFINITY ? 0.f : expf(mrow[j] - mx);
            float ls = 0.f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const float pe = v0 + kt * 16 + r16 < v_hi ? expf(sc2[kt][j] - mx) : 0.f;
                ps[w][4 * g4 + j][kt * 16 + r16] = (f16)pe;
                ls += pe;
            }
            ls = row16_sum(ls);
            lrow[j] = lrow[j] * corr + ls;
            mrow[j] = mx;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) o[dt][j] *= corr;
        }
        __builtin_amdgcn_wave_barrier();                     // LDS is in order within a wave: P and V^T are in place
        const f16x8 pa = *(const f16x8 *)&ps[w][r16][g4 * 8];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            o[dt] = mfma16(pa, *(const f16x8 *)&vt[w][dt * 16 + r16][g4 * 8], o[dt]);
        __builtin_amdgcn_wave_barrier();
    }
    // wave states -> LDS, merged in wave order
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int h = 4 * g4 + j;
        if (r16 == 0) { wm[w][h] = mrow[j]; wl[w][h] = lrow[j]; }
        if (h < G && h < 8) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) wo[w][h][dt * 16 + r16] = o[dt][j];
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * HD; i += blockDim.x) {
        const int h = i / HD, d = i - h * HD;
        float M = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < DEC_WAVES; ++w2) if (wl[w2][h] > 0.f) M = fmaxf(M, wm[w2][h]);
        float L = 0.f, acc = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < DEC_WAVES; ++w2) {
            if (wl[w2][h] > 0.f) {
                const float f = expf(wm[w2][h] - M);
                L += f * wl[w2][h];
                acc += f * wo[w2][h][d];
            }
        }
        if (direct) {
            out[act_off(b, (kvh * G + h) * HD + d, ldo, mtp)] = (f16)(acc / L);
        } else {
            float *pp = a.part + (((size_t)b * a.NH + kvh * G + h) * a.nchunk + split) * part_floats(HD);
            ((f16 *)(pp + 2))[d] = (f16)(L > 0.f ? acc / L : 0.f);
            if (d == 0) { pp[0] = M; pp[1] = L; }
        }
    }
}

// out[b][h*HD + d] (fp16) = sum_c o_c[d] l_c e^{m_c - M} / sum_c l_c e^{m_c - M}; one block (HD threads) per
// (head, column), chunk statistics loaded in parallel.
// The chunk outputs are read in batches of CMB_BATCH with every load of a batch in flight together (the first batch
// before the weights are known); the accumulation runs over the chunks in ascending order.
constexpr int CMB_BATCH = 16;
__global__ void __launch_bounds__(128) k_attn_combine(const float *part, const int *col_nchunk, int NH, int HD,
                                                      int nchunk, f16 *out, int ldo, int mtp) {
    __shared__ float w_s[ATT_MAX_CHUNKS];
    __shared__ float l_s[ATT_MAX_CHUNKS];
    __shared__ float red[16];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, nt = blockDim.x;
    const int nc = col_nchunk[b];
    const int rec = part_floats(HD);
    const float *p = part + ((size_t)b * NH + h) * nchunk * rec;
    const int d = min(tid, HD - 1), last = max(nc - 1, 0);     // clamped: every load is in bounds
    float v[CMB_BATCH];
#pragma unroll
    for (int i = 0; i < CMB_BATCH; ++i) v[i] = (float)((const f16 *)(p + (size_t)min(i, last) * rec + 2))[d];
    float mloc = -INFINITY;
    for (int c = tid; c < nc; c += nt) {
        const float mc = p[(size_t)c * rec], lc = p[(size_t)c * rec + 1];
        w_s[c] = lc > 0.f ? mc : -INFINITY;
        l_s[c] = lc;
        mloc = fmaxf(mloc, w_s[c]);
    }
    // block max
    mloc = wave_max_dpp(mloc);
    if ((tid & 63) == 0) red[tid >> 6] = mloc;
    __syncthreads();
    float M = red[0];
    for (int i = 1; i < (nt + 63) / 64; ++i) M = fmaxf(M, red[i]);
    float lsum = 0.f;
    for (int c = tid; c < nc; c += nt) {
        const float wc = w_s[c] == -INFINITY ? 0.f : expf(w_s[c] - M) * l_s[c];
        w_s[c] = wc;
        lsum += wc;
    }
    __syncthreads();
    const float L = block_sum_dpp(lsum, red + 8);
    float acc = 0.f;
    for (int c0 = 0; c0 < nc; c0 += CMB_BATCH) {
        if (c0 > 0) {
#pragma unroll
            for (int i = 0; i < CMB_BATCH; ++i) v[i] = (float)((const f16 *)(p + (size_t)min(c0 + i, last) * rec + 2))[d];
        }
#pragma unroll
        for (int i = 0; i < CMB_BATCH; ++i)
            if (c0 + i < nc) acc += w_s[c0 + i] * v[i];
    }
    if (tid < HD) out[act_off(b, h * HD + tid, ldo, mtp)] = (f16)(acc / L);
}

// ---------------------------------------------------------------------------------------------------------------
// Two-pass argmax, first index on ties (qwen_engine.py:148 torch.argmax; sampler.hpp:98-99; argmax.comp:2,17).
constexpr int ARGMAX_BLOCKS = 64;
__global__ void __launch_bounds__(256) k_argmax_part(const float *x, int cols, int ld, float *pv, int *pi) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int row = blockIdx.y, blk = blockIdx.x;
    const int per = (cols + ARGMAX_BLOCKS - 1) / ARGMAX_BLOCKS;
    const int lo = blk * per, hi = min(cols, lo + per);
    float bv = -INFINITY; int bi = 0x7fffffff;
    const float *xr = x + (size_t)row * ld;
    for (int i = lo + threadIdx.x; i < hi; i += 256) argmax_merge(bv, bi, xr[i], i);
    wave_argmax(bv, bi);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (lane == 0) { sv[wv] = bv; si[wv] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w2 = 1; w2 < 4; ++w2) argmax_merge(bv, bi, sv[w2], si[w2]);
        pv[row * ARGMAX_BLOCKS + blk] = bv; pi[row * ARGMAX_BLOCKS + blk] = bi;
    }
}
__global__ void __launch_bounds__(64) k_argmax_final(const float *pv, const int *pi, int *out) {
    const int row = blockIdx.x, lane = threadIdx.x;
    float bv = pv[row * ARGMAX_BLOCKS + lane]; int bi = pi[row * ARGMAX_BLOCKS + lane];
    wave_argmax(bv, bi);
    if (lane == 0) out[row] = bi == 0x7fffffff ? 0 : bi;
}

// ---------------------------------------------------------------------------------------------------------------
// K/V slot moves of one sequence, applied in order (one block per layer x kv head).
__global__ void __launch_bounds__(128) k_kv_move(f16 *const *kl, f16 *const *vl, int seq, int NKV, int n_slots, int HD,
                                                 const int *src, const int *dst, int n) {
    const int layer = blockIdx.x / NKV, kvh = blockIdx.x % NKV;
    f16 *k = kl[layer], *v = vl[layer];
    const size_t base = ((size_t)seq * NKV + kvh) * n_slots;
    for (int i = 0; i < n; ++i) {
        const size_t so = (base + src[i]) * HD, dO = (base + dst[i]) * HD;
        f16 tk = 0, tv = 0;
        if (threadIdx.x < HD) { tk = k[so + threadIdx.x]; tv = v[so + threadIdx.x]; }
        __syncthreads();
        if (threadIdx.x < HD) { k[dO + threadIdx.x] = tk; v[dO + threadIdx.x] = tv; }
        __syncthreads();
    }
}

// Growth of the KV pool with live sequences kept: for kept sequence i (keep[3i] = sequence, keep[3i+1] = first position,
// keep[3i+2] = position count) every position p moves from slot p mod old_slots of the old pool to slot p mod new_slots
// of the new one, for one layer's K and V.  Sixteen bytes per thread; blockIdx.y = kept index * NKV + kv head.
__global__ void __launch_bounds__(256) k_kv_regrid(const f16 *ko, const f16 *vo, f16 *kn, f16 *vn, const int *keep,
                                                   int NKV, int HD, int old_slots, int new_slots) {
    const int ki = blockIdx.y / NKV, kvh = blockIdx.y % NKV;
    const int seq = keep[3 * ki], p0 = keep[3 * ki + 1], np = keep[3 * ki + 2];
    const int per_pos = HD / 8;
    const size_t ob = ((size_t)seq * NKV + kvh) * old_slots, nb = ((size_t)seq * NKV + kvh) * new_slots;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < np * per_pos; i += gridDim.x * blockDim.x) {
        const int p = p0 + i / per_pos, c = (i % per_pos) * 8;
        const size_t so = (ob + p % old_slots) * HD + c, dO = (nb + p % new_slots) * HD + c;
        *(uint4 *)(kn + dO) = *(const uint4 *)(ko + so);
        *(uint4 *)(vn + dO) = *(const uint4 *)(vo + so);
    }
}

// Seeded fill of K/V slots (benchmark stand-in for a long prefill): value = scale * (2 * hash01 - 1).
__global__ void __launch_bounds__(256) k_kv_fill(f16 *const *kl, f16 *const *vl, int seq, int NKV, int n_slots, int HD,
                                                 int first, int n, uint64_t seed, float scale) {
    const int layer = blockIdx.y;
    const size_t per_head = (size_t)n * HD;
    const size_t total = per_head * NKV;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int kvh = (int)(i / per_head);
        const size_t r = i - (size_t)kvh * per_head;
        const int slot = first + (int)(r / HD), d = (int)(r % HD);
        const size_t off = (((size_t)seq * NKV + kvh) * n_slots + slot) * HD + d;
        uint64_t x = seed ^ (((uint64_t)layer << 40) + off);
        x += 0x9E3779B97F4A7C15ull;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        x ^= x >> 31;
        const float u1 = (float)(x & 0xffffff) * (1.0f / 16777216.0f), u2 = (float)((x >> 24) & 0xffffff) * (1.0f / 16777216.0f);
        kl[layer][off] = (f16)(scale * (2.f * u1 - 1.f));
        vl[layer][off] = (f16)(scale * (2.f * u2 - 1.f));
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Multi-query attention for groups of columns of one sequence (tree verification, prefill chunks).  The group's
// visible list is the union ring range [lo, lo + nlin) followed by the shared tree block; one block per (chunk of
// ATT_CH keys, kv head, group) stages the chunk's K (row-major) and V (transposed) in LDS once, and every
// (column, query head) row of the group is scored against it on MFMA: S = Q K^T, per-row mask (the column's own
// ring range and tree-mask bits), chunk-local softmax statistics, O = P V.  Partials use the same layout as
// k_attn_part, so k_attn_combine merges them (with the group's chunk count per column).
struct AttnGroup {
    int first_col, ncols, seq, lo, nlin, tree_base, tree_count, pad;
};

struct AttnMqArgs {
    const float *q;        // [n][NH*HD]
    const f16 *kc, *vc;
    const sp_token *toks;
    const AttnGroup *groups;
    int NH, NKV, HD, n_slots, nchunk;
    float scale;
    float *part;
    int splits;            // blocks per (chunk, kv head, group); block s takes row tiles 4s .. 4s+3
};

template <int HD, int G, int CH>
__global__ void __launch_bounds__(256) k_attn_mq(AttnMqArgs a) {
    constexpr int KP = HD + 8, VP = CH + 8;          // padded rows (halves), 16-byte aligned
    constexpr int NST = CH / 16, NS2 = CH / 32, NP2 = CH / 2;   // key tiles, P.V k-steps, key pairs
    constexpr int ST = HD / 32;                      // MFMA k-steps over head dim
    constexpr int CPR = HD / 8;                      // 16-byte pieces per key row
    constexpr int KPER = CH * CPR / 256;         // K pieces per thread
    constexpr int VPER = CH / 2 * CPR / 256;     // V (key pair, piece) items per thread
    static_assert(KPER * 256 == CH * CPR && VPER * 256 == CH / 2 * CPR, "chunk staging split");
    __shared__ __align__(16) f16 k_s[CH][KP];
    __shared__ __align__(16) f16 vt_s[HD][VP];
    __shared__ __align__(16) f16 p_s[4][16][VP];
    __shared__ int kpos_s[CH];                  // ring position of key j, or -(1 + tree index), or INT_MIN
    __shared__ int clo_s[64], chi_s[64], ctc_s[64];
    __shared__ unsigned long long cmask_s[64];

    const int c = blockIdx.x, kvh = blockIdx.y;
    const int split = blockIdx.z % a.splits;
    const AttnGroup gr = a.groups[blockIdx.z / a.splits];
    const int nvis = gr.nlin + gr.tree_count;
    const int v0 = c * CH;
    if (v0 >= nvis) return;
    const int R = gr.ncols * G;
    if (split * 64 >= R) return;                    // 4 row tiles of 16 rows per block
    const int cnt = min(CH, nvis - v0);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r16 = lane & 15, g4 = lane >> 4;
    const int n_tiles = (R + 15) / 16;
    const int rt = split * 4 + wv;                   // this wave's row tile
    const bool active = rt < n_tiles;
    const size_t head_base = ((size_t)gr.seq * a.NKV + kvh) * a.n_slots;
    const f16x8 zero8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    // visible key j of the chunk (j < cnt): its cache slot and its ring position / tree code (~tree index).  Slots
    // of a chunk are consecutive from a per-block base (ring keys) or from tree_base (tree keys), so one modulo per
    // block and a conditional subtraction per key replace a division per key (branch-free: the selects keep the
    // wave converged).
    const int lin_base = (gr.lo + v0) % a.n_slots;   // slot of visible key v0 when it is a ring key
    auto wrap = [&](int x) {                         // x mod n_slots for 0 <= x < n_slots + CH
        x = x >= a.n_slots ? x - a.n_slots : x;
        return a.n_slots >= CH ? x : x % a.n_slots;
    };
    auto key_at = [&](int j, int &kp) {
        const int vis = v0 + j;
        const bool lin = vis < gr.nlin;
        const int tj = vis - gr.nlin;
        kp = lin ? gr.lo + vis : ~tj;
        return wrap(lin ? lin_base + j : gr.tree_base + tj);
    };

    // ---- every global load before the first LDS store.  Keys past cnt load key 0 of the chunk (clamped address,
    // unconditional load) and are replaced by zeros.  K: item i = key i / CPR, piece i % CPR.  V: item i = key pair
    // i % (CH / 2), piece i / (CH / 2) (see the transposed store below).
    f16x8 kf[KPER], vf[VPER][2];
#pragma unroll
    for (int i = 0; i < KPER; ++i) {
        const int idx = tid + 256 * i, j = idx / CPR, ch = idx - j * CPR;
        int kp;
        const int slot = key_at(j < cnt ? j : 0, kp);
        kf[i] = *(const f16x8 *)(a.kc + (head_base + slot) * HD + ch * 8);
    }
#pragma unroll
    for (int i = 0; i < VPER; ++i) {
        const int idx = tid + 256 * i, kp2 = idx % NP2, ch = idx / NP2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int j = 2 * kp2 + h;
            int kp;
            const int slot = key_at(j < cnt ? j : 0, kp);
            vf[i][h] = *(const f16x8 *)(a.vc + (head_base + slot) * HD + ch * 8);
        }
    }
    // Q fragments (A operand) of row rt*16 + r16, dims 32s + 8*g4 .. +8, from a clamped row; rows past R are zero.
    // fp16 values and their fp16 remainders (split_f16), two MFMAs per score step: Q enters at fp32-class precision
    f16x8 qa[ST], ql[ST];
    {
        const int row = rt * 16 + r16;
        const int rowc = row < R ? row : R - 1;
        const int col = rowc / G, h = rowc - col * G;
        const float *qp = a.q + (size_t)(gr.first_col + col) * a.NH * HD + (kvh * G + h) * HD + 8 * g4;
        f32x4 x[ST][2];
#pragma unroll
        for (int s = 0; s < ST; ++s) {
            x[s][0] = *(const f32x4 *)(qp + 32 * s);
            x[s][1] = *(const f32x4 *)(qp + 32 * s + 4);
        }
        const float qs = row < R ? a.scale : 0.f;
#pragma unroll
        for (int s = 0; s < ST; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                f16 hi, lo;
                split_f16(x[s][e >> 2][e & 3] * qs, hi, lo);
                qa[s][e] = hi;
                ql[s][e] = lo;
            }
    }
    const sp_token ct = a.toks[gr.first_col + min(tid, gr.ncols - 1)];

    // ---- LDS: K row-major; V transposed, two keys per dword: lane (key pair p, piece ch) writes the dword holding
    // keys 2p, 2p+1 of dims 8ch .. 8ch+7.  A wave's 64 items hit 64 distinct banks (64-key chunks: 32 pairs x 2
    // pieces whose rows are 8 * 36 dwords apart; 128-key chunks: 64 consecutive pairs of one row).
#pragma unroll
    for (int i = 0; i < KPER; ++i) {
        const int idx = tid + 256 * i, j = idx / CPR, ch = idx - j * CPR;
        *(f16x8 *)&k_s[j][ch * 8] = j < cnt ? kf[i] : zero8;
    }
#pragma unroll
    for (int i = 0; i < VPER; ++i) {
        const int idx = tid + 256 * i, kp2 = idx % NP2, ch = idx / NP2;
        const f16x8 va = 2 * kp2 < cnt ? vf[i][0] : zero8, vb = 2 * kp2 + 1 < cnt ? vf[i][1] : zero8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const f16x2 pr = (f16x2){va[e], vb[e]};
            *(f16x2 *)&vt_s[ch * 8 + e][2 * kp2] = pr;
        }
    }
    if (tid < CH) {
        int kp = INT_MIN;
        if (tid < cnt) (void)key_at(tid, kp);
        kpos_s[tid] = kp;
    }
    if (tid < gr.ncols) { clo_s[tid] = ct.ctx_lo; chi_s[tid] = ct.ctx_hi; ctc_s[tid] = ct.tree_count; cmask_s[tid] = ct.tree_mask; }
    __syncthreads();
    if (!active) return;                             // no block-wide barrier follows

    // ---- S = Q K^T: 4 slot tiles of 16; lane holds S[row 4*g4 + j][slot 16*st + r16]
    f32x4 sc[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) {
        f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < ST; ++s) {
            const f16x8 kb = *(const f16x8 *)&k_s[16 * st + r16][32 * s + 8 * g4];
            acc = mfma16(qa[s], kb, acc);
            acc = mfma16(ql[s], kb, acc);
        }
        sc[st] = acc;
    }
    // ---- mask, chunk-local max / exp / sum per row.  The key codes of the lane's 4 slot tiles and the range / tree
    // bits of its 4 rows are read once; the mask is selects only (ring key: inside the column's range; tree key:
    // its bit set in the column's ancestor mask; padding key: never).
    // A chunk of ring keys that every column of the group sees whole (the prefix of a tree pass): the mask keeps
    // every key, so only rows past R are masked (the same scores as the per-key test below gives there).
    bool whole = v0 + CH <= gr.nlin;
    if (whole) {
        const int k_lo = gr.lo + v0, k_hi = gr.lo + v0 + CH - 1;
        whole = __all(lane >= gr.ncols || (clo_s[lane] <= k_lo && chi_s[lane] >= k_hi));
    }
    float mrow[4], lrow[4];
    if (whole) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool live = rt * 16 + 4 * g4 + j < R;
#pragma unroll
            for (int st = 0; st < NST; ++st) sc[st][j] = live ? sc[st][j] : -INFINITY;
        }
    } else {
        int kpv[NST];
#pragma unroll
        for (int st = 0; st < NST; ++st) kpv[st] = kpos_s[16 * st + r16];
        int clo[4], chi[4], ctc[4];
        unsigned long long cmk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = rt * 16 + 4 * g4 + j;
            const int col = row < R ? row / G : 0;
            clo[j] = clo_s[col]; chi[j] = chi_s[col]; ctc[j] = ctc_s[col]; cmk[j] = cmask_s[col];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = rt * 16 + 4 * g4 + j;
#pragma unroll
            for (int st = 0; st < NST; ++st) {
                const int kp = kpv[st];
                const int tj = ~kp;                      // tree index of a tree key (kp = ~tj < 0)
                const bool in_ring = (kp >= clo[j]) & (kp <= chi[j]);
                const bool in_tree = (tj < ctc[j]) & (((cmk[j] >> (tj & 63)) & 1ull) != 0);
                const bool ok = (row < R) & (kp != INT_MIN) & (kp >= 0 ? in_ring : in_tree);
                sc[st][j] = ok ? sc[st][j] : -INFINITY;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float m = -INFINITY;
#pragma unroll
        for (int st = 0; st < NST; ++st) m = fmaxf(m, sc[st][j]);
        m = row16_max(m);
        float l = 0.f;
#pragma unroll
        for (int st = 0; st < NST; ++st) {
            // the hardware exponential (one v_exp_f32 of x log2 e): P is rounded to fp16 before P V anyway
            const float e = (m == -INFINITY || sc[st][j] == -INFINITY) ? 0.f : __expf(sc[st][j] - m);
            sc[st][j] = e;
            l += e;
        }
        l = row16_sum(l);
        mrow[j] = m; lrow[j] = l;
    }
    // ---- P (fp16) to this wave's LDS rows, read back as the A operand (LDS is in order within a wave)
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
        for (int j = 0; j < 4; ++j) p_s[wv][4 * g4 + j][16 * st + r16] = (f16)sc[st][j];
    __builtin_amdgcn_wave_barrier();
    f16x8 pa[NS2];
#pragma unroll
    for (int s2 = 0; s2 < NS2; ++s2) pa[s2] = *(const f16x8 *)&p_s[wv][r16][32 * s2 + 8 * g4];
    // ---- O = P V over HD/16 dim tiles; lane holds O[row 4*g4 + j][dim 16*dt + r16]
    f32x4 o[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) {
        o[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < NS2; ++s2) {
            const f16x8 vb = *(const f16x8 *)&vt_s[16 * dt + r16][32 * s2 + 8 * g4];
            o[dt] = mfma16(pa[s2], vb, o[dt]);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = rt * 16 + 4 * g4 + j;
        if (row < R) {
            const int col = row / G, h = row - col * G;
            float *out = a.part + (((size_t)(gr.first_col + col) * a.NH + kvh * G + h) * a.nchunk + c) * part_floats(HD);
            f16 *oh = (f16 *)(out + 2);
            const float il = lrow[j] > 0.f ? 1.f / lrow[j] : 0.f;
#pragma unroll
            for (int dt = 0; dt < HD / 16; ++dt) oh[16 * dt + r16] = (f16)(o[dt][j] * il);
            if (r16 == 0) { out[0] = mrow[j]; out[1] = lrow[j]; }
        }
    }
}
