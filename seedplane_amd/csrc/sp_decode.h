// Persistent single-column decode step: the whole Qwen2 forward for one new token (all layers, final norm, LM head,
// argmax) in one cooperative launch of one 512-thread block per CU.
//
// Why: at batch 1 the step is a chain of ~260 small dependent kernels; on this GPU a dependent kernel costs about
// 4 us however little it reads.  Here the chain becomes 6 hand-offs per layer between co-resident blocks.
//
// Hand-off ("LL" words): every value that crosses blocks is written as one 64-bit word, payload in the low 32 bits
// and a 32-bit tag in the high bits, with relaxed agent-scope atomic stores; consumers poll the words with relaxed
// agent-scope atomic loads until every tag matches.  A word is single-copy atomic, so no fence is needed (an
// agent-scope fence writes back / invalidates a whole XCD L2).  Tag = (launch id << 12) | hop id: every hop of a
// launch writes a region of its own (nothing is overwritten inside a launch), and a stale word from an earlier
// launch carries an older launch id.  Every wait is bounded; a timeout sets the error word and every block exits.
//
// The residual stream x is private to every block (each block applies the same partial sums in the same order), so
// only partial sums travel.  Per layer (S1 / S3 / S5 = k-splits of qkv / o / down):
//   P1  x += down partials; xn = norm(x); qkv items (row group, k-split)          -> qkv partials
//   P2  attention items (kv head, chunk of ATT_CH keys): q / k / v from the qkv partials + bias, RoPE, the new key
//       and value taken from registers and written to their cache slot         -> {m, l, acc} per query head
//   P2b combine (one block per query head)                                     -> attention output
//   P3  o_proj items                                                           -> o partials
//   P4  x += o partials; xn = norm(x); gate_up pair items, SiLU(gate) * up      -> act (fp16)
//   P5  down items                                                             -> down partials
// then x += down partials, final norm, LM head items (logits + per-block argmax), block 0 reduces the argmax.
//
// Replaces, for one decode column, the same reference computation as the kernel chain in sp_engine::step
// (seedplane/qwen_engine.py:117-148).
#pragma once
#include "sp_attn.h"
#include "sp_gemv.h"

namespace mk {

constexpr int NT = 256, NWV = NT / 64;     // one wave per SIMD: 512 registers per wave (VGPR + AGPR)
constexpr long MAX_POLLS = 1l << 21;

// Phase timestamps for profiling builds (-DSP_DECODE_TRACE): thread 0 of each block records the 100 MHz clock at
// phase boundaries of the first layers.  Compiled out otherwise.
#ifdef SP_DECODE_TRACE
__device__ unsigned long long trace_buf[1024][64];
#define MK_TRACE(ev) do { if (threadIdx.x == 0 && (ev) < 32) trace_buf[blockIdx.x][(ev)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#define MK_TRACE_ATT(ev) do { if (threadIdx.x == 0) trace_buf[blockIdx.x][32 + (ev)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define MK_TRACE(ev) do { } while (0)
#define MK_TRACE_ATT(ev) do { } while (0)
#endif
typedef unsigned long long u64;

struct Mat {
    const uint8_t *w;
    const f16 *sz;
    int nkt;         // k-tiles per row group
    int groups;      // row groups (units for a paired matrix)
    int rows;        // real rows (paired: rows of one half)
};

struct LayerW {
    Mat qkv, o, gu, down;
    const float *qkv_b, *in_norm, *post_norm;
    f16 *kc, *vc;    // this layer's cache [seq][kvh][slot][HD]
};

struct Args {
    const LayerW *layers;
    Mat embed, head;
    const float *final_norm, *inv_freq;
    const sp_token *tok;
    int L, H, NH, NKV, I, V, n_slots;
    float eps, scale;
    int S1, S3, S5;
    u64 *ll;                 // LL region base
    size_t lw_qkv, lw_part, lw_attn, lw_o, lw_act, lw_d, lw_layer;   // per-layer region offsets / stride (words)
    size_t lw_am;            // argmax words (after all layers)
    int nchunk_max;
    unsigned tag0;
    unsigned *err;
    float *logits;           // may be NULL
    int *out_id;
};

__device__ __forceinline__ void ll_put(u64 *p, unsigned tag, unsigned payload) {
    __hip_atomic_store(p, ((u64)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 ll_peek(const u64 *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool err_set(unsigned *err) {
    return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Wait until words src[0..n) carry `tag`; payloads go to dst[0..n) (LDS, 32-bit).  Block-wide; returns false (in
// every thread) on timeout or when another block reported one.  Each thread polls GATHER_PER consecutive words
// (one address register, immediate offsets).
constexpr int GATHER_PER = 18;
__device__ __forceinline__ bool ll_gather(unsigned *err, const u64 *src, int n, unsigned tag, unsigned *dst) {
    for (int base = 0; base < n; base += NT * GATHER_PER) {
        const int w0 = base + (int)threadIdx.x * GATHER_PER;
        const u64 *p = src + w0;
        unsigned pending = 0;
#pragma unroll
        for (int j = 0; j < GATHER_PER; ++j)
            if (w0 + j < n) pending |= 1u << j;
        bool fail = false;
        long polls = 0;
        while (pending) {
            u64 w[GATHER_PER];
#pragma unroll
            for (int j = 0; j < GATHER_PER; ++j)
                if (pending & (1u << j)) w[j] = ll_peek(p + j);
#pragma unroll
            for (int j = 0; j < GATHER_PER; ++j)
                if ((pending & (1u << j)) && (unsigned)(w[j] >> 32) == tag) {
                    dst[w0 + j] = (unsigned)w[j];
                    pending &= ~(1u << j);
                }
            if (!pending) break;
            ++polls;
            if ((polls & 63) == 0 && (polls > MAX_POLLS || err_set(err))) {
                if (polls > MAX_POLLS) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                fail = true;
                break;
            }
        }
        if (__syncthreads_or(fail)) return false;
    }
    return true;
}

// ----------------------------------------------------------------------------------------------- shared memory
constexpr int MAX_H = 2048, MAX_K = 9216, STAGE = 4608, MAX_G = 8, MAX_CHUNKS = 64;
constexpr int RING_BYTES = 96 * 1024, RING_WAVE = RING_BYTES / NWV;
struct AttnLds {
    __align__(16) f16 qh[16][128 + 8];         // scaled, rotated queries of the group (rows >= G zero)
    __align__(16) f16 k_s[ATT_CH][128 + 8];   // keys of the chunk, row-major (B operand of S = Q K^T)
    __align__(16) f16 vt_s[128][ATT_CH + 8];  // values of the chunk, transposed (B operand of O = P V)
    __align__(16) f16 p_s[16][ATT_CH + 8];    // softmax numerators, row = query head (A operand of O = P V)
    float tmp[10 * 128];                      // q / k / v rows of the group (+ bias) before RoPE
    float rc[64], rs[64];                     // RoPE cos / sin of this position
    float amax[NWV + 1][16], asum[NWV][16];   // per-wave row maxima / sums of the chunk softmax
    __align__(16) f16 kn[128], vn[128];
};
struct Smem {
    float x[MAX_H];             // residual stream (private copy)
    __align__(16) f16 a[MAX_K]; // A operand of the current GEMV (fp16, absolute k index, zero past K)
    unsigned stage[STAGE];      // gathered payloads
    f32x4 red[NWV * 2 * 64];    // wave partials of one GEMV item
    float w[MAX_CHUNKS];
    float redf[16];
    union {
        AttnLds att;                                   // attention items
        __align__(16) unsigned char ring[RING_BYTES];  // weight tiles prefetched by DMA, one region per wave
    } u;
};
__shared__ Smem S;

// xn = fp16((x * rsqrt(mean(x^2) + eps)) * w) into S.a[0..H), zeros up to kpad
__device__ void norm_to_a(const float *w, int H, int kpad, float eps) {
    Smem &s = S;
    float ss = 0.f;
    for (int k = threadIdx.x; k < H; k += NT) ss += s.x[k] * s.x[k];
    ss = block_sum(ss, s.redf);
    const float rs = 1.0f / sqrtf(ss / (float)H + eps);
    for (int k = threadIdx.x; k < kpad; k += NT) s.a[k] = k < H ? (f16)((s.x[k] * rs) * w[k]) : (f16)0.f;
    __syncthreads();
}

// ------------------------------------------------------------------------------------------ GEMV phases
// A phase's items (row group or gate/up pair `unit`, k-split `sp`) are dealt round-robin to blocks.  A block takes
// its items in batches of up to 8; inside a batch wave w works on item w % nb and k-tiles kt0 + sub, kt0 + sub +
// nsub, ... (sub = w / nb, nsub = waves on that item).  The first batch's weight tiles are loaded into registers
// before the phase input is awaited, so HBM latency overlaps the hand-off; waves of an item are then reduced
// through LDS in wave order (deterministic).
template <int FMT, int RG> struct MaxT { static constexpr int V = (FMT == 3 ? 4 : 8) / RG; };   // tiles per wave per round

template <int FMT, int RG>
struct WaveTiles {
    static constexpr int M = MaxT<FMT, RG>::V;
    u32x4 wt[M][RG];
    uint32_t s8[M][RG];
    u32x4 s4[M][RG];
};

struct WaveJob {
    int unit, sp, kt0, nsub, count;     // tiles kt0 + j * nsub, j < count
};

template <int FMT, int RG>
__device__ __forceinline__ void tiles_load(const Mat &m, const WaveJob &j, int first, int round, WaveTiles<FMT, RG> &t) {
    constexpr int M = MaxT<FMT, RG>::V;
    const int lane = threadIdx.x & 63, r = lane & 15;
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int idx = first + round * M + i;
        if (idx >= j.count) break;
        const int kt = j.kt0 + idx * j.nsub;
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const size_t tile = (size_t)(j.unit * RG + rg) * m.nkt + kt;
            t.wt[i][rg] = __builtin_nontemporal_load((const u32x4 *)(m.w + tile * TILE_BYTES) + lane);
            if constexpr (FMT == 2) t.s8[i][rg] = *((const uint32_t *)(m.sz + tile * 32) + r);
            if constexpr (FMT == 3) t.s4[i][rg] = *((const u32x4 *)(m.sz + tile * 128) + r);
        }
    }
}

template <int FMT, int RG>
__device__ __forceinline__ void tiles_mac(const WaveJob &j, int first, int round, const WaveTiles<FMT, RG> &t, f32x4 acc[RG]);

// Number of items block b holds in a phase of `items` items.
__device__ __forceinline__ int my_items(int items) {
    return items > (int)blockIdx.x ? (items - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
}

// ------------------------------------------------------------------------------------------ DMA ring
// Weight tiles can be copied straight into LDS (global_load_lds_dwordx4: lane l's 16 bytes land at the wave's LDS
// base + 16 l, no registers involved) well before a phase's input arrives: each wave owns RING_WAVE bytes and
// prefetches the first CAP tiles (or gate/up pairs) of its job in the next phase.
template <int FMT> struct SideBytes { static constexpr int V = FMT == 1 ? 0 : FMT == 2 ? 64 : 256; };
template <int FMT, int RG> struct Ring {
    static constexpr int CAP = RING_WAVE / (RG * (TILE_BYTES + SideBytes<FMT>::V));
    static constexpr int SIDE = CAP * RG * TILE_BYTES;     // offset of the side data inside a wave region
};

__device__ __forceinline__ void dma16(const void *g, unsigned char *l) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)l, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *g, unsigned char *l) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)l, 4, 0, 0);
}

template <int FMT, int RG>
__device__ __forceinline__ void ring_issue(const Mat &m, const WaveJob &j, int npf) {
    unsigned char *base = S.u.ring + (threadIdx.x >> 6) * RING_WAVE;
    const int lane = threadIdx.x & 63;
    for (int idx = 0; idx < npf; ++idx) {
        const int kt = j.kt0 + idx * j.nsub;
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const size_t tile = (size_t)(j.unit * RG + rg) * m.nkt + kt;
            const int slot = idx * RG + rg;
            dma16(m.w + tile * TILE_BYTES + lane * 16, base + slot * TILE_BYTES);
            if constexpr (FMT == 2) { if (lane < 16) dma4(m.sz + tile * 32 + lane * 2, base + Ring<FMT, RG>::SIDE + slot * 64); }
            if constexpr (FMT == 3) { if (lane < 16) dma16(m.sz + tile * 128 + lane * 8, base + Ring<FMT, RG>::SIDE + slot * 256); }
        }
    }
}

// One tile (or gate/up pair) k-tile kt: codes wt[rg], side data s8 / s4, A fragments from S.a.
template <int FMT, int RG>
__device__ __forceinline__ void mac_tile(int kt, const u32x4 *wt, const uint32_t *s8, const u32x4 *s4, f32x4 acc[RG]) {
    constexpr int KT = TileGeom<FMT>::KT, ST = TileGeom<FMT>::STEPS;
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const f16x8 zero8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
    for (int st = 0; st < ST; ++st) {
        const f16x8 xa = r == 0 ? *(const f16x8 *)(S.a + kt * KT + st * 32 + 8 * g) : zero8;
        f32x4 xs = (f32x4){0.f, 0.f, 0.f, 0.f};
        if constexpr (FMT == 3) xs = mfma16(xa, ones8, xs);
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const f16x8 b = unpack_step<FMT>(wt[rg], st);
            if constexpr (FMT == 1) {
                acc[rg] = mfma16(xa, b, acc[rg]);
            } else if constexpr (FMT == 2) {
                const uint32_t d = s8[rg];
                const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(st == 0 ? (d & 0xffffu) : (d >> 16)));
                acc[rg] += scale * mfma16(xa, b, (f32x4){0.f, 0.f, 0.f, 0.f});
            } else {
                uint32_t d;
                if (st == 0) d = s4[rg].x; else if (st == 1) d = s4[rg].y; else if (st == 2) d = s4[rg].z; else d = s4[rg].w;
                const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                const float zero = (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
                const f32x4 dd = mfma16(xa, b, (f32x4){0.f, 0.f, 0.f, 0.f});
                acc[rg] += scale * (dd - zero * xs);
            }
        }
    }
}

template <int FMT, int RG>
__device__ __forceinline__ void ring_mac(const WaveJob &j, int npf, f32x4 acc[RG]) {
    const unsigned char *base = S.u.ring + (threadIdx.x >> 6) * RING_WAVE;
    const int lane = threadIdx.x & 63, r = lane & 15;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");      // this wave's DMA copies have landed
    for (int idx = 0; idx < npf; ++idx) {
        u32x4 wt[RG], s4[RG];
        uint32_t s8[RG];
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const int slot = idx * RG + rg;
            wt[rg] = *(const u32x4 *)(base + slot * TILE_BYTES + lane * 16);
            if constexpr (FMT == 2) s8[rg] = *(const uint32_t *)(base + Ring<FMT, RG>::SIDE + slot * 64 + r * 4);
            if constexpr (FMT == 3) s4[rg] = *(const u32x4 *)(base + Ring<FMT, RG>::SIDE + slot * 256 + r * 16);
        }
        mac_tile<FMT, RG>(j.kt0 + idx * j.nsub, wt, s8, s4, acc);
    }
}

template <int FMT, int RG>
__device__ __forceinline__ void tiles_mac(const WaveJob &j, int first, int round, const WaveTiles<FMT, RG> &t, f32x4 acc[RG]) {
    constexpr int M = MaxT<FMT, RG>::V;
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int idx = first + round * M + i;
        if (idx >= j.count) break;
        mac_tile<FMT, RG>(j.kt0 + idx * j.nsub, t.wt[i], t.s8[i], t.s4[i], acc);
    }
}

// One batch of a block's items in a GEMV phase: the wave's job, how many of its tiles sit in the ring, and the
// register-prefetched first round of the rest.
template <int FMT, int RG>
struct Phase {
    WaveJob j;
    WaveTiles<FMT, RG> t;
    int nb, npf;
};

// Wave job for batch b0 of the block's `mine` items (see the work decomposition above).
template <int FMT, int RG>
__device__ __forceinline__ WaveJob phase_job(const Mat &m, int nsplit, int b0, int mine, int &nb) {
    const int wv = threadIdx.x >> 6;
    nb = min(NWV, mine - b0);
    const int il = wv % nb, sub = wv / nb, nsub = (NWV - il + nb - 1) / nb;
    const int it = (int)blockIdx.x + (b0 + il) * (int)gridDim.x;
    WaveJob j;
    j.unit = it / nsplit; j.sp = it - j.unit * nsplit;
    const int k0 = (int)((long)m.nkt * j.sp / nsplit), k1 = (int)((long)m.nkt * (j.sp + 1) / nsplit);
    j.kt0 = k0 + sub; j.nsub = nsub;
    j.count = k1 - k0 > sub ? (k1 - k0 - sub + nsub - 1) / nsub : 0;
    return j;
}

// DMA-prefetch this block's first batch of a phase into the ring (call when the ring is free).
template <int FMT, int RG>
__device__ __forceinline__ void phase_prefetch(const Mat &m, int nsplit) {
    const int mine = my_items(m.groups * nsplit);
    if (mine == 0) return;
    int nb;
    const WaveJob j = phase_job<FMT, RG>(m, nsplit, 0, mine, nb);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");    // earlier LDS reads of the ring are complete
    ring_issue<FMT, RG>(m, j, min(j.count, Ring<FMT, RG>::CAP));
}

// Sets up batch b0 and issues the register loads of the first round past the ring-resident tiles.
template <int FMT, int RG>
__device__ __forceinline__ void phase_load(const Mat &m, int nsplit, int b0, int mine, bool prefetched, Phase<FMT, RG> &p) {
    p.j = phase_job<FMT, RG>(m, nsplit, b0, mine, p.nb);
    p.npf = prefetched && b0 == 0 ? min(p.j.count, Ring<FMT, RG>::CAP) : 0;
    tiles_load<FMT, RG>(m, p.j, p.npf, 0, p.t);
}

// Multiply-accumulates the batch against S.a -- ring tiles first, then rounds of M register tiles (software
// pipelined over two register sets) -- and reduces every item over its waves.  Returns true in lanes 0..15 of the
// wave that reduced an item; out[rg] = row unit * 16 + lane.
template <int FMT, int RG>
__device__ __forceinline__ bool phase_finish(const Mat &m, Phase<FMT, RG> &p, float out[RG]) {
    constexpr int M = MaxT<FMT, RG>::V;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    f32x4 acc[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) acc[rg] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (RG == 2) MK_TRACE_ATT(6);
    if (p.npf > 0) ring_mac<FMT, RG>(p.j, p.npf, acc);
    if (RG == 2) MK_TRACE_ATT(7);
    const int rounds = (p.j.count - p.npf + M - 1) / M;
    WaveTiles<FMT, RG> t1;
    for (int r = 0; r < rounds; r += 2) {
        if (r + 1 < rounds) tiles_load<FMT, RG>(m, p.j, p.npf, r + 1, t1);
        tiles_mac<FMT, RG>(p.j, p.npf, r, p.t, acc);
        if (r + 2 < rounds) tiles_load<FMT, RG>(m, p.j, p.npf, r + 2, p.t);
        if (r + 1 < rounds) tiles_mac<FMT, RG>(p.j, p.npf, r + 1, t1, acc);
    }
    if (RG == 2) MK_TRACE_ATT(8);
    __syncthreads();                          // the previous batch's readers of S.red are done
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) S.red[(wv * RG + rg) * 64 + lane] = acc[rg];
    __syncthreads();
    if (RG == 2) MK_TRACE_ATT(9);
    if (wv >= p.nb) return false;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {         // wave il reduces item il over its waves il, il + nb, ...
        f32x4 v = S.red[(wv * RG + rg) * 64 + lane];
        for (int w2 = wv + p.nb; w2 < NWV; w2 += p.nb) v += S.red[(w2 * RG + rg) * 64 + lane];
        out[rg] = v[0];                       // D row 0 (the column) is register 0 of lanes 0..15
    }
    return lane < 16;
}

// x[k] += sum over splits of the gathered partials (fixed split order), k < H
__device__ void add_partials(int nsplit, int H) {
    for (int k = threadIdx.x; k < H; k += NT) {
        float t = __uint_as_float(S.stage[k]);
        for (int sp = 1; sp < nsplit; ++sp) t += __uint_as_float(S.stage[sp * H + k]);
        S.x[k] += t;
    }
    __syncthreads();
}

// The fields the attention steps need, copied out of the kernel arguments (passed by value).
struct AttnCtx {
    int NH, NKV, S1, n_slots, nchunk_max;
    float scale;
    size_t lw_qkv, lw_part, lw_attn;
    const float *inv_freq;
    unsigned *err;
};

// LL position of qkv row `row` of split sp: group-major, so an attention item's q rows, key row and value row of
// every split are one contiguous run: [group][split][G*HD q | HD k | HD v].
__device__ __forceinline__ size_t qkv_pos(int row, int sp, int nsplit, int NH, int NKV, int HD) {
    const int G = NH / NKV;
    int g, off;
    if (row < NH * HD) { g = row / (G * HD); off = row - g * G * HD; }
    else if (row < (NH + NKV) * HD) { const int r2 = row - NH * HD; g = r2 / HD; off = G * HD + (r2 - g * HD); }
    else { const int r2 = row - (NH + NKV) * HD; g = r2 / HD; off = (G + 1) * HD + (r2 - g * HD); }
    return ((size_t)g * nsplit + sp) * (G + 2) * HD + off;
}

// Attention item (kv head g, chunk c of ATT_CH visible keys) of one layer.  Everything that does not depend on
// this step's q / k / v -- the chunk's cached keys / values into LDS (values transposed), the qkv bias, the RoPE
// cos / sin of this position -- is done before the q / k / v partials are awaited.  The new key / value (last
// visible position) come from the partials (+ bias, RoPE); the item owning the last chunk writes them to their
// slot.  S = Q K^T and O = P V run on MFMA (rows = the group's query heads), one key tile / two dim tiles per wave.
// Output: {m, l, acc[HD]} per query head of the group as LL words.
template <int HD>
__device__ __forceinline__ bool attn_item(const AttnCtx a, const LayerW &W, u64 *R, unsigned tg, const sp_token &t,
                                          int g, int c, int nch) {
    Smem &s = S;
    const int NH = a.NH, NKV = a.NKV, G = NH / NKV;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nlin = t.ctx_hi - t.ctx_lo + 1;
    const int v0 = c * ATT_CH, cnt = min(ATT_CH, nlin - v0);
    const size_t head_base = ((size_t)t.seq * NKV + g) * a.n_slots;
    constexpr int HALF = HD / 2, CPR = HD / 8, PER = (ATT_CH * CPR + NT - 1) / NT;
    constexpr int NB_PER = (10 * HD + NT - 1) / NT;               // bias values per thread ((G + 2) * HD <= 10 HD)
    const int qrow0 = g * G * HD, krow0 = NH * HD + g * HD, vrow0 = (NH + NKV) * HD + g * HD;
    // ---- independent of this step: K / V chunk, bias, rope table
    f16x8 kr[PER], vr[PER];
    float bias[NB_PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = threadIdx.x + i * NT, jr = e / CPR, ch = e - jr * CPR;
        const int kp = t.ctx_lo + v0 + jr;
        if (e < ATT_CH * CPR && jr < cnt && kp != t.ctx_hi) {
            const size_t off = (head_base + kp % a.n_slots) * HD + ch * 8;
            kr[i] = *(const f16x8 *)(W.kc + off);
            vr[i] = *(const f16x8 *)(W.vc + off);
        }
    }
#pragma unroll
    for (int i = 0; i < NB_PER; ++i) {
        const int e = threadIdx.x + i * NT;
        const int row = e < G * HD ? qrow0 + e : (e < (G + 1) * HD ? krow0 + e - G * HD : vrow0 + e - (G + 1) * HD);
        bias[i] = e < (G + 2) * HD ? W.qkv_b[row] : 0.f;
    }
    if ((int)threadIdx.x < HALF) {
        const float ph = (float)t.pos * a.inv_freq[threadIdx.x];
        s.u.att.rc[threadIdx.x] = cosf(ph);
        s.u.att.rs[threadIdx.x] = sinf(ph);
    }
    const f16x8 zero8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = threadIdx.x + i * NT, jr = e / CPR, ch = e - jr * CPR;
        if (e < ATT_CH * CPR) {
            const bool live = jr < cnt && t.ctx_lo + v0 + jr != t.ctx_hi;   // the new key is filled in below
            const f16x8 kk = live ? kr[i] : zero8, vv = live ? vr[i] : zero8;
            *(f16x8 *)&s.u.att.k_s[jr][ch * 8] = kk;
#pragma unroll
            for (int q = 0; q < 8; ++q) s.u.att.vt_s[ch * 8 + q][jr] = vv[q];
        }
    }
    MK_TRACE_ATT(0);
    // ---- this step's q / k / v partials
    const int nw = a.S1 * (G + 2) * HD;
    if (!ll_gather(a.err, R + a.lw_qkv + (size_t)g * nw, nw, tg | 1, s.stage)) return false;
    MK_TRACE_ATT(1);
    float *tmp = s.u.att.tmp;
#pragma unroll
    for (int i = 0; i < NB_PER; ++i) {
        const int e = threadIdx.x + i * NT;
        if (e < (G + 2) * HD) {
            float v = __uint_as_float(s.stage[e]);
            for (int sp = 1; sp < a.S1; ++sp) v += __uint_as_float(s.stage[sp * (G + 2) * HD + e]);
            tmp[e] = v + bias[i];
        }
    }
    __syncthreads();
    MK_TRACE_ATT(2);
    // RoPE (non-interleaved halves) on the G query heads (-> fp16, scaled) and the key; the value as is
    for (int i = threadIdx.x; i < (G + 1) * HALF; i += NT) {
        const int head = i / HALF, j = i - head * HALF;
        const float cs = s.u.att.rc[j], sn = s.u.att.rs[j];
        const float x1 = tmp[head * HD + j], x2 = tmp[head * HD + j + HALF];
        const float o1 = __fadd_rn(__fmul_rn(x1, cs), __fmul_rn(-x2, sn));
        const float o2 = __fadd_rn(__fmul_rn(x2, cs), __fmul_rn(x1, sn));
        if (head < G) { s.u.att.qh[head][j] = (f16)(o1 * a.scale); s.u.att.qh[head][j + HALF] = (f16)(o2 * a.scale); }
        else { s.u.att.kn[j] = (f16)o1; s.u.att.kn[j + HALF] = (f16)o2; }
    }
    for (int i = threadIdx.x; i < HD; i += NT) s.u.att.vn[i] = (f16)tmp[(G + 1) * HD + i];
    for (int i = threadIdx.x; i < (16 - G) * HD; i += NT) s.u.att.qh[G + i / HD][i % HD] = (f16)0.f;
    __syncthreads();
    const int jn = t.ctx_hi - t.ctx_lo - v0;      // row of the new key in this chunk (if any)
    if (jn >= 0 && jn < cnt) {
        for (int i = threadIdx.x; i < HD; i += NT) { s.u.att.k_s[jn][i] = s.u.att.kn[i]; s.u.att.vt_s[i][jn] = s.u.att.vn[i]; }
    }
    if (c == nch - 1) {                           // this item owns the new position: write its key / value
        for (int i = threadIdx.x; i < HD; i += NT) {
            W.kc[(head_base + t.slot) * HD + i] = s.u.att.kn[i];
            W.vc[(head_base + t.slot) * HD + i] = s.u.att.vn[i];
        }
    }
    __syncthreads();
    MK_TRACE_ATT(3);
    // ---- S = Q K^T: wave w takes key tile w (16 keys); lane l holds rows 4 (l / 16) + j, key l % 16
    constexpr int ST = HD / 32, NDT = HD / 16;
    static_assert(ATT_CH == 16 * NWV, "one key tile per wave");
    const int r16 = lane & 15, g4 = lane >> 4;
    f32x4 sc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < ST; ++st)
        sc = mfma16(*(const f16x8 *)&s.u.att.qh[r16][st * 32 + g4 * 8], *(const f16x8 *)&s.u.att.k_s[wv * 16 + r16][st * 32 + g4 * 8], sc);
    const bool live = wv * 16 + r16 < cnt;
#pragma unroll
    for (int j = 0; j < 4; ++j) {                 // per-row max over this wave's 16 keys
        float m = live ? sc[j] : -INFINITY;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, SP_WAVE));
        if (r16 == 0) s.u.att.amax[wv][4 * g4 + j] = m;
    }
    __syncthreads();
    float lsum[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int h = 4 * g4 + j;
        float M = s.u.att.amax[0][h];
#pragma unroll
        for (int w2 = 1; w2 < NWV; ++w2) M = fmaxf(M, s.u.att.amax[w2][h]);
        const float pe = live ? expf(sc[j] - M) : 0.f;
        s.u.att.p_s[h][wv * 16 + r16] = (f16)pe;
        float l = pe;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) l += __shfl_xor(l, o, SP_WAVE);
        lsum[j] = l;
        if (wv == 0 && r16 == 0) s.u.att.amax[NWV][h] = M;
    }
    if (r16 == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s.u.att.asum[wv][4 * g4 + j] = lsum[j];
    }
    __syncthreads();
    // ---- O = P V: wave w takes dim tiles w, w + NWV, ...
    u64 *P0 = R + a.lw_part;
#pragma unroll
    for (int dt = wv; dt < NDT; dt += NWV) {
        f32x4 ov = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < ATT_CH / 32; ++ks)
            ov = mfma16(*(const f16x8 *)&s.u.att.p_s[r16][ks * 32 + g4 * 8], *(const f16x8 *)&s.u.att.vt_s[dt * 16 + r16][ks * 32 + g4 * 8], ov);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int h = 4 * g4 + j;
            if (h < G) ll_put(P0 + ((size_t)(g * G + h) * a.nchunk_max + c) * (HD + 2) + 2 + dt * 16 + r16, tg | 2, __float_as_uint(ov[j]));
        }
    }
    if (wv == 0 && lane < G) {                    // m and l of query head `lane` (l summed over waves in order)
        float L = s.u.att.asum[0][lane];
        for (int w2 = 1; w2 < NWV; ++w2) L += s.u.att.asum[w2][lane];
        u64 *dst = P0 + ((size_t)(g * G + lane) * a.nchunk_max + c) * (HD + 2);
        ll_put(dst, tg | 2, __float_as_uint(s.u.att.amax[NWV][lane]));
        ll_put(dst + 1, tg | 2, __float_as_uint(L));
    }
    __syncthreads();
    MK_TRACE_ATT(5);
    return true;
}

// Combine of query head h over its nch chunk partials -> attention output (LL words, fp32)
template <int HD>
__device__ __forceinline__ bool combine_head(const AttnCtx a, u64 *R, unsigned tg, int h, int nch) {
    Smem &s = S;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const u64 *P = R + a.lw_part + (size_t)h * a.nchunk_max * (HD + 2);
    if (!ll_gather(a.err, P, nch * (HD + 2), tg | 2, s.stage)) return false;
    const float *p = (const float *)s.stage;
    if (wv == 0) {
        float M = -INFINITY;
        for (int c = lane; c < nch; c += 64) {
            const float lc = p[c * (HD + 2) + 1];
            M = fmaxf(M, lc > 0.f ? p[c * (HD + 2)] : -INFINITY);
        }
        M = wave_max(M);
        float L = 0.f;
        for (int c = lane; c < nch; c += 64) {
            const float lc = p[c * (HD + 2) + 1];
            const float wc = lc > 0.f ? expf(p[c * (HD + 2)] - M) : 0.f;
            s.w[c] = wc;
            L += wc * lc;
        }
        L = wave_sum(L);
        if (lane == 0) s.redf[0] = L;
    }
    __syncthreads();
    const float L = s.redf[0];
    u64 *A = R + a.lw_attn;
    for (int d = threadIdx.x; d < HD; d += NT) {
        float acc = 0.f;
        for (int c = 0; c < nch; ++c) acc += s.w[c] * p[c * (HD + 2) + 2 + d];
        ll_put(A + h * HD + d, tg | 3, __float_as_uint(acc / L));
    }
    __syncthreads();
    return true;
}

template <int FMT, int HD>
__global__ void __launch_bounds__(NT) k_decode(Args a) {
    // kernel arguments are only read field by field (taking their address would copy them to scratch)
    const sp_token t = *a.tok;
    constexpr int KT = TileGeom<FMT>::KT;
    const int H = a.H, NH = a.NH, NKV = a.NKV, I = a.I, V = a.V, L = a.L;
    const int S1 = a.S1, S3 = a.S3, S5 = a.S5;
    const float eps = a.eps;
    unsigned *const err = a.err;
    const size_t lw_qkv = a.lw_qkv, lw_attn = a.lw_attn, lw_o = a.lw_o, lw_act = a.lw_act, lw_d = a.lw_d;
    const size_t lw_layer = a.lw_layer;
    u64 *const ll = a.ll;
    const unsigned tag0 = a.tag0;
    const AttnCtx ac{NH, NKV, S1, a.n_slots, a.nchunk_max, a.scale, lw_qkv, a.lw_part, lw_attn, a.inv_freq, err};
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nlin = t.ctx_hi - t.ctx_lo + 1;                    // visible keys (the new one is the last)
    const int nch = (nlin + ATT_CH - 1) / ATT_CH;

    // embedding row (every block keeps its own residual copy)
    {
        const Mat em = a.embed;
        for (int k = threadIdx.x; k < H; k += NT) S.x[k] = packed_elem<FMT>(em.w, em.sz, em.nkt, t.token, k);
        __syncthreads();
    }

    phase_prefetch<FMT, 1>(L > 0 ? a.layers[0].qkv : a.head, L > 0 ? S1 : 1);
    MK_TRACE(0);
    for (int l = 0; l <= L; ++l) {
        const int te = 1 + l * 12;                              // trace event base of this layer
        // ---------------- P1 (l < L: qkv; l == L: LM head): x += previous layer's down partials, norm, GEMV
        const bool head = l == L;
        const LayerW W = a.layers[head ? 0 : l];
        const Mat m1 = head ? a.head : W.qkv;
        const float *nw1 = head ? a.final_norm : W.in_norm;
        u64 *const R = ll + (size_t)l * lw_layer;                // head: unused past the last layer's region
        const unsigned tg = tag0 | (unsigned)(l * 8);
        {
            const int nsplit = head ? 1 : S1;
            const int mine = my_items(m1.groups * nsplit);
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            for (int b0 = 0; b0 == 0 || b0 < mine; b0 += NWV) {
                Phase<FMT, 1> p;
                if (mine > 0) phase_load<FMT, 1>(m1, nsplit, b0, mine, true, p);
                if (b0 == 0) {
                    MK_TRACE(te);
                    if (l > 0) {
                        const unsigned tgp = tag0 | (unsigned)((l - 1) * 8);
                        if (!ll_gather(err, ll + (size_t)(l - 1) * lw_layer + lw_d, S5 * H, tgp | 6, S.stage)) return;
                        add_partials(S5, H);
                    }
                    MK_TRACE(te + 1);
                    norm_to_a(nw1, H, m1.nkt * KT, eps);
                }
                if (mine == 0) break;
                float out[1];
                if (phase_finish<FMT, 1>(m1, p, out)) {
                    const int row = p.j.unit * 16 + lane;
                    if (!head) {
                        if (row < m1.rows) ll_put(R + lw_qkv + qkv_pos(row, p.j.sp, S1, NH, NKV, HD), tg | 1, __float_as_uint(out[0]));
                    } else if (row < V) {
                        if (a.logits) a.logits[row] = out[0];
                        argmax_merge(bv, bi, out[0], row);
                    }
                }
            }
            if (head) {
                // block argmax over the candidates of lanes 0..15 of every wave, then across blocks by block 0
                float v = bv;
                int idx = bi;
                wave_argmax(v, idx);
                __syncthreads();
                if (lane == 0) { S.redf[wv] = v; S.stage[wv] = (unsigned)idx; }
                __syncthreads();
                u64 *AM = ll + a.lw_am;
                const unsigned tgh = tag0 | (unsigned)(L * 8 + 7);
                if (threadIdx.x == 0) {
                    for (int w2 = 1; w2 < NWV; ++w2) argmax_merge(v, idx, S.redf[w2], (int)S.stage[w2]);
                    ll_put(AM + 2 * blockIdx.x, tgh, __float_as_uint(v));
                    ll_put(AM + 2 * blockIdx.x + 1, tgh, (unsigned)idx);
                }
                if (blockIdx.x == 0) {
                    if (!ll_gather(err, AM, 2 * gridDim.x, tgh, S.stage)) return;
                    if (wv == 0) {
                        float v2 = -INFINITY;
                        int i2 = 0x7fffffff;
                        for (int b = lane; b < (int)gridDim.x; b += 64)
                            argmax_merge(v2, i2, __uint_as_float(S.stage[2 * b]), (int)S.stage[2 * b + 1]);
                        wave_argmax(v2, i2);
                        if (lane == 0) *a.out_id = i2;
                    }
                }
                return;
            }
        }
        // ---------------- P2: attention items (kv head, chunk); P2b: combine, one block per query head
        MK_TRACE(te + 2);
        for (int it = blockIdx.x; it < NKV * nch; it += gridDim.x)
            if (!attn_item<HD>(ac, W, R, tg, t, it / nch, it % nch, nch)) return;
        MK_TRACE(te + 3);
        phase_prefetch<FMT, 1>(W.o, S3);                       // the ring is free again: o_proj tiles
        for (int h = blockIdx.x; h < NH; h += gridDim.x)
            if (!combine_head<HD>(ac, R, tg, h, nch)) return;
        MK_TRACE(te + 4);
        // ---------------- P3: o_proj partials (blocks without an item skip its input)
        {
            const int mine = my_items(W.o.groups * S3);
            for (int b0 = 0; b0 < mine; b0 += NWV) {
                Phase<FMT, 1> p;
                phase_load<FMT, 1>(W.o, S3, b0, mine, true, p);
                if (b0 == 0) {
                    if (!ll_gather(err, R + lw_attn, NH * HD, tg | 3, S.stage)) return;
                    MK_TRACE(te + 5);
                    for (int k = threadIdx.x; k < W.o.nkt * KT; k += NT)
                        S.a[k] = k < NH * HD ? (f16)__uint_as_float(S.stage[k]) : (f16)0.f;
                    __syncthreads();
                }
                float out[1];
                if (phase_finish<FMT, 1>(W.o, p, out)) {
                    const int row = p.j.unit * 16 + lane;
                    if (row < W.o.rows) ll_put(R + lw_o + (size_t)p.j.sp * H + row, tg | 4, __float_as_uint(out[0]));
                }
            }
        }
        // ---------------- P4: x += o partials; xn = norm(x); gate_up pairs -> act = SiLU(gate) * up (fp16)
        phase_prefetch<FMT, 2>(W.gu, 1);
        MK_TRACE(te + 6);
        {
            const int mine = my_items(W.gu.groups);
            for (int b0 = 0; b0 == 0 || b0 < mine; b0 += NWV) {
                Phase<FMT, 2> p;
                if (mine > 0) phase_load<FMT, 2>(W.gu, 1, b0, mine, true, p);
                if (b0 == 0) {
                    if (!ll_gather(err, R + lw_o, S3 * H, tg | 4, S.stage)) return;
                    MK_TRACE(te + 7);
                    add_partials(S3, H);
                    norm_to_a(W.post_norm, H, W.gu.nkt * KT, eps);
                }
                if (mine == 0) break;
                float out[2];
                if (phase_finish<FMT, 2>(W.gu, p, out)) {
                    const int row = p.j.unit * 16 + lane;
                    if (row < W.gu.rows) {
                        const f16 v = (f16)(silu_f(out[0]) * out[1]);
                        ll_put(R + lw_act + row, tg | 5, (unsigned)__builtin_bit_cast(uint16_t, v));
                    }
                }
            }
        }
        // ---------------- P5: down partials; the input is the act slice this block's items read
        phase_prefetch<FMT, 1>(W.down, S5);
        MK_TRACE(te + 8);
        {
            const int mine = my_items(W.down.groups * S5);
            int kmin = 1 << 30, kmax = 0;
            for (int i = 0; i < mine; ++i) {
                const int sp = ((int)blockIdx.x + i * (int)gridDim.x) % S5;
                kmin = min(kmin, (int)((long)W.down.nkt * sp / S5) * KT);
                kmax = max(kmax, (int)((long)W.down.nkt * (sp + 1) / S5) * KT);
            }
            for (int b0 = 0; b0 < mine; b0 += NWV) {
                Phase<FMT, 1> p;
                phase_load<FMT, 1>(W.down, S5, b0, mine, true, p);
                if (b0 == 0) {
                    if (!ll_gather(err, R + lw_act + kmin, min(I, kmax) - kmin, tg | 5, S.stage)) return;
                    MK_TRACE(te + 9);
                    for (int k = threadIdx.x; k < kmax - kmin; k += NT)
                        S.a[kmin + k] = kmin + k < I ? __builtin_bit_cast(f16, (uint16_t)S.stage[k]) : (f16)0.f;
                    __syncthreads();
                }
                float out[1];
                if (phase_finish<FMT, 1>(W.down, p, out)) {
                    const int row = p.j.unit * 16 + lane;
                    if (row < W.down.rows) ll_put(R + lw_d + (size_t)p.j.sp * H + row, tg | 6, __float_as_uint(out[0]));
                }
            }
        }
        // next layer's qkv tiles (or the LM head's) into the ring while the down partials travel
        phase_prefetch<FMT, 1>(l + 1 < L ? a.layers[l + 1].qkv : a.head, l + 1 < L ? S1 : 1);
        MK_TRACE(te + 10);
    }
}

}  // namespace mk
