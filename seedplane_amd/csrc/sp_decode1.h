// Persistent one-column decode step: every layer of one new token (embedding, RMSNorms, qkv with bias, RoPE and the
// K/V write, windowed GQA attention with a split-K combine, o_proj, SwiGLU MLP, residual adds, the final RMSNorm) in
// one cooperative launch of one block per CU.  The LM head and the argmax then run as the kernel chain's GEMV and
// argmax kernels.  Replaces, for one decode column, the same reference computation as the chain in sp_engine::step
// (seedplane/qwen_engine.py:117-144; native/vulkan_decode/qwen_vk.cpp:372-412 records the whole step once and
// submits it once per token).
//
// Why: a one-column step is a chain of ~170 dependent kernels, each paying launch, ramp-up and the end-of-kernel L2
// write-back (about 3-4 us each) for 1-30 MB of weights.  Here the phases of a layer hand their outputs to each other
// inside one kernel, and a block that has no work in the early phases of a layer issues the weight loads of its later
// phases at once, so weights stream while the early phases wait on each other.
//
// Hand-offs: every value crossing blocks is a 64-bit word, payload (fp32 bits) in the low half and a 32-bit tag in the
// high half, written with one relaxed agent-scope atomic store and read with relaxed agent-scope atomic loads (these
// bypass the XCD-private L2s, so no fence and no cache write-back is needed; a 64-bit atomic is single-copy, so a
// reader sees either the old word or the whole new one).  A consumer polls exactly the words it needs until every tag
// is the current (launch, layer, phase) tag: there is no grid barrier.  Every poll is bounded; a block that runs out
// sets the error word and leaves, and the blocks waiting on it run out in turn, so the grid always drains.
// Buffers are reused from layer to layer: a block overwrites a region of layer l + 1 only after its own inputs of
// layer l + 1 arrived, and each of those depends on every reader of that region in layer l (the phases form a chain in
// which every consumer needs every producer of the phase before: qkv -> attention chunks -> per-head combine -> o_proj
// -> gate_up -> down -> next qkv; the down items that read o_proj rows feed every qkv tile of the next layer, which
// feeds every o_proj tile), so no word is overwritten before it has been read.
//
// Phases of layer l and their blocks (nb = blocks = CUs; item counts for the Qwen2-1.5B shape):
//   P1 qkv      item i < NQ (128 row tiles of 16 rows, full K = H)        blocks 0 .. NQ - 1
//   P2 attn     item (kv head, chunk of CH visible keys) (2 x 17)        blocks NQ .. NQ + NKV*CM - 1
//   P2b combine item q head (12)                                          the next NH blocks
//   P3 o_proj   item i < NO (96 row tiles, full K = NH*HD)               the last NO blocks (B3 = nb - NO ..)
//   P4 gate_up  units u (560 gate+up row tile pairs, full K = H)         blocks below B3 take up to MAXU units
//                                                                         each (u % B3), the rest one per o_proj block
//   P5 down     item (row tile, k half) (96 x 2)                          the last ND blocks (B5 = nb - ND ..)
// So the blocks without o_proj work hold most gate_up units and issue their weight loads as soon as their earlier
// phases are done, while qkv, attention and o_proj still run; the o_proj blocks, idle during gate_up, load their
// down weights meanwhile; and blocks below B5 load the next layer's qkv tiles while gate_up and down run.
// Residual stream: o_proj writes XM = x + attn_out W_o^T; the down item of k half 0 adds XM to its half, so the input
// of layer l + 1 is x = DP0 + DP1 = (XM + down_0) + down_1 (the embedding row at l = 0).
// GEMV tiles and numerics are those of the chain (sp_pack.h tiles, exact code unpacking, fp32 MFMA accumulation with
// the block scale per quant block); activations enter the MFMA as fp16 value (A row 0) + fp16 remainder (A row 1).
//
// Registers: a phase holds its weight tiles (5 registers per tile and lane) from before its hand-off until its dot
// products.  Nothing else may stay live across the layer loop, so every phase reads the launch constants afresh
// through a constant-space pointer and its lane ids afresh (both laundered through an empty asm, so the compiler can
// neither hoist them out of the loop nor keep them in registers from phase to phase), and the dot products keep at
// most two tiles (or one row group) of MFMA results in flight.
#pragma once
#include <algorithm>
#include <cstddef>
#include <type_traits>
#include <vector>

#include "sp_gemv.h"

namespace d1 {

typedef unsigned long long u64;
constexpr int NT = 512, NW = 8;         // threads and waves per block
constexpr int CH = 64;                  // visible keys per attention chunk
constexpr int MAXU = 3;                 // gate_up units per block
constexpr int KS = 2;                   // k halves of the down projection
constexpr long POLL_LIMIT = 1l << 20;   // failed polls of one batch before the block gives up (~0.5 s)
constexpr int MAX_L = 32;               // layers a tag can name
constexpr int MAX_H = 2048;             // hidden size (the norm's LDS row)
constexpr int MAX_K = 4608;             // widest GEMV input a block stages (halves): max(H, NH*HD, I / KS)
constexpr int MAX_G = 8;                // query heads per kv head
constexpr int MAX_HD = 128;
constexpr int MAX_CM = 64;              // attention chunks per kv head (one lane each in the combine)
constexpr int MAX_T5 = 9;               // k-tiles per wave of a down item whose tiles can wait in LDS

// Tag of (launch sequence, layer, phase): unique per launch and per (layer, phase) within it.
enum { PH_QKV = 1, PH_PART = 2, PH_ATT = 3, PH_XM = 4, PH_ACT = 5, PH_DP = 6 };
__host__ __device__ inline unsigned tag_of(unsigned seq, int l, int p) { return (seq << 8) | (unsigned)(l * 8 + p); }
// 16-bit tag of the packed activation words of (launch, layer): never 0 (the words' initial state) and different for
// consecutive launches.  Every activation word is rewritten in every layer of every launch, so a word that carries
// the current tag was written in this layer of this launch.
__host__ __device__ inline unsigned tag16_of(unsigned seq, int l) { return (((seq % 2047u) + 1u) << 5) | (unsigned)l; }

struct LayerPtr {
    const uint8_t *w[4];        // packed qkv, o, gate_up, down
    const f16 *sz[4];
    const float *qkv_b, *n_in, *n_post;
    f16 *kc, *vc;               // this layer's K / V ring [seq][kv head][slot][HD]
};

// Shape, work split and region offsets (in 64-bit words) of one engine; built on the host (make_geom) and checked
// there (check_geom) before any launch.
struct Geom {
    int L, H, NH, NKV, HD, I, V, Nqkv, n_slots;
    int fmt, KT;                 // tile format and k per tile
    int nkt_h, nkt_a, nkt_i;     // k-tiles of K = H, K = NH * HD, K = I
    int nb;                      // blocks (one per CU)
    int NQ, CM, NO, NU, ND;      // items: qkv row tiles, chunks per kv head, o row tiles, gate_up units, down items
    int nu_max;                  // gate_up units of the busiest block
    int B2, B2b, B3, B5;         // first block of attention chunks, combiners, o_proj, down
    int nk5;                     // k-tiles per down item
    size_t o_qkv, o_part, o_att, o_xm, o_act, o_dp, words;
};

// What every launch of one engine reads and no token changes: in device memory, written once when the step is
// prepared.
struct Static {
    Geom g;
    const LayerPtr *layers;
    const uint8_t *emb_w;
    const f16 *emb_sz;
    const float *final_norm, *inv_freq;
    float eps, scale;
    u64 *ll;                    // tagged words
    unsigned *err;              // 0 = fine; a block that gave up writes its code
    f16 *xn;                    // the final RMSNorm output (fp16) for the head GEMV
};
// The token's own arguments (passed by value).
struct Step {
    sp_token tok;
    const int *feed;            // NULL, or the previous step's argmax id (the token, clamped to the vocabulary)
    unsigned seq;               // launch sequence number (tags)
};

// ------------------------------------------------------------------------------------------------------- plan
// The host builds the geometry with these rules; check_geom proves that every item lands on a block < nb and every
// region index stays inside `words` for the shape.
__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

// Item -> block maps (the kernel and the host check share them).
__host__ __device__ inline int blk_p1(const Geom &g, int i) { return i; }
__host__ __device__ inline int blk_p2(const Geom &g, int kvh, int c) { return g.B2 + kvh * g.CM + c; }
__host__ __device__ inline int blk_p2b(const Geom &g, int qh) { return g.B2b + qh; }
__host__ __device__ inline int blk_p3(const Geom &g, int i) { return g.B3 + i; }
__host__ __device__ inline int blk_p4(const Geom &g, int u) { return u < MAXU * g.B3 ? u % g.B3 : g.B3 + (u - MAXU * g.B3); }
// Units of block b: b + i * B3 (i < MAXU) below B3; above, the one overflow unit MAXU * B3 + (b - B3).
__host__ __device__ inline int p4_unit(const Geom &g, int b, int i) {
    return b < g.B3 ? b + i * g.B3 : MAXU * g.B3 + (b - g.B3);
}
__host__ __device__ inline int p4_count(const Geom &g, int b) {
    int n = 0;
    if (b < g.B3) {
        for (int i = 0; i < MAXU; ++i) n += b + i * g.B3 < g.NU;
    } else {
        n = MAXU * g.B3 + (b - g.B3) < g.NU;
    }
    return n;
}
__host__ __device__ inline int blk_p5(const Geom &g, int d) { return g.B5 + d; }

// Region word offsets.
__host__ __device__ inline size_t w_qkv(const Geom &g, int i) { return g.o_qkv + i; }
__host__ __device__ inline size_t w_part(const Geom &g, int qh, int c, int j) {
    return g.o_part + ((size_t)qh * g.CM + c) * (2 + g.HD) + j;
}
__host__ __device__ inline size_t w_att(const Geom &g, int i) { return g.o_att + i; }
__host__ __device__ inline size_t w_xm(const Geom &g, int i) { return g.o_xm + i; }
// Activation words hold two values each: word i = activations 2i, 2i + 1.
__host__ __device__ inline size_t w_act(const Geom &g, int i) { return g.o_act + i; }
__host__ __device__ inline size_t w_dp(const Geom &g, int s, int i) { return g.o_dp + (size_t)s * g.H + i; }

// ------------------------------------------------------------------------------------------------------- device
// Constant-space views of the launch constants (the host pass, which only emits the launch stub, sees plain pointers).
#if defined(__HIP_DEVICE_COMPILE__)
typedef const __attribute__((address_space(4))) Static CStatic;
typedef const __attribute__((address_space(4))) LayerPtr CLayer;
#else
typedef const Static CStatic;
typedef const LayerPtr CLayer;
#endif

// The launch constants through a pointer the compiler must treat as new: loads through it are scalar loads that
// cannot be hoisted out of the layer loop.
__device__ __forceinline__ CStatic *fresh(const Static *p) {
    CStatic *q = (CStatic *)p;
    asm volatile("" : "+s"(q));
    return q;
}
__device__ __forceinline__ CLayer *layer_of(CStatic *S, int l) {
    CLayer *q = (CLayer *)S->layers + l;
    asm volatile("" : "+s"(q));
    return q;
}
// threadIdx.x as a value computed here (lane-dependent values derived from it stay inside the phase).
__device__ __forceinline__ int fresh_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ u64 ld_word(const u64 *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_word(u64 *p, float v, unsigned tag) {
    __hip_atomic_store(p, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One range of tagged words to wait for: src[0 .. n) carrying `tag` -> the LDS floats at dst.
struct Range {
    const u64 *src;
    int n;
    float *dst;
    unsigned tag;
};
// The source word, destination float and tag of slot k of the concatenated ranges (src NULL: past the end).  Every
// range is selected with a compile-time index, so the ranges stay in registers.
template <int NR>
__device__ __forceinline__ const u64 *slot_of(const Range (&rg)[NR], int k, float *&dst, unsigned &tag) {
    const u64 *src = nullptr;
    dst = nullptr;
    tag = 0;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        const bool here = k >= 0 && k < rg[j].n;
        src = here ? rg[j].src + k : src;
        dst = here ? rg[j].dst + k : dst;
        tag = here ? rg[j].tag : tag;
        k -= rg[j].n;
    }
    return src;
}
// The block waits for every word of up to NR ranges to carry its range's tag and copies the payloads to LDS.  The
// ranges are one index space; each thread issues the loads of its PER words (of every range) together and re-polls
// only the words that were not ready.  Returns false (after writing the error word) when a batch stays stale for
// POLL_LIMIT rounds; the caller then leaves the kernel.  Ends with a block barrier.
template <int PER, int NR>
__device__ bool gather(unsigned *err, const Range (&rg)[NR]) {
    int total = 0;
#pragma unroll
    for (int i = 0; i < NR; ++i) total += rg[i].n;
    bool ok = true;
    const int tid = threadIdx.x;
    for (int base = 0; base < total; base += PER * NT) {
        u64 w[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            float *d;
            unsigned t;
            const u64 *src = slot_of(rg, base + j * NT + tid, d, t);
            w[j] = src ? ld_word(src) : 0ull;         // an empty slot expects and holds tag 0
        }
        long spins = 0;
        while (true) {
            bool all = true;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                float *d;
                unsigned t;
                (void)slot_of(rg, base + j * NT + tid, d, t);
                all = all && (unsigned)(w[j] >> 32) == t;
            }
            if (all) break;
            if (++spins > POLL_LIMIT) { ok = false; break; }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                float *d;
                unsigned t;
                const u64 *src = slot_of(rg, base + j * NT + tid, d, t);
                if (src && (unsigned)(w[j] >> 32) != t) w[j] = ld_word(src);
            }
        }
        if (!ok) break;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            float *d;
            unsigned t;
            if (slot_of(rg, base + j * NT + tid, d, t)) *d = __uint_as_float((unsigned)w[j]);
        }
    }
    // every thread of the block leaves together (a thread that gave up makes the whole block leave)
    const int bad = __syncthreads_or(!ok);
    if (bad && threadIdx.x == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return !bad;
}

// One range of tagged words whose payloads stay in the registers of the threads that poll them: the tag is the word's
// bits from `shift` up (32: one fp32 payload; 48: two 24-bit payloads).
struct RRange {
    const u64 *src;
    int n;
    unsigned tag;
    int shift = 32;
};
// The block waits for every word of NR ranges, as gather does, but thread tid keeps word tid + NT * j of range r in
// out[r][j] (the tag alone where that word is past the range): no LDS copy and no barrier before the caller uses its
// values.  Returns false (after writing the error word) when the words stay stale for POLL_LIMIT rounds.
template <int NPT, int NR>
__device__ bool gather_w(unsigned *err, const RRange (&rg)[NR], u64 (&out)[NR][NPT], int tid) {
    // While the producers are still at work, each thread polls one word only (its last element of range 0) and
    // issues its other loads once that word is current: an early block does not stream its whole input through the
    // memory system once per round trip.  (Every word's own tag is still checked below.)
    bool ok = true;
    {
        int js = -1;
#pragma unroll
        for (int j = 0; j < NPT; ++j) js = tid + NT * j < rg[0].n ? j : js;
        if (js >= 0) {
            const u64 *p = rg[0].src + tid + NT * js;
            long spins = 0;
            while ((unsigned)(ld_word(p) >> rg[0].shift) != rg[0].tag) {
                if (++spins > POLL_LIMIT) { ok = false; break; }
                __builtin_amdgcn_s_sleep(1);
            }
        }
    }
    u64 w[NR][NPT];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int k = tid + NT * j;
            w[r][j] = k < rg[r].n ? ld_word(rg[r].src + k) : ((u64)rg[r].tag << rg[r].shift);
        }
    long spins = 0;
    while (ok) {
        bool all = true;
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int j = 0; j < NPT; ++j) all = all && (unsigned)(w[r][j] >> rg[r].shift) == rg[r].tag;
        if (all) break;
        if (++spins > POLL_LIMIT) { ok = false; break; }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int j = 0; j < NPT; ++j)
                if ((unsigned)(w[r][j] >> rg[r].shift) != rg[r].tag) w[r][j] = ld_word(rg[r].src + tid + NT * j);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < NPT; ++j) out[r][j] = w[r][j];
    const int bad = __syncthreads_or(!ok);
    if (bad && threadIdx.x == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return !bad;
}
// gather_w with fp32 payloads: out[r][j] = element tid + NT * j of range r (0 past the range).
template <int NPT, int NR>
__device__ bool gather_r(unsigned *err, const RRange (&rg)[NR], float (&out)[NR][NPT], int tid) {
    u64 w[NR][NPT];
    const bool ok = gather_w<NPT, NR>(err, rg, w, tid);
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < NPT; ++j) out[r][j] = __uint_as_float((unsigned)w[r][j]);
    return ok;
}

// fp32 -> the 24 high bits of its encoding, rounded to nearest even (sign, exponent, 15 fraction bits; finite values
// of the activations' range stay finite), and back (exact).
__device__ __forceinline__ uint32_t f24_of(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u + 0x7Fu + ((u >> 8) & 1u)) >> 8;
}
__device__ __forceinline__ float f32_of24(uint32_t b) { return __uint_as_float(b << 8); }

// LDS of one block (phases reuse it).
struct Smem {
    float red[NW * MAXU * 2 * 16];            // per-wave row sums
    float wsum[32];                           // block reductions
    __align__(16) f16 xh[MAX_K + 8];          // GEMV input (fp16) + a zero line
    __align__(16) f16 xl[MAX_K + 8];          // its remainders
    // attention chunk
    __align__(16) f16 ks[CH][MAX_HD + 8];
    __align__(16) f16 vs[CH][MAX_HD];
    float qs[MAX_G][MAX_HD];
    float es[MAX_G][CH];
    float cs[MAX_HD];                         // cos, then sin, of the RoPE phases
    float knew[MAX_HD], vnew[MAX_HD];
    float cw[MAX_CM];                         // the combine's chunk weights
    float stage[MAX_K + 16];                  // gathered words (the attention's qkv rows, the combine's chunk records)
};
// Dynamic LDS of a launch: at least 84 KiB, so that no CU (160 KiB of LDS) can hold two blocks and the grid of one
// block per CU is spread over every CU.  The kernel adds a static array for the down tiles (at most MAX_T5 KiB per
// wave).
constexpr size_t SMEM_BYTES = sizeof(Smem) > 84 * 1024 ? sizeof(Smem) : 84 * 1024;
static_assert(SMEM_BYTES + NW * MAX_T5 * TILE_BYTES <= 160 * 1024, "one block's LDS fits a CU");

// Block barrier for LDS data only: waits for the wave's LDS (and scalar) operations, not for its vector memory loads,
// so global-to-LDS weight copies issued earlier stay in flight across it (a __syncthreads() waits for those too).
// The memory clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Block-wide sum of one value per thread, in a fixed order (DPP per wave, then the wave sums in wave order).
__device__ __forceinline__ float block_sum_fixed(float v, float *wsum) {
    v = wave_sum_dpp(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) wsum[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int j = 0; j < NW; ++j) t += wsum[j];
    __syncthreads();
    return t;
}

// The norm weights of the thread's elements k = tid + NT * j of a row of n <= MAX_H, loaded before the hand-off they
// will scale (a load after it would add a memory round trip to the phase).
constexpr int NPT = MAX_H / NT;
struct NormW {
    float w[NPT];
    __device__ __forceinline__ void load(const float *wp, int n, int tid) {
#pragma unroll
        for (int j = 0; j < NPT; ++j) w[j] = wp[min(tid + NT * j, n - 1)];
    }
};
// The RMSNorm scale of a GEMV input is one scalar, so W (x rs w) = rs (W (x w)): the GEMV takes x w (x[j] = element
// tid + NT * j in registers, n elements) as fp16 pairs and the scale is applied to its sums.  prenorm_pairs writes
// the pairs and each wave's sum of squares of x (each square rounded, the thread's elements in index order, DPP within
// the wave) and ends with a block barrier; norm_scale then adds the wave sums in wave order: rs = 1 / sqrt(ss / n +
// eps), the same value as a norm computed before the GEMV.
__device__ __forceinline__ void prenorm_pairs(Smem &s, const float (&x)[NPT], int n, const NormW &nw, int tid) {
    float ss = 0.f;
    {
#pragma clang fp contract(off)
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const float v = tid + NT * j < n ? x[j] : 0.f;
            ss += v * v;
        }
    }
    ss = wave_sum_dpp(ss);
    if ((tid & 63) == 0) s.wsum[tid >> 6] = ss;
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
        const int k = tid + NT * j;
        if (k < n) {
            f16 hi, lo;
            split_f16(x[j] * nw.w[j], hi, lo);
            s.xh[k] = hi;
            s.xl[k] = lo;
        }
    }
    if (tid < 8) s.xh[MAX_K + tid] = (f16)0.f;
    lds_barrier();
}
__device__ __forceinline__ float norm_scale(const Smem &s, int n, float eps) {
    float t = 0.f;
    for (int j = 0; j < NW; ++j) t += s.wsum[j];
    return 1.0f / sqrtf(t / (float)n + eps);
}
// x[j] = element tid + NT * j (registers, n elements) -> fp16 pairs
template <int N>
__device__ __forceinline__ void pairs(Smem &s, const float (&x)[N], int n, int tid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const int k = tid + NT * j;
        if (k < n) {
            f16 hi, lo;
            split_f16(x[j], hi, lo);
            s.xh[k] = hi;
            s.xl[k] = lo;
        }
    }
    if (tid < 8) s.xh[MAX_K + tid] = (f16)0.f;
    lds_barrier();
}

// Weight tiles of one row group: wave w takes the T consecutive k-tiles kt0 + w T .. (one address per row group, the
// tiles at immediate offsets), loaded unconditionally (tiles past kt1 re-read tile kt0 and count zero).
template <int FMT> struct SideOf { typedef uint32_t type; };        // Q8: the two block scales of a row
template <> struct SideOf<3> { typedef u32x4 type; };                // Q4: four (scale, zero) pairs of a row
template <int FMT, int T>
struct Tiles {
    u32x4 wt[T];
    typename SideOf<FMT>::type sd[FMT == 1 ? 1 : T];
    int nvalid;                                   // tiles t < nvalid are real
    __device__ __forceinline__ void load(const uint8_t *w, const f16 *sz, int nkt, int grp, int kt0, int kt1, int wv,
                                         int lane) {
        const int first = kt0 + wv * T;
        nvalid = max(0, min(T, kt1 - first));
        // a wave with no real tile reads tile kt0 (in bounds) and uses none of it
        const int base = nvalid > 0 ? first : kt0;
        const u32x4 *wb = (const u32x4 *)(w + ((size_t)grp * nkt + base) * TILE_BYTES) + lane;
        const int r = lane & 15;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int tt = t < nvalid ? t : 0;        // tiles past the range re-read the first one
            wt[t] = __builtin_nontemporal_load(wb + tt * (TILE_BYTES / 16));
            if constexpr (FMT == 2) sd[t] = *((const uint32_t *)(sz + ((size_t)grp * nkt + base + tt) * 32) + r);
            if constexpr (FMT == 3) sd[t] = *((const u32x4 *)(sz + ((size_t)grp * nkt + base + tt) * 128) + r);
        }
    }
    // tile t may not be unpacked or multiplied before v is known (keeps MFMA results from piling up in registers)
    __device__ __forceinline__ void after(int t, float v) { asm volatile("" : "+v"(wt[t]) : "v"(v)); }
    __device__ __forceinline__ void after_all(float v) {
#pragma unroll
        for (int t = 0; t < T; ++t) after(t, v);
    }
};

// Block scale and code offset of step st of tile t (quantized formats).
template <int FMT, int T>
__device__ __forceinline__ float tile_scale(const Tiles<FMT, T> &tl, int t, int st, float &offs) {
    if constexpr (FMT == 2) {
        const uint32_t d = tl.sd[t];
        offs = QBias<FMT>::V;
        return (float)__builtin_bit_cast(f16, (uint16_t)(st == 0 ? (d & 0xffffu) : (d >> 16)));
    } else {
        uint32_t d;
        if (st == 0) d = tl.sd[t].x; else if (st == 1) d = tl.sd[t].y; else if (st == 2) d = tl.sd[t].z; else d = tl.sd[t].w;
        offs = QBias<FMT>::V + (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
        return (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
    }
}

// A operand of step st of the wave's tile t of the staged input (xh / xl, k measured from the staged input's start =
// tile kt0): row 0 the fp16 values, row 1 their remainders, rows 2..15 (and dead tiles) the zero line.
// The three sources are picked by integer selects on one byte offset from xh, not by choosing among pointers: a
// pointer choice compiled to divergent branches around every read, which kept the read from being issued ahead of
// the MFMAs before it (each step then paid the full LDS latency).
template <int FMT, int T>
__device__ __forceinline__ f16x8 x_operand(const Smem &s, int t, int st, bool live, int wv, int lane, int kdep) {
    constexpr int KT = TileGeom<FMT>::KT;
    constexpr int XL = (int)((offsetof(Smem, xl) - offsetof(Smem, xh)) / sizeof(f16));
    const int r = lane & 15, g = lane >> 4;
    const int xo = (wv * T + t) * KT + st * 32 + 8 * g + kdep;
    int o = r == 0 ? xo : XL + xo;
    o = !live || r > 1 ? MAX_K : o;
    return *(const f16x8 *)((const char *)&s + offsetof(Smem, xh) + 2 * o);
}

// One row group's partial dot product with the staged input over the wave's T tiles: lanes 0..15 return the sums of
// rows 0..15 of the group (other lanes: garbage).  Tile t + 2 waits for tile t's sum, so at most two tiles of operands
// and MFMA results are live.
template <int FMT, int T>
__device__ __forceinline__ float stream_dot(const Smem &s, Tiles<FMT, T> &tl, int wv, int lane) {
    constexpr int ST = TileGeom<FMT>::STEPS;
    const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};
    float acc = 0.f;
    f32x4 acc4 = (f32x4){0.f, 0.f, 0.f, 0.f};
    int kdep[2] = {0, 0};
    // software-pipelined like the LDS-tile version below: tile t + 1's A operands are read before tile t's MFMAs
    auto read = [&](int t, f16x8 (&xa)[ST]) {
#pragma unroll
        for (int st = 0; st < ST; ++st) xa[st] = x_operand<FMT, T>(s, t, st, t < tl.nvalid, wv, lane, kdep[t & 1]);
    };
    f16x8 xa_cur[ST], xa_nxt[ST];
    read(0, xa_cur);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        if (t + 1 < T) read(t + 1, xa_nxt);
        if constexpr (FMT == 1) {
#pragma unroll
            for (int st = 0; st < ST; ++st) acc4 = mfma16(xa_cur[st], __builtin_bit_cast(f16x8, tl.wt[t]), acc4);
        } else {
            f32x4 sx[ST], dd[ST];
#pragma unroll
            for (int st = 0; st < ST; ++st) {
                sx[st] = mfma16(xa_cur[st], ones8, (f32x4){0.f, 0.f, 0.f, 0.f});
                dd[st] = mfma16(xa_cur[st], biased_step<FMT>(tl.wt[t], st), (f32x4){0.f, 0.f, 0.f, 0.f});
            }
#pragma unroll
            for (int st = 0; st < ST; ++st) {
                float offs;
                const float scale = tile_scale<FMT, T>(tl, t, st, offs);
                acc = fmaf(scale, fmaf(-offs, sx[st][0], dd[st][0]) + fmaf(-offs, sx[st][1], dd[st][1]), acc);
            }
        }
        const float v = FMT == 1 ? acc4[0] : acc;
        asm volatile("" : "+v"(kdep[t & 1]) : "v"(v));
        if (t + 2 < T) tl.after(t + 2, v);
        if (t + 1 < T) {
#pragma unroll
            for (int st = 0; st < ST; ++st) xa_cur[st] = xa_nxt[st];
        }
    }
    return FMT == 1 ? acc4[0] + acc4[1] : acc;
}

// One 16-byte global-to-LDS copy per lane (global_load_lds_dwordx4): lane i's 16 bytes at g land at LDS byte address
// lds + 16 i.  Written as inline asm so that the compiler does not track the copy: it would otherwise make every LDS
// access of the block that it cannot prove disjoint from the copy, inside the layer loop all of them, wait for every
// outstanding vector memory operation (the cache and hand-off stores included).  The copy completes in order with
// the wave's other vector memory loads; the reader of the tiles waits for it explicitly (copy_wait).  M0 (the LDS
// address) is set here; no other code of this kernel uses M0.
__device__ __forceinline__ void lds_copy16(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(g), "s"(lds) : "memory");
}
__device__ __forceinline__ void copy_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Weight tiles of one row group whose 16-byte lane slices wait in LDS (an array of their own; tile t of wave w at (w T
// + t) KiB, the lane's slice at 16 lane) instead of registers.  The scales stay in registers.  Each wave reads only
// the tiles it copied, after copy_wait.
template <int FMT, int T>
struct LdsTiles {
    typename SideOf<FMT>::type sd[FMT == 1 ? 1 : T];
    int nvalid;
    uint8_t *lds;
    __device__ __forceinline__ void load(uint8_t *wl, const uint8_t *w, const f16 *sz, int nkt, int grp, int kt0,
                                         int kt1, int wv, int lane) {
        lds = wl;
        static_assert(T <= MAX_T5, "the LDS holds MAX_T5 tiles per wave");
        const int first = kt0 + wv * T;
        nvalid = max(0, min(T, kt1 - first));
        const int base = nvalid > 0 ? first : kt0;
        const uint8_t *wb = w + ((size_t)grp * nkt + base) * TILE_BYTES + lane * 16;
        const int r = lane & 15;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int tt = t < nvalid ? t : 0;
            const uint32_t la = (uint32_t)(size_t)((__attribute__((address_space(3))) uint8_t *)wl) + (wv * T + t) * TILE_BYTES;
            lds_copy16(wb + tt * TILE_BYTES, __builtin_amdgcn_readfirstlane(la));
            if constexpr (FMT == 2) sd[t] = *((const uint32_t *)(sz + ((size_t)grp * nkt + base + tt) * 32) + r);
            if constexpr (FMT == 3) sd[t] = *((const u32x4 *)(sz + ((size_t)grp * nkt + base + tt) * 128) + r);
        }
    }
};
template <int FMT, int T>
__device__ __forceinline__ float tile_scale(const LdsTiles<FMT, T> &tl, int t, int st, float &offs) {
    if constexpr (FMT == 2) {
        const uint32_t d = tl.sd[t];
        offs = QBias<FMT>::V;
        return (float)__builtin_bit_cast(f16, (uint16_t)(st == 0 ? (d & 0xffffu) : (d >> 16)));
    } else {
        uint32_t d;
        if (st == 0) d = tl.sd[t].x; else if (st == 1) d = tl.sd[t].y; else if (st == 2) d = tl.sd[t].z; else d = tl.sd[t].w;
        offs = QBias<FMT>::V + (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
        return (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
    }
}
// stream_dot over LDS tiles, software-pipelined: iteration t first reads tile t + 1's weights and A operands (their
// reads wait for tile t - 1's sum, which bounds the operands in flight to two tiles), then issues tile t's MFMAs on
// the operands read one iteration earlier, then adds their results.  The reads of one tile thus overlap the matrix
// work of the tile before it (written step by step, the compiler kept every read behind the previous step's
// results).  Same sums in the same order as the register-tile version.
template <int FMT, int T>
__device__ __forceinline__ float stream_dot(const Smem &s, const LdsTiles<FMT, T> &tl, int wv, int lane) {
    constexpr int ST = TileGeom<FMT>::STEPS;
    const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};
    float acc = 0.f;
    f32x4 acc4 = (f32x4){0.f, 0.f, 0.f, 0.f};
    int kdep[2] = {0, 0};
    copy_wait();
    auto read = [&](int t, u32x4 &wt, f16x8 (&xa)[ST]) {
        const int kd = kdep[t & 1];
        wt = *(const u32x4 *)(tl.lds + (wv * T + t) * TILE_BYTES + lane * 16 + 4 * kd);
#pragma unroll
        for (int st = 0; st < ST; ++st) xa[st] = x_operand<FMT, T>(s, t, st, t < tl.nvalid, wv, lane, kd);
    };
    u32x4 wt_cur, wt_nxt;
    f16x8 xa_cur[ST], xa_nxt[ST];
    read(0, wt_cur, xa_cur);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        if (t + 1 < T) read(t + 1, wt_nxt, xa_nxt);
        if constexpr (FMT == 1) {
#pragma unroll
            for (int st = 0; st < ST; ++st) acc4 = mfma16(xa_cur[st], __builtin_bit_cast(f16x8, wt_cur), acc4);
        } else {
            f32x4 sx[ST], dd[ST];
#pragma unroll
            for (int st = 0; st < ST; ++st) {
                sx[st] = mfma16(xa_cur[st], ones8, (f32x4){0.f, 0.f, 0.f, 0.f});
                dd[st] = mfma16(xa_cur[st], biased_step<FMT>(wt_cur, st), (f32x4){0.f, 0.f, 0.f, 0.f});
            }
#pragma unroll
            for (int st = 0; st < ST; ++st) {
                float offs;
                const float scale = tile_scale<FMT, T>(tl, t, st, offs);
                acc = fmaf(scale, fmaf(-offs, sx[st][0], dd[st][0]) + fmaf(-offs, sx[st][1], dd[st][1]), acc);
            }
        }
        const float v = FMT == 1 ? acc4[0] : acc;
        asm volatile("" : "+v"(kdep[t & 1]) : "v"(v));
        if (t + 1 < T) {
            wt_cur = wt_nxt;
#pragma unroll
            for (int st = 0; st < ST; ++st) xa_cur[st] = xa_nxt[st];
        }
    }
    return FMT == 1 ? acc4[0] + acc4[1] : acc;
}

// The A operands of the wave's T tiles, shared by several row groups over the same k range, and (quantized formats)
// the block sums of A rows 0 and 1.
template <int FMT, int T>
struct XOps {
    static constexpr int ST = TileGeom<FMT>::STEPS;
    f16x8 a[T][ST];
    float s0[T][ST], s1[T][ST];
    __device__ __forceinline__ void load(const Smem &s, int nvalid, int wv, int lane) {
        const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int st = 0; st < ST; ++st) {
                a[t][st] = x_operand<FMT, T>(s, t, st, t < nvalid, wv, lane, 0);
                if constexpr (FMT != 1) {
                    const f32x4 sx = mfma16(a[t][st], ones8, (f32x4){0.f, 0.f, 0.f, 0.f});
                    s0[t][st] = sx[0];
                    s1[t][st] = sx[1];
                }
            }
    }
};
// stream_dot of one row group against shared operands (same sums, bit for bit).
template <int FMT, int T>
__device__ __forceinline__ float group_dot(const XOps<FMT, T> &x, const Tiles<FMT, T> &tl) {
    constexpr int ST = TileGeom<FMT>::STEPS;
    float acc = 0.f;
    f32x4 acc4 = (f32x4){0.f, 0.f, 0.f, 0.f};
    if constexpr (FMT == 1) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int st = 0; st < ST; ++st) acc4 = mfma16(x.a[t][st], __builtin_bit_cast(f16x8, tl.wt[t]), acc4);
    } else {
        // every MFMA of the group first, then the sums in the same order: the products overlap in the matrix core
        // instead of each waiting for the one before it to be read
        f32x4 dd[T][ST];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int st = 0; st < ST; ++st)
                dd[t][st] = mfma16(x.a[t][st], biased_step<FMT>(tl.wt[t], st), (f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int st = 0; st < ST; ++st) {
                float offs;
                const float scale = tile_scale<FMT, T>(tl, t, st, offs);
                acc = fmaf(scale, fmaf(-offs, x.s0[t][st], dd[t][st][0]) + fmaf(-offs, x.s1[t][st], dd[t][st][1]), acc);
            }
    }
    return FMT == 1 ? acc4[0] + acc4[1] : acc;
}

// The 8 waves' partial sums of `nsum` row groups (red[(w * nsum + i) * 16 + r]) reduced in wave order by lanes 0..15
// of wave 0; returns the row sum of group i for lane r < 16.
__device__ __forceinline__ float wave_total(const Smem &s, int nsum, int i, int r) {
    float t = s.red[i * 16 + r];
    for (int w = 1; w < NW; ++w) t += s.red[(w * nsum + i) * 16 + r];
    return t;
}

// The two residual parts of layer l's input rows [r0, r0 + n): DP0 and DP1 of layer l - 1 (l > 0), as register ranges.
__device__ __forceinline__ void residual_ranges(const Geom &g, u64 *ll, unsigned seq, int l, int r0, int n, RRange *out) {
    out[0] = RRange{ll + w_dp(g, 0, r0), n, tag_of(seq, l - 1, PH_DP)};
    out[1] = RRange{ll + w_dp(g, 1, r0), n, tag_of(seq, l - 1, PH_DP)};
}

// The down tiles of block b's P5 item (row tile, k half), into LDS.
template <int FMT, int T5>
__device__ __forceinline__ void down_tiles(uint8_t *wl, LdsTiles<FMT, T5> &t5, const Geom &g, CLayer *lp, int b, int wv,
                                           int lane) {
    const int d = b - g.B5, rt = d % g.NO, kh = d / g.NO;
    const int kt0 = kh * g.nk5, kt1 = min(g.nkt_i, kt0 + g.nk5);
    t5.load(wl, lp->w[3], lp->sz[3], g.nkt_i, rt, kt0, kt1, wv, lane);
}
template <int FMT, int T5>
__device__ __forceinline__ void down_tiles(uint8_t *, Tiles<FMT, T5> &t5, const Geom &g, CLayer *lp, int b, int wv,
                                           int lane) {
    const int d = b - g.B5, rt = d % g.NO, kh = d / g.NO;
    const int kt0 = kh * g.nk5, kt1 = min(g.nkt_i, kt0 + g.nk5);
    t5.load(lp->w[3], lp->sz[3], g.nkt_i, rt, kt0, kt1, wv, lane);
}

// P4 of one block whose NU <= NG gate_up units' tiles are loaded: RMSNorm of the o_proj output XM (scale applied to
// the sums), the gate and up row groups of every unit, SwiGLU, and the activations as packed words.  False when the
// hand-off timed out (the caller leaves the kernel).
template <int FMT, int TH, int NG>
__device__ __forceinline__ bool gate_up(Smem &s, CStatic *S, const Geom &g, CLayer *lp, int l, unsigned seq, int b,
                                        int nu, Tiles<FMT, TH> *tg, Tiles<FMT, TH> *tu, int tid) {
    const int lane = tid & 63, wv = tid >> 6, r = lane & 15;
    u64 *ll = S->ll;
    NormW nw;
    nw.load(lp->n_post, g.H, tid);
    RRange rg[1] = {RRange{ll + w_xm(g, 0), g.H, tag_of(seq, l, PH_XM)}};
    float xm[1][NPT];
    if (!gather_r<NPT, 1>(S->err, rg, xm, tid)) return false;
    prenorm_pairs(s, xm[0], g.H, nw, tid);
    // the norm's scale is final once prenorm_pairs' barrier has passed: taken now, it is off the epilogue's path
    const float rs = norm_scale(s, g.H, S->eps);
    XOps<FMT, TH> xo;
    xo.load(s, tg[0].nvalid, wv, lane);
    // one row group at a time: group j + 1's products start after group j's sum (absent units are skipped by
    // scalar branches: nu is block-uniform)
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        if (i < nu) {
            const float vg = group_dot<FMT, TH>(xo, tg[i]);
            tu[i].after_all(vg);
            const float vu = group_dot<FMT, TH>(xo, tu[i]);
            if (i + 1 < NG) tg[i + 1].after_all(vu);
            if (lane < 16) {
                s.red[(wv * 2 * MAXU + 2 * i) * 16 + lane] = vg;
                s.red[(wv * 2 * MAXU + 2 * i + 1) * 16 + lane] = vu;
            }
        }
    }
    lds_barrier();
    if (tid < 16 * NG) {
        // lane 16 i + r: row r of unit i; rows r (even) and r + 1 go out as one word of two 24-bit values
        const int i = tid >> 4;
        const float gt = rs * wave_total(s, 2 * MAXU, 2 * i, r), up = rs * wave_total(s, 2 * MAXU, 2 * i + 1, r);
        const uint32_t a = f24_of(silu_f(gt) * up);
        const uint32_t an = (uint32_t)__shfl_xor((int)a, 1);
        if (i < nu && (r & 1) == 0)
            __hip_atomic_store(ll + w_act(g, p4_unit(g, b, i) * 8 + r / 2),
                               ((u64)tag16_of(seq, l) << 48) | ((u64)an << 24) | a, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    lds_barrier();
    return true;
}

// ------------------------------------------------------------------------------------------------------- kernel
// TH: k-tiles per wave for K = H (and K = NH * HD); T5: k-tiles per wave for one down item.
template <int FMT, int HD, int TH, int T5>
__global__ void __launch_bounds__(NT, 1) k_decode1(const Static *sp, Step stp) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem &s = *(Smem *)smem_raw;
    // the down tiles of a P5 item wait in LDS where they fit (else in registers, loaded in P5)
    constexpr bool DMA5 = T5 <= MAX_T5;
    typedef std::conditional_t<DMA5, LdsTiles<FMT, T5>, Tiles<FMT, T5>> T5T;
    __shared__ __align__(16) uint8_t wt5[DMA5 ? NW * T5 * TILE_BYTES : 16];
    const int b = blockIdx.x;
    const unsigned seq = stp.seq;
    const sp_token &tk = stp.tok;

    for (int l = 0; l < MAX_L; ++l) {
        {
            CStatic *S = fresh(sp);
            if (l >= S->g.L) break;
        }
        // ---------------------------------------------------------------- P1: RMSNorm + qkv row tile (+ bias)
        {
            CStatic *S = fresh(sp);
            const Geom g = S->g;
            if (b < g.NQ) {
                const int tid = fresh_tid(), lane = tid & 63, wv = tid >> 6, r = lane & 15;
                CLayer *lp = layer_of(S, l);
                u64 *ll = S->ll;
                const int item = b;
                NormW nw;
                nw.load(lp->n_in, g.H, tid);
                const float bias = lp->qkv_b[item * 16 + r];
                Tiles<FMT, TH> tl;
                tl.load(lp->w[0], lp->sz[0], g.nkt_h, item, 0, g.nkt_h, wv, lane);
                float x[NPT];
                if (l == 0) {
                    const int token = stp.feed ? min(max(stp.feed[0], 0), g.V - 1) : tk.token;
#pragma unroll
                    for (int j = 0; j < NPT; ++j)
                        x[j] = tid + NT * j < g.H ? packed_elem<FMT>(S->emb_w, S->emb_sz, g.nkt_h, token, tid + NT * j) : 0.f;
                } else {
                    RRange rg[2];
                    residual_ranges(g, ll, seq, l, 0, g.H, rg);
                    float v[2][NPT];
                    if (!gather_r<NPT, 2>(S->err, rg, v, tid)) return;
#pragma unroll
                    for (int j = 0; j < NPT; ++j) x[j] = v[0][j] + v[1][j];
                }
                prenorm_pairs(s, x, g.H, nw, tid);
                const float v = stream_dot<FMT, TH>(s, tl, wv, lane);
                if (lane < 16) s.red[wv * 16 + lane] = v;
                lds_barrier();
                if (tid < 16)
                    st_word(ll + w_qkv(g, item * 16 + r), norm_scale(s, g.H, S->eps) * wave_total(s, 1, 0, r) + bias,
                            tag_of(seq, l, PH_QKV));
            }
        }
        // ---------------------------------------------------------------- P2: attention over one chunk of keys
        {
            CStatic *S = fresh(sp);
            const Geom g = S->g;
            if (b >= g.B2 && b < g.B2 + g.NKV * g.CM) {
                const int tid = fresh_tid(), lane = tid & 63, wv = tid >> 6;
                CLayer *lp = layer_of(S, l);
                u64 *ll = S->ll;
                const int G = g.NH / g.NKV;
                const int nvis = tk.ctx_hi - tk.ctx_lo + 1;
                const int kvh = (b - g.B2) / g.CM, c = (b - g.B2) - kvh * g.CM;
                const int v0 = c * CH;
                if (v0 < nvis) {
                    const int cnt = min(CH, nvis - v0);
                    const bool has_new = v0 + cnt == nvis;        // the chunk holding the column's own (new) key
                    const size_t head_base = ((size_t)tk.seq * g.NKV + kvh) * g.n_slots;
                    f16 *kc = lp->kc, *vc = lp->vc;
                    constexpr int half = HD / 2;
                    // the RoPE table of the column's position (the chain's embedding kernel computes the same values)
                    const float fpos = (float)tk.pos;
                    for (int j = tid; j < half; j += NT) {
                        const float ph = fpos * S->inv_freq[j];
                        s.cs[j] = cosf(ph);
                        s.cs[half + j] = sinf(ph);
                    }
                    // K / V of the cached keys (the new key's row comes from the projection)
                    constexpr int CPR = HD / 8;
                    for (int i = tid; i < cnt * CPR; i += NT) {
                        const int j = i / CPR, ch = i - j * CPR;
                        if (has_new && j == cnt - 1) continue;
                        const int slot = (tk.ctx_lo + v0 + j) % g.n_slots;
                        const size_t off = (head_base + slot) * HD + ch * 8;
                        *(f16x8 *)&s.ks[j][ch * 8] = *(const f16x8 *)(kc + off);
                        *(f16x8 *)&s.vs[j][ch * 8] = *(const f16x8 *)(vc + off);
                    }
                    // q of the group's heads and (chunk of the new key) its key / value, in one hand-off
                    const unsigned tq = tag_of(seq, l, PH_QKV);
                    Range rg[3] = {Range{ll + w_qkv(g, kvh * G * HD), G * HD, s.stage, tq},
                                   Range{ll + w_qkv(g, (g.NH + kvh) * HD), has_new ? HD : 0, s.knew, tq},
                                   Range{ll + w_qkv(g, (g.NH + g.NKV + kvh) * HD), has_new ? HD : 0, s.vnew, tq}};
                    if (!gather<(MAX_G * MAX_HD + 2 * MAX_HD) / NT, 3>(S->err, rg)) return;
                    const float qscale = S->scale;
                    for (int i = tid; i < G * half; i += NT) {
                        const int h = i / half, j = i - h * half;
                        float o1, o2;
                        rope_pair(s.stage[h * HD + j], s.stage[h * HD + j + half], s.cs[j], s.cs[half + j], o1, o2);
                        s.qs[h][j] = o1 * qscale;
                        s.qs[h][j + half] = o2 * qscale;
                    }
                    if (has_new) {
                        const int jn = cnt - 1;
                        f16 *kdst = kc + (head_base + tk.slot) * HD, *vdst = vc + (head_base + tk.slot) * HD;
                        for (int j = tid; j < half; j += NT) {
                            float o1, o2;
                            rope_pair(s.knew[j], s.knew[j + half], s.cs[j], s.cs[half + j], o1, o2);
                            const f16 k1 = (f16)o1, k2 = (f16)o2;
                            s.ks[jn][j] = k1;
                            s.ks[jn][j + half] = k2;
                            kdst[j] = k1;
                            kdst[j + half] = k2;
                        }
                        for (int j = tid; j < HD; j += NT) {
                            const f16 vv = (f16)s.vnew[j];
                            s.vs[jn][j] = vv;
                            vdst[j] = vv;
                        }
                    }
                    lds_barrier();
                    // wave h (< G): query head kvh * G + h; lane j scores key j
                    if (wv < G) {
                        const int h = wv;
                        float sc = -INFINITY;
                        if (lane < cnt) {
                            float acc = 0.f;
#pragma unroll 4
                            for (int d = 0; d < HD; d += 8) {
                                const f16x8 kv = *(const f16x8 *)&s.ks[lane][d];
#pragma unroll
                                for (int e = 0; e < 8; ++e) acc += s.qs[h][d + e] * (float)kv[e];
                            }
                            sc = acc;
                        }
                        const float m = wave_max_dpp(sc);
                        const float ex = sc == -INFINITY ? 0.f : expf(sc - m);
                        const float lsum = wave_sum_dpp(ex);
                        s.es[h][lane] = ex;
                        __builtin_amdgcn_wave_barrier();
                        // lane: dims DPL * lane .. DPL * lane + DPL - 1, read together (one 2- or 4-byte LDS read per
                        // key, measured faster than one read per dim); each dim's sum runs over the keys in order
                        constexpr int DPL = HD / 64;
                        typedef std::conditional_t<DPL == 2, f16x2, f16> VT;
                        float o[DPL];
#pragma unroll
                        for (int i = 0; i < DPL; ++i) o[i] = 0.f;
                        for (int j = 0; j < cnt; ++j) {
                            const float p = s.es[h][j];
                            const VT vv = *(const VT *)&s.vs[j][DPL * lane];
                            if constexpr (DPL == 2) {
                                o[0] += p * (float)vv[0];
                                o[1] += p * (float)vv[1];
                            } else {
                                o[0] += p * (float)vv;
                            }
                        }
                        const float il = lsum > 0.f ? 1.f / lsum : 0.f;
                        const unsigned tp = tag_of(seq, l, PH_PART);
                        const int qh = kvh * G + h;
#pragma unroll
                        for (int i = 0; i < DPL; ++i) st_word(ll + w_part(g, qh, c, 2 + DPL * lane + i), o[i] * il, tp);
                        if (lane == 0) {
                            st_word(ll + w_part(g, qh, c, 0), m, tp);
                            st_word(ll + w_part(g, qh, c, 1), lsum, tp);
                        }
                    }
                    lds_barrier();
                }
            }
        }
        // ---------------------------------------------------------------- P2b: combine one query head's chunks
        {
            CStatic *S = fresh(sp);
            const Geom g = S->g;
            if (b >= g.B2b && b < g.B2b + g.NH) {
                const int tid = fresh_tid();
                u64 *ll = S->ll;
                const int qh = b - g.B2b;
                const int rec = 2 + HD;
                const int C = cdiv(tk.ctx_hi - tk.ctx_lo + 1, CH);     // chunks holding visible keys
                // the C records of the head are contiguous: chunk c at (qh * CM + c) * rec
                Range rg[1] = {Range{ll + w_part(g, qh, 0, 0), C * rec, s.stage, tag_of(seq, l, PH_PART)}};
                if (!gather<5, 1>(S->err, rg)) return;
                // M = max m_c, w_c = l_c exp(m_c - M) (lane c of wave 0), then out = sum_c w_c o_c / sum_c w_c
                if (tid < 64) {
                    const float lc = tid < C ? s.stage[tid * rec + 1] : 0.f;
                    const float mc = lc > 0.f ? s.stage[tid * rec] : -INFINITY;
                    const float M = wave_max_dpp(mc);
                    const float wc = lc > 0.f ? expf(mc - M) * lc : 0.f;
                    const float L = wave_sum_dpp(wc);
                    if (tid < MAX_CM) s.cw[tid] = wc;
                    if (tid == 0) s.wsum[0] = L;
                }
                lds_barrier();
                if (tid < HD) {
                    float acc = 0.f;
#pragma unroll 4
                    for (int c = 0; c < C; ++c) acc += s.cw[c] * s.stage[c * rec + 2 + tid];
                    st_word(ll + w_att(g, qh * HD + tid), acc / s.wsum[0], tag_of(seq, l, PH_ATT));
                }
                lds_barrier();
            }
        }
        // ---------------------------------------------------------------- P3, P4 and P5 share the down tiles.
        // Loads complete in order, and a load issued between a hand-off's arrival and the block's own publishing
        // stores delays those stores, so weights are issued only right before a phase's wait, and bulk loads at the
        // start of a layer slow the attention phase (its loads and stores share the memory system with them).  A
        // block with three gate_up units (P4 waits ~10 us for the o_proj output) copies the down tiles of its P5 item
        // to LDS together with its gate_up tiles; its activation poll in P5 then does not queue behind 70 KiB of its
        // own loads.  The other P5 blocks load the down tiles when P5 starts.
        T5T t5;
        bool have5 = false;                        // block-uniform
        // ---------------------------------------------------------------- P3: o_proj row tile + residual
        {
            CStatic *S = fresh(sp);
            const Geom g = S->g;
            if (b >= g.B3 && b < g.B3 + g.NO) {
                const int tid = fresh_tid(), lane = tid & 63, wv = tid >> 6, r = lane & 15;
                CLayer *lp = layer_of(S, l);
                u64 *ll = S->ll;
                const int item = b - g.B3;
                Tiles<FMT, TH> tl;
                tl.load(lp->w[1], lp->sz[1], g.nkt_a, item, 0, g.nkt_a, wv, lane);
                // the attention output and (l > 0) the residual parts of the tile's rows, in one hand-off (threads
                // 0..15 hold the residual parts of row tid)
                RRange rg[3];
                rg[0] = RRange{ll + w_att(g, 0), g.NH * HD, tag_of(seq, l, PH_ATT)};
                if (l == 0) {
                    rg[1] = rg[2] = RRange{ll, 0, 0u};
                } else {
                    residual_ranges(g, ll, seq, l, item * 16, 16, rg + 1);
                }
                float v3[3][NPT];
                if (!gather_r<NPT, 3>(S->err, rg, v3, tid)) return;
                if (l == 0 && tid < 16) {
                    const int token = stp.feed ? min(max(stp.feed[0], 0), g.V - 1) : tk.token;
                    v3[1][0] = packed_elem<FMT>(S->emb_w, S->emb_sz, g.nkt_h, token, item * 16 + tid);
                    v3[2][0] = 0.f;
                }
                pairs<NPT>(s, v3[0], g.NH * HD, tid);
                const float v = stream_dot<FMT, TH>(s, tl, wv, lane);
                if (lane < 16) s.red[wv * 16 + lane] = v;
                lds_barrier();
                if (tid < 16) {
                    const float x = v3[1][0] + v3[2][0];
                    st_word(ll + w_xm(g, item * 16 + r), x + wave_total(s, 1, 0, r), tag_of(seq, l, PH_XM));
                }
            }
        }
        // ---------------------------------------------------------------- P4: RMSNorm + gate_up units + SwiGLU
        {
            CStatic *S = fresh(sp);
            const Geom g = S->g;
            const int nu = p4_count(g, b);
            const bool is5 = b >= g.B5 && b < g.B5 + g.ND;
            if (nu > 0) {
                const int tid = fresh_tid(), lane = tid & 63, wv = tid >> 6;
                CLayer *lp = layer_of(S, l);
                if (b < g.B3) {
                    Tiles<FMT, TH> tg[MAXU], tu[MAXU];
#pragma unroll
                    for (int i = 0; i < MAXU; ++i) {
                        if (i < nu) {
                            const int u = p4_unit(g, b, i);
                            tg[i].load(lp->w[2], lp->sz[2], g.nkt_h, 2 * u, 0, g.nkt_h, wv, lane);
                            tu[i].load(lp->w[2], lp->sz[2], g.nkt_h, 2 * u + 1, 0, g.nkt_h, wv, lane);
                        }
                    }
                    if (DMA5 && is5) {
                        down_tiles(wt5, t5, g, lp, b, wv, lane);
                        have5 = true;
                    }
                    if (!gate_up<FMT, TH, MAXU>(s, S, g, lp, l, seq, b, nu, tg, tu, tid)) return;
                } else {
                    Tiles<FMT, TH> tg1, tu1;
                    const int u = p4_unit(g, b, 0);
                    tg1.load(lp->w[2], lp->sz[2], g.nkt_h, 2 * u, 0, g.nkt_h, wv, lane);
                    tu1.load(lp->w[2], lp->sz[2], g.nkt_h, 2 * u + 1, 0, g.nkt_h, wv, lane);
                    if (!gate_up<FMT, TH, 1>(s, S, g, lp, l, seq, b, 1, &tg1, &tu1, tid)) return;
                }
            }
        }
        // ---------------------------------------------------------------- P5: down row tile, one k half
        {
            CStatic *S = fresh(sp);
            const Geom g = S->g;
            if (b >= g.B5 && b < g.B5 + g.ND) {
                const int tid = fresh_tid(), lane = tid & 63, wv = tid >> 6, r = lane & 15;
                CLayer *lp = layer_of(S, l);
                u64 *ll = S->ll;
                const int d = b - g.B5, rt = d % g.NO, kh = d / g.NO;
                const int kt0 = kh * g.nk5, kt1 = min(g.nkt_i, kt0 + g.nk5);
                if (!have5) down_tiles(wt5, t5, g, lp, b, wv, lane);
                const int klen = (kt1 - kt0) * TileGeom<FMT>::KT;
                // the activations of the k half and (k half 0) the o_proj rows of the tile, which it adds (threads
                // 0..15 hold row tid's)
                constexpr int NPK = (MAX_K / 2 + NT - 1) / NT;     // activation words (two values each) per thread
                RRange rg[2] = {RRange{ll + w_act(g, kt0 * TileGeom<FMT>::KT / 2), klen / 2, tag16_of(seq, l), 48},
                                RRange{ll + w_xm(g, rt * 16), kh == 0 ? 16 : 0, tag_of(seq, l, PH_XM)}};
                u64 v5[2][NPK];
                if (!gather_w<NPK, 2>(S->err, rg, v5, tid)) return;
#pragma unroll
                for (int j = 0; j < NPK; ++j) {
                    const int m = tid + NT * j;
                    if (m < klen / 2) {
                        f16 h0, l0, h1, l1;
                        split_f16(f32_of24((uint32_t)v5[0][j] & 0xFFFFFFu), h0, l0);
                        split_f16(f32_of24((uint32_t)(v5[0][j] >> 24) & 0xFFFFFFu), h1, l1);
                        *(f16x2 *)&s.xh[2 * m] = (f16x2){h0, h1};
                        *(f16x2 *)&s.xl[2 * m] = (f16x2){l0, l1};
                    }
                }
                if (tid < 8) s.xh[MAX_K + tid] = (f16)0.f;
                lds_barrier();
                const float v = stream_dot<FMT, T5>(s, t5, wv, lane);
                if (lane < 16) s.red[wv * 16 + lane] = v;
                lds_barrier();
                if (tid < 16) {
                    const float dv = wave_total(s, 1, 0, r);
                    st_word(ll + w_dp(g, kh, rt * 16 + r), kh == 0 ? __uint_as_float((unsigned)v5[1][0]) + dv : dv,
                            tag_of(seq, l, PH_DP));
                }
                lds_barrier();
            }
        }
    }
    // ---------------------------------------------------------------- final RMSNorm (block 0) for the head GEMV
    if (b == 0) {
        CStatic *S = fresh(sp);
        const Geom g = S->g;
        const int tid = fresh_tid();
        NormW nw;
        nw.load(S->final_norm, g.H, tid);
        RRange rg[2];
        residual_ranges(g, S->ll, seq, g.L, 0, g.H, rg);
        float v[2][NPT], x[NPT];
        if (!gather_r<NPT, 2>(S->err, rg, v, tid)) return;
        float ss = 0.f;
        {
#pragma clang fp contract(off)
#pragma unroll
            for (int j = 0; j < NPT; ++j) {
                x[j] = v[0][j] + v[1][j];
                const float xv = tid + NT * j < g.H ? x[j] : 0.f;
                ss += xv * xv;
            }
        }
        const float tot = block_sum_fixed(ss, s.wsum);
        const float rs = 1.0f / sqrtf(tot / (float)g.H + S->eps);
        f16 *xn = S->xn;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int k = tid + NT * j;
            if (k < g.H) xn[k] = (f16)((x[j] * rs) * nw.w[j]);
        }
    }
}

// ------------------------------------------------------------------------------------------------------- host
// The geometry of a model shape on nb blocks, or false (with the reason) when the persistent step does not apply.
inline bool make_geom(const sp_model_desc &d, int n_slots, int nb, Geom &g, const char **why) {
    auto no = [&](const char *m) { *why = m; return false; };
    g = Geom{};
    g.L = d.n_layers; g.H = d.hidden; g.NH = d.n_heads; g.NKV = d.n_kv_heads; g.HD = d.head_dim; g.I = d.intermediate;
    g.V = d.vocab; g.Nqkv = (g.NH + 2 * g.NKV) * g.HD; g.n_slots = n_slots; g.fmt = d.weight_format; g.nb = nb;
    g.KT = g.fmt == SP_FMT_F16 ? 32 : g.fmt == SP_FMT_Q8 ? 64 : 128;
    if (g.fmt != SP_FMT_F16 && g.fmt != SP_FMT_Q8 && g.fmt != SP_FMT_Q4) return no("weight format");
    if (g.L < 1 || g.L > MAX_L) return no("layers: at most 32");
    if (g.H > MAX_H || g.H % g.KT || g.I % g.KT || (g.NH * g.HD) % g.KT) return no("hidden / intermediate sizes");
    if (g.HD > MAX_HD || g.NH % g.NKV || g.NH / g.NKV > MAX_G || g.NH / g.NKV > NW) return no("heads");
    if (g.NH * g.HD > MAX_H) return no("attention width");
    if (n_slots < 1) return no("KV slots");
    g.nkt_h = g.H / g.KT; g.nkt_a = g.NH * g.HD / g.KT; g.nkt_i = g.I / g.KT;
    g.NQ = g.Nqkv / 16; g.CM = cdiv(n_slots, CH); g.NO = g.H / 16; g.NU = g.I / 16;
    g.ND = g.NO * KS; g.nk5 = cdiv(g.nkt_i, KS);
    if (g.Nqkv % 16 || g.H % 16 || g.I % 16) return no("row tiles");
    if (g.CM > MAX_CM) return no("attention chunks per kv head");
    g.B2 = g.NQ; g.B2b = g.B2 + g.NKV * g.CM; g.B3 = nb - g.NO; g.B5 = nb - g.ND;
    if (g.B2b + g.NH > nb) return no("qkv tiles + attention chunks + combiners exceed the blocks");
    if (g.B3 < 1 || g.B5 < 0) return no("o_proj / down items exceed the blocks");
    g.nu_max = std::min(MAXU, cdiv(g.NU, g.B3));
    if (g.NU > MAXU * g.B3 + g.NO) return no("gate_up units per block");
    if (g.nk5 * g.KT > MAX_K) return no("down k half");
    if ((size_t)g.CM * (2 + g.HD) > MAX_K + 16 || g.NH / g.NKV * g.HD > MAX_K + 16) return no("staging");
    size_t o = 0;
    g.o_qkv = o; o += g.Nqkv;
    g.o_part = o; o += (size_t)g.NH * g.CM * (2 + g.HD);
    g.o_att = o; o += (size_t)g.NH * g.HD;
    g.o_xm = o; o += g.H;
    g.o_act = o; o += g.I / 2;
    g.o_dp = o; o += (size_t)KS * g.H;
    g.words = o;
    return true;
}

// Walks every item of every phase the way the kernel does and checks: the block it runs on, every tagged word it
// reads or writes (inside its region and inside `words`), every weight row group and k-tile (inside the matrix), the
// staged element counts (inside the LDS arrays and the gathers' per-thread batches), and the per-wave tile counts
// TH / T5 of the instantiation.
inline bool check_geom(const Geom &g, int TH, int T5, const char **why) {
    auto no = [&](const char *m) { *why = m; return false; };
    const int G = g.NH / g.NKV, rec = 2 + g.HD;
    auto in = [&](size_t lo, size_t n, size_t rlo, size_t rhi) { return lo >= rlo && lo + n <= rhi; };
    const size_t e_qkv = g.o_part, e_part = g.o_att, e_att = g.o_xm, e_xm = g.o_act, e_act = g.o_dp, e_dp = g.words;
    if (TH * NW < g.nkt_h || TH * NW < g.nkt_a || T5 * NW < g.nk5) return no("tiles per wave");
    if (g.CM > MAX_CM || g.CM * rec > MAX_K + 16) return no("combine records");
    for (int i = 0; i < g.NQ; ++i) {
        if (blk_p1(g, i) >= g.nb) return no("qkv block");
        if (!in(w_qkv(g, i * 16), 16, g.o_qkv, e_qkv) || (i + 1) * 16 > g.Nqkv) return no("qkv words");
    }
    for (int kvh = 0; kvh < g.NKV; ++kvh)
        for (int c = 0; c < g.CM; ++c) {
            if (blk_p2(g, kvh, c) >= g.nb) return no("attention block");
            if (!in(w_qkv(g, kvh * G * g.HD), G * g.HD, g.o_qkv, e_qkv)) return no("query words");
            if (!in(w_qkv(g, (g.NH + kvh) * g.HD), g.HD, g.o_qkv, e_qkv)) return no("key words");
            if (!in(w_qkv(g, (g.NH + g.NKV + kvh) * g.HD), g.HD, g.o_qkv, e_qkv)) return no("value words");
            if (G * g.HD + 2 * g.HD > MAX_G * MAX_HD + 2 * MAX_HD) return no("attention gather");
            for (int h = 0; h < G; ++h)
                if (!in(w_part(g, kvh * G + h, c, 0), rec, g.o_part, e_part)) return no("partial words");
        }
    for (int qh = 0; qh < g.NH; ++qh) {
        if (blk_p2b(g, qh) >= g.nb) return no("combiner block");
        if (!in(w_part(g, qh, 0, 0), (size_t)g.CM * rec, g.o_part, e_part)) return no("combiner words");
        if (!in(w_att(g, qh * g.HD), g.HD, g.o_att, e_att)) return no("attention words");
    }
    for (int i = 0; i < g.NO; ++i) {
        if (blk_p3(g, i) >= g.nb || blk_p3(g, i) < 0) return no("o_proj block");
        if (!in(w_xm(g, i * 16), 16, g.o_xm, e_xm)) return no("residual words");
        for (int sl = 0; sl < KS; ++sl)
            if (!in(w_dp(g, sl, i * 16), 16, g.o_dp, e_dp)) return no("down words");
    }
    std::vector<int> per(g.nb, 0), seen(g.NU, 0);
    for (int u = 0; u < g.NU; ++u) {
        const int bk = blk_p4(g, u);
        if (bk < 0 || bk >= g.nb) return no("gate_up block");
        if (++per[bk] > MAXU) return no("gate_up units per block");
        if (!in(w_act(g, u * 8), 8, g.o_act, e_act) || 2 * u + 1 >= 2 * g.NU) return no("activation words");
    }
    for (int bk = 0; bk < g.nb; ++bk) {             // the kernel's per-block list is exactly the units mapped there
        const int n = p4_count(g, bk);
        if (n != per[bk] || n > MAXU) return no("gate_up unit list");
        for (int i = 0; i < n; ++i) {
            const int u = p4_unit(g, bk, i);
            if (u < 0 || u >= g.NU || blk_p4(g, u) != bk || seen[u]++) return no("gate_up unit list");
        }
    }
    for (int dd = 0; dd < g.ND; ++dd) {
        const int bk = blk_p5(g, dd);
        if (bk < 0 || bk >= g.nb) return no("down block");
        const int rt = dd % g.NO, kh = dd / g.NO;
        const int kt0 = kh * g.nk5, kt1 = std::min(g.nkt_i, kt0 + g.nk5);
        if (kt0 >= kt1 || rt * 16 + 16 > g.H) return no("down item");
        if (!in(w_act(g, kt0 * g.KT / 2), (size_t)(kt1 - kt0) * g.KT / 2, g.o_act, e_act)) return no("down input words");
        if ((kt1 - kt0) * g.KT > MAX_K) return no("down input staging");
        if (!in(w_xm(g, rt * 16), 16, g.o_xm, e_xm)) return no("down residual words");
        if (!in(w_dp(g, kh, rt * 16), 16, g.o_dp, e_dp)) return no("down output words");
    }
    if (!in(w_xm(g, 0), g.H, g.o_xm, e_xm)) return no("residual gather");
    return true;
}

}  // namespace d1
