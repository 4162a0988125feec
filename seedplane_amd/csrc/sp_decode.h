// Persistent single-column decode step: the whole Qwen2 forward for one new token (all layers, final norm, LM head,
// argmax) in one cooperative launch of one block per CU.
//
// Why: at batch 1 the step is a chain of ~150-260 small dependent kernels, and on this GPU every kernel boundary
// costs about 4 us (launch, the L2 write-back / invalidate at kernel edges, a cold HBM round trip), far more than
// the 3-30 MB each of them streams.  Inside one kernel a hand-off of a 64-bit word between blocks on different XCDs
// costs about 0.4 us (relaxed agent-scope atomic store / load, measured by ping-pong), so the step becomes a chain of
// cheap hand-offs while the weights stream continuously.
//
// Block layout: NWK worker waves + one poller wave (the last).
//   * Worker waves never touch global memory except through LDS DMA (global_load_lds): each one streams its share of
//     every weight tile of the step (and of the K/V chunk of its block's attention item) into a private LDS ring, in
//     one fixed order over the whole forward, and keeps up to DT tiles in flight.  Vector-memory loads of a wave
//     complete in order, so "tile e has landed" is `s_waitcnt vmcnt(<entries issued after e>)`; the DMA of a tile
//     for a later phase (or layer) is issued as soon as a ring slot frees, so weights keep streaming while the block
//     waits for its next input.
//   * The poller wave does every global access that is not weight streaming: it gathers a phase's input from the
//     other blocks, publishes the phase's outputs, and runs the small scalar steps (RMSNorm, RoPE, the attention
//     combine, epilogues).  Its polls therefore never queue behind weight DMAs.
// Work is owned, not split: every GEMV row group (16 rows; 16 gate + 16 up rows for gate_up) belongs to one block
// (host-side balancing over the whole layer), and the block's workers take its k-tiles w, w + NWK, ... and are reduced
// through LDS in wave order (deterministic).  So every hand-off carries final values: the residual stream, q/k/v
// rows, attention partials, the attention output, the SwiGLU activation, and per-block argmax candidates.
//
// Hand-off ("LL" words): payload in the low 32 bits, a 32-bit tag in the high bits, written with one relaxed
// agent-scope 64-bit atomic store; consumers poll with relaxed agent-scope 64-bit atomic loads until every tag
// matches (single-copy atomic words: no fence anywhere; an agent-scope fence writes back a whole XCD L2).
// Tag = (launch id << 12) | (layer * 8 + region): every region of every layer is written once per launch.  Every
// wait is bounded; a timeout sets the error word, and every block leaves at its next barrier.
//
// Per layer l (phases a block does not own are skipped):
//   QKV  x_l (gathered; the embedding row at l = 0) -> RMSNorm -> qkv rows (+ bias)          -> R_QKV
//   ATT  (kv head g, chunk c of CH visible keys): q/k/v rows of g, RoPE, the new key / value patched into the chunk
//        (and written to its cache slot by the owner of the last chunk), scores, chunk softmax, P.V -> {m, l, acc}
//   CMB  one query head: merge the chunk partials                                          -> attention output
//   O    x_mid rows = x_l rows + o_proj(attention output)                                    -> R_XMID
//   GU   RMSNorm(x_mid) -> SiLU(gate) * up, fp16 pairs                                      -> R_ACT
//   DN   x_{l+1} rows = x_mid rows + down(act)                                               -> R_X
// then HEAD: RMSNorm(x_L) -> logits rows of the block's head row groups + block argmax -> block 0 picks the token.
//
// Replaces, for one decode column, the same reference computation as the kernel chain in sp_engine::step
// (seedplane/qwen_engine.py:117-148).
#pragma once
#include "sp_attn.h"
#include "sp_gemv.h"

namespace mk {

typedef unsigned long long u64;
constexpr int NWK = 8;                 // worker waves
constexpr int NT = 64 * (NWK + 1);     // + the poller
constexpr int PW = NWK;                // poller wave index
constexpr int MAXI = 8;                // items of one GEMV phase per block (LM-head items per batch)
constexpr int MAX_L = 48;              // layers of the on-chip pointer table
constexpr int MAX_K = 9216;            // widest GEMV input (the fp16 A operand)
constexpr int STAGE = 4608;            // gathered words
constexpr int CH = 64;                 // keys per attention item
constexpr int MAX_G = 8;               // query heads per kv head
constexpr int MAX_HN = 32;             // hidden size / 64 held in the poller's registers (H <= 2048)
constexpr int MAX_NCH = 64;            // attention chunks per kv head
constexpr int EMAX = 48;               // DMA instructions in flight per worker wave (vmcnt counts to 63)
constexpr long MAX_POLLS = 1l << 20;

enum { PH_KV = 0, PH_QKV = 1, PH_O = 2, PH_GU = 3, PH_DN = 4, PH_HEAD = 5, PH_END = 6 };
enum { R_QKV = 1, R_PART = 2, R_ATT = 3, R_XMID = 4, R_ACT = 5, R_X = 6, R_AM = 7 };

template <int FMT> struct RingGeom {
    static constexpr int SIDE = FMT == 1 ? 0 : FMT == 2 ? 64 : 256;   // scale (+ zero) bytes of a tile
    static constexpr int SLOT = TILE_BYTES + SIDE;
#ifdef MK_DT
    static constexpr int DT = MK_DT;
#else
    static constexpr int DT = FMT == 3 ? 7 : 8;                        // tiles in flight per worker wave
#endif
    static constexpr int EPT = FMT == 1 ? 1 : 2;                       // DMA instructions per tile
};

// Host-built work plan of one block (identical for every layer).
struct Plan {
    short item[4][MAXI];   // row groups (gate/up pairs for GU) of QKV, O, GU, DN
    int n[4];
    int att;               // attention item kv_head * nch_max + chunk, or -1
    int cmb;               // query head merged by this block, or -1
    int h0, h1;            // LM-head row groups [h0, h1)
};

// Weight / cache pointers the workers stream from (QKV, O, GU, DN).
struct LayerPtr {
    const uint8_t *w[4];
    const f16 *sz[4];
    const f16 *kc, *vc;
};
// Per-layer operands only the poller reads.
struct LayerAux {
    const float *qkv_b, *in_norm, *post_norm;
    f16 *kc, *vc;
};

struct Args {
    const Plan *plans;
    const LayerPtr *lp;
    const LayerAux *aux;
    const uint8_t *emb_w; const f16 *emb_sz; int emb_nkt;
    const uint8_t *head_w; const f16 *head_sz;
    const float *final_norm, *inv_freq;
    sp_token tok;            // the decode column (by value)
    int nkt[6];              // per phase: KV pieces, then k-tiles of QKV, O, GU, DN, HEAD
    int L, H, NH, NKV, I, V, Nqkv, n_slots, nch_max;
    float eps, scale;
    u64 *ll;
    size_t o_part, o_att, o_xmid, o_act, o_x, stride, o_am;
    int nb_head;             // blocks holding LM-head rows: 0 .. nb_head - 1
    unsigned tag0;
    unsigned *err;
    float *logits;           // may be NULL
    int *out_id;             // the chosen token (written by block 0)
};

template <int FMT, int HD>
struct Smem {
    using RG_ = RingGeom<FMT>;
    __align__(16) unsigned char ring[NWK][RG_::DT * RG_::SLOT];
    __align__(16) f16 a[MAX_K];               // A operand of the current GEMV (fp16, zero past K)
    __align__(16) unsigned stage[STAGE];      // gathered payloads / attention P.V partials
    __align__(16) f16 kv[2][CH][HD];          // K and V rows of the block's attention chunk (row-major)
    __align__(16) float red[MAXI * NWK * 2 * 16];   // per-wave row sums of a phase (head: two RG=1 buffers)
    LayerPtr lp[MAX_L + 1];                   // per layer, then the LM head in row L
    Plan plan;
    float qf[MAX_G][HD];                      // rotated, scaled queries
    float sc[MAX_G][CH];                      // scores, then probabilities
    float xr[2][MAXI][16];                    // residual rows of the block's O / DN items
    float mh[MAX_G], lh[MAX_G];
    __align__(16) f16 kn[HD], vn[HD];
    int vote[2][16];                          // per-wave flags of bar_or (two alternating sets)
};

// Phase timestamps for profiling builds (-DSP_DECODE_TRACE): lane 0 of the poller records the 100 MHz clock at
// phase boundaries of the first layers.  Compiled out otherwise.
#ifdef SP_DECODE_TRACE
__device__ unsigned long long trace_buf[1024][64];
#define MK_TRACE(ev) do { if (threadIdx.x == 64 * PW && (ev) < 48) trace_buf[blockIdx.x][(ev)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#define MK_TRACE2(ev) do { if (threadIdx.x == 64 * PW && l == 1) trace_buf[blockIdx.x][48 + (ev)] = __builtin_amdgcn_s_memrealtime(); } while (0)
__device__ unsigned long long wtrace[1024][16][4];   // per block, wave: wait cycles, issue cycles, mac cycles
#define MK_T0() const unsigned long long t0_ = __builtin_amdgcn_s_memtime()
#define MK_TACC(slot) do { st.tacc[slot] += __builtin_amdgcn_s_memtime() - t0_; } while (0)
#else
#define MK_TRACE(ev) do { } while (0)
#define MK_TRACE2(ev) do { } while (0)
#define MK_T0() do { } while (0)
#define MK_TACC(slot) do { } while (0)
#endif

__device__ __forceinline__ void ll_put(u64 *p, unsigned tag, unsigned payload) {
    __hip_atomic_store(p, ((u64)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 ll_peek(const u64 *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool err_set(const unsigned *err) {
    return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// s_waitcnt vmcnt(n) for a wave-uniform n (the counter field holds 0..63).
__device__ __forceinline__ void wait_vm(int n) {
#define MK_W(i) case i: asm volatile("s_waitcnt vmcnt(" #i ")" ::: "memory"); break;
    switch (n < 0 ? 0 : n) {
        MK_W(0) MK_W(1) MK_W(2) MK_W(3) MK_W(4) MK_W(5) MK_W(6) MK_W(7) MK_W(8) MK_W(9) MK_W(10) MK_W(11) MK_W(12)
        MK_W(13) MK_W(14) MK_W(15) MK_W(16) MK_W(17) MK_W(18) MK_W(19) MK_W(20) MK_W(21) MK_W(22) MK_W(23) MK_W(24)
        MK_W(25) MK_W(26) MK_W(27) MK_W(28) MK_W(29) MK_W(30) MK_W(31) MK_W(32) MK_W(33) MK_W(34) MK_W(35) MK_W(36)
        MK_W(37) MK_W(38) MK_W(39) MK_W(40) MK_W(41) MK_W(42) MK_W(43) MK_W(44) MK_W(45) MK_W(46) MK_W(47) MK_W(48)
        MK_W(49) MK_W(50) MK_W(51) MK_W(52) MK_W(53) MK_W(54) MK_W(55) MK_W(56) MK_W(57) MK_W(58) MK_W(59) MK_W(60)
        MK_W(61) MK_W(62)
        default: asm volatile("s_waitcnt vmcnt(63)" ::: "memory"); break;
    }
#undef MK_W
}

// LDS reads of DMA destinations go through inline asm: the compiler cannot tell which LDS DMA a read depends on and
// would otherwise wait for every DMA in flight (vmcnt(0)) before each one.  The waits are explicit instead: vmcnt for
// the DMA, then lgkmcnt(0) before the values are used.
__device__ __forceinline__ unsigned lds_addr(const void *p) {
    return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ __forceinline__ u32x4 lds_ld128(const void *p) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}
__device__ __forceinline__ uint32_t lds_ld32(const void *p) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}
__device__ __forceinline__ uint32_t lds_ldu16(const void *p) {
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}
__device__ __forceinline__ u64 lds_ld64(const void *p) {
    u64 v;
    asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}
__device__ __forceinline__ void lgkm_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Waits for the outstanding LDS reads and ties `v` to the wait: the compiler treats the asm reads above as complete
// when they issue, so without this data dependence it may schedule a use of `v` before the wait.
template <class T>
__device__ __forceinline__ void lgkm_tie(T &v) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v) :: "memory"); }
// Wave-uniform LDS values read by worker waves: read and wait in one asm statement, then a scalar copy.
__device__ __forceinline__ int lds_int(const int *p) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return __builtin_amdgcn_readfirstlane((int)v);
}
template <class T>
__device__ __forceinline__ T *lds_ptr(T *const *p) {
    u64 v;
    asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T *)(((u64)hi << 32) | lo);
}

// LDS DMA.  The worker streams issue it through inline asm, invisible to the compiler: otherwise the compiler, which
// cannot tell which LDS bytes a DMA writes, waits for every DMA in flight (vmcnt(0)) before LDS accesses and
// barriers, which would serialise the stream.  Every read of DMA-written LDS is preceded by an explicit
// `s_waitcnt vmcnt(n)` (in-order completion) and goes through the asm reads above.
__device__ __forceinline__ void sdma16(const void *g, unsigned char *l) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr(l))) : "memory", "m0");
}
__device__ __forceinline__ void sdma4(const void *g, unsigned char *l) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr(l))) : "memory", "m0");
}
// Block barrier without a memory fence: a fence at work-group scope makes the compiler wait for all vector memory
// operations of the wave (vmcnt(0)), which would include the DMA stream.  LDS traffic is ordered by lgkmcnt(0);
// global hand-offs never need the barrier.
__device__ __forceinline__ void bar() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Kernel-uniform facts a worker wave needs to walk its stream (scalar registers; phase-indexed reads are selects).
struct Walk {
    int L, w;                            // layers, this worker wave
    int nkt[6];                          // per phase (PH_KV: 1-KiB pieces of the K/V chunk); only indexed by constants
    int cnt[6];                          // items of this block per phase (PH_KV: 1 when the attention item is live)
    int h0;                              // first LM-head row group of the block
    int kv_g, kv_v0, kv_cnt;             // attention item: kv head, first visible key of the chunk, keys in it
};
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int sel6(const int (&v)[6], int ph) {
    return ph == 0 ? v[0] : ph == 1 ? v[1] : ph == 2 ? v[2] : ph == 3 ? v[3] : ph == 4 ? v[4] : v[5];
}

// Position in a worker wave's DMA stream.  Order: per layer [K/V pieces w, w + NWK, ...] [QKV] [O] [GU] [DN], then
// [HEAD]; inside a GEMV phase: items in plan order, k-tiles w, w + NWK, ...  A step is one k-tile of one item: its
// RG tiles (gate, up) with EPT instructions each (codes, then side data), or one K/V piece.  The step's addresses
// advance by constant strides; tables are read only when an item or a phase begins.
struct Cursor {
    int l, ph, i, k;        // layer, phase, item; k = next K/V piece (PH_KV)
    int ks;                 // steps left in the current item
    int n;                  // instructions issued so far
    int tiles;              // tiles so far (ring slot = tiles % DT)
    int nkt, cnt, rg;       // current phase: k-tiles, items, tiles per step
    const uint8_t *pc;      // codes of the next step's first tile
    const uint8_t *ps;      // side data of the next step's first tile
    long rgc, rgs;          // bytes from the gate tile to the up tile (codes, side data)
    const void *p0, *p1;    // codes / side data base (PH_KV: key / value cache of the layer)
};

template <int FMT> struct SideB { static constexpr int V = FMT == 2 ? 64 : FMT == 3 ? 256 : 0; };

__device__ __forceinline__ void cur_next_phase(Cursor &c, const Walk &wk) {
    c.i = 0;
    if (c.ph == PH_DN) {
        if (c.l + 1 < wk.L) { ++c.l; c.ph = PH_KV; } else c.ph = PH_HEAD;
    } else if (c.ph == PH_HEAD) {
        c.ph = PH_END;
    } else {
        ++c.ph;
    }
    c.nkt = sel6(wk.nkt, c.ph);
    c.cnt = c.ph == PH_END ? 0 : sel6(wk.cnt, c.ph);
    c.rg = c.ph == PH_GU ? 2 : 1;
}
template <int FMT, int HD>
__device__ __forceinline__ void cur_enter_item(Smem<FMT, HD> &S, Cursor &c, const Walk &wk) {
    c.ks = (c.nkt - wk.w + NWK - 1) / NWK;
    if (c.ph == PH_KV) { c.k = wk.w; return; }
    const int unit = c.ph == PH_HEAD ? wk.h0 + c.i
                                     : (lds_int((const int *)&S.plan.item[c.ph - 1][c.i & ~1]) >> (16 * (c.i & 1))) & 0xffff;
    const long tile0 = (long)unit * c.rg * c.nkt + wk.w;
    c.pc = (const uint8_t *)c.p0 + tile0 * TILE_BYTES;
    c.ps = (const uint8_t *)c.p1 + tile0 * SideB<FMT>::V;
    c.rgc = (long)c.nkt * TILE_BYTES;
    c.rgs = (long)c.nkt * SideB<FMT>::V;
}
// Moves past phases in which this wave has nothing to stream; loads the pointers of the phase it stops in.
template <int FMT, int HD>
__device__ __forceinline__ void cur_settle(Smem<FMT, HD> &S, Cursor &c, const Walk &wk) {
    while (c.ph != PH_END && (c.i >= c.cnt || wk.w >= c.nkt)) cur_next_phase(c, wk);
    if (c.ph == PH_END) return;
    if (c.ph == PH_KV) {
        c.p0 = lds_ptr(&S.lp[c.l].kc);
        c.p1 = lds_ptr(&S.lp[c.l].vc);
    } else {
        // LM head pointers sit in row L of the table (slot 0)
        const LayerPtr &P = S.lp[c.ph == PH_HEAD ? wk.L : c.l];
        const int mi = c.ph == PH_HEAD ? 0 : c.ph - 1;
        c.p0 = lds_ptr(&P.w[mi]);
        c.p1 = FMT == 1 ? nullptr : (const void *)lds_ptr(&P.sz[mi]);
    }
    cur_enter_item(S, c, wk);
}

// Worker-side state of the DMA stream.
struct Stream {
    Cursor iss;             // next step to issue
    int cons_n, cons_tiles; // consumed instructions / tiles
    int att_done;           // last layer whose attention item this block finished (K/V area free after it)
    bool bad;               // the consumer needed an instruction the issuer could not issue (logic error)
#ifdef SP_DECODE_TRACE
    unsigned long long tacc[3];
#endif
};

template <int FMT, int HD>
__device__ __forceinline__ void issue_step(Smem<FMT, HD> &S, const Args &a, const Walk &wk, const sp_token &t, Stream &st) {
    using G = RingGeom<FMT>;
    const int lane = threadIdx.x & 63;
    Cursor &c = st.iss;
    if (c.ph == PH_KV) {
        // piece p: 1 KiB of K (p < NP/2) or V rows of the chunk; lane -> (key, 16-byte part)
        const int np2 = c.nkt >> 1, p = c.k, isv = p >= np2, pp = isv ? p - np2 : p;
        constexpr int LPK = HD / 8;                      // lanes per key (16 bytes each)
        constexpr int KPP = 64 / LPK;                    // keys per piece
        const int j = pp * KPP + lane / LPK, part = lane % LPK;
        const int kp = t.ctx_lo + wk.kv_v0 + (j < wk.kv_cnt ? j : 0);
        const size_t off = (((size_t)t.seq * a.NKV + wk.kv_g) * a.n_slots + kp % a.n_slots) * HD + part * 8;
        const f16 *src = (const f16 *)(isv ? c.p1 : c.p0) + off;
        sdma16(src, (unsigned char *)&S.kv[isv][0][0] + pp * 1024);
        c.k += NWK;
        c.n += 1;
    } else {
        unsigned char *ring = S.ring[wk.w];
        for (int r = 0; r < c.rg; ++r) {
            unsigned char *slot = ring + (c.tiles % G::DT) * G::SLOT;
            sdma16(c.pc + r * c.rgc + lane * 16, slot);
            if constexpr (FMT == 2) { if (lane < 16) sdma4(c.ps + r * c.rgs + lane * 4, slot + TILE_BYTES); }
            if constexpr (FMT == 3) { if (lane < 16) sdma16(c.ps + r * c.rgs + lane * 16, slot + TILE_BYTES); }
            ++c.tiles;
        }
        c.pc += NWK * TILE_BYTES;
        c.ps += NWK * SideB<FMT>::V;
        c.n += c.rg * G::EPT;
    }
    if (--c.ks > 0) return;
    if (++c.i < c.cnt) cur_enter_item(S, c, wk);
    else cur_settle(S, c, wk);
}

// Issues stream steps while ring slots, the in-flight limit and the K/V-area rule allow.
template <int FMT, int HD>
__device__ __forceinline__ void pump(Smem<FMT, HD> &S, const Args &a, const Walk &wk, const sp_token &t, Stream &st) {
    using G = RingGeom<FMT>;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");       // ring reads of consumed slots are complete
    while (st.iss.ph != PH_END) {
        if (st.iss.ph == PH_KV) {
            if (st.iss.l > st.att_done + 1 || st.iss.n + 1 - st.cons_n > EMAX) break;   // K/V area still in use
        } else if (st.iss.tiles + st.iss.rg - st.cons_tiles > G::DT || st.iss.n + st.iss.rg * G::EPT - st.cons_n > EMAX) {
            break;                                                                     // no free ring slot
        }
        issue_step<FMT, HD>(S, a, wk, t, st);
    }
}

// Makes instructions [cons_n, cons_n + n) available (landed) and consumes them.
template <int FMT, int HD>
__device__ __forceinline__ void consume(Smem<FMT, HD> &S, const Args &a, const Walk &wk, const sp_token &t, Stream &st, int n) {
    const int last = st.cons_n + n - 1;
    if (st.iss.n <= last) pump<FMT, HD>(S, a, wk, t, st);
    if (st.iss.n <= last) { st.bad = true; st.cons_n += n; return; }
    MK_T0();
    wait_vm(st.iss.n - last - 1);
    MK_TACC(0);
    st.cons_n += n;
}

// One k-tile step (RG tiles) against S.a: codes / side data from the ring, exact unpack, MFMA, block scales.
template <int FMT, int HD, int RG>
__device__ __forceinline__ void mac_step(Smem<FMT, HD> &S, Stream &st, int w, int kt, f32x4 acc[RG]) {
    using G = RingGeom<FMT>;
    constexpr int KT = TileGeom<FMT>::KT, ST = TileGeom<FMT>::STEPS;
    const int lane = threadIdx.x & 63, r = lane & 15, gq = lane >> 4;
    u32x4 wt[RG];
    uint32_t s8[RG];
    u32x4 s4[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        const unsigned char *slot = S.ring[w] + ((st.cons_tiles + rg) % G::DT) * G::SLOT;
        wt[rg] = lds_ld128(slot + lane * 16);
        if constexpr (FMT == 2) s8[rg] = lds_ld32(slot + TILE_BYTES + r * 4);
        if constexpr (FMT == 3) s4[rg] = lds_ld128(slot + TILE_BYTES + r * 16);
    }
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        lgkm_tie(wt[rg]);
        if constexpr (FMT == 2) lgkm_tie(s8[rg]);
        if constexpr (FMT == 3) lgkm_tie(s4[rg]);
    }
    st.cons_tiles += RG;
    const f16x8 zero8 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    const f16x8 ones8 = (f16x8){1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
    for (int s = 0; s < ST; ++s) {
        f16x8 xa = zero8;
        if (r == 0) {
            u32x4 xr = lds_ld128(S.a + kt * KT + s * 32 + 8 * gq);
            lgkm_tie(xr);
            xa = __builtin_bit_cast(f16x8, xr);
        }
        f32x4 xs = (f32x4){0.f, 0.f, 0.f, 0.f};
        if constexpr (FMT == 3) xs = mfma16(xa, ones8, xs);
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const f16x8 b = unpack_step<FMT>(wt[rg], s);
            if constexpr (FMT == 1) {
                acc[rg] = mfma16(xa, b, acc[rg]);
            } else if constexpr (FMT == 2) {
                const uint32_t d = s8[rg];
                const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(s == 0 ? (d & 0xffffu) : (d >> 16)));
                acc[rg] += scale * mfma16(xa, b, (f32x4){0.f, 0.f, 0.f, 0.f});
            } else {
                const uint32_t d = s == 0 ? s4[rg].x : s == 1 ? s4[rg].y : s == 2 ? s4[rg].z : s4[rg].w;
                const float scale = (float)__builtin_bit_cast(f16, (uint16_t)(d & 0xffffu));
                const float zero = (float)__builtin_bit_cast(f16, (uint16_t)(d >> 16));
                const f32x4 dd = mfma16(xa, b, (f32x4){0.f, 0.f, 0.f, 0.f});
                acc[rg] += scale * (dd - zero * xs);
            }
        }
    }
}

// A worker wave's part of a GEMV phase: items [i0, i0 + ni) of the phase, k-tiles w, w + NWK, ...; the wave's row
// sums (row 0 of D = register 0 of lanes 0..15) go to red[(i * NWK + w) * RG + rg][16] at buffer offset `rbase`.
template <int FMT, int HD, int RG>
__device__ __forceinline__ void gemv_items(Smem<FMT, HD> &S, const Args &a, const Walk &wk, const sp_token &t, Stream &st,
                                           int ph, int ni, float *rbase) {
    using G = RingGeom<FMT>;
    const int lane = threadIdx.x & 63, w = wk.w;
    const int nkt = sel6(wk.nkt, ph);
    for (int i = 0; i < ni; ++i) {
        f32x4 acc[RG];
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) acc[rg] = (f32x4){0.f, 0.f, 0.f, 0.f};
        for (int kt = w; kt < nkt; kt += NWK) {
            consume<FMT, HD>(S, a, wk, t, st, RG * G::EPT);
            {
                MK_T0();
                mac_step<FMT, HD, RG>(S, st, w, kt, acc);
                MK_TACC(2);
            }
            {
                MK_T0();
                pump<FMT, HD>(S, a, wk, t, st);
                MK_TACC(1);
            }
        }
        if (lane < 16) {
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) rbase[((i * NWK + w) * RG + rg) * 16 + lane] = acc[rg][0];
        }
    }
}

// ------------------------------------------------------------------------------------------------- poller side
// Gathers words src[0..n) carrying `tag` into dst[0..n) (LDS, 32-bit payloads); n <= 64 * U per wave.  While the
// producers are still busy the wave probes only its first 64 words (one load per lane) and sleeps between probes:
// uncached polls of every word by ~2000 waves would swamp the memory system the weight stream needs.  Once the probe
// is complete, everything is read in one round and misses are re-polled.  Bounded; returns false on timeout or when
// another block reported one.
constexpr int GATHER_U = 8;
__device__ __forceinline__ bool gather(const u64 *src, int n, unsigned tag, unsigned *dst, unsigned *err) {
    const int lane = threadIdx.x & 63;
    constexpr int U = GATHER_U;
    long polls = 0;
    auto give_up = [&]() {
        ++polls;
        if ((polls & 15) == 0) {
            const bool stop = polls > MAX_POLLS || err_set(err);
            if (__any(stop)) {
                if (polls > MAX_POLLS && lane == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return true;
            }
        }
        __builtin_amdgcn_s_sleep(4);
        return false;
    };
    // probe
    while (true) {
        const bool mine = lane < n;
        const u64 v = mine ? ll_peek(src + lane) : 0;
        if (!__any(mine && (unsigned)(v >> 32) != tag)) break;
        if (give_up()) return false;
    }
    for (int base = 0; base < n; base += 64 * U) {
        unsigned pending = 0;
#pragma unroll
        for (int j = 0; j < U; ++j)
            if (base + j * 64 + lane < n) pending |= 1u << j;
        while (__any(pending != 0)) {
            u64 v[U];
#pragma unroll
            for (int j = 0; j < U; ++j)
                if (pending & (1u << j)) v[j] = ll_peek(src + base + j * 64 + lane);
#pragma unroll
            for (int j = 0; j < U; ++j)
                if ((pending & (1u << j)) && (unsigned)(v[j] >> 32) == tag) {
                    dst[base + j * 64 + lane] = (unsigned)v[j];
                    pending &= ~(1u << j);
                }
            if (__any(pending != 0) && give_up()) return false;
        }
    }
    return true;
}

// Position of qkv row `row` in its hand-off region: grouped by kv head, [q rows of the group | key row | value row],
// so an attention item's input is one contiguous range.
__device__ __forceinline__ int qkv_pos(int row, int NH, int NKV, int HD) {
    const int G = NH / NKV;
    int g, off;
    if (row < NH * HD) { g = row / (G * HD); off = row - g * G * HD; }
    else if (row < (NH + NKV) * HD) { const int r2 = row - NH * HD; g = r2 / HD; off = G * HD + (r2 - g * HD); }
    else { const int r2 = row - (NH + NKV) * HD; g = r2 / HD; off = (G + 1) * HD + (r2 - g * HD); }
    return g * (G + 2) * HD + off;
}

// Block-wide gather: wave v polls words [v * per, (v + 1) * per) (per = n / 9 rounded up to 64), so all waves' loads
// are in flight together and a phase input costs one round trip.  Workers' loads complete after their DMAs in
// flight (in-order vector memory), which they need next anyway.
__device__ __forceinline__ void slice_of(int n, int wv, int &w0, int &cnt) {
    const int per = ((n + NWK) / (NWK + 1) + 63) & ~63;
    w0 = wv * per;
    cnt = min(per, n - w0);
}
__device__ __forceinline__ bool gather_blk(const u64 *src, int n, unsigned tag, unsigned *dst, unsigned *err, int wv) {
    int w0, cnt;
    slice_of(n, wv, w0, cnt);
    return cnt <= 0 || gather(src + w0, cnt, tag, dst + w0, err);
}

// The norm weight w[0..H) is brought into stage[NW_OFF ..) by LDS DMA (one 1-KiB copy per 256 floats, lanes past H
// re-read the last 16 bytes), so no register holds it while the poller waits for the phase input in stage[0..H).
constexpr int NW_OFF = STAGE - 64 * MAX_HN;
__device__ __forceinline__ void dma_norm_w(const float *w, int H, unsigned *stage) {
    const int lane = threadIdx.x & 63;
    for (int b = 0; b < H; b += 256) {
        const int e = min(b + lane * 4, H - 4);
        sdma16(w + e, (unsigned char *)(stage + NW_OFF + b));
    }
}

// fp32 x[0..H) (stage) -> S.a = fp16((x * rsqrt(mean(x^2) + eps)) * w), zeros up to kpad; w at stage[NW_OFF ..).
template <int FMT, int HD>
__device__ __forceinline__ void poll_norm(Smem<FMT, HD> &S, int H, int kpad, float eps) {
    const int lane = threadIdx.x & 63;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");          // the norm weight DMA has landed
    const float *x = (const float *)S.stage;
    const float *w = (const float *)(S.stage + NW_OFF);
    float ss = 0.f;
    for (int k = lane; k < H; k += 64) ss += x[k] * x[k];
    ss = wave_sum(ss);
    const float rs = 1.0f / sqrtf(ss / (float)H + eps);
    for (int k = lane; k < H; k += 64) S.a[k] = (f16)((x[k] * rs) * w[k]);
    for (int k = H + lane; k < kpad; k += 64) S.a[k] = (f16)0.f;
}

// Embedding row elements [k0, k1) of the token into dst (fp32).
template <int FMT>
__device__ __forceinline__ void embed_range(const Args &a, int token, int k0, int k1, float *dst) {
    for (int k = k0 + (int)(threadIdx.x & 63); k < k1; k += 64) dst[k - k0] = packed_elem<FMT>(a.emb_w, a.emb_sz, a.emb_nkt, token, k);
}

// ------------------------------------------------------------------------------------------------- the kernel
template <int FMT, int HD>
__global__ void __launch_bounds__(NT) k_decode(Args a) {
    __shared__ Smem<FMT, HD> S;
    using G_ = RingGeom<FMT>;
    constexpr int KT = TileGeom<FMT>::KT, HALF = HD / 2;
    const sp_token t = a.tok;
    const int lane = threadIdx.x & 63, wv = uni(threadIdx.x >> 6);
    const bool poller = wv == PW;
    const int L = a.L, H = a.H, NH = a.NH, NKV = a.NKV, I = a.I, V = a.V, Nqkv = a.Nqkv;
    const int G = NH / NKV;
    u64 *const ll = a.ll;
    unsigned *const err = a.err;
    const unsigned tag0 = a.tag0;
    const int nlin = t.ctx_hi - t.ctx_lo + 1;
    const int nch = (nlin + CH - 1) / CH;

    // ---- plan and pointer table into LDS
    {
        const int *src = (const int *)(a.plans + blockIdx.x);
        int *dst = (int *)&S.plan;
        for (int i = threadIdx.x; i < (int)(sizeof(Plan) / 4); i += NT) dst[i] = src[i];
        const u64 *ps = (const u64 *)a.lp;
        u64 *pd = (u64 *)S.lp;
        for (int i = threadIdx.x; i < (L + 1) * (int)(sizeof(LayerPtr) / 8); i += NT) pd[i] = ps[i];
    }
    bar();
    const int n_q = S.plan.n[0], n_o = S.plan.n[1], n_gu = S.plan.n[2], n_dn = S.plan.n[3];
    const int att = S.plan.att, cmb = S.plan.cmb, h0 = S.plan.h0, h1 = S.plan.h1;
    const int att_g = att >= 0 ? att / a.nch_max : 0, att_c = att >= 0 ? att - att_g * a.nch_max : 0;
    const bool att_live = att >= 0 && att_c < nch;

    Walk wk;
    wk.L = L; wk.w = wv;
#pragma unroll
    for (int p = 0; p < 6; ++p) wk.nkt[p] = a.nkt[p];
    wk.cnt[PH_KV] = att_live ? 1 : 0;
    wk.cnt[PH_QKV] = n_q; wk.cnt[PH_O] = n_o; wk.cnt[PH_GU] = n_gu; wk.cnt[PH_DN] = n_dn;
    wk.cnt[PH_HEAD] = h1 - h0;
    wk.h0 = h0;
    wk.kv_g = att_g; wk.kv_v0 = att_c * CH; wk.kv_cnt = min(CH, nlin - att_c * CH);
    Stream st;
    st.iss = Cursor{};
    st.iss.ph = PH_KV; st.iss.nkt = a.nkt[PH_KV]; st.iss.cnt = wk.cnt[PH_KV]; st.iss.rg = 1;
    st.cons_n = 0; st.cons_tiles = 0; st.att_done = -1; st.bad = false;
#ifdef SP_DECODE_TRACE
    st.tacc[0] = st.tacc[1] = st.tacc[2] = 0;
#endif
    if (!poller) {
        cur_settle(S, st.iss, wk);
        pump<FMT, HD>(S, a, wk, t, st);
    }
    bool ok = true;                       // every gather of this wave so far succeeded

    // Block barrier; every wave leaves together when the poller (or a worker) flagged a failure.
    int nvote = 0;
    auto bar_or = [&](bool pred) {
        const int p = nvote & 1;
        ++nvote;
        if (lane == 0) S.vote[p][wv] = pred ? 1 : 0;
        bar();
        int any = 0;
        for (int w = 0; w <= NWK; ++w) any |= S.vote[p][w];
        return any != 0;
    };
#define MK_SYNC_OR_LEAVE()                                                                                   \
    do {                                                                                                     \
        const bool bad_ = !ok || st.bad;                                                                     \
        if (bar_or(bad_)) {                                                                                  \
            if (st.bad && lane == 0) __hip_atomic_store(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); \
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                                                 \
            return;                                                                                          \
        }                                                                                                    \
    } while (0)

    for (int l = 0; l < L; ++l) {
        u64 *const R = ll + (size_t)l * a.stride;
        const u64 *const Rp = l > 0 ? ll + (size_t)(l - 1) * a.stride : nullptr;
        const unsigned tg = tag0 | (unsigned)(l * 8);
        const unsigned tgp = tag0 | (unsigned)((l - 1) * 8);
        LayerAux ax{};
        if (poller) ax = a.aux[l];
        MK_TRACE(l * 8 + 0);
        // ------------------------------------------------------------------ QKV
        if (n_q > 0) {
            if (poller) dma_norm_w(ax.in_norm, H, S.stage);
            if (l == 0) { if (poller) embed_range<FMT>(a, t.token, 0, H, (float *)S.stage); }
            else ok = ok && gather_blk(Rp + a.o_x, H, tgp | R_X, S.stage, err, wv);
            MK_SYNC_OR_LEAVE();
            MK_TRACE2(0);
            if (poller) poll_norm(S, H, a.nkt[PH_QKV] * KT, a.eps);
            bar();
            MK_TRACE2(1);
            float bias[MAXI];
            if (!poller) {
                if (att_live) consume<FMT, HD>(S, a, wk, t, st, wv < a.nkt[PH_KV] ? (a.nkt[PH_KV] - wv + NWK - 1) / NWK : 0);
                gemv_items<FMT, HD, 1>(S, a, wk, t, st, PH_QKV, n_q, S.red);
            } else {
#pragma unroll
                for (int i = 0; i < MAXI; ++i) {
                    const int row = (i < n_q ? S.plan.item[0][i] : 0) * 16 + (lane & 15);
                    bias[i] = i < n_q && row < Nqkv ? ax.qkv_b[row] : 0.f;
                }
            }
            bar();
            MK_TRACE2(2);
            if (poller && lane < 16) {
#pragma unroll
                for (int i = 0; i < MAXI; ++i) {
                    if (i < n_q) {
                        float v = 0.f;
                        for (int w = 0; w < NWK; ++w) v += S.red[(i * NWK + w) * 16 + lane];
                        const int row = S.plan.item[0][i] * 16 + lane;
                        if (row < Nqkv) ll_put(R + qkv_pos(row, NH, NKV, HD), tg | R_QKV, __float_as_uint(v + bias[i]));
                    }
                }
            }
        }
        MK_TRACE(l * 8 + 1);
        // ------------------------------------------------------------------ ATT
        if (att_live) {
            const int g = att_g, c = att_c;
            const int v0 = c * CH, cnt = min(CH, nlin - v0);
            const int jn = nlin - 1 - v0;                       // row of the new key in this chunk (if < cnt)
            if (!poller && n_q == 0)
                consume<FMT, HD>(S, a, wk, t, st, wv < a.nkt[PH_KV] ? (a.nkt[PH_KV] - wv + NWK - 1) / NWK : 0);
            // q rows of the group, then the key row, then the value row (one contiguous range)
            ok = ok && gather_blk(R + g * (G + 2) * HD, (G + 2) * HD, tg | R_QKV, S.stage, err, wv);
            MK_SYNC_OR_LEAVE();
            MK_TRACE2(3);
            if (poller) {
                const float *x = (const float *)S.stage;
                const float fpos = (float)t.pos;
                for (int i = lane; i < (G + 1) * HALF; i += 64) {
                    const int head = i / HALF, j = i - head * HALF;
                    const float ph = fpos * a.inv_freq[j];
                    const float cs = cosf(ph), sn = sinf(ph);
                    const float x1 = x[head * HD + j], x2 = x[head * HD + j + HALF];
                    const float o1 = __fadd_rn(__fmul_rn(x1, cs), __fmul_rn(-x2, sn));
                    const float o2 = __fadd_rn(__fmul_rn(x2, cs), __fmul_rn(x1, sn));
                    if (head < G) { S.qf[head][j] = o1 * a.scale; S.qf[head][j + HALF] = o2 * a.scale; }
                    else { S.kn[j] = (f16)o1; S.kn[j + HALF] = (f16)o2; }
                }
                for (int d = lane; d < HD; d += 64) S.vn[d] = (f16)x[(G + 1) * HD + d];
                if (jn >= 0 && jn < cnt) {
                    // the chunk holds the new position: patch its row; the owner also writes its cache slot
                    const size_t off = (((size_t)t.seq * NKV + g) * a.n_slots + t.slot) * HD;
                    for (int d = lane; d < HD; d += 64) {
                        S.kv[0][jn][d] = S.kn[d];
                        S.kv[1][jn][d] = S.vn[d];
                        ax.kc[off + d] = S.kn[d];
                        ax.vc[off + d] = S.vn[d];
                    }
                }
            }
            bar();
            if (!poller) {
                // scores: thread -> (key j, 1/8 of the dims); the 8 parts summed by a butterfly over 8 lanes
                constexpr int DP = HD / 8;
                const int tid = threadIdx.x, j = tid >> 3, part = tid & 7;
                float s[MAX_G];
#pragma unroll
                for (int h = 0; h < MAX_G; ++h) s[h] = 0.f;
#pragma unroll
                for (int d8 = 0; d8 < DP; d8 += 8) {
                    u32x4 kr = lds_ld128(&S.kv[0][j][part * DP + d8]);
                    lgkm_tie(kr);
                    const f16x8 kk = __builtin_bit_cast(f16x8, kr);
#pragma unroll
                    for (int h = 0; h < MAX_G; ++h) {
                        if (h < G) {
#pragma unroll
                            for (int e = 0; e < 8; ++e) s[h] += S.qf[h][part * DP + d8 + e] * (float)kk[e];
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < MAX_G; ++h) {
                    if (h < G) {
                        float v = s[h];
                        v += __shfl_xor(v, 1, SP_WAVE);
                        v += __shfl_xor(v, 2, SP_WAVE);
                        v += __shfl_xor(v, 4, SP_WAVE);
                        if (part == 0) S.sc[h][j] = j < cnt ? v : -INFINITY;
                    }
                }
            }
            bar();
            if (!poller && wv < G) {
                const int h = wv;
                const float v = S.sc[h][lane];
                const float m = wave_max(v);
                const float p = lane < cnt ? expf(v - m) : 0.f;
                const float lsum = wave_sum(p);
                S.sc[h][lane] = p;
                if (lane == 0) { S.mh[h] = m; S.lh[h] = lsum; }
            }
            bar();
            constexpr int NJR = NWK * 64 / HD, JPR = CH / NJR;   // key ranges of P.V and keys per range
            float *pv = (float *)S.stage;                        // [NJR][MAX_G][HD]
            if (!poller) {
                const int tid = threadIdx.x, d = tid % HD, jr = tid / HD;
                float o[MAX_G];
#pragma unroll
                for (int h = 0; h < MAX_G; ++h) o[h] = 0.f;
                uint32_t vb[JPR];
#pragma unroll
                for (int jj = 0; jj < JPR; ++jj) vb[jj] = lds_ldu16(&S.kv[1][jr * JPR + jj][d]);
#pragma unroll
                for (int jj = 0; jj < JPR; ++jj) lgkm_tie(vb[jj]);
#pragma unroll
                for (int jj = 0; jj < JPR; ++jj) {
                    const int j = jr * JPR + jj;
                    const float vv = (float)__builtin_bit_cast(f16, (uint16_t)vb[jj]);
#pragma unroll
                    for (int h = 0; h < MAX_G; ++h)
                        if (h < G) o[h] += S.sc[h][j] * vv;
                }
#pragma unroll
                for (int h = 0; h < MAX_G; ++h)
                    if (h < G) pv[(jr * MAX_G + h) * HD + d] = o[h];
            }
            bar();
            if (poller) {
                u64 *P = R + a.o_part;
                for (int h = 0; h < G; ++h) {
                    u64 *dst = P + ((size_t)(g * G + h) * a.nch_max + c) * (HD + 2);
                    for (int d = lane; d < HD; d += 64) {
                        float acc = 0.f;
                        for (int jr = 0; jr < NJR; ++jr) acc += pv[(jr * MAX_G + h) * HD + d];
                        ll_put(dst + 2 + d, tg | R_PART, __float_as_uint(acc));
                    }
                    if (lane == 0) {
                        ll_put(dst, tg | R_PART, __float_as_uint(S.mh[h]));
                        ll_put(dst + 1, tg | R_PART, __float_as_uint(S.lh[h]));
                    }
                }
            }
            bar();                                              // the partials in stage are read
            st.att_done = l;
            if (!poller) pump<FMT, HD>(S, a, wk, t, st);
        } else {
            st.att_done = l;
        }
        MK_TRACE(l * 8 + 2);
        // ------------------------------------------------------------------ CMB
        if (cmb >= 0) {
            const int h = cmb;
            ok = ok && gather_blk(R + a.o_part + (size_t)h * a.nch_max * (HD + 2), nch * (HD + 2), tg | R_PART, S.stage, err, wv);
            MK_SYNC_OR_LEAVE();
            if (poller) {
                const float *p = (const float *)S.stage;
                float M = -INFINITY;
                for (int cc = lane; cc < nch; cc += 64) M = fmaxf(M, p[cc * (HD + 2) + 1] > 0.f ? p[cc * (HD + 2)] : -INFINITY);
                M = wave_max(M);
                float Lsum = 0.f;
                float wc = 0.f;
                if (lane < nch) {
                    const float lc = p[lane * (HD + 2) + 1];
                    wc = lc > 0.f ? expf(p[lane * (HD + 2)] - M) : 0.f;
                    Lsum = wc * lc;
                }
                Lsum = wave_sum(Lsum);
                u64 *A = R + a.o_att + (size_t)h * HD;
                for (int d = lane; d < HD; d += 64) {
                    float acc = 0.f;
                    for (int cc = 0; cc < nch; ++cc) acc += __shfl(wc, cc, SP_WAVE) * p[cc * (HD + 2) + 2 + d];
                    ll_put(A + d, tg | R_ATT, __float_as_uint(acc / Lsum));
                }
            }
            bar();                                              // stage is free again
        }
        MK_TRACE(l * 8 + 3);
        // ------------------------------------------------------------------ O
        if (n_o > 0) {
            {
                // every wave gathers and converts its slice of the attention output; the poller adds the x rows
                const int K = NH * HD;
                ok = ok && gather_blk(R + a.o_att, K, tg | R_ATT, S.stage, err, wv);
                int w0, cnt;
                slice_of(K, wv, w0, cnt);
                const float *x = (const float *)S.stage;
                for (int k = w0 + lane; k < w0 + cnt && ok; k += 64) S.a[k] = (f16)x[k];
                if (poller) {
                    for (int k = K + lane; k < a.nkt[PH_O] * KT; k += 64) S.a[k] = (f16)0.f;
                    for (int i = 0; i < n_o && ok; ++i) {
                        const int row0 = S.plan.item[1][i] * 16;
                        if (l == 0) embed_range<FMT>(a, t.token, row0, min(row0 + 16, H), S.xr[0][i]);
                        else ok = gather(Rp + a.o_x + row0, min(16, H - row0), tgp | R_X, (unsigned *)S.xr[0][i], err);
                    }
                }
            }
            MK_SYNC_OR_LEAVE();
            MK_TRACE2(6);
            if (!poller) gemv_items<FMT, HD, 1>(S, a, wk, t, st, PH_O, n_o, S.red);
            bar();
            MK_TRACE2(7);
            if (poller && lane < 16) {
                for (int i = 0; i < n_o; ++i) {
                    float v = 0.f;
                    for (int w = 0; w < NWK; ++w) v += S.red[(i * NWK + w) * 16 + lane];
                    const int row = S.plan.item[1][i] * 16 + lane;
                    if (row < H) ll_put(R + a.o_xmid + row, tg | R_XMID, __float_as_uint(S.xr[0][i][lane] + v));
                }
            }
        }
        MK_TRACE(l * 8 + 4);
        // ------------------------------------------------------------------ GU
        if (n_gu > 0) {
            if (poller) dma_norm_w(ax.post_norm, H, S.stage);
            ok = ok && gather_blk(R + a.o_xmid, H, tg | R_XMID, S.stage, err, wv);
            MK_SYNC_OR_LEAVE();
            MK_TRACE2(8);
            if (poller) poll_norm(S, H, a.nkt[PH_GU] * KT, a.eps);
            bar();
            MK_TRACE2(9);
            if (!poller) gemv_items<FMT, HD, 2>(S, a, wk, t, st, PH_GU, n_gu, S.red);
            bar();
            MK_TRACE2(10);
            if (poller) {
                for (int i = 0; i < n_gu; ++i) {
                    float gs = 0.f, us = 0.f;
                    if (lane < 16) {
                        for (int w = 0; w < NWK; ++w) {
                            gs += S.red[((i * NWK + w) * 2 + 0) * 16 + lane];
                            us += S.red[((i * NWK + w) * 2 + 1) * 16 + lane];
                        }
                    }
                    const f16 v = (f16)(silu_f(gs) * us);
                    const unsigned bits = (unsigned)__builtin_bit_cast(uint16_t, v);
                    const unsigned hi = __shfl_down(bits, 1, SP_WAVE);
                    const int row = S.plan.item[2][i] * 16 + lane;
                    if (lane < 16 && (lane & 1) == 0 && row < I) ll_put(R + a.o_act + row / 2, tg | R_ACT, bits | (hi << 16));
                }
            }
        }
        MK_TRACE(l * 8 + 5);
        // ------------------------------------------------------------------ DN
        if (n_dn > 0) {
            ok = ok && gather_blk(R + a.o_act, I / 2, tg | R_ACT, (unsigned *)S.a, err, wv);
            if (poller) {
                for (int i = 0; i < n_dn && ok; ++i) {
                    const int row0 = S.plan.item[3][i] * 16;
                    ok = gather(R + a.o_xmid + row0, min(16, H - row0), tg | R_XMID, (unsigned *)S.xr[1][i], err);
                }
                for (int k = I + lane; k < a.nkt[PH_DN] * KT; k += 64) S.a[k] = (f16)0.f;
            }
            MK_SYNC_OR_LEAVE();
            MK_TRACE2(12);
            if (!poller) gemv_items<FMT, HD, 1>(S, a, wk, t, st, PH_DN, n_dn, S.red);
            bar();
            MK_TRACE2(13);
            if (poller && lane < 16) {
                for (int i = 0; i < n_dn; ++i) {
                    float v = 0.f;
                    for (int w = 0; w < NWK; ++w) v += S.red[(i * NWK + w) * 16 + lane];
                    const int row = S.plan.item[3][i] * 16 + lane;
                    if (row < H) ll_put(R + a.o_x + row, tg | R_X, __float_as_uint(S.xr[1][i][lane] + v));
                }
            }
        }
        MK_TRACE(l * 8 + 6);
    }

    // ---------------------------------------------------------------------- LM head + argmax
    const unsigned tga = tag0 | (unsigned)(L * 8 + R_AM);
    if (h1 > h0) {
        const u64 *Rl = ll + (size_t)(L - 1) * a.stride;
        const unsigned tgl = tag0 | (unsigned)((L - 1) * 8);
        if (poller) dma_norm_w(a.final_norm, H, S.stage);
        ok = ok && gather_blk(Rl + a.o_x, H, tgl | R_X, S.stage, err, wv);
        MK_SYNC_OR_LEAVE();
        if (poller) poll_norm(S, H, a.nkt[PH_HEAD] * KT, a.eps);
        bar();
        const int nbat = (h1 - h0 + MAXI - 1) / MAXI;
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        auto head_reduce = [&](int j) {
            const int b0 = h0 + j * MAXI, nb = min(MAXI, h1 - b0);
            const float *rb = S.red + (j & 1) * (MAXI * NWK * 16);
            if (lane < 16) {
                for (int i = 0; i < nb; ++i) {
                    float v = 0.f;
                    for (int w = 0; w < NWK; ++w) v += rb[(i * NWK + w) * 16 + lane];
                    const int row = (b0 + i) * 16 + lane;
                    if (row < V) {
                        if (a.logits) a.logits[row] = v;
                        argmax_merge(bv, bi, v, row);
                    }
                }
            }
        };
        for (int j = 0; j < nbat; ++j) {
            if (!poller) {
                const int b0 = h0 + j * MAXI, nb = min(MAXI, h1 - b0);
                gemv_items<FMT, HD, 1>(S, a, wk, t, st, PH_HEAD, nb, S.red + (j & 1) * (MAXI * NWK * 16));
            } else if (j > 0) {
                head_reduce(j - 1);
            }
            MK_SYNC_OR_LEAVE();
        }
        if (poller) {
            head_reduce(nbat - 1);
            wave_argmax(bv, bi);
            if (lane == 0) {
                ll_put(ll + a.o_am + 2 * blockIdx.x, tga, __float_as_uint(bv));
                ll_put(ll + a.o_am + 2 * blockIdx.x + 1, tga, (unsigned)bi);
            }
        }
    }
    MK_TRACE(L * 8 + 7 < 64 ? L * 8 + 7 : 63);
    if (blockIdx.x == 0 && poller && ok) {
        ok = gather(ll + a.o_am, 2 * a.nb_head, tga, S.stage, err);
        if (ok) {
            float v = -INFINITY;
            int idx = 0x7fffffff;
            for (int b = lane; b < a.nb_head; b += 64) argmax_merge(v, idx, __uint_as_float(S.stage[2 * b]), (int)S.stage[2 * b + 1]);
            wave_argmax(v, idx);
            if (lane == 0) *a.out_id = idx;
        }
    }
    if (!poller) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#ifdef SP_DECODE_TRACE
    if (lane == 0) for (int k = 0; k < 3; ++k) wtrace[blockIdx.x][wv][k] = st.tacc[k];
#endif
#undef MK_SYNC_OR_LEAVE
}

}  // namespace mk
