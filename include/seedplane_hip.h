/*
 * seedplane_hip.h - C ABI of the MI355X (gfx950) Qwen2 decode / speculative-verify library.
 *
 * The library is a plain C ABI over hand-written HIP kernels: no torch types cross it.  Pointers named *_dev are
 * device pointers (e.g. a torch tensor's data_ptr()); every other pointer is host memory owned by the caller.
 * Every entry point returns an int status (SP_OK == 0).  On failure, sp_engine_last_error() (engine calls) or
 * sp_last_error() (calls without an engine) returns a message that stays valid until the next failing call.
 *
 * Threading: one engine is driven by one host thread on one HIP stream; calls on one engine are not thread-safe,
 * matching the single-threaded reference engines (seedplane/qwen_engine.py:32, native/vulkan_decode/qwen_vk.cpp:92).
 *
 * Each declaration names the reference interface it replaces (paths relative to the reference repository).
 */
#ifndef SEEDPLANE_HIP_H
#define SEEDPLANE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status codes */
enum {
    SP_OK = 0,
    SP_EINVAL = 1,      /* bad argument (maps to ValueError in Python)          */
    SP_ENOMEM = 2,      /* device allocation failed                              */
    SP_EHIP = 3,        /* a HIP runtime call failed (maps to RuntimeError)      */
    SP_ESTATE = 4,      /* call out of order, e.g. forward before weights loaded */
    SP_ECAPACITY = 5    /* KV slots / token count exceeded (ValueError)          */
};

/* ---------------------------------------------------------------- weight formats (canonical host layouts)
 * SP_FMT_F16: fp16 row-major [rows][cols].
 * SP_FMT_Q8 : int8 codes row-major [rows][cols] + fp16 scales [rows][cols/32]; w = code * scale (blocks of 32
 *             along K, symmetric).
 * SP_FMT_Q4 : uint8 packed codes [rows][cols/2] (byte j: k=2j in the low nibble, k=2j+1 in the high nibble,
 *             codes 0..15) + fp16 scales [rows][cols/32] + fp16 zeros [rows][cols/32];
 *             w = (code - zero) * scale (groups of 32 along K).
 * SP_FMT_F32: fp32 row-major; accepted for norms and biases only. */
enum { SP_FMT_F32 = 0, SP_FMT_F16 = 1, SP_FMT_Q8 = 2, SP_FMT_Q4 = 3 };

/* ---------------------------------------------------------------- tensor kinds for sp_engine_load
 * The fused matrices follow the reference's inference packing (seedplane/qwen_engine.py:64-80):
 * QKV = cat(q_proj, k_proj, v_proj) rows, QKV_BIAS = cat of the biases, GATE_UP = cat(gate_proj, up_proj) rows. */
enum {
    SP_T_EMBED = 0,       /* [vocab][hidden]                                     */
    SP_T_HEAD = 1,        /* [vocab][hidden]; omit when the head is tied         */
    SP_T_FINAL_NORM = 2,  /* fp32 [hidden]                                       */
    SP_T_IN_NORM = 3,     /* fp32 [hidden], per layer                            */
    SP_T_POST_NORM = 4,   /* fp32 [hidden], per layer                            */
    SP_T_QKV = 5,         /* [(heads + 2*kv_heads)*head_dim][hidden], per layer  */
    SP_T_QKV_BIAS = 6,    /* fp32 [(heads + 2*kv_heads)*head_dim], per layer     */
    SP_T_O = 7,           /* [hidden][heads*head_dim], per layer                 */
    SP_T_GATE_UP = 8,     /* [2*intermediate][hidden], per layer                 */
    SP_T_DOWN = 9         /* [hidden][intermediate], per layer                   */
};

/* ---------------------------------------------------------------- forward flags */
enum {
    SP_F_LOGITS = 1,      /* run the final norm + LM head and produce fp32 logits for every column   */
    SP_F_ARGMAX = 2,      /* also produce the greedy id per column (first index on ties)             */
    SP_F_GRAPH = 4,       /* record the step as graphs once; replayed when the caller waits per step */
    SP_F_PERSISTENT = 8,  /* accepted for compatibility: one plain decode column runs the persistent  */
                          /* step by default wherever sp_engine_persistent_status says it applies    */
    SP_F_UNFUSED = 16,    /* one column: run every RMSNorm and attention combine as a kernel of its   */
                          /* own instead of inside the next GEMV (same results; for checking)        */
    SP_F_FEED = 32,       /* column b's token is the argmax id of column b of the last SP_F_ARGMAX   */
                          /* call (on the device; the token field is ignored), so a greedy loop     */
                          /* needs no host round trip per step                                       */
    SP_F_CHAIN = 64,      /* run the kernel chain even where the persistent one-column step applies  */
    SP_F_DEVCOLS = 128    /* column b's token (and tree mask) come from the device arrays set by      */
                          /* sp_engine_set_device_columns, read when the step runs (always the chain) */
};

typedef struct sp_model_desc {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab;
    int32_t weight_format;   /* SP_FMT_F16 / SP_FMT_Q8 / SP_FMT_Q4 for every projection, embed and head      */
    int32_t tied_head;       /* 1: the LM head is the embedding matrix (seedplane/qwen_engine.py:142)        */
    int32_t max_tokens;      /* most columns (batch rows + tree nodes) one sp_engine_forward call may carry  */
    float rms_eps;
    float reserved0;
    const float *inv_freq;   /* head_dim/2 RoPE inverse frequencies, fp32, computed as qwen_engine.py:52     */
} sp_model_desc;

/* One column of a forward call: a token, the KV cache (sequence) it belongs to and what it attends to.
 * Visible keys = ring positions [ctx_lo, ctx_hi] (slot = position mod n_slots) followed by the tree block:
 * slots (tree_base + j) mod n_slots for j < tree_count whose bit j is set in tree_mask.  The token's own K/V is
 * written to `slot` before attention, so a plain decode column has ctx_hi == pos and slot == pos mod n_slots.
 * This is the (slot range, positions) contract of the reference attention (native/vulkan_decode/shaders/
 * attn_part.comp:18, rope_kv.comp:16,25) generalised with an ancestor mask for tree verification. */
typedef struct sp_token {
    int32_t token;
    int32_t seq;
    int32_t pos;          /* RoPE position (qwen_engine.py:99-103, 115)  */
    int32_t slot;         /* KV slot this column writes                  */
    int32_t ctx_lo, ctx_hi;
    int32_t tree_base, tree_count;
    uint64_t tree_mask;
} sp_token;

typedef struct sp_engine sp_engine;

/* Replaces Qwen2Engine.__init__ (seedplane/qwen_engine.py:35-63) and Engine::init's shape checks
 * (native/vulkan_decode/qwen_vk.cpp:283-308).  Shapes are general: any head_dim in {64, 128}, hidden and
 * intermediate multiples of 128, any vocab. */
int sp_engine_create(const sp_model_desc *desc, sp_engine **out);
void sp_engine_destroy(sp_engine *e);
const char *sp_engine_last_error(const sp_engine *e);
/* Last error of a call that has no engine (create, sp_op_*), per host thread. */
const char *sp_last_error(void);

/* Use `hip_stream` (a hipStream_t, e.g. torch.cuda.current_stream().cuda_stream) for every later call. */
int sp_engine_set_stream(sp_engine *e, void *hip_stream);

/* Replaces the weight upload of Engine::init (qwen_vk.cpp:311-322) and the fused packing of Qwen2Engine.__init__
 * (qwen_engine.py:64-80).  Host buffers in the canonical layout of `fmt`; the library re-tiles them for the
 * kernels and copies them to HBM.  `layer` is ignored for the global kinds. */
int sp_engine_load(sp_engine *e, int32_t kind, int32_t layer, int32_t fmt, int32_t rows, int32_t cols,
                   const void *data, const void *scales, const void *zeros);

/* Replaces KVCache.allocate / Qwen2Engine.new_cache (qwen_engine.py:25-29, 82-85) and the window buffers of
 * Engine::init (qwen_vk.cpp:314-316).  Allocates fp16 K and V for `n_seq` sequences x `n_slots` ring slots for
 * every layer (layout [layer][seq][kv_head][slot][head_dim]).  Re-reserving frees the previous cache. */
int sp_engine_kv_reserve(sp_engine *e, int32_t n_seq, int32_t n_slots);

/* Read access to the cache tensors (reference: KVCache.keys / KVCache.values, seedplane/qwen_engine.py:18-29, which
 * are per-layer tensors).  k_dev / v_dev receive layer `layer`'s K and V pool: fp16 [n_seq][n_kv_heads][n_slots]
 * [head_dim] (sp_engine_kv_reserve's sizes), position p of sequence s at slot p mod n_slots.  The pointers stay
 * valid until the pool is reserved or grown again, or the engine is destroyed. */
int sp_engine_kv_layer(sp_engine *e, int32_t layer, void **k_dev, void **v_dev);

/* Replaces the independence of the reference's per-cache tensors (Qwen2Engine.new_cache allocates a fresh KVCache
 * per call and never touches the others, qwen_engine.py:82-85): grows the pool to n_seq x n_slots (neither smaller
 * than now) while keeping the live sequences.  For kept sequence keep_seq[i] of length keep_len[i], positions
 * [max(0, len - old n_slots), len) move from slot p mod old n_slots to slot p mod n_slots, in every layer; other
 * sequences start empty.  On failure the old pool is untouched.  Synchronous. */
int sp_engine_kv_grow(sp_engine *e, int32_t n_seq, int32_t n_slots, int32_t n_keep, const int32_t *keep_seq,
                      const int32_t *keep_len);

/* Replaces Qwen2Engine.forward (qwen_engine.py:105-144) and the recorded one-token / K/V-batch command buffers
 * (qwen_vk.cpp:374-437).  Runs `n` columns (any mix of sequences) through every layer.  Without SP_F_LOGITS the
 * call is K/V-only: the last layer stops after writing its K/V (qwen_vk.cpp:426).  logits_dev, when not NULL,
 * receives fp32 [n][vocab]; argmax_host, when not NULL (requires SP_F_ARGMAX), receives the greedy ids and the call
 * waits for the stream. */
int sp_engine_forward(sp_engine *e, int32_t n, const sp_token *toks, int32_t flags, float *logits_dev,
                      int32_t *argmax_host);

/* Introspection (no counterpart in the reference): which implementation ran the last sp_engine_forward call:
 * 0 = the kernel chain, 1 = the persistent one-column step (one kernel launch for every layer, then the head
 * GEMV and the argmax), -1 = none yet. */
int sp_engine_last_path(const sp_engine *e);

/* Device-side columns (no counterpart in the reference, whose speculative forest is built from host token lists,
 * seedplane/speculative.py:19-38; the drafter uses it to run its levels without reading tokens back).  For calls
 * with SP_F_DEVCOLS: tokens_dev[b]
 * replaces column b's token (clamped to [0, vocab)) and, when masks_dev is not NULL, masks_dev[b] its tree_mask; the
 * arrays are read on the engine's stream when the step runs, so a kernel queued before the call may write them.
 * The host records still give every other field (positions, slots, ranges, tree block).  Pointers stay set until the
 * next call of this function; tokens_dev NULL clears them. */
int sp_engine_set_device_columns(sp_engine *e, const int32_t *tokens_dev, const uint64_t *masks_dev);

/* Introspection (no counterpart in the reference; the reference records its whole one-token step once and submits
 * it once per token, native/vulkan_decode/qwen_vk.cpp:372-412): 1 when a plain decode column (one column, no tree
 * block, writing the slot of its newest visible position) runs the persistent step on this engine's weights and KV
 * pool, 0 when it runs the kernel chain -- `why` (why_len bytes, may be NULL) then receives the reason -- and -1 on
 * an error.  Prepares the step's buffers on the first call after a weight load or pool change. */
int sp_engine_persistent_status(sp_engine *e, char *why, int32_t why_len);

/* Host function, no GPU call (no counterpart in the reference): the persistent step's work split for a model shape
 * on n_blocks blocks (one per CU) and n_slots KV slots, after the bounds walk that precedes every launch (every
 * item's block, tagged words, weight tiles and staged counts).  info receives 12 values: qkv tiles, attention chunks,
 * combiners, o_proj tiles, gate_up units, down items, gate_up units of the busiest block, first attention block,
 * first o_proj block, first down block, tagged words, LDS bytes per block.  SP_EINVAL (with sp_last_error) when the
 * step does not apply. */
int sp_persistent_geometry(const sp_model_desc *desc, int32_t n_slots, int32_t n_blocks, int32_t *info);

/* Introspection (no counterpart in the reference; its decode report counts dispatches per token,
 * native/vulkan_decode/qwen_vk.cpp:866-870): kernels launched by the last sp_engine_forward call with SP_F_GRAPH
 * (the kernel nodes of its recorded step), -1 after a call without it. */
int sp_engine_last_dispatches(const sp_engine *e);

/* Host function, no GPU call (no counterpart in the reference: its verification is a linear batch whose positions
 * the engine derives from the cache length, qwen_engine.py:99-103): fills the n columns of one tree pass over a
 * cache of `length` positions.
 * Node i (parents before children, depth[i] = its distance from the root, mask[i] = bit j set for every ancestor j
 * and for i itself) gets pos = length + depth[i], slot = (length + i) mod n_slots, ctx = [max(0, pos - window + 1)
 * (0 when window == 0, full attention), length - 1], tree_base = length mod n_slots, tree_count = n, and its token
 * and mask.  n in [1, 64]; SP_EINVAL for NULL arrays or out-of-range sizes. */
int sp_tree_columns(int32_t n, const int32_t *token, const int32_t *depth, const uint64_t *mask, int32_t seq,
                    int64_t length, int32_t n_slots, int32_t window, sp_token *out);

/* Device pointer to the engine's fp32 logits buffer [max_tokens][vocab] holding the last SP_F_LOGITS call. */
int sp_engine_logits(sp_engine *e, float **logits_dev);

/* Replaces the KV rollback by `cache.length = ...` (experiments/hive_scaling/benchmark_speculative.py:119,127) and
 * the slot copies of copy_slots (qwen_vk.cpp:441-451): for every layer copies K/V of slot src[i] to dst[i] of
 * sequence `seq`, in order i = 0..n-1 (tree compaction after acceptance). */
int sp_engine_kv_move(sp_engine *e, int32_t seq, int32_t n, const int32_t *src_slots, const int32_t *dst_slots);

/* Replaces the per-token host read of the greedy id in Qwen2Engine.generate (qwen_engine.py:158-166): enqueue a copy of
 * the last SP_F_ARGMAX call's ids (n <= its column count) to host memory on the engine's stream and return without
 * waiting; `host` holds them after the stream synchronises (sp_engine_sync).  Pinned host memory keeps the copy
 * asynchronous. */
int sp_engine_copy_ids(sp_engine *e, int32_t n, int32_t *host);

/* Wait for all work queued by the engine. */
int sp_engine_sync(sp_engine *e);

/* Measurement hook (no counterpart in the reference): launch the engine's own GEMV for matrix `kind` of `layer`
 * (same packing, split and epilogue as the decode step) `iters` times over n_cols columns on the engine's stream,
 * timed with HIP events.  layer -1 (per-layer kinds) cycles launch i through layer i mod n_layers, so the weights
 * stream from HBM as in a decode step.  Returns the average launch duration in microseconds and the packed bytes one
 * launch reads.  Clobbers the activation buffers (not the KV cache); call between forward passes only. */
int sp_engine_time_gemv(sp_engine *e, int32_t kind, int32_t layer, int32_t n_cols, int32_t iters, float *avg_us,
                        uint64_t *bytes);

/* Measurement hook (no counterpart in the reference): launch the attention kernel that a forward call over these n
 * columns would run (RoPE not fused; q = 0), `iters` times on the engine's stream cycling through the layers, timed
 * with HIP events.  Returns the average launch duration in microseconds and the K/V bytes one launch reads (each
 * visible key's fp16 K and V once per kv head; once per group for multi-query groups).  Clobbers the activation
 * buffers (not the KV cache); call between forward passes only. */
int sp_engine_time_attention(sp_engine *e, int32_t n, const sp_token *toks, int32_t iters, float *avg_us,
                             uint64_t *bytes);

/* Measurement hook (no counterpart in the reference): launch the persistent one-column step's kernel (every layer of
 * one decode column; no head GEMV, no argmax) for column *tok `iters` times on the engine's stream, timed with HIP
 * events.  Returns the average launch duration in microseconds and the algorithmic bytes one launch reads: every
 * layer's packed weights and scales, norm weights and qkv bias, the visible keys' K and V, the embedding row.  The
 * column must be a plain decode column where the step applies (SP_ESTATE otherwise); its K/V slot is rewritten with
 * the same values each time.  Clobbers the activation buffers; call between forward passes only. */
int sp_engine_time_persistent(sp_engine *e, const sp_token *tok, int32_t iters, float *avg_us, uint64_t *bytes);

/* Benchmark utility (no counterpart in the reference): fill slots [first_slot, first_slot + n) of sequence `seq`
 * in every layer's K and V with seeded pseudo-random fp16 values in [-scale, scale], standing in for a long prefill
 * when only the decode step is measured (the step reads the same bytes whatever the values). */
int sp_engine_kv_fill(sp_engine *e, int32_t seq, int32_t first_slot, int32_t n, uint64_t seed, float scale);

/* Bytes of HBM the engine holds for weights / KV (for roofline accounting). */
int sp_engine_bytes(const sp_engine *e, uint64_t *weight_bytes, uint64_t *kv_bytes);

/* ---------------------------------------------------------------- standalone operators */

/* Replaces the greedy branch of Qwen2Engine.sample (qwen_engine.py:147-148) and argmax.comp: two-pass
 * wavefront argmax over each row of logits_dev [rows][cols] (fp32), first index on ties, into out_dev (int32).
 * workspace_dev must hold sp_op_argmax_workspace(rows, cols) bytes. */
size_t sp_op_argmax_workspace(int32_t rows, int32_t cols);
int sp_op_argmax(const float *logits_dev, int32_t rows, int32_t cols, int32_t *out_dev, void *workspace_dev,
                 void *hip_stream);

/* No counterpart in the reference.  sp_op_argmax for callers that cannot allocate (code under HIP graph capture,
 * serving loops that forbid allocation): the same kernels and ids, with the partials in a device array of the
 * library's own (256 KiB per GPU, held until the process ends) instead of a workspace.  No hipMalloc / hipFree or
 * other allocating call is made.  rows <= 512 (SP_EINVAL beyond).  Every call on one GPU shares that array: calls that
 * overlap on one GPU (on different streams, or from different host threads without ordering) race. */
int sp_op_argmax_noalloc(const float *logits_dev, int32_t rows, int32_t cols, int32_t *out_dev, void *hip_stream);

/* A packed projection matrix in HBM, for kernel-level tests and roofline measurement of the GEMV alone.
 * Replaces the per-matrix path of F.linear (qwen_engine.py:121,136,138-139,143) and gemv.comp. */
typedef struct sp_weight sp_weight;
int sp_weight_create(int32_t fmt, int32_t rows, int32_t cols, const void *data, const void *scales,
                     const void *zeros, sp_weight **out);
void sp_weight_destroy(sp_weight *w);
/* HBM bytes of the packed codes + scales + zeros. */
uint64_t sp_weight_bytes(const sp_weight *w);
/* Host-only: the tiled layout sp_weight_create uploads, written into caller buffers (for inspection and for
 * callers that cache packed weights).  With out_codes/out_side NULL only the sizes are returned.  pair_halves
 * selects the SwiGLU row-group interleave used for SP_T_GATE_UP. */
int sp_pack_matrix(int32_t fmt, int32_t rows, int32_t cols, const void *data, const void *scales, const void *zeros,
                   int32_t pair_halves, void *out_codes, uint64_t *codes_bytes, void *out_side, uint64_t *side_bytes);
/* y_dev[m][r] = sum_k W[r][k] * x_dev[m][k] for m < m_cols (x fp16 [m_cols][cols], y fp32 [m_cols][rows]).
 * The kernel needs no scratch: sp_op_gemv_workspace returns 0 and workspace_dev may be NULL (kept so callers
 * need not change if a later kernel needs one). */
size_t sp_op_gemv_workspace(const sp_weight *w, int32_t m_cols);
int sp_op_gemv(const sp_weight *w, const void *x_dev, int32_t m_cols, float *y_dev, void *workspace_dev,
               void *hip_stream);

/* ---------------------------------------------------------------- seeded sampling and speculative acceptance
 * Distributions are softmax(logits / temperature) of fp32 rows, evaluated in float64 with a fixed summation order
 * (rows cut into 1024 contiguous chunks, each summed in index order, chunk sums added in chunk order), so a CPU
 * restatement reproduces every draw and decision from the same logits and uniforms. */

/* Replaces the T > 0 branch of Qwen2Engine.sample (qwen_engine.py:149-156, torch.multinomial) and the native
 * Sampler::draw inverse CDF (native/vulkan_decode/sampler.hpp:93-97) with seeded uniforms: out_dev[s] = the first
 * index whose cumulative softmax mass of row row_dev[s] exceeds u_dev[s] * total.  All pointers are device memory.
 * Each draw runs on many blocks through a per-device scratch area: calls on one device must not overlap. */
int sp_op_sample(const float *logits_dev, int32_t vocab, int32_t ld, const int32_t *row_dev, const double *u_dev,
                 int32_t n, double temperature, int32_t *out_dev, void *hip_stream);

/* Replaces Qwen2Engine.sample with top_k / top_p (qwen_engine.py:149-156) and the native Sampler::distribution +
 * draw (native/vulkan_decode/sampler.hpp:22-57, 93-97) on the GPU: z = fp32(logits / T); top_k > 0 (and < vocab)
 * keeps z >= the k-th largest z (ties kept); top_p < 1 keeps the prefix of the z-descending order (ties by index)
 * whose exclusive cumulative mass is <= top_p of the kept mass; out_dev[s] = the inverse-CDF draw over what is kept
 * with uniform u_dev[s] (masses are 64-bit fixed point, exp(z - z_max) * 2^40, so every sum is exact).  Each draw
 * runs over many blocks (a short launch per radix level) with a histogram scratch the library keeps per device: calls
 * on one device must not overlap.  All pointers are device memory.  Errors: NULL pointers, bad sizes,
 * temperature <= 0, top_p <= 0. */
int sp_op_sample_filtered(const float *logits_dev, int32_t vocab, int32_t ld, const int32_t *row_dev,
                          const double *u_dev, int32_t n, double temperature, int32_t top_k, double top_p,
                          int32_t *out_dev, void *hip_stream);

/* No counterpart in the reference, whose verifier is greedy only (seedplane/speculative.py:55-92; README.md:69):
 * speculative acceptance over a draft tree with residual resampling.  Node 0 is the root (the last committed
 * token).  The trials of node i are trials_dev[trial_start[i] .. trial_start[i] + n_trials[i]): the child each
 * draft branch through node i drew, in branch (draw) order, repeats kept.  p_logits_dev: target logits per node;
 * q_logits_dev: drafter logits per node (read for nodes with trials).  A trial of child x is accepted iff
 * u < p(x) / q(x); a rejection replaces p by norm(max(p - q, 0)); with every trial rejected the final token is drawn
 * from that residual, after an accepted leaf (or max_depth levels) a bonus token is drawn from the target.
 * Uniforms u_dev[0..n_u) are consumed in that order.  out_dev (int32, max_depth + 4 entries): [0] accepted count k,
 * [1..k] accepted node ids, [max_depth+1] final token, [max_depth+2] uniforms used, [max_depth+3] 1 for a bonus
 * draw.  resid_dev is unused (kept for callers of the first signature; may be NULL).  token/trial_start/n_trials
 * are device int32 [n_nodes].  The residual after j rejections is evaluated as max(p - c_j q, 0) / S_j with c_1 = 1,
 * c_{j+1} = c_j + S_j (the same distribution as renormalising max(p - q, 0) after each rejection).  Float64 sums
 * use 64 x 256 contiguous chunks: sequential inside a chunk, over the 256 chunk sums of each group of 256, then
 * over the 64 group sums.  Synchronous: returns after the walk has finished (it polls completion tags the kernel
 * writes to pinned host memory, so later work on the stream may still be queued), SP_EHIP if its cross-block
 * exchange timed out.  out_host (may be NULL): host copy of out_dev, written by the kernel itself. */
int sp_op_accept_tree(const float *p_logits_dev, const float *q_logits_dev, int32_t vocab, int32_t ld, int32_t n_nodes,
                      const int32_t *token_dev, const int32_t *trial_start_dev, const int32_t *n_trials_dev,
                      const int32_t *trials_dev, int32_t n_trials_total, const double *u_dev, int32_t n_u,
                      double temperature, int32_t max_depth, double *resid_dev, int32_t *out_dev, void *hip_stream,
                      int32_t *out_host);

/* sp_op_accept_tree with the tree arrays and the uniforms in ordinary host memory (the same reference interface and
 * decision rule): token / trial_start / n_trials [n_nodes], trials [n_trials_total] and u [n_u] are copied by the CPU
 * into a pinned block the library keeps per device, which the kernel reads directly (no copy on the stream, so the
 * walk starts as soon as the stream reaches it).  Before refilling that block the call waits for the previous walk
 * that read it; calls on one device must not overlap.  Same limits, outputs and errors as sp_op_accept_tree. */
int sp_op_accept_tree_host(const float *p_logits_dev, const float *q_logits_dev, int32_t vocab, int32_t ld,
                           int32_t n_nodes, const int32_t *token, const int32_t *trial_start, const int32_t *n_trials,
                           const int32_t *trials, int32_t n_trials_total, const double *u, int32_t n_u,
                           double temperature, int32_t max_depth, int32_t *out_dev, void *hip_stream, int32_t *out_host);

/* sp_op_accept_tree_host with the drafter's rows given by index (no counterpart in the reference; it replaces a
 * gather of the drafter rows into node order): node i's drafter logits are row q_row[i] (host array [n_nodes], each
 * < n_q_rows for a node with trials; leaves' entries are not read) of q_logits_dev [n_q_rows][ld].  Same decision
 * rule, limits, outputs and errors. */
int sp_op_accept_tree_rows(const float *p_logits_dev, const float *q_logits_dev, int32_t n_q_rows, int32_t vocab,
                           int32_t ld, int32_t n_nodes, const int32_t *token, const int32_t *trial_start,
                           const int32_t *n_trials, const int32_t *trials, int32_t n_trials_total,
                           const int32_t *q_row, const double *u, int32_t n_u, double temperature, int32_t max_depth,
                           int32_t *out_dev, void *hip_stream, int32_t *out_host);

/* Library teardown (no counterpart in the reference): frees what the sampling and acceptance entry points keep per
 * device (draw and histogram scratch, the walk's exchange words, its pinned result and staging blocks and their
 * event) after waiting for each such device's work; a later call of those entry points creates them again.  Engines
 * are not touched (sp_engine_destroy frees an engine).  The Python layer calls it at interpreter exit, after the
 * engines' own finalizers, so no HIP object of the library is left for the HIP runtime's own teardown.  Must not
 * overlap a call of the entry points it serves. */
int sp_library_release(void);

/* One level of a drafter's proposal on the device (no counterpart in the reference; with SP_F_DEVCOLS it lets a
 * drafter run its levels without reading tokens back).  tokens_dev [levels][n_branches]: the tokens drawn so far,
 * level-major.  For `level`, canon_dev[level][b] = the first branch whose tokens at levels 0..level equal branch b's
 * (the branch whose row every branch through that tree node draws from); masks_dev[b] = the tree mask of column b of
 * that level (bit l' * n_branches + canon_dev[l'][b] for every earlier level l', and bit level * n_branches + b);
 * rows_dev[b] = canon_dev[level][b].  canon_dev rows of earlier levels must hold this function's earlier results.
 * Requires n_branches * (level + 1) <= 64.  All pointers are device memory; one small launch on hip_stream. */
int sp_op_draft_link(const int32_t *tokens_dev, int32_t n_branches, int32_t level, int32_t *canon_dev,
                     uint64_t *masks_dev, int32_t *rows_dev, void *hip_stream);

#ifdef __cplusplus
}
#endif
#endif /* SEEDPLANE_HIP_H */
