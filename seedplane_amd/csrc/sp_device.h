// Device-side building blocks shared by every kernel: vector types, exact code->fp16 unpacking, the gfx950
// 16x16x32 fp16 MFMA, wavefront reductions.  gfx950 only: wave64, MFMA, LDS.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define SP_WAVE 64

// ----------------------------------------------------------------------------------------------------------------
// Packed tile geometry (host packer in sp_pack.h writes exactly this; see the layout notes there).
//   Every format tiles a matrix into 16-row groups x KT columns; one tile is 1024 code bytes, one dwordx4 per lane.
//   Lane l of a wave owns row (l % 16) and k-subset g = l / 16 of the tile.
constexpr int TILE_ROWS = 16;
constexpr int TILE_BYTES = 1024;
template <int FMT> struct TileGeom;
// FMT values mirror SP_FMT_*: 1 = F16, 2 = Q8, 3 = Q4.
template <> struct TileGeom<1> { static constexpr int KT = 32;  static constexpr int STEPS = 1; static constexpr int SZ_BYTES = 0;   };
template <> struct TileGeom<2> { static constexpr int KT = 64;  static constexpr int STEPS = 2; static constexpr int SZ_BYTES = 64;  };
template <> struct TileGeom<3> { static constexpr int KT = 128; static constexpr int STEPS = 4; static constexpr int SZ_BYTES = 256; };

// ----------------------------------------------------------------------------------------------------------------
// Activation layouts (fp16 GEMV inputs).  Row-major: element (m, k) at m * ld + k.  Fragment-major, for steps of
// several columns padded to mtp tiles of 16: the 16 x 32 block (column tile mt, k-block kb) is one contiguous 1 KiB
// in the order of the MFMA A operand (lane g * 16 + r holds column 16 mt + r, k = 32 kb + 8 g .. + 7), so a wave
// reads a whole fragment with one fully coalesced dwordx4 load; blocks run k-block major:
//   (m, k) -> ((k / 32) * mtp + m / 16) * 512 + ((k / 8) % 4) * 128 + (m % 16) * 8 + k % 8.
__host__ __device__ __forceinline__ size_t act_off(int m, int k, int ld, int mtp) {
    return mtp ? ((size_t)(k >> 5) * mtp + (m >> 4)) * 512 + ((k >> 3) & 3) * 128 + (m & 15) * 8 + (k & 7)
               : (size_t)m * ld + k;
}

// ----------------------------------------------------------------------------------------------------------------
// Exact unpacking.  int8 code c (two's complement) -> fp16: the byte c^0x80 = c+128 is placed under the exponent
// byte 0x64, giving the fp16 value 1024 + c + 128 exactly; subtracting 1152 (exact in fp16) leaves c.
__device__ __forceinline__ f16x2 q8_pair(uint32_t u, uint32_t sel) {
    // u already xor-ed with 0x80808080; sel picks two bytes of u interleaved with 0x64.
    uint32_t h = __builtin_amdgcn_perm(0x64646464u, u, sel);
    return __builtin_bit_cast(f16x2, h) - (f16x2){(f16)1152.0f, (f16)1152.0f};
}
// 8 int8 codes (two dwords, k order) -> 8 fp16 in k order.
__device__ __forceinline__ f16x8 q8_unpack8(uint32_t d0, uint32_t d1) {
    d0 ^= 0x80808080u; d1 ^= 0x80808080u;
    f16x2 a = q8_pair(d0, 0x04010400u), b = q8_pair(d0, 0x04030402u);
    f16x2 c = q8_pair(d1, 0x04010400u), d = q8_pair(d1, 0x04030402u);
    return (f16x8){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
// The same codes offset by 1152 (1024 + 128): fp16 1152 + c, exact, without the subtraction.  A GEMV that takes these
// removes 1152 * sum(x) from the fp32 MFMA result instead (one correction per quant block, not per weight).
__device__ __forceinline__ f16x8 q8_biased8(uint32_t d0, uint32_t d1) {
    d0 ^= 0x80808080u; d1 ^= 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, d0, 0x04010400u), b = __builtin_amdgcn_perm(0x64646464u, d0, 0x04030402u);
    const uint32_t c = __builtin_amdgcn_perm(0x64646464u, d1, 0x04010400u), d = __builtin_amdgcn_perm(0x64646464u, d1, 0x04030402u);
    return __builtin_bit_cast(f16x8, (u32x4){a, b, c, d});
}
// 8 uint4 codes of one dword -> 8 fp16 1024 + c (exact; see q4_unpack8 for the nibble order).
__device__ __forceinline__ f16x8 q4_biased8(uint32_t v) {
    const uint32_t a = (v & 0x000F000Fu) | 0x64006400u, b = ((v >> 4) & 0x000F000Fu) | 0x64006400u;
    const uint32_t c = ((v >> 8) & 0x000F000Fu) | 0x64006400u, d = ((v >> 12) & 0x000F000Fu) | 0x64006400u;
    return __builtin_bit_cast(f16x8, (u32x4){a, b, c, d});
}
// 8 uint4 codes of one dword -> 8 fp16 in k order.  The packer stores k-order codes c0..c7 at nibble positions
// 0,4,1,5,2,6,3,7 so that (v >> 4j) & 0x000F000F yields the pair (c_{2j}, c_{2j+1}) in the two fp16 halves; OR-ing
// 0x6400 gives 1024 + c exactly, and subtracting 1024 leaves c.
__device__ __forceinline__ f16x2 q4_pair(uint32_t v, int j) {
    uint32_t h = ((v >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
    return __builtin_bit_cast(f16x2, h) - (f16x2){(f16)1024.0f, (f16)1024.0f};
}
__device__ __forceinline__ f16x8 q4_unpack8(uint32_t v) {
    f16x2 a = q4_pair(v, 0), b = q4_pair(v, 1), c = q4_pair(v, 2), d = q4_pair(v, 3);
    return (f16x8){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// D(16x16, fp32) += A(16x32 fp16) * B(32x16 fp16).  Lane l: A row (l%16) k-subset (l/16); B column (l%16)
// k-subset (l/16); D column (l%16), rows 4*(l/16) + r in register r.
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ----------------------------------------------------------------------------------------------------------------
// Wavefront reductions (wave64, butterfly over all lanes).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, SP_WAVE);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, SP_WAVE));
    return v;
}
// Reductions over the 16 lanes of a DPP row (lanes 16k .. 16k+15) on DPP moves instead of LDS-routed shuffles:
// pair with lane ^ 1, lane ^ 2 (quad permutes), then the mirror lane within 8 and within 16.  Every step combines
// two equal partial results of a pair in both orders, so all 16 lanes end with the same bits.
// (The identity element is returned where a source lane is disabled.)
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v, float identity) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// v is pinned as a register value first: otherwise a caller's product feeding v can fuse into the first DPP add
// (fma(x, x, neighbour's rounded x * x)), and the two lanes of a pair then hold different bits.
__device__ __forceinline__ float row16_sum(float v) {
    asm volatile("" : "+v"(v));
    v += dpp_mov<0xB1>(v, 0.f);      // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v, 0.f);      // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v, 0.f);     // row_half_mirror
    v += dpp_mov<0x140>(v, 0.f);     // row_mirror
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v, -INFINITY));
    v = fmaxf(v, dpp_mov<0x4E>(v, -INFINITY));
    v = fmaxf(v, dpp_mov<0x141>(v, -INFINITY));
    v = fmaxf(v, dpp_mov<0x140>(v, -INFINITY));
    return v;
}
// Whole-wave sum / max: the four row results combined in row order (uniform across the wave).
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = row16_sum(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = row16_max(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// (value, index) max with the smallest index winning ties.
__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}
__device__ __forceinline__ void wave_argmax(float &v, int &i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float v2 = __shfl_xor(v, o, SP_WAVE); int i2 = __shfl_xor(i, o, SP_WAVE);
        argmax_merge(v, i, v2, i2);
    }
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024); `red` holds >= 16 floats of LDS.
__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int j = 0; j < nw; ++j) t += red[j];
    return t;
}

// Block-wide sum on DPP wave reductions (same contract as block_sum).
__device__ __forceinline__ float block_sum_dpp(float v, float *red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum_dpp(v);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int j = 0; j < nw; ++j) t += red[j];
    return t;
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// An fp32 activation as the unevaluated sum of two fp16 values: hi = fp16(v), lo = fp16(v - hi).  v - hi is exact in
// fp32, so hi + lo holds about 22 significant bits where hi alone holds 11.  A GEMV that feeds both halves to the
// matrix cores (a second MFMA, or MFMA row 1 of a one-column product) sums x * w with fp32-class inputs while the
// operands stay fp16.  hi and lo must both come from v as rounded to fp32: otherwise the compiler may fold a caller's
// product into the conversion (v_fma_mix: the exact product rounded once to fp16) or into the subtraction (an FMA),
// and two kernels forming the same v could disagree in hi or lo.  The empty asm makes v an fp32 register value (it
// emits no instruction), and contraction is off for the subtraction.
__device__ __forceinline__ void split_f16(float v, f16 &hi, f16 &lo) {
#pragma clang fp contract(off)
    asm volatile("" : "+v"(v));
    hi = (f16)v;
    lo = (f16)(v - (float)hi);
}
