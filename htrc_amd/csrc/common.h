// Shared device helpers for the flat-HTRC HIP kernels (gfx950 / CDNA4 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace htrc {

constexpr int D = 128;      // head dimension the kernels are specialised for
constexpr int TILE = 64;    // query rows per tile (one expansion centre)
constexpr int WAVE = 64;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));

// fp32(1/127) = 0x3C010204, the per-row int8 scale factor.
__device__ constexpr float R127 = 1.0f / 127.0f;
__device__ constexpr float R448 = 1.0f / 448.0f;   // e4m3 state scales (h3/htrc_flat_triton.py:67-68)
__device__ constexpr float LOG2E = 1.4426950408889634f;
__device__ constexpr float LN2 = 0.6931471805599453f;

constexpr uint32_t NXCD = 8;   // MI355X: 8 accelerator dies, each with its own L2

// Workgroups of a 1-D grid of n are dispatched round-robin over the XCDs (workgroup i runs on
// XCD i % 8).  This maps i to the logical block x * q + min(x, r) + i / 8 (q = n / 8,
// r = n % 8): a bijection of [0, n) under which every XCD walks one contiguous range of
// logical blocks, so neighbouring blocks (the same head, adjacent tiles) share one L2.
__device__ __forceinline__ uint32_t xcd_block(uint32_t i, uint32_t n) {
    const uint32_t x = i % NXCD, q = n / NXCD, r = n % NXCD;
    return x * q + (x < r ? x : r) + i / NXCD;
}

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even (quiet NaN kept).
__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// where(x >= 0, x + 0.5, x - 0.5) in fp32, then truncation toward zero: the same fp32 sum
// as x + copysign(0.5, x) (for x = -0 both truncate to 0), and v_cvt_i32_f32 truncates.
__device__ __forceinline__ int round_away(float x) { return (int)__fadd_rn(x, copysignf(0.5f, x)); }

// Four int8 values (given as int32 in [-128, 127]) packed little-endian into a dword.
__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) | ((uint32_t)d << 24);
}

// rint (half to even) clamped to +-127.
__device__ __forceinline__ int round_even_clamp(float x) {
    float y = rintf(x);
    y = y > 127.0f ? 127.0f : y;
    y = y < -127.0f ? -127.0f : y;
    return (int)y;
}

// x / s rounded to nearest from y = x / s's correctly rounded reciprocal y = RN(1 / s):
// q = x y, r = x - q s (exact, one FMA), q + r y (Markstein's correction).  For |x| <= 127 s
// (row quantisation: s = max|x| / 127) it equals the IEEE quotient whenever |x / s| >= 0.25,
// and below that both round to the integer 0 (checked for every bf16 x against every bf16
// row maximum and on 3.5e8 random fp32 pairs); three VALU operations instead of ten.
__device__ __forceinline__ float div_by(float x, float s, float y) {
    const float q = __fmul_rn(x, y);
    return __fmaf_rn(__fmaf_rn(-q, s, x), y, q);
}

__device__ __forceinline__ float row_scale(float amax, float floor_) {
    float s = __fmul_rn(amax, R127);
    return s < floor_ ? floor_ : s;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// Reductions across the four 16-lane groups that share a column of an MFMA C tile, with the
// gfx950 lane swaps: with both operands equal, the two results of v_permlane{16,32}_swap hold
// {v[i], v[i ^ 16]} (resp. {v[i], v[i ^ 32]}) in each lane, so one max / add reduces a pair.
// Maximum of two values that are never NaN: one v_max_f32 (fmaxf on the swapped words would
// first quiet each operand with a v_max_f32 of its own).
__device__ __forceinline__ float max_nonan(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return max_nonan(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return max_nonan(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float grp_max(float v) { return xor32_max(xor16_max(v)); }

// Orders one wave's LDS writes before its lanes' later reads of them (and reads before later
// writes): a lane reading what another lane of its wave wrote is a cross-thread access, which
// the compiler may otherwise move across the writes.  Wave scope, no workgroup barrier.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ln z for z >= 1 (a partition sum whose largest term is exp(0) = 1): log2 z by v_log_f32 (no
// subnormal input to rescale, no infinity to pass through), times ln 2 as hi + lo with hi = ln 2
// truncated to 24 bits (0x3f317217) and lo = fp32(ln 2 - hi) (0x3377d1cf), the product y hi
// carried exactly by an FMA: log2 z ln 2 to within about an ulp.
__device__ __forceinline__ float ln_ge1(float z) {
    const float y = __builtin_amdgcn_logf(z);
    const float hi = __uint_as_float(0x3f317217u), lo = __uint_as_float(0x3377d1cfu);
    const float p = __fmul_rn(y, hi);
    return __fadd_rn(p, __fmaf_rn(y, lo, __fmaf_rn(y, hi, -p)));
}
__device__ __forceinline__ float grp_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __fadd_rn(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __fadd_rn(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// a in lanes 32..63 <-> b in lanes 0..31 (v_permlane32_swap), and a in the odd 16-lane rows
// <-> b in the even rows (v_permlane16_swap).
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}

// 4 x 4 block transpose across the four 16-lane rows: row g holds blocks B_g[c] = (x[2c],
// x[2c+1]) (c = 0..3); afterwards row g holds B_c[g] in (x[2c], x[2c+1]).  When x[j] of row g
// is the dword of dims 16j + 4g.. of an MFMA C column, row g ends with dims 32g + 4c in x[2c]
// and 32g + 16 + 4c in x[2c + 1].
__device__ __forceinline__ void rows_transpose(uint32_t (&x)[8]) {
    swap32(x[0], x[4]);
    swap32(x[1], x[5]);
    swap32(x[2], x[6]);
    swap32(x[3], x[7]);
    swap16(x[0], x[2]);
    swap16(x[1], x[3]);
    swap16(x[4], x[6]);
    swap16(x[5], x[7]);
}

// Max across the 16 lanes of one group (the columns of an MFMA C tile) with DPP: xor 1,
// xor 2 (quad permutes), then half-row and row mirrors; every lane ends with the maximum.
// Four v_max_f32 with the DPP operand folded in (fmaxf on a DPP move costs a move, the DPP
// move, a NaN-quieting max and the max); inputs are never NaN.  Each DPP read of a VGPR
// written by the previous VALU instruction needs two wait states (s_nop 1).
__device__ __forceinline__ float col_max(float v) {
    float r;
    asm("s_nop 1\n\t"
        "v_max_f32_dpp %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf"
        : "=&v"(r) : "v"(v));
    return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ bf16x8 as_bf16x8(u32x2 lo, u32x2 hi) {
    u32x4 u = {lo.x, lo.y, hi.x, hi.y};
    return __builtin_bit_cast(bf16x8, u);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 pair with the hardware conversion (v_cvt_pk_bf16_f32, round to
// nearest even): a in the low half, b in the high half.
__device__ __forceinline__ uint32_t pack2bf(float a, float b) {
    const bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// Two fp32 -> packed fp16 pair, round to nearest even (v_cvt_pk_f16_f32): a in the low half,
// b in the high half.
__device__ __forceinline__ uint32_t pack2h(float a, float b) {
    const h16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// fp32 rounded to TF32 (10 explicit mantissa bits), to nearest with ties away from zero, the
// conversion of a TF32 tensor-core operand (cvt.rna.tf32.f32); infinities and NaN pass unchanged.
__device__ __forceinline__ float tf32_rna(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u & 0x7f800000u) == 0x7f800000u ? x : __uint_as_float((u + 0x1000u) & 0xffffe000u);
}

// fp32 rounded to the nearest bf16 value (returned as fp32).
__device__ __forceinline__ float bf16_round(float x) { return (float)(__bf16)x; }

// Eight fp32 -> bf16x8 (round to nearest even).
__device__ __forceinline__ bf16x8 to_bf16x8(const float* x) {
    u32x4 u = {pack2bf(x[0], x[1]), pack2bf(x[2], x[3]), pack2bf(x[4], x[5]), pack2bf(x[6], x[7])};
    return as_bf16x8(u);
}

// x minus the fp16 value in the low (sub_h_lo) or high (sub_h_hi) half of h, in one
// v_fma_mix_f32 (x + (-h) * 1 with h widened to fp32, one rounding): exact when h is x rounded
// to fp16, the residual of the split below.
__device__ __forceinline__ float sub_h_lo(float x, uint32_t h) {
    float r;
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    return r;
}
__device__ __forceinline__ float sub_h_hi(float x, uint32_t h) {
    float r;
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    return r;
}

// Two-term fp16 split of eight fp32 values, x = hi + lo (both rounded to nearest even): 22
// significant bits while lo stays normal (|x| >= 2^-3), an absolute 2^-25 below that; callers
// scale x into [2^-3, 2^15].  Packed pairs in element order, the layout of an MFMA operand.
__device__ __forceinline__ void split2h8(const float* x, u32x4& hi, u32x4& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h[j] = pack2h(x[2 * j], x[2 * j + 1]);
        l[j] = pack2h(sub_h_lo(x[2 * j], h[j]), sub_h_hi(x[2 * j + 1], h[j]));
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
}

__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
// Two e4m3 codes (bits 0..7, 8..15) -> an fp16 pair holding value * 2^-8, exactly: the code's
// exponent and mantissa fields shifted into fp16 position (biases 7 and 15 differ by 8), which
// also maps e4m3 subnormals onto fp16 subnormals.
__device__ __forceinline__ uint32_t e4m3x2_to_h2(uint32_t b2) {
    const uint32_t t = (b2 & 0xffu) | ((b2 & 0xff00u) << 8);
    return ((t & 0x007f007fu) << 7) | ((t & 0x00800080u) << 8);
}
// Eight e4m3 codes -> eight fp16 (value * 2^-8).
__device__ __forceinline__ u32x4 e4m3x8_to_h8(u32x2 b) {
    return u32x4{e4m3x2_to_h2(b.x & 0xffffu), e4m3x2_to_h2(b.x >> 16), e4m3x2_to_h2(b.y & 0xffffu), e4m3x2_to_h2(b.y >> 16)};
}
// The same eight values with gfx950's conversion instruction (v_cvt_scalef32_pk_f16_fp8, OCP
// e4m3, scale 2^-8): one instruction per pair.  Every finite code converts exactly (the fp16
// grid holds all e4m3 values times 2^-8, subnormals included); htrc_selftest_e4m3 checks all
// 256 codes against e4m3x8_to_h8 on the device.  The state never holds the NaN codes 0x7f / 0xff.
__device__ __forceinline__ uint32_t e4m3x2_to_h2_cvt(uint32_t w, bool hi) {
    return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 0x1p-8f, true)
                                           : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 0x1p-8f, false));
}
__device__ __forceinline__ u32x4 e4m3x8_to_h8_cvt(u32x2 b) {
    return u32x4{e4m3x2_to_h2_cvt(b.x, false), e4m3x2_to_h2_cvt(b.x, true), e4m3x2_to_h2_cvt(b.y, false),
                 e4m3x2_to_h2_cvt(b.y, true)};
}
__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Transposing 64-bit LDS read (ds_read_b64_tr_b16).  Within each 16-lane group, lane i
// receives element i % 4 of the 8-byte reads of lanes 4j + i / 4, j = 0..3.  When lane L of
// a group points at 4 consecutive bf16 of row (R0 + L / 4) at column C0 + 4 (L % 4), lane i
// gets X[R0 + j][C0 + i] for j = 0..3: four consecutive keys at one column, the k-items of
// a PV-type MFMA operand, read straight from row-major data.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
    return __builtin_bit_cast(u32x2, v);
}

// gfx950 transposing 8-bit read: within each group of 16 lanes, lanes 2j and 2j + 1 address the
// two 8-byte halves of a 16-byte piece of "row" j (j = 0..7), and lane L receives byte L % 16 of
// rows 0..7 in order (checked on the device: a byte column of eight rows per lane).
typedef int v2i_lds __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i_lds lds_v2i;
__device__ __forceinline__ u32x2 lds_read_tr8(const void* p) {
    const v2i_lds v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(p));
    return __builtin_bit_cast(u32x2, v);
}

// XOR swizzle of the 16-byte chunks of a 256-byte LDS row: row r keeps chunk c at c ^ swz(r),
// a linear map of r's low four bits (period 16).  Both read patterns on such rows are free of
// bank conflicts whether the LDS serves 128 or 256 bytes per cycle: the 16-byte QK operand
// reads (rows r0 .. r0 + 15 at one chunk: every 8 consecutive rows hit 8 different chunks
// modulo 8, all 16 rows 16 different chunks) and the transposing reads (4 or 8 consecutive
// rows at a chunk pair: 8 or 16 different chunks).  The previous swizzle, 2 (r & 7) + (r >> 3),
// left rows r and r + 4 on one bank group for the QK reads, which the LDS serves 8 lanes
// (128 bytes) at a time: measured, 9.9e7 conflict cycles per stats launch at cfg3.
__device__ __forceinline__ int swz(int r) {
    return ((r & 3) << 1) | ((r >> 2) & 1) | ((((r >> 2) ^ (r >> 3)) & 1) << 3);
}

// Order-preserving uint32 key of a float (larger float -> larger key); -0 maps to +0.
__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

}  // namespace htrc
